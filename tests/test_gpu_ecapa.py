"""Parity of the ECAPA-TDNN GPU path (src/encoder.cpp) against the oracle.

Per layer, at the 4 s / batch-64 shape (T = 398 frames): every TDNN conv
form the encoder uses (block0 k=5 over reflect-padded FBank, the dilated k=3
Res2Net group convs written into their channel slice, 1x1 layers over channel
slices, the ASP attention convs with per-clip bias / tanh / f32 logits) within
2e-3 relative of the oracle's f32 conv1d + ReLU + BatchNorm; the data-movement
kernels bit-exact against numpy; the reductions (SE mean, gate, ASP stats and
pooling, FC+ReLU) against f64 closed forms.  End to end: a random-init
ECAPA-TDNN (C=1024, scale 8, MFA 1536, 192-d) behind the C ABI, pooled
statistics within 2e-3 relative L2 and embeddings at cosine >= 0.9999.
"""
import os
import tempfile

import numpy as np
import pytest

import pyoracle as O
from gpu_util import announce, check_every_clip, close_report, cosine, device_ok
from vdamd import gguf, lib, synth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not device_ok(), reason="no HIP device")]

RTOL = 2e-3
ATOL_RMS = 2e-3
B = 64
N4S = 64000
T4S = 398
CLIPS = (0, 31, 63)


def _sync():
    lib.check(lib.lib().vdk_synchronize())


def _f16w(rng, oc, ic, k):
    return (rng.standard_normal((oc, ic, k), dtype=np.float32) * np.sqrt(2.0 / (ic * k))).astype(np.float16)


def _bn_params(rng, c):
    return (1.0 + 0.1 * rng.standard_normal(c, dtype=np.float32), 0.1 * rng.standard_normal(c, dtype=np.float32),
            0.1 * rng.standard_normal(c, dtype=np.float32), 0.5 + rng.random(c, dtype=np.float32))


def _scale_shift(bn):
    g, b, m, v = bn
    s = (g / np.sqrt(v + np.float32(1e-5))).astype(np.float32)
    return s, (b - s * m).astype(np.float32)


def tdnn_gpu(x_ptr, batch, W, IC, xs, w, dil, bias_dev, y_ptr, ys, bias_bs=0, bn=None, relu=True, tanh=False,
             y_f32=False, ic_pad=None):
    """One vdk_conv2d_ex launch of a time-major TDNN layer (H = 1, pad 0)."""
    OC, ic_w, K = w.shape
    icp = ic_pad or IC
    wp = np.zeros((OC, K, icp), dtype=np.float16)
    wp[:, :, :ic_w] = w.transpose(0, 2, 1)
    dw = lib.DeviceBuffer.from_array(wp)
    keep = [dw]
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride = x_ptr, batch, 1, W, icp, xs
    d.w, d.OC, d.KH, d.KW = dw.ptr, OC, 1, K
    d.stride_h, d.stride_w, d.pad_h, d.pad_w, d.dil_h, d.dil_w = 1, 1, 0, 0, 1, dil
    d.bias, d.bias_batch_stride = bias_dev.ptr, bias_bs
    if bn is not None:
        s, t = _scale_shift(bn)
        ds, dt = lib.DeviceBuffer.from_array(s), lib.DeviceBuffer.from_array(t)
        keep += [ds, dt]
        d.post_scale, d.post_shift = ds.ptr, dt.ptr
    d.act, d.tanh_after = (lib.ACT_RELU if relu else lib.ACT_NONE), int(tanh)
    d.y, d.y_stride, d.y_f32 = y_ptr, ys, int(y_f32)
    d.tile = -1
    lib.check(lib.lib().vdk_conv2d_ex(d, None))
    _sync()


def _oracle_tdnn(x_ct, w, b, dil, bn=None, relu=True):
    y = O.conv1d_same(x_ct, w.astype(np.float32), b, dilation=dil)
    if relu:
        y = np.maximum(y, 0)
    if bn is not None:
        y = O.bn_apply(y, *bn)
    return y


def _assert_close(got, ref, tag):
    ok, ratio, rel = close_report(got, ref, RTOL, ATOL_RMS)
    assert ok and rel <= 2e-3, f"{tag}: max tol ratio {ratio:.3f}, rel-L2 {rel:.2e}"
    return rel


def test_block0_reflect_pad_and_k5_conv():
    rng = np.random.default_rng(11)
    T, nm, C = T4S, 80, 1024
    feats = (3.0 * rng.standard_normal((B, nm, T), dtype=np.float32))
    announce(f"ecapa block0 B={B} T={T} 80->1024 k5")
    L = lib.lib()
    df = lib.DeviceBuffer.from_array(feats)
    x0p = lib.DeviceBuffer(B * (T + 4) * 96 * 2)
    lib.check(L.vdk_feats_tmajor(df.ptr, None, B, nm, T, 2, 96, x0p.ptr, None))
    _sync()
    got_x = x0p.to_array(np.float16, (B, T + 4, 96))
    want = np.zeros((B, T + 4, 96), dtype=np.float16)
    want[:, :, :nm] = np.pad(feats, ((0, 0), (0, 0), (2, 2)), mode="reflect").transpose(0, 2, 1).astype(np.float16)
    assert np.array_equal(got_x.view(np.uint16), want.view(np.uint16))
    w = _f16w(rng, C, nm, 5)
    b = (0.01 * rng.standard_normal(C)).astype(np.float32)
    bn = _bn_params(rng, C)
    db = lib.DeviceBuffer.from_array(b)
    y = lib.DeviceBuffer(B * T * C * 2)
    tdnn_gpu(x0p.ptr, B, T + 4, 96, 96, w, 1, db, y.ptr, C, bn=bn, ic_pad=96)
    got = y.to_array(np.float16, (B, T, C)).astype(np.float32)
    for c in CLIPS:
        rel = _assert_close(got[c].T, _oracle_tdnn(feats[c], w, b, 1, bn), f"block0 clip {c}")
        announce(f"block0 clip {c} rel-L2 {rel:.2e}")


@pytest.mark.parametrize("T", [1, 2, 60, 62, 130, T4S])
def test_feats_tmajor_tiled_matches_elementwise(T):
    """vdk_feats_tmajor's LDS-tiled transpose (c_pad a multiple of 8) against
    its element-wise path (c_pad = 100) and numpy, with per-row means:
    frame blocks cut at 64 frames, reflect padding of short clips."""
    rng = np.random.default_rng(90 + T)
    nb, nm, pad = 3, 80, 2
    feats = (3.0 * rng.standard_normal((nb, nm, T), dtype=np.float32))
    rmean = rng.standard_normal((nb, nm), dtype=np.float32)
    L = lib.lib()
    df, dmn = lib.DeviceBuffer.from_array(feats), lib.DeviceBuffer.from_array(rmean)
    Tp = T + 2 * pad
    outs = {}
    for cp in (96, 100):
        d = lib.DeviceBuffer.from_array(np.full((nb, Tp, cp), 7.0, np.float16))
        lib.check(L.vdk_feats_tmajor(df.ptr, dmn.ptr, nb, nm, T, pad, cp, d.ptr, None))
        _sync()
        outs[cp] = d.to_array(np.float16, (nb, Tp, cp))
    assert np.array_equal(outs[96].view(np.uint16), outs[100][:, :, :96].view(np.uint16))
    assert not outs[100][:, :, 96:].any()
    idx = np.array([min(max(abs(j - pad) if j < pad + T else 2 * (T - 1) - (j - pad), 0), T - 1)
                    for j in range(Tp)])
    want = np.zeros((nb, Tp, 96), np.float16)
    want[:, :, :nm] = (feats[:, :, idx] - rmean[:, :, None]).transpose(0, 2, 1).astype(np.float16)
    assert np.array_equal(outs[96].view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("dil", [2, 3, 4])
def test_reflect_pad_add_kernel(dil):
    """vdk_reflect_pad_add: the Res2Net group input x_j + y_{j-1}, reflect padded, bit-exact."""
    rng = np.random.default_rng(20 + dil)
    T, C, G, j = T4S, 1024, 128, 3
    announce(f"ecapa reflect_pad_add B={B} T={T} dil={dil}")
    t1 = rng.standard_normal((B, T, C), dtype=np.float32).astype(np.float16)
    L = lib.lib()
    dt1 = lib.DeviceBuffer.from_array(t1)
    padb = lib.DeviceBuffer(B * (T + 2 * dil) * G * 2)
    lib.check(L.vdk_reflect_pad_add(dt1.ptr + j * G * 2, C, dt1.ptr + (j - 1) * G * 2, C, B, T, G, dil, padb.ptr,
                                    None))
    _sync()
    s = t1[:, :, j * G:(j + 1) * G].astype(np.float32) + t1[:, :, (j - 1) * G:j * G].astype(np.float32)
    want = np.pad(s, ((0, 0), (dil, dil), (0, 0)), mode="reflect").astype(np.float16)
    got_pad = padb.to_array(np.float16, (B, T + 2 * dil, G))
    assert np.array_equal(got_pad.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("batch,T,dil", [(B, T4S, 2), (B, T4S, 3), (B, T4S, 4), (3, 9, 4), (2, 5, 2)])
def test_res2net_group_conv_reflect_and_next_input(batch, T, dil):
    """The encoder's Res2Net group conv: k=3 dilated over a channel slot of a
    wide time-major tensor with SpeechBrain's reflect padding done by the conv
    (no padded copy), + bias -> ReLU -> BN written into another slot, and the
    second output y + r2 (the next group's input y_j + x_{j+1}); the other
    slots stay untouched."""
    rng = np.random.default_rng(30 + dil + T)
    G = 128
    S = 9 * G
    announce(f"ecapa res2 group conv (reflect fold) B={batch} T={T} dil={dil}")
    t1 = rng.standard_normal((batch, T, S), dtype=np.float32).astype(np.float16)
    L = lib.lib()
    dt1 = lib.DeviceBuffer.from_array(t1)
    dy2 = lib.DeviceBuffer(batch * T * G * 2)
    w = _f16w(rng, G, G, 3)
    b = (0.01 * rng.standard_normal(G)).astype(np.float32)
    bn = _bn_params(rng, G)
    sc, sh = _scale_shift(bn)
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(w.transpose(0, 2, 1))), lib.DeviceBuffer.from_array(b),
            lib.DeviceBuffer.from_array(sc), lib.DeviceBuffer.from_array(sh)]
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride = dt1.ptr + 2 * G * 2, batch, 1, T, G, S
    d.w, d.OC, d.KH, d.KW = keep[0].ptr, G, 1, 3
    d.stride_h, d.stride_w, d.pad_h, d.pad_w, d.dil_h, d.dil_w = 1, 1, 0, dil, 1, dil
    d.reflect_pad = 1
    d.bias, d.post_scale, d.post_shift = keep[1].ptr, keep[2].ptr, keep[3].ptr
    d.act = lib.ACT_RELU
    d.y, d.y_stride = dt1.ptr, S
    d.y2, d.y2_stride, d.res2, d.res2_stride = dy2.ptr, G, dt1.ptr + 3 * G * 2, S
    d.tile = -1
    lib.check(L.vdk_conv2d_ex(d, None))
    _sync()
    out = dt1.to_array(np.float16, (batch, T, S))
    assert np.array_equal(out[:, :, G:].view(np.uint16), t1[:, :, G:].view(np.uint16))
    got = out[:, :, :G].astype(np.float32)
    got2 = dy2.to_array(np.float16, (batch, T, G)).astype(np.float32)
    r2 = t1[:, :, 3 * G:4 * G].astype(np.float32)
    for c in sorted({0, batch // 2, batch - 1}):
        x = t1[c, :, 2 * G:3 * G].astype(np.float32).T
        ref = _oracle_tdnn(x, w, b, dil, bn)
        rel = _assert_close(got[c].T, ref, f"res2 dil {dil} clip {c}")
        _assert_close(got2[c].T, ref + r2[c].T, f"res2 next input dil {dil} clip {c}")
        # y2 = f16(v + r2) and y = f16(v) of the same v: within one f16 rounding of each other
        lim = 2.0 ** -10 * (np.abs(got2[c]) + np.abs(got[c]) + np.abs(r2[c])) + 1e-6
        assert np.all(np.abs(got2[c] - (got[c] + r2[c])) <= lim)
        announce(f"res2 dil {dil} clip {c} rel-L2 {rel:.2e}")
    # the same conv without reflect padding reads zeros past the edges: the
    # first / last dil frames must differ from the reflected result
    d.reflect_pad = 0
    dz = lib.DeviceBuffer(batch * T * S * 2)
    d.y, d.y2 = dz.ptr, None
    d.res2 = None
    lib.check(L.vdk_conv2d_ex(d, None))
    _sync()
    z = dz.to_array(np.float16, (batch, T, S))[:, :, :G].astype(np.float32)
    assert np.array_equal(z[:, dil:T - dil], got[:, dil:T - dil])
    assert not np.array_equal(z[:, :dil], got[:, :dil])


@pytest.mark.parametrize("batch,T,dil,scale", [(B, T4S, 2, 8), (B, T4S, 3, 8), (B, T4S, 4, 8), (3, 37, 4, 8),
                                              (2, 1001, 2, 8), (5, 61, 3, 4), (1, 5, 4, 8)])
def test_res2net_block_one_launch_matches_group_chain(batch, T, dil, scale):
    """vdk_res2_block (all scale - 1 groups of a Res2Net in one launch per time
    tile, halo recomputed) writes the same bits into the same slots as the
    groups run one conv at a time (reflect padding, y_j to slot 0 / j, the
    next input f16(v + x_{j+1}) as the conv's second output), and leaves the
    x slots alone; also a check of group 1 against the oracle conv."""
    rng = np.random.default_rng(40 + dil + T + scale)
    G = 128
    S = (scale + 1) * G
    announce(f"ecapa res2 block B={batch} T={T} dil={dil} scale={scale}")
    t1 = rng.standard_normal((batch, T, S), dtype=np.float32).astype(np.float16)
    L = lib.lib()
    keep, rw = [], lib.Res2Weights()
    ws, bs, bns = [], [], []
    for j in range(scale - 1):
        w = _f16w(rng, G, G, 3)
        b = (0.01 * rng.standard_normal(G)).astype(np.float32)
        bn = _bn_params(rng, G)
        sc, sh = _scale_shift(bn)
        bufs = [lib.DeviceBuffer.from_array(np.ascontiguousarray(w.transpose(0, 2, 1))), lib.DeviceBuffer.from_array(b),
                lib.DeviceBuffer.from_array(sc), lib.DeviceBuffer.from_array(sh)]
        keep += bufs
        rw.w[j], rw.bias[j], rw.scale[j], rw.shift[j] = (x.ptr for x in bufs)
        ws.append(w), bs.append(b), bns.append(bn)
    # the chain: group j reads x_1 (slot 2) or the previous group's second
    # output, writes slot 0 (j = 1) or slot j, and f16(v + x_{j+1}) to a side buffer
    dchain = lib.DeviceBuffer.from_array(t1)
    side = [lib.DeviceBuffer(batch * T * G * 2) for _ in range(2)]
    for j in range(1, scale):
        last = j + 1 == scale
        d = lib.ConvDesc()
        if j == 1:
            d.x, d.x_stride = dchain.ptr + 2 * G * 2, S
        else:
            d.x, d.x_stride = side[j & 1].ptr, G
        d.batch, d.H, d.W, d.IC = batch, 1, T, G
        d.w, d.OC, d.KH, d.KW = rw.w[j - 1], G, 1, 3
        d.stride_h, d.stride_w, d.pad_h, d.pad_w, d.dil_h, d.dil_w = 1, 1, 0, dil, 1, dil
        d.reflect_pad = 1
        d.bias, d.post_scale, d.post_shift = rw.bias[j - 1], rw.scale[j - 1], rw.shift[j - 1]
        d.act = lib.ACT_RELU
        d.y, d.y_stride = dchain.ptr + (0 if j == 1 else j) * G * 2, S
        if not last:
            d.y2, d.y2_stride, d.res2, d.res2_stride = side[(j + 1) & 1].ptr, G, dchain.ptr + (j + 2) * G * 2, S
        d.tile = -1
        lib.check(L.vdk_conv2d_ex(d, None))
    dblk = lib.DeviceBuffer.from_array(t1)
    lib.check(L.vdk_res2_block(dblk.ptr, S, batch, T, G, scale, dil, rw, None))
    _sync()
    want = dchain.to_array(np.float16, (batch, T, S))
    got = dblk.to_array(np.float16, (batch, T, S))
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    assert np.array_equal(got[:, :, scale * G:].view(np.uint16), t1[:, :, scale * G:].view(np.uint16))
    c = batch - 1
    ref = _oracle_tdnn(t1[c, :, 2 * G:3 * G].astype(np.float32).T, ws[0], bs[0], dil, bns[0])
    _assert_close(got[c, :, :G].astype(np.float32).T, ref, f"res2 block group 1 clip {c}")


def test_1x1_layers_over_channel_slices():
    rng = np.random.default_rng(31)
    T, C, M = T4S, 1024, 1536
    announce(f"ecapa 1x1 slices B={B} T={T}")
    cat = rng.standard_normal((B, T, 3 * C), dtype=np.float32).astype(np.float16)
    dcat = lib.DeviceBuffer.from_array(cat)
    # tdnn1 of block 3 reads slice 1 of the MFA input (stride 3C)
    w = _f16w(rng, C, C, 1)
    b = (0.01 * rng.standard_normal(C)).astype(np.float32)
    bn = _bn_params(rng, C)
    db = lib.DeviceBuffer.from_array(b)
    y = lib.DeviceBuffer(B * T * C * 2)
    tdnn_gpu(dcat.ptr + C * 2, B, T, C, 3 * C, w, 1, db, y.ptr, C, bn=bn)
    got = y.to_array(np.float16, (B, T, C)).astype(np.float32)
    for c in CLIPS:
        _assert_close(got[c].T, _oracle_tdnn(cat[c, :, C:2 * C].astype(np.float32).T, w, b, 1, bn),
                      f"tdnn1 slice clip {c}")
    # MFA over the whole concatenation
    wm = _f16w(rng, M, 3 * C, 1)
    bm = (0.01 * rng.standard_normal(M)).astype(np.float32)
    bnm = _bn_params(rng, M)
    dbm = lib.DeviceBuffer.from_array(bm)
    ym = lib.DeviceBuffer(B * T * M * 2)
    tdnn_gpu(dcat.ptr, B, T, 3 * C, 3 * C, wm, 1, dbm, ym.ptr, M, bn=bnm)
    gotm = ym.to_array(np.float16, (B, T, M)).astype(np.float32)
    for c in CLIPS:
        rel = _assert_close(gotm[c].T, _oracle_tdnn(cat[c].astype(np.float32).T, wm, bm, 1, bnm), f"mfa clip {c}")
        announce(f"mfa clip {c} rel-L2 {rel:.2e}")


def test_asp_attention_convs():
    rng = np.random.default_rng(41)
    T, M, A = T4S, 1536, 128
    announce(f"ecapa asp convs B={B} T={T}")
    x = np.abs(rng.standard_normal((B, T, M), dtype=np.float32) * 4).astype(np.float16)
    dx = lib.DeviceBuffer.from_array(x)
    w = _f16w(rng, A, M, 1)
    pb = rng.standard_normal((B, A), dtype=np.float32)
    bn = _bn_params(rng, A)
    dpb = lib.DeviceBuffer.from_array(pb)
    a1 = lib.DeviceBuffer(B * T * A * 2)
    tdnn_gpu(dx.ptr, B, T, M, M, w, 1, dpb, a1.ptr, A, bias_bs=A, bn=bn, tanh=True)
    ga1 = a1.to_array(np.float16, (B, T, A))
    for c in CLIPS:
        ref = np.tanh(_oracle_tdnn(x[c].astype(np.float32).T, w, pb[c], 1, bn))
        _assert_close(ga1[c].astype(np.float32).T, ref, f"asp.tdnn clip {c}")
    wc = _f16w(rng, M, A, 1)
    bc = (0.01 * rng.standard_normal(M)).astype(np.float32)
    dbc = lib.DeviceBuffer.from_array(bc)
    lg = lib.DeviceBuffer(B * T * M * 4)
    tdnn_gpu(a1.ptr, B, T, A, A, wc, 1, dbc, lg.ptr, M, relu=False, y_f32=True)
    glg = lg.to_array(np.float32, (B, T, M))
    for c in CLIPS:
        ref = _oracle_tdnn(ga1[c].astype(np.float32).T, wc, bc, 1, None, relu=False)
        rel = _assert_close(glg[c].T, ref, f"asp.conv clip {c}")
        announce(f"asp.conv clip {c} rel-L2 {rel:.2e}")


def test_se_and_asp_reductions():
    rng = np.random.default_rng(51)
    T, C, M = T4S, 1024, 1536
    L = lib.lib()
    announce(f"ecapa reductions B={B} T={T}")
    # SE squeeze over a channel slice of a wider tensor
    t2 = rng.standard_normal((B, T, 2 * C), dtype=np.float32).astype(np.float16)
    dt2 = lib.DeviceBuffer.from_array(t2)
    dm = lib.DeviceBuffer(B * C * 4)
    lib.check(L.vdk_channel_mean(dt2.ptr + C * 2, 2 * C, B, T, C, dm.ptr, None))
    _sync()
    want = t2[:, :, C:].astype(np.float64).mean(axis=1)
    assert np.abs(dm.to_array(np.float32, (B, C)) - want).max() <= 1e-6 * max(1.0, np.abs(want).max())
    # gate + residual into a slice of the MFA input
    gate = rng.standard_normal((B, C), dtype=np.float32) * 3
    res = rng.standard_normal((B, T, C), dtype=np.float32).astype(np.float16)
    dg, dr = lib.DeviceBuffer.from_array(gate), lib.DeviceBuffer.from_array(res)
    cat = np.zeros((B, T, 3 * C), dtype=np.float16)
    dcat = lib.DeviceBuffer.from_array(cat)
    lib.check(L.vdk_se_gate_residual(dt2.ptr, 2 * C, dg.ptr, dr.ptr, C, B, T, C, dcat.ptr + 2 * C * 2, 3 * C, None))
    _sync()
    gcat = dcat.to_array(np.float16, (B, T, 3 * C))
    sig = 1.0 / (1.0 + np.exp(-gate.astype(np.float64)))
    want = t2[:, :, :C].astype(np.float64) * sig[:, None, :] + res.astype(np.float64)
    got = gcat[:, :, 2 * C:].astype(np.float64)
    assert np.all(np.abs(got - want) <= 2.0 ** -10 * np.abs(want) + 1e-6)
    assert not gcat[:, :, :2 * C].any()
    # the same with the sigmoid taken once per (clip, channel) by the FC's
    # reduce (VDK_ACT_SIGMOID, the model's path): the same bits
    ident = np.eye(C, dtype=np.float32)
    dgi, dsig = lib.DeviceBuffer.from_array(np.ascontiguousarray(gate)), lib.DeviceBuffer(B * C * 4)
    dwi = lib.DeviceBuffer.from_array(ident)
    wsz = L.vdk_linear_workspace_size(B, C, C)
    dwk = lib.DeviceBuffer(wsz)
    lib.check(L.vdk_linear_ex(dgi.ptr, B, C, dwi.ptr, None, None, C, lib.ACT_SIGMOID, dsig.ptr, dwk.ptr, wsz, None))
    dcat2 = lib.DeviceBuffer.from_array(cat)
    lib.check(L.vdk_se_scale_residual(dt2.ptr, 2 * C, dsig.ptr, dr.ptr, C, B, T, C, dcat2.ptr + 2 * C * 2, 3 * C,
                                      None))
    _sync()
    assert np.array_equal(dcat2.to_array(np.float16, (B, T, 3 * C)).view(np.uint16), gcat.view(np.uint16))
    # ASP global statistics and attentive pooling
    x = (rng.standard_normal((B, T, M), dtype=np.float32) * 2 + 1).astype(np.float16)
    x[1, :, 5] = 0.5           # a constant channel: variance clamps to eps
    dx = lib.DeviceBuffer.from_array(x)
    ds = lib.DeviceBuffer(B * 2 * M * 4)
    lib.check(L.vdk_asp_stats(dx.ptr, M, B, T, M, 1e-12, ds.ptr, None))
    _sync()
    xs = x.astype(np.float64)
    mu = xs.mean(axis=1)
    sd = np.sqrt(np.maximum(((xs - mu[:, None, :]) ** 2).mean(axis=1), 1e-12))
    gs = ds.to_array(np.float32, (B, 2 * M))
    assert np.allclose(gs[:, :M], mu, rtol=1e-5, atol=1e-6)
    assert np.allclose(gs[:, M:], sd, rtol=1e-5, atol=1e-6)
    assert gs[1, M + 5] == np.float32(1e-6)
    logits = rng.standard_normal((B, T, M), dtype=np.float32) * 4
    dl = lib.DeviceBuffer.from_array(logits)
    dp = lib.DeviceBuffer(B * 2 * M * 4)
    lib.check(L.vdk_asp_pool(dl.ptr, M, dx.ptr, M, B, T, M, 1e-12, dp.ptr, None))
    _sync()
    lg = logits.astype(np.float64)
    a = np.exp(lg - lg.max(axis=1, keepdims=True))
    a /= a.sum(axis=1, keepdims=True)
    mu = (a * xs).sum(axis=1)
    sd = np.sqrt(np.maximum((a * (xs - mu[:, None, :]) ** 2).sum(axis=1), 1e-12))
    gp = dp.to_array(np.float32, (B, 2 * M))
    assert np.allclose(gp[:, :M], mu, rtol=1e-5, atol=1e-5)
    assert np.allclose(gp[:, M:], sd, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("batch,T", [(64, 398), (3, 1), (2, 63), (2, 64), (2, 65), (2, 130), (1, 998)])
def test_asp_attention_pool_fused(batch, T):
    """vdk_asp_attn_pool (the asp.conv logits and the pooling in one launch)
    against the f64 softmax pooling of the same f16 operands and against the
    two-launch path (f32 logits from the conv kernel, then vdk_asp_pool); T
    covers one frame, the 64-frame chunk edges and a 10 s clip."""
    L = lib.lib()
    rng = np.random.default_rng(batch * 1000 + T)
    M, A = 1536, 128
    announce(f"asp attn pool B={batch} T={T}")
    a1 = np.tanh(rng.standard_normal((batch, T, A), dtype=np.float32)).astype(np.float16)
    w = (rng.standard_normal((M, A), dtype=np.float32) * 0.3).astype(np.float16)
    bc = (rng.standard_normal(M) * 0.5).astype(np.float32)
    x = (rng.standard_normal((batch, T, M), dtype=np.float32) * 2 + 1).astype(np.float16)
    x[:, :, 7] = 0.25                      # constant channel: the variance clamps to eps
    w[11] *= 16                            # sharp attention on channel 11: the running max moves a lot
    da1, dw, db, dx = (lib.DeviceBuffer.from_array(v) for v in (a1, w, bc, x))
    dp = lib.DeviceBuffer(batch * 2 * M * 4)
    lib.check(L.vdk_asp_attn_pool(da1.ptr, A, dw.ptr, db.ptr, A, dx.ptr, M, batch, T, M, 1e-12, dp.ptr, None))
    _sync()
    got = dp.to_array(np.float32, (batch, 2 * M)).astype(np.float64)
    lg = a1.astype(np.float64) @ w.astype(np.float64).T + bc
    a = np.exp(lg - lg.max(axis=1, keepdims=True))
    a /= a.sum(axis=1, keepdims=True)
    xs = x.astype(np.float64)
    mu = (a * xs).sum(axis=1)
    sd = np.sqrt(np.maximum((a * (xs - mu[:, None, :]) ** 2).sum(axis=1), 1e-12))
    assert np.allclose(got[:, :M], mu, rtol=1e-5, atol=1e-5), np.abs(got[:, :M] - mu).max()
    assert np.allclose(got[:, M:], sd, rtol=1e-5, atol=1e-5), np.abs(got[:, M:] - sd).max()
    assert np.all(got[:, M + 7] == np.float32(1e-6))
    # the two-launch path on the same operands
    lgd = lib.DeviceBuffer(batch * T * M * 4)
    tdnn_gpu(da1.ptr, batch, T, A, A, w.reshape(M, A, 1), 1, db, lgd.ptr, M, relu=False, y_f32=True)
    dq = lib.DeviceBuffer(batch * 2 * M * 4)
    lib.check(L.vdk_asp_pool(lgd.ptr, M, dx.ptr, M, batch, T, M, 1e-12, dq.ptr, None))
    _sync()
    two = dq.to_array(np.float32, (batch, 2 * M)).astype(np.float64)
    assert np.allclose(got, two, rtol=1e-5, atol=1e-5), np.abs(got - two).max()


def test_linear_relu():
    rng = np.random.default_rng(61)
    L = lib.lib()
    Bn, I, Oo = 64, 1024, 128
    x = rng.standard_normal((Bn, I), dtype=np.float32)
    w = (rng.standard_normal((Oo, I), dtype=np.float32) / 32).astype(np.float32)
    b = rng.standard_normal(Oo, dtype=np.float32)
    dx, dw, db = (lib.DeviceBuffer.from_array(a) for a in (x, w, b))
    dy = lib.DeviceBuffer(Bn * Oo * 4)
    nw = L.vdk_linear_workspace_size(Bn, I, Oo)
    work = lib.DeviceBuffer(nw)
    lib.check(L.vdk_linear_ex(dx.ptr, Bn, I, dw.ptr, db.ptr, None, Oo, 1, dy.ptr, work.ptr, nw, None))
    _sync()
    want = np.maximum(x.astype(np.float64) @ w.astype(np.float64).T + b, 0)
    got = dy.to_array(np.float32, (Bn, Oo))
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)
    assert (got == 0).sum() == (want == 0).sum()


# ------------------------------------------------------------------ end to end

@pytest.fixture(scope="module")
def ecapa():
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "ecapa_f16.gguf")
    synth.write_ecapa(path, seed=7)
    ctx = lib.Context(path)
    net = O.OracleEcapa(gguf.GGUFFile(path))
    yield path, ctx, net
    ctx.close()


def test_ecapa_batch64_matches_oracle(ecapa):
    path, ctx, net = ecapa
    pcm = synth.clips(4711, B, N4S)
    announce("e2e ecapa B=64 4s capture")
    cap = ctx.capture(pcm)
    assert cap["pooled"].shape[1] == 2 * 1536
    for c in CLIPS:
        feats = O.fbank(pcm[c])
        assert np.abs(cap["feats"][c] - feats).max() <= 1e-4
        emb, caps = net.forward(feats, capture=True)
        rel = np.linalg.norm(cap["pooled"][c] - caps["pooled"]) / np.linalg.norm(caps["pooled"])
        assert rel <= 2e-3, f"pooled rel-L2 {rel:.2e} clip {c}"
        assert cosine(cap["pre_norm"][c], caps["pre_norm"]) >= 0.9999
        cs = cosine(cap["emb"][c], emb)
        announce(f"ecapa clip {c}: cosine {cs:.7f} pooled rel {rel:.2e}")
        assert cs >= 0.9999
        assert abs(np.linalg.norm(cap["emb"][c]) - 1.0) < 1e-5
    check_every_clip(ctx, net, pcm, cap["emb"], "ecapa B=64", invariance=(1, 32, 62))
    # batch invariance: the same clip alone gives the same bits
    one = ctx.embed_batch(pcm[31:32])
    assert np.array_equal(one[0], cap["emb"][31])


@pytest.mark.parametrize("n", [1040, 4000, 40000])   # 1040 samples = 5 frames, the fewest ECAPA takes
def test_ecapa_embed_pcm_lengths(ecapa, n):
    path, ctx, net = ecapa
    announce(f"e2e ecapa B=1 n={n}")
    pcm = synth.clip(900 + n, n)
    got = ctx.embed_pcm(pcm)
    ref = net.forward(O.fbank(pcm))
    assert got.shape == (192,)
    assert cosine(got, ref) >= 0.9999


def test_ecapa_verify_matches_oracle(ecapa, golden_dir):
    path, ctx, net = ecapa
    announce("e2e ecapa verify")
    a = synth.clip(1, 48000)
    b = synth.clip(2, 56000)
    d_gpu, _ = ctx.verify_pcm(a, b, 0.5)
    ea, eb = net.forward(O.fbank(a)), net.forward(O.fbank(b))
    d_ref = 1.0 - float(np.dot(ea.astype(np.float64), eb.astype(np.float64)))
    assert abs(d_gpu - d_ref) <= 2e-3
    for thr in (d_ref - 5e-3, d_ref + 5e-3):
        assert ctx.verify_pcm(a, b, thr)[1] == (d_ref <= thr)


def test_ecapa_real_checkpoint_widths_q8_0_batch64():
    """The published SpeechBrain layout (models/ecapa_tdnn_manifest.txt: MFA
    3072, asp.tdnn 9216 -> 128, asp_bn 6144, fc 6144 -> 192) with the mfa
    weight stored as 2-D Q8_0 the way the converter's q8_0 plan stores it;
    B=64 x 4 s, every clip against the oracle on the same dequantised weights."""
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "ecapa_real_q8_0.gguf")
    synth.write_ecapa(path, seed=17, mfa=3072, wtype=gguf.GGML_Q8_0)
    g = gguf.GGUFFile(path)
    assert g.tensors["mfa.conv.conv.weight"][0] == gguf.GGML_Q8_0
    assert g.tensors["mfa.conv.conv.weight"][1] == [3072, 3072]
    ctx = lib.Context(path)
    try:
        net = O.OracleEcapa(g)
        pcm = synth.clips(4713, B, N4S)
        announce("e2e ecapa MFA 3072 q8_0 B=64 4s capture")
        cap = ctx.capture(pcm)
        assert cap["pooled"].shape[1] == 2 * 3072
        for c in CLIPS:
            emb, caps = net.forward(O.fbank(pcm[c]), capture=True)
            rel = np.linalg.norm(cap["pooled"][c] - caps["pooled"]) / np.linalg.norm(caps["pooled"])
            assert rel <= 2e-3, f"pooled rel-L2 {rel:.2e} clip {c}"
            cs = cosine(cap["emb"][c], emb)
            announce(f"ecapa-3072 clip {c}: cosine {cs:.7f} pooled rel {rel:.2e}")
            assert cs >= 0.9999
        check_every_clip(ctx, net, pcm, cap["emb"], "ecapa MFA 3072 q8_0 B=64", invariance=(0, 40))
    finally:
        ctx.close()
