"""Parity of the CAM++ GPU path (src/encoder_campplus.cpp) against the oracle.

Per layer at the 10 s / batch-32 shape (T = 998 frames, T' = 499): the FCM
convs with a frequency-only stride, the final FCM conv's time-major store
feeding the k=5 stride-2 TDNN (input channels permuted from the reference's
c*H + h), the dilated linear_local with the per-segment context gate stored
into its slice of the dense state; the BN+ReLU, segment-sum and context-MLP
kernels against closed forms.  End to end: a random-init CAM++ with q8_0 1x1
weights behind the C ABI, pooled statistics within 2e-3 relative L2 and
embeddings at cosine >= 0.9999 vs the oracle on the same dequantised weights.
"""
import os
import tempfile

import numpy as np
import pytest

import pyoracle as O
from gpu_util import announce, check_every_clip, close_report, conv_ex, cosine, device_ok
from vdamd import gguf, lib, synth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not device_ok(), reason="no HIP device")]

RTOL = 2e-3
ATOL_RMS = 2e-3
B = 32
N10S = 160000
T10S = 998
TP = 499
CLIPS = (0, 15, 31)


def _sync():
    lib.check(lib.lib().vdk_synchronize())


def _assert_close(got, ref, tag):
    ok, ratio, rel = close_report(got, ref, RTOL, ATOL_RMS)
    assert ok and rel <= 2e-3, f"{tag}: max tol ratio {ratio:.3f}, rel-L2 {rel:.2e}"
    return rel


def _w(rng, oc, ic, kh, kw):
    return (rng.standard_normal((oc, ic, kh, kw), dtype=np.float32) * np.sqrt(2.0 / (ic * kh * kw))).astype(
        np.float16)


def test_fcm_freq_stride_convs():
    """3x3 stride (2, 1) pad 1 and the 1x1 stride (2, 1) shortcut on [B][80][T][32]."""
    rng = np.random.default_rng(71)
    H, T, C = 80, T10S, 32
    announce(f"campp fcm convs B={B} H={H} T={T}")
    x = np.maximum(rng.standard_normal((B, H, T, C), dtype=np.float32), 0).astype(np.float16)
    dx = lib.DeviceBuffer.from_array(x)
    Ho = 40
    for K, pad, tag in ((3, 1, "conv1"), (1, 0, "shortcut")):
        w = _w(rng, C, C, K, K)
        b = rng.uniform(-0.5, 0.5, C).astype(np.float32)
        y = lib.DeviceBuffer(B * Ho * T * C * 2)
        conv_ex(dx.ptr, B, H, T, C, 0, w.transpose(0, 2, 3, 1), C, K, K, y.ptr, sh=2, sw=1, ph=pad, pw=pad,
                bias=b, act=lib.ACT_RELU if K == 3 else lib.ACT_NONE)
        got = y.to_array(np.float16, (B, Ho, T, C)).astype(np.float32)
        for c in CLIPS[:2]:
            ref = O.conv2d_g(x[c].astype(np.float32).transpose(2, 0, 1), w.astype(np.float32), sh=2, sw=1, ph=pad,
                             pw=pad, bias=b, relu=K == 3)
            rel = _assert_close(got[c].transpose(2, 0, 1), ref, f"fcm {tag} clip {c}")
            announce(f"fcm {tag} clip {c} rel-L2 {rel:.2e}")


def test_fcm_out_time_major_and_tdnn():
    """Final FCM conv stored time-major, then the k=5 stride-2 TDNN whose 320
    input channels are the reference's c*10 + h, read here at h*32 + c."""
    rng = np.random.default_rng(72)
    H, T, C, OCT = 20, T10S, 32, 128
    announce(f"campp fcm_out + tdnn B={B} T={T}")
    x = np.maximum(rng.standard_normal((B, H, T, C), dtype=np.float32), 0).astype(np.float16)
    dx = lib.DeviceBuffer.from_array(x)
    w = _w(rng, C, C, 3, 3)
    b = rng.uniform(-0.5, 0.5, C).astype(np.float32)
    yt = lib.DeviceBuffer(B * T * 10 * C * 2)
    conv_ex(dx.ptr, B, H, T, C, 0, w.transpose(0, 2, 3, 1), C, 3, 3, yt.ptr, sh=2, ph=1, pw=1, bias=b,
            act=lib.ACT_RELU, y_time_major=1)
    got = yt.to_array(np.float16, (B, T, 10, C))
    fcm = []
    for c in CLIPS:
        ref = O.conv2d_g(x[c].astype(np.float32).transpose(2, 0, 1), w.astype(np.float32), sh=2, ph=1, pw=1,
                         bias=b, relu=True)                                     # [32][10][T]
        _assert_close(got[c].astype(np.float32).transpose(2, 1, 0), ref, f"fcm_out clip {c}")
        fcm.append(got[c].astype(np.float32).transpose(2, 1, 0).reshape(C * 10, T))   # channel c*10 + h
    wt = _w(rng, OCT, C * 10, 1, 5)[:, :, 0, :]                                # reference [OC][c*10+h][k]
    bt = rng.uniform(-0.5, 0.5, OCT).astype(np.float32)
    wp = wt.reshape(OCT, C, 10, 5).transpose(0, 3, 2, 1).reshape(OCT, 1, 5, 10 * C)   # [OC][1][k][h*32+c]
    dense = lib.DeviceBuffer(B * TP * 512 * 2)
    conv_ex(yt.ptr, B, 1, T, 10 * C, 0, wp, OCT, 1, 5, dense.ptr, ys=512, sw=2, pw=2, bias=bt, act=lib.ACT_RELU)
    gd = dense.to_array(np.float16, (B, TP, 512))
    for i, c in enumerate(CLIPS):
        ref = O.conv2d_g(fcm[i][:, None, :], wt[:, :, None, :].astype(np.float32), sw=2, pw=2, bias=bt,
                         relu=True)[:, 0, :]
        rel = _assert_close(gd[c, :, :OCT].astype(np.float32).T, ref, f"tdnn clip {c}")
        announce(f"tdnn clip {c} rel-L2 {rel:.2e}")


@pytest.mark.parametrize("dil", [1, 2])
def test_linear_local_gated_into_dense_slice(dil):
    rng = np.random.default_rng(80 + dil)
    T, BC, G, CMAX, C0, SEG = TP, 128, 32, 512, 160, 100
    nseg = (T + SEG - 1) // SEG
    announce(f"campp linear_local dil={dil} B={B} T'={T}")
    cc = np.maximum(rng.standard_normal((B, T, BC), dtype=np.float32), 0).astype(np.float16)
    gate = rng.uniform(0, 1, (B, nseg, G)).astype(np.float32)
    dense = rng.standard_normal((B, T, CMAX), dtype=np.float32).astype(np.float16)
    dcc, dd = lib.DeviceBuffer.from_array(cc), lib.DeviceBuffer.from_array(dense)
    w = _w(rng, G, BC, 1, 3)
    conv_ex(dcc.ptr, B, 1, T, BC, 0, w.transpose(0, 2, 3, 1), G, 1, 3, dd.ptr + C0 * 2, ys=CMAX, pw=dil, dw=dil,
            gate=gate, gate_seg=SEG, gate_nseg=nseg)
    out = dd.to_array(np.float16, (B, T, CMAX))
    keep = np.ones(CMAX, dtype=bool)
    keep[C0:C0 + G] = False
    assert np.array_equal(out[:, :, keep].view(np.uint16), dense[:, :, keep].view(np.uint16))
    seg_of_t = np.arange(T) // SEG
    for c in CLIPS:
        y = O.conv2d_g(cc[c].astype(np.float32).T[:, None, :], w.astype(np.float32), pw=dil, dw=dil)[:, 0, :]
        ref = y * gate[c][seg_of_t].T
        rel = _assert_close(out[c, :, C0:C0 + G].astype(np.float32).T, ref, f"linear_local dil {dil} clip {c}")
        announce(f"linear_local dil {dil} clip {c} rel-L2 {rel:.2e}")


def test_bn_act_segment_sums_and_context():
    rng = np.random.default_rng(90)
    L = lib.lib()
    T, C, XS, SEG, H1, G = TP, 384, 512, 100, 64, 32
    announce(f"campp helpers B={B} T'={T}")
    x = rng.standard_normal((B, T, XS), dtype=np.float32).astype(np.float16)
    s = rng.uniform(0.5, 1.5, C).astype(np.float32)
    t = rng.uniform(-0.5, 0.5, C).astype(np.float32)
    dx, ds, dt = (lib.DeviceBuffer.from_array(a) for a in (x, s, t))
    dy = lib.DeviceBuffer(B * T * C * 2)
    lib.check(L.vdk_bn_act(dx.ptr, XS, B * T, C, ds.ptr, dt.ptr, lib.ACT_RELU, dy.ptr, C, None))
    _sync()
    got = dy.to_array(np.float16, (B, T, C)).astype(np.float64)
    want = np.maximum(x[:, :, :C].astype(np.float64) * s + t, 0)
    assert np.all(np.abs(got - want) <= 2.0 ** -10 * np.abs(want) + 1e-6)
    # segment sums over a 128-channel map with a partial last segment
    BC = 128
    cc = np.maximum(rng.standard_normal((B, T, BC), dtype=np.float32), 0).astype(np.float16)
    dcc = lib.DeviceBuffer.from_array(cc)
    nseg = (T + SEG - 1) // SEG
    dsum = lib.DeviceBuffer(B * nseg * BC * 4)
    lib.check(L.vdk_segment_sums(dcc.ptr, BC, B, T, BC, SEG, dsum.ptr, None))
    _sync()
    sums = dsum.to_array(np.float32, (B, nseg, BC))
    ref = np.stack([cc[:, i * SEG:(i + 1) * SEG].astype(np.float64).sum(axis=1) for i in range(nseg)], axis=1)
    assert np.allclose(sums, ref, rtol=1e-6, atol=1e-5)
    # context MLP: Q-matrix form of the context (mean over T' + segment average / 100)
    w1 = rng.standard_normal((H1, BC), dtype=np.float32) / 8
    b1 = rng.standard_normal(H1, dtype=np.float32) / 4
    w2 = rng.standard_normal((G, H1), dtype=np.float32) / 8
    b2 = rng.standard_normal(G, dtype=np.float32) / 4
    dw1, db1, dw2, db2 = (lib.DeviceBuffer.from_array(a) for a in (w1, b1, w2, b2))
    dg = lib.DeviceBuffer(B * nseg * G * 4)
    lib.check(L.vdk_cam_context(dsum.ptr, B, T, BC, SEG, dw1.ptr, db1.ptr, H1, dw2.ptr, db2.ptr, G, dg.ptr, None))
    _sync()
    gate = dg.to_array(np.float32, (B, nseg, G))
    xc = cc.astype(np.float64)
    ctx = xc.mean(axis=1)[:, None, :] + ref / SEG                              # [B][nseg][BC]
    h = np.maximum(ctx @ w1.T.astype(np.float64) + b1, 0)
    want = 1.0 / (1.0 + np.exp(-(h @ w2.T.astype(np.float64) + b2)))
    assert np.allclose(gate, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("batch,T,dil,bias", [(B, TP, 1, False), (B, TP, 2, True), (3, 257, 2, True), (2, 40, 1, True)])
def test_cam_local_fused_layer(batch, T, dil, bias):
    """vdk_cam_local (context sums, mask MLP and the gated k=3 linear_local in
    one launch) against the f64 context of the dense Q-matrix form and the
    oracle's conv, and against the three-launch path (segment sums, context,
    gated conv); the other channels of the dense buffer stay untouched."""
    rng = np.random.default_rng(100 + T + dil)
    L = lib.lib()
    BC, G, H1, SEG, CMAX, C0 = 128, 32, 64, 100, 384, 224
    nseg = (T + SEG - 1) // SEG
    announce(f"campp cam_local B={batch} T'={T} dil={dil} bias={bias}")
    cc = np.maximum(rng.standard_normal((batch, T, BC), dtype=np.float32), 0).astype(np.float16)
    dense = rng.standard_normal((batch, T, CMAX), dtype=np.float32).astype(np.float16)
    w1 = rng.standard_normal((H1, BC), dtype=np.float32) / 8
    b1 = rng.standard_normal(H1, dtype=np.float32) / 4
    w2 = rng.standard_normal((G, H1), dtype=np.float32) / 8
    b2 = rng.standard_normal(G, dtype=np.float32) / 4
    w = _w(rng, G, BC, 1, 3)                                             # [G][BC][1][3] f16
    bl = (rng.standard_normal(G, dtype=np.float32) * 0.1) if bias else None
    dcc, dd = lib.DeviceBuffer.from_array(cc), lib.DeviceBuffer.from_array(dense)
    dw1, db1, dw2, db2 = (lib.DeviceBuffer.from_array(a) for a in (w1, b1, w2, b2))
    dwl = lib.DeviceBuffer.from_array(np.ascontiguousarray(w[:, :, 0, :].transpose(0, 2, 1)))   # [G][3][BC]
    dbl = lib.DeviceBuffer.from_array(bl) if bias else None
    lib.check(L.vdk_cam_local(dcc.ptr, BC, batch, T, BC, SEG, dil, dw1.ptr, db1.ptr, H1, dw2.ptr, db2.ptr, dwl.ptr,
                              dbl.ptr if dbl else None, dd.ptr + C0 * 2, CMAX, None, None, None))
    _sync()
    out = dd.to_array(np.float16, (batch, T, CMAX))
    keep = np.ones(CMAX, dtype=bool)
    keep[C0:C0 + G] = False
    assert np.array_equal(out[:, :, keep].view(np.uint16), dense[:, :, keep].view(np.uint16))
    xc = cc.astype(np.float64)
    segs = np.stack([xc[:, i * SEG:(i + 1) * SEG].sum(axis=1) for i in range(nseg)], axis=1)
    ctx = xc.mean(axis=1)[:, None, :] + segs / SEG
    h = np.maximum(ctx @ w1.T.astype(np.float64) + b1, 0)
    gate = 1.0 / (1.0 + np.exp(-(h @ w2.T.astype(np.float64) + b2)))         # [batch][nseg][G]
    seg_of_t = np.arange(T) // SEG
    for c in sorted({0, batch // 2, batch - 1}):
        y = O.conv2d_g(cc[c].astype(np.float32).T[:, None, :], w.astype(np.float32), pw=dil, dw=dil,
                       bias=bl)[:, 0, :]
        ref = y * gate[c][seg_of_t].T
        rel = _assert_close(out[c, :, C0:C0 + G].astype(np.float32).T, ref, f"cam_local clip {c}")
        announce(f"cam_local clip {c} rel-L2 {rel:.2e}")
    # the three-launch path on the same inputs
    dsum = lib.DeviceBuffer(batch * nseg * BC * 4)
    dg = lib.DeviceBuffer(batch * nseg * G * 4)
    lib.check(L.vdk_segment_sums(dcc.ptr, BC, batch, T, BC, SEG, dsum.ptr, None))
    lib.check(L.vdk_cam_context(dsum.ptr, batch, T, BC, SEG, dw1.ptr, db1.ptr, H1, dw2.ptr, db2.ptr, G, dg.ptr, None))
    _sync()
    g3 = dg.to_array(np.float32, (batch, nseg, G))
    assert np.allclose(g3, gate, rtol=1e-5, atol=1e-6)
    d3 = lib.DeviceBuffer(batch * T * G * 2)
    conv_ex(dcc.ptr, batch, 1, T, BC, 0, w.transpose(0, 2, 3, 1), G, 1, 3, d3.ptr, ys=G, pw=dil, dw=dil, bias=bl,
            gate=g3, gate_seg=SEG, gate_nseg=nseg)
    y3 = d3.to_array(np.float16, (batch, T, G)).astype(np.float32)
    got = out[:, :, C0:C0 + G].astype(np.float32)
    # same products and sums; the gates agree to f32 rounding
    assert np.all(np.abs(got - y3) <= 2.0 ** -9 * np.abs(y3) + 1e-6)


# ------------------------------------------------------------------ end to end

@pytest.fixture(scope="module")
def campp():
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "campplus_q8_0.gguf")
    synth.write_campplus(path, seed=5)
    g = gguf.GGUFFile(path)
    assert sum(1 for v in g.tensors.values() if v[0] == gguf.GGML_Q8_0) > 50
    ctx = lib.Context(path)
    net = O.OracleCampplus(g)
    yield path, ctx, net
    ctx.close()


def test_campplus_batch32_matches_oracle(campp):
    path, ctx, net = campp
    pcm = synth.clips(5150, B, N10S)
    announce("e2e campplus B=32 10s capture")
    cap = ctx.capture(pcm)
    assert cap["pooled"].shape[1] == 1024
    for c in CLIPS:
        feats = O.fbank(pcm[c])
        assert np.abs(cap["feats"][c] - feats).max() <= 1e-4
        emb, caps = net.forward(feats, capture=True)
        rel = np.linalg.norm(cap["pooled"][c] - caps["pooled"]) / np.linalg.norm(caps["pooled"])
        assert rel <= 2e-3, f"pooled rel-L2 {rel:.2e} clip {c}"
        assert cosine(cap["pre_norm"][c], caps["pre_norm"]) >= 0.9999
        cs = cosine(cap["emb"][c], emb)
        announce(f"campplus clip {c}: cosine {cs:.7f} pooled rel {rel:.2e}")
        assert cs >= 0.9999
    one = ctx.embed_batch(pcm[15:16])
    assert np.array_equal(one[0], cap["emb"][15])
    check_every_clip(ctx, net, pcm, cap["emb"], "campplus B=32", invariance=(1, 16, 30))


def test_campplus_batch8_3s_every_clip(campp):
    """3 s clips (T' = 149: segments of 100 and 49 frames, so linear1's pixel
    tiles run over three segments at clip boundaries) at batch 8: every clip
    against the oracle and bitwise batch invariance."""
    path, ctx, net = campp
    pcm = synth.clips(5170, 8, 48000)
    announce("e2e campplus B=8 3s")
    emb = ctx.embed_batch(pcm)
    check_every_clip(ctx, net, pcm, emb, "campplus B=8 3s", invariance=(0, 3, 7))


@pytest.mark.parametrize("n", [400, 4000, 40000])
def test_campplus_embed_pcm_lengths(campp, n):
    path, ctx, net = campp
    announce(f"e2e campplus B=1 n={n}")
    pcm = synth.clip(700 + n, n)
    got = ctx.embed_pcm(pcm)
    ref = net.forward(O.fbank(pcm))
    assert got.shape == (192,)
    assert cosine(got, ref) >= 0.9999


def test_campplus_verify_matches_oracle(campp):
    path, ctx, net = campp
    announce("e2e campplus verify")
    a = synth.clip(11, 48000)
    b = synth.clip(12, 56000)
    d_gpu, _ = ctx.verify_pcm(a, b, 0.5)
    ea, eb = net.forward(O.fbank(a)), net.forward(O.fbank(b))
    d_ref = 1.0 - float(np.dot(ea.astype(np.float64), eb.astype(np.float64)))
    assert abs(d_gpu - d_ref) <= 2e-3
    for thr in (d_ref - 5e-3, d_ref + 5e-3):
        assert ctx.verify_pcm(a, b, thr)[1] == (d_ref <= thr)


@pytest.mark.parametrize("batch,T,cin,dil", [(B, TP, 128, 1), (3, 257, 480, 2), (8, 149, 160, 2),
                                             (2, 40, 992, 2), (12, 3, 128, 1), (4, 101, 224, 2)])
def test_cam_dense_equals_cam_then_linear1(batch, T, cin, dil):
    """One launch of a dense layer's CAM and the next layer's linear1
    (vdk_cam_dense) against vdk_cam_local followed by the linear1 conv with
    its BN+ReLU prologue and segment sums: the block buffer (the 32 new
    channels, nothing else touched), the next h and its per-segment sums
    bit for bit; a short last segment (T' = 149, 101), one short segment
    (40), clips of 3 frames, the widest input (992 + 32 = 1024 channels)."""
    rng = np.random.default_rng(31 * T + cin + dil)
    L = lib.lib()
    BC, G, H1, SEG, CMAX = 128, 32, 64, 100, 1024
    nseg = (T + SEG - 1) // SEG
    cn = cin + G
    announce(f"campp cam_dense B={batch} T'={T} cin={cin} dil={dil}")
    dense = rng.standard_normal((batch, T, CMAX), dtype=np.float32).astype(np.float16)
    h = np.maximum(rng.standard_normal((batch, T, BC), dtype=np.float32), 0).astype(np.float16)
    hd = h.astype(np.float64)
    seg = np.stack([hd[:, i * SEG:(i + 1) * SEG].sum(axis=1) for i in range(nseg)], axis=1)   # exact
    w1 = rng.standard_normal((H1, BC), dtype=np.float32) / 8
    b1 = rng.standard_normal(H1, dtype=np.float32) / 4
    w2 = rng.standard_normal((G, H1), dtype=np.float32) / 8
    b2 = rng.standard_normal(G, dtype=np.float32) / 4
    wl = (rng.standard_normal((G, 3, BC), dtype=np.float32) / np.sqrt(3 * BC)).astype(np.float16)
    bl = (rng.standard_normal(G, dtype=np.float32) * 0.1).astype(np.float32)
    wn = (rng.standard_normal((BC, cn), dtype=np.float32) / np.sqrt(cn)).astype(np.float16)
    bn = (rng.standard_normal(BC, dtype=np.float32) * 0.1).astype(np.float32)
    sc = (rng.random(cn, dtype=np.float32) + 0.5).astype(np.float32)
    sh = (rng.standard_normal(cn, dtype=np.float32) * 0.2).astype(np.float32)
    keep = [lib.DeviceBuffer.from_array(a) for a in (h, seg, w1, b1, w2, b2, wl, bl, wn, bn, sc, sh)]
    dh, dseg, dw1, db1, dw2, db2, dwl, dbl, dwn, dbn, dsc, dsh = keep
    # reference: the CAM launch, then linear1 as a conv accumulating into cleared sums
    dA = lib.DeviceBuffer.from_array(dense)
    lib.check(L.vdk_cam_local(dh.ptr, BC, batch, T, BC, SEG, dil, dw1.ptr, db1.ptr, H1, dw2.ptr, db2.ptr, dwl.ptr,
                              dbl.ptr, dA.ptr + 2 * cin, CMAX, dseg.ptr, None, None))
    hA = lib.DeviceBuffer(batch * T * BC * 2)
    segA = lib.DeviceBuffer.from_array(np.zeros((batch, nseg, BC)))
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride = dA.ptr, batch, 1, T, cn, CMAX
    d.w, d.OC, d.KH, d.KW = dwn.ptr, BC, 1, 1
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
    d.bias, d.act = dbn.ptr, lib.ACT_RELU
    d.in_scale, d.in_shift = dsc.ptr, dsh.ptr
    d.seg_sum, d.seg_len = segA.ptr, SEG
    d.y, d.y_stride, d.tile = hA.ptr, BC, -1
    lib.check(L.vdk_conv2d_ex(d, None))
    # one launch
    dB = lib.DeviceBuffer.from_array(dense)
    hB = lib.DeviceBuffer(batch * T * BC * 2)
    segB = lib.DeviceBuffer.from_array(np.full((batch, nseg, BC), 7.0))
    lib.check(L.vdk_cam_dense(dh.ptr, batch, T, SEG, dil, dw1.ptr, db1.ptr, H1, dw2.ptr, db2.ptr, dwl.ptr, dbl.ptr,
                              dB.ptr, CMAX, cin, dseg.ptr, dwn.ptr, dbn.ptr, dsc.ptr, dsh.ptr, hB.ptr, segB.ptr, None))
    _sync()
    a, b = dA.to_array(np.uint16, dense.shape), dB.to_array(np.uint16, dense.shape)
    assert np.array_equal(a, b)
    assert np.array_equal(np.delete(b, np.s_[cin:cn], axis=2), np.delete(dense.view(np.uint16), np.s_[cin:cn], axis=2))
    assert np.array_equal(hA.to_array(np.uint16, (batch, T, BC)), hB.to_array(np.uint16, (batch, T, BC)))
    assert np.array_equal(segA.to_array(np.float64, (batch, nseg, BC)), segB.to_array(np.float64, (batch, nseg, BC)))
    assert L.vdk_cam_dense(dh.ptr, batch, T, SEG, dil, dw1.ptr, db1.ptr, H1, dw2.ptr, db2.ptr, dwl.ptr, dbl.ptr,
                           dB.ptr, CMAX, cin, dseg.ptr, dwn.ptr, dbn.ptr, dsc.ptr, dsh.ptr, dh.ptr, segB.ptr, None) != 0


@pytest.mark.parametrize("batch,T,c_in", [(B, TP, 320), (3, 257, 160), (2, 40, 128),
                                          (8, 149, 128), (8, 49, 160), (16, 101, 256), (12, 3, 128)])
def test_linear1_segment_sums_feed_cam_local(batch, T, c_in):
    """linear1 with seg_sum (the per-(clip, segment) f64 sums of its stored
    f16 outputs, accumulated in the conv's epilogue) equals the exact f64
    sums of h and leaves h bit-identical; cam_local fed those sums (and
    clearing the next layer's buffer) writes the same bits as cam_local
    summing h itself.  T' = 149 (last segment 49 frames), 49 (one short
    segment per clip), 101 (a one-frame last segment) and 3 (clips shorter
    than any pixel tile) put three or more segments into one pixel tile."""
    rng = np.random.default_rng(7 * T + c_in)
    L = lib.lib()
    BC, G, H1, SEG, CMAX = 128, 32, 64, 100, 512
    nseg = (T + SEG - 1) // SEG
    announce(f"campp linear1 seg sums B={batch} T'={T} c_in={c_in}")
    dense = rng.standard_normal((batch, T, CMAX), dtype=np.float32).astype(np.float16)
    s1 = (rng.random(c_in, dtype=np.float32) + 0.5).astype(np.float32)
    t1 = (rng.standard_normal(c_in, dtype=np.float32) * 0.2).astype(np.float32)
    w = (rng.standard_normal((BC, c_in), dtype=np.float32) / np.sqrt(c_in)).astype(np.float16)
    bias = (rng.standard_normal(BC, dtype=np.float32) * 0.1).astype(np.float32)
    dd, ds1, dt1, dw, db = (lib.DeviceBuffer.from_array(a) for a in (dense, s1, t1, w, bias))

    def linear1(seg_buf):
        dh = lib.DeviceBuffer(batch * T * BC * 2)
        d = lib.ConvDesc()
        d.x, d.batch, d.H, d.W, d.IC, d.x_stride = dd.ptr, batch, 1, T, c_in, CMAX
        d.w, d.OC, d.KH, d.KW = dw.ptr, BC, 1, 1
        d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
        d.bias, d.act = db.ptr, lib.ACT_RELU
        d.in_scale, d.in_shift = ds1.ptr, dt1.ptr
        d.y, d.y_stride, d.tile = dh.ptr, BC, -1
        if seg_buf is not None:
            d.seg_sum, d.seg_len = seg_buf.ptr, SEG
        lib.check(L.vdk_conv2d_ex(d, None))
        _sync()
        return dh

    seg = lib.DeviceBuffer.from_array(np.zeros((batch, nseg, BC), dtype=np.float64))
    dh = linear1(seg)
    h = dh.to_array(np.float16, (batch, T, BC))
    h0 = linear1(None).to_array(np.float16, (batch, T, BC))
    assert np.array_equal(h.view(np.uint16), h0.view(np.uint16))
    got = seg.to_array(np.float64, (batch, nseg, BC))
    hd = h.astype(np.float64)
    want = np.stack([hd[:, i * SEG:(i + 1) * SEG].sum(axis=1) for i in range(nseg)], axis=1)
    assert np.array_equal(got, want), np.abs(got - want).max()
    # cam_local from the sums against cam_local summing h itself
    w1 = rng.standard_normal((H1, BC), dtype=np.float32) / 8
    b1 = rng.standard_normal(H1, dtype=np.float32) / 4
    w2 = rng.standard_normal((G, H1), dtype=np.float32) / 8
    b2 = rng.standard_normal(G, dtype=np.float32) / 4
    wl = (rng.standard_normal((G, 3, BC), dtype=np.float32) / np.sqrt(3 * BC)).astype(np.float16)
    bl = (rng.standard_normal(G, dtype=np.float32) * 0.1).astype(np.float32)
    dw1, db1, dw2, db2, dwl, dbl = (lib.DeviceBuffer.from_array(a) for a in (w1, b1, w2, b2, wl, bl))
    nxt = lib.DeviceBuffer.from_array(rng.standard_normal((batch, nseg, BC)))
    outs = []
    for use in (False, True):
        dy = lib.DeviceBuffer(batch * T * G * 2)
        lib.check(L.vdk_cam_local(dh.ptr, BC, batch, T, BC, SEG, 2, dw1.ptr, db1.ptr, H1, dw2.ptr, db2.ptr, dwl.ptr,
                                  dbl.ptr, dy.ptr, G, seg.ptr if use else None, nxt.ptr if use else None, None))
        _sync()
        outs.append(dy.to_array(np.float16, (batch, T, G)))
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
    assert not nxt.to_array(np.float64, (batch, nseg, BC)).any()


@pytest.mark.parametrize("batch,T,c_in", [(B, TP, 320), (B, TP, 1024), (3, 257, 160), (8, 149, 288),
                                          (8, 49, 160), (16, 101, 256), (12, 3, 128)])
def test_linear1_tiles_bitwise(batch, T, c_in):
    """linear1 (BN + ReLU prologue, bias, ReLU, segment sums) on the GEMM
    kernel's narrow tiles with producer / compute waves: the register-staged
    tiles' bits, outputs and f64 segment sums alike (same operand rounding,
    K order and exact sums), including pixel tiles that reach three
    segments."""
    rng = np.random.default_rng(11 * T + c_in)
    L = lib.lib()
    BC, SEG, CMAX = 128, 100, 1056
    nseg = (T + SEG - 1) // SEG
    announce(f"campp linear1 tiles B={batch} T'={T} c_in={c_in}")
    dense = rng.standard_normal((batch, T, CMAX), dtype=np.float32).astype(np.float16)
    s1 = (rng.random(c_in, dtype=np.float32) + 0.5).astype(np.float32)
    t1 = (rng.standard_normal(c_in, dtype=np.float32) * 0.2).astype(np.float32)
    w = (rng.standard_normal((BC, c_in), dtype=np.float32) / np.sqrt(c_in)).astype(np.float16)
    bias = (rng.standard_normal(BC, dtype=np.float32) * 0.1).astype(np.float32)
    dd, ds1, dt1, dw, db = (lib.DeviceBuffer.from_array(a) for a in (dense, s1, t1, w, bias))
    outs = {}
    for tile in (63, 80, 85, 86, 87, 88):
        d = lib.ConvDesc()
        d.x, d.batch, d.H, d.W, d.IC, d.x_stride = dd.ptr, batch, 1, T, c_in, CMAX
        d.w, d.OC, d.KH, d.KW = dw.ptr, BC, 1, 1
        d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
        d.bias, d.act = db.ptr, lib.ACT_RELU
        d.in_scale, d.in_shift = ds1.ptr, dt1.ptr
        seg = lib.DeviceBuffer.from_array(np.zeros((batch, nseg, BC), dtype=np.float64))
        d.seg_sum, d.seg_len = seg.ptr, SEG
        dh = lib.DeviceBuffer(batch * T * BC * 2)
        d.y, d.y_stride, d.tile = dh.ptr, BC, tile
        if not L.vdk_conv2d_tile_fits_ex(tile, d):
            continue
        lib.check(L.vdk_conv2d_ex(d, None))
        _sync()
        outs[tile] = (dh.to_array(np.uint16, (batch, T, BC)), seg.to_array(np.float64, (batch, nseg, BC)))
    assert 63 in outs and sum(t >= 85 for t in outs) >= 3, sorted(outs)
    for t, (h, sg) in outs.items():
        assert np.array_equal(h, outs[63][0]), f"tile {t} outputs"
        assert np.array_equal(sg, outs[63][1]), f"tile {t} segment sums"
