"""Parity of the ERes2Net GPU path (src/encoder_eres2net.cpp) against the oracle.

Per layer at the 20 s / batch-16 shape (T = 1998 frames): the Res2Net 3x3
convs over channel slices with the Hardtanh(0, 20) clamp (including the
16-channel chunks of layer 1, masked output rows), the strided 1x1 conv1 /
shortcut with residual + clamp, the cross-stage 3x3 stride-2 downsample
stored into its half of the concatenation buffer, the AFF local_att convs
(SiLU, tanh epilogues) and the AFF combine.  End to end: a random-init
ERes2Net base (m_channels 32, q8_0 1x1 weights, 512-d) behind the C ABI,
pooled statistics within 2e-3 relative L2 and embeddings at cosine >= 0.9999.
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
B = 16
N20S = 320000
T20S = 1998


def _assert_close(got, ref, tag):
    ok, ratio, rel = close_report(got, ref, RTOL, ATOL_RMS)
    assert ok and rel <= 2e-3, f"{tag}: max tol ratio {ratio:.3f}, rel-L2 {rel:.2e}"
    return rel


def _w(rng, oc, ic, k):
    return (rng.standard_normal((oc, ic, k, k), dtype=np.float32) * np.sqrt(2.0 / (ic * k * k))).astype(np.float16)


def _clamp(v):
    return np.clip(v, 0.0, 20.0)


def test_chunk_convs_over_slices_with_clamp():
    """Layer-1 shapes: [chunk0 | chunk1 | sp0 | sp1] with w = 16 at 80 x 1998."""
    rng = np.random.default_rng(101)
    H, T, w = 80, T20S, 16
    S = 4 * w
    announce(f"eres chunk convs B={B} H={H} T={T} w={w}")
    s4 = (np.abs(rng.standard_normal((B, H, T, S), dtype=np.float32)) * 3).astype(np.float16)
    d4 = lib.DeviceBuffer.from_array(s4)
    wa = _w(rng, w, w, 3)
    ba = rng.uniform(-0.5, 0.5, w).astype(np.float32)
    # chunk 0 read as [chunk0 | chunk1] with zero weights on chunk1 -> sp0
    wpad = np.zeros((w, 2 * w, 3, 3), dtype=np.float16)
    wpad[:, :w] = wa
    conv_ex(d4.ptr, B, H, T, 2 * w, S, wpad.transpose(0, 2, 3, 1), w, 3, 3, d4.ptr + 2 * w * 2, ys=S, ph=1, pw=1,
            bias=ba, act=lib.ACT_RELU)
    out = d4.to_array(np.float16, (B, H, T, S))
    for c in (0, B - 1):
        ref = O.conv2d_g(s4[c, :, :, :w].astype(np.float32).transpose(2, 0, 1), wa.astype(np.float32), ph=1, pw=1,
                         bias=ba, relu=True)
        rel = _assert_close(out[c, :, :, 2 * w:3 * w].astype(np.float32).transpose(2, 0, 1), ref, f"chunk0 clip {c}")
        announce(f"chunk0 clip {c} rel-L2 {rel:.2e}")
    assert np.array_equal(out[..., :2 * w].view(np.uint16), s4[..., :2 * w].view(np.uint16))
    wb = _w(rng, w, w, 3)
    bb = rng.uniform(-0.5, 0.5, w).astype(np.float32)
    wdup = np.concatenate([wb, wb], axis=1)
    d = lib.ConvDesc()
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(wdup.transpose(0, 2, 3, 1))),
            lib.DeviceBuffer.from_array(bb)]
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride = d4.ptr + w * 2, B, H, T, 2 * w, S
    d.w, d.OC, d.KH, d.KW = keep[0].ptr, w, 3, 3
    d.stride_h = d.stride_w = 1
    d.pad_h = d.pad_w = 1
    d.dil_h = d.dil_w = 1
    d.bias = keep[1].ptr
    d.act, d.clamp_hi = lib.ACT_RELU, 20.0
    d.y, d.y_stride, d.tile = d4.ptr + 3 * w * 2, S, -1
    lib.check(lib.lib().vdk_conv2d_ex(d, None))
    lib.check(lib.lib().vdk_synchronize())
    out2 = d4.to_array(np.float16, (B, H, T, S))
    for c in (0, B - 1):
        xin = out[c, :, :, w:2 * w].astype(np.float32) + out[c, :, :, 2 * w:3 * w].astype(np.float32)
        ref = _clamp(O.conv2d_g(xin.transpose(2, 0, 1), wb.astype(np.float32), ph=1, pw=1, bias=bb))
        rel = _assert_close(out2[c, :, :, 3 * w:].astype(np.float32).transpose(2, 0, 1), ref, f"chunk1 clip {c}")
        announce(f"chunk1 (sum folded) clip {c} rel-L2 {rel:.2e}")


def test_strided_1x1_with_residual_clamp_and_downsample_into_cat():
    rng = np.random.default_rng(102)
    H, T, C = 40, 999, 128
    announce(f"eres strided convs B={B} H={H} T={T}")
    x = (np.abs(rng.standard_normal((B, H, T, C), dtype=np.float32)) * 4).astype(np.float16)
    dx = lib.DeviceBuffer.from_array(x)
    Ho, Wo = 20, 500
    w1 = _w(rng, 2 * C, C, 1)
    b1 = rng.uniform(-0.5, 0.5, 2 * C).astype(np.float32)
    res = (np.abs(rng.standard_normal((B, Ho, Wo, 2 * C), dtype=np.float32)) * 8).astype(np.float16)
    dres = lib.DeviceBuffer.from_array(res)
    y = lib.DeviceBuffer(B * Ho * Wo * 2 * C * 2)
    d = lib.ConvDesc()
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(w1.transpose(0, 2, 3, 1))),
            lib.DeviceBuffer.from_array(b1)]
    d.x, d.batch, d.H, d.W, d.IC = dx.ptr, B, H, T, C
    d.w, d.OC, d.KH, d.KW = keep[0].ptr, 2 * C, 1, 1
    d.stride_h = d.stride_w = 2
    d.dil_h = d.dil_w = 1
    d.bias, d.residual = keep[1].ptr, dres.ptr
    d.act, d.clamp_hi = lib.ACT_RELU, 20.0
    d.y, d.tile = y.ptr, -1
    lib.check(lib.lib().vdk_conv2d_ex(d, None))
    lib.check(lib.lib().vdk_synchronize())
    got = y.to_array(np.float16, (B, Ho, Wo, 2 * C))
    for c in (0, B - 1):
        ref = _clamp(O.conv2d_g(x[c].astype(np.float32).transpose(2, 0, 1), w1.astype(np.float32), sh=2, sw=2,
                                bias=b1, residual=res[c].astype(np.float32).transpose(2, 0, 1)))
        rel = _assert_close(got[c].astype(np.float32).transpose(2, 0, 1), ref, f"1x1 s2 clip {c}")
        announce(f"1x1 s2 + residual + clamp clip {c} rel-L2 {rel:.2e} (clamped {np.mean(ref == 20.0):.3f})")
    # 3x3 stride-2 downsample (no bias) into the second half of a [.. 4C] buffer
    wd = _w(rng, 2 * C, C, 3)
    cat = lib.DeviceBuffer(B * Ho * Wo * 4 * C * 2)
    conv_ex(dx.ptr, B, H, T, C, 0, wd.transpose(0, 2, 3, 1), 2 * C, 3, 3, cat.ptr + 2 * C * 2, ys=4 * C, sh=2, sw=2,
            ph=1, pw=1)
    gc = cat.to_array(np.float16, (B, Ho, Wo, 4 * C))
    for c in (0, B - 1):
        ref = O.conv2d_g(x[c].astype(np.float32).transpose(2, 0, 1), wd.astype(np.float32), sh=2, sw=2, ph=1, pw=1)
        _assert_close(gc[c, :, :, 2 * C:].astype(np.float32).transpose(2, 0, 1), ref, f"downsample clip {c}")


def test_aff_local_att_and_combine():
    rng = np.random.default_rng(103)
    L = lib.lib()
    H, T, C = 20, 500, 64
    announce(f"eres aff B={B} H={H} T={T} C={C}")
    cat = rng.standard_normal((B, H, T, 2 * C), dtype=np.float32).astype(np.float16)   # [ds | x]
    dcat = lib.DeviceBuffer.from_array(cat)
    w1 = _w(rng, C // 4, 2 * C, 1)
    b1 = rng.uniform(-0.5, 0.5, C // 4).astype(np.float32)
    z = lib.DeviceBuffer(B * H * T * (C // 4) * 2)
    conv_ex(dcat.ptr, B, H, T, 2 * C, 0, w1.transpose(0, 2, 3, 1), C // 4, 1, 1, z.ptr, bias=b1, act=lib.ACT_SILU)
    gz = z.to_array(np.float16, (B, H, T, C // 4))
    w2 = _w(rng, C, C // 4, 1)
    b2 = rng.uniform(-0.5, 0.5, C).astype(np.float32)
    z2 = lib.DeviceBuffer(B * H * T * C * 2)
    d = lib.ConvDesc()
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(w2.transpose(0, 2, 3, 1))),
            lib.DeviceBuffer.from_array(b2)]
    d.x, d.batch, d.H, d.W, d.IC = z.ptr, B, H, T, C // 4
    d.w, d.OC, d.KH, d.KW = keep[0].ptr, C, 1, 1
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
    d.bias, d.act, d.tanh_after = keep[1].ptr, lib.ACT_NONE, 1
    d.y, d.tile = z2.ptr, -1
    lib.check(L.vdk_conv2d_ex(d, None))
    lib.check(L.vdk_synchronize())
    gt = z2.to_array(np.float16, (B, H, T, C))
    for c in (0, B - 1):
        pre = O.conv2d_g(cat[c].astype(np.float32).transpose(2, 0, 1), w1.astype(np.float32), bias=b1)
        ref = pre / (1.0 + np.exp(-pre))
        _assert_close(gz[c].astype(np.float32).transpose(2, 0, 1), ref, f"aff silu clip {c}")
        ref2 = np.tanh(O.conv2d_g(gz[c].astype(np.float32).transpose(2, 0, 1), w2.astype(np.float32), bias=b2))
        _assert_close(gt[c].astype(np.float32).transpose(2, 0, 1), ref2, f"aff tanh clip {c}")
    y = lib.DeviceBuffer(B * H * T * C * 2)
    lib.check(L.vdk_aff_combine(z2.ptr, C, 0, dcat.ptr + C * 2, 2 * C, 0, dcat.ptr, 2 * C, 0, B * H * T, C, 0, y.ptr,
                                C, 0, None))
    lib.check(L.vdk_synchronize())
    gy = y.to_array(np.float16, (B, H, T, C)).astype(np.float64)
    xv, dv, tv = cat[..., C:].astype(np.float64), cat[..., :C].astype(np.float64), gt.astype(np.float64)
    want = xv * (1 + tv) + dv * (1 - tv)            # the module's form x*x_att + ds*(2 - x_att)
    assert np.all(np.abs(gy - want) <= 2.0 ** -10 * np.abs(want) + 2e-3)
    # the combine as the second conv's epilogue (aff_x / aff_ds): the same
    # values with tanh's result kept in f32 instead of rounded to f16 first
    y2 = lib.DeviceBuffer(B * H * T * C * 2)
    d.y = y2.ptr
    d.aff_x, d.aff_x_stride, d.aff_ds, d.aff_ds_stride = dcat.ptr + C * 2, 2 * C, dcat.ptr, 2 * C
    lib.check(L.vdk_conv2d_ex(d, None))
    lib.check(L.vdk_synchronize())
    gf = y2.to_array(np.float16, (B, H, T, C)).astype(np.float64)
    for c in (0, B - 1):
        tf = np.tanh(O.conv2d_g(gz[c].astype(np.float32).transpose(2, 0, 1), w2.astype(np.float32), bias=b2,
                                f64=True)).transpose(1, 2, 0)
        wf = xv[c] * (1 + tf) + dv[c] * (1 - tf)
        assert np.all(np.abs(gf[c] - wf) <= 2.0 ** -10 * np.abs(wf) + 2e-3)
    assert np.abs(gf - gy).max() <= 2.0 ** -9 * np.abs(gy).max()


def test_aff_combine_epilogue_split():
    """The AFF combine in the second local_att conv's epilogue on split-f16
    maps (x and ds as [ds | x] slices of one split tensor, as the cross-stage
    AFF reads them) against the f64 module form, to split-f16 accuracy."""
    rng = np.random.default_rng(105)
    Bt, H, T, C, Z = 2, 20, 250, 64, 32
    announce(f"eres aff combine epilogue split B={Bt} H={H} T={T} C={C}")
    cat = rng.standard_normal((Bt, H, T, 2 * C)).astype(np.float32)              # [x | ds]
    z = rng.standard_normal((Bt, H, T, Z)).astype(np.float32)
    w = (rng.standard_normal((C, Z)) * np.sqrt(1.0 / Z)).astype(np.float16).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, C).astype(np.float32)
    dcat = lib.DeviceBuffer.from_array(np.concatenate(_split(cat), axis=3))    # [hi 2C | lo 2C]
    dz = lib.DeviceBuffer.from_array(np.concatenate(_split(z), axis=3))
    wh = w.astype(np.float16)[:, None, None, :]
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(np.concatenate([wh, wh], axis=3))),
            lib.DeviceBuffer.from_array(b)]
    y = lib.DeviceBuffer(Bt * H * T * 2 * C * 2)
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride, d.x_lo = dz.ptr, Bt, H, T, Z, 2 * Z, Z
    d.w, d.OC, d.KH, d.KW = keep[0].ptr, C, 1, 1
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
    d.bias, d.act, d.tanh_after, d.split = keep[1].ptr, lib.ACT_NONE, 1, 2
    d.y, d.y_stride, d.y_lo = y.ptr, 2 * C, C
    d.aff_x, d.aff_x_stride, d.aff_x_lo = dcat.ptr, 4 * C, 2 * C
    d.aff_ds, d.aff_ds_stride, d.aff_ds_lo = dcat.ptr + C * 2, 4 * C, 2 * C
    d.tile = -1
    lib.check(lib.lib().vdk_conv2d_ex(d, None))
    lib.check(lib.lib().vdk_synchronize())
    o = y.to_array(np.float16, (Bt, H, T, 2 * C))
    got = o[..., :C].astype(np.float64) + o[..., C:].astype(np.float64)
    t = np.tanh(z.astype(np.float64) @ w.T.astype(np.float64) + b)
    xv, dv = cat[..., :C].astype(np.float64), cat[..., C:].astype(np.float64)
    want = xv * (1 + t) + dv * (1 - t)
    err = np.abs(got - want).max() / np.abs(want).max()
    announce(f"aff combine epilogue split: max err / max {err:.2e}")
    assert err <= 2e-6


def _split(a):
    """f32 -> (hi, lo) f16 with hi + lo ~ a to ~2^-22."""
    hi = a.astype(np.float16)
    lo = (a - hi.astype(np.float32)).astype(np.float16)
    return hi, lo


@pytest.mark.parametrize("terms,IC,OC,tile", [(3, 64, 64, -1), (2, 64, 64, -1), (2, 32, 16, 27), (3, 32, 32, 28),
                                          (2, 64, 32, 28), (3, 128, 64, 30), (2, 64, 64, 17)])
def test_split_f16_conv_is_f32_accurate(terms, IC, OC, tile):
    """Split-f16 convs (3x3 s1 with clamp, 1x1 s2 with split residual) match the
    f64 brute force to ~1e-6 relative, where plain f16 is ~1e-3.  terms = 2:
    weights that f16 holds exactly, packed [hi | hi] (split = 2), which must
    equal the three-term form with its all-zero lo plane."""
    rng = np.random.default_rng(104 + IC + OC + terms)
    H, T = 20, 250
    announce(f"eres split-f16 convs B={B} H={H} T={T} IC={IC} OC={OC} terms={terms} tile={tile}")
    x = rng.standard_normal((B, H, T, IC)).astype(np.float32) * 3
    xh, xl = _split(x)
    xs = np.concatenate([xh, xl], axis=3)                       # [hi(IC) | lo(IC)] per pixel
    dx = lib.DeviceBuffer.from_array(xs)
    for K, stride in ((3, 1), (1, 2)):
        w = (rng.standard_normal((OC, IC, K, K)) * np.sqrt(2.0 / (IC * K * K))).astype(np.float32)
        if terms == 2:
            w = w.astype(np.float16).astype(np.float32)          # exact in f16: lo = 0
        b = rng.uniform(-0.5, 0.5, OC).astype(np.float32)
        wh, wl = _split(w.transpose(0, 2, 3, 1))
        # [OC][K][K][3*IC], or [OC][K][K][2*IC] for two terms
        wpack = np.concatenate([wh, wh, wl] if terms == 3 else [wh, wh], axis=3)
        Ho, Wo = (H - 1) // stride + 1, (T - 1) // stride + 1
        res = rng.standard_normal((B, Ho, Wo, OC)).astype(np.float32) * 4 if stride == 2 else None
        dres = lib.DeviceBuffer.from_array(np.concatenate(_split(res), axis=3)) if res is not None else None
        y = lib.DeviceBuffer(B * Ho * Wo * 2 * OC * 2)
        d = lib.ConvDesc()
        keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(wpack)), lib.DeviceBuffer.from_array(b)]
        d.x, d.batch, d.H, d.W, d.IC, d.x_stride = dx.ptr, B, H, T, IC, 2 * IC
        d.w, d.OC, d.KH, d.KW = keep[0].ptr, OC, K, K
        d.stride_h = d.stride_w = stride
        d.pad_h = d.pad_w = (K - 1) // 2
        d.dil_h = d.dil_w = 1
        d.bias = keep[1].ptr
        if dres is not None:
            d.residual, d.res_stride, d.res_lo = dres.ptr, 2 * OC, OC
        d.act, d.clamp_hi = lib.ACT_RELU, 20.0
        d.y, d.y_stride = y.ptr, 2 * OC
        d.split, d.x_lo, d.y_lo = (1 if terms == 3 else 2), IC, OC
        d.tile = tile if K == 3 else -1
        lib.check(lib.lib().vdk_conv2d_ex(d, None))
        lib.check(lib.lib().vdk_synchronize())
        got = y.to_array(np.float16, (B, Ho, Wo, 2 * OC)).astype(np.float64)
        if terms == 2:
            assert not np.any(wl)
            keep.append(lib.DeviceBuffer.from_array(np.ascontiguousarray(np.concatenate([wh, wh, wl], axis=3))))
            d.w, d.split = keep[-1].ptr, 1
            y3 = lib.DeviceBuffer(B * Ho * Wo * 2 * OC * 2)
            d.y = y3.ptr
            lib.check(lib.lib().vdk_conv2d_ex(d, None))
            lib.check(lib.lib().vdk_synchronize())
            # the same sums (the skipped products are all zero), up to the sign of zero
            assert np.array_equal(y3.to_array(np.float16, (B, Ho, Wo, 2 * OC)).astype(np.float64), got)
        got = got[..., :OC] + got[..., OC:]
        for c in (0, B - 1):
            ref = O.conv2d_g(x[c].transpose(2, 0, 1), w, sh=stride, sw=stride, ph=(K - 1) // 2, pw=(K - 1) // 2,
                             bias=b, residual=None if res is None else res[c].transpose(2, 0, 1), f64=True)
            ref = np.clip(ref, 0.0, 20.0)
            err = np.abs(got[c].transpose(2, 0, 1) - ref).max() / np.abs(ref).max()
            announce(f"split-f16 K={K} s={stride} clip {c}: max err / max {err:.2e}")
            assert err <= 2e-6


@pytest.mark.parametrize("IC,OC,tile,ref_tile", [(32, 16, 70, 27), (16, 16, 71, None), (32, 32, 72, 27),
                                                 (64, 32, 73, 28), (64, 32, 74, 28), (64, 64, 75, 30)])
def test_split_register_weight_3x3(IC, OC, tile, ref_tile):
    """The split-f16 register-weight 3x3 kernel on channel slices of the Res2Net
    [chunk0 | chunk1 | sp0 | sp1] layout (pixel rows [hi S | lo S]) on a 42 x 300
    map (partial last row tile and 32-column tile), bias + ReLU + clamp.  Against the f64 brute force (<= 2e-6 of the max,
    split-f16's accuracy) and the halo kernel: bit for bit for the 32x32 MFMA
    tiles (same MFMA order), to f32 rounding for the 16x16x32 ones; channels
    outside the output slice keep their bytes."""
    rng = np.random.default_rng(700 + IC + OC + tile)
    Bt, H, T = 2, 42, 300
    S = 256                                      # channels per plane of a pixel row
    cin, cout = 16, 128                          # input / output slice offsets (disjoint slices)
    announce(f"eres split register-weight 3x3 B={Bt} H={H} T={T} IC={IC} OC={OC} tile={tile} ref={ref_tile}")
    x = (rng.standard_normal((Bt, H, T, IC)).astype(np.float32) * 3)
    xh, xl = _split(x)
    buf = rng.standard_normal((Bt, H, T, 2 * S)).astype(np.float16)
    buf[..., cin:cin + IC] = xh
    buf[..., S + cin:S + cin + IC] = xl
    w = (rng.standard_normal((OC, IC, 3, 3)) * np.sqrt(2.0 / (IC * 9))).astype(np.float16).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, OC).astype(np.float32)
    wh = w.transpose(0, 2, 3, 1).astype(np.float16)
    wpack = np.ascontiguousarray(np.concatenate([wh, wh], axis=3))
    wch = np.zeros_like(wpack)
    lib.lib().vdk_conv_pack_chunked(wpack.ctypes.data, OC, 3, 3, 2 * IC, wch.ctypes.data)
    keep = [lib.DeviceBuffer.from_array(wpack), lib.DeviceBuffer.from_array(wch), lib.DeviceBuffer.from_array(b)]

    def run(t, chunked):
        d4 = lib.DeviceBuffer.from_array(buf)
        d = lib.ConvDesc()
        d.x, d.batch, d.H, d.W, d.IC, d.x_stride = d4.ptr + cin * 2, Bt, H, T, IC, 2 * S
        d.w, d.OC, d.KH, d.KW = keep[0].ptr, OC, 3, 3
        d.w_chunked = keep[1].ptr if chunked else None
        d.stride_h = d.stride_w = 1
        d.pad_h = d.pad_w = 1
        d.dil_h = d.dil_w = 1
        d.bias = keep[2].ptr
        d.act, d.clamp_hi = lib.ACT_RELU, 20.0
        d.y, d.y_stride = d4.ptr + cout * 2, 2 * S
        d.split, d.x_lo, d.y_lo = 2, S, S
        d.tile = t
        lib.check(lib.lib().vdk_conv2d_ex(d, None))
        lib.check(lib.lib().vdk_synchronize())
        return d4.to_array(np.float16, (Bt, H, T, 2 * S))

    out = run(tile, True)
    assert np.array_equal(run(tile, False), out)             # the weight copy changes nothing
    keepmask = np.ones(2 * S, bool)
    keepmask[cout:cout + OC] = keepmask[S + cout:S + cout + OC] = False
    assert np.array_equal(out[..., keepmask], buf[..., keepmask])
    got = out[..., cout:cout + OC].astype(np.float64) + out[..., S + cout:S + cout + OC].astype(np.float64)
    if ref_tile is not None:
        ref = run(ref_tile, False)
        rsum = ref[..., cout:cout + OC].astype(np.float64) + ref[..., S + cout:S + cout + OC].astype(np.float64)
        if tile in (72, 74, 75):
            assert np.array_equal(out, ref)
        else:
            assert np.abs(got - rsum).max() <= 1e-6 * np.abs(rsum).max()
    for c in (0, Bt - 1):
        want = O.conv2d_g(x[c].transpose(2, 0, 1), w, sh=1, sw=1, ph=1, pw=1, bias=b, f64=True)
        want = np.clip(want, 0.0, 20.0)
        err = np.abs(got[c].transpose(2, 0, 1) - want).max() / np.abs(want).max()
        announce(f"split register-weight 3x3 clip {c}: max err / max {err:.2e}")
        assert err <= 2e-6


def _grouped(vals, groups, g=16):
    """f32 [.., g * n] -> f16 rows of `groups` g-channel groups [hi g | lo g]."""
    hi, lo = _split(vals)
    out = np.zeros(vals.shape[:-1] + (2 * g * groups,), np.float16)
    for k in range(vals.shape[-1] // g):
        out[..., 2 * g * k:2 * g * k + g] = hi[..., g * k:g * k + g]
        out[..., 2 * g * k + g:2 * g * (k + 1)] = lo[..., g * k:g * k + g]
    return out


def _ungroup(rows, g0, n, g=16):
    """The split values of groups g0 .. g0+n of grouped rows, as f64."""
    parts = [rows[..., 2 * g * k:2 * g * k + g].astype(np.float64) +
             rows[..., 2 * g * k + g:2 * g * (k + 1)].astype(np.float64) for k in range(g0, g0 + n)]
    return np.concatenate(parts, axis=-1)


@pytest.mark.parametrize("case,g", [("3x3_32_16", 16), ("3x3_16_16", 16), ("1x1_32_64_res", 16), ("1x1_64_32", 16),
                                    ("3x3_32_32", 32), ("3x3_64_32", 32), ("1x1_64_128_res", 32),
                                    ("1x1_128_64", 32)])
def test_split_grouped_layout(case, g):
    """Split-f16 tensors stored as g-channel groups [hi g | lo g] (group stride
    2g, lo offset g: layer 1 / 2's Res2Net chunks as whole 64-byte pieces /
    128-byte lines): the 3x3 group convs on the split register-weight kernel
    and the LDS-DMA kernel, and the 1x1 convs around them (grouped input with a
    contiguous split residual; contiguous input into grouped output) on the
    LDS-DMA kernel, against the f64 brute force; bytes outside the output
    groups keep their values."""
    rng = np.random.default_rng(880 + len(case) + g)
    Bt, H, T, G = 2, 42, 300, 4                           # 4 groups per pixel row
    K, IC, OC = {"3x3_32_16": (3, 32, 16), "3x3_16_16": (3, 16, 16), "1x1_32_64_res": (1, 32, 64),
                 "1x1_64_32": (1, 64, 32), "3x3_32_32": (3, 32, 32), "3x3_64_32": (3, 64, 32),
                 "1x1_64_128_res": (1, 64, 128), "1x1_128_64": (1, 128, 64)}[case]
    announce(f"eres grouped split layout {case} group {g} B={Bt} H={H} T={T}")
    w = (rng.standard_normal((OC, IC, K, K)) * np.sqrt(2.0 / (IC * K * K))).astype(np.float16).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, OC).astype(np.float32)
    wh = w.transpose(0, 2, 3, 1).astype(np.float16)
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(np.concatenate([wh, wh], axis=3))),
            lib.DeviceBuffer.from_array(bias)]
    x = rng.standard_normal((Bt, H, T, IC)).astype(np.float32) * 3
    res = None
    d = lib.ConvDesc()
    d.batch, d.H, d.W, d.IC = Bt, H, T, IC
    d.w, d.OC, d.KH, d.KW = keep[0].ptr, OC, K, K
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
    d.pad_h = d.pad_w = K // 2
    d.bias, d.act, d.clamp_hi, d.split = keep[1].ptr, lib.ACT_RELU, 20.0, 2
    res_case = case.endswith("_res")
    if K == 3 or res_case:                                 # grouped input from group 1, grouped / contiguous out
        rows = rng.standard_normal((Bt, H, T, 2 * g * G)).astype(np.float16)
        rows[..., 2 * g:2 * g + 2 * IC] = _grouped(x, IC // g, g)
        din = lib.DeviceBuffer.from_array(rows)
        d.x, d.x_stride, d.x_lo, d.x_group_stride, d.x_group = din.ptr + 2 * g * 2, 2 * g * G, g, 2 * g, g
    else:
        din = lib.DeviceBuffer.from_array(np.concatenate(_split(x), axis=3))
        d.x, d.x_stride, d.x_lo = din.ptr, 2 * IC, IC
    if res_case:                                           # contiguous split output and residual
        res = rng.standard_normal((Bt, H, T, OC)).astype(np.float32) * 2
        dres = lib.DeviceBuffer.from_array(np.concatenate(_split(res), axis=3))
        d.residual, d.res_stride, d.res_lo = dres.ptr, 2 * OC, OC
        yrows = np.zeros((Bt, H, T, 2 * OC), np.float16)
        dy = lib.DeviceBuffer.from_array(yrows)
        d.y, d.y_stride, d.y_lo = dy.ptr, 2 * OC, OC
    else:                                                  # grouped output into group 3 (K = 3) or 1
        g0 = 3 if K == 3 else 1
        yrows = rows.copy() if K == 3 else rng.standard_normal((Bt, H, T, 2 * g * G)).astype(np.float16)
        dy = din if K == 3 else lib.DeviceBuffer.from_array(yrows)
        d.y, d.y_stride, d.y_lo, d.y_group_stride, d.y_group = dy.ptr + 2 * g * g0 * 2, 2 * g * G, g, 2 * g, g
    tiles = {"3x3_32_16": [70, 14], "3x3_16_16": [71], "1x1_32_64_res": [-1, 16], "1x1_64_32": [-1, 14],
             "3x3_32_32": [72, 14], "3x3_64_32": [73, 74, 14], "1x1_64_128_res": [-1, 39],
             "1x1_128_64": [-1, 15]}[case]
    if K == 1:   # the GEMM kernel's tiles where they fit: the LDS-DMA tile's bits
        tiles += [t for t in (81, 82, 83, 84) if lib.lib().vdk_conv2d_tile_fits_ex(t, d)]
    outs, raw = [], {}
    for t in tiles:
        if K == 3:
            dy.copy_from(rows)
        d.tile = t
        lib.check(lib.lib().vdk_conv2d_ex(d, None))
        lib.check(lib.lib().vdk_synchronize())
        if res_case:
            o = dy.to_array(np.float16, (Bt, H, T, 2 * OC))
            got = o[..., :OC].astype(np.float64) + o[..., OC:].astype(np.float64)
        else:
            o = dy.to_array(np.float16, (Bt, H, T, 2 * g * G))
        raw[t] = o.copy()
        if not res_case:
            got = _ungroup(o, g0, OC // g, g)
            mask = np.ones(2 * g * G, bool)
            mask[2 * g * g0:2 * g * (g0 + OC // g)] = False
            assert np.array_equal(o[..., mask], yrows[..., mask])
        outs.append(got)
        for c in (0, Bt - 1):
            want = O.conv2d_g(x[c].transpose(2, 0, 1), w, ph=K // 2, pw=K // 2, bias=bias,
                              residual=None if res is None else res[c].transpose(2, 0, 1), f64=True)
            want = np.clip(want, 0.0, 20.0)
            err = np.abs(got[c].transpose(2, 0, 1) - want).max() / np.abs(want).max()
            announce(f"grouped {case} tile {t} clip {c}: max err / max {err:.2e}")
            assert err <= 2e-6
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() <= 1e-6 * np.abs(outs[0]).max()
    if K == 1:
        gemm = [t for t in raw if t >= 81]
        assert gemm, "no GEMM tile fits"
        for t in gemm:
            assert np.array_equal(raw[t], raw[tiles[1]]), f"GEMM tile {t} vs LDS-DMA tile {tiles[1]}"


@pytest.mark.parametrize("IC,OC,res", [(64, 128, True), (128, 64, False), (256, 512, True)])
def test_gemm_ws_split_three_terms_bitwise(IC, OC, res):
    """Split-f16 1x1 convs with q8_0-style weights f16 does not hold (three
    MFMA terms: x_hi.w_hi + x_lo.w_hi + x_hi.w_lo, K over [hi | lo | hi]) on
    the GEMM kernel's tiles: the LDS-DMA tile's bits (same K order), with a
    split residual, ReLU and the clamp."""
    rng = np.random.default_rng(IC + OC)
    Bt, H, T = 2, 20, 333
    announce(f"gemm split 3-term 1x1 B={Bt} H={H} T={T} {IC}->{OC} res={res}")
    x = rng.standard_normal((Bt, H, T, IC)).astype(np.float32) * 3
    w = (rng.standard_normal((OC, IC)) * np.sqrt(2.0 / IC)).astype(np.float32)
    wh, wl = _split(w)
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(np.concatenate([wh, wh, wl], axis=1))),
            lib.DeviceBuffer.from_array(rng.uniform(-0.5, 0.5, OC).astype(np.float32)),
            lib.DeviceBuffer.from_array(np.concatenate(_split(x), axis=3))]
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride, d.x_lo = keep[2].ptr, Bt, H, T, IC, 2 * IC, IC
    d.w, d.OC, d.KH, d.KW = keep[0].ptr, OC, 1, 1
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
    d.bias, d.act, d.clamp_hi, d.split = keep[1].ptr, lib.ACT_RELU, 20.0, 1
    if res:
        keep.append(lib.DeviceBuffer.from_array(np.concatenate(_split(
            rng.standard_normal((Bt, H, T, OC)).astype(np.float32)), axis=3)))
        d.residual, d.res_stride, d.res_lo = keep[-1].ptr, 2 * OC, OC
    dy = lib.DeviceBuffer(Bt * H * T * 2 * OC * 2)
    d.y, d.y_stride, d.y_lo = dy.ptr, 2 * OC, OC
    outs = {}
    for t in (39, 15, 81, 82, 83, 84):
        d.tile = t
        if not lib.lib().vdk_conv2d_tile_fits_ex(t, d):
            continue
        lib.check(lib.lib().vdk_conv2d_ex(d, None))
        lib.check(lib.lib().vdk_synchronize())
        outs[t] = dy.to_array(np.uint16, (Bt, H, T, 2 * OC))
    ref = 39 if 39 in outs else 15
    assert ref in outs and sum(t >= 81 for t in outs) >= 2, sorted(outs)
    for t, o in outs.items():
        assert np.array_equal(o, outs[ref]), f"tile {t}"


# ------------------------------------------------------------------ end to end

@pytest.fixture(scope="module")
def eres():
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "eres2net_q8_0.gguf")
    synth.write_eres2net(path, seed=9)
    g = gguf.GGUFFile(path)
    assert sum(1 for v in g.tensors.values() if v[0] == gguf.GGML_Q8_0) > 40
    ctx = lib.Context(path)
    net = O.OracleEres2net(g)
    yield path, ctx, net
    ctx.close()


def test_eres2net_batch16_matches_oracle(eres):
    path, ctx, net = eres
    pcm = synth.clips(9090, B, N20S)
    announce("e2e eres2net B=16 20s capture")
    cap = ctx.capture(pcm)
    assert cap["pooled"].shape[1] == 2 * 512 * 10
    for c in (0, B - 1):
        feats = O.fbank(pcm[c])
        assert np.abs(cap["feats"][c] - feats).max() <= 1e-4
        emb, caps = net.forward(feats, capture=True)
        rel = np.linalg.norm(cap["pooled"][c] - caps["pooled"]) / np.linalg.norm(caps["pooled"])
        assert rel <= 2e-3, f"pooled rel-L2 {rel:.2e} clip {c}"
        assert cosine(cap["pre_norm"][c], caps["pre_norm"]) >= 0.9999
        cs = cosine(cap["emb"][c], emb)
        announce(f"eres2net clip {c}: cosine {cs:.7f} pooled rel {rel:.2e}")
        assert cs >= 0.9999
    one = ctx.embed_batch(pcm[B - 1:B])
    assert np.array_equal(one[0], cap["emb"][B - 1])
    check_every_clip(ctx, net, pcm, cap["emb"], "eres2net B=16", invariance=(0, 7, 14))


@pytest.mark.parametrize("n", [400, 4000, 48000])
def test_eres2net_embed_pcm_lengths(eres, n):
    path, ctx, net = eres
    announce(f"e2e eres2net B=1 n={n}")
    pcm = synth.clip(300 + n, n)
    got = ctx.embed_pcm(pcm)
    ref = net.forward(O.fbank(pcm))
    assert got.shape == (512,)
    assert cosine(got, ref) >= 0.9999


def test_eres2net_verify_matches_oracle(eres):
    path, ctx, net = eres
    announce("e2e eres2net verify")
    a = synth.clip(21, 48000)
    b = synth.clip(22, 40000)
    d_gpu, _ = ctx.verify_pcm(a, b, 0.5)
    ea, eb = net.forward(O.fbank(a)), net.forward(O.fbank(b))
    d_ref = 1.0 - float(np.dot(ea.astype(np.float64), eb.astype(np.float64)))
    assert abs(d_gpu - d_ref) <= 2e-3
    for thr in (d_ref - 5e-3, d_ref + 5e-3):
        assert ctx.verify_pcm(a, b, thr)[1] == (d_ref <= thr)


@pytest.mark.parametrize("Bt,H,T", [(2, 42, 301), (B, 80, T20S)])
def test_res2_pair_equals_two_convs(Bt, H, T):
    """The fused Res2Net pair (layer 1's conv_a -> conv_b with sp0 kept on chip)
    on grouped [hi 16 | lo 16] rows equals the two one-conv launches (conv_a on
    c0, conv_b on [c1 | sp0] with its weights on both halves) bit for bit, at
    partial row / column tiles and at the 80 x 1998 layer-1 map; sp0 and sp1
    against the f64 brute force on the small map."""
    rng = np.random.default_rng(990 + H)
    announce(f"eres res2 pair B={Bt} H={H} T={T}")
    c = rng.standard_normal((Bt, H, T, 32)).astype(np.float32) * 3     # [c0 | c1]
    rows = rng.standard_normal((Bt, H, T, 128)).astype(np.float16)
    rows[..., :64] = _grouped(c, 2)
    wa = (rng.standard_normal((16, 16, 3, 3)) * np.sqrt(2.0 / 144)).astype(np.float16)
    wb = (rng.standard_normal((16, 16, 3, 3)) * np.sqrt(2.0 / 144)).astype(np.float16)
    ba = rng.uniform(-0.5, 0.5, 16).astype(np.float32)
    bb = rng.uniform(-0.5, 0.5, 16).astype(np.float32)
    wah, wbh = wa.transpose(0, 2, 3, 1), wb.transpose(0, 2, 3, 1)      # [16][3][3][16]
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(wah)), lib.DeviceBuffer.from_array(ba),
            lib.DeviceBuffer.from_array(np.ascontiguousarray(wbh)), lib.DeviceBuffer.from_array(bb),
            lib.DeviceBuffer.from_array(np.ascontiguousarray(np.concatenate([wah, wah], axis=3))),
            lib.DeviceBuffer.from_array(np.ascontiguousarray(np.concatenate([wbh, wbh, wbh, wbh], axis=3)))]
    L = lib.lib()
    # two one-conv launches on the grouped rows: sp0 -> group 2, sp1 -> group 3
    d2 = lib.DeviceBuffer.from_array(rows)
    for xg, IC, w, bias, yg, tile in ((0, 16, keep[4], keep[1], 2, 71), (1, 32, keep[5], keep[3], 3, 70)):
        d = lib.ConvDesc()
        d.x, d.batch, d.H, d.W, d.IC, d.x_stride = d2.ptr + 32 * xg * 2, Bt, H, T, IC, 128
        d.x_lo, d.x_group_stride = 16, 32
        d.w, d.OC, d.KH, d.KW = w.ptr, 16, 3, 3
        d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
        d.pad_h = d.pad_w = 1
        d.bias, d.act, d.clamp_hi = bias.ptr, lib.ACT_RELU, 20.0
        d.y, d.y_stride, d.y_lo, d.y_group_stride = d2.ptr + 32 * yg * 2, 128, 16, 32
        d.split, d.tile = 2, tile
        lib.check(L.vdk_conv2d_ex(d, None))
    d1 = lib.DeviceBuffer.from_array(rows)
    lib.check(L.vdk_res2_pair3x3(d1.ptr, 128, d1.ptr + 64 * 2, 128, Bt, H, T, keep[0].ptr, keep[1].ptr, keep[2].ptr,
                                 keep[3].ptr, 20.0, None))
    lib.check(L.vdk_synchronize())
    two = d2.to_array(np.float16, (Bt, H, T, 128))
    one = d1.to_array(np.float16, (Bt, H, T, 128))
    assert np.array_equal(one[..., :64], rows[..., :64])
    assert np.array_equal(one, two)
    if Bt == B:
        return
    sp = _ungroup(one, 2, 2)
    for ci in (0, Bt - 1):
        s0 = np.clip(O.conv2d_g(c[ci, :, :, :16].transpose(2, 0, 1), wa.astype(np.float32), ph=1, pw=1, bias=ba,
                                f64=True), 0.0, 20.0)
        err0 = np.abs(sp[ci, :, :, :16].transpose(2, 0, 1) - s0).max() / np.abs(s0).max()
        xin = sp[ci, :, :, :16] + c[ci, :, :, 16:].astype(np.float64)
        s1 = np.clip(O.conv2d_g(xin.transpose(2, 0, 1).astype(np.float32), wb.astype(np.float32), ph=1, pw=1,
                                bias=bb, f64=True), 0.0, 20.0)
        err1 = np.abs(sp[ci, :, :, 16:].transpose(2, 0, 1) - s1).max() / np.abs(s1).max()
        announce(f"res2 pair clip {ci}: sp0 err {err0:.2e}, sp1 err {err1:.2e}")
        assert err0 <= 2e-6 and err1 <= 4e-6


@pytest.mark.parametrize("Bt,H,T,terms,tile", [(2, 42, 301, 3, 16), (2, 42, 301, 2, -1), (B, 80, T20S, 3, -1)])
def test_res2_pair_conv3_equals_pair_then_conv3(Bt, H, T, terms, tile):
    """The Res2Net pair with the block's conv3 fused (sp0, sp1 kept on chip)
    equals the pair followed by the LDS-DMA conv3 over [sp0 | sp1] (split-f16
    weights of two or three terms, bias, split residual, ReLU, clamp) bit for
    bit, at partial tiles and at the 80 x 1998 layer-1 map."""
    rng = np.random.default_rng(1990 + H + terms)
    announce(f"eres res2 pair + conv3 B={Bt} H={H} T={T} terms={terms} tile={tile}")
    c = rng.standard_normal((Bt, H, T, 32)).astype(np.float32) * 3
    rows = np.zeros((Bt, H, T, 128), np.float16)
    rows[..., :64] = _grouped(c, 2)
    res = rng.standard_normal((Bt, H, T, 64)).astype(np.float32) * 2
    wa = (rng.standard_normal((16, 16, 3, 3)) * np.sqrt(2.0 / 144)).astype(np.float16)
    wb = (rng.standard_normal((16, 16, 3, 3)) * np.sqrt(2.0 / 144)).astype(np.float16)
    ba = rng.uniform(-0.5, 0.5, 16).astype(np.float32)
    bb = rng.uniform(-0.5, 0.5, 16).astype(np.float32)
    w3 = (rng.standard_normal((64, 32)) * np.sqrt(2.0 / 32)).astype(np.float32)
    if terms == 2:
        w3 = w3.astype(np.float16).astype(np.float32)
    w3h, w3l = _split(w3)
    w3p = np.ascontiguousarray(np.concatenate([w3h, w3h, w3l] if terms == 3 else [w3h, w3h], axis=1))
    b3 = rng.uniform(-0.5, 0.5, 64).astype(np.float32)
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(wa.transpose(0, 2, 3, 1))), lib.DeviceBuffer.from_array(ba),
            lib.DeviceBuffer.from_array(np.ascontiguousarray(wb.transpose(0, 2, 3, 1))), lib.DeviceBuffer.from_array(bb),
            lib.DeviceBuffer.from_array(w3p), lib.DeviceBuffer.from_array(b3),
            lib.DeviceBuffer.from_array(np.concatenate(_split(res), axis=3))]
    L = lib.lib()
    # the pair into groups 2, 3, then conv3 from them
    d1 = lib.DeviceBuffer.from_array(rows)
    lib.check(L.vdk_res2_pair3x3(d1.ptr, 128, d1.ptr + 64 * 2, 128, Bt, H, T, keep[0].ptr, keep[1].ptr, keep[2].ptr,
                                 keep[3].ptr, 20.0, None))
    y1 = lib.DeviceBuffer(Bt * H * T * 128 * 2)
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride = d1.ptr + 64 * 2, Bt, H, T, 32, 128
    d.x_lo, d.x_group_stride = 16, 32
    d.w, d.OC, d.KH, d.KW = keep[4].ptr, 64, 1, 1
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
    d.bias, d.act, d.clamp_hi = keep[5].ptr, lib.ACT_RELU, 20.0
    d.residual, d.res_stride, d.res_lo = keep[6].ptr, 128, 64
    d.y, d.y_stride, d.y_lo = y1.ptr, 128, 64
    d.split, d.tile = (1 if terms == 3 else 2), tile
    lib.check(L.vdk_conv2d_ex(d, None))
    # fused
    d2 = lib.DeviceBuffer.from_array(rows)
    y2 = lib.DeviceBuffer(Bt * H * T * 128 * 2)
    lib.check(L.vdk_res2_pair3x3_conv3(d2.ptr, 128, Bt, H, T, keep[0].ptr, keep[1].ptr, keep[2].ptr, keep[3].ptr,
                                       keep[4].ptr, keep[5].ptr, terms, keep[6].ptr, 128, 64, y2.ptr, 128, 64, 20.0,
                                       None))
    lib.check(L.vdk_synchronize())
    a = y1.to_array(np.float16, (Bt, H, T, 128))
    b = y2.to_array(np.float16, (Bt, H, T, 128))
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    assert np.array_equal(d2.to_array(np.float16, (Bt, H, T, 128)).view(np.uint16), rows.view(np.uint16))


@pytest.mark.parametrize("Bt,H,T,ic1,resx,t1,terms", [(2, 42, 301, 64, True, 3, 2), (2, 42, 301, 64, False, 2, 3),
                                                      (2, 42, 301, 32, False, 2, 2), (1, 3, 5, 64, True, 2, 3),
                                                      (3, 7, 61, 32, False, 3, 3), (B, 80, T20S, 64, True, 3, 3),
                                                      (B, 80, T20S, 32, False, 3, 3)])
def test_res2_bottleneck_equals_conv1_then_pair_conv3(Bt, H, T, ic1, resx, t1, terms):
    """The whole layer-1 block in one launch (conv1 over an LDS x halo into the
    [c0 | c1] halo, the pair, conv3 + residual) equals vdk_conv2d_ex's split
    conv1 into grouped [c0 | c1] rows followed by vdk_res2_pair3x3_conv3, bit
    for bit: x as the residual (64 channels) or a separate map, two- and
    three-term conv1 / conv3 weights, maps smaller than one tile, partial
    tiles and the 80 x 1998 layer-1 map at batch 16."""
    rng = np.random.default_rng(2990 + H + ic1 + terms + 10 * t1)
    announce(f"eres bottleneck B={Bt} H={H} T={T} ic1={ic1} resx={resx} t1={t1} terms={terms}")
    xv = rng.standard_normal((Bt, H, T, ic1)).astype(np.float32) * 2
    xh, xl = _split(xv)
    xrows = np.ascontiguousarray(np.concatenate([xh, xl], axis=3))            # [hi ic1 | lo ic1]
    w1 = (rng.standard_normal((32, ic1)) * np.sqrt(2.0 / ic1)).astype(np.float32)
    if t1 == 2:
        w1 = w1.astype(np.float16).astype(np.float32)
    w1h, w1l = _split(w1)
    w1p = np.ascontiguousarray(np.concatenate([w1h, w1h, w1l] if t1 == 3 else [w1h, w1h], axis=1))
    b1 = rng.uniform(-0.5, 0.5, 32).astype(np.float32)
    wa = (rng.standard_normal((16, 16, 3, 3)) * np.sqrt(2.0 / 144)).astype(np.float16)
    wb = (rng.standard_normal((16, 16, 3, 3)) * np.sqrt(2.0 / 144)).astype(np.float16)
    ba = rng.uniform(-0.5, 0.5, 16).astype(np.float32)
    bb = rng.uniform(-0.5, 0.5, 16).astype(np.float32)
    w3 = (rng.standard_normal((64, 32)) * np.sqrt(2.0 / 32)).astype(np.float32)
    if terms == 2:
        w3 = w3.astype(np.float16).astype(np.float32)
    w3h, w3l = _split(w3)
    w3p = np.ascontiguousarray(np.concatenate([w3h, w3h, w3l] if terms == 3 else [w3h, w3h], axis=1))
    b3 = rng.uniform(-0.5, 0.5, 64).astype(np.float32)
    keep = [lib.DeviceBuffer.from_array(w1p), lib.DeviceBuffer.from_array(b1),
            lib.DeviceBuffer.from_array(np.ascontiguousarray(wa.transpose(0, 2, 3, 1))), lib.DeviceBuffer.from_array(ba),
            lib.DeviceBuffer.from_array(np.ascontiguousarray(wb.transpose(0, 2, 3, 1))), lib.DeviceBuffer.from_array(bb),
            lib.DeviceBuffer.from_array(w3p), lib.DeviceBuffer.from_array(b3)]
    d_x = lib.DeviceBuffer.from_array(xrows)
    if resx:
        d_res, rs, rlo = d_x, 128, 64
    else:
        d_res = lib.DeviceBuffer.from_array(np.concatenate(_split(rng.standard_normal((Bt, H, T, 64)).astype(
            np.float32) * 2), axis=3))
        rs, rlo = 128, 64
    L = lib.lib()
    # conv1 into grouped [c0 | c1] rows, then the pair with conv3
    rows = lib.DeviceBuffer(Bt * H * T * 128 * 2)
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride, d.x_lo = d_x.ptr, Bt, H, T, ic1, 2 * ic1, ic1
    d.w, d.OC, d.KH, d.KW = keep[0].ptr, 32, 1, 1
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
    d.bias, d.act, d.clamp_hi = keep[1].ptr, lib.ACT_RELU, 20.0
    d.y, d.y_stride, d.y_lo, d.y_group_stride = rows.ptr, 128, 16, 32
    d.split, d.tile = (2 if t1 == 2 else 1), -1
    lib.check(L.vdk_conv2d_ex(d, None))
    y1 = lib.DeviceBuffer(Bt * H * T * 128 * 2)
    lib.check(L.vdk_res2_pair3x3_conv3(rows.ptr, 128, Bt, H, T, keep[2].ptr, keep[3].ptr, keep[4].ptr, keep[5].ptr,
                                       keep[6].ptr, keep[7].ptr, terms, d_res.ptr, rs, rlo, y1.ptr, 128, 64, 20.0,
                                       None))
    y2 = lib.DeviceBuffer(Bt * H * T * 128 * 2)
    lib.check(L.vdk_res2_bottleneck(d_x.ptr, 2 * ic1, ic1, ic1, Bt, H, T, keep[0].ptr, t1, keep[1].ptr, keep[2].ptr,
                                    keep[3].ptr, keep[4].ptr, keep[5].ptr, keep[6].ptr, keep[7].ptr, terms,
                                    None if resx else d_res.ptr, rs, rlo, y2.ptr, 128, 64, 20.0, None))
    lib.check(L.vdk_synchronize())
    a = y1.to_array(np.uint16, (Bt, H, T, 128))
    b = y2.to_array(np.uint16, (Bt, H, T, 128))
    assert np.array_equal(a, b)
    assert np.array_equal(d_x.to_array(np.float16, xrows.shape).view(np.uint16), xrows.view(np.uint16))
