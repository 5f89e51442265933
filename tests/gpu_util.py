"""Helpers shared by the GPU parity tests: run single vdk kernels through the
C ABI on host arrays, and the parity metrics (the reference's atol + rtol*|ref|
form of tests/parity.hpp:44-70, cosine)."""
import ctypes as C
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from vdamd import lib


def device_ok():
    """Whether a HIP device is visible.  A library that fails to load raises
    here (every GPU test then errors) instead of reading as "no device"."""
    return lib.lib().vdk_device_count() > 0


def announce(msg):
    print(f"[gpu-case] {msg}", flush=True)


def conv_gpu(x_nhwc, w_oihw, bias=None, residual=None, stride=1, pad=1, relu=False, tile=-1):
    """x [B,H,W,IC] f16, w [OC,IC,KH,KW] (f16 values) -> y [B,Ho,Wo,OC] f16 via vdk_conv2d_nhwc."""
    L = lib.lib()
    x = np.ascontiguousarray(x_nhwc, dtype=np.float16)
    B, H, W, IC = x.shape
    OC, IC2, KH, KW = w_oihw.shape
    assert IC == IC2
    Ho, Wo = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    wp = np.ascontiguousarray(np.asarray(w_oihw, dtype=np.float16).transpose(0, 2, 3, 1))
    dx = lib.DeviceBuffer.from_array(x)
    dw = lib.DeviceBuffer.from_array(wp)
    db = lib.DeviceBuffer.from_array(np.asarray(bias, dtype=np.float32)) if bias is not None else None
    dr = None
    if residual is not None:
        r = np.ascontiguousarray(residual, dtype=np.float16)
        assert r.shape == (B, Ho, Wo, OC)
        dr = lib.DeviceBuffer.from_array(r)
    dy = lib.DeviceBuffer(B * Ho * Wo * OC * 2)
    rc = L.vdk_conv2d_nhwc_tile(dx.ptr, B, H, W, IC, dw.ptr, OC, KH, KW, stride, pad,
                                db.ptr if db else None, dr.ptr if dr else None, int(relu), dy.ptr, None, tile)
    lib.check(rc)
    lib.check(L.vdk_synchronize())
    return dy.to_array(np.float16, (B, Ho, Wo, OC))


def tile_fits(tile, B, H, W, IC, OC, K, stride, pad, residual=True, relu=True):
    """Whether conv tile `tile` takes this exact shape (map width included,
    which the width-limited band kernels need), via vdk_conv2d_tile_fits_ex."""
    d = lib.ConvDesc()
    d.batch, d.H, d.W, d.IC, d.OC, d.KH, d.KW = B, H, W, IC, OC, K, K
    d.stride_h = d.stride_w = stride
    d.pad_h = d.pad_w = pad
    d.residual = 16 if residual else None   # only its presence matters
    d.act = lib.ACT_RELU if relu else lib.ACT_NONE
    return bool(lib.lib().vdk_conv2d_tile_fits_ex(tile, d))


def close_report(got, ref, rtol, atol_rel_rms):
    """Elementwise |got-ref| <= atol + rtol*|ref| with atol = atol_rel_rms * rms(ref).
    Returns (ok, max_excess_ratio, rel_l2)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref ** 2)) if ref.size else 0.0
    tol = atol_rel_rms * rms + rtol * np.abs(ref)
    d = np.abs(got - ref)
    ratio = float(np.max(d / np.maximum(tol, 1e-30))) if ref.size else 0.0
    rel_l2 = float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))
    return ratio <= 1.0, ratio, rel_l2


def cosine(a, b):
    a = np.asarray(a, dtype=np.float64).reshape(-1)
    b = np.asarray(b, dtype=np.float64).reshape(-1)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def conv_ex(x_ptr, batch, H, W, IC, xs, w_khkwic, OC, KH, KW, y_ptr, ys=0, sh=1, sw=1, ph=0, pw=0, dh=1, dw=1,
            bias=None, residual=None, act=lib.ACT_NONE, gate=None, gate_seg=0, gate_nseg=0, y_time_major=0,
            clamp_hi=0.0, tanh_after=0):
    """One vdk_conv2d_ex launch; w_khkwic is the packed f16 [OC][KH][KW][IC] weight."""
    keep = [lib.DeviceBuffer.from_array(np.ascontiguousarray(w_khkwic, dtype=np.float16))]
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride = x_ptr, batch, H, W, IC, xs
    d.w, d.OC, d.KH, d.KW = keep[0].ptr, OC, KH, KW
    d.stride_h, d.stride_w, d.pad_h, d.pad_w, d.dil_h, d.dil_w = sh, sw, ph, pw, dh, dw
    if bias is not None:
        keep.append(lib.DeviceBuffer.from_array(bias.astype(np.float32)))
        d.bias = keep[-1].ptr
    if residual is not None:
        d.residual = residual
    if gate is not None:
        keep.append(lib.DeviceBuffer.from_array(gate.astype(np.float32)))
        d.gate, d.gate_seg, d.gate_nseg = keep[-1].ptr, gate_seg, gate_nseg
    d.act, d.clamp_hi, d.tanh_after = act, clamp_hi, tanh_after
    d.y, d.y_stride, d.y_time_major = y_ptr, ys, y_time_major
    d.tile = -1
    lib.check(lib.lib().vdk_conv2d_ex(d, None))
    lib.check(lib.lib().vdk_synchronize())


def oracle_embed_all(net, pcm, threads=8):
    """The oracle's embedding of every clip of a batch, clip-parallel on up to
    `threads` threads (the C oracle runs outside the GIL)."""
    import pyoracle as O
    n = max(1, min(threads, os.cpu_count() or 1))
    with ThreadPoolExecutor(n) as ex:
        return np.stack(list(ex.map(lambda k: net.forward(O.fbank(pcm[k])), range(len(pcm)))))


def check_every_clip(ctx, net, pcm, emb, label, invariance=()):
    """Every clip's GPU embedding (emb, from one batch) at cosine >= 0.9999 to
    the oracle's, and the clips in `invariance` bit-identical when embedded alone."""
    ref = oracle_embed_all(net, pcm)
    cs = np.array([cosine(emb[c], ref[c]) for c in range(len(pcm))])
    announce(f"{label}: all {len(pcm)} clips, min cosine {cs.min():.7f} (clip {int(cs.argmin())})")
    assert cs.min() >= 0.9999, f"{label}: clip {int(cs.argmin())} cosine {cs.min():.7f}"
    for c in invariance:
        one = ctx.embed_batch(pcm[c:c + 1])
        assert np.array_equal(one[0], emb[c]), f"{label}: clip {c} alone differs from its batch row"
