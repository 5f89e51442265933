"""Parity of the wav2vec2 analyze path on the GPU (src/analyze_w2v2.cpp)
against the oracle (oracle/oracle_w2v2.py, itself pinned to HF transformers).

Kernels: attention, LayerNorm (+GELU, weighted accumulation), conv layer 0
with GroupNorm / LayerNorm / waveform normalisation, time mean, and the conv
epilogue forms the analyze path adds (exact GELU, f32 residual, residual after
the activation, cropped output width) against f64 numpy.  End to end: random
wav2vec2 emotion and age/gender models through the C ABI against the oracle.

Tolerances.  The GPU multiplies f16 operands with f32 accumulation, so its
error budget is that of f16 rounding (2^-11 relative per operand), not the
1e-4 the reference's f32 graph holds to HF.  Kernels are checked elementwise
as |got - ref| <= atol * rms(ref) + rtol |ref|.  End to end, hidden states
and logits are held to the reference's own gates (tests/test_analyze.cpp:
enc_layer 5e-3, emotion_logits 1e-2, emotion_probs 1e-3; tests/
test_age_gender.cpp: age_raw and gender logits 1e-2, probabilities 1e-3),
applied relative to the rms of each tensor.
"""
import json
import os
import tempfile
import zlib

import numpy as np
import pytest

import oracle_w2v2 as W
from gpu_util import announce, close_report, device_ok
from vdamd import lib, synth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not device_ok(), reason="no HIP device")]


def _sync():
    lib.check(lib.lib().vdk_synchronize())


def _rng(tag):
    return np.random.default_rng(zlib.crc32(repr(tag).encode()))


# ---------------------------------------------------------------- attention
def attention_ref(qkv, nh):
    B, T, H3 = qkv.shape
    H = H3 // 3
    hd = H // nh
    q = qkv[..., :H].astype(np.float64).reshape(B, T, nh, hd).transpose(0, 2, 1, 3)
    k = qkv[..., H:2 * H].astype(np.float64).reshape(B, T, nh, hd).transpose(0, 2, 1, 3)
    v = qkv[..., 2 * H:].astype(np.float64).reshape(B, T, nh, hd).transpose(0, 2, 1, 3)
    s = q @ k.transpose(0, 1, 3, 2) / np.sqrt(hd)
    s = np.exp(s - s.max(axis=-1, keepdims=True))
    p = s / s.sum(axis=-1, keepdims=True)
    return (p @ v).transpose(0, 2, 1, 3).reshape(B, T, H)


def attention_gpu(qkv, nh):
    B, T, H3 = qkv.shape
    H = H3 // 3
    dq = lib.DeviceBuffer.from_array(np.ascontiguousarray(qkv, dtype=np.float16))
    do = lib.DeviceBuffer(B * T * H * 2)
    lib.check(lib.lib().vdk_attention(dq.ptr, B, T, nh, H // nh, 1.0 / np.sqrt(H // nh), do.ptr, None))
    _sync()
    return do.to_array(np.float16, (B, T, H))


@pytest.mark.parametrize("case", [(2, 1, 1), (1, 5, 2), (2, 64, 1), (1, 65, 3), (3, 149, 12), (1, 300, 2),
                                  (1, 999, 1)])
def test_attention(case):
    B, T, nh = case
    announce(f"attention B={B} T={T} heads={nh}")
    rng = _rng(("att", case))
    qkv = (rng.standard_normal((B, T, 3 * 64 * nh)) * 1.5).astype(np.float16)
    got = attention_gpu(qkv, nh)
    ref = attention_ref(qkv, nh)
    ok, ratio, rel = close_report(got, ref, 4e-3, 4e-3)
    assert ok, f"ratio {ratio:.2f} rel-L2 {rel:.2e}"


def test_attention_sharp_and_flat():
    """Large scores (a near one-hot softmax) and identical keys (a uniform one)."""
    rng = _rng("att-sharp")
    B, T, nh = 1, 130, 1
    qkv = rng.standard_normal((B, T, 192)).astype(np.float32)
    qkv[..., :64] *= 8.0
    qkv[..., 64:128] *= 8.0
    qkv = qkv.astype(np.float16)
    ok, ratio, rel = close_report(attention_gpu(qkv, nh), attention_ref(qkv, nh), 4e-3, 4e-3)
    assert ok, f"sharp: ratio {ratio:.2f} rel-L2 {rel:.2e}"
    flat = qkv.copy()
    flat[..., 64:128] = flat[:, :1, 64:128]
    got = attention_gpu(flat, nh).astype(np.float64)
    want = flat[..., 128:].astype(np.float64).mean(axis=1, keepdims=True)
    assert np.abs(got - want).max() < 2e-3 * np.abs(want).max() + 1e-3


def test_attention_rejects_bad_head_dim():
    d = lib.DeviceBuffer(1 << 12)
    assert lib.lib().vdk_attention(d.ptr, 1, 4, 2, 32, 0.1, d.ptr, None) != 0
    assert "head_dim" in lib.lib().vdk_last_error().decode()


# ---------------------------------------------------------------- LayerNorm
@pytest.mark.parametrize("C", [64, 512, 768, 1024, 3072])
def test_layer_norm(C):
    announce(f"layer_norm C={C}")
    rng = _rng(("ln", C))
    rows = 37
    x = (rng.standard_normal((rows, C)) * 3 + 0.5).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C)).astype(np.float32)
    acc0 = rng.standard_normal((rows, C)).astype(np.float32)
    L = lib.lib()
    dx, dg, db = (lib.DeviceBuffer.from_array(a) for a in (x, g, b))
    ref = W.layer_norm(x.astype(np.float64), g, b, 1e-5)
    # f32 in, f16 out + GELU, acc = acc + 0.25 * out
    dy, dacc = lib.DeviceBuffer(rows * C * 2), lib.DeviceBuffer.from_array(acc0)
    lib.check(L.vdk_layer_norm(dx.ptr, rows, C, dg.ptr, db.ptr, 1e-5, 1 | 4, dy.ptr, dacc.ptr, 0.25, None))
    _sync()
    y = dy.to_array(np.float16, (rows, C)).astype(np.float64)
    assert np.abs(y - W.gelu(ref)).max() < 2e-3 * (1 + np.abs(W.gelu(ref)).max())
    acc = dacc.to_array(np.float32, (rows, C))
    assert np.abs(acc - (acc0 + 0.25 * W.gelu(ref))).max() < 1e-5 * (1 + np.abs(ref).max())
    # f16 in, f32 out, acc initialised from the input
    xh = x.astype(np.float16)
    dxh, dy32 = lib.DeviceBuffer.from_array(xh), lib.DeviceBuffer(rows * C * 4)
    lib.check(L.vdk_layer_norm(dxh.ptr, rows, C, dg.ptr, db.ptr, 1e-5, 2 | 8 | 16, dy32.ptr, dacc.ptr, 0.5, None))
    _sync()
    ref16 = W.layer_norm(xh.astype(np.float64), g, b, 1e-5)
    assert np.abs(dy32.to_array(np.float32, (rows, C)) - ref16).max() < 1e-5 * (1 + np.abs(ref16).max())
    assert np.abs(dacc.to_array(np.float32, (rows, C)) - 0.5 * xh.astype(np.float32)).max() == 0


# ---------------------------------------------------------------- conv layer 0
def conv0_ref(x, w, bias, K, S, norm, g, b, eps, normalize):
    x = x.astype(np.float64)
    if normalize:
        x = (x - x.mean()) / np.sqrt(x.var() + 1e-7)
    y = W.conv1d_strided(x[:, None], w[:, None, :].astype(np.float64), S)
    if bias is not None:
        y = y + bias
    if norm == 1:
        mu = y.mean(axis=0)
        y = (y - mu) / np.sqrt(((y - mu) ** 2).mean(axis=0) + eps) * g + b
    elif norm == 2:
        y = W.layer_norm(y, g, b, eps)
    return W.gelu(y)


@pytest.mark.parametrize("case", [
    # (B, n, C, norm, bias, normalize)
    (2, 16000, 512, 1, False, False),
    (1, 48000, 512, 1, False, False),
    (2, 9001, 512, 2, True, True),
    (1, 4000, 256, 1, True, True),
    (3, 777, 1024, 2, True, False),
    (1, 12, 512, 0, False, False),
])
def test_conv0(case):
    B, n, C, norm, use_bias, normalize = case
    announce(f"w2v2_conv0 {case}")
    rng = _rng(("c0", case))
    K, S = 10, 5
    x = (0.3 * rng.standard_normal((B, n)) + 0.05).astype(np.float32)
    w = (rng.standard_normal((C, K)) * np.sqrt(0.2)).astype(np.float32)
    bias = (0.05 * rng.standard_normal(C)).astype(np.float32) if use_bias else None
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C)).astype(np.float32)
    L = lib.lib()
    T0 = (n - K) // S + 1
    dx, dw, dg, db = (lib.DeviceBuffer.from_array(a) for a in (x, w, g, b))
    dbias = lib.DeviceBuffer.from_array(bias) if bias is not None else None
    dst = lib.DeviceBuffer(8 * B)
    if normalize:
        lib.check(L.vdk_wave_stats(dx.ptr, B, n, 1e-7, dst.ptr, None))
    ws = L.vdk_w2v2_conv0_workspace_size(B, n, C, K, S)
    dwk = lib.DeviceBuffer(ws)
    dy = lib.DeviceBuffer(B * T0 * C * 2)
    lib.check(L.vdk_w2v2_conv0(dx.ptr, B, n, dst.ptr if normalize else None, dw.ptr, dbias.ptr if dbias else None,
                               C, K, S, norm, dg.ptr, db.ptr, 1e-5, dwk.ptr, ws, dy.ptr, None))
    _sync()
    y = dy.to_array(np.float16, (B, T0, C))
    for i in range(B):
        ref = conv0_ref(x[i], w, bias, K, S, norm, g, b, 1e-5, normalize)
        ok, ratio, rel = close_report(y[i], ref, 2e-3, 2e-3)
        assert ok, f"clip {i}: ratio {ratio:.2f} rel-L2 {rel:.2e}"


def test_wave_stats_and_time_mean():
    rng = _rng("stats")
    L = lib.lib()
    x = (rng.standard_normal((3, 50001)) * 0.2 + 0.1).astype(np.float32)
    dx, ds = lib.DeviceBuffer.from_array(x), lib.DeviceBuffer(24)
    lib.check(L.vdk_wave_stats(dx.ptr, 3, 50001, 1e-7, ds.ptr, None))
    _sync()
    st = ds.to_array(np.float32, (3, 2))
    x64 = x.astype(np.float64)
    np.testing.assert_allclose(st[:, 0], x64.mean(axis=1), rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(st[:, 1], 1 / np.sqrt(x64.var(axis=1) + 1e-7), rtol=1e-6)
    h = (rng.standard_normal((2, 149, 200)) * 2).astype(np.float32)
    for arr, f32 in ((h, 1), (h.astype(np.float16), 0)):
        dh, do = lib.DeviceBuffer.from_array(arr), lib.DeviceBuffer(2 * 200 * 4)
        lib.check(L.vdk_time_mean(dh.ptr, f32, 2, 149, 200, do.ptr, None))
        _sync()
        m = arr.astype(np.float64).mean(axis=1)
        np.testing.assert_allclose(do.to_array(np.float32, (2, 200)), m, rtol=1e-6, atol=1e-6)
        # weighted accumulation: out = 0.25 m, then out += -0.5 m
        lib.check(L.vdk_time_mean_acc(dh.ptr, f32, 2, 149, 200, 0.25, 0, do.ptr, None))
        lib.check(L.vdk_time_mean_acc(dh.ptr, f32, 2, 149, 200, -0.5, 1, do.ptr, None))
        _sync()
        np.testing.assert_allclose(do.to_array(np.float32, (2, 200)), -0.25 * m, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- conv epilogue forms
def test_conv_epilogue_gelu_residual_crop():
    """Grouped positional-conv slice: y (f32) = x_slice + gelu(conv(x_slice) + b),
    pad K/2 with the last step dropped, and an f32 in-place residual GEMM."""
    rng = _rng("epi")
    L = lib.lib()
    B, T, Hs, icg, K = 2, 37, 96, 48, 16
    x = rng.standard_normal((B, T, Hs)).astype(np.float16)
    w = (rng.standard_normal((icg, icg, K)) * np.sqrt(1.0 / (icg * K))).astype(np.float16)
    bias = (0.1 * rng.standard_normal(icg)).astype(np.float32)
    dx, dw = lib.DeviceBuffer.from_array(x), lib.DeviceBuffer.from_array(np.ascontiguousarray(w.transpose(0, 2, 1)))
    db = lib.DeviceBuffer.from_array(bias)
    dy = lib.DeviceBuffer.from_array(np.zeros((B, T, Hs), np.float32))
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride = dx.ptr + icg * 2, B, 1, T, icg, Hs
    d.w, d.OC, d.KH, d.KW = dw.ptr, icg, 1, K
    d.stride_h = d.stride_w = 1
    d.pad_w, d.dil_h, d.dil_w = K // 2, 1, 1
    d.bias, d.act = db.ptr, lib.ACT_GELU
    d.residual, d.res_stride, d.res_after_act = dx.ptr + icg * 2, Hs, 1
    d.y, d.y_stride, d.y_f32, d.out_w, d.tile = dy.ptr + icg * 4, Hs, 1, T, -1
    lib.check(L.vdk_conv2d_ex(C_ref(d), None))
    _sync()
    y = dy.to_array(np.float32, (B, T, Hs))
    for i in range(B):
        xs = x[i, :, icg:].astype(np.float64)
        conv = W.conv1d_strided(xs, w.astype(np.float64), 1, K // 2)[:T] + bias
        ref = xs + W.gelu(conv)
        ok, ratio, rel = close_report(y[i, :, icg:], ref, 2e-3, 2e-3)
        assert ok, f"clip {i}: ratio {ratio:.2f} rel-L2 {rel:.2e}"
        assert np.all(y[i, :, :icg] == 0)
    # f32 residual, in place: z = z + (a @ W^T + b)
    z0 = rng.standard_normal((B * T, 128)).astype(np.float32)
    a = rng.standard_normal((B * T, 64)).astype(np.float16)
    wl = (rng.standard_normal((128, 64)) * 0.125).astype(np.float16)
    bl = (0.1 * rng.standard_normal(128)).astype(np.float32)
    dz, da, dwl, dbl = (lib.DeviceBuffer.from_array(v) for v in (z0, a, wl, bl))
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC = da.ptr, B, 1, T, 64
    d.w, d.OC, d.KH, d.KW = dwl.ptr, 128, 1, 1
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
    d.bias, d.residual, d.res_f32 = dbl.ptr, dz.ptr, 1
    d.y, d.y_f32, d.tile = dz.ptr, 1, -1
    lib.check(L.vdk_conv2d_ex(C_ref(d), None))
    _sync()
    ref = z0 + a.astype(np.float64) @ wl.astype(np.float64).T + bl
    ok, ratio, rel = close_report(dz.to_array(np.float32, (B * T, 128)), ref, 2e-3, 2e-3)
    assert ok, f"f32 residual: ratio {ratio:.2f} rel-L2 {rel:.2e}"


@pytest.mark.parametrize("case", [
    # (B, T, H, groups, K): base (48 per group) and large-robust (64) shapes,
    # clips shorter than the kernel, longer than one 192-frame workgroup
    (2, 149, 768, 16, 128),
    (1, 400, 1024, 16, 128),
    (3, 7, 192, 4, 16),
    (1, 1, 128, 2, 128),
    (2, 193, 96, 2, 33),
])
def test_pos_conv(case):
    B, T, H, G, K = case
    announce(f"pos_conv {case}")
    rng = _rng(("pos", case))
    icg = H // G
    x = rng.standard_normal((B, T, H)).astype(np.float16)
    w = (rng.standard_normal((G, icg, icg, K)) * np.sqrt(1.0 / (icg * K))).astype(np.float16)   # [g][o][i][k]
    bias = (0.1 * rng.standard_normal(H)).astype(np.float32)
    wp = np.zeros((G, 64, K, icg), np.float16)
    wp[:, :icg] = w.transpose(0, 1, 3, 2)
    dx, dw, db = lib.DeviceBuffer.from_array(x), lib.DeviceBuffer.from_array(wp), lib.DeviceBuffer.from_array(bias)
    dy = lib.DeviceBuffer(B * T * H * 4)
    lib.check(lib.lib().vdk_pos_conv(dx.ptr, B, T, H, G, dw.ptr, db.ptr, K, K // 2, dy.ptr, None))
    _sync()
    y = dy.to_array(np.float32, (B, T, H))
    for i in range(B):
        xs = x[i].astype(np.float64)
        conv = np.concatenate([W.conv1d_strided(xs[:, g * icg:(g + 1) * icg], w[g].astype(np.float64), 1, K // 2)[:T]
                               for g in range(G)], axis=1)
        ref = xs + W.gelu(conv + bias)
        ok, ratio, rel = close_report(y[i], ref, 2e-3, 2e-3)
        assert ok, f"clip {i}: ratio {ratio:.2f} rel-L2 {rel:.2e}"


def C_ref(d):
    import ctypes
    return ctypes.byref(d)


# ---------------------------------------------------------------- end to end
SMALL = dict(hidden=256, n_layers=3, n_heads=4, ff=512, conv_dims=(512,) * 7, pos_k=32, pos_groups=4, proj=64)


def _model(kind, seed, dims):
    announce(f"writing a random {kind} model {dims or 'at the published size'}")
    path = os.path.join(tempfile.mkdtemp(), f"w2v2_{kind}.gguf")
    synth.write_w2v2(path, seed, kind, **dims)
    return path


def _gates(kind, got_hidden, ref_hidden, got_raw, ref_raw, tag):
    ok, ratio, rel = close_report(got_hidden, ref_hidden, 5e-3, 5e-3)
    print(f"[{tag}] last hidden: ratio {ratio:.3f} rel-L2 {rel:.2e}", flush=True)
    assert ok, f"{tag}: last hidden state ratio {ratio:.2f} rel-L2 {rel:.2e}"
    ok, ratio, rel = close_report(got_raw, ref_raw, 1e-2, 1e-2)
    print(f"[{tag}] raw outputs: ratio {ratio:.3f} rel-L2 {rel:.2e}", flush=True)
    assert ok, f"{tag}: head outputs ratio {ratio:.2f} rel-L2 {rel:.2e}"
    logits = got_raw[1:] if kind == "age_gender" else got_raw
    rlog = ref_raw[1:] if kind == "age_gender" else ref_raw
    assert np.abs(W.probs_f32(logits) - W.probs_f32(rlog)).max() <= 1e-3


@pytest.mark.parametrize("kind,dims", [("emotion", SMALL), ("age_gender", SMALL),
                                       ("emotion", dict(SMALL, pos_groups=8))],   # 32 channels per pos-conv group
                         ids=["emotion", "age_gender", "emotion-pos32"])
def test_analyze_small_matches_oracle(kind, dims):
    path = _model(kind, 5, dims)
    orc = W.OracleW2V2(path)
    ctx = lib.Context(path)
    try:
        n = 8000
        pcm = synth.clips(31, 3, n)
        announce(f"analyze {kind} small B=3 n={n}")
        feat, hid, raw = ctx.analyze_capture(pcm, 512, dims["hidden"])
        assert raw.shape == (3, ctx.analyze_outputs())
        for i in range(3):
            rfeat = orc.conv_encoder(pcm[i])
            ok, ratio, rel = close_report(feat[i], rfeat, 5e-3, 5e-3)
            print(f"[{kind} clip {i}] feat: ratio {ratio:.3f} rel-L2 {rel:.2e}", flush=True)
            assert ok, f"clip {i}: conv features ratio {ratio:.2f} rel-L2 {rel:.2e}"
            states = orc.hidden_states(pcm[i])
            _gates(kind, hid[i], states[-1], raw[i], orc.raw_outputs(pcm[i]), f"{kind} clip {i}")
        # batch independence: one clip alone gives the same outputs
        solo = ctx.analyze_pcm(pcm[1:2])
        assert np.array_equal(solo[0], raw[1])
    finally:
        ctx.close()


@pytest.mark.parametrize("kind", ["emotion", "age_gender"])
def test_analyze_full_size(kind):
    """The published shapes (base: 768 x 12 layers; large-robust: 1024 x 24)
    on two 1 s clips."""
    path = _model(kind, 7, {})
    orc = W.OracleW2V2(path)
    ctx = lib.Context(path)
    try:
        pcm = synth.clips(41, 2, 16000)
        announce(f"analyze {kind} full size B=2 n=16000")
        _, hid, raw = ctx.analyze_capture(pcm, 512, orc.hidden)
        for i in range(2):
            states = orc.hidden_states(pcm[i])
            _gates(kind, hid[i], states[-1], raw[i], orc.raw_outputs(pcm[i]), f"{kind} full clip {i}")
    finally:
        ctx.close()


def test_analyze_json_and_errors():
    path = _model("emotion", 9, SMALL)
    orc = W.OracleW2V2(path)
    ctx = lib.Context(path)
    try:
        wav = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "clip_a.wav")
        announce("analyze_path_json clip_a.wav")
        js = json.loads(ctx.analyze_path_json(wav))
        assert set(js) == {"emotion"}
        scores = js["emotion"]["scores"]
        assert list(scores) == synth.EMOTION_LABELS
        assert js["emotion"]["label"] == max(scores, key=scores.get)
        L = lib.lib()
        n = L.vdk_load_wav_16k(wav.encode(), None, 0)
        pcm = np.zeros(n, np.float32)
        assert L.vdk_load_wav_16k(wav.encode(), pcm.ctypes.data, n) == n
        ref = json.loads(orc.analyze_json(pcm))
        for k in scores:
            assert abs(scores[k] - ref["emotion"]["scores"][k]) <= 1e-3
        with pytest.raises(lib.VdkError, match="too short"):
            ctx.analyze_pcm(np.zeros((1, 300), np.float32))
        with pytest.raises(lib.VdkError, match="no speaker embedding"):
            ctx.embed_batch(np.zeros((1, 16000), np.float32))
    finally:
        ctx.close()
