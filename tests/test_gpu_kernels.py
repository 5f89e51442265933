"""Per-kernel parity of the HIP path against the oracle, through the vdk C ABI.

Gates: FBank within 1e-4 absolute of the oracle (and of the reference's golden
vectors); every conv layer shape of ResNet34 at batch 64 (the real launch
shape) within |d| <= 2e-3*|ref| + 2e-3*rms(ref) of the oracle's f32 conv fed
the same f16 input and weights, checked on the first, a middle and the last
clip of the batch; stats pooling, FC and L2 against the oracle at 1e-5..1e-4.
"""
import os
import zlib

import numpy as np
import pytest

import pyoracle as O
from gpu_util import announce, close_report, conv_gpu, device_ok, tile_fits
from test_oracle_fbank import _cases, _cfg, golden_pcm
from vdamd import gguf, lib, synth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not device_ok(), reason="no HIP device")]

CONV_RTOL = 2e-3
CONV_ATOL_RMS = 2e-3


def fbank_gpu(pcm_batch, cfg):
    L = lib.lib()
    pcm = np.ascontiguousarray(pcm_batch, dtype=np.float32)
    B, n = pcm.shape
    T = 1 + (n - cfg.win_length) // cfg.hop_length
    size = L.vdk_fbank_tables_size(cfg)
    assert size > 0
    tab = lib.DeviceBuffer(size)
    lib.check(L.vdk_fbank_tables_fill(cfg, tab.ptr))
    dp = lib.DeviceBuffer.from_array(pcm)
    df = lib.DeviceBuffer(B * cfg.n_mels * T * 4)
    lib.check(L.vdk_fbank(cfg, tab.ptr, dp.ptr, B, n, df.ptr, None))
    lib.check(L.vdk_synchronize())
    return df.to_array(np.float32, (B, cfg.n_mels, T))


def test_fbank_matches_goldens_and_oracle(golden_dir):
    z = np.load(os.path.join(golden_dir, "fbank_golden.npz"))
    for name in _cases(z):
        announce(f"fbank golden {name}")
        ocfg = _cfg(z, name)
        cfg = lib.fbank_cfg(n_mels=ocfg.n_mels, n_fft=ocfg.n_fft, win=ocfg.win_length, hop=ocfg.hop_length,
                            preemph=ocfg.preemph, low=ocfg.low_freq, high=ocfg.high_freq, cmn=bool(ocfg.cmn))
        pcm = golden_pcm(z, name)
        got = fbank_gpu(pcm[None], cfg)[0]
        ref = z[name + "/fbank"]
        assert got.shape == ref.shape, name
        assert np.abs(got - ref).max() <= 1e-4, (name, np.abs(got - ref).max())
        assert np.abs(got - O.fbank(pcm, ocfg)).max() <= 1e-4


@pytest.mark.parametrize("seconds,batch", [(3.0, 64), (4.0, 8), (10.0, 4), (20.0, 2)])
def test_fbank_batched_config_lengths(seconds, batch):
    n = synth.seconds_to_samples(seconds)
    announce(f"fbank batch={batch} n={n}")
    pcm = synth.clips(100 + int(seconds), batch, n)
    got = fbank_gpu(pcm, lib.fbank_cfg())
    for b in sorted({0, batch // 2, batch - 1}):
        ref = O.fbank(pcm[b])
        assert np.abs(got[b] - ref).max() <= 1e-4
    # CMN: every mel bin has zero mean over time
    assert np.abs(got.mean(axis=2)).max() < 1e-5


def _fbank_ex(L, cfg, tab, dp, B, n, T, d_mean):
    df = lib.DeviceBuffer(B * cfg.n_mels * T * 4)
    wsz = L.vdk_fbank_workspace_size(cfg, B, n)
    work = lib.DeviceBuffer.from_array(np.full(wsz, 0xA5, dtype=np.uint8))   # no initial contents needed
    lib.check(L.vdk_fbank_ex(cfg, tab.ptr, dp.ptr, B, n, df.ptr, d_mean, work.ptr, wsz, None))
    lib.check(L.vdk_synchronize())
    return df, work


@pytest.mark.parametrize("seconds,batch", [(3.0, 64), (3.0, 1), (10.0, 5), (0.05, 3)])
def test_fbank_deferred_cmn_means(seconds, batch):
    """vdk_fbank_ex with a mean output: the features come out before the CMN
    subtraction and features - means is bit-identical to vdk_fbank's output;
    the means agree with the f64 means of the raw rows; the consumers'
    row-mean arguments (stem, ECAPA's time-major copy)
    reproduce their outputs on the normalised features bit for bit."""
    L = lib.lib()
    cfg = lib.fbank_cfg()
    n = max(400, synth.seconds_to_samples(seconds))
    T = 1 + (n - cfg.win_length) // cfg.hop_length
    announce(f"fbank_ex deferred CMN batch={batch} n={n}")
    pcm = synth.clips(300 + batch, batch, n)
    tab = lib.DeviceBuffer(L.vdk_fbank_tables_size(cfg))
    lib.check(L.vdk_fbank_tables_fill(cfg, tab.ptr))
    dp = lib.DeviceBuffer.from_array(pcm)
    dm = lib.DeviceBuffer(batch * cfg.n_mels * 4)
    draw, work = _fbank_ex(L, cfg, tab, dp, batch, n, T, dm.ptr)
    raw = draw.to_array(np.float32, (batch, cfg.n_mels, T))
    mean = dm.to_array(np.float32, (batch, cfg.n_mels))
    want_mean = raw.astype(np.float64).mean(axis=2)
    assert np.all(np.abs(mean - want_mean) <= 1e-6 * np.maximum(1.0, np.abs(want_mean)))
    norm = fbank_gpu(pcm, cfg)
    assert np.array_equal((raw - mean[:, :, None]).view(np.uint32), norm.view(np.uint32))
    # vdk_fbank_ex without a mean output normalises in place, like vdk_fbank
    dn, _ = _fbank_ex(L, cfg, tab, dp, batch, n, T, None)
    assert np.array_equal(dn.to_array(np.float32, (batch, cfg.n_mels, T)).view(np.uint32), norm.view(np.uint32))
    # a second call on the same workspace gives the same bits
    d2 = lib.DeviceBuffer(batch * cfg.n_mels * T * 4)
    lib.check(L.vdk_fbank_ex(cfg, tab.ptr, dp.ptr, batch, n, d2.ptr, dm.ptr, work.ptr, work.nbytes, None))
    lib.check(L.vdk_synchronize())
    assert np.array_equal(d2.to_array(np.float32, (batch, cfg.n_mels, T)).view(np.uint32), raw.view(np.uint32))
    assert np.array_equal(dm.to_array(np.float32, (batch, cfg.n_mels)).view(np.uint32), mean.view(np.uint32))
    # consumers: the stem and ECAPA's time-major copy with the row means
    dnorm = lib.DeviceBuffer.from_array(norm)
    rng = np.random.default_rng(5)
    for OC, split in ((32, 0), (64, 1), (16, 0)):
        w = (rng.standard_normal((OC, 9)) * 0.4).astype(np.float32)
        bias = (rng.standard_normal(OC) * 0.1).astype(np.float32)
        dw, db = lib.DeviceBuffer.from_array(w), lib.DeviceBuffer.from_array(bias)
        ch = OC * (2 if split else 1)
        outs = []
        for src, m in ((dnorm, None), (draw, dm.ptr)):
            dy = lib.DeviceBuffer(batch * cfg.n_mels * T * ch * 2)
            lib.check(L.vdk_stem_conv3x3_ex(src.ptr, m, batch, cfg.n_mels, T, dw.ptr, db.ptr, OC, 1, split, dy.ptr,
                                            None))
            lib.check(L.vdk_synchronize())
            outs.append(dy.to_array(np.uint16, (batch * cfg.n_mels * T * ch,)))
        assert np.array_equal(outs[0], outs[1]), (OC, split)
    if T >= 3:
        outs = []
        for src, m in ((dnorm, None), (draw, dm.ptr)):
            dx = lib.DeviceBuffer(batch * (T + 4) * 96 * 2)
            lib.check(L.vdk_feats_tmajor(src.ptr, m, batch, cfg.n_mels, T, 2, 96, dx.ptr, None))
            lib.check(L.vdk_synchronize())
            outs.append(dx.to_array(np.uint16, (batch * (T + 4) * 96,)))
        assert np.array_equal(outs[0], outs[1])


def test_fbank_rejects_short_input():
    L = lib.lib()
    cfg = lib.fbank_cfg()
    tab = lib.DeviceBuffer(L.vdk_fbank_tables_size(cfg))
    d = lib.DeviceBuffer(1024)
    assert L.vdk_fbank(cfg, tab.ptr, d.ptr, 1, 399, d.ptr, None) != 0
    assert "no frames" in L.vdk_last_error().decode()


def _rand_act(rng, shape, scale=1.0):
    return np.maximum(rng.standard_normal(shape, dtype=np.float32) * scale, 0).astype(np.float16)


def _check_conv(x, w, b, res, stride, pad, relu, clips, tag):
    announce(f"conv {tag} x={x.shape} w={w.shape} s={stride} p={pad} res={res is not None}")
    got = conv_gpu(x, w, b, res, stride, pad, relu)
    wf = w.astype(np.float32)
    for c in clips:
        r = None if res is None else res[c].astype(np.float32).transpose(2, 0, 1)
        ref = O.conv2d(x[c].astype(np.float32).transpose(2, 0, 1), wf, stride, pad, bias=b, residual=r, relu=relu)
        ok, ratio, rel = close_report(got[c].astype(np.float32).transpose(2, 0, 1), ref, CONV_RTOL, CONV_ATOL_RMS)
        assert ok, f"{tag} clip {c}: max tol ratio {ratio:.3f}, rel-L2 {rel:.2e}"
        assert rel <= 2e-3, f"{tag} clip {c}: rel-L2 {rel:.2e}"
    return got


# every distinct conv of WeSpeaker ResNet34 at B=64, 3 s clips (H=80 mel, W=298 frames)
RESNET34_LAYERS = [
    # (tag, IC, OC, H, W, K, stride, pad, residual)
    ("s1_conv", 32, 32, 80, 298, 3, 1, 1, True),
    ("s2_conv1", 32, 64, 80, 298, 3, 2, 1, False),
    ("s2_down", 32, 64, 80, 298, 1, 2, 0, False),
    ("s2_conv", 64, 64, 40, 149, 3, 1, 1, True),
    ("s3_conv1", 64, 128, 40, 149, 3, 2, 1, False),
    ("s3_down", 64, 128, 40, 149, 1, 2, 0, False),
    ("s3_conv", 128, 128, 20, 75, 3, 1, 1, True),
    ("s4_conv1", 128, 256, 20, 75, 3, 2, 1, False),
    ("s4_down", 128, 256, 20, 75, 1, 2, 0, False),
    ("s4_conv", 256, 256, 10, 38, 3, 1, 1, True),
]


@pytest.mark.parametrize("layer", RESNET34_LAYERS, ids=[l[0] for l in RESNET34_LAYERS])
def test_conv_resnet34_layer_shapes_batch64(layer):
    tag, IC, OC, H, W, K, s, p, with_res = layer
    rng = np.random.default_rng(zlib.crc32(tag.encode()))
    B = 64
    x = _rand_act(rng, (B, H, W, IC))
    w = (rng.standard_normal((OC, IC, K, K), dtype=np.float32) * np.sqrt(2.0 / (IC * K * K))).astype(np.float16)
    b = (rng.standard_normal(OC, dtype=np.float32) * 0.1).astype(np.float32)
    Ho, Wo = (H + 2 * p - K) // s + 1, (W + 2 * p - K) // s + 1
    res = _rand_act(rng, (B, Ho, Wo, OC)) if with_res else None
    _check_conv(x, w, b, res, s, p, relu=True, clips=(0, 37, 63), tag=tag)


@pytest.mark.parametrize("case", [
    # (B, H, W, IC, OC, K, stride, pad, relu, bias, res)
    (1, 5, 7, 16, 16 * 2, 3, 1, 1, False, False, False),   # IC=16 chunking, tiny map
    (3, 11, 20, 32, 64, 3, 1, 1, True, True, False),       # test_blocked.cpp shapes
    (2, 11, 20, 64, 128, 3, 2, 1, True, True, False),
    (2, 9, 15, 32, 64, 1, 2, 0, False, False, False),
    (2, 9, 13, 48, 96, 3, 1, 0, False, True, True),        # valid conv, OC=96, IC=48
    (1, 1, 1, 32, 32, 3, 1, 1, True, True, True),          # single pixel
    (5, 3, 300, 64, 64, 3, 1, 1, True, True, True),        # long time axis
])
def test_conv_edge_shapes(case):
    B, H, W, IC, OC, K, s, p, relu, with_b, with_res = case
    rng = np.random.default_rng(B * 1000 + H * 10 + W)
    x = (rng.standard_normal((B, H, W, IC), dtype=np.float32)).astype(np.float16)
    w = rng.uniform(-1, 1, (OC, IC, K, K)).astype(np.float16)
    b = rng.uniform(-1, 1, OC).astype(np.float32) if with_b else None
    Ho, Wo = (H + 2 * p - K) // s + 1, (W + 2 * p - K) // s + 1
    res = rng.standard_normal((B, Ho, Wo, OC)).astype(np.float16) if with_res else None
    _check_conv(x, w, b, res, s, p, relu, clips=range(B), tag=f"edge{case}")


TILE_SHAPES = [
    # (B, H, W, IC, OC, K, stride, pad): small maps with ragged tile edges per kernel family
    (2, 13, 75, 32, 32, 3, 1, 1), (2, 9, 70, 64, 64, 3, 1, 1), (2, 7, 38, 128, 128, 3, 1, 1),
    (2, 6, 19, 256, 256, 3, 1, 1), (2, 11, 37, 32, 64, 3, 2, 1), (2, 11, 37, 64, 128, 1, 2, 0),
    (2, 1, 301, 256, 136, 1, 1, 0), (3, 5, 37, 128, 64, 1, 1, 0),
]


@pytest.mark.parametrize("shape", TILE_SHAPES, ids=[f"{s[3]}to{s[4]}k{s[5]}s{s[6]}" for s in TILE_SHAPES])
def test_conv_every_tile_config(shape):
    """Every kernel/tile variant the dispatcher can pick, on shapes with partial tiles."""
    L = lib.lib()
    B, H, W, IC, OC, K, s, p = shape
    rng = np.random.default_rng(IC * 7 + OC + K)
    x = rng.standard_normal((B, H, W, IC)).astype(np.float16)
    w = (rng.standard_normal((OC, IC, K, K)) * np.sqrt(1.0 / (IC * K * K))).astype(np.float16)
    b = rng.uniform(-1, 1, OC).astype(np.float32)
    Ho, Wo = (H + 2 * p - K) // s + 1, (W + 2 * p - K) // s + 1
    res = rng.standard_normal((B, Ho, Wo, OC)).astype(np.float16)
    refs = []
    for c in range(B):
        refs.append(O.conv2d(x[c].astype(np.float32).transpose(2, 0, 1), w.astype(np.float32), s, p, bias=b,
                             residual=res[c].astype(np.float32).transpose(2, 0, 1), relu=True))
    n = 0
    for t in range(L.vdk_conv2d_tile_count()):
        if not tile_fits(t, B, H, W, IC, OC, K, s, p):
            continue
        announce(f"tile {t} shape {shape}")
        got = conv_gpu(x, w, b, res, s, p, True, tile=t)
        for c in range(B):
            ok, ratio, rel = close_report(got[c].astype(np.float32).transpose(2, 0, 1), refs[c], CONV_RTOL,
                                          CONV_ATOL_RMS)
            assert ok and rel <= 2e-3, f"tile {t} clip {c}: ratio {ratio:.3f} rel {rel:.2e}"
        n += 1
    assert n >= 2


@pytest.mark.parametrize("case", [
    # (B, H, W, C, bias, residual, relu): the other epilogues of the
    # persistent register-weight and band 3x3 kernels (tiles 53+; every tile
    # above runs bias + residual + ReLU)
    (2, 9, 70, 64, False, False, False),
    (1, 5, 33, 64, True, False, True),
    (3, 4, 31, 32, True, True, False),
    (1, 1, 1, 64, True, True, True),
    (2, 9, 75, 128, True, False, True),      # band kernels: the widest map, no residual
    (1, 5, 38, 128, False, True, False),
    (3, 4, 31, 128, True, True, True),
])
def test_conv_register_weight_tiles_plain_epilogues(case):
    L = lib.lib()
    B, H, W, C, with_bias, with_res, relu = case
    rng = np.random.default_rng(B * 1000 + H * 10 + W + C)
    x = rng.standard_normal((B, H, W, C)).astype(np.float16)
    w = (rng.standard_normal((C, C, 3, 3)) * np.sqrt(1.0 / (9 * C))).astype(np.float16)
    b = rng.uniform(-1, 1, C).astype(np.float32) if with_bias else None
    res = rng.standard_normal((B, H, W, C)).astype(np.float16) if with_res else None
    n = 0
    for t in range(L.vdk_conv2d_tile_count()):
        if not tile_fits(t, B, H, W, C, C, 3, 1, 1, residual=with_res, relu=relu) or t < 53:
            continue
        announce(f"rw tile {t} case {case}")
        got = conv_gpu(x, w, b, res, 1, 1, relu, tile=t)
        for c in range(B):
            r = None if res is None else res[c].astype(np.float32).transpose(2, 0, 1)
            ref = O.conv2d(x[c].astype(np.float32).transpose(2, 0, 1), w.astype(np.float32), 1, 1, bias=b,
                           residual=r, relu=relu)
            ok, ratio, rel = close_report(got[c].astype(np.float32).transpose(2, 0, 1), ref, CONV_RTOL,
                                          CONV_ATOL_RMS)
            assert ok and rel <= 2e-3, f"tile {t} clip {c}: ratio {ratio:.3f} rel {rel:.2e}"
        n += 1
    assert n >= 1


@pytest.mark.parametrize("case", [
    # (B, H, W, C, residual, relu): ResNet34's 128- and 256-channel maps at
    # batch 1 and 3 (ragged last band), with and without residual
    (1, 20, 75, 128, True, True), (3, 20, 75, 128, False, True), (2, 17, 61, 128, True, False),
    (1, 10, 38, 256, True, True), (3, 7, 38, 256, False, True),
])
def test_one_row_band_tiles_equal_five_row_bands(case):
    """Tiles 76-79 (one-row bands, picked for small batches) give the 5-row band
    kernel's bits: each output's sum runs over the same chunks and taps in the
    same order, so batch-1 and batch-64 embeddings stay bit-identical."""
    B, H, W, C, with_res, relu = case
    rng = np.random.default_rng(B * 100 + H + C)
    x = rng.standard_normal((B, H, W, C)).astype(np.float16)
    w = (rng.standard_normal((C, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, C).astype(np.float32)
    res = rng.standard_normal((B, H, W, C)).astype(np.float16) if with_res else None
    base = 64 if C == 128 else 65
    ref = conv_gpu(x, w, b, res, 1, 1, relu, tile=base)
    for t in ((76, 77) if C == 128 else (78, 79)):
        announce(f"one-row band tile {t} case {case}")
        got = conv_gpu(x, w, b, res, 1, 1, relu, tile=t)
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), f"tile {t} differs from tile {base}"
    assert np.array_equal(conv_gpu(x, w, b, res, 1, 1, relu).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("case", [(1, 40, 149, True, True), (3, 40, 149, False, True), (2, 13, 37, True, False)])
def test_small_batch_64_channel_halo_tile_equals_register_weight(case):
    """Tile 31 (halo kernel, one 64-channel chunk) gives the register-weight
    kernel's bits for 64 -> 64 convs at small batches: both sum tap-major,
    channel-minor, so either may serve a batch without breaking batch
    invariance."""
    B, H, W, with_res, relu = case
    rng = np.random.default_rng(B * 31 + H)
    x = rng.standard_normal((B, H, W, 64)).astype(np.float16)
    w = (rng.standard_normal((64, 64, 3, 3)) * np.sqrt(2.0 / 576)).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, 64).astype(np.float32)
    res = rng.standard_normal((B, H, W, 64)).astype(np.float16) if with_res else None
    announce(f"64-channel halo tile vs register-weight {case}")
    ref = conv_gpu(x, w, b, res, 1, 1, relu, tile=66)
    assert np.array_equal(conv_gpu(x, w, b, res, 1, 1, relu, tile=31).view(np.uint16), ref.view(np.uint16))
    assert np.array_equal(conv_gpu(x, w, b, res, 1, 1, relu).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("case", [
    # (B, H, W, C, residual): enough tiles that each persistent workgroup
    # walks several, with walk lengths of every remainder modulo the ring
    # depths across the cases (13, 4, 5, 8 and 2 tiles per workgroup for the
    # 4-row tiles on 256 CUs)
    (64, 40, 149, 64, True), (16, 40, 149, 64, False), (24, 40, 149, 64, True), (36, 40, 149, 64, False),
    (7, 40, 149, 64, True), (64, 80, 298, 32, True), (9, 80, 298, 32, False),
])
def test_conv_register_weight_rings_bitwise(case):
    """The register-weight kernels (tiles 53-56: 2-stage ring with 2-, 4- and
    6-row tiles; 66-69: 3- and 4-stage rings) return the same bits for every
    tile height and ring depth, on maps where each workgroup walks several
    tiles; the 4-row 2-stage kernel's last clip is checked against the
    oracle."""
    B, H, W, C, with_res = case
    rng = np.random.default_rng(B * 7 + H + C)
    x = np.maximum(rng.standard_normal((B, H, W, C)), 0).astype(np.float16)
    w = (rng.standard_normal((C, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float16)
    b = rng.uniform(-0.1, 0.1, C).astype(np.float32)
    res = rng.standard_normal((B, H, W, C)).astype(np.float16) if with_res else None
    ref_tile = 53 if C == 64 else 56
    assert tile_fits(ref_tile, B, H, W, C, C, 3, 1, 1, residual=with_res)
    want = conv_gpu(x, w, b, res, 1, 1, True, tile=ref_tile)
    r0 = None if res is None else res[B - 1].astype(np.float32).transpose(2, 0, 1)
    ref = O.conv2d(x[B - 1].astype(np.float32).transpose(2, 0, 1), w.astype(np.float32), 1, 1, bias=b,
                   residual=r0, relu=True)
    ok, ratio, rel = close_report(want[B - 1].astype(np.float32).transpose(2, 0, 1), ref, CONV_RTOL, CONV_ATOL_RMS)
    assert ok and rel <= 2e-3, f"tile {ref_tile}: ratio {ratio:.3f} rel {rel:.2e}"
    n = 0
    for t in (53, 54, 55, 56, 66, 67, 68, 69):
        if t == ref_tile or not tile_fits(t, B, H, W, C, C, 3, 1, 1, residual=with_res):
            continue
        announce(f"rw tile {t} case {case}")
        got = conv_gpu(x, w, b, res, 1, 1, True, tile=t)
        bad = np.flatnonzero(got.view(np.uint16) != want.view(np.uint16))
        assert bad.size == 0, f"tile {t}: {bad.size} values differ from tile {ref_tile}, first at {bad[0]}"
        n += 1
    assert n >= 1


@pytest.mark.parametrize("shape", [(2, 7, 75, 128, True), (3, 20, 75, 128, False), (1, 6, 40, 256, True),
                                   (5, 40, 149, 64, True), (3, 21, 149, 64, False), (4, 80, 298, 32, True)])
def test_conv_chunked_weights_bitwise(shape):
    """A conv given the chunk-major weight copy (vdk_conv_pack_chunked) as
    w_chunked returns the same bits as without it, on every tile that fits
    (the band kernels stream it, the register-weight kernels load their
    weight fragments from it; the others ignore it)."""
    L = lib.lib()
    B, H, W, C, with_res = shape
    rng = np.random.default_rng(B * 100 + H + W + C)
    x = np.maximum(rng.standard_normal((B, H, W, C)), 0).astype(np.float16)
    w = (rng.standard_normal((C, 3, 3, C)) * np.sqrt(2.0 / (9 * C))).astype(np.float16)
    b = rng.uniform(-0.1, 0.1, C).astype(np.float32)
    res = rng.standard_normal((B, H, W, C)).astype(np.float16) if with_res else None
    wc = np.zeros(w.size, dtype=np.uint16)
    L.vdk_conv_pack_chunked(w.view(np.uint16).ctypes.data, C, 3, 3, C, wc.ctypes.data)
    dx, dw, dwc, db = (lib.DeviceBuffer.from_array(a) for a in (x, w, wc, b))
    dr = lib.DeviceBuffer.from_array(res) if with_res else None
    n = 0
    for t in range(L.vdk_conv2d_tile_count()):
        if not tile_fits(t, B, H, W, C, C, 3, 1, 1, residual=with_res):
            continue
        outs = []
        for chunked in (False, True):
            d = lib.ConvDesc()
            d.x, d.batch, d.H, d.W, d.IC = dx.ptr, B, H, W, C
            d.w, d.OC, d.KH, d.KW = dw.ptr, C, 3, 3
            d.stride_h = d.stride_w = 1
            d.pad_h = d.pad_w = 1
            d.bias, d.act, d.tile = db.ptr, lib.ACT_RELU, t
            d.residual = dr.ptr if dr else None
            d.w_chunked = dwc.ptr if chunked else None
            dy = lib.DeviceBuffer(B * H * W * C * 2)
            d.y = dy.ptr
            announce(f"chunked weights tile {t} shape {shape} chunked={chunked}")
            lib.check(L.vdk_conv2d_ex(d, None))
            lib.check(L.vdk_synchronize())
            outs.append(dy.to_array(np.uint16, (B, H, W, C)))
        assert np.array_equal(outs[0], outs[1]), f"tile {t}"
        n += 1
    assert n >= 2


@pytest.mark.parametrize("case", [
    # (B, H, T, IC, OC, x_stride, KH, KW, stride, pad, epilogue)
    (2, 1, 301, 1024, 1024, 1024, 1, 1, 1, 0, "bias_relu_bn"), (3, 1, 149, 3072, 768, 3072, 1, 1, 1, 0, "bias_res"),
    (2, 1, 37, 768, 2304, 776, 1, 1, 1, 0, "gelu"), (1, 1, 5, 256, 136, 256, 1, 1, 1, 0, "res_f32_y_f32"),
    (2, 1, 70, 4608, 128, 4608, 1, 1, 1, 0, "tmajor"), (2, 1, 301, 512, 512, 512, 1, 3, 2, 0, "gelu"),
    (3, 1, 99, 512, 512, 520, 1, 2, 2, 0, "gelu"), (2, 1, 40, 256, 256, 256, 1, 5, 1, 2, "bias_relu_bn"),
    (2, 9, 31, 64, 128, 64, 1, 1, 2, 0, "bias_res"), (2, 11, 37, 64, 128, 64, 3, 3, 2, 1, "bias_res"),
    (2, 7, 19, 128, 256, 128, 3, 3, 1, 1, "bias_relu_bn"),
    (2, 1, 45, 32, 256, 32, 1, 1, 1, 0, "bias_res"), (3, 1, 77, 64, 384, 72, 1, 1, 1, 0, "gelu"),
])
def test_gemm_ws_tiles_bitwise(case):
    """The GEMM kernel with producer / compute waves (tiles 81-84) returns
    the LDS-DMA kernel's bits (same MFMA shape, K order and staged epilogue)
    for every epilogue form the models use: bias + ReLU + post-BN, f16
    residual, exact GELU, f32 residual into an f32 output, a time-major
    store; 1x1 GEMMs, strided 2- / 3-tap convs (wav2vec2's feature encoder),
    a zero-padded 5-tap conv and a 2-D 1x1 stride-2 shortcut; ragged pixel
    counts, output channels off the tile grid, padded input strides, and K
    of one or two chunks (the ring's shortest walks)."""
    L = lib.lib()
    B, H, T, IC, OC, xs, KH, KW, st, pad, epi = case
    rng = np.random.default_rng(B * 10 + T + IC + OC + KW + KH)
    announce(f"gemm_ws B={B} H={H} T={T} {IC}->{OC} k{KH}x{KW} s{st} p{pad} {epi}")
    sh, ph = (st, pad) if KH > 1 or H > 1 else (1, 0)
    Ho = (H + 2 * ph - KH) // sh + 1
    To = (T + 2 * pad - KW) // st + 1
    dx = lib.DeviceBuffer.from_array((rng.standard_normal((B, H, T, xs)) * 0.5).astype(np.float16))
    dw = lib.DeviceBuffer.from_array((rng.standard_normal((OC, KH, KW, IC)) * np.sqrt(1.0 / (KH * KW * IC))).astype(
        np.float16))
    db = lib.DeviceBuffer.from_array(rng.standard_normal(OC).astype(np.float32))
    dsc = lib.DeviceBuffer.from_array(rng.uniform(0.5, 1.5, OC).astype(np.float32))
    dsh = lib.DeviceBuffer.from_array(rng.standard_normal(OC).astype(np.float32))
    f32 = epi == "res_f32_y_f32"
    dr = lib.DeviceBuffer.from_array(rng.standard_normal((B, Ho, To, OC)).astype(np.float32 if f32 else np.float16))
    outs = {}
    for t in (36, 81, 82, 83, 84):
        d = lib.ConvDesc()
        d.x, d.batch, d.H, d.W, d.IC, d.x_stride = dx.ptr, B, H, T, IC, xs
        d.w, d.OC, d.KH, d.KW = dw.ptr, OC, KH, KW
        d.stride_h, d.pad_h = sh, ph
        d.stride_w, d.pad_w = st, pad
        d.dil_h = d.dil_w = 1
        d.bias = db.ptr
        if epi == "bias_relu_bn":
            d.act, d.post_scale, d.post_shift = lib.ACT_RELU, dsc.ptr, dsh.ptr
        elif epi == "bias_res":
            d.residual = dr.ptr
        elif epi == "gelu":
            d.act = lib.ACT_GELU
        elif f32:
            d.residual, d.res_f32, d.y_f32 = dr.ptr, 1, 1
        else:
            d.act, d.y_time_major = lib.ACT_RELU, 1
        dy = lib.DeviceBuffer(B * Ho * To * OC * 4)
        d.y, d.tile = dy.ptr, t
        if not L.vdk_conv2d_tile_fits_ex(t, d):
            continue
        lib.check(L.vdk_conv2d_ex(d, None))
        lib.check(L.vdk_synchronize())
        outs[t] = dy.to_array(np.uint32 if f32 else np.uint16, (B, Ho, To, OC))
    assert 36 in outs and len(outs) >= (2 if IC % 64 else 3), sorted(outs)
    for t, o in outs.items():
        assert np.array_equal(o, outs[36]), f"tile {t}"


def test_conv_invariants_delta_and_zero():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 6, 70, 32)).astype(np.float16)
    w = np.zeros((32, 32, 3, 3), dtype=np.float16)
    for c in range(32):
        w[c, c, 1, 1] = 1.0                        # identity kernel
    y = conv_gpu(x, w, None, None, 1, 1, False)
    assert np.array_equal(y, x)                    # exact: one product per output
    b = rng.uniform(-1, 1, 32).astype(np.float32)
    y0 = conv_gpu(x, np.zeros_like(w), b, None, 1, 1, False)
    assert np.array_equal(y0, np.broadcast_to(b.astype(np.float16), y0.shape))


def test_conv_rejects_bad_shapes():
    L = lib.lib()
    d = lib.DeviceBuffer(1 << 16)
    assert L.vdk_conv2d_nhwc(d.ptr, 1, 4, 4, 24, d.ptr, 32, 3, 3, 1, 1, None, None, 0, d.ptr, None) != 0
    assert "IC" in L.vdk_last_error().decode()
    assert L.vdk_conv2d_nhwc(d.ptr, 1, 4, 4, 32, d.ptr, 20, 3, 3, 1, 1, None, None, 0, d.ptr, None) != 0
    assert "OC" in L.vdk_last_error().decode()
    assert L.vdk_conv2d_nhwc(None, 1, 4, 4, 32, d.ptr, 32, 3, 3, 1, 1, None, None, 0, d.ptr, None) != 0
    assert L.vdk_conv2d_nhwc(d.ptr, 1, 1, 1, 32, d.ptr, 32, 3, 3, 1, 0, None, None, 0, d.ptr, None) != 0


@pytest.mark.parametrize("IC,OC,npix,prologue", [(128, 128, 15968, True), (352, 128, 15968, True),
                                               (1024, 512, 4096, True), (96, 40, 777, False), (32, 64, 300, True)])
def test_conv_q8_0_weights_dequantised_in_registers(IC, OC, npix, prologue):
    """1x1 convs reading q8_0 blocks straight from the model-file layout
    (vdk_conv_desc.w_q8_0) equal, bit for bit, the same convs on the
    host-dequantised f16 weights f16(q * d), on every register-staged tile
    that takes the shape, with and without the BN+ReLU input prologue."""
    L = lib.lib()
    rng = np.random.default_rng(IC + OC + npix)
    announce(f"q8_0 1x1 IC={IC} OC={OC} npix={npix} prologue={prologue}")
    w = (rng.standard_normal((OC, IC)) * np.sqrt(2.0 / IC)).astype(np.float32)
    w[3 % OC, :32] = 0.0                                   # an all-zero block (d = 0)
    raw = gguf.quantize_q8_0(w)                            # [OC][IC/32] blocks of 34 bytes
    wdeq = gguf.dequantize_q8_0(raw.tobytes(), OC * IC).reshape(OC, IC)
    wf16 = wdeq.astype(np.float16)                         # what the host upload stores
    x = rng.standard_normal((1, 1, npix, IC)).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, OC).astype(np.float32)
    sc = rng.uniform(0.5, 1.5, IC).astype(np.float32)
    sh = rng.uniform(-0.5, 0.5, IC).astype(np.float32)
    keep = [lib.DeviceBuffer.from_array(a) for a in (x, wf16, raw, b, sc, sh)]
    dx, dwf, dwq, db, dsc, dsh = keep
    outs = {}
    for q8 in (False, True):
        for t in range(L.vdk_conv2d_tile_count()):
            d = lib.ConvDesc()
            d.x, d.batch, d.H, d.W, d.IC = dx.ptr, 1, 1, npix, IC
            d.w, d.OC, d.KH, d.KW = (None if q8 else dwf.ptr), OC, 1, 1
            d.w_q8_0 = dwq.ptr if q8 else None
            d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
            d.bias, d.act = db.ptr, lib.ACT_RELU
            if prologue:
                d.in_scale, d.in_shift = dsc.ptr, dsh.ptr
            if not L.vdk_conv2d_tile_fits_ex(t, d) or (t >= 14 and t < 62):
                continue
            dy = lib.DeviceBuffer(npix * OC * 2)
            d.y, d.tile = dy.ptr, t
            lib.check(L.vdk_conv2d_ex(d, None))
            lib.check(L.vdk_synchronize())
            outs[(q8, t)] = dy.to_array(np.float16, (npix, OC))
    tiles = sorted(t for (q, t) in outs if q)   # the register-staged tiles (the only q8_0 readers)
    assert tiles and all((False, t) in outs for t in tiles)
    for t in tiles:
        assert np.array_equal(outs[(True, t)].view(np.uint16), outs[(False, t)].view(np.uint16)), f"tile {t}"
    # and the f16 path against the oracle's conv on the dequantised weights
    xin = x[0, 0].astype(np.float32)
    if prologue:
        xin = np.maximum(xin * sc + sh, 0).astype(np.float16).astype(np.float32)
    ref = np.maximum(xin @ wf16.astype(np.float32).T + b, 0)
    ok, ratio, rel = close_report(outs[(True, tiles[0])].astype(np.float32), ref, CONV_RTOL, CONV_ATOL_RMS)
    assert ok, (ratio, rel)


@pytest.mark.parametrize("IC,OC,npix", [(320, 128, 15968), (128, 128, 15968), (512, 128, 1000), (96, 32, 777),
                                        (1024, 512, 15968), (512, 256, 4001)])
def test_conv_input_prologue_every_tile_bitwise(IC, OC, npix):
    """1x1 convs with the BN+ReLU input prologue relu(x * in_scale +
    in_shift): every tile that takes the shape (register-staged: applied on
    the operand loads; LDS-DMA and GEMM kernels: applied to the B fragments
    leaving LDS) gives the same bits, and the oracle's conv of the prologued
    input agrees; the last two shapes are CAM++'s transits (B=32 x 499
    frames, and a ragged pixel count)."""
    L = lib.lib()
    rng = np.random.default_rng(3 * IC + OC + npix)
    announce(f"prologue 1x1 IC={IC} OC={OC} npix={npix}")
    x = rng.standard_normal((1, 1, npix, IC)).astype(np.float16)
    w = (rng.standard_normal((OC, IC)) * np.sqrt(2.0 / IC)).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, OC).astype(np.float32)
    sc = rng.uniform(0.5, 1.5, IC).astype(np.float32)
    sh = rng.uniform(-0.5, 0.5, IC).astype(np.float32)
    dx, dw, db, dsc, dsh = (lib.DeviceBuffer.from_array(a) for a in (x, w, b, sc, sh))
    outs = {}
    for t in range(L.vdk_conv2d_tile_count()):
        d = lib.ConvDesc()
        d.x, d.batch, d.H, d.W, d.IC = dx.ptr, 1, 1, npix, IC
        d.w, d.OC, d.KH, d.KW = dw.ptr, OC, 1, 1
        d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
        d.bias, d.act = db.ptr, lib.ACT_RELU
        d.in_scale, d.in_shift = dsc.ptr, dsh.ptr
        if not L.vdk_conv2d_tile_fits_ex(t, d):
            continue
        dy = lib.DeviceBuffer(npix * OC * 2)
        d.y, d.tile = dy.ptr, t
        lib.check(L.vdk_conv2d_ex(d, None))
        lib.check(L.vdk_synchronize())
        outs[t] = dy.to_array(np.float16, (npix, OC))
    assert any(t < 14 for t in outs) and any(14 <= t < 62 for t in outs)
    ref_t = min(outs)
    for t, o in outs.items():
        assert np.array_equal(o.view(np.uint16), outs[ref_t].view(np.uint16)), f"tile {t} vs {ref_t}"
    xin = np.maximum(x[0, 0].astype(np.float32) * sc + sh, 0).astype(np.float16).astype(np.float32)
    ref = np.maximum(xin @ w.astype(np.float32).T + b, 0)
    ok, ratio, rel = close_report(outs[ref_t].astype(np.float32), ref, CONV_RTOL, CONV_ATOL_RMS)
    assert ok, (ratio, rel)


@pytest.mark.parametrize("B,H,W,OC,split", [(64, 80, 298, 32, 0), (3, 7, 37, 64, 0), (2, 9, 33, 32, 1),
                                           (2, 5, 31, 16, 0), (1, 80, 1998, 32, 1)])
def test_stem_conv_matches_oracle(B, H, W, OC, split):
    """The stem (f32 MFMA for 32 / 64 channels, the f32 FMA loop for 16)
    against the oracle's f32 conv; in split-f16 the stored hi + lo pair holds
    the f32 result to ~2^-21 relative."""
    L = lib.lib()
    rng = np.random.default_rng(3 + OC + W)
    announce(f"stem B={B} H={H} W={W} OC={OC} split={split}")
    feats = rng.standard_normal((B, H, W)).astype(np.float32) * 3
    w = rng.standard_normal((OC, 1, 3, 3)).astype(np.float32) * 0.4
    b = rng.standard_normal(OC).astype(np.float32) * 0.1
    df = lib.DeviceBuffer.from_array(feats)
    dw = lib.DeviceBuffer.from_array(w.reshape(OC, 9))
    db = lib.DeviceBuffer.from_array(b)
    ch = OC * (2 if split else 1)
    dy = lib.DeviceBuffer(B * H * W * ch * 2)
    lib.check(L.vdk_stem_conv3x3_ex(df.ptr, None, B, H, W, dw.ptr, db.ptr, OC, 1, split, dy.ptr, None))
    lib.check(L.vdk_synchronize())
    y = dy.to_array(np.float16, (B, H, W, ch)).astype(np.float32)
    got = y[..., :OC] + y[..., OC:] if split else y
    for c in sorted({0, B // 2, B - 1}):
        ref = O.conv2d(feats[c][None], w, 1, 1, bias=b, relu=True)
        g = got[c].transpose(2, 0, 1)
        if split:
            assert np.abs(g - ref).max() <= 2e-6 * np.abs(ref).max() + 1e-6
        else:
            ok, ratio, rel = close_report(g, ref, CONV_RTOL, CONV_ATOL_RMS)
            assert ok, (ratio, rel)
            # f16 rounding of an f32-accurate value: within one f16 ulp
            assert np.all(np.abs(g - ref) <= np.abs(ref) * 2.0 ** -10 + 1e-6)


def test_tstp_linear_l2_match_oracle():
    L = lib.lib()
    rng = np.random.default_rng(4)
    B, H, W, C, E = 64, 10, 38, 256, 256
    announce("tstp/linear/l2")
    x = (rng.standard_normal((B, H, W, C)) * 30).astype(np.float16)
    dx = lib.DeviceBuffer.from_array(x)
    P = 2 * C * H
    dp = lib.DeviceBuffer(B * P * 4)
    lib.check(L.vdk_tstp(dx.ptr, B, H, W, C, 1e-8, dp.ptr, None))
    wfc = (rng.standard_normal((E, P)) * np.sqrt(2.0 / P)).astype(np.float32)
    bfc = rng.standard_normal(E).astype(np.float32) * 0.01
    mv = rng.standard_normal(E).astype(np.float32) * 0.05
    dw, db, dm = (lib.DeviceBuffer.from_array(a) for a in (wfc, bfc, mv))
    dy = lib.DeviceBuffer(B * E * 4)
    wsz = L.vdk_linear_workspace_size(B, P, E)
    dwk = lib.DeviceBuffer(wsz)
    assert L.vdk_linear(dp.ptr, B, P, dw.ptr, db.ptr, dm.ptr, E, dy.ptr, dwk.ptr, wsz - 4, None) != 0
    lib.check(L.vdk_linear(dp.ptr, B, P, dw.ptr, db.ptr, dm.ptr, E, dy.ptr, dwk.ptr, wsz, None))
    lib.check(L.vdk_synchronize())
    pooled = dp.to_array(np.float32, (B, P))
    pre = dy.to_array(np.float32, (B, E))
    dn = lib.DeviceBuffer(B * E * 4)
    lib.check(L.vdk_l2norm_to(dy.ptr, B, E, dn.ptr, None))     # out of place: y keeps the pre-norm rows
    lib.check(L.vdk_l2norm(dy.ptr, B, E, None))
    lib.check(L.vdk_synchronize())
    emb = dy.to_array(np.float32, (B, E))
    assert np.array_equal(dn.to_array(np.float32, (B, E)), emb)
    for c in (0, 17, 63):
        rp = O.tstp(x[c].astype(np.float32).transpose(2, 0, 1), 1e-8)
        assert np.allclose(pooled[c], rp, rtol=1e-5, atol=1e-5)
        rl = O.linear(pooled[c], wfc, bfc, mv)
        assert np.allclose(pre[c], rl, rtol=1e-4, atol=1e-4)
        assert np.allclose(emb[c], O.l2norm(pre[c]), rtol=1e-6, atol=1e-6)
    # zero vectors stay zero (norm 0 is skipped)
    z = lib.DeviceBuffer.from_array(np.zeros((2, 8), np.float32))
    lib.check(L.vdk_l2norm(z.ptr, 2, 8, None))
    lib.check(L.vdk_synchronize())
    assert np.array_equal(z.to_array(np.float32, (2, 8)), np.zeros((2, 8), np.float32))
    # the FC with the L2 normalisation in its reduce: the same pre-norm bits,
    # normalised rows within an f32 rounding of vdk_l2norm_to's
    dpre, dl2 = lib.DeviceBuffer(B * E * 4), lib.DeviceBuffer(B * E * 4)
    lib.check(L.vdk_linear_l2_ex(dp.ptr, B, P, dw.ptr, db.ptr, dm.ptr, E, dpre.ptr, dl2.ptr, dwk.ptr, wsz, None))
    lib.check(L.vdk_synchronize())
    assert np.array_equal(dpre.to_array(np.float32, (B, E)).view(np.uint32), pre.view(np.uint32))
    assert np.abs(dl2.to_array(np.float32, (B, E)) - emb).max() <= 1.2e-7
    assert L.vdk_linear_l2_ex(dp.ptr, B, P, dw.ptr, db.ptr, dm.ptr, E, dpre.ptr, dpre.ptr, dwk.ptr, wsz, None) != 0


@pytest.mark.parametrize("B,H,W,C,lo", [(3, 10, 38, 256, 0), (2, 5, 250, 512, 512), (2, 4, 37, 200, 0),
                                         (1, 3, 2, 64, 0), (2, 3, 128, 264, 0)])
def test_tstp_vector_and_scalar_paths(B, H, W, C, lo):
    """TSTP on 16-byte channel vectors (16-byte aligned rows, C % 8 == 0)
    and, for the same values through a view 4 bytes off alignment, on the
    scalar path; split-f16 inputs (value = hi + lo); against the oracle's
    two-pass statistics."""
    L = lib.lib()
    rng = np.random.default_rng(B * 100 + C)
    xs = C * (2 if lo else 1)
    x = (rng.standard_normal((B, H, W, xs)) * 20).astype(np.float16)
    announce(f"tstp B={B} H={H} W={W} C={C} lo={lo}")
    for off in (0, 2):   # off = 2 elements: a 4-byte aligned view, the scalar kernel
        buf = np.zeros(x.size + 8, dtype=np.float16)
        buf[off:off + x.size] = x.reshape(-1)
        dx = lib.DeviceBuffer.from_array(buf)
        dp = lib.DeviceBuffer(B * 2 * C * H * 4)
        lib.check(L.vdk_tstp_ex(dx.ptr + 2 * off, xs, lo, B, H, W, C, 1e-8, dp.ptr, None))
        lib.check(L.vdk_synchronize())
        got = dp.to_array(np.float32, (B, 2 * C * H))
        v = x.astype(np.float32)
        if lo:
            v = v[..., :C] + v[..., C:]
        for c in range(B):
            rp = O.tstp(v[c].transpose(2, 0, 1), 1e-8)
            assert np.allclose(got[c], rp, rtol=2e-5, atol=2e-5), (off, c)


@pytest.mark.parametrize("case", [(1, 3, 5, 0), (70, 130, 33, 1), (130, 5120, 200, 2), (64, 1024, 1024, 5),
                                  (64, 128, 1024, 2), (3, 769, 64, 0)])
def test_linear_shapes_and_batch_invariance(case):
    """y = act(W x + b - mv) against numpy f64 over ragged shapes: K not a
    multiple of 4 (scalar loads), several batch tiles, output counts off the
    tile grid, both per-thread blockings; each clip's row is bitwise the
    same computed alone (every output sums its slice in k order)."""
    L = lib.lib()
    B, I, E, act = case
    rng = np.random.default_rng(B * 1000 + I + E)
    x = rng.standard_normal((B, I)).astype(np.float32)
    w = (rng.standard_normal((E, I)) / np.sqrt(I)).astype(np.float32)
    b = (0.1 * rng.standard_normal(E)).astype(np.float32)
    mv = (0.05 * rng.standard_normal(E)).astype(np.float32)
    dx, dw, db, dm = (lib.DeviceBuffer.from_array(a) for a in (x, w, b, mv))
    dy = lib.DeviceBuffer(B * E * 4)
    wsz = L.vdk_linear_workspace_size(B, I, E)
    dwk = lib.DeviceBuffer(wsz)
    announce(f"linear {case}")
    lib.check(L.vdk_linear_ex(dx.ptr, B, I, dw.ptr, db.ptr, dm.ptr, E, act, dy.ptr, dwk.ptr, wsz, None))
    lib.check(L.vdk_synchronize())
    got = dy.to_array(np.float32, (B, E))
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b - mv
    ref = {0: ref, 1: np.maximum(ref, 0), 2: 1 / (1 + np.exp(-ref)), 5: np.tanh(ref)}[act]   # VDK_ACT_* codes
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)
    for c in sorted({0, B // 2, B - 1}):
        d1 = lib.DeviceBuffer.from_array(x[c:c + 1])
        w1 = L.vdk_linear_workspace_size(1, I, E)
        k1 = lib.DeviceBuffer(w1)
        lib.check(L.vdk_linear_ex(d1.ptr, 1, I, dw.ptr, db.ptr, dm.ptr, E, act, dy.ptr, k1.ptr, w1, None))
        lib.check(L.vdk_synchronize())
        assert np.array_equal(dy.to_array(np.float32, (1, E))[0], got[c]), c


@pytest.mark.parametrize("case", [
    # (B, T, IC, x_stride, OC): CAM++ dense-layer linear1 shapes (the BatchNorm +
    # ReLU of the concatenated features folded into the GEMM's operand loads)
    (2, 499, 128, 512, 128),
    (1, 97, 480, 896, 128),
    (3, 33, 96, 96, 64),
    (1, 5, 64, 64, 32),
    (2, 40, 32, 32, 64),   # one K chunk on the 32-wide tiles (the two-slot loop's shortest trip)
    (1, 9, 16, 16, 32),    # one K chunk on the 16-wide tiles
])
def test_conv_input_prologue(case):
    """y = relu(W relu(x*s + t) + b) for every tile that takes the input prologue,
    against numpy with the prologue rounded to f16 (as the GPU feeds it to the MFMA)."""
    L = lib.lib()
    B, T, IC, xs, OC = case
    rng = np.random.default_rng(IC + OC + T)
    x = rng.standard_normal((B, T, xs)).astype(np.float16)
    s = (0.5 + rng.random(IC)).astype(np.float32)
    t = (0.3 * rng.standard_normal(IC)).astype(np.float32)
    w = (rng.standard_normal((OC, IC)) * np.sqrt(1.0 / IC)).astype(np.float16)
    b = (0.1 * rng.standard_normal(OC)).astype(np.float32)
    u = np.maximum(x[..., :IC].astype(np.float32) * s + t, 0).astype(np.float16).astype(np.float64)
    ref = np.maximum(u @ w.astype(np.float64).T + b, 0)
    dx, dw, db, ds, dt = (lib.DeviceBuffer.from_array(a) for a in (x, w, b, s, t))
    dy = lib.DeviceBuffer(B * T * OC * 2)
    d = lib.ConvDesc()
    d.x, d.batch, d.H, d.W, d.IC, d.x_stride = dx.ptr, B, 1, T, IC, xs
    d.w, d.OC, d.KH, d.KW = dw.ptr, OC, 1, 1
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
    d.bias, d.act, d.y = db.ptr, lib.ACT_RELU, dy.ptr
    d.in_scale, d.in_shift = ds.ptr, dt.ptr
    n = 0
    for tile in [-1] + list(range(L.vdk_conv2d_tile_count())):
        if tile >= 0 and not L.vdk_conv2d_tile_fits_ex(tile, d):
            continue
        d.tile = tile
        announce(f"input prologue tile {tile} {case}")
        lib.check(L.vdk_conv2d_ex(d, None))
        lib.check(L.vdk_synchronize())
        got = dy.to_array(np.float16, (B, T, OC)).astype(np.float64)
        ok, ratio, rel = close_report(got, ref, CONV_RTOL, CONV_ATOL_RMS)
        assert ok, f"tile {tile}: ratio {ratio:.3f} rel {rel:.2e}"
        n += 1
    assert n >= 3
    # the prologue needs a 1x1 conv without padding
    d.KW, d.pad_w, d.tile = 3, 1, -1
    assert L.vdk_conv2d_ex(d, None) != 0
    assert "input prologue" in L.vdk_last_error().decode()


@pytest.mark.parametrize("B,H,W,IC,OC,K,res", [(3, 17, 45, 96, 192, 3, True), (1, 1, 5000, 768, 384, 1, False),
                                               (1, 1, 4096, 3072, 3072, 1, False)])
def test_conv_autotune_same_bits_and_cached(B, H, W, IC, OC, K, res):
    """Shapes no built-in rule was measured on (a 96 -> 192 3x3 with a
    residual, 1-D GEMMs of 768 -> 384 and the real ECAPA MFA's 3072 -> 3072):
    with the run-time tuner on, the first call (tuning) and the second (the
    cached choice) give the default tile's bits, and the chosen tile fits."""
    L = lib.lib()
    rng = np.random.default_rng(H * W + IC + OC)
    announce(f"autotune conv B={B} {H}x{W} {IC}->{OC} k={K} res={res}")
    x = rng.standard_normal((B, H, W, IC)).astype(np.float16)
    w = (rng.standard_normal((OC, K, K, IC)) * np.sqrt(2.0 / (IC * K * K))).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, OC).astype(np.float32)
    r = rng.standard_normal((B, H, W, OC)).astype(np.float16)
    dx, dw, db, dr = (lib.DeviceBuffer.from_array(a) for a in (x, w, b, r))
    outs = []
    def run():
        d = lib.ConvDesc()
        d.x, d.batch, d.H, d.W, d.IC = dx.ptr, B, H, W, IC
        d.w, d.OC, d.KH, d.KW = dw.ptr, OC, K, K
        d.stride_h = d.stride_w = d.dil_h = d.dil_w = 1
        d.pad_h = d.pad_w = K // 2
        d.bias, d.act = db.ptr, lib.ACT_RELU
        if res:
            d.residual = dr.ptr
        dy = lib.DeviceBuffer(B * H * W * OC * 2)
        d.y, d.tile = dy.ptr, -1
        lib.check(L.vdk_conv2d_ex(d, None))
        lib.check(L.vdk_synchronize())
        outs.append(dy.to_array(np.uint16, (B, H, W, OC)))
        return d
    run()
    lib.check(L.vdk_conv_set_autotune(1))
    try:
        d = run()
        run()
        t = L.vdk_conv_tuned_tile(d)
    finally:
        lib.check(L.vdk_conv_set_autotune(0))
    assert np.array_equal(outs[1], outs[0]) and np.array_equal(outs[2], outs[0])
    assert t >= 0 and L.vdk_conv2d_tile_fits_ex(t, d)
