"""Registry scoring / identify on the GPU (vdk_registry_topk and the
voicedetect_gpu_identify_* entry points) against the oracle's registry_topk.

The GPU forms each f32 x f32 product exactly in f64 and sums in f64, as the
oracle does, so the ranking must match exactly (rows tie only when their
scores are equal, and then the lower row comes first) and the f32 scores to
within one f32 rounding of the f64 value.
"""
import os
import tempfile
import zlib

import numpy as np
import pytest

import pyoracle as O
from gpu_util import announce, device_ok
from vdamd import lib, synth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not device_ok(), reason="no HIP device")]


def _unit(rng, n, d):
    x = rng.standard_normal((n, d)).astype(np.float32)
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


def topk_gpu(q, reg, k):
    L = lib.lib()
    B, D = q.shape
    N = reg.shape[0]
    dq, dr = lib.DeviceBuffer.from_array(q), lib.DeviceBuffer.from_array(reg)
    ws = L.vdk_registry_topk_workspace_size(B, N, k)
    dw = lib.DeviceBuffer(ws)
    di, ds = lib.DeviceBuffer(B * k * 4), lib.DeviceBuffer(B * k * 4)
    lib.check(L.vdk_registry_topk(dq.ptr, B, dr.ptr, N, D, k, dw.ptr, ws, di.ptr, ds.ptr, None))
    lib.check(L.vdk_synchronize())
    return di.to_array(np.int32, (B, k)), ds.to_array(np.float32, (B, k))


def _check(q, reg, k):
    gi, gs = topk_gpu(q, reg, k)
    oi, os_ = O.registry_topk(q, reg, k)
    bad = np.argwhere(gi != oi)
    assert bad.size == 0, f"{len(bad)} ranks differ, first at {bad[0].tolist()}: gpu {gi[tuple(bad[0])]} " \
                          f"oracle {oi[tuple(bad[0])]}"
    assert np.all(np.abs(gs.astype(np.float64) - os_) <= 6e-8 * np.maximum(1.0, np.abs(os_)))


@pytest.mark.parametrize("case", [
    # (B, N, D, k): partial 64-row tiles, B over one 64-query tile, k = 1 / 64 / N
    (5, 1000, 256, 10),
    (70, 3001, 192, 64),
    (1, 64, 512, 1),
    (3, 7, 256, 7),
    (64, 100000, 256, 10),
    (2, 40000, 192, 64),     # 157 x 64 candidates per query: the merge scans them in global memory
])
def test_registry_topk_matches_oracle(case):
    B, N, D, k = case
    announce(f"registry_topk B={B} N={N} D={D} k={k}")
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    _check(_unit(rng, B, D), _unit(rng, N, D), k)


def test_registry_topk_ties_and_self_match():
    rng = np.random.default_rng(11)
    reg = _unit(rng, 300, 256)
    reg[200] = reg[3]                   # a duplicate row ties with row 3
    reg[250:260] = reg[120]             # ten copies of row 120
    q = reg[[3, 120, 299, 0]].copy()
    announce("registry_topk ties")
    gi, gs = topk_gpu(q, reg, 12)
    assert gi[0, 0] == 3 and gi[0, 1] == 200 and gs[0, 0] == gs[0, 1]
    assert gi[1, :11].tolist() == [120] + list(range(250, 260))
    assert gi[2, 0] == 299 and gi[3, 0] == 0
    _check(q, reg, 12)


def test_registry_topk_rejects_bad_arguments():
    L = lib.lib()
    d = lib.DeviceBuffer(1 << 16)
    assert L.vdk_registry_topk(d.ptr, 1, d.ptr, 5, 8, 6, d.ptr, 1 << 16, d.ptr, d.ptr, None) != 0
    assert "exceeds the registry" in L.vdk_last_error().decode()
    assert L.vdk_registry_topk(d.ptr, 1, d.ptr, 500, 8, 65, d.ptr, 1 << 16, d.ptr, d.ptr, None) != 0
    assert "1..64" in L.vdk_last_error().decode()
    assert L.vdk_registry_topk(d.ptr, 64, d.ptr, 10000, 8, 10, d.ptr, 64, d.ptr, d.ptr, None) != 0
    assert "workspace" in L.vdk_last_error().decode()
    assert L.vdk_registry_topk(d.ptr, 1, d.ptr, 500, 6, 5, d.ptr, 1 << 16, d.ptr, d.ptr, None) != 0
    assert "multiple of 4" in L.vdk_last_error().decode()


def test_identify_pcm_end_to_end():
    """Enrol GPU embeddings of three clips among random rows, identify the clips
    from PCM: each is its own best match, and the whole ranking matches the
    oracle on the same embeddings."""
    path = os.path.join(tempfile.mkdtemp(), "resnet34.gguf")
    synth.write_resnet34(path, seed=2024)
    ctx = lib.Context(path)
    try:
        pcm = synth.clips(77, 3, 48000)
        emb = ctx.embed_batch(pcm)
        rng = np.random.default_rng(21)
        reg = _unit(rng, 500, ctx.dim)
        rows = [5, 17, 42]
        reg[rows] = emb
        ctx.registry_set(reg)
        announce("identify_pcm 3 clips vs 500 rows")
        idx, score = ctx.identify_pcm(pcm, 8)
        assert idx[:, 0].tolist() == rows
        assert np.all(np.abs(score[:, 0] - 1.0) < 1e-5)
        oi, os_ = O.registry_topk(emb, reg, 8)
        assert np.array_equal(idx, oi)
        assert np.all(np.abs(score.astype(np.float64) - os_) <= 6e-8 * np.maximum(1.0, np.abs(os_)))
        # distance = 1 - score is verify's distance for the best pair
        d, ok = ctx.verify_pcm(pcm[0], pcm[0], 0.5)
        assert abs(d) < 1e-5 and ok
        with pytest.raises(lib.VdkError, match="k must be"):
            ctx.identify_pcm(pcm, 65)
        ctx.registry_set(np.zeros((0, ctx.dim), dtype=np.float32))
        with pytest.raises(lib.VdkError, match="no registry"):
            ctx.identify_pcm(pcm, 1)
        assert ctx.L.voicedetect_gpu_registry_set(ctx.ctx, reg.ctypes.data, 10, ctx.dim + 1) != 0
        assert "registry dim" in ctx.last_error()
    finally:
        ctx.close()
