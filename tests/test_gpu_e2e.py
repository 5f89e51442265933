"""End-to-end parity of the GPU path behind the C ABI against the oracle.

WeSpeaker ResNet34 with random-init f16 weights (folded BN), seeded synthetic
3 s clips: batch 64 (the throughput config) and batch 1 (the per-clip config).
Gates: FBank features within 1e-4, pooled statistics within 2e-3 relative
L2, embeddings at cosine >= 0.9999, identical verify verdicts; plus the
size-independent properties batch invariance and run-to-run determinism.
"""
import os
import tempfile

import numpy as np
import pytest

import pyoracle as O
from gpu_util import announce, check_every_clip, cosine, device_ok
from vdamd import gguf, lib, synth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not device_ok(), reason="no HIP device")]

N3S = 48000


@pytest.fixture(scope="module")
def resnet():
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "resnet34_f16.gguf")
    synth.write_resnet34(path, seed=2024)
    ctx = lib.Context(path)
    net = O.OracleResNet(gguf.GGUFFile(path))
    yield path, ctx, net
    ctx.close()


def test_resnet34_batch64_matches_oracle(resnet):
    path, ctx, net = resnet
    pcm = synth.clips(777, 64, N3S)
    announce("e2e resnet34 B=64 3s capture")
    cap = ctx.capture(pcm)
    check = [0, 21, 42, 63]
    ref = net.embed_batch(pcm[check], n_threads=4)
    for i, c in enumerate(check):
        feats = O.fbank(pcm[c])
        assert np.abs(cap["feats"][c] - feats).max() <= 1e-4
        emb, caps = net.forward(feats, capture=True)
        assert np.allclose(emb, ref[i], atol=1e-6)
        rel = np.linalg.norm(cap["pooled"][c] - caps["pooled"]) / np.linalg.norm(caps["pooled"])
        assert rel <= 2e-3, f"pooled rel-L2 {rel:.2e} clip {c}"
        assert cosine(cap["pre_norm"][c], caps["pre_norm"]) >= 0.9999
        cs = cosine(cap["emb"][c], emb)
        announce(f"clip {c}: cosine {cs:.7f} pooled rel {rel:.2e}")
        assert cs >= 0.9999
        assert abs(np.linalg.norm(cap["emb"][c]) - 1.0) < 1e-5
    check_every_clip(ctx, net, pcm, cap["emb"], "resnet34 B=64", invariance=(1, 32, 62))


def test_resnet34_batch1_embed_pcm_matches_oracle(resnet):
    path, ctx, net = resnet
    pcm = synth.clip(4242, N3S)
    announce("e2e resnet34 B=1 embed_pcm")
    got = ctx.embed_pcm(pcm)
    assert got.shape == (256,)
    assert cosine(got, net.forward(O.fbank(pcm))) >= 0.9999


def test_batch_invariance_and_determinism(resnet):
    path, ctx, net = resnet
    pcm = synth.clips(31, 16, N3S)
    announce("e2e determinism / batch invariance")
    a = ctx.embed_batch(pcm)
    b = ctx.embed_batch(pcm)
    assert np.array_equal(a, b)
    for c in (0, 9, 15):
        assert np.array_equal(ctx.embed_batch(pcm[c:c + 1])[0], a[c])
    # the device-resident path gives the same bits
    dp = lib.DeviceBuffer.from_array(pcm)
    do = lib.DeviceBuffer(16 * 256 * 4)
    ctx.embed_device_async(dp.ptr, 16, N3S, do.ptr)
    ctx.synchronize()
    assert np.array_equal(do.to_array(np.float32, (16, 256)), a)


def test_verify_fixture_wavs_same_verdict_as_oracle(resnet, golden_dir):
    path, ctx, net = resnet
    z = np.load(os.path.join(golden_dir, "fbank_golden.npz"))
    emb = {}
    for name in ("clip_a", "clip_b_same", "clip_c_diff"):
        wav = os.path.join(golden_dir, name + ".wav")
        got = ctx.embed_path(wav)
        ref = net.forward(O.fbank(z[f"wav_{name}/pcm"]))
        assert cosine(got, ref) >= 0.9999
        emb[name] = ref
    for a, b in (("clip_a", "clip_b_same"), ("clip_a", "clip_c_diff"), ("clip_b_same", "clip_c_diff")):
        thr = 0.25
        d_ref = 1.0 - float(np.dot(emb[a].astype(np.float64), emb[b].astype(np.float64)))
        d, ok = ctx.verify_paths(os.path.join(golden_dir, a + ".wav"), os.path.join(golden_dir, b + ".wav"), thr)
        assert abs(d - d_ref) <= 2e-3
        assert ok == (d_ref <= thr)
        # identical verdicts at thresholds just outside the 2e-3 distance tolerance band
        for t in (d_ref - 5e-3, d_ref + 5e-3):
            path_a, path_b = os.path.join(golden_dir, a + ".wav"), os.path.join(golden_dir, b + ".wav")
            assert ctx.verify_paths(path_a, path_b, t)[1] == (d_ref <= t)


def test_other_lengths_and_mean_vec():
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "small.gguf")
        synth.write_resnet34(path, seed=8, mean_vec=True)
        ctx = lib.Context(path)
        net = O.OracleResNet(gguf.GGUFFile(path))
        for n in (400, 4000, 64000):
            announce(f"e2e mean_vec model n={n}")
            pcm = synth.clips(n, 2, n)
            got = ctx.embed_batch(pcm)
            for c in range(2):
                assert cosine(got[c], net.forward(O.fbank(pcm[c]))) >= 0.9999
        # resampling path: 8 kHz input is resampled to 16 kHz before FBank
        x8 = synth.clip(5, 24000)
        x16 = np.zeros(48000, dtype=np.float32)
        n16 = lib.lib().vdk_resample_linear(x8.ctypes.data, len(x8), 8000, 16000, x16.ctypes.data, len(x16))
        assert n16 == 48000
        assert cosine(ctx.embed_pcm(x8, sample_rate=8000), net.forward(O.fbank(x16))) >= 0.9999
        ctx.close()


def test_autotuned_tiles_keep_the_bits(resnet):
    """The run-time tile tuner (vdk_conv_set_autotune) only ever picks a tile
    whose output equals the default's bit for bit: ResNet34 embeddings of a
    4-clip batch are the same with it on (first call: tuning, second: the
    cached choices) as with it off, and the tuner recorded a choice for a
    shape it handled."""
    path, ctx, net = resnet
    L = lib.lib()
    pcm = synth.clips(41, 4, N3S)
    announce("e2e autotune: reference pass")
    ref = ctx.embed_batch(pcm)
    lib.check(L.vdk_conv_set_autotune(1))
    try:
        announce("e2e autotune: tuning pass")
        a = ctx.embed_batch(pcm)
        b = ctx.embed_batch(pcm)
    finally:
        lib.check(L.vdk_conv_set_autotune(0))
    assert np.array_equal(a, ref) and np.array_equal(b, ref)
