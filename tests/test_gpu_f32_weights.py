"""End to end with F32 conv weights that f16 does not hold exactly.

The reference converter keeps k > 1 conv weights F32 (and, unquantised, the
1x1 ones too); the GPU path stores them as f16 MFMA operands (ERes2Net as
split-f16 hi + lo, exact to ~2^-22).  These models carry full-precision F32
weights, so the gates below measure that weight rounding against the oracle,
which computes with the f32 weights: pooled statistics within 2e-3 relative
L2 and embeddings at cosine >= 0.9999, the gates of the f16-exact models.
"""
import os
import tempfile

import numpy as np
import pytest

import pyoracle as O
from gpu_util import announce, cosine, device_ok
from vdamd import gguf, lib, synth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not device_ok(), reason="no HIP device")]


def _check(ctx, net, pcm, clips, tag):
    cap = ctx.capture(pcm)
    for c in clips:
        feats = O.fbank(pcm[c])
        emb, caps = net.forward(feats, capture=True)
        rel = np.linalg.norm(cap["pooled"][c] - caps["pooled"]) / np.linalg.norm(caps["pooled"])
        cs = cosine(cap["emb"][c], emb)
        announce(f"{tag} clip {c}: cosine {cs:.7f} pooled rel {rel:.2e}")
        assert rel <= 2e-3, f"{tag} pooled rel-L2 {rel:.2e} clip {c}"
        assert cs >= 0.9999


def _model(write, name, **kw):
    path = os.path.join(tempfile.mkdtemp(), name)
    write(path, **kw)
    g = gguf.GGUFFile(path)
    # at least one F32 conv weight that f16 does not represent
    assert any(v[0] == gguf.GGML_F32 and len(v[1]) >= 3 and
               not np.array_equal(g.array(k), g.array(k).astype(np.float16).astype(np.float32))
               for k, v in g.tensors.items())
    return path, g


def test_resnet34_f32_weights():
    path, g = _model(synth.write_resnet34, "resnet34_f32.gguf", seed=61, wtype=gguf.GGML_F32)
    announce("f32 weights: resnet34 B=8 3s")
    ctx = lib.Context(path)
    _check(ctx, O.OracleResNet(g), synth.clips(610, 8, 48000), (0, 7), "resnet34 f32")
    ctx.close()


def test_ecapa_f32_weights():
    path, g = _model(synth.write_ecapa, "ecapa_f32.gguf", seed=62, wtype=gguf.GGML_F32, f16_exact=False)
    announce("f32 weights: ecapa B=4 4s")
    ctx = lib.Context(path)
    _check(ctx, O.OracleEcapa(g), synth.clips(620, 4, 64000), (0, 3), "ecapa f32")
    ctx.close()


def test_campplus_f32_weights():
    path, g = _model(synth.write_campplus, "campplus_f32.gguf", seed=63, wtype=gguf.GGML_F32, f16_exact=False)
    announce("f32 weights: campplus B=2 4s")
    ctx = lib.Context(path)
    _check(ctx, O.OracleCampplus(g), synth.clips(630, 2, 64000), (0, 1), "campplus f32")
    ctx.close()


def test_eres2net_f32_weights():
    path, g = _model(synth.write_eres2net, "eres2net_f32.gguf", seed=64, wtype=gguf.GGML_F32, f16_exact=False)
    announce("f32 weights: eres2net B=2 3s")
    ctx = lib.Context(path)
    _check(ctx, O.OracleEres2net(g), synth.clips(640, 2, 48000), (0, 1), "eres2net f32")
    ctx.close()
