"""Pins the oracle's ResNet34 wiring (src/encoder_resnet.cpp:94-185) with an
independent float64 composition: f64 brute-force convs, numpy statistics
pooling (C-outer/H-inner flatten, unbiased std + eps), numpy FC and L2.
A wrong stride, shortcut, flatten order or eps placement fails here."""
import os
import tempfile

import numpy as np

import pyoracle as O
from vdamd import gguf, synth


def _tiny_model(tmp, mean_vec):
    path = os.path.join(tmp, "tiny.gguf")
    kv, tensors = synth.make_resnet34(11, wtype=gguf.GGML_F32, channels=(4, 8, 8, 16),
                                      blocks=(2, 1, 2, 1), emb_dim=12, n_mels=24, mean_vec=mean_vec)
    gguf.write_gguf(path, kv, tensors)
    return gguf.GGUFFile(path)


def _f64_forward(g, feats):
    kv = g.kv
    p = "voicedetect.resnet."
    A = lambda n: g.array(n).astype(np.float32)  # noqa: E731
    x = O.conv2d(feats[None], A(kv[p + "stem_weight"]), 1, 1, bias=A(kv[p + "stem_bias"]), relu=True, f64=True)
    for i in range(len(kv[p + "conv1_weight"])):
        s = kv[p + "stride"][i]
        xf = x.astype(np.float32)
        h = O.conv2d(xf, A(kv[p + "conv1_weight"][i]), s, 1, bias=A(kv[p + "conv1_bias"][i]), relu=True, f64=True)
        if kv[p + "down_weight"][i]:
            sc = O.conv2d(xf, A(kv[p + "down_weight"][i]), s, 0, bias=A(kv[p + "down_bias"][i]), f64=True)
        else:
            sc = x
        y = O.conv2d(h.astype(np.float32), A(kv[p + "conv2_weight"][i]), 1, 1, bias=A(kv[p + "conv2_bias"][i]),
                     f64=True)
        x = np.maximum(y + sc, 0.0)
    mean = x.mean(axis=2).reshape(-1)
    std = np.sqrt(x.var(axis=2, ddof=1) + kv[p + "var_eps"]).reshape(-1)
    pooled = np.concatenate([mean, std])
    emb = A(kv[p + "seg_weight"]).astype(np.float64) @ pooled + A(kv[p + "seg_bias"])
    if kv[p + "mean_vec"]:
        emb = emb - A(kv[p + "mean_vec"])
    return pooled, emb, emb / np.linalg.norm(emb)


def test_resnet_wiring_against_f64_composition():
    rng = np.random.default_rng(8)
    for mean_vec in (False, True):
        with tempfile.TemporaryDirectory() as tmp:
            g = _tiny_model(tmp, mean_vec)
            net = O.OracleResNet(g)
            feats = rng.standard_normal((24, 37)).astype(np.float32)
            emb, caps = net.forward(feats, capture=True)
            pooled, pre, unit = _f64_forward(g, feats)
            assert caps["pooled"].shape == pooled.shape
            assert np.allclose(caps["pooled"], pooled, rtol=1e-4, atol=1e-4)
            assert np.allclose(caps["pre_norm"], pre, rtol=1e-4, atol=1e-4)
            assert np.allclose(emb, unit, atol=1e-5)


def test_block_shapes_follow_strides():
    with tempfile.TemporaryDirectory() as tmp:
        net = O.OracleResNet(_tiny_model(tmp, False))
        assert net.block_shapes(37)[-1] == (16, 3, 5)
        full = synth.resnet34_spec()
        assert len(full) == 16 and sum(1 for b in full if b[3]) == 3
