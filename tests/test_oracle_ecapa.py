"""Pins the oracle's ECAPA-TDNN (oracle/oracle_ecapa.c, following src/encoder.cpp)
with an independent float64 numpy implementation of the same published
SpeechBrain structure: reflect padding via numpy's "reflect" mode (reflection
without repeating the edge sample, the rule of src/encoder.cpp:39-45),
Conv -> ReLU -> BN TDNN blocks, hierarchical Res2Net groups, SE gating, MFA,
attentive statistics pooling with global context (clamp, not add, 1e-12),
asp_bn, fc, L2."""
import os
import tempfile

import numpy as np

import pyoracle as O
from vdamd import gguf, synth


def _np_conv1d(x, w, b, dil):
    oc, ic, k = w.shape
    pad = (k - 1) // 2 * dil
    xp = np.pad(x, ((0, 0), (pad, pad)), mode="reflect") if pad else x
    T = x.shape[1]
    y = np.zeros((oc, T))
    for j in range(k):
        y += w[:, :, j] @ xp[:, j * dil: j * dil + T]
    return y + b[:, None]


def _np_bn(x, g, pre):
    s = g.array(pre + ".weight") / np.sqrt(g.array(pre + ".running_var").astype(np.float64) + 1e-5)
    return x * s[:, None] + (g.array(pre + ".bias") - s * g.array(pre + ".running_mean"))[:, None]


def _w(g, name):
    a = g.array(name).astype(np.float64)
    return a[:, :, None] if a.ndim == 2 else a


def _tdnn(g, pre, x, dil=1, conv="conv.conv", norm="norm.norm"):
    y = _np_conv1d(x, _w(g, f"{pre}.{conv}.weight"), g.array(f"{pre}.{conv}.bias"), dil)
    return _np_bn(np.maximum(y, 0.0), g, f"{pre}.{norm}")


def _np_ecapa(g, feats, scale, R):
    x = _tdnn(g, "blocks.0", feats.astype(np.float64))
    outs = [x]
    for i in range(1, R + 1):
        p = f"blocks.{i}"
        t1 = _tdnn(g, p + ".tdnn1", x)
        groups = np.split(t1, scale, axis=0)
        ys = [groups[0]]
        for j in range(1, scale):
            inp = groups[j] if j == 1 else groups[j] + ys[-1]
            ys.append(_tdnn(g, f"{p}.res2net_block.blocks.{j - 1}", inp, dil=i + 1))
        t2 = _tdnn(g, p + ".tdnn2", np.concatenate(ys, axis=0))
        s = t2.mean(axis=1, keepdims=True)
        s = np.maximum(_np_conv1d(s, _w(g, p + ".se_block.conv1.conv.weight"),
                                  g.array(p + ".se_block.conv1.conv.bias"), 1), 0.0)
        s = _np_conv1d(s, _w(g, p + ".se_block.conv2.conv.weight"), g.array(p + ".se_block.conv2.conv.bias"), 1)
        x = t2 * (1.0 / (1.0 + np.exp(-s))) + x
        outs.append(x)
    m = _tdnn(g, "mfa", np.concatenate(outs[1:], axis=0))
    T = m.shape[1]
    gm = m.mean(axis=1, keepdims=True)
    gs = np.sqrt(np.maximum(((m - gm) ** 2).mean(axis=1, keepdims=True), 1e-12))
    ctx = np.concatenate([m, np.repeat(gm, T, 1), np.repeat(gs, T, 1)], axis=0)
    a = np.tanh(_tdnn(g, "asp.tdnn", ctx))
    lg = _np_conv1d(a, _w(g, "asp.conv.conv.weight"), g.array("asp.conv.conv.bias"), 1)
    e = np.exp(lg - lg.max(axis=1, keepdims=True))
    att = e / e.sum(axis=1, keepdims=True)
    mu = (att * m).sum(axis=1)
    sd = np.sqrt(np.maximum((att * (m - mu[:, None]) ** 2).sum(axis=1), 1e-12))
    pooled = np.concatenate([mu, sd])
    nb = _np_bn(pooled[:, None], g, "asp_bn.norm")
    emb = _np_conv1d(nb, _w(g, "fc.conv.weight"), g.array("fc.conv.bias"), 1)[:, 0]
    return outs, m, pooled, emb, emb / np.linalg.norm(emb)


def test_ecapa_oracle_against_f64_numpy():
    rng = np.random.default_rng(12)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "tiny_ecapa.gguf")
        synth.write_ecapa(path, 9, channels=64, mfa=96, n_mels=24, scale=4, se_ch=16, att_ch=16, emb_dim=12,
                          n_res_blocks=3)
        g = gguf.GGUFFile(path)
        net = O.OracleEcapa(g)
        assert net.net.scale == 4 and net.net.n_res == 3
        feats = rng.standard_normal((24, 29)).astype(np.float32)
        emb, caps = net.forward(feats, capture=True)
        outs, m, pooled, pre, unit = _np_ecapa(g, feats, 4, 3)
        for i, o in enumerate(outs):
            got = caps[f"block{i}"]
            assert np.abs(got - o).max() <= 1e-4 * (1 + np.abs(o).max()), i
        assert np.allclose(caps["mfa"], m, rtol=1e-4, atol=1e-4)
        assert np.allclose(caps["pooled"], pooled, rtol=1e-4, atol=1e-4)
        assert np.allclose(caps["pre_norm"], pre, rtol=1e-4, atol=1e-4)
        assert np.allclose(emb, unit, atol=1e-5)


def test_conv1d_reflect_rule_and_dilation():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 11)).astype(np.float32)
    # one-hot taps read x[t + (j - (k-1)/2) * dil] with reflection at both ends
    for k, dil in ((3, 1), (3, 4), (5, 1), (5, 2)):
        pad = (k - 1) // 2 * dil
        xp = np.pad(x, ((0, 0), (pad, pad)), mode="reflect")
        for j in range(k):
            w = np.zeros((3, 3, k), dtype=np.float32)
            w[[0, 1, 2], [0, 1, 2], j] = 1.0
            y = O.conv1d_same(x, w, np.zeros(3, np.float32), dil)
            assert np.array_equal(y, xp[:, j * dil: j * dil + 11])
    # explicit reflect index rule of the reference: left pad-j, right (T-2)-(j-pad-T)
    T, pad = 11, 4
    idx = [pad - j if j < pad else (j - pad if j < pad + T else (T - 2) - (j - pad - T)) for j in range(T + 2 * pad)]
    assert idx == list(np.pad(np.arange(T), pad, mode="reflect"))
