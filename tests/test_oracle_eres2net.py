"""Pins the oracle's ERes2Net (oracle/oracle_eres2net.c, following
src/encoder_eres2net.cpp) with an independent float64 numpy implementation
written from the 3D-Speaker module semantics: BasicBlockERes2Net (conv1 ->
Hardtanh(0, 20), torch.split into width chunks, sp = sp + spx[i] or
AFF(sp, spx[i]) in the diff_AFF blocks, conv3 + shortcut -> Hardtanh), AFF as
x * (1 + tanh(z)) + ds * (1 - tanh(z)) (the module's own form, not the
reference's constant-free rewrite), the bottom-up cross-stage fusion, TSTP
with unbiased variance + 1e-8, seg_1, L2.  The conv weights are walked in
module order, so a manifest-order slip in the oracle fails here too."""
import os
import tempfile

import numpy as np
import pytest

import pyoracle as O
from vdamd import gguf, synth


def _conv(x, w, b, stride):
    """x [ic, H, W], w [oc, ic, k, k] (f64), zero pad (k-1)/2, stride on both axes."""
    oc, ic, kh, kw = w.shape
    _, H, W = x.shape
    p = (kh - 1) // 2
    xp = np.pad(x, ((0, 0), (p, p), (p, p)))
    Ho, Wo = (H + 2 * p - kh) // stride + 1, (W + 2 * p - kw) // stride + 1
    y = np.zeros((oc, Ho, Wo))
    for i in range(kh):
        for j in range(kw):
            y += np.einsum("oc,chw->ohw", w[:, :, i, j],
                           xp[:, i: i + (Ho - 1) * stride + 1: stride, j: j + (Wo - 1) * stride + 1: stride])
    return y if b is None else y + b[:, None, None]


class _Walk:
    def __init__(self, g):
        kv = g.kv
        self.w = [np.asarray(O._weight4(g, n), dtype=np.float64) for n in kv["voicedetect.eres2net.conv_weight"]]
        self.b = [np.asarray(g.array(n), dtype=np.float64) if n else None
                  for n in kv["voicedetect.eres2net.conv_bias"]]
        self.s = list(kv["voicedetect.eres2net.conv_stride"])
        self.i = 0

    def conv(self, x):
        y = _conv(x, self.w[self.i], self.b[self.i], self.s[self.i])
        self.i += 1
        return y


def _np_eres2net(g, feats):
    kv = g.kv
    walk = _Walk(g)
    ht = lambda v: np.clip(v, 0.0, 20.0)

    def aff(x, ds):
        z = walk.conv(np.concatenate([x, ds], axis=0))
        z = z / (1.0 + np.exp(-z))
        xa = 1.0 + np.tanh(walk.conv(z))
        return x * xa + ds * (2.0 - xa)

    def block(x, planes, stride, diff_aff, in_planes):
        out = ht(walk.conv(x))
        spx = np.split(out, 2, axis=0)
        outs = []
        sp = None
        for i in range(2):
            if i == 0:
                sp = spx[0]
            elif diff_aff:
                sp = aff(sp, spx[i])
            else:
                sp = sp + spx[i]
            sp = ht(walk.conv(sp))
            outs.append(sp)
        y = walk.conv(np.concatenate(outs, axis=0))
        res = walk.conv(x) if (stride != 1 or in_planes != 2 * planes) else x
        return ht(y + res)

    M = int(kv["voicedetect.eres2net.m_channels"])
    nb = list(kv["voicedetect.eres2net.num_blocks"])
    x = np.maximum(walk.conv(feats.astype(np.float64)[None]), 0.0)
    stem = x.copy()
    in_planes = M
    outs = []
    for li in range(4):
        planes = M * 2 ** li
        for bi in range(nb[li]):
            x = block(x, planes, (1 if li == 0 else 2) if bi == 0 else 1, li >= 2, in_planes)
            in_planes = 2 * planes
        outs.append(x)
        if li == 1:
            fused = aff(outs[1], walk.conv(outs[0]))
        elif li >= 2:
            fused = aff(outs[li], walk.conv(fused))
    assert walk.i == len(walk.w)
    C, H, W = fused.shape
    mean = fused.mean(axis=2)
    # unbiased variance; a single frame keeps the biased value 0 like the
    # reference (src/encoder_eres2net.cpp:233-236)
    var = fused.var(axis=2, ddof=1) if W > 1 else np.zeros_like(mean)
    std = np.sqrt(var + 1e-8)
    pooled = np.concatenate([mean.reshape(-1), std.reshape(-1)])
    sw = g.array("seg_1.weight").astype(np.float64)
    pre = sw @ pooled + g.array("seg_1.bias")
    return stem, fused, pooled, pre


@pytest.fixture(scope="module")
def tiny():
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "eres2net_tiny.gguf")
    synth.write_eres2net(path, seed=4, n_mels=16, m_ch=8, emb_dim=24, wtype=gguf.GGML_F32)
    g = gguf.GGUFFile(path)
    return g, O.OracleEres2net(g)


@pytest.mark.parametrize("T", [45, 8])
def test_eres2net_oracle_against_f64_numpy(tiny, T):
    g, net = tiny
    rng = np.random.default_rng(T)
    feats = rng.standard_normal((16, T)).astype(np.float32) * 2
    emb, caps = net.forward(feats, capture=True)
    stem, fused, pooled, pre = _np_eres2net(g, feats)
    tol = lambda ref: 2e-4 * (1 + np.abs(ref).max())
    assert np.abs(caps["stem"] - stem).max() <= tol(stem)
    assert np.abs(caps["fused"] - fused).max() <= tol(fused)
    assert np.abs(caps["pooled"] - pooled).max() <= tol(pooled)
    assert np.abs(caps["pre_norm"] - pre).max() <= tol(pre)
    assert np.allclose(emb, pre / np.linalg.norm(pre), atol=1e-5)


def test_eres2net_manifest_counts():
    """96 convs for num_blocks [3,4,6,3], scale 2 (the converter's check); the
    three cross-stage downsample convs are the only bias-free ones."""
    kv, _ = synth.make_eres2net(1, n_mels=16, m_ch=8, emb_dim=24)
    assert len(kv["voicedetect.eres2net.conv_weight"]) == 96
    assert sum(1 for b in kv["voicedetect.eres2net.conv_bias"] if b == "") == 3
    assert sum(1 for s in kv["voicedetect.eres2net.conv_stride"] if s == 2) == 3 * 2 + 3
