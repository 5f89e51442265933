"""Pins the oracle's CAM++ (oracle/oracle_campplus.c, following
src/encoder_campplus.cpp) with an independent float64 numpy implementation of
the published 3D-Speaker structure, written from the torch module semantics
rather than the oracle's loops:

* FCM: Conv2d with stride (freq, 1), residual blocks, then torch's
  reshape(B, C*H, T) (channel c*H + h);
* TDNN Conv1d k=5 stride 2 pad 2 (zero padding) via im2col;
* dense layers with the context mask computed from the DENSE time-mixing matrix
  Q[t', t] = 1/T' + [same 100-frame segment]/100 (the form the reference
  factorises, src/encoder_campplus.cpp:159-182), so the per-segment evaluation
  of the oracle and the count_include_pad rule for a partial last segment are
  both checked;
* transits, mean + unbiased std (no eps), dense head, affine-free BN, L2.
"""
import os
import tempfile

import numpy as np
import pytest

import pyoracle as O
from vdamd import gguf, synth


def _conv1d(x, w, b, stride=1, pad=0, dil=1):
    """x [ic, T], w [oc, ic, k] (f64), zero padding."""
    oc, ic, k = w.shape
    T = x.shape[1]
    xp = np.pad(x, ((0, 0), (pad, pad)))
    To = (T + 2 * pad - (k - 1) * dil - 1) // stride + 1
    cols = np.stack([xp[:, j * dil: j * dil + (To - 1) * stride + 1: stride] for j in range(k)], axis=1)
    y = np.einsum("oik,ikt->ot", w, cols)
    return y if b is None else y + b[:, None]


def _conv2d(x, w, b, sh, ph):
    """x [ic, H, T], w [oc, ic, kh, kw]; stride (sh, 1), pad (ph, ph)."""
    oc, ic, kh, kw = w.shape
    _, H, T = x.shape
    xp = np.pad(x, ((0, 0), (ph, ph), (ph, ph)))
    Ho = (H + 2 * ph - kh) // sh + 1
    y = np.zeros((oc, Ho, T))
    for i in range(kh):
        for j in range(kw):
            y += np.einsum("oc,cht->oht", w[:, :, i, j], xp[:, i: i + (Ho - 1) * sh + 1: sh, j: j + T])
    return y + b[:, None, None]


class _Net:
    def __init__(self, g):
        kv = g.kv
        self.g = g
        self.w = [np.asarray(O._weight4(g, n), dtype=np.float64) for n in kv["voicedetect.campplus.conv_weight"]]
        self.b = [np.asarray(g.array(n), dtype=np.float64) if n else None for n in kv["voicedetect.campplus.conv_bias"]]
        self.bn = kv["voicedetect.campplus.bn_prefix"]
        self.ci = 0
        self.bi = 0

    def conv(self):
        w, b = self.w[self.ci], self.b[self.ci]
        self.ci += 1
        return w, b

    def bn_relu(self, x):
        p = self.bn[self.bi]
        self.bi += 1
        g = self.g
        s = g.array(p + ".weight") / np.sqrt(g.array(p + ".running_var").astype(np.float64) + 1e-5)
        y = x * s[:, None] + (g.array(p + ".bias") - s * g.array(p + ".running_mean"))[:, None]
        return np.maximum(y, 0.0)


def _np_campplus(g, feats):
    n = _Net(g)
    relu = lambda v: np.maximum(v, 0.0)
    x = feats.astype(np.float64)[None]
    w, b = n.conv()
    x = relu(_conv2d(x, w, b, 1, 1))
    for stride in (2, 1, 2, 1):
        w1, b1 = n.conv()
        w2, b2 = n.conv()
        h = relu(_conv2d(x, w1, b1, stride, 1))
        h = _conv2d(h, w2, b2, 1, 1)
        if stride != 1:
            ws, bs = n.conv()
            sc = _conv2d(x, ws, bs, stride, 0)
        else:
            sc = x
        x = relu(h + sc)
    w, b = n.conv()
    x = relu(_conv2d(x, w, b, 2, 1))
    C, H, T = x.shape
    fcm = x.reshape(C * H, T)
    w, b = n.conv()
    h = relu(_conv1d(fcm, w[:, :, 0, :], b, stride=2, pad=2))
    tdnn = h.copy()
    Tp = h.shape[1]
    seg = np.arange(Tp) // 100
    Q = np.full((Tp, Tp), 1.0 / Tp) + (seg[:, None] == seg[None, :]) / 100.0   # Q[t', t]
    blocks = []
    for bi, (nl, dil) in enumerate(zip((12, 24, 16), (1, 2, 2))):
        for _ in range(nl):
            a = n.bn_relu(h)
            w1, b1 = n.conv()
            cc = relu(_conv1d(a, w1[:, :, 0, :], b1))
            wl, bl = n.conv()
            y = _conv1d(cc, wl[:, :, 0, :], bl, pad=dil, dil=dil)
            ctx = cc @ Q.T                                  # ctx[c, t'] = sum_t Q[t', t] cc[c, t]
            wc1, bc1 = n.conv()
            wc2, bc2 = n.conv()
            m = relu(_conv1d(ctx, wc1[:, :, 0, :], bc1))
            m = 1.0 / (1.0 + np.exp(-_conv1d(m, wc2[:, :, 0, :], bc2)))
            h = np.concatenate([h, y * m], axis=0)
        wt, bt = n.conv()
        h = _conv1d(n.bn_relu(h), wt[:, :, 0, :], bt)
        if bi == 2:
            h = relu(h)
        blocks.append(h)
    mean = h.mean(axis=1)
    std = np.sqrt(h.var(axis=1, ddof=1)) if Tp > 1 else np.zeros_like(mean)
    pooled = np.concatenate([mean, std])
    wd, bd = n.conv()
    e = wd[:, :, 0, 0] @ pooled + (0 if bd is None else bd)
    kv = g.kv
    mu = g.array(kv["voicedetect.campplus.emb_bn_mean"]).astype(np.float64)
    var = g.array(kv["voicedetect.campplus.emb_bn_var"]).astype(np.float64)
    pre = (e - mu) / np.sqrt(var + 1e-5)
    assert n.ci == len(n.w) and n.bi == len(n.bn)
    return fcm, tdnn, blocks, pooled, pre


@pytest.fixture(scope="module")
def tiny():
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "campplus_tiny.gguf")
    synth.write_campplus(path, seed=3, n_mels=16, m_ch=8, init_ch=32, growth=8, bn_ch=32, emb_dim=12,
                         wtype=gguf.GGML_F32)
    g = gguf.GGUFFile(path)
    return g, O.OracleCampplus(g)


@pytest.mark.parametrize("T", [259, 41])
def test_campplus_oracle_against_f64_numpy(tiny, T):
    g, net = tiny
    rng = np.random.default_rng(T)
    feats = rng.standard_normal((16, T)).astype(np.float32) * 2
    emb, caps = net.forward(feats, capture=True)
    fcm, tdnn, blocks, pooled, pre = _np_campplus(g, feats)
    tol = lambda ref: 2e-4 * (1 + np.abs(ref).max())
    assert np.abs(caps["fcm"] - fcm).max() <= tol(fcm)
    assert np.abs(caps["tdnn"] - tdnn).max() <= tol(tdnn)
    for b in range(3):
        assert np.abs(caps[f"block{b}"] - blocks[b]).max() <= tol(blocks[b]), b
    assert np.abs(caps["pooled"] - pooled).max() <= tol(pooled)
    assert np.abs(caps["pre_norm"] - pre).max() <= tol(pre)
    assert np.allclose(emb, pre / np.linalg.norm(pre), atol=1e-5)


def test_campplus_manifest_counts():
    """225 convs and 55 affine BNs for the standard topology (the converter's check)."""
    kv, tensors = synth.make_campplus(1, n_mels=16, m_ch=8, init_ch=32, growth=8, bn_ch=32, emb_dim=12)
    assert len(kv["voicedetect.campplus.conv_weight"]) == 225
    assert len(kv["voicedetect.campplus.bn_prefix"]) == 55
    assert sum(1 for b in kv["voicedetect.campplus.conv_bias"] if b == "") == 52 + 2 + 1
