"""numpy (f64) restatement of the reference's wav2vec2 analyze path.

TEST INFRASTRUCTURE ONLY: imported by the test suite, the smoke check and the
CPU-baseline leg of bench.py.  Results are compared against it; it is never
the thing measured.

Follows src/analyze_w2v2.cpp of the reference, function by function:
  conv feature encoder      build_conv_encoder        :52-131 (conv1d_strided :34-45)
  feature projection        build_transformer_states  :381-392 (layer_norm :187-193, linear :196-201)
  positional conv embedding positional_conv           :280-326, weights :333-359
  transformer stack         build_transformer_states  :398-468, self_attention :222-270
  emotion head              emotion_logits            :503-558, analyze_json :561-594
  age/gender head           age_gender_raw            :596-630, analyze_age_gender_json :632-668
The reference builds ggml graphs in f32; this restatement computes in f64.
Activations are returned time-major ([T', C]), the layout of the GPU path.

Pinned by tests/test_oracle_w2v2.py against HF transformers' Wav2Vec2 modules
run in f64 on the same weights (the library the reference's golden tensors
come from), and by closed forms (GroupNorm / LayerNorm moments, weight-norm row
norms, attention over identical keys).
"""
import numpy as np
from scipy.special import erf

import os
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "voice-detect.cpp_amd"))
from vdamd import gguf as G  # noqa: E402

WAVE_NORM_EPS = 1e-7    # src/analyze_w2v2.cpp:63-70 (do_normalize)
GROUP_NORM_EPS = 1e-5   # src/analyze_w2v2.cpp:57-60


def gelu(x):
    """Exact erf GELU (src/analyze_w2v2.cpp:126-128)."""
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def layer_norm(x, g, b, eps):
    """LayerNorm over the last axis, biased variance (src/analyze_w2v2.cpp:187-193)."""
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def conv1d_strided(x, w, stride, pad=0):
    """x [T, IC] time-major, w [OC, IC, K] -> [OL, OC], OL = (T + 2 pad - K) / stride + 1
    (src/analyze_w2v2.cpp:34-45: im2col + mul_mat, no bias)."""
    OC, IC, K = w.shape
    if pad:
        x = np.concatenate([np.zeros((pad, IC)), x, np.zeros((pad, IC))], axis=0)
    T = x.shape[0]
    OL = (T - K) // stride + 1
    cols = np.lib.stride_tricks.sliding_window_view(x, K, axis=0)[: (OL - 1) * stride + 1: stride]   # [OL, IC, K]
    return np.tensordot(cols, w, axes=([1, 2], [1, 2]))   # [OL, OC]


def softmax(v):
    v = np.asarray(v, dtype=np.float64)
    e = np.exp(v - v.max())
    return e / e.sum()


class OracleW2V2:
    """A wav2vec2 analyze GGUF (arch wav2vec2_emotion / wav2vec2_age_gender)."""

    def __init__(self, path):
        g = G.GGUFFile(path)
        kv = g.kv
        self.arch = kv["voicedetect.arch"]
        p = "voicedetect.w2v2."
        self.hidden = int(kv[p + "hidden_size"])
        self.n_layers = int(kv[p + "n_layers"])
        self.n_heads = int(kv[p + "n_heads"])
        self.ff = int(kv[p + "ff_dim"])
        self.conv_dims = [int(v) for v in kv[p + "conv_dims"]]
        self.kernels = [int(v) for v in kv[p + "conv_kernels"]]
        self.strides = [int(v) for v in kv[p + "conv_strides"]]
        self.norm = kv[p + "feat_extract_norm"]
        self.conv_bias = bool(kv.get(p + "conv_bias", False))
        self.do_normalize = bool(kv.get(p + "do_normalize", False))
        self.stable = bool(kv.get(p + "do_stable_layer_norm", False))
        self.eps = float(kv.get(p + "layer_norm_eps", 1e-5))
        self.pos_k = int(kv[p + "num_conv_pos_embeddings"])
        self.pos_groups = int(kv[p + "num_conv_pos_embedding_groups"])
        self.weighted = bool(kv.get(p + "use_weighted_layer_sum", False))
        self.emotion_labels = list(kv.get("voicedetect.analyze.emotion_labels", []))
        self.gender_labels = list(kv.get("voicedetect.analyze.gender_labels", []))
        self.W = {name: g.array(name).astype(np.float64) for name in g.tensors}

    def w(self, name):
        return self.W[name]

    def frames(self, n):
        """T' of the conv stack for n samples (0 when too short)."""
        t = n
        for k, s in zip(self.kernels, self.strides):
            if t < k:
                return 0
            t = (t - k) // s + 1
        return t

    # -- conv feature encoder (src/analyze_w2v2.cpp:52-131) ---------------------
    def conv_encoder(self, pcm):
        x = np.asarray(pcm, dtype=np.float64)
        if self.do_normalize:   # :68-70, biased variance, eps 1e-7
            x = (x - x.mean()) / np.sqrt(x.var() + WAVE_NORM_EPS)
        h = x[:, None]          # [L, IC=1]
        for i, (k, s) in enumerate(zip(self.kernels, self.strides)):
            pre = f"w2v2.feature_extractor.conv_layers.{i}"
            y = conv1d_strided(h, self.w(pre + ".conv.weight"), s)
            if self.conv_bias:
                y = y + self.w(pre + ".conv.bias")
            if self.norm == "group" and i == 0:   # :99-104: per channel over time
                mu = y.mean(axis=0, keepdims=True)
                var = ((y - mu) ** 2).mean(axis=0, keepdims=True)
                y = (y - mu) / np.sqrt(var + GROUP_NORM_EPS) * self.w(pre + ".layer_norm.weight") + \
                    self.w(pre + ".layer_norm.bias")
            elif self.norm == "layer":            # :105-124: per frame over channels
                y = layer_norm(y, self.w(pre + ".layer_norm.weight"), self.w(pre + ".layer_norm.bias"), self.eps)
            h = gelu(y)
        return h   # [T', conv_dim]

    # -- positional conv embedding (src/analyze_w2v2.cpp:280-326, 333-359) ------
    def pos_conv_weight(self):
        """w[oc, ic, k] = g[k] v[oc, ic, k] / ||v[:, :, k]|| (norm over oc and ic)."""
        v = self.w("w2v2.encoder.pos_conv_embed.conv.weight_v")   # [H, H/groups, K]
        g = self.w("w2v2.encoder.pos_conv_embed.conv.weight_g").reshape(-1)   # [K]
        norm = np.sqrt((v * v).sum(axis=(0, 1)))
        s = np.where(norm > 0, g / np.where(norm > 0, norm, 1.0), 0.0)
        return v * s[None, None, :]

    def pos_conv(self, proj):
        """proj [T, H] -> gelu(grouped conv(pad K/2) + b) with the last step dropped for even K."""
        T, H = proj.shape
        K, groups = self.pos_k, self.pos_groups
        icg = H // groups
        w = self.pos_conv_weight()
        out = np.concatenate([conv1d_strided(proj[:, g * icg:(g + 1) * icg], w[g * icg:(g + 1) * icg], 1, K // 2)
                              for g in range(groups)], axis=1)
        out = out + self.w("w2v2.encoder.pos_conv_embed.conv.bias")
        if K % 2 == 0:
            out = out[:-1]
        return gelu(out)

    # -- transformer (src/analyze_w2v2.cpp:222-270, 370-468) --------------------
    def linear(self, x, name):
        return x @ self.w(name + ".weight").T + self.w(name + ".bias")

    def attention(self, h, pre):
        T, H = h.shape
        nh = self.n_heads
        hd = H // nh
        q = self.linear(h, pre + ".q_proj").reshape(T, nh, hd).transpose(1, 0, 2)
        k = self.linear(h, pre + ".k_proj").reshape(T, nh, hd).transpose(1, 0, 2)
        v = self.linear(h, pre + ".v_proj").reshape(T, nh, hd).transpose(1, 0, 2)
        s = (q @ k.transpose(0, 2, 1)) / np.sqrt(hd)              # [nh, Tq, Tk]
        s = np.exp(s - s.max(axis=-1, keepdims=True))
        p = s / s.sum(axis=-1, keepdims=True)
        o = (p @ v).transpose(1, 0, 2).reshape(T, H)
        return self.linear(o, pre + ".out_proj")

    def feed_forward(self, h, pre):
        f = gelu(self.linear(h, pre + ".feed_forward.intermediate_dense"))
        return self.linear(f, pre + ".feed_forward.output_dense")

    def ln(self, x, name):
        return layer_norm(x, self.w(name + ".weight"), self.w(name + ".bias"), self.eps)

    def hidden_states(self, pcm):
        """All n_layers + 1 hidden states [T', H] in HF's output_hidden_states order."""
        feat = self.conv_encoder(pcm)
        h = self.ln(feat, "w2v2.feature_projection.layer_norm")
        proj = self.linear(h, "w2v2.feature_projection.projection")
        hs = proj + self.pos_conv(proj)
        states = []
        if self.stable:   # :398-427: pre-norm layers, one final LayerNorm
            states.append(hs)
            for i in range(self.n_layers):
                pre = f"w2v2.encoder.layers.{i}"
                hs = hs + self.attention(self.ln(hs, pre + ".layer_norm"), pre + ".attention")
                hs = hs + self.feed_forward(self.ln(hs, pre + ".final_layer_norm"), pre)
                if i < self.n_layers - 1:
                    states.append(hs)
            states.append(self.ln(hs, "w2v2.encoder.layer_norm"))
            return states
        hs = self.ln(hs, "w2v2.encoder.layer_norm")   # :429-468: post-norm
        states.append(hs)
        for i in range(self.n_layers):
            pre = f"w2v2.encoder.layers.{i}"
            hs = self.ln(hs + self.attention(hs, pre + ".attention"), pre + ".layer_norm")
            hs = self.ln(hs + self.feed_forward(hs, pre), pre + ".final_layer_norm")
            states.append(hs)
        return states

    # -- heads ------------------------------------------------------------------
    def layer_weights(self):
        """softmax(layer_weights) when the weighted layer sum is on (:511-521), else None."""
        if not self.weighted or "layer_weights" not in self.W:
            return None
        return softmax(self.w("layer_weights").reshape(-1))

    def raw_outputs(self, pcm):
        """Emotion logits [N], or [age_raw, gender logits...] for the age/gender arch."""
        states = self.hidden_states(pcm)
        if self.arch == "wav2vec2_age_gender":   # :596-630
            pooled = states[-1].mean(axis=0)

            def head(name):
                return self.linear(np.tanh(self.linear(pooled, name + ".dense")), name + ".out_proj")
            return np.concatenate([head("age"), head("gender")])
        lw = self.layer_weights()                # :528-558
        hs = sum(wi * s for wi, s in zip(lw, states)) if lw is not None and len(lw) == len(states) else states[-1]
        proj = self.linear(hs, "projector")
        return self.linear(proj.mean(axis=0), "classifier")

    def analyze_json(self, pcm):
        """The reference's analyze JSON for one clip (:561-594, :632-668)."""
        raw = self.raw_outputs(pcm)
        return format_json(self.arch, raw, self.emotion_labels, self.gender_labels)


def _fnum(x):
    return "%.6g" % x


def probs_f32(logits):
    """The reference's host softmax (:566-575): e_i = (float)exp((double)l_i - max),
    s = sum of the rounded e_i in double, p_i = (float)(e_i / s)."""
    l = np.asarray(logits, dtype=np.float32)
    if l.size == 0:
        return l
    e = np.exp(l.astype(np.float64) - float(l.max())).astype(np.float32)
    s = float(np.sum(e.astype(np.float64)))
    return (e.astype(np.float64) / s).astype(np.float32)


def format_json(arch, raw, emotion_labels, gender_labels):
    """JSON text from the raw f32 head outputs (first maximum wins the argmax)."""
    raw = np.asarray(raw, dtype=np.float32)
    if arch == "wav2vec2_age_gender":
        age = float(raw[0]) * 100.0 if raw.size else 0.0
        logits = raw[1:]
        probs = probs_f32(logits)
        am = int(np.argmax(logits)) if logits.size else 0
        dom = gender_labels[am] if am < len(gender_labels) else ""
        js = '{"age":' + _fnum(age) + ',"gender":{"label":"' + dom + '"'
        for i, lab in enumerate(gender_labels):
            js += ',"' + lab + '":' + _fnum(float(probs[i]) if i < probs.size else 0.0)
        return js + "}}"
    probs = probs_f32(raw)
    am = int(np.argmax(raw)) if raw.size else 0
    dom = emotion_labels[am] if am < len(emotion_labels) else ""
    js = '{"emotion":{"label":"' + dom + '","scores":{'
    js += ",".join('"' + lab + '":' + _fnum(float(probs[i]) if i < probs.size else 0.0)
                   for i, lab in enumerate(emotion_labels))
    return js + "}}}"
