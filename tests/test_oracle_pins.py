"""Closed-form pins of the oracle's ECAPA and ResNet34 composition.

Each check drives the oracle (oracle/oracle_ecapa.c, oracle/oracle.c) with
weights chosen so that the reference's layer rules reduce to a formula that
can be written down without restating them:

* attentive statistics pooling (src/encoder.cpp:262-295): logits constant in
  time give uniform attention, so the pooled pair is the plain mean and
  sqrt(clamp(biased variance, 1e-12)); one dominant logit picks one frame
  (mean = that frame, std = sqrt(1e-12)); and the global context
  [x ; mean ; std] (biased std, clamped) decides, through a threshold built
  into the attention TDNN, whether attention is one-hot or uniform;
* SE-Res2Net blocks (src/encoder.cpp:174-244) with identity 1x1 convs,
  centre-tap identity group convs and identity BatchNorms on non-negative
  input: group 0 passes through, group j >= 1 is the prefix sum
  x_1 + ... + x_j, and the block output is t2 * sigmoid(gate) + x with the
  gate read from the time mean of one chosen channel;
* the ResNet BasicBlock (src/encoder_resnet.cpp:37-48): centre-tap identity
  convs give relu(2x + b2), a zero conv2 gives relu(b2 + shortcut), and a
  strided 1x1 channel map in the downsample gives relu(b2 + bd + k x[::2, ::2]).

The mutation tests then compile copies of the oracle sources with one
plausible misreading each (softmax over channels, eps added instead of
clamped, variance about 0, unbiased global std, Res2Net chain through group 0,
SE gate on the sum, SE squeeze of the block input, ReLU before the residual
add, swapped global-context channels) and require that a pin fails on every
copy.
"""
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

import pyoracle as O
from vdamd import gguf, synth

ORACLE_DIR = os.path.dirname(os.path.abspath(O.__file__))
F32 = np.float32
BN_UNIT = np.sqrt(F32(1.0) + F32(1e-5))   # gamma with gamma / sqrt(1 + eps) == 1 in f32
SQRT_EPS = float(np.sqrt(F32(1e-12)))


def _set(tensors, name, arr):
    """Replace tensor `name` by an f32 tensor of the same stored shape."""
    for i, (n, _t, shape, _a) in enumerate(tensors):
        if n == name:
            a = np.asarray(arr, dtype=F32).reshape(shape)
            tensors[i] = (n, gguf.GGML_F32, list(shape), a)
            return
    raise KeyError(name)


def _unit_bn(tensors, prefix, c):
    _set(tensors, prefix + ".weight", np.full(c, BN_UNIT, F32))
    _set(tensors, prefix + ".bias", np.zeros(c, F32))
    _set(tensors, prefix + ".running_mean", np.zeros(c, F32))
    _set(tensors, prefix + ".running_var", np.ones(c, F32))


def _load(tmp, name, kv, tensors):
    path = os.path.join(tmp, name)
    gguf.write_gguf(path, kv, tensors)
    return gguf.GGUFFile(path)


# ------------------------------------------------------------------ ECAPA ASP

M, A = 8, 4    # MFA channels, attention channels of the tiny ECAPA


def _tiny_ecapa():
    return synth.make_ecapa(5, channels=16, mfa=M, n_mels=6, scale=4, se_ch=4, att_ch=A, emb_dim=4,
                            n_res_blocks=3, wtype=gguf.GGML_F32)


def _asp(tensors_fn, x):
    kv, tensors = _tiny_ecapa()
    tensors_fn(tensors)
    with tempfile.TemporaryDirectory() as tmp:
        net = O.OracleEcapa(_load(tmp, "ecapa.gguf", kv, tensors))
        out = O.ecapa_asp(net, np.ascontiguousarray(x, dtype=F32))
    return out[:M].astype(np.float64), out[M:].astype(np.float64)


def check_asp_uniform_attention():
    """asp.conv weights zero, per-channel biases: softmax over time is uniform."""
    def edit(t):
        _set(t, "asp.conv.conv.weight", np.zeros((M, A, 1)))
        _set(t, "asp.conv.conv.bias", np.linspace(-3.0, 3.0, M))
    T = 8
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((M, T)) + np.linspace(-2.0, 2.0, M)[:, None]).astype(F32)
    # channels 0-2: +-a about 0 (biased variance a^2 near or below the 1e-12 clamp)
    for c, a in enumerate((1e-7, 5e-7, 2e-6)):
        x[c] = F32(a) * np.where(np.arange(T) % 2 == 0, 1.0, -1.0)
    mu, sd = _asp(edit, x)
    x64 = x.astype(np.float64)
    want_mu = x64.mean(axis=1)
    want_sd = np.sqrt(np.maximum(x64.var(axis=1), 1e-12))
    np.testing.assert_allclose(mu, want_mu, rtol=1e-5, atol=1e-6 * np.abs(x64).max())
    np.testing.assert_allclose(sd, want_sd, rtol=1e-4)


def check_asp_one_dominant_frame():
    """The attention TDNN reads x channel 0 (identity BN), asp.conv scales it by
    2000 for every channel: the spike frame t0 takes all the attention."""
    def edit(t):
        w = np.zeros((A, 3 * M, 1))
        w[0, 0, 0] = 1.0
        _set(t, "asp.tdnn.conv.conv.weight", w)
        _set(t, "asp.tdnn.conv.conv.bias", np.zeros(A))
        _unit_bn(t, "asp.tdnn.norm.norm", A)
        wc = np.zeros((M, A, 1))
        wc[:, 0, 0] = 2000.0
        _set(t, "asp.conv.conv.weight", wc)
        _set(t, "asp.conv.conv.bias", np.linspace(-1.0, 1.0, M))
    T, t0 = 9, 5
    rng = np.random.default_rng(22)
    x = rng.standard_normal((M, T)).astype(F32)
    x[0] = 0.0
    x[0, t0] = 5.0
    mu, sd = _asp(edit, x)
    np.testing.assert_allclose(mu, x[:, t0].astype(np.float64), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(sd, np.full(M, SQRT_EPS), rtol=1e-6)


def check_asp_global_context_threshold():
    """Attention row r of the TDNN is S_r * (x_r - mean_r - kappa_r * std_r)
    over the context [x ; mean ; std]; it is positive only at the frames where
    x_r exceeds mean_r + kappa_r * std_r, and kappa_r sits between the value
    that the biased, clamped global std passes and the one a wrong std would.
      channel 0: x = [1, -1/3, -1/3, -1/3] + 2 (mean 2, biased std 1/sqrt(3),
        unbiased 2/3), kappa 1.6: frame 0 passes -> one-hot attention;
      channel 1: x = +-5e-7 (biased var 2.5e-13, clamped to 1e-12 -> std 1e-6;
        added eps would give 1.118e-6), kappa 0.47: frames 0 and 2 pass -> mean
        5e-7, std sqrt(1e-12).
    The other channels keep uniform attention."""
    S = (10.0, 1e8)
    kappa = (1.6, 0.47)

    def edit(t):
        w = np.zeros((A, 3 * M, 1))
        for r in range(2):
            w[r, r, 0] = S[r]
            w[r, M + r, 0] = -S[r]
            w[r, 2 * M + r, 0] = -S[r] * kappa[r]
        _set(t, "asp.tdnn.conv.conv.weight", w)
        _set(t, "asp.tdnn.conv.conv.bias", np.zeros(A))
        _unit_bn(t, "asp.tdnn.norm.norm", A)
        wc = np.zeros((M, A, 1))
        wc[0, 0, 0] = 2000.0
        wc[1, 1, 0] = 2000.0
        _set(t, "asp.conv.conv.weight", wc)
        _set(t, "asp.conv.conv.bias", np.zeros(M))
    T = 4
    rng = np.random.default_rng(23)
    x = rng.standard_normal((M, T)).astype(F32)
    x[0] = np.array([1.0, -1 / 3, -1 / 3, -1 / 3], F32) + F32(2.0)
    x[1] = np.array([5e-7, -5e-7, 5e-7, -5e-7], F32)
    mu, sd = _asp(edit, x)
    x64 = x.astype(np.float64)
    want_mu = x64.mean(axis=1)
    want_sd = np.sqrt(np.maximum(x64.var(axis=1), 1e-12))
    want_mu[0], want_sd[0] = x64[0, 0], SQRT_EPS
    want_mu[1], want_sd[1] = 5e-7, SQRT_EPS
    np.testing.assert_allclose(mu, want_mu, rtol=1e-5, atol=1e-12)
    np.testing.assert_allclose(sd, want_sd, rtol=1e-4)


# ------------------------------------------------------------ SE-Res2Net block

C_E, G_E, N_MELS = 16, 4, 6


def _ecapa_blocks(feats):
    """Tiny ECAPA with identity pieces; returns the oracle's block outputs and
    the closed form."""
    kv, t = _tiny_ecapa()
    w0 = np.zeros((C_E, N_MELS, 5))
    scale0 = 1.0 + np.arange(C_E) // N_MELS
    for c in range(C_E):
        w0[c, c % N_MELS, 2] = scale0[c]          # centre tap of the k=5 block0 conv
    _set(t, "blocks.0.conv.conv.weight", w0)
    _set(t, "blocks.0.conv.conv.bias", np.zeros(C_E))
    _unit_bn(t, "blocks.0.norm.norm", C_E)
    beta = np.linspace(-1.0, 1.0, C_E)
    bias2 = np.linspace(0.5, -0.5, C_E)
    for i in range(1, 4):
        p = f"blocks.{i}"
        for name in ("tdnn1", "tdnn2"):
            _set(t, f"{p}.{name}.conv.conv.weight", np.eye(C_E)[:, :, None])
            _set(t, f"{p}.{name}.conv.conv.bias", np.zeros(C_E))
            _unit_bn(t, f"{p}.{name}.norm.norm", C_E)
        for j in range(3):
            wg = np.zeros((G_E, G_E, 3))
            wg[:, :, 1] = np.eye(G_E)
            _set(t, f"{p}.res2net_block.blocks.{j}.conv.conv.weight", wg)
            _set(t, f"{p}.res2net_block.blocks.{j}.conv.conv.bias", np.zeros(G_E))
            _unit_bn(t, f"{p}.res2net_block.blocks.{j}.norm.norm", G_E)
        w1 = np.zeros((4, C_E, 1))
        w1[0, 12, 0] = 1.0                          # squeeze reads channel 12 (group 3)
        _set(t, f"{p}.se_block.conv1.conv.weight", w1)
        _set(t, f"{p}.se_block.conv1.conv.bias", np.zeros(4))
        w2 = np.zeros((C_E, 4, 1))
        w2[:, 0, 0] = beta
        _set(t, f"{p}.se_block.conv2.conv.weight", w2)
        _set(t, f"{p}.se_block.conv2.conv.bias", bias2)
    with tempfile.TemporaryDirectory() as tmp:
        net = O.OracleEcapa(_load(tmp, "ecapa_blocks.gguf", kv, t))
        _, caps = net.forward(np.ascontiguousarray(feats, dtype=F32), capture=True)
    # closed form in f64
    f = feats.astype(np.float64)
    x = np.maximum(scale0[:, None] * f[np.arange(C_E) % N_MELS], 0.0)
    want = [x]
    for _ in range(3):
        g = [x[k * G_E:(k + 1) * G_E] for k in range(4)]
        t2 = np.concatenate([g[0], g[1], g[1] + g[2], g[1] + g[2] + g[3]])
        gate = 1.0 / (1.0 + np.exp(-(beta * max(t2[12].mean(), 0.0) + bias2)))
        x = t2 * gate[:, None] + x
        want.append(x)
    return [caps[f"block{i}"].astype(np.float64) for i in range(4)], want


def check_se_res2net_blocks():
    rng = np.random.default_rng(31)
    feats = rng.standard_normal((N_MELS, 13)).astype(F32)
    got, want = _ecapa_blocks(feats)
    for i, (g, w) in enumerate(zip(got, want)):
        np.testing.assert_allclose(g, w, rtol=2e-6, atol=2e-6 * np.abs(w).max(), err_msg=f"block {i}")


# ------------------------------------------------------------ ResNet BasicBlock

def _resnet_blocks(feats):
    kv, t = synth.make_resnet34(13, wtype=gguf.GGML_F32, channels=(4, 8, 8, 16), blocks=(2, 1, 2, 1),
                                emb_dim=6, n_mels=feats.shape[0])
    p = "voicedetect.resnet."
    name = lambda key, i: kv[p + key][i]   # noqa: E731
    s = np.array([1.0, 0.5, 2.0, 1.5])
    ws = np.zeros((4, 1, 3, 3))
    ws[:, 0, 1, 1] = s
    _set(t, kv[p + "stem_weight"], ws)
    _set(t, kv[p + "stem_bias"], np.zeros(4))
    centre = np.zeros((4, 4, 3, 3))
    centre[:, :, 1, 1] = np.eye(4)
    # block 0 (4 -> 4, stride 1): identity convs, b2 = -0.7 -> relu(2x - 0.7)
    _set(t, name("conv1_weight", 0), centre)
    _set(t, name("conv1_bias", 0), np.zeros(4))
    _set(t, name("conv2_weight", 0), centre)
    _set(t, name("conv2_bias", 0), np.full(4, -0.7))
    # block 1 (4 -> 4, stride 1): conv2 zero -> relu(b2 + x)
    b2 = np.array([-0.5, 0.3, -0.2, 0.1])
    _set(t, name("conv2_weight", 1), np.zeros((4, 4, 3, 3)))
    _set(t, name("conv2_bias", 1), b2)
    # block 2 (4 -> 8, stride 2, downsample): conv2 zero, 1x1 channel map k
    b2s = np.linspace(-0.4, 0.4, 8)
    bd = np.linspace(0.2, -0.3, 8)
    k = 1.0 + np.arange(8) // 4
    wd = np.zeros((8, 4, 1, 1))
    wd[np.arange(8), np.arange(8) % 4, 0, 0] = k
    _set(t, name("conv2_weight", 2), np.zeros((8, 8, 3, 3)))
    _set(t, name("conv2_bias", 2), b2s)
    _set(t, name("down_weight", 2), wd)
    _set(t, name("down_bias", 2), bd)
    with tempfile.TemporaryDirectory() as tmp:
        net = O.OracleResNet(_load(tmp, "resnet_blocks.gguf", kv, t))
        _, caps = net.forward(np.ascontiguousarray(feats, dtype=F32), capture=True)
    f = feats.astype(np.float64)
    x0 = np.maximum(s[:, None, None] * f[None], 0.0)
    y0 = np.maximum(2.0 * x0 - 0.7, 0.0)
    y1 = np.maximum(b2[:, None, None] + y0, 0.0)
    y2 = np.maximum((b2s + bd)[:, None, None] + k[:, None, None] * y1[np.arange(8) % 4][:, ::2, ::2], 0.0)
    got = [caps["stem"], caps["block0"], caps["block1"], caps["block2"]]
    return [g.astype(np.float64) for g in got], [x0, y0, y1, y2]


def check_resnet_blocks():
    rng = np.random.default_rng(41)
    feats = rng.standard_normal((12, 15)).astype(F32)
    got, want = _resnet_blocks(feats)
    for i, (g, w) in enumerate(zip(got, want)):
        assert g.shape == w.shape, (i, g.shape, w.shape)
        np.testing.assert_allclose(g, w, rtol=1e-6, atol=1e-6, err_msg=f"stage {i}")


PINS = {
    "asp_uniform": check_asp_uniform_attention,
    "asp_one_frame": check_asp_one_dominant_frame,
    "asp_global_context": check_asp_global_context_threshold,
    "se_res2net": check_se_res2net_blocks,
    "resnet_block": check_resnet_blocks,
}


@pytest.mark.parametrize("pin", sorted(PINS))
def test_oracle_meets_closed_form(pin):
    PINS[pin]()


# ------------------------------------------------------------------ mutations

def _sub(old, new, count=1):
    return (old, new, count)


# file -> substitutions; each names a misreading of the reference rule
MUTANTS = {
    "asp_softmax_over_channels": ("oracle_ecapa.c", [
        _sub("""        float mx = l[0];
        for (int t = 1; t < T; ++t) if (l[t] > mx) mx = l[t];
        double z = 0.0;
        for (int t = 0; t < T; ++t) { l[t] = expf(l[t] - mx); z += l[t]; }
        for (int t = 0; t < T; ++t) l[t] = (float)(l[t] / z);       /* softmax over time */
""", ""),
        _sub("""    for (int c = 0; c < C; ++c) {
        float* l = lg + (size_t)c * T;""", """    for (int t = 0; t < T; ++t) {
        float mx = lg[t];
        for (int c = 1; c < C; ++c) if (lg[(size_t)c * T + t] > mx) mx = lg[(size_t)c * T + t];
        double z = 0.0;
        for (int c = 0; c < C; ++c) { lg[(size_t)c * T + t] = expf(lg[(size_t)c * T + t] - mx); z += lg[(size_t)c * T + t]; }
        for (int c = 0; c < C; ++c) lg[(size_t)c * T + t] = (float)(lg[(size_t)c * T + t] / z);
    }
    for (int c = 0; c < C; ++c) {
        float* l = lg + (size_t)c * T;"""),
    ]),
    "asp_eps_added": ("oracle_ecapa.c", [_sub("if (v < kAspEps) v = kAspEps;", "v += kAspEps;", 2)]),
    "asp_variance_about_zero": ("oracle_ecapa.c", [_sub("const float d = r[t] - muf;", "const float d = r[t];")]),
    "asp_global_std_unbiased": ("oracle_ecapa.c", [_sub("float v = (float)(s2 / T);",
                                                        "float v = (float)(s2 / (T - 1));")]),
    "asp_context_order_swapped": ("oracle_ecapa.c", [
        _sub("ctx[(size_t)(C + c) * T + t] = m;", "ctx[(size_t)(C + c) * T + t] = sd;"),
        _sub("ctx[(size_t)(2 * C + c) * T + t] = sd;", "ctx[(size_t)(2 * C + c) * T + t] = m;"),
    ]),
    "res2net_chain_through_group0": ("oracle_ecapa.c", [
        _sub("if (j == 1) memcpy(in, xj, sizeof(float) * (size_t)G * T);\n            else {",
             "{")]),
    "se_gate_on_sum": ("oracle_ecapa.c", [
        _sub("out[(size_t)c * T + t] = t2[(size_t)c * T + t] * g + x[(size_t)c * T + t];",
             "out[(size_t)c * T + t] = (t2[(size_t)c * T + t] + x[(size_t)c * T + t]) * g;")]),
    "se_squeeze_of_input": ("oracle_ecapa.c", [
        _sub("se[c] = mean_row(t2 + (size_t)c * T, T);", "se[c] = mean_row(x + (size_t)c * T, T);")]),
    "resnet_relu_before_residual": ("oracle.c", [
        _sub("orc_conv2d_f32(h, oc, Ho, Wo, net->conv2_w[i], oc, 3, 3, 1, 1, net->conv2_b[i], sc, 1, y);",
             "orc_conv2d_f32(h, oc, Ho, Wo, net->conv2_w[i], oc, 3, 3, 1, 1, net->conv2_b[i], NULL, 1, y);\n"
             "        for (size_t q = 0; q < n; ++q) y[q] += sc[q];")]),
}


def _build_mutant(tmp, name):
    fname, subs = MUTANTS[name]
    return _build_mutant_from(tmp, name, fname, subs)


def _build_mutant_from(tmp, name, fname, subs):
    """The oracle sources copied to tmp/name with `subs` applied to `fname`,
    built as a shared library; returns its path."""
    d = os.path.join(tmp, name)
    os.makedirs(d)
    for f in os.listdir(ORACLE_DIR):
        if f.endswith((".c", ".h")):
            shutil.copy(os.path.join(ORACLE_DIR, f), d)
    src = open(os.path.join(d, fname)).read()
    for old, new, count in subs:
        assert src.count(old) == count, (name, old)
        src = src.replace(old, new)
    open(os.path.join(d, fname), "w").write(src)
    out = os.path.join(d, "liboracle_mutant.so")
    cfiles = sorted(os.path.join(d, f) for f in os.listdir(d) if f.endswith(".c"))
    subprocess.run(["gcc", "-O1", "-fPIC", "-shared", "-std=gnu11", "-w", "-o", out] + cfiles + ["-lm", "-lpthread"],
                   check=True)
    return out


# the pin that must fail on each mutant
CATCHES = {
    "asp_softmax_over_channels": "asp_uniform",
    "asp_eps_added": "asp_uniform",
    "asp_variance_about_zero": "asp_uniform",
    "asp_global_std_unbiased": "asp_global_context",
    "asp_context_order_swapped": "asp_global_context",
    "res2net_chain_through_group0": "se_res2net",
    "se_gate_on_sum": "se_res2net",
    "se_squeeze_of_input": "se_res2net",
    "resnet_relu_before_residual": "resnet_block",
}


def _fails(pin):
    try:
        PINS[pin]()
    except AssertionError:
        return True
    return False


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc to build the mutant oracles")
@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_pins_catch_mutant(mutant):
    with tempfile.TemporaryDirectory() as tmp:
        path = _build_mutant(tmp, mutant)
        with O.using_library(path):
            assert _fails(CATCHES[mutant]), f"pin {CATCHES[mutant]} does not fail on the {mutant} mutant"
