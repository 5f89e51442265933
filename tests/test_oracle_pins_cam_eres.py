"""Closed-form pins of the oracle's CAM++ and ERes2Net composition.

Each check drives the oracle (oracle/oracle_campplus.c, oracle/oracle_eres2net.c)
with weights chosen so that the reference's layer rules reduce to a formula
that can be written down without restating them:

* CAM++ transits (src/encoder_campplus.cpp:250-281): BN -> ReLU -> 1x1, with
  the ReLU after the conv on the last transit only.  Transit weights of -1 /
  +1 on chosen channels make each block's output a signed copy of TDNN output
  channels, so a ReLU after transit 1 or 2 (zeroing the negative copies) or a
  missing one after transit 3 shows up as a wrong sign;
* CAM++ statistics pooling (src/encoder_campplus.cpp:284-296): an all-zero
  channel pools to std exactly 0 (no eps), a copied channel to its mean and
  unbiased std;
* CAM++ context (src/encoder_campplus.cpp:159-182): a dense layer whose
  linear1 output is the constant k sees ctx = k + k * L / 100 in a segment of
  L frames (the 100-frame average counts the missing frames of a short last
  segment as zeros), and its gated output k * sigmoid(ctx - 1) reaches a
  block output through the transit;
* ERes2Net blocks (src/encoder_eres2net.cpp:111-137): with a zero conv3 and a
  zero-weight shortcut the block output is clamp(b3 + residual, 0, 20), the
  clamp after the residual add, chained over the blocks of the last layer;
* ERes2Net AFF (src/encoder_eres2net.cpp:91-101): a zero second attention
  conv with bias z gives (x + ds) + tanh(z) (x - ds) with x the deep branch
  and ds the downsampled fused branch (here 0: a zero downsample conv);
* the ERes2Net shortcut rule (src/encoder_eres2net.cpp:130-134): a shortcut
  conv exactly when stride != 1 or in_planes != 2 * planes; any other rule
  walks the manifest differently and the fused map no longer matches.

The mutation tests compile copies of the oracle with one misreading each and
require the pin to fail; they run in a child process, since a misread
manifest walk can read past a buffer.
"""
import os
import shutil
import subprocess
import sys
import tempfile

import numpy as np
import pytest

import pyoracle as O
from test_oracle_pins import _build_mutant_from, _load, _set, _unit_bn
from vdamd import gguf, synth

F32 = np.float32
HERE = os.path.dirname(os.path.abspath(__file__))

# ------------------------------------------------------------------ CAM++

CM = dict(n_mels=16, m_ch=4, init_ch=8, growth=4, bn_ch=8, emb_dim=4, wtype=gguf.GGML_F32)
T_CAM = 297            # T' = 149: segments of 100 and 49 frames
K_CTX = F32(0.5)       # the constant linear1 output of the observed dense layer


def _campp_net():
    kv, T = synth.make_campplus(11, **CM)
    convs = kv["voicedetect.campplus.conv_weight"]
    biases = kv["voicedetect.campplus.conv_bias"]
    shapes = {n: s for n, _t, s, _a in T}
    init, g, bc = CM["init_ch"], CM["growth"], CM["bn_ch"]
    # block 1, layer 1: linear1 -> constant K_CTX on channel 0, linear_local
    # -> its centre tap, context MLP hidden0 = ctx0, gate0 = sigmoid(hidden0 - 1)
    p = "xvector.block1.tdnnd1"
    l1 = convs.index(p + ".cam_layer.linear_local.weight") - 1
    _set(T, convs[l1], np.zeros(shapes[convs[l1]], F32))
    b = np.zeros(bc, F32)
    b[0] = K_CTX
    _set(T, biases[l1], b)
    w = np.zeros((g, bc, 3), F32)
    w[0, 0, 1] = 1.0
    _set(T, p + ".cam_layer.linear_local.weight", w)
    w = np.zeros((bc // 2, bc, 1), F32)
    w[0, 0, 0] = 1.0
    _set(T, p + ".cam_layer.linear1.weight", w)
    _set(T, p + ".cam_layer.linear1.bias", np.zeros(bc // 2, F32))
    w = np.zeros((g, bc // 2, 1), F32)
    w[0, 0, 0] = 1.0
    _set(T, p + ".cam_layer.linear2.weight", w)
    b = np.zeros(g, F32)
    b[0] = -1.0
    _set(T, p + ".cam_layer.linear2.bias", b)
    # transits: unit BNs and signed channel copies
    c1 = init + 12 * g
    c2 = c1 // 2 + 24 * g
    c3 = c2 // 2 + 16 * g
    for i, c in ((1, c1), (2, c2), (3, c3)):
        _unit_bn(T, f"xvector.transit{i}.nonlinear.batchnorm", c)
    w = np.zeros((c1 // 2, c1, 1), F32)
    w[0, 0, 0], w[1, 1, 0], w[2, 2, 0], w[3, init, 0] = -1.0, 1.0, 1.0, 1.0
    _set(T, "xvector.transit1.linear.weight", w)
    w = np.zeros((c2 // 2, c2, 1), F32)
    w[0, 1, 0], w[1, 2, 0] = -1.0, 1.0
    _set(T, "xvector.transit2.linear.weight", w)
    t3 = convs[-2]                       # the folded last transit, before the dense head
    w = np.zeros((c3 // 2, c3, 1), F32)
    w[0, 1, 0], w[1, 1, 0] = -1.0, 1.0
    _set(T, t3, w)
    _set(T, biases[-2], np.zeros(c3 // 2, F32))
    return kv, T


def _campp_forward():
    kv, T = _campp_net()
    with tempfile.TemporaryDirectory() as tmp:
        net = O.OracleCampplus(_load(tmp, "campp.gguf", kv, T))
        feats = np.random.default_rng(2).standard_normal((CM["n_mels"], T_CAM)).astype(F32)
        _, caps = net.forward(feats, capture=True)
    return caps


def _sigmoid32(x):
    x = F32(x)
    return F32(1.0) / (F32(1.0) + np.exp(-x, dtype=F32))


def check_campp_transit_relu_rule():
    caps = _campp_forward()
    t = caps["tdnn"]
    assert (t[:3] > 0).any(axis=1).all(), "the copied TDNN channels must be positive somewhere"
    b0, b1, b2 = caps["block0"], caps["block1"], caps["block2"]
    assert np.array_equal(b0[0], -t[0]) and np.array_equal(b0[1], t[1]) and np.array_equal(b0[2], t[2])
    assert np.array_equal(b1[0], -t[1]) and np.array_equal(b1[1], t[2])
    assert np.array_equal(b2[0], np.zeros_like(t[2])) and np.array_equal(b2[1], t[2])


def check_campp_stats_pooling():
    caps = _campp_forward()
    t2 = caps["tdnn"][2].astype(np.float64)
    C = caps["block2"].shape[0]
    pooled = caps["pooled"]
    assert pooled[0] == 0.0 and pooled[C] == 0.0            # a zero channel: std 0, no eps
    assert abs(pooled[1] - t2.mean()) <= 1e-6 * max(1.0, abs(t2.mean()))
    assert abs(pooled[C + 1] - t2.std(ddof=1)) <= 1e-5 * t2.std(ddof=1)


def check_campp_segment_context():
    caps = _campp_forward()
    Tp = caps["block0"].shape[1]
    assert Tp == 149
    got = caps["block0"][3]
    for lo, hi in ((0, 100), (100, Tp)):
        L = hi - lo
        ctx = F32(K_CTX) + F32(K_CTX * L / 100.0)           # mean over T' + segment sum / 100
        want = K_CTX * _sigmoid32(F32(ctx) - F32(1.0))
        assert np.allclose(got[lo:hi], want, rtol=2e-6, atol=0), (lo, hi, got[lo], want)


# ------------------------------------------------------------------ ERes2Net

EM = dict(n_mels=16, m_ch=4, num_blocks=(1, 1, 1, 2), scale=2, emb_dim=8, wtype=gguf.GGML_F32)
T_ERES = 40
NC = 16 * EM["m_ch"]                    # channels of the last layer and the fused map


def _eres_values():
    c = np.arange(NC)
    s0 = (((c * 7) % 13) * 3.0 - 12.0).astype(F32)            # shortcut bias of block 0
    b30 = (((c * 5) % 11) * 3.0 - 9.0).astype(F32)            # conv3 biases
    b31 = (((c * 3) % 7) * 5.0 - 16.0).astype(F32)
    z = (((c * 11) % 9) * 0.45 - 1.8).astype(F32)             # final AFF logit
    return s0, b30, b31, z


def _eres_net():
    kv, T = synth.make_eres2net(13, **EM)
    convs = kv["voicedetect.eres2net.conv_weight"]
    biases = kv["voicedetect.eres2net.conv_bias"]
    shapes = {n: s for n, _t, s, _a in T}
    s0, b30, b31, z = _eres_values()

    def zero(i, bias=None):
        _set(T, convs[i], np.zeros(shapes[convs[i]], F32))
        if bias is not None:
            _set(T, biases[i], bias)

    # from the end of the manifest: final AFF (conv1, conv2), the downsample of
    # the fused map, then the last layer's two blocks (block 1: conv1,
    # convs[0], AFF pair, convs[1], conv3; block 0 the same plus its shortcut)
    zero(-1, z)
    zero(-3)
    zero(-4, b31)
    zero(-10, s0)
    zero(-11, b30)
    return kv, T


def _eres_fused():
    kv, T = _eres_net()
    with tempfile.TemporaryDirectory() as tmp:
        net = O.OracleEres2net(_load(tmp, "eres.gguf", kv, T))
        feats = np.random.default_rng(4).standard_normal((EM["n_mels"], T_ERES)).astype(F32)
        _, caps = net.forward(feats, capture=True)
    return caps["fused"]


def _eres_expect():
    s0, b30, b31, z = _eres_values()
    o0 = np.clip(b30 + s0, F32(0), F32(20))
    o1 = np.clip(b31 + o0, F32(0), F32(20))
    t = np.tanh(z, dtype=F32)
    return (o1 + F32(0)) + t * (o1 - F32(0)), o0, o1, t


def check_eres_block_clamp_after_residual():
    fused = _eres_fused()
    want, o0, o1, t = _eres_expect()
    # the chosen biases cross both clamp bounds, before and after the add
    assert (o0 == 20).any() and (o0 == 0).any() and (o1 == 20).any() and (o1 == 0).any()
    got = fused.reshape(NC, -1)
    assert np.allclose(got, want[:, None], rtol=2e-6, atol=1e-6), np.abs(got - want[:, None]).max()


def check_eres_aff_order():
    fused = _eres_fused()
    want, _, o1, t = _eres_expect()
    assert ((o1 != 0) & (np.abs(t) > 0.1)).sum() >= 16
    got = fused.reshape(NC, -1)
    assert np.allclose(got, want[:, None], rtol=2e-6, atol=1e-6)


PINS = {
    "campp_transit_relu": check_campp_transit_relu_rule,
    "campp_stats_pooling": check_campp_stats_pooling,
    "campp_segment_context": check_campp_segment_context,
    "eres_clamp_after_residual": check_eres_block_clamp_after_residual,
    "eres_aff_order": check_eres_aff_order,
}


@pytest.mark.parametrize("pin", sorted(PINS))
def test_oracle_meets_closed_form(pin):
    PINS[pin]()


# ------------------------------------------------------------------ mutations

def _sub(old, new, count=1):
    return (old, new, count)


MUTANTS = {
    "campp_relu_after_every_transit": ("oracle_campplus.c", [
        _sub("conv1d(tr, a, Tp, 1, 0, 1, b == 2, h);", "conv1d(tr, a, Tp, 1, 0, 1, 1, h);")]),
    "campp_no_relu_after_last_transit": ("oracle_campplus.c", [
        _sub("conv1d(tr, a, Tp, 1, 0, 1, b == 2, h);", "conv1d(tr, a, Tp, 1, 0, 1, 0, h);")]),
    "campp_std_with_eps": ("oracle_campplus.c", [
        _sub("orc_tstp(h, Ccur, 1, Tp, 0.0f, pooled);", "orc_tstp(h, Ccur, 1, Tp, eps, pooled);")]),
    "campp_segment_average_excludes_pad": ("oracle_campplus.c", [
        _sub("ctx[(size_t)c * nseg + sg] = m + (float)(ss / kSeg);",
             "ctx[(size_t)c * nseg + sg] = m + (float)(ss / (t1 - sg * kSeg));")]),
    "campp_context_without_global_mean": ("oracle_campplus.c", [
        _sub("ctx[(size_t)c * nseg + sg] = m + (float)(ss / kSeg);",
             "ctx[(size_t)c * nseg + sg] = (float)(ss / kSeg);")]),
    "eres_clamp_before_residual": ("oracle_eres2net.c", [
        _sub("""    orc_conv2d_f32_g(acc.d, acc.C, acc.H, acc.W, c3->w, c3->oc, c3->kh, c3->kw, s3, s3, 0, 0, 1, 1, c3->b, res.d, 0,
                     y.d);""", """    orc_conv2d_f32_g(acc.d, acc.C, acc.H, acc.W, c3->w, c3->oc, c3->kh, c3->kw, s3, s3, 0, 0, 1, 1, c3->b, NULL, 0,
                     y.d);
    hclamp(y.d, fm_n(y), hi);
    for (size_t q = 0; q < fm_n(y); ++q) y.d[q] += res.d[q];
    if (0)"""),
    ]),
    "eres_relu_instead_of_clamp": ("oracle_eres2net.c", [
        _sub("x[i] = x[i] < 0.0f ? 0.0f : (x[i] > hi ? hi : x[i]);", "x[i] = x[i] < 0.0f ? 0.0f : x[i];")]),
    "eres_aff_order_swapped": ("oracle_eres2net.c", [
        _sub("z2.d[i] = (a + b) + tanhf(z2.d[i]) * (a - b);", "z2.d[i] = (a + b) + tanhf(z2.d[i]) * (b - a);")]),
    "eres_shortcut_on_stride_only": ("oracle_eres2net.c", [
        _sub("if (stride != 1 || *in_planes != 2 * planes) {", "if (stride != 1) {")]),
    "eres_shortcut_without_expansion": ("oracle_eres2net.c", [
        _sub("if (stride != 1 || *in_planes != 2 * planes) {", "if (stride != 1 || *in_planes != planes) {")]),
}

CATCHES = {
    "campp_relu_after_every_transit": "campp_transit_relu",
    "campp_no_relu_after_last_transit": "campp_transit_relu",
    "campp_std_with_eps": "campp_stats_pooling",
    "campp_segment_average_excludes_pad": "campp_segment_context",
    "campp_context_without_global_mean": "campp_segment_context",
    "eres_clamp_before_residual": "eres_clamp_after_residual",
    "eres_relu_instead_of_clamp": "eres_clamp_after_residual",
    "eres_aff_order_swapped": "eres_aff_order",
    "eres_shortcut_on_stride_only": "eres_clamp_after_residual",
    "eres_shortcut_without_expansion": "eres_clamp_after_residual",
}

# child: run one pin against a mutant oracle; exit 0 when the pin fails (an
# assertion, or the oracle reporting a manifest it cannot walk), 3 when it passes
_CHILD = """
import sys
sys.path[:0] = sys.argv[3].split(":")
import pyoracle as O
import test_oracle_pins_cam_eres as P
with O.using_library(sys.argv[1]):
    try:
        P.PINS[sys.argv[2]]()
    except AssertionError:
        sys.exit(0)
sys.exit(3)
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc to build the mutant oracles")
@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_pins_catch_mutant(mutant):
    fname, subs = MUTANTS[mutant]
    with tempfile.TemporaryDirectory() as tmp:
        path = _build_mutant_from(tmp, mutant, fname, subs)
        paths = ":".join(p for p in sys.path if p)
        r = subprocess.run([sys.executable, "-c", _CHILD, path, CATCHES[mutant], HERE + ":" + paths],
                           capture_output=True, text=True, timeout=600)
        # 0: the pin failed; a signal: the misread walk crashed the oracle
        assert r.returncode == 0 or r.returncode < 0, (
            f"pin {CATCHES[mutant]} does not fail on the {mutant} mutant (rc {r.returncode})\n{r.stderr[-2000:]}")
