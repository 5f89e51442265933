"""Pins the numpy wav2vec2 oracle (oracle/oracle_w2v2.py).

The reference's analyze goldens are HF transformers outputs
(scripts/gen_baseline.py --analyze; tests/test_analyze.cpp,
tests/test_age_gender.cpp).  tests/golden/make_w2v2_golden.py builds HF's own
Wav2Vec2 modules offline from a small config with seeded random weights, runs
them in f64 and stores their weights (under the reference converter's names,
w2v2_store_name) and outputs in tests/golden/w2v2_golden.npz; here the weights
go into a GGUF and the oracle run on it must reproduce every hidden state and
the head outputs to ~1e-10.  The checks cover both reference variants:
wav2vec2-base emotion (group-norm conv0, post-norm layers, weighted layer sum,
projector + classifier) and wav2vec2-large-robust age/gender (layer-norm convs
with bias, do_normalize, pre-norm layers, two tanh heads).  Closed forms pin the
pieces on their own.  No torch or transformers import happens here.
"""
import json
import os
import tempfile

import numpy as np
import pytest

import oracle_w2v2 as W
from vdamd import gguf as G
from vdamd import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w2v2_golden.npz")


def _golden():
    return np.load(GOLDEN, allow_pickle=False)


def _oracle(z, kind, labels):
    prefix = f"{kind}/w/"
    tensors = [(k[len(prefix):], G.GGML_F32, list(z[k].shape), z[k]) for k in z.files if k.startswith(prefix)]
    c = json.loads(str(z[f"{kind}/config"]))
    kv = synth.w2v2_kv(kind, c["hidden"], c["n_layers"], c["n_heads"], c["ff"], tuple(c["conv_dims"]),
                       tuple(c["conv_kernels"]), tuple(c["conv_strides"]), c["pos_k"], c["pos_groups"], c["proj"],
                       labels, c["eps"])
    path = os.path.join(tempfile.mkdtemp(), kind + ".gguf")
    G.write_gguf(path, kv, tensors)
    return W.OracleW2V2(path)


def _pcm(n, seed):
    return synth.clip(seed, n).astype(np.float64)


@pytest.fixture(scope="module")
def emotion_pair():
    z = _golden()
    return z, _oracle(z, "emotion", synth.EMOTION_LABELS)


@pytest.fixture(scope="module")
def age_gender_pair():
    z = _golden()
    return z, _oracle(z, "age_gender", synth.GENDER_LABELS)


def _close(a, b, tol=1e-9):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    err = np.abs(a - b).max() / max(1.0, np.abs(b).max())
    assert err < tol, err


@pytest.mark.parametrize("n", [4000, 8000, 12345])
def test_emotion_matches_hf(emotion_pair, n):
    z, orc = emotion_pair
    pcm = _pcm(n, 100 + n)
    g = f"emotion/n{n}/"
    _close(orc.conv_encoder(pcm), z[g + "feat"])
    states = orc.hidden_states(pcm)
    hidden = z[g + "hidden"]
    assert len(states) == len(hidden) == orc.n_layers + 1
    assert states[0].shape[0] == orc.frames(n)
    for s, h in zip(states, hidden):
        _close(s, h)
    _close(orc.raw_outputs(pcm), z[g + "raw"])


@pytest.mark.parametrize("n", [4000, 9001])
def test_age_gender_matches_hf(age_gender_pair, n):
    z, orc = age_gender_pair
    pcm = _pcm(n, 200 + n)
    g = f"age_gender/n{n}/"
    # do_normalize is the feature extractor's zero-mean / unit-variance step;
    # it normalises in f32, so the conv stack is compared on its output
    x = z[g + "normalized"]
    orc.do_normalize = False
    try:
        _close(orc.conv_encoder(x), z[g + "feat"])
        states = orc.hidden_states(x)
        hidden = z[g + "hidden"]
        assert len(states) == len(hidden)
        for s, h in zip(states, hidden):
            _close(s, h)
        _close(orc.raw_outputs(x), z[g + "raw"])
    finally:
        orc.do_normalize = True
    # and the oracle's own normalisation agrees with the extractor's to f32 rounding
    xn = (pcm - pcm.mean()) / np.sqrt(pcm.var() + W.WAVE_NORM_EPS)
    assert np.abs(xn - x).max() < 1e-5


def test_conv_stack_lengths(emotion_pair):
    _, orc = emotion_pair
    for n in (400, 401, 1000, 16000):
        T = n
        for k, s in zip(orc.kernels, orc.strides):
            T = (T - k) // s + 1
        assert orc.frames(n) == T
        if T > 0:
            assert orc.conv_encoder(_pcm(n, 5)).shape == (T, orc.conv_dims[-1])
    assert orc.frames(9) == 0


def test_pos_conv_weight_norm(emotion_pair):
    _, orc = emotion_pair
    w = orc.pos_conv_weight()
    g = orc.w("w2v2.encoder.pos_conv_embed.conv.weight_g").reshape(-1)
    np.testing.assert_allclose(np.sqrt((w * w).sum(axis=(0, 1))), np.abs(g), rtol=1e-12)


def test_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((7, 33)) * 3 + 1
    y = W.layer_norm(x, np.ones(33), np.zeros(33), 0.0)
    np.testing.assert_allclose(y.mean(axis=1), 0, atol=1e-12)
    np.testing.assert_allclose(y.var(axis=1), 1, rtol=1e-12)
    # gelu: x * Phi(x); Phi(0) = 1/2, odd part x/2
    np.testing.assert_allclose(W.gelu(np.array([0.0, 1.0, -1.0])), [0.0, 0.8413447460685429, -0.15865525393145707],
                               rtol=1e-12)
    # strided conv against a direct double loop
    w = rng.standard_normal((3, 2, 4))
    x = rng.standard_normal((11, 2))
    ref = np.array([[sum(w[o, i, k] * x[t * 3 + k, i] for i in range(2) for k in range(4)) for o in range(3)]
                    for t in range((11 - 4) // 3 + 1)])
    np.testing.assert_allclose(W.conv1d_strided(x, w, 3), ref, rtol=1e-12)
    # reference host softmax: probabilities sum to ~1 and keep the logit order
    p = W.probs_f32(np.array([1.0, 3.0, 2.0], np.float32))
    assert p.dtype == np.float32 and abs(float(p.sum()) - 1) < 1e-6 and list(np.argsort(p)) == [0, 2, 1]


def test_attention_identical_keys(emotion_pair):
    """With every token equal, attention returns out_proj(v_proj(x)) for each token."""
    _, orc = emotion_pair
    x = np.tile(np.linspace(-1, 1, orc.hidden)[None], (5, 1))
    pre = "w2v2.encoder.layers.0.attention"
    want = orc.linear(orc.linear(x, pre + ".v_proj"), pre + ".out_proj")
    np.testing.assert_allclose(orc.attention(x, pre), want, rtol=1e-12, atol=1e-12)


def test_json_shapes(emotion_pair, age_gender_pair):
    _, orc = emotion_pair
    js = json.loads(orc.analyze_json(_pcm(6000, 9)))
    assert set(js) == {"emotion"} and js["emotion"]["label"] in synth.EMOTION_LABELS
    assert abs(sum(js["emotion"]["scores"].values()) - 1) < 1e-5
    _, orc2 = age_gender_pair
    js = json.loads(orc2.analyze_json(_pcm(6000, 9)))
    assert set(js) == {"age", "gender"} and js["gender"]["label"] in synth.GENDER_LABELS
    assert abs(sum(v for k, v in js["gender"].items() if k != "label") - 1) < 1e-5
    raw = orc2.raw_outputs(_pcm(6000, 9))
    assert js["age"] == pytest.approx(float(np.float32(raw[0])) * 100.0, rel=1e-5)
