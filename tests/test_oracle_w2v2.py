"""Pins the numpy wav2vec2 oracle (oracle/oracle_w2v2.py).

The reference's analyze goldens are HF transformers outputs
(scripts/gen_baseline.py --analyze; tests/test_analyze.cpp,
tests/test_age_gender.cpp).  Here HF's own Wav2Vec2 modules are built offline
from a small config with random weights, run in f64, exported through the
reference converter's naming (w2v2_store_name) into a GGUF, and the oracle run
on that GGUF must reproduce every hidden state and the head outputs to ~1e-10.
The checks cover both reference variants: wav2vec2-base emotion (group-norm conv0,
post-norm layers, weighted layer sum, projector + classifier) and
wav2vec2-large-robust age/gender (layer-norm convs with bias, do_normalize,
pre-norm layers, two tanh heads).  Closed forms pin the pieces on their own.
"""
import json
import os
import tempfile

import numpy as np
import pytest

import oracle_w2v2 as W
from vdamd import gguf as G
from vdamd import synth

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")
os.environ.setdefault("HF_HUB_OFFLINE", "1")
os.environ.setdefault("TRANSFORMERS_OFFLINE", "1")

CONV = dict(conv_dim=(32, 32, 32, 32, 32, 32, 32), conv_kernel=(10, 3, 3, 3, 3, 2, 2),
            conv_stride=(5, 2, 2, 2, 2, 2, 2))


def _hf_config(large):
    from transformers import Wav2Vec2Config
    return Wav2Vec2Config(
        hidden_size=64, num_hidden_layers=3, num_attention_heads=4, intermediate_size=96, **CONV,
        feat_extract_norm="layer" if large else "group", conv_bias=large, do_stable_layer_norm=large,
        num_conv_pos_embeddings=16, num_conv_pos_embedding_groups=4, use_weighted_layer_sum=not large,
        classifier_proj_size=24, num_labels=4, layer_norm_eps=1e-5, hidden_dropout=0.0, attention_dropout=0.0,
        activation_dropout=0.0, feat_proj_dropout=0.0, final_dropout=0.0, layerdrop=0.0, mask_time_prob=0.0)


def _export(state, kind, cfg, labels, path):
    tensors = []
    for name, t in state.items():
        if name.startswith("wav2vec2.masked_spec_embed"):
            continue
        a = t.detach().cpu().numpy().astype(np.float32)
        tensors.append((synth.w2v2_store_name(name), G.GGML_F32, list(a.shape), a))
    kv = synth.w2v2_kv(kind, cfg.hidden_size, cfg.num_hidden_layers, cfg.num_attention_heads,
                       cfg.intermediate_size, cfg.conv_dim, cfg.conv_kernel, cfg.conv_stride,
                       cfg.num_conv_pos_embeddings, cfg.num_conv_pos_embedding_groups,
                       cfg.classifier_proj_size, labels, cfg.layer_norm_eps)
    G.write_gguf(path, kv, tensors)
    return path


def _f32_weights(model):
    # the GGUF stores f32: round the f64 model's weights to f32 so both sides
    # see the same values
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(p.float().double())


def _pcm(n, seed):
    return synth.clip(seed, n).astype(np.float64)


@pytest.fixture(scope="module")
def emotion_pair():
    from transformers import Wav2Vec2ForSequenceClassification
    torch.manual_seed(7)
    cfg = _hf_config(False)
    m = Wav2Vec2ForSequenceClassification(cfg).double().eval()
    with torch.no_grad():
        m.layer_weights.copy_(torch.randn(cfg.num_hidden_layers + 1, dtype=torch.float64))
    _f32_weights(m)
    path = _export(m.state_dict(), "emotion", cfg, synth.EMOTION_LABELS,
                   os.path.join(tempfile.mkdtemp(), "emo.gguf"))
    return m, W.OracleW2V2(path)


class _AgeGender(torch.nn.Module):
    """audeering AgeGenderModel: Wav2Vec2Model + two ModelHeads
    out_proj(tanh(dense(mean_t(last_hidden_state))))."""

    def __init__(self, cfg):
        super().__init__()
        from transformers import Wav2Vec2Model
        self.wav2vec2 = Wav2Vec2Model(cfg)
        H = cfg.hidden_size
        self.age = torch.nn.ModuleDict(dict(dense=torch.nn.Linear(H, H), out_proj=torch.nn.Linear(H, 1)))
        self.gender = torch.nn.ModuleDict(dict(dense=torch.nn.Linear(H, H), out_proj=torch.nn.Linear(H, 3)))

    def forward(self, x):
        out = self.wav2vec2(x, output_hidden_states=True)
        pooled = out.last_hidden_state.mean(dim=1)
        heads = [h["out_proj"](torch.tanh(h["dense"](pooled))) for h in (self.age, self.gender)]
        return out, torch.cat(heads, dim=1)


@pytest.fixture(scope="module")
def age_gender_pair():
    torch.manual_seed(11)
    cfg = _hf_config(True)
    m = _AgeGender(cfg).double().eval()
    _f32_weights(m)
    path = _export(m.state_dict(), "age_gender", cfg, synth.GENDER_LABELS,
                   os.path.join(tempfile.mkdtemp(), "ag.gguf"))
    return m, W.OracleW2V2(path)


def _close(a, b, tol=1e-9):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    err = np.abs(a - b).max() / max(1.0, np.abs(b).max())
    assert err < tol, err


@pytest.mark.parametrize("n", [4000, 8000, 12345])
def test_emotion_matches_hf(emotion_pair, n):
    m, orc = emotion_pair
    pcm = _pcm(n, 100 + n)
    with torch.no_grad():
        out = m(torch.from_numpy(pcm)[None], output_hidden_states=True)
        feat = m.wav2vec2.feature_extractor(torch.from_numpy(pcm)[None]).transpose(1, 2)[0].numpy()
    _close(orc.conv_encoder(pcm), feat)
    states = orc.hidden_states(pcm)
    assert len(states) == len(out.hidden_states) == orc.n_layers + 1
    assert states[0].shape[0] == orc.frames(n)
    for s, h in zip(states, out.hidden_states):
        _close(s, h[0].numpy())
    _close(orc.raw_outputs(pcm), out.logits[0].numpy())


@pytest.mark.parametrize("n", [4000, 9001])
def test_age_gender_matches_hf(age_gender_pair, n):
    from transformers import Wav2Vec2FeatureExtractor
    m, orc = age_gender_pair
    pcm = _pcm(n, 200 + n)
    # do_normalize is the feature extractor's zero-mean / unit-variance step
    fe = Wav2Vec2FeatureExtractor(do_normalize=True, feature_size=1, sampling_rate=16000, padding_value=0.0)
    x = np.asarray(fe(pcm, sampling_rate=16000).input_values[0], dtype=np.float64)
    with torch.no_grad():
        out, raw = m(torch.from_numpy(x)[None])
        feat = m.wav2vec2.feature_extractor(torch.from_numpy(x)[None]).transpose(1, 2)[0].numpy()
    # the feature extractor normalises in f32; compare the conv stack on its input
    orc.do_normalize = False
    try:
        _close(orc.conv_encoder(x), feat)
        states = orc.hidden_states(x)
        for s, h in zip(states, out.hidden_states):
            _close(s, h[0].numpy())
        _close(orc.raw_outputs(x), raw[0].numpy())
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
