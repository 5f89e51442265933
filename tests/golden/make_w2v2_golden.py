"""Write the wav2vec2 golden vectors from HF transformers.

The reference's analyze goldens are HF transformers outputs
(scripts/gen_baseline.py --analyze; tests/test_analyze.cpp,
tests/test_age_gender.cpp).  This script builds HF's own Wav2Vec2 modules
offline from a small config with seeded random weights, runs them in f64 and
stores, per variant, the weights (under the reference converter's tensor names,
scripts/convert_voicedetect_to_gguf.py:127-140, rounded to f32 as a GGUF holds
them), the config (the input clips are vdamd.synth's seeded clips, regenerated
by the test) and every output the oracle is checked
against: the conv feature encoder output, every hidden state and the head
outputs.  Output: tests/golden/w2v2_golden.npz.

Variants: wav2vec2-base emotion (Wav2Vec2ForSequenceClassification: group-norm
conv0, post-norm layers, weighted layer sum, projector + classifier) and
wav2vec2-large-robust age/gender (Wav2Vec2Model with layer-norm convs with
bias, pre-norm layers, the audeering two-head AgeGenderModel, inputs through
Wav2Vec2FeatureExtractor(do_normalize=True)).

Runs in the development container only (needs torch and transformers, which
tests never import).  transformers version used: printed into the file.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "voice-detect.cpp_amd"))
os.environ.setdefault("HF_HUB_OFFLINE", "1")
os.environ.setdefault("TRANSFORMERS_OFFLINE", "1")

import torch  # noqa: E402
import transformers  # noqa: E402
from transformers import (Wav2Vec2Config, Wav2Vec2FeatureExtractor, Wav2Vec2ForSequenceClassification,  # noqa: E402
                          Wav2Vec2Model)

from vdamd import synth  # noqa: E402

CONV = dict(conv_dim=(32, 32, 32, 32, 32, 32, 32), conv_kernel=(10, 3, 3, 3, 3, 2, 2),
            conv_stride=(5, 2, 2, 2, 2, 2, 2))
EMOTION_LENGTHS = (4000, 8000, 12345)
AGE_GENDER_LENGTHS = (4000, 9001)


def hf_config(large):
    return Wav2Vec2Config(
        hidden_size=64, num_hidden_layers=3, num_attention_heads=4, intermediate_size=96, **CONV,
        feat_extract_norm="layer" if large else "group", conv_bias=large, do_stable_layer_norm=large,
        num_conv_pos_embeddings=16, num_conv_pos_embedding_groups=4, use_weighted_layer_sum=not large,
        classifier_proj_size=24, num_labels=4, layer_norm_eps=1e-5, hidden_dropout=0.0, attention_dropout=0.0,
        activation_dropout=0.0, feat_proj_dropout=0.0, final_dropout=0.0, layerdrop=0.0, mask_time_prob=0.0)


class AgeGender(torch.nn.Module):
    """audeering AgeGenderModel: Wav2Vec2Model + two ModelHeads
    out_proj(tanh(dense(mean_t(last_hidden_state))))."""

    def __init__(self, cfg):
        super().__init__()
        self.wav2vec2 = Wav2Vec2Model(cfg)
        H = cfg.hidden_size
        self.age = torch.nn.ModuleDict(dict(dense=torch.nn.Linear(H, H), out_proj=torch.nn.Linear(H, 1)))
        self.gender = torch.nn.ModuleDict(dict(dense=torch.nn.Linear(H, H), out_proj=torch.nn.Linear(H, 3)))

    def forward(self, x):
        out = self.wav2vec2(x, output_hidden_states=True)
        pooled = out.last_hidden_state.mean(dim=1)
        heads = [h["out_proj"](torch.tanh(h["dense"](pooled))) for h in (self.age, self.gender)]
        return out, torch.cat(heads, dim=1)


def f32_weights(model):
    """Round the f64 model's weights to f32 so the GGUF and HF see the same values."""
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(p.float().double())


def store(out, prefix, model, cfg):
    for name, t in model.state_dict().items():
        if name.startswith("wav2vec2.masked_spec_embed"):
            continue
        out[f"{prefix}/w/{synth.w2v2_store_name(name)}"] = t.detach().cpu().numpy().astype(np.float32)
    out[f"{prefix}/config"] = np.array(json.dumps(dict(
        hidden=cfg.hidden_size, n_layers=cfg.num_hidden_layers, n_heads=cfg.num_attention_heads,
        ff=cfg.intermediate_size, conv_dims=list(cfg.conv_dim), conv_kernels=list(cfg.conv_kernel),
        conv_strides=list(cfg.conv_stride), pos_k=cfg.num_conv_pos_embeddings,
        pos_groups=cfg.num_conv_pos_embedding_groups, proj=cfg.classifier_proj_size, eps=cfg.layer_norm_eps)))


def main():
    out = {"transformers_version": np.array(transformers.__version__)}
    # emotion
    torch.manual_seed(7)
    cfg = hf_config(False)
    m = Wav2Vec2ForSequenceClassification(cfg).double().eval()
    with torch.no_grad():
        m.layer_weights.copy_(torch.randn(cfg.num_hidden_layers + 1, dtype=torch.float64))
    f32_weights(m)
    store(out, "emotion", m, cfg)
    for n in EMOTION_LENGTHS:
        pcm = synth.clip(100 + n, n).astype(np.float64)
        with torch.no_grad():
            r = m(torch.from_numpy(pcm)[None], output_hidden_states=True)
            feat = m.wav2vec2.feature_extractor(torch.from_numpy(pcm)[None]).transpose(1, 2)[0].numpy()
        p = f"emotion/n{n}"   # input: vdamd.synth.clip(100 + n, n), regenerated by the test
        out[p + "/feat"] = feat
        out[p + "/hidden"] = np.stack([h[0].numpy() for h in r.hidden_states])
        out[p + "/raw"] = r.logits[0].numpy()
    # age / gender
    torch.manual_seed(11)
    cfg = hf_config(True)
    m = AgeGender(cfg).double().eval()
    f32_weights(m)
    store(out, "age_gender", m, cfg)
    fe = Wav2Vec2FeatureExtractor(do_normalize=True, feature_size=1, sampling_rate=16000, padding_value=0.0)
    for n in AGE_GENDER_LENGTHS:
        pcm = synth.clip(200 + n, n).astype(np.float64)
        x = np.asarray(fe(pcm, sampling_rate=16000).input_values[0], dtype=np.float64)
        with torch.no_grad():
            r, raw = m(torch.from_numpy(x)[None])
            feat = m.wav2vec2.feature_extractor(torch.from_numpy(x)[None]).transpose(1, 2)[0].numpy()
        p = f"age_gender/n{n}"   # input: vdamd.synth.clip(200 + n, n)
        out[p + "/normalized"] = x          # the feature extractor's do_normalize output
        out[p + "/feat"] = feat
        out[p + "/hidden"] = np.stack([h[0].numpy() for h in r.hidden_states])
        out[p + "/raw"] = raw[0].numpy()
    path = os.path.join(HERE, "w2v2_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, transformers {transformers.__version__})")


if __name__ == "__main__":
    main()
