"""Seeded synthetic clips and random-init speaker-encoder models.

Clip (16 kHz mono f32): x[n] = sum_{h=1..5} 0.1 sin(2 pi h f0 n / 16000) + N(0, 0.01)
with f0 ~ U(100, 250) Hz; phase 0, noise standard deviation 0.01.  The stream
seeds are derived from (seed, clip index) with `rng.derive_seed`.

Models follow the shapes of the published encoders with random weights:
conv weights N(0, sqrt(2 / fan_in)) with fan_in = IC*KH*KW; a BatchNorm after
every conv with mean N(0, 0.1), var U(0.5, 1.5), gamma 1, beta 0, eps 1e-5,
folded into the conv (w' = w * g/sqrt(var+eps), b' = beta - mean*g/sqrt(var+eps))
in f32 before the weight is stored as f16 (or Q8_0).  Biases stay f32.

The GGUF layout mirrors the reference converter's WeSpeaker ResNet34 schema
(docs/conversion.md "WeSpeaker ResNet34 block manifest"): conv weights with
ggml ne = [KW, KH, IC, OC], a per-block manifest in `voicedetect.resnet.*`.
"""
import numpy as np

from . import gguf as G
from .rng import derive_seed, normal, uniform

SR = 16000
BN_EPS = 1e-5


def clip(seed, n_samples, index=0):
    """One synthetic clip as float32[n_samples]."""
    s = derive_seed(seed, 0xC11B, index)
    f0 = 100.0 + 150.0 * uniform(derive_seed(s, 1), 1)[0]
    n = np.arange(n_samples, dtype=np.float64)
    x = np.zeros(n_samples, dtype=np.float64)
    for h in range(1, 6):
        x += 0.1 * np.sin(2.0 * np.pi * h * f0 * n / SR)
    x += 0.01 * normal(derive_seed(s, 2), n_samples)
    return x.astype(np.float32)


def clips(seed, batch, n_samples):
    """float32[batch, n_samples]; clip b uses stream (seed, b)."""
    return np.stack([clip(seed, n_samples, b) for b in range(batch)])


def seconds_to_samples(sec):
    return int(round(sec * SR))


def frames_for(n_samples, win=400, hop=160):
    """Kaldi snip_edges frame count (src/fbank.cpp:130)."""
    return 0 if n_samples < win else 1 + (n_samples - win) // hop


class _WeightStream:
    """Hands out per-tensor seeds in creation order so a model is a pure function of its seed."""

    def __init__(self, seed):
        self.seed = seed
        self.k = 0

    def next(self):
        self.k += 1
        return derive_seed(self.seed, 0x5EED, self.k)


def conv_bn_folded(ws, oc, ic, kh, kw, bn=True):
    """Random conv (+ folded BN) -> (w f32 [OC,IC,KH,KW], b f32 [OC])."""
    fan_in = ic * kh * kw
    w = normal(ws.next(), oc * ic * kh * kw).reshape(oc, ic, kh, kw) * np.sqrt(2.0 / fan_in)
    w = w.astype(np.float32)
    if not bn:
        return w, np.zeros(oc, dtype=np.float32)
    mean = (0.1 * normal(ws.next(), oc)).astype(np.float32)
    var = (0.5 + uniform(ws.next(), oc)).astype(np.float32)
    scale = (np.float32(1.0) / np.sqrt(var + np.float32(BN_EPS))).astype(np.float32)
    return (w * scale[:, None, None, None]).astype(np.float32), (-mean * scale).astype(np.float32)


def _fbank_kv(n_mels=80):
    return {
        "voicedetect.fbank.sample_rate": 16000,
        "voicedetect.fbank.n_mels": n_mels,
        "voicedetect.fbank.n_fft": 512,
        "voicedetect.fbank.win_length": 400,
        "voicedetect.fbank.hop_length": 160,
        "voicedetect.fbank.preemph": G.F32(0.97),
        "voicedetect.fbank.low_freq": G.F32(20.0),
        "voicedetect.fbank.high_freq": G.F32(0.0),
        "voicedetect.fbank.use_energy": False,
        "voicedetect.fbank.cmn": True,
        "voicedetect.fbank.window": "povey",
    }


def resnet34_spec(channels=(32, 64, 128, 256), blocks=(3, 4, 6, 3), emb_dim=256, n_mels=80):
    """Block list of WeSpeaker ResNet34: (in_c, out_c, stride, has_down)."""
    out = []
    in_c = channels[0]
    for si, (c, nb) in enumerate(zip(channels, blocks)):
        for bi in range(nb):
            stride = 2 if (si > 0 and bi == 0) else 1
            down = stride != 1 or in_c != c
            out.append((in_c, c, stride, down))
            in_c = c
    return out


def make_resnet34(seed, wtype=G.GGML_F16, channels=(32, 64, 128, 256), blocks=(3, 4, 6, 3),
                  emb_dim=256, n_mels=80, mean_vec=False):
    """Random-init WeSpeaker ResNet34 -> (kv dict, tensor list) ready for gguf.write_gguf."""
    ws = _WeightStream(seed)
    tensors = []

    def add(name, w, b):
        tensors.append((name + ".weight", wtype, list(w.shape), w))
        tensors.append((name + ".bias", G.GGML_F32, [w.shape[0]], b))

    c0 = channels[0]
    w, b = conv_bn_folded(ws, c0, 1, 3, 3)
    add("front.conv1", w, b)
    m = {k: [] for k in ("conv1_weight", "conv1_bias", "conv2_weight", "conv2_bias",
                         "down_weight", "down_bias", "stride")}
    spec = resnet34_spec(channels, blocks, emb_dim, n_mels)
    li, bi = 1, 0
    counts = list(blocks)
    for (ic, oc, stride, down) in spec:
        pre = f"front.layer{li}.{bi}"
        w, b = conv_bn_folded(ws, oc, ic, 3, 3)
        add(pre + ".conv1", w, b)
        w, b = conv_bn_folded(ws, oc, oc, 3, 3)
        add(pre + ".conv2", w, b)
        m["conv1_weight"].append(pre + ".conv1.weight")
        m["conv1_bias"].append(pre + ".conv1.bias")
        m["conv2_weight"].append(pre + ".conv2.weight")
        m["conv2_bias"].append(pre + ".conv2.bias")
        if down:
            w, b = conv_bn_folded(ws, oc, ic, 1, 1)
            add(pre + ".shortcut.0", w, b)
            m["down_weight"].append(pre + ".shortcut.0.weight")
            m["down_bias"].append(pre + ".shortcut.0.bias")
        else:
            m["down_weight"].append("")
            m["down_bias"].append("")
        m["stride"].append(G.I32(stride))
        bi += 1
        if bi == counts[li - 1]:
            li, bi = li + 1, 0
    h_out = n_mels
    for s in range(len(channels) - 1):
        h_out = (h_out - 1) // 2 + 1
    pooled = 2 * channels[-1] * h_out
    seg_w = (normal(ws.next(), emb_dim * pooled).reshape(emb_dim, pooled) * np.sqrt(2.0 / pooled)).astype(np.float32)
    seg_b = (0.01 * normal(ws.next(), emb_dim)).astype(np.float32)
    tensors.append(("seg_1.weight", wtype, [emb_dim, pooled], seg_w))
    tensors.append(("seg_1.bias", G.GGML_F32, [emb_dim], seg_b))
    kv = {
        "general.architecture": "voicedetect",
        "general.name": f"synthetic-wespeaker-resnet34-seed{seed}",
        "voicedetect.arch": "wespeaker_resnet34",
        "voicedetect.embedding_dim": emb_dim,
        "voicedetect.l2_normalize": True,
    }
    kv.update(_fbank_kv(n_mels))
    kv.update({
        "voicedetect.resnet.stem_weight": "front.conv1.weight",
        "voicedetect.resnet.stem_bias": "front.conv1.bias",
        "voicedetect.resnet.conv1_weight": m["conv1_weight"],
        "voicedetect.resnet.conv1_bias": m["conv1_bias"],
        "voicedetect.resnet.conv2_weight": m["conv2_weight"],
        "voicedetect.resnet.conv2_bias": m["conv2_bias"],
        "voicedetect.resnet.down_weight": m["down_weight"],
        "voicedetect.resnet.down_bias": m["down_bias"],
        "voicedetect.resnet.stride": m["stride"],
        "voicedetect.resnet.seg_weight": "seg_1.weight",
        "voicedetect.resnet.seg_bias": "seg_1.bias",
        "voicedetect.resnet.mean_vec": "mean_vec" if mean_vec else "",
        "voicedetect.resnet.var_eps": G.F32(1e-8),
    })
    if mean_vec:
        tensors.append(("mean_vec", G.GGML_F32, [emb_dim], (0.05 * normal(ws.next(), emb_dim)).astype(np.float32)))
    return kv, tensors


def write_resnet34(path, seed, **kw):
    kv, tensors = make_resnet34(seed, **kw)
    G.write_gguf(path, kv, tensors)
    return path


# ---------------------------------------------------------------- ECAPA-TDNN

def _bn(ws, prefix, c, tensors):
    """Eval-mode BatchNorm1d parameters (gamma 1, beta 0, mean N(0,0.1), var U(0.5,1.5))."""
    tensors.append((prefix + ".weight", G.GGML_F32, [c], np.ones(c, dtype=np.float32)))
    tensors.append((prefix + ".bias", G.GGML_F32, [c], np.zeros(c, dtype=np.float32)))
    tensors.append((prefix + ".running_mean", G.GGML_F32, [c], (0.1 * normal(ws.next(), c)).astype(np.float32)))
    tensors.append((prefix + ".running_var", G.GGML_F32, [c], (0.5 + uniform(ws.next(), c)).astype(np.float32)))


def _f16_exact(a, on=True):
    """a rounded to f16-representable f32 values (on=False: a unchanged, f32)."""
    a = np.asarray(a, dtype=np.float32)
    return a.astype(np.float16).astype(np.float32) if on else a


def make_ecapa(seed, channels=1024, mfa=1536, n_mels=80, scale=8, se_ch=128, att_ch=128, emb_dim=192,
               n_res_blocks=3, k0=5, wtype=G.GGML_F16, f16_exact=True):
    """Random-init SpeechBrain ECAPA-TDNN in the reference GGUF schema.

    Tensor names and torch shapes follow models/ecapa_tdnn_manifest.txt of the
    reference.  Weight values are f16-representable; storage follows the
    reference converter's f16 plan (scripts/convert_voicedetect_to_gguf.py
    quant_plan): 1x1 weights outside fc/asp/se/tdnn1/tdnn2 (i.e. mfa) are stored
    F16 as a 2-D [OC, IC] matrix, everything else F32 (so k>1 convs keep the
    [OC, IC, K] F32 layout the reference's im2col path needs).  BatchNorm
    follows the ReLU (Conv -> ReLU -> BN), so it is kept as explicit eval-mode
    parameters, not folded.
    """
    ws = _WeightStream(seed)
    T = []

    def conv(name, oc, ic, k, quantizable=False):
        w = _f16_exact(normal(ws.next(), oc * ic * k).reshape(oc, ic, k) * np.sqrt(2.0 / (ic * k)), f16_exact)
        b = (0.01 * normal(ws.next(), oc)).astype(np.float32)
        if quantizable and k == 1 and wtype != G.GGML_F32:
            T.append((name + ".weight", wtype, [oc, ic], w.reshape(oc, ic)))
        else:
            T.append((name + ".weight", G.GGML_F32, [oc, ic, k], w))
        T.append((name + ".bias", G.GGML_F32, [oc], b))

    conv("blocks.0.conv.conv", channels, n_mels, k0)
    _bn(ws, "blocks.0.norm.norm", channels, T)
    g = channels // scale
    for i in range(1, n_res_blocks + 1):
        p = f"blocks.{i}"
        conv(p + ".tdnn1.conv.conv", channels, channels, 1)
        _bn(ws, p + ".tdnn1.norm.norm", channels, T)
        for j in range(scale - 1):
            conv(f"{p}.res2net_block.blocks.{j}.conv.conv", g, g, 3)
            _bn(ws, f"{p}.res2net_block.blocks.{j}.norm.norm", g, T)
        conv(p + ".tdnn2.conv.conv", channels, channels, 1)
        _bn(ws, p + ".tdnn2.norm.norm", channels, T)
        conv(p + ".se_block.conv1.conv", se_ch, channels, 1)
        conv(p + ".se_block.conv2.conv", channels, se_ch, 1)
    conv("mfa.conv.conv", mfa, channels * n_res_blocks, 1, quantizable=True)
    _bn(ws, "mfa.norm.norm", mfa, T)
    conv("asp.tdnn.conv.conv", att_ch, 3 * mfa, 1)
    _bn(ws, "asp.tdnn.norm.norm", att_ch, T)
    conv("asp.conv.conv", mfa, att_ch, 1)
    _bn(ws, "asp_bn.norm", 2 * mfa, T)
    conv("fc.conv", emb_dim, 2 * mfa, 1)
    kv = {
        "general.architecture": "voicedetect",
        "general.name": f"synthetic-ecapa-tdnn-seed{seed}",
        "voicedetect.arch": "ecapa_tdnn",
        "voicedetect.embedding_dim": emb_dim,
        "voicedetect.l2_normalize": True,
        "voicedetect.ecapa.channels": channels,
        "voicedetect.ecapa.n_blocks": n_res_blocks + 1,
        "voicedetect.ecapa.se_channels": se_ch,
        "voicedetect.ecapa.res2net_scale": scale,
        "voicedetect.ecapa.attention_channels": att_ch,
    }
    kv.update(_fbank_kv(n_mels))
    return kv, T


def write_ecapa(path, seed, **kw):
    kv, tensors = make_ecapa(seed, **kw)
    G.write_gguf(path, kv, tensors)
    return path


# ---------------------------------------------------------------- CAM++

def _q8_eligible(kh, kw, ic, oc):
    """The converter's quantisation rule (scripts/convert_voicedetect_to_gguf.py
    quant_plan): only 1x1 Conv1d / linear weights, blocked by 32 along IC."""
    return kh == 1 and kw == 1 and ic % 32 == 0 and ic >= 32 and oc >= 32


def _put_conv(T, wname, bname, w, b, wtype, conv1d, f16_exact=True):
    """Store a conv weight: q8_0/f16-eligible 1x1 Conv1d weights squeezed to a 2-D
    [OC, IC] matrix of `wtype`, everything else F32 ([OC,IC,K] for Conv1d,
    [OC,IC,KH,KW] for Conv2d) with f16-representable values."""
    oc, ic, kh, kw = w.shape
    if conv1d and wtype != G.GGML_F32 and _q8_eligible(kh, kw, ic, oc):
        T.append((wname, wtype, [oc, ic], w.reshape(oc, ic)))
    elif conv1d:
        T.append((wname, G.GGML_F32, [oc, ic, kw], _f16_exact(w.reshape(oc, ic, kw), f16_exact)))
    else:
        T.append((wname, G.GGML_F32, [oc, ic, kh, kw], _f16_exact(w, f16_exact)))
    if bname:
        T.append((bname, G.GGML_F32, [oc], b.astype(np.float32)))


def make_campplus(seed, n_mels=80, m_ch=32, init_ch=128, growth=32, bn_ch=128, emb_dim=192,
                  layers=(12, 24, 16), wtype=G.GGML_Q8_0, f16_exact=True):
    """Random-init 3D-Speaker CAM++ in the reference GGUF schema
    (src/model_loader.hpp:82-99, scripts/convert_voicedetect_to_gguf.py
    parse_campplus_onnx): flat execution-order conv / BN manifests.

    Convs whose BatchNorm the ONNX export folds (FCM, TDNN, each dense layer's
    linear1, the last transit) carry opaque `onnx::Conv_*` names and a bias;
    the others keep semantic names (linear_local without bias, the CAM linear1 /
    linear2 with bias, transit 1-2 and the dense head without).  Standalone
    affine BNs: each layer's nonlinear1 and each transit's nonlinear; the head
    BN is affine-free.  Weight storage follows the converter's kernel==1 rule.
    """
    ws = _WeightStream(seed)
    T = []
    conv_w, conv_b, bn_prefix = [], [], []
    nid = [0]

    def onnx_name():
        nid[0] += 1
        return f"onnx::Conv_{1000 + 2 * nid[0]}", f"onnx::Conv_{1001 + 2 * nid[0]}"

    def folded(oc, ic, kh, kw, conv1d):
        wn, bn = onnx_name()
        w, b = conv_bn_folded(ws, oc, ic, kh, kw)
        _put_conv(T, wn, bn, w, b, wtype, conv1d, f16_exact)
        conv_w.append(wn)
        conv_b.append(bn)

    def plain(name, oc, ic, k, bias):
        w = (normal(ws.next(), oc * ic * k).reshape(oc, ic, 1, k) * np.sqrt(2.0 / (ic * k))).astype(np.float32)
        b = (0.01 * normal(ws.next(), oc)).astype(np.float32) if bias else None
        _put_conv(T, name + ".weight", name + ".bias" if bias else "", w, b, wtype, True, f16_exact)
        conv_w.append(name + ".weight")
        conv_b.append(name + ".bias" if bias else "")

    def affine_bn(prefix, c):
        _bn(ws, prefix, c, T)
        bn_prefix.append(prefix)

    # FCM: stem, 2 x (stride-2 block with shortcut, stride-1 block), final conv
    folded(m_ch, 1, 3, 3, False)
    for stride in (2, 1, 2, 1):
        folded(m_ch, m_ch, 3, 3, False)
        folded(m_ch, m_ch, 3, 3, False)
        if stride != 1:
            folded(m_ch, m_ch, 1, 1, False)
    folded(m_ch, m_ch, 3, 3, False)
    H = n_mels
    for _ in range(3):
        H = (H - 1) // 2 + 1
    fcm_out = m_ch * H
    # TDNN 320 -> init_ch, k=5 s2 (BN folded)
    folded(init_ch, fcm_out, 1, 5, True)
    C = init_ch
    for b, nl in enumerate(layers, start=1):
        for l in range(1, nl + 1):
            p = f"xvector.block{b}.tdnnd{l}"
            affine_bn(p + ".nonlinear1.batchnorm", C)
            folded(bn_ch, C, 1, 1, True)                                   # linear1 (+ nonlinear2 BN)
            plain(p + ".cam_layer.linear_local", growth, bn_ch, 3, False)
            plain(p + ".cam_layer.linear1", bn_ch // 2, bn_ch, 1, True)
            plain(p + ".cam_layer.linear2", growth, bn_ch // 2, 1, True)
            C += growth
        affine_bn(f"xvector.transit{b}.nonlinear.batchnorm", C)
        if b < len(layers):
            plain(f"xvector.transit{b}.linear", C // 2, C, 1, False)
        else:
            folded(C // 2, C, 1, 1, True)                                  # transit3 (+ out BN)
        C //= 2
    plain("xvector.dense.linear", emb_dim, 2 * C, 1, False)
    mean = (0.1 * normal(ws.next(), emb_dim)).astype(np.float32)
    var = (0.5 + uniform(ws.next(), emb_dim)).astype(np.float32)
    T.append(("xvector.dense.nonlinear.batchnorm.running_mean", G.GGML_F32, [emb_dim], mean))
    T.append(("xvector.dense.nonlinear.batchnorm.running_var", G.GGML_F32, [emb_dim], var))
    kv = {
        "general.architecture": "voicedetect",
        "general.name": f"synthetic-campplus-seed{seed}",
        "voicedetect.arch": "campplus",
        "voicedetect.embedding_dim": emb_dim,
        "voicedetect.l2_normalize": True,
        "voicedetect.campplus.conv_weight": conv_w,
        "voicedetect.campplus.conv_bias": conv_b,
        "voicedetect.campplus.bn_prefix": bn_prefix,
        "voicedetect.campplus.emb_bn_mean": "xvector.dense.nonlinear.batchnorm.running_mean",
        "voicedetect.campplus.emb_bn_var": "xvector.dense.nonlinear.batchnorm.running_var",
        "voicedetect.campplus.bn_eps": 1e-5,
    }
    kv.update(_fbank_kv(n_mels))
    return kv, T


def write_campplus(path, seed, **kw):
    kv, tensors = make_campplus(seed, **kw)
    G.write_gguf(path, kv, tensors)
    return path


# ---------------------------------------------------------------- ERes2Net

def make_eres2net(seed, n_mels=80, m_ch=32, num_blocks=(3, 4, 6, 3), base_width=32, scale=2, emb_dim=512,
                  wtype=G.GGML_Q8_0, f16_exact=True):
    """Random-init 3D-Speaker ERes2Net in the reference GGUF schema
    (src/model_loader.hpp:68-79, scripts/convert_voicedetect_to_gguf.py
    parse_eres2net_onnx): every conv BN-folded with an opaque `onnx::Conv_*`
    name and a bias, except the three bias-free cross-stage downsample convs;
    the flat manifest lists the convs in forward order with their strides.
    Storage follows the converter's kernel==1 rule (1x1 convs and seg_1 as
    2-D matrices of `wtype`, 3x3 convs F32 with f16-representable values)."""
    ws = _WeightStream(seed)
    T = []
    conv_w, conv_b, conv_s = [], [], []
    nid = [0]

    def conv(oc, ic, k, stride, bias=True):
        nid[0] += 1
        wn, bn = f"onnx::Conv_{3000 + 2 * nid[0]}", f"onnx::Conv_{3001 + 2 * nid[0]}"
        w, b = conv_bn_folded(ws, oc, ic, k, k, bn=bias)
        if k == 1 and wtype != G.GGML_F32 and _q8_eligible(1, 1, ic, oc):
            T.append((wn, wtype, [oc, ic], w.reshape(oc, ic)))
        else:
            T.append((wn, G.GGML_F32, [oc, ic, k, k], _f16_exact(w, f16_exact)))
        if bias:
            T.append((bn, G.GGML_F32, [oc], b))
        conv_w.append(wn)
        conv_b.append(bn if bias else "")
        conv_s.append(stride)

    def aff(channels):
        inter = channels // 4
        conv(inter, 2 * channels, 1, 1)
        conv(channels, inter, 1, 1)

    conv(m_ch, 1, 3, 1)                                     # stem
    in_planes = m_ch
    for li, (nb, stride) in enumerate(zip(num_blocks, (1, 2, 2, 2))):
        planes = m_ch * (2 ** li)
        width = planes * base_width // 64
        for bi in range(nb):
            s = stride if bi == 0 else 1
            conv(width * scale, in_planes, 1, s)            # conv1
            for i in range(scale):
                if i > 0 and li >= 2:
                    aff(width)                              # diff_AFF scale fusion
                conv(width, width, 3, 1)                    # convs[i]
            conv(2 * planes, width * scale, 1, 1)           # conv3
            if s != 1 or in_planes != 2 * planes:
                conv(2 * planes, in_planes, 1, s)           # shortcut
            in_planes = 2 * planes
        if li >= 1:
            # after layer li+1: downsample of the previous fused feature, then AFF
            conv(2 * planes, planes, 3, 2, bias=False)
            aff(2 * planes)
    H = n_mels // 8
    stats = 2 * in_planes * H
    w = (normal(ws.next(), emb_dim * stats).reshape(emb_dim, stats) * np.sqrt(1.0 / stats)).astype(np.float32)
    b = (0.01 * normal(ws.next(), emb_dim)).astype(np.float32)
    if wtype != G.GGML_F32 and stats % 32 == 0:
        T.append(("seg_1.weight", wtype, [emb_dim, stats], w))
    else:
        T.append(("seg_1.weight", G.GGML_F32, [emb_dim, stats], _f16_exact(w)))
    T.append(("seg_1.bias", G.GGML_F32, [emb_dim], b))
    kv = {
        "general.architecture": "voicedetect",
        "general.name": f"synthetic-eres2net-seed{seed}",
        "voicedetect.arch": "eres2net",
        "voicedetect.embedding_dim": emb_dim,
        "voicedetect.l2_normalize": True,
        "voicedetect.eres2net.conv_weight": conv_w,
        "voicedetect.eres2net.conv_bias": conv_b,
        "voicedetect.eres2net.conv_stride": [G.I32(s) for s in conv_s],
        "voicedetect.eres2net.num_blocks": [G.I32(n) for n in num_blocks],
        "voicedetect.eres2net.m_channels": m_ch,
        "voicedetect.eres2net.scale": scale,
        "voicedetect.eres2net.seg_weight": "seg_1.weight",
        "voicedetect.eres2net.seg_bias": "seg_1.bias",
        "voicedetect.eres2net.relu_clamp": 20.0,
        "voicedetect.eres2net.var_eps": 1e-8,
    }
    kv.update(_fbank_kv(n_mels))
    return kv, T


def write_eres2net(path, seed, **kw):
    kv, tensors = make_eres2net(seed, **kw)
    G.write_gguf(path, kv, tensors)
    return path


# ---------------------------------------------------------------- wav2vec2 analyze

EMOTION_LABELS = ["neu", "hap", "ang", "sad"]
GENDER_LABELS = ["female", "male", "child"]


def w2v2_store_name(name):
    """The reference converter's name transform for the analyze archs
    (scripts/convert_voicedetect_to_gguf.py:127-140): module prefix wav2vec2. ->
    w2v2., weight-norm parametrization original0/original1 -> weight_g/weight_v."""
    if name.startswith("wav2vec2."):
        name = "w2v2." + name[len("wav2vec2."):]
    name = name.replace(".parametrizations.weight.original0", ".weight_g")
    return name.replace(".parametrizations.weight.original1", ".weight_v")


def w2v2_kv(kind, hidden, n_layers, n_heads, ff, conv_dims, conv_kernels, conv_strides, pos_k, pos_groups,
            proj, labels, eps=1e-5):
    """KV of an analyze GGUF (scripts/convert_voicedetect_to_gguf.py:725-763;
    docs/conversion.md "wav2vec2 emotion / age-gender analyze head")."""
    large = kind == "age_gender"
    kv = {
        "general.architecture": "voicedetect",
        "voicedetect.arch": "wav2vec2_age_gender" if large else "wav2vec2_emotion",
        "voicedetect.analyze.present": True,
        "voicedetect.analyze.kind": kind,
        "voicedetect.analyze.pooling": "mean",
        "voicedetect.w2v2.conv_bias": large,
        "voicedetect.w2v2.do_normalize": large,
        "voicedetect.w2v2.hidden_size": hidden,
        "voicedetect.w2v2.n_layers": n_layers,
        "voicedetect.w2v2.n_heads": n_heads,
        "voicedetect.w2v2.ff_dim": ff,
        "voicedetect.w2v2.num_conv_layers": len(conv_dims),
        "voicedetect.w2v2.conv_dims": [G.I32(v) for v in conv_dims],
        "voicedetect.w2v2.conv_kernels": [G.I32(v) for v in conv_kernels],
        "voicedetect.w2v2.conv_strides": [G.I32(v) for v in conv_strides],
        "voicedetect.w2v2.feat_extract_norm": "layer" if large else "group",
        "voicedetect.w2v2.feat_extract_activation": "gelu",
        "voicedetect.w2v2.hidden_act": "gelu",
        "voicedetect.w2v2.do_stable_layer_norm": large,
        "voicedetect.w2v2.layer_norm_eps": float(eps),
        "voicedetect.w2v2.num_conv_pos_embeddings": pos_k,
        "voicedetect.w2v2.num_conv_pos_embedding_groups": pos_groups,
        "voicedetect.w2v2.pos_conv_weight_norm_dim": 2,
        "voicedetect.w2v2.use_weighted_layer_sum": not large,
        "voicedetect.w2v2.classifier_proj_size": proj,
    }
    if large:
        kv["voicedetect.analyze.gender_labels"] = list(labels)
        kv["voicedetect.analyze.num_genders"] = len(labels)
    else:
        kv["voicedetect.analyze.emotion_labels"] = list(labels)
        kv["voicedetect.analyze.num_emotions"] = len(labels)
    return kv


W2V2_BASE = dict(hidden=768, n_layers=12, n_heads=12, ff=3072, conv_dims=(512,) * 7,
                 conv_kernels=(10, 3, 3, 3, 3, 2, 2), conv_strides=(5, 2, 2, 2, 2, 2, 2), pos_k=128,
                 pos_groups=16, proj=256)
W2V2_LARGE = dict(W2V2_BASE, hidden=1024, n_layers=24, n_heads=16, ff=4096)


def make_w2v2(seed, kind="emotion", labels=None, **dims):
    """Random-init wav2vec2 analyze model (emotion: wav2vec2-base with the
    weighted-layer-sum classifier; age_gender: wav2vec2-large-robust with the
    audeering age/gender heads) in the reference GGUF schema, all tensors F32
    as the reference converter stores them.  Matrix values are f16-exact.

    Init: conv N(0, sqrt(2/fan_in)); linear N(0, sqrt(1/fan_in)), bias N(0, 0.02);
    LayerNorm / GroupNorm gamma 1 + N(0, 0.1), beta N(0, 0.1); positional conv
    weight_v N(0, 1), weight_g U(1, 3); layer_weights N(0, 1).
    """
    d = dict(W2V2_LARGE if kind == "age_gender" else W2V2_BASE)
    d.update(dims)
    large = kind == "age_gender"
    if labels is None:
        labels = GENDER_LABELS if large else EMOTION_LABELS
    H, L, FF = d["hidden"], d["n_layers"], d["ff"]
    ws = _WeightStream(seed)
    T = []

    def put(name, arr):
        arr = np.asarray(arr, dtype=np.float32)
        T.append((w2v2_store_name(name), G.GGML_F32, list(arr.shape), arr))

    def mat(shape, std):
        n = int(np.prod(shape))
        return _f16_exact(normal(ws.next(), n).reshape(shape) * std)

    def vec(n, std, mean=0.0):
        return (mean + std * normal(ws.next(), n)).astype(np.float32)

    def norm(name, c):
        put(name + ".weight", vec(c, 0.1, 1.0))
        put(name + ".bias", vec(c, 0.1))

    def linear(name, o, i):
        put(name + ".weight", mat((o, i), np.sqrt(1.0 / i)))
        put(name + ".bias", vec(o, 0.02))

    ic = 1
    for i, (oc, k) in enumerate(zip(d["conv_dims"], d["conv_kernels"])):
        p = f"wav2vec2.feature_extractor.conv_layers.{i}"
        put(p + ".conv.weight", mat((oc, ic, k), np.sqrt(2.0 / (ic * k))))
        if large:
            put(p + ".conv.bias", vec(oc, 0.02))
            norm(p + ".layer_norm", oc)
        elif i == 0:
            norm(p + ".layer_norm", oc)
        ic = oc
    norm("wav2vec2.feature_projection.layer_norm", ic)
    linear("wav2vec2.feature_projection.projection", H, ic)
    K, groups = d["pos_k"], d["pos_groups"]
    pc = "wav2vec2.encoder.pos_conv_embed.conv"
    put(pc + ".parametrizations.weight.original0", (1.0 + 2.0 * uniform(ws.next(), K)).reshape(1, 1, K))
    put(pc + ".parametrizations.weight.original1", mat((H, H // groups, K), 1.0))
    put(pc + ".bias", vec(H, 0.02))
    norm("wav2vec2.encoder.layer_norm", H)
    for i in range(L):
        p = f"wav2vec2.encoder.layers.{i}"
        for n in ("q_proj", "k_proj", "v_proj", "out_proj"):
            linear(f"{p}.attention.{n}", H, H)
        norm(p + ".layer_norm", H)
        linear(p + ".feed_forward.intermediate_dense", FF, H)
        linear(p + ".feed_forward.output_dense", H, FF)
        norm(p + ".final_layer_norm", H)
    if large:
        for head, n_out in (("age", 1), ("gender", len(labels))):
            linear(head + ".dense", H, H)
            linear(head + ".out_proj", n_out, H)
    else:
        put("layer_weights", vec(L + 1, 1.0))
        linear("projector", d["proj"], H)
        linear("classifier", len(labels), d["proj"])
    kv = w2v2_kv(kind, H, L, d["n_heads"], FF, d["conv_dims"], d["conv_kernels"], d["conv_strides"], K, groups,
                 d["proj"], labels)
    kv["general.name"] = f"synthetic-wav2vec2-{kind}-seed{seed}"
    return kv, T


def write_w2v2(path, seed, kind="emotion", **kw):
    kv, tensors = make_w2v2(seed, kind, **kw)
    G.write_gguf(path, kv, tensors)
    return path
