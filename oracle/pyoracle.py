"""ctypes binding of the oracle (liboracle.so) and of oracle/_ref/libref.so.

TEST INFRASTRUCTURE ONLY: imported by the test suite, the smoke check and the
CPU-baseline leg of bench.py.  Results are compared against it; it is never
the thing measured.
"""
import contextlib
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

F32P = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
F64P = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")


class FbankCfg(C.Structure):
    _fields_ = [("sample_rate", C.c_int), ("n_mels", C.c_int), ("n_fft", C.c_int),
                ("win_length", C.c_int), ("hop_length", C.c_int), ("preemph", C.c_float),
                ("low_freq", C.c_float), ("high_freq", C.c_float), ("cmn", C.c_int)]


MAXB = 32
_fp = C.POINTER(C.c_float)


class ResNet(C.Structure):
    _fields_ = [("n_mels", C.c_int), ("stem_oc", C.c_int), ("stem_w", _fp), ("stem_b", _fp),
                ("n_blocks", C.c_int),
                ("in_c", C.c_int * MAXB), ("out_c", C.c_int * MAXB), ("stride", C.c_int * MAXB),
                ("conv1_w", _fp * MAXB), ("conv1_b", _fp * MAXB),
                ("conv2_w", _fp * MAXB), ("conv2_b", _fp * MAXB),
                ("down_w", _fp * MAXB), ("down_b", _fp * MAXB),
                ("seg_w", _fp), ("seg_b", _fp), ("mean_vec", _fp),
                ("emb_dim", C.c_int), ("var_eps", C.c_float), ("l2_normalize", C.c_int)]


class ResNetCaps(C.Structure):
    _fields_ = [("stem", _fp), ("block", _fp * MAXB), ("pooled", _fp), ("pre_norm", _fp)]


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle not built: {path} (run make -C oracle)")
        _LIB = _load(path)
    return _LIB


@contextlib.contextmanager
def using_library(path):
    """Run the oracle wrappers against another build of the oracle sources
    (the mutation tests' deliberately broken copies), then restore."""
    global _LIB
    saved = _LIB
    _LIB = _load(path)
    try:
        yield _LIB
    finally:
        _LIB = saved


def _load(path):
    L = C.CDLL(path)
    L.orc_fbank_frames.argtypes = [C.c_int, C.POINTER(FbankCfg)]
    L.orc_fbank.argtypes = [F32P, C.c_int, C.POINTER(FbankCfg), F32P]
    L.orc_powspec.argtypes = [F32P, C.c_int, C.c_int, C.c_int, F64P]
    L.orc_mel_filters.argtypes = [C.POINTER(FbankCfg), F64P]
    L.orc_povey_window.argtypes = [C.c_int, F64P]
    conv = [F32P, C.c_int, C.c_int, C.c_int, F32P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
            C.c_void_p, C.c_void_p, C.c_int]
    L.orc_conv2d_f32.argtypes = conv + [F32P]
    L.orc_conv2d_f64.argtypes = conv + [F64P]
    L.orc_tstp.argtypes = [F32P, C.c_int, C.c_int, C.c_int, C.c_float, F32P]
    L.orc_linear.argtypes = [F32P, C.c_int, F32P, C.c_void_p, C.c_void_p, C.c_int, F32P]
    L.orc_l2norm.argtypes = [F32P, C.c_int]
    L.orc_resnet34_forward.argtypes = [C.POINTER(ResNet), F32P, C.c_int, F32P, C.POINTER(ResNetCaps)]
    L.orc_embed_batch.argtypes = [C.POINTER(ResNet), C.POINTER(FbankCfg), F32P, C.c_int, C.c_int,
                                  C.c_int, F32P]
    return L


def ref_lib():
    """oracle/_ref/libref.so (the reference's own FBank/WAV code) or None if not built."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libref.so")
        if not os.path.exists(path):
            return None
        L = C.CDLL(path)
        L.ref_fbank.argtypes = [F32P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                C.c_float, C.c_float, C.c_int, F32P, C.c_long]
        L.ref_fbank.restype = C.c_int
        L.ref_load_wav.argtypes = [C.c_char_p, F32P, C.c_long]
        L.ref_load_wav.restype = C.c_long
        L.ref_resample.argtypes = [F32P, C.c_long, C.c_int, C.c_int, F32P, C.c_long]
        L.ref_resample.restype = C.c_long
        _REF = L
    return _REF


def fbank_cfg(n_mels=80, n_fft=512, win=400, hop=160, preemph=0.97, low=20.0, high=0.0, cmn=True,
              sample_rate=16000):
    return FbankCfg(sample_rate, n_mels, n_fft, win, hop, preemph, low, high, int(cmn))


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def fbank(pcm, cfg=None):
    cfg = cfg or fbank_cfg()
    pcm = np.ascontiguousarray(pcm, dtype=np.float32)
    T = lib().orc_fbank_frames(len(pcm), C.byref(cfg))
    out = np.zeros((cfg.n_mels, max(T, 1)), dtype=np.float32)
    T2 = lib().orc_fbank(pcm, len(pcm), C.byref(cfg), out)
    assert T2 == T
    return out[:, :T]


def ref_fbank(pcm, cfg=None):
    cfg = cfg or fbank_cfg()
    L = ref_lib()
    pcm = np.ascontiguousarray(pcm, dtype=np.float32)
    cap = cfg.n_mels * (len(pcm) // max(cfg.hop_length, 1) + 2)
    out = np.zeros(cap, dtype=np.float32)
    T = L.ref_fbank(pcm, len(pcm), cfg.n_mels, cfg.n_fft, cfg.win_length, cfg.hop_length,
                    cfg.preemph, cfg.low_freq, cfg.high_freq, cfg.cmn, out, cap)
    assert T >= 0
    return out[: cfg.n_mels * T].reshape(cfg.n_mels, T)


def powspec(frame, n_fft, use_dft=False):
    frame = np.ascontiguousarray(frame, dtype=np.float32)
    out = np.zeros(n_fft // 2 + 1)
    lib().orc_powspec(frame, len(frame), n_fft, int(use_dft), out)
    return out


def mel_filters(cfg=None):
    cfg = cfg or fbank_cfg()
    fb = np.zeros((cfg.n_mels, cfg.n_fft // 2 + 1))
    lib().orc_mel_filters(C.byref(cfg), fb)
    return fb


def povey(win):
    w = np.zeros(win)
    lib().orc_povey_window(win, w)
    return w


def conv2d(x, w, stride=1, pad=1, bias=None, residual=None, relu=False, f64=False):
    """x [IC,H,W] f32, w [OC,IC,KH,KW] -> [OC,Ho,Wo] (f32 or f64)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    IC, H, W = x.shape
    OC, IC2, KH, KW = w.shape
    assert IC == IC2
    Ho, Wo = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    r = None if residual is None else np.ascontiguousarray(residual, dtype=np.float32)
    if r is not None:
        assert r.shape == (OC, Ho, Wo)
    y = np.zeros((OC, Ho, Wo), dtype=np.float64 if f64 else np.float32)
    fn = lib().orc_conv2d_f64 if f64 else lib().orc_conv2d_f32
    fn(x, IC, H, W, w, OC, KH, KW, stride, pad, _p(b), _p(r), int(relu), y)
    return y


def tstp(x, eps=1e-8):
    x = np.ascontiguousarray(x, dtype=np.float32)
    Cc, H, W = x.shape
    out = np.zeros(2 * Cc * H, dtype=np.float32)
    lib().orc_tstp(x, Cc, H, W, eps, out)
    return out


def linear(x, w, b=None, mean_vec=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out_dim, in_dim = w.shape
    y = np.zeros(out_dim, dtype=np.float32)
    bb = None if b is None else np.ascontiguousarray(b, dtype=np.float32)
    mv = None if mean_vec is None else np.ascontiguousarray(mean_vec, dtype=np.float32)
    lib().orc_linear(x, in_dim, w, _p(bb), _p(mv), out_dim, y)
    return y


def l2norm(v):
    v = np.array(v, dtype=np.float32, copy=True)
    lib().orc_l2norm(v, len(v))
    return v


def verify_distance(ea, eb):
    """The reference's verify distance, 1 - sum(ea * eb) accumulated in double
    (src/model.cpp:65-78)."""
    return 1.0 - float(np.dot(np.asarray(ea, dtype=np.float64), np.asarray(eb, dtype=np.float64)))


def registry_topk(q, reg, k):
    """Identify against an enrolled registry (no reference function: README.md:15
    promises identify; the score follows verify, src/model.cpp:65-78): scores
    q @ reg.T in f64 over f32 values (each product exact), the k best rows per
    query, highest score first, equal scores by the lower row index.
    Returns (idx [B][k] int32, score [B][k] f64)."""
    s = np.asarray(q, dtype=np.float32).astype(np.float64) @ np.asarray(reg, dtype=np.float32).astype(np.float64).T
    idx = np.argsort(-s, axis=1, kind="stable")[:, :k]   # stable: equal scores keep the lower row first
    return idx.astype(np.int32), np.take_along_axis(s, idx, axis=1)


class OracleResNet:
    """orc_resnet built from a parsed GGUF (vdamd.gguf.GGUFFile), weights dequantised to f32."""

    def __init__(self, g):
        kv = g.kv
        self.keep = []
        n = ResNet()

        def ptr(name):
            a = np.ascontiguousarray(g.array(name), dtype=np.float32)
            self.keep.append(a)
            return a.ctypes.data_as(_fp)

        pre = "voicedetect.resnet."
        n.n_mels = int(kv.get("voicedetect.fbank.n_mels", 80))
        stem = g.array(kv[pre + "stem_weight"])
        n.stem_oc = stem.shape[0]
        n.stem_w = ptr(kv[pre + "stem_weight"])
        n.stem_b = ptr(kv[pre + "stem_bias"])
        nb = len(kv[pre + "conv1_weight"])
        assert nb <= MAXB
        n.n_blocks = nb
        for i in range(nb):
            w1 = g.array(kv[pre + "conv1_weight"][i])
            n.out_c[i], n.in_c[i] = w1.shape[0], w1.shape[1]
            n.stride[i] = kv[pre + "stride"][i]
            n.conv1_w[i] = ptr(kv[pre + "conv1_weight"][i])
            n.conv1_b[i] = ptr(kv[pre + "conv1_bias"][i])
            n.conv2_w[i] = ptr(kv[pre + "conv2_weight"][i])
            n.conv2_b[i] = ptr(kv[pre + "conv2_bias"][i])
            dw = kv[pre + "down_weight"][i]
            n.down_w[i] = ptr(dw) if dw else None
            n.down_b[i] = ptr(kv[pre + "down_bias"][i]) if dw else None
        seg = g.array(kv[pre + "seg_weight"])
        n.emb_dim = seg.shape[0]
        n.seg_w = ptr(kv[pre + "seg_weight"])
        n.seg_b = ptr(kv[pre + "seg_bias"]) if kv.get(pre + "seg_bias") else None
        mv = kv.get(pre + "mean_vec", "")
        n.mean_vec = ptr(mv) if mv else None
        n.var_eps = float(kv.get(pre + "var_eps", 1e-8))
        n.l2_normalize = int(bool(kv.get("voicedetect.l2_normalize", True)))
        self.net = n
        self.blocks = [(n.in_c[i], n.out_c[i], n.stride[i]) for i in range(nb)]

    def block_shapes(self, T):
        H, W = self.net.n_mels, T
        out = []
        for (_, oc, s) in self.blocks:
            H, W = (H - 1) // s + 1, (W - 1) // s + 1
            out.append((oc, H, W))
        return out

    def forward(self, feats, capture=False):
        feats = np.ascontiguousarray(feats, dtype=np.float32)
        T = feats.shape[1]
        emb = np.zeros(self.net.emb_dim, dtype=np.float32)
        caps = ResNetCaps()
        bufs = {}
        if capture:
            bufs["stem"] = np.zeros((self.net.stem_oc, self.net.n_mels, T), dtype=np.float32)
            caps.stem = bufs["stem"].ctypes.data_as(_fp)
            for i, shp in enumerate(self.block_shapes(T)):
                bufs[f"block{i}"] = np.zeros(shp, dtype=np.float32)
                caps.block[i] = bufs[f"block{i}"].ctypes.data_as(_fp)
            oc, H, W = self.block_shapes(T)[-1]
            bufs["pooled"] = np.zeros(2 * oc * H, dtype=np.float32)
            caps.pooled = bufs["pooled"].ctypes.data_as(_fp)
            bufs["pre_norm"] = np.zeros(self.net.emb_dim, dtype=np.float32)
            caps.pre_norm = bufs["pre_norm"].ctypes.data_as(_fp)
        rc = lib().orc_resnet34_forward(C.byref(self.net), feats, T, emb, C.byref(caps))
        assert rc == 0
        return (emb, bufs) if capture else emb

    def embed_batch(self, pcm, n_threads=1, cfg=None):
        cfg = cfg or fbank_cfg(n_mels=self.net.n_mels)
        pcm = np.ascontiguousarray(pcm, dtype=np.float32)
        B, n = pcm.shape
        out = np.zeros((B, self.net.emb_dim), dtype=np.float32)
        rc = lib().orc_embed_batch(C.byref(self.net), C.byref(cfg), pcm, B, n, n_threads, out)
        assert rc == 0
        return out


# ---------------------------------------------------------------- ECAPA-TDNN

class Conv1d(C.Structure):
    _fields_ = [("w", _fp), ("b", _fp), ("oc", C.c_int), ("ic", C.c_int), ("k", C.c_int)]


class BN(C.Structure):
    _fields_ = [("gamma", _fp), ("beta", _fp), ("mean", _fp), ("var", _fp), ("c", C.c_int)]


MAXR, MAXS = 8, 16


class Ecapa(C.Structure):
    _fields_ = [("n_mels", C.c_int), ("channels", C.c_int), ("scale", C.c_int), ("n_res", C.c_int),
                ("mfa_ch", C.c_int), ("emb_dim", C.c_int), ("l2_normalize", C.c_int),
                ("block0", Conv1d), ("bn0", BN),
                ("tdnn1", Conv1d * MAXR), ("tdnn2", Conv1d * MAXR), ("se1", Conv1d * MAXR), ("se2", Conv1d * MAXR),
                ("bn_t1", BN * MAXR), ("bn_t2", BN * MAXR),
                ("res", (Conv1d * MAXS) * MAXR), ("bn_res", (BN * MAXS) * MAXR),
                ("mfa", Conv1d), ("bn_mfa", BN),
                ("asp_tdnn", Conv1d), ("bn_asp", BN), ("asp_conv", Conv1d), ("asp_bn", BN),
                ("fc", Conv1d)]


class EcapaCaps(C.Structure):
    _fields_ = [("block", _fp * (MAXR + 1)), ("mfa", _fp), ("pooled", _fp), ("pre_norm", _fp)]


def _ecapa_sigs():
    L = lib()
    if not hasattr(L, "_ecapa_ready"):
        L.orc_conv1d_same.argtypes = [F32P, C.c_int, C.POINTER(Conv1d), C.c_int, F32P]
        L.orc_bn_apply.argtypes = [F32P, C.c_int, C.POINTER(BN)]
        L.orc_ecapa_asp.argtypes = [C.POINTER(Ecapa), F32P, C.c_int, F32P]
        L.orc_ecapa_forward.argtypes = [C.POINTER(Ecapa), F32P, C.c_int, F32P, C.POINTER(EcapaCaps)]
        L._ecapa_ready = True
    return L


class OracleEcapa:
    """orc_ecapa built from a parsed ECAPA GGUF (weights as stored, dequantised to f32)."""

    def __init__(self, g):
        self.keep = []
        self.g = g
        kv = g.kv
        n = Ecapa()

        def arr(name):
            a = np.ascontiguousarray(g.array(name), dtype=np.float32)
            self.keep.append(a)
            return a

        def conv(dst, prefix):
            w = arr(prefix + ".weight")
            if w.ndim == 2:
                w = w.reshape(w.shape[0], w.shape[1], 1)
                self.keep.append(w)
            dst.w = w.ctypes.data_as(_fp)
            dst.b = arr(prefix + ".bias").ctypes.data_as(_fp)
            dst.oc, dst.ic, dst.k = w.shape

        def bn(dst, prefix):
            dst.gamma = arr(prefix + ".weight").ctypes.data_as(_fp)
            dst.beta = arr(prefix + ".bias").ctypes.data_as(_fp)
            dst.mean = arr(prefix + ".running_mean").ctypes.data_as(_fp)
            v = arr(prefix + ".running_var")
            dst.var = v.ctypes.data_as(_fp)
            dst.c = v.shape[0]

        n.n_mels = int(kv.get("voicedetect.fbank.n_mels", 80))
        conv(n.block0, "blocks.0.conv.conv")
        bn(n.bn0, "blocks.0.norm.norm")
        n.channels = n.block0.oc
        R = 0
        while f"blocks.{R + 1}.tdnn1.conv.conv.weight" in g.tensors:
            R += 1
        n.n_res = R
        scale = 1
        while f"blocks.1.res2net_block.blocks.{scale - 1}.conv.conv.weight" in g.tensors:
            scale += 1
        n.scale = scale
        for i in range(R):
            p = f"blocks.{i + 1}"
            conv(n.tdnn1[i], p + ".tdnn1.conv.conv")
            bn(n.bn_t1[i], p + ".tdnn1.norm.norm")
            conv(n.tdnn2[i], p + ".tdnn2.conv.conv")
            bn(n.bn_t2[i], p + ".tdnn2.norm.norm")
            conv(n.se1[i], p + ".se_block.conv1.conv")
            conv(n.se2[i], p + ".se_block.conv2.conv")
            for j in range(scale - 1):
                conv(n.res[i][j], f"{p}.res2net_block.blocks.{j}.conv.conv")
                bn(n.bn_res[i][j], f"{p}.res2net_block.blocks.{j}.norm.norm")
        conv(n.mfa, "mfa.conv.conv")
        bn(n.bn_mfa, "mfa.norm.norm")
        n.mfa_ch = n.mfa.oc
        conv(n.asp_tdnn, "asp.tdnn.conv.conv")
        bn(n.bn_asp, "asp.tdnn.norm.norm")
        conv(n.asp_conv, "asp.conv.conv")
        bn(n.asp_bn, "asp_bn.norm")
        conv(n.fc, "fc.conv")
        n.emb_dim = n.fc.oc
        n.l2_normalize = int(bool(kv.get("voicedetect.l2_normalize", True)))
        self.net = n

    def forward(self, feats, capture=False):
        L = _ecapa_sigs()
        feats = np.ascontiguousarray(feats, dtype=np.float32)
        T = feats.shape[1]
        n = self.net
        emb = np.zeros(n.emb_dim, dtype=np.float32)
        caps = EcapaCaps()
        bufs = {}
        if capture:
            for i in range(n.n_res + 1):
                bufs[f"block{i}"] = np.zeros((n.channels, T), dtype=np.float32)
                caps.block[i] = bufs[f"block{i}"].ctypes.data_as(_fp)
            bufs["mfa"] = np.zeros((n.mfa_ch, T), dtype=np.float32)
            caps.mfa = bufs["mfa"].ctypes.data_as(_fp)
            bufs["pooled"] = np.zeros(2 * n.mfa_ch, dtype=np.float32)
            caps.pooled = bufs["pooled"].ctypes.data_as(_fp)
            bufs["pre_norm"] = np.zeros(n.emb_dim, dtype=np.float32)
            caps.pre_norm = bufs["pre_norm"].ctypes.data_as(_fp)
        assert L.orc_ecapa_forward(C.byref(n), feats, T, emb, C.byref(caps)) == 0
        return (emb, bufs) if capture else emb


def conv1d_same(x, w, b, dilation=1):
    """Oracle reflect-padded conv1d: x [ic, T], w [oc, ic, k] -> [oc, T]."""
    L = _ecapa_sigs()
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    c = Conv1d(w.ctypes.data_as(_fp), b.ctypes.data_as(_fp), w.shape[0], w.shape[1], w.shape[2])
    y = np.zeros((w.shape[0], x.shape[1]), dtype=np.float32)
    L.orc_conv1d_same(x, x.shape[1], C.byref(c), dilation, y)
    return y


def bn_apply(x, gamma, beta, mean, var):
    """Oracle eval BatchNorm1d on x [C, T] (returns a new array)."""
    L = _ecapa_sigs()
    y = np.array(x, dtype=np.float32, order="C", copy=True)
    keep = [np.ascontiguousarray(a, dtype=np.float32) for a in (gamma, beta, mean, var)]
    bn = BN(*(a.ctypes.data_as(_fp) for a in keep), y.shape[0])
    L.orc_bn_apply(y, y.shape[1], C.byref(bn))
    return y


def ecapa_asp(net, x):
    """Oracle attentive statistics pooling of an OracleEcapa on x [mfa, T] -> [2*mfa]."""
    L = _ecapa_sigs()
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(2 * x.shape[0], dtype=np.float32)
    L.orc_ecapa_asp(C.byref(net.net), x, x.shape[1], out)
    return out


# ---------------------------------------------------------------- CAM++

class Conv(C.Structure):
    _fields_ = [("w", _fp), ("b", _fp), ("oc", C.c_int), ("ic", C.c_int), ("kh", C.c_int), ("kw", C.c_int)]


class Campplus(C.Structure):
    _fields_ = [("n_mels", C.c_int), ("n_conv", C.c_int), ("n_bn", C.c_int), ("l2_normalize", C.c_int),
                ("bn_eps", C.c_float), ("conv", Conv * 256), ("bn", BN * 64),
                ("emb_mean", _fp), ("emb_var", _fp)]


class CampplusCaps(C.Structure):
    _fields_ = [("fcm", _fp), ("tdnn", _fp), ("block", _fp * 3), ("pooled", _fp), ("pre_norm", _fp)]


def _campplus_sigs():
    L = lib()
    if not hasattr(L, "_campplus_ready"):
        L.orc_campplus_forward.argtypes = [C.POINTER(Campplus), F32P, C.c_int, F32P, C.POINTER(CampplusCaps)]
        L.orc_campplus_forward.restype = C.c_int
        L.orc_conv2d_f32_g.argtypes = [F32P, C.c_int, C.c_int, C.c_int, F32P, C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                       _fp, _fp, C.c_int, F32P]
        L.orc_conv2d_f64_g.argtypes = [F32P, C.c_int, C.c_int, C.c_int, F32P, C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                       _fp, _fp, C.c_int, np.ctypeslib.ndpointer(dtype=np.float64,
                                                                               flags="C_CONTIGUOUS")]
        L._campplus_ready = True
    return L


def conv2d_g(x, w, sh=1, sw=1, ph=0, pw=0, dh=1, dw=1, bias=None, residual=None, relu=False, f64=False):
    """Oracle conv with per-axis stride / zero pad / dilation: x [IC,H,W], w [OC,IC,KH,KW]."""
    L = _campplus_sigs()
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    IC, H, W = x.shape
    OC, _, KH, KW = w.shape
    Ho = (H + 2 * ph - (KH - 1) * dh - 1) // sh + 1
    Wo = (W + 2 * pw - (KW - 1) * dw - 1) // sw + 1
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    r = None if residual is None else np.ascontiguousarray(residual, dtype=np.float32)
    y = np.zeros((OC, Ho, Wo), dtype=np.float64 if f64 else np.float32)
    fn = L.orc_conv2d_f64_g if f64 else L.orc_conv2d_f32_g
    fn(x, IC, H, W, w, OC, KH, KW, sh, sw, ph, pw, dh, dw,
       None if b is None else b.ctypes.data_as(_fp), None if r is None else r.ctypes.data_as(_fp), int(relu), y)
    return y


def _weight4(g, name):
    """A manifest conv weight as [OC, IC, KH, KW] f32 (1-D convs KH = 1, 2-D matrices 1x1)."""
    w = np.asarray(g.array(name), dtype=np.float32)
    if w.ndim == 2:
        return w.reshape(w.shape[0], w.shape[1], 1, 1)
    if w.ndim == 3:
        return w.reshape(w.shape[0], w.shape[1], 1, w.shape[2])
    return w


class OracleCampplus:
    """orc_campplus built from a parsed CAM++ GGUF (weights dequantised to f32)."""

    def __init__(self, g):
        self.keep = []
        kv = g.kv
        n = Campplus()
        names_w = kv["voicedetect.campplus.conv_weight"]
        names_b = kv["voicedetect.campplus.conv_bias"]
        bns = kv["voicedetect.campplus.bn_prefix"]
        n.n_mels = int(kv.get("voicedetect.fbank.n_mels", 80))
        n.n_conv = len(names_w)
        n.n_bn = len(bns)
        n.bn_eps = float(kv.get("voicedetect.campplus.bn_eps", 1e-5))
        n.l2_normalize = int(bool(kv.get("voicedetect.l2_normalize", True)))

        def arr(a):
            a = np.ascontiguousarray(a, dtype=np.float32)
            self.keep.append(a)
            return a.ctypes.data_as(_fp)

        self.weights = []
        for i, (wn, bn) in enumerate(zip(names_w, names_b)):
            w = _weight4(g, wn)
            self.weights.append(w)
            c = n.conv[i]
            c.w = arr(w)
            c.b = arr(g.array(bn)) if bn else None
            c.oc, c.ic, c.kh, c.kw = w.shape
        for i, p in enumerate(bns):
            b = n.bn[i]
            b.gamma = arr(g.array(p + ".weight"))
            b.beta = arr(g.array(p + ".bias"))
            b.mean = arr(g.array(p + ".running_mean"))
            v = np.asarray(g.array(p + ".running_var"), dtype=np.float32)
            b.var = arr(v)
            b.c = v.shape[0]
        n.emb_mean = arr(g.array(kv["voicedetect.campplus.emb_bn_mean"]))
        n.emb_var = arr(g.array(kv["voicedetect.campplus.emb_bn_var"]))
        self.net = n
        self.emb_dim = n.conv[n.n_conv - 1].oc

    def forward(self, feats, capture=False):
        L = _campplus_sigs()
        feats = np.ascontiguousarray(feats, dtype=np.float32)
        T = feats.shape[1]
        Tp = (T - 1) // 2 + 1
        n = self.net
        emb = np.zeros(self.emb_dim, dtype=np.float32)
        caps = CampplusCaps()
        bufs = {}
        if capture:
            H = n.n_mels
            for _ in range(3):
                H = (H - 1) // 2 + 1
            bufs["fcm"] = np.zeros((n.conv[11].oc * H, T), dtype=np.float32)
            caps.fcm = bufs["fcm"].ctypes.data_as(_fp)
            bufs["tdnn"] = np.zeros((n.conv[12].oc, Tp), dtype=np.float32)
            caps.tdnn = bufs["tdnn"].ctypes.data_as(_fp)
            # transit convs: the last conv of each block (index walk over the fixed topology)
            ci = 13
            for b, nl in enumerate((12, 24, 16)):
                ci += 4 * nl
                bufs[f"block{b}"] = np.zeros((n.conv[ci].oc, Tp), dtype=np.float32)
                caps.block[b] = bufs[f"block{b}"].ctypes.data_as(_fp)
                ci += 1
            c_out = n.conv[ci - 1].oc
            bufs["pooled"] = np.zeros(2 * c_out, dtype=np.float32)
            caps.pooled = bufs["pooled"].ctypes.data_as(_fp)
            bufs["pre_norm"] = np.zeros(self.emb_dim, dtype=np.float32)
            caps.pre_norm = bufs["pre_norm"].ctypes.data_as(_fp)
        rc = L.orc_campplus_forward(C.byref(n), feats, T, emb, C.byref(caps))
        assert rc == 0, "CAM++ manifest does not match the fixed topology"
        return (emb, bufs) if capture else emb


# ---------------------------------------------------------------- ERes2Net

class Eres2net(C.Structure):
    _fields_ = [("n_mels", C.c_int), ("n_conv", C.c_int), ("m_channels", C.c_int), ("scale", C.c_int),
                ("emb_dim", C.c_int), ("l2_normalize", C.c_int), ("num_blocks", C.c_int * 4),
                ("relu_clamp", C.c_float), ("var_eps", C.c_float), ("conv", Conv * 128), ("stride", C.c_int * 128),
                ("seg_w", _fp), ("seg_b", _fp)]


class Eres2netCaps(C.Structure):
    _fields_ = [("stem", _fp), ("fused", _fp), ("pooled", _fp), ("pre_norm", _fp)]


class OracleEres2net:
    """orc_eres2net built from a parsed ERes2Net GGUF (weights dequantised to f32)."""

    def __init__(self, g):
        self.keep = []
        kv = g.kv
        n = Eres2net()
        names_w = kv["voicedetect.eres2net.conv_weight"]
        names_b = kv["voicedetect.eres2net.conv_bias"]
        strides = kv["voicedetect.eres2net.conv_stride"]
        n.n_mels = int(kv.get("voicedetect.fbank.n_mels", 80))
        n.n_conv = len(names_w)
        n.m_channels = int(kv["voicedetect.eres2net.m_channels"])
        n.scale = int(kv.get("voicedetect.eres2net.scale", 2))
        for i, v in enumerate(kv["voicedetect.eres2net.num_blocks"]):
            n.num_blocks[i] = int(v)
        n.relu_clamp = float(kv.get("voicedetect.eres2net.relu_clamp", 20.0))
        n.var_eps = float(kv.get("voicedetect.eres2net.var_eps", 1e-8))
        n.l2_normalize = int(bool(kv.get("voicedetect.l2_normalize", True)))

        def arr(a):
            a = np.ascontiguousarray(a, dtype=np.float32)
            self.keep.append(a)
            return a.ctypes.data_as(_fp)

        for i, (wn, bn) in enumerate(zip(names_w, names_b)):
            w = _weight4(g, wn)
            c = n.conv[i]
            c.w = arr(w)
            c.b = arr(g.array(bn)) if bn else None
            c.oc, c.ic, c.kh, c.kw = w.shape
            n.stride[i] = int(strides[i])
        sw = np.asarray(g.array(kv["voicedetect.eres2net.seg_weight"]), dtype=np.float32)
        n.seg_w = arr(sw)
        n.seg_b = arr(g.array(kv["voicedetect.eres2net.seg_bias"]))
        n.emb_dim = sw.shape[0]
        self.net = n

    def forward(self, feats, capture=False):
        L = lib()
        if not hasattr(L, "_eres_ready"):
            L.orc_eres2net_forward.argtypes = [C.POINTER(Eres2net), F32P, C.c_int, F32P, C.POINTER(Eres2netCaps)]
            L.orc_eres2net_forward.restype = C.c_int
            L._eres_ready = True
        feats = np.ascontiguousarray(feats, dtype=np.float32)
        T = feats.shape[1]
        n = self.net
        emb = np.zeros(n.emb_dim, dtype=np.float32)
        caps = Eres2netCaps()
        bufs = {}
        if capture:
            M = n.m_channels
            H, W = n.n_mels, T
            bufs["stem"] = np.zeros((M, H, W), dtype=np.float32)
            for _ in range(3):
                H, W = (H - 1) // 2 + 1, (W - 1) // 2 + 1
            bufs["fused"] = np.zeros((16 * M, H, W), dtype=np.float32)
            bufs["pooled"] = np.zeros(2 * 16 * M * H, dtype=np.float32)
            bufs["pre_norm"] = np.zeros(n.emb_dim, dtype=np.float32)
            for k in ("stem", "fused", "pooled", "pre_norm"):
                setattr(caps, k, bufs[k].ctypes.data_as(_fp))
        rc = L.orc_eres2net_forward(C.byref(n), feats, T, emb, C.byref(caps))
        assert rc == 0, "ERes2Net manifest does not match the topology"
        return (emb, bufs) if capture else emb
