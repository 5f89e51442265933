"""C-ABI checks that need no GPU: the library loads, exports every symbol the
headers declare, and follows the reference's error/ownership contract
(src/voicedetect_capi.cpp:61-178) on the paths that fail before any device work.
Also pins the host utilities: WAV decode against the reference's dr_wav-based
loader output (golden PCM), the resampler and f16 packing against closed forms.
"""
import ctypes as C
import os
import re
import tempfile

import numpy as np
import pytest

import pyoracle as O
from vdamd import gguf, lib, synth


def _declared(header):
    src = open(os.path.join(lib.INCLUDE_DIR, header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b((?:voicedetect_capi|voicedetect_gpu|vdk)_\w+)\s*\(", src))


def test_library_exports_every_declared_symbol():
    L = lib.lib()
    declared = set()
    for h in ("voicedetect_capi.h", "voicedetect_gpu.h", "vdk.h"):
        declared |= _declared(h)
    assert len(declared) >= 35
    for name in sorted(declared):
        assert hasattr(L, name), name
    # the binding covers exactly the declared surface
    assert declared == set(lib.exported_symbols())
    frozen = {"voicedetect_capi_abi_version", "voicedetect_capi_load", "voicedetect_capi_free",
              "voicedetect_capi_last_error", "voicedetect_capi_free_string", "voicedetect_capi_free_vec",
              "voicedetect_capi_embed_path", "voicedetect_capi_embed_pcm", "voicedetect_capi_verify_paths",
              "voicedetect_capi_analyze_path_json"}
    assert frozen <= declared


def test_abi_version_and_null_safety():
    L = lib.lib()
    assert L.voicedetect_capi_abi_version() == 1
    assert L.voicedetect_capi_load(None) is None
    assert L.voicedetect_capi_load(b"/nonexistent/model.gguf") is None
    assert L.voicedetect_capi_last_error(None) == b""
    L.voicedetect_capi_free(None)
    L.voicedetect_capi_free_vec(None)
    L.voicedetect_capi_free_string(None)
    vec = C.POINTER(C.c_float)()
    dim = C.c_int(7)
    assert L.voicedetect_capi_embed_pcm(None, None, 0, 16000, C.byref(vec), C.byref(dim)) == 1
    assert not vec and dim.value == 0
    assert L.voicedetect_capi_verify_paths(None, b"a", b"b", 0.25, None, None) == 1
    assert L.voicedetect_capi_analyze_path_json(None, b"a") is None


def test_load_rejects_bad_files():
    L = lib.lib()
    with tempfile.TemporaryDirectory() as tmp:
        p = os.path.join(tmp, "junk.gguf")
        open(p, "wb").write(b"not a gguf at all")
        assert L.voicedetect_capi_load(p.encode()) is None
        # valid container without voicedetect.embedding_dim (src/model_loader.cpp:212-214)
        q = os.path.join(tmp, "nodim.gguf")
        gguf.write_gguf(q, {"voicedetect.arch": "wespeaker_resnet34"}, [])
        assert L.voicedetect_capi_load(q.encode()) is None


def _with_extra_tensor(src, dst, ne_words, gtype=0, offset=0, truncate_to=None):
    """Copy GGUF `src` to `dst` with one more tensor info (raw u64 dim words,
    type, offset) after the existing ones; the data section is moved to the
    new aligned base so every existing offset stays valid."""
    import struct
    g = gguf.GGUFFile(src)
    end = g.pos                                   # end of the tensor infos
    buf = g.buf
    old_base = (end + 31) // 32 * 32
    (nt,) = struct.unpack_from("<Q", buf, 8)
    info = struct.pack("<Q", 5) + b"bogus" + struct.pack("<I", len(ne_words))
    info += b"".join(struct.pack("<Q", w & (2 ** 64 - 1)) for w in ne_words) + struct.pack("<IQ", gtype, offset)
    head = bytearray(buf[:end]) + info
    head[8:16] = struct.pack("<Q", nt + 1)
    head += b"\0" * ((-len(head)) % 32)
    out = bytes(head) + buf[old_base:]
    if truncate_to is not None:
        out = out[:truncate_to]
    open(dst, "wb").write(out)


def test_load_rejects_corrupt_tensor_headers():
    """Tensor infos a corrupt or crafted file can hold: negative dims, dims whose
    product overflows int64, offsets that wrap the bounds check, unaligned
    offsets, data cut short.  Each makes load return NULL; the same file with a
    well-formed extra tensor loads (the construction itself is sound)."""
    L = lib.lib()
    with tempfile.TemporaryDirectory() as tmp:
        base = os.path.join(tmp, "base.gguf")
        synth.write_resnet34(base, seed=5, channels=(32, 32, 64, 64), blocks=(1, 1, 1, 1), emb_dim=64)
        ok = os.path.join(tmp, "ok.gguf")
        _with_extra_tensor(base, ok, [8])
        ctx = L.voicedetect_capi_load(ok.encode())
        assert ctx is not None
        L.voicedetect_capi_free(ctx)
        cases = {
            "negative_dim": dict(ne_words=[-8, 4]),
            "dim_past_int32": dict(ne_words=[2 ** 31, 1]),
            "product_overflow": dict(ne_words=[2 ** 31 - 1, 2 ** 31 - 1, 2 ** 31 - 1, 4]),
            "offset_wraps": dict(ne_words=[8], offset=2 ** 64 - 64),
            "offset_past_end": dict(ne_words=[8], offset=1 << 40),
            "offset_unaligned": dict(ne_words=[8], offset=4),
            "larger_than_file": dict(ne_words=[1 << 30, 4]),
        }
        for name, kw in cases.items():
            bad = os.path.join(tmp, name + ".gguf")
            _with_extra_tensor(base, bad, **kw)
            assert L.voicedetect_capi_load(bad.encode()) is None, name
        cut = os.path.join(tmp, "truncated.gguf")
        _with_extra_tensor(base, cut, [8], truncate_to=os.path.getsize(ok) - 100)
        assert L.voicedetect_capi_load(cut.encode()) is None


def test_ecapa_refuses_clips_shorter_than_its_reflect_pad():
    """ECAPA's reflect padding needs pad < T (src/encoder.cpp:32-52; the widest
    pad is the last SE-Res2Net block's dilation, 4): 1039 samples give 4 FBank
    frames and are refused before any device work, with a clear message."""
    L = lib.lib()
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "ecapa.gguf")
        synth.write_ecapa(path, 3, channels=64, mfa=96, n_mels=80, scale=2, se_ch=16, att_ch=32, emb_dim=16)
        ctx = lib.Context(path)
        vec, dim = C.POINTER(C.c_float)(), C.c_int(5)
        x = np.zeros(1039, dtype=np.float32)
        assert L.voicedetect_capi_embed_pcm(ctx.ctx, x.ctypes.data, 1039, 16000, C.byref(vec), C.byref(dim)) == 1
        assert "clip too short for reflect padding (4 frames, the model needs 5)" in ctx.last_error()
        assert not vec and dim.value == 0
        ctx.close()


@pytest.fixture(scope="module")
def tiny_model():
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "tiny.gguf")
    synth.write_resnet34(path, seed=5, channels=(32, 32, 64, 64), blocks=(1, 1, 1, 1), emb_dim=64)
    return path


def test_error_contract_without_device_work(tiny_model):
    ctx = lib.Context(tiny_model)
    L = ctx.L
    assert ctx.dim == 64
    assert ctx.last_error() == ""
    vec = C.POINTER(C.c_float)()
    dim = C.c_int(5)
    # NULL pcm / negative length: "invalid pcm buffer", outputs reset
    assert L.voicedetect_capi_embed_pcm(ctx.ctx, None, 10, 16000, C.byref(vec), C.byref(dim)) == 1
    assert ctx.last_error() == "invalid pcm buffer" and not vec and dim.value == 0
    x = np.zeros(100, dtype=np.float32)
    assert L.voicedetect_capi_embed_pcm(ctx.ctx, x.ctypes.data, -1, 16000, C.byref(vec), C.byref(dim)) == 1
    # fewer samples than one window (src/fbank.cpp:126-127, src/model.cpp:27-28)
    assert L.voicedetect_capi_embed_pcm(ctx.ctx, x.ctypes.data, 100, 16000, C.byref(vec), C.byref(dim)) == 1
    assert "FBank produced no frames" in ctx.last_error()
    # verify with NULL path / unreadable file
    d, v = C.c_float(-7.0), C.c_int(-7)
    assert L.voicedetect_capi_verify_paths(ctx.ctx, None, b"x", 0.25, C.byref(d), C.byref(v)) == 1
    assert ctx.last_error() == "clip path is NULL" and d.value == -7.0 and v.value == -7
    assert L.voicedetect_capi_verify_paths(ctx.ctx, b"/nonexistent.wav", b"/n2.wav", 0.25, C.byref(d),
                                           C.byref(v)) == 1
    assert "failed to load audio" in ctx.last_error() and d.value == -7.0
    assert L.voicedetect_capi_embed_path(ctx.ctx, None, C.byref(vec), C.byref(dim)) == 1
    assert ctx.last_error() == "wav_path is NULL"
    # a speaker model has no analyze heads: NULL + the reference's message
    assert L.voicedetect_capi_analyze_path_json(ctx.ctx, b"x.wav") is None
    assert ctx.last_error() == "voicedetect: this model has no age/gender/emotion analyze heads"
    if L.vdk_device_count() == 0:
        y = np.zeros(16000, dtype=np.float32)
        assert L.voicedetect_capi_embed_pcm(ctx.ctx, y.ctypes.data, 16000, 16000, C.byref(vec), C.byref(dim)) == 1
        assert "no HIP device" in ctx.last_error()
    ctx.close()


def test_wav_reader_matches_reference_decoder(golden_dir):
    z = np.load(os.path.join(golden_dir, "fbank_golden.npz"))
    L = lib.lib()
    for name in ("clip_a", "clip_b_same", "clip_c_diff"):
        path = os.path.join(golden_dir, name + ".wav").encode()
        n = L.vdk_load_wav_16k(path, None, 0)
        assert n == 48000
        out = np.zeros(n, dtype=np.float32)
        assert L.vdk_load_wav_16k(path, out.ctypes.data, n) == n
        assert np.array_equal(out, z[f"wav_{name}/pcm"])   # bit-exact vs dr_wav
    assert L.vdk_load_wav_16k(b"/nonexistent.wav", None, 0) == -1


def test_wav_formats_and_downmix():
    L = lib.lib()
    with tempfile.TemporaryDirectory() as tmp:
        import wave
        p = os.path.join(tmp, "st.wav")
        left = (np.arange(320) * 50 - 8000).astype(np.int16)
        right = (-left).astype(np.int16)
        inter = np.stack([left, right], axis=1).reshape(-1)
        with wave.open(p, "wb") as w:
            w.setnchannels(2)
            w.setsampwidth(2)
            w.setframerate(16000)
            w.writeframes(inter.tobytes())
        out = np.zeros(320, dtype=np.float32)
        assert L.vdk_load_wav_16k(p.encode(), out.ctypes.data, 320) == 320
        assert np.all(out == 0.0)                 # L + R cancel exactly
        p8 = os.path.join(tmp, "k.wav")
        with wave.open(p8, "wb") as w:
            w.setnchannels(1)
            w.setsampwidth(2)
            w.setframerate(8000)
            w.writeframes(left.tobytes())
        n = L.vdk_load_wav_16k(p8.encode(), None, 0)
        assert n == 640                           # 8 kHz -> 16 kHz doubles the length


def test_resampler_closed_form():
    L = lib.lib()
    x = np.arange(10, dtype=np.float32)
    out = np.zeros(20, dtype=np.float32)
    assert L.vdk_resample_linear(x.ctypes.data, 10, 8000, 16000, out.ctypes.data, 20) == 20
    # linear interpolation of a ramp, last point holds the final sample
    assert np.allclose(out[:19], np.arange(19) / 2.0) and out[19] == 9.0
    same = np.zeros(10, dtype=np.float32)
    assert L.vdk_resample_linear(x.ctypes.data, 10, 16000, 16000, same.ctypes.data, 10) == 10
    assert np.array_equal(same, x)
    # 48 kHz -> 16 kHz: every output sits on an input sample (src = 3i exactly)
    y = np.random.default_rng(4).standard_normal(3001).astype(np.float32)
    dec = np.zeros(1000, dtype=np.float32)
    assert L.vdk_resample_linear(y.ctypes.data, 3001, 48000, 16000, dec.ctypes.data, 1000) == 1000
    assert np.array_equal(dec, y[0:3000:3])


@pytest.mark.parametrize("in_sr,out_sr", [(44100, 16000), (22050, 16000), (48000, 16000), (8000, 16000),
                                          (11025, 16000), (32000, 16000), (16000, 8000), (16000, 44100)])
def test_resampler_bit_exact_with_reference(in_sr, out_sr):
    """vdk_resample_linear against the reference's own resample_linear
    (src/audio_io.cpp:9-23, compiled from the reference sources into
    oracle/_ref/libref.so): identical output length and bits at non-integer
    ratios, on a noisy clip and on a ramp."""
    R = O.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref/libref.so not built (the reference checkout is absent)")
    L = lib.lib()
    rng = np.random.default_rng(in_sr + out_sr)
    for x in (rng.standard_normal(in_sr * 37 // 100).astype(np.float32),
              np.linspace(-1.0, 1.0, 4801, dtype=np.float32)):
        cap = int(len(x) * out_sr / in_sr) + 4
        got, want = np.zeros(cap, np.float32), np.zeros(cap, np.float32)
        n = L.vdk_resample_linear(x.ctypes.data, len(x), in_sr, out_sr, got.ctypes.data, cap)
        m = R.ref_resample(x, len(x), in_sr, out_sr, want, cap)
        assert n == m and n > 0
        assert np.array_equal(got[:n].view(np.uint32), want[:m].view(np.uint32))


def test_f16_packing_matches_ieee_round_to_nearest_even():
    L = lib.lib()
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * s for s in (1e-6, 1e-3, 1.0, 1e3, 3e4)])
    x = np.concatenate([x, np.array([0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 5.96e-8, 2.98e-8, 6.1e-5,
                                     np.inf, -np.inf], dtype=np.float32)])
    out = np.zeros(len(x), dtype=np.uint16)
    L.vdk_f32_to_f16(x.ctypes.data, out.ctypes.data, len(x))
    assert np.array_equal(out, x.astype(np.float16).view(np.uint16))


def test_analyze_model_host_side(tmp_path):
    """An analyze GGUF (wav2vec2 emotion / age-gender) loads through the C ABI;
    its shape queries and error paths need no GPU (src/model.cpp:80-101)."""
    from vdamd import synth
    L = lib.lib()
    small = dict(hidden=128, n_layers=1, n_heads=2, ff=256, conv_dims=(256,) * 7, pos_k=8, pos_groups=2, proj=32)
    for kind, n_out in (("emotion", 4), ("age_gender", 4)):
        path = str(tmp_path / f"{kind}.gguf")
        synth.write_w2v2(path, 3, kind, **small)
        ctx = lib.Context(path)
        assert ctx.analyze_outputs() == n_out
        # T' = 49 for 1 s at 16 kHz (kernels 10,3,3,3,3,2,2, strides 5,2,...)
        assert ctx.analyze_frames(16000) == 49 and ctx.analyze_frames(399) == 0 and ctx.analyze_frames(400) == 1
        vec, dim = C.POINTER(C.c_float)(), C.c_int(-1)
        x = np.zeros(16000, dtype=np.float32)
        assert L.voicedetect_capi_embed_pcm(ctx.ctx, x.ctypes.data, 16000, 16000, C.byref(vec), C.byref(dim)) == 1
        assert "no speaker embedding head" in ctx.last_error() and not vec and dim.value == 0
        assert L.voicedetect_capi_analyze_path_json(ctx.ctx, b"/nonexistent.wav") is None
        assert "failed to load audio" in ctx.last_error()
        ctx.close()


def test_conv_pack_chunked_layout():
    """vdk_conv_pack_chunked: [OC][KH][KW][IC] -> [IC/16][KH*KW][OC][16], element
    (oc, tap, ic) at ((ic // 16) * taps + tap) * OC * 16 + oc * 16 + ic % 16."""
    L = lib.lib()
    OC, KH, KW, IC = 96, 3, 3, 48
    w = np.random.default_rng(5).integers(0, 65536, (OC, KH, KW, IC), dtype=np.uint16)
    out = np.zeros(w.size, dtype=np.uint16)
    L.vdk_conv_pack_chunked(w.ctypes.data, OC, KH, KW, IC, out.ctypes.data)
    want = w.reshape(OC, KH * KW, IC // 16, 16).transpose(2, 1, 0, 3).reshape(-1)
    assert np.array_equal(out, want)
    oc, tap, ic = 37, 5, 33
    assert out[((ic // 16) * 9 + tap) * OC * 16 + oc * 16 + ic % 16] == w[oc, tap // 3, tap % 3, ic]
