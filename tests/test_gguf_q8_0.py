"""Q8_0 tensors and the real ECAPA checkpoint layout, on the CPU.

The Q8_0 block (ggml's public format, read by src/model_loader.cpp:114-215
through ggml): 34 bytes per 32 elements along ne[0], an IEEE f16 scale d
then 32 int8 quants q, element = q * d.  The file below is assembled byte by
byte here (not by this package's writer) with scales whose f16 bit patterns
and values are written out by hand, and both readers (the library's C++
GgufFile behind vdk_gguf_tensor_f32 and vdamd.gguf) must return q * d.

tests/golden/ecapa_tdnn_manifest.txt is the reference's
models/ecapa_tdnn_manifest.txt (SpeechBrain spkrec-ecapa-voxceleb state_dict
names and torch shapes), kept as data.
"""
import os
import struct

import numpy as np
import pytest

from vdamd import gguf, lib, synth

HERE = os.path.dirname(os.path.abspath(__file__))

# (f16 bits, value) written out by hand: 0.5, 0.0999755859375 (= 1638 / 2^14),
# -2.0, 2^-24 (the smallest subnormal), 65504 (the largest finite f16)
SCALES = [(0x3800, 0.5), (0x2E66, 1638.0 / 16384.0), (0xC000, -2.0), (0x0001, 2.0 ** -24), (0x7BFF, 65504.0)]


def _quants():
    q = [list(range(-16, 16)),
         [127, -127, -128, 0, 1, -1] + [5] * 26,
         [(-1) ** k * k for k in range(32)],
         [100] * 32,
         [-3, 3] * 16]
    return [np.array(b, dtype=np.int8) for b in q]


def _gguf_bytes(tensors):
    """GGUF v3: no key/values, tensors (name, ne, ggml type, payload) at
    32-byte aligned offsets."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 0))
    off = 0
    offs = []
    for name, ne, gtype, payload in tensors:
        nb = name.encode()
        out += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(ne))
        out += b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", gtype, off)
        offs.append(off)
        off = (off + len(payload) + 31) // 32 * 32
    out += b"\0" * ((-len(out)) % 32)
    base = len(out)
    for (name, ne, gtype, payload), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out))
        out += payload
    return bytes(out)


def test_q8_0_hand_assembled_blocks_both_readers(tmp_path):
    qs = _quants()
    blocks = b"".join(struct.pack("<H", bits) + q.tobytes() for (bits, _), q in zip(SCALES, qs))
    assert len(blocks) == 5 * 34
    # a 2-D [IC = 32, OC = 5] weight (one block per output row) and a 1-D
    # tensor of the same 160 elements
    want = np.concatenate([q.astype(np.float64) * v for (_, v), q in zip(SCALES, qs)])
    f16_bits = np.array([0x3C00, 0xC400, 0x0400, 0x8001], dtype=np.uint16).tobytes()   # 1, -4, 2^-14, -2^-24
    path = str(tmp_path / "q8.gguf")
    with open(path, "wb") as f:
        f.write(_gguf_bytes([("w2d", [32, 5], 8, blocks), ("w1d", [160], 8, blocks), ("h", [4], 1, f16_bits)]))
    # every product q * d is exact in f32
    assert np.array_equal(want.astype(np.float32).astype(np.float64), want)
    g = gguf.GGUFFile(path)
    assert g.tensors["w2d"][1] == [32, 5]
    assert np.array_equal(g.array("w2d").astype(np.float64), want.reshape(5, 32))
    assert np.array_equal(g.array("w1d").astype(np.float64), want)
    assert np.array_equal(g.array("h"), np.array([1.0, -4.0, 2.0 ** -14, -(2.0 ** -24)], dtype=np.float32))
    L = lib.lib()
    for name in ("w2d", "w1d"):
        out = np.empty(160, dtype=np.float32)
        lib.check(L.vdk_gguf_tensor_f32(path.encode(), name.encode(), out.ctypes.data, 160))
        assert np.array_equal(out.astype(np.float64), want), name
    out = np.empty(4, dtype=np.float32)
    lib.check(L.vdk_gguf_tensor_f32(path.encode(), b"h", out.ctypes.data, 4))
    assert np.array_equal(out, np.array([1.0, -4.0, 2.0 ** -14, -(2.0 ** -24)], dtype=np.float32))
    # wrong element count and a missing name are errors, not reads
    assert L.vdk_gguf_tensor_f32(path.encode(), b"w1d", out.ctypes.data, 4) != 0
    assert b"element count" in L.vdk_last_error()
    assert L.vdk_gguf_tensor_f32(path.encode(), b"nope", out.ctypes.data, 4) != 0


def test_q8_0_writer_round_trip_through_both_readers(tmp_path):
    """The package's writer (the synthetic models' Q8_0 weights) read back by
    both readers: identical values, within one quantisation step of the input."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 96)).astype(np.float32)
    path = str(tmp_path / "w.gguf")
    gguf.write_gguf(path, {"general.architecture": "voicedetect"}, [("x", gguf.GGML_Q8_0, [6, 96], x)])
    got = gguf.GGUFFile(path).array("x")
    out = np.empty(x.size, dtype=np.float32)
    lib.check(lib.lib().vdk_gguf_tensor_f32(path.encode(), b"x", out.ctypes.data, x.size))
    assert np.array_equal(out.reshape(6, 96), got)
    # the quants are rounded against the f32 scale d, which is then stored as
    # f16: |q * f16(d) - x| <= d / 2 + 127 * |f16(d) - d| <= d * (1/2 + 127 * 2^-11)
    d = np.abs(x.reshape(-1, 32)).max(axis=1, keepdims=True) / 127.0
    assert np.all(np.abs(got.reshape(-1, 32) - x.reshape(-1, 32)) <= d * (0.5 + 127 * 2.0 ** -11) + 1e-7)


def _manifest():
    rows = []
    with open(os.path.join(HERE, "golden", "ecapa_tdnn_manifest.txt")) as f:
        for line in f:
            if line.startswith("#") or not line.strip():
                continue
            name, _, shape = line.rstrip("\n").partition("\t")
            rows.append((name, [int(v) for v in shape.split(",")] if shape else []))
    return rows


# scripts/convert_voicedetect_to_gguf.py quant_plan: which weights a q8_0
# conversion stores as 2-D Q8_0 [OC, IC] (1x1 .conv/.linear weights outside
# fc / asp / se_block / tdnn1 / tdnn2 with IC, OC >= 32 and IC % 32 == 0)
def _q8_0_by_converter_rule(name, shape):
    import re
    if not re.search(r"\.conv\.weight$|\.linear\.weight$", name):
        return False
    if re.search(r"^fc\.|^asp\.|\.se_block\.|\.tdnn1\.|\.tdnn2\.", name):
        return False
    oc, ic, k = shape if len(shape) == 3 else (shape[0], shape[1], 1)
    return k == 1 and oc >= 32 and ic >= 32 and ic % 32 == 0


def test_synthetic_ecapa_matches_real_checkpoint_manifest():
    """make_ecapa at the published widths (MFA 3072, asp.tdnn 9216 -> 128,
    asp_bn 6144, fc 6144 -> 192) has every manifest tensor with its torch
    shape, nothing else, and stores as Q8_0 exactly what the converter's
    rule quantises.  BatchNorm's num_batches_tracked (a training counter,
    empty shape, never read by the encoder) is the one manifest entry the
    synthetic file leaves out."""
    man = _manifest()
    assert len(man) == 231
    counters = [n for n, s in man if n.endswith(".num_batches_tracked")]
    assert len(counters) == 31 and all(s == [] for n, s in man if n in counters)
    want = {n: s for n, s in man if not n.endswith(".num_batches_tracked")}
    assert len(want) == 200
    assert want["mfa.conv.conv.weight"] == [3072, 3072, 1]
    assert want["asp.tdnn.conv.conv.weight"] == [128, 9216, 1]
    assert want["asp_bn.norm.running_mean"] == [6144]
    assert want["fc.conv.weight"] == [192, 6144, 1]
    kv, T = synth.make_ecapa(seed=1, mfa=3072, wtype=gguf.GGML_Q8_0)
    got = {name: (gtype, list(shape)) for name, gtype, shape, _ in T}
    assert set(got) == set(want)
    for name, shape in want.items():
        gtype, s = got[name]
        if gtype == gguf.GGML_Q8_0:
            assert s + [1] == shape, name      # stored squeezed to 2-D [OC, IC]
        else:
            assert s == shape, name
        assert (gtype == gguf.GGML_Q8_0) == _q8_0_by_converter_rule(name, shape), name
    assert kv["voicedetect.ecapa.channels"] == 1024 and kv["voicedetect.embedding_dim"] == 192
