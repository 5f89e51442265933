"""Minimal GGUF v3 writer/reader (numpy only).

GGUF is the model container the reference's `ModelLoader::load` reads
(src/model_loader.cpp:114-215): a header, `voicedetect.*` key/values and named
tensors whose dims are listed fastest-first (ggml `ne` order).  This module
writes and reads the subset the speaker encoders use: scalar/string/array KV and
F32, F16 and Q8_0 tensors.

Q8_0 is ggml's public block format: 32 consecutive elements of a row share one
f16 scale `d`; the block stores d (2 bytes) then 32 int8 quants (34 bytes in
all) and dequantises as q * d.  The quantiser follows gguf-py's published
recipe: d = max|x| / 127, q = round-half-away-from-zero(x / d).
"""
import struct

import numpy as np

GGUF_MAGIC = 0x46554747  # "GGUF" little-endian
GGUF_VERSION = 3
ALIGNMENT = 32

# value types
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
# ggml tensor types
GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8
QK8_0 = 32
Q8_0_BLOCK_BYTES = 34

_SCALAR_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
               T_F32: "<f", T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


class U32(int):
    pass


class I32(int):
    pass


class F32(float):
    pass


def quantize_q8_0(x):
    """Quantise the last axis (length a multiple of 32) into Q8_0 block bytes."""
    x = np.asarray(x, dtype=np.float32)
    assert x.shape[-1] % QK8_0 == 0, "Q8_0 rows must be a multiple of 32"
    blocks = x.reshape(-1, QK8_0)
    d = np.abs(blocks).max(axis=1) / np.float32(127.0)
    with np.errstate(divide="ignore"):
        inv = np.where(d == 0, np.float32(0), np.float32(1.0) / d).astype(np.float32)
    v = blocks * inv[:, None]
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)
    out = np.empty((blocks.shape[0], Q8_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def dequantize_q8_0(raw, n):
    b = np.frombuffer(raw, dtype=np.uint8).reshape(-1, Q8_0_BLOCK_BYTES)[: n // QK8_0]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    q = b[:, 2:].copy().view(np.int8).astype(np.float32)
    return (q * d).reshape(-1)


def _tensor_nbytes(ggml_type, n):
    if ggml_type == GGML_F32:
        return 4 * n
    if ggml_type == GGML_F16:
        return 2 * n
    if ggml_type == GGML_Q8_0:
        return (n // QK8_0) * Q8_0_BLOCK_BYTES
    raise ValueError(f"unsupported ggml type {ggml_type}")


def _pstr(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _kv_value(v):
    """Encode (type, payload) for a python value; ints default to u32."""
    if isinstance(v, bool):
        return T_BOOL, struct.pack("<?", v)
    if isinstance(v, I32):
        return T_I32, struct.pack("<i", int(v))
    if isinstance(v, int):
        return T_U32, struct.pack("<I", int(v))
    if isinstance(v, float):
        return T_F32, struct.pack("<f", float(v))
    if isinstance(v, str):
        return T_STR, _pstr(v)
    if isinstance(v, (list, tuple)):
        if len(v) and all(isinstance(e, str) for e in v) or (len(v) == 0):
            payload = struct.pack("<IQ", T_STR, len(v)) + b"".join(_pstr(e) for e in v)
            return T_ARR, payload
        if all(isinstance(e, int) and not isinstance(e, bool) for e in v):
            payload = struct.pack("<IQ", T_I32, len(v)) + b"".join(struct.pack("<i", int(e)) for e in v)
            return T_ARR, payload
        if all(isinstance(e, float) for e in v):
            payload = struct.pack("<IQ", T_F32, len(v)) + b"".join(struct.pack("<f", e) for e in v)
            return T_ARR, payload
    raise TypeError(f"cannot encode KV value {v!r}")


def write_gguf(path, kv, tensors):
    """kv: dict key -> value; tensors: list of (name, ggml_type, shape_rowmajor, ndarray).

    `shape_rowmajor` is the numpy (slowest-first) shape; it is stored reversed
    as the ggml `ne`.  F32/F16 data is cast; Q8_0 data is quantised row-wise.
    """
    infos = []
    blobs = []
    offset = 0
    for name, gtype, shape, arr in tensors:
        arr = np.asarray(arr)
        n = int(np.prod(shape)) if len(shape) else 1
        assert arr.size == n, (name, arr.shape, shape)
        if gtype == GGML_F32:
            raw = np.ascontiguousarray(arr, dtype=np.float32).tobytes()
        elif gtype == GGML_F16:
            raw = np.ascontiguousarray(arr, dtype=np.float16).tobytes()
        elif gtype == GGML_Q8_0:
            raw = quantize_q8_0(arr.reshape(-1, shape[-1])).tobytes()
        else:
            raise ValueError(gtype)
        assert len(raw) == _tensor_nbytes(gtype, n)
        infos.append((name, list(reversed(shape)), gtype, offset))
        pad = (-len(raw)) % ALIGNMENT
        blobs.append(raw + b"\0" * pad)
        offset += len(raw) + pad
    head = bytearray()
    head += struct.pack("<IIQQ", GGUF_MAGIC, GGUF_VERSION, len(infos), len(kv))
    for k, v in kv.items():
        t, payload = _kv_value(v)
        head += _pstr(k) + struct.pack("<I", t) + payload
    for name, ne, gtype, off in infos:
        head += _pstr(name) + struct.pack("<I", len(ne))
        for d in ne:
            head += struct.pack("<Q", d)
        head += struct.pack("<IQ", gtype, off)
    head += b"\0" * ((-len(head)) % ALIGNMENT)
    with open(path, "wb") as f:
        f.write(bytes(head))
        for b in blobs:
            f.write(b)


class GGUFFile:
    """Parsed GGUF: .kv (dict) and .tensors (name -> (ggml_type, ne, raw bytes))."""

    def __init__(self, path):
        with open(path, "rb") as f:
            self.buf = f.read()
        self.pos = 0
        magic, ver, nt, nkv = self._unpack("<IIQQ")
        if magic != GGUF_MAGIC:
            raise ValueError("not a GGUF file")
        if ver not in (2, 3):
            raise ValueError(f"unsupported GGUF version {ver}")
        self.kv = {}
        for _ in range(nkv):
            key = self._str()
            (t,) = self._unpack("<I")
            self.kv[key] = self._value(t)
        align = int(self.kv.get("general.alignment", ALIGNMENT))
        infos = []
        for _ in range(nt):
            name = self._str()
            (nd,) = self._unpack("<I")
            ne = [self._unpack("<Q")[0] for _ in range(nd)]
            gtype, off = self._unpack("<IQ")
            infos.append((name, ne, gtype, off))
        base = (self.pos + align - 1) // align * align
        self.tensors = {}
        for name, ne, gtype, off in infos:
            n = int(np.prod(ne)) if ne else 1
            nb = _tensor_nbytes(gtype, n)
            self.tensors[name] = (gtype, ne, self.buf[base + off: base + off + nb])

    def _unpack(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.pos)
        self.pos += struct.calcsize(fmt)
        return v

    def _str(self):
        (n,) = self._unpack("<Q")
        s = self.buf[self.pos:self.pos + n].decode("utf-8")
        self.pos += n
        return s

    def _value(self, t):
        if t == T_STR:
            return self._str()
        if t == T_ARR:
            et, n = self._unpack("<IQ")
            return [self._value(et) for _ in range(n)]
        return self._unpack(_SCALAR_FMT[t])[0]

    def array(self, name):
        """Tensor as float32 numpy array in row-major (slowest-first) shape."""
        gtype, ne, raw = self.tensors[name]
        n = int(np.prod(ne)) if ne else 1
        if gtype == GGML_F32:
            a = np.frombuffer(raw, dtype=np.float32)
        elif gtype == GGML_F16:
            a = np.frombuffer(raw, dtype=np.float16).astype(np.float32)
        elif gtype == GGML_Q8_0:
            a = dequantize_q8_0(raw, n)
        else:
            raise ValueError(gtype)
        return a.reshape(list(reversed(ne)))
