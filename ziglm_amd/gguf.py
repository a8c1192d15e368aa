"""GGUF files on the host side: the reader over the C-ABI of include/zl_gguf.h (the
library's zl_gguf_* entry points, replacing ziglm's src/gguf.zig GGUFFile) and a writer.

Reader: `GGUFFile.open(path)` / `GGUFFile.from_buffer(bytes)` parse in native code and
raise GGUFError with the reference's error name ("InvalidGGUFMagic", "UnexpectedEOF", ...)
on the files GGUFFile.parse rejects. The getters mirror gguf.zig:319-397 (getMetadata,
getU32, getU64, getF32, getString, getTensor) and `params` is ModelParams as extracted by
gguf.zig:399-451. Tensor data is a zero-copy numpy view of the mapped file.

Writer: `GGUFWriter` lays out a GGUF v3 file (header, metadata, tensor infos, padding to
the alignment, tensor data) -- the counterpart of the reference's BufferWriter
(gguf.zig:465-506) and synthetic.zig's generator. It shares no code with the reader, so a
write -> read round trip checks one against the other.
"""
import ctypes
import struct
from dataclasses import dataclass, field

import numpy as np

from . import bridge as B

MAGIC = 0x46554747

# GGUFValueType (gguf.zig:11-26)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)

# GGMLType ids (types.zig:4-31) used here
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q6_K, GGML_BF16 = 0, 1, 2, 8, 14, 30

ARCH_NAMES = ["llama", "qwen2", "mistral", "gemma", "gemma2", "gemma4", "phi", "phi3", "deepseek",
              "starcoder2", "gpt2", "unknown"]
GEMMA_ARCHS = ("gemma", "gemma2", "gemma4")

ERRORS = {-10: "FileOpenFailed", -11: "InvalidGGUFFile", -12: "InvalidGGUFMagic", -13: "UnsupportedGGUFVersion",
          -14: "UnexpectedEOF", -15: "UnsupportedGGUFValueType", -16: "InvalidTensorDimensions",
          -17: "TensorDataOutOfBounds", -18: "InvalidAlignment", -19: "OutOfMemory", -20: "InvalidArgument",
          -21: "DestinationTooSmall"}


class KV(ctypes.Structure):
    _fields_ = [("key", ctypes.c_void_p), ("key_len", ctypes.c_uint64), ("type", ctypes.c_uint32),
                ("array_type", ctypes.c_uint32), ("array_len", ctypes.c_uint64), ("data", ctypes.c_void_p),
                ("data_bytes", ctypes.c_uint64)]


class TensorC(ctypes.Structure):
    _fields_ = [("name", ctypes.c_void_p), ("name_len", ctypes.c_uint64), ("type", ctypes.c_uint32),
                ("n_dims", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64),
                ("data", ctypes.c_void_p), ("size_bytes", ctypes.c_uint64)]


class ParamsC(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_int32), ("use_gemma_rms_unit_offset", ctypes.c_int32),
                ("context_length", ctypes.c_uint64), ("embedding_length", ctypes.c_uint64),
                ("feed_forward_length", ctypes.c_uint64), ("head_count", ctypes.c_uint64),
                ("head_count_kv", ctypes.c_uint64), ("block_count", ctypes.c_uint64),
                ("head_size", ctypes.c_uint64), ("vocab_size", ctypes.c_uint64),
                ("layer_norm_rms_epsilon", ctypes.c_float), ("rope_freq_base", ctypes.c_float),
                ("rope_freq_scale", ctypes.c_float), ("attn_logit_softcapping", ctypes.c_float),
                ("final_logit_softcapping", ctypes.c_float), ("rope_type", ctypes.c_int32),
                ("rope_dim_count", ctypes.c_uint64), ("expert_count", ctypes.c_uint64),
                ("expert_used_count", ctypes.c_uint64), ("sliding_window", ctypes.c_uint64),
                ("num_kv_shared_layers", ctypes.c_uint64)]


_v, _u32, _u64, _i64, _i = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64, ctypes.c_int
_P = ctypes.POINTER

# name -> (restype, argtypes), in header order (include/zl_gguf.h).
SIGNATURES = {
    "zl_gguf_open": (_i, [ctypes.c_char_p, _P(_v)]),
    "zl_gguf_open_buffer": (_i, [_v, _u64, _P(_v)]),
    "zl_gguf_close": (None, [_v]),
    "zl_gguf_error_name": (ctypes.c_char_p, [_i]),
    "zl_gguf_version": (_u32, [_v]),
    "zl_gguf_tensor_count": (_u64, [_v]),
    "zl_gguf_metadata_count": (_u64, [_v]),
    "zl_gguf_alignment": (_u64, [_v]),
    "zl_gguf_data_offset": (_u64, [_v]),
    "zl_gguf_file_size": (_u64, [_v]),
    "zl_gguf_base": (_v, [_v]),
    "zl_gguf_metadata": (_i, [_v, _u64, _P(KV)]),
    "zl_gguf_find_metadata": (_i64, [_v, ctypes.c_char_p]),
    "zl_gguf_get_u32": (_i, [_v, ctypes.c_char_p, _P(_u32)]),
    "zl_gguf_get_u64": (_i, [_v, ctypes.c_char_p, _P(_u64)]),
    "zl_gguf_get_f32": (_i, [_v, ctypes.c_char_p, _P(ctypes.c_float)]),
    "zl_gguf_get_string": (_i, [_v, ctypes.c_char_p, _P(_v), _P(_u64)]),
    "zl_gguf_tensor": (_i, [_v, _u64, _P(TensorC)]),
    "zl_gguf_find_tensor": (_i64, [_v, ctypes.c_char_p, _P(TensorC)]),
    "zl_ggml_block_size": (_u64, [_u32]),
    "zl_ggml_type_size": (_u64, [_u32]),
    "zl_gguf_params": (None, [_v, _P(ParamsC)]),
    "zl_gguf_upload_tensors": (_i, [_v, _P(_u64), _P(_v), _P(_u64), _u64, _v]),
    "zl_gguf_upload": (_i, [_v, _u64, _v, _u64, _v]),
    "zl_upload_host": (_i, [_v, _v, _u64, _v]),
}

_lib = None


def lib():
    """The zl_gguf_* entry points of libhip_bridge.so (typed)."""
    global _lib
    if _lib is None:
        L = ctypes.CDLL(B.LIB_PATH) if not B._bridge else B._bridge.lib
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


class GGUFError(RuntimeError):
    def __init__(self, code, what):
        self.code = code
        self.name = ERRORS.get(code) or lib().zl_gguf_error_name(code).decode()
        super().__init__(f"{what}: {self.name} ({code})")


@dataclass
class Tensor:
    """types.zig:296-330 Tensor: GGUF-order shape (shape[0] contiguous), raw bytes."""
    name: str
    type: int
    n_dims: int
    shape: tuple
    offset: int
    size_bytes: int
    data: np.ndarray  # uint8 view into the file
    index: int

    def elements(self):
        n = 1
        for d in self.shape[:self.n_dims]:
            n *= d
        return n

    def row_bytes(self):
        """getRowBytes (types.zig:320-324)."""
        return self.shape[0] // block_size(self.type) * type_size(self.type)


@dataclass
class ModelParams:
    """types.zig:246-267, as GGUFFile.extractParams leaves it."""
    arch: str = "llama"
    use_gemma_rms_unit_offset: bool = False
    context_length: int = 2048
    embedding_length: int = 4096
    feed_forward_length: int = 11008
    head_count: int = 32
    head_count_kv: int = 32
    block_count: int = 32
    head_size: int = 0
    vocab_size: int = 32000
    layer_norm_rms_epsilon: float = 1e-5
    rope_freq_base: float = 10000.0
    rope_freq_scale: float = 1.0
    attn_logit_softcapping: float = 0.0
    final_logit_softcapping: float = 0.0
    rope_type: int = 0
    rope_dim_count: int = 0
    expert_count: int = 0
    expert_used_count: int = 0
    sliding_window: int = 0
    num_kv_shared_layers: int = 0


def block_size(t):
    return lib().zl_ggml_block_size(t)


def type_size(t):
    return lib().zl_ggml_type_size(t)


def _decode_scalar(t, raw):
    fmt = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<B", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}[t]
    v = struct.unpack(fmt, raw)[0]
    return bool(v) if t == BOOL else v


class GGUFFile:
    """A parsed GGUF file (gguf.zig:55-71). Close it (or use `with`) to unmap."""

    def __init__(self, handle, keepalive=None):
        self._h = ctypes.c_void_p(handle)
        self._keep = keepalive
        L = lib()
        self.version = L.zl_gguf_version(self._h)
        self.tensor_count = L.zl_gguf_tensor_count(self._h)
        self.metadata_count = L.zl_gguf_metadata_count(self._h)
        self.alignment = L.zl_gguf_alignment(self._h)
        self.data_offset = L.zl_gguf_data_offset(self._h)
        self.size = L.zl_gguf_file_size(self._h)
        p = ParamsC()
        L.zl_gguf_params(self._h, ctypes.byref(p))
        self.params = ModelParams(**{n: getattr(p, n) for n, _ in ParamsC._fields_ if n != "arch"})
        self.params.arch = ARCH_NAMES[p.arch]
        self.params.use_gemma_rms_unit_offset = bool(p.use_gemma_rms_unit_offset)
        base = L.zl_gguf_base(self._h)
        self._buf = (ctypes.c_uint8 * self.size).from_address(base) if self.size else None
        self._base = base

    @classmethod
    def open(cls, path):
        h = ctypes.c_void_p()
        rc = lib().zl_gguf_open(str(path).encode(), ctypes.byref(h))
        if rc != 0:
            raise GGUFError(rc, f"open {path}")
        return cls(h.value)

    @classmethod
    def from_buffer(cls, data):
        """Parse an in-memory image (initFromBuffer); the bytes are kept alive here."""
        buf = (ctypes.c_uint8 * len(data)).from_buffer_copy(bytes(data)) if len(data) else (ctypes.c_uint8 * 1)()
        h = ctypes.c_void_p()
        rc = lib().zl_gguf_open_buffer(ctypes.addressof(buf), len(data), ctypes.byref(h))
        if rc != 0:
            raise GGUFError(rc, "parse buffer")
        return cls(h.value, keepalive=buf)

    def close(self):
        if self._h is not None and self._h.value:
            lib().zl_gguf_close(self._h)
        self._h = None
        self._buf = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def handle(self):
        return self._h

    def _bytes(self, ptr, n):
        return ctypes.string_at(ptr, n) if n else b""

    # ---- metadata -------------------------------------------------------------------
    def metadata(self):
        """All entries in file order: list of (key, type, value); arrays give
        (element_type, [values]) and strings str (undecodable bytes: bytes)."""
        out = []
        for i in range(self.metadata_count):
            kv = KV()
            lib().zl_gguf_metadata(self._h, i, ctypes.byref(kv))
            out.append((self._bytes(kv.key, kv.key_len).decode(errors="surrogateescape"), kv.type, self._value(kv)))
        return out

    def _value(self, kv):
        raw = self._bytes(kv.data, kv.data_bytes)
        if kv.type == STRING:
            return _str(raw)
        if kv.type == ARRAY:
            return kv.array_type, _array(kv.array_type, kv.array_len, raw)
        return _decode_scalar(kv.type, raw)

    def getMetadata(self, key):
        i = lib().zl_gguf_find_metadata(self._h, key.encode())
        if i < 0:
            return None
        kv = KV()
        lib().zl_gguf_metadata(self._h, i, ctypes.byref(kv))
        return kv.type, self._value(kv)

    def getU32(self, key):
        v = ctypes.c_uint32()
        return v.value if lib().zl_gguf_get_u32(self._h, key.encode(), ctypes.byref(v)) else None

    def getU64(self, key):
        v = ctypes.c_uint64()
        return v.value if lib().zl_gguf_get_u64(self._h, key.encode(), ctypes.byref(v)) else None

    def getF32(self, key):
        v = ctypes.c_float()
        return v.value if lib().zl_gguf_get_f32(self._h, key.encode(), ctypes.byref(v)) else None

    def getString(self, key):
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        if not lib().zl_gguf_get_string(self._h, key.encode(), ctypes.byref(p), ctypes.byref(n)):
            return None
        return _str(self._bytes(p.value, n.value))

    # ---- tensors ----------------------------------------------------------------------
    def _tensor(self, t, index):
        start = t.data - self._base if t.data else 0
        data = np.frombuffer(self._buf, np.uint8, t.size_bytes, start) if t.size_bytes else np.zeros(0, np.uint8)
        return Tensor(self._bytes(t.name, t.name_len).decode(errors="surrogateescape"), t.type, t.n_dims,
                      tuple(int(s) for s in t.shape), t.offset, t.size_bytes, data, index)

    def tensor(self, i):
        t = TensorC()
        if lib().zl_gguf_tensor(self._h, i, ctypes.byref(t)) != 0:
            raise IndexError(i)
        return self._tensor(t, i)

    def tensors(self):
        return [self.tensor(i) for i in range(self.tensor_count)]

    def getTensor(self, name):
        t = TensorC()
        i = lib().zl_gguf_find_tensor(self._h, name.encode(), ctypes.byref(t))
        return None if i < 0 else self._tensor(t, i)

    # ---- device tables ------------------------------------------------------------------
    def upload(self, tensors, bufs, stream=None):
        """Copy each tensor's bytes into the matching device buffer (DeviceBuffer) through
        the pinned ring; returns when done."""
        n = len(tensors)
        idx = (ctypes.c_uint64 * n)(*[t.index for t in tensors])
        dst = (ctypes.c_void_p * n)(*[b.ptr for b in bufs])
        cap = (ctypes.c_uint64 * n)(*[b.size_bytes for b in bufs])
        rc = lib().zl_gguf_upload_tensors(self._h, idx, dst, cap, n, stream)
        if rc != 0:
            raise GGUFError(rc, "upload")


def _str(raw):
    try:
        return raw.decode()
    except UnicodeDecodeError:
        return raw


def _array(et, n, raw):
    if et == STRING:
        out, p = [], 0
        for _ in range(n):
            ln = struct.unpack_from("<Q", raw, p)[0]
            out.append(_str(raw[p + 8:p + 8 + ln]))
            p += 8 + ln
        return out
    if et == ARRAY:
        out, p = [], 0
        for _ in range(n):
            sub_t, sub_n = struct.unpack_from("<IQ", raw, p)
            sub_raw, used = _array_extent(sub_t, sub_n, raw, p + 12)
            out.append((sub_t, _array(sub_t, sub_n, sub_raw)))
            p = used
        return out
    dt = {UINT8: "<u1", INT8: "<i1", UINT16: "<u2", INT16: "<i2", UINT32: "<u4", INT32: "<i4", FLOAT32: "<f4",
          BOOL: "<u1", UINT64: "<u8", INT64: "<i8", FLOAT64: "<f8"}.get(et)
    if dt is None:
        return []  # empty array of an unknown type
    return np.frombuffer(raw, dt, n).tolist()


def _array_extent(t, n, raw, p):
    """(bytes of a nested array's elements, position after them)."""
    start = p
    size = {UINT8: 1, INT8: 1, BOOL: 1, UINT16: 2, INT16: 2, UINT32: 4, INT32: 4, FLOAT32: 4, UINT64: 8, INT64: 8,
            FLOAT64: 8}.get(t)
    if size is not None:
        p += n * size
    elif t == STRING:
        for _ in range(n):
            p += 8 + struct.unpack_from("<Q", raw, p)[0]
    elif t == ARRAY:
        for _ in range(n):
            st, sn = struct.unpack_from("<IQ", raw, p)
            _, p = _array_extent(st, sn, raw, p + 12)
    return raw[start:p], p


# ---------------------------------------------------------------------------------------
# Writer
# ---------------------------------------------------------------------------------------

_SCALAR_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
               BOOL: "<B", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def _enc_str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _enc_value(t, v):
    if t == STRING:
        return _enc_str(v)
    if t == ARRAY:
        et, items = v
        out = [struct.pack("<IQ", et, len(items))]
        out.extend(_enc_value(et, x) for x in items)
        return b"".join(out)
    return struct.pack(_SCALAR_FMT[t], v)


@dataclass
class GGUFWriter:
    """Builds a GGUF image: add metadata with `kv(key, type, value)` (arrays: value =
    (element_type, list)) and tensors with `tensor(name, ggml_type, shape, raw_bytes)`
    (shape in GGUF order, shape[0] contiguous). Tensor data is placed back to back, each
    start rounded up to `alignment` (GGUF's convention; the reference's synthetic writer
    packs them unpadded, synthetic.zig:217-226, which `pad_tensors=False` reproduces)."""
    version: int = 3
    alignment: int = 32
    pad_tensors: bool = True
    kvs: list = field(default_factory=list)
    infos: list = field(default_factory=list)

    def kv(self, key, t, value):
        self.kvs.append((key, t, value))
        return self

    def tensor(self, name, ggml_type, shape, data):
        self.infos.append((name, ggml_type, tuple(int(s) for s in shape), memoryview(np.ascontiguousarray(data)).cast("B")))
        return self

    def _layout(self):
        offs, off = [], 0
        for _, _, _, data in self.infos:
            if self.pad_tensors:
                off = (off + self.alignment - 1) // self.alignment * self.alignment
            offs.append(off)
            off += data.nbytes
        return offs, off

    def header(self):
        offs, _ = self._layout()
        out = [struct.pack("<IIQQ", MAGIC, self.version, len(self.infos), len(self.kvs))]
        for key, t, v in self.kvs:
            out.append(_enc_str(key) + struct.pack("<I", t) + _enc_value(t, v))
        for (name, gt, shape, _), off in zip(self.infos, offs):
            out.append(_enc_str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", s) for s in shape)
                       + struct.pack("<IQ", gt, off))
        head = b"".join(out)
        pad = (-len(head)) % self.alignment
        return head + b"\0" * pad

    def tobytes(self):
        parts = [self.header()]
        offs, _ = self._layout()
        pos = 0
        for (_, _, _, data), off in zip(self.infos, offs):
            parts.append(b"\0" * (off - pos))
            parts.append(data.tobytes())
            pos = off + data.nbytes
        return b"".join(parts)

    def write(self, path):
        """Stream the file (tensor data is not concatenated in memory)."""
        offs, _ = self._layout()
        with open(path, "wb") as f:
            f.write(self.header())
            pos = 0
            for (_, _, _, data), off in zip(self.infos, offs):
                f.write(b"\0" * (off - pos))
                f.write(data)
                pos = off + data.nbytes
        return path
