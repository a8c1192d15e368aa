"""CPU restatement of ziglm's GGUF reader (src/gguf.zig GGUFFile.parse + extractParams,
src/types.zig sizes and initComputed) in plain Python, for differential tests of the
native reader (include/zl_gguf.h). Test infrastructure only: nothing in the product
imports it.

parse(buf) returns a dict with version, counts, alignment, data_offset, metadata
[(key, type, raw value bytes)], tensors [(name, type, n_dims, shape4, offset, size)] and
params, or raises RefError(name) with the Zig error name. It follows the reference
step by step:
  header          gguf.zig:242-256
  metadata loop   gguf.zig:258-267 (parseValue 213-239; only a UINT32 general.alignment
                  counts, 264-266)
  tensor infos    gguf.zig:269-297 (n_dims > 4 rejected, shape defaults to 1)
  data offset     gguf.zig:299-301 (align up with a mask)
  bounds          gguf.zig:303-311 (size = elements / block * type size, types.zig:313-318)
  params          gguf.zig:399-451, getters 326-389, initComputed types.zig:269-285
The one deliberate difference of the native reader, an error for general.alignment 0 or
a non-power of two (where the reference's mask arithmetic overflows or misaligns), is
mirrored here as RefError("InvalidAlignment") so the two stay comparable.
"""
import struct

# types.zig:33-40
_BLOCK1 = {0, 1, 16, 17, 18, 19, 20, 30}
_BLOCK256 = {10, 11, 12, 13, 14, 15, 21, 23, 24, 25}
# types.zig:42-67 (and the BlockQ* sizes asserted at types.zig:375-388)
_TYPE_SIZE = {0: 4, 1: 2, 30: 2, 16: 1, 17: 2, 18: 4, 19: 8, 20: 8, 2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 9: 36,
              10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 15: 292, 22: 18}
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}
_U64 = (1 << 64) - 1


class RefError(Exception):
    pass


def block_size(t):
    return 1 if t in _BLOCK1 else 256 if t in _BLOCK256 else 32


def type_size(t):
    return _TYPE_SIZE.get(t, 1)


class _Reader:
    def __init__(self, buf):
        self.b, self.p = buf, 0

    def take(self, n):
        if self.p + n > len(self.b):
            raise RefError("UnexpectedEOF")
        v = self.b[self.p:self.p + n]
        self.p += n
        return v

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def string(self):
        return self.take(self.u64())

    def value(self, t):
        """parseValue (gguf.zig:213-239): returns the raw bytes of the value."""
        start = self.p
        if t in _SCALAR:
            self.take(struct.calcsize(_SCALAR[t]))
        elif t == 8:
            self.string()
        elif t == 9:
            et, n = self.u32(), self.u64()
            for _ in range(n):
                self.value(et)
        else:
            raise RefError("UnsupportedGGUFValueType")
        return self.b[start:self.p]


def parse(buf):
    buf = bytes(buf)
    r = _Reader(buf)
    if r.u32() != 0x46554747:
        raise RefError("InvalidGGUFMagic")
    version = r.u32()
    if version not in (2, 3):
        raise RefError("UnsupportedGGUFVersion")
    tensor_count, metadata_count = r.u64(), r.u64()
    alignment = 32
    metadata = []
    for _ in range(metadata_count):
        key = r.string()
        t = r.u32()
        raw = r.value(t)
        metadata.append((key, t, raw))
        if key == b"general.alignment" and t == 4:
            alignment = struct.unpack("<I", raw)[0]
    tensors = []
    for _ in range(tensor_count):
        name = r.string()
        n_dims = r.u32()
        if n_dims > 4:
            raise RefError("InvalidTensorDimensions")
        shape = [1, 1, 1, 1]
        for d in range(n_dims):
            shape[d] = r.u64()
        t, off = r.u32(), r.u64()
        tensors.append([name, t, n_dims, tuple(shape), off, 0])
    if alignment == 0 or alignment & (alignment - 1):
        raise RefError("InvalidAlignment")
    data_offset = (r.p + alignment - 1) & ~(alignment - 1)
    for rec in tensors:
        elems = 1
        for d in range(rec[2]):
            elems = (elems * rec[3][d]) & _U64
        size = (elems // block_size(rec[1]) * type_size(rec[1])) & _U64
        rec[5] = size
        a = data_offset + rec[4]
        if a > _U64 or a + size > len(buf):
            raise RefError("TensorDataOutOfBounds")
    out = {"version": version, "tensor_count": tensor_count, "metadata_count": metadata_count,
           "alignment": alignment, "data_offset": data_offset, "metadata": metadata,
           "tensors": [tuple(t) for t in tensors]}
    out["params"] = params(out)
    return out


# ---- getters (gguf.zig:319-389) -----------------------------------------------------
def _first(meta, key):
    for k, t, raw in meta:
        if k == key:
            return t, raw
    return None


def _scalar(t, raw):
    return struct.unpack(_SCALAR[t], raw[:struct.calcsize(_SCALAR[t])])[0]


def get_u32(meta, key):
    e = _first(meta, key)
    if e is None:
        return None
    t, raw = e
    if t == 4:
        return _scalar(4, raw)
    if t == 10:
        return _scalar(10, raw) & 0xFFFFFFFF
    if t == 5:
        v = _scalar(5, raw)
        return v if v >= 0 else None
    return None


def get_u64(meta, key):
    e = _first(meta, key)
    if e is None:
        return None
    t, raw = e
    if t == 9:
        et, n = struct.unpack_from("<IQ", raw)
        if n == 0 or et not in (4, 10, 5, 11):
            return None
        t, raw = et, raw[12:]
    if t in (10, 4):
        return _scalar(t, raw)
    if t in (11, 5):
        v = _scalar(t, raw)
        return v if v >= 0 else None
    return None


def get_f32(meta, key):
    e = _first(meta, key)
    if e is None:
        return None
    t, raw = e
    if t == 6:
        return _scalar(6, raw)
    if t == 12:
        return struct.unpack("<f", struct.pack("<f", _scalar(12, raw)))[0]
    if t == 9:
        et, n = struct.unpack_from("<IQ", raw)
        if n > 0 and et == 6:
            return _scalar(6, raw[12:])
    return None


def get_string(meta, key):
    e = _first(meta, key)
    if e is None or e[0] != 8:
        return None
    return e[1][8:]


_ARCH = {b"llama": "llama", b"qwen2": "qwen2", b"qwen2.5": "qwen2", b"mistral": "mistral", b"gemma": "gemma",
         b"gemma2": "gemma2", b"gemma4": "gemma4", b"gemma_4": "gemma4", b"phi": "phi", b"phi2": "phi",
         b"phi3": "phi3", b"deepseek": "deepseek", b"starcoder2": "starcoder2", b"gpt2": "gpt2"}


def params(f):
    """extractParams (gguf.zig:399-451) + initComputed (types.zig:269-285)."""
    meta = f["metadata"]
    p = dict(arch="llama", use_gemma_rms_unit_offset=False, context_length=2048, embedding_length=4096,
             feed_forward_length=11008, head_count=32, head_count_kv=32, block_count=32, head_size=0,
             vocab_size=32000, layer_norm_rms_epsilon=struct.unpack("<f", struct.pack("<f", 1e-5))[0],
             rope_freq_base=10000.0, rope_freq_scale=1.0, rope_dim_count=0, sliding_window=0,
             final_logit_softcapping=0.0)
    arch = get_string(meta, b"general.architecture")
    if arch is None:
        arch = b"llama"
    p["arch"] = _ARCH.get(arch, "unknown")

    def key(name):
        k = arch + b"." + name.encode()
        return k if len(k) <= 128 else None

    for name, field in [("context_length", "context_length"), ("embedding_length", "embedding_length"),
                        ("feed_forward_length", "feed_forward_length"), ("block_count", "block_count"),
                        ("attention.head_count", "head_count")]:
        k = key(name)
        v = get_u64(meta, k) if k else None
        if v is not None:
            p[field] = v
    k = key("attention.head_count_kv")
    v = get_u64(meta, k) if k else None
    p["head_count_kv"] = v if v is not None else p["head_count"]
    for name, field in [("attention.key_length", "head_size"), ("attention.sliding_window", "sliding_window")]:
        k = key(name)
        v = get_u64(meta, k) if k else None
        if v is not None:
            p[field] = v
    for name, field in [("attention.layer_norm_rms_epsilon", "layer_norm_rms_epsilon"),
                        ("rope.freq_base", "rope_freq_base"), ("rope.freq_scale", "rope_freq_scale")]:
        k = key(name)
        v = get_f32(meta, k) if k else None
        if v is not None:
            p[field] = v
    k = key("rope.dimension_count")
    v = get_u64(meta, k) if k else None
    if v is not None:
        p["rope_dim_count"] = v
    k = key("final_logit_softcapping")
    v = get_f32(meta, k) if k else None
    if v is not None:
        p["final_logit_softcapping"] = v
    embd = [t for t in f["tensors"] if t[0] == b"token_embd.weight"]
    if embd:
        p["vocab_size"] = embd[-1][3][1]
    if p["head_count"] > 0 and p["head_size"] == 0:
        p["head_size"] = p["embedding_length"] // p["head_count"]
    if p["rope_dim_count"] == 0:
        p["rope_dim_count"] = p["head_size"]
    if p["head_count_kv"] == 0:
        p["head_count_kv"] = p["head_count"]
    if p["arch"] in ("gemma", "gemma2"):
        p["use_gemma_rms_unit_offset"] = True
    elif p["arch"] == "gemma4":
        p["use_gemma_rms_unit_offset"] = False
    return p
