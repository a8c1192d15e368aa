"""The native GGUF reader (include/zl_gguf.h) on the CPU: the reference's own GGUF tests
(gguf.zig:508-527, synthetic.zig:450-463, types.zig:375-399), each reject path of
GGUFFile.parse, the getters' conversions, parameter extraction, and a differential test
against the Python restatement of gguf.zig (oracle/gguf_ref.py) on random files and on
every truncation / many byte mutations of them (same accept/reject, same error name, same
parsed fields)."""
import struct

import numpy as np
import pytest

from oracle import gguf_ref as R
from ziglm_amd import gguf as G


def header(version=3, n_tensors=0, n_kv=0, magic=G.MAGIC):
    return struct.pack("<IIQQ", magic, version, n_tensors, n_kv)


def s(x):
    b = x.encode() if isinstance(x, str) else x
    return struct.pack("<Q", len(b)) + b


def kv_u32(key, v):
    return s(key) + struct.pack("<II", G.UINT32, v)


def expect_error(data, name):
    with pytest.raises(G.GGUFError) as e:
        G.GGUFFile.from_buffer(data)
    assert e.value.name == name
    with pytest.raises(R.RefError) as e2:
        R.parse(data)
    assert str(e2.value) == name


# ---------------------------------------------------------------------------------------
# The reference's tests
# ---------------------------------------------------------------------------------------

def test_reference_in_memory_validation():
    """gguf.zig:508-527: a v3 header with one STRING entry parses; arch llama."""
    data = header(3, 0, 1) + s("general.architecture") + struct.pack("<I", G.STRING) + s("llama")
    with G.GGUFFile.from_buffer(data) as f:
        assert f.version == 3
        assert f.params.arch == "llama"
        assert f.tensor_count == 0 and f.metadata_count == 1


def sample_gguf(arch="llama", block_count=2, dim=64, ffn=128, n_head=4, n_kv=2, vocab=32, ctx=128, seed=42):
    """synthetic.zig:30-250 generateSampleGGUF restated: 15 metadata entries, 3 + 9 per
    block F32 tensors packed back to back from offset 0 (no per-tensor padding), header
    padded to 32, weights (u - 0.5) * 0.02 and norms 1 (numpy's generator stands in for
    Zig's DefaultPrng, so the weight values differ; the layout is the reference's)."""
    w = G.GGUFWriter(pad_tensors=False)
    w.kv("general.architecture", G.STRING, arch)
    for k, v in [("block_count", block_count), ("context_length", ctx), ("embedding_length", dim),
                 ("feed_forward_length", ffn), ("attention.head_count", n_head), ("attention.head_count_kv", n_kv)]:
        w.kv(f"{arch}.{k}", G.UINT32, v)
    w.kv(f"{arch}.attention.layer_norm_rms_epsilon", G.FLOAT32, 1e-5)
    w.kv(f"{arch}.rope.freq_base", G.FLOAT32, 10000.0)
    w.kv(f"{arch}.rope.dimension_count", G.UINT32, dim // n_head)
    w.kv("tokenizer.ggml.model", G.STRING, "gpt2")
    w.kv("tokenizer.ggml.bos_token_id", G.UINT32, 0)
    w.kv("tokenizer.ggml.eos_token_id", G.UINT32, 1)
    toks = ["<s>", "</s>", "<unk>", "Hello", "world", "!", "The", "capital", "of", "France", "is", "Paris"]
    toks += [chr(ord("A") + i) for i in range(20)]
    w.kv("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, [toks[i] if i < len(toks) else f"tok_{i}" for i in range(vocab)]))
    w.kv("tokenizer.ggml.merges", G.ARRAY, (G.STRING, ["t h", "Ġ t"]))
    hs = dim // n_head
    kvd = n_kv * hs
    shapes = [("token_embd.weight", (dim, vocab))]
    for i in range(block_count):
        shapes += [(f"blk.{i}.attn_norm.weight", (dim, 1)), (f"blk.{i}.attn_q.weight", (dim, dim)),
                   (f"blk.{i}.attn_k.weight", (dim, kvd)), (f"blk.{i}.attn_v.weight", (dim, kvd)),
                   (f"blk.{i}.attn_output.weight", (dim, dim)), (f"blk.{i}.ffn_norm.weight", (dim, 1)),
                   (f"blk.{i}.ffn_gate.weight", (dim, ffn)), (f"blk.{i}.ffn_up.weight", (dim, ffn)),
                   (f"blk.{i}.ffn_down.weight", (ffn, dim))]
    shapes += [("output_norm.weight", (dim, 1)), ("output.weight", (dim, vocab))]
    rng = np.random.default_rng(seed)
    arrays = {}
    for name, shp in shapes:
        a = (rng.random(shp[0] * shp[1], dtype=np.float32) - np.float32(0.5)) * np.float32(0.02)
        if name.endswith("norm.weight"):
            a[:] = 1.0
        arrays[name] = a
        w.tensor(name, G.GGML_F32, shp, a)
    return w, arrays


def test_reference_generate_and_load_sample(tmp_path):
    """synthetic.zig:450-463: write the sample model to a file, open it (mmap path)."""
    w, arrays = sample_gguf()
    path = w.write(tmp_path / "sample.gguf")
    with G.GGUFFile.open(path) as f:
        p = f.params
        assert (p.arch, p.block_count, p.embedding_length) == ("llama", 2, 64)
        # beyond the reference's three checks: everything the generator wrote
        assert f.tensor_count == 3 + 2 * 9 and f.metadata_count == 15
        assert (p.feed_forward_length, p.head_count, p.head_count_kv, p.context_length) == (128, 4, 2, 128)
        assert (p.vocab_size, p.head_size, p.rope_dim_count, p.use_gemma_rms_unit_offset) == (32, 16, 16, False)
        assert p.layer_norm_rms_epsilon == np.float32(1e-5) and p.rope_freq_base == 10000.0
        assert f.getString("tokenizer.ggml.model") == "gpt2"
        toks = f.getMetadata("tokenizer.ggml.tokens")
        assert toks[0] == G.ARRAY and toks[1][0] == G.STRING and toks[1][1][:4] == ["<s>", "</s>", "<unk>", "Hello"]
        for name, a in arrays.items():
            t = f.getTensor(name)
            assert t is not None and t.type == G.GGML_F32 and t.size_bytes == a.nbytes
            np.testing.assert_array_equal(t.data.view(np.float32), a)
        # packed data: tensor i starts where i-1 ends, data section 32-aligned
        ts = f.tensors()
        assert ts[0].offset == 0 and all(ts[i].offset == ts[i - 1].offset + ts[i - 1].size_bytes for i in range(1, len(ts)))
        assert f.data_offset % 32 == 0 and f.data_offset + ts[-1].offset + ts[-1].size_bytes == f.size


def test_reference_type_sizes():
    """types.zig:375-399 (block structs and block sizes)."""
    sizes = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 9: 36, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 15: 292, 22: 18}
    for t, n in sizes.items():
        assert G.type_size(t) == n == R.type_size(t)
    for t in (2, 6, 8):
        assert G.block_size(t) == 32
    for t in (10, 11, 12, 13, 14, 15):
        assert G.block_size(t) == 256
    for t in (0, 1, 30, 16, 17, 18, 19, 20):
        assert G.block_size(t) == 1 == R.block_size(t)
    # the fallbacks (types.zig:38, 65): unsized types count 1 byte per 32 / 256 elements
    assert (G.type_size(25), G.block_size(25), G.type_size(99), G.block_size(99)) == (1, 256, 1, 32)


# ---------------------------------------------------------------------------------------
# Reject paths of GGUFFile.parse / open
# ---------------------------------------------------------------------------------------

def test_bad_magic_and_versions():
    expect_error(header(magic=0x46554748), "InvalidGGUFMagic")
    for v in (0, 1, 4, 0xFFFFFFFF):
        expect_error(header(version=v), "UnsupportedGGUFVersion")
    for v in (2, 3):
        with G.GGUFFile.from_buffer(header(version=v)) as f:
            assert f.version == v and f.params.arch == "llama"


def test_open_short_file_and_missing(tmp_path):
    p = tmp_path / "short.gguf"
    p.write_bytes(header()[:23])
    with pytest.raises(G.GGUFError) as e:
        G.GGUFFile.open(p)
    assert e.value.name == "InvalidGGUFFile"            # gguf.zig:80 (file shorter than 24 bytes)
    expect_error(header()[:23], "UnexpectedEOF")        # the buffer path has no size check
    with pytest.raises(G.GGUFError) as e:
        G.GGUFFile.open(tmp_path / "absent.gguf")
    assert e.value.name == "FileOpenFailed"


def test_value_types():
    ok = header(3, 0, 2) + s("a") + struct.pack("<IIQ", G.ARRAY, 77, 0) + kv_u32("b", 5)
    with G.GGUFFile.from_buffer(ok) as f:      # an empty array of an unknown type is accepted
        assert f.getU32("b") == 5
    expect_error(header(3, 0, 1) + s("a") + struct.pack("<II", 13, 0), "UnsupportedGGUFValueType")
    expect_error(header(3, 0, 1) + s("a") + struct.pack("<IIQ", G.ARRAY, 13, 1) + b"\0" * 8,
                 "UnsupportedGGUFValueType")
    expect_error(header(3, 0, 1) + s("a") + struct.pack("<IIQ", G.ARRAY, G.UINT64, 3) + b"\0" * 23, "UnexpectedEOF")
    expect_error(header(3, 0, 1) + s("a") + struct.pack("<IQ", G.STRING, 10) + b"abc", "UnexpectedEOF")


def test_tensor_info_errors():
    ti = s("t") + struct.pack("<I", 5) + struct.pack("<5Q", 1, 1, 1, 1, 1) + struct.pack("<IQ", 0, 0)
    expect_error(header(3, 1, 0) + ti, "InvalidTensorDimensions")
    # 4 f32 elements at offset 0 need 16 bytes after the aligned header
    ti = s("t") + struct.pack("<IQ", 1, 4) + struct.pack("<IQ", 0, 0)
    head = header(3, 1, 0) + ti
    pad = (-len(head)) % 32
    expect_error(head + b"\0" * (pad + 15), "TensorDataOutOfBounds")
    with G.GGUFFile.from_buffer(head + b"\0" * pad + struct.pack("<4f", 1, 2, 3, 4)) as f:
        np.testing.assert_array_equal(f.getTensor("t").data.view(np.float32), [1, 2, 3, 4])
    # offset + size past 2^64
    ti = s("t") + struct.pack("<IQ", 1, 4) + struct.pack("<IQ", 0, (1 << 64) - 8)
    expect_error(header(3, 1, 0) + ti + b"\0" * 64, "TensorDataOutOfBounds")


def test_alignment_rules():
    def build(align_kv):
        head = header(3, 1, 1) + align_kv + s("t") + struct.pack("<IQ", 1, 2) + struct.pack("<IQ", 0, 0)
        return head
    # UINT32 general.alignment is honoured (gguf.zig:264-266)
    head = build(kv_u32("general.alignment", 64))
    data = head + b"\0" * ((-len(head)) % 64) + struct.pack("<2f", 7, 8)
    with G.GGUFFile.from_buffer(data) as f:
        assert f.alignment == 64 and f.data_offset % 64 == 0 and f.data_offset >= len(head)
        np.testing.assert_array_equal(f.getTensor("t").data.view(np.float32), [7, 8])
    # a UINT64 alignment is ignored: 32 stays
    head = build(s("general.alignment") + struct.pack("<IQ", G.UINT64, 64))
    with G.GGUFFile.from_buffer(head + b"\0" * 128) as f:
        assert f.alignment == 32 and f.data_offset == (len(head) + 31) // 32 * 32
    # 0 and non-powers of two are refused (the reference's mask arithmetic breaks on them)
    for a in (0, 24):
        expect_error(build(kv_u32("general.alignment", a)) + b"\0" * 128, "InvalidAlignment")


# ---------------------------------------------------------------------------------------
# Getters and parameters
# ---------------------------------------------------------------------------------------

def test_getters_conversions():
    w = G.GGUFWriter()
    w.kv("u64big", G.UINT64, (1 << 40) + 7).kv("i32", G.INT32, 12).kv("i32neg", G.INT32, -3)
    w.kv("i64", G.INT64, 1 << 35).kv("arr_u32", G.ARRAY, (G.UINT32, [9, 10])).kv("arr_i64", G.ARRAY, (G.INT64, [-1]))
    w.kv("arr_empty", G.ARRAY, (G.UINT32, [])).kv("arr_f32", G.ARRAY, (G.FLOAT32, [2.5, 1.0]))
    w.kv("f64", G.FLOAT64, 0.1).kv("str", G.STRING, "x").kv("b", G.BOOL, True).kv("u16", G.UINT16, 3)
    w.kv("dup", G.UINT32, 1).kv("dup", G.UINT32, 2)
    with G.GGUFFile.from_buffer(w.tobytes()) as f:
        assert f.getU32("u64big") == 7                      # truncated (gguf.zig:330)
        assert f.getU64("u64big") == (1 << 40) + 7
        assert f.getU32("i32") == 12 and f.getU64("i32") == 12
        assert f.getU32("i32neg") is None and f.getU64("i32neg") is None
        assert f.getU32("i64") is None and f.getU64("i64") == 1 << 35
        assert f.getU64("arr_u32") == 9 and f.getU32("arr_u32") is None   # first element
        assert f.getU64("arr_i64") is None and f.getU64("arr_empty") is None
        assert f.getF32("arr_f32") == 2.5 and f.getF32("f64") == np.float32(0.1)
        assert f.getF32("i32") is None and f.getString("i32") is None and f.getString("str") == "x"
        assert f.getU64("b") is None and f.getU32("u16") is None   # no other conversions
        assert f.getU32("dup") == 1                          # first entry wins (getMetadata)
        assert f.getU32("absent") is None and f.getMetadata("absent") is None
        md = dict((k, v) for k, _, v in reversed(f.metadata()))
        assert md["b"] is True and md["arr_u32"] == (G.UINT32, [9, 10]) and md["u16"] == 3


def test_duplicate_tensor_names_last_wins():
    w = G.GGUFWriter()
    w.tensor("t", G.GGML_F32, (2,), np.array([1, 2], np.float32))
    w.tensor("t", G.GGML_F32, (2,), np.array([3, 4], np.float32))
    with G.GGUFFile.from_buffer(w.tobytes()) as f:
        t = f.getTensor("t")
        assert t.index == 1 and list(t.data.view(np.float32)) == [3, 4]


def gemma_kvs(arch, w, **over):
    vals = dict(context_length=8192, embedding_length=2560, feed_forward_length=10240, block_count=34,
                **{"attention.head_count": 8, "attention.head_count_kv": 4, "attention.key_length": 256,
                   "attention.sliding_window": 1024})
    vals.update(over)
    w.kv("general.architecture", G.STRING, arch)
    for k, v in vals.items():
        w.kv(f"{arch}.{k}", G.UINT32, v)
    w.kv(f"{arch}.attention.layer_norm_rms_epsilon", G.FLOAT32, 1e-6)
    w.kv(f"{arch}.rope.freq_base", G.FLOAT32, 1e6)
    w.kv(f"{arch}.final_logit_softcapping", G.FLOAT32, 30.0)
    return w


@pytest.mark.parametrize("arch,unit", [("gemma", True), ("gemma2", True), ("gemma4", False), ("gemma_4", False),
                                       ("gemma3", False), ("qwen2.5", False)])
def test_params_gemma_family(arch, unit):
    w = gemma_kvs(arch, G.GGUFWriter())
    w.tensor("token_embd.weight", G.GGML_Q4_0, (2560, 64), np.zeros(64 * 80 * 18, np.uint8))
    with G.GGUFFile.from_buffer(w.tobytes()) as f:
        p = f.params
        assert p.use_gemma_rms_unit_offset == unit
        assert p.arch == {"gemma_4": "gemma4", "gemma3": "unknown", "qwen2.5": "qwen2"}.get(arch, arch)
        assert (p.embedding_length, p.feed_forward_length, p.block_count, p.head_count, p.head_count_kv) == \
            (2560, 10240, 34, 8, 4)
        assert (p.head_size, p.rope_dim_count, p.sliding_window, p.vocab_size, p.context_length) == \
            (256, 256, 1024, 64, 8192)
        assert p.layer_norm_rms_epsilon == np.float32(1e-6) and p.rope_freq_base == 1e6
        assert p.final_logit_softcapping == 30.0 and p.attn_logit_softcapping == 0.0  # GGUF never sets it
        assert f.getTensor("token_embd.weight").row_bytes() == 2560 // 32 * 18


def test_params_defaults_and_fallbacks():
    w = G.GGUFWriter()
    w.kv("general.architecture", G.STRING, "llama").kv("llama.attention.head_count", G.ARRAY, (G.UINT32, [16, 8]))
    w.kv("llama.embedding_length", G.UINT64, 1024)
    with G.GGUFFile.from_buffer(w.tobytes()) as f:
        p = f.params
        assert p.head_count == 16 and p.head_count_kv == 16         # kv falls back to head_count
        assert p.head_size == 64 and p.rope_dim_count == 64 and p.vocab_size == 32000
        assert (p.block_count, p.context_length, p.feed_forward_length) == (32, 2048, 11008)
    # a key longer than the reference's 128-byte buffer is never found
    arch = "a" * 114  # "{arch}.block_count" is 126 bytes, "{arch}.context_length" 129
    w = G.GGUFWriter().kv("general.architecture", G.STRING, arch).kv(f"{arch}.block_count", G.UINT32, 3)
    w.kv(f"{arch}.context_length", G.UINT32, 99)
    with G.GGUFFile.from_buffer(w.tobytes()) as f:
        assert f.params.block_count == 3 and f.params.context_length == 2048 and f.params.arch == "unknown"
    # head_count 0: head_size stays 0
    w = G.GGUFWriter().kv("general.architecture", G.STRING, "llama").kv("llama.attention.head_count", G.UINT32, 0)
    with G.GGUFFile.from_buffer(w.tobytes()) as f:
        assert f.params.head_count == 0 and f.params.head_size == 0 and f.params.head_count_kv == 0


# ---------------------------------------------------------------------------------------
# Differential: native reader vs the Python restatement
# ---------------------------------------------------------------------------------------

def native_view(data):
    """The native reader's result in the restatement's shape, or its error name."""
    try:
        f = G.GGUFFile.from_buffer(data)
    except G.GGUFError as e:
        return e.name
    with f:
        md = []
        for i in range(f.metadata_count):
            kv = G.KV()
            G.lib().zl_gguf_metadata(f.handle, i, kv)
            key = G.ctypes.string_at(kv.key, kv.key_len) if kv.key_len else b""
            raw = G.ctypes.string_at(kv.data, kv.data_bytes) if kv.data_bytes else b""
            if kv.type == G.STRING:
                raw = struct.pack("<Q", len(raw)) + raw
            elif kv.type == G.ARRAY:
                raw = struct.pack("<IQ", kv.array_type, kv.array_len) + raw
            md.append((key, kv.type, raw))
        ts = [(t.name.encode(errors="surrogateescape"), t.type, t.n_dims, t.shape, t.offset, t.size_bytes)
              for t in f.tensors()]
        p = dict(vars(f.params))
        return {"version": f.version, "tensor_count": f.tensor_count, "metadata_count": f.metadata_count,
                "alignment": f.alignment, "data_offset": f.data_offset, "metadata": md, "tensors": ts, "params": p}


def ref_view(data):
    try:
        r = R.parse(data)
    except R.RefError as e:
        return str(e)
    return r


def compare(data, what):
    a, b = native_view(data), ref_view(data)
    if isinstance(a, str) or isinstance(b, str):
        assert a == b, f"{what}: native {a!r} vs reference {b if isinstance(b, str) else 'ok'}"
        return a
    for k in ("version", "tensor_count", "metadata_count", "alignment", "data_offset", "metadata", "tensors"):
        assert a[k] == b[k], f"{what}: {k}"
    for k, v in b["params"].items():
        assert a["params"][k] == v, f"{what}: params.{k}"
    return "ok"


def random_gguf(rng):
    w = G.GGUFWriter(version=int(rng.choice([2, 3])), pad_tensors=bool(rng.integers(2)))
    arch = str(rng.choice(["gemma4", "gemma2", "llama", "qwen2"]))
    w.kv("general.architecture", G.STRING, arch)
    scalars = [(G.UINT8, 200), (G.INT8, -5), (G.UINT16, 60000), (G.INT16, -7), (G.UINT32, 123456), (G.INT32, -9),
               (G.FLOAT32, 1.25), (G.BOOL, 1), (G.UINT64, 1 << 50), (G.INT64, -(1 << 40)), (G.FLOAT64, 2.5)]
    for i in range(int(rng.integers(0, 8))):
        t, v = scalars[int(rng.integers(len(scalars)))]
        w.kv(f"k{i}", t, v)
    for k in ("block_count", "embedding_length", "attention.head_count", "attention.head_count_kv"):
        if rng.random() < 0.7:
            w.kv(f"{arch}.{k}", int(rng.choice([G.UINT32, G.UINT64, G.INT32])), int(rng.integers(1, 64)))
    if rng.random() < 0.5:
        w.kv(f"{arch}.rope.freq_base", int(rng.choice([G.FLOAT32, G.FLOAT64])), 10000.0)
    if rng.random() < 0.5:
        w.kv("tok", G.ARRAY, (G.STRING, [f"t{j}" for j in range(int(rng.integers(0, 5)))]))
    if rng.random() < 0.3:
        w.kv("nest", G.ARRAY, (G.ARRAY, [(G.UINT16, [1, 2]), (G.STRING, ["x"])]))
    if rng.random() < 0.3:
        w.kv("general.alignment", G.UINT32, int(rng.choice([8, 16, 64])))
        w.alignment = [v for k, t, v in w.kvs if k == "general.alignment"][-1]
    for j in range(int(rng.integers(0, 5))):
        gt = int(rng.choice([G.GGML_F32, G.GGML_F16, G.GGML_Q4_0, G.GGML_Q8_0, G.GGML_BF16]))
        cols = 32 * int(rng.integers(1, 4))
        rows = int(rng.integers(1, 4))
        nbytes = cols * rows // G.block_size(gt) * G.type_size(gt)
        name = "token_embd.weight" if j == 0 and rng.random() < 0.5 else f"t{j}"
        w.tensor(name, gt, (cols, rows) if rng.random() < 0.8 else (cols * rows,),
                 rng.integers(0, 256, nbytes, dtype=np.uint8))
    return w.tobytes()


def test_differential_random_files():
    rng = np.random.default_rng(1234)
    for i in range(150):
        data = random_gguf(rng)
        assert compare(data, f"file {i}") == "ok"


def test_differential_truncations():
    """Every prefix of a few files: both readers fail (or succeed) the same way."""
    rng = np.random.default_rng(99)
    outcomes = set()
    for i in range(4):
        data = random_gguf(rng)
        for n in range(len(data) + 1):
            outcomes.add(compare(data[:n], f"file {i} prefix {n}"))
    assert {"UnexpectedEOF", "ok"} <= outcomes


def test_differential_mutations():
    """Random byte flips: same verdicts and parsed fields (exercises magic, version, counts,
    lengths, types and offsets)."""
    rng = np.random.default_rng(7)
    outcomes = {}
    for i in range(60):
        base = bytearray(random_gguf(rng))
        for j in range(25):
            data = bytearray(base)
            for _ in range(int(rng.integers(1, 4))):
                pos = int(rng.integers(0, min(len(data), 400)))
                data[pos] = int(rng.integers(0, 256))
            r = compare(bytes(data), f"file {i} mutation {j}")
            outcomes[r] = outcomes.get(r, 0) + 1
    assert outcomes.get("ok", 0) > 100 and len(outcomes) >= 4, outcomes
