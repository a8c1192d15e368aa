"""GGUF files to device tables (include/zl_gguf.h uploader, ziglm_amd/model.py loader)
and the decode step on a loaded model, on the GPU.

  * upload: every tensor's bytes arrive bit for bit, across the pinned ring's slot
    boundaries; too-small destinations and bad indices are refused before any copy;
  * loader: the resolved per-layer configuration equals the oracle's independent
    restatement of model.zig:156-300 / 600-616 (oracle/model_ref.py); norm vectors equal
    the oracle's dequantization bit for bit (F16 / BF16 norms go through the device
    gather); matrices equal the file's bytes;
  * decode: a gemma4 file with per-layer embeddings, KV sharing, head_dim 512 layers,
    8 query heads per KV head, layer scalars and mixed tensor types, and a gemma2 file,
    decoded step by step (eager and graph) against the oracle's forward pass
    (RefModel.forward, itself checked against float64 in test_model_ref_cpu.py);
    also at position 700 over prefilled caches (sliding window 512 vs global layers).
Logits tolerance 2e-4 * (|logit| + std(logits)): each op differs from the CPU's only in
summation order (a few f32 ulps relative), compounded over ~20 layers; the greedy token
must agree wherever the top-2 gap exceeds twice that.
"""

import numpy as np
import pytest

from oracle import model_ref as MR
from ziglm_amd import bridge as B
from ziglm_amd import gguf as G
from ziglm_amd import synth
from ziglm_amd import synth_gguf as S
from ziglm_amd.decode import DecodeModel
from ziglm_amd.model import Model

pytestmark = pytest.mark.gpu

GEMMA4 = S.GgufModelConfig(arch="gemma4", dim=256, n_layers=20, n_heads=8, n_kv_heads=1, head_dim=64,
                           global_head_dim=512, global_every=5, inter=512, vocab=1024,
                           types={"q": B.Q8_0, "o": B.BF16, "down": B.F16, "ple_out": B.F32, "v": B.Q8_0},
                           norm_type=B.F16, no_kv_from=18, scalars={3: (B.BF16, 0.75), 7: (B.F32, 1.5)},
                           tile_rows=0)
GEMMA2 = S.GgufModelConfig(arch="gemma2", dim=256, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=128,
                           global_every=0, inter=512, vocab=1024, ple=False, norm_type=B.BF16, tile_rows=0,
                           types={"up": B.BF16})
# a Q4_K_M-like mix: K-quant projections, Q6_K embedding / LM head and down projection
GEMMA2K = S.GgufModelConfig(arch="gemma2", dim=512, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=128,
                            global_every=0, inter=1024, vocab=1024, ple=False, tile_rows=0, weight_type=B.Q4_K,
                            types={"emb": B.Q6_K, "down": B.Q6_K, "v": B.Q6_K})


def gguf_bytes(cfg, seed=9):
    return S.build(cfg, seed=seed).tobytes()


# ---------------------------------------------------------------------------------------
# Upload
# ---------------------------------------------------------------------------------------

def test_upload_tensors_bit_exact(dev, tmp_path):
    rng = np.random.default_rng(3)
    sizes = [4, 100, (16 << 20) + 36, 3 << 20, 40_000_004, 8]   # spans the 16 MiB slots
    w = G.GGUFWriter()
    arrays = []
    for i, n in enumerate(sizes):
        a = rng.integers(0, 256, n, dtype=np.uint8)
        arrays.append(a)
        w.tensor(f"t{i}", G.GGML_F32, (n // 4,), a)
    path = w.write(tmp_path / "u.gguf")
    with G.GGUFFile.open(path) as f:
        ts = f.tensors()
        bufs = [dev.alloc(t.size_bytes + 64) for t in ts]
        for b in bufs:
            b.fill(0x5A)
        f.upload(ts, bufs, dev.stream)
        for t, b, a in zip(ts, bufs, arrays):
            got = b.to_numpy((t.size_bytes + 64,), np.uint8)
            assert np.array_equal(got[:t.size_bytes], a), t.name
            assert np.all(got[t.size_bytes:] == 0x5A), t.name  # nothing past the tensor
        # one tensor at a time, reversed order
        for t, b in zip(reversed(ts), reversed(bufs)):
            b.fill(0)
            assert G.lib().zl_gguf_upload(f.handle, t.index, b.ptr, b.size_bytes, dev.stream) == 0
            assert np.array_equal(b.to_numpy((t.size_bytes,), np.uint8), arrays[t.index])


def test_upload_errors(dev):
    w = G.GGUFWriter().tensor("t", G.GGML_F32, (16,), np.arange(16, dtype=np.float32))
    with G.GGUFFile.from_buffer(w.tobytes()) as f:
        small = dev.alloc(32)
        small.fill(0x11)
        L = G.lib()
        assert L.zl_gguf_upload(f.handle, 0, small.ptr, 32, dev.stream) == -21      # DestinationTooSmall
        assert L.zl_gguf_upload(f.handle, 1, small.ptr, 64, dev.stream) == -20      # bad index
        assert L.zl_gguf_upload(f.handle, 0, None, 64, dev.stream) == -20           # NULL destination
        assert np.all(small.to_numpy((32,), np.uint8) == 0x11)


def test_upload_host_ring(dev):
    a = np.random.default_rng(4).integers(0, 256, 70_000_001, dtype=np.uint8)
    b = dev.alloc(a.nbytes)
    assert G.lib().zl_upload_host(b.ptr, a.ctypes.data, a.nbytes, dev.stream) == 0
    assert np.array_equal(b.to_numpy((a.nbytes,), np.uint8), a)


# ---------------------------------------------------------------------------------------
# Loader
# ---------------------------------------------------------------------------------------

def test_loader_matches_oracle_restatement(dev, oracle):
    data = gguf_bytes(GEMMA4)
    ref = MR.RefModel(oracle, data, max_seq=8)
    with G.GGUFFile.from_buffer(data) as f:
        m = Model.from_gguf(dev, f)
        try:
            assert m.arch == "gemma4" and not m.unit_offset and m.final_softcap == 30.0
            assert m.embed_scale == np.sqrt(np.float32(256)) and m.lm_head is m.token_embd
            for ly, r in zip(m.layers, ref.layers):
                assert (ly.head_dim, ly.n_heads, ly.n_kv_heads, ly.intermediate_size) == \
                    (r["head_dim"], r["n_heads"], r["n_kv"], r["inter"])
                assert (ly.rope_theta, ly.rotary_dim, ly.sliding_window) == (r["theta"], r["rotary"], r["window"])
                assert (ly.kv_shared, ly.kv_layer, ly.layer_scalar) == (r["shared"], r["donor"], r["scalar"])
                assert ly.attn_scale == 1.0 and ly.v_norm
                for name, key in [("input_layernorm", "in"), ("post_attention_layernorm", "post_attn"),
                                  ("pre_feedforward_layernorm", "pre_ffn"),
                                  ("post_feedforward_layernorm", "post_ffn"),
                                  ("post_per_layer_input_norm", "post_ple"), ("attn_q_norm", "q_norm")]:
                    want = r[key]
                    got = getattr(ly, name).to_numpy(want.shape, np.float32)
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (ly.index, name)
                for name, key in [("attn_q", "q"), ("attn_output", "o"), ("ffn_gate", "gate"), ("ffn_up", "up"),
                                  ("ffn_down", "down"), ("per_layer_input_gate", "ple_gate"),
                                  ("per_layer_projection", "ple_proj")]:
                    t = getattr(ly, name)
                    qtype, raw = r[key]
                    assert t.qtype == qtype and t.rows == raw.shape[0], (ly.index, name)
                    assert np.array_equal(t.buf.to_numpy((raw.size,), np.uint8), raw.reshape(-1)), (ly.index, name)
                if r["shared"]:
                    assert ly.attn_k is None and ly.attn_v is None
            on = m.output_norm.to_numpy((m.dim,), np.float32)
            assert np.array_equal(on.view(np.uint32), ref.output_norm.view(np.uint32))
            pn = m.ple_proj_norm.to_numpy((256,), np.float32)
            assert np.array_equal(pn.view(np.uint32), ref.ple_norm.view(np.uint32))
        finally:
            m.free()


def test_loader_rejects_bad_tables(dev):
    cfg = S.GgufModelConfig(arch="gemma4", dim=256, n_layers=2, n_heads=2, n_kv_heads=1, head_dim=64,
                            global_every=0, inter=512, vocab=64, ple=False, tile_rows=0)
    w = S.build(cfg)
    # blk.1.ffn_down with one row too few
    w.infos = [(n, t, (s[0], s[1] - 1) if n == "blk.1.ffn_down.weight" else s,
                d[:-(512 // 32 * 18)] if n == "blk.1.ffn_down.weight" else d) for n, t, s, d in w.infos]
    with G.GGUFFile.from_buffer(w.tobytes()) as f:
        with pytest.raises(Exception, match="ffn_down"):
            Model.from_gguf(dev, f)
    # a matrix type the GEMV kernels do not take (Q5_K)
    w = S.build(cfg)
    w.infos = [(n, 13 if n == "blk.0.attn_q.weight" else t, s, d) for n, t, s, d in w.infos]
    with G.GGUFFile.from_buffer(w.tobytes()) as f:
        with pytest.raises(Exception, match="attn_q"):
            Model.from_gguf(dev, f)


# ---------------------------------------------------------------------------------------
# Decode on a loaded model
# ---------------------------------------------------------------------------------------

def check_logits(got, ref, what):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    tol = 2e-4 * (np.abs(ref) + ref.std())
    err = np.abs(got - ref)
    assert np.all(err <= tol), f"{what}: max err/tol {float(np.max(err / tol)):.3g}"
    return tol


def check_token(gtok, ref, tol, what):
    top = np.sort(ref[1:])[-2:]
    if top[1] - top[0] > 2 * tol.max():
        assert gtok == int(np.argmax(ref[1:])) + 1, what


FUSE_SETS = [True, set(), {"qkv", "ffn", "ple", "head"}, {"attn", "ple"}]
FUSE_IDS = ["default", "unfused", "prologues", "qk_attention"]


@pytest.mark.parametrize("fused", FUSE_SETS, ids=FUSE_IDS)
@pytest.mark.parametrize("cfg", [GEMMA4, GEMMA2, GEMMA2K], ids=["gemma4", "gemma2", "gemma2_kquants"])
def test_decode_loaded_model_vs_oracle(dev, oracle, cfg, fused):
    data = gguf_bytes(cfg)
    ref = MR.RefModel(oracle, data, max_seq=32)
    with G.GGUFFile.from_buffer(data) as f:
        dm = DecodeModel(dev, Model.from_gguf(dev, f), max_seq=32, own_model=True, fused=fused)
    try:
        dm.reset(0)
        for pos, tok in enumerate([3, 17, 101, 250, 77, 1000]):
            dm.set_token(tok)
            dm.step(pos, graph=False)
            got = dm.logits.to_numpy((dm.V,), np.float32)
            want = ref.forward(tok, pos)
            tol = check_logits(got, want, f"{cfg.arch} pos {pos}")
            check_token(dm.read_token(), want.astype(np.float64), tol, f"{cfg.arch} pos {pos}")
    finally:
        dm.free()


def test_decode_e2b_full_shape_vs_oracle(dev, oracle, tmp_path):
    """The gemma-4-E2B-shaped model the benchmark decodes (35 layers, 1536 hidden, 8/1 heads
    x 256 with a 512 window | 512 with rotary 128, FFN 6144, per-layer embeddings, 15
    unshared KV layers, tied 262144-row LM head; Q4_0; the default fuse set, so the fused QK
    attention and the prologue GEMVs run at their real shapes): three decode steps against
    the oracle's forward pass over the same file."""
    path = str(tmp_path / "e2b.gguf")
    S.build(S.E2B, seed=11).write(path)  # streamed: 2.3 GB
    with open(path, "rb") as fh:
        data = fh.read()
    ref = MR.RefModel(oracle, data, max_seq=16)
    with G.GGUFFile.open(path) as f:
        dm = DecodeModel(dev, Model.from_gguf(dev, f), max_seq=16, own_model=True)
    try:
        dm.reset(0)
        for pos, tok in enumerate([2, 1234, 99999]):
            dm.set_token(tok)
            dm.step(pos, graph=False)
            got = dm.logits.to_numpy((dm.V,), np.float32)
            want = ref.forward(tok, pos)
            tol = check_logits(got, want, f"e2b pos {pos}")
            check_token(dm.read_token(), want.astype(np.float64), tol, f"e2b pos {pos}")
    finally:
        dm.free()


@pytest.mark.parametrize("fused", FUSE_SETS, ids=FUSE_IDS)
def test_decode_loaded_graph_equals_eager(dev, fused):
    data = gguf_bytes(GEMMA4)
    with G.GGUFFile.from_buffer(data) as f:
        dm = DecodeModel(dev, Model.from_gguf(dev, f), max_seq=32, own_model=True, fused=fused)
    try:
        dm.reset(5)
        eager = []
        for p in range(4):
            dm.step(p, graph=False)
            eager.append((dm.logits.to_numpy((dm.V,), np.float32).copy(), dm.read_token()))
        dm.reset(5)
        dm.capture()
        for p in range(4):
            dm.step(p, graph=True)
            dev.sync()
            np.testing.assert_array_equal(dm.logits.to_numpy((dm.V,), np.float32), eager[p][0], err_msg=f"pos {p}")
            assert dm.read_token() == eager[p][1]
        dm.reset(5)
        dm.run(0, 4)
        np.testing.assert_array_equal(dm.logits.to_numpy((dm.V,), np.float32), eager[3][0])
    finally:
        dm.free()


def test_decode_loaded_long_context(dev, oracle):
    """Position 700 over caches prefilled with the same random rows on both sides: the
    local layers see the last 512 positions, the head_dim-512 layers all 701, the
    KV-shared layers their donors' rows."""
    data = gguf_bytes(GEMMA4, seed=21)
    max_seq, pos = 1024, 700
    ref = MR.RefModel(oracle, data, max_seq=max_seq)
    with G.GGUFFile.from_buffer(data) as f:
        dm = DecodeModel(dev, Model.from_gguf(dev, f), max_seq=max_seq, own_model=True)
    try:
        L, kvd = dm.L, dm.kv_dim
        kc = np.zeros((L * max_seq, kvd), np.float32)
        vc = np.zeros_like(kc)
        for l, ly in enumerate(dm.model.layers):
            if ly.kv_shared:
                continue
            n = ly.n_kv_heads * ly.head_dim
            kc[l * max_seq:l * max_seq + pos, :n] = synth.normal_f32(31, f"k{l}", (pos, n))
            vc[l * max_seq:l * max_seq + pos, :n] = synth.normal_f32(31, f"v{l}", (pos, n))
        ref.kc[:] = kc
        ref.vc[:] = vc
        dm.kc.upload(kc)
        dm.vc.upload(vc)
        for step, tok in enumerate([42, 900]):
            dm.set_token(tok)
            dm.step(pos + step, graph=False)
            got = dm.logits.to_numpy((dm.V,), np.float32)
            want = ref.forward(tok, pos + step)
            check_logits(got, want, f"pos {pos + step}")
    finally:
        dm.free()
