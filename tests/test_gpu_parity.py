"""GPU parity: every hip_bridge entry point against the CPU oracle on seeded inputs.

All calls go through the C-ABI (ziglm_amd.device.HipDevice -> libhip_bridge.so).
Tolerances:
  gathers, KV copies, residual add/scale ....... bit-exact
  f32 norm / RoPE / GeGLU / soft-cap ............ 1e-5 relative; RoPE outputs relative to
      the norm of their rotation pair (a rotated coordinate can cancel to ~0); GeGLU adds
      the reference's own cancellation bound in 1 + tanh(z): |x*up| * 2^-23
  bf16 outputs .................................. 1 bf16 ulp, with the same floors
"""
import numpy as np
import pytest

from oracle import oracle as O
from tol import assert_bf16, assert_bitexact, assert_rel
from ziglm_amd import bridge as B
from ziglm_amd import synth

pytestmark = pytest.mark.gpu

SQRT = {2560: np.float32(np.sqrt(np.float32(2560))), 5376: np.float32(np.sqrt(np.float32(5376)))}


def f16_table(seed, rows, cols):
    return synth.f16_bits(synth.normal_f32(seed, "f16tab", (rows, cols), 0, 0.5)).view(np.uint8).reshape(rows, cols * 2)


def f32_table(seed, rows, cols):
    return synth.normal_f32(seed, "f32tab", (rows, cols)).view(np.uint8).reshape(rows, cols * 4)


def q6k_table(seed, rows, cols):
    return synth.q6_k_table(seed, rows, cols)


def make_table(qtype, seed, rows, cols):
    return {
        B.Q8_0: synth.q8_0_table, B.Q4_0: synth.q4_0_table, B.BF16: synth.bf16_table,
        B.F16: f16_table, B.F32: f32_table, B.Q6_K: q6k_table, B.Q4_K: synth.q4_k_table,
    }[qtype](seed, rows, cols)


# ---------------------------------------------------------------------------------------
# Embedding gather
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("out_dtype", [B.F32, B.BF16])
@pytest.mark.parametrize("qtype,dim", [(B.Q8_0, 2560), (B.Q4_0, 2560), (B.BF16, 2560), (B.F16, 2560),
                                       (B.F32, 2560), (B.Q6_K, 2560), (B.Q8_0, 96), (B.Q4_0, 160),
                                       (B.BF16, 2562), (B.F32, 100),
                                       # partial last segment / byte-staged rows
                                       (B.Q8_0, 5376), (B.Q4_0, 5376), (B.Q6_K, 5376),
                                       (B.BF16, 5376), (B.Q8_0, 800), (B.F16, 1000),
                                       (B.Q4_K, 2560), (B.Q4_K, 5376), (B.Q4_K, 256)])
def test_embed_gather_bitexact(dev, oracle, qtype, dim, out_dtype):
    vocab = 700
    table = make_table(qtype, 2, vocab, dim)
    ids = synth.gather_ids(2, 320, vocab, n_repeat=20)
    bad = np.array([-1, vocab, vocab + 77, -5], np.int32)
    all_ids = np.concatenate([ids, bad])
    scale = np.float32(np.sqrt(np.float32(dim)))
    ref = oracle.embed_gather(table, qtype, ids, dim, scale)
    ref = np.concatenate([ref, np.zeros((bad.size, dim), np.float32)])
    d_tab, d_ids = dev.from_numpy(table), dev.from_numpy(all_ids)
    es = 4 if out_dtype == B.F32 else 2
    d_out = dev.alloc(all_ids.size * dim * es)
    d_out.fill(0xAB)
    dev.embedGather(d_tab, qtype, vocab, d_ids, out_dtype, d_out, all_ids.size, dim, scale)
    if out_dtype == B.F32:
        got = d_out.to_numpy((all_ids.size, dim), np.float32)
        assert_bitexact(got, ref, f"gather qtype={qtype} dim={dim}")
    else:
        got = d_out.to_numpy((all_ids.size, dim), np.uint16)
        assert_bitexact(got, oracle.f32_to_bf16(ref), f"gather bf16-out qtype={qtype} dim={dim}")


@pytest.mark.parametrize("out_dtype", [B.F32, B.BF16])
@pytest.mark.parametrize("qtype", [B.Q8_0, B.Q4_0])
@pytest.mark.parametrize("dim", [5376, 2560])
def test_embed_gather_many_segments_bitexact(dev, oracle, qtype, dim, out_dtype):
    """Prefill-sized gathers (4100 ids; a row of 5376 is 11 segments of f32 output, the last
    partial, or 6 of bf16; one of 2560 is 5 or 3) over several rounds of waves, out-of-range
    ids among them giving zero rows. Bit-exact against the oracle."""
    vocab = 700
    table = make_table(qtype, 4, vocab, dim)
    ids = synth.gather_ids(4, 4096, vocab, n_repeat=64)
    bad = np.array([-1, vocab, vocab + 77, -5], np.int32)
    all_ids = np.concatenate([ids[:1000], bad, ids[1000:]])
    ok = (all_ids >= 0) & (all_ids < vocab)
    scale = np.float32(np.sqrt(np.float32(dim)))
    ref = np.zeros((all_ids.size, dim), np.float32)
    ref[ok] = oracle.embed_gather(table, qtype, all_ids[ok], dim, scale)
    d_tab, d_ids = dev.from_numpy(table), dev.from_numpy(all_ids)
    es = 4 if out_dtype == B.F32 else 2
    d_out = dev.alloc(all_ids.size * dim * es)
    d_out.fill(0xAB)
    dev.embedGather(d_tab, qtype, vocab, d_ids, out_dtype, d_out, all_ids.size, dim, scale)
    if out_dtype == B.F32:
        assert_bitexact(d_out.to_numpy((all_ids.size, dim), np.float32), ref, f"gather qtype={qtype}")
    else:
        assert_bitexact(d_out.to_numpy((all_ids.size, dim), np.uint16), oracle.f32_to_bf16(ref),
                        f"gather bf16-out qtype={qtype}")


@pytest.mark.parametrize("qtype,offset", [(B.Q8_0, 1), (B.Q4_0, 1), (B.Q8_0, 2), (B.Q4_0, 6),
                                          (B.BF16, 2), (B.F16, 6), (B.F32, 4), (B.Q6_K, 8), (B.Q4_K, 1)])
@pytest.mark.parametrize("out_dtype", [B.F32, B.BF16])
def test_embed_gather_misaligned_table(dev, oracle, qtype, offset, out_dtype):
    """Tables at an odd or non-16-byte address take the byte-staged / scalar paths."""
    vocab, dim = 90, 2560
    table = make_table(qtype, 3, vocab, dim)
    ids = synth.gather_ids(3, 64, vocab, n_repeat=8)
    scale = SQRT[dim]
    ref = oracle.embed_gather(table, qtype, ids, dim, scale)
    d_raw = dev.alloc(table.nbytes + 16)
    d_tab = d_raw.at(offset)
    d_tab.upload(table.reshape(-1))
    es = 4 if out_dtype == B.F32 else 2
    d_out = dev.alloc(ids.size * dim * es)
    dev.embedGather(d_tab, qtype, vocab, dev.from_numpy(ids), out_dtype, d_out, ids.size, dim, scale)
    if out_dtype == B.F32:
        assert_bitexact(d_out.to_numpy((ids.size, dim), np.float32), ref, f"qtype={qtype} +{offset}")
    else:
        assert_bitexact(d_out.to_numpy((ids.size, dim), np.uint16), oracle.f32_to_bf16(ref),
                        f"bf16-out qtype={qtype} +{offset}")


@pytest.mark.parametrize("qtype", [B.Q8_0, B.Q4_0, B.BF16, B.Q6_K, B.Q4_K])
def test_embed_lookup_mirrors(dev, oracle, qtype):
    vocab, dim = 300, 2560
    table = make_table(qtype, 5, vocab, dim)
    scale = SQRT[dim]
    ids = np.array([0, 299, 7, 7, 150], np.int32)
    ref = oracle.embed_gather(table, qtype, ids, dim, scale)
    d_tab = dev.from_numpy(table)
    d_out = dev.alloc(ids.size * dim * 4)
    dev.embedLookupBatch(d_tab, qtype, dev.from_numpy(ids), d_out, ids.size, dim, scale)
    assert_bitexact(d_out.to_numpy((ids.size, dim), np.float32), ref, "embedLookupBatch")
    d_one = dev.alloc(dim * 4)
    dev.embedLookup(d_tab, qtype, 299, d_one, dim, scale)
    assert_bitexact(d_one.to_numpy((dim,), np.float32), ref[1], "embedLookup")


def test_gather_unsupported_qtype_is_noop(dev):
    d_tab = dev.alloc(1024)
    d_ids = dev.from_numpy(np.zeros(1, np.int32))
    d_out = dev.alloc(256 * 4)
    d_out.fill(0x11)
    dev.strict = False
    try:
        dev.embedLookupBatch(d_tab, 13, d_ids, d_out, 1, 256, 1.0)  # Q5_K: not supported
        assert dev.b.last_error() == B.EUNSUPPORTED
    finally:
        dev.strict = True
    assert np.all(d_out.to_numpy((1024,), np.uint8) == 0x11)


# ---------------------------------------------------------------------------------------
# RMSNorm family
# ---------------------------------------------------------------------------------------

EPS = np.float32(1e-6)


@pytest.mark.parametrize("n", [2560, 5376, 256, 2561, 16384])
@pytest.mark.parametrize("uo", [True, False])
def test_rmsnorm_f32(dev, oracle, n, uo):
    x = synth.normal_f32(0, "x", (n,))
    w = synth.normal_f32(0, "w", (n,), 0, 0.1)
    ref = oracle.rms_norm(x, w, EPS, uo)
    d_x, d_w, d_o = dev.from_numpy(x), dev.from_numpy(w), dev.alloc(n * 4)
    dev.rmsNorm(d_x, d_w, d_o, n, EPS, uo)
    assert_rel(d_o.to_numpy((n,), np.float32), ref, 1e-5, what=f"rmsNorm n={n}")
    dev.rmsNorm(d_x, None, d_o, n, EPS, uo)  # no weight: rmsNormNoScale
    assert_rel(d_o.to_numpy((n,), np.float32), oracle.rms_norm(x, None, EPS), 1e-5, what="rmsNorm w=NULL")


def test_rmsnorm_batched_inplace(dev, oracle):
    q = synth.normal_f32(0, "q", (8, 256))
    wq = synth.normal_f32(0, "wq", (256,), 0, 0.1)
    d_q, d_w = dev.from_numpy(q), dev.from_numpy(wq)
    dev.rmsNormBatched(d_q, d_w, d_q, 256, 8, EPS, True)
    assert_rel(d_q.to_numpy((8, 256), np.float32), oracle.rms_norm(q, wq, EPS, True), 1e-5)


@pytest.mark.parametrize("batch", [1, 64])
def test_add_rmsnorm_out_aliases_residual(dev, oracle, batch):
    n = 2560
    x = synth.normal_f32(1, "x", (batch, n))
    r = synth.normal_f32(1, "r", (batch, n))
    w = synth.normal_f32(1, "w", (n,), 0, 0.1)
    x_ref, out_ref = oracle.add_rms_norm(x, r, w, EPS, True)
    d_x, d_r, d_w = dev.from_numpy(x), dev.from_numpy(r), dev.from_numpy(w)
    if batch == 1:
        dev.addRmsNorm(d_x, d_r, d_w, d_r, n, EPS, True)  # out = residual, as cuda_model.zig:935
    else:
        dev.addRmsNormBatched(d_x, d_r, d_w, d_r, n, batch, EPS, True)
    assert_bitexact(d_x.to_numpy((batch, n), np.float32), x_ref, "x += r")
    assert_rel(d_r.to_numpy((batch, n), np.float32), out_ref, 1e-5, what="norm(x+r)")


def test_rmsnorm_add(dev, oracle):
    n = 2560
    x = synth.normal_f32(2, "x", (n,))
    inp = synth.normal_f32(2, "in", (n,))
    w = synth.normal_f32(2, "w", (n,), 0, 0.1)
    ref = oracle.rms_norm_add(x, inp, w, EPS, True)
    d_x = dev.from_numpy(x)
    dev.rmsnormAdd(d_x, dev.from_numpy(inp), dev.from_numpy(w), n, EPS, True)
    # x + norm(in): relative to the larger of the two summands (the sum can cancel)
    floor = 1e-5 * np.abs(x)
    assert_rel(d_x.to_numpy((n,), np.float32), ref, 1e-5, floor=floor, what="rmsnormAdd")


@pytest.mark.parametrize("n,rows", [(2560, 64), (5376, 16), (2568, 8), (12000, 4)])
def test_bf16_rows(dev, oracle, n, rows):
    x = synth.normal_bf16(3, "x", (rows, n))
    r = synth.normal_bf16(3, "r", (rows, n))
    w = synth.normal_f32(3, "w", (n,), 0, 0.1)
    x_ref, out_ref = oracle.add_rms_norm_bf16(x, r, w, EPS, True)
    d_x, d_r, d_w, d_o = dev.from_numpy(x), dev.from_numpy(r), dev.from_numpy(w), dev.alloc(x.nbytes)
    dev.addRmsNormRows(B.BF16, d_x, d_r, d_w, d_o, rows, n, EPS, True)
    assert_bitexact(d_x.to_numpy(x.shape, np.uint16), x_ref, "bf16 x+r")
    assert_bf16(d_o.to_numpy(x.shape, np.uint16), out_ref, 1, what="bf16 add+norm")
    # plain norm rows
    d_o2 = dev.alloc(x.nbytes)
    dev.rmsNormRows(B.BF16, dev.from_numpy(x), d_w, d_o2, rows, n, EPS, True)
    assert_bf16(d_o2.to_numpy(x.shape, np.uint16), oracle.rms_norm_bf16(x, w, EPS, True), 1, what="bf16 norm")


@pytest.mark.parametrize("dtype,n,rows", [(B.F32, 2560, 8), (B.BF16, 2560, 64), (B.BF16, 5376, 8),
                                          (B.F32, 2561, 3)])
def test_rmsnorm_add_rmsnorm(dev, oracle, dtype, n, rows):
    if dtype == B.F32:
        x = synth.normal_f32(4, "x", (rows, n))
        xb = synth.normal_f32(4, "xb", (rows, n))
    else:
        x = synth.normal_bf16(4, "x", (rows, n))
        xb = synth.normal_bf16(4, "xb", (rows, n))
    w1 = synth.normal_f32(4, "w1", (n,), 0, 0.1)
    w2 = synth.normal_f32(4, "w2", (n,), 0, 0.1)
    x_ref, out_ref = oracle.rms_norm_add_rms_norm(x, xb, w1, w2, EPS, True)
    d_x, d_xb = dev.from_numpy(x), dev.from_numpy(xb)
    dev.rmsNormAddRmsNorm(dtype, d_x, d_xb, dev.from_numpy(w1), dev.from_numpy(w2), d_xb, rows, n, EPS, True)
    gx, go = d_x.to_numpy(x.shape, x.dtype), d_xb.to_numpy(x.shape, x.dtype)
    # s = x + a, a = norm1(xb): an ulp-level difference in a moves s by ~1e-7*|a| even where
    # the sum cancels, so s is checked relative to its summands, and norm2(s) = s*inv2*(1+w2)
    # relative to (|x| + |a|)*inv2*|1+w2|.
    f = O.get().bf16_to_f32
    xf = (x if dtype == B.F32 else f(x)).astype(np.float64)
    a = oracle.rms_norm(xb if dtype == B.F32 else f(xb), w1, EPS, True).astype(np.float64)
    s = xf + a
    inv2 = 1.0 / np.sqrt(np.mean(s * s, axis=-1, keepdims=True) + float(EPS))
    floor_x = 1e-5 * (np.abs(xf) + np.abs(a))
    floor_o = 1e-5 * (np.abs(xf) + np.abs(a)) * inv2 * np.abs(1.0 + w2.astype(np.float64))
    if dtype == B.F32:
        assert_rel(gx, x_ref, 1e-5, floor=floor_x, what="x + norm1(xb)")
        assert_rel(go, out_ref, 1e-5, floor=floor_o, what="norm2(x)")
    else:
        assert_bf16(gx, x_ref, 1, floor=floor_x, what="bf16 x + norm1(xb)")
        assert_bf16(go, out_ref, 1, floor=floor_o, what="bf16 norm2(x)")


@pytest.mark.parametrize("dtype,n,rows", [(B.F32, 2560, 64), (B.BF16, 2560, 2048), (B.BF16, 5376, 64)])
def test_rmsnorm_add_rmsnorm_cancellation(dev, oracle, dtype, n, rows):
    """post-attn norm + add + pre-FFN norm where the residual stream nearly cancels the
    normalised branch: x = -norm1(xb) + delta * noise, delta in {0, 1e-4, 1e-2, 1} by row
    (s = x + norm1(xb) is ~delta, so the second statistic is a sum of cancelled terms), with
    the same tolerances as test_rmsnorm_add_rmsnorm."""
    f = O.get().bf16_to_f32
    bf = dtype == B.BF16
    xb = synth.normal_bf16(6, "xb", (rows, n)) if bf else synth.normal_f32(6, "xb", (rows, n))
    w1 = synth.normal_f32(6, "w1", (n,), 0, 0.1)
    w2 = synth.normal_f32(6, "w2", (n,), 0, 0.1)
    a32 = oracle.rms_norm(f(xb) if bf else xb, w1, EPS, True)
    delta = np.array([0.0, 1e-4, 1e-2, 1.0], np.float32)[np.arange(rows) % 4][:, None]
    x32 = (-a32 + delta * synth.normal_f32(6, "noise", (rows, n))).astype(np.float32)
    x = O.get().f32_to_bf16(x32) if bf else x32
    x_ref, out_ref = oracle.rms_norm_add_rms_norm(x, xb, w1, w2, EPS, True)
    d_x, d_o = dev.from_numpy(x), dev.alloc(x.nbytes)
    dev.rmsNormAddRmsNorm(dtype, d_x, dev.from_numpy(xb), dev.from_numpy(w1), dev.from_numpy(w2), d_o, rows, n,
                          EPS, True)
    gx, go = d_x.to_numpy(x.shape, x.dtype), d_o.to_numpy(x.shape, x.dtype)
    xf = (f(x) if bf else x).astype(np.float64)
    a = a32.astype(np.float64)
    s = xf + a
    inv2 = 1.0 / np.sqrt(np.mean(s * s, axis=-1, keepdims=True) + float(EPS))
    floor_x = 1e-5 * (np.abs(xf) + np.abs(a))
    floor_o = 1e-5 * (np.abs(xf) + np.abs(a)) * inv2 * np.abs(1.0 + w2.astype(np.float64))
    if bf:
        assert_bf16(gx, x_ref, 1, floor=floor_x, what="bf16 x + norm1(xb), cancelling")
        assert_bf16(go, out_ref, 1, floor=floor_o, what="bf16 norm2(x), cancelling")
    else:
        assert_rel(gx, x_ref, 1e-5, floor=floor_x, what="x + norm1(xb), cancelling")
        assert_rel(go, out_ref, 1e-5, floor=floor_o, what="norm2(x), cancelling")


@pytest.mark.parametrize("dtype,n,rows", [(B.BF16, 2560, 4097), (B.BF16, 5376, 2049), (B.F32, 2560, 2049),
                                          (B.BF16, 1024, 777), (B.F32, 5376, 512), (B.BF16, 5376, 4099),
                                          (B.F32, 2560, 4101)])
def test_norm_modes_many_rows(dev, oracle, dtype, n, rows):
    """Prefill-sized row counts. rows * waves-per-row >= 8192 takes two rows per lane group
    (the odd counts leave the last group's second row out of range; 5376 x 4099 bf16 and
    2560 x 4101 f32 at four waves a row); 1024 x 777 and 5376 x 512 f32 take one row per
    group."""
    f = O.get().bf16_to_f32
    bf = dtype == B.BF16
    gen = synth.normal_bf16 if bf else synth.normal_f32
    up = (lambda a: f(a).astype(np.float64)) if bf else (lambda a: a.astype(np.float64))
    x = gen(9, "x", (rows, n))
    r = gen(9, "r", (rows, n))
    w1 = synth.normal_f32(9, "w1", (n,), 0, 0.1)
    w2 = synth.normal_f32(9, "w2", (n,), 0, 0.1)
    npdt = x.dtype

    def check(got, ref, what, floor=0.0):
        if bf:
            assert_bf16(got, ref, 1, floor=floor, what=what)
        else:
            assert_rel(got, ref, 1e-5, floor=floor, what=what)

    # NORM
    d_o = dev.alloc(x.nbytes)
    dev.rmsNormRows(dtype, dev.from_numpy(x), dev.from_numpy(w1), d_o, rows, n, EPS, True)
    ref = oracle.rms_norm_bf16(x, w1, EPS, True) if bf else oracle.rms_norm(x, w1, EPS, True)
    check(d_o.to_numpy(x.shape, npdt), ref, "norm")
    # ADD_NORM
    d_x, d_o = dev.from_numpy(x), dev.alloc(x.nbytes)
    dev.addRmsNormRows(dtype, d_x, dev.from_numpy(r), dev.from_numpy(w1), d_o, rows, n, EPS, True)
    x_ref, o_ref = (oracle.add_rms_norm_bf16 if bf else oracle.add_rms_norm)(x, r, w1, EPS, True)
    assert_bitexact(d_x.to_numpy(x.shape, npdt), x_ref, "x + r")
    check(d_o.to_numpy(x.shape, npdt), o_ref, "norm(x + r)")
    # NORM_ADD: x + norm(r), relative to its summands
    a = oracle.rms_norm(up(r).astype(np.float32), w1, EPS, True).astype(np.float64)
    floor = 1e-5 * (np.abs(up(x)) + np.abs(a))
    d_x = dev.from_numpy(x)
    dev.rmsnormAddRows(dtype, d_x, dev.from_numpy(r), dev.from_numpy(w1), rows, n, EPS, True)
    check(d_x.to_numpy(x.shape, npdt), oracle.rms_norm_add(x, r, w1, EPS, True), "x + norm(r)", floor)
    # NORM_ADD_NORM
    d_x, d_r = dev.from_numpy(x), dev.from_numpy(r)
    dev.rmsNormAddRmsNorm(dtype, d_x, d_r, dev.from_numpy(w1), dev.from_numpy(w2), d_r, rows, n, EPS, True)
    x_ref, o_ref = oracle.rms_norm_add_rms_norm(x, r, w1, w2, EPS, True)
    s_ = up(x) + a
    inv2 = 1.0 / np.sqrt(np.mean(s_ * s_, axis=-1, keepdims=True) + float(EPS))
    check(d_x.to_numpy(x.shape, npdt), x_ref, "x + norm1(r)", floor)
    check(d_r.to_numpy(x.shape, npdt), o_ref, "norm2(x + norm1(r))",
          floor * inv2 * np.abs(1.0 + w2.astype(np.float64)))


@pytest.mark.parametrize("dtype,n", [(B.BF16, 5376), (B.BF16, 4104), (B.BF16, 8192), (B.F32, 2560)])
@pytest.mark.parametrize("weighted", [True, False])
def test_norm_pipelined_rows_equal_row_kernel(dev, oracle, dtype, n, weighted):
    """Launches of 16384 or more waves at four waves a row (4099 rows here) take the
    persistent, pipelined row kernels (norm + add + norm its one-barrier-per-row form), whose
    workgroups walk several rows each (an odd count for some); the same rows in two launches
    under that size take the one-shot row kernel. Both do the same arithmetic in the same
    order, so every output is bit-equal between the two; the norm is also checked against the
    oracle. 4104 leaves part of each row's last chunk column empty, 8192 fills four chunks per
    lane; no weight takes the other factor form. add + norm writes its output over the
    residual, as the reference's decode step does."""
    rows, split = 4099, 2050
    bf = dtype == B.BF16
    gen = synth.normal_bf16 if bf else synth.normal_f32
    npdt = np.uint16 if bf else np.float32
    es = 2 if bf else 4
    x = gen(21, "x", (rows, n))
    r = gen(21, "r", (rows, n))
    w = synth.normal_f32(21, "w", (n,), 0, 0.1) if weighted else None
    uo = weighted  # weighted: (1 + w); otherwise no weight at all
    d_w = dev.from_numpy(w) if weighted else None
    d_w2 = dev.from_numpy(synth.normal_f32(21, "w2", (n,), 0, 0.1)) if weighted else None

    def both(run):
        """run(x_view, r_view, out_view, rows) over all rows at once, then in two launches."""
        outs = []
        for parts in ([(0, rows)], [(0, split), (split, rows - split)]):
            d_x, d_r, d_o = dev.from_numpy(x), dev.from_numpy(r), dev.alloc(x.nbytes)
            d_o.fill(0)  # the modes that write no separate output leave it zero in both runs
            for r0, cnt in parts:
                off = r0 * n * es
                run(d_x.at(off), d_r.at(off), d_o.at(off), cnt)
            dev.sync()
            outs.append(tuple(b.to_numpy(x.shape, npdt) for b in (d_x, d_r, d_o)))
            for b in (d_x, d_r, d_o):
                b.deinit()
        for k, what in enumerate(("x", "r", "out")):
            assert_bitexact(outs[0][k], outs[1][k], what)
        return outs[0]

    _, _, o = both(lambda dx, dr, do, cnt: dev.rmsNormRows(dtype, dx, d_w, do, cnt, n, EPS, uo))
    if bf:  # the bf16 oracle is the f32 one between exact widening and RNE narrowing
        ref = oracle.f32_to_bf16(oracle.rms_norm(O.get().bf16_to_f32(x), w, EPS, uo))
        assert_bf16(o, ref, 1, what="norm")
    else:
        assert_rel(o, oracle.rms_norm(x, w, EPS, uo), 1e-5, what="norm")
    both(lambda dx, dr, do, cnt: dev.addRmsNormRows(dtype, dx, dr, d_w, dr, cnt, n, EPS, uo))
    both(lambda dx, dr, do, cnt: dev.rmsnormAddRows(dtype, dx, dr, d_w, cnt, n, EPS, uo))
    # norm + add + norm, its output over its input r (the reference's fused call does that)
    both(lambda dx, dr, do, cnt: dev.rmsNormAddRmsNorm(dtype, dx, dr, d_w, d_w2, dr, cnt, n, EPS, uo))
    both(lambda dx, dr, do, cnt: dev.rmsNormAddRmsNorm(dtype, dx, dr, d_w, d_w2, do, cnt, n, EPS, uo))


# ---------------------------------------------------------------------------------------
# QK-norm + RoPE + KV append
# ---------------------------------------------------------------------------------------

def pair_floor(ref, D, rot, rtol=1e-5):
    """rtol * |(r_i, r_{i+half})| for rotated coordinates, 0 elsewhere; ref [..., D]."""
    r = np.asarray(ref, np.float64)
    eff = D if (rot == 0 or rot > D) else rot
    h = eff // 2
    f = np.zeros_like(r)
    pn = np.sqrt(r[..., :h] ** 2 + r[..., h:2 * h] ** 2)
    f[..., :h] = rtol * pn
    f[..., h:2 * h] = rtol * pn
    return f


def qk_case(dev, oracle, dtype, T, nh, nkv, D, rot, base, positions, slots=None, v_norm=False,
            max_seq=4096, use_pos_array=True, layer=0, seed=7):
    gen = synth.normal_bf16 if dtype == B.BF16 else synth.normal_f32
    q = gen(seed, "q", (T, nh, D))
    k = gen(seed, "k", (T, nkv, D))
    v = gen(seed, "v", (T, nkv, D))
    wq = synth.normal_f32(seed, "wq", (D,), 0, 0.1)
    wk = synth.normal_f32(seed, "wk", (D,), 0, 0.1)
    max_kv_dim = nkv * D
    n_layers = layer + 1
    cache_rows = n_layers * max_seq if slots is None else int(np.max(slots)) + 1
    cdt = np.uint16 if dtype == B.BF16 else np.float32
    kc = np.zeros((cache_rows, max_kv_dim), cdt)
    vc = np.zeros((cache_rows, max_kv_dim), cdt)
    pos = np.asarray(positions, np.int32)
    q_ref = oracle.qk_norm_rope_kv(q, k, v, wq, wk, kc, vc, v_norm=v_norm, layer=layer,
                                   max_seq=max_seq, max_kv_dim=max_kv_dim, pos=pos,
                                   slots=slots, n_heads=nh, n_kv_heads=nkv, head_dim=D,
                                   rotary_dim=rot, base=base, eps=EPS)
    d_q, d_k, d_v = dev.from_numpy(q), dev.from_numpy(k), dev.from_numpy(v)
    d_kc, d_vc = dev.alloc(kc.nbytes), dev.alloc(vc.nbytes)
    d_kc.fill(0)
    d_vc.fill(0)
    d_pos = dev.from_numpy(pos) if use_pos_array else None
    d_slot = dev.from_numpy(np.asarray(slots, np.int64)) if slots is not None else None
    pos_base = int(pos[0]) if not use_pos_array else 0
    dev.qkNormRopeKv(dtype, d_q, d_k, d_v, dev.from_numpy(wq), dev.from_numpy(wk), v_norm, d_kc, d_vc,
                     cache_rows, layer, max_seq, max_kv_dim, d_pos, pos_base, d_slot, T, nh, nkv, D,
                     rot, base, 1.0, EPS, True)
    gq = d_q.to_numpy(q.shape, cdt)
    gk = d_kc.to_numpy(kc.shape, cdt)
    gv = d_vc.to_numpy(vc.shape, cdt)
    kref = kc.reshape(cache_rows, nkv, D)
    if dtype == B.F32:
        assert_rel(gq, q_ref, 1e-5, floor=pair_floor(q_ref, D, rot), what="Q norm+rope")
        assert_rel(gk.reshape(cache_rows, nkv, D), kref, 1e-5, floor=pair_floor(kref, D, rot), what="K cache")
        assert_rel(gv, vc, 1e-5, what="V cache")
        if not v_norm:
            assert_bitexact(gv, vc, "V cache copy")
    else:
        f = O.get().bf16_to_f32
        assert_bf16(gq, q_ref, 1, floor=pair_floor(f(q_ref), D, rot), what="bf16 Q")
        assert_bf16(gk.reshape(cache_rows, nkv, D), kref, 1, floor=pair_floor(f(kref), D, rot), what="bf16 K cache")
        if v_norm:
            assert_bf16(gv, vc, 1, what="bf16 V cache")
        else:
            assert_bitexact(gv, vc, "bf16 V cache copy")


def test_qk_c1_decode_f32(dev, oracle):
    qk_case(dev, oracle, B.F32, 1, 8, 4, 256, 0, 10000.0, [1234])


def test_qk_c1_decode_f32_by_value_pos(dev, oracle):
    qk_case(dev, oracle, B.F32, 1, 8, 4, 256, 0, 10000.0, [1234], use_pos_array=False)


def test_qk_prefill_bf16_d256(dev, oracle):
    qk_case(dev, oracle, B.BF16, 64, 8, 4, 256, 0, 10000.0, np.arange(1000, 1064), max_seq=4096)


@pytest.mark.parametrize("base", [10000.0, 1e6])
def test_qk_prefill_bf16_d128(dev, oracle, base):
    qk_case(dev, oracle, B.BF16, 24, 32, 16, 128, 0, base, np.arange(8000, 8024), max_seq=8192, layer=1)


def test_qk_batched_decode_slots_f32(dev, oracle):
    B_ = 8
    pos = synth.uniform_int(4, "pos", (B_,), 0, 32767).astype(np.int32)
    slots = np.arange(B_, dtype=np.int64) * 32768 + pos
    qk_case(dev, oracle, B.F32, B_, 8, 4, 256, 0, 10000.0, pos, slots=slots, max_seq=32768)


def test_qk_v_norm_d64(dev, oracle):
    qk_case(dev, oracle, B.F32, 5, 4, 2, 64, 0, 10000.0, np.arange(5), v_norm=True)


@pytest.mark.parametrize("D,rot", [(256, 128), (512, 128), (512, 0), (128, 64)])
def test_qk_partial_rotary(dev, oracle, D, rot):
    """Fused path with a rotary width below head_dim (lanes split into RoPE pairs and the
    unrotated tail) and head_dim 512; one token (workgroups per pass of head rows) and a
    few."""
    qk_case(dev, oracle, B.F32, 1, 8, 1, D, rot, 1e6, [1234])
    qk_case(dev, oracle, B.F32, 3, 4, 2, D, rot, 1e6, [3, 900, 4095])
    qk_case(dev, oracle, B.BF16, 3, 4, 2, D, rot, 1e6, [3, 900, 4095])


@pytest.mark.parametrize("dtype,nh,nkv,D,rot,v_norm", [
    (B.BF16, 32, 16, 128, 0, False),  # Gemma-27B heads (the c4 shape)
    (B.F32, 8, 4, 256, 0, False),
    (B.BF16, 16, 4, 256, 128, False),  # partial rotary
    (B.BF16, 64, 16, 64, 0, True),  # Gemma-4 V no-scale norm
])
def test_qk_many_tokens_equal_split_launches(dev, oracle, dtype, nh, nkv, D, rot, v_norm):
    """A launch of 4100 tokens whose head rows take two passes of a workgroup, against the same
    tokens in two launches (views into the same buffers and position array): Q and both
    caches bit-equal, so a token's result depends on nothing but its own rows and position.
    Positions come from a device array, all distinct, some at or past max_seq (those tokens'
    K / V rows are not written). The whole launch is also checked against the oracle at
    in-range positions."""
    T, split, max_seq = 4100, 2050, 8192
    bf = dtype == B.BF16
    gen = synth.normal_bf16 if bf else synth.normal_f32
    cdt = np.uint16 if bf else np.float32
    es = 2 if bf else 4
    q = gen(31, "q", (T, nh, D))
    k = gen(31, "k", (T, nkv, D))
    v = gen(31, "v", (T, nkv, D))
    d_wq = dev.from_numpy(synth.normal_f32(31, "wq", (D,), 0, 0.1))
    d_wk = dev.from_numpy(synth.normal_f32(31, "wk", (D,), 0, 0.1))
    rng = np.random.default_rng(31)
    pos = rng.permutation(max_seq + 64)[:T].astype(np.int32)
    assert np.any(pos >= max_seq)

    def run(parts):
        d_q, d_k, d_v, d_pos = dev.from_numpy(q), dev.from_numpy(k), dev.from_numpy(v), dev.from_numpy(pos)
        d_kc, d_vc = dev.alloc(max_seq * nkv * D * es), dev.alloc(max_seq * nkv * D * es)
        d_kc.fill(0)
        d_vc.fill(0)
        for t0, cnt in parts:
            dev.qkNormRopeKv(dtype, d_q.at(t0 * nh * D * es), d_k.at(t0 * nkv * D * es),
                             d_v.at(t0 * nkv * D * es), d_wq, d_wk, v_norm, d_kc, d_vc, max_seq, 0,
                             max_seq, nkv * D, d_pos.at(t0 * 4), 0, None, cnt, nh, nkv, D, rot, 10000.0,
                             1.0, EPS, True)
        dev.sync()
        out = (d_q.to_numpy(q.shape, cdt), d_kc.to_numpy((max_seq, nkv * D), cdt),
               d_vc.to_numpy((max_seq, nkv * D), cdt))
        for b in (d_q, d_k, d_v, d_pos, d_kc, d_vc):
            b.deinit()
        return out

    whole, halves = run([(0, T)]), run([(0, split), (split, T - split)])
    for got, ref, what in zip(whole, halves, ("Q", "K cache", "V cache")):
        assert_bitexact(got, ref, what)
    qk_case(dev, oracle, dtype, T, nh, nkv, D, rot, 10000.0, rng.permutation(max_seq)[:T], v_norm=v_norm,
            max_seq=max_seq, seed=32)


@pytest.mark.parametrize("D,rot", [(96, 0), (128, 24)])
def test_qk_generic_path(dev, oracle, D, rot):
    """Generic path: head_dim outside the fused set, or (bf16) a rotary half that is not a
    whole number of 16-byte chunks."""
    qk_case(dev, oracle, B.F32, 3, 4, 2, D, rot, 1e6, [3, 900, 4095])
    qk_case(dev, oracle, B.BF16, 3, 4, 2, D, rot, 1e6, [3, 900, 4095])


def test_qk_many_tokens_loop_over_head_rows(dev, oracle):
    """More than 64 tokens: one workgroup per token takes its head rows in passes."""
    qk_case(dev, oracle, B.BF16, 96, 32, 16, 128, 0, 1e6, np.arange(500, 596), max_seq=1024)
    qk_case(dev, oracle, B.F32, 80, 8, 1, 512, 128, 1e6, np.arange(10, 90), max_seq=1024)


@pytest.mark.parametrize("dtype", [B.BF16, B.F32])
def test_qk_two_tokens_per_workgroup_odd_count(dev, oracle, dtype):
    """From 1024 tokens with every head row in one pass, a workgroup takes two tokens; an odd
    token count leaves the last workgroup one token (its second slot reads and writes
    nothing)."""
    T = 1031
    qk_case(dev, oracle, dtype, T, 8, 4, 256, 0, 10000.0, np.arange(3000, 3000 + T), max_seq=4096)
    qk_case(dev, oracle, dtype, T, 8, 2, 256, 128, 1e6, np.arange(T)[::-1], max_seq=2048)


def test_rope_mirrors(dev, oracle):
    nh, nkv, D = 8, 4, 256
    q = synth.normal_f32(9, "q", (nh, D))
    k = synth.normal_f32(9, "k", (nkv, D))
    qr, kr = oracle.apply_rope(q, k, 1234, D, 0, nh, nkv, 10000.0)
    d_q, d_k = dev.from_numpy(q), dev.from_numpy(k)
    dev.rope(None, d_k, 1234, 0, nkv, D, 0, 10000.0)  # K first, as cuda_model.zig:658
    dev.rope(d_q, None, 1234, nh, 0, D, 0, 10000.0)
    assert_rel(d_q.to_numpy(q.shape, np.float32), qr, 1e-5, floor=pair_floor(qr, D, 0))
    assert_rel(d_k.to_numpy(k.shape, np.float32), kr, 1e-5, floor=pair_floor(kr, D, 0))
    # device-side position
    d_q2 = dev.from_numpy(q)
    dev.ropeInd(d_q2, None, dev.from_numpy(np.array([1234], np.int32)), nh, 0, D, 0, 10000.0)
    assert_rel(d_q2.to_numpy(q.shape, np.float32), qr, 1e-5, floor=pair_floor(qr, D, 0))
    # batched: token b at pos + b
    Bt = 5
    qb = synth.normal_f32(9, "qb", (Bt, nh, D))
    d_qb = dev.from_numpy(qb)
    dev.ropeBatched(d_qb, None, 100, Bt, nh, 0, D, 0, 10000.0)
    ref = np.stack([oracle.apply_rope(qb[b], None, 100 + b, D, 0, nh, 0, 10000.0)[0] for b in range(Bt)])
    assert_rel(d_qb.to_numpy(qb.shape, np.float32), ref, 1e-5, floor=pair_floor(ref, D, 0))


def test_kv_cache_put_mirrors(dev, oracle):
    nkv, D, max_seq, layers = 4, 256, 64, 3
    max_kv_dim = nkv * D + 64  # padded rows, as the reference's max_kv_dim allows
    kc = np.zeros((layers * max_seq, max_kv_dim), np.float32)
    vc = np.zeros_like(kc)
    d_kc, d_vc = dev.alloc(kc.nbytes), dev.alloc(vc.nbytes)
    d_kc.fill(0)
    d_vc.fill(0)
    k = synth.normal_f32(10, "k", (6, nkv, D))
    v = synth.normal_f32(10, "v", (6, nkv, D))
    d_k, d_v = dev.from_numpy(k), dev.from_numpy(v)
    dev.kvCachePut(d_kc, d_vc, d_k, d_v, 1, 17, max_seq, nkv, D, max_kv_dim)
    oracle.kv_cache_put(kc, vc, k[0], v[0], 1, 17, max_seq, nkv, D, max_kv_dim)
    dev.kvCachePutInd(d_kc, d_vc, d_k.at(k[0].nbytes), d_v.at(v[0].nbytes), 2,
                      dev.from_numpy(np.array([63], np.int32)), max_seq, nkv, D, max_kv_dim)
    oracle.kv_cache_put(kc, vc, np.ascontiguousarray(k[1]), np.ascontiguousarray(v[1]), 2, 63, max_seq, nkv, D, max_kv_dim)
    dev.kvCachePutBatched(d_kc, d_vc, d_k.at(2 * k[0].nbytes), d_v.at(2 * v[0].nbytes), 0, 60, 4,
                          max_seq, nkv, D, max_kv_dim)  # rows 60..63 (the 4th at 63 is the last slot)
    for b in range(4):
        oracle.kv_cache_put(kc, vc, np.ascontiguousarray(k[2 + b]), np.ascontiguousarray(v[2 + b]), 0,
                            60 + b, max_seq, nkv, D, max_kv_dim)
    assert_bitexact(d_kc.to_numpy(kc.shape, np.float32), kc, "K cache")
    assert_bitexact(d_vc.to_numpy(vc.shape, np.float32), vc, "V cache")
    # out-of-range position: skipped, cache untouched
    dev.kvCachePut(d_kc, d_vc, d_k, d_v, 0, max_seq, max_seq, nkv, D, max_kv_dim)
    assert_bitexact(d_kc.to_numpy(kc.shape, np.float32), kc, "K cache after pos=max_seq")


# ---------------------------------------------------------------------------------------
# GeGLU, soft-cap, add, scale
# ---------------------------------------------------------------------------------------

EXTREMES = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-4, -1e-4, 0.5, -0.5, 3.0, -3.0, 5.0, -5.0, 9.0,
                     -9.0, 20.0, -20.0, 60.0, -60.0, 1e4, -1e4], np.float32)


def geglu_floor(g, u):
    return np.abs(np.asarray(g, np.float64) * np.asarray(u, np.float64)) * 2.0 ** -23


@pytest.mark.parametrize("n", [10240, 10240 + 3, 7])
def test_geglu_f32(dev, oracle, n):
    g = synth.normal_f32(0, "gate", (n,))
    u = synth.normal_f32(0, "up", (n,))
    g[: min(n, EXTREMES.size)] = EXTREMES[: min(n, EXTREMES.size)]
    ref = oracle.geglu(g, u)
    d_g, d_u, d_o = dev.from_numpy(g), dev.from_numpy(u), dev.alloc(g.nbytes)
    dev.geglu(d_g, d_u, d_o, n)
    assert_rel(d_o.to_numpy((n,), np.float32), ref, 1e-5, floor=geglu_floor(g, u), what="geglu f32")
    dev.geglu(d_g, d_u, d_g, n)  # out aliases gate (math.zig geglu in place, model.zig:736-738)
    assert_rel(d_g.to_numpy((n,), np.float32), ref, 1e-5, floor=geglu_floor(g, u), what="geglu in place")


@pytest.mark.parametrize("n", [64 * 10240, 4096 + 5])
def test_geglu_bf16(dev, oracle, n):
    g = synth.normal_bf16(1, "gate", (n,))
    u = synth.normal_bf16(1, "up", (n,))
    g[:EXTREMES.size] = synth.f32_to_bf16(EXTREMES)
    ref = oracle.geglu(g, u)
    d_o = dev.alloc(g.nbytes)
    dev.gegluEx(B.BF16, dev.from_numpy(g), dev.from_numpy(u), d_o, n)
    f = O.get().bf16_to_f32
    assert_bf16(d_o.to_numpy((n,), np.uint16), ref, 1, floor=geglu_floor(f(g), f(u)), what="geglu bf16")


@pytest.mark.parametrize("cap,n,sigma", [(50.0, 8 * 1235, 20.0), (30.0, 4 * 262144, 15.0), (30.0, 1001, 100.0)])
def test_softcap_f32(dev, oracle, cap, n, sigma):
    x = synth.normal_f32(4, "logits", (n,), 0, sigma)
    x[:EXTREMES.size] = EXTREMES
    ref = oracle.softcap(x, cap)
    d_x = dev.from_numpy(x)
    dev.tanhSoftcap(d_x, cap, n)
    assert_rel(d_x.to_numpy((n,), np.float32), ref, 1e-5, what=f"softcap cap={cap}")


def test_softcap_bf16(dev, oracle):
    n = 3 * 4096 + 1
    x = synth.normal_bf16(4, "s", (n,), 0, 20)
    ref = oracle.f32_to_bf16(oracle.softcap(oracle.bf16_to_f32(x), 50.0))
    d_x = dev.from_numpy(x)
    dev.tanhSoftcapEx(B.BF16, d_x, 50.0, n)
    assert_bf16(d_x.to_numpy((n,), np.uint16), ref, 1, what="softcap bf16")


# SwiGLU: relative 1e-5; where exp(-gate) overflows in f32 (gate < -88.7) or the quotient
# is subnormal, the CPU gives x / inf = -0 or a value below 2e-37, so the floor is
# |up| * 1e-36.
SILU_EXTREMES = np.array([-87.0, -88.5, -88.75, -89.0, -100.0, -1e4, 87.0, 88.8, 1e4, -1e-40, 1e-40,
                          np.float32(1e-37), -16.6, 16.6], np.float32)


@pytest.mark.parametrize("n", [10240, 10240 + 3, 7])
def test_swiglu_f32(dev, oracle, n):
    g = synth.normal_f32(6, "gate", (n,), 0, 4)
    u = synth.normal_f32(6, "up", (n,))
    ext = np.concatenate([EXTREMES, SILU_EXTREMES])
    m = min(n, ext.size)
    g[:m] = ext[:m]
    ref = oracle.swiglu(g, u)
    floor = np.abs(u.astype(np.float64)) * 1e-36
    d_g, d_u, d_o = dev.from_numpy(g), dev.from_numpy(u), dev.alloc(g.nbytes)
    dev.swiglu(d_g, d_u, d_o, n)
    assert_rel(d_o.to_numpy((n,), np.float32), ref, 1e-5, floor=floor, what="swiglu f32")
    dev.swiglu(d_g, d_u, d_u, n)  # out aliases up
    assert_rel(d_u.to_numpy((n,), np.float32), ref, 1e-5, floor=floor, what="swiglu in place")


@pytest.mark.parametrize("n", [64 * 10240, 4096 + 5])
def test_swiglu_bf16(dev, oracle, n):
    g = synth.normal_bf16(6, "gate", (n,), 0, 4)
    u = synth.normal_bf16(6, "up", (n,))
    g[:EXTREMES.size] = synth.f32_to_bf16(EXTREMES)
    ref = oracle.swiglu(g, u)
    d_o = dev.alloc(g.nbytes)
    dev.swigluEx(B.BF16, dev.from_numpy(g), dev.from_numpy(u), d_o, n)
    floor = np.abs(O.get().bf16_to_f32(u).astype(np.float64)) * 1e-36
    assert_bf16(d_o.to_numpy((n,), np.uint16), ref, 1, floor=floor, what="swiglu bf16")


@pytest.mark.parametrize("n", [256, 35 * 256, 35 * 256 * 8 + 3])
def test_ple_gate_gelu(dev, oracle, n):
    """cuda_ple_gate_gelu (cuda_bridge.h:171) against model.zig:762-768."""
    g = synth.normal_f32(7, "pg", (n,), 0, 2)
    sl = synth.normal_f32(7, "ps", (n,))
    g[:EXTREMES.size] = EXTREMES
    ref = oracle.ple_gate_gelu(g, sl)
    d_o = dev.alloc(g.nbytes)
    dev.pleGateGelu(dev.from_numpy(g), dev.from_numpy(sl), d_o, n)
    assert_rel(d_o.to_numpy((n,), np.float32), ref, 1e-5, floor=geglu_floor(g, sl), what="ple gate gelu")


@pytest.mark.parametrize("add", [True, False])
@pytest.mark.parametrize("n", [35 * 256, 8 * 35 * 256 + 5, 3])
def test_ple_ctx_fuse_bitexact(dev, oracle, n, add):
    """cuda_ple_ctx_fuse (cuda_bridge.h:172) against model.zig:525-535: one rounding of the
    sum, one of the product by f32(1/sqrt 2), so bit-exact."""
    ctx = synth.normal_f32(8, "ctx", (n,), 0, 16)
    s = synth.normal_f32(8, "scr", (n,))
    ref = oracle.ple_ctx_fuse(ctx, s, add)
    d_c = dev.from_numpy(ctx)
    dev.pleCtxFuse(d_c, dev.from_numpy(s), n, add)
    assert_bitexact(d_c.to_numpy((n,), np.float32), ref, f"ple ctx fuse add={add}")


def test_add_scale_mirrors(dev):
    n = 2560 + 1
    x = synth.normal_f32(5, "x", (n,))
    r = synth.normal_f32(5, "r", (n,))
    d_x = dev.from_numpy(x)
    dev.add(d_x, dev.from_numpy(r), n)
    assert_bitexact(d_x.to_numpy((n,), np.float32), (x + r).astype(np.float32), "add")
    dev.scale(d_x, np.float32(0.37), n)
    assert_bitexact(d_x.to_numpy((n,), np.float32), ((x + r) * np.float32(0.37)).astype(np.float32), "scale")


@pytest.mark.parametrize("base", [10000.0, 1e6])
@pytest.mark.parametrize("D", [256, 128, 64])
def test_rope_angles(dev, oracle, base, D):
    """RoPE alone (no norm). The angles are the oracle's theta = f32(pos) / D_i (same D_i,
    IEEE divide); cos / sin come from the kernel's own evaluation (an exact double-precision
    reduction and fitted f32 polynomials), which must lie within 2 ulp of the correctly
    rounded values the oracle uses. Rotating the unit pairs (1, 0) reads them out directly:
    h[i] = cos(theta_i), h[i + D/2] = sin(theta_i). Random heads are then checked within the
    1e-5 pair-norm tolerance, positions up to 32767 at both RoPE bases."""
    nh, nkv = 4, 2
    positions = [0, 1, 2, 17, 100, 1234, 2047, 4095, 8191, 16383, 32767]
    half = D // 2
    unit = np.zeros((len(positions), nh, D), np.float32)
    unit[..., :half] = 1.0
    d_u = dev.from_numpy(unit)
    for i, p in enumerate(positions):
        dev.rope(d_u.at(i * nh * D * 4), None, p, nh, nkv, D, 0, base)
    gu = d_u.to_numpy(unit.shape, np.float32)
    for i, p in enumerate(positions):
        ref_c = np.empty(half, np.float32)
        ref_s = np.empty(half, np.float32)
        for j in range(half):
            ref_c[j], ref_s[j] = oracle.rope_cos_sin(np.float32(p), oracle.rope_denominator(base, j, D))
        for h in range(nh):
            for got, ref, what in ((gu[i, h, :half], ref_c, "cos"), (gu[i, h, half:], ref_s, "sin")):
                err = np.abs(got.astype(np.float64) - ref)
                ulp = np.spacing(np.abs(ref)).astype(np.float64)
                assert np.all(err <= 2.0 * ulp + 1e-45), \
                    f"{what} at pos {p}: {np.max(err / np.maximum(ulp, 1e-45)):.2f} ulp"
    q = synth.normal_f32(11, "q", (len(positions), nh, D))
    k = synth.normal_f32(11, "k", (len(positions), nkv, D))
    qr = np.stack([oracle.apply_rope(q[i], k[i], p, D, 0, nh, nkv, base)[0] for i, p in enumerate(positions)])
    kr = np.stack([oracle.apply_rope(q[i], k[i], p, D, 0, nh, nkv, base)[1] for i, p in enumerate(positions)])
    d_q, d_k = dev.from_numpy(q), dev.from_numpy(k)
    for i, p in enumerate(positions):
        dev.rope(d_q.at(i * nh * D * 4), d_k.at(i * nkv * D * 4), p, nh, nkv, D, 0, base)
    gq, gk = d_q.to_numpy(q.shape, np.float32), d_k.to_numpy(k.shape, np.float32)
    for g, r, name in ((gq, qr, "Q"), (gk, kr, "K")):
        assert_rel(g, r, 1e-5, floor=pair_floor(r, D, 0), what=f"rope {name}")
