"""Prefill-sized GEMM on the matrix cores (hip_gemm from its threshold, hip_gemm_ex: gemm.hip) against
float64 and the oracle's math.gemm (math.zig:440-616), through the C-ABI.

The activations are split into three bf16 terms and the weights into one (Q4_0, Q8_0, BF16,
Q4_K, Q6_K), two (F16) or three (F32) exact bf16 terms, so
  * integer-valued operands give the exact integer dot product, bit for bit (every term but
    the first is zero and every partial sum is exact): indexing, nibble order, block scales,
    ragged tiles in both dimensions, the two workgroup shapes;
  * on random operands the result and the oracle's both lie within 2^-20 * sum |w_i x_i| of
    the float64 product of the dequantised weights, the bound the decode GEMV meets.
"""
import numpy as np
import pytest

from oracle import oracle as O
from test_oracle_gemv_cpu import bound, int_matrix, random_matrix
from ziglm_amd import bridge as B
from ziglm_amd import synth

pytestmark = pytest.mark.gpu

TYPES = [B.Q4_0, B.Q8_0, B.F16, B.BF16, B.F32]


def run(dev, qtype, raw, X, rows, cols):
    batch = X.shape[0]
    d_w = dev.from_numpy(np.ascontiguousarray(raw).reshape(-1))
    d_x = dev.from_numpy(np.ascontiguousarray(X, np.float32).reshape(-1))
    d_y = dev.alloc(batch * rows * 4)
    d_y.fill(0xAB)
    dev.gemm(qtype, d_w, d_x, d_y, batch, rows, cols)
    return d_y.to_numpy((batch, rows), np.float32)


# Workgroup tiles (tokens x rows) by launch size: 128 x 128 from 512 such tiles (e.g. 4096 rows
# x 2048 tokens), else 64 x 128 from 512 (4096 x 1024; 2560 x 2048, 2500 x 1900 with a ragged
# last tile), else 64 x 64.
@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("rows,cols,batch", [(128, 64, 32), (200, 96, 37), (129, 2560, 128), (77, 160, 300),
                                             (256, 512, 64), (4096, 96, 2048), (4100, 64, 2050),
                                             (4096, 64, 1024), (4097, 96, 1000), (2560, 256, 2048),
                                             (2500, 96, 1900)])
def test_gemm_mfma_integer_bitexact(dev, qtype, rows, cols, batch):
    raw, wd = int_matrix(qtype, rows, cols, seed=rows * cols + qtype + batch, scale_pow=-1)
    X = np.random.default_rng(batch).integers(-3, 4, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24)
    got = run(dev, qtype, raw, X, rows, cols)
    np.testing.assert_array_equal(got, exact.astype(np.float32), err_msg=f"qtype={qtype} {rows}x{cols} b={batch}")


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("rows,cols,batch", [(256, 2560, 128), (300, 1024, 77), (1024, 2560, 512),
                                             (128, 10240, 64), (4096, 512, 2048), (4096, 1024, 1024),
                                             (2560, 1024, 2048)])
def test_gemm_mfma_vs_f64_and_oracle(dev, oracle, qtype, rows, cols, batch):
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + cols + batch)
    X = synth.normal_f32(rows + batch, "X", (batch, cols), 0, 2)
    exact = X.astype(np.float64) @ wd.T
    bd = bound(wd, X)
    got = run(dev, qtype, raw, X, rows, cols).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))
    if rows * cols * batch <= 1 << 28:
        ref = oracle.gemm(qtype, raw, X).astype(np.float64)
        assert np.all(np.abs(ref - exact) <= bd)


def test_gemm_mfma_extreme_activations(dev):
    """Activations over a wide dynamic range (1e-30 .. 1e30 in one row) and exact zeros: the
    three-term split keeps every element's 24 bits."""
    rows, cols, batch = 96, 256, 40
    raw, wd = random_matrix(B.BF16, rows, cols, seed=9)
    rng = np.random.default_rng(9)
    X = (rng.standard_normal((batch, cols)) * 10.0 ** rng.integers(-30, 31, (batch, cols))).astype(np.float32)
    X[:, ::17] = 0.0
    exact = X.astype(np.float64) @ wd.T
    got = run(dev, B.BF16, raw, X, rows, cols).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bound(wd, X))


# ---- hip_gemm_ex: bf16 activations (one exact term), bf16 output, gate.up GeGLU ----------

def bf16_bits(a):
    return O.get().f32_to_bf16(np.ascontiguousarray(a, np.float32))


def run_ex(dev, qtype, raw, X, rows, cols, x_dtype, y_dtype, raw_up=None):
    batch = X.shape[0]
    xb = bf16_bits(X) if x_dtype == B.BF16 else np.ascontiguousarray(X, np.float32)
    d_w = dev.from_numpy(np.ascontiguousarray(raw).reshape(-1))
    d_u = dev.from_numpy(np.ascontiguousarray(raw_up).reshape(-1)) if raw_up is not None else None
    d_x = dev.from_numpy(xb.reshape(-1))
    es = 2 if y_dtype == B.BF16 else 4
    d_y = dev.alloc(batch * rows * es)
    d_y.fill(0xAB)
    dev.gemmEx(qtype, d_w, d_u, x_dtype, d_x, y_dtype, d_y, batch, rows, cols)
    if y_dtype == B.BF16:
        return d_y.to_numpy((batch, rows), np.uint16)
    return d_y.to_numpy((batch, rows), np.float32)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("rows,cols,batch", [(128, 64, 32), (200, 96, 37), (129, 2560, 5), (4100, 64, 2050),
                                             (4096, 64, 1024), (77, 160, 300), (2560, 256, 2048), (2500, 96, 1900)])
def test_gemm_ex_bf16_activations_integer_bitexact(dev, qtype, rows, cols, batch):
    """Integer activations are exact in bf16, so the bf16-input product of integer operands is
    the exact integer dot product (f32 output) and its bf16 rounding (bf16 output)."""
    raw, wd = int_matrix(qtype, rows, cols, seed=rows * cols + qtype + batch + 1, scale_pow=-1)
    X = np.random.default_rng(batch + 7).integers(-3, 4, (batch, cols)).astype(np.float32)
    exact = (X.astype(np.float64) @ wd.T).astype(np.float32)
    got = run_ex(dev, qtype, raw, X, rows, cols, B.BF16, B.F32)
    np.testing.assert_array_equal(got, exact, err_msg=f"qtype={qtype} {rows}x{cols} b={batch}")
    got16 = run_ex(dev, qtype, raw, X, rows, cols, B.BF16, B.BF16)
    np.testing.assert_array_equal(got16, bf16_bits(exact))


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("rows,cols,batch", [(256, 2560, 128), (300, 1024, 77), (1024, 2560, 512), (4096, 512, 2048)])
def test_gemm_ex_bf16_activations_vs_f64_and_oracle(dev, oracle, qtype, rows, cols, batch):
    """bf16 activations against the float64 product of the same (bf16-valued) activations and
    the oracle's math.gemm on them: within 2^-20 * sum |w_i x_i|."""
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + cols + batch + 3)
    Xf = O.get().bf16_to_f32(bf16_bits(synth.normal_f32(rows + batch, "Xb", (batch, cols), 0, 2)))
    exact = Xf.astype(np.float64) @ wd.T
    bd = bound(wd, Xf)
    got = run_ex(dev, qtype, raw, Xf, rows, cols, B.BF16, B.F32).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))
    if rows * cols * batch <= 1 << 27:
        ref = oracle.gemm(qtype, raw, Xf).astype(np.float64)
        assert np.all(np.abs(ref - exact) <= bd)


def _gelu64(g):
    return 0.5 * g * (1.0 + np.tanh(0.7978845608 * (g + 0.044715 * g ** 3)))


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0, B.BF16, B.Q4_K, B.Q6_K])
@pytest.mark.parametrize("x_dtype,y_dtype", [(B.BF16, B.BF16), (B.BF16, B.F32), (B.F32, B.F32)])
@pytest.mark.parametrize("rows,cols,batch", [(320, 256, 96), (1000, 512, 200), (2560, 2560, 2048)])
def test_gemm_ex_geglu_pair(dev, oracle, qtype, x_dtype, y_dtype, rows, cols, batch):
    """y = gelu_tanh(W x) * (U x) in one launch against float64: g = W x and u = U x each lie
    within the product bound bd_g / bd_u of their exact values, and gelu has |gelu'| < 1.13,
    so |y - gelu(g64) u64| <= 1.13 bd_g |u64| + |gelu(g64)| bd_u + bd_g bd_u, plus the kernel's
    own GELU and product rounding (a few ulp: 1e-5 relative and, for the reference's 1 + tanh(z)
    cancellation, 2^-22 |g u|), plus one bf16 ulp for a bf16 output. Also against the oracle's
    composition (math.gemm twice, then math.geglu) at the smallest size."""
    raw_g, wg = random_matrix(qtype, rows, cols, seed=rows + batch + 11)
    raw_u, wu = random_matrix(qtype, rows, cols, seed=rows + batch + 12)
    X = synth.normal_f32(rows + batch + 13, "Xg", (batch, cols), 0, 1)
    if x_dtype == B.BF16:
        X = O.get().bf16_to_f32(bf16_bits(X))
    g64, u64 = X.astype(np.float64) @ wg.T, X.astype(np.float64) @ wu.T
    bd_g, bd_u = bound(wg, X), bound(wu, X)
    ref = _gelu64(g64) * u64
    tol = 1.13 * bd_g * np.abs(u64) + np.abs(_gelu64(g64)) * bd_u + bd_g * bd_u + 1e-5 * np.abs(ref) \
        + 2.0 ** -22 * np.abs(g64 * u64)
    got = run_ex(dev, qtype, raw_g, X, rows, cols, x_dtype, y_dtype, raw_up=raw_u)
    if y_dtype == B.BF16:
        got = O.get().bf16_to_f32(got)
        tol = tol + np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) * 65536.0
    got = got.astype(np.float64)
    bad = np.abs(got - ref) > tol
    assert not bad.any(), (int(bad.sum()), float(np.max(np.abs(got - ref) / tol)))
    if rows == 320:
        og = oracle.gemm(qtype, raw_g, X)
        ou = oracle.gemm(qtype, raw_u, X)
        oref = oracle.geglu(og, ou).astype(np.float64)
        assert np.all(np.abs(oref - ref) <= tol)


# ---- hip_split_terms and the F32_TERMS input ----------------------------------------------

def split_terms_ref(x):
    """h = bf16(x), m = bf16(x - h), l = bf16(x - h - m), RNE, float32 arithmetic (numpy)."""
    o = O.get()
    x = np.ascontiguousarray(x, np.float32)
    h = o.f32_to_bf16(x)
    r = (x - o.bf16_to_f32(h)).astype(np.float32)
    m = o.f32_to_bf16(r)
    r2 = (r - o.bf16_to_f32(m)).astype(np.float32)
    return np.stack([h, m, o.f32_to_bf16(r2)])


def test_split_terms_bitexact(dev):
    rng = np.random.default_rng(31)
    n = 4 * 40000
    x = (rng.standard_normal(n) * 10.0 ** rng.integers(-30, 31, n)).astype(np.float32)
    x[::97] = 0.0
    x[1::101] = -0.0
    d_p = dev.alloc(3 * n * 2)
    dev.splitTerms(dev.from_numpy(x), d_p, n)
    got = d_p.to_numpy((3, n), np.uint16)
    assert_eq = np.testing.assert_array_equal
    assert_eq(got, split_terms_ref(x))
    o = O.get()
    # h + m + l = x to 2^-24 relative; where x is below ~2^-110 the small terms are bf16
    # subnormals, whose last place is 2^-133 (the absolute floor)
    s = sum(o.bf16_to_f32(got[u]).astype(np.float64) for u in range(3))
    assert np.all(np.abs(s - x) <= 2.0 ** -24 * np.abs(x) + 2.0 ** -133)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("rows,cols,batch", [(256, 2560, 128), (300, 1024, 130), (4096, 512, 2048), (129, 160, 140),
                                             (2500, 96, 1900)])
def test_gemm_ex_split_terms_equal_f32_product(dev, qtype, rows, cols, batch):
    """Activations split beforehand (hip_split_terms, F32_TERMS input) give hip_gemm's f32
    product bit for bit where hip_gemm runs on the matrix cores (128 tokens and more for
    these row counts): the kernel stages the same three terms it would form itself."""
    raw, _ = random_matrix(qtype, rows, cols, seed=rows + cols + batch + 21)
    X = synth.normal_f32(rows + batch + 22, "Xs", (batch, cols), 0, 3)
    ref = run(dev, qtype, raw, X, rows, cols)
    d_x = dev.from_numpy(X.reshape(-1))
    d_p = dev.alloc(3 * batch * cols * 2)
    dev.splitTerms(d_x, d_p, batch * cols)
    d_w = dev.from_numpy(np.ascontiguousarray(raw).reshape(-1))
    d_y = dev.alloc(batch * rows * 4)
    d_y.fill(0xAB)
    dev.gemmEx(qtype, d_w, None, B.F32_TERMS, d_p, B.F32, d_y, batch, rows, cols)
    np.testing.assert_array_equal(d_y.to_numpy((batch, rows), np.float32), ref)
    # the GeGLU pair on split activations against the pair on f32 activations
    if qtype == B.Q4_0:
        raw_u, _ = random_matrix(qtype, rows, cols, seed=rows + cols + batch + 23)
        a = run_ex(dev, qtype, raw, X, rows, cols, B.F32, B.F32, raw_up=raw_u)
        d_u = dev.from_numpy(np.ascontiguousarray(raw_u).reshape(-1))
        dev.gemmEx(qtype, d_w, d_u, B.F32_TERMS, d_p, B.F32, d_y, batch, rows, cols)
        np.testing.assert_array_equal(d_y.to_numpy((batch, rows), np.float32), a)


# ---- K-quant weights (Q4_K, Q6_K) on the matrix cores --------------------------------------
# Q4_K: quants 0..15 exact in bf16, each 32-column sub-block's partial sum scaled by d * sc_j
# and the min term dmin * m_j * sum(x) subtracted (the x sums formed while staging); Q6_K:
# u - 32 exact in bf16, each 16-column half's partial sum scaled by d * sc.

KTYPES = [B.Q4_K, B.Q6_K]


@pytest.mark.parametrize("qtype", KTYPES)
@pytest.mark.parametrize("rows,cols,batch", [(128, 256, 32), (200, 512, 37), (129, 2560, 128), (77, 768, 300),
                                             (4096, 256, 2048), (4100, 256, 2050), (4096, 256, 1024),
                                             (2560, 512, 2048), (2500, 256, 1900)])
def test_gemm_mfma_kquant_integer_bitexact(dev, qtype, rows, cols, batch):
    """Integer-valued K-quant weights and activations: the exact integer dot product, f32 and
    bf16 activations alike (every tile shape, ragged tiles, tokens and rows past the ends)."""
    raw, wd = int_matrix(qtype, rows, cols, seed=rows * cols + qtype + batch, scale_pow=-1)
    X = np.random.default_rng(batch).integers(-3, 4, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24)
    got = run(dev, qtype, raw, X, rows, cols)
    np.testing.assert_array_equal(got, exact.astype(np.float32), err_msg=f"qtype={qtype} {rows}x{cols} b={batch}")
    got_b = run_ex(dev, qtype, raw, X, rows, cols, B.BF16, B.F32)
    np.testing.assert_array_equal(got_b, exact.astype(np.float32), err_msg="bf16 activations")


def q6_k_full_scales(rng, rows, cols, d):
    """Q6_K rows with int8 scales over their whole range (-128..127), so values d * sc * (u -
    32) span 13 bits; packed by the format description: super-block {ql[128],
    qh[64], scales[16], f16 d}, column c = 128 h + 32 k + l takes nibble k // 2 of
    ql[64 h + 32 (k % 2) + l], bits 2k, 2k + 1 of qh[32 h + l] and scale c // 16."""
    nsb = cols // 256
    u = rng.integers(0, 64, (rows, nsb, 256))
    sc = rng.integers(-128, 128, (rows, nsb, 16))
    raw = np.zeros((rows, nsb, 210), np.uint8)
    ql = np.zeros((rows, nsb, 128), np.int64)
    qh = np.zeros((rows, nsb, 64), np.int64)
    for c in range(256):
        h, i = divmod(c, 128)
        k, l = divmod(i, 32)
        ql[..., 64 * h + 32 * (k % 2) + l] |= (u[..., c] & 15) << (4 * (k // 2))
        qh[..., 32 * h + l] |= (u[..., c] >> 4) << (2 * k)
    raw[..., 0:128] = ql.astype(np.uint8)
    raw[..., 128:192] = qh.astype(np.uint8)
    raw[..., 192:208] = sc.astype(np.int8).view(np.uint8)
    raw[..., 208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    val = d * np.repeat(sc, 16, axis=-1) * (u - 32)
    return raw.reshape(rows, -1), val.reshape(rows, cols).astype(np.float64)


@pytest.mark.parametrize("rows,cols,batch", [(130, 512, 64), (300, 256, 257)])
def test_gemm_mfma_q6_k_full_scale_range_exact(dev, rows, cols, batch):
    """Full-range int8 scales (|sc * (u - 32)| up to 4096, 13 bits) and every half's own
    scale: integer products are exact."""
    raw, wd = q6_k_full_scales(np.random.default_rng(rows), rows, cols, 0.5)
    X = np.random.default_rng(batch).integers(-1, 2, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24) and np.max(np.abs(wd)) > 1000
    np.testing.assert_array_equal(run(dev, B.Q6_K, raw, X, rows, cols), exact.astype(np.float32))
    np.testing.assert_array_equal(run_ex(dev, B.Q6_K, raw, X, rows, cols, B.BF16, B.F32), exact.astype(np.float32))


@pytest.mark.parametrize("qtype", KTYPES)
@pytest.mark.parametrize("rows,cols,batch", [(256, 2560, 128), (300, 1024, 77), (1024, 2560, 512),
                                             (128, 10240, 64), (4096, 512, 2048), (2560, 1024, 2048)])
def test_gemm_mfma_kquant_vs_f64_and_oracle(dev, oracle, qtype, rows, cols, batch):
    """Random K-quant weights and N(0, 2) activations: within 2^-20 * sum |w_i x_i| of the
    float64 product of the dequantised weights, as is the oracle's math.gemm."""
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + cols + batch + 5)
    X = synth.normal_f32(rows + batch + 5, "Xk", (batch, cols), 0, 2)
    exact = X.astype(np.float64) @ wd.T
    bd = bound(wd, X)
    got = run(dev, qtype, raw, X, rows, cols).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))
    if rows * cols * batch <= 1 << 27:
        ref = oracle.gemm(qtype, raw, X).astype(np.float64)
        assert np.all(np.abs(ref - exact) <= bd)


@pytest.mark.parametrize("qtype", KTYPES)
@pytest.mark.parametrize("rows,cols,batch", [(256, 2560, 128), (1024, 2560, 512), (4096, 512, 2048)])
def test_gemm_ex_kquant_bf16_activations_vs_f64(dev, qtype, rows, cols, batch):
    """bf16 activations (one exact term) with K-quant weights, f32 and bf16 output."""
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + cols + batch + 6)
    Xf = O.get().bf16_to_f32(bf16_bits(synth.normal_f32(rows + batch + 6, "Xkb", (batch, cols), 0, 2)))
    exact = Xf.astype(np.float64) @ wd.T
    bd = bound(wd, Xf)
    got = run_ex(dev, qtype, raw, Xf, rows, cols, B.BF16, B.F32).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))
    got16 = O.get().bf16_to_f32(run_ex(dev, qtype, raw, Xf, rows, cols, B.BF16, B.BF16)).astype(np.float64)
    tol16 = bd + np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64) * 65536.0
    assert np.all(np.abs(got16 - exact) <= tol16)


@pytest.mark.parametrize("qtype", KTYPES)
@pytest.mark.parametrize("rows,cols,batch", [(256, 2560, 128), (4096, 512, 2048), (129, 256, 100)])
def test_gemm_ex_kquant_split_terms_and_geglu(dev, qtype, rows, cols, batch):
    """Pre-split activations (F32_TERMS) give hip_gemm's f32 product bit for bit for Q6_K; for
    Q4_K, whose min term sums each plane of the split activations instead of x itself, both
    lie within the product bound of the float64 product. The gate.up GeGLU pair on the planes
    equals (Q6_K) or matches within the bound (Q4_K) the pair on the f32 activations."""
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + cols + batch + 7)
    raw_u, wu = random_matrix(qtype, rows, cols, seed=rows + cols + batch + 8)
    X = synth.normal_f32(rows + batch + 7, "Xks", (batch, cols), 0, 3)
    ref = run(dev, qtype, raw, X, rows, cols)
    d_p = dev.alloc(3 * batch * cols * 2)
    dev.splitTerms(dev.from_numpy(X.reshape(-1)), d_p, batch * cols)
    d_w = dev.from_numpy(np.ascontiguousarray(raw).reshape(-1))
    d_u = dev.from_numpy(np.ascontiguousarray(raw_u).reshape(-1))
    d_y = dev.alloc(batch * rows * 4)
    d_y.fill(0xAB)
    dev.gemmEx(qtype, d_w, None, B.F32_TERMS, d_p, B.F32, d_y, batch, rows, cols)
    got = d_y.to_numpy((batch, rows), np.float32)
    pair = run_ex(dev, qtype, raw, X, rows, cols, B.F32, B.F32, raw_up=raw_u)
    dev.gemmEx(qtype, d_w, d_u, B.F32_TERMS, d_p, B.F32, d_y, batch, rows, cols)
    got_pair = d_y.to_numpy((batch, rows), np.float32)
    if qtype == B.Q6_K:
        np.testing.assert_array_equal(got, ref)
        np.testing.assert_array_equal(got_pair, pair)
        return
    g64, u64 = X.astype(np.float64) @ wd.T, X.astype(np.float64) @ wu.T
    bd_g, bd_u = bound(wd, X), bound(wu, X)
    assert np.all(np.abs(got.astype(np.float64) - g64) <= bd_g)
    assert np.all(np.abs(ref.astype(np.float64) - g64) <= bd_g)
    # the pair, both forms against float64 with test_gemm_ex_geglu_pair's tolerance
    ref_pair = _gelu64(g64) * u64
    tol = 1.13 * bd_g * np.abs(u64) + np.abs(_gelu64(g64)) * bd_u + bd_g * bd_u + 1e-5 * np.abs(ref_pair) \
        + 2.0 ** -22 * np.abs(g64 * u64)
    assert np.all(np.abs(got_pair.astype(np.float64) - ref_pair) <= tol)
    assert np.all(np.abs(pair.astype(np.float64) - ref_pair) <= tol)


def test_gemm_kquant_refuses_partial_super_blocks(dev):
    """K-quant rows that are not whole 256-column super-blocks are refused by hip_gemm_ex
    (nothing written)."""
    w, x, y = dev.alloc(1 << 16), dev.alloc(1 << 16), dev.alloc(64 * 64 * 4)
    y.fill(0x11)
    dev.strict = False
    try:
        for qt in KTYPES:
            dev.gemmEx(qt, w, None, B.BF16, x, B.F32, y, 64, 64, 224)
            assert dev.b.last_error() == B.EUNSUPPORTED
    finally:
        dev.strict = True
    assert np.all(y.to_numpy((64 * 64 * 4,), np.uint8) == 0x11)


# ---- two K halves (deep products, f32 output, fewer than two rounds of workgroups) -------------

@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0, B.BF16, B.Q4_K, B.Q6_K])
@pytest.mark.parametrize("rows,cols,batch", [(2560, 10240, 256), (300, 4352, 130), (77, 8192, 300)])
def test_gemm_split_k_integer_bitexact_and_random(dev, qtype, rows, cols, batch):
    """Deep products (cols >= 4096) whose tiles number fewer than two rounds run each tile as two
    K halves added into zeroed y: integer operands give the exact product bit for bit, random
    ones stay within 2^-20 * sum |w_i x_i| of float64, and a second call gives the same bits
    (two addends: 0 + a + b in either order)."""
    raw, wd = int_matrix(qtype, rows, cols, seed=rows + cols + batch + qtype, scale_pow=-3)
    X = np.random.default_rng(rows + batch).integers(-2, 3, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24)
    np.testing.assert_array_equal(run(dev, qtype, raw, X, rows, cols), exact.astype(np.float32))
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + cols + batch + 31)
    X = synth.normal_f32(rows + batch + 31, "Xsk", (batch, cols), 0, 2)
    exact = X.astype(np.float64) @ wd.T
    got = run(dev, qtype, raw, X, rows, cols)
    bd = bound(wd, X)
    assert np.all(np.abs(got.astype(np.float64) - exact) <= bd), float(np.max(np.abs(got - exact) / bd))
    np.testing.assert_array_equal(run(dev, qtype, raw, X, rows, cols), got)


@pytest.mark.parametrize("qtype,rows,cols,batch", [(B.Q4_0, 2560, 10240, 256), (B.Q4_0, 2560, 10240, 40),
                                                   (B.Q4_K, 2560, 4096, 200)])
def test_split_products_replay_in_a_graph(dev, qtype, rows, cols, batch):
    """The split products (a zero-fill kernel, then two halves added into y) captured in a
    hipGraph: three replays, with eager products on other buffers between them, each equal
    to the eager result bit for bit."""
    from ziglm_amd.device import Graph
    raw, _ = random_matrix(qtype, rows, cols, seed=rows + batch + 41)
    X = synth.normal_f32(rows + batch + 41, "Xg", (batch, cols), 0, 2)
    d_w = dev.from_numpy(np.ascontiguousarray(raw).reshape(-1))
    d_x = dev.from_numpy(np.ascontiguousarray(X).reshape(-1))
    d_y = dev.alloc(batch * rows * 4)
    dev.gemm(qtype, d_w, d_x, d_y, batch, rows, cols)
    ref = d_y.to_numpy((batch, rows), np.float32)
    g = Graph(dev, lambda: dev.gemm(qtype, d_w, d_x, d_y, batch, rows, cols))
    d_o = dev.alloc(batch * rows * 4)
    for i in range(3):
        d_y.fill(0x7F)
        dev.sync()
        g.launch()
        dev.sync()
        np.testing.assert_array_equal(d_y.to_numpy((batch, rows), np.float32), ref, err_msg=f"replay {i}")
        dev.gemm(qtype, d_w, d_x, d_o, batch, rows, cols)  # eager work between replays
        dev.sync()
        np.testing.assert_array_equal(d_o.to_numpy((batch, rows), np.float32), ref)
    g.destroy()
