"""Small-batch products on the matrix cores (gemv.hip k_gemv_mb: from 2 tokens up to the
prefill GEMM's threshold, 96 tokens for 8192 rows or more, 64 for narrower products at
least 4096 deep, else 128; Q4_0 / Q8_0 / BF16 weights) through the C-ABI, over its
launch choices: 1, 2 or 4 sixteen-row tiles per wave and 4, 8 or 16 waves splitting the
blocks of a row, rows too long for that in two halves added into zeroed y (so row counts that leave tiles and tile groups partly empty, block counts
that the waves split unevenly, one or two 16-token tiles, tokens that leave a tile partly
empty), and the shapes it leaves to the vector kernels (x not 16-byte aligned, other types,
a column count that is not a whole number of blocks).

Integer-valued weights and activations make every partial sum exact in f32 (the three bf16
terms of an integer x are x, 0, 0), so each product must equal the exact (float64) one bit
for bit; on random operands the result must lie within 2^-20 * sum |w_i x_i| of the float64
product, the bound every GEMV path meets.
"""
import numpy as np
import pytest

from ziglm_amd import bridge as B
from ziglm_amd import synth
from test_oracle_gemv_cpu import bound, int_matrix, random_matrix

pytestmark = pytest.mark.gpu

MB_TYPES = [B.Q4_0, B.Q8_0, B.BF16]


def gemm(dev, qtype, raw, X, rows, cols, batch, x_offset=0):
    d_w = dev.from_numpy(np.ascontiguousarray(raw).reshape(-1))
    flat = np.ascontiguousarray(X, np.float32).reshape(-1)
    if x_offset:
        d_xb = dev.alloc(flat.nbytes + 16)
        d_xb.at(x_offset).upload(flat)
        d_x = d_xb.at(x_offset)
    else:
        d_x = dev.from_numpy(flat)
    d_y = dev.alloc(batch * rows * 4)
    d_y.fill(0xAB)
    dev.gemm(qtype, d_w, d_x, d_y, batch, rows, cols)
    return d_y.to_numpy((batch, rows), np.float32)


@pytest.mark.parametrize("qtype", MB_TYPES)
@pytest.mark.parametrize("rows,cols,batch", [
    (10240, 2560, 8),   # 4 tiles per wave, 8 waves per workgroup
    (2560, 10240, 8),   # rows too long for 16 waves of 10 blocks: the vector kernels below 12 tokens,
    (2500, 10240, 40), (130, 6144, 20), (2560, 10240, 12),  # two halves added into y from 12
    (4096, 2560, 2), (1000, 2560, 16), (37, 2560, 17), (300, 1536, 31), (19, 96, 3),
    (5, 32, 2), (64, 160, 9), (777, 4096, 24), (100, 64, 5)])
def test_mb_integer_bitexact(dev, qtype, rows, cols, batch):
    raw, wd = int_matrix(qtype, rows, cols, seed=rows + cols + batch, scale_pow=-2)
    X = np.random.default_rng(rows + batch).integers(-3, 4, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24)
    np.testing.assert_array_equal(gemm(dev, qtype, raw, X, rows, cols, batch), exact.astype(np.float32),
                                  err_msg=f"qtype={qtype} {rows}x{cols} b={batch}")


@pytest.mark.parametrize("qtype", MB_TYPES)
@pytest.mark.parametrize("rows,cols,batch", [(10240, 2560, 8), (2560, 10240, 4), (333, 2048, 31), (48, 512, 2)])
def test_mb_random_vs_f64(dev, qtype, rows, cols, batch):
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + 7 * batch)
    X = synth.normal_f32(rows + batch, "X", (batch, cols), 0, 2)
    exact = X.astype(np.float64) @ wd.T
    bd = bound(wd, X)
    got = gemm(dev, qtype, raw, X, rows, cols, batch).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))


def test_mb_wide_range_activations(dev):
    """Activations over many binades (tiny, huge, mixed signs): the three bf16 terms carry
    each x's 24 bits wherever its exponent lies."""
    rows, cols, batch = 96, 1024, 6
    raw, wd = random_matrix(B.Q8_0, rows, cols, seed=5)
    rng = np.random.default_rng(6)
    X = (rng.standard_normal((batch, cols)) * 2.0 ** rng.integers(-60, 60, (batch, cols))).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    bd = bound(wd, X)
    got = gemm(dev, B.Q8_0, raw, X, rows, cols, batch).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))


@pytest.mark.parametrize("qtype", [B.Q4_0, B.F16, B.Q4_K])
def test_mb_leaves_other_cases_to_the_vector_kernels(dev, qtype):
    """x not 16-byte aligned (Q4_0), and types the kernel does not take: same exact results."""
    rows, cols, batch = 45, 512, 5
    raw, wd = int_matrix(qtype, rows, cols, seed=3, scale_pow=-2)
    X = np.random.default_rng(4).integers(-3, 4, (batch, cols)).astype(np.float32)
    exact = (X.astype(np.float64) @ wd.T).astype(np.float32)
    np.testing.assert_array_equal(gemm(dev, qtype, raw, X, rows, cols, batch, x_offset=4 if qtype == B.Q4_0 else 0),
                                  exact)


@pytest.mark.parametrize("qtype,rows,cols,batch", [
    (B.Q4_0, 10240, 2560, 95), (B.Q8_0, 8192, 1024, 64), (B.Q4_0, 2560, 10240, 60), (B.BF16, 4096, 1024, 127),
    (B.Q4_K, 2560, 2560, 63), (B.Q6_K, 10240, 2560, 12), (B.Q6_K, 2048, 1024, 95), (B.F16, 1024, 512, 100),
    (B.F32, 512, 512, 77), (B.Q4_K, 8192, 512, 7), (B.Q4_K, 2560, 4096, 31), (B.Q6_K, 1024, 8192, 47)])
def test_below_matrix_core_threshold_vs_f64(dev, qtype, rows, cols, batch):
    """Batches below the prefill GEMM's threshold for their type and shape (8192 rows or more
    / narrower but at least 4096 deep / the rest: Q4_0 and the dense types 96 / 64 / 128, Q4_K
    128 / 96 / 96, Q6_K 64 / 96 / 96 tokens) take the small-batch or the vector kernels: within
    2^-20 * sum |w_i x_i| of float64."""
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + 5 * batch)
    X = synth.normal_f32(rows + batch + 1, "Xt", (batch, cols), 0, 2)
    exact = X.astype(np.float64) @ wd.T
    got = gemm(dev, qtype, raw, X, rows, cols, batch).astype(np.float64)
    bd = bound(wd, X)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))


@pytest.mark.parametrize("qtype", [B.Q4_K, B.Q6_K])
@pytest.mark.parametrize("rows,cols,batch", [(10240, 2560, 8), (2560, 10240, 16), (1000, 2560, 3), (37, 2048, 31),
                                             (300, 1536, 17), (2500, 10240, 40), (64, 256, 2)])
def test_mb_kquant_integer_bitexact_and_random(dev, qtype, rows, cols, batch):
    """K-quants on the small-batch kernel. Q4_K: each 32-column block is one sub-block of a
    256-column super-block, scaled by d * sc_j with dmin * m_j * sum x subtracted (scale and min
    decoded from the 12 packed bytes); Q6_K: sc * (u - 32) per 16 columns as two exact bf16
    terms, d per super-block. Integer operands exact, random ones within the bound."""
    raw, wd = int_matrix(qtype, rows, cols, seed=rows + cols + batch, scale_pow=-2)
    X = np.random.default_rng(rows + batch).integers(-3, 4, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24)
    np.testing.assert_array_equal(gemm(dev, qtype, raw, X, rows, cols, batch), exact.astype(np.float32))
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + 3 * batch)
    X = synth.normal_f32(rows + batch + 2, "Xk", (batch, cols), 0, 2)
    exact = X.astype(np.float64) @ wd.T
    got = gemm(dev, qtype, raw, X, rows, cols, batch).astype(np.float64)
    bd = bound(wd, X)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))


@pytest.mark.parametrize("rows,cols,batch", [(130, 512, 9), (77, 1024, 20)])
def test_mb_q6_k_full_scale_range_exact(dev, rows, cols, batch):
    """Q6_K int8 scales over their whole range (|sc * (u - 32)| up to 4096): both bf16 terms
    carry it exactly, integer products bit for bit."""
    from test_gpu_gemm import q6_k_full_scales
    raw, wd = q6_k_full_scales(np.random.default_rng(rows + batch), rows, cols, 0.5)
    X = np.random.default_rng(batch).integers(-1, 2, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24) and np.max(np.abs(wd)) > 1000
    np.testing.assert_array_equal(gemm(dev, B.Q6_K, raw, X, rows, cols, batch), exact.astype(np.float32))
