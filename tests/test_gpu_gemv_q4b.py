"""The batch-1 block kernel (gemv.hip k_gemv_q4b, Q4_0 and Q8_0) over its selection rules, through the
C-ABI: every column count it takes (multiples of 256 up to 12288 columns: 8 to 384 blocks
per row, so 8, 16, 32 or 64 lanes per row and 1 to 6 blocks per lane), row counts that leave the
last row set partly empty, enough rows for two rows per set, the fused GeGLU and QKV forms and
the 20-byte block windows at both ends of a row (first block even, last block odd).

Integer-valued weights and activations make every partial sum exact in f32, so each product
must equal the exact (float64) dot product bit for bit whatever the lane / wave order; the
fused GeGLU must equal the elementwise GeGLU kernel (the same gelu_fast) applied to the two
plain products, bit for bit; QKV must equal three plain products.
"""
import numpy as np
import pytest

from test_oracle_gemv_cpu import bound, int_matrix, random_matrix
from ziglm_amd import bridge as B
from ziglm_amd import synth

pytestmark = pytest.mark.gpu

COLS = [256, 512, 768, 1024, 1280, 1536, 2048, 2560, 3072, 4096, 5120, 6144, 10240, 12288]


def int_x(seed, cols):
    return np.random.default_rng(seed).integers(-3, 4, cols).astype(np.float32)


def gemv(dev, raw, x, rows, cols, qtype=B.Q4_0):
    d_y = dev.alloc(rows * 4)
    d_y.fill(0xAB)
    dev.gemv(qtype, dev.from_numpy(np.ascontiguousarray(raw).reshape(-1)), dev.from_numpy(x), d_y, rows, cols)
    return d_y.to_numpy((rows,), np.float32)


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0])
@pytest.mark.parametrize("cols", COLS)
@pytest.mark.parametrize("rows", [1, 37, 4099])
def test_q4b_integer_bitexact(dev, qtype, rows, cols):
    raw, wd = int_matrix(qtype, rows, cols, seed=rows + cols + qtype, scale_pow=-1)
    x = int_x(cols, cols)
    exact = wd @ x.astype(np.float64)
    assert np.all(np.abs(exact) < 2 ** 24)
    np.testing.assert_array_equal(gemv(dev, raw, x, rows, cols, qtype), exact.astype(np.float32),
                                  err_msg=f"qtype {qtype} {rows} x {cols}")


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0])
@pytest.mark.parametrize("rows,cols", [(40000, 2560), (33001, 512), (16389, 5120)])
def test_q4b_two_rows_per_set(dev, qtype, rows, cols):
    """Row counts that take two rows per row set (the LM-head shape class), ragged at the end."""
    raw, wd = int_matrix(qtype, rows, cols, seed=rows + qtype, scale_pow=-2)
    x = int_x(rows, cols)
    exact = wd @ x.astype(np.float64)
    np.testing.assert_array_equal(gemv(dev, raw, x, rows, cols, qtype), exact.astype(np.float32),
                                  err_msg=f"qtype {qtype} {rows} x {cols}")


@pytest.mark.parametrize("rows,cols", [(77, 1536), (5003, 2560), (300, 6144), (64, 10240), (1536, 256)])
def test_q4b_geglu_equals_unfused(dev, rows, cols):
    gw, _ = int_matrix(B.Q4_0, rows, cols, seed=1 + rows, scale_pow=-3)
    uw, _ = int_matrix(B.Q4_0, rows, cols, seed=2 + rows, scale_pow=-3)
    x = int_x(3 + cols, cols)
    d_x = dev.from_numpy(x)
    d_g, d_u = dev.from_numpy(gw.reshape(-1)), dev.from_numpy(uw.reshape(-1))
    d_o = dev.alloc(rows * 4)
    dev.gemvGegluQ4_0(d_g, d_u, d_x, d_o, rows, cols)
    g, u = dev.alloc(rows * 4), dev.alloc(rows * 4)
    dev.gemv(B.Q4_0, d_g, d_x, g, rows, cols)
    dev.gemv(B.Q4_0, d_u, d_x, u, rows, cols)
    ref = dev.alloc(rows * 4)
    dev.geglu(g, u, ref, rows)
    np.testing.assert_array_equal(d_o.to_numpy((rows,), np.float32), ref.to_numpy((rows,), np.float32))


@pytest.mark.parametrize("q_rows,k_rows,v_rows,cols", [(2048, 1024, 1024, 2560), (21, 3, 5, 1536),
                                                       (8, 8, 8, 512), (4096, 512, 512, 3072)])
def test_q4b_qkv_segments(dev, q_rows, k_rows, v_rows, cols):
    """Row sets that straddle the Q / K / V boundaries read each row from its own matrix."""
    mats = [int_matrix(B.Q4_0, r, cols, seed=40 + i + r, scale_pow=-1) for i, r in enumerate((q_rows, k_rows, v_rows))]
    x = int_x(41, cols)
    d_x = dev.from_numpy(x)
    d_w = [dev.from_numpy(np.ascontiguousarray(m[0]).reshape(-1)) for m in mats]
    d_o = [dev.alloc(m[0].shape[0] * 4) for m in mats]
    dev.gemvQkvQ4_0(d_w[0], d_w[1], d_w[2], d_x, d_o[0], d_o[1], d_o[2], q_rows, k_rows, v_rows, cols)
    for i, (raw, wd) in enumerate(mats):
        exact = wd @ x.astype(np.float64)
        np.testing.assert_array_equal(d_o[i].to_numpy((raw.shape[0],), np.float32), exact.astype(np.float32),
                                      err_msg=f"matrix {i}")


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0])
@pytest.mark.parametrize("rows,cols", [(300, 2560), (4096, 10240), (2000, 3072)])
def test_q4b_random_vs_f64(dev, qtype, rows, cols):
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + 7)
    x = synth.normal_f32(rows, "x", (cols,), 0, 2)
    exact = wd @ x.astype(np.float64)
    got = gemv(dev, raw, x, rows, cols, qtype).astype(np.float64)
    bd = bound(wd, x)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0])
def test_q4b_two_byte_aligned_weights_take_the_group_kernel(dev, qtype):
    """Block rows are only 2-byte aligned in GGUF files; a matrix whose base is not 4-byte
    aligned is left to the group-wise kernel (16-bit loads) and is as exact."""
    rows, cols = 37, 2560
    raw, wd = int_matrix(qtype, rows, cols, seed=5 + qtype, scale_pow=-1)
    x = int_x(6, cols)
    d_w = dev.alloc(raw.nbytes + 16)
    d_w.at(2).upload(np.ascontiguousarray(raw).reshape(-1))
    d_y = dev.alloc(rows * 4)
    dev.gemv(qtype, d_w.at(2), dev.from_numpy(x), d_y, rows, cols)
    np.testing.assert_array_equal(d_y.to_numpy((rows,), np.float32), (wd @ x.astype(np.float64)).astype(np.float32))
