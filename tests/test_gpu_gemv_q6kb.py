"""The batch-1 Q6_K quarter-chunk kernel (gemv.hip k_gemv_q6kb) over its selection rules,
through the C-ABI: every column count it takes (multiples of 512 up to 12288: 8 to 192
quarters of 64 columns per row, so 8, 16, 32 or 64 lanes per row and 1 to 6 quarters per
lane), row counts that leave the last row set partly empty, LM-head-sized row counts, the
fused QKV form (row sets across the Q / K / V boundaries), the norm prologue, a matrix that
starts 2 bytes past a dword (every super-block then starts off a dword), and the shapes it
leaves to the group kernels (256-column multiples that 512 does not divide).

Integer-valued weights (6-bit codes, signed int8 scales, power-of-two d) and integer
activations make every partial sum exact in f32, so each product must equal the exact
(float64) dot product bit for bit whatever the lane / wave order; on random operands the
result must lie within 2^-20 * sum |w_i x_i| of the float64 product, the bound every GEMV
path meets.
"""
import numpy as np
import pytest

from test_oracle_gemv_cpu import bound, int_matrix, random_matrix
from ziglm_amd import bridge as B
from ziglm_amd import synth

pytestmark = pytest.mark.gpu

COLS = [512, 1024, 1536, 2048, 2560, 3072, 4096, 5120, 6144, 10240, 12288]


def int_x(seed, cols):
    return np.random.default_rng(seed).integers(-3, 4, cols).astype(np.float32)


def gemv(dev, raw, x, rows, cols, offset=0):
    d_y = dev.alloc(rows * 4)
    d_y.fill(0xAB)
    flat = np.ascontiguousarray(raw).reshape(-1)
    if offset:
        d_w = dev.alloc(flat.nbytes + 16)
        d_w.at(offset).upload(flat)
        w = d_w.at(offset)
    else:
        w = dev.from_numpy(flat)
    dev.gemv(B.Q6_K, w, dev.from_numpy(x), d_y, rows, cols)
    return d_y.to_numpy((rows,), np.float32)


@pytest.mark.parametrize("cols", COLS + [768, 1280])  # (768, 1280: the group kernels)
@pytest.mark.parametrize("rows", [1, 37, 4099])
def test_q6kb_integer_bitexact(dev, rows, cols):
    raw, wd = int_matrix(B.Q6_K, rows, cols, seed=rows + cols, scale_pow=-3)
    x = int_x(cols, cols)
    exact = wd @ x.astype(np.float64)
    assert np.all(np.abs(exact) < 2 ** 24)
    np.testing.assert_array_equal(gemv(dev, raw, x, rows, cols), exact.astype(np.float32),
                                  err_msg=f"{rows} x {cols}")


@pytest.mark.parametrize("rows,cols", [(65601, 2560), (33001, 512), (16389, 5120)])
def test_q6kb_lm_head_sized(dev, rows, cols):
    raw, wd = int_matrix(B.Q6_K, rows, cols, seed=rows, scale_pow=-4)
    x = int_x(rows, cols)
    exact = wd @ x.astype(np.float64)
    np.testing.assert_array_equal(gemv(dev, raw, x, rows, cols), exact.astype(np.float32),
                                  err_msg=f"{rows} x {cols}")


@pytest.mark.parametrize("rows,cols", [(300, 2560), (4096, 10240), (2000, 3072), (20000, 2560)])
def test_q6kb_random_vs_f64(dev, rows, cols):
    raw, wd = random_matrix(B.Q6_K, rows, cols, seed=rows + 13)
    x = synth.normal_f32(rows, "x", (cols,), 0, 2)
    got = gemv(dev, raw, x, rows, cols).astype(np.float64)
    exact = wd @ x.astype(np.float64)
    bd = bound(wd, x)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))


@pytest.mark.parametrize("rows,cols", [(37, 2560), (1001, 1024)])
def test_q6kb_matrix_off_a_dword(dev, rows, cols):
    """A matrix 2 bytes past a dword: even super-blocks then start off a dword too."""
    raw, wd = int_matrix(B.Q6_K, rows, cols, seed=9 + rows, scale_pow=-3)
    x = int_x(10, cols)
    np.testing.assert_array_equal(gemv(dev, raw, x, rows, cols, offset=2),
                                  (wd @ x.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("q_rows,k_rows,v_rows,cols", [(2048, 1024, 1024, 2560), (21, 3, 5, 1536),
                                                       (8, 8, 8, 512), (4096, 512, 512, 3072)])
def test_q6kb_qkv_segments(dev, q_rows, k_rows, v_rows, cols):
    """Row sets that straddle the Q / K / V boundaries read each row from its own matrix."""
    mats = [int_matrix(B.Q6_K, r, cols, seed=60 + i + r, scale_pow=-3) for i, r in enumerate((q_rows, k_rows, v_rows))]
    x = int_x(61, cols)
    d_x = dev.from_numpy(x)
    d_w = [dev.from_numpy(np.ascontiguousarray(m[0]).reshape(-1)) for m in mats]
    d_o = [dev.alloc(m[0].shape[0] * 4) for m in mats]
    dev.gemvQkvPro(B.Q6_K, d_w[0], d_w[1], d_w[2], d_x, d_o[0], d_o[1], d_o[2], q_rows, k_rows, v_rows, cols, None)
    for i, (raw, wd) in enumerate(mats):
        exact = wd @ x.astype(np.float64)
        np.testing.assert_array_equal(d_o[i].to_numpy((raw.shape[0],), np.float32), exact.astype(np.float32),
                                      err_msg=f"matrix {i}")
