"""Prefill-sized GEMM on the matrix cores (hip_gemm with batch >= 32: gemm.hip) against
float64 and the oracle's math.gemm (math.zig:440-616), through the C-ABI.

The activations are split into three bf16 terms and the weights into one (Q4_0, Q8_0, BF16),
two (F16) or three (F32) exact bf16 terms, so
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
# x 2048 tokens), else 64 x 128 from 512 (4096 x 1024), else 64 x 64.
@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("rows,cols,batch", [(128, 64, 32), (200, 96, 37), (129, 2560, 128), (77, 160, 300),
                                             (256, 512, 64), (4096, 96, 2048), (4100, 64, 2050),
                                             (4096, 64, 1024), (4097, 96, 1000)])
def test_gemm_mfma_integer_bitexact(dev, qtype, rows, cols, batch):
    raw, wd = int_matrix(qtype, rows, cols, seed=rows * cols + qtype + batch, scale_pow=-1)
    X = np.random.default_rng(batch).integers(-3, 4, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24)
    got = run(dev, qtype, raw, X, rows, cols)
    np.testing.assert_array_equal(got, exact.astype(np.float32), err_msg=f"qtype={qtype} {rows}x{cols} b={batch}")


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("rows,cols,batch", [(256, 2560, 128), (300, 1024, 77), (1024, 2560, 512),
                                             (128, 10240, 64), (4096, 512, 2048), (4096, 1024, 1024)])
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
