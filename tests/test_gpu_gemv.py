"""GEMV / small-batch GEMM on the GPU against the oracle (math.zig:25-330, 652-846).

The kernels sum in a different order from ziglm's CPU code, so the checks are
  * bit-exact on integer-valued inputs (every partial sum is exact in f32, so any order
    gives the exact integer dot product): indexing, nibble order, offsets, scales, tails;
  * on random inputs, both the GPU result and the oracle's lie within
    2^-20 * sum |w_i x_i| of the exact (float64) dot product of the dequantised row.
Fused forms: QKV must equal three separate GEMVs bit for bit (same per-row arithmetic);
GeGLU is gelu(g) * u of the two products, checked against float64 with the propagated
bound of the two dot products plus the GELU's own 1e-5 relative / |x*up|*2^-23 floor.
"""
import numpy as np
import pytest

from oracle import oracle as O
from ziglm_amd import bridge as B
from ziglm_amd import synth
from test_oracle_gemv_cpu import bound, int_matrix, random_matrix

pytestmark = pytest.mark.gpu

QTYPES = [B.Q4_0, B.Q8_0, B.BF16, B.F16, B.F32]


def run_gemm(dev, qtype, raw, X, rows, cols, batch):
    d_w = dev.from_numpy(np.ascontiguousarray(raw).reshape(-1))
    d_x = dev.from_numpy(np.ascontiguousarray(X, np.float32).reshape(-1))
    d_y = dev.alloc(batch * rows * 4)
    d_y.fill(0xAB)
    if batch == 1:
        dev.gemv(qtype, d_w, d_x, d_y, rows, cols)
    else:
        dev.gemm(qtype, d_w, d_x, d_y, batch, rows, cols)
    return d_y.to_numpy((batch, rows), np.float32)


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("rows,cols,batch", [(37, 2560, 1), (16, 96, 1), (9, 10240, 1), (11, 512, 2),
                                             (13, 2560, 3), (6, 256, 7)])
def test_gemv_integer_bitexact(dev, qtype, rows, cols, batch):
    raw, wd = int_matrix(qtype, rows, cols, seed=rows * cols + qtype, scale_pow=-1)
    X = np.random.default_rng(rows).integers(-3, 4, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24)
    got = run_gemm(dev, qtype, raw, X, rows, cols, batch)
    np.testing.assert_array_equal(got, exact.astype(np.float32), err_msg=f"qtype={qtype} {rows}x{cols} b={batch}")


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("rows,cols,batch", [(64, 2560, 1), (40, 10240, 1), (24, 2560, 4), (7, 1024, 5)])
def test_gemv_vs_f64(dev, oracle, qtype, rows, cols, batch):
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + cols)
    X = synth.normal_f32(rows, "X", (batch, cols))
    exact = X.astype(np.float64) @ wd.T
    bd = bound(wd, X)
    got = run_gemm(dev, qtype, raw, X, rows, cols, batch).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bd), float(np.max(np.abs(got - exact) / bd))
    ref = oracle.gemm(qtype, raw, X).astype(np.float64)
    assert np.all(np.abs(ref - exact) <= bd)


def test_gemv_mirrors_and_misaligned_paths(dev, oracle):
    rows, cols = 20, 2560
    raw, wd = random_matrix(B.Q4_0, rows, cols, seed=3)
    x = synth.normal_f32(3, "x", (cols,))
    exact, bd = wd @ x.astype(np.float64), bound(wd, x)
    d_w, d_x = dev.from_numpy(raw.reshape(-1)), dev.from_numpy(x)
    d_y = dev.alloc(rows * 4)
    dev.b.hip_gemv_q4_0(d_w.ptr, d_x.ptr, d_y.ptr, rows, cols, dev.stream)
    y1 = d_y.to_numpy((rows,), np.float32)
    dev.gemmQ4_0(d_w, d_x, d_y, 1, rows, cols)
    np.testing.assert_array_equal(d_y.to_numpy((rows,), np.float32), y1)
    assert np.all(np.abs(y1 - exact) <= bd)
    # x at a 4-byte offset: the per-row scalar kernel
    d_x2 = dev.alloc(cols * 4 + 16)
    d_x2.at(4).upload(x)
    dev.gemv(B.Q4_0, d_w, d_x2.at(4), d_y, rows, cols)
    assert np.all(np.abs(d_y.to_numpy((rows,), np.float32) - exact) <= bd)
    # bf16 weights at a 2-byte offset: scalar kernel
    rawb, wdb = random_matrix(B.BF16, rows, 1000, seed=4)
    xb = synth.normal_f32(4, "x", (1000,))
    d_wb = dev.alloc(rawb.nbytes + 16)
    d_wb.at(2).upload(rawb.reshape(-1))
    dev.gemv(B.BF16, d_wb.at(2), dev.from_numpy(xb), d_y, rows, 1000)
    assert np.all(np.abs(d_y.to_numpy((rows,), np.float32) - wdb @ xb.astype(np.float64)) <= bound(wdb, xb))


@pytest.mark.parametrize("q_rows,k_rows,v_rows", [(2048, 1024, 1024), (13, 0, 6), (0, 5, 3)])
def test_gemv_qkv_equals_three_gemvs(dev, q_rows, k_rows, v_rows):
    cols = 2560
    mats = [random_matrix(B.Q4_0, max(r, 1), cols, seed=20 + i)[0][:r] for i, r in enumerate((q_rows, k_rows, v_rows))]
    x = synth.normal_f32(20, "x", (cols,))
    d_x = dev.from_numpy(x)
    d_w = [dev.from_numpy(np.ascontiguousarray(m).reshape(-1)) if m.shape[0] else None for m in mats]
    d_o = [dev.alloc(max(m.shape[0], 1) * 4) for m in mats]
    dev.gemvQkvQ4_0(d_w[0], d_w[1], d_w[2], d_x, d_o[0], d_o[1], d_o[2], q_rows, k_rows, v_rows, cols)
    fused = [d.to_numpy((max(m.shape[0], 1),), np.float32)[: m.shape[0]] for d, m in zip(d_o, mats)]
    for i, m in enumerate(mats):
        if m.shape[0] == 0:
            continue
        d_y = dev.alloc(m.shape[0] * 4)
        dev.gemv(B.Q4_0, d_w[i], d_x, d_y, m.shape[0], cols)
        np.testing.assert_array_equal(fused[i], d_y.to_numpy((m.shape[0],), np.float32), err_msg=f"matrix {i}")


@pytest.mark.parametrize("rows", [10240, 77])
def test_gemv_geglu_q4_0(dev, oracle, rows):
    cols = 2560
    gw, gd = random_matrix(B.Q4_0, rows, cols, seed=30)
    uw, ud = random_matrix(B.Q4_0, rows, cols, seed=31)
    x = synth.normal_f32(30, "x", (cols,))
    d_o = dev.alloc(rows * 4)
    dev.gemvGegluQ4_0(dev.from_numpy(gw.reshape(-1)), dev.from_numpy(uw.reshape(-1)), dev.from_numpy(x), d_o,
                      rows, cols)
    got = d_o.to_numpy((rows,), np.float32).astype(np.float64)
    g, u = gd @ x.astype(np.float64), ud @ x.astype(np.float64)
    bg, bu = bound(gd, x), bound(ud, x)
    gelu = 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3)))
    exact = gelu * u
    # |d gelu/dg| <= 1.13; GELU/product rounding: 1e-5 relative plus the 1+tanh cancellation
    tol = 1.13 * bg * np.abs(u) + np.abs(gelu) * bu + bg * bu + 1e-5 * np.abs(exact) + np.abs(g * u) * 2.0 ** -23
    assert np.all(np.abs(got - exact) <= tol), float(np.max(np.abs(got - exact) / tol))
    # and the oracle's CPU composition (gemv, gemv, geglu) within the same bound
    ref = oracle.geglu(oracle.gemv(O.Q4_0, gw, x), oracle.gemv(O.Q4_0, uw, x)).astype(np.float64)
    assert np.all(np.abs(ref - exact) <= tol)


def test_gemv_unsupported_qtype_is_noop(dev):
    d_w, d_x, d_y = dev.alloc(4096), dev.alloc(1024), dev.alloc(64)
    d_y.fill(0x11)
    dev.strict = False
    try:
        dev.gemv(12, d_w, d_x, d_y, 4, 256)  # Q4_K: not supported here
        assert dev.b.last_error() == B.EUNSUPPORTED
    finally:
        dev.strict = True
    assert np.all(d_y.to_numpy((64,), np.uint8) == 0x11)
