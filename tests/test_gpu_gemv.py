"""GEMV / small-batch GEMM on the GPU against the oracle (math.zig:25-330, 440-616, 652-846).
Shapes include LM-head-sized row counts (>= 65536 rows: the wave-owned-rows kernel), with
one, two and three column steps per lane and a last step that only some lanes fill.

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
from tol import assert_bitexact, assert_rel

pytestmark = pytest.mark.gpu

QTYPES = [B.Q4_0, B.Q8_0, B.Q4_K, B.Q6_K, B.BF16, B.F16, B.F32]
K_QUANTS = (B.Q4_K, B.Q6_K)


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


_INT_SHAPES = [(37, 2560, 1), (16, 96, 1), (9, 10240, 1), (11, 512, 2), (13, 2560, 3), (6, 256, 7),
               (65601, 256, 1), (65601, 768, 1), (65537, 1280, 1)]


# super-block types take whole 256-column super-blocks (the 96-column shape is for the others)
@pytest.mark.parametrize("qtype,rows,cols,batch", [(q, *sh) for q in QTYPES for sh in _INT_SHAPES
                                                   if q not in K_QUANTS or sh[1] % 256 == 0])
def test_gemv_integer_bitexact(dev, qtype, rows, cols, batch):
    raw, wd = int_matrix(qtype, rows, cols, seed=rows * cols + qtype, scale_pow=-1)
    X = np.random.default_rng(rows).integers(-3, 4, (batch, cols)).astype(np.float32)
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(exact) < 2 ** 24)
    got = run_gemm(dev, qtype, raw, X, rows, cols, batch)
    np.testing.assert_array_equal(got, exact.astype(np.float32), err_msg=f"qtype={qtype} {rows}x{cols} b={batch}")


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("rows,cols,batch", [(64, 2560, 1), (40, 10240, 1), (24, 2560, 4), (7, 1024, 5),
                                             (65540, 512, 1)])
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
    # K-quant reference-ABI mirrors (cuda_bridge.h:38-39) equal the qtype dispatch
    d_xk = dev.from_numpy(x)
    for qt, fn in ((B.Q4_K, dev.b.hip_gemv_q4_k), (B.Q6_K, dev.b.hip_gemv_q6_k)):
        rawk, _ = random_matrix(qt, rows, cols, seed=6)
        d_wk = dev.from_numpy(rawk.reshape(-1))
        fn(d_wk.ptr, d_xk.ptr, d_y.ptr, rows, cols, dev.stream)
        y_m = d_y.to_numpy((rows,), np.float32)
        dev.gemv(qt, d_wk, d_xk, d_y, rows, cols)
        np.testing.assert_array_equal(y_m, d_y.to_numpy((rows,), np.float32))
    # K-quant rows below their load alignment (Q4_K: 4 bytes, Q6_K: 2 bytes): scalar kernel
    for qt, off in ((B.Q4_K, 2), (B.Q6_K, 1)):
        rawk, wdk = random_matrix(qt, rows, cols, seed=5)
        d_wk = dev.alloc(rawk.nbytes + 16)
        d_wk.at(off).upload(rawk.reshape(-1))
        dev.gemv(qt, d_wk.at(off), d_xk, d_y, rows, cols)
        assert np.all(np.abs(d_y.to_numpy((rows,), np.float32) - wdk @ x.astype(np.float64)) <= bound(wdk, x)), qt


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


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0])
@pytest.mark.parametrize("rows,cols", [(77, 256), (1001, 2560), (10240, 2560), (333, 4096), (65, 12288),
                                       (20001, 512), (6144, 1536)])
def test_gemv_geglu_pairs_bitexact(dev, qtype, rows, cols):
    """The fused gate.up product (pairs over two row sets of a wave where its lanes per row
    leave several sets; both rows in every lane at 64 lanes per row) equals gelu(g) * u of
    the two single products bit for bit on integer operands (every sum exact in f32)."""
    gw, _ = int_matrix(qtype, rows, cols, seed=rows + 1, scale_pow=-3)
    uw, _ = int_matrix(qtype, rows, cols, seed=rows + 2, scale_pow=-3)
    x = np.random.default_rng(cols).integers(-3, 4, cols).astype(np.float32)
    d_gw, d_uw, d_x = dev.from_numpy(gw.reshape(-1)), dev.from_numpy(uw.reshape(-1)), dev.from_numpy(x)
    d_act, d_g, d_u = dev.alloc(rows * 4), dev.alloc(rows * 4), dev.alloc(rows * 4)
    d_act.fill(0xAB)
    dev.gemvPro(qtype, d_gw, d_uw, d_x, d_act, rows, cols, None)
    dev.gemv(qtype, d_gw, d_x, d_g, rows, cols)
    dev.gemv(qtype, d_uw, d_x, d_u, rows, cols)
    dev.geglu(d_g, d_u, d_g, rows)
    assert_bitexact(d_act.to_numpy((rows,), np.float32), d_g.to_numpy((rows,), np.float32),
                    f"geglu pair {rows} x {cols}")


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
        dev.gemv(13, d_w, d_x, d_y, 4, 256)  # Q5_K: not supported here
        assert dev.b.last_error() == B.EUNSUPPORTED
    finally:
        dev.strict = True
    assert np.all(d_y.to_numpy((64,), np.uint8) == 0x11)


# ---------------------------------------------------------------------------------------
# Input prologue (hip_gemv_pro / hip_gemv_qkv_pro)
# ---------------------------------------------------------------------------------------

def pro_ref(oracle, x, r=None, r_w=None, r_uo=False, scale=1.0, w=None, uo=False, eps=1e-6):
    """The prologue as the reference's separate ops: x1 = (x + [norm](r)) * scale,
    v = [norm](x1); returns (x1, v, y) with y the branch term added to x."""
    x1 = x.astype(np.float32)
    y = None
    if r is not None:
        y = r if r_w is None else oracle.rms_norm(r, r_w, eps, r_uo)
        x1 = (x1 + y).astype(np.float32)
    if scale != 1.0:
        x1 = (x1 * np.float32(scale)).astype(np.float32)
    v = x1 if w is None else oracle.rms_norm(x1, w, eps, uo)
    return x1, v, y


def check_pro_outputs(got_y, wd, v, got_v=None, got_x1=None, x1=None, y=None, what=""):
    """v within 1e-5 relative (the norm kernels' bar); y = W v within twice the dot-product
    bound plus the change a 1e-5-relative v can make (1e-5 * sum |w| |v|)."""
    if got_v is not None:
        assert_rel(got_v, v, 1e-5, what=f"{what} v")
    if got_x1 is not None:
        floor = 1e-5 * np.abs(y) if y is not None else 0.0
        assert_rel(got_x1, x1, 2.0 ** -23, floor=floor, what=f"{what} x1")
    ref = wd @ v.astype(np.float64)
    tol = 2 * bound(wd, v[None])[0] + 1e-5 * (np.abs(wd) @ np.abs(v.astype(np.float64)))
    err = np.abs(np.asarray(got_y, np.float64) - ref)
    assert np.all(err <= tol), f"{what}: max err/tol {float(np.max(err / tol)):.3g}"


PRO_CASES = {
    "norm": dict(w=True, uo=True),
    "add_raw_norm": dict(r="raw", w=True, uo=True),
    "add_norm_norm": dict(r="norm", r_uo=True, w=True, uo=True, outs=True),
    "add_norm_scale": dict(r="norm", r_uo=False, scale=0.75, outs=True),
    "add_norm_norm_w": dict(r="norm", r_uo=False, w=True, uo=False, outs=True),
}


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("case", list(PRO_CASES))
@pytest.mark.parametrize("rows,cols", [(1536, 2048), (37, 1536), (300, 256), (64, 6144)])
def test_gemv_prologue_norm(dev, oracle, qtype, case, rows, cols):
    """Input widths up to 4096 take the register prologue, 6144 the looping one."""
    c = PRO_CASES[case]
    raw, wd = random_matrix(qtype, rows, cols, seed=rows + cols)
    x = synth.normal_f32(51, "x", (cols,), 0, 3.0)
    r = synth.normal_f32(51, "r", (cols,), 0, 0.5) if "r" in c else None
    r_w = synth.normal_f32(51, "rw", (cols,), 0, 0.1) if c.get("r") == "norm" else None
    w = synth.normal_f32(51, "w", (cols,), 0, 0.1) if c.get("w") else None
    x1, v, y = pro_ref(oracle, x, r, r_w, c.get("r_uo", False), c.get("scale", 1.0), w, c.get("uo", False))
    d = {k: (dev.from_numpy(a) if a is not None else None) for k, a in dict(x=x, r=r, r_w=r_w, w=w).items()}
    d_y, d_x1, d_v, d_w = dev.alloc(rows * 4), dev.alloc(cols * 4), dev.alloc(cols * 4), dev.from_numpy(raw.reshape(-1))
    outs = c.get("outs", False)
    pro = dev.prologue(B.PRO_NORM, r=d["r"], r_weight=d["r_w"], r_unit_offset=c.get("r_uo", False),
                       scale=c.get("scale", 1.0), x_out=d_x1 if outs else None, weight=d["w"],
                       unit_offset=c.get("uo", False), eps=1e-6, xb_out=d_v if outs else None)
    dev.gemvPro(qtype, d_w, None, d["x"], d_y, rows, cols, pro)
    got_y = d_y.to_numpy((rows,), np.float32)
    if outs:
        check_pro_outputs(got_y, wd, v, d_v.to_numpy((cols,), np.float32), d_x1.to_numpy((cols,), np.float32), x1,
                          y, what=case)
    else:
        check_pro_outputs(got_y, wd, v, what=case)


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0, B.F32])
@pytest.mark.parametrize("rows,cols", [(1536, 256), (96, 6144)])
def test_gemv_prologue_geglu_input(dev, oracle, qtype, rows, cols):
    """v = gelu(x) * r (the per-layer-embedding projection's input), register and looping
    prologues."""
    raw, wd = random_matrix(qtype, rows, cols, seed=77)
    g = synth.normal_f32(52, "g", (cols,), 0, 2.0)
    u = synth.normal_f32(52, "u", (cols,))
    v = oracle.geglu(g, u)
    d_y, d_v, d_u, d_g, d_w = dev.alloc(rows * 4), dev.alloc(cols * 4), dev.from_numpy(u), dev.from_numpy(g), \
        dev.from_numpy(raw.reshape(-1))
    pro = dev.prologue(B.PRO_GEGLU, r=d_u, xb_out=d_v)
    dev.gemvPro(qtype, d_w, None, d_g, d_y, rows, cols, pro)
    got_v = d_v.to_numpy((cols,), np.float32)
    assert_rel(got_v, v, 1e-5, floor=np.abs(g.astype(np.float64) * u) * 2.0 ** -23, what="gelu(x)*r")
    check_pro_outputs(d_y.to_numpy((rows,), np.float32), wd, v, what="geglu input")


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0, B.BF16])
def test_gemv_prologue_geglu_matrices_and_qkv(dev, oracle, qtype):
    """GeGLU pair and Q/K/V segments with a prologue: the same per-row arithmetic as the
    single-matrix form over the same input (QKV bit for bit; GeGLU against gelu(g) * u of
    the two single products, which it computes from the same sums)."""
    cols, I = 1536, 1024
    x = synth.normal_f32(53, "x", (cols,))
    r = synth.normal_f32(53, "r", (cols,))
    rw = synth.normal_f32(53, "rw", (cols,), 0, 0.1)
    w = synth.normal_f32(53, "w", (cols,), 0, 0.1)
    d_x, d_r, d_rw, d_w = (dev.from_numpy(a) for a in (x, r, rw, w))
    pro = dev.prologue(B.PRO_NORM, r=d_r, r_weight=d_rw, r_unit_offset=True, weight=d_w, unit_offset=True)
    mats = [random_matrix(qtype, n, cols, seed=90 + n) for n in (2048, 512, 512)]
    d_m = [dev.from_numpy(m[0].reshape(-1)) for m in mats]
    outs = [dev.alloc(n * 4) for n in (2048, 512, 512)]
    dev.gemvQkvPro(qtype, *d_m, d_x, *outs, 2048, 512, 512, cols, pro)
    for (raw, wd), dm, o, n in zip(mats, d_m, outs, (2048, 512, 512)):
        single = dev.alloc(n * 4)
        dev.gemvPro(qtype, dm, None, d_x, single, n, cols, pro)
        assert_bitexact(o.to_numpy((n,), np.float32), single.to_numpy((n,), np.float32), "qkv segment")
    _, v, _ = pro_ref(oracle, x, r, rw, True, 1.0, w, True)
    check_pro_outputs(outs[0].to_numpy((2048,), np.float32), mats[0][1], v, what="qkv q")
    gm, um = random_matrix(qtype, I, cols, seed=5), random_matrix(qtype, I, cols, seed=6)
    d_act, d_g, d_u = dev.alloc(I * 4), dev.alloc(I * 4), dev.alloc(I * 4)
    d_gm, d_um = dev.from_numpy(gm[0].reshape(-1)), dev.from_numpy(um[0].reshape(-1))
    dev.gemvPro(qtype, d_gm, d_um, d_x, d_act, I, cols, pro)
    dev.gemvPro(qtype, d_gm, None, d_x, d_g, I, cols, pro)
    dev.gemvPro(qtype, d_um, None, d_x, d_u, I, cols, pro)
    gg, uu = d_g.to_numpy((I,), np.float32), d_u.to_numpy((I,), np.float32)
    dev.geglu(d_g, d_u, d_g, I)
    assert_bitexact(d_act.to_numpy((I,), np.float32), d_g.to_numpy((I,), np.float32), "geglu pair")
    check_pro_outputs(gg, gm[1], v, what="gate")
    check_pro_outputs(uu, um[1], v, what="up")


def test_gemv_prologue_rejects(dev):
    w = dev.alloc(18 * 1024)
    x = dev.alloc(4 * 20000)
    y = dev.alloc(4 * 64)
    y.fill(0x33)
    dev.strict = False
    try:
        pro = dev.prologue(B.PRO_NORM, weight=x)
        dev.gemvPro(B.Q4_0, w, None, x, y, 1, 16416, pro)                     # input beyond LDS
        assert dev.b.last_error() == B.EUNSUPPORTED
        dev.gemvPro(B.Q4_0, w, None, x, y, 4, 256, dev.prologue(B.PRO_NORM, weight=x, x_out=y.at(4)))  # misaligned
        assert dev.b.last_error() == B.EUNSUPPORTED
        dev.gemvPro(B.Q4_0, w, None, x, y, 4, 256, dev.prologue(B.PRO_GEGLU))    # GEGLU needs r
        assert dev.b.last_error() == B.EINVAL
        dev.gemvPro(B.Q4_0, w, None, x, y, 4, 256, dev.prologue(B.PRO_NORM, r_weight=x))  # r weight without r
        assert dev.b.last_error() == B.EINVAL
    finally:
        dev.strict = True
    assert np.all(y.to_numpy((256,), np.uint8) == 0x33)
