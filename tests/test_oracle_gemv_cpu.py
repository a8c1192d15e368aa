"""Pins the oracle's dot products, GEMV and GEMM (oracle/ziglm_oracle_gemv.c, restating
math.zig:25-330 and 652-846) before they are trusted as the checker for the HIP GEMV.

* Closed form: with integer-valued weights, activations and power-of-two block scales every
  partial sum is an integer below 2^24, so each f32 sum is exact whatever its order and the
  result must equal the exact integer dot product bit for bit. A dropped or repeated block,
  a wrong nibble order (low nibbles are elements 0..15), a missing -8 offset, a wrong sign
  or scale index, or a lost 8-element tail fails this.
* float64: random rows agree with the exact dot product of the dequantised row within
  2^-20 * sum |w_i x_i| (f32 summation error of a few thousand terms).
* Structure: gemv is dotRow per row; gemm with batch 1 is gemv; gemm with batch > 1 is the
  dequantise-then-dotF32F32 definition (math.zig:780-806).
Unpinned at the last bit: @reduce(.Add)'s lane order.
"""
import numpy as np
import pytest

from oracle import oracle as O
from ziglm_amd import synth

QTYPES = [O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K, O.BF16, O.F16, O.F32]


@pytest.fixture(scope="module")
def o():
    return O.get()


def f16_bytes(v):
    """Little-endian bytes of the f16 value v."""
    return np.array([v], np.float16).view(np.uint8)


def int_matrix(qtype, rows, cols, seed, scale_pow=0):
    """Integer-valued weights in `qtype` layout, their exact float64 values, and scale 2^p."""
    rng = np.random.default_rng(seed)
    d = np.float64(2.0 ** scale_pow)
    if qtype == O.Q8_0:
        q = rng.integers(-127, 128, (rows, cols))
        raw = np.zeros((rows, cols // 32, 34), np.uint8)
        raw[:, :, 0:2] = f16_bytes(d)
        raw[:, :, 2:] = q.reshape(rows, cols // 32, 32).astype(np.int8).view(np.uint8)
        return raw.reshape(rows, -1), q * d
    if qtype == O.Q4_0:
        q = rng.integers(0, 16, (rows, cols))
        qb = q.reshape(rows, cols // 32, 32)
        raw = np.zeros((rows, cols // 32, 18), np.uint8)
        raw[:, :, 0:2] = f16_bytes(d)
        raw[:, :, 2:] = (qb[:, :, :16] | (qb[:, :, 16:] << 4)).astype(np.uint8)
        return raw.reshape(rows, -1), (q - 8) * d
    if qtype == O.Q4_K:
        return q4_k_encode(rng, rows, cols, d)
    if qtype == O.Q6_K:
        return q6_k_encode(rng, rows, cols, d)
    w = rng.integers(-100, 101, (rows, cols)).astype(np.float64) * d
    if qtype == O.F32:
        return w.astype(np.float32).view(np.uint8).reshape(rows, -1), w
    if qtype == O.F16:
        return w.astype(np.float16).view(np.uint8).reshape(rows, -1), w
    bits = (w.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)  # exact: small ints
    return bits.view(np.uint8).reshape(rows, -1), w


def q4_k_encode(rng, rows, cols, d):
    """Q4_K rows from intended values, packed by the GGUF format description (not by
    inverting the decoder): a 256-column super-block is {f16 d, f16 dmin, 12 scale bytes,
    128 quant bytes}; column c of a super-block belongs to 32-column sub-block j = c // 32,
    whose value is q * (d * sc_j) - dmin * m_j with 6-bit sc_j, m_j; the quant byte of c is
    qs[32 (j // 2) + c % 32], low nibble for even j, high for odd j; sc_j, m_j for j < 4 are
    the low 6 bits of bytes j and j + 4, for j >= 4 the low / high nibble of byte j + 4 with
    their top 2 bits in bits 6-7 of bytes j - 4 / j. Scales and mins are kept small so every
    integer sum stays exact in f32."""
    nsb = cols // 256
    q = rng.integers(0, 16, (rows, nsb, 8, 32))
    sc = rng.integers(0, 8, (rows, nsb, 8))
    sc[..., 4:] |= rng.integers(0, 2, (rows, nsb, 4)) << 4   # exercise the high bits of j >= 4
    sc[..., 4:] = np.minimum(sc[..., 4:], 23)
    mn = rng.integers(0, 8, (rows, nsb, 8))
    mn[..., 4:] |= rng.integers(0, 2, (rows, nsb, 4)) << 4
    mn[..., 4:] = np.minimum(mn[..., 4:], 23)
    dmin = np.float64(d) / 2
    raw = np.zeros((rows, nsb, 144), np.uint8)
    raw[..., 0:2] = f16_bytes(d)
    raw[..., 2:4] = f16_bytes(dmin)
    b = np.zeros((rows, nsb, 12), np.int64)
    for j in range(4):
        b[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        b[..., j + 4] = (mn[..., j] & 63) | ((mn[..., j + 4] >> 4) << 6)
        b[..., j + 8] = (sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)
    raw[..., 4:16] = b.astype(np.uint8)
    for jj in range(4):
        raw[..., 16 + 32 * jj:48 + 32 * jj] = (q[:, :, 2 * jj] | (q[:, :, 2 * jj + 1] << 4)).astype(np.uint8)
    val = q * (d * sc[..., None]) - dmin * mn[..., None]
    return raw.reshape(rows, -1), val.reshape(rows, cols).astype(np.float64)


def q6_k_encode(rng, rows, cols, d):
    """Q6_K rows from intended values, packed by the format description: a 256-column
    super-block is {ql[128], qh[64], int8 scales[16], f16 d}; column c has value
    d * scales[c // 16] * (u - 32), u a 6-bit code whose low 4 bits sit in ql and top 2 bits in
    qh: with h = c // 128, i = c % 128, l = i % 32 and quadrant k = i // 32, the low bits are
    nibble (k // 2) of ql[64 h + 32 (k % 2) + l] and the top bits are bits 2k, 2k + 1 of
    qh[32 h + l]."""
    nsb = cols // 256
    u = rng.integers(0, 64, (rows, nsb, 256))
    sc = rng.integers(-8, 8, (rows, nsb, 16))
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
    raw[..., 208:210] = f16_bytes(d)
    val = d * np.repeat(sc, 16, axis=-1) * (u - 32)
    return raw.reshape(rows, -1), val.reshape(rows, cols).astype(np.float64)


def random_matrix(qtype, rows, cols, seed):
    """Synthetic weights in `qtype` layout and their dequantised float64 values."""
    if qtype == O.Q8_0:
        raw = synth.q8_0_table(seed, rows, cols)
    elif qtype == O.Q4_0:
        raw = synth.q4_0_table(seed, rows, cols)
    elif qtype == O.BF16:
        raw = synth.bf16_table(seed, rows, cols)
    elif qtype == O.Q4_K:
        raw = synth.q4_k_table(seed, rows, cols)
    elif qtype == O.Q6_K:
        raw = synth.q6_k_table(seed, rows, cols)
    elif qtype == O.F16:
        raw = synth.f16_bits(synth.normal_f32(seed, "w16", (rows, cols), 0, 0.05)).view(np.uint8).reshape(rows, -1)
    else:
        raw = synth.normal_f32(seed, "w32", (rows, cols), 0, 0.05).view(np.uint8).reshape(rows, -1)
    o = O.get()
    deq = np.empty((rows, cols), np.float32)
    for r in range(rows):
        deq[r] = o.embed_gather(raw, qtype, np.array([r], np.int32), cols, np.float32(1.0))[0]
    return raw, deq.astype(np.float64)


def bound(wd, x):
    """2^-20 * sum |w_i x_i| per output (rows of wd against each x)."""
    return np.abs(x).astype(np.float64) @ np.abs(wd).T * 2.0 ** -20


def _valid_cols(qtype, cols):
    """Block types take whole 32-column blocks, super-block types whole 256-column ones."""
    if qtype in (O.Q4_0, O.Q8_0):
        return cols % 32 == 0
    if qtype in (O.Q4_K, O.Q6_K):
        return cols % 256 == 0
    return True


@pytest.mark.parametrize("qtype,cols", [(q, c) for q in QTYPES for c in (32, 64, 96, 2560, 264)
                                        if _valid_cols(q, c)])
def test_dot_integer_closed_form(o, qtype, cols):
    for p in (0, -1, 3):
        raw, wd = int_matrix(qtype, 5, cols, seed=cols + p + 100 * qtype, scale_pow=p)
        x = np.random.default_rng(cols).integers(-3, 4, cols).astype(np.float32)
        exact = wd @ x.astype(np.float64)
        assert np.all(np.abs(exact) < 2 ** 24)
        y = o.gemv(qtype, raw, x)
        np.testing.assert_array_equal(y, exact.astype(np.float32), err_msg=f"qtype={qtype} cols={cols} 2^{p}")


def test_dot_f32_tails(o):
    """dotF32F32's 32-, 8- and scalar-tail loops (n = 37 = 32 + 0*8 + 5, 45 = 32 + 8 + 5)."""
    for n in (5, 8, 37, 45, 77):
        a = np.arange(1, n + 1, dtype=np.float32)
        b = (np.arange(n, dtype=np.float32) % 7) - 3
        got = o.lib.zo_dot_f32(o.fp(a), o.fp(b), n)
        assert got == float(np.dot(a.astype(np.float64), b.astype(np.float64))), n


def test_q4_0_nibble_order_single_element(o):
    """One nonzero weight at a time: element e of block 1 is the low nibble of byte e
    (e < 16) or the high nibble of byte e - 16, offset by -8."""
    cols = 64
    x = np.arange(1, cols + 1, dtype=np.float32)
    for e in (0, 5, 15, 16, 21, 31):
        blk = np.zeros((2, 18), np.uint8)
        blk[:, 0:2] = f16_bytes(1.0)
        blk[:, 2:] = 0x88  # every nibble 8 -> weight 0
        byte = e % 16
        blk[1, 2 + byte] = 0xC8 if e >= 16 else 0x8C  # that nibble 12 -> weight 4
        y = o.dot_row(O.Q4_0, blk.reshape(-1), x)
        assert y == 4.0 * x[32 + e], (e, y)


def test_k_quant_dequant_matches_encoder(o):
    """The dequantisation (quant.zig:276-309, 357-385) returns the values the format-level
    encoders above intended, element for element (Q4_K: every scale / min byte position,
    both nibbles; Q6_K: every quadrant, both qh bit pairs, signed scales)."""
    rng = np.random.default_rng(5)
    for qt, enc in ((O.Q4_K, q4_k_encode), (O.Q6_K, q6_k_encode)):
        for d in (1.0, 0.5, 8.0):
            raw, val = enc(rng, 3, 512, d)
            for r in range(3):
                got = o.dequantize_row(qt, raw[r], 512).astype(np.float64)
                np.testing.assert_array_equal(got, val[r], err_msg=f"qtype {qt} d {d} row {r}")


def test_q8_0_sign_and_scale(o):
    cols = 64
    blk = np.zeros((2, 34), np.uint8)
    blk[0, 0:2] = f16_bytes(0.25)
    blk[1, 0:2] = f16_bytes(-2.0)
    blk[0, 2 + 3] = np.uint8(np.int8(-5).view(np.uint8))
    blk[1, 2 + 30] = 7
    x = np.arange(cols, dtype=np.float32) + 1
    assert o.dot_row(O.Q8_0, blk.reshape(-1), x) == np.float32(-5 * 0.25 * 4 + 7 * -2.0 * 63)


@pytest.mark.parametrize("qtype", QTYPES)
def test_gemv_vs_f64(o, qtype):
    rows, cols = 48, 2560
    raw, wd = random_matrix(qtype, rows, cols, seed=11)
    x = synth.normal_f32(11, "x", (cols,))
    y = o.gemv(qtype, raw, x).astype(np.float64)
    exact = wd @ x.astype(np.float64)
    assert np.all(np.abs(y - exact) <= bound(wd, x)), np.max(np.abs(y - exact) / bound(wd, x))
    for r in (0, 17, rows - 1):
        assert o.dot_row(qtype, raw[r], x) == y[r]


@pytest.mark.parametrize("qtype", QTYPES)
def test_gemm_definition(o, qtype):
    rows, cols, batch = 24, 512, 3
    raw, wd = random_matrix(qtype, rows, cols, seed=12)
    X = synth.normal_f32(12, "X", (batch, cols))
    Y = o.gemm(qtype, raw, X)
    np.testing.assert_array_equal(o.gemm(qtype, raw, X[:1])[0], o.gemv(qtype, raw, X[0]))
    exact = X.astype(np.float64) @ wd.T
    assert np.all(np.abs(Y - exact) <= bound(wd, X)), "gemm vs f64"
    # batch > 1 uses dequantise + dotF32F32 (math.zig:780-806)
    wf = wd.astype(np.float32)
    for b in range(batch):
        for r in (0, rows - 1):
            ref = o.lib.zo_dot_f32(o.fp(np.ascontiguousarray(wf[r])), o.fp(np.ascontiguousarray(X[b])), cols)
            assert Y[b, r] == np.float32(ref)


# ---------------------------------------------------------------------------------------
# Decode attention (model.zig:658-700, math.softmax math.zig:1088-1106)
# ---------------------------------------------------------------------------------------

from attn_ref import attention_f64  # noqa: E402


@pytest.mark.parametrize("nh,nkv,d", [(8, 4, 256), (4, 4, 128), (8, 2, 64)])
@pytest.mark.parametrize("softcap,window", [(0.0, 0), (50.0, 0), (0.0, 40)])
def test_attention_vs_f64(o, nh, nkv, d, softcap, window):
    rows, pos, row0 = 300, 250, 20
    kc = synth.normal_f32(7, "kc", (rows, nkv * d))
    vc = synth.normal_f32(7, "vc", (rows, nkv * d))
    q = synth.normal_f32(7, "q", (nh * d,), 0, 0.25)
    scale = float(np.float32(1.0 / np.sqrt(d)))
    got = o.attention(q, kc, vc, row0, pos, nh, nkv, d, scale, softcap, window).astype(np.float64)
    ref, tol = attention_f64(q, kc, vc, row0, pos, nh, nkv, d, scale, softcap, window)
    assert np.all(np.abs(got - ref) <= tol), float(np.max(np.abs(got - ref) / tol))


def test_attention_closed_forms(o):
    nh, nkv, d = 8, 4, 128
    kc = synth.normal_f32(8, "kc", (64, nkv * d))
    vc = synth.normal_f32(8, "vc", (64, nkv * d))
    q = synth.normal_f32(8, "q", (nh * d,))
    # one position (pos 0, or a window of 1): weight exactly 1, out = v of that position
    for pos, window in ((0, 0), (37, 1)):
        out = o.attention(q, kc, vc, 0, pos, nh, nkv, d, 0.1, 0.0, window).reshape(nh, d)
        for h in range(nh):
            np.testing.assert_array_equal(out[h], vc[pos, (h // 2) * d:(h // 2 + 1) * d])
    # q = 0: equal scores, out = the mean of v over [0, pos]
    out = o.attention(np.zeros(nh * d, np.float32), kc, vc, 0, 19, nh, nkv, d, 0.1).reshape(nh, d)
    mean = vc[:20].astype(np.float64).mean(axis=0)
    for h in range(nh):
        np.testing.assert_allclose(out[h], mean[(h // 2) * d:(h // 2 + 1) * d], rtol=0, atol=2e-6)
    # bf16 cache = the same attention over the upconverted values
    kb, vb = o.f32_to_bf16(kc), o.f32_to_bf16(vc)
    a = o.attention(q, kb, vb, 0, 40, nh, nkv, d, 0.1)
    b = o.attention(q, o.bf16_to_f32(kb), o.bf16_to_f32(vb), 0, 40, nh, nkv, d, 0.1)
    np.testing.assert_array_equal(a, b)


# ---------------------------------------------------------------------------------------
# Greedy selection (sampler.zig:158-170)
# ---------------------------------------------------------------------------------------

def greedy_brute(x):
    """First index i >= 1 of the strictly greatest value scanning from index 1 (Python)."""
    if len(x) <= 1:
        return 0
    best, m = 1, x[1]
    for i in range(2, len(x)):
        if x[i] > m:
            best, m = i, x[i]
    return best


def test_argmax_sampler_zig_173(o):
    assert o.argmax(np.array([0.1, 2.5, 0.3, -1.0], np.float32)) == 1


@pytest.mark.parametrize("case", ["random", "ties", "index0", "nan1", "nan_mid", "inf", "short"])
def test_argmax_brute_force(o, case):
    rng = np.random.default_rng(abs(hash(case)) % 1000)
    x = rng.normal(0, 1, 5000).astype(np.float32)
    if case == "ties":
        x[[7, 3000, 4999]] = 9.0
    elif case == "index0":
        x[0] = 100.0
    elif case == "nan1":
        x[1] = np.nan
    elif case == "nan_mid":
        x[[5, 17, 4000]] = np.nan
        x[4001] = 50.0
    elif case == "inf":
        x[:] = -np.inf
        x[2500] = np.inf
    elif case == "short":
        for n in (0, 1, 2, 3):
            assert o.argmax(x[:n]) == greedy_brute(list(x[:n]))
        return
    assert o.argmax(x) == greedy_brute(list(x))
