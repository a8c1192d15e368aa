"""Decode attention on the GPU (model.zig:658-700) against float64 with the f32 bound of
attn_ref.py, and against the oracle's CPU restatement with twice that bound.

Covers: head sizes 64/128/256/512, 1/2/4/8 query heads per kv head, soft-cap, sliding window,
f32 and bf16 caches, per-token positions and per-sequence cache rows (positions up to 32767),
the split-over-positions path (workspace) and the unsplit one, the reference-ABI mirrors
(single token, device position, causal chunk), and tokens whose cache rows are out of range
(zero output)."""
import numpy as np
import pytest

from attn_ref import attention_f64
from tol import assert_bf16, assert_bitexact, assert_rel
from oracle import oracle as O
from ziglm_amd import bridge as B
from ziglm_amd import synth

pytestmark = pytest.mark.gpu


def check(got, q, kc_f32, vc_f32, row0, pos, nh, nkv, d, scale, softcap, window, what, oracle=None, kc=None, vc=None):
    ref, tol = attention_f64(q, kc_f32, vc_f32, row0, pos, nh, nkv, d, scale, softcap, window)
    err = np.abs(np.asarray(got, np.float64) - ref)
    assert np.all(err <= tol), f"{what}: max err/tol {float(np.max(err / tol)):.3g}"
    if oracle is not None:
        o = oracle.attention(q, kc if kc is not None else kc_f32, vc if vc is not None else vc_f32, row0, pos,
                             nh, nkv, d, scale, softcap, window).astype(np.float64)
        assert np.all(np.abs(o - ref) <= tol), f"{what}: oracle outside the bound"


@pytest.mark.parametrize("kv_dtype", [B.F32, B.BF16])
@pytest.mark.parametrize("nh,nkv,d", [(8, 4, 256), (4, 4, 128), (8, 2, 64), (16, 4, 128), (8, 1, 256), (8, 1, 512),
                                      (4, 2, 512)])
@pytest.mark.parametrize("softcap,window", [(0.0, 0), (50.0, 0), (0.0, 300)])
@pytest.mark.parametrize("split", [False, True])
def test_attention_decode_per_sequence(dev, oracle, kv_dtype, nh, nkv, d, softcap, window, split):
    B_, cap = 3, 2048                     # 3 sequences, 2048 cache rows each
    positions = np.array([0, 1234, 2047], np.int32)
    rows = B_ * cap
    kc = synth.normal_f32(11, "kc", (rows, nkv * d))
    vc = synth.normal_f32(11, "vc", (rows, nkv * d))
    if kv_dtype == B.BF16:
        kc_dev, vc_dev = oracle.f32_to_bf16(kc), oracle.f32_to_bf16(vc)
        kc, vc = oracle.bf16_to_f32(kc_dev), oracle.bf16_to_f32(vc_dev)
    else:
        kc_dev, vc_dev = kc, vc
    q = synth.normal_f32(11, "q", (B_, nh * d), 0, 0.3)
    scale = float(np.float32(1.0 / np.sqrt(d)))
    row_base = np.arange(B_, dtype=np.int64) * cap
    d_out = dev.alloc(B_ * nh * d * 4)
    ws_bytes = dev.attentionWorkspaceBytes(B_, nh, nkv, d, cap, window) if split else 0
    d_ws = dev.alloc(ws_bytes) if ws_bytes else None
    if split:
        assert ws_bytes > 0
    dev.attentionDecode(kv_dtype, dev.from_numpy(q), dev.from_numpy(kc_dev), dev.from_numpy(vc_dev), d_out, rows,
                        nkv * d, dev.from_numpy(row_base), 0, dev.from_numpy(positions), 0, cap, B_, nh, nkv, d,
                        scale, softcap, window, d_ws, ws_bytes)
    got = d_out.to_numpy((B_, nh * d), np.float32)
    for b in range(B_):
        check(got[b], q[b], kc, vc, int(row_base[b]), int(positions[b]), nh, nkv, d, scale, softcap, window,
              f"seq {b} pos {positions[b]}", oracle if b == 1 else None, kc_dev, vc_dev)


def test_attention_decode_long_context(dev, oracle):
    """Positions up to 32767 in per-sequence caches (the c5 layout), bf16, split."""
    nh, nkv, d, cap = 8, 4, 256, 32768
    positions = np.array([32767, 5], np.int32)
    rows = 2 * cap
    kc16 = oracle.f32_to_bf16(synth.normal_f32(12, "kc", (rows, nkv * d)))
    vc16 = oracle.f32_to_bf16(synth.normal_f32(12, "vc", (rows, nkv * d)))
    q = synth.normal_f32(12, "q", (2, nh * d), 0, 0.3)
    ws = dev.attentionWorkspaceBytes(2, nh, nkv, d, cap)
    d_out = dev.alloc(2 * nh * d * 4)
    dev.attentionDecode(B.BF16, dev.from_numpy(q), dev.from_numpy(kc16), dev.from_numpy(vc16), d_out, rows, nkv * d,
                        dev.from_numpy(np.array([0, cap], np.int64)), 0, dev.from_numpy(positions), 0, cap, 2, nh, nkv,
                        d, 1.0 / 16, 0.0, 0, dev.alloc(ws), ws)
    got = d_out.to_numpy((2, nh * d), np.float32)
    kc, vc = oracle.bf16_to_f32(kc16), oracle.bf16_to_f32(vc16)
    check(got[0], q[0], kc, vc, 0, 32767, nh, nkv, d, 1.0 / 16, 0.0, 0, "pos 32767")
    check(got[1], q[1], kc, vc, cap, 5, nh, nkv, d, 1.0 / 16, 0.0, 0, "pos 5")


def test_attention_reference_mirrors(dev, oracle):
    nh, nkv, d, max_seq, layer = 8, 4, 256, 512, 1
    max_kv_dim = nkv * d + 64                      # padded rows
    kc = synth.normal_f32(13, "kc", (2 * max_seq, max_kv_dim))
    vc = synth.normal_f32(13, "vc", (2 * max_seq, max_kv_dim))
    d_kc, d_vc = dev.from_numpy(kc), dev.from_numpy(vc)
    scale = 1.0 / 16
    # single token by value and through a device position
    q = synth.normal_f32(13, "q", (nh * d,), 0, 0.3)
    d_q, d_out = dev.from_numpy(q), dev.alloc(nh * d * 4)
    for pos in (0, 300, 511):
        dev.attentionForward(d_q, d_kc, d_vc, d_out, layer, pos, max_seq, nh, nkv, d, max_kv_dim, scale, 30.0, 0)
        check(d_out.to_numpy((nh * d,), np.float32), q, kc, vc, layer * max_seq, pos, nh, nkv, d, scale, 30.0, 0,
              f"forward pos {pos}", oracle)
        dev.attentionForwardInd(d_q, d_kc, d_vc, d_out, layer, dev.from_numpy(np.array([pos], np.int32)), max_seq,
                                nh, nkv, d, max_kv_dim, scale, 0.0, 128)
        check(d_out.to_numpy((nh * d,), np.float32), q, kc, vc, layer * max_seq, pos, nh, nkv, d, scale, 0.0, 128,
              f"forward_ind pos {pos}")
    # causal chunk: token b at position pos + b
    T, pos = 5, 100
    qb = synth.normal_f32(14, "q", (T, nh * d), 0, 0.3)
    d_outb = dev.alloc(T * nh * d * 4)
    dev.attentionBatched(dev.from_numpy(qb), d_kc, d_vc, d_outb, layer, pos, T, max_seq, nh, nkv, d, max_kv_dim,
                         scale, 0.0, 0)
    got = d_outb.to_numpy((T, nh * d), np.float32)
    for b in range(T):
        check(got[b], qb[b], kc, vc, layer * max_seq, pos + b, nh, nkv, d, scale, 0.0, 0, f"batched token {b}")


@pytest.mark.parametrize("split", [False, True])
def test_attention_out_of_range_rows_give_zeros(dev, split):
    """Out-of-range tokens write zeros from the attention kernel itself (one split) or from
    the merge, which then reads none of their splits (workspace given)."""
    nh, nkv, d, cap = 4, 2, 128, 64
    kc = synth.normal_f32(15, "kc", (2 * cap, nkv * d))
    q = synth.normal_f32(15, "q", (3, nh * d))
    d_out = dev.alloc(3 * nh * d * 4)
    d_out.fill(0x7f)
    # token 0: position beyond max_len; token 1: row past the cache; token 2: valid
    pos = np.array([cap, cap - 1, 3], np.int32)
    base = np.array([0, cap + 8, 0], np.int64)
    ws = dev.attentionWorkspaceBytes(3, nh, nkv, d, cap) if split else 0
    assert ws > 0 or not split
    dev.attentionDecode(B.F32, dev.from_numpy(q), dev.from_numpy(kc), dev.from_numpy(kc), d_out, 2 * cap, nkv * d,
                        dev.from_numpy(base), 0, dev.from_numpy(pos), 0, cap, 3, nh, nkv, d, 0.1, 0.0, 0,
                        dev.alloc(ws) if ws else None, ws)
    got = d_out.to_numpy((3, nh * d), np.float32)
    assert np.all(got[0] == 0) and np.all(got[1] == 0)
    ref, tol = attention_f64(q[2], kc, kc, 0, 3, nh, nkv, d, 0.1)
    assert np.all(np.abs(got[2] - ref) <= tol)


def test_attention_unsupported_group_is_noop(dev):
    d_buf = dev.alloc(1 << 16)
    d_out = dev.alloc(32 * 64 * 4)
    d_out.fill(0x11)
    dev.strict = False
    try:
        dev.attentionForward(d_buf, d_buf, d_buf, d_out, 0, 3, 16, 32, 2, 64, 128, 1.0, 0.0, 0)  # 16 q per kv head
        assert dev.b.last_error() == B.EUNSUPPORTED
        dev.attentionForward(d_buf, d_buf, d_buf, d_out, 0, 3, 16, 4, 2, 96, 192, 1.0, 0.0, 0)   # head_dim 96
        assert dev.b.last_error() == B.EUNSUPPORTED
    finally:
        dev.strict = True
    assert np.all(d_out.to_numpy((32 * 64 * 4,), np.uint8) == 0x11)


@pytest.mark.parametrize("kv_dtype", [B.F32, B.BF16])
@pytest.mark.parametrize("qk", [False, True], ids=["plain", "qk"])
def test_attention_decode_long_splits(dev, oracle, kv_dtype, qk):
    """Splits of up to 1024 positions (8 sequences x 2 kv heads of a 32768-row cache: the
    double-buffered step loop), plain and QK mode (q normalised and rotated in the kernel, the
    cache only read), positions at both ends of the cache and in between."""
    B_, nh, nkv, d, cap = 8, 8, 2, 128, 32768
    positions = np.array([32767, 0, 1, 31, 1024, 20000, 32766, 777], np.int32)
    rows = B_ * cap
    kc = synth.normal_f32(13, "kc", (rows, nkv * d))
    vc = synth.normal_f32(13, "vc", (rows, nkv * d))
    if kv_dtype == B.BF16:
        kc_dev, vc_dev = oracle.f32_to_bf16(kc), oracle.f32_to_bf16(vc)
        kc, vc = oracle.bf16_to_f32(kc_dev), oracle.bf16_to_f32(vc_dev)
    else:
        kc_dev, vc_dev = kc, vc
    q = synth.normal_f32(13, "q", (B_, nh * d), 0, 0.3 if not qk else 1.0)
    scale = float(np.float32(1.0 / np.sqrt(d)))
    row_base = np.arange(B_, dtype=np.int64) * cap
    ws = dev.attentionWorkspaceBytes(B_, nh, nkv, d, cap)
    d_out = dev.alloc(B_ * nh * d * 4)
    keep = [dev.from_numpy(a) for a in (q, kc_dev, vc_dev, row_base, positions)]
    d_q, d_kc, d_vc, d_rb, d_pos = keep
    if qk:
        wq = synth.normal_f32(13, "wq", (d,), 0, 0.1)
        eps = np.float32(1e-6)
        kc_ref, vc_ref = kc.copy(), vc.copy()
        q_att = oracle.qk_norm_rope_kv(q.reshape(B_, nh, d), np.zeros((B_, 0), np.float32),
                                       np.zeros((B_, 0), np.float32), wq, None, kc_ref, vc_ref, v_norm=False,
                                       max_seq=cap, max_kv_dim=nkv * d, pos=positions, slots=row_base + positions,
                                       n_heads=nh, n_kv_heads=0, head_dim=d, rotary_dim=0, base=1e4, eps=eps,
                                       unit_offset=True).reshape(B_, nh * d)
        d_wq = dev.from_numpy(wq)
        keep.append(d_wq)
        dev.attentionDecodeQk(kv_dtype, d_q, None, None, d_wq, None, False, d_kc, d_vc, d_out, rows, nkv * d, d_rb,
                              0, d_pos, 0, cap, B_, nh, nkv, d, 0, 1e4, 1.0, float(eps), True, scale, 0.0, 0,
                              dev.alloc(ws), ws)
    else:
        q_att = q
        dev.attentionDecode(kv_dtype, d_q, d_kc, d_vc, d_out, rows, nkv * d, d_rb, 0, d_pos, 0, cap, B_, nh, nkv, d,
                            scale, 0.0, 0, dev.alloc(ws), ws)
    got = d_out.to_numpy((B_, nh * d), np.float32)
    for b in range(B_):
        check(got[b], q_att[b], kc, vc, int(row_base[b]), int(positions[b]), nh, nkv, d, scale, 0.0, 0,
              f"seq {b} pos {positions[b]}")


QK_SHAPES = [(8, 4, 256, 0), (8, 1, 512, 128), (8, 1, 256, 0), (4, 2, 64, 0), (16, 4, 128, 64)]


@pytest.mark.parametrize("kv_dtype", [B.F32, B.BF16])
@pytest.mark.parametrize("nh,nkv,d,rot", QK_SHAPES)
@pytest.mark.parametrize("own", [True, False], ids=["own_kv", "reads_only"])
@pytest.mark.parametrize("split", [False, True])
def test_attention_decode_qk(dev, oracle, kv_dtype, nh, nkv, d, rot, own, split):
    """hip_attention_decode_qk against the oracle's QK-norm + RoPE + KV append followed by a
    float64 attention over the updated cache: the written cache rows (f32 within 1e-5 of the
    rotated pair's norm, bf16 within 1 ulp), the untouched rows bit for bit, and the outputs
    within the f32 attention bound. own_kv: the token's K/V row is formed in the kernel;
    reads_only (KV-shared layers): q only, the row is already in the cache."""
    B_, cap = 3, 2048
    positions = np.array([0, 777, 2047], np.int32)
    window = 300 if (d == 256 and nkv == 1) else 0
    softcap = 30.0 if d == 128 else 0.0
    v_norm = nkv == 1
    base = 1e6 if rot else 1e4
    eps = np.float32(1e-6)
    rows = B_ * cap
    row_base = np.arange(B_, dtype=np.int64) * cap
    slots = row_base + positions
    kc = synth.normal_f32(21, "kc", (rows, nkv * d))
    vc = synth.normal_f32(21, "vc", (rows, nkv * d))
    if kv_dtype == B.BF16:
        kc, vc = oracle.bf16_to_f32(oracle.f32_to_bf16(kc)), oracle.bf16_to_f32(oracle.f32_to_bf16(vc))
    q = synth.normal_f32(21, "q", (B_, nh, d))
    k = synth.normal_f32(21, "k", (B_, nkv, d))
    v = synth.normal_f32(21, "v", (B_, nkv, d))
    wq = synth.normal_f32(21, "wq", (d,), 0, 0.1)
    wk = synth.normal_f32(21, "wk", (d,), 0, 0.1)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    q_ref = oracle.qk_norm_rope_kv(q, k if own else np.zeros((B_, 0), np.float32),
                                   v if own else np.zeros((B_, 0), np.float32), wq, wk if own else None,
                                   kc_ref, vc_ref, v_norm=v_norm and own, max_seq=cap, max_kv_dim=nkv * d,
                                   pos=positions, slots=slots, n_heads=nh, n_kv_heads=nkv if own else 0,
                                   head_dim=d, rotary_dim=rot, base=base, eps=eps, unit_offset=True)
    if kv_dtype == B.BF16:  # the cache holds the rows rounded to bf16
        kc_att, vc_att = oracle.bf16_to_f32(oracle.f32_to_bf16(kc_ref)), oracle.bf16_to_f32(oracle.f32_to_bf16(vc_ref))
        d_kc, d_vc = dev.from_numpy(oracle.f32_to_bf16(kc)), dev.from_numpy(oracle.f32_to_bf16(vc))
    else:
        kc_att, vc_att = kc_ref, vc_ref
        d_kc, d_vc = dev.from_numpy(kc), dev.from_numpy(vc)
    scale = float(np.float32(1.0 / np.sqrt(d)))
    ws = dev.attentionWorkspaceBytes(B_, nh, nkv, d, cap, window) if split else 0
    d_out = dev.alloc(B_ * nh * d * 4)
    keep = []  # device buffers alive until the launch has run
    keep += [dev.from_numpy(a) for a in (q, k, v, wq, wk, row_base, positions)]
    d_q, d_k, d_v, d_wq, d_wk, d_rb, d_pos = keep
    dev.attentionDecodeQk(kv_dtype, d_q, d_k if own else None, d_v if own else None, d_wq, d_wk if own else None,
                          v_norm and own, d_kc, d_vc, d_out, rows, nkv * d, d_rb, 0, d_pos, 0, cap, B_, nh, nkv, d,
                          rot, base, 1.0, float(eps), True, scale, softcap, window,
                          dev.alloc(ws) if ws else None, ws)
    got = d_out.to_numpy((B_, nh * d), np.float32)
    cdt = np.uint16 if kv_dtype == B.BF16 else np.float32
    gk = d_kc.to_numpy(kc.shape, cdt)
    gv = d_vc.to_numpy(vc.shape, cdt)
    others = np.setdiff1d(np.arange(rows), slots if own else [])
    ref_k0 = oracle.f32_to_bf16(kc) if kv_dtype == B.BF16 else kc
    ref_v0 = oracle.f32_to_bf16(vc) if kv_dtype == B.BF16 else vc
    assert_bitexact(gk[others], ref_k0[others], "untouched K rows")
    assert_bitexact(gv[others], ref_v0[others], "untouched V rows")
    if own:
        kr = kc_ref[slots].reshape(B_, nkv, d)
        vr = vc_ref[slots].reshape(B_, nkv, d)
        if kv_dtype == B.BF16:
            assert_bf16(gk[slots].reshape(B_, nkv, d), oracle.f32_to_bf16(kr), 1, what="bf16 K row")
            assert_bf16(gv[slots].reshape(B_, nkv, d), oracle.f32_to_bf16(vr), 1, what="bf16 V row")
        else:
            eff = d if rot == 0 else rot
            h = eff // 2
            pn = np.sqrt(kr[..., :h].astype(np.float64) ** 2 + kr[..., h:2 * h].astype(np.float64) ** 2)
            floor = np.zeros(kr.shape)
            floor[..., :h] = 1e-5 * pn
            floor[..., h:2 * h] = 1e-5 * pn
            assert_rel(gk[slots].reshape(B_, nkv, d), kr, 1e-5, floor=floor, what="K row")
            assert_rel(gv[slots].reshape(B_, nkv, d), vr, 1e-5, what="V row")
    for b in range(B_):
        check(got[b], q_ref[b].reshape(-1), kc_att, vc_att, int(row_base[b]), int(positions[b]), nh, nkv, d, scale,
              softcap, window, f"seq {b} pos {positions[b]}")


def test_attention_decode_qk_unsupported_rotary(dev):
    """A rotary half that is not a power-of-two number of 8-element lane slices is
    reported, nothing launched."""
    d_buf = dev.alloc(1 << 20)
    d_out = dev.alloc(4 * 256 * 4)
    d_out.fill(0x11)
    dev.strict = False
    try:
        dev.attentionDecodeQk(B.F32, d_buf, d_buf, d_buf, None, None, False, d_buf, d_buf, d_out, 16, 256, None, 0,
                              None, 3, 16, 1, 4, 1, 256, 96, 1e4, 1.0, 1e-6, True, 0.0625, 0.0, 0)
        assert dev.b.last_error() == B.EUNSUPPORTED
    finally:
        dev.strict = True
    assert np.all(d_out.to_numpy((4 * 256 * 4,), np.uint8) == 0x11)
