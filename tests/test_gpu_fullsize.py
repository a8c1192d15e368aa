"""Parity at BASELINE.json's full sizes, through the C-ABI, against the CPU oracle on the
configs' own seeded inputs (ziglm_amd/synth.py, seeds 1-4):

  c2  Gemma-4B prefill, T = 2048 tokens, bf16 activations, seed 1, positions 0..2047: every op
      of the chain launched on its own at full size (the launch shapes the benchmark times,
      the input RMSNorm instance included), then the 5-op and the 4-op (cross-layer) chains;
  c3  embedding gather from full 262144 x 2560 Q8_0 / Q4_0 / BF16 tables in device memory,
      4096 ids (4032 uniform + 64 repeats), seed 2, bit-exact. The rows the ids select hold
      the seeded table's bytes (synth.table_rows draws them from the generator's streams at
      their offsets); every other row holds 0xFF bytes (an f16/bf16 NaN), so a gather from a
      wrong row cannot pass;
  c4  Gemma-27B prefill, T = 8192, bf16, seed 3, positions 0..8191: every op, the QK op at the
      local (theta 1e4) and global (theta 1e6) RoPE bases;
  c5  batched decode, B in {1, 8, 64, 256}, f32, seed 4, positions ~U[0, 32767], per-sequence
      cache slots (b * 32768 + pos): every op and the 5-op chain, then the final RMSNorm and
      the soft-cap 30 tanh(z / 30) over f32[B x 262144] logits ~N(0, 15).

Tolerances are the ones the smaller tests state: bf16 outputs within 1 bf16 ulp, f32 within
1e-5 relative; rotated coordinates relative to their rotation pair's norm; GeGLU with the
reference's 1 + tanh cancellation floor |x * up| * 2^-23; a sum x + norm(r) relative to its
summands and a norm of that sum scaled accordingly; copies and x + r bit-exact.
"""
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from test_gpu_parity import geglu_floor, pair_floor
from tol import assert_bf16, assert_bitexact, assert_rel
from ziglm_amd import bridge as B
from ziglm_amd import layer as LY
from ziglm_amd import synth

pytestmark = pytest.mark.gpu


def _f(a):
    return O.get().bf16_to_f32(a) if a.dtype == np.uint16 else a


def _close(got, ref, floor=0.0, what=""):
    """1 bf16 ulp (bf16) or 1e-5 relative (f32), plus `floor`."""
    if ref.dtype == np.uint16:
        assert_bf16(got, ref, 1, floor=floor, what=what)
    else:
        assert_rel(got, ref, 1e-5, floor=floor, what=what)


class Case:
    """One seeded layer instance on the device plus its host copy."""

    def __init__(self, dev, shape, T, dtype, seed, pos, cache_rows=None, slots=None, max_seq=None):
        self.dev, self.s, self.T, self.dtype = dev, shape, T, dtype
        self.max_seq = max_seq or shape.max_seq
        self.L = LY.LayerBuffers(dev, shape, T, dtype, cache_rows=cache_rows)
        self.h = self.L.fill_random(seed=seed)
        self.pos = np.asarray(pos, np.int32)
        self.L.pos.upload(self.pos)
        self.slots = slots
        self.d_slot = dev.from_numpy(np.asarray(slots, np.int64)) if slots is not None else None
        s = shape
        self.w = {k: synth.normal_f32(seed, "w_" + k, (s.H,), 0, 0.1) for k in self.L.w}
        self.wq = synth.normal_f32(seed, "wq", (s.D,), 0, 0.1)
        self.wk = synth.normal_f32(seed, "wk", (s.D,), 0, 0.1)
        self.np = np.uint16 if dtype == B.BF16 else np.float32
        self.eps = np.float32(s.eps)

    def restore(self):
        """Inputs the ops update in place back to the seeded values; caches zeroed."""
        for k in ("x", "q"):
            getattr(self.L, k).upload(self.h[k])
        self.L.kc.fill(0)
        self.L.vc.fill(0)

    def get(self, name, shape):
        return getattr(self.L, name).to_numpy(shape, self.np)

    def run(self, name, theta=None):
        s = self.s if theta is None else dataclasses.replace(self.s, theta=theta)
        if name == "qk_norm_rope_kv":
            self.dev.qkNormRopeKv(self.dtype, self.L.q, self.L.k, self.L.v, self.L.wq, self.L.wk, 0, self.L.kc,
                                  self.L.vc, self.L.cache_rows, 0, self.max_seq, s.nkv * s.D, self.L.pos, 0,
                                  self.d_slot, self.T, s.nh, s.nkv, s.D, 0, s.theta, 1.0, s.eps, s.uo)
        else:
            LY.OPS[name](self.dev, self.L)

    # ---- oracle and checks, per op --------------------------------------------------------
    def oracle_norm_add(self, x, r, w):
        """(x + norm(r), floor of that sum) for bf16 or f32 x."""
        o = O.get()
        xf = _f(x).astype(np.float64)
        a = o.rms_norm(_f(r).astype(np.float32), w, self.eps, True).astype(np.float64)
        return o.rms_norm_add(x, r, w, self.eps, True), 1e-5 * (np.abs(xf) + np.abs(a)), xf + a

    def check_op(self, name, theta=None):
        o, s, T, h, w, eps = O.get(), self.s, self.T, self.h, self.w, self.eps
        bf = self.dtype == B.BF16
        H, I = s.H, s.I
        if name == "input_norm":
            ref = o.rms_norm_bf16(h["x"], w["in"], eps, True) if bf else o.rms_norm(h["x"], w["in"], eps, True)
            _close(self.get("xb", (T, H)), ref, what="input norm")
        elif name == "add_rmsnorm":
            x_ref, o_ref = (o.add_rms_norm_bf16 if bf else o.add_rms_norm)(h["x"], h["ao"], w["pre_ffn"], eps, True)
            assert_bitexact(self.get("x", (T, H)), x_ref, "x + r")
            _close(self.get("xb", (T, H)), o_ref, what="norm(x + r)")
        elif name in ("norm_add_norm", "norm_add_norm_next"):
            r, w1, w2 = (h["ao"], w["post_attn"], w["pre_ffn"]) if name == "norm_add_norm" else \
                (h["fo"], w["post_ffn"], w["in"])
            x_ref, o_ref = o.rms_norm_add_rms_norm(h["x"], r, w1, w2, eps, True)
            _, floor, s_ = self.oracle_norm_add(h["x"], r, w1)
            inv2 = 1.0 / np.sqrt(np.mean(s_ * s_, axis=-1, keepdims=True) + float(eps))
            _close(self.get("x", (T, H)), x_ref, floor, "x + norm1(r)")
            _close(self.get("xb", (T, H)), o_ref, floor * inv2 * np.abs(1.0 + w2.astype(np.float64)),
                   "norm2(x + norm1(r))")
        elif name == "norm_add":
            ref, floor, _ = self.oracle_norm_add(h["x"], h["fo"], w["post_ffn"])
            _close(self.get("x", (T, H)), ref, floor, "x + norm(fo)")
        elif name == "geglu":
            _close(self.get("act", (T, I)), o.geglu(h["gate"], h["up"]),
                   geglu_floor(_f(h["gate"]), _f(h["up"])), "GeGLU")
        elif name == "qk_norm_rope_kv":
            self.check_qk(theta or s.theta)
        else:
            raise KeyError(name)

    def check_qk(self, theta):
        o, s, T = O.get(), self.s, self.T
        kn = s.nkv * s.D
        # the oracle writes row i for token i (compact cache); the device rows are the slots
        rows = self.slots if self.slots is not None else self.pos
        kc = np.zeros((T, kn), self.np)
        vc = np.zeros_like(kc)
        q_ref = o.qk_norm_rope_kv(self.h["q"].reshape(T, s.nh, s.D), self.h["k"].reshape(T, s.nkv, s.D),
                                  self.h["v"].reshape(T, s.nkv, s.D), self.wq, self.wk, kc, vc, max_seq=T,
                                  max_kv_dim=kn, pos=self.pos, slots=np.arange(T), n_heads=s.nh,
                                  n_kv_heads=s.nkv, head_dim=s.D, base=theta, eps=self.eps)
        _close(self.get("q", (T, s.nh, s.D)), q_ref, pair_floor(_f(q_ref), s.D, 0), "Q")
        es = 2 if self.np == np.uint16 else 4
        if self.slots is None and np.array_equal(rows, np.arange(T)):
            gk = self.L.kc.to_numpy((T, kn), self.np)
            gv = self.L.vc.to_numpy((T, kn), self.np)
        else:
            gk = np.stack([self.L.kc.at(int(r) * kn * es).to_numpy((kn,), self.np) for r in rows])
            gv = np.stack([self.L.vc.at(int(r) * kn * es).to_numpy((kn,), self.np) for r in rows])
            # the rows next to a written slot stay untouched (zero)
            for r in list(rows[:4]) + list(rows[-4:]):
                for nb in (int(r) - 1, int(r) + 1):
                    if 0 <= nb < self.L.cache_rows and nb not in set(int(x) for x in rows):
                        assert not np.any(self.L.kc.at(nb * kn * es).to_numpy((kn,), self.np)), f"row {nb}"
        kr = kc.reshape(T, s.nkv, s.D)
        _close(gk.reshape(T, s.nkv, s.D), kr, pair_floor(_f(kr), s.D, 0), "K cache")
        assert_bitexact(gv, vc, "V cache")

    def check_chain(self, fused, theta=None):
        """The 5-op chain (or the 4-op chain with the next layer's input norm) against the
        oracle's composition: every output after a residual update inherits a one-ulp
        difference of that update, hence the floors. theta: the RoPE base the chain ran at."""
        o, s, T, h, w, eps = O.get(), self.s, self.T, self.h, self.w, self.eps
        bf = self.dtype == B.BF16
        H = s.H
        x3, xb3 = o.rms_norm_add_rms_norm(h["x"], h["ao"], w["post_attn"], w["pre_ffn"], eps, True)
        if fused:
            x5, xb5 = o.rms_norm_add_rms_norm(x3, h["fo"], w["post_ffn"], w["in"], eps, True)
        else:
            x5 = o.rms_norm_add(x3, h["fo"], w["post_ffn"], eps, True)
        # x3 = x + norm(ao) may differ by 1e-5 of its summands (and, in bf16, by the one ulp
        # its rounding can then flip); x5 = x3 + norm(fo) adds 1e-5 of its own summands
        _, floor3, _ = self.oracle_norm_add(h["x"], h["ao"], w["post_attn"])
        if bf:
            floor3 = floor3 + np.spacing(np.abs(_f(x3))).astype(np.float64) * 65536.0
        nfo = o.rms_norm(_f(h["fo"]).astype(np.float32), w["post_ffn"], eps, True).astype(np.float64)
        floor_x = floor3 + 1e-5 * (np.abs(_f(x3)) + np.abs(nfo))
        _close(self.get("x", (T, H)), x5, floor_x, "x after the layer")
        gxb = self.get("xb", (T, H))
        if fused:
            s5 = _f(x5).astype(np.float64)
            inv = 1.0 / np.sqrt(np.mean(s5 * s5, axis=-1, keepdims=True) + float(eps))
            _close(gxb, xb5, floor_x * inv * np.abs(1.0 + w["in"].astype(np.float64)), "next-layer input norm")
        else:
            _, floor, s3 = self.oracle_norm_add(h["x"], h["ao"], w["post_attn"])
            inv = 1.0 / np.sqrt(np.mean(s3 * s3, axis=-1, keepdims=True) + float(eps))
            _close(gxb, xb3, floor * inv * np.abs(1.0 + w["pre_ffn"].astype(np.float64)), "pre-FFN norm")
        self.check_op("geglu")
        self.check_qk(theta or s.theta)


OPS_ALL = ["input_norm", "add_rmsnorm", "qk_norm_rope_kv", "norm_add_norm", "geglu", "norm_add",
           "norm_add_norm_next"]


# ---------------------------------------------------------------------------------------
# c2: Gemma-4B, 2048-token prefill, bf16, seed 1
# ---------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def c2(dev):
    print("[fullsize] c2 Gemma-4B T=2048 bf16 seed 1", flush=True)
    c = Case(dev, LY.GEMMA_4B, 2048, B.BF16, seed=1, pos=np.arange(2048))
    yield c
    LY_free(c)


def LY_free(c):
    from ziglm_amd.device import DeviceBuffer
    for v in list(vars(c.L).values()) + list(c.L.w.values()):
        if isinstance(v, DeviceBuffer):
            v.deinit()
    if c.d_slot is not None:
        c.d_slot.deinit()


@pytest.mark.parametrize("op", OPS_ALL)
def test_c2_op_full_size(c2, op):
    c2.restore()
    c2.run(op)
    c2.check_op(op)


@pytest.mark.parametrize("fused", [False, True], ids=["5op", "4op"])
def test_c2_chain_full_size(c2, fused):
    c2.restore()
    LY.run_chain(c2.dev, c2.L, fused=fused)
    c2.check_chain(fused)


# ---------------------------------------------------------------------------------------
# c3: gather from full 262144 x 2560 tables, 4096 ids, seed 2
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("kind,qtype", [("q8_0", B.Q8_0), ("q4_0", B.Q4_0), ("bf16", B.BF16)])
def test_c3_gather_full_table(dev, oracle, kind, qtype):
    vocab, dim = 262144, 2560
    print(f"[fullsize] c3 gather {kind} {vocab}x{dim}, 4096 ids, seed 2", flush=True)
    ids = synth.gather_ids(2, 4096, vocab, n_repeat=64)
    uniq = np.unique(ids)
    rows = synth.table_rows(kind, 2, uniq, dim)
    rb = rows.shape[1]
    d_tab = dev.alloc(vocab * rb)
    d_tab.fill(0xFF)
    for r, row in zip(uniq, rows):
        d_tab.at(int(r) * rb).upload(row)
    scale = np.float32(np.sqrt(np.float32(dim)))
    where = np.searchsorted(uniq, ids)
    ref = oracle.embed_gather(rows, qtype, where.astype(np.int32), dim, scale)
    d_ids, d_out = dev.from_numpy(ids), dev.alloc(ids.size * dim * 4)
    dev.embedGather(d_tab, qtype, vocab, d_ids, B.F32, d_out, ids.size, dim, scale)
    assert_bitexact(d_out.to_numpy((ids.size, dim), np.float32), ref, f"c3 gather {kind}")
    # the reference ABI mirror over the same table (no vocabulary bound)
    dev.embedLookupBatch(d_tab, qtype, d_ids, d_out, ids.size, dim, scale)
    assert_bitexact(d_out.to_numpy((ids.size, dim), np.float32), ref, f"c3 embed_lookup_batch {kind}")
    d_tab.deinit()


# ---------------------------------------------------------------------------------------
# c4: Gemma-27B, 8192-token prefill, bf16, seed 3, local and global RoPE bases
# ---------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def c4(dev):
    print("[fullsize] c4 Gemma-27B T=8192 bf16 seed 3", flush=True)
    c = Case(dev, LY.GEMMA_27B, 8192, B.BF16, seed=3, pos=np.arange(8192))
    yield c
    LY_free(c)


@pytest.mark.parametrize("op,theta", [("input_norm", None), ("add_rmsnorm", None), ("qk_norm_rope_kv", 1e4),
                                      ("qk_norm_rope_kv", 1e6), ("norm_add_norm", None), ("geglu", None),
                                      ("norm_add", None), ("norm_add_norm_next", None)])
def test_c4_op_full_size(c4, op, theta):
    c4.restore()
    c4.run(op, theta)
    c4.check_op(op, theta)


@pytest.mark.parametrize("fused,theta", [(False, 1e4), (True, 1e6)], ids=["5op-local", "4op-global"])
def test_c4_chain_full_size(c4, fused, theta):
    """The whole c4 chain in sequence at a local (1e4) and a global (1e6) RoPE base."""
    c4.restore()
    for op in (LY.CHAIN_FUSED if fused else LY.CHAIN):
        c4.run(op, theta if op == "qk_norm_rope_kv" else None)
    c4.check_chain(fused, theta)


# ---------------------------------------------------------------------------------------
# c5: batched decode, f32, seed 4, positions ~U[0, 32767], per-sequence slots
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("batch", [1, 8, 64, 256])
def test_c5_batched_decode(dev, oracle, batch):
    max_seq = 32768
    print(f"[fullsize] c5 decode B={batch}, f32, per-sequence caches of {max_seq} rows", flush=True)
    pos = synth.uniform_int(4, "pos", (batch,), 0, max_seq - 1).astype(np.int32)
    slots = np.arange(batch, dtype=np.int64) * max_seq + pos
    c = Case(dev, LY.GEMMA_4B, batch, B.F32, seed=4, pos=pos, cache_rows=batch * max_seq, slots=slots,
             max_seq=max_seq)
    try:
        for op in OPS_ALL:
            c.restore()
            c.run(op)
            c.check_op(op)
        c.restore()
        for op in LY.CHAIN:
            c.run(op)
        c.check_chain(False)
        # final RMSNorm (output norm) and the LM-head soft-cap over B x 262144 logits
        V = 262144
        w_out = synth.normal_f32(4, "w_out", (c.s.H,), 0, 0.1)
        x = c.get("x", (batch, c.s.H))
        d_w, d_o = dev.from_numpy(w_out), dev.alloc(x.nbytes)
        dev.rmsNormRows(B.F32, c.L.x, d_w, d_o, batch, c.s.H, c.s.eps, True)
        assert_rel(d_o.to_numpy(x.shape, np.float32), oracle.rms_norm(x, w_out, c.eps, True), 1e-5,
                   what="final norm")
        z = synth.normal_f32(4, "logits", (batch, V), 0, 15.0)
        d_z = dev.from_numpy(z)
        dev.tanhSoftcap(d_z, 30.0, batch * V)
        assert_rel(d_z.to_numpy(z.shape, np.float32), oracle.softcap(z, 30.0), 1e-5, what="soft-cap 30")
    finally:
        LY_free(c)
