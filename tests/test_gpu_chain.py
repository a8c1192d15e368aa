"""The per-layer fused chain as bench.py runs it (ziglm_amd/layer.py), checked end to end
against the oracle's composition of the same ops on the same seeded inputs.

Every output after a bf16 residual update inherits a possible one-ulp difference of that
update, so the floors below are one bf16 ulp of the intermediate plus 1e-5 of the summands.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tol import assert_bf16, assert_bitexact
from ziglm_amd import bridge as B
from ziglm_amd import layer as LY

pytestmark = pytest.mark.gpu


def bf16_ulp(x):
    x = np.abs(np.asarray(x, np.float32))
    return np.spacing(x).astype(np.float64) * 65536.0


@pytest.mark.parametrize("shape,T,fused", [(LY.GEMMA_4B, 48, False), (LY.GEMMA_4B, 48, True),
                                           (LY.GEMMA_27B, 16, False)])
def test_chain_bf16(dev, oracle, shape, T, fused):
    s = shape
    L = LY.LayerBuffers(dev, s, T, B.BF16)
    h = L.fill_random(seed=21, pos0=100)
    LY.run_chain(dev, L, fused=fused)
    f = O.get().bf16_to_f32
    w = {k: L.w[k].to_numpy((s.H,), np.float32) for k in L.w}
    wq, wk = L.wq.to_numpy((s.D,), np.float32), L.wk.to_numpy((s.D,), np.float32)

    # oracle composition
    eps = np.float32(s.eps)
    xb1 = oracle.rms_norm_bf16(h["x"], w["in"], eps, True)
    kc = np.zeros((s.max_seq, s.nkv * s.D), np.uint16)
    vc = np.zeros_like(kc)
    q_ref = oracle.qk_norm_rope_kv(h["q"].reshape(T, s.nh, s.D), h["k"].reshape(T, s.nkv, s.D),
                                   h["v"].reshape(T, s.nkv, s.D), wq, wk, kc, vc, max_seq=s.max_seq,
                                   max_kv_dim=s.nkv * s.D, pos=np.arange(100, 100 + T, dtype=np.int32),
                                   n_heads=s.nh, n_kv_heads=s.nkv, head_dim=s.D, base=s.theta, eps=eps)
    x3, xb3 = oracle.rms_norm_add_rms_norm(h["x"], h["ao"], w["post_attn"], w["pre_ffn"], eps, True)
    act = oracle.geglu(h["gate"], h["up"])
    if fused:
        x5, xb5 = oracle.rms_norm_add_rms_norm(x3, h["fo"], w["post_ffn"], w["in"], eps, True)
    else:
        x5 = oracle.rms_norm_add(x3, h["fo"], w["post_ffn"], eps, True)

    gx = L.x.to_numpy((T, s.H), np.uint16)
    gxb = L.xb.to_numpy((T, s.H), np.uint16)
    nfo = oracle.rms_norm(f(h["fo"]), w["post_ffn"], eps, True).astype(np.float64)
    floor_x = bf16_ulp(f(x3)) + 1e-5 * (np.abs(f(x3)) + np.abs(nfo))
    assert_bf16(gx, x5, 1, floor=floor_x, what="x after the layer")
    if fused:
        s5 = f(x5).astype(np.float64)
        inv = 1.0 / np.sqrt(np.mean(s5 * s5, axis=-1, keepdims=True) + float(eps))
        floor_xb = floor_x * inv * np.abs(1.0 + w["in"].astype(np.float64))
        assert_bf16(gxb, xb5, 1, floor=floor_xb, what="next-layer input norm")
    else:
        assert xb1.shape == gxb.shape
        s3 = f(x3).astype(np.float64)
        inv = 1.0 / np.sqrt(np.mean(s3 * s3, axis=-1, keepdims=True) + float(eps))
        a = oracle.rms_norm(f(h["ao"]), w["post_attn"], eps, True).astype(np.float64)
        floor_xb = 1e-5 * (np.abs(f(h["x"])) + np.abs(a)) * inv * np.abs(1.0 + w["pre_ffn"].astype(np.float64))
        assert_bf16(gxb, xb3, 1, floor=floor_xb, what="pre-FFN norm")
    from test_gpu_parity import geglu_floor, pair_floor
    assert_bf16(L.act.to_numpy((T, s.I), np.uint16), act, 1, floor=geglu_floor(f(h["gate"]), f(h["up"])), what="GeGLU")
    assert_bf16(L.q.to_numpy((T, s.nh, s.D), np.uint16), q_ref, 1, floor=pair_floor(f(q_ref), s.D, 0), what="Q")
    gk = L.kc.to_numpy(kc.shape, np.uint16).reshape(s.max_seq, s.nkv, s.D)
    kr = kc.reshape(s.max_seq, s.nkv, s.D)
    assert_bf16(gk, kr, 1, floor=pair_floor(f(kr), s.D, 0), what="K cache")
    assert_bitexact(L.vc.to_numpy(vc.shape, np.uint16), vc, "V cache")
