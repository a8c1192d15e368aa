"""Golden fixtures (tests/golden/make_golden.py): the oracle reproduces them bit for bit
(CPU), and the HIP kernels match them through the C-ABI (GPU) -- bit-exact for the gather
and the KV V copy, 1e-5 relative (pair-norm / GeGLU floors as in test_gpu_parity.py)
otherwise."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from tol import assert_bitexact, assert_rel
from ziglm_amd import bridge as B

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
EPS = np.float32(1e-6)


def load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_c1_fixture():
    o, g = O.get(), load("c1_decode_seed0.npz")
    H, nh, nkv, D, I, pos = (int(v) for v in g["meta"])
    x_out, norm_out = o.add_rms_norm(g["x"], g["residual"], g["w"], EPS, True)
    assert_bitexact(x_out, g["x_out"], "x+r")
    assert_bitexact(norm_out, g["norm_out"], "norm")
    kc = np.zeros((4096, nkv * D), np.float32)
    vc = np.zeros_like(kc)
    q_out = o.qk_norm_rope_kv(g["q"], g["k"], g["v"], g["wq"], g["wk"], kc, vc, max_seq=4096, max_kv_dim=nkv * D,
                              pos=np.array([pos], np.int32), n_heads=nh, n_kv_heads=nkv, head_dim=D, base=10000.0,
                              eps=EPS)
    assert_bitexact(q_out, g["q_out"], "q")
    assert_bitexact(kc[pos], g["k_row"], "k row")
    assert_bitexact(vc[pos], g["v_row"], "v row")
    assert_bitexact(o.geglu(g["gate"], g["up"]), g["geglu_out"], "geglu")
    assert_bitexact(o.softcap(g["scores"], 50.0), g["softcap_out"], "softcap")


def test_oracle_reproduces_gather_fixture():
    o, g = O.get(), load("gather_seed2.npz")
    for name, qt in (("q8_0", O.Q8_0), ("q4_0", O.Q4_0), ("bf16", O.BF16), ("q6_k", O.Q6_K)):
        assert_bitexact(o.embed_gather(g[name], qt, g["ids"], 256, np.float32(16.0)), g["out_" + name], name)


@pytest.mark.gpu
def test_gpu_matches_c1_fixture(dev):
    from test_gpu_parity import geglu_floor, pair_floor
    g = load("c1_decode_seed0.npz")
    H, nh, nkv, D, I, pos = (int(v) for v in g["meta"])
    d_x, d_r, d_w, d_o = dev.from_numpy(g["x"]), dev.from_numpy(g["residual"]), dev.from_numpy(g["w"]), dev.alloc(H * 4)
    dev.addRmsNorm(d_x, d_r, d_w, d_o, H, EPS, True)
    assert_bitexact(d_x.to_numpy((H,), np.float32), g["x_out"], "x+r")
    assert_rel(d_o.to_numpy((H,), np.float32), g["norm_out"], 1e-5, what="norm")
    d_q = dev.from_numpy(g["q"])
    d_kc, d_vc = dev.alloc(4096 * nkv * D * 4), dev.alloc(4096 * nkv * D * 4)
    d_kc.fill(0)
    d_vc.fill(0)
    dev.qkNormRopeKv(B.F32, d_q, dev.from_numpy(g["k"]), dev.from_numpy(g["v"]), dev.from_numpy(g["wq"]),
                     dev.from_numpy(g["wk"]), 0, d_kc, d_vc, 4096, 0, 4096, nkv * D, None, pos, None, 1, nh, nkv,
                     D, 0, 10000.0, 1.0, EPS, True)
    q = d_q.to_numpy(g["q"].shape, np.float32)
    assert_rel(q, g["q_out"], 1e-5, floor=pair_floor(g["q_out"], D, 0), what="q")
    kc = d_kc.to_numpy((4096, nkv * D), np.float32)
    kr = g["k_row"].reshape(nkv, D)
    assert_rel(kc[pos].reshape(nkv, D), kr, 1e-5, floor=pair_floor(kr, D, 0), what="k row")
    assert_bitexact(d_vc.to_numpy((4096, nkv * D), np.float32)[pos], g["v_row"], "v row")
    d_a = dev.alloc(I * 4)
    dev.geglu(dev.from_numpy(g["gate"]), dev.from_numpy(g["up"]), d_a, I)
    assert_rel(d_a.to_numpy((I,), np.float32), g["geglu_out"], 1e-5, floor=geglu_floor(g["gate"], g["up"]), what="geglu")
    d_s = dev.from_numpy(g["scores"])
    dev.tanhSoftcap(d_s, 50.0, g["scores"].size)
    assert_rel(d_s.to_numpy(g["scores"].shape, np.float32), g["softcap_out"], 1e-5, what="softcap")


@pytest.mark.gpu
def test_gpu_matches_gather_fixture(dev):
    g = load("gather_seed2.npz")
    ids = g["ids"]
    for name, qt in (("q8_0", B.Q8_0), ("q4_0", B.Q4_0), ("bf16", B.BF16), ("q6_k", B.Q6_K)):
        d_out = dev.alloc(ids.size * 256 * 4)
        dev.embedGather(dev.from_numpy(g[name]), qt, g[name].shape[0], dev.from_numpy(ids), B.F32, d_out, ids.size,
                        256, np.float32(16.0))
        assert_bitexact(d_out.to_numpy((ids.size, 256), np.float32), g["out_" + name], name)
