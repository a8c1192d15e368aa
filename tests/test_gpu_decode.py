"""On-device greedy selection (sampler.zig:158-170) against the oracle, bit-exact (an
index), including in a replayed graph."""
import numpy as np
import pytest

from oracle import oracle as O
from ziglm_amd import synth
from ziglm_amd.device import Graph

pytestmark = pytest.mark.gpu


def argmax_dev(dev, x):
    d_x = dev.from_numpy(np.ascontiguousarray(x, np.float32))
    d_o = dev.alloc(16)
    d_o.fill(0xEE)
    dev.argmax(d_x, len(x), d_o)
    return int(d_o.to_numpy((4,), np.uint32)[0])


@pytest.mark.parametrize("n", [262144, 1000, 2, 1, 100003])
def test_argmax_random(dev, oracle, n):
    x = synth.normal_f32(n, "logits", (n,), 0, 10.0)
    assert argmax_dev(dev, x) == oracle.argmax(x)


def test_argmax_edge_cases(dev, oracle):
    n = 262144
    base = synth.normal_f32(9, "logits", (n,))
    cases = {}
    x = base.copy(); x[[11, 70000, 262143]] = 50.0; cases["ties"] = x
    x = base.copy(); x[0] = 1e9; cases["index0"] = x
    x = base.copy(); x[1] = np.nan; cases["nan1"] = x
    x = base.copy(); x[[5, 1000, 200000]] = np.nan; x[199999] = 40.0; cases["nan_mid"] = x
    x = np.full(n, -np.inf, np.float32); x[123456] = np.inf; cases["inf"] = x
    x = np.full(n, -np.inf, np.float32); cases["all_minus_inf"] = x
    x = np.full(n, np.nan, np.float32); cases["all_nan"] = x
    for name, x in cases.items():
        assert argmax_dev(dev, x) == oracle.argmax(x), name
    assert argmax_dev(dev, np.array([0.1, 2.5, 0.3, -1.0], np.float32)) == 1  # sampler.zig:173-177


def test_argmax_graph_replays(dev, oracle):
    """Captured once, replayed on changing logits with eager work in between."""
    n = 262144
    d_x = dev.alloc(n * 4)
    d_o = dev.alloc(16)
    g = Graph(dev, lambda: dev.argmax(d_x, n, d_o))
    for rep in range(3):
        x = synth.normal_f32(40 + rep, "logits", (n,), 0, 5.0)
        d_x.upload(x)
        g.launch()
        dev.sync()
        assert int(d_o.to_numpy((4,), np.uint32)[0]) == oracle.argmax(x), rep
        assert argmax_dev(dev, x[::-1].copy()) == oracle.argmax(x[::-1].copy())
    g.destroy()


# ---------------------------------------------------------------------------------------
# Graph-captured decode step (ziglm_amd/decode.py)
# ---------------------------------------------------------------------------------------

from ziglm_amd.decode import DecodeModel  # noqa: E402
from ziglm_amd.layer import GEMMA_4B  # noqa: E402


def reset(m, token):
    m.kc.fill(0)
    m.vc.fill(0)
    m.set_token(token)


FUSE_SETS = [set(), {"qkv", "ffn", "ple", "head"}, {"attn"}]


@pytest.mark.parametrize("fused", FUSE_SETS, ids=["unfused", "prologues", "qk_attention"])
def test_decode_graph_equals_eager(dev, fused):
    """The captured step replays the eager step bit for bit, token fed back on the device."""
    m = DecodeModel.synthetic(dev, GEMMA_4B, n_layers=2, vocab=4096, max_seq=64, fused=fused)
    try:
        reset(m, 5)
        eager = []
        for p in range(4):
            m.step(p, graph=False)
            eager.append((m.logits.to_numpy((m.V,), np.float32).copy(), m.read_token()))
        reset(m, 5)
        m.capture()
        for p in range(4):
            m.step(p, graph=True)
            dev.sync()
            np.testing.assert_array_equal(m.logits.to_numpy((m.V,), np.float32), eager[p][0], err_msg=f"pos {p}")
            assert m.read_token() == eager[p][1]
        reset(m, 5)
        m.run(0, 4)  # pinned positions, no host sync between replays
        np.testing.assert_array_equal(m.logits.to_numpy((m.V,), np.float32), eager[3][0])
        assert m.read_token() == eager[3][1]
    finally:
        m.free()


@pytest.mark.parametrize("fused", FUSE_SETS, ids=["unfused", "prologues", "qk_attention"])
def test_decode_step_vs_oracle(dev, oracle, fused):
    """Three decode steps of a 2-layer model against the oracle's composition of the same
    ops (same tokens fed to both). Each op is parity-tested on its own; this checks the
    wiring of the step. Logits within 2e-3 * (1 + |logit|) (a chain of ~25 f32 ops whose
    sums differ in order), and the greedy token equal wherever the top-2 gap exceeds that."""
    s = GEMMA_4B
    L, V, max_seq, tok0 = 2, 4096, 16, 7
    m = DecodeModel.synthetic(dev, s, n_layers=L, vocab=V, max_seq=max_seq, host_weights=True, fused=fused)
    try:
        reset(m, tok0)
        h, eps = m.host, np.float32(s.eps)
        H, qn, kn = s.H, s.nh * s.D, s.nkv * s.D
        kc = np.zeros((L * max_seq, kn), np.float32)
        vc = np.zeros_like(kc)
        tok = tok0
        for p in range(3):
            m.step(p, graph=False)
            got = m.logits.to_numpy((V,), np.float32).astype(np.float64)
            gtok = m.read_token()
            # oracle composition
            x = oracle.embed_gather(h["emb"], O.Q4_0, np.array([tok], np.int32), H, np.float32(np.sqrt(np.float32(H))))[0]
            xb = oracle.rms_norm(x, h["in0"], eps, True)
            for l in range(L):
                q = oracle.gemv(O.Q4_0, h[f"wq{l}"], xb)
                k = oracle.gemv(O.Q4_0, h[f"wk{l}"], xb)
                v = oracle.gemv(O.Q4_0, h[f"wv{l}"], xb)
                q = oracle.qk_norm_rope_kv(q.reshape(1, s.nh, s.D), k.reshape(1, s.nkv, s.D), v.reshape(1, s.nkv, s.D),
                                           h[f"q_norm{l}"], h[f"k_norm{l}"], kc, vc, layer=l, max_seq=max_seq,
                                           max_kv_dim=kn, pos=np.array([p], np.int32), n_heads=s.nh,
                                           n_kv_heads=s.nkv, head_dim=s.D, base=s.theta, eps=eps)
                attn = oracle.attention(q.reshape(-1), kc, vc, l * max_seq, p, s.nh, s.nkv, s.D, 1.0)
                ao = oracle.gemv(O.Q4_0, h[f"wo{l}"], attn)
                x2, xb = oracle.rms_norm_add_rms_norm(x[None], ao[None], h[f"post_attn{l}"], h[f"pre_ffn{l}"], eps, True)
                act = oracle.geglu(oracle.gemv(O.Q4_0, h[f"wg{l}"], xb[0]), oracle.gemv(O.Q4_0, h[f"wu{l}"], xb[0]))
                fo = oracle.gemv(O.Q4_0, h[f"wd{l}"], act)
                nxt = h[f"in{l + 1}"] if l + 1 < L else h["final_norm"]
                x3, xb = oracle.rms_norm_add_rms_norm(x2, fo[None], h[f"post_ffn{l}"], nxt, eps, True)
                x, xb = x3[0], xb[0]
            logits = oracle.softcap(oracle.gemv(O.Q4_0, h["emb"], xb), 30.0).astype(np.float64)
            tol = 2e-3 * (1.0 + np.abs(logits))
            assert np.all(np.abs(got - logits) <= tol), (p, float(np.max(np.abs(got - logits) / tol)))
            top = np.sort(logits[1:])[-2:]
            if top[1] - top[0] > 2 * tol.max():
                assert gtok == oracle.argmax(logits.astype(np.float32)), p
            tok = gtok
    finally:
        m.free()
