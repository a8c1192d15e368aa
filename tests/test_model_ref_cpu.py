"""The oracle's model restatement (oracle/model_ref.py) on the CPU: its per-layer
configuration against the reference's rules worked out by hand for a small gemma4 file
(model.zig:246-300, 600-616), and its f32 forward pass against an independent float64
forward (tests/model_f64.py) over several decode steps, for gemma4 (PLE, KV sharing,
no-scale V norm, head_dim 512 layers, layer scalar, mixed tensor types, F16 / BF16 norms)
and gemma2 ((1+w) norms, 1/sqrt(head_dim) attention scale)."""
import numpy as np
import pytest

from model_f64 import F64Model
from oracle import model_ref as MR
from oracle import oracle as O
from ziglm_amd import bridge as B
from ziglm_amd import synth_gguf as S

TINY4 = S.GgufModelConfig(arch="gemma4", dim=128, n_layers=20, n_heads=4, n_kv_heads=1, head_dim=32,
                          global_head_dim=512, global_every=5, inter=256, vocab=512,
                          types={"q": B.Q8_0, "o": B.BF16, "down": B.F16, "ple_out": B.F32, "v": B.Q8_0},
                          norm_type=B.F16, no_kv_from=18, scalars={3: (B.BF16, 0.75), 7: (B.F32, 1.5)},
                          tile_rows=0)
TINY2 = S.GgufModelConfig(arch="gemma2", dim=128, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=64,
                          global_every=0, inter=256, vocab=512, ple=False, norm_type=B.BF16, tile_rows=0)


@pytest.fixture(scope="module")
def o():
    return O.get()


def test_ref_config_follows_reference_rules(o):
    data = S.build(TINY4, seed=5).tobytes()
    r = MR.RefModel(o, data, max_seq=32)
    assert r.arch == "gemma4" and not r.uo and r.gemma
    for i, ly in enumerate(r.layers):
        glob = (i + 1) % 5 == 0
        assert ly["head_dim"] == (512 if glob else 32)
        assert (ly["theta"], ly["rotary"], ly["window"]) == ((1e6, 128, 0) if glob else (1e4, 32, 512))
        assert (ly["n_heads"], ly["n_kv"], ly["inter"]) == (4, 1, 256)
        # 20 gemma4 layers: 15 unshared; 18, 19 also lack attn_k
        assert ly["shared"] == (i >= 15)
        if i >= 15:
            assert ly["donor"] == (14 if glob else 13)   # last unshared layer of equal head_dim
        else:
            assert ly["donor"] == i
    assert r.layers[3]["scalar"] == 0.75 and r.layers[7]["scalar"] == 1.5 and r.layers[4]["scalar"] == 1.0
    assert r.ple is not None and r.ple_proj is not None and r.ple_norm is not None and r.output is None


@pytest.mark.parametrize("cfg,steps", [(TINY4, 4), (TINY2, 3)], ids=["gemma4", "gemma2"])
def test_ref_forward_matches_float64(o, cfg, steps):
    """Distinct tokens per step (a repeated token gives equal V rows, which would hide
    the attention weights). Tolerance 1e-5 * (|logit| + std(logits)): the f32 chain
    stays within ~1e-6 of that scale here."""
    data = S.build(cfg, seed=9).tobytes()
    r = MR.RefModel(o, data, max_seq=16)
    f = F64Model(r)
    for pos, tok in enumerate([3, 17, 101, 250, 77][:steps]):
        got = r.forward(tok, pos).astype(np.float64)
        ref = f.forward(tok, pos)
        tol = 1e-5 * (np.abs(ref) + ref.std())
        assert np.all(np.abs(got - ref) <= tol), (pos, float(np.max(np.abs(got - ref) / tol)))
    # planted mistakes are caught: no embedding scale; attention over the wrong window
    for plant in ("scale", "window"):
        r2 = MR.RefModel(o, data, max_seq=16)
        f2 = F64Model(MR.RefModel(o, data, max_seq=16))
        if plant == "scale":
            r2.gemma = False
        else:
            for ly in r2.layers:
                ly["window"] = 2
        bad = 0.0
        for pos, tok in enumerate([3, 17, 101, 250]):
            got = r2.forward(tok, pos).astype(np.float64)
            ref = f2.forward(tok, pos)
            bad = max(bad, float(np.max(np.abs(got - ref) / (1e-5 * (np.abs(ref) + ref.std())))))
        assert bad > 10, plant
