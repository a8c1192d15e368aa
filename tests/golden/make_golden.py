"""Writes the committed golden fixtures under tests/golden/ (run from the repo root):

    python tests/golden/make_golden.py

c1_decode_seed0.npz  BASELINE.json configs[0] (one decode step, seed 0), inputs from
                     ziglm_amd.synth and outputs from the CPU oracle:
                     residual add + RMSNorm(1+w) over f32[2560] (eps 1e-6); per-head
                     QK-RMSNorm(1+w) + RoPE (theta 1e4, half-split, pos 1234) of
                     Q f32[8x256], K f32[4x256] and the K/V append into cache row 1234;
                     GeGLU over f32[10240]; soft-cap 50*tanh(s/50) over f32[8x1235].
gather_seed2.npz     small Q8_0 / Q4_0 / BF16 / Q6_K tables (32 rows x 256 columns, the
                     c3 generator at reduced size) and 40 ids with repeats, gathered with
                     scale sqrt(256) = 16 (f32 outputs, bit-exact targets).

The fixtures pin the oracle over time (tests/test_golden.py) and are the GPU tests'
committed targets; regenerate them only when the oracle's definition changes on purpose.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from ziglm_amd import synth  # noqa: E402

EPS = np.float32(1e-6)


def c1(o):
    s = 0
    H, nh, nkv, D, I, pos = 2560, 8, 4, 256, 10240, 1234
    d = {
        "x": synth.normal_f32(s, "x", (H,)),
        "residual": synth.normal_f32(s, "residual", (H,)),
        "w": synth.normal_f32(s, "w", (H,), 0, 0.1),
        "q": synth.normal_f32(s, "q", (1, nh, D)),
        "k": synth.normal_f32(s, "k", (1, nkv, D)),
        "v": synth.normal_f32(s, "v", (1, nkv, D)),
        "wq": synth.normal_f32(s, "wq", (D,), 0, 0.1),
        "wk": synth.normal_f32(s, "wk", (D,), 0, 0.1),
        "gate": synth.normal_f32(s, "gate", (I,)),
        "up": synth.normal_f32(s, "up", (I,)),
        "scores": synth.normal_f32(s, "scores", (nh, pos + 1), 0, 20),
    }
    d["x_out"], d["norm_out"] = o.add_rms_norm(d["x"], d["residual"], d["w"], EPS, True)
    kc = np.zeros((4096, nkv * D), np.float32)
    vc = np.zeros_like(kc)
    d["q_out"] = o.qk_norm_rope_kv(d["q"], d["k"], d["v"], d["wq"], d["wk"], kc, vc, max_seq=4096,
                                   max_kv_dim=nkv * D, pos=np.array([pos], np.int32), n_heads=nh,
                                   n_kv_heads=nkv, head_dim=D, base=10000.0, eps=EPS)
    d["k_row"], d["v_row"] = kc[pos].copy(), vc[pos].copy()
    d["geglu_out"] = o.geglu(d["gate"], d["up"])
    d["softcap_out"] = o.softcap(d["scores"], 50.0)
    d["meta"] = np.array([H, nh, nkv, D, I, pos], np.int64)
    return d


def gather(o):
    s, rows, cols = 2, 32, 256
    d = {
        "q8_0": synth.q8_0_table(s, rows, cols),
        "q4_0": synth.q4_0_table(s, rows, cols),
        "bf16": synth.bf16_table(s, rows, cols),
        "ids": synth.gather_ids(s, 40, rows, n_repeat=8),
    }
    raw = synth.uniform_int(s, "q6k", (rows, 210), 0, 255).astype(np.uint8)
    raw[:, 208:210] = synth.f16_bits(synth.uniform_f32(s, "q6k.d", (rows,), 1e-3, 2e-2)).reshape(rows, 1).view(np.uint8)
    d["q6_k"] = raw
    scale = np.float32(16.0)
    for name, qt in (("q8_0", O.Q8_0), ("q4_0", O.Q4_0), ("bf16", O.BF16), ("q6_k", O.Q6_K)):
        d["out_" + name] = o.embed_gather(d[name], qt, d["ids"], cols, scale)
    return d


def main():
    o = O.get()
    np.savez_compressed(os.path.join(HERE, "c1_decode_seed0.npz"), **c1(o))
    np.savez_compressed(os.path.join(HERE, "gather_seed2.npz"), **gather(o))
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
