"""float64 decode attention and its f32 error bound, shared by the oracle and GPU tests.

For query head h (kv head h // (n_heads // n_kv_heads)) at position pos over cache rows
row0 + [start, pos]: s_t = (q_h . k_t) * scale, optionally cap * tanh(s_t / cap), w =
softmax(s), out_h = sum_t w_t v_t (model.zig:658-700).

Bound. An f32 implementation rounds each score by at most ds_t = 2^-20 * scale * sum_i |q_i
k_ti| (dot-product rounding; the soft-cap's tanh adds a few ulp of |s|, covered by the
1e-6 * |s| term). A score perturbation ds moves the output by at most
2 * max_t ds_t * sum_t w_t |v_t - out|; the weights' exp / normalisation and the weighted
sum add at most 2^-19 * sum_t w_t |v_t|.
"""
import numpy as np


def attention_f64(q, kc, vc, row0, pos, n_heads, n_kv_heads, d, scale, softcap=0.0, window=0):
    """Returns (out f64[n_heads*d], tol f64[n_heads*d]); kc / vc are [rows, row_stride] f32
    (bf16 caches: pass the upconverted f32 values)."""
    q = np.asarray(q, np.float64).reshape(n_heads, d)
    seq = pos + 1
    start = seq - window if (window > 0 and seq > window) else 0
    g = n_heads // n_kv_heads
    out = np.zeros((n_heads, d))
    tol = np.zeros((n_heads, d))
    for h in range(n_heads):
        kh = h // g
        K = np.asarray(kc[row0 + start: row0 + seq, kh * d:(kh + 1) * d], np.float64)
        V = np.asarray(vc[row0 + start: row0 + seq, kh * d:(kh + 1) * d], np.float64)
        s = (K @ q[h]) * scale
        ds = 2.0 ** -20 * scale * (np.abs(K) @ np.abs(q[h]))
        if softcap > 0.0:
            s = softcap * np.tanh(s / softcap)
            ds = ds + 1e-6 * np.abs(s)
        w = np.exp(s - s.max())
        w /= w.sum()
        o = w @ V
        out[h] = o
        tol[h] = 2.0 * ds.max() * (w @ np.abs(V - o)) + 2.0 ** -19 * (w @ np.abs(V)) + 1e-7
    return out.reshape(-1), tol.reshape(-1)
