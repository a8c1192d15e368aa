"""Gemma-4 per-layer-embedding (PLE) steps on the GPU, driven in the reference's own call
sequence through the reference-ABI methods (cuda_model.zig:488-523 token inputs, 710-724
injection: embedLookup, copy + scale, gemv, rmsNormBatched, pleCtxFuse; gemv, pleGateGelu,
gemv, rmsnormAdd), against the oracle's model.zig:506-540 / 757-781.

The GEMVs sum in another order than the CPU, so each stage is checked on its own input:
  * the gathered PLE row and the fuse are bit-exact (one rounding each, as the CPU's);
  * a GEMV lies within 2^-20 * sum |w x| of the float64 product, as the oracle's does;
  * the norm and GELU stages, fed the GPU's own previous stage, are within 1e-5 relative
    of the oracle applied to that same input (GELU with its |x * slice| * 2^-23 floor).
"""
import numpy as np
import pytest

from oracle import oracle as O
from test_oracle_gemv_cpu import bound, random_matrix
from tol import assert_bitexact, assert_rel
from ziglm_amd import bridge as B
from ziglm_amd import synth

pytestmark = pytest.mark.gpu

PLE = 256


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0, B.BF16])
@pytest.mark.parametrize("token_path", [True, False])
def test_ple_token_inputs_reference_sequence(dev, oracle, qtype, token_path):
    L, dim, vocab, eps = 35, 1536, 64, np.float32(1e-6)
    n = L * PLE
    table = random_matrix(qtype, vocab, n, seed=21)[0]
    proj_raw, proj_wd = random_matrix(qtype, n, dim, seed=22)
    norm = synth.normal_f32(23, "pn", (PLE,), 1, 0.1)
    x = synth.normal_f32(23, "x", (dim,), 0, 40)
    token = 17
    d_tab, d_proj, d_norm = dev.from_numpy(table.reshape(-1)), dev.from_numpy(proj_raw.reshape(-1)), dev.from_numpy(norm)
    d_x, d_xb = dev.from_numpy(x), dev.alloc(dim * 4)
    d_ple, d_scr = dev.alloc(n * 4), dev.alloc(n * 4)
    d_ple.fill(0x7F)
    scale16 = np.float32(np.sqrt(np.float32(PLE)))
    if token_path:
        dev.embedLookup(d_tab, qtype, token, d_ple, n, scale16)                 # cuda_model.zig:493
    else:
        dev.scale(d_ple, 0.0, n)                                                # cuda_model.zig:502
    d_xb.copy_from(d_x, dim * 4, dev.stream)                                   # cuda_model.zig:510
    dev.scale(d_xb, np.float32(1.0) / np.sqrt(np.float32(dim)), dim)           # cuda_model.zig:511
    dev.gemv(qtype, d_proj, d_xb, d_scr, n, dim)                                # cuda_model.zig:514
    ctx = d_scr.to_numpy((n,), np.float32)
    dev.rmsNormBatched(d_scr, d_norm, d_scr, PLE, L, eps, False)                # cuda_model.zig:519
    normed = d_scr.to_numpy((n,), np.float32)
    ple0 = d_ple.to_numpy((n,), np.float32)
    dev.pleCtxFuse(d_ple, d_scr, n, token_path)                                 # cuda_model.zig:523
    got = d_ple.to_numpy((n,), np.float32)

    row = oracle.dequantize_row(qtype, table[token], n)
    ple_ref = (row * scale16).astype(np.float32) if token_path else np.zeros(n, np.float32)
    assert_bitexact(ple0, ple_ref, "PLE row gather")
    xb = (x * (np.float32(1.0) / np.sqrt(np.float32(dim)))).astype(np.float32)
    exact = proj_wd @ xb.astype(np.float64)
    assert np.all(np.abs(ctx - exact) <= bound(proj_wd, xb)), "projection GEMV"
    assert_rel(normed, oracle.rms_norm(ctx.reshape(L, PLE), norm, eps, False).reshape(-1), 1e-5,
               what="per-layer projection norm")
    assert_bitexact(got, oracle.ple_ctx_fuse(ple0, normed, token_path), "ctx fuse")
    # end to end against the oracle's model.zig:506-540 (its own GEMV order): the GEMV bound
    # carried through the norm, which divides by the row's rms
    ref = oracle.ple_token_inputs(row if token_path else None, x, qtype, proj_raw, norm, L, eps, token_path)
    rms = np.sqrt(np.mean(exact.reshape(L, PLE) ** 2, axis=1)).repeat(PLE)
    floor = 4 * bound(proj_wd, xb) / rms * np.abs(np.tile(norm, L)) + 1e-6 * np.abs(ref)
    assert_rel(got, ref, 1e-5, floor=floor, what="PLE token inputs vs oracle")


@pytest.mark.parametrize("qtype", [B.Q4_0, B.BF16])
def test_ple_inject_reference_sequence(dev, oracle, qtype):
    dim, eps = 1536, np.float32(1e-6)
    gate_raw, gate_wd = random_matrix(qtype, PLE, dim, seed=31)
    proj_raw, proj_wd = random_matrix(qtype, dim, PLE, seed=32)
    post = synth.normal_f32(33, "post", (dim,), 1, 0.1)
    x = synth.normal_f32(33, "x", (dim,), 0, 4)
    sl = synth.normal_f32(33, "slice", (PLE,), 0, 2)
    d_x, d_gate, d_buf, d_xb = dev.from_numpy(x), dev.alloc(PLE * 4), dev.alloc(PLE * 4), dev.alloc(dim * 4)
    d_gw, d_pw, d_post, d_sl = (dev.from_numpy(gate_raw.reshape(-1)), dev.from_numpy(proj_raw.reshape(-1)),
                                dev.from_numpy(post), dev.from_numpy(sl))
    dev.gemv(qtype, d_gw, d_x, d_gate, PLE, dim)                                # cuda_model.zig:716
    gate = d_gate.to_numpy((PLE,), np.float32)
    dev.pleGateGelu(d_gate, d_sl, d_buf, PLE)                                   # cuda_model.zig:717
    buf = d_buf.to_numpy((PLE,), np.float32)
    dev.gemv(qtype, d_pw, d_buf, d_xb, dim, PLE)                                # cuda_model.zig:719
    d = d_xb.to_numpy((dim,), np.float32)
    dev.rmsnormAdd(d_x, d_xb, d_post, dim, eps, False)                          # cuda_model.zig:722
    got = d_x.to_numpy((dim,), np.float32)

    assert np.all(np.abs(gate - gate_wd @ x.astype(np.float64)) <= bound(gate_wd, x)), "gate GEMV"
    assert_rel(buf, oracle.ple_gate_gelu(gate, sl), 1e-5,
               floor=np.abs(gate.astype(np.float64) * sl) * 2.0 ** -23, what="pleGateGelu")
    assert np.all(np.abs(d - proj_wd @ buf.astype(np.float64)) <= bound(proj_wd, buf)), "projection GEMV"
    assert_rel(got, oracle.rms_norm_add(x, d, post, eps, False), 1e-5, floor=1e-6 * np.abs(x),
               what="post-PLE norm + add")
