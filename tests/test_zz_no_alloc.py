"""hip_attention_decode_noalloc (the no-allocation entry point) against hip_attention_decode
with a caller workspace, through the C-ABI: two calls in a row, the second with a smaller
input, each bit-identical to the workspace entry point (same kernels, same split count, same
partials); a call that needs no workspace (the unsplit path); the call captured in a
hipGraph and replayed over the shared scratch with new positions; and a call whose workspace
would exceed the static scratch is refused with HIP_BRIDGE_ESCRATCH and leaves its output
untouched."""
import numpy as np
import pytest

from ziglm_amd import bridge as B
from ziglm_amd import synth
from ziglm_amd.bridge import HipError
from ziglm_amd.device import Graph

pytestmark = pytest.mark.gpu


def _case(dev, seed, batch, n_heads, n_kv, D, max_len, window, kv_dtype):
    """Per-sequence caches [batch][max_len][n_kv * D], queries, positions ~U[0, max_len)."""
    kvd = n_kv * D
    gen = synth.normal_bf16 if kv_dtype == B.BF16 else synth.normal_f32
    kc = gen(seed, "kc", (batch * max_len, kvd))
    vc = gen(seed, "vc", (batch * max_len, kvd))
    q = synth.normal_f32(seed, "q", (batch, n_heads * D))
    pos = synth.uniform_int(seed, "pos", (batch,), 0, max_len - 1).astype(np.int32)
    rb = np.arange(batch, dtype=np.int64) * max_len
    bufs = {k: dev.from_numpy(v) for k, v in (("kc", kc), ("vc", vc), ("q", q), ("pos", pos), ("rb", rb))}
    return bufs, dict(batch=batch, n_heads=n_heads, n_kv=n_kv, D=D, max_len=max_len, window=window,
                      kv_dtype=kv_dtype, rows=batch * max_len, kvd=kvd)


def _noalloc(dev, bufs, c, out):
    dev.attentionDecodeNoalloc(c["kv_dtype"], bufs["q"], bufs["kc"], bufs["vc"], out, c["rows"], c["kvd"], bufs["rb"],
                               0, bufs["pos"], 0, c["max_len"], c["batch"], c["n_heads"], c["n_kv"], c["D"], 1.0, 30.0,
                               c["window"])


def _with_workspace(dev, bufs, c):
    """hip_attention_decode with a caller workspace: (output, workspace bytes)."""
    n = c["batch"] * c["n_heads"] * c["D"]
    out_ws = dev.alloc(n * 4)
    out_ws.fill(0xCD)
    need = dev.attentionWorkspaceBytes(c["batch"], c["n_heads"], c["n_kv"], c["D"], c["max_len"], c["window"])
    ws = dev.alloc(max(need, 16))
    dev.attentionDecode(c["kv_dtype"], bufs["q"], bufs["kc"], bufs["vc"], out_ws, c["rows"], c["kvd"], bufs["rb"], 0,
                        bufs["pos"], 0, c["max_len"], c["batch"], c["n_heads"], c["n_kv"], c["D"], 1.0, 30.0,
                        c["window"], ws, need)
    return out_ws.to_numpy((c["batch"], c["n_heads"] * c["D"]), np.float32), need


def _run_pair(dev, bufs, c):
    """(no-alloc output, workspace output) of the same call."""
    n = c["batch"] * c["n_heads"] * c["D"]
    out_na = dev.alloc(n * 4)
    out_na.fill(0xAB)
    _noalloc(dev, bufs, c, out_na)
    ref, need = _with_workspace(dev, bufs, c)
    return out_na.to_numpy(ref.shape, np.float32), ref, need


def test_noalloc_matches_workspace_entry_point_twice(dev):
    # call 1: 8 sequences of Gemma-4B heads (8 / 4 x 256) over 4096-row f32 caches (split)
    bufs, c = _case(dev, 41, 8, 8, 4, 256, 4096, 0, B.F32)
    got, ref, need = _run_pair(dev, bufs, c)
    assert need > 0, "the call should split (use the scratch)"
    assert np.all(np.isfinite(ref))
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    # call 2, smaller: 2 sequences of 8 / 1 x 128 heads, bf16 caches of 1024 rows, window 256
    bufs2, c2 = _case(dev, 42, 2, 8, 1, 128, 1024, 256, B.BF16)
    got2, ref2, need2 = _run_pair(dev, bufs2, c2)
    assert 0 < need2 < need
    assert np.all(np.isfinite(ref2))
    np.testing.assert_array_equal(got2.view(np.uint32), ref2.view(np.uint32))


def test_noalloc_refuses_calls_beyond_its_scratch(dev):
    """256 sequences of Gemma-4B heads over 32768 positions need 68 MB of partials (more than
    the 32 MiB scratch): not launched, HIP_BRIDGE_ESCRATCH, output untouched."""
    batch, nh, nkv, D, max_len = 256, 8, 4, 256, 32768
    need = dev.attentionWorkspaceBytes(batch, nh, nkv, D, max_len, 0)
    assert need > 32 << 20
    q = dev.alloc(batch * nh * D * 4)
    kv = dev.alloc(16 * nkv * D * 4)  # never read: the call is refused before any launch
    out = dev.alloc(batch * nh * D * 4)
    out.fill(0x5A)
    with pytest.raises(HipError) as e:
        dev.attentionDecodeNoalloc(B.F32, q, kv, kv, out, 16, nkv * D, None, 0, None, 0, max_len, batch, nh, nkv, D,
                                   1.0, 0.0, 0)
    assert f"{B.ESCRATCH} " in str(e.value)
    assert np.all(out.to_numpy((batch * nh * D * 4,), np.uint8) == 0x5A)


def test_noalloc_unsplit_shape(dev):
    """A call that needs no workspace (8-row caches: one split): the no-allocation entry point
    takes the unsplit path and matches the workspace entry point bit for bit."""
    bufs, c = _case(dev, 46, 3, 8, 4, 256, 8, 0, B.F32)
    got, ref, need = _run_pair(dev, bufs, c)
    assert need == 0
    assert np.all(np.isfinite(ref))
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_noalloc_captured_in_a_graph(dev):
    """The use the entry point is for: one eager call (the scratch address is looked up
    outside capture), then the call captured in a hipGraph and replayed twice over the
    shared static scratch with new positions written into d_pos between the replays; each
    replay bit-identical to hip_attention_decode with a workspace over the same positions."""
    bufs, c = _case(dev, 43, 4, 8, 4, 256, 4096, 0, B.F32)
    n = c["batch"] * c["n_heads"] * c["D"]
    out_g = dev.alloc(n * 4)
    _noalloc(dev, bufs, c, out_g)
    dev.sync()
    g = Graph(dev, lambda: _noalloc(dev, bufs, c, out_g))
    try:
        for seed in (44, 45):
            pos = synth.uniform_int(seed, "pos", (c["batch"],), 0, c["max_len"] - 1).astype(np.int32)
            bufs["pos"].upload(pos)
            out_g.fill(0xAB)
            dev.sync()
            g.launch()
            dev.sync()
            got = out_g.to_numpy((c["batch"], c["n_heads"] * c["D"]), np.float32)
            ref, need = _with_workspace(dev, bufs, c)
            assert need > 0
            assert np.all(np.isfinite(ref))
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    finally:
        g.destroy()
