"""bench.py host logic that needs no GPU: the profiler guard and the rotation sizing."""
import math
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from ziglm_amd import layer as LY  # noqa: E402


def test_profiler_attached_detects_preload_and_settings():
    assert not bench.profiler_attached({})
    assert not bench.profiler_attached({"LD_PRELOAD": "/usr/lib/libfoo.so", "HOME": "/root"})
    assert bench.profiler_attached({"LD_PRELOAD": "/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so"})
    assert bench.profiler_attached({"ROCPROF_KERNEL_TRACE": "1"})
    assert bench.profiler_attached({"ROCP_TOOL_LIBRARIES": "x"})


def test_op_rotation_exceeds_infinity_cache_for_every_op():
    """make_sets sizes the rotation by the op with the fewest bytes, so every op timed over
    the sets moves at least 3x the 256 MB Infinity Cache before it revisits a set."""
    for shape, T in ((LY.GEMMA_4B, 2048), (LY.GEMMA_27B, 8192)):
        ob = LY.op_bytes(shape, T, 2)
        nsets = min(64, max(2, math.ceil(3 * bench.MALL_BYTES / min(ob.values()))))
        for name, b in ob.items():
            assert nsets * b >= 3 * bench.MALL_BYTES, (shape.name, name)


def test_in_place_mixes():
    mix = bench.op_mix(LY.GEMMA_4B, 2048, 2)
    assert mix["norm_add"][3] and mix["norm_add_norm"][3] and mix["add_rmsnorm"][3]
    assert not mix["input_norm"][3] and not mix["geglu"][3]


def test_op_streams_match_mixes():
    """The op-buffer ceiling reads and writes what op_mix says each op moves: the same number
    of streams, in place exactly where the op rewrites its first input."""
    class L:  # stand-in buffers: only identity matters
        pass
    lb = L()
    for name in ("x", "xb", "ao", "fo", "gate", "up", "act"):
        setattr(lb, name, object())
    mix = bench.op_mix(LY.GEMMA_4B, 2048, 2)
    covered = 0
    for name, (r, w, _, inplace) in mix.items():
        st = bench.op_streams(name, lb)
        if st is None:
            assert name == "qk_norm_rope_kv"
            continue
        covered += 1
        n_in, n_out, i0, i1, o0, o1 = st
        assert (n_in, n_out) == (r, w), name
        assert (i1 is not None) == (n_in == 2) and (o1 is not None) == (n_out == 2), name
        assert (o0 is i0) == inplace, name
    assert covered == 6


def test_qk_copies_match_op_bytes():
    """The QK ceiling's copies read and write the QK op's activation bytes (its algorithmic
    bytes less the two norm-weight rows and the positions): Q in place, K / V to the caches."""
    class L:
        pass
    s, T = LY.GEMMA_4B, 2048
    lb = L()
    lb.shape, lb.T, lb.esize = s, T, 2
    for name in ("q", "k", "v", "kc", "vc"):
        setattr(lb, name, object())
    pairs = bench.op_copies("qk_norm_rope_kv", lb)
    assert [(a is lb.q, b is lb.q) for a, b, _ in pairs][0] == (True, True)
    assert pairs[1][0] is lb.k and pairs[1][1] is lb.kc and pairs[2][0] is lb.v and pairs[2][1] is lb.vc
    algo = LY.op_bytes(s, T, 2, pos_array=True)["qk_norm_rope_kv"] - 2 * 4 * s.D - 4 * T
    assert 2 * sum(nb for _, _, nb in pairs) == algo
    assert bench.op_copies("geglu", lb) is None
