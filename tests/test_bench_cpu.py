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
