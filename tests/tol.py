"""Parity tolerances for the HIP kernels against the CPU oracle (stated per test)."""
import numpy as np


def assert_bitexact(gpu, ref, what=""):
    g = np.ascontiguousarray(gpu)
    r = np.ascontiguousarray(ref)
    assert g.shape == r.shape and g.dtype == r.dtype, (what, g.shape, r.shape, g.dtype, r.dtype)
    ut = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[g.dtype.itemsize]
    gb, rb = g.view(ut).reshape(-1), r.view(ut).reshape(-1)
    bad = np.flatnonzero(gb != rb)
    if bad.size:
        i = bad[:5]
        raise AssertionError(f"{what}: not bit-exact, {bad.size} of {gb.size} differ; idx {i} "
                             f"gpu={g.reshape(-1)[i]} ref={r.reshape(-1)[i]}")


def assert_rel(gpu, ref, rtol=1e-5, floor=0.0, what=""):
    """|gpu - ref| <= rtol*|ref| + floor elementwise (floor: scalar or array)."""
    g = np.asarray(gpu, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    assert np.all(np.isfinite(g) == np.isfinite(r)), f"{what}: finiteness differs"
    fin = np.isfinite(r)
    err = np.abs(g - r)
    bound = rtol * np.abs(r) + floor
    bad = np.flatnonzero(fin & (err > bound))
    if bad.size:
        i = bad[:5]
        raise AssertionError(
            f"{what}: {bad.size} of {r.size} outside rtol={rtol} (+floor); idx {i} "
            f"gpu={g.reshape(-1)[i]} ref={r.reshape(-1)[i]} "
            f"max rel={np.max(err.reshape(-1)[bad] / np.maximum(np.abs(r.reshape(-1)[bad]), 1e-300)):.3e}")


def bf16_key(u):
    u = np.asarray(u, dtype=np.uint16).astype(np.int32)
    return np.where(u & 0x8000, -(u & 0x7FFF), u)


def bf16_f32(u):
    return (np.asarray(u, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_bf16(gpu_u16, ref_u16, max_ulp=1, floor=None, what=""):
    """bf16 outputs within max_ulp units in the last place; where `floor` (f32 array/scalar)
    is given, a difference up to floor + one bf16 ulp of the larger value also passes."""
    d = np.abs(bf16_key(gpu_u16) - bf16_key(ref_u16))
    ok = d <= max_ulp
    if floor is not None:
        g = bf16_f32(gpu_u16).astype(np.float64)
        r = bf16_f32(ref_u16).astype(np.float64)
        mag = np.maximum(np.abs(g), np.abs(r)).astype(np.float32)
        ulp = np.spacing(mag.astype(np.float32)).astype(np.float64) * 65536.0
        ok |= np.abs(g - r) <= floor + ulp
    bad = np.flatnonzero(~ok.reshape(-1))
    if bad.size:
        i = bad[:5]
        raise AssertionError(f"{what}: {bad.size} of {d.size} beyond {max_ulp} bf16 ulp; idx {i} "
                             f"gpu={bf16_f32(gpu_u16).reshape(-1)[i]} ref={bf16_f32(ref_u16).reshape(-1)[i]} "
                             f"ulp={d.reshape(-1)[i]}")
    return int(d.max()) if d.size else 0
