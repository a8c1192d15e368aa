"""The C++ host interface (include/hip_device.hpp, mirroring ziglm's CudaDevice) compiles
and links against libhip_bridge.so (CPU), and a C++ decode step in the reference's own op
order reproduces the golden c1 fixture on the GPU."""
import os
import subprocess

import numpy as np
import pytest

from tol import assert_bitexact, assert_rel
from ziglm_amd import bridge

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "cpp", "decode_step.cpp")


def build(tmp_path):
    exe = str(tmp_path / "decode_step")
    libdir = os.path.dirname(bridge.LIB_PATH)
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), SRC, "-o",
                    exe, "-L", libdir, "-lhip_bridge", f"-Wl,-rpath,{libdir}"], check=True)
    return exe


def test_cpp_host_interface_compiles_and_links(tmp_path):
    exe = build(tmp_path)
    assert os.path.exists(exe)
    # every symbol the program uses resolves at load time (no GPU call is made: bad usage)
    p = subprocess.run([exe], capture_output=True)
    assert p.returncode == 2


@pytest.mark.gpu
def test_cpp_decode_step_matches_fixture(tmp_path):
    from test_golden import load
    from test_gpu_parity import geglu_floor, pair_floor
    exe = build(tmp_path)
    g = load("c1_decode_seed0.npz")
    order = ["x", "residual", "w", "q", "k", "v", "wq", "wk", "gate", "up", "scores"]
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(fin, "wb") as f:
        for k in order:
            f.write(np.ascontiguousarray(g[k], np.float32).tobytes())
    subprocess.run([exe, str(fin), str(fout)], check=True, timeout=120)
    out = np.fromfile(fout, np.float32)
    H, nh, nkv, D, I, pos = (int(v) for v in g["meta"])
    sizes = [H, H, nh * D, nkv * D, nkv * D, I, g["scores"].size]
    parts = np.split(out, np.cumsum(sizes)[:-1])
    x, n, q, k, v, a, s = parts
    assert_bitexact(x, g["x_out"], "x+r")
    assert_rel(n, g["norm_out"], 1e-5, what="norm")
    assert_rel(q.reshape(nh, D), g["q_out"].reshape(nh, D), 1e-5, floor=pair_floor(g["q_out"].reshape(nh, D), D, 0))
    kr = g["k_row"].reshape(nkv, D)
    assert_rel(k.reshape(nkv, D), kr, 1e-5, floor=pair_floor(kr, D, 0))
    assert_bitexact(v, g["v_row"], "v row")
    assert_rel(a, g["geglu_out"], 1e-5, floor=geglu_floor(g["gate"], g["up"]))
    assert_rel(s, g["softcap_out"].reshape(-1), 1e-5)
