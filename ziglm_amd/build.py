"""Build recipe for libhip_bridge.so (gfx950) and the CPU oracle.

    python -m ziglm_amd.build            # compile everything
    python -m ziglm_amd.build --check    # compile, then load the library (no GPU needed)

Every HIP source is compiled with:
  --offload-arch=gfx950        MI355X only
  -ffp-contract=off            no implicit FMA: f32 expressions round as written, matching
                               ziglm's CPU arithmetic (kernels call fmaf where they want one)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                               no packed-FP32 VALU instructions (v_pk_*_f32)
The library links only the HIP runtime; it never loads the oracle.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libhip_bridge.so")
ORACLE_DIR = os.path.join(ROOT, "oracle")

SOURCES = ["runtime.hip", "embed.hip", "norm.hip", "rope_kv.hip", "elementwise.hip", "gemv.hip", "gemm.hip",
           "attention.hip", "argmax.hip", "stream.hip", "gguf.cpp"]

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"),
]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32-ops feature; that warning is harmless.
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def compile_one(src, extra=()):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    out = _run(cmd)
    return obj, out


def build_bridge(verbose=False, jobs=None, out=LIB, defines=()):
    """Compile all sources and link `out`; `defines` are extra -D flags (variants)."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    extra = tuple(f"-D{d}" for d in defines)
    tag = "_".join(d.replace("=", "") for d in defines)

    def one(src):
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + (f".{tag}" if tag else "") + ".o")
        cmd = [HIPCC, *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        return obj, _run(cmd)

    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(one, SOURCES))
    for obj, msg in results:
        if msg and verbose:
            print(msg)
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *[o for o, _ in results]])
    os.replace(tmp, out)
    return out


def build_oracle():
    _run(["make", "-s", "-B", "-C", ORACLE_DIR])
    return [os.path.join(ORACLE_DIR, n) for n in ("liboracle.so", "liboracle_simd.so")]


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true", help="load the built library afterwards")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args(argv)
    lib = build_bridge(verbose=a.verbose)
    print("built", lib)
    for p in build_oracle():
        print("built", p)
    if a.check:
        sys.path.insert(0, ROOT)
        from ziglm_amd import bridge

        b = bridge.load()
        print("loaded", b.path, "-", b.version())


if __name__ == "__main__":
    main()
