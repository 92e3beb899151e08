"""Build recipe for the gfx950 kernel library and its host-side companions.

Outputs (in-tree, git-ignored, shipped with the source tree to the GPU box):

* ``lib/libq3k.so``           HIP kernels + the C ABI (``include/q3k_abi.h``),
                               compiled for gfx950 with hipcc.
* ``lib/libq3k_bench.so``     the benchmark's measurement kernels
                               (``include/q3k_bench.h``), kept out of libq3k.so.
* ``lib/libqwen3_runtime.so`` the C++ ``qwen3::`` core tensor layer and the
                               ``qwen3::ops`` drop-in API, linked to libq3k.so.
* ``tests/cpp/build/*``       C++ test executables (built only when their
                               sources exist).
* ``bin/q3k_weight_io_bench``  the weight IO measurement (``bench/*.cpp``).
* ``oracle/build/libq3k_oracle.so`` the CPU oracle (test infrastructure),
                               built through ``oracle/Makefile``.
* ``oracle/_ref/*``           the reference's own test programs compiled
                               against this library (``oracle/reference_programs.mk``),
                               only where the reference's sources are present.

Every call recompiles everything (``build()`` is the "does it build" check).
"""
from __future__ import annotations

import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
OBJ_DIR = os.path.join(PKG_DIR, "build")
KERNEL_DIR = os.path.join(PKG_DIR, "csrc", "kernels")
HOST_DIRS = [os.path.join(PKG_DIR, "csrc", d) for d in ("core", "ops", "model", "generation", "io")]
ORACLE_DIR = os.path.join(REPO_DIR, "oracle")
CPP_TEST_DIR = os.path.join(REPO_DIR, "tests", "cpp")
BENCH_DIR = os.path.join(PKG_DIR, "bench")
BIN_DIR = os.path.join(PKG_DIR, "bin")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# Device flags: gfx950 only; no fp contraction (rounding points are part of
# the contract); packed-fp32 instructions disabled.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core accumulators in ordinary VGPRs: the attention loop rescales
    # them with VALU ops, and AGPR copies would cost ~128 moves per key tile
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE_DIR}",
]
CXX_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
    f"-I{INCLUDE_DIR}", f"-I{os.path.join(ROCM, 'include')}",
]
RPATH = [f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-Wl,-rpath,$ORIGIN"]

# Per-file device flags.  Element-wise and RoPE kernels: arguments preloaded
# into SGPRs at wave launch instead of loaded from the kernarg segment
# (SwiGLU [64, 12288] replayed from a HIP graph: 2.43 against 2.55 us;
# [8192, 1536]: 13.8 against 14.1 us; config 4's Q/K norm + RoPE 27.1 against
# 27.4 us, RoPE over Q and K 26.8 against 27.1 us, in alternating runs on one
# box).  Not for the RMSNorm file: add + RMSNorm at config 4 ran 43.1 against
# 42.9 us with it.
_PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]
FILE_FLAGS = {"elementwise.hip": _PRELOAD, "rope.hip": _PRELOAD}


def _run(cmd, cwd=None, verbose=False):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip() and verbose:
        print(out, flush=True)
    return out


def _parallel(jobs, verbose):
    workers = min(8, max(1, len(jobs)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        futures = [pool.submit(_run, cmd, None, verbose) for cmd in jobs]
        for f in futures:
            f.result()


def build_kernels(verbose=False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    obj_dir = os.path.join(OBJ_DIR, "kernels")
    os.makedirs(obj_dir, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(KERNEL_DIR, "*.hip")))
    objects, jobs = [], []
    for src in sources:
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        objects.append(obj)
        jobs.append([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj])
    _parallel(jobs, verbose)
    out = os.path.join(LIB_DIR, "libq3k.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objects, *RPATH], verbose=verbose)
    os.replace(tmp, out)
    return out


def build_bench_kernels(verbose=False) -> str:
    """lib/libq3k_bench.so: the benchmark's measurement kernels (include/q3k_bench.h)."""
    src = os.path.join(BENCH_DIR, "bench_kernels.hip")
    obj = os.path.join(OBJ_DIR, "bench_kernels.hip.o")
    os.makedirs(OBJ_DIR, exist_ok=True)
    _run([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj], verbose=verbose)
    out = os.path.join(LIB_DIR, "libq3k_bench.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, obj, *RPATH], verbose=verbose)
    os.replace(tmp, out)
    return out


def build_runtime(verbose=False) -> str | None:
    sources = []
    for d in HOST_DIRS:
        sources += sorted(glob.glob(os.path.join(d, "*.cpp")))
    if not sources:
        return None
    obj_dir = os.path.join(OBJ_DIR, "host")
    os.makedirs(obj_dir, exist_ok=True)
    objects, jobs = [], []
    for src in sources:
        rel = os.path.relpath(src, os.path.join(PKG_DIR, "csrc")).replace(os.sep, "_")
        obj = os.path.join(obj_dir, rel + ".o")
        objects.append(obj)
        jobs.append(["g++", *CXX_FLAGS, "-pthread", "-c", src, "-o", obj])
    _parallel(jobs, verbose)
    out = os.path.join(LIB_DIR, "libqwen3_runtime.so")
    tmp = out + ".tmp"
    _run(["g++", "-shared", "-pthread", "-o", tmp, *objects, f"-L{LIB_DIR}", "-lq3k",
          f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64", *RPATH], verbose=verbose)
    os.replace(tmp, out)
    return out


def build_oracle(verbose=False) -> str:
    _run(["make", "-B", "-C", ORACLE_DIR], verbose=verbose)
    return os.path.join(ORACLE_DIR, "build", "libq3k_oracle.so")


def build_reference_programs(verbose=False) -> str | None:
    """The reference's own test programs against this library (``oracle/reference_programs.mk``), where the
    reference's sources are present; None elsewhere."""
    ref = os.environ.get("Q3K_REFERENCE_DIR", "/root/reference")
    if not os.path.isdir(os.path.join(ref, "tests", "unit")):
        return None
    _run(["make", "-B", "-j8", "-C", ORACLE_DIR, "-f", "reference_programs.mk", f"REF={ref}"], verbose=verbose)
    return os.path.join(ORACLE_DIR, "_ref")


def build_cpp_tests(verbose=False) -> list[str]:
    sources = sorted(glob.glob(os.path.join(CPP_TEST_DIR, "*.cpp")))
    if not sources:
        return []
    out_dir = os.path.join(CPP_TEST_DIR, "build")
    os.makedirs(out_dir, exist_ok=True)
    jobs, outs = [], []
    for src in sources:
        exe = os.path.join(out_dir, os.path.splitext(os.path.basename(src))[0])
        outs.append(exe)
        jobs.append(["g++", *CXX_FLAGS, f"-I{ORACLE_DIR}", src, "-o", exe,
                     f"-L{LIB_DIR}", "-lqwen3_runtime", "-lq3k",
                     os.path.join(ORACLE_DIR, "build", "libq3k_oracle.so"),
                     f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64",
                     "-Wl,-rpath,$ORIGIN/" + os.path.relpath(LIB_DIR, out_dir),
                     "-Wl,-rpath,$ORIGIN/" + os.path.relpath(os.path.join(ORACLE_DIR, "build"), out_dir),
                     f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-pthread"])
    _parallel(jobs, verbose)
    return outs


def build_benches(verbose=False) -> list[str]:
    sources = sorted(glob.glob(os.path.join(BENCH_DIR, "*.cpp")))
    os.makedirs(BIN_DIR, exist_ok=True)
    jobs, outs = [], []
    for src in sources:
        exe = os.path.join(BIN_DIR, "q3k_" + os.path.splitext(os.path.basename(src))[0])
        outs.append(exe)
        jobs.append(["g++", *CXX_FLAGS, src, "-o", exe, f"-L{LIB_DIR}", "-lqwen3_runtime", "-lq3k",
                     f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64",
                     "-Wl,-rpath,$ORIGIN/" + os.path.relpath(LIB_DIR, BIN_DIR),
                     f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-pthread"])
    _parallel(jobs, verbose)
    return outs


def build_all(verbose=False) -> dict:
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    result = {"kernels": build_kernels(verbose), "bench_kernels": build_bench_kernels(verbose),
              "oracle": build_oracle(verbose)}
    result["runtime"] = build_runtime(verbose)
    result["cpp_tests"] = build_cpp_tests(verbose) if result["runtime"] else []
    result["reference_programs"] = build_reference_programs(verbose) if result["runtime"] else None
    result["benches"] = build_benches(verbose) if result["runtime"] else []
    return result


if __name__ == "__main__":
    res = build_all(verbose="-v" in sys.argv)
    for k, v in res.items():
        print(f"{k}: {v}")
