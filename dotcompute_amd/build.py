"""Offline build of the gfx950 HIP backend (no JIT, no torch extension machinery).

Produces, in-tree:
  dotcompute_amd/lib/libdotcompute_hip.so     the C-ABI library (include/dotcompute_hip.h)
  dotcompute_amd/lib/dc_kernels_gfx950.hsaco  code object for the generic module-load path: the
                                              kernels generated from dotcompute_amd/kernels/*.cs
  dotcompute_amd/lib/libdotcompute_host.so    C++ host layer (orchestrator, LINQ provider, algorithms)
  dotcompute_amd/lib/libdotcompute_bench.so   measurement-only streaming probes (bench.py's ceilings;
                                              not part of the product library)
  dotcompute_amd/lib/dc_host_tests             C++ tests of the host layer
  dotcompute_amd/lib/dc_orchestrator_bench     end-to-end orchestrator timing (bench.py runs it)
Run: python -m dotcompute_amd.build
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
LIB = os.path.join(PKG, "lib")
BUILD = os.path.join(PKG, "_build")
GENERATED = os.path.join(BUILD, "generated")
KERNELS = os.path.join(PKG, "kernels")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Device flags: gfx950 only; packed-FP32 instructions disabled; one rounding per float operation
# (bit-exact LINQ maps); correctly rounded fp32 divide/sqrt (as .NET).
HIP_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
HIP_SOURCES = ["dc_runtime.hip", "dc_streaming.hip", "dc_linq.hip", "dc_gemm.hip", "dc_spmv.hip"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build_hip_library(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    out = os.path.join(LIB, "libdotcompute_hip.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out + ".tmp", *objs, "-lpthread", "-ldl"])
    os.replace(out + ".tmp", out)
    return out


def build_probe_library() -> str:
    """The measurement-only streaming probes (dotcompute_amd/probes), a library of their own so that
    the product library carries no benchmark code."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    obj = os.path.join(BUILD, "dc_bench_probes.o")
    _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(PKG, "probes", "dc_bench_probes.hip"), "-o", obj])
    out = os.path.join(LIB, "libdotcompute_bench.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out + ".tmp", obj])
    os.replace(out + ".tmp", out)
    return out


def generate_kernels() -> list:
    """Translates the [Kernel] methods of dotcompute_amd/kernels/*.cs: the HIP kernels go into the
    code object, the registry into the host library (KernelRegistry.g.cpp)."""
    sys.path.insert(0, ROOT)
    from dotcompute_amd.generator import generate

    cs = sorted(os.path.join(KERNELS, f) for f in os.listdir(KERNELS) if f.endswith(".cs"))
    return generate(cs, GENERATED, root=ROOT)


def build_code_object() -> str:
    """The code object of the module-load path: generated kernels + csr_spmv. -fwrapv gives signed
    integer overflow C#'s wrapping meaning; divide and sqrt are correctly rounded, as in .NET."""
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "dc_kernels_gfx950.hsaco")
    _run([HIPCC, "--genco", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-ffp-contract=off", "-fwrapv",
          "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", GENERATED, "-I", CSRC, os.path.join(CSRC, "dc_module_kernels.hip"), "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_host_layer() -> str:
    """C++ host layer (g++, links libdotcompute_hip.so) and its test binary (tests/cpp, which also
    links the CPU oracle as its checker)."""
    srcs = sorted(os.path.join(HOST, "src", f) for f in os.listdir(os.path.join(HOST, "src")) if f.endswith(".cpp"))
    srcs.append(os.path.join(GENERATED, "KernelRegistry.g.cpp"))
    inc = ["-I", os.path.join(HOST, "include"), "-I", os.path.join(ROOT, "include")]
    flags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter", "-pthread", "-ffp-contract=off"]
    out = os.path.join(LIB, "libdotcompute_host.so")
    _run(["g++", *flags, *inc, "-shared", "-o", out + ".tmp", *srcs, "-L", LIB, "-ldotcompute_hip",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(out + ".tmp", out)
    tests = os.path.join(ROOT, "tests", "cpp")
    tsrcs = sorted(os.path.join(tests, f) for f in os.listdir(tests) if f.endswith(".cpp"))
    tbin = os.path.join(LIB, "dc_host_tests")
    oracle_dir = os.path.join(ROOT, "oracle")
    _run(["g++", *flags, *inc, "-o", tbin + ".tmp", *tsrcs, "-L", LIB, "-ldotcompute_host", "-ldotcompute_hip",
          "-L", oracle_dir, "-loracle", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,$ORIGIN/../../oracle"])
    os.replace(tbin + ".tmp", tbin)
    bbin = os.path.join(LIB, "dc_orchestrator_bench")
    _run(["g++", *flags, *inc, "-o", bbin + ".tmp", os.path.join(HOST, "bench", "orchestrator_bench.cpp"), "-L", LIB,
          "-ldotcompute_host", "-ldotcompute_hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(bbin + ".tmp", bbin)
    return out


def build_oracle() -> str:
    subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle")], check=True)
    return os.path.join(ROOT, "oracle", "liboracle.so")


def build_all() -> None:
    generate_kernels()
    with cf.ThreadPoolExecutor(max_workers=4) as ex:
        f_lib = ex.submit(build_hip_library)
        f_co = ex.submit(build_code_object)
        f_or = ex.submit(build_oracle)
        f_pr = ex.submit(build_probe_library)
        f_lib.result()
        f_pr.result()
        f_co.result()
        f_or.result()
    build_host_layer()


if __name__ == "__main__":
    build_all()
    print("built:", sorted(os.listdir(LIB)))
