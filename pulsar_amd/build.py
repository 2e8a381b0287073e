"""In-tree build of the W4A16 libraries (no GPU needed: hipcc cross-compiles).

    python -m pulsar_amd.build

produces, next to this file,
  libpulsar_w4a16.so          HIP kernels + the C ABI of include/pulsar_w4a16.h
  _pulsar_w4a16_torch.so      at::Tensor API + torch.ops.pulsar registration, and the
                              C++ model layer of include/pulsar_w4a16_model.hpp
                              (torch.classes.pulsar.Qwen3W4A16Layer)
  libpw4_probe.so             a streaming-read probe that bench.py times for the
                              read-only HBM ceiling (measurement only; not part of
                              the library or its ABI)
  pw4_selftest                a torch-free C++ program that calls the C ABI on
                              hipMalloc'd memory and checks the results on the CPU
                              (links libpulsar_w4a16.so and the HIP runtime only)
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_SOURCES = ["repack.hip", "gemm_decode.hip", "gemm_prefill.hip", "gemm_prefill_256.hip", "capi.hip"]
LIB_NAME = "libpulsar_w4a16.so"
TORCH_LIB_NAME = "_pulsar_w4a16_torch.so"
TORCH_SOURCES = ["torch_ops.cpp", "model.cpp"]
PROBE_SOURCE = "probe.hip"
PROBE_LIB_NAME = "libpw4_probe.so"
SELFTEST_SOURCE = "capi_selftest.cpp"
SELFTEST_NAME = "pw4_selftest"

# gfx950 only.  Packed-fp32 instructions are disabled for the device pass; the
# host pass prints a harmless "not a recognized feature" warning for it.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    p = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found; the W4A16 library needs ROCm's hipcc")
    return p


def _run_parallel(cmds: list[list[str]], verbose: bool) -> None:
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for cmd, p in procs:
        out, _ = p.communicate()
        noise = "is not a recognized feature for this target"
        lines = [ln for ln in (out or "").splitlines() if noise not in ln]
        if p.returncode != 0:
            failed.append((cmd, "\n".join(lines)))
        elif verbose and lines:
            print("\n".join(lines))
    if failed:
        msg = "\n\n".join(f"$ {' '.join(c)}\n{o}" for c, o in failed)
        raise RuntimeError(f"build failed:\n{msg}")


# Per-file extras.  The decode GEMM keeps its small MFMA accumulators in
# VGPRs (no v_accvgpr moves around every 128-K step); the prefill GEMM needs
# the AGPRs for its large accumulator tile.
HIPCC_FILE_FLAGS = {
    "gemm_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def build_hip(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    objs, cmds = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *HIPCC_FILE_FLAGS.get(src, []), f"-I{INCLUDE}", f"-I{CSRC}", "-c",
                     os.path.join(CSRC, src), "-o", obj])
    _run_parallel(cmds, verbose)
    out = os.path.join(HERE, LIB_NAME)
    tmp = out + ".tmp"
    _run_parallel([[hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
                    "-Wl,--no-undefined", "-Wl,-soname," + LIB_NAME]], verbose)
    os.replace(tmp, out)
    return out


def build_torch(verbose: bool = False) -> str:
    import torch
    from torch.utils import cpp_extension

    torch_lib = cpp_extension.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{p}" for p in cpp_extension.include_paths()]
    py_inc = sysconfig.get_paths()["include"]
    out = os.path.join(HERE, TORCH_LIB_NAME)
    tmp = out + ".tmp"
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *inc, f"-I{py_inc}", f"-I{ROCM}/include", f"-I{INCLUDE}",
        *[os.path.join(CSRC, f) for f in TORCH_SOURCES], "-o", tmp,
        f"-L{HERE}", "-lpulsar_w4a16", f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
        "-ltorch_hip", f"-L{ROCM}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
    ]
    _run_parallel([cmd], verbose)
    os.replace(tmp, out)
    return out


def build_probe(verbose: bool = False) -> str:
    out = os.path.join(HERE, PROBE_LIB_NAME)
    tmp = out + ".tmp"
    _run_parallel([[_hipcc(), *HIPCC_FLAGS, "-shared", os.path.join(CSRC, PROBE_SOURCE), "-o", tmp]], verbose)
    os.replace(tmp, out)
    return out


def build_selftest(verbose: bool = False) -> str:
    """Host-only C++ (g++): no torch and no device code of its own."""
    out = os.path.join(HERE, SELFTEST_NAME)
    tmp = out + ".tmp"
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__=1",
        f"-I{ROCM}/include", f"-I{INCLUDE}", os.path.join(CSRC, SELFTEST_SOURCE), "-o", tmp,
        f"-L{HERE}", "-lpulsar_w4a16", f"-L{ROCM}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM}/lib",
    ]
    _run_parallel([cmd], verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    build_hip(verbose)
    build_torch(verbose)
    build_probe(verbose)
    build_selftest(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", os.path.join(HERE, LIB_NAME), os.path.join(HERE, TORCH_LIB_NAME))
