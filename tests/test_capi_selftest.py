"""The torch-free C++ caller of the C ABI (pulsar_amd/csrc/capi_selftest.cpp,
built as pulsar_amd/pw4_selftest by pulsar_amd/build.py).

It stands for a non-ATen C++ caller of the reference's operators
(pulsar-core/inc/pulsar/ops.hpp:156-189): hipMalloc'd memory, one workspace
cleared once, pw4_repack_w4a16 then GEMM calls that take the decode, K-split,
prefill and compressed-tensors plans, status codes for the reference's
precondition checks, each result checked against a double-precision CPU GEMM.

The CPU test checks that the program links the library and the HIP runtime but
no part of torch.  The GPU test runs it as a child process of pytest (which
does not touch the GPU itself in this test) and requires exit status 0.
"""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "pulsar_amd", "pw4_selftest")


def _exe() -> str:
    if not os.path.exists(EXE):
        raise RuntimeError(f"{EXE} not built; run `python -m pulsar_amd.build`")
    return EXE


@pytest.mark.skipif(shutil.which("ldd") is None, reason="ldd not available")
def test_selftest_links_no_torch():
    out = subprocess.run(["ldd", _exe()], capture_output=True, text=True, check=True).stdout
    libs = [ln.split()[0] for ln in out.splitlines() if ln.strip()]
    assert any(name.startswith("libpulsar_w4a16.so") for name in libs), out
    assert any(name.startswith("libamdhip64.so") for name in libs), out
    assert not [n for n in libs if "torch" in n or n.startswith("libc10")], out


@pytest.mark.gpu
def test_selftest_passes_on_gpu():
    print(f"running {EXE}", flush=True)
    r = subprocess.run([_exe(), "-v"], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all cases passed" in r.stdout
    assert "FAIL" not in r.stdout
    assert sum(ln.startswith("ok ") for ln in r.stdout.splitlines()) >= 11, r.stdout
    assert any(ln.startswith("ok ") and "K windows" in ln for ln in r.stdout.splitlines()), r.stdout
