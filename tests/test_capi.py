"""CPU-side checks of the drop-in boundary: the C ABI library loads and exports
every entry point include/pulsar_w4a16.h declares, argument checks fire before
any launch, workspace queries are consistent, and the torch op schemas and
fake kernels match the reference (pulsar/ext/ops.cpp:39-52,
pulsar/src/pulsar/core/ops.py:117-165).  No kernel runs here."""

import ctypes
import os
import re

import pytest
import torch

import pulsar_amd
from pulsar_amd import ops
from pw4_capi import declare

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pulsar_w4a16.h")

P = ctypes.c_void_p
I64 = ctypes.c_int64


@pytest.fixture(scope="module")
def lib():
    return declare(pulsar_amd.capi())


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pw4_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), f"{name} declared in pulsar_w4a16.h but not exported"


def test_status_strings_and_version(lib):
    assert lib.pw4_status_string(0) == b"ok"
    for code in (-1, -2, -3, -4, -5):
        assert lib.pw4_status_string(code) != b"unknown status"
    assert lib.pw4_abi_version() == 2


def test_timing_hook_arguments(lib):
    # one event without the other is rejected and arms nothing; (NULL, NULL) disarms
    assert lib.pw4_time_next_kernel(None, P(0x1000)) == -1
    assert lib.pw4_time_next_kernel(P(0x1000), None) == -1
    assert lib.pw4_time_next_kernel(None, None) == 0


def test_marlin_words_matches_oracle(lib, orc):
    for n, k in [(128, 256), (100, 136), (4096, 14336), (1, 8), (0, 64)]:
        assert lib.pw4_marlin_words(n, k) == orc.marlin_words(n, k)


def test_argument_checks_fire_before_launch(lib):
    dummy = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    # group_size not a multiple of 16 (reference w4a16_gemm.cu:339)
    assert lib.pw4_gemm_w4a16(dummy, 0, dummy, dummy, dummy, 4, 64, 128, 24, 0, None, 0, None) == -2
    # K not a multiple of group_size (w4a16_gemm.cu:344)
    assert lib.pw4_gemm_w4a16(dummy, 0, dummy, dummy, dummy, 4, 64, 160, 64, 0, None, 0, None) == -2
    # K % 8 != 0 (w4a16_gemm.cu:340-343)
    assert lib.pw4_gemm_w4a16(dummy, 0, dummy, dummy, dummy, 4, 64, 20, 16, 0, None, 0, None) == -2
    # bad x dtype / null pointers / negative splits
    assert lib.pw4_gemm_w4a16(dummy, 7, dummy, dummy, dummy, 4, 64, 128, 64, 0, None, 0, None) == -1
    assert lib.pw4_gemm_w4a16(None, 0, dummy, dummy, dummy, 4, 64, 128, 64, 0, None, 0, None) == -1
    assert lib.pw4_gemm_w4a16(dummy, 0, dummy, dummy, dummy, 4, 64, 128, 64, -1, None, 0, None) == -1
    # x and the weight words must be 16-byte aligned (read as 16-byte vectors)
    odd = ctypes.c_void_p(18)
    assert lib.pw4_gemm_w4a16(odd, 0, dummy, dummy, dummy, 4, 64, 128, 64, 0, None, 0, None) == -1
    assert lib.pw4_gemm_w4a16_marlin(dummy, 0, odd, dummy, 2, None, None, dummy, 4, 64, 128, 64, 0, None, 0,
                                     None) == -1
    # SiLU-gated GEMM: N (gate|up interleaved by 8) must be a multiple of 16; scale dtype
    assert lib.pw4_gemm_w4a16_silu_mul(dummy, 0, dummy, dummy, 0, None, None, dummy, 4, 24, 128, 64, None, 0,
                                       None) == -2
    assert lib.pw4_gemm_w4a16_silu_mul(dummy, 0, dummy, dummy, 7, None, None, dummy, 4, 32, 128, 64, None, 0,
                                       None) == -1
    assert lib.pw4_gemm_w4a16_silu_mul(None, 0, None, None, 0, None, None, None, 0, 32, 128, 64, None, 0, None) == 0
    assert lib.pw4_gemm_w4a16_silu_mul_workspace_size(4, 24, 128, 64, 0) == 0
    # M == 0 and N == 0 are no-ops (w4a16_gemm.cu:355-357)
    assert lib.pw4_gemm_w4a16(None, 0, None, None, None, 0, 64, 128, 64, 0, None, 0, None) == 0
    assert lib.pw4_gemm_w4a16(None, 0, None, None, None, 4, 0, 128, 64, 0, None, 0, None) == 0
    # marlin: fp32/fp16 scales only; qzeros need N % 8 == 0
    assert lib.pw4_gemm_w4a16_marlin(dummy, 0, dummy, dummy, 1 + 1 + 5, None, None, dummy, 4, 64, 128, 64, 0,
                                     None, 0, None) == -1
    assert lib.pw4_gemm_w4a16_marlin(dummy, 0, dummy, dummy, 2, dummy, None, dummy, 4, 60, 128, 64, 0, None, 0,
                                     None) == -2
    # repack: group size, dtype
    assert lib.pw4_repack_w4a16(dummy, dummy, 2, 64, 128, 48, dummy, dummy, None) == -2
    assert lib.pw4_repack_w4a16(dummy, dummy, 9, 64, 128, 64, dummy, dummy, None) == -1
    # gidx: K % G
    assert lib.pw4_gidx_to_perm(dummy, 100, 64, dummy, dummy, None) == -2
    assert lib.pw4_repack_gptq(dummy, None, 64, 12, dummy, None) == -2


def test_workspace_queries(lib):
    # forced split: [splits, M, N] fp32 partials
    ws = lib.pw4_gemm_w4a16_workspace_size(4, 256, 512, 64, 3)
    assert ws >= 3 * 4 * 256 * 4
    assert lib.pw4_gemm_w4a16_workspace_size(0, 256, 512, 64, 3) == 0
    # act-order prefill needs room for the permuted activations
    ws_perm = lib.pw4_gemm_w4a16_marlin_workspace_size(512, 256, 512, 64, 1, 0)
    ws_noperm = lib.pw4_gemm_w4a16_marlin_workspace_size(512, 256, 512, 64, 0, 0)
    assert ws_perm >= ws_noperm + 512 * 512 * 2
    # act-order decode gathers x once per call into the workspace as well
    ws_perm1 = lib.pw4_gemm_w4a16_marlin_workspace_size(1, 256, 512, 64, 1, 0)
    assert ws_perm1 >= (16 << 20) + 512 * 2


def test_plan_overrides_are_live(lib):
    """The tests that pin a plan through PW4_* variables (tests/conftest.py
    enables them for the process) would compare a plan with itself if the
    library ignored them: an unforced prefill plan must follow
    PW4_PREFILL_SPLITS, which the workspace query shows as its fp32 partials."""
    M, N, K, G = 512, 4096, 4096, 128
    old = os.environ.get("PW4_PREFILL_SPLITS")
    try:
        os.environ["PW4_PREFILL_SPLITS"] = "1"
        unsplit = lib.pw4_gemm_w4a16_marlin_workspace_size(M, N, K, G, 0, 0)
        os.environ["PW4_PREFILL_SPLITS"] = "3"
        split3 = lib.pw4_gemm_w4a16_marlin_workspace_size(M, N, K, G, 0, 0)
    finally:
        if old is None:
            os.environ.pop("PW4_PREFILL_SPLITS", None)
        else:
            os.environ["PW4_PREFILL_SPLITS"] = old
    assert unsplit == 0
    assert split3 >= 3 * M * N * 4


def test_missing_workspace_is_rejected(lib):
    dummy = ctypes.c_void_p(16)
    assert lib.pw4_gemm_w4a16(dummy, 0, dummy, dummy, dummy, 4, 256, 512, 64, 3, None, 0, None) == -3


# ---- torch boundary ---------------------------------------------------------------------

REFERENCE_SCHEMAS = {
    "gemm_w4a16": "pulsar::gemm_w4a16(Tensor x, Tensor weight_packed, Tensor weight_scale, int group_size) -> Tensor",
    "gemm_w4a16_split": "pulsar::gemm_w4a16_split(Tensor x, Tensor weight_packed, Tensor weight_scale, "
                        "int group_size, int num_splits) -> Tensor",
    "repack_w4a16": "pulsar::repack_w4a16(Tensor weight_packed, Tensor weight_scale, int group_size) "
                    "-> (Tensor, Tensor)",
    "gemm_w4a16_marlin": "pulsar::gemm_w4a16_marlin(Tensor x, Tensor weight_marlin, Tensor scale_marlin, "
                         "int group_size) -> Tensor",
}


def test_reference_schemas_verbatim():
    for name, schema in REFERENCE_SCHEMAS.items():
        assert str(getattr(torch.ops.pulsar, name).default._schema) == schema


def test_fake_kernels_shapes():
    m, n, k, g = 5, 100, 136, 8
    x = torch.empty(m, k, dtype=torch.float16, device="meta")
    wp = torch.empty(n, k // 8, dtype=torch.int32, device="meta")
    ws = torch.empty(n, k // g, dtype=torch.float16, device="meta")
    assert torch.ops.pulsar.gemm_w4a16(x, wp, ws, g).shape == (m, n)
    assert torch.ops.pulsar.gemm_w4a16_split(x, wp, ws, g, 3).shape == (m, n)
    wm, sm = torch.ops.pulsar.repack_w4a16(wp, ws, g)
    assert wm.shape == (128 * 192 // 8,) and wm.dtype == torch.int32
    assert sm.shape == (k // g, n) and sm.dtype == torch.float32
    assert torch.ops.pulsar.gemm_w4a16_marlin(x, wm, sm, g).shape == (m, n)
    qw = torch.empty(k // 8, n, dtype=torch.int32, device="meta")
    wm2, perm = torch.ops.pulsar.repack_w4a16_gptq(qw, None, g)
    assert wm2.shape == wm.shape and perm.shape == (0,)
    gi = torch.empty(k, dtype=torch.int32, device="meta")
    assert torch.ops.pulsar.repack_w4a16_gptq(qw, gi, g)[1].shape == (k,)
    assert ops.gemm_w4a16_gptq(x, wm, sm.half(), None, None, g).shape == (m, n)
