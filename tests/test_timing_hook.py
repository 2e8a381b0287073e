"""The kernel timing hook (pw4_time_next_kernel): an armed GEMM call launches the
decode kernel through hipExtLaunchKernel with the caller's events, which then
bracket that dispatch alone; an armed repack call brackets its one repack
dispatch (words and scales together).  The output is the same as an unarmed call's, the interval is
positive and inside the events recorded around the call, and the arming is used
up by one call."""

import numpy as np
import pytest
import torch

import pulsar_amd
from oracle import oracle as O
from pulsar_amd import ops

pytestmark = pytest.mark.gpu


def test_armed_launch_times_the_kernel_alone():
    lib = pulsar_amd.capi()
    n, k, g = 4096, 4096, 128
    rng = np.random.default_rng(5)
    u = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
    s = torch.from_numpy((np.abs(rng.standard_normal((k // g, n))) * 0.02 + 1e-3).astype(np.float16)).cuda()
    wm, _ = ops.repack_w4a16_gptq(torch.from_numpy(O.pack_gptq(u)).cuda(), None, g)
    x = torch.randn(4, k, device="cuda:0").half()
    stream = torch.cuda.current_stream()
    y0 = ops.gemm_w4a16_gptq(x, wm, s, None, None, g)

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in ev:
        e.record(stream)  # creates the events
    ev[0].record(stream)
    assert lib.pw4_time_next_kernel(ev[2], ev[3]) == 0
    y1 = ops.gemm_w4a16_gptq(x, wm, s, None, None, g)
    ev[1].record(stream)
    torch.cuda.synchronize()
    kernel_ms, call_ms = ev[2].elapsed_time(ev[3]), ev[0].elapsed_time(ev[1])
    assert torch.equal(y0, y1)
    assert 0.0 < kernel_ms <= call_ms
    # used up: a second call leaves the kernel events where they were
    y2 = ops.gemm_w4a16_gptq(x, wm, s, None, None, g)
    torch.cuda.synchronize()
    assert torch.equal(y0, y2)
    assert ev[2].elapsed_time(ev[3]) == kernel_ms


def test_armed_repack_times_its_kernels():
    lib = pulsar_amd.capi()
    n, k, g = 4096, 4096, 128
    packed = torch.randint(-(2 ** 31), 2 ** 31, (n, k // 8), dtype=torch.int32, device="cuda:0")
    scale = (torch.randn(n, k // g, device="cuda:0") * 0.02).abs_().add_(1e-3).half()
    stream = torch.cuda.current_stream()
    w0, s0 = ops.repack_w4a16(packed, scale, g)

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in ev:
        e.record(stream)  # creates the events
    ev[0].record(stream)
    assert lib.pw4_time_next_kernel(ev[2], ev[3]) == 0
    w1, s1 = ops.repack_w4a16(packed, scale, g)
    ev[1].record(stream)
    torch.cuda.synchronize()
    kernel_ms, call_ms = ev[2].elapsed_time(ev[3]), ev[0].elapsed_time(ev[1])
    assert torch.equal(w0, w1) and torch.equal(s0, s1)
    assert 0.0 < kernel_ms <= call_ms
    # used up: the next GEMM call is not timed into these events
    x = torch.randn(1, k, device="cuda:0").half()
    ops.gemm_w4a16_marlin(x, w1, s1, g)
    torch.cuda.synchronize()
    assert ev[2].elapsed_time(ev[3]) == kernel_ms


def test_armed_gptq_repack_times_its_kernel():
    lib = pulsar_amd.capi()
    n, k, g = 1024, 4096, 128
    rng = np.random.default_rng(8)
    qweight = torch.from_numpy(O.pack_gptq(rng.integers(0, 16, size=(n, k)).astype(np.uint8))).cuda()
    stream = torch.cuda.current_stream()
    w0, _ = ops.repack_w4a16_gptq(qweight, None, g)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in ev:
        e.record(stream)  # creates the events
    ev[0].record(stream)
    assert lib.pw4_time_next_kernel(ev[2], ev[3]) == 0
    w1, _ = ops.repack_w4a16_gptq(qweight, None, g)
    ev[1].record(stream)
    torch.cuda.synchronize()
    kernel_ms, call_ms = ev[2].elapsed_time(ev[3]), ev[0].elapsed_time(ev[1])
    assert torch.equal(w0, w1)
    assert 0.0 < kernel_ms <= call_ms
