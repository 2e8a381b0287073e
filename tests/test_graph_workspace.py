"""The torch shim's per-stream workspace under HIP graph capture.

The C ABI needs the zero region at the start of a GEMM workspace to be zero on
entry (K-slice arrival counters and exchange slots) and leaves it zero.  The
shim keeps one workspace per (device, stream); these tests replay captured
graphs after the things that used to break them:

* an eager call on the capture stream that needs a larger workspace (the old
  buffer, baked into the graph, must stay alive and untouched);
* a first allocation inside a capture (its zero fill is a graph node that
  never ran eagerly: eager calls on that stream must still see zeros);
* a warm-up on a side stream, then torch's own capture stream;
* two graphs captured on one stream whose second capture grows the workspace.

Every replay must equal the eager result bit for bit: the plans are the same
and every reduction is in a fixed order.
"""

import pytest
import torch

from pulsar_amd import ops

pytestmark = pytest.mark.gpu

G = 128


def _weights(k, n, seed, act_order=False):
    gen = torch.Generator(device="cuda:0").manual_seed(seed)
    qweight = torch.randint(-(2 ** 31), 2 ** 31, (k // 8, n), dtype=torch.int32, device="cuda:0", generator=gen)
    g_idx = None
    if act_order:
        p = torch.randperm(k, device="cuda:0", generator=gen)
        g_idx = torch.empty(k, dtype=torch.int32, device="cuda:0")
        g_idx[p] = torch.arange(k, device="cuda:0", dtype=torch.int32) // G
    wm, perm = ops.repack_w4a16_gptq(qweight, g_idx, G)
    scales = (torch.randn(k // G, n, device="cuda:0", generator=gen) * 0.02).abs_().add_(1e-3).half()
    qz = torch.randint(-(2 ** 31), 2 ** 31, (k // G, n // 8), dtype=torch.int32, device="cuda:0", generator=gen)
    return wm, scales, qz if act_order else None, perm if act_order else None


def _x(m, k, seed):
    gen = torch.Generator(device="cuda:0").manual_seed(seed)
    return torch.randn(m, k, device="cuda:0", generator=gen).half()


def _gemm(x, w):
    return ops.gemm_w4a16_gptq(x, w[0], w[1], w[2], w[3], G)


def _capture(stream, fn):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        out = fn()
    return g, out


def test_replay_after_eager_growth_on_capture_stream():
    """Capture a tree-split decode GEMM (down, M = 8: K slices reduced through
    the exchange slots of the zero region), then run a larger eager split-K
    prefill call on the same stream, then replay."""
    down = _weights(14336, 4096, seed=1)
    x8 = _x(8, 14336, seed=2)
    ref = _gemm(x8, down).clone()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        _gemm(x8, down)  # warm-up on the capture stream
    s.synchronize()
    g, out = _capture(s, lambda: _gemm(x8, down))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # a much larger workspace on the same stream: forced K slices write fp32 partials
    o = _weights(4096, 4096, seed=3)
    wm_ref, sm_ref = o[0], o[1].float()
    x256 = _x(256, 4096, seed=4)
    with torch.cuda.stream(s):
        big = ops.gemm_w4a16_marlin_split(x256, wm_ref, sm_ref, G, 8)
    s.synchronize()
    assert torch.equal(big, ops.gemm_w4a16_marlin_split(x256, wm_ref, sm_ref, G, 8))
    for _ in range(3):
        out.zero_()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert torch.equal(out, ref)


def test_first_allocation_inside_capture():
    """A fresh stream whose first GEMM call is captured: the workspace is
    allocated and zero-filled inside the graph.  Replays, and eager calls on
    that stream between them, must all be exact."""
    down = _weights(14336, 4096, seed=5)
    x8 = _x(8, 14336, seed=6)
    ref = _gemm(x8, down).clone()
    s = torch.cuda.Stream()
    g, out = _capture(s, lambda: _gemm(x8, down))
    for _ in range(2):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        with torch.cuda.stream(s):
            eager = _gemm(x8, down)
        s.synchronize()
        assert torch.equal(eager, ref)


def test_side_stream_warmup_then_default_capture_stream():
    """PyTorch's usual pattern: warm up on a side stream, capture with
    torch.cuda.graph's own capture stream."""
    down = _weights(14336, 4096, seed=7)
    x16 = _x(16, 14336, seed=8)
    ref = _gemm(x16, down).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _gemm(x16, down)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = _gemm(x16, down)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


def test_two_graphs_on_one_stream_growing_workspace():
    """Act-order GEMMs gather x[:, perm] into the workspace: capturing M = 1 and
    then M = 16 on one stream grows it during the second capture.  The first
    graph keeps its own (smaller) buffer."""
    w = _weights(8192, 1024, seed=9, act_order=True)
    x1, x16 = _x(1, 8192, seed=10), _x(16, 8192, seed=11)
    ref1, ref16 = _gemm(x1, w).clone(), _gemm(x16, w).clone()
    s = torch.cuda.Stream()
    g1, out1 = _capture(s, lambda: _gemm(x1, w))
    g16, out16 = _capture(s, lambda: _gemm(x16, w))
    for _ in range(2):
        out1.zero_()
        out16.zero_()
        g1.replay()
        g16.replay()
        g1.replay()
        torch.cuda.synchronize()
        assert torch.equal(out1, ref1)
        assert torch.equal(out16, ref16)
        with torch.cuda.stream(s):
            e1 = _gemm(x1, w)
        s.synchronize()
        assert torch.equal(e1, ref1)


def _graph_nodes(g) -> int:
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
    hip.hipGraphGetNodes.restype = ctypes.c_int
    n = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(ctypes.c_void_p(g.raw_cuda_graph()), None, ctypes.byref(n)) == 0
    return n.value


def _fresh_stream():
    """A stream the shim has never seen (its workspace cache is keyed by stream)."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamCreate.restype = ctypes.c_int
    p = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(p)) == 0
    return torch.cuda.ExternalStream(p.value)


def test_one_zero_fill_per_capture():
    """Several split calls captured on a stream with no eager call before: the
    graph holds ONE fill of the workspace's zero region (not one per call, not
    of the whole buffer), and its replays and the eager calls between them are
    exact.  Node counts are compared with the same calls captured on a stream
    whose workspace an eager call has already cleared (no fill at all)."""
    down = _weights(14336, 4096, seed=12)
    o = _weights(4096, 4096, seed=13)
    x8, x256 = _x(8, 14336, seed=14), _x(256, 4096, seed=15)
    sm = o[1].float()

    # the largest workspace first: a buffer that grows inside the capture is a
    # new allocation, which needs (and gets) a fill of its own
    def calls():
        return [ops.gemm_w4a16_marlin_split(x256, o[0], sm, G, 4),  # K-slice partials + combine
                _gemm(x8, down),                                   # exchange-tree decode
                _gemm(x8, down)]

    refs = [t.clone() for t in calls()]
    warm = _fresh_stream()
    with torch.cuda.stream(warm):
        calls()
    warm.synchronize()
    gw = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(gw, stream=warm):
        calls()
    cold = _fresh_stream()
    gc = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(gc, stream=cold):
        outs = calls()
    assert _graph_nodes(gc) == _graph_nodes(gw) + 1, (_graph_nodes(gc), _graph_nodes(gw))
    for _ in range(3):
        for t in outs:
            t.zero_()
        gc.replay()
        torch.cuda.synchronize()
        for t, r in zip(outs, refs):
            assert torch.equal(t, r)
        with torch.cuda.stream(cold):
            eager = calls()
        cold.synchronize()
        for t, r in zip(eager, refs):
            assert torch.equal(t, r)
