"""pw4_gemm_w4a16_marlin_noalloc, through the C ABI: the GEMM with no workspace
argument, whose scratch is a fixed device array in the library.  Each call's
output must equal pw4_gemm_w4a16_marlin's (same kernels, same plan, a
caller-owned workspace) bit for bit, on calls in a row that need the scratch
(exchange-tree slots and counters in its zero region, fp32 partials and the
act-order copy of x after it), each smaller than the one before; a call whose
plan needs more than PW4_NOALLOC_SCRATCH_BYTES is rejected before it launches."""

import numpy as np
import pytest

import pulsar_amd
from oracle import oracle as O
from pw4_capi import DTYPE_F16, DTYPE_F32, PW4_NOALLOC_SCRATCH_BYTES, Hip, declare

pytestmark = pytest.mark.gpu

G = 128


@pytest.fixture(scope="module")
def env():
    lib = declare(pulsar_amd.capi())
    hip = Hip()
    yield lib, hip
    hip.free_all()


def _operands(lib, hip, p):
    n, k = p.n, p.k
    wm = hip.malloc(lib.pw4_marlin_words(n, k) * 4)
    if p.g_idx is None:
        packed = hip.upload(p.ct_packed())
        sc = hip.upload(p.scale_nk.astype(np.float32))
        sm = hip.malloc(n * (k // G) * 4)
        assert lib.pw4_repack_w4a16(packed, sc, DTYPE_F32, n, k, G, wm, sm, None) == 0
        return wm, sm, DTYPE_F32, None, None
    gi = hip.upload(p.g_idx.astype(np.int32))
    perm = hip.malloc(k * 4)
    status = hip.malloc(4)
    assert lib.pw4_gidx_to_perm(gi, k, G, perm, status, None) == 0
    qw = hip.upload(p.qweight())
    assert lib.pw4_repack_gptq(qw, perm, n, k, wm, None) == 0
    return wm, hip.upload(O.f32_to_f16_bits(p.scale_kn)), DTYPE_F16, hip.upload(p.qzeros()), perm


# (M, N, K, num_splits, act_order), each call smaller than the one before
CALLS = [
    (300, 1040, 2048, 4, False),   # prefill K slices: partials in the scratch, combine
    (24, 2112, 28672, 0, False),   # decode, K windows (more slices than the tree takes; no scratch)
    (16, 2048, 14336, 0, False),   # decode, exchange-tree K slices in the zero region
    (8, 1024, 8192, 0, True),      # act-order: x[:, perm] gathered into the scratch
    (4, 512, 4096, 3, False),      # decode, forced K slices: counters + partials
    (1, 256, 1024, 0, False),      # decode, direct store (no scratch needed)
]


def test_noalloc_matches_workspace_entry_point(env):
    lib, hip = env
    for i, (m, n, k, splits, act) in enumerate(CALLS):
        p = O.make_problem(m, n, k, G, seed=90 + i, symmetric=not act, act_order=act)
        wm, sc, sdt, qz, perm = _operands(lib, hip, p)
        x = hip.upload(p.x16)
        need = lib.pw4_gemm_w4a16_marlin_workspace_size(m, n, k, G, int(act), splits)
        ws = hip.malloc(max(need, 1))
        hip.memset(ws, 0, max(need, 1))
        y_ws = hip.malloc(m * n * 2)
        y_na = hip.malloc(m * n * 2)
        hip.memset(y_na, 0xff, m * n * 2)
        assert lib.pw4_gemm_w4a16_marlin(x, DTYPE_F16, wm, sc, sdt, qz, perm, y_ws, m, n, k, G, splits, ws, need,
                                         None) == 0
        rc = lib.pw4_gemm_w4a16_marlin_noalloc(x, DTYPE_F16, wm, sc, sdt, qz, perm, y_na, m, n, k, G, splits, None)
        assert rc == 0, (lib.pw4_status_string(rc), lib.pw4_last_hip_error())
        a = hip.download(y_ws, (m, n), np.uint16)
        b = hip.download(y_na, (m, n), np.uint16)
        assert np.array_equal(a, b), f"call {i} (M={m} N={n} K={k}): noalloc differs from the workspace entry point"
        # and both meet the oracle
        ref = p.reference()
        got = b.view(np.float16).astype(np.float64)
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-3


def test_noalloc_rejects_plans_beyond_the_scratch(env):
    lib, hip = env
    # act-order gathers x[:, perm] (M * K * 2 bytes) into the scratch: 4096 x 8192 is 64 MiB
    m, n, k = 4096, 256, 8192
    assert m * k * 2 > PW4_NOALLOC_SCRATCH_BYTES - (16 << 20)
    x = hip.malloc(m * k * 2)
    wm = hip.malloc(lib.pw4_marlin_words(n, k) * 4)
    sc = hip.malloc((k // G) * n * 2)
    perm = hip.upload(np.arange(k, dtype=np.int32))
    y = hip.malloc(m * n * 2)
    assert lib.pw4_gemm_w4a16_marlin_noalloc(x, DTYPE_F16, wm, sc, DTYPE_F16, None, perm, y, m, n, k, G, 0,
                                             None) == -3
    # forced K slices whose partials do not fit are rejected too (automatic plans run unsplit)
    assert lib.pw4_gemm_w4a16_marlin_noalloc(x, DTYPE_F16, wm, sc, DTYPE_F16, None, None, y, m, n, k, G, 16,
                                             None) == -3


# ---- under HIP graph capture ------------------------------------------------
# (M, N, K, num_splits, act_order): every kind of scratch use, as above
CAPTURE_CALLS = [
    (16, 2048, 14336, 0, False),   # exchange-tree slots in the zero region
    (4, 512, 4096, 3, False),      # forced K slices: counters + partials
    (300, 1040, 2048, 4, False),   # prefill K-slice partials + combine
    (8, 1024, 8192, 0, True),      # act-order copy of x
]


def _capture_check() -> None:
    """Run in a fresh process, so that its first no-alloc call is made while a
    stream is capturing.  Checks, bit for bit against the workspace entry
    point: replays of graphs captured before any eager no-alloc call (the
    zero-region fill recorded once per graph, ahead of its first call), an
    eager call after them, and a graph captured after that (no fill)."""
    lib = declare(pulsar_amd.capi())
    hip = Hip()
    cases = []
    for i, (m, n, k, splits, act) in enumerate(CAPTURE_CALLS):
        p = O.make_problem(m, n, k, G, seed=120 + i, symmetric=not act, act_order=act)
        wm, sc, sdt, qz, perm = _operands(lib, hip, p)
        x = hip.upload(p.x16)
        need = lib.pw4_gemm_w4a16_marlin_workspace_size(m, n, k, G, int(act), splits)
        ws = hip.malloc(max(need, 1))
        hip.memset(ws, 0, max(need, 1))
        y_ws = hip.malloc(m * n * 2)
        assert lib.pw4_gemm_w4a16_marlin(x, DTYPE_F16, wm, sc, sdt, qz, perm, y_ws, m, n, k, G, splits, ws, need,
                                         None) == 0
        want = hip.download(y_ws, (m, n), np.uint16)
        cases.append(dict(args=(x, DTYPE_F16, wm, sc, sdt, qz, perm), shape=(m, n, k, splits),
                          y=hip.malloc(m * n * 2), want=want))

    def call(case, s):
        x, xd, wm, sc, sdt, qz, perm = case["args"]
        m, n, k, splits = case["shape"]
        rc = lib.pw4_gemm_w4a16_marlin_noalloc(x, xd, wm, sc, sdt, qz, perm, case["y"], m, n, k, G, splits, s)
        assert rc == 0, (lib.pw4_status_string(rc), lib.pw4_last_hip_error())

    def check(which, tag):
        for i in which:
            c = cases[i]
            m, n = c["shape"][:2]
            got = hip.download(c["y"], (m, n), np.uint16)
            assert np.array_equal(got, c["want"]), f"{tag}: call {i} {c['shape']} differs from the workspace entry point"

    def replay(ge, s, which, tag, times):
        for r in range(times):
            for i in which:
                m, n = cases[i]["shape"][:2]
                hip.memset(cases[i]["y"], 0xFF, m * n * 2)
            hip.sync()
            hip.launch_graph(ge, s)
            hip.stream_sync(s)
            check(which, f"{tag} replay {r}")

    s = hip.stream()
    # cold: no no-alloc call has run in this process
    _, n1 = hip.capture(s, lambda st: call(cases[0], st))
    g3, n3 = hip.capture(s, lambda st: [call(cases[0], st) for _ in range(3)])
    # one fill node per graph, however many calls it holds
    assert n3 == 3 * n1 - 2, f"cold graphs: {n1} nodes for one call, {n3} for three (one fill expected in each)"
    gall, _ = hip.capture(s, lambda st: [call(c, st) for c in cases])
    e3, eall = hip.instantiate(g3), hip.instantiate(gall)
    replay(eall, s, range(len(cases)), "cold graph of every kind", 3)
    replay(e3, s, [0], "cold graph of three calls", 2)
    # an eager call clears the region for good ...
    call(cases[1], s)
    hip.stream_sync(s)
    check([1], "eager call after the cold graphs")
    # ... so a graph captured after it records no fill
    g3w, n3w = hip.capture(s, lambda st: [call(cases[0], st) for _ in range(3)])
    assert n3w == n3 - 1, f"warm graph of three calls: {n3w} nodes against {n3} with the fill"
    e3w = hip.instantiate(g3w)
    replay(e3w, s, [0], "warm graph", 2)
    replay(eall, s, range(len(cases)), "cold graph after the eager call", 2)
    # a stream of the current device is required; the default stream is one
    hip.sync()
    hip.free_all()
    print("capture check ok", flush=True)


def test_noalloc_under_graph_capture():
    """The first no-alloc call of a process made under stream capture, then
    replays, eager calls and a warm capture (see _capture_check); run in a
    child process so that the call really is the process's first."""
    import os
    import subprocess
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([here, os.path.dirname(here), env.get("PYTHONPATH", "")])
    r = subprocess.run([sys.executable, "-u", os.path.abspath(__file__), "capture"], env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0 and "capture check ok" in r.stdout, f"child failed ({r.returncode}):\n{r.stdout}\n{r.stderr}"


if __name__ == "__main__":
    import sys as _sys

    if len(_sys.argv) > 1 and _sys.argv[1] == "capture":
        _capture_check()
