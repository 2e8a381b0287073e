"""ctypes declarations of the C ABI (include/pulsar_w4a16.h) and a minimal HIP
runtime binding (libamdhip64: hipMalloc / hipMemcpy / hipMemset / hipFree), so
that tests can drive libpulsar_w4a16.so the way a non-torch caller would."""

from __future__ import annotations

import ctypes

import numpy as np

P = ctypes.c_void_p
I64 = ctypes.c_int64
SZ = ctypes.c_size_t
INT = ctypes.c_int

PW4_ZERO_REGION_BYTES = 16 << 20
PW4_NOALLOC_SCRATCH_BYTES = 64 << 20
DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2


def declare(L: ctypes.CDLL) -> ctypes.CDLL:
    sig = {
        "pw4_status_string": (ctypes.c_char_p, [INT]),
        "pw4_last_hip_error": (ctypes.c_char_p, []),
        "pw4_marlin_words": (I64, [I64, I64]),
        "pw4_gemm_w4a16": (INT, [P, INT, P, P, P, I64, I64, I64, I64, I64, P, SZ, P]),
        "pw4_gemm_w4a16_marlin": (INT, [P, INT, P, P, INT, P, P, P, I64, I64, I64, I64, I64, P, SZ, P]),
        "pw4_gemm_w4a16_workspace_size": (SZ, [I64, I64, I64, I64, I64]),
        "pw4_gemm_w4a16_marlin_workspace_size": (SZ, [I64, I64, I64, I64, INT, I64]),
        "pw4_gemm_w4a16_silu_mul": (INT, [P, INT, P, P, INT, P, P, P, I64, I64, I64, I64, P, SZ, P]),
        "pw4_gemm_w4a16_silu_mul_workspace_size": (SZ, [I64, I64, I64, I64, INT]),
        "pw4_repack_w4a16": (INT, [P, P, INT, I64, I64, I64, P, P, P]),
        "pw4_gidx_to_perm": (INT, [P, I64, I64, P, P, P]),
        "pw4_repack_gptq": (INT, [P, P, I64, I64, P, P]),
        "pw4_abi_version": (INT, []),
        "pw4_time_next_kernel": (INT, [P, P]),
        "pw4_observe_next_call": (INT, [P]),
        "pw4_plan_describe": (INT, [INT, INT, INT, INT, INT, INT, I64, I64, I64, I64, I64, ctypes.c_char_p, SZ]),
        "pw4_gemm_w4a16_marlin_noalloc": (INT, [P, INT, P, P, INT, P, P, P, I64, I64, I64, I64, I64, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


class Hip:
    """The few HIP runtime calls the ABI tests need (device 0, default stream)."""

    H2D, D2H = 1, 2

    def __init__(self):
        # by soname: the runtime the process already has loaded (torch's copy
        # and ROCm's share it), never a second copy
        self.lib = ctypes.CDLL("libamdhip64.so.7")
        L = self.lib
        L.hipMalloc.argtypes = [ctypes.POINTER(P), SZ]
        L.hipFree.argtypes = [P]
        L.hipMemcpy.argtypes = [P, P, SZ, INT]
        L.hipMemset.argtypes = [P, INT, SZ]
        L.hipDeviceSynchronize.argtypes = []
        for f in (L.hipMalloc, L.hipFree, L.hipMemcpy, L.hipMemset, L.hipDeviceSynchronize):
            f.restype = INT
        self._live: list[int] = []

    def _ok(self, rc: int, what: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")

    def malloc(self, nbytes: int) -> int:
        p = P()
        self._ok(self.lib.hipMalloc(ctypes.byref(p), max(int(nbytes), 1)), "hipMalloc")
        self._live.append(p.value)
        return p.value

    def upload(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        d = self.malloc(a.nbytes)
        self._ok(self.lib.hipMemcpy(d, a.ctypes.data, a.nbytes, self.H2D), "hipMemcpy H2D")
        return d

    def download(self, d: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        self.sync()
        self._ok(self.lib.hipMemcpy(out.ctypes.data, d, out.nbytes, self.D2H), "hipMemcpy D2H")
        return out

    def memset(self, d: int, value: int, nbytes: int) -> None:
        self._ok(self.lib.hipMemset(d, value, nbytes), "hipMemset")

    def sync(self) -> None:
        self._ok(self.lib.hipDeviceSynchronize(), "hipDeviceSynchronize")

    # ---- streams and graph capture (for the capture tests) ----------------
    CAPTURE_GLOBAL = 0

    def _declare_graph_calls(self) -> None:
        L = self.lib
        if getattr(self, "_graph_calls", False):
            return
        L.hipStreamCreate.argtypes = [ctypes.POINTER(P)]
        L.hipStreamDestroy.argtypes = [P]
        L.hipStreamSynchronize.argtypes = [P]
        L.hipStreamBeginCapture.argtypes = [P, INT]
        L.hipStreamEndCapture.argtypes = [P, ctypes.POINTER(P)]
        L.hipGraphGetNodes.argtypes = [P, P, ctypes.POINTER(SZ)]
        L.hipGraphInstantiate.argtypes = [ctypes.POINTER(P), P, P, P, SZ]
        L.hipGraphLaunch.argtypes = [P, P]
        L.hipGraphExecDestroy.argtypes = [P]
        L.hipGraphDestroy.argtypes = [P]
        for f in (L.hipStreamCreate, L.hipStreamDestroy, L.hipStreamSynchronize, L.hipStreamBeginCapture,
                  L.hipStreamEndCapture, L.hipGraphGetNodes, L.hipGraphInstantiate, L.hipGraphLaunch,
                  L.hipGraphExecDestroy, L.hipGraphDestroy):
            f.restype = INT
        self._graph_calls = True

    def stream(self) -> int:
        self._declare_graph_calls()
        s = P()
        self._ok(self.lib.hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        return s.value

    def stream_sync(self, s: int) -> None:
        self._ok(self.lib.hipStreamSynchronize(s), "hipStreamSynchronize")

    def capture(self, s: int, record) -> tuple[int, int]:
        """Capture what record(s) launches on stream s; returns (graph, node count)."""
        self._declare_graph_calls()
        self._ok(self.lib.hipStreamBeginCapture(s, self.CAPTURE_GLOBAL), "hipStreamBeginCapture")
        try:
            record(s)
        finally:
            g = P()
            rc = self.lib.hipStreamEndCapture(s, ctypes.byref(g))
        self._ok(rc, "hipStreamEndCapture")
        n = SZ(0)
        self._ok(self.lib.hipGraphGetNodes(g, None, ctypes.byref(n)), "hipGraphGetNodes")
        return g.value, n.value

    def instantiate(self, g: int) -> int:
        ge = P()
        self._ok(self.lib.hipGraphInstantiate(ctypes.byref(ge), g, None, None, 0), "hipGraphInstantiate")
        return ge.value

    def launch_graph(self, ge: int, s: int) -> None:
        self._ok(self.lib.hipGraphLaunch(ge, s), "hipGraphLaunch")

    def free_all(self) -> None:
        self.sync()
        for p in self._live:
            self.lib.hipFree(p)
        self._live.clear()
