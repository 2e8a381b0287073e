"""A stack of W4A16 linear layers replayed as one HIP graph per step.

The decode step of a Llama-3-8B-shaped transformer runs seven quantized
linears per layer -- q, k, v, o, gate, up, down -- whose weights (3.49 GB of
int4 plus 0.11 GB of fp16 scales over 32 layers) stream from HBM once per
token.  `W4A16LinearStack` holds those weights in the MARLIN layout, captures
every linear of every layer into one graph for a fixed batch M, and replays it
per step, so the per-token cost is the kernels' own HBM time with no host
launch gaps.

Activations are not chained from layer to layer: the attention and norm
maths between the linears is outside this path, and chaining raw GEMM outputs
would grow the values by ~6x per GEMM until fp16 overflows.  Every linear reads
a fixed input of its K (x_attn [M, 4096] for q/k/v/o/gate/up, x_mlp [M, 14336]
for down), which leaves each kernel's work and traffic exactly what it is in
the model.  The one exception is the MLP with its gate fused
(`fuse_layers(..., silu_gate=True)`): there down reads the W4A16SiluGate's
output silu(gate) * up, exactly as in the model.

The reference has no such runner (its engine calls bf16 at::linear at
pulsar-core/src/models/qwen3.cpp:82-119); this is the drop-in's counterpart of
that decode step's linear layers, built on W4A16Linear (pulsar_amd.linear).
"""

from __future__ import annotations

import torch

from . import capi
from .linear import W4A16Linear, W4A16SiluGate

# (name, K, N) of the seven linears of one Llama-3-8B layer (hidden 4096, 8 KV
# heads of 128, MLP 14336).
LLAMA3_8B_LINEARS = (
    ("q", 4096, 4096),
    ("k", 4096, 1024),
    ("v", 4096, 1024),
    ("o", 4096, 4096),
    ("gate", 4096, 14336),
    ("up", 4096, 14336),
    ("down", 14336, 4096),
)


# The same layer with q|k|v and gate|up each fused into one N-concatenated
# linear (the decode-sweep shapes qkv 4096x6144 and gate_up 4096x28672).
LLAMA3_8B_FUSED = (("qkv", ("q", "k", "v")), ("o", ("o",)), ("gate_up", ("gate", "up")), ("down", ("down",)))


def random_layers(num_layers: int, shapes=LLAMA3_8B_LINEARS, group_size: int = 128, device="cuda:0",
                  seed: int = 0, stats: dict | None = None) -> list[list[W4A16Linear]]:
    """Random symmetric int4 GPTQ weights (u ~ U{0..15}, zero 8) and |N(0, 0.02)| + 1e-3 fp16
    scales, generated on the device and repacked to the MARLIN layout, as a checkpoint load
    would.  With `stats`, the repack bytes (qweight read, MARLIN words written) and times are
    accumulated: stats["repack_ms"] the repack kernels' own intervals (the library's timing
    hook, pw4_time_next_kernel, armed for each repack), stats["repack_call_ms"] HIP events
    around each from_gptq call, which also hold its host time."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    lib = capi() if stats is not None else None
    events, kernel_events = [], []
    nbytes = 0
    layers = []
    for _ in range(num_layers):
        layer = []
        for name, k, n in shapes:
            qweight = torch.randint(-(2 ** 31), 2 ** 31, (k // 8, n), dtype=torch.int32, device=device,
                                    generator=gen)
            scales = (torch.randn(k // group_size, n, device=device, generator=gen) * 0.02).abs_().add_(1e-3).half()
            if lib is not None:
                ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                kev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                for e in kev:
                    e.record()  # create the events before handing them over
                ev[0].record()
                if lib.pw4_time_next_kernel(kev[0], kev[1]) != 0:
                    raise RuntimeError("pw4_time_next_kernel failed")
            lin = W4A16Linear.from_gptq(qweight, scales, group_size)
            if lib is not None:
                ev[1].record()
                events.append(ev)
                kernel_events.append(kev)
                nbytes += qweight.numel() * 4 + lin.weight_marlin.numel() * 4
            lin.name = name
            layer.append(lin)
            del qweight
        layers.append(layer)
    if stats is not None:
        torch.cuda.synchronize()
        stats["repack_ms"] = stats.get("repack_ms", 0.0) + sum(a.elapsed_time(b) for a, b in kernel_events)
        stats["repack_call_ms"] = stats.get("repack_call_ms", 0.0) + sum(a.elapsed_time(b) for a, b in events)
        stats["repack_bytes"] = stats.get("repack_bytes", 0) + nbytes
    return layers


def fuse_layers(layers: list[list[W4A16Linear]], groups=LLAMA3_8B_FUSED,
                silu_gate: bool = False) -> list[list[W4A16Linear]]:
    """N-concatenate linears that share their input (W4A16Linear.concat: the members' MARLIN
    words back to back, their scales along N).  With `silu_gate`, gate|up becomes a
    W4A16SiluGate (silu(gate) * up, columns interleaved by 8) whose output feeds down."""
    fused = []
    for layer in layers:
        by_name = {lin.name: lin for lin in layer}
        out = []
        for name, members in groups:
            parts = [by_name[m] for m in members]
            if silu_gate and members == ("gate", "up"):
                lin = W4A16SiluGate.from_members(*parts)
            else:
                lin = W4A16Linear.concat(parts)
            if len(members) > 1:
                lin.name = name
            out.append(lin)
        fused.append(out)
    return fused


class W4A16LinearStack:
    """Every linear of `layers` at batch `m`, eager or as one captured graph.

    `forward()` runs the linears eagerly on the current stream and returns
    their outputs; `capture()` records the same launches into a graph whose
    outputs are `self.outputs` (fixed buffers); `step()` replays it.  Inputs are
    `self.inputs[k]`, one [m, k] fp16 buffer per distinct K, which the caller
    may overwrite between steps.
    """

    def __init__(self, layers: list[list[W4A16Linear]], m: int, group_size: int = 128, device="cuda:0",
                 seed: int = 1):
        self.layers = layers
        self.m = m
        self.group_size = group_size
        self.device = torch.device(device)
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        ks = sorted({lin.in_features for layer in layers for lin in layer})
        self.inputs = {k: torch.randn(m, k, device=self.device, generator=gen).half() for k in ks}
        self.graph: torch.cuda.CUDAGraph | None = None
        self.outputs: list[torch.Tensor] = []
        self.stream = torch.cuda.Stream(device=self.device)

    def forward(self) -> list[torch.Tensor]:
        outs = []
        for layer in self.layers:
            prev = None
            for lin in layer:
                x = outs[-1] if isinstance(prev, W4A16SiluGate) else self.inputs[lin.in_features]
                outs.append(lin(x))
                prev = lin
        return outs

    def capture(self) -> None:
        # One eager pass on the capture stream first: it sizes the shared
        # split-K workspace and loads the code objects outside the capture.
        with torch.cuda.stream(self.stream):
            self.forward()
        self.stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.outputs = self.forward()

    def step(self) -> None:
        if self.graph is None:
            raise RuntimeError("W4A16LinearStack.step() before capture()")
        self.graph.replay()

    def bytes_per_step(self) -> int:
        return sum(lin.bytes_per_call(self.m) for layer in self.layers for lin in layer)

    def launches_per_step(self) -> int:
        return sum(len(layer) for layer in self.layers)
