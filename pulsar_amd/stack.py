"""A stack of W4A16 linear layers replayed as one HIP graph per step.

The decode step of a Llama-3-8B-shaped transformer runs seven quantized
linears per layer -- q, k, v, o, gate, up, down -- whose weights (3.49 GB of
int4 plus 0.11 GB of fp16 scales over 32 layers) stream from HBM once per
token.  `W4A16LinearStack` holds those weights in the MARLIN layout, captures
every linear of every layer into one graph for a fixed batch M, and replays it
per step, so the per-token cost is the kernels' own HBM time with no host
launch gaps.

Activations are not chained through the layers: the attention and MLP maths
between the linears is outside this path, and chaining raw GEMM outputs would
grow the values by ~6x per GEMM until fp16 overflows.  Every linear reads a
fixed input of its K (x_attn [M, 4096] for q/k/v/o/gate/up, x_mlp [M, 14336]
for down), which leaves each kernel's work and traffic exactly what it is in
the model.

The reference has no such runner (its engine calls bf16 at::linear at
pulsar-core/src/models/qwen3.cpp:82-119); this is the drop-in's counterpart of
that decode step's linear layers, built on the ops in pulsar_amd.ops.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops

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


@dataclass
class QuantLinear:
    """One linear in the MARLIN layout: weight_marlin int32 words, fp16 scales [K/G, N]."""

    name: str
    k: int
    n: int
    weight_marlin: torch.Tensor
    scales: torch.Tensor

    def bytes_per_call(self, m: int, group_size: int) -> int:
        """Algorithmic HBM bytes of one call: int4 weights, fp16 scales, x, y."""
        return self.n * self.k // 2 + self.n * (self.k // group_size) * 2 + m * self.k * 2 + m * self.n * 2


def random_layers(num_layers: int, shapes=LLAMA3_8B_LINEARS, group_size: int = 128, device="cuda:0",
                  seed: int = 0) -> list[list[QuantLinear]]:
    """Random symmetric int4 weights (u ~ U{0..15}, zero 8) and |N(0, 0.02)| + 1e-3
    fp16 scales, generated on the device and repacked to the MARLIN layout."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    layers = []
    for _ in range(num_layers):
        layer = []
        for name, k, n in shapes:
            qweight = torch.randint(-(2 ** 31), 2 ** 31, (k // 8, n), dtype=torch.int32, device=device,
                                    generator=gen)
            wm, _ = ops.repack_w4a16_gptq(qweight, None, group_size)
            del qweight
            scales = (torch.randn(k // group_size, n, device=device, generator=gen) * 0.02).abs_().add_(1e-3).half()
            layer.append(QuantLinear(name, k, n, wm, scales))
        layers.append(layer)
    return layers


def fuse_layers(layers: list[list[QuantLinear]], groups=LLAMA3_8B_FUSED) -> list[list[QuantLinear]]:
    """N-concatenate linears that share their input.  The MARLIN word order is
    column-block major (64-column blocks, each holding all of K), so for
    members whose N is a multiple of 64 the fused weight is the members'
    weight buffers back to back; the scales concatenate along N."""
    fused = []
    for layer in layers:
        by_name = {lin.name: lin for lin in layer}
        out = []
        for name, members in groups:
            parts = [by_name[m] for m in members]
            k = parts[0].k
            if any(p.k != k for p in parts) or any(p.n % 64 for p in parts[:-1]):
                raise ValueError(f"cannot fuse {members}: K differs or N not a multiple of 64")
            wm = torch.cat([p.weight_marlin for p in parts]) if len(parts) > 1 else parts[0].weight_marlin
            sc = torch.cat([p.scales for p in parts], dim=1) if len(parts) > 1 else parts[0].scales
            out.append(QuantLinear(name, k, sum(p.n for p in parts), wm, sc))
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

    def __init__(self, layers: list[list[QuantLinear]], m: int, group_size: int = 128, device="cuda:0",
                 seed: int = 1):
        self.layers = layers
        self.m = m
        self.group_size = group_size
        self.device = torch.device(device)
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        ks = sorted({lin.k for layer in layers for lin in layer})
        self.inputs = {k: torch.randn(m, k, device=self.device, generator=gen).half() for k in ks}
        self.graph: torch.cuda.CUDAGraph | None = None
        self.outputs: list[torch.Tensor] = []
        self.stream = torch.cuda.Stream(device=self.device)

    def _input_for(self, lin: QuantLinear) -> torch.Tensor:
        return self.inputs[lin.k]

    def forward(self) -> list[torch.Tensor]:
        outs = []
        for layer in self.layers:
            for lin in layer:
                outs.append(ops.gemm_w4a16_gptq(self._input_for(lin), lin.weight_marlin, lin.scales, None, None,
                                                self.group_size))
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
        return sum(lin.bytes_per_call(self.m, self.group_size) for layer in self.layers for lin in layer)

    def launches_per_step(self) -> int:
        return sum(len(layer) for layer in self.layers)
