"""W4A16 linear layer: the drop-in for the engine's dense `at::linear` sites.

The reference decode step runs `at::linear(h, W)` on dense bf16/fp16 weights
for q, k, v, o, gate, up and down (pulsar-core/src/model/qwen3.cpp:82-119,
qwen2.cpp:78-93).  A `W4A16Linear` holds one such weight in the MARLIN layout
(int4 words, fp16 or fp32 scales [K/G, N], optional GPTQ zero points and
act-order permutation) and computes y = x @ W^T (+ bias) through the library's
GEMM for any leading shape of x, so a model swaps `at::linear(h, W)` for
`W(h)`.

`W4A16Linear.concat` builds the N-concatenated q|k|v and gate|up linears from
already repacked members (no requantisation): the MARLIN words are column-block
major (64-column blocks, each holding all of K), so for members whose N is a
multiple of 64 the fused weight is their word buffers back to back.
"""

from __future__ import annotations

import torch

from . import ops


class W4A16Linear(torch.nn.Module):
    """y = x @ dequant(W)^T (+ bias), W int4 [out_features, in_features] in the MARLIN layout."""

    def __init__(self, weight_marlin: torch.Tensor, scales: torch.Tensor, group_size: int, in_features: int,
                 out_features: int, qzeros: torch.Tensor | None = None, perm: torch.Tensor | None = None,
                 bias: torch.Tensor | None = None):
        super().__init__()
        k, n, g = int(in_features), int(out_features), int(group_size)
        if g <= 0 or k % g or k % 8:
            raise ValueError(f"W4A16Linear: in_features {k} must be a multiple of 8 and of group_size {g}")
        if tuple(scales.shape) != (k // g, n) or scales.dtype not in (torch.float16, torch.float32):
            raise ValueError(f"W4A16Linear: scales must be fp16/fp32 [{k // g}, {n}], got {scales.dtype} "
                             f"{tuple(scales.shape)}")
        if qzeros is not None and tuple(qzeros.shape) != (k // g, n // 8):
            raise ValueError(f"W4A16Linear: qzeros must be int32 [{k // g}, {n // 8}]")
        if perm is not None and perm.numel() == 0:
            perm = None
        if perm is not None and tuple(perm.shape) != (k,):
            raise ValueError(f"W4A16Linear: perm must be int32 [{k}]")
        if bias is not None and tuple(bias.shape) != (n,):
            raise ValueError(f"W4A16Linear: bias must be [{n}]")
        self.in_features, self.out_features, self.group_size = k, n, g
        self.register_buffer("weight_marlin", weight_marlin)
        self.register_buffer("scales", scales)
        self.register_buffer("qzeros", qzeros)
        self.register_buffer("perm", perm)
        self.register_buffer("bias", bias)

    # ---- construction from checkpoint tensors -------------------------------------------

    @classmethod
    def from_packed(cls, weight_packed: torch.Tensor, weight_scale: torch.Tensor, group_size: int,
                    bias: torch.Tensor | None = None) -> "W4A16Linear":
        """The reference's quantized weight: `weight_packed` int32 [N, K/8] (nibble k % 8 of word
        [n, k / 8], two's complement, ops.hpp:148-152) and `weight_scale` [N, K/G]; repacked with
        repack_w4a16, which keeps the reference's fp32 `scale_marlin` [K/G, N]."""
        n, k = weight_packed.shape[0], weight_packed.shape[1] * 8
        wm, sm = ops.repack_w4a16(weight_packed.contiguous(), weight_scale.contiguous(), group_size)
        return cls(wm, sm, group_size, k, n, bias=bias)

    @classmethod
    def from_gptq(cls, qweight: torch.Tensor, scales: torch.Tensor, group_size: int,
                  qzeros: torch.Tensor | None = None, g_idx: torch.Tensor | None = None,
                  bias: torch.Tensor | None = None) -> "W4A16Linear":
        """A GPTQ checkpoint's tensors: qweight int32 [K/8, N] (nibble k % 8 = u, unsigned),
        scales [K/G, N], qzeros int32 [K/G, N/8] holding z itself (convert the original
        AutoGPTQ "z - 1" storage with `gptq_v1_to_v2_zeros` first), g_idx [K] for act-order.
        A g_idx equal to k // G is the natural order and needs no permutation."""
        k, n = qweight.shape[0] * 8, qweight.shape[1]
        if g_idx is not None:
            natural = torch.arange(k, device=g_idx.device, dtype=torch.int32) // group_size
            if torch.equal(g_idx.to(torch.int32), natural):
                g_idx = None
        wm, perm = ops.repack_w4a16_gptq(qweight.contiguous(),
                                         None if g_idx is None else g_idx.to(torch.int32).contiguous(), group_size)
        sc = scales if scales.dtype in (torch.float16, torch.float32) else scales.float()
        return cls(wm, sc.contiguous(), group_size, k, n,
                   qzeros=None if qzeros is None else qzeros.contiguous(),
                   perm=perm if g_idx is not None else None, bias=bias)

    # ---- compute ------------------------------------------------------------------------

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.in_features:
            raise ValueError(f"W4A16Linear: x has {x.shape[-1]} features, expected {self.in_features}")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        y = ops.gemm_w4a16_gptq(x2, self.weight_marlin, self.scales, self.qzeros, self.perm, self.group_size)
        if self.bias is not None:
            # at::linear's bias (Qwen2's q, k, v): summed in fp32 with the GEMM output,
            # which is already rounded to x's dtype, and rounded again (at::linear
            # rounds x @ W^T + b once)
            y.add_(self.bias)
        return y.reshape(*lead, self.out_features)

    def bytes_per_call(self, m: int) -> int:
        """Algorithmic HBM bytes of one call at batch m: int4 weights, scales, zero points,
        permutation, x and y."""
        k, n, kg = self.in_features, self.out_features, self.in_features // self.group_size
        b = n * k // 2 + n * kg * self.scales.element_size() + m * k * 2 + m * n * 2
        if self.qzeros is not None:
            b += n * kg // 2
        if self.perm is not None:
            b += k * 4
        return b

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, group_size={self.group_size}, "
                f"zero_points={self.qzeros is not None}, act_order={self.perm is not None}, "
                f"bias={self.bias is not None}")

    # ---- fusion ---------------------------------------------------------------------------

    @staticmethod
    def can_concat(parts: list["W4A16Linear"]) -> bool:
        """Whether `concat` accepts these members (see there)."""
        if not parts:
            return False
        p0 = parts[0]
        for i, p in enumerate(parts):
            if isinstance(p, W4A16SiluGate):
                return False
            if (p.in_features, p.group_size, p.scales.dtype) != (p0.in_features, p0.group_size, p0.scales.dtype):
                return False
            if (p.qzeros is None) != (p0.qzeros is None) or (p.bias is None) != (p0.bias is None):
                return False
            if (p.perm is None) != (p0.perm is None) or (p.perm is not None and not torch.equal(p.perm, p0.perm)):
                return False
            if i + 1 < len(parts) and p.out_features % 64:
                return False
        return True

    @staticmethod
    def concat(parts: list["W4A16Linear"]) -> "W4A16Linear":
        """N-concatenation of linears that share their input (q|k|v, gate|up).  Every member but
        the last needs N % 64 == 0 (no MARLIN padding inside the fused words); all need the same
        K, group size, scale dtype, zero-point presence and act-order permutation."""
        if not parts:
            raise ValueError("W4A16Linear.concat: no parts")
        if len(parts) == 1:
            return parts[0]
        p0 = parts[0]
        for p in parts:
            if (p.in_features, p.group_size, p.scales.dtype) != (p0.in_features, p0.group_size, p0.scales.dtype):
                raise ValueError("W4A16Linear.concat: members differ in K, group size or scale dtype")
            if (p.qzeros is None) != (p0.qzeros is None) or (p.bias is None) != (p0.bias is None):
                raise ValueError("W4A16Linear.concat: members differ in zero points or bias")
            if (p.perm is None) != (p0.perm is None) or (p.perm is not None and not torch.equal(p.perm, p0.perm)):
                raise ValueError("W4A16Linear.concat: members have different act-order permutations")
        if any(p.out_features % 64 for p in parts[:-1]):
            raise ValueError("W4A16Linear.concat: every member but the last needs out_features % 64 == 0")
        return W4A16Linear(
            torch.cat([p.weight_marlin for p in parts]),
            torch.cat([p.scales for p in parts], dim=1),
            p0.group_size, p0.in_features, sum(p.out_features for p in parts),
            qzeros=None if p0.qzeros is None else torch.cat([p.qzeros for p in parts], dim=1),
            perm=p0.perm,
            bias=None if p0.bias is None else torch.cat([p.bias for p in parts]))


def gptq_v1_to_v2_zeros(qzeros: torch.Tensor) -> torch.Tensor:
    """AutoGPTQ's original checkpoints store each zero point as (z - 1) mod 16 (its kernels add
    the 1 back); this library's qzeros hold z.  Adds 1 to every nibble, mod 16."""
    w = qzeros.to(torch.int64) & 0xFFFFFFFF
    out = torch.zeros_like(w)
    for i in range(8):
        out |= (((w >> (4 * i)) + 1) & 0xF) << (4 * i)
    return out.to(torch.int32)


def _groups8(words: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """MARLIN words of an [n, k] weight as its 8-column groups: [n/8, Kpad/64, 2, 32] (a
    64-column block's chunk half holds 8 groups of 8 columns, 32 words each)."""
    ncb, nch = n // 64, -(-k // 64)
    return words.view(ncb, nch, 2, 8, 32).permute(0, 3, 1, 2, 4).reshape(ncb * 8, nch, 2, 32)


class W4A16SiluGate(W4A16Linear):
    """The SwiGLU gate of an MLP in one GEMM: y = silu(x @ Wg^T) * (x @ Wu^T), [..., F].

    Holds gate and up as one weight of 2F columns interleaved by 8 (fused columns 16j..16j+7
    are gate 8j..8j+7, 16j+8..16j+15 are up 8j..8j+7), so every 16-column strip the kernels
    finish together carries matching gate and up columns; the reference runs two at::linear
    calls and at::silu(gate) * up (pulsar-core/src/model/qwen3.cpp:116-118)."""

    @staticmethod
    def can_fuse(gate: W4A16Linear, up: W4A16Linear) -> bool:
        """Whether `from_members` accepts these two linears (see there)."""
        return (W4A16Linear.can_concat([gate, up]) and gate.out_features == up.out_features and
                gate.out_features % 64 == 0 and gate.bias is None)

    @classmethod
    def from_members(cls, gate: W4A16Linear, up: W4A16Linear) -> "W4A16SiluGate":
        """Interleave two repacked linears (same K, group size, scale dtype, zero points and
        act-order; F % 64 == 0) by regrouping their MARLIN words: no requantisation."""
        f, k = gate.out_features, gate.in_features
        if (up.out_features, up.in_features, up.group_size, up.scales.dtype) != \
                (f, k, gate.group_size, gate.scales.dtype):
            raise ValueError("W4A16SiluGate: gate and up differ in shape, group size or scale dtype")
        if f % 64:
            raise ValueError("W4A16SiluGate: the intermediate size must be a multiple of 64")
        if (gate.qzeros is None) != (up.qzeros is None) or (gate.bias is not None or up.bias is not None):
            raise ValueError("W4A16SiluGate: zero points must match; biases are not supported")
        if (gate.perm is None) != (up.perm is None) or (gate.perm is not None and not torch.equal(gate.perm, up.perm)):
            raise ValueError("W4A16SiluGate: gate and up have different act-order permutations")
        nch = -(-k // 64)
        groups = torch.stack([_groups8(gate.weight_marlin, f, k), _groups8(up.weight_marlin, f, k)], dim=1)
        words = groups.reshape(2 * f // 64, 8, nch, 2, 32).permute(0, 2, 3, 1, 4).reshape(-1).contiguous()
        kg = k // gate.group_size

        def inter(a: torch.Tensor, b: torch.Tensor, width: int) -> torch.Tensor:
            return torch.stack([a.view(kg, -1, width), b.view(kg, -1, width)], dim=2).reshape(kg, -1).contiguous()

        return cls(words, inter(gate.scales, up.scales, 8), gate.group_size, k, 2 * f,
                   qzeros=None if gate.qzeros is None else inter(gate.qzeros, up.qzeros, 1), perm=gate.perm)

    @property
    def intermediate(self) -> int:
        return self.out_features // 2

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.in_features:
            raise ValueError(f"W4A16SiluGate: x has {x.shape[-1]} features, expected {self.in_features}")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        y = ops.gemm_w4a16_silu_mul(x2, self.weight_marlin, self.scales, self.qzeros, self.perm, self.group_size)
        return y.reshape(*lead, self.intermediate)

    def bytes_per_call(self, m: int) -> int:
        return super().bytes_per_call(m) - m * self.intermediate * 2
