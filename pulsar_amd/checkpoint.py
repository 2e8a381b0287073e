"""Quantization-aware checkpoint loading: W4A16 linears repacked at load.

The reference loader (pulsar/src/pulsar/checkpoint.py:123-141, `load_weights`)
reads every safetensors tensor of a model archive and casts it to the model
dtype, which turns int32 packed weights into floats.  This loader reads the
same archive layout -- a zip with `config.json` and `weights/*.safetensors`
(checkpoint.py:144-158), or a plain directory of `*.safetensors` shards with a
`config.json` -- and:

  * leaves integer tensors in their own dtype (only floating tensors take
    `dtype`);
  * finds the quantized linears by their tensor names, in either of two
    formats:
      - "packed": the reference's own quantized weight, `<p>.weight_packed`
        int32 [N, K/8] + `<p>.weight_scale` [N, K/G] (+ optional
        `<p>.weight_shape`), the inputs of gemm_w4a16 / repack_w4a16
        (pulsar-core/inc/pulsar/ops.hpp:148-182);
      - "gptq": `<p>.qweight` int32 [K/8, N], `<p>.scales` [K/G, N],
        `<p>.qzeros` int32 [K/G, N/8], optional `<p>.g_idx` [K];
  * repacks each one to the MARLIN layout on the device, once, and returns it
    as a `W4A16Linear` under `<p>.weight`, the key the engine looks up
    (pulsar-core/src/model/qwen3.cpp:48-70), in place of the dense tensor.

The group size and the GPTQ conventions come from `config.json`'s
`quantization_config` (or the `quant` argument): for GPTQ, `bits` (4),
`group_size`, `desc_act`, `sym` and `checkpoint_format` ("gptq": zero points
stored as z - 1, AutoGPTQ's original format; "gptq_v2": stored as z); for the
packed format, `group_size` and `nibbles` ("twos": two's complement, the
reference's convention, default; "offset": value + 8).  Symmetric GPTQ zero
points that are all 8 are dropped, so such layers run the symmetric kernels.
"""

from __future__ import annotations

import io
import json
import os
import zipfile
from dataclasses import dataclass

import torch

from .linear import W4A16Linear, W4A16SiluGate, gptq_v1_to_v2_zeros

PACKED_SUFFIXES = ("weight_packed", "weight_scale", "weight_shape")
GPTQ_SUFFIXES = ("qweight", "qzeros", "scales", "g_idx")


class CheckpointError(RuntimeError):
    """A checkpoint this loader cannot turn into W4A16 linears (the reference raises
    PulsarModelLoadingError for archives it cannot read, checkpoint.py:18-19)."""


@dataclass(frozen=True)
class QuantConfig:
    fmt: str                  # "packed" or "gptq"
    group_size: int
    symmetric: bool = True
    act_order: bool = False
    v1_zeros: bool = False    # GPTQ zero points stored as (z - 1) mod 16
    nibbles: str = "twos"     # packed format: "twos" or "offset"


def parse_quant_config(q: dict) -> QuantConfig:
    """`quantization_config` of a config.json (or the same keys given directly)."""
    method = str(q.get("quant_method", q.get("format", "gptq"))).lower()
    if method == "gptq":
        bits = int(q.get("bits", 4))
        if bits != 4:
            raise CheckpointError(f"GPTQ checkpoint with {bits}-bit weights: only 4-bit is supported")
        g = int(q.get("group_size", 128))
        if g <= 0:
            raise CheckpointError("GPTQ group_size must be positive (per-column quantisation, group_size -1, "
                                  "is not supported)")
        return QuantConfig("gptq", g, symmetric=bool(q.get("sym", True)), act_order=bool(q.get("desc_act", False)),
                           v1_zeros=str(q.get("checkpoint_format", "gptq")).lower() != "gptq_v2")
    if method in ("packed", "pulsar", "w4a16"):
        nib = str(q.get("nibbles", "twos")).lower()
        if nib not in ("twos", "offset"):
            raise CheckpointError(f"packed format: nibbles must be 'twos' or 'offset', not {nib!r}")
        return QuantConfig("packed", int(q.get("group_size", 128)), nibbles=nib)
    raise CheckpointError(f"unsupported quant_method {method!r} (expected 'gptq' or 'packed')")


def find_quantized(names) -> dict[str, str]:
    """Linear prefixes and their format, from tensor names: `<p>.weight_packed` -> "packed",
    `<p>.qweight` -> "gptq"."""
    out = {}
    for name in names:
        if name.endswith(".weight_packed"):
            out[name[: -len(".weight_packed")]] = "packed"
        elif name.endswith(".qweight"):
            out[name[: -len(".qweight")]] = "gptq"
    return out


def _is_member(name: str, prefixes: dict[str, str]) -> bool:
    p, _, suffix = name.rpartition(".")
    return p in prefixes and suffix in (PACKED_SUFFIXES if prefixes[p] == "packed" else GPTQ_SUFFIXES)


# ---- reading shards ----------------------------------------------------------------------


def _read_config(source: str) -> dict:
    if os.path.isdir(source):
        path = os.path.join(source, "config.json")
        if not os.path.exists(path):
            return {}
        with open(path) as f:
            return json.load(f)
    with zipfile.ZipFile(source) as z:
        try:
            return json.loads(z.read("config.json"))
        except KeyError:
            return {}


def _shard_files(source: str) -> list[str]:
    roots = [source, os.path.join(source, "weights")]
    return sorted({os.path.join(r, f) for r in roots if os.path.isdir(r) for f in os.listdir(r)
                   if f.endswith(".safetensors")})


def _zip_members(z: zipfile.ZipFile) -> list[str]:
    return sorted(n for n in z.namelist() if n.startswith("weights/") and n.endswith(".safetensors"))


def _header_names(f) -> list[str]:
    """Tensor names from a safetensors header (8-byte little-endian length, then JSON),
    without reading the tensor data."""
    n = int.from_bytes(f.read(8), "little")
    return [k for k in json.loads(f.read(n)) if k != "__metadata__"]


def _tensor_names(source: str) -> list[str]:
    """Every tensor name of `source` (directory or zip archive), from the shard headers only."""
    names = []
    if os.path.isdir(source):
        for path in _shard_files(source):
            with open(path, "rb") as f:
                names += _header_names(f)
        return names
    with zipfile.ZipFile(source) as z:
        for member in _zip_members(z):
            with z.open(member) as f:
                names += _header_names(f)
    return names


def _iter_shards(source: str):
    """(name, cpu tensor) over every safetensors shard of `source` (directory or zip archive),
    one tensor at a time: a directory's shards are memory-mapped, a zip member is read whole
    (one shard in host memory at a time)."""
    from safetensors import safe_open
    from safetensors.torch import load as st_load

    if os.path.isdir(source):
        for path in _shard_files(source):
            with safe_open(path, framework="pt", device="cpu") as f:
                for name in f.keys():
                    yield name, f.get_tensor(name)
        return
    with zipfile.ZipFile(source) as z:
        for member in _zip_members(z):
            shard = st_load(z.read(member))
            while shard:
                name = next(iter(shard))
                yield name, shard.pop(name)
            del shard


# ---- the loader ----------------------------------------------------------------------------


def build_linear(fmt: str, parts: dict[str, torch.Tensor], qc: QuantConfig, prefix: str) -> W4A16Linear:
    """One W4A16Linear from its checkpoint tensors (already on the target device)."""
    g = qc.group_size
    if fmt == "packed":
        wp, ws = parts.get("weight_packed"), parts.get("weight_scale")
        if wp is None or ws is None:
            raise CheckpointError(f"{prefix}: weight_packed needs weight_scale")
        if wp.dtype != torch.int32 or wp.dim() != 2:
            raise CheckpointError(f"{prefix}.weight_packed must be int32 [N, K/8]")
        n, k = wp.shape[0], wp.shape[1] * 8
        if "weight_shape" in parts:
            shp = [int(v) for v in parts["weight_shape"].flatten().tolist()]
            if shp != [n, k]:
                raise CheckpointError(f"{prefix}.weight_shape {shp} does not match weight_packed [N, K/8] = "
                                      f"[{n}, {k // 8}]")
        if k % g or tuple(ws.shape) != (n, k // g):
            raise CheckpointError(f"{prefix}.weight_scale must be [{n}, {k // g}] for group size {g}")
        if qc.nibbles == "offset":
            wp = wp ^ torch.tensor(0x88888888 - (1 << 32), dtype=torch.int32, device=wp.device)
        return W4A16Linear.from_packed(wp, ws, g)
    qw, sc = parts.get("qweight"), parts.get("scales")
    if qw is None or sc is None:
        raise CheckpointError(f"{prefix}: qweight needs scales")
    if qw.dtype != torch.int32 or qw.dim() != 2:
        raise CheckpointError(f"{prefix}.qweight must be int32 [K/8, N]")
    k, n = qw.shape[0] * 8, qw.shape[1]
    if k % g or tuple(sc.shape) != (k // g, n):
        raise CheckpointError(f"{prefix}.scales must be [{k // g}, {n}] for group size {g}")
    qz = parts.get("qzeros")
    if qz is not None:
        if qz.dtype != torch.int32 or tuple(qz.shape) != (k // g, n // 8):
            raise CheckpointError(f"{prefix}.qzeros must be int32 [{k // g}, {n // 8}]")
        if qc.v1_zeros:
            qz = gptq_v1_to_v2_zeros(qz)
        if bool((qz == torch.tensor(0x88888888 - (1 << 32), dtype=torch.int32, device=qz.device)).all()):
            qz = None  # every zero point is the implicit 8: the symmetric kernels apply
    g_idx = parts.get("g_idx")
    if g_idx is not None and tuple(g_idx.shape) != (k,):
        raise CheckpointError(f"{prefix}.g_idx must be [{k}]")
    sc = sc if sc.dtype in (torch.float16, torch.float32) else sc.float()
    return W4A16Linear.from_gptq(qw, sc, g, qzeros=qz, g_idx=g_idx)


def load_weights(source: str, *, device: torch.device | str, dtype: torch.dtype | None = None,
                 quant: dict | None = None, fuse: bool = False,
                 silu_gate: bool = False) -> dict[str, "torch.Tensor | W4A16Linear"]:
    """Every tensor of the checkpoint at `source`, on `device`; quantized linears come back as
    W4A16Linear under `<prefix>.weight`.  `quant` overrides config.json's quantization_config.
    With `fuse`, q|k|v and gate|up of each layer are N-concatenated into `<layer>.self_attn.
    qkv_proj.weight` and `<layer>.mlp.gate_up_proj.weight` (the members are dropped); with
    `silu_gate` as well, the latter is a W4A16SiluGate computing silu(gate) * up."""
    device = torch.device(device)
    cfg = _read_config(source)
    qraw = quant if quant is not None else cfg.get("quantization_config")
    prefixes = find_quantized(_tensor_names(source))  # from the shard headers, before any data
    if prefixes and qraw is None:
        raise CheckpointError("quantized linears found but no quantization_config (pass quant=...)")
    qc = parse_quant_config(qraw) if prefixes else None
    if qc is not None and any(f != qc.fmt for f in prefixes.values()):
        raise CheckpointError(f"quantization_config says {qc.fmt!r} but the checkpoint holds "
                              f"{sorted(set(prefixes.values()))} linears")
    out: dict = {}
    groups: dict[str, dict[str, torch.Tensor]] = {p: {} for p in prefixes}
    # each tensor goes to the device as it is read, so host memory holds one shard at most
    for name, t in _iter_shards(source):
        if _is_member(name, prefixes):
            p, _, suffix = name.rpartition(".")
            groups[p][suffix] = t.to(device)
        else:
            out[name] = t.to(device=device, dtype=dtype if (dtype is not None and t.is_floating_point()) else None)
        del t
    for p, fmt in prefixes.items():
        lin = build_linear(fmt, groups.pop(p), qc, p)
        bias = out.pop(p + ".bias", None)
        if bias is not None:
            lin.bias = bias.to(torch.float32)
        out[p + ".weight"] = lin
    if fuse:
        fuse_projections(out, silu_gate=silu_gate)
    return out


def fuse_projections(weights: dict, silu_gate: bool = False) -> None:
    """In place: `<l>.self_attn.{q,k,v}_proj.weight` -> `<l>.self_attn.qkv_proj.weight` and
    `<l>.mlp.{gate,up}_proj.weight` -> `<l>.mlp.gate_up_proj.weight` (a W4A16SiluGate with
    `silu_gate`), for every layer whose members are all W4A16Linear (Llama / Qwen naming) and
    can share one GEMM.  Members that cannot (different act-order permutations, as desc_act
    checkpoints usually have, or zero points kept on some and dropped as all-8 on others) stay
    separate linears under their own names."""
    for key in [k for k in weights if k.endswith(".self_attn.q_proj.weight")]:
        base = key[: -len("q_proj.weight")]
        names = [base + m + "_proj.weight" for m in ("q", "k", "v")]
        if all(isinstance(weights.get(n), W4A16Linear) for n in names) and \
                W4A16Linear.can_concat([weights[n] for n in names]):
            weights[base + "qkv_proj.weight"] = W4A16Linear.concat([weights.pop(n) for n in names])
    for key in [k for k in weights if k.endswith(".mlp.gate_proj.weight")]:
        base = key[: -len("gate_proj.weight")]
        names = [base + m + "_proj.weight" for m in ("gate", "up")]
        if not all(isinstance(weights.get(n), W4A16Linear) for n in names):
            continue
        members = [weights[n] for n in names]
        if silu_gate and W4A16SiluGate.can_fuse(*members):
            weights[base + "gate_up_proj.weight"] = W4A16SiluGate.from_members(*[weights.pop(n) for n in names])
        elif not silu_gate and W4A16Linear.can_concat(members):
            weights[base + "gate_up_proj.weight"] = W4A16Linear.concat([weights.pop(n) for n in names])


def save_archive(path: str, config: dict, tensors: dict[str, torch.Tensor], shards: int = 1) -> None:
    """Write a model archive in the reference's layout (config.json + weights/*.safetensors in a
    zip); used to build test checkpoints."""
    from safetensors.torch import save

    names = sorted(tensors)
    with zipfile.ZipFile(path, "w") as z:
        z.writestr("config.json", json.dumps(config))
        for s in range(shards):
            part = {n: tensors[n].contiguous().cpu() for n in names[s::shards]}
            z.writestr(f"weights/model-{s:05d}.safetensors", io.BytesIO(save(part)).getvalue())
