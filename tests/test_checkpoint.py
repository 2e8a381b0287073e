"""Checkpoint ingestion: the quantization-aware loader and W4A16Linear.

CPU tests pin the host logic: quantization_config parsing, grouping of tensor
names into linears, the AutoGPTQ v1 -> v2 zero-point conversion (against the
oracle's GPTQ zero packer), and the dense path, which keeps integer tensors in
their dtype where the reference's load_weights casts everything
(pulsar/src/pulsar/checkpoint.py:123-141).

GPU tests write small two-layer Llama-shaped checkpoints in both formats (the
reference's packed weights; GPTQ with v1 zero points and act-order), load them
through the reference archive layout, and check every linear's forward
against the fp32 oracle, and the fused q|k|v and gate|up linears against the
separate ones.
"""

import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsar_amd.checkpoint import (CheckpointError, QuantConfig, find_quantized, load_weights, parse_quant_config,
                                   save_archive)
from pulsar_amd.linear import W4A16Linear, gptq_v1_to_v2_zeros
from w4a16_case import check, to_device_x

G = 64
HIDDEN, FF, KV = 256, 512, 128
# (name, K, N) of one Llama-shaped layer at test size
LINEARS = (("self_attn.q_proj", HIDDEN, HIDDEN), ("self_attn.k_proj", HIDDEN, KV), ("self_attn.v_proj", HIDDEN, KV),
           ("self_attn.o_proj", HIDDEN, HIDDEN), ("mlp.gate_proj", HIDDEN, FF), ("mlp.up_proj", HIDDEN, FF),
           ("mlp.down_proj", FF, HIDDEN))


# ---- host logic (no GPU) ---------------------------------------------------------------------


def test_parse_quant_config():
    q = parse_quant_config({"quant_method": "gptq", "bits": 4, "group_size": 64, "desc_act": True, "sym": False})
    assert q == QuantConfig("gptq", 64, symmetric=False, act_order=True, v1_zeros=True)
    assert parse_quant_config({"quant_method": "gptq", "checkpoint_format": "gptq_v2"}).v1_zeros is False
    assert parse_quant_config({"quant_method": "packed", "group_size": 32, "nibbles": "offset"}) == \
        QuantConfig("packed", 32, nibbles="offset")
    for bad in ({"quant_method": "gptq", "bits": 8}, {"quant_method": "gptq", "group_size": -1},
                {"quant_method": "awq"}, {"quant_method": "packed", "nibbles": "sign"}):
        with pytest.raises(CheckpointError):
            parse_quant_config(bad)


def test_find_quantized():
    names = ["model.layers.0.self_attn.q_proj.qweight", "model.layers.0.self_attn.q_proj.scales",
             "model.layers.0.mlp.down_proj.weight_packed", "model.layers.0.mlp.down_proj.weight_scale",
             "model.norm.weight", "model.layers.0.input_layernorm.weight"]
    assert find_quantized(names) == {"model.layers.0.self_attn.q_proj": "gptq", "model.layers.0.mlp.down_proj": "packed"}


@pytest.mark.parametrize("seed", [0, 1])
def test_gptq_v1_zeros_convert(seed):
    """v1 storage packs (z - 1) mod 16; after the conversion the words equal the oracle's
    packing of z itself, for every z in 0..15 (z = 0 is stored as 15 in v1)."""
    rng = np.random.default_rng(seed)
    z = rng.integers(0, 16, size=(6, 64)).astype(np.uint8)
    z[0, :16] = np.arange(16)
    v1 = O.pack_gptq_zeros(((z.astype(np.int16) - 1) % 16).astype(np.uint8))
    v2 = gptq_v1_to_v2_zeros(torch.from_numpy(v1))
    assert v2.dtype == torch.int32
    assert np.array_equal(v2.numpy(), O.pack_gptq_zeros(z))


def test_dense_checkpoint_keeps_integer_dtypes(tmp_path):
    """Floating tensors take the model dtype, integer tensors keep theirs; zip archives and
    directories read the same."""
    t = {"model.norm.weight": torch.randn(16), "model.embed_tokens.weight": torch.randn(8, 16, dtype=torch.float16),
         "model.position_ids": torch.arange(10, dtype=torch.int64), "model.flags": torch.tensor([1, 0], dtype=torch.int32)}
    arch = str(tmp_path / "m.pulsar")
    save_archive(arch, {"hidden_size": 16}, t, shards=2)
    d = tmp_path / "dir"
    d.mkdir()
    from safetensors.torch import save_file
    save_file({k: v.contiguous() for k, v in t.items()}, str(d / "model.safetensors"))
    for src in (arch, str(d)):
        w = load_weights(src, device="cpu", dtype=torch.bfloat16)
        assert set(w) == set(t)
        assert w["model.norm.weight"].dtype == torch.bfloat16
        assert w["model.embed_tokens.weight"].dtype == torch.bfloat16
        assert w["model.position_ids"].dtype == torch.int64 and torch.equal(w["model.position_ids"], t["model.position_ids"])
        assert w["model.flags"].dtype == torch.int32


def test_quantized_without_config_is_rejected(tmp_path):
    t = {"l.qweight": torch.zeros(4, 64, dtype=torch.int32), "l.scales": torch.ones(1, 64, dtype=torch.float16)}
    arch = str(tmp_path / "q.pulsar")
    save_archive(arch, {}, t)
    with pytest.raises(CheckpointError):
        load_weights(arch, device="cpu")
    save_archive(arch, {"quantization_config": {"quant_method": "packed"}}, t)
    with pytest.raises(CheckpointError):  # config says packed, tensors are GPTQ
        load_weights(arch, device="cpu")


# ---- end to end on the GPU -----------------------------------------------------------------


def _gptq_layer(rng, k, n, act_order):
    u = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
    z = rng.integers(0, 16, size=(k // G, n)).astype(np.uint8)
    s = (np.abs(rng.standard_normal((k // G, n))) * 0.02 + 1e-3).astype(np.float16)
    if act_order:
        p = rng.permutation(k)
        g_idx = np.empty(k, dtype=np.int32)
        g_idx[p] = np.arange(k) // G
    else:
        g_idx = (np.arange(k) // G).astype(np.int32)
    w = (u.astype(np.float32) - z[g_idx].T.astype(np.float32)) * s[g_idx].T.astype(np.float32)  # [N, K]
    tensors = {"qweight": torch.from_numpy(O.pack_gptq(u)),
               "qzeros": torch.from_numpy(O.pack_gptq_zeros(((z.astype(np.int16) - 1) % 16).astype(np.uint8))),
               "scales": torch.from_numpy(s), "g_idx": torch.from_numpy(g_idx)}
    return tensors, w


def _packed_layer(rng, k, n, offset):
    vals = rng.integers(-8, 8, size=(n, k)).astype(np.int8)
    s = (rng.random((n, k // G)) * 0.04 + 0.01).astype(np.float16)
    packed = O.pack_ct(vals)
    if offset:
        packed = packed ^ np.int32(0x88888888 - (1 << 32))
    w = vals.astype(np.float32) * np.repeat(s.astype(np.float32), G, axis=1)
    return {"weight_packed": torch.from_numpy(packed), "weight_scale": torch.from_numpy(s),
            "weight_shape": torch.tensor([n, k], dtype=torch.int64)}, w


def _model(fmt, act_order=False, offset=False, layers=2, seed=0):
    rng = np.random.default_rng(seed)
    tensors, dense_w = {}, {}
    for li in range(layers):
        for name, k, n in LINEARS:
            p = f"model.layers.{li}.{name}"
            parts, w = _gptq_layer(rng, k, n, act_order) if fmt == "gptq" else _packed_layer(rng, k, n, offset)
            for suffix, t in parts.items():
                tensors[f"{p}.{suffix}"] = t
            dense_w[p] = w
        tensors[f"model.layers.{li}.input_layernorm.weight"] = torch.ones(HIDDEN)
    tensors["model.norm.weight"] = torch.ones(HIDDEN)
    if fmt == "gptq":
        q = {"quant_method": "gptq", "bits": 4, "group_size": G, "desc_act": act_order, "sym": False,
             "checkpoint_format": "gptq"}
    else:
        q = {"quant_method": "packed", "group_size": G, "nibbles": "offset" if offset else "twos"}
    return tensors, dense_w, {"hidden_size": HIDDEN, "quantization_config": q}


def _check_linears(weights, dense_w, m, seed):
    rng = np.random.default_rng(seed)
    for p, w in dense_w.items():
        lin = weights[p + ".weight"]
        assert isinstance(lin, W4A16Linear), p
        k = w.shape[1]
        x16 = rng.standard_normal((m, k)).astype(np.float16)
        y = lin(to_device_x(x16, torch.float16))
        check(y, x16.astype(np.float32) @ w.T, torch.float16, f"{p} m={m}")


@pytest.mark.gpu
@pytest.mark.parametrize("act_order", [False, True])
@pytest.mark.parametrize("m", [1, 80])
def test_gptq_checkpoint_end_to_end(tmp_path, act_order, m):
    tensors, dense_w, cfg = _model("gptq", act_order=act_order)
    arch = str(tmp_path / "gptq.pulsar")
    save_archive(arch, cfg, tensors, shards=3)
    w = load_weights(arch, device="cuda:0", dtype=torch.float16)
    assert w["model.norm.weight"].dtype == torch.float16 and w["model.norm.weight"].is_cuda
    lin = w["model.layers.0.self_attn.q_proj.weight"]
    assert lin.qzeros is not None and (lin.perm is not None) == act_order
    _check_linears(w, dense_w, m, seed=7)


@pytest.mark.gpu
@pytest.mark.parametrize("offset", [False, True])
def test_packed_checkpoint_end_to_end(tmp_path, offset):
    tensors, dense_w, cfg = _model("packed", offset=offset, seed=3)
    d = tmp_path / "packed"
    d.mkdir()
    (d / "config.json").write_text(json.dumps(cfg))
    from safetensors.torch import save_file
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(d / "model.safetensors"))
    w = load_weights(str(d), device="cuda:0", dtype=torch.float16)
    _check_linears(w, dense_w, 4, seed=8)
    # the repack is the reference's: bit-exact MARLIN words
    p = "model.layers.1.mlp.down_proj"
    packed = tensors[p + ".weight_packed"].numpy()
    if offset:
        packed = packed ^ np.int32(0x88888888 - (1 << 32))
    assert np.array_equal(w[p + ".weight"].weight_marlin.cpu().numpy(), O.repack_marlin(packed))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["gptq", "packed"])
def test_fused_projections_match_members(tmp_path, fmt):
    """fuse=True N-concatenates q|k|v and gate|up: each fused output's column slices equal the
    members' outputs (same kernels, one launch), and 3-D activations keep their shape."""
    tensors, _, cfg = _model(fmt, act_order=False, seed=5)
    arch = str(tmp_path / "m.pulsar")
    save_archive(arch, cfg, tensors)
    sep = load_weights(arch, device="cuda:0")
    fused = load_weights(arch, device="cuda:0", fuse=True)
    assert "model.layers.0.self_attn.q_proj.weight" not in fused
    x = torch.randn(2, 3, HIDDEN, device="cuda:0").half()
    for base, members in (("self_attn.", ("q", "k", "v")), ("mlp.", ("gate", "up"))):
        f = fused[f"model.layers.1.{base}{'qkv' if len(members) == 3 else 'gate_up'}_proj.weight"]
        yf = f(x)
        assert yf.shape == (2, 3, f.out_features)
        ys = torch.cat([sep[f"model.layers.1.{base}{m}_proj.weight"](x) for m in members], dim=-1)
        torch.testing.assert_close(yf.float(), ys.float(), rtol=2 ** -10, atol=1e-4)


@pytest.mark.gpu
def test_fusion_skipped_when_members_differ(tmp_path):
    """Members that cannot share one GEMM stay separate linears under their own names:
    act-order q, k, v (each permuted differently, as desc_act checkpoints are), and q whose
    zero points are all 8 (dropped at load: symmetric kernels) next to asymmetric k and v."""
    tensors, dense_w, cfg = _model("gptq", act_order=True, seed=11)
    arch = str(tmp_path / "act.pulsar")
    save_archive(arch, cfg, tensors, shards=2)
    w = load_weights(arch, device="cuda:0", dtype=torch.float16, fuse=True, silu_gate=True)
    for li in range(2):
        assert f"model.layers.{li}.self_attn.qkv_proj.weight" not in w
        assert f"model.layers.{li}.mlp.gate_up_proj.weight" not in w
    _check_linears(w, dense_w, 5, seed=12)

    tensors, dense_w, cfg = _model("gptq", act_order=False, seed=13)
    q = "model.layers.0.self_attn.q_proj"
    kq, nq = HIDDEN, HIDDEN
    tensors[q + ".qzeros"] = torch.full((kq // G, nq // 8), 0x77777777, dtype=torch.int32)  # v1: z - 1 = 7
    u = O.unpack_gptq(tensors[q + ".qweight"].numpy()).astype(np.float32)          # [N, K]
    s = tensors[q + ".scales"].numpy().astype(np.float32)                             # [K/G, N]
    dense_w[q] = (u - 8.0) * np.repeat(s, G, axis=0).T
    arch = str(tmp_path / "mixed.pulsar")
    save_archive(arch, cfg, tensors)
    w = load_weights(arch, device="cuda:0", dtype=torch.float16, fuse=True)
    assert w[q + ".weight"].qzeros is None
    assert "model.layers.0.self_attn.qkv_proj.weight" not in w     # q symmetric, k/v not: separate
    assert "model.layers.1.self_attn.qkv_proj.weight" in w         # layer 1 fuses as before
    assert "model.layers.0.mlp.gate_up_proj.weight" in w
    _check_linears({k: v for k, v in w.items()}, {p: d for p, d in dense_w.items() if "layers.0.self_attn" in p
                                                  and "o_proj" not in p}, 3, seed=14)


@pytest.mark.gpu
@pytest.mark.parametrize("bdtype", [torch.float32, torch.float16])
def test_linear_bias(bdtype):
    """W4A16Linear with a bias, as Qwen2's q, k and v projections carry one
    (at::linear(h, W, b), pulsar-core/src/model/qwen2.cpp:78-80): the rounded
    GEMM output plus the bias, rounded once, against the fp32 oracle plus bias."""
    m, n, k, g = 5, 320, 1024, 128
    p = O.make_problem(m, n, k, g, seed=11)
    rng = np.random.default_rng(11)
    b = (0.5 * rng.standard_normal(n)).astype(np.float32)
    if bdtype == torch.float16:
        b = b.astype(np.float16).astype(np.float32)
    lin = W4A16Linear.from_packed(torch.from_numpy(p.ct_packed()).cuda(),
                                  torch.from_numpy(p.scale_nk).cuda(), g,
                                  bias=torch.from_numpy(b).to(bdtype).cuda())
    x = torch.from_numpy(p.x16.view(np.float16)).cuda()
    y = lin(x)
    assert y.shape == (m, n) and y.dtype == torch.float16
    check(y, O.gemm_f32(p.xf, p.dequant()) + b, torch.float16, f"bias {bdtype}")
