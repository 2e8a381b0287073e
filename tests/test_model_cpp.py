"""The C++ model layer (include/pulsar_w4a16_model.hpp) on the GPU, reached
through its torch class pulsar.Qwen3W4A16Layer: the W4A16 linears at the
at::linear sites of Qwen3Model::block (pulsar-core/src/model/qwen3.cpp:77-121),
built in C++ from a checkpoint's weights map (both quantized formats, fused
q|k|v and SiLU-gated gate|up, or separate linears when act-order permutations
differ), checked against the fp32 oracle.  The Qwen2 cases add the q, k and v
biases of Qwen2Model::block (at::linear(h, W, b), qwen2.cpp:78-80) to the map.

The whole-block check uses attention over a one-token context (each token
attends only to itself, so o = v repeated per query head) and restates the
block's arithmetic in numpy around the oracle's GEMMs, rounding to fp16 where
the C++ path does (each GEMM output, the residual adds, the norms): what is
left is fp32 summation order, held to the reference's relative bar and the
north star's rel-L2 bar.
"""

import numpy as np
import pytest
import torch

import pulsar_amd  # noqa: F401  (loads the torch class)
from oracle import oracle as O
from w4a16_case import check

pytestmark = pytest.mark.gpu

G = 128
EPS = 1e-6
PROJ = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
        "mlp.up_proj", "mlp.down_proj")


def _shapes(hidden, heads, kv_heads, head_dim, inter):
    q, kv = heads * head_dim, kv_heads * head_dim
    return {"self_attn.q_proj": (hidden, q), "self_attn.k_proj": (hidden, kv), "self_attn.v_proj": (hidden, kv),
            "self_attn.o_proj": (q, hidden), "mlp.gate_proj": (hidden, inter), "mlp.up_proj": (hidden, inter),
            "mlp.down_proj": (inter, hidden)}


def _layer(fmt, shapes, seed, act_order=False, bias=False):
    """A weights map for one layer (device tensors), each projection's fp32 dense
    weight, and (bias=True) fp16 biases of q, k and v as Qwen2 has them."""
    weights, dense, biases = {}, {}, {}
    rng = np.random.default_rng(seed)
    for i, name in enumerate(PROJ):
        k, n = shapes[name]
        p = O.make_problem(1, n, k, G, seed=seed + i, symmetric=fmt == "packed", act_order=act_order)
        key = f"model.layers.0.{name}."
        if fmt == "packed":
            weights[key + "weight_packed"] = torch.from_numpy(p.ct_packed()).cuda()
            weights[key + "weight_scale"] = torch.from_numpy(O.f32_to_f16_bits(p.scale_nk).view(np.float16)).cuda()
        else:
            weights[key + "qweight"] = torch.from_numpy(p.qweight()).cuda()
            weights[key + "scales"] = torch.from_numpy(O.f32_to_f16_bits(p.scale_kn).view(np.float16)).cuda()
            weights[key + "qzeros"] = torch.from_numpy(p.qzeros()).cuda()
            if act_order:
                weights[key + "g_idx"] = torch.from_numpy(p.g_idx).cuda()
        dense[name] = p.dequant()
        if bias and name in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"):
            b = _f16(0.5 * rng.standard_normal(n))
            weights[key + "bias"] = torch.from_numpy(b.astype(np.float16)).cuda()
            biases[name] = b
    return weights, dense, biases


def _f16(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def _rms(x, w):
    inv = 1.0 / np.sqrt((x.astype(np.float32) ** 2).mean(axis=-1, keepdims=True) + np.float32(EPS))
    return _f16(x * inv * w)


def _block_ref(x, ln1, ln2, dense, heads, kv_heads, head_dim, biases):
    h = _rms(x, ln1)
    v = _f16(O.gemm_f32(h, dense["self_attn.v_proj"]))
    if "self_attn.v_proj" in biases:
        v = _f16(v + biases["self_attn.v_proj"])
    o = np.repeat(v.reshape(len(x), kv_heads, 1, head_dim), heads // kv_heads, axis=2).reshape(len(x), -1)
    x1 = _f16(x + _f16(O.gemm_f32(o, dense["self_attn.o_proj"])))
    h2 = _rms(x1, ln2)
    g = O.gemm_f32(h2, dense["mlp.gate_proj"])
    u = O.gemm_f32(h2, dense["mlp.up_proj"])
    a = _f16(g / (1.0 + np.exp(-g.astype(np.float64))) * u)
    return _f16(x1 + _f16(O.gemm_f32(a, dense["mlp.down_proj"])))


# (format, act-order, q/k/v biases (Qwen2), hidden, heads, kv heads, head dim, intermediate, tokens)
CASES = [
    ("gptq", False, False, 512, 8, 2, 64, 1024, 1),
    ("gptq", False, False, 512, 8, 2, 64, 1024, 300),
    ("packed", False, False, 512, 8, 2, 64, 1024, 16),
    ("gptq", True, False, 512, 8, 2, 64, 1024, 7),         # act-order: separate linears
    ("packed", False, False, 4096, 32, 8, 128, 14336, 4),  # Llama-3-8B layer
    ("packed", False, True, 896, 14, 2, 64, 4864, 5),      # Qwen2-0.5B layer, biased q|k|v
    ("gptq", True, True, 512, 8, 2, 64, 1024, 3),          # Qwen2-style, act-order: separate biased q, k, v
]


@pytest.mark.parametrize("fmt,act,bias,hidden,heads,kv_heads,head_dim,inter,t", CASES)
def test_qwen3_layer_linears(fmt, act, bias, hidden, heads, kv_heads, head_dim, inter, t):
    shapes = _shapes(hidden, heads, kv_heads, head_dim, inter)
    weights, dense, biases = _layer(fmt, shapes, seed=hidden + t + (7 if act else 0), act_order=act, bias=bias)
    layer = torch.classes.pulsar.Qwen3W4A16Layer(weights, "model.layers.0.", G, heads, kv_heads, head_dim)
    assert tuple(layer.fusion()) == ((3, 2) if act else (1, 1))
    rng = np.random.default_rng(t)
    x = _f16(rng.standard_normal((t, hidden)))
    xd = torch.from_numpy(x.astype(np.float16)).cuda()
    # the three projections of h = x
    q, k, v = layer.qkv(xd)
    for got, name in ((q, "self_attn.q_proj"), (k, "self_attn.k_proj"), (v, "self_attn.v_proj")):
        ref = O.gemm_f32(x, dense[name]) + biases.get(name, np.float32(0))
        check(got, ref, torch.float16, f"{fmt} {name} t={t} bias={bias}")
    # the MLP residual on its own: x + down(silu(gate(x)) * up(x))
    g = O.gemm_f32(x, dense["mlp.gate_proj"])
    u = O.gemm_f32(x, dense["mlp.up_proj"])
    a = g / (1.0 + np.exp(-g.astype(np.float64))) * u
    ref_mlp = x + O.gemm_f32(_f16(a), dense["mlp.down_proj"])
    check(layer.mlp_residual(xd, xd), ref_mlp, torch.float16, f"{fmt} mlp t={t}", abs_excess=False)
    # the whole block with one-token attention
    ln1 = _f16(1.0 + 0.1 * rng.standard_normal(hidden))
    ln2 = _f16(1.0 + 0.1 * rng.standard_normal(hidden))
    y = layer.block_self_attention(xd, torch.from_numpy(ln1.astype(np.float16)).cuda(),
                                   torch.from_numpy(ln2.astype(np.float16)).cuda(), EPS)
    assert y.shape == (t, hidden) and y.dtype == torch.float16
    ref = _block_ref(x, ln1, ln2, dense, heads, kv_heads, head_dim, biases)
    check(y, ref, torch.float16, f"{fmt} block t={t}", abs_excess=False)


def test_missing_weight_is_reported():
    shapes = _shapes(512, 8, 2, 64, 1024)
    weights, _, _ = _layer("gptq", shapes, seed=3)
    del weights["model.layers.0.mlp.up_proj.qweight"]
    with pytest.raises(RuntimeError, match="mlp.up_proj"):
        torch.classes.pulsar.Qwen3W4A16Layer(weights, "model.layers.0.", G, 8, 2, 64)
