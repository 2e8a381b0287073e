"""The Llama-3-8B linear stack as one captured graph.

* every replay reproduces the eager launches bit for bit, with the program's
  own eager work and synchronisations between replays, and follows new input
  values written between replays;
* through the graph, linears built from oracle weights match the fp32 oracle
  (dequantize-then-matmul) at M = 1 and M = 32.
"""

import pytest
import torch

from oracle import oracle as O
from pulsar_amd import ops
from pulsar_amd.linear import W4A16Linear
from pulsar_amd.stack import LLAMA3_8B_LINEARS, W4A16LinearStack, fuse_layers, random_layers
from w4a16_case import check, to_device_x

pytestmark = pytest.mark.gpu

G = 128


@pytest.mark.parametrize("m", [1, 32])
def test_stack_graph_replays_match_eager(m):
    layers = random_layers(2, device="cuda:0", seed=3)
    st = W4A16LinearStack(layers, m)
    st.capture()
    assert st.launches_per_step() == 14 and len(st.outputs) == 14
    assert [tuple(o.shape) for o in st.outputs[:7]] == [(m, n) for _, _, n in LLAMA3_8B_LINEARS]
    for rep in range(3):
        st.step()
        torch.cuda.synchronize()
        want = st.forward()  # eager, same inputs
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(st.outputs, want)):
            assert torch.equal(got, ref), f"replay {rep}, linear {i}"
        # new inputs between replays: the graph reads the same buffers
        for x in st.inputs.values():
            x.copy_(torch.randn_like(x, dtype=torch.float32).half())


@pytest.mark.parametrize("m", [1, 32])
def test_stack_graph_matches_oracle(m):
    probs = {k: O.make_problem(m, n, k, G, seed=20 + i) for i, (_, k, n) in enumerate([("k", 4096, 1024),
                                                                                    ("down", 14336, 4096)])}
    layer = []
    for name, (k, p) in zip(("k", "down"), probs.items()):
        qweight = torch.from_numpy(O.pack_gptq(p.u)).cuda()
        wm, _ = ops.repack_w4a16_gptq(qweight, None, G)
        scales = torch.from_numpy(p.scale_kn).half().cuda()  # exact: the values are fp16
        lin = W4A16Linear(wm, scales, G, k, p.n)
        lin.name = name
        layer.append(lin)
    st = W4A16LinearStack([layer], m)
    for k, p in probs.items():
        st.inputs[k].copy_(to_device_x(p.x16, torch.float16))
    st.capture()
    for _ in range(2):
        st.step()
        torch.cuda.synchronize()
        for (k, p), y in zip(probs.items(), st.outputs):
            y_ref = O.gemm_f32(p.xf, p.dequant())
            check(y, y_ref, torch.float16, f"stack m={m} k={k}")


def _close16(a, b):
    # Fused and separate linears may get different plans (unit width, K
    # slices), hence a different fp32 summation order: equal up to the fp16
    # rounding of the output (one ulp, 2^-10 relative), or, for outputs near
    # zero after cancellation, up to the reordering error of fp32 sums whose
    # terms are O(1) (1e-4 absolute).
    torch.testing.assert_close(a.float(), b.float(), rtol=2 ** -10, atol=1e-4)


@pytest.mark.parametrize("m", [1, 32])
def test_fused_stack_equals_unfused(m):
    """q|k|v and gate|up fused along N compute every column as the separate
    linears do, to the last bit where the plans agree and within one fp16 ulp
    where they do not."""
    layers = random_layers(1, device="cuda:0", seed=5)
    fused = fuse_layers(layers)
    assert [(l.name, l.in_features, l.out_features) for l in fused[0]] == [("qkv", 4096, 6144), ("o", 4096, 4096),
                                                      ("gate_up", 4096, 28672), ("down", 14336, 4096)]
    a = W4A16LinearStack(layers, m, seed=7)
    b = W4A16LinearStack(fused, m, seed=7)
    for k in a.inputs:
        assert torch.equal(a.inputs[k], b.inputs[k])
    a.capture()
    b.capture()
    a.step()
    b.step()
    torch.cuda.synchronize()
    ya, yb = a.outputs, b.outputs
    _close16(yb[0], torch.cat(ya[0:3], dim=1))
    _close16(yb[2], torch.cat(ya[4:6], dim=1))
    # o and down are the same linear in both stacks: same plan, same bits
    torch.testing.assert_close(yb[1], ya[3], rtol=0, atol=0)
    torch.testing.assert_close(yb[3], ya[6], rtol=0, atol=0)
    if m == 1:
        # one K slice, and gate|up takes the 64-column units that gate and up take alone:
        # identical plans, the same bits (q|k|v takes 32-column units where q, k and v
        # take 16: a different fp32 summation order, held to one ulp above)
        torch.testing.assert_close(yb[2], torch.cat(ya[4:6], dim=1), rtol=0, atol=0)


@pytest.mark.parametrize("m", [1, 32])
def test_silu_gated_stack(m):
    """fuse_layers(silu_gate=True): gate|up is one W4A16SiluGate whose output feeds down, as
    in the model; through the graph its output equals silu(gate) * up of the separate
    linears (up to their fp16 rounding) and down's output equals down applied eagerly to it."""
    layers = random_layers(1, device="cuda:0", seed=9)
    plain = W4A16LinearStack(layers, m, seed=4)
    gated = W4A16LinearStack(fuse_layers(layers, silu_gate=True), m, seed=4)
    assert gated.launches_per_step() == 4
    plain.capture()
    gated.capture()
    for _ in range(2):
        plain.step()
        gated.step()
        torch.cuda.synchronize()
        g, u = plain.outputs[4].float(), plain.outputs[5].float()
        ref = torch.nn.functional.silu(g) * u
        h = gated.outputs[2]
        assert h.shape == (m, 14336)
        torch.testing.assert_close(h.float(), ref, rtol=4e-3, atol=4e-3 * ref.abs().max().item())
        down = gated.layers[0][3]
        torch.testing.assert_close(gated.outputs[3], down(h), rtol=0, atol=0)


@pytest.mark.parametrize("variant", ["plain", "gated"])
@pytest.mark.parametrize("m", [1, 32])
def test_full_32_layer_graph_matches_eager(variant, m):
    """BASELINE config 5 at its real size: the 32-layer Llama-3-8B stack (224 linears, or
    128 launches with q|k|v fused and gate|up as the SiLU-gated GEMM feeding down), captured
    as one graph.  After two replays every output of every launch equals the eager launch
    on the same inputs, bit for bit; one linear of the last layer is also held to the
    oracle through its dequantized weights."""
    layers = random_layers(32, device="cuda:0", seed=9)
    if variant == "gated":
        layers = fuse_layers(layers, silu_gate=True)
    st = W4A16LinearStack(layers, m)
    st.capture()
    assert len(st.outputs) == st.launches_per_step() == (224 if variant == "plain" else 128)
    for _ in range(2):
        st.step()
    torch.cuda.synchronize()
    want = st.forward()
    torch.cuda.synchronize()
    for i, (got, ref) in enumerate(zip(st.outputs, want)):
        assert torch.equal(got, ref), f"{variant} m={m}: launch {i} differs from eager"
    del want
    if variant == "plain":
        # the last layer's k projection (K = 4096, N = 1024) against the oracle
        lin = layers[-1][1]
        k, n = lin.in_features, lin.out_features
        u = O.marlin_to_u(lin.weight_marlin.cpu().numpy(), n, k)
        w = (u.astype("float32") - 8.0) * lin.scales.float().cpu().numpy().repeat(G, axis=0).T
        x = st.inputs[k].float().cpu().numpy()
        check(st.outputs[-6], O.gemm_f32(x, w), torch.float16, f"stack layer 31 k_proj m={m}")
