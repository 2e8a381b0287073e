"""The plans the library picks for the BASELINE layers, read through pw4_plan_describe
(host logic only: nothing launches).  Each pinned choice is the measured-faster plan on
MI355X (256 CUs; graph periods in the comments, us, fp16 x):

* M = 29..32 on the decode kernel, except Llama-3-70B gate_up (8192 x 57344: M = 32 128
  decode / 118 prefill tile) and down (28672 x 8192: M = 32 69.5 / 61.7), which are faster
  on the 128-row prefill tile; at M = 28 and below the decode kernel (70B down M = 28 55.5 /
  61.6, 70B gate_up M = 24 101 / 115; M = 28 123 / 116 is the one measured miss), and at
  M = 32 on every other 8B and 70B layer (70B qkv 27.0 / 30.0, 8B gate_up 29.1 / 36.3, 8B
  down 25.0 / 32.0).
* Prefill K slices and K halves (128-row tiles whose 8-wave workgroup sums two K halves in
  LDS): Llama-3-8B qkv M = 1024 in K halves 56.6 (69.0 unsplit or on 2 slices), o M = 2048
  in K halves 65.7 (73.2 unsplit), o M = 1024 on 2 slices in K halves 46.9 (50.0 without),
  gate_up M = 256 in K halves 63.1 (69.8 unsplit), down M = 2048 in K halves 216.5 (224.3 on
  2 slices), down M = 256 on 8 slices in K halves 42.4 (44.7 without), o M = 256 on 8
  slices in K halves 24.7 (24.2 without: within 2%), and unsplit single-half tiles at
  M = 4096 (qkv 183.6 against 193.2 in K halves, gate_up 815 against 878).
"""

import ctypes
import os

import pytest

import pulsar_amd
from pw4_capi import DTYPE_BF16, DTYPE_F16, declare

LAYOUT_CT, LAYOUT_MARLIN = 0, 1
G = 128
L8 = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 28672), "down": (14336, 4096)}
L70 = {"qkv": (8192, 10240), "gate_up": (8192, 57344), "down": (28672, 8192)}
L70o = {"o": (8192, 8192)}
OVERRIDES = ("PW4_PREFILL_ROWS", "PW4_PREFILL_SPLITS", "PW4_PREFILL_KHALVES", "PW4_PREFILL_EXACT",
             "PW4_PREFILL_TILE", "PW4_DECODE", "PW4_DECODE_BLOCK_SCALES", "PW4_DECODE_PERM_LDS", "PW4_DECODE_NB",
             "PW4_DECODE_SPLITS", "PW4_DECODE_WPS", "PW4_DECODE_WIN")


@pytest.fixture(scope="module")
def lib():
    saved = {k: os.environ.pop(k) for k in OVERRIDES if k in os.environ}
    yield declare(pulsar_amd.capi())
    os.environ.update(saved)


def plan(lib, m, k, n, dtype=DTYPE_F16, layout=LAYOUT_MARLIN, zp=0, perm=0, silu=0, splits=0):
    buf = ctypes.create_string_buffer(160)
    rc = lib.pw4_plan_describe(layout, dtype, DTYPE_F16, zp, perm, silu, m, n, k, G, splits, buf, len(buf))
    assert rc == 0, rc
    return buf.value.decode()


@pytest.mark.parametrize("layer", ["gate_up", "down"])
@pytest.mark.parametrize("m", [29, 32])
@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_BF16])
def test_70b_large_layers_take_the_prefill_tile_from_m29(lib, layer, m, dtype):
    k, n = L70[layer]
    assert plan(lib, m, k, n, dtype).startswith("prefill256"), plan(lib, m, k, n, dtype)
    # act-order with zero points (config 4) plans the same way
    assert plan(lib, m, k, n, dtype, zp=1, perm=1).startswith("prefill256")


@pytest.mark.parametrize("layer", ["gate_up", "down"])
@pytest.mark.parametrize("m", [1, 16, 17, 24, 28])
def test_70b_large_layers_decode_to_m28(lib, layer, m):
    k, n = L70[layer]
    assert plan(lib, m, k, n).startswith("decode"), plan(lib, m, k, n)


@pytest.mark.parametrize("layer", ["8b_qkv", "8b_o", "8b_gate_up", "8b_down", "70b_qkv"])
@pytest.mark.parametrize("m", [1, 16, 28, 32])
def test_other_layers_decode_up_to_m32(lib, layer, m):
    model, name = layer.split("_", 1)
    k, n = (L8 if model == "8b" else L70)[name]
    assert plan(lib, m, k, n).startswith("decode"), (layer, m, plan(lib, m, k, n))


def test_m33_leaves_the_decode_kernel(lib):
    k, n = L8["down"]
    assert plan(lib, 33, k, n).startswith("prefill256")


def test_forced_splits_keep_the_decode_kernel(lib):
    # gemm_w4a16_marlin_split at decode sizes: the reference's split path, on the decode kernel
    # (8 slices: a 32-row slice of K / 8 fits the decode kernel's LDS, K / 4 does not)
    k, n = L70["gate_up"]
    assert plan(lib, 32, k, n, splits=8).startswith("decode"), plan(lib, 32, k, n, splits=8)


@pytest.mark.parametrize("layer,m,want", [
    ("o", 2048, "prefill256 rows=128 splits=1 exact=1 khalves=2"),
    ("o", 1024, "prefill256 rows=128 splits=2 exact=1 khalves=2"),
    ("o", 256, "prefill256 rows=128 splits=8 exact=1 khalves=2"),
    ("gate_up", 256, "prefill256 rows=128 splits=1 exact=1 khalves=2"),
    ("gate_up", 1024, "prefill256 rows=128 splits=1 exact=1 khalves=1"),
    ("gate_up", 4096, "prefill256 rows=128 splits=1 exact=1 khalves=1"),
    ("qkv", 1024, "prefill256 rows=128 splits=1 exact=1 khalves=2"),
    ("qkv", 2048, "prefill256 rows=128 splits=1 exact=1 khalves=1"),
    ("qkv", 4096, "prefill256 rows=128 splits=1 exact=1 khalves=1"),
    ("down", 256, "prefill256 rows=128 splits=8 exact=1 khalves=2"),
    ("down", 1024, "prefill256 rows=128 splits=4 exact=1 khalves=1"),
    ("down", 2048, "prefill256 rows=128 splits=1 exact=1 khalves=2"),
    ("down", 4096, "prefill256 rows=128 splits=1 exact=1 khalves=1"),
])
def test_prefill_splits_8b(lib, layer, m, want):
    k, n = L8[layer]
    assert plan(lib, m, k, n) == want


@pytest.mark.parametrize("layer,m,want", [
    ("qkv", 256, "splits=3 exact=1 khalves=2"), ("qkv", 1024, "splits=3"), ("qkv", 2048, "splits=2"),
    ("qkv", 4096, "splits=1"), ("gate_up", 1024, "splits=1"), ("down", 256, "splits=8"), ("down", 1024, "splits=2"),
    ("down", 2048, "splits=1"),
])
def test_prefill_splits_70b(lib, layer, m, want):
    k, n = L70[layer]
    assert want in plan(lib, m, k, n), plan(lib, m, k, n)


@pytest.mark.parametrize("layer,m,want", [
    ("qkv", 1024, "rows=128 splits=1 exact=0 khalves=2"), ("o", 1536, "rows=128 splits=1 exact=0 khalves=2"),
    ("gate_up", 256, "rows=128 splits=1 exact=0 khalves=2"), ("down", 2048, "rows=128 splits=1 exact=0 khalves=2"),
    ("qkv", 4096, "rows=256 splits=1"), ("gate_up", 4096, "rows=256 splits=1"),
])
def test_prefill_bf16_tail_rounds(lib, layer, m, want):
    """bf16 x (rounded scaling, 256-row tiles allowed).  A 256-row plan whose tail columns would
    run as 128-row tiles at one per CU is priced at that lone rate (1.1 us a chunk against
    1.6 for a 256-row tile): the 8B layers below take K halves instead.  Graph periods, us,
    two runs each, 256-row plan / K halves: qkv M = 1024 83.4, 82.0 / 72.8, 73.8; o M = 1536
    82.0, 81.8 / 73.1, 73.3; gate_up M = 256 84.5, 83.8 / 75.2, 74.8; down M = 2048 307,
    299 / 255, 267.  M = 4096 keeps 256-row tiles."""
    k, n = L8[layer]
    assert want in plan(lib, m, k, n, DTYPE_BF16), plan(lib, m, k, n, DTYPE_BF16)


def test_ct_layout_repacks_past_the_decode_range(lib):
    k, n = L8["o"]
    assert plan(lib, 16, k, n, layout=LAYOUT_CT).startswith("decode")
    assert plan(lib, 64, k, n, layout=LAYOUT_CT).endswith("repack")


def test_describe_rejects_bad_arguments(lib):
    buf = ctypes.create_string_buffer(8)
    assert lib.pw4_plan_describe(LAYOUT_MARLIN, DTYPE_F16, DTYPE_F16, 0, 0, 0, 1, 4096, 4096, G, 0, buf, 8) == -1
    big = ctypes.create_string_buffer(160)
    assert lib.pw4_plan_describe(7, DTYPE_F16, DTYPE_F16, 0, 0, 0, 1, 4096, 4096, G, 0, big, 160) == -1
    assert lib.pw4_plan_describe(LAYOUT_MARLIN, DTYPE_F16, DTYPE_F16, 0, 0, 0, 1, 4096, 4100, G, 0, big, 160) == -2


@pytest.mark.parametrize("layer,want", [("8b_gate_up", 1), ("8b_down", 1), ("70b_qkv", 1), ("70b_gate_up", 1),
                                        ("70b_down", 1), ("8b_qkv", 0), ("8b_o", 0)])
@pytest.mark.parametrize("m", [1, 16])
def test_decode_block_scales_on_large_layers(lib, layer, want, m):
    """One scale load per four steps on layers of 24 MiB or more (8B gate_up 3.0-3.2% and down
    0.8-2.6% faster, kernel-only medians of six runs), one per step on the small ones (o
    3.8-6.1% and qkv 0-3.6% slower with them)."""
    model, name = layer.split("_", 1)
    k, n = (L8 if model == "8b" else L70)[name]
    p = plan(lib, m, k, n)
    assert p.startswith("decode") and f" bs={want}" in p, p


@pytest.mark.parametrize("layer,m,want", [
    ("o", 1, 32), ("o", 4, 32), ("o", 8, 32), ("gate_up", 1, 32), ("gate_up", 8, 32), ("down", 1, 32),
    ("qkv", 1, 16), ("qkv", 8, 16),
])
@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_BF16])
def test_decode_unit_width_70b(lib, layer, m, want, dtype):
    """One slice over K >= 8192: 32-column units where the busiest CU gets no more columns than
    with 16 (one workgroup per CU, twice the steps per K wave between unit ends).  Kernel only,
    us, 16 / 32 columns, fp16: 70B o M = 1 9.44 / 8.70, M = 8 10.28 / 9.76; gate_up M = 2
    44.96 / 39.88, M = 8 45.27 / 40.96; down M = 1 24.48 / 23.66.  70B qkv keeps 16 (48
    columns on the busiest CU against 64 at 32)."""
    k, n = L70o[layer] if layer == "o" else L70[layer]
    p = plan(lib, m, k, n, dtype)
    assert p.startswith("decode") and f"nb={want} " in p, p


@pytest.mark.parametrize("layer,want", [("qkv", 32), ("gate_up", 64), ("o", 16), ("down", 16)])
@pytest.mark.parametrize("m", [1, 4, 8])
def test_decode_unit_width_8b(lib, layer, want, m):
    """One slice over K = 4096 at M <= 8: the widest units (at most 16 steps per K wave) whose
    workgroups cover 3/4 of the CUs with at most 1.15x the busiest CU's columns.  Kernel only,
    us, 16 columns / wider: qkv at 32 M = 1 5.64 / 5.28, M = 4 6.40 / 5.66, M = 8 6.52 / 6.28;
    gate_up at 64 M = 1 13.28 / 12.36, M = 4 13.60 / 12.76.  o keeps 16 (32 columns would
    leave half the CUs idle), and so does down (K = 14336; at M = 8 on the exchange tree)."""
    k, n = L8[layer]
    p = plan(lib, m, k, n)
    assert p.startswith("decode") and (f"nb={want} " in p or (layer == "down" and " tree=1" in p)), p


@pytest.mark.parametrize("layer,k,n,m,want", [
    ("70b_down", 28672, 8192, 4, 64), ("70b_down", 28672, 8192, 8, 64), ("70b_o", 8192, 8192, 16, 32),
    ("8b_down", 14336, 4096, 16, 32), ("8b_down", 14336, 4096, 8, 32),
])
def test_decode_tree_units_64_on_long_slices(lib, layer, k, n, m, want):
    """Exchange-tree plans take 64-column units where their slices split evenly over the CUs
    and each K wave of a unit streams 24 steps or more (70B down, K = 28672, M = 4 / 8:
    kernel only, 32 / 64 columns, 24.3 / 22.7 and 28.1 / 25.6 us, fp16).  Shorter units keep
    32 columns (70B o at M = 16, 8B down at M = 8-16)."""
    p = plan(lib, m, k, n)
    assert " tree=1" in p and f"nb={want} " in p, p
