"""The hip backend without a GPU: generated source, launch plans, statistics, the C ABI library.

The counterpart of the reference's GPU-less codegen tests (tests/test_cuda.py:107-276): lowering
decisions are asserted on the generated text and statistics, every operator family is cross-compiled
for gfx950 with hipcc, and the runtime library is checked to export every entry point of
include/chroma_hip.h.
"""

from __future__ import annotations

import ctypes
import json
import re
from pathlib import Path

import pytest
import torch

from chroma_amd._src import native
from chroma_amd._src.build import build
from chroma_amd._src.codegen.hip import HIPCodegen
from chroma_amd._src.compiler import Compiler, compile_for_backend, lower_program
from chroma_amd.models.gpt_oss import RMSNorm
from tests.helpers import Function, export, random_transformer, small_config

ROOT = Path(__file__).resolve().parents[1]


def lower(module, *inputs, blas=True):
    return lower_program(export(module, *inputs), HIPCodegen(blas=blas))


class Bandwidth(torch.nn.Module):
    def forward(self, x, y):
        z = torch.tanh(x * 0.5 + y) * torch.sigmoid(y) - torch.exp(torch.clamp(x, -8, 8)) * 1e-3
        return torch.softmax(z, -1)


def test_bandwidth_graph_is_one_single_pass_kernel():
    generated = lower(Bandwidth(), torch.rand(64, 8192), torch.rand(64, 8192))
    source = generated.files["model.hip"]
    assert generated.stats["kernels"] == 1 and generated.stats["workspace_bytes"] == 0
    assert generated.stats["backend"] == "hip"
    # x and y are each read once with 128-bit loads; the softmax output is written in place (promoted).
    assert source.count("reinterpret_cast<const float4*>") == 2
    # 8192-wide rows split evenly into two float4 steps of 1024 threads: 16 waves per row
    assert "__launch_bounds__(1024)" in source
    assert "chroma::fast_tanh" in source and "chroma::block_max<16>" in source and "chroma::block_sum<16>" in source
    plan = generated.files["model.plan"].splitlines()
    launches = [line for line in plan if line.startswith("launch ")]
    assert len(launches) == 1 and launches[0].split()[2:5] == ["64", "1", "1"]


def test_dev_model_reuses_kernels_across_layers():
    from chroma_amd.models.dev import make_dev_model

    generated = lower(make_dev_model(0), torch.arange(8, dtype=torch.int64))
    stats = generated.stats
    assert stats["expert_contractions"] == 24
    assert stats["workspace_bytes"] < stats["unreused_workspace_bytes"]
    # Small concatenations, clones of views and multi-consumer expressions fuse into their consumers, the
    # attention chain is one launch that also computes the output projection, RMSNorms fold into the
    # kernels that stage their rows, the router (gate linear, top-k, softmax) is one launch and the
    # weighted sum of the four selected experts is an expression: 5 launches per layer plus the final norm
    # (stored, as the wide unembedding would repeat it in every workgroup) and the unembedding (the
    # reference's CUDA backend: 361).
    assert stats["fused_attentions"] == 12 and stats["fused_routers"] == 12 and stats["small_contractions"] == 12
    assert stats["attention_epilogues"] == 12
    # The residual stream is stored every layer, by the next layer's first kernel, which evaluates the sum
    # while staging its rows anyway (no copy launches).
    assert stats["write_through_stores"] == 11
    assert stats["launches"] == stats["kernels"] <= 12 * 5 + 2
    # Kernels are deduplicated across layers: the attention and second expert product kernels are shared by
    # all twelve layers (the kernels that fold a norm read the layer's own residual expression).
    plan = [line.split()[1] for line in generated.files["model.plan"].splitlines() if line.startswith("launch ")]
    shared = [name for name in set(plan) if plan.count(name) == 12]
    assert len(shared) >= 2 and stats["unique_kernels"] == len(set(plan)) < stats["launches"] * 2 // 3


def test_wide_topk_takes_two_stages():
    """A top-k over a vocabulary-wide row cannot hold the row in one wave's registers: per-chunk selection,
    then a merge of the chunk lists (two launches, scratch for the lists)."""
    class TopK(torch.nn.Module):
        def forward(self, x):
            return torch.topk(x, 40, dim=-1)

    generated = lower(TopK(), torch.randn(2, 201088))
    source = generated.files["model.hip"]
    assert "chroma_topk_chunks" in source and "chroma_topk_merge" in source
    assert generated.stats["launches"] == 2
    narrow = lower(TopK(), torch.randn(2, 2048)).files["model.hip"]
    assert "chroma_topk_chunks" not in narrow


def test_linear_kernel_selection():
    module = torch.nn.Linear(16, 7).eval()
    for blas, rows, kind in ((True, 3, "linear_stream"), (True, 40, "linear_mfma"), (False, 3, "linear_scalar")):
        generated = lower(module, torch.ones(rows, 16), blas=blas)
        assert kind in generated.files["model.hip"], kind
        assert generated.stats["workspace_bytes"] == 0  # the result is written straight into the output
    assert "linear_tiled" in lower(torch.nn.Linear(17, 7).eval(), torch.ones(40, 17)).files["model.hip"]
    # rows that are not a whole number of 16-byte chunks keep the 4-element skinny kernel
    assert "linear_skinny" in lower(torch.nn.Linear(12, 7).bfloat16().eval(), torch.ones(3, 12, dtype=torch.bfloat16)).files["model.hip"]
    # bfloat16 with K a multiple of 64 takes the direct-to-LDS body on 512 threads; other K the register-staged ones
    direct = lower(torch.nn.Linear(64, 7).bfloat16().eval(), torch.ones(40, 64, dtype=torch.bfloat16)).files["model.hip"]
    assert "mfma_linear<uint16_t, 2>" in direct and "__launch_bounds__(512, 2)" in direct
    assert "mfma_linear<uint16_t, 0>" in lower(torch.nn.Linear(40, 7).bfloat16().eval(), torch.ones(40, 40, dtype=torch.bfloat16)).files["model.hip"]
    # products with at least 200 of the wide body's 256 x 192 tiles take it (4 waves, one workgroup per CU);
    # one tile row fewer takes the mid ring body (at least 160 tiles of 128 x 192), fewer tiles the 128 x 128 body
    wide = lower(torch.nn.Linear(32, 4800).bfloat16().eval(), torch.ones(2048, 32, dtype=torch.bfloat16)).files["model.hip"]
    assert "chroma::mfma_linear_wide<uint16_t>" in wide and "__launch_bounds__(256, 1)" in wide
    narrow = lower(torch.nn.Linear(32, 4800).bfloat16().eval(), torch.ones(1792, 32, dtype=torch.bfloat16)).files["model.hip"]
    assert "mfma_linear_wide" not in narrow and "chroma::mfma_linear_mid<uint16_t>" in narrow
    small = lower(torch.nn.Linear(32, 4800).bfloat16().eval(), torch.ones(640, 32, dtype=torch.bfloat16)).files["model.hip"]
    assert "mfma_linear_mid" not in small and "mfma_linear<uint16_t, 0>" in small
    # bfloat16 keeps float accumulation in both paths
    generated = lower(torch.nn.Linear(17, 7).bfloat16().eval(), torch.ones(3, 5, 17, dtype=torch.bfloat16))
    assert generated.inputs[0]["dtype"] == "bfloat16" and generated.outputs[0]["dtype"] == "bfloat16"
    source = generated.files["model.hip"]
    assert "chroma::tiled_linear<uint16_t>" in source  # float accumulators, one bf16 rounding at the store


def test_large_weights_are_read_ahead_of_their_matrix_core_product():
    """Matrix-core linears over 4-64 MiB of constant weights get a read-ahead launch (chroma_prefetch) just
    before them; smaller weights, streamed few-row products and weights computed in the graph do not."""
    big = lower(torch.nn.Linear(2048, 2048, bias=False).bfloat16().eval(), torch.ones(512, 2048, dtype=torch.bfloat16))
    plan = [line.split()[1] for line in big.files["model.plan"].splitlines() if line.startswith("launch ")]
    assert big.stats["weight_prefetches"] == 1 and plan[0].startswith("chroma_prefetch_") and len(plan) == 2
    assert "chroma::prefetch_bytes(" in big.files["model.hip"] and f"{2048 * 2048 * 2}ull" in big.files["model.hip"]
    small = lower(torch.nn.Linear(1024, 1024, bias=False).bfloat16().eval(), torch.ones(512, 1024, dtype=torch.bfloat16))
    few = lower(torch.nn.Linear(2048, 2048, bias=False).bfloat16().eval(), torch.ones(2, 2048, dtype=torch.bfloat16))
    computed = lower(Function(lambda x, w: torch.nn.functional.linear(x, w * 2)), torch.ones(512, 2048).bfloat16(),
                     torch.ones(2048, 2048).bfloat16())
    assert small.stats["weight_prefetches"] == few.stats["weight_prefetches"] == computed.stats["weight_prefetches"] == 0


def test_shared_expressions_and_workspace_reuse():
    def fn(x, w):
        first = torch.nn.functional.linear(x, w)
        shared = first.sin()
        second = torch.nn.functional.linear(shared + 1, w)
        third = torch.nn.functional.linear(second + shared, w)
        return third, first[:, 1:], shared

    compiler = Compiler.from_export(export(Function(fn), torch.ones(40, 16), torch.eye(16)), HIPCodegen())
    generated = compiler.lower()
    assert generated.stats["workspace_bytes"] > 0
    allocations = list(compiler.codegen.allocations.values())
    for i, a in enumerate(allocations):
        for b in allocations[i + 1 :]:
            if a.start <= b.end and b.start <= a.end:
                assert a.offset + a.size <= b.offset or b.offset + b.size <= a.offset
    assert generated.stats["workspace_bytes"] < generated.stats["unreused_workspace_bytes"]


def test_long_expressions_stay_bounded():
    def fn(x):
        for _ in range(80):
            x = x.clamp(-1, 1)
        return x

    generated = lower(Function(fn), torch.ones(257))
    assert generated.stats["kernels"] == 4
    assert len(generated.files["model.hip"]) < 60_000


def test_plan_regions_are_aligned_disjoint_and_every_argument_is_inside_the_allocation():
    generated = lower(random_transformer(small_config(), seed=5, std=0.1), torch.tensor([1, 4, 2, 7]))
    lines = generated.files["model.plan"].splitlines()
    arena = int(next(l for l in lines if l.startswith("arena")).split()[1])
    regions = []
    for line in lines:
        if line.startswith(("input", "output")):
            _, _, offset, size = line.split()
            assert int(offset) % 256 == 0
            regions.append((int(offset), int(offset) + int(size)))
    regions.sort()
    for (a0, a1), (b0, b1) in zip(regions, regions[1:]):
        assert a1 <= b0
    for line in lines:
        if line.startswith("launch"):
            fields = line.split()
            count = int(fields[7])
            offsets = list(map(int, fields[8 : 8 + count]))
            assert len(offsets) == count and all(0 <= o < arena for o in offsets)
    # the error region (error word, router and decode-attention tickets) is 1 KiB that no region overlaps
    error = int(next(l for l in lines if l.startswith("error")).split()[1])
    assert all(start >= error + 1024 or end <= error for start, end in regions)


class CachedAttention(torch.nn.Module):
    """The workload's attention with sinks over past and new keys (gpt_oss.py sdpa, cached.py:38-48)."""

    def forward(self, q, k_past, k_new, v_past, v_new, mask, sinks):
        tokens, kv_heads, group, dim = q.shape
        k = torch.cat((k_past, k_new))[:, :, None, :].expand(-1, -1, group, -1)
        v = torch.cat((v_past, v_new))[:, :, None, :].expand(-1, -1, group, -1)
        scores = torch.einsum("qhmd,khmd->hmqk", q, k) * (1 / dim**0.5) + mask[None, None, :, :]
        s = sinks.reshape(kv_heads, group, 1, 1).expand(-1, -1, tokens, -1)
        weights = torch.softmax(torch.cat([scores, s], dim=-1), dim=-1)[..., :-1]
        return torch.einsum("hmqk,khmd->qhmd", weights, v)


def cached_attention_inputs(tokens, past, kv_heads, group, dim):
    dtype = torch.bfloat16
    mask = torch.zeros(tokens, past + tokens, dtype=dtype)
    return (torch.randn(tokens, kv_heads, group, dim).to(dtype), torch.randn(past, kv_heads, dim).to(dtype),
            torch.randn(tokens, kv_heads, dim).to(dtype), torch.randn(past, kv_heads, dim).to(dtype),
            torch.randn(tokens, kv_heads, dim).to(dtype), mask, torch.randn(kv_heads * group).to(dtype))


class NormLinear(torch.nn.Module):
    def __init__(self, width, columns):
        super().__init__()
        self.norm = RMSNorm(width)
        self.linear = torch.nn.Linear(width, columns, bias=False)

    def forward(self, x, y):
        return self.linear(self.norm(x + y))


def test_staging_loops_request_every_trip_before_their_arithmetic():
    """A one-row product whose X is a norm of a sum (a decode step's QKV product at hidden size 2880):
    the prologue's staging loops run a fixed 12 trips per thread with a clamped index, and the loop that
    loads the sum's two operands first requests every trip's loads into per-trip arrays, then does the
    arithmetic past a scheduling barrier."""
    module = NormLinear(2880, 512).to(torch.bfloat16)
    x, y = torch.randn(1, 2880).to(torch.bfloat16), torch.randn(1, 2880).to(torch.bfloat16)
    source = lower(module, x, y).files["model.hip"]
    assert "linear_stream" in source
    assert "for (uint32_t trip = 0; trip < 12u; ++trip) {" in source
    assert "const uint32_t i = slot < 2880u ? slot : 2879u;" in source
    arrays = re.findall(r"float (pre\d+)\[12\];", source)
    assert len(arrays) >= 2 and '__asm__ volatile("" ::: "memory");' in source
    for array in arrays:
        assert f"{array}[trip] = " in source  # filled in the loads-only loop ...
        assert source.count(f"{array}[trip]") >= 2  # ... and read in the arithmetic loop


def test_rotary_halves_are_written_by_one_thread():
    """A rotary embedding's concatenation of two equal halves along the last dimension: one thread writes
    both halves of a position (half as many vectors, two 16-byte stores, no branch on the part), and the
    loads the halves share (x1, x2, cos, sin) appear once."""

    def rotary(x, cos, sin):
        x1, x2 = x[..., :32], x[..., 32:]
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1)

    x = torch.randn(256, 8, 64).to(torch.bfloat16)
    cos, sin = torch.randn(256, 1, 32).to(torch.bfloat16), torch.randn(256, 1, 32).to(torch.bfloat16)
    source = lower(Function(rotary), x, cos, sin).files["model.hip"]
    kernel = source[source.index("chroma_concat_"):]
    kernel = kernel[: kernel.index("\n}\n")]
    assert f"v < {256 * 8 * 64 // 8 // 2}u" in kernel
    assert kernel.count("*reinterpret_cast<uint4*>(b0 + ") == 2
    assert "if (j" not in kernel
    loads = re.findall(r"reinterpret_cast<const uint4\*>\((b\d+ \+ [^)]*)\)", kernel)
    assert len(loads) == len(set(loads)) == 4  # x1, x2, cos, sin: 16 bytes each, once


@pytest.mark.parametrize("dtype, dim", [(torch.float32, 128), (torch.bfloat16, 256)])
def test_long_cache_attention_with_wide_heads_cross_compiles(tmp_path, dtype, dim):
    """Head dimensions whose split would give a decode-attention thread more than 8 keys take the general
    split-key kernels, and the program builds for gfx950."""
    mask = torch.zeros(1, 1001, dtype=dtype)
    inputs = (torch.randn(1, 2, 4, dim).to(dtype), torch.randn(1000, 2, dim).to(dtype), torch.randn(1, 2, dim).to(dtype),
              torch.randn(1000, 2, dim).to(dtype), torch.randn(1, 2, dim).to(dtype), mask, torch.randn(8).to(dtype))
    generated = lower(CachedAttention(), *inputs)
    assert "attention_decode" not in generated.files["model.hip"] and generated.stats["fused_attentions"] == 1
    build(generated, tmp_path / "program", load=False)


def test_grouped_prefill_attention_takes_two_heads_per_wave():
    """A bfloat16 prefill over a mask shared by every head (the workloads' case) runs ``attention_heads`` with
    two query heads per wave when the group is even and the head dimension at most 64 (half the waves: 256
    threads for a group of 8, compiled for three resident workgroups per compute unit), one otherwise."""
    dtype = torch.bfloat16
    for group, heads, threads in ((8, 2, 256), (3, 1, 192)):
        mask = torch.zeros(128, 160, dtype=dtype)
        inputs = (torch.randn(128, 1, group, 64).to(dtype), torch.randn(32, 1, 64).to(dtype), torch.randn(128, 1, 64).to(dtype),
                  torch.randn(32, 1, 64).to(dtype), torch.randn(128, 1, 64).to(dtype), mask, torch.randn(group).to(dtype))
        source = lower(CachedAttention(), *inputs).files["model.hip"]
        assert f"chroma::attention_heads_mfma_bf16<64, {group}, true, {heads}>(a);" in source
        bounds = f"__launch_bounds__({threads}, 3)" if heads == 2 else f"__launch_bounds__({threads})"
        assert re.search(re.escape(bounds) + r" chroma_attention_heads_", source), source[:300]
        # the live-tile table of a mask whose rows are whole 16-byte chunks: one wave per tile
        assert "chroma::attention_live_tiles_wave(" in source
    ragged = (torch.randn(128, 1, 8, 64).to(dtype), torch.randn(36, 1, 64).to(dtype), torch.randn(128, 1, 64).to(dtype),
              torch.randn(36, 1, 64).to(dtype), torch.randn(128, 1, 64).to(dtype), torch.zeros(128, 164, dtype=dtype), torch.randn(8).to(dtype))
    source = lower(CachedAttention(), *ragged).files["model.hip"]
    assert "chroma::attention_live_tiles(" in source and "attention_live_tiles_wave" not in source  # 164-key rows


def test_decode_attention_is_two_launches_with_tickets_inside_the_error_region():
    """A long cache read by few (query row, head) rows: scores and statistics, then partial sums whose last
    split adds them (no combine launch); each row's ticket word lies in the error region's decode-attention
    words (64-127). 64 or more rows take the general split-key kernels instead."""
    generated = lower(CachedAttention(), *cached_attention_inputs(1, 4096, 8, 8, 64))
    kernels = [line.split()[1] for line in generated.files["model.plan"].splitlines() if line.startswith("launch ")]
    assert [re.sub(r"_[0-9a-f]{8}$", "", name) for name in kernels] == ["chroma_attention_decode1", "chroma_attention_decode2"]
    source = generated.files["model.hip"]
    assert source.count("error + chroma::kAttentionTicketWord + blockIdx.x * 8u + blockIdx.y") == 2
    header = (ROOT / "chroma_amd/csrc/include/chroma_hip/attention.h").read_text()
    word = int(re.search(r"kAttentionTicketWord = (\d+)", header).group(1))
    rows = int(re.search(r"kAttentionTickets = (\d+)", header).group(1))
    assert word >= 64 and (word + rows) * 4 <= 1024  # router tickets end at word 63; the region is 1 KiB
    wide = lower(CachedAttention(), *cached_attention_inputs(8, 1024, 8, 1, 64))  # 64 rows
    assert "chroma_attention_decode" not in wide.files["model.hip"]


class GroupedExperts(torch.nn.Module):
    def forward(self, weights, indices, x, per_slot):
        selected = weights[indices]
        return torch.einsum("beck,bk->bec", selected, x), torch.einsum("beck,bek->bec", selected, per_slot)


def test_expert_ring_bodies_cross_compile_with_tall_last_tiles(tmp_path):
    """Every ring tile width builds for gfx950 with its bodies in one kernel (the live-row variants of the
    128-slot tile, and the 160-slot last tile where its rule takes it), and both products of a layer share
    one routing."""
    from chroma_amd._src.codegen.hip import RING_EXPERT_TILES

    for width, waves, last in RING_EXPERT_TILES:
        experts, tokens, selected, inner = 4, 160, 2, 64
        inputs = (torch.randn(experts, width, inner).to(torch.bfloat16), torch.randint(0, experts, (tokens, selected)),
                  torch.randn(tokens, inner).to(torch.bfloat16), torch.randn(tokens, selected, inner).to(torch.bfloat16))
        generated = lower(GroupedExperts(), *inputs)
        source = generated.files["model.hip"]
        assert source.count(f", 3, {width}, 1, {waves}, {last}>(") == 2
        assert source.count("chroma::route_slots(") == 1
        build(generated, tmp_path / f"ring{width}", load=False)


def test_gated_activation_is_the_first_expert_products_epilogue(tmp_path, monkeypatch):
    """The MoE MLP's clamped SwiGLU (and the first product's bias) between its two expert products is
    computed in the first product's epilogue: one launch fewer, and the first product is not stored when
    nothing else reads it; when the graph also returns it, the fused kernel stores it too. Both build for
    gfx950."""
    from chroma_amd._src.codegen import hip as codegen
    from tests.helpers import ExpertMLP

    x = torch.randn(256, 64).to(torch.bfloat16)
    monkeypatch.setattr(codegen, "NORM_EPILOGUES", False)  # counted on their own below
    monkeypatch.setattr(codegen, "ACTIVATION_EPILOGUES", False)
    plain = lower(ExpertMLP(), x)
    assert plain.stats["expert_epilogues"] == 0
    monkeypatch.setattr(codegen, "ACTIVATION_EPILOGUES", True)
    fused = lower(ExpertMLP(), x)
    assert fused.stats["expert_epilogues"] == 1 and fused.stats["unstored_products"] == 1
    assert fused.stats["launches"] == plain.stats["launches"] - 1
    source = fused.files["model.hip"]
    assert "auto epilogue = [&]" in source and ", epilogue);" in source and "uint2{" not in source
    build(fused, tmp_path / "fused", load=False)
    both = lower(ExpertMLP(product=True), x)
    assert both.stats["expert_epilogues"] == 1 and both.stats["unstored_products"] == 0
    assert "uint2{" in both.files["model.hip"]  # the epilogue stores the product as well
    build(both, tmp_path / "both", load=False)


def test_norm_cast_is_the_norm_kernels_epilogue(tmp_path, monkeypatch):
    """The bfloat16 cast a workload's RMSNorm ends with is written by the norm kernel itself (one launch
    fewer, no float round trip); when the graph also returns the float rows, the fused kernel keeps
    writing them. Both build for gfx950."""
    from chroma_amd._src.codegen import hip as codegen
    from tests.helpers import NormThenLinear

    x = torch.randn(256, 256).to(torch.bfloat16)
    monkeypatch.setattr(codegen, "NORM_EPILOGUES", False)
    plain = lower(NormThenLinear(), x)
    monkeypatch.setattr(codegen, "NORM_EPILOGUES", True)
    fused = lower(NormThenLinear(), x)
    assert plain.stats["norm_epilogues"] == 0 and fused.stats["norm_epilogues"] == 1
    assert fused.stats["launches"] == plain.stats["launches"] - 1 and fused.stats["unstored_products"] == 1
    build(fused, tmp_path / "fused", load=False)
    both = lower(NormThenLinear(both=True), x)
    assert both.stats["norm_epilogues"] == 1 and both.stats["unstored_products"] == 0
    build(both, tmp_path / "both", load=False)


def test_constant_tables_are_computed_once():
    """A stored map that reads only weights and graph inputs is launched once per distinct kernel and
    bindings: the prefill's per-layer rotary cos/sin tables (a transcendental table stored for its many
    readers) are computed by the first layer and read by the others."""
    from chroma_amd.models.cached import export_cached

    # tables of 512 steps x 16 frequencies: large enough to be stored, in each of 3 layers
    model = random_transformer(small_config(num_hidden_layers=3, head_dim=32, num_attention_heads=2, num_key_value_heads=1),
                               seed=1, std=0.1)
    generated = lower_program(export_cached(model, 512, 512), HIPCodegen())
    assert generated.stats["reused_maps"] == 4, generated.stats["reused_maps"]  # cos and sin of layers 1 and 2
    plan = [line.split()[1] for line in generated.files["model.plan"].splitlines() if line.startswith("launch ")]
    assert len(plan) == generated.stats["launches"]


OPERATIONS_SOURCE = """
def fn(x, y, ids):
    selected = x[ids]
    values, indices = selected.topk(2, dim=0, largest=False, sorted=False)
    return (selected.sum(0), selected.mean(1, keepdim=True), selected.softmax(0), values, indices,
            torch.cat((selected, y), dim=0), torch.triu(selected, 1), torch.tril(selected, -1),
            torch.einsum("ij,kj->ik", selected, y))
"""


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_every_operation_family_cross_compiles_for_gfx950(tmp_path, dtype):
    namespace = {"torch": torch}
    exec(OPERATIONS_SOURCE, namespace)
    generated = lower(Function(namespace["fn"]), torch.randn(6, 4, dtype=dtype), torch.randn(2, 4, dtype=dtype), torch.tensor([4, -1, 0]))
    assert generated.outputs[3]["dtype"] == str(dtype).removeprefix("torch.")
    assert generated.outputs[4]["dtype"] == "int64"
    build(generated, tmp_path / "ops", load=False)
    norm = lower(RMSNorm(65).to(dtype).eval(), torch.randn(4, 65, dtype=dtype))
    build(norm, tmp_path / "norm", load=False)
    model = random_transformer(small_config(), seed=5, std=0.1, dtype=dtype)
    build(lower(model, torch.tensor([1, 4, 2, 7])), tmp_path / "model", load=False)
    from chroma_amd.models.cached import export_cached

    for steps in (1, 5):
        cached = lower_program(export_cached(model, 5, steps), HIPCodegen())
        assert [o["dtype"] for o in cached.outputs] == [str(dtype).removeprefix("torch.")] * 3
        build(cached, tmp_path / f"cached{steps}", load=False)


def test_build_publishes_and_replaces_artifacts(tmp_path):
    x = torch.arange(4, dtype=torch.float32)
    build(lower(torch.nn.Linear(4, 4).eval(), x), tmp_path, load=False)
    build(lower(torch.nn.Linear(4, 2).eval(), x), tmp_path, load=False)
    assert len(list(tmp_path.glob("_chroma_*.hsaco"))) == 1
    assert len(list(tmp_path.glob("weights-*.bin"))) == 1
    manifest = json.loads((tmp_path / "model.json").read_text())
    assert manifest["version"] == 2 and manifest["stats"]["backend"] == "hip"
    plan = (tmp_path / "model.plan").read_text().splitlines()
    assert plan[0] == "chroma-hip-plan 2" and any(line.startswith("signature ") for line in plan)
    assert (tmp_path / manifest["library"]).stat().st_size > 0


def test_backend_dispatch_and_unsupported_dtypes():
    exported = torch.export.export(torch.nn.Identity(), (torch.ones(4),))
    with pytest.raises(ValueError, match="Unknown runtime backend"):
        compile_for_backend(exported, "unused", backend="cuda")
    with pytest.raises(ValueError, match="Unsupported dtype torch.float16"):
        lower(torch.nn.Identity(), torch.ones(4, dtype=torch.float16))


def test_c_abi_library_exports_every_declared_entry_point():
    header = (ROOT / "include" / "chroma_hip.h").read_text()
    declared = sorted(set(re.findall(r"\b(chroma_hip_\w+)\s*\(", header)))
    assert declared == sorted(native.EXPORTED)
    if not native.LIBRARY.exists():
        native.build_runtime()
    library = ctypes.CDLL(str(native.LIBRARY))
    for name in declared:
        assert hasattr(library, name), name


def test_program_load_fails_loudly_without_a_built_library(tmp_path, monkeypatch):
    from chroma_amd._src import native as module

    monkeypatch.setattr(module, "LIBRARY", tmp_path / "missing.so")
    monkeypatch.setattr(module, "_library", None)
    with pytest.raises(RuntimeError, match="not built"):
        module.library()


def test_dev_model_arena_lifetimes_cover_every_launch():
    """Every arena allocation is live (and so not shared) at every launch that reads or writes it, also
    when a fused launch replaces an earlier one (the router takes the gate linear's place)."""
    from chroma_amd.models.dev import make_dev_model

    compiler = Compiler.from_export(export(make_dev_model(0), torch.arange(8, dtype=torch.int64)), HIPCodegen())
    generated = compiler.lower()
    codegen = compiler.codegen
    assert generated.stats["fused_routers"] == 12
    allocations = codegen.allocations
    for index, launch in enumerate(codegen.launches):
        for binding in launch.bindings:
            if binding.kind == "arena" and binding.index in allocations:
                allocation = allocations[binding.index]
                assert allocation.start <= index <= allocation.end, (launch.kernel, binding.index)
    live = list(allocations.values())
    for i, a in enumerate(live):
        for b in live[i + 1 :]:
            if a.start <= b.end and b.start <= a.end:
                assert a.offset + a.size <= b.offset or b.offset + b.size <= a.offset


def _function_text(source: str, marker: str) -> str:
    """The text of the device function that contains ``marker`` (from its signature to its closing brace)."""
    at = source.index(marker)
    start = source.rindex("__device__ __forceinline__ void", 0, at)
    end = source.index("\n}\n", at)
    return source[start:end]


def test_in_kernel_handoffs_use_device_scope_accesses():
    """The two kernels that pass data between workgroups inside one launch (the split router's logits and
    the decode attention's phase-2 partial sums, each handed over behind a ticket) touch that data only
    through ``store_device`` / ``load_device`` (device-scope atomics, which the compiler keeps as such and
    the hardware writes through / reads past the XCD's L2), and each returns its ticket word to zero."""
    include = ROOT / "chroma_amd" / "csrc" / "include" / "chroma_hip"
    router = _function_text((include / "linear.h").read_text(), "void router_split(")
    uses = [line.strip() for line in router.splitlines() if "row_logits" in line and "T* row_logits =" not in line]
    assert uses and all("store_device(row_logits" in line or "load_device(row_logits" in line for line in uses), uses
    assert "atomicExch(counter + row, 0u)" in router and "device_stores_complete();" in router
    decode = _function_text((include / "attention.h").read_text(), "auto finish = [&]()")
    uses = [line.strip() for line in decode.splitlines() if "partial" in line and not line.strip().startswith("//")
            and "float* partial = split.partial" not in line]
    assert uses and all("store_device(" in line or "load_device(" in line for line in uses), uses
    assert "atomicExch(ticket_word, 0u)" in decode and "device_stores_complete();" in decode
