"""Shared test helpers: wrap functions for torch.export, build small seeded transformers, compare arrays."""

from __future__ import annotations

import dataclasses
from typing import Any, Callable

import numpy as np
import torch

from chroma_amd._src.dtypes import BFLOAT16, bf16_to_float32
from chroma_amd.models.gpt_oss import ModelConfig, Transformer
from chroma_amd.models.variants import dev


class Function(torch.nn.Module):
    """Wraps a plain function so torch.export can trace it."""

    def __init__(self, fn: Callable[..., Any]) -> None:
        super().__init__()
        self.fn = fn

    def forward(self, *args: Any) -> Any:
        return self.fn(*args)


def export(module: torch.nn.Module, *inputs: torch.Tensor) -> torch.export.ExportedProgram:
    with torch.no_grad():
        return torch.export.export(module.eval(), inputs)


def random_transformer(config: ModelConfig, *, seed: int, std: float, dtype: torch.dtype = torch.float32) -> Transformer:
    """Unit norm scales and N(0, std) elsewhere, drawn in fp32 without disturbing the global RNG."""
    with torch.random.fork_rng(devices=[]), torch.no_grad():
        torch.manual_seed(seed)
        model = Transformer(config, device=torch.device("cpu")).float().eval().requires_grad_(False)
        for name, parameter in model.named_parameters():
            if name.endswith(".scale"):
                parameter.fill_(1)
            else:
                parameter.normal_(std=std)
    return model.to(dtype)


def small_config(**changes: Any) -> ModelConfig:
    base = dict(
        num_hidden_layers=1,
        num_experts=2,
        experts_per_token=2,
        vocab_size=17,
        hidden_size=8,
        intermediate_size=8,
        head_dim=4,
        num_attention_heads=2,
        num_key_value_heads=1,
        sliding_window=3,
    )
    base.update(changes)
    return dataclasses.replace(dev, **base)


def numpy_of(value: Any) -> np.ndarray:
    if isinstance(value, np.ndarray):
        return value
    tensor = value.detach().contiguous()
    if tensor.dtype == torch.bfloat16:
        return tensor.view(torch.uint16).numpy().view(BFLOAT16)
    return tensor.numpy()


def as_float(array: np.ndarray) -> np.ndarray:
    if array.dtype == BFLOAT16:
        return bf16_to_float32(array)
    return np.asarray(array)


def assert_close(actual: Any, expected: Any, *, rtol: float = 2e-5, atol: float = 2e-6) -> None:
    """Compare one array (NumPy result) with an expected tensor/array: int64 exactly, floats within tolerance."""
    expected = numpy_of(expected)
    actual = np.asarray(actual) if not isinstance(actual, np.ndarray) else actual
    assert actual.dtype == expected.dtype, (actual.dtype, expected.dtype)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    if expected.dtype == np.int64:
        np.testing.assert_array_equal(actual, expected)
    else:
        np.testing.assert_allclose(as_float(actual), as_float(expected), rtol=rtol, atol=atol, equal_nan=True)


def leaves(value: Any) -> list:
    if isinstance(value, (tuple, list)):
        out = []
        for item in value:
            out.extend(leaves(item))
        return out
    if hasattr(value, "values") and hasattr(value, "indices") and not isinstance(value, (np.ndarray, torch.Tensor)):
        return [value.values, value.indices]
    return [value]


def gathered_routing(runs) -> tuple:
    """(expert ids [layers, positions, k], gate logits [layers, positions, experts] as float32) over the
    runs of ``Decoder.extras`` (first position, tokens, [gate logits, expert ids]) of routing probes, in
    position order."""
    runs = sorted(runs, key=lambda run: run[0])
    ids = np.concatenate([arrays[1][:, :count] for _, count, arrays in runs], axis=1)
    logits = np.concatenate([as_float(arrays[0][:, :count]) for _, count, arrays in runs], axis=1)
    return ids, logits


class ExpertMLP(torch.nn.Module):
    """The workload's mixture-of-experts MLP (gpt_oss.py MLPBlock) at a chosen size, bfloat16, weights
    N(0, ``std``) from ``seed``; with ``product`` the first expert product is returned as well."""

    def __init__(self, hidden: int = 64, intermediate: int = 192, experts: int = 8, selected: int = 4, *, seed: int = 0,
                 std: float = 0.1, product: bool = False) -> None:
        super().__init__()
        import dataclasses

        from chroma_amd.models.gpt_oss import MLPBlock
        from chroma_amd.models.variants import gpt_oss_20b

        config = dataclasses.replace(gpt_oss_20b, hidden_size=hidden, intermediate_size=intermediate, num_experts=experts,
                                     experts_per_token=selected)
        with torch.device("meta"):
            self.block = MLPBlock(config)
        self.block = self.block.to_empty(device="cpu")
        generator = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            for name, parameter in self.block.named_parameters():
                if name.endswith("scale"):
                    parameter.fill_(1.0)
                else:
                    parameter.copy_(torch.randn(parameter.shape, generator=generator) * std)
        self.product = product

    def forward(self, x):
        if not self.product:
            return self.block(x)
        from chroma_amd.models.gpt_oss import swiglu

        b = self.block
        t = b.norm(x)
        experts = torch.topk(b.gate(t), k=b.experts_per_token, dim=-1, sorted=True)
        weights = torch.nn.functional.softmax(experts.values, dim=1)
        up = torch.einsum("beck,bk->bec", b.mlp1_weight[experts.indices, ...], t)
        t = swiglu(up + b.mlp1_bias[experts.indices, ...], limit=b.swiglu_limit)
        t = torch.einsum("beck,bek->bec", b.mlp2_weight[experts.indices, ...], t) + b.mlp2_bias[experts.indices, ...]
        return x + torch.einsum("bec,be->bc", t, weights), up


class NormThenLinear(torch.nn.Module):
    """The workloads' RMSNorm (float32 chain, cast back to bfloat16) feeding a linear; with ``both`` the
    float32 normalised rows are returned as well."""

    def __init__(self, width: int = 256, columns: int = 384, *, both: bool = False, seed: int = 0) -> None:
        super().__init__()
        generator = torch.Generator().manual_seed(seed)
        self.scale = torch.nn.Parameter(torch.rand(width, generator=generator) + 0.5)
        self.weight = torch.nn.Parameter((torch.randn(columns, width, generator=generator) * 0.05).to(torch.bfloat16))
        self.both = both

    def forward(self, x):
        h = x.float()
        y = h * torch.rsqrt(torch.mean(h**2, dim=-1, keepdim=True) + 1e-5) * self.scale
        out = torch.nn.functional.linear(y.to(torch.bfloat16), self.weight)
        return (out, y) if self.both else out
