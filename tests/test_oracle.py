"""The CPU oracle against eager torch and the reference's known answers.

These are the reference's own CPU-backend checks (tests/test_runtime.py, tests/test_bf16.py,
tests/test_backend_conformance.py, tests/runtime_core.cc) applied to the restatement: eager torch at the
reference's tolerances, exact bfloat16 answers, the bfloat16 rounding table and index errors.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from chroma_amd._src.dtypes import bf16_bits, bf16_to_float32, float32_to_bf16
from oracle import compile_cpu
from tests.helpers import Function, as_float, assert_close, export, leaves, numpy_of, random_transformer

TABLE = [
    (0x00000000, 0x0000), (0x80000000, 0x8000), (0x3F808000, 0x3F80), (0x3F818000, 0x3F82),
    (0xBF808000, 0xBF80), (0x00008000, 0x0000), (0x00010000, 0x0001), (0x7F800000, 0x7F80),
    (0xFF800000, 0xFF80), (0x7F800001, 0x7FC0), (0x7FFFFFFF, 0x7FC0), (0x7F7FFFFF, 0x7F80),
]


def run(tmp_path, module, *inputs, blas=False, name="p"):
    program = compile_cpu(export(module, *inputs), tmp_path / name, blas=blas)
    return program, program(*[numpy_of(v) for v in inputs])


def close(actual, expected, **tol):
    for got, want in zip(leaves(actual), leaves(expected)):
        assert_close(got, want, **(tol or dict(rtol=2e-5, atol=2e-6)))


def test_bfloat16_rounding_table_host_and_oracle(tmp_path):
    """The reference's 12-entry RNE table (tests/runtime_core.cc:26-35) through Python and the oracle."""
    words = np.array([w for w, _ in TABLE], dtype=np.uint32)
    expected = np.array([b for _, b in TABLE], dtype=np.uint16)
    floats = words.view(np.float32)
    np.testing.assert_array_equal([bf16_bits(float(f)) for f in floats], expected)
    np.testing.assert_array_equal(float32_to_bf16(floats).view(np.uint16), expected)
    _, out = run(tmp_path, Function(lambda y: y.bfloat16()), torch.from_numpy(floats.copy()))
    np.testing.assert_array_equal(out.view(np.uint16), expected)
    np.testing.assert_array_equal(bf16_to_float32(out).view(np.uint32), expected.astype(np.uint32) << 16)


def test_views_broadcast_reduction_and_aliases(tmp_path):
    def fn(x, y):
        z = x + y * 2
        r = z.transpose(0, 1).reshape(2, 6)
        s = r[:, 1::2]
        return (s.sin() * s).mean(dim=0), z, z, z.sum(dim=(0, 1), keepdim=True), y

    inputs = (torch.randn(3, 4), torch.randn(4))
    program, out = run(tmp_path, Function(fn), *inputs)
    close(out, Function(fn)(*inputs))
    assert not np.shares_memory(out[1], out[2])


def test_inplace_is_functionalized(tmp_path):
    def fn(x):
        z = x * 2
        alias = z[:, ::2]
        z.add_(3)
        return z, alias, x

    inputs = (torch.randn(3, 4),)
    _, out = run(tmp_path, Function(fn), *inputs)
    close(out, Function(fn)(*inputs))


def test_indexing_softmax_topk_nonfinite_and_index_errors(tmp_path):
    def fn(x, indices):
        selected = x[indices]
        values, positions = torch.topk(selected, 3, dim=0, largest=False)
        return values, positions, selected.softmax(dim=1), torch.triu(selected, diagonal=-1)

    inputs = (torch.randn(6, 4), torch.tensor([4, -1, 0, 2], dtype=torch.int64))
    program, out = run(tmp_path, Function(fn), *inputs)
    close(out, fn(*inputs))
    x = inputs[0].clone()
    x[0, 1] = float("nan")
    x[2, 2] = float("-inf")
    close(program(x.numpy(), inputs[1].numpy()), fn(x, inputs[1]))
    with pytest.raises(IndexError):
        program(inputs[0].numpy(), np.array([6, 0, 0, 0]))


def test_topk_ties_return_distinct_indices(tmp_path):
    for width in (12, 256):
        program, (values, indices) = run(tmp_path, Function(lambda x: torch.topk(x, 4)), torch.zeros(2, width), name=f"t{width}")
        np.testing.assert_array_equal(values, 0)
        assert all(len(set(row)) == 4 for row in indices)
        x = torch.rand(2, width)
        close(program(x.numpy()), torch.topk(x, 4))


def test_portable_linear_scalar_outputs_einsum_and_constant_graph(tmp_path):
    module = torch.nn.Linear(8, 3).eval()
    x = torch.randn(8)
    close(run(tmp_path, module, x, name="linear")[1], module(x))
    close(run(tmp_path, Function(lambda x: ((x + 1).mean(), x * 2)), torch.tensor(3.0), name="scalar")[1], ((torch.tensor(3.0) + 1).mean(), torch.tensor(6.0)))
    a, b = torch.randn(2, 3, 4), torch.randn(1, 4, 5)
    close(run(tmp_path, Function(lambda a, b: torch.einsum("bij,bjk->bik", a, b)), a, b, name="einsum")[1], torch.einsum("bij,bjk->bik", a, b), rtol=2e-4, atol=2e-5)
    close(run(tmp_path, Function(lambda: torch.arange(7).to(torch.float32).cos()), name="constant")[1], torch.arange(7).to(torch.float32).cos())


def test_long_expression_chain_is_bounded(tmp_path):
    def fn(x):
        for _ in range(180):
            x = (x * 0.99 + 0.02).sin()
        return x

    x = torch.randn(4, 5)
    program, out = run(tmp_path, Function(fn), x)
    close(out, fn(x))
    assert program.stats["kernels"] < 25


def test_lengths_sliding_window_and_yarn(tmp_path):
    from chroma_amd.models.variants import dev

    for length in (1, 17):
        config = dataclasses.replace(dev, num_hidden_layers=2, hidden_size=16, head_dim=64, num_attention_heads=4, num_key_value_heads=2,
                                     vocab_size=257, sliding_window=3, initial_context_length=4096, rope_scaling_factor=32.0)
        model = random_transformer(config, seed=length, std=0.04)
        tokens = torch.arange(length, dtype=torch.int64)
        program, out = run(tmp_path, model, tokens, blas=True, name=f"yarn{length}")
        close(out, model(tokens), rtol=2e-5, atol=4e-6)
        tokens = (tokens * 19 + 23) % config.vocab_size
        close(program(tokens.numpy()), model(tokens), rtol=2e-5, atol=4e-6)


def test_bfloat16_operations_and_fused_rounding(tmp_path):
    def fn(x, y, full, ids, one):
        values, indices = x.topk(3, dim=-1)
        return (x + y, x - y, x * y, x / y, x.sin(), x.cos(), x.exp(), x.sigmoid(), x.abs(), -x, x.square(), x.clamp(-0.25, 0.5),
                x.pow(2), (x.square() + 1).rsqrt(), x.sum(dim=1), x.mean(dim=0), x.sum(dtype=torch.float32), x.softmax(dim=-1), values,
                indices, x[ids], torch.cat((x, y.unsqueeze(0)), dim=0), torch.triu(x), torch.tril(x, diagonal=-1), x + full,
                (one + 2**-8) + 2**-8, (one * 0.333984375) - 0.333, torch.add(one * -0.30078125, one * 3, alpha=0.1))

    inputs = (torch.linspace(-1, 1, 96).reshape(3, 32).bfloat16(), torch.linspace(0.5, 1.5, 32).bfloat16(),
              torch.linspace(-0.1, 0.1, 96).reshape(3, 32), torch.tensor([-1, 0], dtype=torch.int64), torch.ones(1, dtype=torch.bfloat16))
    expected = fn(*inputs)
    program, actual = run(tmp_path, Function(fn), *inputs)
    close(actual, expected, rtol=0.02, atol=0.01)
    mixed, rounded, cancelled, scaled = actual[-4:]
    np.testing.assert_array_equal(as_float(rounded), np.ones(1, dtype=np.float32))
    np.testing.assert_allclose(as_float(mixed), expected[-4].numpy(), rtol=2e-5, atol=2e-6)
    close((cancelled, scaled), expected[-2:], rtol=0, atol=0)
    with pytest.raises(IndexError):
        program(*[numpy_of(v) for v in inputs[:3]], np.array([-4, 0]), numpy_of(inputs[4]))


@pytest.mark.parametrize("blas", [False, True])
def test_bfloat16_linear_einsum_and_sum_known_answers(tmp_path, blas):
    def fn(x, weight, bias):
        return torch.nn.functional.linear(x, weight, bias), torch.einsum("mk,nk->mn", x, weight), weight.sum(dim=1)

    x = torch.ones(2, 17, dtype=torch.bfloat16)
    weight = torch.full((5, 17), 2**-8, dtype=torch.bfloat16)
    weight[:, 0] = 1
    bias = torch.full((5,), 2**-5, dtype=torch.bfloat16)
    _, actual = run(tmp_path, Function(fn), x, weight, bias, blas=blas)
    np.testing.assert_array_equal(as_float(actual[0]), np.full((2, 5), 1.09375))
    np.testing.assert_array_equal(as_float(actual[1]), np.full((2, 5), 1.0625))
    np.testing.assert_array_equal(as_float(actual[2]), np.full(5, 1.0625))


def test_explicit_bfloat16_reductions_and_scalar_axes(tmp_path):
    class DTypeSemantics(torch.nn.Module):
        def forward(self, x):
            return x.sum(-1, dtype=torch.bfloat16), x.mean(-1, dtype=torch.bfloat16), x.softmax(-1, dtype=torch.bfloat16)

    class ScalarAxes(torch.nn.Module):
        def forward(self, x):
            values, indices = x.topk(1)
            return x.sum(0), x.softmax(-1), values, indices

    x = torch.tensor([[1.003, 1.003, -2.0], [10.01, -10.0, 0.01], [256.5, 256.0, -1000.0]])
    _, out = run(tmp_path, DTypeSemantics(), x, name="dtype")
    for got, want in zip(out, DTypeSemantics()(x)):
        np.testing.assert_array_equal(got.view(np.uint16), want.view(torch.uint16).numpy())
    _, out = run(tmp_path, ScalarAxes(), torch.tensor(2.5), name="scalar")
    close(out, ScalarAxes()(torch.tensor(2.5)))


def test_expert_contraction_broadcasts(tmp_path):
    class ExpertBroadcast(torch.nn.Module):
        def forward(self, weights, narrow_weights, indices, batch_x, narrow_x, x, batch_expert_x, narrow_expert_x, expert_x):
            selected, narrow_selected = weights[indices], narrow_weights[indices]
            return (torch.einsum("beck,bk->bec", selected, batch_x), torch.einsum("beck,bk->bec", selected, narrow_x),
                    torch.einsum("beck,bk->bec", narrow_selected, x), torch.einsum("beck,bek->bec", selected, batch_expert_x),
                    torch.einsum("beck,bek->bec", selected, narrow_expert_x), torch.einsum("beck,bek->bec", narrow_selected, expert_x))

    weights = torch.arange(24, dtype=torch.float32).reshape(3, 2, 4)
    batch_x = torch.tensor([[1.0, 2.0, 3.0, 4.0]])
    narrow_x = torch.tensor([[2.0], [3.0]])
    x = torch.arange(8, dtype=torch.float32).reshape(2, 4) + 1
    inputs = (weights, weights[:, :, :1].clone(), torch.tensor([[0], [1]]), batch_x, narrow_x, x, batch_x.unsqueeze(1), narrow_x.unsqueeze(1), x.unsqueeze(1))
    _, out = run(tmp_path, ExpertBroadcast(), *inputs)
    close(out, ExpertBroadcast()(*inputs))


def test_dev_model_matches_eager(tmp_path):
    from chroma_amd.models.dev import make_dev_model

    model = make_dev_model(0)
    tokens = torch.arange(8, dtype=torch.int64)
    program, out = run(tmp_path, model, tokens, blas=True)
    with torch.no_grad():
        for values in (tokens, (tokens * 7919 + 17) % 201088, torch.zeros_like(tokens), tokens.flip(0)):
            close(program(values.numpy()), model(values))
    with pytest.raises(IndexError):
        program(np.full(8, 201088, dtype=np.int64))
    with pytest.raises(IndexError):
        program(np.full(8, -1, dtype=np.int64))


@pytest.mark.parametrize("name", ["tanh", "silu"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_extension_unaries_match_eager(tmp_path, name, dtype):
    """The two operators the oracle adds to the reference's table (``aten.tanh``: ``std::tanh``;
    ``aten.silu``: ``x * (1 / (1 + exp(-x)))``, the reference's sigmoid form times x) against eager torch:
    +-inf, NaN, signed zeros, |x| < 0.05 (where tanh is x to first order), |x| > 20 (saturation, and
    exp(-x) overflowing for silu), the float extremes and a normal sample. fp32 within 2 ulp; bfloat16,
    whose inputs and outputs both round, within one bfloat16 ulp."""
    special = [np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-8, -3e-4, 0.049, -0.0499, 0.051, 20.5, -20.5, 45.0, -88.0, -104.0,
               3.0e38, -3.0e38, 1e-38, 0.5, -1.0]
    x = torch.cat([torch.tensor(special), torch.randn(200, generator=torch.Generator().manual_seed(3)) * 6]).to(dtype)
    fn = getattr(torch, name) if name == "tanh" else torch.nn.functional.silu
    _, out = run(tmp_path, Function(fn), x)
    got = as_float(out)
    want = fn(x).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want)), name
    finite = np.isfinite(want)
    np.testing.assert_array_equal(got[~finite & ~np.isnan(want)], want[~finite & ~np.isnan(want)])
    rtol = 2.4e-7 if dtype == torch.float32 else 7.9e-3
    np.testing.assert_allclose(got[finite], want[finite], rtol=rtol, atol=1e-37)
    # sign of zero and of tiny results is kept
    np.testing.assert_array_equal(np.signbit(got[finite & (want == 0)]), np.signbit(want[finite & (want == 0)]))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_logsumexp_and_log_match_eager(tmp_path, dtype):
    """The oracle's ``logsumexp`` (an extension: torch's m + log(sum(exp(x - m))), m the maximum, 0 when
    infinite) and ``log`` against eager torch: ordinary rows, a row with NaN, a row with +inf, a row of
    -inf, a row with -inf among finite values, a constant row (exactly m + log(n)); the last axis, the
    first axis and a middle axis of a 3-d tensor; and the closed form on the constant row."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(9, 300, generator=g) * 4
    x[1, 17] = float("nan")
    x[2, 5] = float("inf")
    x[3] = -float("inf")
    x[4, ::3] = -float("inf")
    x[5] = 2.5
    x = x.to(dtype)
    cube = (torch.randn(3, 70, 5, generator=g) * 3).to(dtype)

    def fn(x, cube):
        return (torch.logsumexp(x, -1), torch.logsumexp(x, 0, keepdim=True), torch.logsumexp(cube, 1),
                torch.log(x.abs() + 0.5), torch.logsumexp(x * 0.5, dim=1, keepdim=True))

    _, out = run(tmp_path, Function(fn), x, cube)
    for got, want in zip(out, Function(fn)(x, cube)):
        got, want = as_float(got), want.float().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(want))
        finite = np.isfinite(want)
        np.testing.assert_array_equal(got[~finite & ~np.isnan(want)], want[~finite & ~np.isnan(want)])
        np.testing.assert_allclose(got[finite], want[finite], rtol=2e-6 if dtype == torch.float32 else 8e-3, atol=1e-6)
    lse = as_float(out[0])
    assert np.isnan(lse[1]) and lse[2] == np.inf and lse[3] == -np.inf
    # a constant row of 2.5: 2.5 + log(300) (float64), within the float sum's rounding
    assert abs(lse[5] - (2.5 + np.log(300.0))) <= (1e-6 if dtype == torch.float32 else 0.04)
    # brute force in float64 on an ordinary row
    row = x[0].double().numpy()
    assert abs(lse[0] - (row.max() + np.log(np.exp(row - row.max()).sum()))) <= 2e-6 * abs(lse[0]) + (0 if dtype == torch.float32 else 0.05)
