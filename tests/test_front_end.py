"""Front end (import, folding, lowering, planning) pinned against the reference's published compile
statistics and its rejection rules.

The reference's CPU backend reports, for the dev model (docs/benchmarks/benchmark.json:66-74) and its
cached prefill/decode graphs (docs/benchmarks/decode-benchmark.json:58-82), the number of kernels, fused
expressions, folded constants, matrix and expert contractions, the planned and unreused arena sizes and
the weight/output bytes. The same graphs lowered here through the oracle's CPU codegen must give the same
numbers: a missed fusion, a different materialisation rule, a changed fold limit or planner would move
at least one of them.
"""

import pytest
import torch

from chroma_amd._src.compiler import Compiler, lower_program
from chroma_amd._src.graph import prepare
from chroma_amd.models.cached import export_cached
from chroma_amd.models.dev import DEV_PARAMETERS, make_dev_model
from oracle.cpu_codegen import CPUCodegen
from tests.helpers import Function, export

PUBLISHED = {
    "forward": {"kernels": 289, "expressions": 505, "folded_constants": 36, "matrix_contractions": 24, "workspace_bytes": 75776,
                "unreused_workspace_bytes": 1989120, "weight_bytes": 236089856, "output_bytes": 6434816, "expert_contractions": 24},
    "prefill": {"kernels": 352, "expressions": 554, "folded_constants": 12, "matrix_contractions": 24, "workspace_bytes": 17129472,
                "unreused_workspace_bytes": 213369344, "weight_bytes": 236089152, "output_bytes": 1197568, "expert_contractions": 24},
    "decode": {"kernels": 316, "expressions": 482, "folded_constants": 12, "matrix_contractions": 24, "workspace_bytes": 59328,
               "unreused_workspace_bytes": 927488, "weight_bytes": 236089152, "output_bytes": 805888, "expert_contractions": 24},
}


@pytest.fixture(scope="module")
def dev_model():
    return make_dev_model(0)


def test_dev_model_shape(dev_model):
    assert sum(p.numel() for p in dev_model.parameters()) == DEV_PARAMETERS


@pytest.mark.parametrize("graph", ["forward", "prefill", "decode"])
def test_published_compile_statistics(dev_model, graph):
    if graph == "forward":
        exported = export(dev_model, torch.arange(8, dtype=torch.int64))
    else:
        exported = export_cached(dev_model, 256, 256 if graph == "prefill" else 1)
    stats = lower_program(exported, CPUCodegen(blas=True)).stats
    for key, value in PUBLISHED[graph].items():
        assert stats[key] == value, (key, stats[key], value)


def test_rejections_at_import():
    with pytest.raises(NotImplementedError, match="unsupported operator"):
        prepare(export(Function(lambda x: torch.linalg.det(x)), torch.eye(3)))
    with pytest.raises(ValueError, match="Unsupported dtype torch.float16"):
        prepare(export(torch.nn.Identity(), torch.ones(4, dtype=torch.float16)))
    with pytest.raises(ValueError, match="dtype"):
        prepare(export(torch.nn.Linear(2, 2).double(), torch.ones(2, dtype=torch.float64)))
    with pytest.raises(TypeError, match="Only tensor inputs"):
        prepare(torch.export.export(Function(lambda x, scale: x * scale), (torch.ones(4), 2)))

    class Mutation(torch.nn.Module):
        def forward(self, x):
            return x.add_(1)

    class BufferMutation(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.register_buffer("count", torch.zeros(2))

        def forward(self, x):
            self.count.add_(1)
            return x + self.count

    for module in (Mutation(), BufferMutation()):
        with pytest.raises(ValueError, match="mutation"):
            prepare(export(module, torch.ones(2)))
    with pytest.raises(TypeError, match="Only tensor outputs"):
        prepare(export(Function(lambda x: (x, 3)), torch.ones(2)))
    dynamic = torch.export.export(
        Function(lambda x: x.sin()), (torch.ones(4),), dynamic_shapes=(({0: torch.export.Dim("length", min=1, max=16)},),)
    )
    with pytest.raises(ValueError, match="Dynamic"):
        prepare(dynamic)


def test_rmsnorm_chain_is_fused_and_nn_rmsnorm_is_not():
    from chroma_amd.models.gpt_oss import RMSNorm

    program = prepare(export(RMSNorm(16), torch.randn(3, 16)))
    targets = [str(n.target) for n in program.graph.nodes if n.op == "call_function"]
    assert any("_rmsnorm" in t for t in targets) and "aten.rsqrt.default" not in targets
    with pytest.raises(NotImplementedError, match="rms_norm"):
        prepare(export(torch.nn.RMSNorm(16), torch.randn(3, 16)))


def test_folded_state_is_stored_once_and_large_folds_are_bounded():
    class Constant(torch.nn.Module):
        def __init__(self, size):
            super().__init__()
            self.register_buffer("weight", torch.arange(size, dtype=torch.float32))

        def forward(self, x):
            return x + self.weight.sin()

    small = Constant(8)
    codegen = CPUCodegen()
    Compiler.from_export(export(small, torch.ones(8)), codegen).lower()
    assert len(codegen.weights) == 64
    import numpy as np

    np.testing.assert_array_equal(np.frombuffer(bytes(codegen.weights), dtype=np.float32)[:8], small.weight.sin().numpy())
    compiler = Compiler.from_export(export(Constant(262145), torch.ones(262145)), CPUCodegen())
    compiler.lower()
    assert compiler.folded == set()


def test_reshape_linear_does_not_allocate_an_input_copy():
    fn = Function(lambda x, w: torch.nn.functional.linear(x.reshape(-1, 17), w))
    stats = lower_program(export(fn, torch.randn(3, 5, 17), torch.randn(7, 17)), CPUCodegen()).stats
    assert stats["workspace_bytes"] == 0


@pytest.mark.parametrize(
    "eqn, a, b",
    [("mk,nk->mn", (35, 67), (33, 67)), ("qhd,khd->hqk", (35, 3, 17), (67, 3, 17)), ("hqk,khd->qhd", (3, 35, 67), (67, 3, 33)),
     ("bik,bkj->bij", (2, 35, 67), (1, 67, 33))],
)
def test_matrix_contractions_are_recognised(eqn, a, b):
    fn = Function(lambda x, y: torch.einsum(eqn, x, y))
    assert lower_program(export(fn, torch.randn(a), torch.randn(b)), CPUCodegen()).stats["matrix_contractions"] == 1
