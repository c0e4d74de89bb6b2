"""The oracle's restated kernel headers against the reference's own headers, bit for bit.

The same generated program (oracle CPU codegen, portable mode) is compiled twice: against
oracle/include and against /root/reference/chroma/_src (prebuilt into oracle/_ref by
``oracle.ref.build_reference_fixtures``). Identical source, flags and libm mean any difference is a
difference between the two header sets - a dropped term, a reordered sum, a wrong rounding or tie rule.
"""

import numpy as np
import pytest
import torch

from chroma_amd._src.compiler import lower_program
from oracle.cpu_build import build_cpu
from oracle.cpu_codegen import CPUCodegen
from oracle.ref import GRAPHS, build_reference_fixtures, graph, load_reference
from tests.helpers import leaves, numpy_of


@pytest.fixture(scope="module")
def reference_built():
    built = build_reference_fixtures()
    if not built and load_reference("bandwidth") is None:
        pytest.skip("reference headers unavailable and no prebuilt oracle/_ref")
    return True


def inputs_for(name, inputs, variant):
    """The example inputs, and a second seeded set that changes routing and values."""
    if variant == 0:
        return inputs
    generator = torch.Generator().manual_seed(100 + variant)
    changed = []
    for value in inputs:
        if value.dtype == torch.int64:
            high = {"routing": 6, "transformer": 17, "transformer_bf16": 17}.get(name, 2)
            changed.append(torch.randint(-high if name == "routing" else 0, high, value.shape, generator=generator))
        else:
            changed.append((torch.randn(value.shape, generator=generator) * 2).to(value.dtype))
    return tuple(changed)


@pytest.mark.parametrize("name", sorted(GRAPHS()))
def test_own_headers_match_reference_headers_bit_for_bit(name, tmp_path, reference_built):
    module, inputs = graph(name)
    reference = load_reference(name)
    assert reference is not None
    own = build_cpu(lower_program(torch.export.export(module, inputs), CPUCodegen(blas=False)), tmp_path / "own")
    for variant in range(3):
        values = [numpy_of(v) for v in inputs_for(name, inputs, variant)]
        got, want = own(*values), reference(*values)
        for a, b in zip(leaves(got), leaves(want)):
            np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("name", ["mlp_block", "transformer", "contractions"])
def test_blas_mode_matches_portable_mode(name, tmp_path, reference_built):
    module, inputs = graph(name)
    exported = torch.export.export(module, inputs)
    portable = build_cpu(lower_program(exported, CPUCodegen(blas=False)), tmp_path / "portable")
    blas = build_cpu(lower_program(exported, CPUCodegen(blas=True)), tmp_path / "blas")
    assert blas.stats["math_library"] == "cblas" and portable.stats["math_library"] == "portable"
    values = [numpy_of(v) for v in inputs]
    for a, b in zip(leaves(blas(*values)), leaves(portable(*values))):
        np.testing.assert_allclose(a, b, rtol=2e-5, atol=2e-6)
