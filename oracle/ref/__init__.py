"""ORACLE - test infrastructure only. Builds of the oracle's generated programs against the reference's
own kernel headers.

Recipe (run by ``__graft_entry__.build()`` when /root/reference is present): each graph in ``GRAPHS`` is
lowered with the oracle's CPU codegen in portable mode (no BLAS; the reference's CBLAS mode needs a
``cblas.h`` this image lacks, so it is not built) and the emitted program is compiled with
``-I /root/reference/chroma/_src`` - the reference's ``codegen/cpu/kernels.h``, ``expressions.h`` and
``core/*.h`` exactly where they lie - into ``oracle/_ref/<name>/``. Nothing from the reference is copied;
the outputs stay out of git (``.gitignore``) but travel with the tree. ``tests/test_oracle_pinning.py``
runs the same programs compiled against the oracle's restated headers and requires identical bits.
"""

from __future__ import annotations

import json
import shutil
import tempfile
from pathlib import Path
from typing import Callable, Dict, Tuple

REFERENCE_HEADERS = Path("/root/reference/chroma/_src")
OUTPUT = Path(__file__).resolve().parents[1] / "_ref"


def _graphs() -> Dict[str, Callable[[], Tuple[object, tuple]]]:
    import torch

    from tests.helpers import Function, random_transformer, small_config

    def seeded(seed: int, *shape: int, low: float = -4.0, high: float = 4.0) -> "torch.Tensor":
        generator = torch.Generator().manual_seed(seed)
        return torch.rand(*shape, generator=generator) * (high - low) + low

    def bandwidth():
        def fn(x, y):
            z = torch.tanh(x * 0.5 + y) * torch.sigmoid(y) - torch.exp(torch.clamp(x, -8, 8)) * 1e-3
            return torch.softmax(z, -1)

        return Function(fn), (seeded(1, 16, 512), seeded(2, 16, 512))

    def mlp_block():
        return mlp_module(128, 256, seed=0), (torch.randn(8, 128, generator=torch.Generator().manual_seed(0)),)

    def routing():
        def fn(x, indices):
            selected = x[indices]
            values, positions = torch.topk(selected, 3, dim=0, largest=False)
            return values, positions, selected.softmax(dim=1), torch.triu(selected, diagonal=-1), selected.sum(0), selected.mean(1, keepdim=True)

        return Function(fn), (seeded(3, 6, 4), torch.tensor([4, -1, 0, 2], dtype=torch.int64))

    def bf16_ops():
        def fn(x, y, one):
            values, indices = x.topk(3, dim=-1)
            return (x + y, x * y, x / y, x.sigmoid(), x.exp(), x.clamp(-0.25, 0.5), (x.square() + 1).rsqrt(), x.sum(dim=1),
                    x.softmax(dim=-1), values, indices, (one + 2**-8) + 2**-8, (one * 0.333984375) - 0.333,
                    torch.add(one * -0.30078125, one * 3, alpha=0.1))

        return Function(fn), (
            torch.linspace(-1, 1, 96).reshape(3, 32).bfloat16(),
            torch.linspace(0.5, 1.5, 32).bfloat16(),
            torch.ones(1, dtype=torch.bfloat16),
        )

    def contractions():
        def fn(a, b, c, d):
            return torch.einsum("bik,bkj->bij", a, b), torch.einsum("km,kn->mn", c, d), torch.einsum("ij,ik->ijk", c, d)

        return Function(fn), (seeded(4, 2, 3, 17), seeded(5, 1, 17, 5), seeded(6, 17, 3), seeded(7, 17, 5))

    def transformer():
        model = random_transformer(small_config(num_hidden_layers=2, hidden_size=16, intermediate_size=16, head_dim=8,
                                                num_attention_heads=4, num_key_value_heads=2, num_experts=4), seed=5, std=0.1)
        return model, (torch.tensor([1, 4, 2, 7, 0, 16], dtype=torch.int64),)

    def transformer_bf16():
        model = random_transformer(small_config(), seed=5, std=0.1, dtype=torch.bfloat16)
        return model, (torch.tensor([1, 4, 2, 7], dtype=torch.int64),)

    return {
        "bandwidth": bandwidth,
        "mlp_block": mlp_block,
        "routing": routing,
        "bf16_ops": bf16_ops,
        "contractions": contractions,
        "transformer": transformer,
        "transformer_bf16": transformer_bf16,
    }


GRAPHS = _graphs


def mlp_module(hidden: int, intermediate: int, seed: int):
    """BASELINE config C1's block (``chroma_amd.models.blocks.mlp_block``) at the given widths."""
    from chroma_amd.models.blocks import mlp_block

    return mlp_block(hidden, intermediate, seed)


def graph(name: str):
    """(module, example inputs) of a pinning graph."""
    return _graphs()[name]()


def build_reference_fixtures(force: bool = False) -> bool:
    """Compile every pinning graph against the reference's headers; False when they are absent."""
    if not REFERENCE_HEADERS.exists():
        return False
    import torch

    from chroma_amd._src.compiler import lower_program
    from oracle.cpu_build import compile_library
    from oracle.cpu_codegen import CPUCodegen

    OUTPUT.mkdir(parents=True, exist_ok=True)
    for name, make in _graphs().items():
        target = OUTPUT / name
        if (target / "spec.json").exists() and not force:
            continue
        module, inputs = make()
        generated = lower_program(torch.export.export(module, inputs), CPUCodegen(blas=False))
        with tempfile.TemporaryDirectory(prefix=f".{name}-", dir=OUTPUT) as stage:
            stage = Path(stage)
            (stage / "model.cc").write_text(generated.files["model.cc"])
            compile_library(stage / "model.cc", stage / "model.so", generated.flags, REFERENCE_HEADERS)
            generated.weights.write_to(stage / "weights.bin")
            (stage / "spec.json").write_text(json.dumps({"inputs": generated.inputs, "outputs": generated.outputs, "stats": generated.stats}))
            if target.exists():
                shutil.rmtree(target)
            shutil.move(str(stage), str(target))
    return True


def load_reference(name: str):
    """The reference-header build of ``name`` as an OracleProgram, or None when it was not built."""
    from oracle.cpu_build import OracleProgram

    target = OUTPUT / name
    if not (target / "spec.json").exists():
        return None
    spec = json.loads((target / "spec.json").read_text())
    return OracleProgram(target / "model.so", target / "weights.bin", spec["inputs"], spec["outputs"], spec["stats"])


def build_oracle_selftest() -> None:
    """Compile one pinning graph with the oracle's own headers (both BLAS modes) as a build check."""
    import torch

    from chroma_amd._src.compiler import lower_program
    from oracle.cpu_build import build_cpu
    from oracle.cpu_codegen import CPUCodegen

    module, inputs = graph("mlp_block")
    with tempfile.TemporaryDirectory(prefix="chroma-oracle-") as work:
        for blas in (False, True):
            build_cpu(lower_program(torch.export.export(module, inputs), CPUCodegen(blas=blas)), Path(work) / str(blas))
