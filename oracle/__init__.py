"""ORACLE - test infrastructure only.

CPU restatement of Chroma's CPU backend, used as the parity oracle for the ``hip`` backend and as the
CPU baseline in ``bench.py``. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it; the ``chroma_amd`` package never does.

How each part is pinned: the kernel headers by compiling the same generated program against the
reference's own headers (oracle/ref, bit-identical results); the front end by the reference's published
graph statistics; the numerics against eager torch at the reference's tolerances, its bf16 known answers
and float64 closed forms; the routing checker (routing.py) against hand-built decisions with planted
mistakes. The tests under tests/ hold each check.
"""

from __future__ import annotations

import os

from oracle.cpu_build import OWN_HEADERS, OracleProgram, build_cpu
from oracle.cpu_codegen import CPUCodegen


def compile_cpu(program, output: "os.PathLike[str]", *, blas: bool = True, include_root=OWN_HEADERS) -> OracleProgram:
    """Import, lower and build ``program`` with the CPU restatement; returns a loaded program."""
    from chroma_amd._src.compiler import lower_program

    return build_cpu(lower_program(program, CPUCodegen(blas=blas)), output, include_root)


__all__ = ["CPUCodegen", "OracleProgram", "compile_cpu"]
