"""chroma_amd: an MI355X-native ``hip`` backend for Chroma's fixed-shape ``torch.export`` compiler.

Public API, mirroring ``chroma`` (reference chroma/__init__.py:14-26):

* ``compile(export, directory, *, blas=True, backend="hip") -> Program``
* ``Program(directory)`` - load a compiled artifact (NumPy only at run time)
* ``Decoder(prefill, decode, *, sliding_window=0)`` - KV-cached generation
* ``jit(fn, *, backend="hip", blas=True)``
"""

from __future__ import annotations

from chroma_amd._src.decoder import Decoder
from chroma_amd._src.jit import jit
from chroma_amd._src.program import Program


def compile(input, output, *, blas: bool = True, backend: str = "hip") -> Program:
    from chroma_amd._src.compiler import compile_for_backend

    return compile_for_backend(input, output, blas=blas, backend=backend)


__all__ = ["Decoder", "Program", "compile", "jit"]
