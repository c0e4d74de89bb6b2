"""Compile a function or module once per input signature (reference chroma/_src/jit.py:38-80)."""

from __future__ import annotations

import threading
from functools import partial, wraps
from pathlib import Path
from tempfile import TemporaryDirectory
from typing import Any, Callable, Optional


def jit(fn: Optional[Callable[..., Any]] = None, *, backend: str = "hip", blas: bool = True):
    if fn is None:
        return partial(jit, backend=backend, blas=blas)
    if not callable(fn):
        raise TypeError(f"callable, got {type(fn).__name__}")
    import torch

    from chroma_amd._src.compiler import compile_for_backend

    class Function(torch.nn.Module):
        def __init__(self, function: Callable[..., Any]) -> None:
            super().__init__()
            self.function = function

        def forward(self, *args: Any) -> Any:
            return self.function(*args)

    module = fn if isinstance(fn, torch.nn.Module) else Function(fn)
    directory = TemporaryDirectory(prefix="chroma-jit-")
    programs = {}
    lock = threading.Lock()

    @wraps(fn)
    def run(*args: Any, out: Any = None) -> Any:
        if any(not isinstance(value, torch.Tensor) or value.device.type != "cpu" for value in args):
            raise TypeError("positional CPU Torch tensor")
        key = tuple((tuple(value.shape), value.dtype) for value in args)
        with lock:
            if key not in programs:
                with torch.no_grad():
                    examples = tuple(value.detach().contiguous() for value in args)
                    exported = torch.export.export(module, examples)
                programs[key] = compile_for_backend(exported, Path(directory.name) / str(len(programs)), backend=backend, blas=blas)
            program = programs[key]
        return program(*args, out=out)

    run._directory = directory  # keeps the artifacts alive as long as the function
    return run
