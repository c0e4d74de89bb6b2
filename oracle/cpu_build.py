"""ORACLE - test infrastructure only. Compiles and runs the CPU restatement's generated programs.

Compilation follows the reference CPU build (chroma/_src/build.py:19-30): ``-std=c++20 -O3 -shared
-fPIC -fvisibility=hidden -ffp-contract=off``, single-threaded. In BLAS mode the program links NumPy's
bundled OpenBLAS and the runner pins it to one thread, matching the reference's 1-thread CPU numbers
(docs/benchmarks.md:12). ``include_root`` selects the kernel headers: the oracle's own (default) or the
reference's (oracle/ref builds, written only under oracle/_ref).
"""

from __future__ import annotations

import ctypes
import glob
import hashlib
import os
import shlex
import subprocess
from pathlib import Path
from typing import List, Optional, Sequence

import numpy as np

from chroma_amd._src.codegen.base import GeneratedCode
from chroma_amd._src.dtypes import numpy_dtype

ORACLE_ROOT = Path(__file__).resolve().parent
OWN_HEADERS = ORACLE_ROOT / "include"
FLAGS = ["-std=c++20", "-O3", "-shared", "-fPIC", "-fvisibility=hidden", "-ffp-contract=off"]


def openblas_library() -> str:
    import numpy

    pattern = os.path.join(os.path.dirname(os.path.dirname(numpy.__file__)), "numpy.libs", "libscipy_openblas64_*.so")
    matches = sorted(glob.glob(pattern))
    if not matches:
        raise RuntimeError("NumPy's bundled OpenBLAS was not found; compile the oracle with blas=False")
    return matches[0]


def compile_library(source: Path, library: Path, flags: Sequence[str], include_root: Path) -> None:
    command = [*shlex.split(os.environ.get("CXX", "g++")), *FLAGS, "-I", str(include_root), str(source), "-o", str(library)]
    if "-DCHROMA_CBLAS" in flags:
        blas = openblas_library()
        command += ["-DCHROMA_CBLAS", blas, f"-Wl,-rpath,{os.path.dirname(blas)}"]
    result = subprocess.run(command, capture_output=True, text=True, check=False)
    if result.returncode:
        raise RuntimeError(f"Oracle compilation failed:\n{result.stderr[-4000:]}")


class OracleProgram:
    """Runs one compiled oracle program on NumPy arrays (inputs and outputs follow the manifest specs)."""

    device = "CPU"

    def __init__(self, library: Path, weights: Path, inputs: List[dict], outputs: List[dict], stats: dict) -> None:
        self.inputs, self.outputs, self.stats = inputs, outputs, stats
        self._lib = ctypes.CDLL(str(library))
        self._lib.oracle_create.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p, ctypes.c_size_t]
        self._lib.oracle_run.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
        self._lib.oracle_destroy.argtypes = [ctypes.c_void_p]
        if stats.get("math_library") == "cblas":
            blas = ctypes.CDLL(openblas_library())
            blas.scipy_openblas_set_num_threads64_.argtypes = [ctypes.c_int]
            blas.scipy_openblas_set_num_threads64_(1)
        handle = ctypes.c_void_p()
        error = ctypes.create_string_buffer(512)
        status = self._lib.oracle_create(str(weights).encode(), ctypes.byref(handle), error, len(error))
        if status:
            raise RuntimeError(error.value.decode())
        self._handle = handle

    def __call__(self, *inputs, out: Optional[Sequence[np.ndarray]] = None):
        arrays = []
        for value, spec in zip(inputs, self.inputs):
            if not isinstance(value, np.ndarray):
                value = _numpy(value)
            array = np.require(value, requirements=["C", "A"])
            if array.dtype != numpy_dtype(spec["dtype"]) or list(array.shape) != spec["shape"]:
                raise ValueError("shape or dtype")
            arrays.append(array)
        if len(arrays) != len(self.inputs):
            raise ValueError("wrong number of arrays")
        results = list(out) if out is not None else [np.empty(s["shape"], dtype=numpy_dtype(s["dtype"])) for s in self.outputs]
        in_ptrs = (ctypes.c_void_p * max(1, len(arrays)))(*[a.ctypes.data for a in arrays])
        out_ptrs = (ctypes.c_void_p * max(1, len(results)))(*[r.ctypes.data for r in results])
        error = ctypes.create_string_buffer(512)
        status = self._lib.oracle_run(self._handle, in_ptrs, out_ptrs, error, len(error))
        if status == 1:
            raise IndexError(error.value.decode())
        if status:
            raise RuntimeError(error.value.decode())
        return results[0] if len(results) == 1 else tuple(results)

    def close(self) -> None:
        if self._handle is not None:
            self._lib.oracle_destroy(self._handle)
            self._handle = None

    def __enter__(self) -> "OracleProgram":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def _numpy(value) -> np.ndarray:
    import torch

    from chroma_amd._src.dtypes import BFLOAT16

    tensor = value.detach().contiguous()
    if tensor.dtype == torch.bfloat16:
        return tensor.view(torch.uint16).numpy().view(BFLOAT16)
    return tensor.numpy()


def build_cpu(generated: GeneratedCode, output: os.PathLike, include_root: Path = OWN_HEADERS) -> OracleProgram:
    directory = Path(output)
    directory.mkdir(parents=True, exist_ok=True)
    source = directory / generated.source_name
    source.write_text(generated.files[generated.source_name])
    digest = hashlib.sha256(source.read_bytes() + str(include_root).encode() + " ".join(generated.flags).encode()).hexdigest()[:16]
    library = directory / f"oracle-{digest}.so"
    if not library.exists():
        compile_library(source, library, generated.flags, include_root)
    weights = directory / "weights.bin"
    generated.weights.write_to(weights)
    return OracleProgram(library, weights, generated.inputs, generated.outputs, generated.stats)
