"""Load and call a compiled hip artifact: the runtime half of the public API.

``Program(directory)`` mirrors the reference loader (chroma/_src/program.py:73-153): it checks the
manifest version and interpreter ABI ("recompile" on mismatch), loads the native program, compares the
tensor signature ("metadata" on mismatch), and serializes calls with one lock. The array checks the
reference performs in its pybind11 layer (chroma/_src/core/bindings.h:17-75) happen here, before the
C ABI is called: argument count, dtype/shape ("shape or dtype"), C-contiguity/alignment/writability of
outputs, and overlap between any output and any other array ("output overlap"). ctypes releases the
GIL for the duration of the native call. Loading needs NumPy only (no torch, no pybind11).
"""

from __future__ import annotations

import ctypes
import json
import sysconfig
import threading
from pathlib import Path
from typing import Any, List, Optional, Sequence, Tuple, Union

import numpy as np

from chroma_amd._src import host, native
from chroma_amd._src.dtypes import BFLOAT16, numpy_dtype
from chroma_amd._src.spec import MANIFEST_VERSION, signature

Array = np.ndarray
KNOWN_INPUT_BYTES = 64 << 10  # input arrays up to this size are remembered once checked


def _checked(value: Any, spec: dict, output: bool) -> np.ndarray:
    _address(value, spec, output)
    return value


def _address(value: Any, spec: dict, output: bool) -> int:
    """The reference's array checks (bindings.h:17-65) for one array; returns its data address."""
    if not isinstance(value, np.ndarray):
        raise TypeError("not a numpy array")
    dtype = numpy_dtype(spec["dtype"])
    if value.dtype != dtype or list(value.shape) != list(spec["shape"]):
        raise ValueError("shape or dtype")
    address = value.ctypes.data
    if not value.flags.c_contiguous or address % dtype.alignment or (output and not value.flags.writeable):
        raise ValueError("want C-contiguous, aligned, writable outputs")
    return address


class NativeModel:
    """The object the reference exposes as the extension's ``Model``: ``.device`` and ``.run``."""

    def __init__(self, directory: Path, inputs: List[dict], outputs: List[dict]) -> None:
        self._lib = native.library()
        self._inputs, self._outputs = inputs, outputs
        handle = ctypes.c_void_p()
        error = ctypes.create_string_buffer(1024)
        native.check(self._lib.chroma_hip_create(str(directory).encode(), ctypes.byref(handle), error, len(error)), error)
        self._handle = handle
        self.device = self._lib.chroma_hip_device_name(handle).decode()
        self.signature = self._lib.chroma_hip_signature(handle).decode()
        # Small input arrays already checked, by object: index -> (array, address). An array's address
        # never changes while it lives, and the entry holds it, so its id cannot be reused; a caller that
        # passes the same arrays every step (the decoder) pays for the address lookup once. Shape and
        # dtype are still compared on every call.
        self._known: dict = {}
        self._specs = [(numpy_dtype(spec["dtype"]), tuple(spec["shape"])) for spec in inputs]

    def _pointers(self, inputs: List[Optional[np.ndarray]], outputs: List[Optional[np.ndarray]], resident: bool) -> Tuple[ctypes.Array, ctypes.Array]:
        """The host pointer arrays of a call, after the reference's array checks (bindings.h:17-65)."""
        if not isinstance(inputs, list) or not isinstance(outputs, list):
            raise TypeError("run takes two lists of arrays")
        if len(inputs) != len(self._inputs) or len(outputs) != len(self._outputs):
            raise ValueError("wrong number of arrays")
        regions: List[Tuple[int, int]] = []
        pointers: List[Optional[int]] = []
        for index, (value, spec) in enumerate(zip(inputs, self._inputs)):
            if value is None and resident:
                pointers.append(None)
                continue
            known = self._known.get(index)
            if known is not None and known[0] is value and value.dtype == self._specs[index][0] and value.shape == self._specs[index][1]:
                begin = known[1]
            else:
                begin = _address(value, spec, False)
                if value.nbytes <= KNOWN_INPUT_BYTES:
                    self._known[index] = (value, begin)
            pointers.append(begin)
            regions.append((begin, begin + value.nbytes))
        for value, spec in zip(outputs, self._outputs):
            if value is None and resident:
                pointers.append(None)
                continue
            begin = _address(value, spec, True)
            end = begin + value.nbytes
            if any(begin < last and first < end for first, last in regions):
                raise ValueError("output overlap")
            regions.append((begin, end))
            pointers.append(begin)
        count = len(inputs)
        return native.pointer_array(pointers[:count]), native.pointer_array(pointers[count:])

    def run(self, inputs: List[np.ndarray], outputs: List[np.ndarray], *, resident: bool = False) -> None:
        """The extension's ``Model.run``. With ``resident`` an input given as None keeps what its device
        staging region holds and an output given as None stays on the device."""
        ins, outs = self._pointers(inputs, outputs, resident)
        error = ctypes.create_string_buffer(1024)
        native.check(self._lib.chroma_hip_run(self._handle, ins, outs, error, len(error)), error)

    def run_top(self, inputs: List[Optional[np.ndarray]], outputs: List[Optional[np.ndarray]], index: int, k: int) -> Tuple[np.ndarray, np.ndarray]:
        """``run`` (resident: None keeps an input's device copy, and leaves an output on the device) that also
        selects the ``k`` largest values of each row of output ``index`` on the device, after the plan on
        the same stream and under the same synchronization; returns (values [rows, k], int64 ids [rows, k])
        in page-locked host arrays."""
        spec = self._outputs[index]
        dtype = numpy_dtype(spec["dtype"])
        if dtype not in (np.dtype(np.float32), BFLOAT16) or not spec["shape"]:
            raise TypeError("run_top selects over float32 or bfloat16 outputs of rank >= 1")
        width = int(spec["shape"][-1])
        rows = int(np.prod(spec["shape"][:-1])) if len(spec["shape"]) > 1 else 1
        ins, outs = self._pointers(inputs, outputs, True)
        values = host.empty((rows, k), dtype)
        ids = host.empty((rows, k), np.int64)
        code = native.FLOAT32 if dtype == np.dtype(np.float32) else native.BFLOAT16
        error = ctypes.create_string_buffer(1024)
        status = self._lib.chroma_hip_run_top(self._handle, ins, outs, index, code, rows, width, k, values.ctypes.data, ids.ctypes.data,
                                              error, len(error))
        native.check(status, error)
        return values, ids

    def input_pointer(self, index: int) -> int:
        return int(self._lib.chroma_hip_input_pointer(self._handle, index) or 0)

    def output_pointer(self, index: int) -> int:
        return int(self._lib.chroma_hip_output_pointer(self._handle, index) or 0)

    def copy_2d(self, dst: int, dst_pitch: int, src: int, src_pitch: int, width: int, height: int, *, queued: bool = False) -> None:
        """Device-to-device copy of ``height`` rows of ``width`` bytes on this program's stream; complete on
        return, or with ``queued`` only ordered before this program's later work (see ``synchronize``)."""
        error = ctypes.create_string_buffer(256)
        copy = self._lib.chroma_hip_copy_2d_queued if queued else self._lib.chroma_hip_copy_2d
        native.check(copy(self._handle, dst, dst_pitch, src, src_pitch, width, height, error, len(error)), error)

    def copy_2d_batch(self, rects: Sequence[Tuple[int, int, int, int, int, int]]) -> None:
        """Up to four queued device-to-device copies, each (dst, dst_pitch, src, src_pitch, width, height),
        in one kernel launch on this program's stream."""
        array = (native.Rect * len(rects))(*[native.Rect(*rect) for rect in rects])
        error = ctypes.create_string_buffer(256)
        native.check(self._lib.chroma_hip_copy_2d_batch_queued(self._handle, array, len(rects), error, len(error)), error)

    def clear_input(self, index: int) -> None:
        """Zero input ``index``'s device staging, queued on this program's stream (see ``synchronize``)."""
        error = ctypes.create_string_buffer(256)
        native.check(self._lib.chroma_hip_clear_input(self._handle, index, error, len(error)), error)

    def decoder_masks(self, slots: np.ndarray, position: int, steps: int, window: int, full_input: int, window_input: int) -> None:
        """Build a multi-step decoder call's two attention masks on the device, in the staging regions of
        inputs ``full_input`` (window = the cache's context) and ``window_input`` (``window``), queued on
        this program's stream ahead of the next resident run, which is then given None for them.
        ``slots`` [context] holds each cache row's time (negative when empty); query t sits at
        ``position + t``; the masks' dtype is the program's for those inputs."""
        table = np.ascontiguousarray(slots, dtype=np.int64)
        dtype = self._specs[full_input][0]
        code = native.FLOAT32 if dtype == np.dtype(np.float32) else native.BFLOAT16
        error = ctypes.create_string_buffer(512)
        status = self._lib.chroma_hip_decoder_masks(self._handle, table.ctypes.data, len(table), position, steps, window, code, full_input,
                                                    window_input, error, len(error))
        native.check(status, error)

    def synchronize(self) -> None:
        """Wait for everything queued on this program's stream."""
        error = ctypes.create_string_buffer(256)
        native.check(self._lib.chroma_hip_synchronize(self._handle, error, len(error)), error)

    # Device-resident helpers (benchmarks and tests): upload once, execute many times, download.
    def upload(self, inputs: Sequence[np.ndarray]) -> None:
        arrays = [_checked(np.require(a, requirements=["C", "A"]), s, False) for a, s in zip(inputs, self._inputs)]
        error = ctypes.create_string_buffer(1024)
        native.check(self._lib.chroma_hip_upload(self._handle, native.pointer_array(a.ctypes.data for a in arrays), error, len(error)), error)

    def execute(self, iterations: int = 1, timed: bool = False) -> Optional[float]:
        error = ctypes.create_string_buffer(1024)
        elapsed = ctypes.c_float(0.0)
        status = self._lib.chroma_hip_execute(self._handle, iterations, ctypes.byref(elapsed) if timed else None, error, len(error))
        native.check(status, error)
        return elapsed.value if timed else None

    def execute_chained(self, copies: int, iterations: int) -> float:
        """Milliseconds per execution of the plan, from ``iterations`` launches of one graph holding
        ``copies`` back-to-back executions (no per-replay host launch in the figure)."""
        error = ctypes.create_string_buffer(1024)
        elapsed = ctypes.c_float(0.0)
        native.check(self._lib.chroma_hip_execute_chained(self._handle, copies, iterations, ctypes.byref(elapsed), error, len(error)), error)
        return elapsed.value / (copies * iterations)

    def download(self, outputs: Sequence[np.ndarray]) -> None:
        for array, spec in zip(outputs, self._outputs):
            _checked(array, spec, True)
        error = ctypes.create_string_buffer(1024)
        native.check(self._lib.chroma_hip_download(self._handle, native.pointer_array(a.ctypes.data for a in outputs), error, len(error)), error)

    def set_graph(self, enabled: bool) -> bool:
        return bool(self._lib.chroma_hip_set_graph(self._handle, int(bool(enabled))))

    @property
    def launch_count(self) -> int:
        return int(self._lib.chroma_hip_launch_count(self._handle))

    def close(self) -> None:
        if self._handle is not None and self._handle.value:
            self._lib.chroma_hip_destroy(self._handle)
        self._handle = None

    def __del__(self) -> None:  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass


class Program:
    def __init__(self, directory: Union[str, Path]) -> None:
        manifest, model = self._load(directory)
        self._lock = threading.Lock()
        self._model: Optional[NativeModel] = model
        self._inputs = manifest["inputs"]
        self._outputs = manifest["outputs"]
        self._stats = manifest["stats"]
        self._device = model.device

    @staticmethod
    def _load(directory: Union[str, Path]):
        directory = Path(directory).resolve()
        manifest = json.loads((directory / "model.json").read_text())
        if manifest.get("version") != MANIFEST_VERSION or manifest.get("python_abi") != sysconfig.get_config_var("SOABI"):
            raise ValueError("Incompatible Chroma artifact; recompile it with this Python interpreter")
        if manifest.get("stats", {}).get("backend") != "hip":
            raise ValueError("Not a hip artifact; recompile it with backend='hip'")
        model = NativeModel(directory, manifest["inputs"], manifest["outputs"])
        if model.signature != signature(manifest["inputs"], manifest["outputs"]):
            model.close()
            raise ValueError("Artifact tensor metadata does not match its native library")
        return manifest, model

    @property
    def device(self) -> str:
        return self._device

    @property
    def inputs(self) -> List[dict]:
        return self._inputs

    @property
    def outputs(self) -> List[dict]:
        return self._outputs

    @property
    def stats(self) -> dict:
        return self._stats

    @staticmethod
    def _array(value: Any) -> Array:
        if isinstance(value, np.ndarray):
            array = value
        else:
            tensor = value.detach()
            if str(tensor.dtype) == "torch.bfloat16":
                import torch

                array = tensor.view(torch.uint16).numpy().view(BFLOAT16)
            else:
                array = tensor.numpy()
        return np.require(array, requirements=["C", "A"])

    def __call__(self, *inputs: Any, out: Union[Array, Sequence[Array], None] = None):
        arrays = [self._array(value) for value in inputs]
        if out is None:
            # page-locked, so the device writes them straight over the link
            results = [host.empty(spec["shape"], numpy_dtype(spec["dtype"])) for spec in self._outputs]
        else:
            results = [out] if isinstance(out, np.ndarray) else list(out)
        with self._lock:
            if self._model is None:
                raise RuntimeError("Model is closed")
            self._model.run(arrays, results)
        return results[0] if len(results) == 1 else tuple(results)

    def run_resident(self, inputs: Sequence[Optional[Array]], outputs: Sequence[Optional[Array]]) -> None:
        """A call that leaves chosen data on the device: an input given as None keeps what the program's
        device copy of it already holds (an earlier upload or device copy), an output given as None is
        not downloaded. The KV-cached ``Decoder`` keeps its cache on the device this way."""
        arrays = [None if value is None else self._array(value) for value in inputs]
        with self._lock:
            if self._model is None:
                raise RuntimeError("Model is closed")
            self._model.run(arrays, list(outputs), resident=True)

    def run_top_resident(self, inputs: Sequence[Optional[Array]], outputs: Sequence[Optional[Array]], index: int, k: int) -> Tuple[Array, Array]:
        """``run_resident`` that also returns the ``k`` largest values of each row of output ``index`` and
        their ids, selected on the device (``NativeModel.run_top``)."""
        arrays = [None if value is None else self._array(value) for value in inputs]
        with self._lock:
            if self._model is None:
                raise RuntimeError("Model is closed")
            return self._model.run_top(arrays, list(outputs), index, k)

    @property
    def native(self) -> NativeModel:
        if self._model is None:
            raise RuntimeError("Model is closed")
        return self._model

    def close(self) -> None:
        with self._lock:
            if self._model is not None:
                self._model.close()
            self._model = None

    def __enter__(self) -> "Program":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()
