"""Locate, build and bind the hip runtime library (``libchroma_hip.so``, C ABI in include/chroma_hip.h).

The library is built in-tree (``chroma_amd/lib``) by ``build_runtime``; loading never builds, so a GPU
host runs exactly the library that was compiled and shipped with the tree. There is no fallback: if the
library is missing, loading a program fails with a message saying how to build it.
"""

from __future__ import annotations

import ctypes
import os
import shlex
import subprocess
import tempfile
import threading
from pathlib import Path

PACKAGE = Path(__file__).resolve().parents[1]
REPO = PACKAGE.parent
LIBRARY = PACKAGE / "lib" / "libchroma_hip.so"
RUNTIME_SOURCE = PACKAGE / "csrc" / "runtime.cpp"
SELECT_SOURCE = PACKAGE / "csrc" / "select.hip"
COPY_SOURCE = PACKAGE / "csrc" / "copy.hip"
MASKS_SOURCE = PACKAGE / "csrc" / "masks.hip"
DEVICE_INCLUDE = PACKAGE / "csrc" / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

OK, INDEX_ERROR, RUNTIME_ERROR = 0, 1, 2
FLOAT32, BFLOAT16 = 0, 1  # CHROMA_HIP_FLOAT32 / CHROMA_HIP_BFLOAT16

_lock = threading.Lock()
_library = None


def build_runtime(output: Path = LIBRARY) -> Path:
    """Build the runtime library: the host runtime (``runtime.cpp``, g++) and the row selection kernels
    (``select.hip``, hipcc for gfx950 with the same device flags as generated programs), linked by hipcc
    against the HIP runtime."""
    from chroma_amd._src.build import DEVICE_FLAGS, architecture

    output.parent.mkdir(parents=True, exist_ok=True)
    temporary = output.with_suffix(".so.tmp")
    hipcc = shlex.split(os.environ.get("HIPCC", str(ROCM / "bin" / "hipcc")))
    device_flags = [flag for flag in DEVICE_FLAGS if flag != "--genco"]
    with tempfile.TemporaryDirectory(prefix="chroma-runtime-") as work:
        host_object, device_object, copy_object = Path(work) / "runtime.o", Path(work) / "select.o", Path(work) / "copy.o"
        masks_object = Path(work) / "masks.o"
        commands = [
            [*shlex.split(os.environ.get("CXX", "g++")), "-std=c++17", "-O2", "-c", "-fPIC", "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__",
             f"-I{ROCM / 'include'}", str(RUNTIME_SOURCE), "-o", str(host_object)],
            [*hipcc, f"--offload-arch={architecture()}", *device_flags, "-c", "-fPIC", "-fvisibility=hidden", f"-I{DEVICE_INCLUDE}",
             str(SELECT_SOURCE), "-o", str(device_object)],
            [*hipcc, f"--offload-arch={architecture()}", *device_flags, "-c", "-fPIC", "-fvisibility=hidden", f"-I{DEVICE_INCLUDE}",
             str(COPY_SOURCE), "-o", str(copy_object)],
            [*hipcc, f"--offload-arch={architecture()}", *device_flags, "-c", "-fPIC", "-fvisibility=hidden", f"-I{DEVICE_INCLUDE}",
             str(MASKS_SOURCE), "-o", str(masks_object)],
            [*hipcc, f"--offload-arch={architecture()}", "-shared", "-fPIC", str(host_object), str(device_object), str(copy_object),
             str(masks_object), "-o", str(temporary),
             f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}", "-lamdhip64"],
        ]
        for command in commands:
            result = subprocess.run(command, capture_output=True, text=True, check=False)
            if result.returncode:
                raise RuntimeError(f"Building the hip runtime failed:\n{' '.join(command)}\n{result.stderr[-4000:]}")
    os.replace(temporary, output)
    return output


class Rect(ctypes.Structure):
    """``chroma_hip_rect``: one device-to-device rectangle copy."""

    _fields_ = [("dst", ctypes.c_void_p), ("dst_pitch", ctypes.c_size_t), ("src", ctypes.c_void_p), ("src_pitch", ctypes.c_size_t),
                ("width", ctypes.c_size_t), ("height", ctypes.c_size_t)]


def library() -> ctypes.CDLL:
    global _library
    with _lock:
        if _library is not None:
            return _library
        if not LIBRARY.exists():
            raise RuntimeError(
                f"The hip runtime library {LIBRARY} is not built; run __graft_entry__.build() "
                "(or chroma_amd._src.native.build_runtime()) first"
            )
        lib = ctypes.CDLL(str(LIBRARY))
        c = ctypes
        lib.chroma_hip_create.argtypes = [c.c_char_p, c.POINTER(c.c_void_p), c.c_char_p, c.c_size_t]
        lib.chroma_hip_run.argtypes = [c.c_void_p, c.c_void_p, c.c_void_p, c.c_char_p, c.c_size_t]
        lib.chroma_hip_device_name.argtypes = [c.c_void_p]
        lib.chroma_hip_device_name.restype = c.c_char_p
        lib.chroma_hip_signature.argtypes = [c.c_void_p]
        lib.chroma_hip_signature.restype = c.c_char_p
        lib.chroma_hip_destroy.argtypes = [c.c_void_p]
        lib.chroma_hip_destroy.restype = None
        lib.chroma_hip_upload.argtypes = [c.c_void_p, c.c_void_p, c.c_char_p, c.c_size_t]
        lib.chroma_hip_execute.argtypes = [c.c_void_p, c.c_int, c.POINTER(c.c_float), c.c_char_p, c.c_size_t]
        lib.chroma_hip_execute_chained.argtypes = [c.c_void_p, c.c_int, c.c_int, c.POINTER(c.c_float), c.c_char_p, c.c_size_t]
        lib.chroma_hip_download.argtypes = [c.c_void_p, c.c_void_p, c.c_char_p, c.c_size_t]
        lib.chroma_hip_set_graph.argtypes = [c.c_void_p, c.c_int]
        lib.chroma_hip_launch_count.argtypes = [c.c_void_p]
        lib.chroma_hip_device_base.argtypes = [c.c_void_p]
        lib.chroma_hip_device_base.restype = c.c_void_p
        for name in ("chroma_hip_input_pointer", "chroma_hip_output_pointer"):
            getattr(lib, name).argtypes = [c.c_void_p, c.c_int]
            getattr(lib, name).restype = c.c_void_p
        lib.chroma_hip_copy_2d.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p, c.c_size_t, c.c_size_t, c.c_size_t, c.c_char_p, c.c_size_t]
        lib.chroma_hip_copy_2d_queued.argtypes = lib.chroma_hip_copy_2d.argtypes
        lib.chroma_hip_copy_2d_batch_queued.argtypes = [c.c_void_p, c.POINTER(Rect), c.c_int, c.c_char_p, c.c_size_t]
        lib.chroma_hip_synchronize.argtypes = [c.c_void_p, c.c_char_p, c.c_size_t]
        lib.chroma_hip_clear_input.argtypes = [c.c_void_p, c.c_int, c.c_char_p, c.c_size_t]
        lib.chroma_hip_decoder_masks.argtypes = [c.c_void_p, c.c_void_p, c.c_int64, c.c_int64, c.c_int64, c.c_int64, c.c_int, c.c_int, c.c_int,
                                                 c.c_char_p, c.c_size_t]
        lib.chroma_hip_host_alloc.argtypes = [c.c_size_t, c.POINTER(c.c_void_p), c.c_char_p, c.c_size_t]
        lib.chroma_hip_host_free.argtypes = [c.c_void_p]
        lib.chroma_hip_host_free.restype = None
        lib.chroma_hip_rows_topk_workspace.argtypes = [c.c_size_t, c.c_size_t, c.c_int]
        lib.chroma_hip_rows_topk_workspace.restype = c.c_size_t
        lib.chroma_hip_rows_topk.argtypes = [c.c_void_p, c.c_int, c.c_size_t, c.c_size_t, c.c_int, c.c_int, c.c_void_p, c.c_void_p,
                                             c.c_void_p, c.c_size_t, c.c_void_p, c.c_char_p, c.c_size_t]
        lib.chroma_hip_rows_topk_static.argtypes = [c.c_void_p, c.c_int, c.c_size_t, c.c_size_t, c.c_int, c.c_int, c.c_void_p, c.c_void_p,
                                                    c.c_void_p, c.c_char_p, c.c_size_t]
        lib.chroma_hip_run_top.argtypes = [c.c_void_p, c.c_void_p, c.c_void_p, c.c_int, c.c_int, c.c_size_t, c.c_size_t, c.c_int,
                                           c.c_void_p, c.c_void_p, c.c_char_p, c.c_size_t]
        _library = lib
        return lib


EXPORTED = (
    "chroma_hip_create",
    "chroma_hip_run",
    "chroma_hip_device_name",
    "chroma_hip_signature",
    "chroma_hip_destroy",
    "chroma_hip_upload",
    "chroma_hip_execute",
    "chroma_hip_execute_chained",
    "chroma_hip_decoder_masks",
    "chroma_hip_clear_input",
    "chroma_hip_download",
    "chroma_hip_set_graph",
    "chroma_hip_launch_count",
    "chroma_hip_device_base",
    "chroma_hip_input_pointer",
    "chroma_hip_output_pointer",
    "chroma_hip_copy_2d",
    "chroma_hip_copy_2d_queued",
    "chroma_hip_copy_2d_batch_queued",
    "chroma_hip_synchronize",
    "chroma_hip_host_alloc",
    "chroma_hip_host_free",
    "chroma_hip_rows_topk_workspace",
    "chroma_hip_rows_topk",
    "chroma_hip_rows_topk_static",
    "chroma_hip_run_top",
)


def check(status: int, error: ctypes.Array) -> None:
    if status == OK:
        return
    message = error.value.decode(errors="replace")
    if status == INDEX_ERROR:
        raise IndexError(message)
    raise RuntimeError(message)


def pointer_array(pointers) -> ctypes.Array:
    pointers = list(pointers)
    return (ctypes.c_void_p * max(1, len(pointers)))(*pointers)
