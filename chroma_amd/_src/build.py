"""Compile generated HIP, write the artifact directory and publish it atomically.

Follows the reference's build/publish (chroma/_src/build.py:50-113): everything is staged in a temporary
directory inside the output, loaded once from there, then moved into place with ``os.replace``; files of
the artifact it replaces are deleted afterwards. The ``nvcc`` branch (build.py:22-30) becomes
``hipcc --genco`` for gfx950: the artifact holds a device code object, not a host extension, and the
prebuilt ``libchroma_hip.so`` runs it.

Artifact contents: ``model.json`` (manifest version 2), ``_chroma_<id>.hsaco`` (code object),
``weights-<XXH3-128 of the blob [:20]>.bin``, ``model.plan`` (launch plan read by the runtime) and the generated
``model.hip``.
"""

from __future__ import annotations

import hashlib
import json
import os
import shlex
import shutil
import subprocess
import sysconfig
import tempfile
import uuid
from pathlib import Path
from typing import Dict, List, Optional, Set

from chroma_amd._src.codegen.base import GeneratedCode
from chroma_amd._src.native import DEVICE_INCLUDE
from chroma_amd._src.spec import MANIFEST_VERSION, signature

# -ffp-contract=off keeps every fused chain's multiply and add separately rounded, as the reference
# backends do; packed fp32 ALU forms are disabled (they are avoided on this hardware pool). MFMA
# accumulators are allocated in VGPRs: with the AGPR form the register allocator rotates the wide GEMM
# body's 192 loop-carried accumulators through copies every stage (the other kernels allocate the same
# either way).
DEVICE_FLAGS = [
    "--genco",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form=1",
]


def architecture() -> str:
    return os.environ.get("CHROMA_HIP_ARCH", "gfx950")


def compiler_command() -> List[str]:
    command = shlex.split(os.environ.get("HIPCC", "/opt/rocm/bin/hipcc"))
    if not command or shutil.which(command[0]) is None:
        raise RuntimeError("HIP compilation requires hipcc; set HIPCC or install ROCm")
    return [*command, f"--offload-arch={architecture()}", *DEVICE_FLAGS, f"-I{DEVICE_INCLUDE}"]


def _header_digest() -> str:
    digest = hashlib.sha256()
    for path in sorted(DEVICE_INCLUDE.rglob("*.h")):
        digest.update(path.name.encode() + path.read_bytes())
    return digest.hexdigest()


def cache_directory() -> Path:
    return Path(os.environ.get("CHROMA_HIP_CACHE", Path.home() / ".cache" / "chroma_amd" / "hsaco"))


def compile_code_object(source: str, destination: Path) -> None:
    """hipcc the generated source to ``destination``; identical sources are served from a cache."""
    command = compiler_command()
    key = hashlib.sha256((source + "\0" + " ".join(command) + "\0" + _header_digest()).encode()).hexdigest()
    cached = cache_directory() / f"{key}.hsaco"
    if cached.exists():
        shutil.copyfile(cached, destination)
        return
    with tempfile.TemporaryDirectory(prefix="chroma-hipcc-") as work:
        path = Path(work) / "model.hip"
        path.write_text(source)
        result = subprocess.run([*command, str(path), "-o", str(destination)], capture_output=True, text=True, check=False)
        if result.returncode:
            raise RuntimeError(f"HIP compilation failed:\n{result.stderr[-6000:]}")
    try:
        cached.parent.mkdir(parents=True, exist_ok=True)
        temporary = cached.with_suffix(f".{uuid.uuid4().hex}.tmp")
        shutil.copyfile(destination, temporary)
        os.replace(temporary, cached)
    except OSError:
        pass


def _artifact_files(directory: Path) -> Set[str]:
    try:
        manifest = json.loads((directory / "model.json").read_text())
        names = {manifest["library"], manifest["weights"]}
    except (OSError, ValueError, KeyError, TypeError):
        return set()
    return {name for name in names if isinstance(name, str) and name == Path(name).name}


# Weights files this process has published, by blob digest: a later artifact with the same blob (the
# prefill and decode graphs of one model) hard-links the file instead of writing gigabytes again.
_published_weights: Dict[str, Path] = {}


def _write_weights(weights, digest: str, destination: Path) -> None:
    existing = _published_weights.get(digest)
    if existing is not None:
        try:
            if existing.stat().st_size == len(weights):
                os.link(existing, destination)
                return
        except OSError:
            pass
    weights.write_to(destination)


def build(generated: GeneratedCode, output, *, load: bool = True):
    """Write the artifact for ``generated`` into ``output`` and return the loaded ``Program``
    (``load=False`` publishes without touching a GPU and returns the directory)."""
    from chroma_amd._src.program import Program

    inputs, outputs, weights = generated.inputs, generated.outputs, generated.weights
    library = f"_chroma_{uuid.uuid4().hex}.hsaco"
    digest = weights.hexdigest()
    weights_name = f"weights-{digest[:20]}.bin"
    output = Path(output).resolve()
    output.mkdir(parents=True, exist_ok=True)
    stale = _artifact_files(output)
    files = dict(generated.files)
    header = [f"signature {signature(inputs, outputs)}", f"code_object {library}", f"weights_file {weights_name}"]
    plan_lines = files["model.plan"].splitlines()
    files["model.plan"] = "\n".join(plan_lines[:1] + header + plan_lines[1:]) + "\n"

    with tempfile.TemporaryDirectory(prefix=".compile-", dir=output) as temporary:
        stage = Path(temporary)
        for name, text in files.items():
            (stage / name).write_text(text)
        compile_code_object(files[generated.source_name], stage / library)
        _write_weights(weights, digest, stage / weights_name)
        manifest = {
            "version": MANIFEST_VERSION,
            "python_abi": sysconfig.get_config_var("SOABI"),
            "library": library,
            "weights": weights_name,
            "inputs": inputs,
            "outputs": outputs,
            "stats": generated.stats,
        }
        (stage / "model.json").write_text(json.dumps(manifest, indent=2) + "\n")
        model: Optional[Program] = Program(stage) if load else None
        try:
            for name in (library, weights_name, *files, "model.json"):
                os.replace(stage / name, output / name)
        except BaseException:
            if model is not None:
                model.close()
            raise
    _published_weights[digest] = output / weights_name
    # The loaded program holds its code object and weights on the device, so replaced files can go.
    for name in stale - {library, weights_name}:
        (output / name).unlink(missing_ok=True)
    return model if load else output
