"""Seeded dev-model weights and their digest.

``make_dev_model(seed)`` restates the reference's benchmark weights (scripts/export.py:16-29): construct
the bf16 model (module initialisers consume the RNG), cast to fp32, then walk ``named_parameters`` and set
norm scales to 1, biases and sinks to 0 and everything else to N(0, 0.02), all inside a forked RNG.
``weights_digest`` is the reference's state-dict digest (scripts/benchmark.py:96-101); for seed 0 it must
equal ``DEV_WEIGHTS_SHA256`` (docs/benchmarks/cuda-benchmark.json:52).
"""

from __future__ import annotations

import hashlib

import torch

from chroma_amd.models.gpt_oss import ModelConfig, Transformer
from chroma_amd.models.variants import dev

DEV_WEIGHTS_SHA256 = "cc57b07e0d327c575801ee9b1287da016df9178395f58c24be513f7362a28726"
DEV_PARAMETERS = 59_079_408


def make_model(config: ModelConfig, seed: int, std: float = 0.02, dtype: torch.dtype = torch.float32) -> Transformer:
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        model = Transformer(config, device=torch.device("cpu")).float().eval()
        with torch.no_grad():
            for name, parameter in model.named_parameters():
                if name.endswith(".scale"):
                    parameter.fill_(1.0)
                elif name.endswith(("bias", ".sinks")):
                    parameter.zero_()
                else:
                    parameter.normal_(mean=0.0, std=std)
    return model.to(dtype).requires_grad_(False)


def make_dev_model(seed: int = 0) -> Transformer:
    return make_model(dev, seed)


def weights_digest(model: torch.nn.Module) -> str:
    digest = hashlib.sha256()
    for name, value in model.state_dict().items():
        digest.update(name.encode())
        digest.update(value.numpy().tobytes())
    return digest.hexdigest()


def make_gpt_oss_20b(seed: int = 2, *, std: float = 0.02, generator_device: str = "cpu", **changes) -> Transformer:
    """The GPT-OSS-20B-shaped bfloat16 workload with seeded random weights: norm scales 1, biases and
    sinks 0, every other parameter N(0, ``std``) drawn in ``named_parameters`` order from one generator
    seeded with ``seed`` on ``generator_device`` ("cpu", or "cuda" to draw 21 billion values in seconds).
    ``changes`` override configuration fields (a reduced slice keeps the widths and drops layers or
    experts). The module is built without initialisers, so no float32 copy of the model ever exists."""
    import dataclasses

    from chroma_amd.models.variants import gpt_oss_20b

    config = dataclasses.replace(gpt_oss_20b, **changes)
    with torch.device("meta"):
        model = Transformer(config)
    model = model.to_empty(device="cpu")
    generator = torch.Generator(device=generator_device).manual_seed(seed)
    chunk = 1 << 26
    with torch.no_grad():
        for name, parameter in model.named_parameters():
            if name.endswith(".scale"):
                parameter.fill_(1.0)
            elif name.endswith(("bias", ".sinks")):
                parameter.zero_()
            else:
                flat = parameter.view(-1)
                for start in range(0, flat.numel(), chunk):
                    piece = flat[start : start + chunk]
                    drawn = torch.empty(piece.numel(), dtype=torch.float32, device=generator_device)
                    drawn.normal_(mean=0.0, std=std, generator=generator)
                    piece.copy_(drawn)
    return model.eval().requires_grad_(False)
