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
