"""KV-cached and padded-uncached exports of the GPT-OSS workload.

``export_cached(model, context, steps)`` exports one prefill chunk (``steps == context``) or decode step
(``steps == 1``) with the cache as explicit inputs, in the order the ``Decoder`` expects: token ids
[steps] int64, positions [steps] fp32, keys and values [layers, context, kv_heads, head_dim], full and
window masks [steps, context + steps] (0 or -inf), and the row whose logits to return [1] int64. It
returns the logits [1, vocab] and the new key and value rows [layers, steps, kv_heads, head_dim]
(reference chroma/models/cached.py:9-91).

``routing=True`` (an addition for parity checks, not in the reference) exports a probe of the same graph
that also returns every layer's router decision: the gate logits [layers, steps, experts] and the chosen
expert ids [layers, steps, k], outputs 3 and 4. The arithmetic of the other outputs is unchanged.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch
from torch import Tensor, nn

from chroma_amd.models.gpt_oss import Transformer


class CachedTransformer(nn.Module):
    def __init__(self, model: Transformer, routing: bool = False, forced: Optional[Tensor] = None) -> None:
        """``forced`` (eager use only): expert ids [layers, steps, k] every layer takes instead of its own
        top-k, so an eager run follows another run's routing decisions."""
        super().__init__()
        self.model = model
        self.routing = routing
        self.forced = forced

    def forward(
        self, tokens: Tensor, positions: Tensor, keys: Tensor, values: Tensor, mask: Tensor, window_mask: Tensor, last: Tensor
    ) -> Tuple[Tensor, ...]:
        x = self.model.embedding(tokens)
        new_keys: List[Tensor] = []
        new_values: List[Tensor] = []
        routing: Optional[List[Tuple[Tensor, Tensor]]] = [] if self.routing else None
        for layer, block in enumerate(self.model.block):
            attention = block.attn
            q, k, v = attention.project(x, positions)
            new_keys.append(k.unsqueeze(0))
            new_values.append(v.unsqueeze(0))
            past = (keys.shape[1], attention.num_key_value_heads, attention.head_dim)
            all_k = torch.cat((keys[layer : layer + 1].reshape(past), k), dim=0)
            all_v = torch.cat((values[layer : layer + 1].reshape(past), v), dim=0)
            steps, kv_heads, group, _ = q.shape
            all_k = all_k[:, :, None, :].expand(-1, -1, group, -1)
            all_v = all_v[:, :, None, :].expand(-1, -1, group, -1)
            scores = torch.einsum("qhmd,khmd->hmqk", q, all_k) * attention.sm_scale
            scores = scores + (window_mask if attention.sliding_window else mask)[None, None, :, :]
            sinks = attention.sinks.reshape(kv_heads, group, 1, 1).expand(-1, -1, steps, -1)
            weights = torch.cat((scores, sinks), dim=-1).softmax(-1)[..., :-1]
            attended = torch.einsum("hmqk,khmd->qhmd", weights, all_v).reshape(steps, -1)
            x = block.mlp(x + attention.out(attended), routing, None if self.forced is None else self.forced[layer])
        logits = self.model.unembedding(self.model.norm(x)[last])
        if routing is None:
            return logits, torch.cat(new_keys, dim=0), torch.cat(new_values, dim=0)
        return (logits, torch.cat(new_keys, dim=0), torch.cat(new_values, dim=0),
                *(torch.cat([layer[i].unsqueeze(0) for layer in routing], dim=0) for i in (0, 1)))


class UncachedTransformer(nn.Module):
    """A full forward over a padded window that projects only the selected position to the vocabulary."""

    def __init__(self, model: Transformer) -> None:
        super().__init__()
        self.model = model

    def forward(self, tokens: Tensor, position: Tensor) -> Tensor:
        x = self.model.embedding(tokens)
        for block in self.model.block:
            x = block(x)
        return self.model.unembedding(self.model.norm(x)[position])


def export_cached(model: Transformer, context: int, steps: int, routing: bool = False) -> torch.export.ExportedProgram:
    if context < 1 or not 1 <= steps <= context:
        raise ValueError(f"{steps} steps, context {context}")
    first = model.block[0].attn
    cache_shape = (len(model.block), context, first.num_key_value_heads, first.head_dim)
    dtype = first.qkv.weight.dtype
    examples = (
        torch.zeros(steps, dtype=torch.int64),
        torch.arange(steps, dtype=torch.float32),
        torch.zeros(cache_shape, dtype=dtype),
        torch.zeros(cache_shape, dtype=dtype),
        torch.zeros(steps, context + steps, dtype=dtype),
        torch.zeros(steps, context + steps, dtype=dtype),
        torch.tensor([steps - 1], dtype=torch.int64),
    )
    with torch.no_grad():
        return torch.export.export(CachedTransformer(model, routing).eval(), examples)


def export_uncached(model: Transformer, context: int) -> torch.export.ExportedProgram:
    tokens = torch.arange(context, dtype=torch.int64) % model.embedding.num_embeddings
    with torch.no_grad():
        return torch.export.export(UncachedTransformer(model).eval(), (tokens, torch.tensor([context - 1], dtype=torch.int64)))
