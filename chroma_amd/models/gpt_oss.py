"""GPT-OSS-style mixture-of-experts transformer used as the benchmark workload.

Architecture and parameter layout follow the reference workload (chroma/models/gpt_oss.py:10-310), which
adapts the gpt-oss PyTorch reference model (Apache-2.0): RMSNorm, YaRN rotary embeddings, grouped-query
attention with learned sinks and optional sliding windows, and a top-k router over SwiGLU experts whose
weights are gathered per (token, slot). The module tree, parameter names, registration order and dtypes
are kept identical on purpose: the seeded dev weights are pinned by a sha256 over the state dict
(docs/benchmarks/benchmark.json), which depends on all four. The arithmetic is written so that
``torch.export`` emits only operators the compiler accepts (the RMSNorm chain is explicit so that
``fuse_norms`` recognises it).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch
from torch import Tensor, nn


@dataclass
class ModelConfig:
    num_hidden_layers: int
    num_experts: int
    experts_per_token: int
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    swiglu_limit: float
    head_dim: int
    num_attention_heads: int
    num_key_value_heads: int
    sliding_window: int
    initial_context_length: int
    rope_theta: float
    rope_scaling_factor: float
    rope_ntk_alpha: float
    rope_ntk_beta: float


class RMSNorm(nn.Module):
    def __init__(self, num_features: int, eps: float = 1e-05, device: Optional[torch.device] = None) -> None:
        super().__init__()
        self.num_features = num_features
        self.eps = eps
        self.scale = nn.Parameter(torch.ones(num_features, device=device, dtype=torch.float32))

    def forward(self, x: Tensor) -> Tensor:
        dtype = x.dtype
        h = x.float()
        inverse = torch.rsqrt(torch.mean(h**2, dim=-1, keepdim=True) + self.eps)
        return (h * inverse * self.scale).to(dtype)


def rotate(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """Rotate the two halves of the last axis of ``x`` [tokens, heads, dim] by per-token angles."""
    cos = cos.unsqueeze(-2).to(x.dtype)
    sin = sin.unsqueeze(-2).to(x.dtype)
    first, second = torch.chunk(x, 2, dim=-1)
    return torch.cat((first * cos - second * sin, second * cos + first * sin), dim=-1)


class RotaryEmbedding(nn.Module):
    """Rotary position embedding with YaRN NTK-by-parts scaling (https://arxiv.org/abs/2309.00071)."""

    def __init__(
        self,
        head_dim: int,
        base: float,
        dtype: torch.dtype,
        initial_context_length: int = 4096,
        scaling_factor: float = 1.0,
        ntk_alpha: float = 1.0,
        ntk_beta: float = 32.0,
        device: Optional[torch.device] = None,
    ) -> None:
        super().__init__()
        self.head_dim = head_dim
        self.base = base
        self.dtype = dtype
        self.initial_context_length = initial_context_length
        self.scaling_factor = scaling_factor
        self.ntk_alpha = ntk_alpha
        self.ntk_beta = ntk_beta
        self.device = device

    def inverse_frequencies(self) -> Tuple[float, Tensor]:
        exponents = torch.arange(0, self.head_dim, 2, dtype=torch.float, device=self.device) / self.head_dim
        freq = self.base**exponents
        if self.scaling_factor <= 1.0:
            return 1.0, 1.0 / freq
        concentration = 0.1 * math.log(self.scaling_factor) + 1.0
        half = self.head_dim / 2
        low = half * math.log(self.initial_context_length / (self.ntk_beta * 2 * math.pi)) / math.log(self.base)
        high = half * math.log(self.initial_context_length / (self.ntk_alpha * 2 * math.pi)) / math.log(self.base)
        assert 0 < low < high < half - 1
        interpolated = 1.0 / (self.scaling_factor * freq)
        extrapolated = 1.0 / freq
        ramp = (torch.arange(half, dtype=torch.float32, device=freq.device) - low) / (high - low)
        keep = 1 - ramp.clamp(0, 1)
        return concentration, interpolated * (1 - keep) + extrapolated * keep

    def angles(self, num_tokens: int, positions: Optional[Tensor]) -> Tuple[Tensor, Tensor]:
        concentration, inverse = self.inverse_frequencies()
        t = torch.arange(num_tokens, dtype=torch.float32, device=self.device) if positions is None else positions
        freqs = torch.einsum("i,j->ij", t, inverse)
        return freqs.cos() * concentration, freqs.sin() * concentration

    def forward(self, query: Tensor, key: Tensor, positions: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
        tokens = query.shape[0]
        cos, sin = self.angles(tokens, positions)
        query_shape, key_shape = query.shape, key.shape
        query = rotate(query.view(tokens, -1, self.head_dim), cos, sin).reshape(query_shape)
        key = rotate(key.view(tokens, -1, self.head_dim), cos, sin).reshape(key_shape)
        return query, key


def sdpa(Q: Tensor, K: Tensor, V: Tensor, S: Tensor, sm_scale: float, sliding_window: int = 0) -> Tensor:
    """Causal grouped-query attention with one learned sink logit per head (dropped after softmax)."""
    tokens, kv_heads, group, _ = Q.shape
    K = K[:, :, None, :].expand(-1, -1, group, -1)
    V = V[:, :, None, :].expand(-1, -1, group, -1)
    S = S.reshape(kv_heads, group, 1, 1).expand(-1, -1, tokens, -1)
    mask = torch.triu(Q.new_full((tokens, tokens), -float("inf")), diagonal=1)
    if sliding_window > 0:
        mask += torch.tril(mask.new_full((tokens, tokens), -float("inf")), diagonal=-sliding_window)
    scores = torch.einsum("qhmd,khmd->hmqk", Q, K)
    scores *= sm_scale
    scores += mask[None, None, :, :]
    weights = torch.softmax(torch.cat([scores, S], dim=-1), dim=-1)[..., :-1]
    attended = torch.einsum("hmqk,khmd->qhmd", weights, V)
    return attended.reshape(tokens, -1)


class AttentionBlock(nn.Module):
    def __init__(self, config: ModelConfig, layer_idx: int = 0, device: Optional[torch.device] = None) -> None:
        super().__init__()
        self.head_dim = config.head_dim
        self.num_attention_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        # Even layers use the sliding window, odd layers attend to the whole context.
        self.sliding_window = config.sliding_window if layer_idx % 2 == 0 else 0
        self.sinks = nn.Parameter(torch.empty(config.num_attention_heads, device=device, dtype=torch.bfloat16))
        self.norm = RMSNorm(config.hidden_size, device=device)
        width = config.head_dim * (config.num_attention_heads + 2 * config.num_key_value_heads)
        self.qkv = nn.Linear(config.hidden_size, width, device=device, dtype=torch.bfloat16)
        self.out = nn.Linear(config.head_dim * config.num_attention_heads, config.hidden_size, device=device, dtype=torch.bfloat16)
        self.sm_scale = 1 / math.sqrt(config.head_dim)
        self.rope = RotaryEmbedding(
            config.head_dim,
            config.rope_theta,
            torch.float32,
            initial_context_length=config.initial_context_length,
            scaling_factor=config.rope_scaling_factor,
            ntk_alpha=config.rope_ntk_alpha,
            ntk_beta=config.rope_ntk_beta,
            device=device,
        )

    def project(self, x: Tensor, positions: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
        qkv = self.qkv(self.norm(x))
        q_width = self.num_attention_heads * self.head_dim
        kv_width = self.num_key_value_heads * self.head_dim
        q = qkv[:, :q_width].contiguous()
        k = qkv[:, q_width : q_width + kv_width].contiguous()
        v = qkv[:, q_width + kv_width : q_width + 2 * kv_width].contiguous()
        group = self.num_attention_heads // self.num_key_value_heads
        q = q.view(-1, self.num_key_value_heads, group, self.head_dim)
        k = k.view(-1, self.num_key_value_heads, self.head_dim)
        v = v.view(-1, self.num_key_value_heads, self.head_dim)
        q, k = self.rope(q, k, positions)
        return q, k, v

    def forward(self, x: Tensor) -> Tensor:
        q, k, v = self.project(x)
        return x + self.out(sdpa(q, k, v, self.sinks, self.sm_scale, self.sliding_window))


def swiglu(x: Tensor, alpha: float = 1.702, limit: float = 7.0) -> Tensor:
    """Clamped SwiGLU over interleaved (glu, linear) channels, with the +1 bias on the linear half."""
    glu, linear = x[..., ::2], x[..., 1::2]
    glu = glu.clamp(min=None, max=limit)
    linear = linear.clamp(min=-limit, max=limit)
    return glu * torch.sigmoid(alpha * glu) * (linear + 1)


class MLPBlock(nn.Module):
    def __init__(self, config: ModelConfig, device: Optional[torch.device] = None) -> None:
        super().__init__()
        self.num_experts = config.num_experts
        self.experts_per_token = config.experts_per_token
        self.swiglu_limit = config.swiglu_limit
        self.norm = RMSNorm(config.hidden_size, device=device)
        self.gate = nn.Linear(config.hidden_size, config.num_experts, device=device, dtype=torch.bfloat16)

        def empty(*shape: int) -> nn.Parameter:
            return nn.Parameter(torch.empty(shape, device=device, dtype=torch.bfloat16))

        self.mlp1_weight = empty(config.num_experts, config.intermediate_size * 2, config.hidden_size)
        self.mlp1_bias = empty(config.num_experts, config.intermediate_size * 2)
        self.mlp2_weight = empty(config.num_experts, config.hidden_size, config.intermediate_size)
        self.mlp2_bias = empty(config.num_experts, config.hidden_size)

    def forward(self, x: Tensor, routing: Optional[List[Tuple[Tensor, Tensor]]] = None, forced: Optional[Tensor] = None) -> Tensor:
        """Two additions, not in the reference (which has neither argument), that leave the arithmetic
        unchanged: with a ``routing`` list the block appends its (gate logits [tokens, experts], expert
        ids [tokens, k]) to it, so that a probe export can return every layer's routing decision; with
        ``forced`` expert ids [tokens, k] an eager run takes those experts (and their gate logits as the
        values) instead of its own top-k, to follow another run's routing."""
        t = self.norm(x)
        gate = self.gate(t)
        if forced is None:
            routed = torch.topk(gate, k=self.experts_per_token, dim=-1, sorted=True)
            values, experts = routed.values, routed.indices
        else:
            values, experts = torch.gather(gate, -1, forced), forced
        if routing is not None:
            routing.append((gate, experts))
        expert_weights = nn.functional.softmax(values, dim=1)
        t = torch.einsum("beck,bk->bec", self.mlp1_weight[experts, ...], t) + self.mlp1_bias[experts, ...]
        t = swiglu(t, limit=self.swiglu_limit)
        t = torch.einsum("beck,bek->bec", self.mlp2_weight[experts, ...], t)
        t += self.mlp2_bias[experts, ...]
        return x + torch.einsum("bec,be->bc", t, expert_weights)


class TransformerBlock(nn.Module):
    def __init__(self, config: ModelConfig, layer_idx: int, device: Optional[torch.device] = None) -> None:
        super().__init__()
        self.layer_idx = layer_idx
        self.attn = AttentionBlock(config, layer_idx, device)
        self.mlp = MLPBlock(config, device)

    def forward(self, x: Tensor, routing: Optional[List[Tuple[Tensor, Tensor]]] = None) -> Tensor:
        return self.mlp(self.attn(x), routing)


class Transformer(nn.Module):
    def __init__(self, config: ModelConfig, device: Optional[torch.device] = None) -> None:
        super().__init__()
        self.embedding = nn.Embedding(config.vocab_size, config.hidden_size, device=device, dtype=torch.bfloat16)
        self.block = nn.ModuleList([TransformerBlock(config, i, device) for i in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, device=device)
        self.unembedding = nn.Linear(config.hidden_size, config.vocab_size, bias=False, device=device, dtype=torch.bfloat16)

    def forward(self, x: Tensor) -> Tensor:
        x = self.embedding(x)
        for block in self.block:
            x = block(x)
        return self.unembedding(self.norm(x))
