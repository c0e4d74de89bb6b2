"""Small benchmark workloads: BASELINE configs C1 (MLP block) and C2 (bandwidth graph), and the row
reductions (RMSNorm, softmax, log-sum-exp) and plain copy the measurement compares against HBM.

Each is an ``nn.Module`` for ``torch.export`` with seeded inputs; none needs a checkpoint.
"""

from __future__ import annotations

from typing import Tuple

import torch


def mlp_block(hidden: int = 1024, intermediate: int = 4096, seed: int = 0) -> torch.nn.Module:
    """C1: explicit RMSNorm (eps 1e-5, weight 1), SiLU(gate) * up, down projection, residual; weights
    N(0, 0.02) drawn with ``seed`` in the order gate, up, down; no biases. The norm is written as the
    explicit chain so the front end's RMSNorm pattern (reference graph.py:58-95) matches it."""

    class MLPBlock(torch.nn.Module):
        def __init__(self) -> None:
            super().__init__()
            generator = torch.Generator().manual_seed(seed)
            self.norm = torch.nn.Parameter(torch.ones(hidden), requires_grad=False)
            self.gate = torch.nn.Parameter(torch.randn(intermediate, hidden, generator=generator) * 0.02, requires_grad=False)
            self.up = torch.nn.Parameter(torch.randn(intermediate, hidden, generator=generator) * 0.02, requires_grad=False)
            self.down = torch.nn.Parameter(torch.randn(hidden, intermediate, generator=generator) * 0.02, requires_grad=False)

        def forward(self, x):
            h = x * torch.rsqrt(torch.mean(x**2, dim=-1, keepdim=True) + 1e-5) * self.norm
            gate = torch.nn.functional.linear(h, self.gate)
            up = torch.nn.functional.linear(h, self.up)
            return torch.nn.functional.linear(torch.nn.functional.silu(gate) * up, self.down) + x

    return MLPBlock().eval()


def mlp_inputs(rows: int = 8, hidden: int = 1024, seed: int = 0) -> Tuple[torch.Tensor]:
    return (torch.randn(rows, hidden, generator=torch.Generator().manual_seed(seed)),)


class BandwidthGraph(torch.nn.Module):
    """C2: a fused elementwise chain and a row softmax over its result."""

    def forward(self, x, y):
        z = torch.tanh(x * 0.5 + y) * torch.sigmoid(y) - torch.exp(torch.clamp(x, -8, 8)) * 1e-3
        return torch.softmax(z, -1)


def bandwidth_inputs(rows: int = 16384, columns: int = 8192, seed: int = 1) -> Tuple[torch.Tensor, torch.Tensor]:
    """x then y ~ U(-4, 4) from one generator seeded with ``seed``."""
    generator = torch.Generator().manual_seed(seed)
    x = torch.rand(rows, columns, generator=generator) * 8 - 4
    y = torch.rand(rows, columns, generator=generator) * 8 - 4
    return x, y


class RowNorm(torch.nn.Module):
    """RMSNorm over the last axis (eps 1e-5, weight 1) as the explicit chain."""

    def __init__(self, width: int) -> None:
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(width), requires_grad=False)

    def forward(self, x):
        return x * torch.rsqrt(torch.mean(x**2, dim=-1, keepdim=True) + 1e-5) * self.weight


class RowSoftmax(torch.nn.Module):
    def forward(self, x):
        return torch.softmax(x, -1)


class RowLogSumExp(torch.nn.Module):
    def forward(self, x):
        return torch.logsumexp(x, -1)


class Copy(torch.nn.Module):
    """A plain copy (``x * 1.0``): one read and one write per element, the practical HBM ceiling."""

    def forward(self, x):
        return x * 1.0
