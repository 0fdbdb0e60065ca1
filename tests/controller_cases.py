"""Controller weights for tests: a stand-in module with the attribute names
of the reference's ``SparseDeltaMemory`` (sdm.py:1032-1052), built from
torch's own LayerNorm and Linear layers, and its parameters as the numpy
dict ``oracle.controller`` takes."""

from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np
import torch
from torch import nn


def make_layer(width: int, *, slots: int, reads: int, writes: int, heads: int = 1,
               seed: int = 0, norm_eps: float = 1e-6, dtype=torch.float64) -> SimpleNamespace:
    """Random weights, biases and norm affines (none left at their zero or
    one initial values, so that every term is exercised)."""

    g = torch.Generator().manual_seed(seed)
    root = math.isqrt(slots)
    key = heads * 2 * root
    std = width ** -0.5

    def lin(out):
        layer = nn.Linear(width, out, bias=True).to(dtype)
        with torch.no_grad():
            layer.weight.copy_(torch.randn(out, width, generator=g, dtype=dtype) * std)
            layer.bias.copy_(torch.randn(out, generator=g, dtype=dtype) * 0.1)
        return layer

    def norm(n, eps):
        layer = nn.LayerNorm(n, eps=eps).to(dtype)
        with torch.no_grad():
            layer.weight.copy_(1.0 + torch.randn(n, generator=g, dtype=dtype) * 0.1)
            layer.bias.copy_(torch.randn(n, generator=g, dtype=dtype) * 0.1)
        return layer

    return SimpleNamespace(
        width=width, slots=slots, reads=reads, writes=writes, memory_heads=heads,
        head_width=width // heads, key_width_per_head=2 * root,
        input_norm=norm(width, 1e-5), read_projection=lin(key), write_projection=lin(key),
        value_projection=lin(width), forget_projection=lin(heads), input_projection=lin(heads),
        A_log=(torch.rand(heads, generator=g, dtype=dtype) * 3.0).log(),
        dt_bias=torch.randn(heads, generator=g, dtype=dtype),
        output_gate=lin(width), output_projection=lin(width),
        readings_norm=norm(width // heads, norm_eps))


def params_of(layer: SimpleNamespace) -> dict:
    """The numpy parameter dict of ``oracle.controller``."""

    def arr(t):
        return t.detach().to(torch.float64).cpu().numpy()

    def lin(m):
        return (arr(m.weight), arr(m.bias))

    def norm(m):
        return (arr(m.weight), arr(m.bias), m.eps)

    return {
        "width": layer.width, "slots": layer.slots, "memory_heads": layer.memory_heads,
        "input_norm": norm(layer.input_norm), "readings_norm": norm(layer.readings_norm),
        "read_projection": lin(layer.read_projection),
        "write_projection": lin(layer.write_projection),
        "value_projection": lin(layer.value_projection),
        "forget_projection": lin(layer.forget_projection),
        "input_projection": lin(layer.input_projection),
        "output_gate": lin(layer.output_gate), "output_projection": lin(layer.output_projection),
        "A_log": arr(layer.A_log), "dt_bias": arr(layer.dt_bias),
    }


def tokens(batch: int, width: int, *, seed: int, dtype=torch.float64) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(batch, 1, width, generator=g, dtype=dtype)
