"""Seeded synthetic SDM routes and step inputs for benchmarks and tests.

Routes follow the shapes the reference's controller produces
(copy_on_write_sdm/sdm.py:96-159): per bank and token, W write and R read
slot indices drawn without replacement and sorted, softmax route weights,
values ~ N(0, 1), input gate = sigmoid(N(0, 1)) (the erase gate defaults to
it), forget log gate = -U(0, 1) as in tests/test_allocator.py:31-38.

``uniform`` draws every slot with equal probability; ``zipf`` draws slot
``perm[k]`` with probability proportional to (k + 1)^-s without replacement
(Gumbel top-k over log-weights), with one fixed random permutation per
(layer, head), drawn from the call's generator or, with ``zipf_seed``, from
a generator of its own, so that calls with different seeds (a prefill and
the decode after it) share their hot slots.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class StepBatch:
    """Inputs of ``steps`` consecutive tokens for ``layers`` layers:
    index/weight tensors are [steps, layers, banks, K], values
    [steps, layers, banks, D], gates [steps, layers, banks]."""

    write_indices: torch.Tensor
    write_weights: torch.Tensor
    values: torch.Tensor
    input_gate: torch.Tensor
    forget_log_gate: torch.Tensor
    read_indices: torch.Tensor
    read_weights: torch.Tensor

    def step(self, s: int, layer: int) -> dict:
        return {
            "write_indices": self.write_indices[s, layer],
            "write_weights": self.write_weights[s, layer],
            "values": self.values[s, layer],
            "input_gate": self.input_gate[s, layer],
            "forget_log_gate": self.forget_log_gate[s, layer],
            "read_indices": self.read_indices[s, layer],
            "read_weights": self.read_weights[s, layer],
        }


def _subset(keys: torch.Tensor, k: int) -> torch.Tensor:
    return keys.topk(k, dim=-1).indices.sort(dim=-1).values


def zipf_log_weights(slots: int, exponent: float, permutation: torch.Tensor) -> torch.Tensor:
    """log-probability (unnormalised) of each slot: slot permutation[k] has
    weight (k+1)^-exponent."""

    ranks = torch.empty(slots, dtype=torch.float32, device=permutation.device)
    ranks[permutation] = torch.arange(1, slots + 1, dtype=torch.float32,
                                      device=permutation.device)
    return -exponent * ranks.log()


def make_steps(
    *,
    steps: int,
    layers: int,
    banks: int,
    slots: int,
    width: int,
    writes: int,
    reads: int,
    seed: int,
    device: torch.device | str = "cpu",
    index_dtype: torch.dtype = torch.int32,
    distribution: str = "uniform",
    zipf_exponent: float = 1.1,
    heads: int = 1,
    zipf_seed: int | None = None,
) -> StepBatch:
    """Generate a seeded batch of synthetic step inputs on ``device``."""

    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (steps, layers, banks)
    if distribution not in ("uniform", "zipf"):
        raise ValueError("distribution must be uniform or zipf")
    if distribution == "zipf" and banks % heads:
        raise ValueError("banks must be a multiple of heads")
    logw = None
    if distribution == "zipf":
        perm_gen = gen
        if zipf_seed is not None:
            perm_gen = torch.Generator(device=device)
            perm_gen.manual_seed(zipf_seed)
        logw = torch.stack([
            torch.stack([
                zipf_log_weights(slots, zipf_exponent,
                                 torch.randperm(slots, generator=perm_gen, device=device))
                for _ in range(heads)])
            for _ in range(layers)])                    # [L, H, N]
        logw = logw.repeat(1, banks // heads, 1)        # bank = seq * H + h

    def keys(n: int) -> torch.Tensor:
        if distribution == "uniform":
            return torch.rand(n, layers, banks, slots, generator=gen, device=device)
        gumbel = -torch.log(-torch.log(
            torch.rand(n, layers, banks, slots, generator=gen, device=device).clamp_min(1e-20)))
        return logw + gumbel

    # one key per (step, layer, bank, slot); large address spaces draw them a
    # few steps at a time (the routes then differ from a single draw)
    per_step = layers * banks * slots
    chunk = steps if steps * per_step <= (1 << 28) else max(1, (1 << 26) // per_step)
    if chunk >= steps:
        write_keys = keys(steps)
        read_keys = keys(steps)
        write_indices = _subset(write_keys, writes).to(index_dtype)
        read_indices = _subset(read_keys, reads).to(index_dtype)
        del write_keys, read_keys
    else:
        w_parts, r_parts = [], []
        for s0 in range(0, steps, chunk):
            n = min(chunk, steps - s0)
            w_parts.append(_subset(keys(n), writes).to(index_dtype))
            r_parts.append(_subset(keys(n), reads).to(index_dtype))
        write_indices = torch.cat(w_parts)
        read_indices = torch.cat(r_parts)
        del w_parts, r_parts
    write_weights = torch.softmax(
        torch.randn(*shape, writes, generator=gen, device=device), dim=-1)
    read_weights = torch.softmax(
        torch.randn(*shape, reads, generator=gen, device=device), dim=-1)
    values = torch.randn(*shape, width, generator=gen, device=device)
    input_gate = torch.sigmoid(torch.randn(*shape, generator=gen, device=device))
    forget_log_gate = -torch.rand(*shape, generator=gen, device=device)
    return StepBatch(
        write_indices=write_indices.contiguous(),
        write_weights=write_weights.contiguous(),
        values=values.contiguous(),
        input_gate=input_gate.contiguous(),
        forget_log_gate=forget_log_gate.contiguous(),
        read_indices=read_indices.contiguous(),
        read_weights=read_weights.contiguous(),
    )


def make_initial_memory(layers: int, heads: int, slots: int, width: int, *, seed: int,
                        device: torch.device | str = "cpu", std: float = 0.02) -> torch.Tensor:
    """M0 per layer ~ N(0, std^2): [layers, heads, slots, width] float32."""

    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return (torch.randn(layers, heads, slots, width, generator=gen, device=device)
            * std).contiguous()
