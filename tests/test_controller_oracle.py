"""Pins of oracle/controller.py (the controller's per-token work,
inference.py:459-535) on the CPU.

* Against torch's own CPU LayerNorm, Linear, softplus and sigmoid, composed
  with the reshapes and permutes the reference applies (inference.py:
  471-518, 528-535): a transposed bank order, a misplaced eps or a wrong
  softplus fails here, since those library routines and torch's
  permute/flatten fix them independently of the oracle's own arithmetic.
* Closed forms: a constant token normalises to the norm's bias; zero
  projections give their biases; zero gate inputs give sigmoid 1/2 and
  forget -exp(A_log) * log 2.
* Planted mistakes in copies of the oracle fail the pins.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from controller_cases import make_layer, params_of, tokens
from oracle import controller as ctl


def torch_prepare(layer, x):
    """The reference's composition (inference.py:470-518) in torch ops."""

    batch = x.shape[0]
    normalized = layer.input_norm(x)
    raw_reads = layer.read_projection(normalized).reshape(
        batch, 1, layer.memory_heads, layer.key_width_per_head)
    raw_writes = layer.write_projection(normalized).reshape_as(raw_reads)
    reads = raw_reads.permute(0, 2, 1, 3).flatten(0, 1)
    writes = raw_writes.permute(0, 2, 1, 3).flatten(0, 1)
    values = (layer.value_projection(normalized)
              .reshape(batch, 1, layer.memory_heads, layer.head_width)
              .permute(0, 2, 1, 3).flatten(0, 1)[:, 0])
    forget = (-torch.exp(layer.A_log) * F.softplus(layer.forget_projection(normalized)
                                                   + layer.dt_bias)).permute(0, 2, 1).flatten()
    input_gate = torch.sigmoid(layer.input_projection(normalized)).permute(0, 2, 1).flatten()
    return {"normalized": normalized, "read_keys": reads, "write_keys": writes,
            "values": values, "input_gate": input_gate, "forget_log_gate": forget}


def torch_finish(layer, normalized, reading):
    """inference.py:528-535 in torch ops."""

    batch = normalized.shape[0]
    r = layer.readings_norm(reading).reshape(batch, layer.memory_heads, layer.head_width)
    r = r.reshape(batch, 1, layer.width)
    gate = torch.sigmoid(layer.output_gate(normalized))
    return layer.output_projection(gate * r)


CASES = [(128, 256, 1, 5), (512, 1024, 4, 3), (96, 64, 2, 4), (64, 16, 4, 1)]


@pytest.mark.parametrize("width,slots,heads,batch", CASES)
def test_prepare_matches_torch_composition(width, slots, heads, batch):
    layer = make_layer(width, slots=slots, reads=8, writes=4, heads=heads, seed=width + heads)
    x = tokens(batch, width, seed=3)
    want = {k: v.detach().numpy() for k, v in torch_prepare(layer, x).items()}
    got = ctl.prepare(params_of(layer), x.numpy())
    assert set(got) == set(want)
    for k in want:
        assert got[k].shape == want[k].shape, k
        np.testing.assert_allclose(got[k], want[k], rtol=1e-12, atol=1e-13, err_msg=k)


@pytest.mark.parametrize("width,slots,heads,batch", CASES)
def test_finish_matches_torch_composition(width, slots, heads, batch):
    layer = make_layer(width, slots=slots, reads=8, writes=4, heads=heads, seed=7 * width)
    x = tokens(batch, width, seed=4)
    normalized = layer.input_norm(x)
    reading = tokens(batch * heads, width // heads, seed=5)[:, 0]
    want = torch_finish(layer, normalized, reading).detach().numpy()
    got = ctl.finish(params_of(layer), normalized.detach().numpy(), reading.numpy())
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-13)


def test_closed_forms():
    width, heads = 8, 2
    layer = make_layer(width, slots=16, reads=4, writes=2, heads=heads, seed=1)
    p = params_of(layer)
    # a constant token has zero variance: it normalises to the bias
    x = np.full((3, 1, width), 2.5)
    out = ctl.prepare(p, x)
    np.testing.assert_allclose(out["normalized"][:, 0], np.broadcast_to(p["input_norm"][1], (3, width)),
                               rtol=0, atol=1e-12)
    # zero projection weights give the biases, in bank order b * H + h
    for name in ("read_projection", "write_projection", "value_projection",
                 "forget_projection", "input_projection"):
        w, b = p[name]
        p[name] = (np.zeros_like(w), b)
    out = ctl.prepare(p, tokens(3, width, seed=9).numpy())
    key = p["read_projection"][1].reshape(heads, 8)
    np.testing.assert_array_equal(out["read_keys"][:, 0], np.tile(key, (3, 1)))
    vb = p["value_projection"][1].reshape(heads, width // heads)
    np.testing.assert_array_equal(out["values"], np.tile(vb, (3, 1)))
    # zero gate inputs: sigmoid(0) = 1/2, softplus(0) = log 2
    p["forget_projection"] = (p["forget_projection"][0], np.zeros(heads))
    p["input_projection"] = (p["input_projection"][0], np.zeros(heads))
    p["dt_bias"] = np.zeros(heads)
    out = ctl.prepare(p, tokens(3, width, seed=9).numpy())
    np.testing.assert_allclose(out["input_gate"], 0.5, rtol=0, atol=0)
    np.testing.assert_allclose(out["forget_log_gate"],
                               np.tile(-np.exp(p["A_log"]) * math.log(2.0), 3), rtol=1e-15)
    # softplus's threshold: the identity above 20
    assert ctl.softplus(np.array([25.0]))[0] == 25.0
    assert abs(ctl.softplus(np.array([-30.0]))[0] - math.exp(-30.0)) < 1e-25
    # finish: zero-variance readings normalise to the bias; a zero output gate is 1/2
    p["output_gate"] = (np.zeros((width, width)), np.zeros(width))
    p["output_projection"] = (np.eye(width), np.zeros(width))
    y = ctl.finish(p, np.zeros((3, 1, width)), np.full((3 * heads, width // heads), 4.0))
    rb = np.tile(p["readings_norm"][1], heads)
    np.testing.assert_allclose(y[:, 0], np.tile(0.5 * rb, (3, 1)), rtol=0, atol=1e-15)


def _mutants():
    """Copies of oracle functions with one plausible mistake each."""

    def head_major(params, x):
        out = ctl.prepare(params, x)
        b, h = x.shape[0], params["memory_heads"]
        for k in ("read_keys", "write_keys", "values"):
            v = out[k]
            out[k] = v.reshape(b, h, *v.shape[1:]).swapaxes(0, 1).reshape(v.shape)
        return out

    def unbiased_variance(params, x):
        out = ctl.prepare(params, x)
        n = params["width"]
        xx = np.asarray(x, np.float64)
        mean = xx.mean(-1, keepdims=True)
        var = ((xx - mean) ** 2).sum(-1, keepdims=True) / (n - 1)
        w, b, eps = params["input_norm"]
        out["normalized"] = (xx - mean) / np.sqrt(var + eps) * w + b
        return out

    def eps_outside(params, x):
        out = ctl.prepare(params, x)
        xx = np.asarray(x, np.float64)
        mean = xx.mean(-1, keepdims=True)
        var = ((xx - mean) ** 2).mean(-1, keepdims=True)
        w, b, eps = params["input_norm"]
        out["normalized"] = (xx - mean) / (np.sqrt(var) + eps) * w + b
        return out

    def dt_bias_dropped(params, x):
        p = dict(params)
        p["dt_bias"] = np.zeros_like(params["dt_bias"])
        return ctl.prepare(p, x)

    return [head_major, unbiased_variance, eps_outside, dt_bias_dropped]


@pytest.mark.parametrize("mutant", _mutants(), ids=lambda f: f.__name__)
def test_planted_mistakes_fail_the_torch_pin(mutant):
    layer = make_layer(96, slots=64, reads=8, writes=4, heads=2, seed=11)
    x = tokens(4, 96, seed=12)
    want = {k: v.detach().numpy() for k, v in torch_prepare(layer, x).items()}
    got = mutant(params_of(layer), x.numpy())
    assert any(not np.allclose(got[k], want[k], rtol=1e-12, atol=1e-13) for k in want)
