"""Float64 numpy restatement of the SDM controller's per-token work around
the copy-on-write step (copy_on_write_sdm/inference.py:459-535).

Test infrastructure only: ``tests/`` use it as the checker of
``copy_on_write_sdm_amd.controller``; nothing in the product imports it.

``params`` is a dict of numpy arrays named after the reference module's
parameters (sdm.py:1032-1052): ``input_norm`` / ``readings_norm`` as
(weight, bias, eps), the projections as (weight [out, in], bias [out]) like
``nn.Linear``, ``A_log`` and ``dt_bias`` [heads], and the sizes ``width``,
``slots``, ``memory_heads``.  Routes are not restated here: the caller runs
``oracle.routes.product_key_routes`` on the keys.

Pinned by ``tests/test_controller_oracle.py``: against torch's CPU
LayerNorm, Linear, softplus, sigmoid, reshape and permute composed as the
reference composes them; closed forms (constant inputs normalise to the
bias, identity projections, the gates at zero); and planted mistakes.
"""

from __future__ import annotations

import math

import numpy as np


def layer_norm(x: np.ndarray, weight, bias, eps: float) -> np.ndarray:
    """torch.nn.LayerNorm over the last axis: the mean, the biased variance,
    (x - mean) / sqrt(var + eps) * weight + bias."""

    x = np.asarray(x, dtype=np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * np.asarray(weight, np.float64) \
        + np.asarray(bias, np.float64)


def linear(x: np.ndarray, layer) -> np.ndarray:
    """nn.Linear: x @ weight.T + bias."""

    weight, bias = layer
    return np.asarray(x, np.float64) @ np.asarray(weight, np.float64).T \
        + np.asarray(bias, np.float64)


def softplus(x: np.ndarray) -> np.ndarray:
    """torch.nn.functional.softplus, beta 1, threshold 20: x above 20, else
    log1p(exp(x))."""

    x = np.asarray(x, np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def prepare(params: dict, tokens: np.ndarray) -> dict:
    """inference.py:459-519 without the routes, for tokens [B, 1, width]:
    the normalised tokens [B, 1, width]; read and write keys
    [B * H, 1, 2*sqrt(N)] (row b * H + h: the permute(0, 2, 1, 3) and
    flatten(0, 1) of the [B, 1, H, key] projections); values [B * H, D];
    input_gate and forget_log_gate [B * H]."""

    width, heads = params["width"], params["memory_heads"]
    key = 2 * math.isqrt(params["slots"])
    head_width = width // heads
    batch = tokens.shape[0]
    normalized = layer_norm(tokens, *params["input_norm"])
    x = normalized[:, 0]

    def per_bank(y: np.ndarray, inner: int) -> np.ndarray:
        # [B, H * inner] -> rows b * H + h
        return y.reshape(batch, heads, inner).reshape(batch * heads, inner)

    reads = per_bank(linear(x, params["read_projection"]), key)[:, None, :]
    writes = per_bank(linear(x, params["write_projection"]), key)[:, None, :]
    values = per_bank(linear(x, params["value_projection"]), head_width)
    forget = (-np.exp(np.asarray(params["A_log"], np.float64))
              * softplus(linear(x, params["forget_projection"])
                         + np.asarray(params["dt_bias"], np.float64))).reshape(-1)
    input_gate = sigmoid(linear(x, params["input_projection"])).reshape(-1)
    return {"normalized": normalized, "read_keys": reads, "write_keys": writes,
            "values": values, "input_gate": input_gate, "forget_log_gate": forget}


def finish(params: dict, normalized: np.ndarray, reading: np.ndarray) -> np.ndarray:
    """inference.py:522-535: readings [B * H, D] normalised per head,
    reshaped to [B, 1, width], times sigmoid(output_gate(normalized)),
    through output_projection."""

    batch = normalized.shape[0]
    width = params["width"]
    r = layer_norm(reading, *params["readings_norm"]).reshape(batch, 1, width)
    gate = sigmoid(linear(normalized, params["output_gate"]))
    return linear(gate * r, params["output_projection"])
