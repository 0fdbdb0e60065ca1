"""Product-key route selection on the device (copy_on_write_sdm/sdm.py:96-159).

``product_key_routes`` keeps the reference's name, arguments, return values
and argument errors; the selection runs in ``cowsdm_product_key_routes``
(csrc/routes.hip), one wave per route row.  The reference calls it twice per
decode step and layer, for the read and the write routes
(inference.py:479-488), on ``[banks, 1, 2*sqrt(N)]`` projections.
"""

from __future__ import annotations

import math

import torch

from . import _native as nat


def product_key_routes(projected: torch.Tensor, *, slots: int, selected: int,
                       out: tuple[torch.Tensor, torch.Tensor] | None = None
                       ) -> tuple[torch.Tensor, torch.Tensor]:
    """Top ``selected`` product keys of each row and the softmax of their scores.

    ``projected`` is ``[B, T, 2*sqrt(N)]``; returns ``(weights, indices)`` of
    shape ``[B, T, K]`` with ``K = min(selected, min(selected, sqrt(N))**2)``,
    indices int64 ascending along the last dimension (sdm.py:96-159).  The HIP
    path takes float32 CUDA tensors with finite scores; equal scores are
    selected lowest position first.  ``out`` (not in the reference): the
    contiguous float32 weights and int64 indices to write, so that a
    captured graph keeps its buffers.
    """

    if projected.ndim != 3:
        raise ValueError("product-key projection must be [B,T,2*sqrt(N)]")
    root = math.isqrt(slots)
    if root * root != slots or projected.shape[-1] != 2 * root:
        raise ValueError("slot count and product-key projection do not match")
    if not 1 <= selected <= slots:
        raise ValueError("selected product keys must be between one and slots")
    if projected.device.type != "cuda":
        raise ValueError("product_key_routes runs on the HIP device only (no CPU path)")
    if projected.dtype != torch.float32:
        raise TypeError("product_key_routes takes float32 projections on the HIP path")
    sub = min(selected, root)
    final = min(selected, sub * sub)
    batch, steps = projected.shape[:2]
    source = projected.contiguous()
    if out is None:
        weights = torch.empty((batch, steps, final), dtype=torch.float32, device=projected.device)
        indices = torch.empty((batch, steps, final), dtype=torch.int64, device=projected.device)
    else:
        weights, indices = out
        if (weights.shape != (batch, steps, final) or indices.shape != (batch, steps, final)
                or weights.dtype != torch.float32 or indices.dtype != torch.int64
                or not weights.is_contiguous() or not indices.is_contiguous()
                or weights.device != projected.device or indices.device != projected.device):
            raise ValueError("product-key route outputs must be contiguous float32 weights and "
                             "int64 indices of shape [B,T,K] on the projection's device")
    rc = nat.lib().cowsdm_product_key_routes(
        source.data_ptr(), batch * steps, slots, selected, weights.data_ptr(),
        indices.data_ptr(), nat.stream_handle(projected.device))
    nat.check(rc, "cowsdm_product_key_routes")
    return weights, indices
