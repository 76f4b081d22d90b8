"""CPU restatement of the MoE-layer steps around the grouped GEMM.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference operator (docs/Task1.md:8-17) starts from int8 activations
with per-token scales and ends at per-row bf16 outputs; it has no router,
activation quantizer, gated activation or combine. These functions define
the steps this build adds on either side, in plain float32 torch / numpy so
that the bit-level choices are explicit:

``quant_per_token_ref``  per-token symmetric int8: ``scale = max(amax, 1e-12)
                         / 127``, ``q = clamp(round_half_even(x / scale), -127,
                         127)`` in float32. The reference's own int8 quantizer
                         (docs/Task3.md:55-66) works per 128-column group and
                         truncates; the GEMM here consumes one scale per token,
                         so the scale is per row and the rounding is to
                         nearest-even. Pinned by hand-worked ties and a Python
                         brute force.
``router_topk_ref``      top-k of the logits (ties: lower index first) and
                         weights ``exp(l - l_max)`` normalised over the chosen k
                         or over all E, in float64. Equal (mathematically) to
                         softmax -> top-k -> renormalise. Pinned by brute-force
                         sorting and closed-form weights.
``silu_mul_quant_ref``   ``y = (g * sigmoid(g)) * u`` in float32 with torch's
                         sigmoid, the forward order of docs/Task3.md:103-110,
                         then ``quant_per_token_ref`` on y. Pinned against
                         float64 math.
``combine_ref``          ``out[m] = bf16(sum_j w[m,j] * y[m*topk + j])`` with
                         float32 product and sum in j order. Pinned by loops.
``moe_layer_ref``        the composition (with ``task1_ref.fused_moe_ref`` for
                         both GEMMs).
"""

from __future__ import annotations

import numpy as np
import torch

from . import task1_ref


def quant_per_token_ref(x: torch.Tensor):
    """``x [M, K]`` (bf16 or fp32) -> ``(q int8 [M, K], scale fp32 [M])``."""
    xf = x.to(torch.float32)
    amax = xf.abs().amax(dim=1).clamp_min(1e-12)
    scale = amax / 127.0
    q = torch.round(xf / scale[:, None]).clamp_(-127, 127).to(torch.int8)
    return q, scale


def router_topk_ref(logits, topk: int, renormalize: bool = True):
    """``logits [M, E]`` fp32 -> ``(ids int32 [M, topk], weights float64 [M, topk])``."""
    lg = np.asarray(logits, dtype=np.float32)
    M, E = lg.shape
    idx = np.arange(E)
    ids = np.zeros((M, topk), dtype=np.int32)
    w = np.zeros((M, topk), dtype=np.float64)
    for m in range(M):
        order = np.lexsort((idx, -lg[m].astype(np.float64)))[:topk]
        ids[m] = order
        top = float(lg[m, order[0]])
        num = np.exp(lg[m, order].astype(np.float64) - top)
        den = num.sum() if renormalize else np.exp(lg[m].astype(np.float64) - top).sum()
        w[m] = num / den
    return ids, w


def silu_mul_y(h: torch.Tensor) -> torch.Tensor:
    """float32 ``y = (g * sigmoid(g)) * u`` of ``h = [gate | up]`` (docs/Task3.md:103-110)."""
    I = h.shape[1] // 2
    g = h[:, :I].to(torch.float32)
    u = h[:, I:].to(torch.float32)
    return (g * torch.sigmoid(g)) * u


def silu_mul_quant_ref(h: torch.Tensor):
    """``h [P, 2I]`` bf16 -> ``(q int8 [P, I], scale fp32 [P])``."""
    return quant_per_token_ref(silu_mul_y(h))


def combine_ref(y: torch.Tensor, topk: int, weights=None) -> torch.Tensor:
    """``y [M*topk, N]`` bf16 -> ``out [M, N]`` bf16 (float32, j order)."""
    yf = y.to(torch.float32).numpy()
    P, N = yf.shape
    M = P // topk
    acc = np.zeros((M, N), dtype=np.float32)
    wt = None if weights is None else np.asarray(weights, dtype=np.float32).reshape(M, topk)
    for j in range(topk):
        rows = yf[j::topk]
        acc = acc + (rows if wt is None else (wt[:, j:j + 1] * rows).astype(np.float32))
    return torch.from_numpy(acc).to(torch.bfloat16)


def moe_layer_ref(x, router_logits, w13_q4, w13_scale, w13_zero, w2_q4, w2_scale, w2_zero, topk,
                  group_size=128, renormalize=True):
    """One MoE layer, composed of the steps above and ``task1_ref.fused_moe_ref``."""
    M, H = x.shape
    x_q, x_scale = quant_per_token_ref(x)
    ids, w = router_topk_ref(router_logits, topk, renormalize)
    ids_t = torch.from_numpy(ids)
    w_t = torch.from_numpy(w.astype(np.float32))
    ones = torch.ones(M, topk, dtype=torch.float32)
    h = task1_ref.fused_moe_ref(x_q, x_scale, w13_q4, w13_scale, w13_zero, ids_t, ones, group_size)
    h_q, h_scale = silu_mul_quant_ref(h)
    P = M * topk
    y = task1_ref.fused_moe_ref(h_q, h_scale, w2_q4, w2_scale, w2_zero, ids_t.reshape(P, 1),
                                w_t.reshape(P, 1), group_size)
    return combine_ref(y, topk), dict(x_q=x_q, x_scale=x_scale, ids=ids, w=w, h=h, h_q=h_q, h_scale=h_scale, y=y)
