"""The MoE layer around the W4A8 grouped GEMM (PyTorch-ROCm tensors -> C ABI).

The reference operator (docs/Task1.md:8-17) starts from quantized
activations and CSR expert offsets and ends at per-row bf16 outputs. These
entry points supply the steps on either side, each a HIP kernel of
libmw4a8.so with no CPU fallback:

* ``quant_per_token``   bf16 activations -> int8 + per-token fp32 scale
* ``router_topk``       router logits -> top-k expert ids + weights
* ``silu_mul_quant``    up/gate GEMM output [gate | up] -> int8 silu(gate)*up
                        + per-row scale (forward half of docs/Task3.md:103-110)
* ``combine_topk``      per-pair rows -> per-token weighted sum
* ``w4a8_moe_layer``    the chain: quant -> router -> up/gate GEMM ->
                        silu*up requant -> down GEMM (top-k weights in its
                        epilogue) -> combine
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .moe import W4A8ShapeError, _dtype, _need, _on_gpu, _ptr, _stream, moe_align_block_size, select_block_m, \
    w4a8_fused_moe


def _rows_ok(t: torch.Tensor, name: str):
    _need(t.dim() == 2 and t.stride(1) == 1, f"{name} must be 2-D with unit inner stride")


def quant_per_token(x: torch.Tensor, out_q: torch.Tensor | None = None, out_scale: torch.Tensor | None = None):
    """bf16 ``x [M, K]`` -> ``(x_q int8 [M, K], x_scale fp32 [M])``.

    ``x_scale = max(amax_k |x|, 1e-12) / 127``,
    ``x_q = clamp(round_half_even(x / x_scale), -127, 127)`` in fp32.
    """
    _dtype(x, "x", torch.bfloat16)
    _rows_ok(x, "x")
    M, K = x.shape
    dev = _on_gpu(dict(x=x))
    q = out_q if out_q is not None else torch.empty(M, K, dtype=torch.int8, device=dev)
    s = out_scale if out_scale is not None else torch.empty(M, dtype=torch.float32, device=dev)
    _need(tuple(q.shape) == (M, K) and q.dtype == torch.int8 and q.stride(1) == 1, "x_q must be int8 [M, K]")
    _need(tuple(s.shape) == (M,) and s.dtype == torch.float32 and s.is_contiguous(), "x_scale must be fp32 [M]")
    rc = _lib.lib().mw4a8_quant_rows(_ptr(x), x.stride(0), M, K, _ptr(q), q.stride(0), _ptr(s),
                                     ctypes.c_void_p(_stream(dev)))
    _lib.check(rc, "mw4a8_quant_rows")
    return q, s


def router_topk(logits: torch.Tensor, topk: int, renormalize: bool = True):
    """fp32 ``logits [M, E]`` -> ``(topk_ids int32 [M, topk], topk_weights fp32 [M, topk])``.

    The ``topk`` largest logits (ties: lower expert index first), in
    descending order; weights ``exp(l - l_max)`` normalised over the chosen
    ``topk`` (``renormalize``) or over all E (plain softmax probabilities).
    """
    _dtype(logits, "logits", torch.float32)
    _rows_ok(logits, "logits")
    M, E = logits.shape
    _need(0 < topk <= min(E, 64) and E <= 1024, f"router supports E <= 1024 and 0 < topk <= min(E, 64)")
    dev = _on_gpu(dict(logits=logits))
    ids = torch.empty(M, topk, dtype=torch.int32, device=dev)
    w = torch.empty(M, topk, dtype=torch.float32, device=dev)
    rc = _lib.lib().mw4a8_router_topk(_ptr(logits), logits.stride(0), M, E, topk, 1 if renormalize else 0,
                                      _ptr(ids), _ptr(w), ctypes.c_void_p(_stream(dev)))
    _lib.check(rc, "mw4a8_router_topk")
    return ids, w


def silu_mul_quant(h: torch.Tensor):
    """bf16 ``h [P, 2I]`` = [gate | up] -> ``(q int8 [P, I], scale fp32 [P])`` of
    ``y = silu(gate) * up`` (fp32, docs/Task3.md:103-110 order), per-row int8."""
    _dtype(h, "h", torch.bfloat16)
    _rows_ok(h, "h")
    P, two_i = h.shape
    _need(two_i % 2 == 0, "h must hold [gate | up] halves")
    I = two_i // 2
    dev = _on_gpu(dict(h=h))
    q = torch.empty(P, I, dtype=torch.int8, device=dev)
    s = torch.empty(P, dtype=torch.float32, device=dev)
    rc = _lib.lib().mw4a8_silu_mul_quant(_ptr(h), h.stride(0), P, I, _ptr(q), q.stride(0), _ptr(s),
                                         ctypes.c_void_p(_stream(dev)))
    _lib.check(rc, "mw4a8_silu_mul_quant")
    return q, s


def combine_topk(y: torch.Tensor, topk: int, topk_weights: torch.Tensor | None = None,
                 out: torch.Tensor | None = None):
    """bf16 ``y [M*topk, N]`` -> bf16 ``out [M, N]`` with
    ``out[m] = sum_j w[m, j] * y[m*topk + j]`` (fp32, j order; w = 1 if None)."""
    _dtype(y, "y", torch.bfloat16)
    _rows_ok(y, "y")
    P, N = y.shape
    _need(topk > 0 and P % topk == 0, f"rows {P} not a multiple of topk={topk}")
    M = P // topk
    tensors = dict(y=y)
    if topk_weights is not None:
        _dtype(topk_weights, "topk_weights", torch.float32)
        _need(tuple(topk_weights.shape) == (M, topk) and topk_weights.is_contiguous(),
              f"topk_weights must be a contiguous [{M}, {topk}] tensor")
        tensors["topk_weights"] = topk_weights
    dev = _on_gpu(tensors)
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    _need(tuple(out.shape) == (M, N) and out.dtype == torch.bfloat16 and out.stride(1) == 1,
          f"out must be bf16 [{M}, {N}]")
    rc = _lib.lib().mw4a8_combine_topk(_ptr(y), y.stride(0), M, topk, N,
                                       _ptr(topk_weights) if topk_weights is not None else None, _ptr(out),
                                       out.stride(0), ctypes.c_void_p(_stream(dev)))
    _lib.check(rc, "mw4a8_combine_topk")
    return out


def w4a8_moe_layer(x: torch.Tensor, router_logits: torch.Tensor, w13_q4: torch.Tensor, w13_scale: torch.Tensor,
                   w13_zero: torch.Tensor, w2_q4: torch.Tensor, w2_scale: torch.Tensor, w2_zero: torch.Tensor,
                   topk: int, group_size: int = 128, renormalize: bool = True, return_intermediates: bool = False,
                   weight_layout: str = "reference"):
    """One W4A8 MoE layer: ``x [M, H]`` bf16 -> ``out [M, H]`` bf16.

    ``w13_*`` hold the up/gate projection ``[E, 2I, H/2]`` (rows ``[0, I)``
    gate, ``[I, 2I)`` up), ``w2_*`` the down projection ``[E, H, I/2]``, both
    in the reference's packed int4 / group-scale / zero-point format
    (docs/Task1.md:8-26), or both converted by ``repack_weights`` with
    ``weight_layout="mfma"``. Steps (each a HIP kernel):

    1. ``x_q, x_scale = quant_per_token(x)``
    2. ``ids, w = router_topk(router_logits, topk, renormalize)``
    3. ``h = up/gate GEMM`` per pair (weight 1)              -> ``[M*topk, 2I]``
    4. ``h_q, h_scale = silu_mul_quant(h)``                  -> ``[M*topk, I]``
    5. ``y = down GEMM`` per pair, times ``w`` in its epilogue -> ``[M*topk, H]``
    6. ``out = combine_topk(y, topk)``
    """
    _dtype(x, "x", torch.bfloat16)
    M, H = x.shape
    E, two_i, h_half = w13_q4.shape
    _need(h_half * 2 == H, f"w13 last dim {h_half} != H/2 with H={H}")
    I = two_i // 2
    _need(tuple(w2_q4.shape) == (E, H, I // 2), f"w2_q4 must be [{E}, {H}, {I // 2}]")
    _need(tuple(router_logits.shape) == (M, E), f"router_logits must be [{M}, {E}]")
    x_q, x_scale = quant_per_token(x)
    ids, w = router_topk(router_logits, topk, renormalize)
    P = M * topk
    bm_up = select_block_m(P, E, two_i, H, group_size)
    routing_up = moe_align_block_size(ids, bm_up, E)
    h = w4a8_fused_moe(x_q, x_scale, w13_q4, w13_scale, w13_zero, ids, None, group_size=group_size,
                       block_m=bm_up, routing=routing_up, weight_layout=weight_layout)
    h_q, h_scale = silu_mul_quant(h)
    # the down GEMM treats every pair as a token routed to one expert: the
    # pair order and expert of row p are those of the up/gate GEMM
    ids_p = ids.view(P, 1)
    bm_down = select_block_m(P, E, H, I, group_size)
    routing_down = routing_up if bm_down == bm_up else moe_align_block_size(ids_p, bm_down, E)
    y = w4a8_fused_moe(h_q, h_scale, w2_q4, w2_scale, w2_zero, ids_p, w.view(P, 1), group_size=group_size,
                       block_m=bm_down, routing=routing_down, weight_layout=weight_layout)
    out = combine_topk(y, topk)
    if return_intermediates:
        return out, dict(x_q=x_q, x_scale=x_scale, topk_ids=ids, topk_weights=w, h=h, h_q=h_q, h_scale=h_scale,
                         y=y)
    return out
