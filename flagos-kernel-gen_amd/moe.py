"""Python entry points of the W4A8 MoE path (PyTorch-ROCm tensors -> C ABI).

``w4a8_group_gemm_moe`` keeps the reference operator's name, argument order,
argument meaning, in-place ``out`` and return value (docs/Task1.md:8-17;
GPU entry Task1/v1.6/task1-codex5.5-all-v1.6.py:986-1030). Shape violations
the reference asserts (docs/Task1.md:74-75) raise ``W4A8ShapeError``, which
is both an ``AssertionError`` (as in the reference) and a ``ValueError``.

``moe_align_block_size`` and ``w4a8_fused_moe`` are the routed extension:
top-k routing ids/weights in, one bf16 row per token-expert pair out. They
have no reference counterpart.

There is no CPU or PyTorch fallback: every entry point runs the HIP kernels
of libmw4a8.so and raises if the library or a GPU tensor is missing.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


class W4A8ShapeError(ValueError, AssertionError):
    """Shape/stride/size violation (AssertionError in the reference)."""


_WORKSPACES: dict = {}


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _capturing(device: torch.device) -> bool:
    return torch.cuda.is_current_stream_capturing()


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-(device, stream) scratch buffer, grown on demand.

    Calls that share a stream are ordered, so they may share this buffer.
    Under HIP-graph capture a fresh buffer is taken from the graph's memory
    pool instead: the graph keeps its address, so a cached buffer that a
    later eager call replaced (and freed) must never be one a graph uses.
    """
    if _capturing(device):
        return torch.empty(max(nbytes, 4096), dtype=torch.uint8, device=device)
    key = (device.index, _stream(device))
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 4096), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = buf
    return buf


_ROUTING: dict = {}


def _routing_buffer(device: torch.device, stream: int, n_int32: int) -> torch.Tensor:
    """Per-(device, stream) int32 buffer for the routing metadata of
    ``w4a8_fused_moe`` calls without precomputed routing, grown on demand.

    A call's routing kernel writes it and the call's GEMM reads it; a later
    call on the same stream runs after both, so the calls may share it.
    Under HIP-graph capture the call gets a fresh buffer from the graph's
    pool (see ``_workspace``).
    """
    if _capturing(device):
        return torch.empty(max(n_int32, 1024), dtype=torch.int32, device=device)
    key = (device.index, stream)
    buf = _ROUTING.get(key)
    if buf is None or buf.numel() < n_int32:
        buf = torch.empty(max(n_int32, 1024), dtype=torch.int32, device=device)
        _ROUTING[key] = buf
    return buf


def _need(cond: bool, msg: str, exc=W4A8ShapeError):
    if not cond:
        raise exc(msg)


def _dtype(t: torch.Tensor, name: str, dtype: torch.dtype):
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def _on_gpu(tensors: dict) -> torch.device:
    dev = None
    for name, t in tensors.items():
        if not t.is_cuda:
            raise RuntimeError(f"{name} is on {t.device}; the W4A8 MoE kernels run on the GPU only "
                               "(no CPU fallback)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{name} is on {t.device}, expected {dev}")
    return dev


def _ptr(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


def _check_weights(w_q4_packed, w_scale, w_zero, K, group_size):
    E, N, K_half = w_q4_packed.shape
    _need(K_half * 2 == K, f"w_q4_packed last dim {K_half} != K/2 with K={K}")
    _need(group_size > 0 and K % group_size == 0, f"K={K} is not a multiple of group_size={group_size}")
    _need(group_size in (64, 128, 256), f"group_size={group_size} not supported (64, 128 or 256)")
    G = K // group_size
    _dtype(w_q4_packed, "w_q4_packed", torch.uint8)
    _dtype(w_scale, "w_scale", torch.float32)
    _dtype(w_zero, "w_zero", torch.int8)
    _need(tuple(w_scale.shape) == (E, N, G), f"w_scale shape {tuple(w_scale.shape)} != {(E, N, G)}")
    _need(tuple(w_zero.shape) == (E, N, G), f"w_zero shape {tuple(w_zero.shape)} != {(E, N, G)}")
    for name, t in (("w_q4_packed", w_q4_packed), ("w_scale", w_scale), ("w_zero", w_zero)):
        _need(t.is_contiguous(), f"{name} must be contiguous")
    return E, N, G


def _check_activations(x_q, x_scale, rows):
    _dtype(x_q, "x_q", torch.int8)
    _dtype(x_scale, "x_scale", torch.float32)
    _need(x_q.dim() == 2, "x_q must be 2-D [rows, K]")
    _need(x_q.stride(1) == 1, "x_q must have unit stride along K")
    _need(x_q.stride(0) % 16 == 0 and x_q.data_ptr() % 16 == 0,
          "x_q rows must start on 16-byte boundaries (row stride a multiple of 16)")
    _need(x_scale.dim() == 1 and x_scale.shape[0] == rows and x_scale.is_contiguous(),
          f"x_scale must be a contiguous [{rows}] vector")


def w4a8_group_gemm_moe(x_q: torch.Tensor, x_scale: torch.Tensor, w_q4_packed: torch.Tensor,
                        w_scale: torch.Tensor, w_zero: torch.Tensor, expert_offsets: torch.Tensor,
                        out: torch.Tensor, group_size: int) -> torch.Tensor:
    """W4A8 grouped GEMM over expert-grouped rows (drop-in for the reference op).

    ``out[m] = bf16(x_scale[m] * sum_g w_scale[e,:,g] * (x_q[m, g] . int8(w[e,:,g] - w_zero[e,:,g])))``
    for every row m in ``[expert_offsets[e], expert_offsets[e+1])``; other
    rows of ``out`` are left untouched. Returns ``out``.
    """
    M_total, K = x_q.shape
    _check_activations(x_q, x_scale, M_total)
    E, N, G = _check_weights(w_q4_packed, w_scale, w_zero, K, group_size)
    _dtype(expert_offsets, "expert_offsets", torch.int32)
    _dtype(out, "out", torch.bfloat16)
    _need(tuple(expert_offsets.shape) == (E + 1,) and expert_offsets.is_contiguous(),
          f"expert_offsets must be a contiguous [{E + 1}] vector")
    _need(out.dim() == 2 and tuple(out.shape) == (M_total, N), f"out shape {tuple(out.shape)} != {(M_total, N)}")
    _need(out.stride(1) == 1, "out must have unit stride along N")
    dev = _on_gpu(dict(x_q=x_q, x_scale=x_scale, w_q4_packed=w_q4_packed, w_scale=w_scale,
                       w_zero=w_zero, expert_offsets=expert_offsets, out=out))
    if M_total == 0:
        return out
    L = _lib.lib()
    nbytes = L.mw4a8_workspace_bytes(M_total, N, K, E, group_size)
    ws = _workspace(dev, nbytes)
    rc = L.mw4a8_grouped_gemm(_ptr(x_q), x_q.stride(0), _ptr(x_scale), _ptr(w_q4_packed), _ptr(w_scale),
                              _ptr(w_zero), _ptr(expert_offsets), _ptr(out), out.stride(0), M_total, N, K, E,
                              group_size, _ptr(ws), ws.numel(), ctypes.c_void_p(_stream(dev)))
    _lib.check(rc, "mw4a8_grouped_gemm")
    return out


def w4a8_group_partials(x_q, w_q4_packed, w_zero, expert_offsets, group_size):
    """Debug export: exact int32 per-group partials ``[M_total, N, G]`` (zeros for unowned rows)."""
    M_total, K = x_q.shape
    _dtype(x_q, "x_q", torch.int8)
    _need(x_q.stride(1) == 1 and x_q.stride(0) % 16 == 0, "x_q layout")
    E, N, K_half = w_q4_packed.shape
    _need(K_half * 2 == K and K % group_size == 0, "shape mismatch")
    G = K // group_size
    dev = _on_gpu(dict(x_q=x_q, w_q4_packed=w_q4_packed, w_zero=w_zero, expert_offsets=expert_offsets))
    out = torch.zeros(M_total, N, G, dtype=torch.int32, device=dev)
    if M_total == 0:
        return out
    L = _lib.lib()
    ws = _workspace(dev, L.mw4a8_workspace_bytes(M_total, N, K, E, group_size))
    rc = L.mw4a8_debug_partials(_ptr(x_q), x_q.stride(0), _ptr(w_q4_packed.contiguous()),
                                _ptr(w_zero.contiguous()), _ptr(expert_offsets), _ptr(out), M_total, N, K, E,
                                group_size, _ptr(ws), ws.numel(), ctypes.c_void_p(_stream(dev)))
    _lib.check(rc, "mw4a8_debug_partials")
    return out


def w4a8_fused_moe_partials(x_q, x_scale, w_q4_packed, w_scale, w_zero, topk_ids, topk_weights,
                            group_size: int = 128, block_m: int | None = None, weight_layout: str = "reference"):
    """Debug export of the routed GEMM: runs the same kernel body as
    ``w4a8_fused_moe`` and returns ``(out, partials)``, where ``partials
    [M*topk, N, G]`` int32 holds the exact group partial sums of every routed
    pair as its int32 MFMA chains computed them (zeros for unrouted pairs)."""
    _need(weight_layout in ("reference", "mfma"), f"unknown weight_layout {weight_layout!r}")
    M, K = x_q.shape
    _check_activations(x_q, x_scale, M)
    E, N, G = _check_weights(w_q4_packed, w_scale, w_zero, K, group_size)
    _dtype(topk_ids, "topk_ids", torch.int32)
    _dtype(topk_weights, "topk_weights", torch.float32)
    topk = topk_ids.shape[1]
    _need(topk_ids.is_contiguous() and tuple(topk_weights.shape) == (M, topk) and topk_weights.is_contiguous(),
          "topk_ids / topk_weights must be contiguous [M, topk]")
    dev = _on_gpu(dict(x_q=x_q, x_scale=x_scale, w_q4_packed=w_q4_packed, w_scale=w_scale, w_zero=w_zero,
                       topk_ids=topk_ids, topk_weights=topk_weights))
    P = M * topk
    if block_m is None:
        block_m = select_block_m(P, E, N, K, group_size)
    sorted_ids, expert_ids, num_post, _ = moe_align_block_size(topk_ids, block_m, E)
    out = torch.zeros(P, N, dtype=torch.bfloat16, device=dev)
    partials = torch.zeros(P, N, G, dtype=torch.int32, device=dev)
    rc = _lib.lib().mw4a8_debug_partials_routed(
        _ptr(x_q), x_q.stride(0), _ptr(x_scale), _ptr(w_q4_packed), _ptr(w_scale), _ptr(w_zero),
        _ptr(sorted_ids), _ptr(expert_ids), _ptr(num_post), _ptr(topk_weights), topk, _ptr(out), out.stride(0),
        _ptr(partials), M, N, K, E, group_size, block_m, 1 if weight_layout == "mfma" else 0,
        ctypes.c_void_p(_stream(dev)))
    _lib.check(rc, "mw4a8_debug_partials_routed")
    return out, partials


def align_buffer_sizes(num_pairs: int, num_experts: int, block_m: int):
    sl, bl = ctypes.c_int(), ctypes.c_int()
    _lib.check(_lib.lib().mw4a8_align_sizes(num_pairs, num_experts, block_m, ctypes.byref(sl), ctypes.byref(bl)),
               "mw4a8_align_sizes")
    return sl.value, bl.value


def select_block_m(num_pairs: int, num_experts: int, N: int, K: int, group_size: int) -> int:
    return int(_lib.lib().mw4a8_select_block_m(num_pairs, num_experts, N, K, group_size))


def moe_align_block_size(topk_ids: torch.Tensor, block_m: int, num_experts: int):
    """Routing metadata for ``topk_ids [M, topk]`` (int32, on the GPU).

    Returns ``(sorted_token_ids, expert_ids, num_tokens_post_padded [1], expert_offsets [E+1])``.
    """
    _dtype(topk_ids, "topk_ids", torch.int32)
    _need(topk_ids.is_contiguous(), "topk_ids must be contiguous")
    _need(num_experts <= 1024, "num_experts > 1024 is not supported", RuntimeError)
    dev = _on_gpu(dict(topk_ids=topk_ids))
    P = topk_ids.numel()
    sl, bl = align_buffer_sizes(P, num_experts, block_m)
    sorted_ids = torch.empty(sl, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(bl, dtype=torch.int32, device=dev)
    num_post = torch.empty(1, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    rc = _lib.lib().mw4a8_moe_align(_ptr(topk_ids), P, num_experts, block_m, _ptr(sorted_ids), _ptr(expert_ids),
                                    _ptr(num_post), _ptr(offsets), ctypes.c_void_p(_stream(dev)))
    _lib.check(rc, "mw4a8_moe_align")
    return sorted_ids, expert_ids, num_post, offsets


def w4a8_fused_moe(x_q: torch.Tensor, x_scale: torch.Tensor, w_q4_packed: torch.Tensor, w_scale: torch.Tensor,
                   w_zero: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor | None,
                   group_size: int = 128, out: torch.Tensor | None = None, block_m: int | None = None,
                   routing=None, weight_layout: str = "reference") -> torch.Tensor:
    """Routed W4A8 MoE GEMM: one bf16 row per token-expert pair.

    ``out[m * topk + j] = bf16((acc_e(x_q[m]) * x_scale[m]) * topk_weights[m, j])``
    with ``e = topk_ids[m, j]`` (``topk_weights=None``: weight 1, as for the
    up/gate GEMM of a MoE layer). ``routing`` may pass precomputed
    ``moe_align_block_size`` results for the same ``block_m``.
    ``weight_layout="mfma"`` takes weights converted by ``repack_weights``
    (bit-identical results).
    """
    _need(weight_layout in ("reference", "mfma"), f"unknown weight_layout {weight_layout!r}")
    M, K = x_q.shape
    _check_activations(x_q, x_scale, M)
    E, N, G = _check_weights(w_q4_packed, w_scale, w_zero, K, group_size)
    _dtype(topk_ids, "topk_ids", torch.int32)
    _need(topk_ids.dim() == 2 and topk_ids.shape[0] == M, f"topk_ids must be [{M}, topk]")
    topk = topk_ids.shape[1]
    tensors = dict(x_q=x_q, x_scale=x_scale, w_q4_packed=w_q4_packed, w_scale=w_scale, w_zero=w_zero,
                   topk_ids=topk_ids)
    if topk_weights is not None:
        _dtype(topk_weights, "topk_weights", torch.float32)
        _need(tuple(topk_weights.shape) == (M, topk) and topk_weights.is_contiguous(),
              f"topk_weights must be a contiguous [{M}, {topk}] tensor")
        tensors["topk_weights"] = topk_weights
    dev = _on_gpu(tensors)
    P = M * topk
    if out is None:
        out = torch.empty(P, N, dtype=torch.bfloat16, device=dev)
    else:
        _dtype(out, "out", torch.bfloat16)
        _need(tuple(out.shape) == (P, N) and out.stride(1) == 1, f"out must be [{P}, {N}] with unit inner stride")
        _on_gpu(dict(out=out))
    if P == 0:
        return out
    if block_m is None:
        block_m = select_block_m(P, E, N, K, group_size)
    if routing is not None:
        sl, bl = align_buffer_sizes(P, E, block_m)
        _need(routing[0].numel() == sl and routing[1].numel() == bl,
              f"routing buffers do not match block_m={block_m} (expected lengths {sl} and {bl})")
        _on_gpu(dict(sorted_ids=routing[0], expert_ids=routing[1], num_tokens_post_padded=routing[2]))
    L = _lib.lib()
    sid = _stream(dev)
    stream = ctypes.c_void_p(sid)
    if routing is None:
        # internal routing metadata: carved from the stream's cached int32
        # buffer (no allocation per call)
        sl, bl = align_buffer_sizes(P, E, block_m)
        rbuf = _routing_buffer(dev, sid, sl + bl + 1)   # held until both launches are enqueued
        base = rbuf.data_ptr()
        sorted_p, expert_p, num_post_p = base, base + 4 * sl, base + 4 * (sl + bl)
        ids = topk_ids if topk_ids.is_contiguous() else topk_ids.contiguous()
        _lib.check(L.mw4a8_moe_align(_ptr(ids), P, E, block_m, sorted_p, expert_p, num_post_p, None, stream),
                   "mw4a8_moe_align")
    else:
        sorted_p, expert_p, num_post_p = routing[0].data_ptr(), routing[1].data_ptr(), routing[2].data_ptr()
    entry = L.mw4a8_fused_moe if weight_layout == "reference" else L.mw4a8_fused_moe_repacked
    rc = entry(_ptr(x_q), x_q.stride(0), _ptr(x_scale), _ptr(w_q4_packed), _ptr(w_scale),
               _ptr(w_zero), sorted_p, expert_p, num_post_p,
               _ptr(topk_weights) if topk_weights is not None else None, topk, _ptr(out),
               out.stride(0), M, N, K, E, group_size, block_m, stream)
    _lib.check(rc, "mw4a8_fused_moe")
    return out


def repack_weights(w_q4_packed: torch.Tensor, inverse: bool = False) -> torch.Tensor:
    """Convert ``[E, N, K/2]`` uint8 int4 weights between the reference packing
    (docs/Task1.md:78-81) and the MFMA order ``w4a8_fused_moe(...,
    weight_layout="mfma")`` reads (``inverse=True``: back). Returns a new
    tensor; the round trip is bit-exact."""
    _dtype(w_q4_packed, "w_q4_packed", torch.uint8)
    _need(w_q4_packed.dim() == 3 and w_q4_packed.is_contiguous(), "w_q4_packed must be a contiguous [E, N, K/2]")
    E, N, K_half = w_q4_packed.shape
    dev = _on_gpu(dict(w_q4_packed=w_q4_packed))
    out = torch.empty_like(w_q4_packed)
    rc = _lib.lib().mw4a8_repack_weights(_ptr(w_q4_packed), _ptr(out), E, N, 2 * K_half, 1 if inverse else 0,
                                         ctypes.c_void_p(_stream(dev)))
    _lib.check(rc, "mw4a8_repack_weights")
    return out
