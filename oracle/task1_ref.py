"""Torch-on-CPU restatement of the reference W4A8 grouped-GEMM MoE operator.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows docs/Task1.md:53-114 of the reference step by step:

=====================  ==========================  =============================
step                   reference lines             function here
=====================  ==========================  =============================
shape checks           docs/Task1.md:72-76         ``_check_shapes``
INT4 unpack            docs/Task1.md:78-81         ``unpack_int4``
zero-point fold        docs/Task1.md:83-85         ``fold_zero``
expert loop, skip      docs/Task1.md:87-92         ``w4a8_group_gemm_moe_ref``
per-group partials     docs/Task1.md:99-104        ``group_partials``
group-scale reduce     docs/Task1.md:106-107       ``_finish_rows``
token scale + bf16     docs/Task1.md:109-112       ``_finish_rows``
=====================  ==========================  =============================

Pinning (checked in tests/test_oracle_cpu.py):

* ``unpack_int4`` -- exhaustive over all 256 byte values against the closed
  form ``u[2p] = b & 15, u[2p+1] = b >> 4`` and a hand-worked byte.
* ``fold_zero`` -- exhaustive 16 x 256 (nibble, zero) table against the
  closed form ``((u - z) + 128) mod 256 - 128`` including the wrap regime.
* ``group_partials`` -- bit-exact against the int64 brute force in
  ``oracle/brute.py`` (values are integers below 2**24, so the fp32 matmul
  here is exact) and against one-hot activations, which select single
  weights and so pin the nibble order and the group index of the zero point.
* ``w4a8_group_gemm_moe_ref`` -- against a float64 brute force within bf16
  rounding, against the closed form ``out = bf16(x_scale * (x @ w.T))`` when
  all group scales are 1, and against the untouched-row rule for empty
  experts and ``offsets[0] != 0``.
* ``fused_moe_ref`` (routed extension, no reference counterpart) -- against
  ``w4a8_group_gemm_moe_ref`` applied to the gathered rows and then the
  top-k weight, and against a pure-Python loop on tiny inputs.

The fp32 summation order of the reference's ``einsum``/``sum`` calls is
internal to torch and is not pinned bit for bit; the product path is checked
against this oracle within a tolerance for the bf16 output.
"""

from __future__ import annotations

import torch


def _check_shapes(x_q, w_q4_packed, group_size):
    """Shape rules of docs/Task1.md:72-76 (raised as AssertionError there)."""
    M_total, K = x_q.shape
    E, N, K_half = w_q4_packed.shape
    assert K_half * 2 == K, "w_q4_packed last dim must be K/2"
    assert K % group_size == 0, "K must be a multiple of group_size"
    return M_total, K, E, N, K // group_size


def unpack_int4(w_q4_packed: torch.Tensor) -> torch.Tensor:
    """Nibbles -> int16 values in [0, 15] (docs/Task1.md:78-81).

    Byte ``p`` of a row holds k = 2p in its low nibble and k = 2p+1 in its
    high nibble; the result has the packed axis expanded to K.
    """
    b = w_q4_packed.to(torch.int16)
    even_k = b & 0x0F
    odd_k = (b >> 4) & 0x0F
    out = torch.empty(*b.shape[:-1], b.shape[-1] * 2, dtype=torch.int16)
    out[..., 0::2] = even_k
    out[..., 1::2] = odd_k
    return out


def fold_zero(u: torch.Tensor, w_zero: torch.Tensor, group_size: int) -> torch.Tensor:
    """int8(int16(u) - int16(z)) with z broadcast over each K-group.

    docs/Task1.md:83-85. The int16 -> int8 cast wraps modulo 256, which only
    matters when ``u - z > 127`` (zero points at or below -113).
    """
    z = w_zero.to(torch.int16).repeat_interleave(group_size, dim=-1)
    return (u - z).to(torch.int8)


def group_partials(xq_rows: torch.Tensor, w_signed: torch.Tensor, group_size: int) -> torch.Tensor:
    """P[m, n, g] = sum_{k in group g} x[m, k] * w[n, k], as fp32.

    docs/Task1.md:99-104 (the ``"mgk,ngk->mng"`` einsum). Every term is an
    integer with |P| <= 128 * 128 * group_size < 2**24, so fp32 holds it
    exactly and the result does not depend on summation order.
    """
    rows, K = xq_rows.shape
    N = w_signed.shape[0]
    G = K // group_size
    xg = xq_rows.reshape(rows, G, group_size).to(torch.float32).permute(1, 0, 2)   # [G, rows, gs]
    wg = w_signed.reshape(N, G, group_size).to(torch.float32).permute(1, 2, 0)     # [G, gs, N]
    return torch.bmm(xg, wg).permute(1, 2, 0).contiguous()                         # [rows, N, G]


def _finish_rows(partial, ws_e, xs_rows, row_weight=None):
    """Group-scale reduce, token scale, optional routing weight, bf16.

    docs/Task1.md:106-112: ``(partial * ws).sum(-1)``, then ``* x_scale``,
    then ``.to(bfloat16)``. ``row_weight`` (routed extension) multiplies the
    fp32 value after the token scale, before rounding.
    """
    acc = (partial * ws_e.unsqueeze(0)).sum(dim=-1)
    acc = acc * xs_rows.unsqueeze(-1)
    if row_weight is not None:
        acc = acc * row_weight.unsqueeze(-1)
    return acc.to(torch.bfloat16)


def _expert_weights(w_q4_packed, w_zero, e, group_size, unpacked=None):
    if unpacked is not None:
        return unpacked[e]
    return fold_zero(unpack_int4(w_q4_packed[e]), w_zero[e], group_size)


def w4a8_group_gemm_moe_ref(x_q, x_scale, w_q4_packed, w_scale, w_zero,
                            expert_offsets, out, group_size, unpack="per_expert"):
    """Reference-layout operator on CPU tensors (docs/Task1.md:53-114).

    Rows ``[off[e], off[e+1])`` of ``x_q`` belong to expert ``e``; experts with
    ``off[e+1] <= off[e]`` are skipped and rows outside every range keep the
    contents of ``out``. Python slicing clamps ranges to ``[0, M_total]``.

    ``unpack="all"`` unpacks every expert before the loop, as the reference
    does (docs/Task1.md:78-85); ``"per_expert"`` unpacks inside the loop and
    gives bitwise-identical output with far less memory.
    """
    M_total, K, E, N, G = _check_shapes(x_q, w_q4_packed, group_size)
    all_w = None
    if unpack == "all":
        all_w = fold_zero(unpack_int4(w_q4_packed), w_zero, group_size)
    offs = [int(v) for v in expert_offsets.tolist()]
    for e in range(E):
        m0, m1 = offs[e], offs[e + 1]
        if m1 <= m0:
            continue
        xq_e = x_q[m0:m1]
        if xq_e.shape[0] == 0:
            continue
        w_e = _expert_weights(w_q4_packed, w_zero, e, group_size, all_w)
        partial = group_partials(xq_e, w_e, group_size)
        out[m0:m1].copy_(_finish_rows(partial, w_scale[e], x_scale[m0:m1]))
    return out


def expert_rows_ref(xq_rows, xs_rows, w_q4_e, ws_e, wz_e, group_size, row_weight=None):
    """Output rows ``[rows, N]`` bf16 of one expert (docs/Task1.md:94-112).

    ``w_q4_e``/``ws_e``/``wz_e`` are that expert's ``[N, ...]`` slices;
    ``row_weight`` is the routed extension's per-row top-k weight.
    """
    w_e = fold_zero(unpack_int4(w_q4_e), wz_e, group_size)
    partial = group_partials(xq_rows, w_e, group_size)
    return _finish_rows(partial, ws_e, xs_rows, row_weight)


def group_partials_ref(x_q, w_q4_packed, w_zero, expert_offsets, group_size):
    """Exact int32 partials ``P[m, n, g]`` for every row owned by an expert.

    Rows owned by no expert are zero. Used to check the product path's
    debug export of its int32 group accumulators.
    """
    M_total, K, E, N, G = _check_shapes(x_q, w_q4_packed, group_size)
    P = torch.zeros(M_total, N, G, dtype=torch.int32)
    offs = [int(v) for v in expert_offsets.tolist()]
    for e in range(E):
        m0, m1 = max(offs[e], 0), min(offs[e + 1], M_total)
        if m1 <= m0:
            continue
        w_e = _expert_weights(w_q4_packed, w_zero, e, group_size)
        P[m0:m1] = group_partials(x_q[m0:m1], w_e, group_size).to(torch.int32)
    return P


def fused_moe_ref(x_q, x_scale, w_q4_packed, w_scale, w_zero, topk_ids,
                  topk_weights, group_size, out=None, pairs=None):
    """Routed extension: one output row per token-expert pair.

    No reference counterpart. Pair ``i = m * topk + j`` routes token ``m`` to
    expert ``topk_ids[m, j]``; its row is

        out[i, :] = bf16((acc_e(x_q[m]) * x_scale[m]) * topk_weights[m, j])

    where ``acc_e`` is the docs/Task1.md:99-107 reduction for expert e. Pairs
    whose expert id is outside ``[0, E)`` are not routed and keep the
    contents of ``out``. ``pairs`` restricts the computation to a subset of
    pair indices (used to check full-size runs on sampled rows).
    """
    M, K = x_q.shape
    E, N, _ = w_q4_packed.shape
    topk = topk_ids.shape[1]
    _check_shapes(x_q, w_q4_packed, group_size)
    if out is None:
        out = torch.zeros(M * topk, N, dtype=torch.bfloat16)
    ids = topk_ids.reshape(-1).to(torch.int64)
    tw = topk_weights.reshape(-1).to(torch.float32)
    sel = torch.arange(M * topk) if pairs is None else torch.as_tensor(pairs, dtype=torch.int64)
    for e in range(E):
        pe = sel[ids[sel] == e]
        if pe.numel() == 0:
            continue
        tok = pe // topk
        w_e = _expert_weights(w_q4_packed, w_zero, e, group_size)
        partial = group_partials(x_q[tok], w_e, group_size)
        out[pe] = _finish_rows(partial, w_scale[e], x_scale[tok], tw[pe])
    return out
