"""Independent brute-force computations that pin the oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

These deliberately take a different route from ``task1_ref``: nibbles are
extracted per element with integer shifts, the zero fold uses modular
arithmetic instead of an int16 -> int8 cast, partial sums are int64 numpy
contractions, and the scale reduction runs in float64. Small inputs only.
"""

from __future__ import annotations

import numpy as np


def signed_weights_i64(w_q4_packed, w_zero, group_size):
    """int64 [..., N, K]: ((nibble - zero + 128) mod 256) - 128."""
    b = np.asarray(w_q4_packed, dtype=np.int64)
    K = b.shape[-1] * 2
    k = np.arange(K)
    byte = b[..., k // 2]
    nib = np.where(k % 2 == 1, byte // 16, byte % 16)
    z = np.asarray(w_zero, dtype=np.int64)[..., k // group_size]
    return (nib - z + 128) % 256 - 128


def partials_i64(x_rows, w_signed_n_k, group_size):
    """int64 [rows, N, G] group partial sums by explicit contraction."""
    x = np.asarray(x_rows, dtype=np.int64)
    rows, K = x.shape
    N = w_signed_n_k.shape[0]
    G = K // group_size
    xg = x.reshape(rows, G, group_size)
    wg = w_signed_n_k.reshape(N, G, group_size)
    return np.einsum("mgk,ngk->mng", xg, wg)


def grouped_gemm_f64(x_q, x_scale, w_q4_packed, w_scale, w_zero, expert_offsets, group_size):
    """float64 outputs and int64 partials for the reference-layout operator.

    Returns ``(out_f64 [M, N], owned [M] bool, partials [M, N, G] int64)``.
    Rows owned by no expert are NaN in ``out_f64`` and zero in ``partials``.
    """
    x = np.asarray(x_q, dtype=np.int64)
    M, K = x.shape
    E, N, _ = np.asarray(w_q4_packed).shape
    G = K // group_size
    out = np.full((M, N), np.nan)
    P = np.zeros((M, N, G), dtype=np.int64)
    owned = np.zeros(M, dtype=bool)
    offs = [int(v) for v in np.asarray(expert_offsets)]
    ws = np.asarray(w_scale, dtype=np.float64)
    xs = np.asarray(x_scale, dtype=np.float64)
    for e in range(E):
        m0, m1 = max(offs[e], 0), min(offs[e + 1], M)
        if m1 <= m0:
            continue
        w = signed_weights_i64(np.asarray(w_q4_packed)[e], np.asarray(w_zero)[e], group_size)
        pe = partials_i64(x[m0:m1], w, group_size)
        P[m0:m1] = pe
        out[m0:m1] = (pe * ws[e][None]).sum(-1) * xs[m0:m1, None]
        owned[m0:m1] = True
    return out, owned, P


def align_loops(topk_ids, num_experts, block_m):
    """Pure-Python loops for the routing metadata (tiny inputs)."""
    ids = [int(v) for v in np.asarray(topk_ids).reshape(-1)]
    P = len(ids)
    E, BM = num_experts, block_m
    sorted_ids, expert_ids, offsets = [], [], [0]
    for e in range(E):
        mine = [i for i in range(P) if ids[i] == e]
        offsets.append(offsets[-1] + len(mine))
        if not mine:
            continue
        nb = (len(mine) + BM - 1) // BM
        sorted_ids += mine + [P] * (nb * BM - len(mine))
        expert_ids += [e] * nb
    num_post = len(sorted_ids)
    total = P + E * (BM - 1)
    sorted_ids += [P] * (total - len(sorted_ids))
    nblocks = (total + BM - 1) // BM
    expert_ids += [-1] * (nblocks - len(expert_ids))
    return sorted_ids, expert_ids, num_post, offsets


def fused_loops(x_q, x_scale, w_q4_packed, w_scale, w_zero, topk_ids, topk_weights, group_size):
    """Routed output in float64 by per-pair loops over experts (tiny inputs)."""
    x = np.asarray(x_q, dtype=np.int64)
    M, K = x.shape
    ids = np.asarray(topk_ids).reshape(M, -1)
    tw = np.asarray(topk_weights, dtype=np.float64).reshape(M, -1)
    topk = ids.shape[1]
    E, N, _ = np.asarray(w_q4_packed).shape
    out = np.full((M * topk, N), np.nan)
    ws = np.asarray(w_scale, dtype=np.float64)
    xs = np.asarray(x_scale, dtype=np.float64)
    for m in range(M):
        for j in range(topk):
            e = int(ids[m, j])
            if not 0 <= e < E:
                continue
            w = signed_weights_i64(np.asarray(w_q4_packed)[e], np.asarray(w_zero)[e], group_size)
            p = partials_i64(x[m:m + 1], w, group_size)[0]
            out[m * topk + j] = (p * ws[e]).sum(-1) * xs[m] * tw[m, j]
    return out
