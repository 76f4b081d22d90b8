"""Closed form of the moe_align_block_size routing metadata (numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference has no routing step: its operator receives rows already grouped
by expert plus CSR ``expert_offsets [E+1]`` (docs/Task1.md:8-17, consumed at
docs/Task1.md:87-92). The routed entry of this build defines the metadata
below; with ``block_m = 1`` its unpadded offsets are exactly the reference's
``expert_offsets`` for rows laid out in ``sorted_token_ids`` order.

Definitions (pairs ``i = m * topk + j`` over the flattened ``topk_ids``):

* ``cnt[e]``                 number of pairs routed to expert e; ids outside
                             ``[0, E)`` are not routed.
* ``block_off[e]``           exclusive prefix sum of ``ceil(cnt[e] / BM)``.
* ``sorted_token_ids``       length ``P + E * (BM - 1)``; slot
                             ``BM * block_off[e] + r`` holds the r-th pair of
                             expert e in ascending pair order; every other
                             slot holds the sentinel ``P``.
* ``expert_ids``             length ``ceil(len(sorted_token_ids) / BM)``;
                             block b holds the expert owning it, -1 past the
                             last used block.
* ``num_tokens_post_padded`` ``BM * block_off[E]``.
* ``expert_offsets``         exclusive prefix sum of ``cnt`` (length E + 1).

Pinning: bit-exact against the pure-Python brute force in ``oracle/brute.py``
on small inputs, and against invariants (permutation of routed pairs,
sentinel padding, block ownership, ``BM = 1`` reproduces the CSR offsets) in
tests/test_oracle_cpu.py.
"""

from __future__ import annotations

import numpy as np


def align_buffer_sizes(num_pairs: int, num_experts: int, block_m: int):
    """Lengths of ``sorted_token_ids`` and ``expert_ids`` buffers."""
    sorted_len = num_pairs + num_experts * (block_m - 1)
    blocks_len = -(-sorted_len // block_m)
    return sorted_len, blocks_len


def moe_align_ref(topk_ids, num_experts: int, block_m: int):
    """Return ``(sorted_token_ids, expert_ids, num_tokens_post_padded, expert_offsets)``."""
    ids = np.asarray(topk_ids, dtype=np.int64).reshape(-1)
    P = ids.size
    E, BM = num_experts, block_m
    valid = (ids >= 0) & (ids < E)
    cnt = np.bincount(ids[valid], minlength=E).astype(np.int64)
    nblk = -(-cnt // BM)
    block_off = np.zeros(E + 1, dtype=np.int64)
    block_off[1:] = np.cumsum(nblk)
    expert_offsets = np.zeros(E + 1, dtype=np.int64)
    expert_offsets[1:] = np.cumsum(cnt)

    sorted_len, blocks_len = align_buffer_sizes(P, E, BM)
    sorted_ids = np.full(sorted_len, P, dtype=np.int64)
    pair_idx = np.nonzero(valid)[0]
    order = pair_idx[np.argsort(ids[pair_idx], kind="stable")]
    pos = 0
    for e in range(E):
        c = int(cnt[e])
        start = int(block_off[e]) * BM
        sorted_ids[start:start + c] = order[pos:pos + c]
        pos += c
    expert_ids = np.full(blocks_len, -1, dtype=np.int64)
    for e in range(E):
        expert_ids[block_off[e]:block_off[e + 1]] = e
    num_post = int(block_off[E]) * BM
    return (sorted_ids.astype(np.int32), expert_ids.astype(np.int32),
            np.int32(num_post), expert_offsets.astype(np.int32))


def grouped_row_order(topk_ids, num_experts: int):
    """Pair indices in (expert, pair) order plus CSR offsets (``BM = 1``).

    Lays the routed pairs out the way the reference operator expects its
    rows (docs/Task1.md:87-92): row r of the grouped activation matrix is
    pair ``order[r]``, and expert e owns rows ``[off[e], off[e+1])``.
    """
    sorted_ids, _, num_post, offs = moe_align_ref(topk_ids, num_experts, 1)
    return sorted_ids[:int(num_post)], offs
