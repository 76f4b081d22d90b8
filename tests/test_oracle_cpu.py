"""Pins for the CPU oracle (no GPU). Each check takes a route independent of
the oracle's own code, so that a plausible mistake -- swapped nibbles, a
zero point applied to the wrong group, a missing wrap, a transposed operand,
a dropped scale -- fails at least one of them."""

import numpy as np
import pytest
import torch
from hypothesis import given, settings, strategies as st

from oracle import brute, routing, task1_ref


# ---------------------------------------------------------------- unpack / fold

def test_unpack_exhaustive_bytes():
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(1, 1, 256)
    u = task1_ref.unpack_int4(b).reshape(256, 2)
    for v in range(256):
        assert int(u[v, 0]) == v % 16 and int(u[v, 1]) == v // 16


def test_unpack_hand_worked_byte():
    # byte 0x21 at position p=0 holds k=0 -> 1 (low nibble), k=1 -> 2 (high nibble)
    u = task1_ref.unpack_int4(torch.tensor([[[0x21, 0xF0]]], dtype=torch.uint8))
    assert u.flatten().tolist() == [1, 2, 0, 15]


def test_fold_zero_exhaustive_with_wrap():
    u = torch.arange(16, dtype=torch.int16).repeat(256).reshape(256, 16)
    z = torch.arange(-128, 128, dtype=torch.int32).to(torch.int8).reshape(256, 1)
    w = task1_ref.fold_zero(u, z, 16)
    for zi in range(256):
        zv = zi - 128
        for uv in range(16):
            want = ((uv - zv + 128) % 256) - 128
            assert int(w[zi, uv]) == want
    # the wrap regime exists: z = -120, u = 15 -> 135 wraps to -121
    assert int(task1_ref.fold_zero(torch.tensor([[15]], dtype=torch.int16),
                                   torch.tensor([[-120]], dtype=torch.int8), 1)) == -121


# ---------------------------------------------------------------- partials

def _rand_case(seed, E=3, M=9, N=24, K=256, gs=64, zero="full"):
    g = torch.Generator().manual_seed(seed)
    x_q = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    x_scale = torch.rand(M, generator=g) + 0.1
    w_q4 = torch.randint(0, 256, (E, N, K // 2), dtype=torch.uint8, generator=g)
    G = K // gs
    w_scale = torch.rand(E, N, G, generator=g) * 0.02 + 0.001
    if zero == "full":
        w_zero = torch.randint(-128, 128, (E, N, G), dtype=torch.int8, generator=g)
    else:
        w_zero = torch.full((E, N, G), 8, dtype=torch.int8)
    cuts = sorted(torch.randint(0, M + 1, (E - 1,), generator=g).tolist())
    offs = torch.tensor([0] + cuts + [M], dtype=torch.int32)
    return x_q, x_scale, w_q4, w_scale, w_zero, offs, gs


@pytest.mark.parametrize("seed,gs", [(0, 64), (1, 128), (2, 32), (3, 256)])
def test_partials_match_int64_brute_force(seed, gs):
    x_q, x_scale, w_q4, w_scale, w_zero, offs, gs = _rand_case(seed, gs=gs)
    P = task1_ref.group_partials_ref(x_q, w_q4, w_zero, offs, gs)
    _, _, Pb = brute.grouped_gemm_f64(x_q.numpy(), x_scale.numpy(), w_q4.numpy(), w_scale.numpy(),
                                      w_zero.numpy(), offs.numpy(), gs)
    np.testing.assert_array_equal(P.numpy().astype(np.int64), Pb)


def test_partials_extreme_values_exact():
    # |P| = 128 * 128 * gs = 2**21 for gs=128: still exact in fp32
    K, gs = 256, 128
    x_q = torch.full((2, K), -128, dtype=torch.int8)
    w_q4 = torch.zeros(1, 3, K // 2, dtype=torch.uint8)      # nibbles 0
    w_zero = torch.full((1, 3, 2), 127, dtype=torch.int8)    # w = 0 - 127 = -127
    w_zero[0, 1] = -128                                      # w = 0 + 128 wraps to -128
    P = task1_ref.group_partials_ref(x_q, w_q4, w_zero, torch.tensor([0, 2], dtype=torch.int32), gs)
    assert int(P[0, 0, 0]) == 128 * 127 * gs
    assert int(P[0, 1, 0]) == 128 * 128 * gs
    assert int(P[1, 2, 1]) == 128 * 127 * gs


def test_one_hot_activation_selects_single_weight():
    """x = e_k picks weight (n, k): pins nibble order and the zero point's group."""
    E, N, K, gs = 1, 5, 128, 64
    g = torch.Generator().manual_seed(7)
    w_q4 = torch.randint(0, 256, (E, N, K // 2), dtype=torch.uint8, generator=g)
    w_zero = torch.randint(-20, 20, (E, N, K // gs), dtype=torch.int8, generator=g)
    x_q = torch.zeros(K, K, dtype=torch.int8)
    x_q[torch.arange(K), torch.arange(K)] = 1
    P = task1_ref.group_partials_ref(x_q, w_q4, w_zero, torch.tensor([0, K], dtype=torch.int32), gs)
    for k in range(K):
        for n in range(N):
            byte = int(w_q4[0, n, k // 2])
            nib = (byte >> 4) if k % 2 else (byte & 15)
            want = nib - int(w_zero[0, n, k // gs])
            assert int(P[k, n, k // gs]) == want
            assert int(P[k, n].abs().sum()) == abs(want)


# ---------------------------------------------------------------- full operator

def test_unit_scales_reduce_to_plain_integer_matmul():
    x_q, _, w_q4, _, w_zero, offs, gs = _rand_case(4, E=1, M=7, N=16, K=256, gs=64)
    offs = torch.tensor([0, 7], dtype=torch.int32)
    ones_ws = torch.ones(1, 16, 4)
    ones_xs = torch.ones(7)
    out = task1_ref.w4a8_group_gemm_moe_ref(x_q, ones_xs, w_q4, ones_ws, w_zero, offs,
                                            torch.zeros(7, 16, dtype=torch.bfloat16), gs)
    w = brute.signed_weights_i64(w_q4.numpy()[0], w_zero.numpy()[0], gs)
    want = torch.from_numpy((x_q.numpy().astype(np.int64) @ w.T).astype(np.float32)).to(torch.bfloat16)
    assert torch.equal(out, want)


@pytest.mark.parametrize("seed", range(4))
def test_reference_output_vs_float64(seed):
    x_q, x_scale, w_q4, w_scale, w_zero, offs, gs = _rand_case(10 + seed)
    sentinel = torch.full((x_q.shape[0], w_q4.shape[1]), 3.0, dtype=torch.bfloat16)
    out = task1_ref.w4a8_group_gemm_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, offs, sentinel.clone(), gs)
    f64, owned, _ = brute.grouped_gemm_f64(x_q.numpy(), x_scale.numpy(), w_q4.numpy(), w_scale.numpy(),
                                           w_zero.numpy(), offs.numpy(), gs)
    got = out.float().numpy()
    # bf16 keeps 8 significant bits: half an ulp is 2**-9 relative, plus fp32 noise
    tol = np.abs(f64[owned]) * 2.0 ** -8 + 1e-6
    assert np.all(np.abs(got[owned] - f64[owned]) <= tol)
    assert np.all(got[~owned] == 3.0)


def test_linearity_in_scales():
    x_q, x_scale, w_q4, w_scale, w_zero, offs, gs = _rand_case(20)
    o1 = task1_ref.w4a8_group_gemm_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, offs,
                                           torch.zeros(x_q.shape[0], 24, dtype=torch.bfloat16), gs)
    o2 = task1_ref.w4a8_group_gemm_moe_ref(x_q, x_scale * 4, w_q4, w_scale, w_zero, offs,
                                           torch.zeros(x_q.shape[0], 24, dtype=torch.bfloat16), gs)
    # scaling by a power of two commutes with bf16 rounding
    assert torch.equal(o2.float(), o1.float() * 4)


def test_empty_experts_and_nonzero_first_offset_leave_rows_untouched():
    x_q, x_scale, w_q4, w_scale, w_zero, _, gs = _rand_case(30, E=4, M=10)
    offs = torch.tensor([2, 2, 6, 6, 8], dtype=torch.int32)   # rows 0-1 and 8-9 owned by nobody
    out = torch.full((10, 24), -7.0, dtype=torch.bfloat16)
    task1_ref.w4a8_group_gemm_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, offs, out, gs)
    assert torch.all(out[[0, 1, 8, 9]] == -7.0)
    assert not torch.any(out[2:8] == -7.0)


def test_all_unpack_equals_per_expert_unpack():
    x_q, x_scale, w_q4, w_scale, w_zero, offs, gs = _rand_case(31)
    a = task1_ref.w4a8_group_gemm_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, offs,
                                          torch.zeros(9, 24, dtype=torch.bfloat16), gs, unpack="all")
    b = task1_ref.w4a8_group_gemm_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, offs,
                                          torch.zeros(9, 24, dtype=torch.bfloat16), gs, unpack="per_expert")
    assert torch.equal(a, b)


def test_shape_asserts_like_reference():
    x_q = torch.zeros(4, 128, dtype=torch.int8)
    with pytest.raises(AssertionError):
        task1_ref.w4a8_group_gemm_moe_ref(x_q, torch.ones(4), torch.zeros(1, 8, 63, dtype=torch.uint8),
                                          None, None, torch.tensor([0, 4], dtype=torch.int32), None, 64)
    with pytest.raises(AssertionError):
        task1_ref.w4a8_group_gemm_moe_ref(x_q, torch.ones(4), torch.zeros(1, 8, 64, dtype=torch.uint8),
                                          None, None, torch.tensor([0, 4], dtype=torch.int32), None, 96)


# ---------------------------------------------------------------- routed extension

@pytest.mark.parametrize("seed", range(3))
def test_fused_ref_vs_loops(seed):
    g = torch.Generator().manual_seed(40 + seed)
    M, E, topk, N, K, gs = 6, 5, 2, 16, 128, 64
    x_q = torch.randint(-127, 128, (M, K), dtype=torch.int8, generator=g)
    x_scale = torch.rand(M, generator=g) + 0.5
    w_q4 = torch.randint(0, 256, (E, N, K // 2), dtype=torch.uint8, generator=g)
    w_scale = torch.rand(E, N, K // gs, generator=g) * 0.01 + 0.005
    w_zero = torch.randint(-128, 128, (E, N, K // gs), dtype=torch.int8, generator=g)
    ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(M)]).to(torch.int32)
    ids[0, 1] = -1           # not routed
    tw = torch.rand(M, topk, generator=g)
    out = task1_ref.fused_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, ids, tw, gs,
                                  out=torch.full((M * topk, N), 9.0, dtype=torch.bfloat16))
    want = brute.fused_loops(x_q.numpy(), x_scale.numpy(), w_q4.numpy(), w_scale.numpy(), w_zero.numpy(),
                             ids.numpy(), tw.numpy(), gs)
    got = out.float().numpy()
    routed = ~np.isnan(want[:, 0])
    assert not routed[1] and np.all(got[1] == 9.0)
    tol = np.abs(want[routed]) * 2.0 ** -8 + 1e-6
    assert np.all(np.abs(got[routed] - want[routed]) <= tol)


def test_fused_ref_pair_subset_matches_full():
    g = torch.Generator().manual_seed(50)
    M, E, topk, N, K, gs = 8, 4, 2, 16, 128, 128
    x_q = torch.randint(-127, 128, (M, K), dtype=torch.int8, generator=g)
    x_scale = torch.rand(M, generator=g) + 0.5
    w_q4 = torch.randint(0, 256, (E, N, K // 2), dtype=torch.uint8, generator=g)
    w_scale = torch.rand(E, N, 1, generator=g) * 0.01
    w_zero = torch.full((E, N, 1), 8, dtype=torch.int8)
    ids = torch.randint(0, E, (M, topk), generator=g).to(torch.int32)
    tw = torch.rand(M, topk, generator=g)
    full = task1_ref.fused_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, ids, tw, gs)
    sub = task1_ref.fused_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, ids, tw, gs, pairs=[3, 0, 11])
    for p in (0, 3, 11):
        assert torch.equal(sub[p], full[p])


# ---------------------------------------------------------------- routing

@pytest.mark.parametrize("P,E,BM", [(0, 4, 16), (1, 8, 16), (8, 256, 16), (37, 5, 4), (100, 7, 1),
                                    (64, 3, 64), (200, 16, 128)])
def test_align_matches_loops(P, E, BM):
    rng = np.random.default_rng(P * 31 + E)
    ids = rng.integers(0, E, size=P).astype(np.int32)
    s, x, n, o = routing.moe_align_ref(ids, E, BM)
    bs, bx, bn, bo = brute.align_loops(ids, E, BM)
    assert s.tolist() == bs and x.tolist() == bx and int(n) == bn and o.tolist() == bo


def test_align_ignores_out_of_range_ids():
    ids = np.array([0, -1, 3, 4, 1, 3, 99], dtype=np.int32)
    s, x, n, o = routing.moe_align_ref(ids, 4, 2)
    assert o.tolist() == [0, 1, 2, 2, 4]
    assert int(n) == 6
    assert s[:6].tolist() == [0, 7, 4, 7, 2, 5]
    assert x.tolist()[:3] == [0, 1, 3]


@settings(max_examples=60, deadline=None)
@given(st.integers(1, 40), st.integers(1, 9), st.integers(1, 4), st.sampled_from([1, 2, 4, 16]),
       st.integers(0, 2 ** 31 - 1))
def test_align_invariants(M, E, topk, BM, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, E, size=(M, topk)).astype(np.int32)
    P = M * topk
    s, x, n, o = routing.moe_align_ref(ids, E, BM)
    n = int(n)
    real = s[s < P]
    assert sorted(real.tolist()) == list(range(P))            # every pair exactly once
    assert np.all(s[n:] == P)                                  # tail is sentinel
    assert n % BM == 0 and np.all(x[n // BM:] == -1)
    flat = ids.reshape(-1)
    for b in range(n // BM):
        slots = s[b * BM:(b + 1) * BM]
        members = slots[slots < P]
        assert members.size > 0 and np.all(flat[members] == x[b])
        assert np.all(np.diff(members) > 0)                    # ascending pair order
    assert np.array_equal(np.diff(o), np.bincount(flat, minlength=E))


def test_align_bm1_gives_reference_csr_offsets():
    rng = np.random.default_rng(3)
    ids = rng.integers(0, 6, size=(50, 2)).astype(np.int32)
    order, offs = routing.grouped_row_order(ids, 6)
    flat = ids.reshape(-1)
    for e in range(6):
        rows = order[offs[e]:offs[e + 1]]
        assert np.all(flat[rows] == e)
    assert offs[-1] == 100


# ---------------------------------------------------------------- planted mistakes

def test_planted_nibble_swap_is_caught(monkeypatch):
    """A swapped nibble order in the oracle must fail the brute-force pin."""
    def swapped(w):
        b = w.to(torch.int16)
        out = torch.empty(*b.shape[:-1], b.shape[-1] * 2, dtype=torch.int16)
        out[..., 0::2] = (b >> 4) & 15
        out[..., 1::2] = b & 15
        return out
    monkeypatch.setattr(task1_ref, "unpack_int4", swapped)
    x_q, x_scale, w_q4, w_scale, w_zero, offs, gs = _rand_case(60)
    P = task1_ref.group_partials_ref(x_q, w_q4, w_zero, offs, gs)
    _, _, Pb = brute.grouped_gemm_f64(x_q.numpy(), x_scale.numpy(), w_q4.numpy(), w_scale.numpy(),
                                      w_zero.numpy(), offs.numpy(), gs)
    assert not np.array_equal(P.numpy().astype(np.int64), Pb)


def test_planted_missing_wrap_is_caught(monkeypatch):
    """Folding the zero point without the int8 wrap must fail the exhaustive table."""
    monkeypatch.setattr(task1_ref, "fold_zero",
                        lambda u, z, gs: (u - z.to(torch.int16).repeat_interleave(gs, -1)).clamp(-128, 127)
                        .to(torch.int8))
    u = torch.tensor([[15]], dtype=torch.int16)
    assert int(task1_ref.fold_zero(u, torch.tensor([[-120]], dtype=torch.int8), 1)) != -121
