"""Pins for the MoE-layer oracle (no GPU): each check takes a route
independent of the oracle's code -- hand-worked values, Python brute force,
float64 closed forms -- so that a wrong rounding mode, a dropped clamp, a
swapped gate/up half, a wrong tie rule or a missing renormalisation fails."""

import math

import numpy as np
import pytest
import torch

from oracle import layer_ref, task1_ref


# ---------------------------------------------------------------- per-token quant

def test_quant_ties_round_half_even_and_clamp():
    # amax = 127 -> scale = 1.0 exactly, so x / scale = x
    x = torch.tensor([[127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -126.5]], dtype=torch.float32)
    q, s = layer_ref.quant_per_token_ref(x)
    assert float(s[0]) == 1.0
    assert q[0].tolist() == [127, 2, 4, -2, -4, 0, 2, -126]


def test_quant_zero_row_and_extremes():
    x = torch.zeros(2, 16, dtype=torch.bfloat16)
    x[1, 3] = -7.0
    q, s = layer_ref.quant_per_token_ref(x)
    assert float(s[0]) == np.float32(1e-12) / np.float32(127.0)
    assert int(q[0].abs().max()) == 0
    assert int(q[1, 3]) == -127 and int(q[1].abs().sum()) == 127


def test_quant_matches_python_brute_force():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(6, 40, generator=g) * 3).to(torch.bfloat16)
    q, s = layer_ref.quant_per_token_ref(x)
    xf = x.float().numpy()
    for m in range(6):
        amax = max(np.float32(max(abs(float(v)) for v in xf[m])), np.float32(1e-12))
        sc = np.float32(amax) / np.float32(127.0)
        assert np.float32(s[m]) == sc
        for k in range(40):
            want = max(-127, min(127, round(float(np.float32(xf[m, k]) / sc))))   # Python round: half-even
            assert int(q[m, k]) == want


def test_reciprocal_rounding_with_division_fallback_equals_division():
    """The quant kernels round a * (1/s) and divide only when that product is
    within 1e-4 of a half-integer; for |a| <= 127 s this gives rint(a / s)
    exactly (float32, round half to even). Half of the samples sit within 4
    ulps of a half-integer multiple of s, where a plain a * (1/s) does differ
    from the quotient."""
    rng = np.random.default_rng(7)
    n = 2_000_000
    amax = (0.5 + rng.random(n, dtype=np.float32)) * np.exp2(rng.integers(-30, 30, n)).astype(np.float32)
    s = np.maximum(amax, np.float32(1e-12)) / np.float32(127)
    inv = np.float32(1) / s
    a = ((rng.random(n, dtype=np.float32) * 2 - 1) * amax).astype(np.float32)
    half = n // 2
    k = (rng.integers(-127, 127, half) + 0.5).astype(np.float32)
    near = (k * s[:half]).view(np.int32) + rng.integers(-4, 5, half).astype(np.int32)
    a[:half] = near.view(np.float32)
    keep = np.abs(a) <= amax
    a, s, inv = a[keep], s[keep], inv[keep]
    exact = np.rint(a / s)
    t = a * inv
    fast = np.where(np.abs((t - np.floor(t)) - np.float32(0.5)) < np.float32(1e-4), np.rint(a / s), np.rint(t))
    assert np.array_equal(fast, exact)
    assert not np.array_equal(np.rint(t), exact)   # the fallback is needed


def test_quant_matches_the_benchmark_generator(pkg):
    g = torch.Generator().manual_seed(9)
    x = torch.randn(7, 96, generator=g).to(torch.bfloat16)
    q, s = layer_ref.quant_per_token_ref(x)
    q2, s2 = pkg.workloads.quantize_per_token(x)
    assert torch.equal(q, q2) and torch.equal(s, s2)


# ---------------------------------------------------------------- router

@pytest.mark.parametrize("E,k,renorm", [(8, 2, True), (16, 5, False), (64, 8, True), (300, 1, True)])
def test_router_matches_brute_force(E, k, renorm):
    g = torch.Generator().manual_seed(E + k)
    lg = torch.randn(5, E, generator=g)
    lg[0, 3] = lg[0, 7] = 4.0            # a tie at the top: lower index first
    ids, w = layer_ref.router_topk_ref(lg, k, renorm)
    for m in range(5):
        row = [float(v) for v in lg[m]]
        order = sorted(range(E), key=lambda e: (-row[e], e))[:k]
        assert ids[m].tolist() == order
        ex = [math.exp(row[e] - row[order[0]]) for e in range(E)]
        den = sum(ex[e] for e in order) if renorm else sum(ex)
        for j, e in enumerate(order):
            assert abs(w[m, j] - ex[e] / den) <= 1e-12
    assert ids[0, 0] == 3 and (k < 2 or ids[0, 1] == 7)


def test_router_renormalised_equals_softmax_topk_renormalised():
    g = torch.Generator().manual_seed(3)
    lg = torch.randn(9, 32, generator=g)
    ids, w = layer_ref.router_topk_ref(lg, 4, True)
    p = torch.softmax(lg.double(), dim=-1)
    pv, pi = torch.topk(p, 4, dim=-1)
    assert np.array_equal(pi.numpy(), ids)
    np.testing.assert_allclose((pv / pv.sum(-1, keepdim=True)).numpy(), w, rtol=1e-12)
    assert np.allclose(w.sum(-1), 1.0)


# ---------------------------------------------------------------- silu * up, requant

def test_silu_mul_against_float64_and_halves():
    g = torch.Generator().manual_seed(11)
    h = (torch.randn(4, 64, generator=g) * 2).to(torch.bfloat16)
    y = layer_ref.silu_mul_y(h).double().numpy()
    hf = h.double().numpy()
    gate, up = hf[:, :32], hf[:, 32:]
    want = gate / (1.0 + np.exp(-gate)) * up
    np.testing.assert_allclose(y, want, rtol=2e-6, atol=1e-30)
    # swapping the halves gives a different function: the gate half is the first
    swapped = up / (1.0 + np.exp(-up)) * gate
    assert not np.allclose(y, swapped, rtol=1e-3)


def test_silu_mul_quant_is_quant_of_y():
    g = torch.Generator().manual_seed(12)
    h = torch.randn(3, 48, generator=g).to(torch.bfloat16)
    q, s = layer_ref.silu_mul_quant_ref(h)
    q2, s2 = layer_ref.quant_per_token_ref(layer_ref.silu_mul_y(h))
    assert torch.equal(q, q2) and torch.equal(s, s2)


# ---------------------------------------------------------------- combine

@pytest.mark.parametrize("weighted", [False, True])
def test_combine_matches_loops(weighted):
    g = torch.Generator().manual_seed(13)
    M, topk, N = 3, 4, 8
    y = torch.randn(M * topk, N, generator=g).to(torch.bfloat16)
    w = torch.rand(M, topk, generator=g) if weighted else None
    out = layer_ref.combine_ref(y, topk, w)
    yf = y.float().numpy()
    for m in range(M):
        for n in range(N):
            acc = np.float32(0)
            for j in range(topk):
                t = np.float32(yf[m * topk + j, n])
                if weighted:
                    t = np.float32(np.float32(w[m, j]) * t)
                acc = np.float32(acc + t)
            assert float(out[m, n]) == float(torch.tensor(float(acc)).to(torch.bfloat16))


# ---------------------------------------------------------------- the layer

def test_layer_with_one_expert_per_token_is_the_down_gemm_of_the_up_gemm(pkg):
    """topk = 1 with renormalisation: every weight is 1 and combine is the
    identity, so the layer is down(silu_quant(up(quant(x)))) row by row."""
    wl = pkg.workloads
    E, H, I, M = 4, 256, 128, 6
    g = torch.Generator().manual_seed(21)
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(M, E, generator=g)
    w13 = wl.make_weights(E, 2 * I, H, 128, seed=31)
    w2 = wl.make_weights(E, H, I, 128, seed=32)
    out, mid = layer_ref.moe_layer_ref(x, logits, *w13, *w2, topk=1)
    assert np.allclose(mid["w"], 1.0)
    x_q, x_s = layer_ref.quant_per_token_ref(x)
    ids = torch.from_numpy(mid["ids"])
    h = task1_ref.fused_moe_ref(x_q, x_s, *w13, ids, torch.ones(M, 1), 128)
    hq, hs = layer_ref.silu_mul_quant_ref(h)
    y = task1_ref.fused_moe_ref(hq, hs, *w2, ids, torch.ones(M, 1), 128)
    assert torch.equal(out, y)


# ---------------------------------------------------------------- weight repack

def test_repack_round_trip_and_element_order():
    from oracle import repack
    g = torch.Generator().manual_seed(41)
    w = torch.randint(0, 256, (3, 5, 64), dtype=torch.int32, generator=g).to(torch.uint8)
    m = repack.to_mfma(w.numpy())
    assert np.array_equal(repack.from_mfma(m), w.numpy())
    # byte i of run r holds elements 8r+i and 8r+i+4 (reference unpack), flipped by 8
    u = task1_ref.unpack_int4(w).numpy()
    for e in range(3):
        for n in range(5):
            for r in range(16):
                for i in range(4):
                    byte = int(m[e, n, 4 * r + i])
                    assert (byte & 0xF) ^ 8 == u[e, n, 8 * r + i]
                    assert (byte >> 4) ^ 8 == u[e, n, 8 * r + i + 4]


def test_repack_hand_worked_run():
    from oracle import repack
    # run elements 0..7 = 0,1,...,7 -> reference bytes 0x10 0x32 0x54 0x76
    ref = np.array([[[0x10, 0x32, 0x54, 0x76]]], dtype=np.uint8)
    # byte i = (i ^ 8) | ((i + 4) ^ 8) << 4 -> 0xC8 0xD9 0xEA 0xFB
    assert repack.to_mfma(ref).tolist() == [[[0xC8, 0xD9, 0xEA, 0xFB]]]
