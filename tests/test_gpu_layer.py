"""Parity of the MoE-layer kernels (through the C ABI) with the CPU oracle.

Bars: per-token quantization bit-exact (IEEE division and round-half-even
on both sides); router ids bit-exact, weights within 2e-6 relative (the
kernel's expf vs float64); combine bit-exact (float32 products and sums in
the same order); silu*up requant: scales within 2e-6 relative, int8 values
within 1 and at least 99.9 % identical (expf rounding can move a value
across a rounding boundary); the whole layer within the GEMM's tolerance
(max|diff| <= 2e-2 * max|ref|, cosine >= 0.9995) since two int8
requantizations sit inside it."""

import numpy as np
import pytest
import torch

from oracle import layer_ref, task1_ref

pytestmark = pytest.mark.gpu


def _close(got, ref, what, rel=2e-2, cos_min=0.9995):
    g = got.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert torch.isfinite(g).all(), what
    d = (g - r).abs().max().item()
    scale = r.abs().max().item()
    cos = torch.nn.functional.cosine_similarity(g.reshape(1, -1).double(), r.reshape(1, -1).double()).item()
    assert d <= rel * scale, f"{what}: max|diff| {d:.4g} vs {scale:.4g}"
    assert cos >= cos_min, f"{what}: cos {cos:.6f}"


# ---------------------------------------------------------------- quant

@pytest.mark.parametrize("M,K", [(1, 8), (5, 1024), (64, 7168), (4096, 2048), (7, 3000), (9, 16384),
                                 (3, 40000)])
def test_quant_rows_bit_exact(pkg, dev, M, K):
    print(f"[quant] M={M} K={K}", flush=True)
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16)
    x[0, :] = 0                      # all-zero row
    if M > 2:
        x[2, 1] = 127.0              # scale 1.0: exact ties below
        x[2, 0] = 2.5
        x[2, 2] = -3.5
    q, s = pkg.quant_per_token(x.to(dev))
    rq, rs = layer_ref.quant_per_token_ref(x)
    assert torch.equal(s.cpu(), rs)
    assert torch.equal(q.cpu(), rq)


def test_quant_rows_strided_input(pkg, dev):
    g = torch.Generator().manual_seed(3)
    big = torch.randn(9, 512 + 64, generator=g).to(torch.bfloat16)
    x = big[:, :512]
    q, s = pkg.quant_per_token(big.to(dev)[:, :512])
    rq, rs = layer_ref.quant_per_token_ref(x)
    assert torch.equal(q.cpu(), rq) and torch.equal(s.cpu(), rs)


# ---------------------------------------------------------------- router

@pytest.mark.parametrize("M,E,k,renorm", [(1, 8, 2, True), (300, 256, 8, True), (77, 128, 8, False),
                                          (33, 1024, 64, True), (40, 64, 1, True), (16, 5, 5, False),
                                          (21, 512, 8, False), (9, 300, 6, True), (12, 200, 3, True)])
def test_router_topk(pkg, dev, M, E, k, renorm):
    print(f"[router] M={M} E={E} k={k} renorm={renorm}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + E)
    lg = torch.randn(M, E, generator=g)
    lg[0, E // 2] = lg[0, E - 1] = 9.0           # tie at the top: lower index first
    ids, w = pkg.router_topk(lg.to(dev), k, renorm)
    rids, rw = layer_ref.router_topk_ref(lg, k, renorm)
    assert np.array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(w.cpu().numpy().astype(np.float64), rw, rtol=2e-6, atol=1e-12)


def test_router_matches_the_benchmark_routing(pkg, dev):
    """Same ids and (to float32 rounding) the same weights as the softmax ->
    top-k -> renormalise routing the benchmark inputs use."""
    M, E, k = 512, 256, 8
    g = torch.Generator().manual_seed(99)
    logits = torch.randn(M, E, generator=g)
    probs = torch.softmax(logits, dim=-1)
    pw, pi = torch.topk(probs, k, dim=-1)
    pw = pw / pw.sum(-1, keepdim=True)
    ids, w = pkg.router_topk(logits.to(dev), k)
    assert torch.equal(ids.cpu().long(), pi)
    torch.testing.assert_close(w.cpu(), pw, rtol=1e-5, atol=1e-7)


# ---------------------------------------------------------------- silu * up

@pytest.mark.parametrize("P,I", [(1, 8), (37, 768), (512, 2048), (4096, 1024), (9, 3000), (7, 6144),
                                 (5, 10000)])
def test_silu_mul_quant(pkg, dev, P, I):
    print(f"[silu] P={P} I={I}", flush=True)
    g = torch.Generator().manual_seed(P + I)
    h = (torch.randn(P, 2 * I, generator=g) * 2).to(torch.bfloat16)
    q, s = pkg.silu_mul_quant(h.to(dev))
    rq, rs = layer_ref.silu_mul_quant_ref(h)
    np.testing.assert_allclose(s.cpu().numpy(), rs.numpy(), rtol=2e-6)
    d = (q.cpu().int() - rq.int()).abs()
    assert int(d.max()) <= 1
    assert float((d == 0).float().mean()) >= 0.999


# ---------------------------------------------------------------- combine

@pytest.mark.parametrize("M,topk,N,weighted", [(1, 1, 8, False), (64, 8, 7168, False), (33, 2, 4096, True),
                                               (4096, 8, 2048, False), (5, 3, 520, True), (7, 6, 1024, True),
                                               (16, 8, 7168, True), (9, 4, 2056, False)])
def test_combine_bit_exact(pkg, dev, M, topk, N, weighted):
    print(f"[combine] M={M} topk={topk} N={N} weighted={weighted}", flush=True)
    g = torch.Generator().manual_seed(M + N)
    y = torch.randn(M * topk, N, generator=g).to(torch.bfloat16)
    w = torch.rand(M, topk, generator=g) if weighted else None
    out = pkg.combine_topk(y.to(dev), topk, None if w is None else w.to(dev))
    ref = layer_ref.combine_ref(y, topk, w)
    assert torch.equal(out.cpu(), ref)


# ---------------------------------------------------------------- GEMM without top-k weights

def test_fused_moe_without_weights_equals_unit_weights(pkg, dev):
    wl = pkg.workloads
    inp = wl.make_routed_inputs(wl.CONFIGS["tiny"], 64, device=dev)
    args = (inp.x_q, inp.x_scale, inp.w_q4, inp.w_scale, inp.w_zero, inp.topk_ids)
    a = pkg.w4a8_fused_moe(*args, None, group_size=128)
    b = pkg.w4a8_fused_moe(*args, torch.ones_like(inp.topk_weights), group_size=128)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


# ---------------------------------------------------------------- the layer

LAYERS = [
    # (name, E, H, I, topk, M)
    ("tiny", 8, 1024, 512, 2, 64),
    ("qwen3-like", 128, 2048, 768, 8, 48),
    ("mixtral-like decode", 8, 4096, 1024, 2, 3),
]


def _layer_inputs(pkg, E, H, I, M, seed):
    wl = pkg.workloads
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(M, E, generator=g)
    w13 = wl.make_weights(E, 2 * I, H, 128, seed=seed + 1)
    w2 = wl.make_weights(E, H, I, 128, seed=seed + 2)
    return x, logits, w13, w2


@pytest.mark.parametrize("name,E,H,I,topk,M", LAYERS)
def test_moe_layer_stagewise_and_end_to_end(pkg, dev, name, E, H, I, topk, M):
    """Each stage against the oracle applied to the GPU's own inputs to that
    stage, then the whole layer against the oracle chain."""
    print(f"[layer] {name} E={E} H={H} I={I} topk={topk} M={M}", flush=True)
    x, logits, w13, w2 = _layer_inputs(pkg, E, H, I, M, seed=E + H + M)
    w13d = [t.to(dev) for t in w13]
    w2d = [t.to(dev) for t in w2]
    out, mid = pkg.w4a8_moe_layer(x.to(dev), logits.to(dev), *w13d, *w2d, topk=topk, return_intermediates=True)
    torch.cuda.synchronize()
    P = M * topk
    # stage 1-2: quant and router are exact / within float rounding
    rq, rs = layer_ref.quant_per_token_ref(x)
    assert torch.equal(mid["x_q"].cpu(), rq) and torch.equal(mid["x_scale"].cpu(), rs)
    rids, rw = layer_ref.router_topk_ref(logits, topk)
    ids = mid["topk_ids"].cpu()
    assert np.array_equal(ids.numpy(), rids)
    # stage 3: up/gate GEMM without weights
    h_ref = task1_ref.fused_moe_ref(rq, rs, *w13, ids, torch.ones(M, topk), 128)
    _close(mid["h"], h_ref, f"{name}: up/gate GEMM", rel=1e-2, cos_min=0.9999)
    # stage 4: silu * up requant of the GPU's h
    hq_ref, hs_ref = layer_ref.silu_mul_quant_ref(mid["h"].cpu())
    np.testing.assert_allclose(mid["h_scale"].cpu().numpy(), hs_ref.numpy(), rtol=2e-6)
    assert int((mid["h_q"].cpu().int() - hq_ref.int()).abs().max()) <= 1
    # stage 5: down GEMM of the GPU's h_q with the routing weights
    w_gpu = mid["topk_weights"].cpu()
    y_ref = task1_ref.fused_moe_ref(mid["h_q"].cpu(), mid["h_scale"].cpu(), *w2, ids.reshape(P, 1),
                                    w_gpu.reshape(P, 1), 128)
    _close(mid["y"], y_ref, f"{name}: down GEMM", rel=1e-2, cos_min=0.9999)
    # stage 6: combine of the GPU's y is exact
    assert torch.equal(out.cpu(), layer_ref.combine_ref(mid["y"].cpu(), topk))
    # end to end against the oracle chain
    ref, _ = layer_ref.moe_layer_ref(x, logits, *w13, *w2, topk)
    _close(out, ref, f"{name}: layer")


# ---------------------------------------------------------------- weight repack

@pytest.mark.parametrize("E,N,K", [(2, 3, 8), (3, 70, 200), (8, 2048, 1024), (1, 1, 24)])
def test_repack_bit_exact_and_round_trip(pkg, dev, E, N, K):
    from oracle import repack
    g = torch.Generator().manual_seed(E * N + K)
    w = torch.randint(0, 256, (E, N, K // 2), dtype=torch.int32, generator=g).to(torch.uint8)
    m = pkg.repack_weights(w.to(dev))
    assert np.array_equal(m.cpu().numpy(), repack.to_mfma(w.numpy()))
    back = pkg.repack_weights(m, inverse=True)
    assert torch.equal(back.cpu(), w)


@pytest.mark.parametrize("gs,zero", [(128, "symmetric"), (128, "full"), (64, "uint4"), (256, "symmetric"),
                                     (256, "full")])
def test_fused_moe_repacked_is_bit_identical(pkg, dev, gs, zero):
    """Same outputs, bit for bit, from the repacked weights on every row-block
    kernel (16 / 32 / 64 / 128 rows) and both unpacking paths."""
    wl = pkg.workloads
    print(f"[repacked] gs={gs} zero={zero}", flush=True)
    E, N, K, M, topk = 8, 512, 2048, 256, 2
    w_q4, w_scale, w_zero = wl.make_weights(E, N, K, gs, seed=gs + 5, device=dev, zero=zero)
    x_q, x_scale = wl.make_activations(M, K, seed=gs + 6, device=dev)
    ids, tw = wl.make_routing(M, E, topk, "softmax", seed=gs + 7, device=dev)
    w_m = pkg.repack_weights(w_q4)
    for bm in (16, 32, 64, 128):
        a = pkg.w4a8_fused_moe(x_q, x_scale, w_q4, w_scale, w_zero, ids, tw, group_size=gs, block_m=bm)
        b = pkg.w4a8_fused_moe(x_q, x_scale, w_m, w_scale, w_zero, ids, tw, group_size=gs, block_m=bm,
                               weight_layout="mfma")
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"gs={gs} zero={zero} block_m={bm}"


def test_moe_layer_repacked_is_bit_identical(pkg, dev):
    x, logits, w13, w2 = _layer_inputs(pkg, 8, 1024, 512, 32, seed=77)
    w13d = [t.to(dev) for t in w13]
    w2d = [t.to(dev) for t in w2]
    a = pkg.w4a8_moe_layer(x.to(dev), logits.to(dev), *w13d, *w2d, topk=2)
    w13m = [pkg.repack_weights(w13d[0]), w13d[1], w13d[2]]
    w2m = [pkg.repack_weights(w2d[0]), w2d[1], w2d[2]]
    b = pkg.w4a8_moe_layer(x.to(dev), logits.to(dev), *w13m, *w2m, topk=2, weight_layout="mfma")
    torch.cuda.synchronize()
    assert torch.equal(a, b)
