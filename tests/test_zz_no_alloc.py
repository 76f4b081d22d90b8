"""The allocation-free reference-layout entry ``mw4a8_grouped_gemm_noalloc``
through the C ABI: its output equals that of ``mw4a8_grouped_gemm`` (the same
kernels, with a caller workspace) bit for bit, on two calls in a row, the
second with a smaller input (fewer row blocks than the first left in the
shared scratch array, which holds the row-block table of calls over more
than 256 experts), and both match the oracle; then on two calls over fewer
experts, whose kernels find their row blocks without the table."""

import ctypes

import pytest
import torch

from oracle import task1_ref

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_matches_workspace_entry(pkg, dev, order):
    from flagos_kernel_gen_amd import _lib
    L = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    # Over more than 256 experts the row-block table lives in the scratch
    # array: a larger table, then a smaller one over the first's leftovers.
    # Then calls that derive the blocks in the kernel (128-row tiles at
    # 150 rows per expert and K = 4608, then 16-row tiles).
    cases = [(300, 6000, 256, 1024, 128, 13), (260, 700, 256, 512, 128, 14),
             (8, 1200, 512, 4608, 128, 11), (4, 40, 384, 1024, 128, 12)]
    for E, M, N, K, gs, seed in cases:
        print(f"[noalloc] E={E} M={M} N={N} K={K}", flush=True)
        x_q, x_scale, w_q4, w_scale, w_zero, offs = pkg.workloads.make_grouped_inputs(E, M, N, K, gs, seed=seed)
        g = [t.to(dev) for t in (x_q, x_scale, w_q4, w_scale, w_zero, offs)]
        out_ws = torch.full((M, N), -3.0, dtype=torch.bfloat16, device=dev)
        pkg.w4a8_group_gemm_moe(*g, out_ws, gs)
        out_na = torch.full((M, N), -3.0, dtype=torch.bfloat16, device=dev)
        rc = L.mw4a8_grouped_gemm_noalloc(_p(g[0]), g[0].stride(0), _p(g[1]), _p(g[2]), _p(g[3]), _p(g[4]),
                                          _p(g[5]), _p(out_na), out_na.stride(0), M, N, K, E, gs, stream)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_ws), f"E={E} M={M}: differs from the workspace entry"
        ref = task1_ref.w4a8_group_gemm_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, offs,
                                                torch.full((M, N), -3.0, dtype=torch.bfloat16), gs)
        d = (out_na.cpu().float() - ref.float()).abs()
        assert bool((d <= 1e-4 * N + 0.016 * ref.float().abs()).all()), f"E={E} M={M}: outside tolerance"
