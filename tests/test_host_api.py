"""The C-ABI library and the Python host layer, without a GPU: the library
loads, exports every symbol include/mw4a8.h declares, its CPU self-test
passes, argument validation rejects bad input before any device work, and
nothing falls back to the CPU."""

import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mw4a8.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mw4a8_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(pkg):
    from flagos_kernel_gen_amd import _lib
    L = _lib.lib()
    names = _declared_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.SIGNATURES)


def test_host_selftest_passes(pkg):
    from flagos_kernel_gen_amd import _lib
    assert _lib.lib().mw4a8_host_selftest() == 0
    assert _lib.lib().mw4a8_abi_version() == 1


def test_sizes_and_tile_selection(pkg):
    assert pkg.align_buffer_sizes(8, 256, 16) == (8 + 256 * 15, -(-(8 + 256 * 15) // 16))
    assert pkg.align_buffer_sizes(0, 4, 1) == (0, 0)
    # decode: ~1 row per touched expert -> smallest block; prefill DSv3 -> 128
    assert pkg.select_block_m(8, 256, 4096, 7168, 128) == 16
    assert pkg.select_block_m(32768, 256, 4096, 7168, 128) == 128
    assert pkg.select_block_m(512, 256, 4096, 7168, 128) == 16
    assert pkg.select_block_m(64 * 8, 8, 2048, 1024, 128) == 64
    assert pkg.select_block_m(64 * 2, 8, 2048, 1024, 128) == 16         # tiny M=64: 16 rows, 128 tiles
    # middle: 8 rows per expert stay on 16-row tiles; from 16 rows (and from
    # 9 rows at K <= 4096) the 64-row tile (measured crossovers)
    assert pkg.select_block_m(32 * 2, 8, 28672, 4096, 128) == 16        # Mixtral M=32: 8 rows
    assert pkg.select_block_m(64 * 2, 8, 28672, 4096, 128) == 64        # Mixtral M=64: 16 rows
    assert pkg.select_block_m(384 * 8, 256, 4096, 7168, 128) == 16     # DSv3 up M=384: 12 rows
    assert pkg.select_block_m(384 * 8, 256, 7168, 2048, 128) == 64     # DSv3 down M=384: 12 rows
    assert pkg.select_block_m(256 * 8, 128, 1536, 2048, 128) == 64     # Qwen3 M=256: 16 rows
    assert pkg.select_block_m(1024 * 8, 256, 4096, 7168, 128) == 64    # DSv3 up M=1024: 32 rows
    # long expert row lists: 128-row tiles from K = 2048 (DSv3 down M=4096,
    # Qwen3 M=2048), 64 below
    assert pkg.select_block_m(32768, 256, 7168, 2048, 128) == 128
    assert pkg.select_block_m(16384, 128, 1536, 2048, 128) == 128
    assert pkg.select_block_m(16384, 128, 1536, 1024, 128) == 64


def test_c_abi_rejects_bad_arguments_without_device_work(pkg):
    from flagos_kernel_gen_amd import _lib
    L = _lib.lib()
    p = ctypes.c_void_p(4096)
    # K not a multiple of group_size
    rc = L.mw4a8_grouped_gemm(p, 256, p, p, p, p, p, p, 64, 4, 64, 200, 2, 128, p, 1 << 20, None)
    assert rc == -1 and "multiple" in _lib.last_error()
    # unsupported group size
    rc = L.mw4a8_grouped_gemm(p, 256, p, p, p, p, p, p, 64, 4, 64, 256, 2, 32, p, 1 << 20, None)
    assert rc == -2
    # null pointer
    rc = L.mw4a8_grouped_gemm(None, 256, p, p, p, p, p, p, 64, 4, 64, 256, 2, 128, p, 1 << 20, None)
    assert rc == -1 and "null" in _lib.last_error()
    # row stride not a multiple of 16
    rc = L.mw4a8_grouped_gemm(p, 260, p, p, p, p, p, p, 64, 4, 64, 256, 2, 128, p, 1 << 20, None)
    assert rc == -1
    # too small a workspace
    rc = L.mw4a8_grouped_gemm(p, 256, p, p, p, p, p, p, 64, 4, 64, 256, 2, 128, p, 16, None)
    assert rc == -3
    # routing: too many experts, bad block_m for the fused GEMM
    assert L.mw4a8_moe_align(p, 8, 2048, 16, p, p, p, None, None) == -2
    rc = L.mw4a8_fused_moe(p, 256, p, p, p, p, p, p, p, p, 2, p, 64, 4, 64, 256, 2, 128, 48, None)
    assert rc == -2
    # zero rows is a no-op
    assert L.mw4a8_grouped_gemm(p, 256, p, p, p, p, p, p, 64, 0, 64, 256, 2, 128, p, 1 << 20, None) == 0
    # the allocation-free entry: same argument checks; a call whose block table
    # exceeds its fixed scratch (800000 rows over 100000 experts: up to 143750
    # 16-row blocks > 65536) is refused before any device work
    rc = L.mw4a8_grouped_gemm_noalloc(p, 256, p, p, p, p, p, p, 64, 4, 64, 200, 2, 128, None)
    assert rc == -1 and "multiple" in _lib.last_error()
    rc = L.mw4a8_grouped_gemm_noalloc(p, 256, p, p, p, p, p, p, 64, 800000, 64, 256, 100000, 128, None)
    assert rc == -2 and "scratch" in _lib.last_error()
    assert L.mw4a8_grouped_gemm_noalloc(p, 256, p, p, p, p, p, p, 64, 0, 64, 256, 2, 128, None) == 0


def test_layer_entries_reject_bad_arguments_without_device_work(pkg):
    from flagos_kernel_gen_amd import _lib
    L = _lib.lib()
    p = ctypes.c_void_p(4096)
    # quant: K not a multiple of 8, misaligned input, null output
    assert L.mw4a8_quant_rows(p, 20, 4, 20, p, 24, p, None) == -1
    assert L.mw4a8_quant_rows(ctypes.c_void_p(4098), 64, 4, 64, p, 64, p, None) == -1
    assert L.mw4a8_quant_rows(p, 64, 4, 64, None, 64, p, None) == -1
    assert L.mw4a8_quant_rows(p, 64, 0, 64, p, 64, p, None) == 0
    # router: too many experts, topk > E, topk > 64
    assert L.mw4a8_router_topk(p, 2048, 4, 2048, 8, 1, p, p, None) == -2
    assert L.mw4a8_router_topk(p, 8, 4, 8, 9, 1, p, p, None) == -2
    assert L.mw4a8_router_topk(p, 256, 4, 256, 65, 1, p, p, None) == -2
    assert L.mw4a8_router_topk(p, 4, 4, 8, 2, 1, p, p, None) == -1          # ld < E
    # silu: row stride shorter than both halves
    assert L.mw4a8_silu_mul_quant(p, 64, 4, 64, p, 64, p, None) == -1
    assert L.mw4a8_silu_mul_quant(p, 128, 4, 12, p, 64, p, None) == -1      # I % 8
    # combine: N not a multiple of 8, null output, misaligned weights
    assert L.mw4a8_combine_topk(p, 12, 4, 2, 12, None, p, 12, None) == -1
    assert L.mw4a8_combine_topk(p, 64, 4, 2, 64, None, None, 64, None) == -1
    assert L.mw4a8_combine_topk(p, 64, 4, 2, 64, ctypes.c_void_p(4098), p, 64, None) == -1


def test_repack_entry_rejects_bad_arguments(pkg):
    from flagos_kernel_gen_amd import _lib
    L = _lib.lib()
    p, q = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    assert L.mw4a8_repack_weights(p, q, 2, 4, 12, 0, None) == -1                      # K % 8
    assert L.mw4a8_repack_weights(p, p, 2, 4, 16, 0, None) == -1                      # in place
    assert L.mw4a8_repack_weights(ctypes.c_void_p(4100), q, 2, 4, 16, 0, None) == -1  # alignment
    assert L.mw4a8_repack_weights(p, q, 0, 4, 16, 0, None) == 0                       # nothing to do


def test_layer_wrappers_fail_loudly_on_cpu(pkg):
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.quant_per_token(x)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.router_topk(torch.zeros(4, 8), 2)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.silu_mul_quant(x)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.combine_topk(x, 2)
    with pytest.raises(TypeError):
        pkg.quant_per_token(x.float())
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.repack_weights(torch.zeros(2, 4, 8, dtype=torch.uint8))


def _cpu_args(M=4, E=2, N=32, K=256, gs=128):
    return (torch.zeros(M, K, dtype=torch.int8), torch.ones(M), torch.zeros(E, N, K // 2, dtype=torch.uint8),
            torch.ones(E, N, K // gs), torch.full((E, N, K // gs), 8, dtype=torch.int8),
            torch.tensor([0, 2, 4], dtype=torch.int32), torch.zeros(M, N, dtype=torch.bfloat16), gs)


def test_python_shape_errors_are_assertion_errors(pkg):
    a = list(_cpu_args())
    a[2] = torch.zeros(2, 32, 100, dtype=torch.uint8)       # K/2 mismatch
    with pytest.raises(AssertionError):
        pkg.w4a8_group_gemm_moe(*a)
    a = list(_cpu_args())
    a[7] = 96                                                # K % group_size != 0
    with pytest.raises(pkg.W4A8ShapeError):
        pkg.w4a8_group_gemm_moe(*a)


def test_python_dtype_errors(pkg):
    a = list(_cpu_args())
    a[0] = a[0].to(torch.int16)
    with pytest.raises(TypeError):
        pkg.w4a8_group_gemm_moe(*a)
    a = list(_cpu_args())
    a[6] = a[6].float()
    with pytest.raises(TypeError):
        pkg.w4a8_group_gemm_moe(*a)


def test_cpu_tensors_fail_loudly_no_fallback(pkg):
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.w4a8_group_gemm_moe(*_cpu_args())
    ids = torch.zeros(4, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.moe_align_block_size(ids, 16, 8)
    a = _cpu_args()
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.w4a8_fused_moe(a[0], a[1], a[2], a[3], a[4], ids, torch.ones(4, 2), group_size=128)


def test_missing_library_raises(monkeypatch, pkg):
    from flagos_kernel_gen_amd import _lib
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libmw4a8.so")
    with pytest.raises(_lib.LibraryNotBuilt):
        _lib.lib()


def test_workload_generators(pkg):
    wl = pkg.workloads
    inp = wl.make_routed_inputs(wl.CONFIGS["tiny"], 64)
    inp2 = wl.make_routed_inputs(wl.CONFIGS["tiny"], 64)
    assert torch.equal(inp.w_q4, inp2.w_q4) and torch.equal(inp.topk_ids, inp2.topk_ids)
    assert inp.x_q.abs().amax(dim=1).eq(127).all()
    assert torch.allclose(inp.topk_weights.sum(-1), torch.ones(64))
    assert inp.topk_ids.shape == (64, 2) and inp.w_zero.eq(8).all()
    assert float(inp.w_scale.min()) >= 0.005 and float(inp.w_scale.max()) <= 0.02
    # each token's experts are distinct
    assert (inp.topk_ids[:, 0] != inp.topk_ids[:, 1]).all()


def test_skewed_routing_meets_its_definition(pkg):
    wl = pkg.workloads
    ids, tw = wl.make_routing(4096, 256, 8, "zipf", seed=4 * 7 + 3)
    load = torch.bincount(ids.reshape(-1).long(), minlength=256)
    assert float(load.max()) > 10 * 4096 * 8 / 256
    assert int((load == 0).sum()) >= 1


def test_stream_read_utility_rejects_bad_arguments(pkg):
    from flagos_kernel_gen_amd import _lib
    L = _lib.lib()
    p, q = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    assert L.mw4a8_stream_read(p, 24, q, 4096, 256, None) == -1          # not a multiple of 16
    assert L.mw4a8_stream_read(p, 1024, q, 1024, 256, None) == -1        # sink too small
    assert L.mw4a8_stream_read(p, 1024, q, 4096, 0, None) == -1          # no workgroups
    assert L.mw4a8_stream_read(ctypes.c_void_p(4100), 1024, q, 4096, 8, None) == -1   # misaligned
    assert L.mw4a8_stream_read(p, 0, q, 4096, 8, None) == 0              # nothing to read
