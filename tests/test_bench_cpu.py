"""bench.py's accounting on the CPU: the algorithmic bytes and int8 ops that
every roofline figure divides by, checked against hand-worked values of the
formula bytes = sum over touched experts of (N*K/2 + 4*N*G + N*G)
+ M*K + 4*M + 8*M*topk + 2*M*topk*N, ops = 2*M*topk*N*K; and the one-GPU
contract of the command line."""

import os
import subprocess
import sys

import torch

from conftest import ROOT

sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_headline_bytes_and_ops_hand_worked(pkg):
    shape = pkg.workloads.CONFIGS["dsv3_up"]
    M = 4096
    ids = torch.arange(M * 8, dtype=torch.int32).reshape(M, 8) % 256     # all 256 experts touched
    a = bench.algorithmic(shape, M, ids)
    # per expert: 4096*3584 packed bytes + 4*4096*56 scale bytes + 4096*56 zero bytes
    per_expert = 14_680_064 + 917_504 + 229_376
    assert per_expert == 15_826_944
    act = 4096 * 7168 + 4 * 4096 + 8 * 4096 * 8           # x_q, x_scale, topk ids + weights
    out = 2 * 4096 * 8 * 4096                              # bf16 pair rows
    assert a["touched_experts"] == 256
    assert a["weight_bytes"] == 256 * per_expert == 4_051_697_664
    assert a["bytes"] == 4_051_697_664 + 29_638_656 + 268_435_456 == 4_349_771_776
    assert a["ops"] == 1_924_145_348_608


def test_touched_experts_count_distinct_ids(pkg):
    shape = pkg.workloads.MoEShape("t", 8, 2, 256, 64, (3,))
    ids = torch.tensor([[5, 5], [1, 5], [1, 1]], dtype=torch.int32)
    a = bench.algorithmic(shape, 3, ids)
    assert a["touched_experts"] == 2                      # experts 1 and 5 only
    G = 256 // 128
    assert a["weight_bytes"] == 2 * (64 * 128 + 4 * 64 * G + 64 * G)
    assert a["bytes"] == a["weight_bytes"] + 3 * 256 + 4 * 3 + 8 * 3 * 2 + 2 * 3 * 2 * 64
    assert a["ops"] == 2 * 3 * 2 * 64 * 256


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""
