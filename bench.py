"""Benchmark of the MI355X W4A8 fused-MoE path (one JSON line on stdout).

Headline workload: DeepSeek-V3 shape, up/gate projection (E=256, topk=8,
K=7168, N=4096, int4 group 128), M=4096 tokens. One step is one routed call
``w4a8_fused_moe`` = routing kernel + grouped GEMM on inputs resident in HBM.

The JSON line carries ``value`` = microseconds per step, the GEMM kernel's
roofline (algorithmic bytes and int8 ops per launch divided by its average
duration from HIP events on the launch stream, >= 50 launches, mean and
median), every other configuration point as ``points`` (decode points with
the rate of a plain cold read of the same byte count beside them), the
drop-in reference-layout operator on the reference's ten workloads as
``dropin`` (with the CPU oracle on the same inputs), two DeepSeek-V3 MoE
layers as ``layers``, and the CPU baseline: the oracle restatement of the
reference operator timed on a bounded sample of the headline workload on the
host cores, scaled to one call.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--points all|none|name:M,...]
                       [--no-cpu] [--cpu-seconds S] [--no-dropin] [--no-layer]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA
HEADLINE = ("dsv3_up", 4096)
ALL_POINTS = ("tiny:64", "mixtral_up:1", "mixtral_up:8", "mixtral_up:32", "qwen3_up:16", "qwen3_up:256",
              "qwen3_up:2048", "dsv3_up:1", "dsv3_up:64", "dsv3_down:1", "dsv3_down:64", "dsv3_down:4096",
              "dsv3_skew:4096")
DEFAULT_POINTS = ALL_POINTS
# decode points (HBM-bound, judged against the >= 70 % of HBM target): each
# also gets the measured rate of a plain cold read of the same byte count
DECODE_POINTS = ("mixtral_up:1", "mixtral_up:8", "mixtral_up:32", "qwen3_up:16", "dsv3_up:1", "dsv3_up:64",
                 "dsv3_down:1", "dsv3_down:64")
ROTATE_BYTES = 1 << 30       # keep > 4x the 256 MB Infinity Cache in rotation
MIN_EVENTS = 50              # HIP-event samples per kernel timing (median of >= 50)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic(shape, M, topk_ids):
    """Bytes and int8 ops one routed call must move/execute (padding excluded)."""
    import torch
    E, N, K, gs, topk = shape.E, shape.N, shape.K, shape.group_size, shape.topk
    G = K // gs
    touched = int(torch.unique(topk_ids).numel())
    w_bytes = touched * (N * K // 2 + 4 * N * G + N * G)
    act = M * K + 4 * M + 8 * M * topk
    out = 2 * M * topk * N
    return {"touched_experts": touched, "bytes": w_bytes + act + out, "weight_bytes": w_bytes,
            "ops": 2 * M * topk * N * K}


class Point:
    """Inputs of one (shape, M) point, with rotation sets for cold-HBM timing."""

    def __init__(self, pkg, name, M, dev):
        import torch
        wl = pkg.workloads
        self.pkg, self.shape, self.M, self.dev = pkg, wl.CONFIGS[name], M, dev
        s = self.shape
        base = wl.make_routed_inputs(s, M, device=dev)
        self.inputs = [base]
        # rotate distinct weight copies while all of them are smaller than ROTATE_BYTES
        wbytes = base.w_q4.numel() + 5 * base.w_zero.numel()
        ncopies = max(1, min(8, -(-ROTATE_BYTES // max(wbytes, 1))))
        for c in range(1, ncopies):
            w, ws, wz = wl.make_weights(s.E, s.N, s.K, s.group_size, seed=9000 + 31 * c, device=dev)
            self.inputs.append(wl.RoutedInputs(s, M, base.x_q, base.x_scale, w, ws, wz, base.topk_ids,
                                               base.topk_weights))
        # small M touches few experts: rotate routings so each call streams cold experts
        self.routings = [(base.topk_ids, base.topk_weights)]
        if M * s.topk < s.E:
            for r in range(1, 16):
                self.routings.append(wl.make_routing(M, s.E, s.topk, s.routing, seed=777 + r, device=dev))
        self.block_m = pkg.select_block_m(M * s.topk, s.E, s.N, s.K, s.group_size)
        self.aligned = [pkg.moe_align_block_size(ids, self.block_m, s.E) for ids, _ in self.routings]
        self.out = torch.empty(M * s.topk, s.N, dtype=torch.bfloat16, device=dev)
        self.weight_layout = "reference"
        self.n_sets = max(len(self.inputs), len(self.routings))
        self.alg = [algorithmic(s, M, self.routings[i % len(self.routings)][0]) for i in range(self.n_sets)]

    def _args(self, i):
        inp = self.inputs[i % len(self.inputs)]
        ids, tw = self.routings[i % len(self.routings)]
        return inp, ids, tw

    def step(self, i):
        """Full routed call: routing kernel + grouped GEMM."""
        inp, ids, tw = self._args(i)
        self.pkg.w4a8_fused_moe(inp.x_q, inp.x_scale, inp.w_q4, inp.w_scale, inp.w_zero, ids, tw,
                                group_size=self.shape.group_size, out=self.out, block_m=self.block_m)

    def gemm(self, i):
        """Grouped GEMM only, on precomputed routing metadata."""
        inp, ids, tw = self._args(i)
        self.pkg.w4a8_fused_moe(inp.x_q, inp.x_scale, inp.w_q4, inp.w_scale, inp.w_zero, ids, tw,
                                group_size=self.shape.group_size, out=self.out, block_m=self.block_m,
                                routing=self.aligned[i % len(self.routings)], weight_layout=self.weight_layout)


def time_steps(fn, n, warmup):
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / n


def kernel_events(fn, n, warmup):
    """Average duration of fn's launches from HIP events on the current stream."""
    import torch
    for i in range(warmup):
        fn(i)
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        fn(i)
        b.record(stream)
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in evs]
    return statistics.mean(ms) * 1e3, statistics.median(ms) * 1e3


def prime(fn, min_ms=100.0):
    """Untimed run of fn until ~min_ms of GPU work has completed, so that the
    timed phases start with the GPU at its working clock (the first timed
    phase after input generation otherwise measured ~5 % slow)."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    i = 0
    while True:
        fn(i)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= min_ms:
                break
    torch.cuda.synchronize()


def cold_read_ceiling(pkg, nbytes, dev, steps, warmup):
    """Memory ceiling of a point: the HBM rate of moving ``nbytes`` cold, by
    two plain streaming kernels over equally sized buffers rotated through
    more than ``ROTATE_BYTES`` (each pass misses the 256 MB Infinity Cache):

    * ``stream``: the library's measurement kernel ``mw4a8_stream_read``
      (coalesced 16-byte loads, eight in flight per thread), the better of a
      2048- and a 256-workgroup grid;
    * ``torch_copy``: ``Tensor.copy_`` of ``nbytes / 2`` (reads and writes
      ``nbytes`` in all) -- the fastest plain torch op on this box (its
      reductions stay below 4 TB/s).

    Returns a dict of GB/s (median of the HIP-event timings) per method."""
    import ctypes
    import torch
    from flagos_kernel_gen_amd import _lib
    L = _lib.lib()
    n16 = max(1, nbytes // 16)
    nbuf = max(2, min(64, -(-ROTATE_BYTES // (16 * n16)) + 1))
    bufs = [torch.empty(16 * n16, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
    sink = torch.zeros(4096, dtype=torch.uint8, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    out = {}
    best = None
    for blocks in (2048, 256):
        def read(i, blocks=blocks):
            _lib.check(L.mw4a8_stream_read(ctypes.c_void_p(bufs[i % nbuf].data_ptr()), 16 * n16,
                                           ctypes.c_void_p(sink.data_ptr()), 4096, blocks, stream),
                       "mw4a8_stream_read")
        prime(read, 20.0)
        _, med_us = kernel_events(read, steps, warmup)
        gbs = 16 * n16 / (med_us * 1e-6) / 1e9
        best = gbs if best is None else max(best, gbs)
    out["stream"] = round(best, 1)
    half = [b[: 8 * n16] for b in bufs]
    dst = torch.empty(8 * n16, dtype=torch.uint8, device=dev)

    def copy(i):
        dst.copy_(half[i % nbuf])

    prime(copy, 20.0)
    _, med_us = kernel_events(copy, steps, warmup)
    out["torch_copy"] = round(16 * n16 / (med_us * 1e-6) / 1e9, 1)
    del bufs, half, dst
    torch.cuda.empty_cache()
    return out


def measure_point(pt, steps, warmup, ceiling=False):
    """Routed call (host clock over ``steps`` calls) and GEMM kernel (HIP
    events over at least ``MIN_EVENTS`` launches: mean and median). With
    ``ceiling`` the point also reports the rate of a plain cold read of its
    algorithmic byte count (``cold_read_ceiling``) and the GEMM's fraction of
    it."""
    prime(pt.step)
    us_step = time_steps(pt.step, steps, warmup) * 1e6
    n_ev = max(steps, MIN_EVENTS)
    us_gemm, us_gemm_med = kernel_events(pt.gemm, n_ev, warmup)
    n = pt.n_sets
    bytes_ = statistics.mean(pt.alg[i % n]["bytes"] for i in range(n_ev))
    ops = pt.alg[0]["ops"]
    gbs = bytes_ / (us_gemm * 1e-6) / 1e9
    gbs_med = bytes_ / (us_gemm_med * 1e-6) / 1e9
    tops = ops / (us_gemm * 1e-6) / 1e12
    res = {
        "workload": f"{pt.shape.name}:M={pt.M}", "E": pt.shape.E, "topk": pt.shape.topk, "K": pt.shape.K,
        "N": pt.shape.N, "block_m": pt.block_m, "us_per_call": round(us_step, 2),
        "gemm_us": round(us_gemm, 2), "gemm_us_median": round(us_gemm_med, 2), "gemm_events": n_ev,
        "touched_experts": pt.alg[0]["touched_experts"], "alg_bytes": int(bytes_), "alg_ops": int(ops),
        "gemm_GBps": round(gbs, 1), "gemm_TOPS": round(tops, 2),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "hbm_frac_median": round(gbs_med / HBM_PEAK_GBS, 4),
        "mfma_frac": round(tops / INT8_PEAK_TOPS, 4),
        "weight_sets": len(pt.inputs), "routing_sets": len(pt.routings),
    }
    if ceiling:
        ceil = cold_read_ceiling(pt.pkg, int(bytes_), pt.dev, n_ev, warmup)
        top = max(ceil.values())
        res["ceiling_GBps"] = ceil
        res["gemm_over_ceiling_median"] = round(gbs_med / top, 4)
    return res


def dropin_algorithmic(E, M, N, K, gs, offsets):
    """Bytes and int8 ops of one reference-layout call: the weights of every
    expert that owns rows, the activation rows with their scales, the CSR
    offsets and the bf16 output rows."""
    G = K // gs
    offs = [min(max(int(v), 0), M) for v in offsets.tolist()]
    rows = [max(0, b - a) for a, b in zip(offs[:-1], offs[1:])]
    touched = sum(1 for r in rows if r > 0)
    covered = sum(rows)
    nbytes = touched * (N * K // 2 + 4 * N * G + N * G) + covered * K + 4 * covered + 4 * (E + 1) + 2 * covered * N
    return {"touched_experts": touched, "rows": covered, "bytes": nbytes, "ops": 2 * covered * N * K}


def measure_dropin(pkg, dev, steps, warmup, cpu=True):
    """The drop-in entry ``w4a8_group_gemm_moe`` on the reference's ten
    workloads (docs/Task1.md:30-41): µs per operator call (HIP events around
    the call: block-table kernel + GEMM; weight copies rotated so every call
    reads cold HBM), algorithmic GB/s and TOPS, and the CPU oracle on the
    same inputs (the reference's own all-expert unpack, docs/Task1.md:78-85)
    on the host cores."""
    import torch
    from oracle import task1_ref
    wl = pkg.workloads
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    results = []
    for idx, (E, M, N, K, gs) in enumerate(wl.TASK1_WORKLOADS):
        x_q, x_scale, w_q4, w_scale, w_zero, offs = wl.make_grouped_inputs(E, M, N, K, gs, seed=idx)
        alg = dropin_algorithmic(E, M, N, K, gs, offs)
        g_in = [t.to(dev) for t in (x_q, x_scale, offs)]
        wbytes = w_q4.numel() + 5 * w_zero.numel()
        ncopies = max(1, min(16, -(-ROTATE_BYTES // wbytes)))
        sets = [tuple(t.to(dev) for t in (w_q4, w_scale, w_zero))]
        for c in range(1, ncopies):
            sets.append(wl.make_weights(E, N, K, gs, seed=4000 + 17 * c + idx, device=dev))
        out = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)

        def call(i):
            w = sets[i % len(sets)]
            pkg.w4a8_group_gemm_moe(g_in[0], g_in[1], w[0], w[1], w[2], g_in[2], out, gs)

        prime(call, 30.0)
        n_ev = max(steps, MIN_EVENTS)
        us, us_med = kernel_events(call, n_ev, warmup)
        res = {"workload": f"task1[{idx}]", "E": E, "M_total": M, "N": N, "K": K, "group_size": gs,
               "op_us": round(us, 2), "op_us_median": round(us_med, 2), "events": n_ev,
               "weight_sets": len(sets), "touched_experts": alg["touched_experts"], "alg_bytes": alg["bytes"],
               "GBps": round(alg["bytes"] / (us * 1e-6) / 1e9, 1),
               "hbm_frac": round(alg["bytes"] / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
               "TOPS": round(alg["ops"] / (us * 1e-6) / 1e12, 3),
               "mfma_frac": round(alg["ops"] / (us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 5)}
        del sets, out, g_in
        torch.cuda.empty_cache()
        if cpu:
            ref_out = torch.zeros(M, N, dtype=torch.bfloat16)
            ts = []
            for rep in range(4):
                t0 = time.perf_counter()
                task1_ref.w4a8_group_gemm_moe_ref(x_q, x_scale, w_q4, w_scale, w_zero, offs, ref_out, gs,
                                                  unpack="all")
                ts.append(time.perf_counter() - t0)
                if sum(ts) > 3.0:
                    break
            cpu_us = statistics.median(ts[1:] if len(ts) > 1 else ts) * 1e6
            res.update({"cpu_us": round(cpu_us, 1), "cpu_cores": cores, "cpu_runs": len(ts),
                        "gpu_speedup_vs_cpu": round(cpu_us / us, 1)})
        results.append(res)
        log(json.dumps(res))
    return results


LAYER_POINTS = ("dsv3_layer:64", "dsv3_layer:4096")


class LayerPoint:
    """One DeepSeek-V3-shape MoE layer (E=256, topk=8, hidden 7168, expert
    intermediate 2048): bf16 tokens + router logits in, bf16 tokens out."""

    E, H, I, TOPK, GS = 256, 7168, 2048, 8, 128

    def __init__(self, pkg, M, dev):
        import torch
        wl = pkg.workloads
        self.pkg, self.M = pkg, M
        g = torch.Generator(device=dev).manual_seed(7000 + M)
        self.x = torch.randn(M, self.H, generator=g, device=dev).to(torch.bfloat16)
        self.logits = torch.randn(M, self.E, generator=g, device=dev)
        self.w13 = wl.make_weights(self.E, 2 * self.I, self.H, self.GS, seed=7101, device=dev)
        self.w2 = wl.make_weights(self.E, self.H, self.I, self.GS, seed=7102, device=dev)
        _, self.mid = self.layer(return_intermediates=True)
        torch.cuda.synchronize()

    def layer(self, i=0, return_intermediates=False):
        return self.pkg.w4a8_moe_layer(self.x, self.logits, *self.w13, *self.w2, topk=self.TOPK,
                                       group_size=self.GS, return_intermediates=return_intermediates)

    def stages(self):
        """(name, fn, algorithmic bytes) of the streaming kernels of the layer."""
        M, H, I, E, k = self.M, self.H, self.I, self.E, self.TOPK
        P = M * k
        pkg, mid = self.pkg, self.mid
        return [
            ("quant_rows", lambda i: pkg.quant_per_token(self.x), M * H * 2 + M * H + 4 * M),
            ("router_topk", lambda i: pkg.router_topk(self.logits, k), M * E * 4 + M * k * 8),
            ("silu_mul_quant", lambda i: pkg.silu_mul_quant(mid["h"]), P * 2 * I * 2 + P * I + 4 * P),
            ("combine_topk", lambda i: pkg.combine_topk(mid["y"], k), P * H * 2 + M * H * 2),
        ]


def measure_layer(pkg, M, dev, steps, warmup):
    import torch
    lp = LayerPoint(pkg, M, dev)
    prime(lp.layer)
    us = time_steps(lp.layer, steps, warmup) * 1e6
    out = {"workload": f"dsv3_layer:M={M}", "E": lp.E, "topk": lp.TOPK, "hidden": lp.H, "intermediate": lp.I,
           "us_per_layer": round(us, 2), "stages": []}
    for name, fn, nbytes in lp.stages():
        t, _ = kernel_events(fn, steps, warmup)
        out["stages"].append({"kernel": name, "us": round(t, 2), "alg_bytes": int(nbytes),
                              "GBps": round(nbytes / (t * 1e-6) / 1e9, 1),
                              "hbm_frac": round(nbytes / (t * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    del lp
    torch.cuda.empty_cache()
    return out


def cpu_baseline(pkg, budget_s):
    """Oracle restatement of the reference operator on the host cores.

    Sample: the headline routing's experts in ascending order, each with all
    of its routed rows, until about ``budget_s`` seconds of work; the time is
    scaled by (touched experts / sampled experts) to one call.
    """
    import torch
    from oracle import task1_ref
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    wl = pkg.workloads
    shape = wl.CONFIGS[HEADLINE[0]]
    M = HEADLINE[1]
    s = wl.seed_for(shape, M)
    x_q, x_scale = wl.make_activations(M, shape.K, s * 7 + 2)
    ids, tw = wl.make_routing(M, shape.E, shape.topk, shape.routing, s * 7 + 3)
    flat = ids.reshape(-1).long()
    experts = torch.unique(flat).tolist()
    G = shape.K // shape.group_size
    times, rows = [], 0
    spent = 0.0
    for i, e in enumerate(experts):
        g = torch.Generator().manual_seed(50_000 + e)
        w_q4 = torch.randint(0, 256, (shape.N, shape.K // 2), dtype=torch.uint8, generator=g)
        ws = torch.empty(shape.N, G).uniform_(0.005, 0.02, generator=g)
        wz = torch.full((shape.N, G), 8, dtype=torch.int8)
        pe = torch.nonzero(flat == e).flatten()
        tok = pe // shape.topk
        t0 = time.perf_counter()
        task1_ref.expert_rows_ref(x_q[tok], x_scale[tok], w_q4, ws, wz, shape.group_size, row_weight=tw.reshape(-1)[pe])
        dt = time.perf_counter() - t0
        if i > 0:            # first expert is warm-up
            times.append(dt)
            rows += pe.numel()
            spent += dt
        if spent >= budget_s or len(times) >= len(experts) - 1:
            break
    per_expert = statistics.mean(times)
    us = per_expert * len(experts) * 1e6
    return {"value": round(us, 1), "unit": "us/call", "cores": cores, "kind": "port",
            "sample": f"oracle (docs/Task1.md:53-114 restatement, per-expert unpack) on {len(times)} of "
                      f"{len(experts)} touched experts ({rows} routed rows) of {shape.name} M={M}, "
                      f"{spent:.1f} s, scaled x{len(experts) / len(times):.1f} to one call"}


def traffic_from_profiles():
    """HBM bytes per GEMM launch from the committed rocprofv3 PMC summary, if any."""
    path = os.path.join(ROOT, "profiles", "traffic_dsv3_up_4096.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--points", default="default")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--headline-only", action="store_true")
    ap.add_argument("--no-layer", action="store_true", help="skip the whole-MoE-layer measurements")
    ap.add_argument("--layers", default=",".join(p.split(":")[1] for p in LAYER_POINTS),
                    help="token counts of the DeepSeek-V3 MoE-layer measurements (comma list)")
    ap.add_argument("--layer-only", action="store_true",
                    help="measure only the MoE layers (profiling; prints their JSON, not the bench line)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB int32 read+write kernel (torch.neg) to calibrate "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE against known bytes")
    ap.add_argument("--workload", default=None,
                    help="name:M to measure instead of the headline (profiling); implies --headline-only")
    ap.add_argument("--no-dropin", action="store_true",
                    help="skip the reference-layout drop-in on the reference's ten workloads")
    ap.add_argument("--dropin-only", action="store_true",
                    help="measure only the drop-in workloads (profiling; prints their JSON, not the bench line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the expert-parallel sharding is a design note, not code)", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__
    pkg = __graft_entry__.import_package()
    dev = torch.device("cuda:0")

    if args.layer_only:
        layers = [measure_layer(pkg, int(m), dev, args.steps, args.warmup) for m in args.layers.split(",")]
        print(json.dumps({"layers": layers}), flush=True)
        return
    if args.dropin_only:
        print(json.dumps({"dropin": measure_dropin(pkg, dev, args.steps, args.warmup, cpu=not args.no_cpu)}),
              flush=True)
        return

    head_name, head_m = HEADLINE
    if args.workload:
        head_name, head_m = args.workload.split(":")[0], int(args.workload.split(":")[1])
        args.headline_only = True
    log(f"headline {head_name} M={head_m}")
    hp = Point(pkg, head_name, head_m, dev)
    head = measure_point(hp, args.steps, args.warmup)
    log(json.dumps(head))
    # the same GEMM on weights converted offline to the MFMA order (opt-in
    # layout; results bit-identical): reported beside the drop-in headline
    head_mfma = None
    if not args.headline_only:
        for inp in hp.inputs:
            inp.w_q4 = pkg.repack_weights(inp.w_q4)
        hp.weight_layout = "mfma"
        us_m, med_m = kernel_events(hp.gemm, max(args.steps, MIN_EVENTS), args.warmup)
        head_mfma = {"workload": head["workload"], "weight_layout": "mfma", "gemm_us": round(us_m, 2),
                     "gemm_us_median": round(med_m, 2),
                     "gemm_GBps": round(head["alg_bytes"] / (us_m * 1e-6) / 1e9, 1),
                     "gemm_TOPS": round(head["alg_ops"] / (us_m * 1e-6) / 1e12, 2)}
        log(json.dumps(head_mfma))
    del hp
    torch.cuda.empty_cache()

    points = []
    if not args.headline_only and args.points != "none":
        names = {"default": DEFAULT_POINTS, "all": ALL_POINTS}.get(args.points, tuple(args.points.split(",")))
        for item in names:
            name, M = item.split(":")
            log(f"point {name} M={M}")
            pt = Point(pkg, name, int(M), dev)
            # side points: at least 10 warm-up and 50 timed calls (mean and median);
            # decode points also measure the cold-read ceiling of their byte count
            points.append(measure_point(pt, max(args.steps, 50), max(args.warmup, 10), ceiling=item in DECODE_POINTS))
            log(json.dumps(points[-1]))
            del pt
            torch.cuda.empty_cache()

    dropin = []
    if not args.headline_only and not args.no_dropin:
        log("drop-in w4a8_group_gemm_moe on the reference's ten workloads")
        dropin = measure_dropin(pkg, dev, args.steps, max(args.warmup, 10), cpu=not args.no_cpu)

    layers = []
    if not args.headline_only and not args.no_layer:
        for M in (int(m) for m in args.layers.split(",")):
            log(f"layer dsv3 M={M}")
            layers.append(measure_layer(pkg, M, dev, max(args.steps, 50), max(args.warmup, 10)))
            log(json.dumps(layers[-1]))

    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(pkg, args.cpu_seconds)
        log(json.dumps(cpu))

    traffic = traffic_from_profiles()
    line = {
        "metric": "us/call + achieved HBM GB/s & int8 TOPS (% roofline), W4A8 MoE DeepSeek-V3 shape",
        "value": head["us_per_call"],
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_call"] / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x int4 -> int32, fp32 scales, bf16 out",
        "data": "synthetic (seeded int4 weights, per-token int8 activations, softmax top-8 routing)",
        "config": {"workload": "DeepSeek-V3 MoE up/gate, routed w4a8_fused_moe (moe_align + grouped GEMM)",
                   "E": 256, "topk": 8, "K": 7168, "N": 4096, "group_size": 128, "tokens": HEADLINE[1],
                   "block_m": head["block_m"]},
        "roofline": {"kernel": "w4a8_gemm_kernel (routed)", "bound": "hbm",
                     "achieved": head["gemm_GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": head["hbm_frac"], "traffic": traffic,
                     "alg_bytes_per_launch": head["alg_bytes"], "kernel_us": head["gemm_us"],
                     "mfma": {"achieved": head["gemm_TOPS"], "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                              "frac": head["mfma_frac"]}},
        "cpu_baseline": cpu,
        "headline": head,
        "headline_mfma_layout": head_mfma,
        "points": points,
        "dropin": dropin,
        "layers": layers,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
