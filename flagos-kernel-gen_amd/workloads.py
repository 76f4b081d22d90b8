"""Named shapes and seeded synthetic inputs for the W4A8 MoE path.

Shapes:

* ``CONFIGS`` -- the five benchmark configurations (tiny, Mixtral-8x7B
  decode, Qwen3-30B-A3B, DeepSeek-V3 up/gate and down, DeepSeek-V3 with
  Zipf-skewed routing).
* ``TASK1_WORKLOADS`` -- the ten (E, M_total, N, K, group_size) workloads
  the reference contest used (docs/Task1.md:30-41), in the reference layout.

Inputs follow one recipe everywhere:

* weights: symmetric int4 ``w ~ U{-8..7}`` stored as nibble ``u = w + 8``
  (so every packed byte is uniform on 0..255), ``w_zero = 8``, group scales
  ``U[0.005, 0.02]``;
* activations: ``x ~ N(0, 1)`` in bf16, per-token scale ``amax|x| / 127``,
  ``x_q = clamp(round_half_even(x / scale), -127, 127)``;
* routing: softmax top-k over ``N(0, 1)`` logits with renormalised weights;
  uniformly random distinct experts for the Qwen3 shape; ``N(0, 1)`` logits
  plus a Zipf(1.2) per-expert bias for the skewed shape.

All generation uses ``torch.Generator`` seeded from the config, on the device
requested, so a run is reproducible on that device.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class MoEShape:
    name: str
    E: int
    topk: int
    K: int
    N: int
    Ms: tuple
    group_size: int = 128
    routing: str = "softmax"   # softmax | uniform | zipf


CONFIGS = {
    "tiny": MoEShape("tiny", 8, 2, 1024, 2048, (64,)),
    "mixtral_up": MoEShape("mixtral_up", 8, 2, 4096, 28672, (1, 8, 32)),
    "qwen3_up": MoEShape("qwen3_up", 128, 8, 2048, 1536, (16, 256, 2048), routing="uniform"),
    "dsv3_up": MoEShape("dsv3_up", 256, 8, 7168, 4096, (1, 64, 4096)),
    "dsv3_down": MoEShape("dsv3_down", 256, 8, 2048, 7168, (1, 64, 4096)),
    "dsv3_skew": MoEShape("dsv3_skew", 256, 8, 7168, 4096, (4096,), routing="zipf"),
}

# (E, M_total, N, K, group_size), docs/Task1.md:30-41
TASK1_WORKLOADS = (
    (4, 32, 512, 512, 128),
    (8, 64, 1024, 1024, 128),
    (8, 128, 1408, 2048, 128),
    (8, 256, 2048, 2048, 128),
    (16, 128, 1024, 1536, 64),
    (16, 256, 1536, 2048, 128),
    (32, 256, 1408, 2048, 128),
    (32, 512, 2048, 4096, 128),
    (64, 512, 1024, 2048, 128),
    (64, 1024, 2048, 4096, 128),
)


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def make_weights(E, N, K, group_size, seed, device="cpu", zero="symmetric"):
    """Packed int4 weights ``[E, N, K/2]`` u8, scales and zero points ``[E, N, G]``.

    ``zero``: ``"symmetric"`` (all 8), ``"uint4"`` (random 0..15) or
    ``"full"`` (random over the whole int8 range, which exercises the
    int16 -> int8 wrap of the zero fold).
    """
    g = _gen(seed, device)
    G = K // group_size
    packed = torch.randint(0, 256, (E, N, K // 2), dtype=torch.uint8, generator=g, device=device)
    scale = torch.empty(E, N, G, dtype=torch.float32, device=device).uniform_(0.005, 0.02, generator=g)
    if zero == "symmetric":
        wz = torch.full((E, N, G), 8, dtype=torch.int8, device=device)
    elif zero == "uint4":
        wz = torch.randint(0, 16, (E, N, G), dtype=torch.int8, generator=g, device=device)
    elif zero == "full":
        wz = torch.randint(-128, 128, (E, N, G), dtype=torch.int8, generator=g, device=device)
    else:
        raise ValueError(f"unknown zero mode {zero!r}")
    return packed, scale, wz


def quantize_per_token(x: torch.Tensor):
    """bf16/fp32 activations -> (int8 [M, K], fp32 scale [M])."""
    xf = x.to(torch.float32)
    amax = xf.abs().amax(dim=1).clamp_min(1e-12)
    scale = amax / 127.0
    xq = torch.round(xf / scale[:, None]).clamp_(-127, 127).to(torch.int8)
    return xq, scale


def make_activations(M, K, seed, device="cpu"):
    g = _gen(seed, device)
    x = torch.randn(M, K, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    return quantize_per_token(x)


def make_routing(M, E, topk, kind, seed, device="cpu"):
    """Return ``(topk_ids int32 [M, topk], topk_weights fp32 [M, topk])``."""
    g = _gen(seed, device)
    if kind == "softmax":
        logits = torch.randn(M, E, generator=g, device=device)
        probs = torch.softmax(logits, dim=-1)
        w, ids = torch.topk(probs, topk, dim=-1)
    elif kind == "uniform":
        logits = torch.rand(M, E, generator=g, device=device)
        _, ids = torch.topk(logits, topk, dim=-1)
        w = torch.softmax(logits, dim=-1).gather(1, ids)
    elif kind == "zipf":
        noise = torch.randn(M, E, generator=g, device=device)
        rank = torch.randperm(E, generator=g, device=device).to(torch.float32) + 1.0
        bias = rank.pow(-1.2)
        c = 8.0
        while True:
            logits = noise + c * bias
            w, ids = torch.topk(torch.softmax(logits, dim=-1), topk, dim=-1)
            load = torch.bincount(ids.reshape(-1).to(torch.int64), minlength=E)
            mean = M * topk / E
            if float(load.max()) > 10.0 * mean and int((load == 0).sum()) >= 1:
                break
            c *= 2.0
            if c > 1e4:
                raise RuntimeError("could not reach the requested routing skew")
    else:
        raise ValueError(f"unknown routing kind {kind!r}")
    w = w / w.sum(dim=-1, keepdim=True)
    return ids.to(torch.int32).contiguous(), w.to(torch.float32).contiguous()


@dataclass
class RoutedInputs:
    shape: MoEShape
    M: int
    x_q: torch.Tensor
    x_scale: torch.Tensor
    w_q4: torch.Tensor
    w_scale: torch.Tensor
    w_zero: torch.Tensor
    topk_ids: torch.Tensor
    topk_weights: torch.Tensor
    extra: dict = field(default_factory=dict)


def seed_for(shape: MoEShape, M: int) -> int:
    base = {"tiny": 0, "mixtral_up": 1, "qwen3_up": 2, "dsv3_up": 3, "dsv3_down": 3, "dsv3_skew": 4}
    return 1000 * base.get(shape.name, 9) + M


def make_routed_inputs(shape: MoEShape, M: int, device="cpu", zero="symmetric") -> RoutedInputs:
    s = seed_for(shape, M)
    w_q4, w_scale, w_zero = make_weights(shape.E, shape.N, shape.K, shape.group_size,
                                         s * 7 + 1 + (11 if shape.name == "dsv3_down" else 0),
                                         device, zero)
    x_q, x_scale = make_activations(M, shape.K, s * 7 + 2, device)
    ids, tw = make_routing(M, shape.E, shape.topk, shape.routing, s * 7 + 3, device)
    return RoutedInputs(shape, M, x_q, x_scale, w_q4, w_scale, w_zero, ids, tw)


def make_grouped_inputs(E, M_total, N, K, group_size, seed, device="cpu", zero="symmetric"):
    """Reference-layout inputs: rows already grouped by expert plus CSR offsets.

    Each row draws its expert uniformly; rows are then laid out by expert,
    so some experts may own no rows.
    """
    g = _gen(seed, device)
    owner = torch.randint(0, E, (M_total,), generator=g, device=device)
    counts = torch.bincount(owner, minlength=E)
    offsets = torch.zeros(E + 1, dtype=torch.int32, device=device)
    offsets[1:] = torch.cumsum(counts, 0).to(torch.int32)
    x_q, x_scale = make_activations(M_total, K, seed * 7 + 2, device)
    w_q4, w_scale, w_zero = make_weights(E, N, K, group_size, seed * 7 + 1, device, zero)
    return x_q, x_scale, w_q4, w_scale, w_zero, offsets
