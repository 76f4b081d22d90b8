"""MI355X-native W4A8 fused-MoE grouped GEMM (hand-written HIP for gfx950).

Public API:

* ``w4a8_group_gemm_moe(x_q, x_scale, w_q4_packed, w_scale, w_zero,
  expert_offsets, out, group_size)`` -- drop-in for the reference operator
  (docs/Task1.md:8-17).
* ``moe_align_block_size(topk_ids, block_m, num_experts)`` -- routing metadata.
* ``w4a8_fused_moe(x_q, x_scale, w_q4_packed, w_scale, w_zero, topk_ids,
  topk_weights, group_size)`` -- routed GEMM with the top-k weight epilogue.
* ``w4a8_group_partials`` / ``w4a8_fused_moe_partials`` -- debug exports of the
  int32 group partial sums (reference layout / routed), from the product kernels.
* ``repack_weights`` -- offline conversion to the MFMA weight order
  (``w4a8_fused_moe(..., weight_layout="mfma")``).
* ``quant_per_token``, ``router_topk``, ``silu_mul_quant``, ``combine_topk``
  and ``w4a8_moe_layer`` -- the MoE layer around the GEMM (layer.py).

The package directory name contains hyphens, so it is imported under the
module name ``flagos_kernel_gen_amd`` (see ``__graft_entry__.import_package``).
"""

from .moe import (W4A8ShapeError, align_buffer_sizes, moe_align_block_size, repack_weights, select_block_m,
                  w4a8_fused_moe, w4a8_fused_moe_partials, w4a8_group_gemm_moe, w4a8_group_partials)
from .layer import combine_topk, quant_per_token, router_topk, silu_mul_quant, w4a8_moe_layer
from . import workloads

__all__ = [
    "W4A8ShapeError",
    "align_buffer_sizes",
    "moe_align_block_size",
    "repack_weights",
    "select_block_m",
    "w4a8_fused_moe",
    "w4a8_fused_moe_partials",
    "w4a8_group_gemm_moe",
    "w4a8_group_partials",
    "workloads",
    "combine_topk",
    "quant_per_token",
    "router_topk",
    "silu_mul_quant",
    "w4a8_moe_layer",
]
