"""CPU oracle for the W4A8 fused-MoE grouped GEMM path.

TEST INFRASTRUCTURE ONLY. Nothing in the product path (the package
``flagos-kernel-gen_amd`` and its HIP library) imports, links or calls this
package. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` use it, and only as the checker or as the timed CPU
baseline, never as the thing that is measured or shipped.

Contents
--------
``task1_ref``  Restatement, in torch on the CPU, of the reference operator
               ``w4a8_group_gemm_moe`` (docs/Task1.md:53-114): INT4 unpack,
               zero-point fold with int16->int8 wrap, per-group int8 partial
               sums (exact in fp32), group-scale reduction, token scale,
               bf16 store. Adds the routed extension (top-k weight epilogue
               and pair-row scatter), which has no reference counterpart.
``routing``    Closed form of the moe_align_block_size routing metadata
               (stable counting sort of token-expert pairs, padded per
               expert to a block multiple). No reference counterpart: the
               reference consumes its result as ``expert_offsets``.
``brute``      Independent int64 / float64 brute force used to pin the two
               modules above on small inputs.
``repack``     The offline weight repack to the MFMA order and back.
``layer_ref``  The MoE-layer steps around the GEMM that this build adds (no
               reference counterpart): per-token int8 quantization, router
               top-k, SiLU-gated product with requantization, top-k combine,
               and their composition into one layer.

Pinning status (how each function is checked before it is trusted) is listed
in each module's docstring.
"""
