// Routing metadata kernels for gfx950.
//
// moe_align_kernel: token-expert pairs -> expert-sorted, block-padded slots.
//   One workgroup of 1024 threads (16 wave64s):
//   1. LDS histogram of expert ids (ids outside [0, E) are not routed).
//   2. Workgroup scan of per-expert block counts and pair counts.
//   3. Padding slots, expert_ids and the tails of both buffers are written
//      directly from the scan (each expert owns at most BM-1 padding slots).
//   4. Stable scatter in rounds of 1024 consecutive pairs. Inside a wave the
//      lanes holding the same expert are found with one ballot per id bit;
//      a lane's rank is the popcount of its peers below it. Wave counts go
//      through LDS so later waves add the counts of earlier ones, and a
//      running per-expert cursor carries counts across rounds. Slot order
//      within an expert is therefore ascending pair index, independent of
//      scheduling, which makes the output bit-exact with a stable sort.
//
// csr_block_table_kernel: CSR expert_offsets (reference layout,
//   docs/Task1.md:87-92) -> list of (expert, first row, end row) blocks of
//   at most BM rows, so the GEMM grid needs no host-side count.
#include "mw4a8_internal.h"

namespace mw4a8 {

constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kAlignMaxE = 1024;

// Exclusive scan of one int per thread across a 1024-thread workgroup.
// `wave_sums` must hold kAlignWaves ints. Returns the exclusive prefix and
// writes the workgroup total to *total (same value in every thread).
__device__ __forceinline__ int block_exclusive_scan(int v, int* wave_sums, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
  if (lane == 63) wave_sums[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    int ws = lane < kAlignWaves ? wave_sums[lane] : 0;
#pragma unroll
    for (int d = 1; d < kAlignWaves; d <<= 1) {
      const int o = __shfl_up(ws, d, 64);
      if (lane >= d) ws += o;
    }
    if (lane < kAlignWaves) wave_sums[lane] = ws;   // inclusive wave prefix
  }
  __syncthreads();
  const int before = wave > 0 ? wave_sums[wave - 1] : 0;
  *total = wave_sums[kAlignWaves - 1];
  __syncthreads();   // wave_sums may be reused by the caller
  return before + inc - v;
}

__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(
    const int32_t* __restrict__ topk_ids, int P, int E, int BM, int id_bits,
    int32_t* __restrict__ sorted_ids, int sorted_len,
    int32_t* __restrict__ expert_ids, int blocks_len,
    int32_t* __restrict__ num_post_pad, int32_t* __restrict__ expert_offsets) {
  __shared__ int s_cnt[kAlignMaxE];
  __shared__ int s_cur[kAlignMaxE];
  __shared__ int s_boff[kAlignMaxE + 1];
  __shared__ uint8_t s_wcnt[kAlignWaves][kAlignMaxE];
  __shared__ int s_wave[kAlignWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int e = tid; e < E; e += kAlignThreads) { s_cnt[e] = 0; s_cur[e] = 0; }
  for (int i = tid; i < kAlignWaves * kAlignMaxE / 4; i += kAlignThreads)
    reinterpret_cast<int*>(&s_wcnt[0][0])[i] = 0;
  __syncthreads();

  // 1. histogram
  for (int i = tid; i < P; i += kAlignThreads) {
    const int e = topk_ids[i];
    if ((unsigned)e < (unsigned)E) atomicAdd(&s_cnt[e], 1);
  }
  __syncthreads();

  // 2. scans (E <= 1024: one expert per thread)
  const int my_cnt = tid < E ? s_cnt[tid] : 0;
  const int my_blk = (my_cnt + BM - 1) / BM;
  int tot_blk, tot_cnt;
  const int blk_ex = block_exclusive_scan(my_blk, s_wave, &tot_blk);
  const int cnt_ex = block_exclusive_scan(my_cnt, s_wave, &tot_cnt);
  if (tid < E) {
    s_boff[tid] = blk_ex;
    if (expert_offsets) expert_offsets[tid] = cnt_ex;
  }
  if (tid == 0) {
    s_boff[E] = tot_blk;
    if (expert_offsets) expert_offsets[E] = tot_cnt;
    num_post_pad[0] = tot_blk * BM;
  }
  __syncthreads();

  // 3. padding slots, block owners, buffer tails
  if (tid < E) {
    const int first = blk_ex * BM;
    for (int s = first + my_cnt; s < first + my_blk * BM; ++s) sorted_ids[s] = P;
    for (int b = blk_ex; b < blk_ex + my_blk; ++b) expert_ids[b] = tid;
  }
  for (int s = tot_blk * BM + tid; s < sorted_len; s += kAlignThreads) sorted_ids[s] = P;
  for (int b = tot_blk + tid; b < blocks_len; b += kAlignThreads) expert_ids[b] = -1;

  // 4. stable scatter
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = 0; base < P; base += kAlignThreads) {
    const int i = base + tid;
    const int e = i < P ? topk_ids[i] : -1;
    const bool valid = (unsigned)e < (unsigned)E;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < id_bits; ++bit) {
      const bool set = (e >> bit) & 1;
      const uint64_t m = __ballot(set);
      peers &= set ? m : ~m;
    }
    const int rank = __popcll(peers & lt_mask);
    const int wcount = __popcll(peers);
    if (valid && rank == 0) s_wcnt[wave][e] = (uint8_t)wcount;
    __syncthreads();
    if (valid) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += s_wcnt[w][e];
      sorted_ids[s_boff[e] * BM + s_cur[e] + before + rank] = i;
    }
    __syncthreads();
    if (valid && rank == 0) {
      atomicAdd(&s_cur[e], wcount);
      s_wcnt[wave][e] = 0;
    }
    __syncthreads();
  }
}

hipError_t launch_moe_align(const int32_t* topk_ids, int num_pairs, int E, int BM,
                            int32_t* sorted_ids, int sorted_len, int32_t* expert_ids, int blocks_len,
                            int32_t* num_post_pad, int32_t* expert_offsets, hipStream_t s) {
  int id_bits = 0;
  while ((1 << id_bits) < E) ++id_bits;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kAlignThreads), 0, s, topk_ids, num_pairs, E, BM,
                     id_bits, sorted_ids, sorted_len, expert_ids, blocks_len, num_post_pad, expert_offsets);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kAlignThreads) void csr_block_table_kernel(
    const int32_t* __restrict__ offsets, int E, int M_total, int BM, int max_blocks,
    int32_t* __restrict__ blk_expert, int32_t* __restrict__ blk_row0, int32_t* __restrict__ blk_row1,
    int32_t* __restrict__ blk_count) {
  __shared__ int s_wave[kAlignWaves];
  const int tid = threadIdx.x;
  int carry = 0;
  for (int e0 = 0; e0 < E; e0 += kAlignThreads) {
    const int e = e0 + tid;
    int r0 = 0, r1 = 0;
    if (e < E) {
      r0 = min(max(offsets[e], 0), M_total);
      r1 = min(max(offsets[e + 1], 0), M_total);
    }
    const int rows = r1 > r0 ? r1 - r0 : 0;
    const int nb = (rows + BM - 1) / BM;
    int chunk_total;
    const int first = carry + block_exclusive_scan(nb, s_wave, &chunk_total);
    for (int j = 0; j < nb; ++j) {
      const int b = first + j;
      if (b >= max_blocks) break;
      blk_expert[b] = e;
      blk_row0[b] = r0 + j * BM;
      blk_row1[b] = min(r0 + (j + 1) * BM, r1);
    }
    carry += chunk_total;
  }
  for (int b = carry + tid; b < max_blocks; b += kAlignThreads) {
    blk_expert[b] = -1;
    blk_row0[b] = 0;
    blk_row1[b] = 0;
  }
  if (tid == 0) {
    blk_count[0] = min(carry, max_blocks);
    blk_count[1] = carry;   // > max_blocks only for overlapping (non-CSR) offsets
  }
}

hipError_t launch_csr_block_table(const int32_t* offsets, int E, int M_total, int BM, int max_blocks,
                                  int32_t* blk_expert, int32_t* blk_row0, int32_t* blk_row1,
                                  int32_t* blk_count, hipStream_t s) {
  hipLaunchKernelGGL(csr_block_table_kernel, dim3(1), dim3(kAlignThreads), 0, s, offsets, E, M_total, BM,
                     max_blocks, blk_expert, blk_row0, blk_row1, blk_count);
  return hipGetLastError();
}

}  // namespace mw4a8
