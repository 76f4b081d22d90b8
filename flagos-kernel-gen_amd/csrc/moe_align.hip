// Routing metadata kernels for gfx950.
//
// moe_align_kernel: token-expert pairs -> expert-sorted, block-padded slots.
//   One workgroup of 1024 threads (16 wave64s):
//   1. Per-wave LDS histograms of expert ids (ids outside [0, E) are not
//      routed).
//   2. Workgroup scan of per-expert block counts and pair counts.
//   3. Padding slots, expert_ids and the tails of both buffers are written
//      directly from the scan (each expert owns at most BM-1 padding slots).
//   4. Stable scatter: wave w owns a contiguous range of pairs and its own
//      per-expert cursors, which start at the expert's padded offset plus the
//      counts of the waves before w. Inside a wave the lanes holding the same
//      expert are found with one ballot per id bit; a lane's rank is the
//      popcount of its peers below it. Slot order within an expert is
//      therefore ascending pair index, independent of scheduling, which makes
//      the output bit-exact with a stable sort. No workgroup barrier is
//      needed after the scan.
//
// moe_align_split_kernel: the same result from NB workgroups, for larger
//   pair counts (one workgroup's scattered stores were the bottleneck).
//   Every workgroup reads all the ids (they are small and stay in L2) and
//   counts, per expert, the pairs before its own segment and from it on; the
//   totals give every workgroup the same padded layout, the counts before the
//   segment its own starting slot per expert. It then scatters only its own
//   segment exactly as above, so the slot of a pair is the same as with one
//   workgroup. Padding slots, expert_ids and the tails are split over the
//   workgroups by expert and by slot. No workgroup depends on another.
//
// moe_align_small_kernel: the same result for at most 64 pairs (decode),
//   with no loop over experts. The first wave holds one pair per lane and
//   takes one ballot per id bit. From those ballots alone (read from the
//   top bit down) a lane gets the pairs of lower experts below it, and an
//   expert's padded block count is the number of its pairs whose rank is a
//   multiple of BM, so the same count over those "block heads" gives every
//   expert's first block. Pairs are stored at once; each head records its
//   block's expert and pair count in LDS. All four waves then write the
//   padding, expert_ids, expert_offsets (the same counts per expert from
//   the ballots, kept in LDS) and the tails (16-byte stores).
//
// csr_block_table_kernel: CSR expert_offsets (reference layout,
//   docs/Task1.md:87-92) -> list of (expert, first row, end row) blocks of
//   at most BM rows, so the GEMM grid needs no host-side count.
#include "mw4a8_internal.h"

namespace mw4a8 {

constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kAlignMaxE = 1024;
constexpr int kAlignCachedPairs = 32768;   // ids kept in LDS (16 bits each) up to this many pairs

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
  // per-wave expert counts; after the scan, each wave's next free slot per expert
  __shared__ int s_wcnt[kAlignWaves][kAlignMaxE];
  __shared__ int s_wave[kAlignWaves];
  // the pairs' expert ids, read once from HBM (0xffff = not routed)
  __shared__ uint16_t s_ids[kAlignCachedPairs];
  const bool cached = P <= kAlignCachedPairs;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int i = tid; i < kAlignWaves * kAlignMaxE; i += kAlignThreads) (&s_wcnt[0][0])[i] = 0;
  __syncthreads();

  // wave w owns the contiguous pair range [p0, p1)
  const int seg = (P + kAlignWaves - 1) / kAlignWaves;
  const int p0 = min(P, wave * seg);
  const int p1 = min(P, p0 + seg);

  // 1. per-wave histograms (ids outside [0, E) are not routed)
  // eight independent loads in flight per lane before any of them is used
  constexpr int kBatch = 8;
  for (int i0 = p0 + lane; i0 < p1; i0 += 64 * kBatch) {
    int ev[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int i = i0 + 64 * j;
      ev[j] = i < p1 ? topk_ids[i] : -1;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int i = i0 + 64 * j;
      const bool ok = (unsigned)ev[j] < (unsigned)E;
      if (cached && i < p1) s_ids[i] = ok ? (uint16_t)ev[j] : (uint16_t)0xffff;
      if (ok) atomicAdd(&s_wcnt[wave][ev[j]], 1);
    }
  }
  __syncthreads();

  // 2. per-expert totals, block and pair offsets (E <= 1024: one expert per
  //    thread), then each wave's first slot for the expert: the expert's
  //    padded start plus the counts of the waves before it
  int my_cnt = 0;
  if (tid < E) {
#pragma unroll
    for (int w = 0; w < kAlignWaves; ++w) my_cnt += s_wcnt[w][tid];
  }
  const int my_blk = (my_cnt + BM - 1) / BM;
  int tot_blk, tot_cnt;
  const int blk_ex = block_exclusive_scan(my_blk, s_wave, &tot_blk);
  const int cnt_ex = block_exclusive_scan(my_cnt, s_wave, &tot_cnt);
  if (tid < E) {
    int run = blk_ex * BM;
#pragma unroll
    for (int w = 0; w < kAlignWaves; ++w) {
      const int c = s_wcnt[w][tid];
      s_wcnt[w][tid] = run;
      run += c;
    }
    if (expert_offsets) expert_offsets[tid] = cnt_ex;
    const int first = blk_ex * BM;
    for (int sl = first + my_cnt; sl < first + my_blk * BM; ++sl) sorted_ids[sl] = P;
    for (int bb = blk_ex; bb < blk_ex + my_blk; ++bb) expert_ids[bb] = tid;
  }
  if (tid == 0) {
    if (expert_offsets) expert_offsets[E] = tot_cnt;
    num_post_pad[0] = tot_blk * BM;
  }
  for (int sl = tot_blk * BM + tid; sl < sorted_len; sl += kAlignThreads) sorted_ids[sl] = P;
  for (int bb = tot_blk + tid; bb < blocks_len; bb += kAlignThreads) expert_ids[bb] = -1;
  __syncthreads();

  // 3. stable scatter, each wave on its own range and its own cursors (no
  //    workgroup barriers): the lanes holding the same expert are found with
  //    one ballot per id bit; a lane's slot is the wave's cursor plus the
  //    number of such lanes below it, and the lowest of them advances the
  //    cursor. The read of the cursor by every lane precedes the leader's
  //    write in the wave's LDS instruction order.
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = p0; base < p1; base += 64) {
    const int i = base + lane;
    int e = -1;
    if (i < p1) e = cached ? (s_ids[i] == 0xffff ? -1 : (int)s_ids[i]) : topk_ids[i];
    const bool valid = (unsigned)e < (unsigned)E;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < id_bits; ++bit) {
      const bool set = (e >> bit) & 1;
      const uint64_t m = __ballot(set);
      peers &= set ? m : ~m;
    }
    const int rank = __popcll(peers & lt_mask);
    const int count = __popcll(peers);
    int slot = 0;
    if (valid) slot = s_wcnt[wave][e] + rank;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      sorted_ids[slot] = i;
      if (rank == 0) s_wcnt[wave][e] = slot + count;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ __launch_bounds__(kAlignThreads) void moe_align_split_kernel(
    const int32_t* __restrict__ topk_ids, int P, int E, int BM, int id_bits,
    int32_t* __restrict__ sorted_ids, int sorted_len,
    int32_t* __restrict__ expert_ids, int blocks_len,
    int32_t* __restrict__ num_post_pad, int32_t* __restrict__ expert_offsets) {
  // per-wave counts of this segment; after the scan, each wave's next free slot
  __shared__ int s_wcnt[kAlignWaves][kAlignMaxE];
  __shared__ int s_pre[kAlignMaxE];    // pairs before the segment, per expert
  __shared__ int s_post[kAlignMaxE];   // pairs from the segment on, per expert
  __shared__ int s_wave[kAlignWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nb = gridDim.x, b = blockIdx.x;

  for (int i = tid; i < kAlignWaves * kAlignMaxE; i += kAlignThreads) (&s_wcnt[0][0])[i] = 0;
  for (int i = tid; i < kAlignMaxE; i += kAlignThreads) {
    s_pre[i] = 0;
    s_post[i] = 0;
  }
  __syncthreads();

  // this workgroup's segment [s0, s1); wave w owns [p0, p1) of it
  const int seg = (P + nb - 1) / nb;
  const int s0 = min(P, b * seg);
  const int s1 = min(P, s0 + seg);
  const int wseg = (s1 - s0 + kAlignWaves - 1) / kAlignWaves;
  const int p0 = min(s1, s0 + wave * wseg);
  const int p1 = min(s1, p0 + wseg);

  // 1. counts over all pairs: before the segment, from it on, and per owning
  //    wave inside it
  constexpr int kBatch = 8;
  for (int i0 = tid; i0 < P; i0 += kAlignThreads * kBatch) {
    int ev[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int i = i0 + kAlignThreads * j;
      ev[j] = i < P ? topk_ids[i] : -1;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int i = i0 + kAlignThreads * j;
      if ((unsigned)ev[j] < (unsigned)E) {
        atomicAdd(i < s0 ? &s_pre[ev[j]] : &s_post[ev[j]], 1);
        if (i >= s0 && i < s1) atomicAdd(&s_wcnt[min((i - s0) / wseg, kAlignWaves - 1)][ev[j]], 1);
      }
    }
  }
  __syncthreads();

  // 2. the padded layout (identical in every workgroup) and this segment's
  //    per-wave starting slots
  int my_cnt = 0, my_pre = 0;
  if (tid < E) {
    my_pre = s_pre[tid];
    my_cnt = my_pre + s_post[tid];
  }
  const int my_blk = (my_cnt + BM - 1) / BM;
  int tot_blk, tot_cnt;
  const int blk_ex = block_exclusive_scan(my_blk, s_wave, &tot_blk);
  const int cnt_ex = block_exclusive_scan(my_cnt, s_wave, &tot_cnt);
  if (tid < E) {
    int run = blk_ex * BM + my_pre;
#pragma unroll
    for (int w = 0; w < kAlignWaves; ++w) {
      const int cnt = s_wcnt[w][tid];
      s_wcnt[w][tid] = run;
      run += cnt;
    }
    // expert tid's padding, block ids and offset: written by one workgroup
    if (tid % nb == b) {
      if (expert_offsets) expert_offsets[tid] = cnt_ex;
      const int first = blk_ex * BM;
      for (int sl = first + my_cnt; sl < first + my_blk * BM; ++sl) sorted_ids[sl] = P;
      for (int bb = blk_ex; bb < blk_ex + my_blk; ++bb) expert_ids[bb] = tid;
    }
  }
  if (b == 0 && tid == 0) {
    if (expert_offsets) expert_offsets[E] = tot_cnt;
    num_post_pad[0] = tot_blk * BM;
  }
  for (int sl = tot_blk * BM + b * kAlignThreads + tid; sl < sorted_len; sl += nb * kAlignThreads) sorted_ids[sl] = P;
  for (int bb = tot_blk + b * kAlignThreads + tid; bb < blocks_len; bb += nb * kAlignThreads) expert_ids[bb] = -1;
  __syncthreads();

  // 3. stable scatter of the segment (as in moe_align_kernel)
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = p0; base < p1; base += 64) {
    const int i = base + lane;
    const int e = i < p1 ? topk_ids[i] : -1;
    const bool valid = (unsigned)e < (unsigned)E;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < id_bits; ++bit) {
      const bool set = (e >> bit) & 1;
      const uint64_t m = __ballot(set);
      peers &= set ? m : ~m;
    }
    const int rank = __popcll(peers & lt_mask);
    const int count = __popcll(peers);
    int slot = 0;
    if (valid) slot = s_wcnt[wave][e] + rank;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      sorted_ids[slot] = i;
      if (rank == 0) s_wcnt[wave][e] = slot + count;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// Workgroups for the split kernel: one per ~1024 pairs, at most 64 (every
// workgroup reads all ids: 64 x the id array of L2 traffic at most).
int align_workgroups(int num_pairs) {
  if (num_pairs < 4096) return 1;
  const int nb = (num_pairs + 1023) / 1024;
  return nb < 64 ? nb : 64;
}

constexpr int kSmallPairs = 64;     // one pair per lane of the first wave
constexpr int kSmallThreads = 256;
constexpr int kIdBits = 10;         // ids below kAlignMaxE = 1024

// pairs among `pm` whose id is below v (v < 1024), from the ballots of each
// id bit: at every bit where v has a 1, the lanes still matching v's higher
// bits and holding a 0 there are below v
__device__ inline int count_below(int v, uint64_t pm, const uint64_t (&m)[kIdBits]) {
  int n = 0;
#pragma unroll
  for (int bit = kIdBits - 1; bit >= 0; --bit) {
    if ((v >> bit) & 1) {
      n += __popcll(pm & ~m[bit]);
      pm &= m[bit];
    } else {
      pm &= ~m[bit];
    }
  }
  return n;
}

__global__ __launch_bounds__(kSmallThreads) void moe_align_small_kernel(
    const int32_t* __restrict__ topk_ids, int P, int E, int BM,
    int32_t* __restrict__ sorted_ids, int sorted_len,
    int32_t* __restrict__ expert_ids, int blocks_len,
    int32_t* __restrict__ num_post_pad, int32_t* __restrict__ expert_offsets) {
  __shared__ uint64_t s_mask[kIdBits + 1];   // ballot of each id bit, then the routed pairs
  __shared__ int s_bexp[kSmallPairs];        // expert of each padded block (>= 1 pair each)
  __shared__ int s_bfill[kSmallPairs];       // pairs in each padded block
  __shared__ int s_totblk;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (wave == 0) {
    const int ev = lane < P ? topk_ids[lane] : -1;
    const bool valid = (unsigned)ev < (unsigned)E;
    const uint64_t vmask = __ballot(valid);
    // the lanes holding the same expert; a lane's rank among them is its
    // pair order within the expert (ids >= E and < 0 are not routed)
    uint64_t m[kIdBits];
    uint64_t peers = vmask;
#pragma unroll
    for (int bit = 0; bit < kIdBits; ++bit) {
      const bool set = (ev >> bit) & 1;
      m[bit] = __ballot(set);
      peers &= set ? m[bit] : ~m[bit];
    }
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int rank = __popcll(peers & lt_mask);
    const int c = __popcll(peers);
    // an expert's padded blocks = its pairs whose rank is a multiple of BM
    const bool head = valid && rank % BM == 0;
    const uint64_t heads = __ballot(head);
    const int bbelow = count_below(ev, vmask & heads, m);
    if (valid) sorted_ids[bbelow * BM + rank] = lane;
    if (head) {
      const int b = bbelow + rank / BM;
      s_bexp[b] = ev;
      s_bfill[b] = min(BM, c - rank);
    }
    if (lane == 0) {
#pragma unroll
      for (int bit = 0; bit < kIdBits; ++bit) s_mask[bit] = m[bit];
      s_mask[kIdBits] = vmask;
      s_totblk = __popcll(heads);
      num_post_pad[0] = __popcll(heads) * BM;
    }
  }
  __syncthreads();
  const int tot_blk = s_totblk;
  // padding slots: wave w takes blocks w, w + 4, ...; lane l holds block l's pairs
  const int fill = lane < tot_blk ? s_bfill[lane] : 0;
  for (int b = wave; b < tot_blk; b += kSmallThreads / 64) {
    const int fb = __builtin_amdgcn_readlane(fill, b);
    for (int q = fb + lane; q < BM; q += 64) sorted_ids[b * BM + q] = P;
  }
  for (int b = tid; b < blocks_len; b += kSmallThreads) expert_ids[b] = b < tot_blk ? s_bexp[b] : -1;
  if (expert_offsets) {
    uint64_t m[kIdBits];
#pragma unroll
    for (int bit = 0; bit < kIdBits; ++bit) m[bit] = s_mask[bit];
    const uint64_t vmask = s_mask[kIdBits];
    for (int e = tid; e <= E; e += kSmallThreads)
      expert_offsets[e] = e < E ? count_below(e, vmask, m) : __popcll(vmask);
  }
  // tail: 16-byte stores from the first aligned slot on
  const int t0 = tot_blk * BM;
  const int mis = (int)((reinterpret_cast<uintptr_t>(sorted_ids + t0) >> 2) & 3);
  const int hd = min(sorted_len, t0 + ((4 - mis) & 3));
  if (tid < hd - t0) sorted_ids[t0 + tid] = P;
  const int nv = (sorted_len - hd) >> 2;
  int4* vt = reinterpret_cast<int4*>(sorted_ids + hd);
  for (int i = tid; i < nv; i += kSmallThreads) vt[i] = make_int4(P, P, P, P);
  const int rest = hd + nv * 4;
  if (tid < sorted_len - rest) sorted_ids[rest + tid] = P;
}

hipError_t launch_moe_align(const int32_t* topk_ids, int num_pairs, int E, int BM,
                            int32_t* sorted_ids, int sorted_len, int32_t* expert_ids, int blocks_len,
                            int32_t* num_post_pad, int32_t* expert_offsets, hipStream_t s) {
  int id_bits = 0;
  while ((1 << id_bits) < E) ++id_bits;
  const int nb = align_workgroups(num_pairs);
  if (num_pairs <= kSmallPairs)
    hipLaunchKernelGGL(moe_align_small_kernel, dim3(1), dim3(kSmallThreads), 0, s, topk_ids, num_pairs, E, BM,
                       sorted_ids, sorted_len, expert_ids, blocks_len, num_post_pad, expert_offsets);
  else if (nb > 1)
    hipLaunchKernelGGL(moe_align_split_kernel, dim3(nb), dim3(kAlignThreads), 0, s, topk_ids, num_pairs, E, BM,
                       id_bits, sorted_ids, sorted_len, expert_ids, blocks_len, num_post_pad, expert_offsets);
  else
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
