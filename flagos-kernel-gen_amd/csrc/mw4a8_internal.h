// Internal interfaces between the C-ABI layer (api.cpp) and the HIP kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mw4a8 {

// Everything a grouped-GEMM launch needs. Exactly one of the two row
// sources is used: the CSR block table (reference layout, rows grouped by
// expert) or the routing metadata (routed layout, rows gathered per pair).
struct GemmArgs {
  const int8_t* x;        // [rows, K] int8, row stride ldx bytes
  int64_t ldx;
  uint32_t x_bytes;       // rows * ldx (< 2^31)
  const float* xs;        // per-row activation scale
  const uint8_t* w;       // [E, N, K/2] packed int4
  const float* ws;        // [E, N, G] group scales
  const int8_t* wz;       // [E, N, G] zero points
  // reference layout: block b covers rows [row0[b], row1[b]) of expert blk_expert[b]
  const int32_t* blk_expert;
  const int32_t* blk_row0;
  const int32_t* blk_row1;
  const int32_t* blk_count;   // [0] = number of valid blocks
  // reference layout without a block table (E <= kCsrScanExperts): every
  // wave derives its block from the clamped CSR offsets [E + 1] itself
  const int32_t* offsets;
  int M_total;
  int max_blocks;             // blocks past this bound are dropped, as by the table
  // routed layout: block b covers sorted slots [b*BM, b*BM+BM)
  const int32_t* sorted_ids;
  const int32_t* expert_ids;
  const int32_t* num_post_pad;
  const float* tw;            // [num_pairs] routing weights
  int topk;
  int num_pairs;
  int sorted_len;             // length of sorted_ids (reads are bounded by it)
  int E;
  uint16_t* out;              // bf16 bits, row stride ldo elements
  int64_t ldo;
  int32_t* dbg;               // debug partials [rows, N, G] (debug kernels only)
  int N, K, G;
  int zs_vec;                 // zero points/scales of a K-chunk load as one vector run per column
  int vec_out;                // output rows may be stored in 16-byte pieces (N, ldo multiples of 8; aligned)
  // launch geometry (see grid_for)
  int n_tiles, R, total_tiles, per_xcd;
  int egroups;                // routed 64/128-row tiles in expert groups (expert_group_tile)
  // persistent launches: this launch's tile queues (one counter per XCD,
  // 16 ints apart, and the count of finished workgroups at [128]); all zero
  // when the launch starts, and left zero by its last workgroup
  int* queue;
};

// Position of block slot i among the gs blocks that share column tile nt in
// the tile list. One XCD's workgroups go to its four shader engines in turn
// (the k-th workgroup of the XCD's run to a fixed engine, k mod 4 -- measured
// with a placement probe; each engine then runs its own queue), so with the
// same block order for every column tile an expert's full block and its
// short last block alternate in the list and all the full blocks land on
// the same engines. The order is rotated by the digit sum of nt in base gs
// (a generalised Thue-Morse sequence), which spreads each block over the
// positions mod 4 (for gs = 2 and 4: evenly over every 4 column tiles).
__host__ __device__ __forceinline__ int group_slot(int i, int nt, int gs) {
  if (gs <= 1) return i;
  int r = 0;
  for (int v = nt; v > 0; v /= gs) r += v % gs;
  return (i + r) % gs;
}

// Expert-grouped tile order of a routed launch. The row blocks of one
// expert's run (expert_ids ascends over the blocks, as moe_align lays them
// out) form groups of up to R blocks counted from the run's first block; a
// group's tiles take the column tiles in turn, its blocks innermost (in the
// rotated order of group_slot), so the tiles that share one column tile of
// one expert's weights are adjacent in the list and run at the same time on
// one XCD. Every block keeps n_tiles tiles inside its group's range, so
// block t / n_tiles lies in the group of tile t. Writes block b, column
// tile nt and expert e of tile t in [0, nblocks * n_tiles); false when the
// block has no expert in [0, E).
// The run start is found by a binary search, which needs ascending
// expert_ids: on a table that is not sorted the returned group may not hold
// block t / n_tiles, so every block of the group is checked to belong to e
// -- a tile never computes a block with another expert's weights (its tiles
// may then be skipped; the C ABI requires the ascending order).
__host__ __device__ __forceinline__ bool expert_group_tile(int t, int n_tiles, int R, int nblocks, const int32_t* expert_ids,
                                                  int E, int& b, int& nt, int& e) {
  const int bb = t / n_tiles;
  e = expert_ids[bb];
  if (e < 0 || e >= E) return false;
  int lo = 0, hi = bb;   // first block of the run: lower bound of e in [0, bb]
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (expert_ids[mid] < e) lo = mid + 1;
    else hi = mid;
  }
  const int g0 = lo + (bb - lo) / R * R;
  if (expert_ids[g0] != e) return false;   // unsorted table
  int gs = 1;
  while (gs < R && g0 + gs < nblocks && expert_ids[g0 + gs] == e) ++gs;
  const int local = t - g0 * n_tiles;
  nt = local / gs;
  b = g0 + group_slot(local - nt * gs, nt, gs);
  return nt < n_tiles;
}

// Scalar byte offset of K-group gg within a weight column (the vector part
// of the address holds the column and the lane's 16-byte piece). Groups past
// the last one -- loaded by a partial last K-chunk, never computed -- read
// the last group again, so the offset stays inside the column: the buffer
// range check does not cover scalar offsets.
__host__ __device__ __forceinline__ int w_group_soffset(int gg, int G, int GS) { return (gg < G ? gg : G - 1) * (GS / 2); }

// Vector byte offset of a lane's weight pieces within one expert's
// [N, K/2] slice: column col, K slot kb (0..3) of the MFMA operand, which
// covers bytes kb * GS / 8 .. + GS / 8 of each group (16-byte pieces, or one
// 8-byte piece at group size 64).
__host__ __device__ __forceinline__ uint32_t w_lane_offset(int col, uint32_t khalf, int kb, int GS) {
  return (uint32_t)col * khalf + (uint32_t)(kb * (GS / 8));
}

// Tile bodies per group size, row source and debug export (gemm_kernel.h;
// instantiated by the gemm_*.hip files).
struct GemmArgs;
struct TileConfig;
template <int GS, int RMODE, bool DEBUGP>
hipError_t dispatch_bm(GemmArgs a, const TileConfig& c, int max_blocks, hipStream_t s);

struct TileConfig {
  int BM;     // rows per block
  int WN;     // columns per wave
  int NW;     // waves per workgroup
  int KCG;    // K-groups staged per chunk
  int R;      // row blocks walked together per column tile (L2 reuse)
};

// Tile choice by expected rows per touched expert (no device sync).
TileConfig select_tiles(int rows, int touched_experts, int N, int K, int group_size);

// The tile configuration of row-block size BM (16, 32, 64 or 128).
TileConfig tiles_for_block_m(int BM, int group_size);

// Upper bound on the number of row blocks for `rows` rows spread over at
// most `experts` experts: every expert adds at most one partial block.
int max_row_blocks(int rows, int experts, int BM);

// Experts up to which a reference-layout launch needs no block table: each
// wave scans the offsets in chunks of 64 experts, one expert per lane.
constexpr int kCsrScanChunks = 4;
constexpr int kCsrScanExperts = 64 * kCsrScanChunks;

// Kernel launchers; return hipSuccess or the launch error.
hipError_t launch_csr_block_table(const int32_t* offsets, int E, int M_total, int BM, int max_blocks,
                                  int32_t* blk_expert, int32_t* blk_row0, int32_t* blk_row1,
                                  int32_t* blk_count, hipStream_t s);

hipError_t launch_moe_align(const int32_t* topk_ids, int num_pairs, int E, int BM,
                            int32_t* sorted_ids, int sorted_len, int32_t* expert_ids, int blocks_len,
                            int32_t* num_post_pad, int32_t* expert_offsets, hipStream_t s);

// max_blocks bounds the row-block index space the grid covers.
// Row sources and weight layout of a GEMM launch.
constexpr int kModeCsr = 0;             // reference layout: CSR expert offsets, reference weight format
constexpr int kModeRouted = 1;          // routed pairs (sorted_ids), reference weight format
constexpr int kModeRoutedRepacked = 2;  // routed pairs, weights in the repacked MFMA order

hipError_t launch_grouped_gemm(GemmArgs a, const TileConfig& cfg, int group_size, int mode, int max_blocks,
                               hipStream_t s);

// The same kernels with the debug export on: a.dbg [rows, N, G] receives
// the exact int32 partial of every (row, column, group) the launch computes.
hipError_t launch_debug_partials(GemmArgs a, const TileConfig& cfg, int group_size, int mode, int max_blocks,
                                 hipStream_t s);

// MoE-layer kernels around the GEMM (moe_layer.hip); shapes checked by the caller.
hipError_t launch_quant_rows(const uint16_t* x, int64_t ldx, int M, int K, int8_t* q, int64_t ldq, float* scale,
                             hipStream_t s);
hipError_t launch_silu_mul_quant(const uint16_t* h, int64_t ldh, int P, int I, int8_t* q, int64_t ldq,
                                 float* scale, hipStream_t s);
hipError_t launch_router_topk(const float* logits, int64_t ld, int M, int E, int k, int renormalize, int32_t* ids,
                              float* weights, hipStream_t s);
hipError_t launch_combine_topk(const uint16_t* y, int64_t ldy, int M, int topk, int N, const float* weights,
                               uint16_t* out, int64_t ldo, hipStream_t s);
// Streaming read of `bytes` (a multiple of 16) at src with `blocks`
// 256-thread workgroups; sink receives at most 4096 bytes (measure.hip).
hipError_t launch_stream_read(const void* src, int64_t bytes, void* sink, int blocks, hipStream_t s);
// Weight repack between the reference int4 packing and the MFMA order
// (inverse != 0: back to the reference packing); n_words 32-bit words.
hipError_t launch_repack_weights(const uint32_t* src, uint32_t* dst, int64_t n_words, int inverse, hipStream_t s);

}  // namespace mw4a8
