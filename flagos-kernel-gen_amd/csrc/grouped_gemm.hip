// Host side of the grouped GEMM: tile selection and dispatch to the kernel
// instantiations. The kernel template lives in gemm_kernel.h; the gemm_*.hip
// files instantiate it once per row source (reference layout, routed,
// routed on repacked weights, and the debug exports of the same bodies), so
// they compile in parallel.
#include "mw4a8_internal.h"

namespace mw4a8 {

template <bool DEBUGP>
static hipError_t dispatch_mode(GemmArgs a, const TileConfig& cfg, int group_size, int mode, int max_blocks,
                                hipStream_t s) {
  switch (group_size) {
    case 64:
      if (mode == kModeCsr) return dispatch_bm<64, kModeCsr, DEBUGP>(a, cfg, max_blocks, s);
      if (mode == kModeRouted) return dispatch_bm<64, kModeRouted, DEBUGP>(a, cfg, max_blocks, s);
      if (mode == kModeRoutedRepacked) return dispatch_bm<64, kModeRoutedRepacked, DEBUGP>(a, cfg, max_blocks, s);
      break;
    case 128:
      if (mode == kModeCsr) return dispatch_bm<128, kModeCsr, DEBUGP>(a, cfg, max_blocks, s);
      if (mode == kModeRouted) return dispatch_bm<128, kModeRouted, DEBUGP>(a, cfg, max_blocks, s);
      if (mode == kModeRoutedRepacked) return dispatch_bm<128, kModeRoutedRepacked, DEBUGP>(a, cfg, max_blocks, s);
      break;
    case 256:
      if (mode == kModeCsr) return dispatch_bm<256, kModeCsr, DEBUGP>(a, cfg, max_blocks, s);
      if (mode == kModeRouted) return dispatch_bm<256, kModeRouted, DEBUGP>(a, cfg, max_blocks, s);
      if (mode == kModeRoutedRepacked) return dispatch_bm<256, kModeRoutedRepacked, DEBUGP>(a, cfg, max_blocks, s);
      break;
  }
  return hipErrorInvalidValue;
}

hipError_t launch_grouped_gemm(GemmArgs a, const TileConfig& cfg, int group_size, int mode, int max_blocks,
                               hipStream_t s) {
  return dispatch_mode<false>(a, cfg, group_size, mode, max_blocks, s);
}

hipError_t launch_debug_partials(GemmArgs a, const TileConfig& cfg, int group_size, int mode, int max_blocks,
                                 hipStream_t s) {
  if (a.dbg == nullptr) return hipErrorInvalidValue;
  return dispatch_mode<true>(a, cfg, group_size, mode, max_blocks, s);
}

int max_row_blocks(int rows, int experts, int BM) {
  if (rows <= 0) return 0;
  const int64_t ne = experts < rows ? experts : rows;
  const int64_t bound = ((int64_t)rows + ne * (BM - 1)) / BM;
  return (int)(bound < rows ? bound : rows);
}

TileConfig tiles_for_block_m(int BM, int group_size) {
  TileConfig c;
  c.NW = 4;
  c.BM = BM;
  switch (BM) {
    case 16: c.WN = 16; c.KCG = 512 / group_size; c.R = 1; break;
    case 32: c.WN = 16; c.KCG = 512 / group_size; c.R = 1; break;
    case 64: c.WN = 32; c.KCG = 256 / group_size; c.R = 2; break;
    default: c.BM = 128; c.WN = 32; c.KCG = 256 / group_size; c.R = 2; c.NW = group_size >= 128 ? 8 : 4; break;
  }
  if (c.KCG < 1) c.KCG = 1;
  return c;
}

TileConfig select_tiles(int rows, int touched_experts, int N, int K, int group_size) {
  const int ne = touched_experts < 1 ? 1 : touched_experts;
  const int per_expert = (rows + ne - 1) / ne;
  // Measured on MI355X (DeepSeek-V3, Qwen3, Mixtral shapes): up to 8 rows per
  // expert the 16-row decode tile streams the weights best; from 16 rows the
  // 64-row tile wins (one block per expert reads its weights once, and its
  // half-height body covers experts of up to 32 rows) -- by 16-40 % at 16-32
  // rows; in between the long K = 7168 still prefers 16 rows, K <= 4096 64.
  // The 32-row tile was never the fastest choice.
  if (per_expert <= 8) return tiles_for_block_m(16, group_size);
  if (per_expert < 16 && K > 4096) return tiles_for_block_m(16, group_size);
  // a small problem keeps the 16-row tiles' larger grid (64-row tiles span
  // 128 columns: fewer than 256 tiles leave CUs idle)
  if (per_expert <= 32 && (int64_t)ne * ((N + 127) / 128) < 256) return tiles_for_block_m(16, group_size);
  // 128-row tiles over more than 64 rows an expert (measured on MI355X with
  // the tail rows and the rotated block order: DeepSeek-V3 up/gate K = 7168
  // 1391 vs 1950 us with 64 rows, down K = 2048 839 vs 961 us, Qwen3 K = 2048
  // 112 either way); shorter K loops keep the 64-row tiles
  if (per_expert <= 64 || K < 2048) return tiles_for_block_m(64, group_size);
  return tiles_for_block_m(128, group_size);
}

}  // namespace mw4a8
