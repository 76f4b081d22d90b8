// Instantiations of the grouped-GEMM kernel: routed pairs, weights in the repacked MFMA order.
#include "gemm_kernel.h"

namespace mw4a8 {

template hipError_t dispatch_bm<64, kModeRoutedRepacked, false>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<128, kModeRoutedRepacked, false>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<256, kModeRoutedRepacked, false>(GemmArgs, const TileConfig&, int, hipStream_t);

}  // namespace mw4a8
