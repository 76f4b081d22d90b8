// Instantiations of the grouped-GEMM kernel: routed pairs, reference weight format.
#include "gemm_kernel.h"

namespace mw4a8 {

template hipError_t dispatch_bm<64, kModeRouted, false>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<128, kModeRouted, false>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<256, kModeRouted, false>(GemmArgs, const TileConfig&, int, hipStream_t);

}  // namespace mw4a8
