// Instantiations of the grouped-GEMM kernel: debug export of the int32 group partials, routed pairs.
#include "gemm_kernel.h"

namespace mw4a8 {

template hipError_t dispatch_bm<64, kModeRouted, true>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<128, kModeRouted, true>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<256, kModeRouted, true>(GemmArgs, const TileConfig&, int, hipStream_t);

}  // namespace mw4a8
