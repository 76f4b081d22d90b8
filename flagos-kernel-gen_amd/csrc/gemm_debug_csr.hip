// Instantiations of the grouped-GEMM kernel: debug export of the int32 group partials, reference layout.
#include "gemm_kernel.h"

namespace mw4a8 {

template hipError_t dispatch_bm<64, kModeCsr, true>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<128, kModeCsr, true>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<256, kModeCsr, true>(GemmArgs, const TileConfig&, int, hipStream_t);

}  // namespace mw4a8
