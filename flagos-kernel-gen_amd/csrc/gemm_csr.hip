// Instantiations of the grouped-GEMM kernel: reference layout (CSR expert offsets).
#include "gemm_kernel.h"

namespace mw4a8 {

template hipError_t dispatch_bm<64, kModeCsr, false>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<128, kModeCsr, false>(GemmArgs, const TileConfig&, int, hipStream_t);
template hipError_t dispatch_bm<256, kModeCsr, false>(GemmArgs, const TileConfig&, int, hipStream_t);

}  // namespace mw4a8
