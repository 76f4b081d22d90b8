// C ABI entry points (declared in include/mw4a8.h): argument validation,
// tile selection, workspace carving and kernel launches. Host code only.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/mw4a8.h"
#include "mw4a8_internal.h"
#include "mw4a8_pack.h"

using namespace mw4a8;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(MW4A8_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

bool supported_group(int gs) { return gs == 64 || gs == 128 || gs == 256; }

// Checks shared by the GEMM entries. Returns MW4A8_OK or an error code.
int check_gemm_args(const int8_t* x_q, int64_t ldx, const float* x_scale, const uint8_t* w_q4,
                    const float* w_scale, const int8_t* w_zero, const void* out, int64_t ldo, int rows,
                    int N, int K, int E, int gs, bool need_scales) {
  if (rows < 0 || N <= 0 || K <= 0 || E <= 0)
    return fail(MW4A8_ERR_INVALID, "bad sizes: rows=%d N=%d K=%d E=%d", rows, N, K, E);
  if (!supported_group(gs)) return fail(MW4A8_ERR_UNSUPPORTED, "group_size %d not in {64,128,256}", gs);
  if (K % gs != 0) return fail(MW4A8_ERR_INVALID, "K=%d is not a multiple of group_size=%d", K, gs);
  if (ldx < K) return fail(MW4A8_ERR_INVALID, "ldx=%lld < K=%d", (long long)ldx, K);
  if (ldo < N) return fail(MW4A8_ERR_INVALID, "ldo=%lld < N=%d", (long long)ldo, N);
  if (ldx % 16 != 0) return fail(MW4A8_ERR_INVALID, "ldx=%lld must be a multiple of 16", (long long)ldx);
  if (!x_q || !w_q4 || !w_zero || !out || (need_scales && (!x_scale || !w_scale)))
    return fail(MW4A8_ERR_INVALID, "null tensor pointer");
  if (!aligned(x_q, 16) || !aligned(w_q4, 16))
    return fail(MW4A8_ERR_INVALID, "x_q and w_q4 must be 16-byte aligned");
  if ((need_scales && (!aligned(x_scale, 4) || !aligned(w_scale, 4))) || !aligned(out, 2))
    return fail(MW4A8_ERR_INVALID, "misaligned scale or output pointer");
  // kernels address each tensor (weights: one expert's slice) with 32-bit offsets
  const int64_t lim = (int64_t)1 << 31;
  if ((int64_t)rows * ldx >= lim || (int64_t)N * (K / 2) >= lim || (int64_t)N * (K / gs) * 4 >= lim)
    return fail(MW4A8_ERR_UNSUPPORTED, "tensor too large for 32-bit offsets (rows*ldx, N*K/2, N*G*4 < 2^31)");
  return MW4A8_OK;
}

struct CsrWorkspace {
  int32_t* count;
  int32_t* expert;
  int32_t* row0;
  int32_t* row1;
};

size_t csr_ws_bytes(int max_blocks) {
  const size_t b = 256 + 3 * sizeof(int32_t) * (size_t)max_blocks;
  return (b + 255) & ~(size_t)255;
}

CsrWorkspace carve(void* ws, int max_blocks) {
  char* p = static_cast<char*>(ws);
  CsrWorkspace w;
  w.count = reinterpret_cast<int32_t*>(p);
  w.expert = reinterpret_cast<int32_t*>(p + 256);
  w.row0 = w.expert + max_blocks;
  w.row1 = w.row0 + max_blocks;
  return w;
}

// rows >= 1 activation rows of K bytes, ldx apart: the kernels' activation
// descriptor ends with the last row's K-th byte (not its row stride)
GemmArgs base_args(const int8_t* x_q, int64_t ldx, int rows, const float* x_scale, const uint8_t* w_q4,
                   const float* w_scale, const int8_t* w_zero, uint16_t* out, int64_t ldo, int N, int K,
                   int gs) {
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.x = x_q;
  a.ldx = ldx;
  a.x_bytes = (uint32_t)((int64_t)(rows - 1) * ldx + K);
  a.xs = x_scale;
  a.w = w_q4;
  a.ws = w_scale;
  a.wz = w_zero;
  a.out = out;
  a.ldo = ldo;
  a.N = N;
  a.K = K;
  a.G = K / gs;
  return a;
}

// Whether a reference-layout launch over E experts builds a block table in
// the workspace: with up to kCsrScanExperts experts the GEMM's waves derive
// their row blocks from the offsets themselves (one launch, no table).
bool csr_uses_table(int E) { return E > kCsrScanExperts; }

// Shared by the reference-layout GEMM and the debug export: the GEMM launch,
// preceded by the block-table launch for many experts. The workspace is
// required either way (its size depends on M_total and E only).
int run_csr(GemmArgs a, const int32_t* offsets, int M_total, int E, int gs, void* workspace, size_t ws_bytes,
            hipStream_t s, bool debug) {
  if (!offsets) return fail(MW4A8_ERR_INVALID, "null expert_offsets");
  const int ne = E < M_total ? E : M_total;
  // the debug export runs the tile the product would select
  const TileConfig cfg = select_tiles(M_total, ne, a.N, a.K, gs);
  const int max_blocks = max_row_blocks(M_total, E, cfg.BM);
  if (max_blocks == 0) return MW4A8_OK;
  if (!workspace || ws_bytes < csr_ws_bytes(max_blocks))
    return fail(MW4A8_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", csr_ws_bytes(max_blocks),
                workspace ? ws_bytes : (size_t)0);
  if (!aligned(workspace, 256)) return fail(MW4A8_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  hipError_t e;
  a.E = E;
  if (csr_uses_table(E)) {
    CsrWorkspace w = carve(workspace, max_blocks);
    e = launch_csr_block_table(offsets, E, M_total, cfg.BM, max_blocks, w.expert, w.row0, w.row1, w.count, s);
    if (e != hipSuccess) return hip_fail(e, "block table launch");
    a.blk_expert = w.expert;
    a.blk_row0 = w.row0;
    a.blk_row1 = w.row1;
    a.blk_count = w.count;
  } else {
    a.offsets = offsets;
    a.M_total = M_total;
    a.max_blocks = max_blocks;
  }
  e = debug ? launch_debug_partials(a, cfg, gs, kModeCsr, max_blocks, s)
            : launch_grouped_gemm(a, cfg, gs, kModeCsr, max_blocks, s);
  if (e != hipSuccess) return hip_fail(e, "grouped GEMM launch");
  return MW4A8_OK;
}

// ---- allocation-free variant of the reference-layout entry ----------------
// mw4a8_grouped_gemm_noalloc keeps its block table (the only device memory
// the reference-layout entry needs beyond inputs and outputs) in `scratch`,
// a file-scope device array: one copy per GPU, held until the process ends,
// sized for kNoallocMaxBlocks row blocks. Host code never passes the array's
// name to a kernel (on the host it is a stand-in, not a device address): the
// first call on a device resolves the device's own address of the array with
// hipGetSymbolAddress, with that device current, and keeps it per device.
// The block-table kernel writes every entry the GEMM reads, so nothing has
// to be cleared between calls. Calls over at most kCsrScanExperts experts
// build no table and leave the array untouched.
constexpr int kNoallocMaxBlocks = 65536;
constexpr size_t kNoallocScratchBytes = 256 + 3 * sizeof(int32_t) * (size_t)kNoallocMaxBlocks;   // 786688
static_assert(kNoallocScratchBytes % 256 == 0, "scratch is whole 256-byte units");
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// This device's address of `scratch` (resolved once per device); the stream
// must belong to the current device.
int noalloc_scratch(hipStream_t s, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(MW4A8_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
  if (s != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(s, &sdev);
    if (e != hipSuccess) return hip_fail(e, "hipStreamGetDevice");
    if (sdev != dev) return fail(MW4A8_ERR_INVALID, "stream is on device %d, current device is %d", (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr || !aligned(ptr, 256)) return fail(MW4A8_ERR_HIP, "unusable scratch address %p", ptr);
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MW4A8_OK;
}

}  // namespace

extern "C" {

const char* mw4a8_last_error(void) { return g_err; }

int mw4a8_abi_version(void) { return 1; }

size_t mw4a8_workspace_bytes(int M_total, int N, int K, int E, int group_size) {
  (void)N;
  (void)K;
  (void)group_size;
  if (M_total <= 0 || E <= 0) return 256;
  return csr_ws_bytes(max_row_blocks(M_total, E, 16));
}

int mw4a8_grouped_gemm(const int8_t* x_q, int64_t ldx, const float* x_scale, const uint8_t* w_q4,
                       const float* w_scale, const int8_t* w_zero, const int32_t* expert_offsets,
                       uint16_t* out_bf16, int64_t ldo, int M_total, int N, int K, int E, int group_size,
                       void* workspace, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  if (M_total == 0) return MW4A8_OK;
  int rc = check_gemm_args(x_q, ldx, x_scale, w_q4, w_scale, w_zero, out_bf16, ldo, M_total, N, K, E,
                           group_size, true);
  if (rc) return rc;
  GemmArgs a = base_args(x_q, ldx, M_total, x_scale, w_q4, w_scale, w_zero, out_bf16, ldo, N, K, group_size);
  return run_csr(a, expert_offsets, M_total, E, group_size, workspace, ws_bytes,
                 static_cast<hipStream_t>(stream), false);
}

int mw4a8_grouped_gemm_noalloc(const int8_t* x_q, int64_t ldx, const float* x_scale, const uint8_t* w_q4,
                               const float* w_scale, const int8_t* w_zero, const int32_t* expert_offsets,
                               uint16_t* out_bf16, int64_t ldo, int M_total, int N, int K, int E, int group_size,
                               void* stream) {
  g_err[0] = 0;
  if (M_total == 0) return MW4A8_OK;
  int rc = check_gemm_args(x_q, ldx, x_scale, w_q4, w_scale, w_zero, out_bf16, ldo, M_total, N, K, E,
                           group_size, true);
  if (rc) return rc;
  // the block table of the tile mw4a8_grouped_gemm would select must fit
  const int ne = E < M_total ? E : M_total;
  const int max_blocks = max_row_blocks(M_total, E, select_tiles(M_total, ne, N, K, group_size).BM);
  if (csr_ws_bytes(max_blocks) > kNoallocScratchBytes)
    return fail(MW4A8_ERR_UNSUPPORTED,
                "mw4a8_grouped_gemm_noalloc: up to %d row blocks exceed its fixed scratch of %d blocks "
                "(%zu bytes); use mw4a8_grouped_gemm with a workspace",
                max_blocks, kNoallocMaxBlocks, kNoallocScratchBytes);
  void* ws = nullptr;
  rc = noalloc_scratch(static_cast<hipStream_t>(stream), &ws);
  if (rc) return rc;
  GemmArgs a = base_args(x_q, ldx, M_total, x_scale, w_q4, w_scale, w_zero, out_bf16, ldo, N, K, group_size);
  return run_csr(a, expert_offsets, M_total, E, group_size, ws, kNoallocScratchBytes,
                 static_cast<hipStream_t>(stream), false);
}

int mw4a8_debug_partials(const int8_t* x_q, int64_t ldx, const uint8_t* w_q4, const int8_t* w_zero,
                         const int32_t* expert_offsets, int32_t* partials, int M_total, int N, int K,
                         int E, int group_size, void* workspace, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  if (M_total == 0) return MW4A8_OK;
  int rc = check_gemm_args(x_q, ldx, nullptr, w_q4, nullptr, w_zero, partials, N, M_total, N, K, E,
                           group_size, false);
  if (rc) return rc;
  GemmArgs a = base_args(x_q, ldx, M_total, nullptr, w_q4, nullptr, w_zero, nullptr, N, N, K, group_size);
  a.dbg = partials;
  return run_csr(a, expert_offsets, M_total, E, group_size, workspace, ws_bytes,
                 static_cast<hipStream_t>(stream), true);
}

int mw4a8_align_sizes(int num_pairs, int E, int block_m, int* sorted_len, int* blocks_len) {
  g_err[0] = 0;
  if (num_pairs < 0 || E <= 0 || block_m <= 0 || !sorted_len || !blocks_len)
    return fail(MW4A8_ERR_INVALID, "bad align sizes arguments");
  const int64_t sl = (int64_t)num_pairs + (int64_t)E * (block_m - 1);
  if (sl > 0x7fffffff) return fail(MW4A8_ERR_UNSUPPORTED, "routing buffer too large");
  *sorted_len = (int)sl;
  *blocks_len = (int)((sl + block_m - 1) / block_m);
  return MW4A8_OK;
}

int mw4a8_select_block_m(int num_pairs, int E, int N, int K, int group_size) {
  const int ne = E < num_pairs ? E : num_pairs;
  return select_tiles(num_pairs, ne, N, K, group_size).BM;
}

int mw4a8_moe_align(const int32_t* topk_ids, int num_pairs, int E, int block_m, int32_t* sorted_ids,
                    int32_t* expert_ids, int32_t* num_post_pad, int32_t* expert_offsets_out, void* stream) {
  g_err[0] = 0;
  if (num_pairs < 0 || E <= 0 || block_m <= 0) return fail(MW4A8_ERR_INVALID, "bad routing sizes");
  if (E > 1024) return fail(MW4A8_ERR_UNSUPPORTED, "E=%d > 1024 experts", E);
  if ((num_pairs > 0 && !topk_ids) || !sorted_ids || !expert_ids || !num_post_pad)
    return fail(MW4A8_ERR_INVALID, "null routing pointer");
  int sorted_len, blocks_len;
  int rc = mw4a8_align_sizes(num_pairs, E, block_m, &sorted_len, &blocks_len);
  if (rc) return rc;
  hipError_t e = launch_moe_align(topk_ids, num_pairs, E, block_m, sorted_ids, sorted_len, expert_ids,
                                  blocks_len, num_post_pad, expert_offsets_out, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "moe_align launch");
  return MW4A8_OK;
}

}  // extern "C"

namespace {

int fused_moe_impl(const int8_t* x_q, int64_t ldx, const float* x_scale, const uint8_t* w_q4, const float* w_scale,
                   const int8_t* w_zero, const int32_t* sorted_ids, const int32_t* expert_ids,
                   const int32_t* num_post_pad, const float* topk_weights, int topk, uint16_t* out_bf16, int64_t ldo,
                   int M, int N, int K, int E, int group_size, int block_m, int mode, void* stream,
                   int32_t* partials = nullptr) {
  g_err[0] = 0;
  if (topk <= 0) return fail(MW4A8_ERR_INVALID, "topk=%d", topk);
  if (M == 0) return MW4A8_OK;
  int rc = check_gemm_args(x_q, ldx, x_scale, w_q4, w_scale, w_zero, out_bf16, ldo, M, N, K, E, group_size,
                           true);
  if (rc) return rc;
  if (!sorted_ids || !expert_ids || !num_post_pad) return fail(MW4A8_ERR_INVALID, "null routing pointer");
  if (!aligned(topk_weights, 4)) return fail(MW4A8_ERR_INVALID, "misaligned topk_weights");
  if (block_m != 16 && block_m != 32 && block_m != 64 && block_m != 128)
    return fail(MW4A8_ERR_UNSUPPORTED, "block_m=%d not in {16,32,64,128}", block_m);
  const int64_t pairs = (int64_t)M * topk;
  if (pairs > 0x7fffffff / 2) return fail(MW4A8_ERR_UNSUPPORTED, "too many pairs");
  GemmArgs a = base_args(x_q, ldx, M, x_scale, w_q4, w_scale, w_zero, out_bf16, ldo, N, K, group_size);
  a.sorted_ids = sorted_ids;
  a.expert_ids = expert_ids;
  a.num_post_pad = num_post_pad;
  a.tw = topk_weights;
  a.topk = topk;
  a.num_pairs = (int)pairs;
  a.E = E;
  int sorted_len, blocks_len;
  rc = mw4a8_align_sizes((int)pairs, E, block_m, &sorted_len, &blocks_len);
  if (rc) return rc;
  a.sorted_len = sorted_len;
  // the routing metadata fixes the row block
  const TileConfig cfg = tiles_for_block_m(block_m, group_size);
  if (cfg.BM != block_m) return fail(MW4A8_ERR_UNSUPPORTED, "block_m must be 16, 32, 64 or 128");
  const int max_blocks = max_row_blocks((int)pairs, E, block_m);
  a.dbg = partials;
  hipError_t e = partials ? launch_debug_partials(a, cfg, group_size, mode, max_blocks, static_cast<hipStream_t>(stream))
                          : launch_grouped_gemm(a, cfg, group_size, mode, max_blocks, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "fused MoE launch");
  return MW4A8_OK;
}

}  // namespace

extern "C" {

int mw4a8_fused_moe(const int8_t* x_q, int64_t ldx, const float* x_scale, const uint8_t* w_q4,
                    const float* w_scale, const int8_t* w_zero, const int32_t* sorted_ids,
                    const int32_t* expert_ids, const int32_t* num_post_pad, const float* topk_weights,
                    int topk, uint16_t* out_bf16, int64_t ldo, int M, int N, int K, int E, int group_size,
                    int block_m, void* stream) {
  return fused_moe_impl(x_q, ldx, x_scale, w_q4, w_scale, w_zero, sorted_ids, expert_ids, num_post_pad,
                        topk_weights, topk, out_bf16, ldo, M, N, K, E, group_size, block_m, kModeRouted, stream);
}

int mw4a8_fused_moe_repacked(const int8_t* x_q, int64_t ldx, const float* x_scale, const uint8_t* w_mfma,
                             const float* w_scale, const int8_t* w_zero, const int32_t* sorted_ids,
                             const int32_t* expert_ids, const int32_t* num_post_pad, const float* topk_weights,
                             int topk, uint16_t* out_bf16, int64_t ldo, int M, int N, int K, int E,
                             int group_size, int block_m, void* stream) {
  return fused_moe_impl(x_q, ldx, x_scale, w_mfma, w_scale, w_zero, sorted_ids, expert_ids, num_post_pad,
                        topk_weights, topk, out_bf16, ldo, M, N, K, E, group_size, block_m, kModeRoutedRepacked,
                        stream);
}

int mw4a8_debug_partials_routed(const int8_t* x_q, int64_t ldx, const float* x_scale, const uint8_t* w_q4,
                                const float* w_scale, const int8_t* w_zero, const int32_t* sorted_ids,
                                const int32_t* expert_ids, const int32_t* num_post_pad, const float* topk_weights,
                                int topk, uint16_t* out_bf16, int64_t ldo, int32_t* partials, int M, int N, int K,
                                int E, int group_size, int block_m, int repacked, void* stream) {
  g_err[0] = 0;
  if (!partials) return fail(MW4A8_ERR_INVALID, "null partials");
  if (!aligned(partials, 4)) return fail(MW4A8_ERR_INVALID, "misaligned partials");
  return fused_moe_impl(x_q, ldx, x_scale, w_q4, w_scale, w_zero, sorted_ids, expert_ids, num_post_pad,
                        topk_weights, topk, out_bf16, ldo, M, N, K, E, group_size, block_m,
                        repacked ? kModeRoutedRepacked : kModeRouted, stream, partials);
}

int mw4a8_repack_weights(const uint8_t* src, uint8_t* dst, int64_t E, int N, int K, int inverse, void* stream) {
  g_err[0] = 0;
  if (E < 0 || N < 0 || K <= 0 || K % 8 != 0)
    return fail(MW4A8_ERR_INVALID, "bad sizes: E=%lld N=%d K=%d (K must be a multiple of 8)", (long long)E, N, K);
  const int64_t bytes = E * (int64_t)N * (K / 2);
  if (bytes == 0) return MW4A8_OK;
  if (!src || !dst) return fail(MW4A8_ERR_INVALID, "null tensor pointer");
  if (!aligned(src, 16) || !aligned(dst, 16)) return fail(MW4A8_ERR_INVALID, "weights must be 16-byte aligned");
  if (src == dst) return fail(MW4A8_ERR_INVALID, "in-place repack is not supported");
  hipError_t e = launch_repack_weights(reinterpret_cast<const uint32_t*>(src), reinterpret_cast<uint32_t*>(dst),
                                       bytes / 4, inverse ? 1 : 0, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "repack launch");
  return MW4A8_OK;
}

// ---------------------------------------------------------------------------
// MoE-layer kernels around the GEMM

int mw4a8_quant_rows(const uint16_t* x_bf16, int64_t ldx, int M, int K, int8_t* x_q, int64_t ldq, float* x_scale,
                     void* stream) {
  g_err[0] = 0;
  if (M < 0 || K <= 0) return fail(MW4A8_ERR_INVALID, "bad sizes: M=%d K=%d", M, K);
  if (M == 0) return MW4A8_OK;
  if (!x_bf16 || !x_q || !x_scale) return fail(MW4A8_ERR_INVALID, "null tensor pointer");
  if (K % 8 != 0 || ldx < K || ldq < K || ldx % 8 != 0 || ldq % 8 != 0)
    return fail(MW4A8_ERR_INVALID, "K=%d, ldx=%lld, ldq=%lld must be multiples of 8 with ld >= K", K,
                (long long)ldx, (long long)ldq);
  if (!aligned(x_bf16, 16) || !aligned(x_q, 8) || !aligned(x_scale, 4))
    return fail(MW4A8_ERR_INVALID, "x must be 16-byte, x_q 8-byte aligned");
  hipError_t e = launch_quant_rows(x_bf16, ldx, M, K, x_q, ldq, x_scale, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "quant_rows launch");
  return MW4A8_OK;
}

int mw4a8_router_topk(const float* logits, int64_t ld, int M, int E, int topk, int renormalize, int32_t* topk_ids,
                      float* topk_weights, void* stream) {
  g_err[0] = 0;
  if (M < 0 || E <= 0 || topk <= 0 || ld < E) return fail(MW4A8_ERR_INVALID, "bad sizes: M=%d E=%d topk=%d", M, E, topk);
  if (E > 1024 || topk > 64 || topk > E)
    return fail(MW4A8_ERR_UNSUPPORTED, "router supports E <= 1024 and topk <= min(E, 64)");
  if (M == 0) return MW4A8_OK;
  if (!logits || !topk_ids || !topk_weights) return fail(MW4A8_ERR_INVALID, "null tensor pointer");
  if (!aligned(logits, 4) || !aligned(topk_ids, 4) || !aligned(topk_weights, 4))
    return fail(MW4A8_ERR_INVALID, "misaligned router pointer");
  hipError_t e = launch_router_topk(logits, ld, M, E, topk, renormalize ? 1 : 0, topk_ids, topk_weights,
                                    static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "router_topk launch");
  return MW4A8_OK;
}

int mw4a8_silu_mul_quant(const uint16_t* h_bf16, int64_t ldh, int P, int I, int8_t* q, int64_t ldq, float* scale,
                         void* stream) {
  g_err[0] = 0;
  if (P < 0 || I <= 0) return fail(MW4A8_ERR_INVALID, "bad sizes: P=%d I=%d", P, I);
  if (P == 0) return MW4A8_OK;
  if (!h_bf16 || !q || !scale) return fail(MW4A8_ERR_INVALID, "null tensor pointer");
  if (I % 8 != 0 || ldh < 2 * (int64_t)I || ldq < I || ldh % 8 != 0 || ldq % 8 != 0)
    return fail(MW4A8_ERR_INVALID, "I=%d, ldh=%lld, ldq=%lld: need I %% 8 == 0, ldh >= 2I, ldq >= I, both %% 8 == 0",
                I, (long long)ldh, (long long)ldq);
  if (!aligned(h_bf16, 16) || !aligned(q, 8) || !aligned(scale, 4))
    return fail(MW4A8_ERR_INVALID, "h must be 16-byte, q 8-byte aligned");
  hipError_t e = launch_silu_mul_quant(h_bf16, ldh, P, I, q, ldq, scale, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "silu_mul_quant launch");
  return MW4A8_OK;
}

int mw4a8_combine_topk(const uint16_t* y_bf16, int64_t ldy, int M, int topk, int N, const float* topk_weights,
                       uint16_t* out_bf16, int64_t ldo, void* stream) {
  g_err[0] = 0;
  if (M < 0 || topk <= 0 || N <= 0) return fail(MW4A8_ERR_INVALID, "bad sizes: M=%d topk=%d N=%d", M, topk, N);
  if (M == 0) return MW4A8_OK;
  if (!y_bf16 || !out_bf16) return fail(MW4A8_ERR_INVALID, "null tensor pointer");
  if (N % 8 != 0 || ldy < N || ldo < N || ldy % 8 != 0 || ldo % 8 != 0)
    return fail(MW4A8_ERR_INVALID, "N=%d, ldy=%lld, ldo=%lld must be multiples of 8 with ld >= N", N,
                (long long)ldy, (long long)ldo);
  if (!aligned(y_bf16, 16) || !aligned(out_bf16, 16) || !aligned(topk_weights, 4))
    return fail(MW4A8_ERR_INVALID, "y and out must be 16-byte aligned");
  if ((int64_t)M * topk > 0x7fffffff) return fail(MW4A8_ERR_UNSUPPORTED, "too many rows");
  hipError_t e = launch_combine_topk(y_bf16, ldy, M, topk, N, topk_weights, out_bf16, ldo,
                                     static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "combine_topk launch");
  return MW4A8_OK;
}

int mw4a8_stream_read(const void* src, int64_t bytes, void* sink, size_t sink_bytes, int blocks, void* stream) {
  g_err[0] = 0;
  if (bytes < 0 || bytes % 16 != 0) return fail(MW4A8_ERR_INVALID, "bytes=%lld must be a non-negative multiple of 16",
                                                (long long)bytes);
  if (blocks < 1 || blocks > 65536) return fail(MW4A8_ERR_INVALID, "blocks=%d not in [1, 65536]", blocks);
  if (!sink || sink_bytes < 4096 || !aligned(sink, 16))
    return fail(MW4A8_ERR_INVALID, "sink must be a 16-byte aligned buffer of at least 4096 bytes");
  if (bytes == 0) return MW4A8_OK;
  if (!src || !aligned(src, 16)) return fail(MW4A8_ERR_INVALID, "src must be a 16-byte aligned device pointer");
  hipError_t e = launch_stream_read(src, bytes, sink, blocks, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "stream_read launch");
  return MW4A8_OK;
}

// ---------------------------------------------------------------------------

int mw4a8_host_selftest(void) {
  int bad = 0;
  // zero fold: every nibble against every zero point, in every byte lane
  for (int z = -128; z <= 127; ++z) {
    const ZeroFold f = make_zero_fold(z);
    for (int u = 0; u < 16; ++u) {
      const int8_t want = (int8_t)(uint8_t)((u - z) & 0xff);
      for (int lane = 0; lane < 4; ++lane) {
        const uint32_t lo_word = (uint32_t)u << (8 * lane);         // nibble in the low half of byte `lane`
        const uint32_t hi_word = (uint32_t)(u << 4) << (8 * lane);  // nibble in the high half
        const int8_t got_lo = (int8_t)((fold_even(lo_word, f) >> (8 * lane)) & 0xff);
        const int8_t got_hi = (int8_t)((fold_odd(hi_word, f) >> (8 * lane)) & 0xff);
        bad += got_lo != want;
        bad += got_hi != want;
      }
    }
  }
  // K relabelling: one lane's 16-k dot product computed from the relabelled
  // activation bytes and the unpacked weight words equals the natural-order dot
  uint32_t state = 12345u;
  auto rnd = [&state]() {
    state = state * 1664525u + 1013904223u;
    return state >> 8;
  };
  for (int trial = 0; trial < 2000; ++trial) {
    int8_t x[16];
    uint8_t packed[8];
    for (int i = 0; i < 16; ++i) x[i] = (int8_t)(rnd() & 0xff);
    for (int i = 0; i < 8; ++i) packed[i] = (uint8_t)(rnd() & 0xff);
    const int z = (int)(rnd() % 256) - 128;
    int64_t want = 0;
    for (int k = 0; k < 16; ++k) {
      const int u = (k & 1) ? (packed[k / 2] >> 4) : (packed[k / 2] & 15);
      want += (int64_t)x[k] * (int8_t)(uint8_t)((u - z) & 0xff);
    }
    uint32_t xd[4], pd[2];
    memcpy(xd, x, 16);
    memcpy(pd, packed, 8);
    const uint32_t a[4] = {even_bytes(xd[0], xd[1]), odd_bytes(xd[0], xd[1]), even_bytes(xd[2], xd[3]),
                           odd_bytes(xd[2], xd[3])};
    const ZeroFold f = make_zero_fold(z);
    const uint32_t bw[4] = {fold_even(pd[0], f), fold_odd(pd[0], f), fold_even(pd[1], f), fold_odd(pd[1], f)};
    int64_t got = 0;
    for (int w = 0; w < 4; ++w)
      for (int by = 0; by < 4; ++by)
        got += (int64_t)(int8_t)((a[w] >> (8 * by)) & 0xff) * (int8_t)((bw[w] >> (8 * by)) & 0xff);
    bad += got != want;
  }
  // expert-grouped tile order: over random expert runs (empty experts, runs
  // of 1..12 blocks), every (block, column tile) is produced exactly once
  // with the block's expert; groups stay inside one run, start at the run's
  // first block plus a multiple of R and hold at most R blocks; the tiles of
  // one group and column tile are consecutive in the list.
  for (int trial = 0; trial < 300; ++trial) {
    int32_t ids[160];
    int nblocks = 0;
    const int E = 1 + (int)(rnd() % 24);
    for (int ex = 0; ex < E && nblocks < 148; ++ex) {
      const int run = (rnd() % 4 == 0) ? 0 : 1 + (int)(rnd() % ((trial & 1) ? 12 : 3));
      for (int j = 0; j < run && nblocks < 148; ++j) ids[nblocks++] = ex;
    }
    if (nblocks == 0) continue;
    const int R = 1 + (int)(rnd() % 4);
    const int n_tiles = 1 + (int)(rnd() % 7);
    static uint8_t seen[160 * 8];
    memset(seen, 0, sizeof(seen));
    int prev_key = -1;
    uint8_t key_done[160 * 8];
    memset(key_done, 0, sizeof(key_done));
    for (int t = 0; t < nblocks * n_tiles; ++t) {
      int b = -1, nt = -1, ex = -1;
      if (!expert_group_tile(t, n_tiles, R, nblocks, ids, E, b, nt, ex) || b < 0 || b >= nblocks ||
          nt < 0 || nt >= n_tiles || ids[b] != ex) {
        ++bad;
        continue;
      }
      bad += seen[b * n_tiles + nt]++ != 0;
      int first = b;   // run start, by walking back
      while (first > 0 && ids[first - 1] == ex) --first;
      const int g0 = first + (b - first) / R * R;
      const int key = g0 * n_tiles + nt;   // (group, column tile)
      if (key != prev_key) {
        bad += key_done[key] != 0;   // a (group, column) seen before must not reappear
        if (prev_key >= 0) key_done[prev_key] = 1;
        prev_key = key;
      }
    }
    for (int i = 0; i < nblocks * n_tiles; ++i) bad += seen[i] != 1;
  }
  // the rotated block order within a column tile (group_slot) is a
  // permutation of the group's slots for every group size and column tile,
  // as both tile orders (expert groups and fixed row-block groups) need
  for (int gs = 1; gs <= 16; ++gs)
    for (int nt = 0; nt < 512; ++nt) {
      uint32_t hit = 0;
      for (int i = 0; i < gs; ++i) {
        const int j = group_slot(i, nt, gs);
        bad += j < 0 || j >= gs;
        if (j >= 0 && j < gs) hit |= 1u << j;
      }
      bad += hit != (gs == 32 ? ~0u : (1u << gs) - 1u);
    }
  // an expert_ids table that is not ascending (not what moe_align writes):
  // the grouped order may skip tiles, but never pairs a block with another
  // expert's weights
  for (int trial = 0; trial < 300; ++trial) {
    int32_t ids[64];
    const int nblocks = 1 + (int)(rnd() % 64), E = 1 + (int)(rnd() % 8);
    for (int i = 0; i < nblocks; ++i) ids[i] = (int)(rnd() % (E + 1)) - (rnd() % 8 == 0 ? 1 : 0);
    const int R = 1 + (int)(rnd() % 4), n_tiles = 1 + (int)(rnd() % 5);
    for (int t = 0; t < nblocks * n_tiles; ++t) {
      int b = -1, nt = -1, ex = -1;
      if (expert_group_tile(t, n_tiles, R, nblocks, ids, E, b, nt, ex))
        bad += b < 0 || b >= nblocks || nt < 0 || nt >= n_tiles || ids[b] != ex;
    }
  }
  // weight loads (w_lane_offset + w_group_soffset, as the kernel forms them):
  // for every group size, chunk length and group count the dispatcher can
  // use, every piece a lane loads -- including the groups past the last one
  // that a partial last chunk requests -- lies inside the expert's [N, K/2]
  // slice, and the pieces of a group gg < G tile exactly its GS/2 bytes of
  // its column
  for (int GS = 64; GS <= 256; GS *= 2) {
    const int piece = GS == 64 ? 8 : 16, pieces = GS == 64 ? 1 : GS / 128;
    for (int KCG = 1; KCG <= 16; KCG *= 2)
      for (int G = 1; G <= 72; ++G)
        for (int N = 1; N <= 3; ++N) {
          const uint32_t khalf = (uint32_t)(G * GS / 2), slice = (uint32_t)N * khalf;
          const int nchunks = (G + KCG - 1) / KCG;
          for (int gg = 0; gg < nchunks * KCG; ++gg)
            for (int col = 0; col < N; ++col) {
              uint8_t cover[128];
              memset(cover, 0, sizeof(cover));
              for (int kb = 0; kb < 4; ++kb)
                for (int h = 0; h < pieces; ++h) {
                  const uint32_t start =
                      w_lane_offset(col, khalf, kb, GS) + 16u * h + (uint32_t)w_group_soffset(gg, G, GS);
                  bad += start + piece > slice;
                  if (gg < G) {
                    const uint32_t g0 = (uint32_t)col * khalf + (uint32_t)(gg * GS / 2);
                    if (start < g0 || start + piece > g0 + GS / 2) {
                      ++bad;
                    } else {
                      for (int i = 0; i < piece; ++i) cover[start - g0 + i]++;
                    }
                  }
                }
              if (gg < G)
                for (int i = 0; i < GS / 2; ++i) bad += cover[i] != 1;
            }
        }
  }
  // activation chunks: the descriptor of chunk ch starts at ch * KC and ends
  // where the tensor ends ((rows - 1) * ldx + K bytes); every unit of real
  // data (k < K) of every row reads inside it, so none is zeroed by the
  // range check
  for (int GS = 64; GS <= 256; GS *= 2)
    for (int KCG = 1; KCG <= 16; KCG *= 2)
      for (int G = 1; G <= 40; ++G)
        for (int rows = 1; rows <= 3; ++rows)
          for (int pad = 0; pad <= 64; pad += 16) {
            const int K = G * GS, KC = KCG * GS, ldx = K + pad;
            const int64_t x_bytes = (int64_t)(rows - 1) * ldx + K;
            for (int ch = 0; ch * KC < K; ++ch) {
              const int64_t size = x_bytes - (int64_t)ch * KC;
              bad += size <= 0;
              for (int r = 0; r < rows; ++r)
                for (int cu = 0; cu < KC / 16; ++cu)
                  if (ch * KC + cu * 16 < K) bad += (int64_t)r * ldx + cu * 16 + 16 > size;
            }
          }
  // bf16 round to nearest even
  struct Case { uint32_t in; uint16_t out; };
  const Case cases[] = {
      {0x3f800000u, 0x3f80}, {0x3f808000u, 0x3f80}, {0x3f818000u, 0x3f82}, {0x3f808001u, 0x3f81},
      {0xbf80ffffu, 0xbf81}, {0x7f7fffffu, 0x7f80}, {0x00000000u, 0x0000}, {0x7fc00000u, 0x7fc0}};
  for (const Case& c : cases) bad += bf16_rne_bits(c.in) != c.out;
  if (bad) fail(MW4A8_ERR_INVALID, "host self-test: %d checks failed", bad);
  return bad;
}

}  // extern "C"
