// Host-side driver for the AddressSanitizer build of the C ABI (built and
// run by tests/test_host_asan.py; needs no GPU). It calls every entry point
// with arguments the validation must reject before any device work, the
// size helpers, and the CPU self-test, and checks each return code. Under
// -fsanitize=address any out-of-bounds or use-after-free access in the host
// code on these paths aborts the run.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "mw4a8.h"

static int failures = 0;

static void expect(int got, int want, const char* what) {
  if (got != want) {
    fprintf(stderr, "FAIL %s: got %d want %d (%s)\n", what, got, want, mw4a8_last_error());
    ++failures;
  }
}

int main() {
  void* p = (void*)4096;
  const int8_t* x = (const int8_t*)p;
  const float* f = (const float*)p;
  const uint8_t* w = (const uint8_t*)p;
  const int8_t* z = (const int8_t*)p;
  const int32_t* o = (const int32_t*)p;
  uint16_t* out = (uint16_t*)p;
  int32_t* i32 = (int32_t*)p;

  expect(mw4a8_host_selftest(), 0, "host self-test");
  expect(mw4a8_abi_version(), 1, "abi version");
  // grouped GEMM: K % group_size, group size, null pointer, row stride, workspace
  expect(mw4a8_grouped_gemm(x, 256, f, w, f, z, o, out, 64, 4, 64, 200, 2, 128, p, 1 << 20, NULL), -1, "K % gs");
  if (strstr(mw4a8_last_error(), "multiple") == NULL) ++failures;
  expect(mw4a8_grouped_gemm(x, 256, f, w, f, z, o, out, 64, 4, 64, 256, 2, 32, p, 1 << 20, NULL), -2, "gs 32");
  expect(mw4a8_grouped_gemm(NULL, 256, f, w, f, z, o, out, 64, 4, 64, 256, 2, 128, p, 1 << 20, NULL), -1, "null x");
  expect(mw4a8_grouped_gemm(x, 260, f, w, f, z, o, out, 64, 4, 64, 256, 2, 128, p, 1 << 20, NULL), -1, "ldx % 16");
  expect(mw4a8_grouped_gemm(x, 256, f, w, f, z, o, out, 64, 4, 64, 256, 2, 128, p, 16, NULL), -3, "workspace");
  expect(mw4a8_grouped_gemm(x, 256, f, w, f, z, o, out, 64, 0, 64, 256, 2, 128, p, 1 << 20, NULL), 0, "no rows");
  expect(mw4a8_grouped_gemm(x, 1 << 20, f, w, f, z, o, out, 64, 4096, 64, 256, 2, 128, p, 1 << 20, NULL), -2,
         "32-bit offsets");
  expect(mw4a8_debug_partials(x, 256, w, z, o, i32, 4, 64, 200, 2, 128, p, 1 << 20, NULL), -1, "debug K % gs");
  expect(mw4a8_grouped_gemm_noalloc(x, 256, f, w, f, z, o, out, 64, 800000, 64, 256, 100000, 128, NULL), -2,
         "noalloc beyond its scratch");
  expect(mw4a8_grouped_gemm_noalloc(x, 260, f, w, f, z, o, out, 64, 4, 64, 256, 2, 128, NULL), -1, "noalloc ldx");
  // routing and the routed GEMM
  expect(mw4a8_moe_align(o, 8, 2048, 16, i32, i32, i32, NULL, NULL), -2, "E > 1024");
  expect(mw4a8_moe_align(NULL, 8, 8, 16, i32, i32, i32, NULL, NULL), -1, "null ids");
  expect(mw4a8_fused_moe(x, 256, f, w, f, z, o, o, o, f, 2, out, 64, 4, 64, 256, 2, 128, 48, NULL), -2, "block_m 48");
  expect(mw4a8_fused_moe(x, 256, f, w, f, z, o, o, o, f, 0, out, 64, 4, 64, 256, 2, 128, 16, NULL), -1, "topk 0");
  expect(mw4a8_fused_moe_repacked(x, 256, f, w, f, z, NULL, o, o, f, 2, out, 64, 4, 64, 256, 2, 128, 16, NULL), -1,
         "null routing");
  expect(mw4a8_debug_partials_routed(x, 256, f, w, f, z, o, o, o, f, 2, out, 64, NULL, 4, 64, 256, 2, 128, 16, 0,
                                     NULL), -1, "null partials");
  expect(mw4a8_repack_weights(w, (uint8_t*)p, 2, 4, 16, 0, NULL), -1, "in place repack");
  expect(mw4a8_repack_weights(w, (uint8_t*)8192, 2, 4, 12, 0, NULL), -1, "repack K % 8");
  // layer kernels
  expect(mw4a8_quant_rows((const uint16_t*)p, 20, 4, 20, (int8_t*)p, 24, (float*)p, NULL), -1, "quant K % 8");
  expect(mw4a8_router_topk(f, 2048, 4, 2048, 8, 1, i32, (float*)p, NULL), -2, "router E");
  expect(mw4a8_silu_mul_quant((const uint16_t*)p, 64, 4, 64, (int8_t*)p, 64, (float*)p, NULL), -1, "silu ldh");
  expect(mw4a8_combine_topk((const uint16_t*)p, 12, 4, 2, 12, NULL, out, 12, NULL), -1, "combine N % 8");
  // size helpers
  int sl = 0, bl = 0;
  expect(mw4a8_align_sizes(8, 256, 16, &sl, &bl), 0, "align sizes");
  expect(sl, 8 + 256 * 15, "sorted_len");
  expect(bl, (8 + 256 * 15 + 15) / 16, "blocks_len");
  expect(mw4a8_align_sizes(-1, 4, 16, &sl, &bl), -1, "negative pairs");
  expect(mw4a8_select_block_m(32768, 256, 4096, 7168, 128), 128, "select_block_m prefill");
  expect(mw4a8_select_block_m(8, 256, 4096, 7168, 128), 16, "select_block_m decode");
  // block table for at most (4096 + 256 * 15) / 16 = 496 row blocks: 256 + 3 * 4 * 496 bytes, 256-aligned
  expect((int)mw4a8_workspace_bytes(4096, 4096, 7168, 256, 128), 6400, "workspace bytes");
  // a long error message stays inside the thread-local buffer
  expect(mw4a8_grouped_gemm(x, 256, f, w, f, z, o, out, 64, -5, 64, 256, 2, 128, p, 1 << 20, NULL), -1, "rows < 0");
  if (strlen(mw4a8_last_error()) == 0) ++failures;
  if (failures) {
    fprintf(stderr, "%d checks failed\n", failures);
    return 1;
  }
  printf("host ABI checks passed\n");
  return 0;
}
