// W4A8 grouped GEMM for gfx950 (int8 MFMA, int32 accumulation per K-group).
//
// One workgroup computes a BM x BN output tile for one expert. Its waves
// split the BN columns (WN columns each) and all share the BM activation
// rows, which are staged through LDS once per K-chunk. Each wave streams its
// own packed int4 weight columns straight from HBM into registers with
// 128-bit loads (four lanes cover the 64 contiguous bytes of one column's
// 128-wide K-group), unpacks them to int8 with the zero point folded in
// (mw4a8_pack.h), and feeds v_mfma_i32_16x16x64_i8.
//
// Per K-group the int32 MFMA accumulators start from zero; at the end of the
// group they are converted to fp32 and multiplied by the group scale into an
// fp32 accumulator (docs/Task1.md:99-107, int32 per group as the Hygon
// kernel does it). The epilogue multiplies by the per-row activation scale
// and, for routed launches, the top-k routing weight, rounds to bf16 and
// stores the row (docs/Task1.md:109-112).
//
// Pipelining: the activation chunk and the weight registers of chunk c+1
// are requested before chunk c is computed; LDS is double-buffered so one
// barrier per chunk suffices.
//
// Grid: a 1-D list of (row block, column tile) pairs, a multiple of 8 long.
// Workgroup L runs on XCD L % 8, so tile t = (L % 8) * per_xcd + L / 8 gives
// every XCD a contiguous run of the list. The list walks R row blocks
// (usually of one expert) across all column tiles before moving on, so the
// activation rows and the weight tile a row block pair shares stay in that
// XCD's L2.
#include "mw4a8_internal.h"
#include "mw4a8_pack.h"

namespace mw4a8 {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int BM, int WN, int NW, int GS, int KCG, bool ROUTED, bool DEBUGP>
__global__ __launch_bounds__(NW * 64) void w4a8_gemm_kernel(const GemmArgs a) {
  constexpr int NT = NW * 64;
  constexpr int MB = BM / 16;         // 16-row blocks per tile
  constexpr int NB = WN / 16;         // 16-column blocks per wave
  constexpr int BN = NW * WN;
  constexpr int S = GS / 64;          // MFMA K-steps per group
  constexpr int WD = 2 * S;           // packed dwords per lane per (group, column block)
  constexpr int KC = KCG * GS;        // activation bytes per row per chunk
  constexpr int PITCH = KC + 16;      // LDS row pitch in bytes
  constexpr int UPR = KC / 16;        // 16-byte units per row and chunk
  constexpr int XU = (BM * UPR + NT - 1) / NT;
  static_assert(BM % 16 == 0 && WN % 16 == 0 && GS % 64 == 0, "tile shape");

  __shared__ __attribute__((aligned(16))) int8_t s_x[2][BM * PITCH];
  __shared__ int s_src[BM];
  __shared__ int s_dst[BM];
  __shared__ float s_xs[BM];
  __shared__ float s_tw[BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int jl = lane & 15;   // row (A) / column (B) within a 16-block
  const int kb = lane >> 4;   // K slot group of the MFMA operands

  // ---- tile decode -------------------------------------------------------
  const int L = blockIdx.x;
  const int t = (L & 7) * a.per_xcd + (L >> 3);
  if (t >= a.total_tiles) return;
  const int span = a.n_tiles * a.R;
  const int chunk_id = t / span;
  const int rem = t - chunk_id * span;
  const int nt = rem / a.R;
  const int b = chunk_id * a.R + (rem - nt * a.R);
  int e;
  if constexpr (ROUTED) {
    // (b + 1) * BM <= sorted_len also bounds expert_ids, whose length is
    // ceil(sorted_len / BM)
    if (b >= a.num_post_pad[0] / BM || (int64_t)(b + 1) * BM > a.sorted_len) return;
    e = a.expert_ids[b];
    if (e >= a.E) return;
  } else {
    if (b >= a.blk_count[0]) return;
    e = a.blk_expert[b];
  }
  if (e < 0) return;

  if (tid < BM) {
    int src = -1, dst = -1;
    float xsv = 0.f, twv = 1.f;
    if constexpr (ROUTED) {
      const int s = a.sorted_ids[b * BM + tid];
      if (s >= 0 && s < a.num_pairs) {
        src = s / a.topk;
        dst = s;
        xsv = a.xs[src];
        twv = a.tw[s];
      }
    } else {
      const int r = a.blk_row0[b] + tid;
      if (r < a.blk_row1[b]) {
        src = dst = r;
        if constexpr (!DEBUGP) xsv = a.xs[r];
      }
    }
    s_src[tid] = src;
    s_dst[tid] = dst;
    s_xs[tid] = xsv;
    s_tw[tid] = twv;
  }
  __syncthreads();

  const int nchunks = (a.G + KCG - 1) / KCG;
  const int col0 = nt * BN + wave * WN;
  const int64_t khalf = a.K / 2;

  // ---- activation chunk: global -> registers -> (relabelled) LDS ---------
  u32x4 xr[XU];
  auto load_x = [&](int ch) {
#pragma unroll
    for (int j = 0; j < XU; ++j) {
      const int u = tid + j * NT;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (u < BM * UPR) {
        const int row = u / UPR;
        const int k = ch * KC + (u - row * UPR) * 16;
        const int src = s_src[row];
        if (src >= 0 && k < a.K) v = *reinterpret_cast<const u32x4*>(a.x + (int64_t)src * a.ldx + k);
      }
      xr[j] = v;
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int j = 0; j < XU; ++j) {
      const int u = tid + j * NT;
      if (u < BM * UPR) {
        const int row = u / UPR;
        const int c = u - row * UPR;
        const u32x4 v = xr[j];
        u32x4 p;
        p.x = even_bytes(v.x, v.y);
        p.y = odd_bytes(v.x, v.y);
        p.z = even_bytes(v.z, v.w);
        p.w = odd_bytes(v.z, v.w);
        *reinterpret_cast<u32x4*>(&s_x[buf][row * PITCH + c * 16]) = p;
      }
    }
  };

  // ---- weights, zero points and scales of one chunk ----------------------
  uint32_t wc[KCG][NB][WD], wn[KCG][NB][WD];
  int zc[KCG][NB], zn[KCG][NB];
  float sc[KCG][NB], sn[KCG][NB];
  auto load_w = [&](int ch, uint32_t (&wd)[KCG][NB][WD], int (&zd)[KCG][NB], float (&sd)[KCG][NB]) {
#pragma unroll
    for (int g = 0; g < KCG; ++g) {
      const int gg = ch * KCG + g;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int col = col0 + nb * 16 + jl;
        const bool ok = gg < a.G && col < a.N;
        const int64_t rowc = (int64_t)e * a.N + col;
        if (ok) {
          const uint8_t* p = a.w + rowc * khalf + (int64_t)gg * (GS / 2) + kb * (GS / 8);
          if constexpr (S == 1) {
            const u32x2 q = *reinterpret_cast<const u32x2*>(p);
            wd[g][nb][0] = q.x;
            wd[g][nb][1] = q.y;
          } else {
#pragma unroll
            for (int h = 0; h < S / 2; ++h) {
              const u32x4 q = *reinterpret_cast<const u32x4*>(p + 16 * h);
              wd[g][nb][4 * h + 0] = q.x;
              wd[g][nb][4 * h + 1] = q.y;
              wd[g][nb][4 * h + 2] = q.z;
              wd[g][nb][4 * h + 3] = q.w;
            }
          }
          zd[g][nb] = a.wz[rowc * a.G + gg];
          if constexpr (!DEBUGP) sd[g][nb] = a.ws[rowc * a.G + gg];
        } else {
#pragma unroll
          for (int d = 0; d < WD; ++d) wd[g][nb][d] = 0u;
          zd[g][nb] = 0;
          sd[g][nb] = 0.f;
        }
      }
    }
  };

  float acc[MB][NB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[mb][nb][r] = 0.f;

  load_x(0);
  load_w(0, wc, zc, sc);

  for (int ch = 0; ch < nchunks; ++ch) {
    const int buf = ch & 1;
    store_x(buf);
    __syncthreads();
    if (ch + 1 < nchunks) {
      load_x(ch + 1);
      load_w(ch + 1, wn, zn, sn);
    }
    const int8_t* xb = s_x[buf];
#pragma unroll
    for (int g = 0; g < KCG; ++g) {
      const int gg = ch * KCG + g;
      if (gg < a.G) {
        i32x4 bfr[NB][S];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const ZeroFold zf = make_zero_fold(zc[g][nb]);
#pragma unroll
          for (int s = 0; s < S; ++s) {
            const uint32_t d0 = wc[g][nb][2 * s];
            const uint32_t d1 = wc[g][nb][2 * s + 1];
            bfr[nb][s].x = (int)fold_even(d0, zf);
            bfr[nb][s].y = (int)fold_odd(d0, zf);
            bfr[nb][s].z = (int)fold_even(d1, zf);
            bfr[nb][s].w = (int)fold_odd(d1, zf);
          }
        }
        i32x4 part[MB][NB];
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            const i32x4 av = *reinterpret_cast<const i32x4*>(
                xb + (mb * 16 + jl) * PITCH + g * GS + kb * (GS / 4) + 16 * s);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              const i32x4 cin = (s == 0) ? i32x4{0, 0, 0, 0} : part[mb][nb];
              part[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bfr[nb][s], cin, 0, 0, 0);
            }
          }
        }
        if constexpr (DEBUGP) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              const int col = col0 + nb * 16 + jl;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int dst = s_dst[mb * 16 + kb * 4 + r];
                if (dst >= 0 && col < a.N)
                  a.dbg[((int64_t)dst * a.N + col) * a.G + gg] = part[mb][nb][r];
              }
            }
        } else {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                acc[mb][nb][r] = __builtin_fmaf((float)part[mb][nb][r], sc[g][nb], acc[mb][nb][r]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < KCG; ++g)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int d = 0; d < WD; ++d) wc[g][nb][d] = wn[g][nb][d];
        zc[g][nb] = zn[g][nb];
        sc[g][nb] = sn[g][nb];
      }
  }

  if constexpr (!DEBUGP) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int col = col0 + nb * 16 + jl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = mb * 16 + kb * 4 + r;
          const int dst = s_dst[row];
          if (dst >= 0 && col < a.N) {
            float v = acc[mb][nb][r] * s_xs[row];
            if constexpr (ROUTED) v = v * s_tw[row];
            a.out[(int64_t)dst * a.ldo + col] = bf16_rne_bits(__float_as_uint(v));
          }
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Launch geometry and dispatch.

static void set_grid(GemmArgs& a, int max_blocks, int BN, int R) {
  a.n_tiles = (a.N + BN - 1) / BN;
  a.R = R;
  const int chunks = (max_blocks + R - 1) / R;
  a.total_tiles = chunks * R * a.n_tiles;
  a.per_xcd = (a.total_tiles + 7) / 8;
}

template <int BM, int WN, int NW, int GS, int KCG, bool ROUTED, bool DEBUGP>
static hipError_t launch_one(GemmArgs a, int max_blocks, int R, hipStream_t s) {
  set_grid(a, max_blocks, NW * WN, R);
  if (a.total_tiles == 0) return hipSuccess;
  hipLaunchKernelGGL((w4a8_gemm_kernel<BM, WN, NW, GS, KCG, ROUTED, DEBUGP>), dim3(8 * a.per_xcd),
                     dim3(NW * 64), 0, s, a);
  return hipGetLastError();
}

template <int GS, bool ROUTED>
static hipError_t dispatch_bm(GemmArgs a, const TileConfig& c, int max_blocks, hipStream_t s) {
  // K-chunk sizes keep KCG * GS at 512 activation bytes per row for small
  // row blocks and 256 for large ones.
  switch (c.BM) {
    case 16: return launch_one<16, 16, 4, GS, 512 / GS, ROUTED, false>(a, max_blocks, c.R, s);
    case 32: return launch_one<32, 16, 4, GS, 512 / GS, ROUTED, false>(a, max_blocks, c.R, s);
    case 64: return launch_one<64, 32, 4, GS, 256 / GS, ROUTED, false>(a, max_blocks, c.R, s);
    case 128: return launch_one<128, 32, 4, GS, 256 / GS, ROUTED, false>(a, max_blocks, c.R, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_grouped_gemm(GemmArgs a, const TileConfig& cfg, int group_size, bool routed,
                               int max_blocks, hipStream_t s) {
  if (group_size == 128)
    return routed ? dispatch_bm<128, true>(a, cfg, max_blocks, s) : dispatch_bm<128, false>(a, cfg, max_blocks, s);
  if (group_size == 64)
    return routed ? dispatch_bm<64, true>(a, cfg, max_blocks, s) : dispatch_bm<64, false>(a, cfg, max_blocks, s);
  if (group_size == 256)
    return routed ? dispatch_bm<256, true>(a, cfg, max_blocks, s) : dispatch_bm<256, false>(a, cfg, max_blocks, s);
  return hipErrorInvalidValue;
}

hipError_t launch_debug_partials(GemmArgs a, int group_size, int max_blocks, hipStream_t s) {
  if (group_size == 128) return launch_one<16, 16, 4, 128, 4, false, true>(a, max_blocks, 1, s);
  if (group_size == 64) return launch_one<16, 16, 4, 64, 8, false, true>(a, max_blocks, 1, s);
  if (group_size == 256) return launch_one<16, 16, 4, 256, 2, false, true>(a, max_blocks, 1, s);
  return hipErrorInvalidValue;
}

int max_row_blocks(int rows, int experts, int BM) {
  if (rows <= 0) return 0;
  const int64_t ne = experts < rows ? experts : rows;
  const int64_t bound = ((int64_t)rows + ne * (BM - 1)) / BM;
  return (int)(bound < rows ? bound : rows);
}

TileConfig select_tiles(int rows, int touched_experts, int N, int K, int group_size) {
  (void)N;
  (void)K;
  (void)group_size;
  const int ne = touched_experts < 1 ? 1 : touched_experts;
  const int per_expert = (rows + ne - 1) / ne;
  TileConfig c;
  c.NW = 4;
  if (per_expert <= 16) {
    c.BM = 16; c.WN = 16; c.KCG = 512 / group_size; c.R = 1;
  } else if (per_expert <= 32) {
    c.BM = 32; c.WN = 16; c.KCG = 512 / group_size; c.R = 1;
  } else if (per_expert <= 64) {
    c.BM = 64; c.WN = 32; c.KCG = 256 / group_size; c.R = 2;
  } else {
    c.BM = 128; c.WN = 32; c.KCG = 256 / group_size; c.R = 2;
  }
  return c;
}

}  // namespace mw4a8
