// W4A8 grouped GEMM for gfx950 (int8 MFMA, int32 accumulation per K-group).
//
// One workgroup computes a BM x BN output tile for one expert. Its waves
// split the BN columns (WN columns each) and all share the BM activation
// rows, which are staged through LDS once per K-chunk. Each wave streams its
// own packed int4 weight columns straight from HBM into registers with
// 128-bit buffer loads (four lanes cover the 64 contiguous bytes of one
// column's 128-wide K-group), unpacks them to int8 with the zero point folded
// in (mw4a8_pack.h), and feeds v_mfma_i32_16x16x64_i8.
//
// Per K-group and 16-row block the int32 MFMA results start from zero; right
// after the block's MFMAs they are converted to fp32 and multiplied by the
// group scale into the fp32 accumulator (docs/Task1.md:99-107, int32 per
// group as the reference's Hygon kernel does it). The epilogue multiplies by
// the per-row activation scale and, for routed launches, the top-k routing
// weight, rounds to bf16 and stores the row (docs/Task1.md:109-112).
//
// Memory access is branch-free: every global read is a raw buffer load whose
// descriptor covers exactly the tensor (or one expert's slice of it), and
// lanes with nothing to read (padding rows, columns past N) use an offset
// beyond the descriptor, which the hardware returns as zero. A tile whose
// valid rows fit in its top half runs a half-height body, so a nearly empty
// last row block of an expert costs at most half a tile of MFMAs.
//
// Pipelining: the activation chunk and the weight registers of chunk c+1 are
// requested before chunk c is computed. Weights ping-pong between two
// register sets (the loop is unrolled by two chunks, so no copies), and LDS
// is double-buffered, so one barrier per chunk suffices.
//
// Grid: a 1-D list of (row block, column tile) pairs, sized on the host for
// the worst-case number of row blocks. Workgroup L runs on XCD L % 8; with
// per_xcd = ceil(actual tiles / 8), tile t = (L % 8) * per_xcd + L / 8 gives
// every XCD an equal, contiguous run of the actual tiles. The list walks R row blocks
// (usually of one expert) across all column tiles before moving on, so the
// activation rows and the weight tile a row block pair shares stay in that
// XCD's L2.
//
// Memory safety of the loads: the hardware range check of a raw buffer load
// covers its vector offset, not the scalar one. Every scalar offset here
// therefore stays inside the tensor by construction: weight groups past the
// last one (a partial last K-chunk) are clamped to the last group, and the
// activation chunk offset moves the descriptor's base (and shrinks its
// size) instead of travelling as a scalar offset, so the range check still
// covers the end of the activation tensor.
//
// This header holds the kernel template and its launch helpers; each
// gemm_*.hip file instantiates dispatch_bm for one row source.
#pragma once
#include <mutex>
#include <type_traits>

#include "mw4a8_internal.h"
#include "mw4a8_pack.h"

namespace mw4a8 {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr uint32_t kOOB = 0x80000000u;   // buffer offset that reads as zero
// float bits of 12582912 = 1.5 * 2^23: adding an integer P with |P| <= 2^22 to
// them gives the float 12582912 + P exactly
constexpr int kMagic = 0x4B400000;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
// two fp32 -> packed bf16 (a low, b high), round to nearest even: one
// v_cvt_pk_bf16_f32 (same bits as bf16_rne_bits for every non-NaN input)
__device__ __forceinline__ uint32_t bf16x2_rne(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
constexpr float kMagicF = 12582912.0f;
constexpr int kRsrcFlags = 0x00020000;   // raw buffer, 32-bit data format

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcFlags);
}

// The thread's index, read so that the compiler cannot reuse an earlier
// read: in a persistent launch every value a tile body derives from it is
// then computed inside the tile loop rather than hoisted out of it and kept
// live across the whole loop (which spilled the 128-row bodies).
__device__ __forceinline__ int opaque_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// KCG consecutive int8 zero points at byte offset `off` (KCG-aligned), kept
// as raw words (zero point g is byte g % 4 of w[g / 4]). They are
// sign-extended where they are used (zero_of), not here: extracting them
// right after the load would make the wave wait for the load, and with it
// for every load issued before it.
template <int KCG>
__device__ __forceinline__ void load_zero_run(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t (&w)[(KCG + 3) / 4]) {
  if constexpr (KCG == 1) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
  } else if constexpr (KCG == 2) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  } else if constexpr (KCG == 4) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  } else if constexpr (KCG == 8) {
    const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    w[0] = q.x;
    w[1] = q.y;
  } else {
    static_assert(KCG % 16 == 0, "zero-point run length");
#pragma unroll
    for (int h = 0; h < KCG / 16; ++h) {
      const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * h, 0, 0);
      w[4 * h] = q.x;
      w[4 * h + 1] = q.y;
      w[4 * h + 2] = q.z;
      w[4 * h + 3] = q.w;
    }
  }
}

template <int KCG>
__device__ __forceinline__ int zero_of(const uint32_t (&w)[(KCG + 3) / 4], int g) {
  return (int)(int8_t)((w[g / 4] >> (8 * (g % 4))) & 0xffu);
}

// KCG consecutive fp32 scales at byte offset `off` (4*KCG-aligned up to 16).
template <int KCG, int NB>
__device__ __forceinline__ void load_scale_run(__amdgpu_buffer_rsrc_t r, uint32_t off, float (&dst)[KCG][NB],
                                               int nb) {
  if constexpr (KCG == 1) {
    dst[0][nb] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  } else if constexpr (KCG == 2) {
    const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    dst[0][nb] = __uint_as_float(q.x);
    dst[1][nb] = __uint_as_float(q.y);
  } else {
    static_assert(KCG % 4 == 0, "scale run length");
#pragma unroll
    for (int h = 0; h < KCG / 4; ++h) {
      const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * h, 0, 0);
      dst[4 * h][nb] = __uint_as_float(q.x);
      dst[4 * h + 1][nb] = __uint_as_float(q.y);
      dst[4 * h + 2][nb] = __uint_as_float(q.z);
      dst[4 * h + 3][nb] = __uint_as_float(q.w);
    }
  }
}

// ---- LDS layout of the staged activations ---------------------------------
// ds_read_b128 / ds_write_b128 are served 32 lanes per cycle across 128
// four-byte banks, i.e. 32 sixteen-byte segments: a cycle is conflict-free
// when its 32 lanes touch 32 distinct segments (mod 32).
//
// Rows are PITCH = KC + 32 bytes apart, so PITCH / 16 = 2 * odd and the 16
// rows of an MFMA A fragment start on 16 distinct even segments. Within a
// K-group, the 16-byte unit that K slot kb of MFMA step s reads (K-order unit
// kb * S + s) is stored at position 4 * s + kb; lanes 0-31 (kb = 0, 1) then
// read 32 distinct segments for every s.
//
// Stores: a 32-lane half writes 32 / UPR rows (UPR 16-byte units per row).
// Rows r and r + XD, with (PITCH / 16) * XD = UPR (mod 32), land on disjoint
// segment ranges, so each half writes such rows: row_of_group() maps the
// q-th row group of the thread order to a row, bijectively within every 16
// rows.
__host__ __device__ constexpr int lds_row_step(int upr) {
  int d = 1;
  while (d < 32 && ((upr + 2) * d) % 32 != upr % 32) ++d;
  return d;
}

template <int UPR>
__device__ __forceinline__ int row_of_group(int q) {
  if constexpr (UPR >= 32) {
    return q;
  } else {
    constexpr int XR = 32 / UPR;            // rows per 32-lane half
    constexpr int XD = lds_row_step(UPR);   // row distance within a half
    static_assert(XR * XD == 16, "row interleave must tile 16 rows");
    const int j = q % XR, b = q / XR;
    return (b % XD) + XD * j + 16 * (b / XD);
  }
}

// LDS byte position of K-order unit cu (16 bytes) within a row's chunk.
template <int GS>
__device__ __forceinline__ int unit_pos(int cu) {
  constexpr int S = GS / 64, UG = GS / 16;
  const int g = cu / UG, v = cu - g * UG;
  return 16 * (g * UG + (v % S) * 4 + v / S);
}

// Chunks per zero-point/scale window (ZSV): the window's runs are read with
// one vector load each per column block. RD chunks (the loop's unroll) while
// the window's scales fit in 8 registers, else one chunk.
// Decode tiles (bm < 64) keep one chunk per window: each ring slot carries
// its chunk's runs, requested with the chunk's weights.
// Runs of 1, 2, 4 or 8 groups have a vector load (load_zero_run /
// load_scale_run); other windows fall back to one chunk.
__host__ __device__ constexpr int zs_window(int kcg, int rd, int bm) {
  return bm < 64 ? 1 : ((kcg * rd <= 8 && (kcg * rd & (kcg * rd - 1)) == 0) ? rd : 1);
}

// Per-tile values shared by the kernel's setup and its tile bodies.
struct TileCtx {
  int e;          // expert
  int blk;        // row block
  int row0, row1; // reference layout: the block's rows [row0, row1)
  int col0;       // first column of this wave
  int tile_col0;  // first column of the workgroup's tile
  int nchunks;    // K-chunks
  int rows;       // rows of the tile holding data (the rest is padding)
  int tail;       // routed tiles with a tail: the block whose first slots follow this block's rows, or -1
};

// Routed slot s of sorted_ids: the pair's activation row (src) and output row
// (dst), or -1 for padding.
__device__ __forceinline__ void routed_slot(const GemmArgs& a, int slot, int& src, int& dst) {
  src = dst = -1;
  const int s = a.sorted_ids[slot];
  if (s >= 0 && s < a.num_pairs) {
    src = s / a.topk;
    dst = s;
  }
}

// Routed block x holds at most T pairs: its slot T is padding. (An expert's
// pairs fill its blocks from the first slot on, so only its last block can
// be short, and its pairs are that block's first slots.)
template <int BM, int T>
__device__ __forceinline__ bool short_block(const GemmArgs& a, int x) {
  const int s = a.sorted_ids[x * BM + T];
  return s < 0 || s >= a.num_pairs;
}

// Row r of the tile's row block: the activation row it reads (src) and the
// output row it writes (dst), -1 for padding. Routed: the pair in slot
// blk * BM + r of sorted_ids; reference layout: row row0 + r below row1.
template <int BM, bool ROUTED>
__device__ __forceinline__ void row_source(const GemmArgs& a, const TileCtx& c, int r, int& src, int& dst) {
  src = dst = -1;
  if constexpr (ROUTED) {
    routed_slot(a, c.blk * BM + r, src, dst);
  } else {
    const int row = c.row0 + r;
    if (row < c.row1) src = dst = row;
  }
}

// Epilogue factors of a row with dst >= 0: activation scale and (routed)
// top-k weight. The reference-layout debug export may pass no scales.
template <bool ROUTED, bool DEBUGP>
__device__ __forceinline__ void row_scales(const GemmArgs& a, int src, int dst, float& xsv, float& twv) {
  xsv = 0.f;
  twv = 1.f;
  if (!DEBUGP || a.xs != nullptr) xsv = a.xs[src];
  if constexpr (ROUTED) twv = a.tw ? a.tw[dst] : 1.f;
}

// Routed decode tiles: the sorted_ids entries a thread needs, requested by
// the kernel entry together with the tile's expert and the block count --
// its own row's (own, threads < BM) and those of the rows of its XU
// activation staging units (unit[j] for unit threadIdx.x + j * threads).
template <int XU>
struct DecodeSlots {
  int own;
  int unit[XU];
};

// Staging units per thread of a BMX-row tile body (16-byte units of the
// activation chunk over the workgroup's threads).
__host__ __device__ constexpr int staging_units(int BMX, int KCG, int GS, int NW) {
  return (BMX * (KCG * GS / 16) + NW * 64 - 1) / (NW * 64);
}

// Work a persistent launch fits into a tile body (see the persistent
// kernel): before_barrier() runs once the body has requested its first
// chunk's loads (before the body's first barrier), before_epilogue() once
// the K loop is done, before_stores() in the epilogue before its first
// global store (values loaded in before_epilogue() are consumed there:
// waiting for a load issued before the output stores, whose number varies
// by row, waits for all of them), and the row factors ep_xs / ep_tw
// (activation scale, routing weight of row threadIdx.x) go to LDS just
// before the epilogue, their loads having run during the K loop. With an
// LDS zero/scale block, the persistent kernel has stored the tile's block
// before the body starts. A plain launch has no hooks.
struct NoHooks {
  static constexpr bool kActive = false;
  float ep_xs = 0.f, ep_tw = 1.f;
  __device__ __forceinline__ void before_barrier() {}
  __device__ __forceinline__ void before_epilogue() {}
  __device__ __forceinline__ void before_stores() {}
};

// Workgroup-wide AND of pred behind one barrier (__syncthreads_and takes
// three, with two LDS round trips): each wave's ballot goes to its own LDS
// word, read by every thread after the barrier. Calls must be separated by
// at least one other barrier (a tile body has several), so that no wave
// writes its word again while another still reads the previous values.
// (Used by the plain-grid prefill tiles: Qwen3 M=2048 -0.7 %; in the decode
// prologue it measured up to 1.3 % slower.)
template <int NW>
__device__ __forceinline__ bool block_and(bool pred) {
  __shared__ int s_wand[NW];
  const int tid = opaque_tid();
  const int w = __ballot(!pred) == 0;
  if ((tid & 63) == 0) s_wand[tid >> 6] = w;
  __syncthreads();
  int r = 1;
#pragma unroll
  for (int i = 0; i < NW; ++i) r &= s_wand[i];
  return r != 0;
}

// Main K loop and epilogue for the first BMX rows of a tile (BMX <= BM).
//
// RD: weight-register ring depth. The weights (and, unless ZS_LDS, the zero
//     points and scales) of chunk c + RD - 1 are requested while chunk c is
//     computed.
// ZSG: when positive, the tile's whole [BN x G] zero-point and scale block
//     (G <= ZSG) is copied into LDS once -- it is contiguous in memory -- so
//     the K loop issues no loads for them. When zero they travel with the
//     weights, one vector run per column and chunk when aligned.
// FAST: the host guarantees that every chunk is full and the chunk count is
//     a multiple of RD (G % (KCG * RD) == 0) and, without ZSG, that the
//     zero-point / scale runs are aligned; the loop then carries no guards.
//     (Used for the 16- and 32-row tiles only: without the guards the
//     compiler schedules the larger bodies into scratch.)
// ZSV (ZSG == 0 only): the zero points and scales of a window of
//     zs_window(KCG, RD, BM) chunks are read as one aligned vector run each per
//     column (host-checked: G a multiple of the window's groups, 16-byte
//     aligned tensors); otherwise one scalar load per group and chunk. Every
//     such load costs the memory pipeline about as much as a 1 KB weight
//     load (each touches one cache line per column), so fewer, wider runs
//     leave more of it to the weights. It is a compile-time choice so that
//     the loads of the next chunk lie on one straight path: with a run-time
//     choice the compiler copied the loaded registers where the two paths
//     join, and waited there for every outstanding load, which serialized
//     the prefetch with the compute.
template <int BMX, int BM, int WN, int NW, int GS, int KCG, int RD, int ZSG, int RMODE, bool DEBUGP, bool FAST,
          bool ZSV, bool SYMT, int BMA = BM, class Hooks = NoHooks, class Pre = std::nullptr_t>
__device__ __forceinline__ void gemm_body(const GemmArgs& a, const TileCtx& c, int8_t* s_x, float* s_scale,
                                          int8_t* s_zero, int* s_src, int* s_dst, float* s_xs, float* s_tw,
                                          Hooks* hk = nullptr, const Pre* pre = nullptr) {
  constexpr int NT = NW * 64;
  constexpr int MB = BMX / 16;        // 16-row blocks computed
  constexpr int NB = WN / 16;         // 16-column blocks per wave
  constexpr int BN = NW * WN;
  constexpr int S = GS / 64;          // MFMA K-steps per group
  constexpr int WD = 2 * S;           // packed dwords per lane per (group, column block)
  constexpr int KC = KCG * GS;        // activation bytes per row per chunk
  constexpr int PITCH = KC + 32;      // LDS row pitch in bytes (see the layout note)
  constexpr int BUF = BMA * PITCH;    // bytes per LDS buffer (BMA rows staged: the block and a tail)
  constexpr int UPR = KC / 16;        // 16-byte units per row and chunk
  constexpr int XU = (BMX * UPR + NT - 1) / NT;
  constexpr bool ZS_LDS = ZSG > 0;
  constexpr bool ROUTED = RMODE != 0;
  constexpr bool REPACKED = RMODE == kModeRoutedRepacked;
  // SYMT: every zero point of the tile is 8 (decided by the kernel entry for
  // tiles with an LDS zero/scale block): symmetric unpack and magic-number
  // fold for every group, scales stored / 16, no zero points needed.
  // DEBUGP changes none of the arithmetic: the same body also writes each
  // exact int32 group partial (decoded from its chain, see fold) to a.dbg.
  constexpr bool MG = SYMT && ZS_LDS;

  const int tid = opaque_tid();
  const int lane = tid & 63;
  const int jl = lane & 15;   // row (A) / column (B) within a 16-block
  const int kb = lane >> 4;   // K slot group of the MFMA operands
  const uint32_t khalf = (uint32_t)a.K / 2;

  // Decode tiles (XDEEP, defined below with the activation ring) read their
  // routing rows here, before any weight load: loads complete in issue order,
  // so waiting for these rows never waits for the weights requested next.
  // PRE: routed decode tiles whose slots the kernel entry has requested
  // (DecodeSlots): no load here, and the activation offsets come from the
  // thread's own slots rather than from LDS, so the first activation chunk
  // is requested with the first weights instead of after a barrier.
  constexpr bool PRE = !std::is_same<Pre, std::nullptr_t>::value;
  int r_src = -1, r_dst = -1;
  if constexpr (BM < 64) {
    if constexpr (PRE) {
      static_assert(ROUTED && BM < 64, "preloaded slots are for routed decode tiles");
      if (tid < BM && pre->own >= 0 && pre->own < a.num_pairs) {
        r_src = pre->own / a.topk;
        r_dst = pre->own;
      }
    } else {
      if (tid < BM) row_source<BM, ROUTED>(a, c, tid, r_src, r_dst);
    }
  }

  // ---- buffer descriptors (one expert's slice for the weights) ------------
  const int64_t expert_cols = (int64_t)c.e * a.N;
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(a.w + expert_cols * khalf, (uint32_t)a.N * khalf);
  const __amdgpu_buffer_rsrc_t z_rsrc = make_rsrc(a.wz + expert_cols * a.G, (uint32_t)(a.N * a.G));
  // the reference-layout debug export passes no scales: an empty descriptor
  // (every scale reads as zero) keeps its loop identical to the product's
  const __amdgpu_buffer_rsrc_t s_rsrc =
      (DEBUGP && a.ws == nullptr) ? make_rsrc(a.wz, 0u)
                                  : make_rsrc(a.ws + expert_cols * a.G, (uint32_t)(a.N * a.G) * 4u);

  // per-lane offsets of this lane's weight columns and activation units
  uint32_t w_off[NB], zs_off[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = c.col0 + nb * 16 + jl;
    const bool ok = col < a.N;
    w_off[nb] = ok ? w_lane_offset(col, khalf, kb, GS) : kOOB;
    zs_off[nb] = ok ? (uint32_t)(col * a.G) : kOOB;
  }
  // Padding rows read zeros (out-of-range offset) and are staged like the
  // others, which keeps the staging loops free of per-lane branches; their
  // results are never stored.
  // The staging units divide evenly over the threads, except on bodies with a
  // tail (144 rows): there the last round's surplus units read nothing (the
  // out-of-range offset) and land in the 32-byte pads that end each staged
  // row (two units a row), which the A fragments never read -- so the
  // staging loops keep no per-lane branch.
  constexpr int XSURPLUS = XU * NT - BMX * UPR;
  static_assert(XSURPLUS == 0 || (PITCH - KC == 32 && XSURPLUS <= 2 * BMX),
                "staging units must divide evenly over the threads or fit the row pads");
  uint32_t x_off[XU];
  int x_lds[XU];   // LDS byte offset within a buffer
  // reads the tile's source rows from LDS (s_src), so only after they are there
  auto init_x = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < XU; ++j) {
      const int u = tid + j * NT;
      if constexpr (XSURPLUS > 0) {
        if (u >= BMX * UPR) {
          const int v = u - BMX * UPR;
          x_off[j] = kOOB;
          x_lds[j] = (v >> 1) * PITCH + KC + 16 * (v & 1);
          continue;
        }
      }
      const int q = u / UPR;
      const int cu = u - q * UPR;
      const int row = row_of_group<UPR>(q);
      int src;
      if constexpr (PRE) {
        static_assert(XSURPLUS == 0, "decode staging units divide evenly");
        const int sid = pre->unit[j];
        src = sid >= 0 && sid < a.num_pairs ? sid / a.topk : -1;
      } else {
        src = s_src[row];
      }
      x_off[j] = src >= 0 ? (uint32_t)(src * a.ldx) + (uint32_t)(cu * 16) : kOOB;
      x_lds[j] = row * PITCH + unit_pos<GS>(cu);
    }
  };
  if constexpr (BM >= 64) init_x();

  // ---- the tile's zero points and scales -> registers (ZS_LDS) -------------
  // [BN columns x G] of each, contiguous from column tile_col0; the
  // descriptors return zero past column N. All loads are issued before any
  // LDS write so their latencies overlap (and overlap the pipeline prologue).
  constexpr int SU = ZS_LDS ? (BN * ZSG / 4 + NT - 1) / NT : 1;    // scale units per thread
  constexpr int ZU = ZS_LDS ? (BN * ZSG / 16 + NT - 1) / NT : 1;   // zero-point units per thread
  const int s_units = BN * a.G / 4;
  const int z_units = BN * a.G / 16;
  u32x4 sq[SU], zq[ZU];
  // PZS: a persistent launch loaded this tile's zero/scale block during the
  // previous tile's epilogue and has stored it to LDS before the body
  constexpr bool PZS = ZS_LDS && Hooks::kActive;
  if constexpr (PZS) {
    // (stored by the persistent kernel)
  } else if constexpr (ZS_LDS) {
    const uint32_t zbase = (uint32_t)(c.tile_col0 * a.G);
#pragma unroll
    for (int j = 0; j < SU; ++j) {
      const int u = tid + j * NT;
      if (u < s_units) sq[j] = __builtin_amdgcn_raw_buffer_load_b128(s_rsrc, zbase * 4u + u * 16u, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < ZU; ++j) {
      const int u = tid + j * NT;
      if (!MG && u < z_units) zq[j] = __builtin_amdgcn_raw_buffer_load_b128(z_rsrc, zbase + u * 16u, 0, 0);
    }
  }
  // LDS index of this lane's columns in the zero/scale block
  int zs_lds[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) zs_lds[nb] = (c.col0 - c.tile_col0 + nb * 16 + jl) * a.G;

  // ---- chunk loaders -----------------------------------------------------
  // Decode tiles (16/32 rows) request a chunk's activations together with
  // its weights, RD - 1 chunks ahead, into a ring of RD register sets. Loads
  // complete in issue order, so the wait for the activations about to be
  // staged then only covers loads issued before them -- the chunk's own and
  // earlier ones -- and the later chunks' weights stay in flight. (With one
  // register set the activations of chunk c + 1 were requested after the
  // weights of chunk c + RD - 1, and staging them waited for those too.)
  constexpr bool XDEEP = BM < 64;
  constexpr int XR = XDEEP ? RD : 1;
  u32x4 xr[XR][XU];
  // the chunk's K offset moves the descriptor (scalar work) rather than going
  // into the unchecked scalar offset: units past K in a partial last chunk of
  // the tensor's last row then read as zero instead of past its end
  auto load_x = [&](int ch, int slot) __attribute__((always_inline)) {
    const uint32_t base = (uint32_t)(ch * KC);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(a.x + base, a.x_bytes - base);
#pragma unroll
    for (int j = 0; j < XU; ++j) xr[slot][j] = __builtin_amdgcn_raw_buffer_load_b128(r, x_off[j], 0, 0);
  };
  auto store_x = [&](int buf, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < XU; ++j) {
      const u32x4 v = xr[slot][j];
      if constexpr (REPACKED) {
        // the repacked weights unpack in natural K order: no relabel
        *reinterpret_cast<u32x4*>(s_x + buf * BUF + x_lds[j]) = v;
      } else {
        u32x4 p;
        p.x = even_bytes(v.x, v.y);
        p.y = odd_bytes(v.x, v.y);
        p.z = even_bytes(v.z, v.w);
        p.w = odd_bytes(v.z, v.w);
        *reinterpret_cast<u32x4*>(s_x + buf * BUF + x_lds[j]) = p;
      }
    }
  };

  struct WChunk {
    uint32_t w[KCG][NB][WD];
    int z[KCG][NB];     // !ZSV: sign-extended zero points
    float s[KCG][NB];   // !ZSV: scales
  };
  // ZSV: one window of ZW chunks (KW groups) of zero points (raw runs) and scales
  constexpr int ZW = zs_window(KCG, RD, BM);
  constexpr int KW = ZW * KCG;
  struct ZsWin {
    uint32_t zr[NB][(KW + 3) / 4];
    float s[KW][NB];
  };
  auto load_zs = [&](int win, ZsWin& d) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint32_t zo = zs_off[nb] + (uint32_t)(win * KW);
      load_zero_run<KW>(z_rsrc, zo, d.zr[nb]);
      load_scale_run<KW, NB>(s_rsrc, zo * 4u, d.s, nb);
    }
  };
  auto load_w = [&](int ch, WChunk& d) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < KCG; ++g) {
      const uint32_t gg = (uint32_t)(ch * KCG + g);
      // groups past the last one (partial last chunk; never computed) load
      // the last group again, so the scalar offset stays inside the column
      const int soff = w_group_soffset((int)gg, a.G, GS);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint32_t off = w_off[nb];
        if constexpr (S == 1) {
          const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(w_rsrc, off, soff, 0);
          d.w[g][nb][0] = q.x;
          d.w[g][nb][1] = q.y;
        } else {
#pragma unroll
          for (int h = 0; h < S / 2; ++h) {
            const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, off + 16 * h, soff, 0);
            d.w[g][nb][4 * h + 0] = q.x;
            d.w[g][nb][4 * h + 1] = q.y;
            d.w[g][nb][4 * h + 2] = q.z;
            d.w[g][nb][4 * h + 3] = q.w;
          }
        }
        if constexpr (!ZS_LDS && !ZSV) {
          d.z[g][nb] = (int)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(z_rsrc, zs_off[nb] + gg, 0, 0);
          d.s[g][nb] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(s_rsrc, (zs_off[nb] + gg) * 4u, 0, 0));
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
  const i32x4 magic4 = {kMagic, kMagic, kMagic, kMagic};

  // ---- one chunk of K ------------------------------------------------------
  // dd: position of the chunk in its zero/scale window (compile-time after unrolling)
  //
  // Fold without a convert: each group's MFMA chain starts from the integer
  // kMagic = 0x4B400000 instead of 0, so the int32 result M + P (|P| <= 2^22
  // for every group size here) read as a float is exactly 12582912 + P. One
  // FMA then folds (12582912 + P) * s; the 12582912 * s of the groups is
  // summed per column (bias) and subtracted from the accumulators every
  // 4 * RD chunks and once after the loop (rebase), which keeps their
  // magnitude, and the extra rounding, small: with scales / 16 the bias of
  // 16 groups at group size 128 stays below ~2^18, an ulp of 2^-5 per fold,
  // far inside the bf16 rounding of the output. (Every 2 * RD chunks
  // measured 0.4-0.7 % slower on the 128-row prefill points: the rebase is
  // 64 subtractions.) Only symmetric tiles with an
  // LDS zero/scale block (SYMT) take this path; every other tile and kernel
  // keeps the plain int32 chain and a convert.
  bool tile_sym = false;   // decode tiles: every zero point of the tile is 8 (set in the prologue)
  float bias[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) bias[nb] = 0.f;
  auto rebase = [&]() __attribute__((always_inline)) {
    if constexpr (MG) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[mb][nb][r] -= bias[nb];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) bias[nb] = 0.f;
    }
  };
  auto compute = [&](int ch, const int8_t* xb, const WChunk& wc, const ZsWin& zw, int dd) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < KCG; ++g) {
      const int gg = ch * KCG + g;
      if (FAST || gg < a.G) {
        int zv[NB];
        float sv[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          if constexpr (ZS_LDS) {
            sv[nb] = s_scale[zs_lds[nb] + gg];
            if constexpr (XDEEP) {
              // decode tiles: a tile whose zero points are all 8 skips the read
              zv[nb] = 8;
              if (!tile_sym) zv[nb] = s_zero[zs_lds[nb] + gg];
            } else {
              zv[nb] = s_zero[zs_lds[nb] + gg];
            }
          } else if constexpr (ZSV) {
            zv[nb] = zero_of<KW>(zw.zr[nb], dd * KCG + g);
            sv[nb] = zw.s[dd * KCG + g][nb];
          } else {
            zv[nb] = wc.z[g][nb];
            sv[nb] = wc.s[g][nb];
          }
        }
        i32x4 bfr[NB][S];
        // Symmetric int4 (every zero point of the tile -- LDS block -- or of
        // this group in the wave is 8):
        // 16 * (u - 8) is the nibble with its top bit flipped, moved into the
        // high half of its byte, so unpacking takes 1.5 ops per int8 dword
        // instead of 3.5. The partials come out 16x larger and the scale is
        // used / 16; both factors are powers of two, so the product fed to
        // the fold is the same real number.
        bool sym = false;
        if constexpr (MG) {
          sym = true;   // scales already / 16
        } else {
          bool z8 = true;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) z8 = z8 && zv[nb] == 8;
          sym = __all(z8);
        }
        if (sym) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            if constexpr (!MG) sv[nb] *= 0.0625f;
#pragma unroll
            for (int s = 0; s < S; ++s) {
              // the top-bit flip (repacked weights store it) is applied after
              // the mask, so each half is a shift and one 3-input op
              const uint32_t flip = REPACKED ? 0u : 0x80808080u;
              const uint32_t t0 = wc.w[g][nb][2 * s];
              const uint32_t t1 = wc.w[g][nb][2 * s + 1];
              bfr[nb][s].x = (int)(((t0 << 4) & 0xF0F0F0F0u) ^ flip);
              bfr[nb][s].y = (int)((t0 & 0xF0F0F0F0u) ^ flip);
              bfr[nb][s].z = (int)(((t1 << 4) & 0xF0F0F0F0u) ^ flip);
              bfr[nb][s].w = (int)((t1 & 0xF0F0F0F0u) ^ flip);
            }
          }
        } else {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const ZeroFold zf = make_zero_fold(zv[nb]);
#pragma unroll
            for (int s = 0; s < S; ++s) {
              const uint32_t flip = REPACKED ? 0x88888888u : 0u;
              const uint32_t d0 = wc.w[g][nb][2 * s] ^ flip;
              const uint32_t d1 = wc.w[g][nb][2 * s + 1] ^ flip;
              bfr[nb][s].x = (int)fold_even(d0, zf);
              bfr[nb][s].y = (int)fold_odd(d0, zf);
              bfr[nb][s].z = (int)fold_even(d1, zf);
              bfr[nb][s].w = (int)fold_odd(d1, zf);
            }
          }
        }
        if constexpr (MG) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) bias[nb] = __builtin_fmaf(kMagicF, sv[nb], bias[nb]);
        }
        // Software-pipelined over 16-row blocks: the A fragments of block
        // mb+1 are read from LDS while block mb's MFMAs run, and block mb-1's
        // int32 partials are folded into the fp32 accumulators after block
        // mb's MFMAs are issued, so neither the LDS latency nor the MFMA
        // result latency sits on the issue path.
        const int8_t* xg = xb + jl * PITCH + g * GS + kb * 16;
        auto read_a = [&](int mb, i32x4 (&av)[S]) __attribute__((always_inline)) {
#pragma unroll
          for (int s = 0; s < S; ++s) av[s] = *reinterpret_cast<const i32x4*>(xg + mb * 16 * PITCH + 64 * s);
        };
        auto fold = [&](int mb, const i32x4 (&part)[NB]) __attribute__((always_inline)) {
          if constexpr (DEBUGP) {
            // the exact partial from the chain's value: minus the seed on
            // magic-seeded chains, / 16 (exact) after the symmetric unpack
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              const int col = c.col0 + nb * 16 + jl;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int dst = s_dst[mb * 16 + kb * 4 + r];
                int p = part[nb][r];
                if constexpr (MG) p -= kMagic;
                if (sym) p >>= 4;
                if (dst >= 0 && col < a.N) a.dbg[((int64_t)dst * a.N + col) * a.G + gg] = p;
              }
            }
          }
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float pf = MG ? __int_as_float(part[nb][r]) : (float)part[nb][r];
              acc[mb][nb][r] = __builtin_fmaf(pf, sv[nb], acc[mb][nb][r]);
            }
        };
        i32x4 av[2][S];
        i32x4 part[2][NB];
        read_a(0, av[0]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          if (mb + 1 < MB) read_a(mb + 1, av[(mb + 1) & 1]);
#pragma unroll
          for (int s = 0; s < S; ++s)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              const i32x4 cin = (s == 0) ? (MG ? magic4 : i32x4{0, 0, 0, 0}) : part[mb & 1][nb];
              part[mb & 1][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mb & 1][s], bfr[nb][s], cin, 0, 0, 0);
            }
          if (mb > 0) fold(mb - 1, part[(mb - 1) & 1]);
        }
        fold(MB - 1, part[(MB - 1) & 1]);
      }
    }
  };

  // ---- main loop: chunk c uses ring slot c % RD ----------------------------
  // 64/128-row tiles issue the next chunk's loads unconditionally, past the
  // end with the chunk index clamped to the last chunk (loaded again, never
  // used): no branch surrounds a load, so no join makes the compiler wait for
  // one (which serialized their prefetch). The 16/32-row tiles run a few
  // chunks per tile, where the extra chunk costs more than the join (measured
  // on the decode points), so they skip the loads past the end.
  constexpr bool CLAMP = BM >= 64;
  static_assert(CLAMP != XDEEP, "decode tiles run the deep ring, prefill tiles the clamped loop");
  const int last_chunk = c.nchunks - 1;
  const int last_win = (c.nchunks + ZW - 1) / ZW - 1;
  WChunk ring[RD];
  // zs_cur serves the current window; zs_next is loaded one window ahead and
  // copied in at each window start (after the activation wait, which has
  // covered its load: it was issued before those activations). Decode tiles
  // instead keep one window (= one chunk, see zs_window) per ring slot.
  ZsWin zs_cur, zs_next;
  ZsWin zs_ring[XDEEP && !ZS_LDS && ZSV ? RD : 1];
  float r_xs = 0.f, r_tw = 1.f;   // decode tiles: this thread's row factors, to LDS in the epilogue
  if constexpr (XDEEP) {
    // chunks 0 .. RD - 2 in flight before the loop: the weights (and zero
    // point / scale runs) first, right after the routing-row loads; then the
    // rows go to LDS -- that wait covers only the row loads, issued first --
    // and the row scales are requested (needed only by the epilogue); then,
    // after the barrier that publishes the rows, the activations
#pragma unroll
    for (int d = 0; d < RD - 1; ++d) {
      if (d < c.nchunks) {
        if constexpr (!ZS_LDS && ZSV) load_zs(d, zs_ring[d]);
        load_w(d, ring[d]);
      }
    }
    if constexpr (PRE) {
      init_x();
#pragma unroll
      for (int d = 0; d < RD - 1; ++d)
        if (d < c.nchunks) load_x(d, d);
    }
    if (tid < BM) {
      s_src[tid] = r_src;
      s_dst[tid] = r_dst;
      if (r_dst >= 0) row_scales<ROUTED, DEBUGP>(a, r_src, r_dst, r_xs, r_tw);
    }
    // the tile's zero points (loaded for its LDS block, before the weights)
    // all 8? Columns past N read zero: such a tile is not taken as symmetric.
    int zok = ZS_LDS ? 1 : 0;
    if constexpr (ZS_LDS) {
#pragma unroll
      for (int j = 0; j < ZU; ++j) {
        const u32x4 q = zq[j];
        if (tid + j * NT < z_units)
          zok &= (q.x == 0x08080808u) & (q.y == 0x08080808u) & (q.z == 0x08080808u) & (q.w == 0x08080808u);
      }
    }
    tile_sym = __syncthreads_and(zok) != 0;
    if constexpr (!PRE) {
      init_x();
#pragma unroll
      for (int d = 0; d < RD - 1; ++d)
        if (d < c.nchunks) load_x(d, d);
    }
  } else {
    if constexpr (!ZS_LDS && ZSV) load_zs(0, zs_next);
    load_x(0, 0);
#pragma unroll
    for (int d = 0; d < RD - 1; ++d) load_w(min(d, last_chunk), ring[d]);
    if constexpr (Hooks::kActive) hk->before_barrier();
  }
  if constexpr (ZS_LDS && !PZS) {
    // visible to all waves after the first barrier of the loop; a symmetric
    // tile stores its scales / 16 for the symmetric unpack (see compute)
#pragma unroll
    for (int j = 0; j < SU; ++j) {
      const int u = tid + j * NT;
      if (u < s_units) {
        u32x4 v = sq[j];
        if constexpr (MG) {
          v.x = __float_as_uint(__uint_as_float(v.x) * 0.0625f);
          v.y = __float_as_uint(__uint_as_float(v.y) * 0.0625f);
          v.z = __float_as_uint(__uint_as_float(v.z) * 0.0625f);
          v.w = __float_as_uint(__uint_as_float(v.w) * 0.0625f);
        }
        *reinterpret_cast<u32x4*>(s_scale + 4 * u) = v;
      }
    }
#pragma unroll
    for (int j = 0; j < ZU; ++j) {
      const int u = tid + j * NT;
      if (!MG && u < z_units) *reinterpret_cast<u32x4*>(s_zero + 16 * u) = zq[j];
    }
  }
  // STAGGER (full-height bodies of 8-wave 256-column tiles, with or without
  // a tail): half of the waves run the chunk
  // interval in the opposite order, so that the CU's load bursts and compute
  // phases overlap: early waves loads(c+1), compute(c), store A(c+1); late
  // waves compute(c), store A(c+1) (loaded one interval earlier), loads(c+2) --
  // into the weight slot compute(c) has just finished with. One barrier per
  // chunk for all waves, as in the plain loop. Waves are placed round-robin
  // (w and w + 4 share a SIMD); of the groupings measured, late = waves 2, 3,
  // 6, 7 (each SIMD's two waves in the same order, two SIMDs each way) was
  // fastest -- faster than the SIMD mates in opposite orders. A wave raises
  // its issue priority for its compute phase, so that a SIMD mate's loads and
  // staging fill the gaps rather than delay the MFMA chain (measured -0.75 %
  // over five interleaved runs).
  constexpr bool STAGGER = NW == 8 && BMX >= BM && CLAMP;
  if constexpr (STAGGER) {
    // one interval of chunk cc (ring parity d); LATE selects the order
    auto interval = [&](int cc, int d, auto late_tag) __attribute__((always_inline)) {
      constexpr bool LATE = decltype(late_tag)::value;
      if constexpr (!ZS_LDS && ZSV) {
        if (d % ZW == 0) {
          zs_cur = zs_next;
          load_zs(min(cc / ZW + 1, last_win), zs_next);
        }
      }
      if constexpr (LATE) {
        __builtin_amdgcn_s_setprio(1);
        compute(cc, s_x + (cc & 1) * BUF, ring[d], zs_cur, d % ZW);
        __builtin_amdgcn_s_setprio(0);
        store_x((cc + 1) & 1, 0);
        load_x(min(cc + 2, last_chunk), 0);
        load_w(min(cc + RD, last_chunk), ring[d]);
      } else {
        load_x(min(cc + 1, last_chunk), 0);
        load_w(min(cc + RD - 1, last_chunk), ring[(d + RD - 1) % RD]);
        __builtin_amdgcn_s_setprio(1);
        compute(cc, s_x + (cc & 1) * BUF, ring[d], zs_cur, d % ZW);
        __builtin_amdgcn_s_setprio(0);
        store_x((cc + 1) & 1, 0);
      }
      __syncthreads();
    };
    // Two separate loops (no join inside either, so no waits for loads
    // there). Each loop iteration runs both intervals unconditionally and an
    // odd last chunk runs after the loop: with the second interval under a
    // condition, the loop header had a predecessor that issued no loads after
    // the current weights, and the wait-count merge there made every other
    // compute phase wait for the loads issued just before the barrier.
    auto run_loop = [&](auto late_tag) __attribute__((always_inline)) {
      int ch = 0;
      for (; ch + RD <= c.nchunks; ch += RD) {
#pragma unroll
        for (int d = 0; d < RD; ++d) interval(ch + d, d, late_tag);
        if ((ch & (3 * RD)) == 3 * RD) rebase();   // every fourth ring turn (see rebase)
      }
      if (ch < c.nchunks) {
#pragma unroll
        for (int d = 0; d < RD; ++d)
          if (ch + d < c.nchunks) interval(ch + d, d, late_tag);
      }
      rebase();
    };
    if (((tid >> 6) >> 1) & 1) {
      // one more chunk in flight: A(1) in registers, W(RD - 1) in the ring
      store_x(0, 0);
      load_x(min(1, last_chunk), 0);
      load_w(min(RD - 1, last_chunk), ring[RD - 1]);
      __syncthreads();
      run_loop(std::true_type{});
    } else {
      store_x(0, 0);
      __syncthreads();
      run_loop(std::false_type{});
    }
  }
  if constexpr (XDEEP) {
    // Decode loop: chunk cc (ring slot cc % RD = d) is staged from the
    // registers its loads filled RD - 1 intervals earlier; after the barrier
    // chunk cc + RD - 1 is requested into the slot chunk cc - 1 has freed.
    // The main loop runs while every such request exists, so it holds no
    // conditional load (a join after one makes the wait-count merge assume
    // the fewest loads in flight); the last chunks follow in a guarded tail.
    auto step = [&](int cc, int d, bool load_next) __attribute__((always_inline)) {
      store_x(cc & 1, d);
      __syncthreads();
      const int nx = cc + RD - 1, slot = (d + RD - 1) % RD;
      if (load_next) {
        if constexpr (!ZS_LDS && ZSV) load_zs(nx, zs_ring[slot]);
        load_x(nx, slot);
        load_w(nx, ring[slot]);
      }
      compute(cc, s_x + (cc & 1) * BUF, ring[d], zs_ring[(!ZS_LDS && ZSV) ? d : 0], 0);
    };
    int ch = 0;
    for (; ch + 2 * RD - 1 <= c.nchunks; ch += RD) {
#pragma unroll
      for (int d = 0; d < RD; ++d) step(ch + d, d, true);
      rebase();
    }
    for (; ch < c.nchunks; ch += RD) {
#pragma unroll
      for (int d = 0; d < RD; ++d) {
        const int cc = ch + d;
        if (cc < c.nchunks) step(cc, d, cc + RD - 1 < c.nchunks);
      }
      rebase();
    }
  }
  if constexpr (!STAGGER && !XDEEP) {
    auto step = [&](int cc, int d) __attribute__((always_inline)) {
      store_x(cc & 1, 0);
      __syncthreads();
      if constexpr (!ZS_LDS && ZSV) {
        if (d % ZW == 0) {
          zs_cur = zs_next;
          load_zs(min(cc / ZW + 1, last_win), zs_next);
        }
      }
      load_x(min(cc + 1, last_chunk), 0);
      load_w(min(cc + RD - 1, last_chunk), ring[(d + RD - 1) % RD]);
      // the 8-wave kernel's half- and quarter-height bodies raise their
      // priority for the compute phase as the staggered loop does (-0.8 %
      // on DeepSeek-V3 up M=4096 over five interleaved runs); in the 4-wave
      // 64-row kernel it measured 1-3 % slower
      if constexpr (NW == 8) __builtin_amdgcn_s_setprio(1);
      compute(cc, s_x + (cc & 1) * BUF, ring[d], zs_cur, d % ZW);
      if constexpr (NW == 8) __builtin_amdgcn_s_setprio(0);
    };
    // whole ring turns without conditions (see the staggered loop), then the
    // remaining chunks
    int ch = 0;
    for (; ch + RD <= c.nchunks; ch += RD) {
#pragma unroll
      for (int d = 0; d < RD; ++d) step(ch + d, d);
      if ((ch & (3 * RD)) == 3 * RD) rebase();   // every fourth ring turn (see rebase)
    }
    if (!FAST && ch < c.nchunks) {
#pragma unroll
      for (int d = 0; d < RD; ++d)
        if (ch + d < c.nchunks) step(ch + d, d);
    }
    rebase();
  }

  if constexpr (Hooks::kActive) {
    hk->before_epilogue();
    // (read by the epilogue only, after its first barrier)
    const int r = opaque_tid();
    if (r < BMA) {
      s_xs[r] = hk->ep_xs;
      s_tw[r] = hk->ep_tw;
    }
  }
  // (the reference-layout debug export passes no output)
  if (!DEBUGP || a.out != nullptr) {
    if constexpr (XDEEP) {
      // the row factors requested in the prologue (s_xs / s_tw are not used
      // before the epilogue)
      if (tid < BM) {
        s_xs[tid] = r_xs;
        s_tw[tid] = r_tw;
      }
      __syncthreads();
    }
    // 128-column tiles: the finished tile goes through LDS (the activation
    // buffers are free now) so that every row leaves as 16-byte stores of
    // its 256 contiguous bytes -- 8 store instructions per wave instead of 64
    // two-byte ones (an MFMA lane holds four rows of one column). Row r's
    // 16-byte segment s sits at r * ROWB + 16 * (s ^ 2 ((r / 4) % 4)): the
    // four rows of one ds_write_b16 (r / 4 % 4 = the lane's K slot, the rows'
    // segment pairs XORed with 0, 2, 4, 6) hit 8 distinct segments, and a
    // ds_read_b128 half-wave reads one row's segments permuted. The XOR term
    // is the lane's own for every write, so each write's address is a lane
    // base plus an immediate (a term with the row's low bits cost ~4 VALU a
    // write).
    constexpr bool TILE_OUT = (BN == 128 || BN == 256) && BM >= 64;
    constexpr int SEG = BN / 8;          // 16-byte segments per tile row
    constexpr int ROWB = BN * 2;         // bytes per tile row
    bool stored = false;
    if constexpr (TILE_OUT) {
      if (a.vec_out) {
        uint8_t* tile = reinterpret_cast<uint8_t*>(s_x);
        __syncthreads();   // every wave has finished reading the activation buffers
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const int cl = c.col0 - c.tile_col0 + nb * 16 + jl;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = mb * 16 + kb * 4 + r;
              v[r] = acc[mb][nb][r] * s_xs[row];
              if constexpr (ROUTED) v[r] = v[r] * s_tw[row];
            }
            // rows r and r + 1 of the column converted as one pair
            const uint32_t pk[2] = {bf16x2_rne(v[0], v[1]), bf16x2_rne(v[2], v[3])};
            // this lane's rows kb * 4 + r of block mb: (row / 4) % 4 = kb
            uint8_t* const lb = tile + kb * 4 * ROWB + (((cl >> 3) ^ (kb << 1)) << 4) + ((cl & 7) << 1);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              *reinterpret_cast<uint16_t*>(lb + (mb * 16 + r) * ROWB) = (uint16_t)(pk[r >> 1] >> (16 * (r & 1)));
          }
        __syncthreads();
        if constexpr (Hooks::kActive) hk->before_stores();
        static_assert((BMX * SEG) % NT == 0, "output rounds");
#pragma unroll
        for (int i = 0; i < BMX * SEG / NT; ++i) {
          const int t = tid + i * NT;
          const int row = t / SEG, seg = t % SEG;
          const u32x4 v = *reinterpret_cast<const u32x4*>(tile + row * ROWB + ((seg ^ (((row >> 2) & 3) << 1)) << 4));
          const int dst = s_dst[row];
          const int col = c.tile_col0 + seg * 8;
          if (dst >= 0 && col < a.N) *reinterpret_cast<u32x4*>(a.out + (int64_t)dst * a.ldo + col) = v;
        }
        stored = true;
      }
    }
    if (!stored) {
      if constexpr (Hooks::kActive) {
        __syncthreads();   // the row factors just stored
        hk->before_stores();
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int col = c.col0 + nb * 16 + jl;
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
  } else if constexpr (Hooks::kActive) {
    hk->before_stores();
  }
}

// Routing rows of a 64/128-row tile, loaded ahead of their use: this
// thread's sorted_ids entry (routed tiles; row tid of the block, or of the
// tail for tid >= BM) and its share of the tile's [BN x G] zero-point block
// for the symmetric check (tiles with an LDS zero/scale block).
template <int ZCU, int SCU = 1>
struct RowsAhead {
  int sid;
  u32x4 zq[ZCU];
  u32x4 sq[SCU];   // persistent launches: the tile's scale block share
};

template <int BN, int NT, int ZSG>
__host__ __device__ constexpr int zero_check_units() {
  return ZSG > 0 ? (BN * ZSG / 16 + NT - 1) / NT : 1;
}

template <int BN, int NT, int ZSG>
__host__ __device__ constexpr int scale_units() {
  return ZSG > 0 ? (BN * ZSG / 4 + NT - 1) / NT : 1;
}

template <int BM, int BN, int NT, int ZSG, int TAIL, bool ROUTED, bool DEBUGP = false, int SCU = 1>
__device__ __forceinline__ void prefill_rows_issue(const GemmArgs& a, const TileCtx& c,
                                                   RowsAhead<zero_check_units<BN, NT, ZSG>(), SCU>& p) {
  constexpr int ZCU = zero_check_units<BN, NT, ZSG>();
  const int tid = opaque_tid();
  p.sid = -1;
  if constexpr (ROUTED) {
    if (tid < BM) p.sid = a.sorted_ids[c.blk * BM + tid];
    else if (tid < BM + TAIL && c.tail >= 0) p.sid = a.sorted_ids[c.tail * BM + (tid - BM)];
  }
  if constexpr (ZSG > 0) {
    const __amdgpu_buffer_rsrc_t zr = make_rsrc(a.wz + (int64_t)c.e * a.N * a.G, (uint32_t)(a.N * a.G));
    const int z_units = BN * a.G / 16;
#pragma unroll
    for (int j = 0; j < ZCU; ++j) {
      const int u = tid + j * NT;
      p.zq[j] = u32x4{0u, 0u, 0u, 0u};
      if (u < z_units) p.zq[j] = __builtin_amdgcn_raw_buffer_load_b128(zr, (uint32_t)(c.tile_col0 * a.G) + u * 16u, 0, 0);
    }
  }
}

// This thread's share of a tile's scale block, loaded ahead (persistent
// launches: during the previous tile's epilogue).
template <int BN, int NT, int ZSG, bool DEBUGP, int SCU>
__device__ __forceinline__ void prefill_scales_issue(const GemmArgs& a, const TileCtx& c,
                                                     RowsAhead<zero_check_units<BN, NT, ZSG>(), SCU>& p) {
  static_assert(SCU == scale_units<BN, NT, ZSG>(), "scale block share");
  const int tid = opaque_tid();
  // the reference-layout debug export passes no scales (read as zero)
  const __amdgpu_buffer_rsrc_t sr =
      (DEBUGP && a.ws == nullptr) ? make_rsrc(a.wz, 0u)
                                  : make_rsrc(a.ws + (int64_t)c.e * a.N * a.G, (uint32_t)(a.N * a.G) * 4u);
  const int s_units = BN * a.G / 4;
#pragma unroll
  for (int j = 0; j < SCU; ++j) {
    const int u = tid + j * NT;
    p.sq[j] = u32x4{0u, 0u, 0u, 0u};
    if (u < s_units)
      p.sq[j] = __builtin_amdgcn_raw_buffer_load_b128(sr, (uint32_t)(c.tile_col0 * a.G) * 4u + u * 16u, 0, 0);
  }
}

// This thread's row of the tile (src: activation row, dst: output row,
// -1 for padding) from its sorted_ids entry, and whether its share of the
// zero-point block is all 8 (columns past N read zero: not symmetric).
template <int BM, int BN, int NT, int ZSG, int TAIL, bool ROUTED, int SCU = 1>
__device__ __forceinline__ void prefill_rows_settle(const GemmArgs& a, const TileCtx& c,
                                                    const RowsAhead<zero_check_units<BN, NT, ZSG>(), SCU>& p, int& zok,
                                                    int& src, int& dst) {
  constexpr int ZCU = zero_check_units<BN, NT, ZSG>();
  const int tid = opaque_tid();
  zok = 1;
  if constexpr (ZSG > 0) {
    const int z_units = BN * a.G / 16;
#pragma unroll
    for (int j = 0; j < ZCU; ++j) {
      const u32x4 q = p.zq[j];
      if (tid + j * NT < z_units)
        zok &= (q.x == 0x08080808u) & (q.y == 0x08080808u) & (q.z == 0x08080808u) & (q.w == 0x08080808u);
    }
  }
  src = dst = -1;
  if (tid < BM + TAIL) {
    if constexpr (ROUTED) {
      if (p.sid >= 0 && p.sid < a.num_pairs) {
        src = p.sid / a.topk;
        dst = p.sid;
      }
    } else {
      if (tid < BM) row_source<BM, false>(a, c, tid, src, dst);
    }
  }
}

// The rows into LDS (s_src, s_dst; s_rows raised to the last row holding
// data, from zero) and this row's epilogue factors requested into xsv / twv.
template <int BM, int TAIL, bool ROUTED, bool DEBUGP>
__device__ __forceinline__ void prefill_rows_place(const GemmArgs& a, int src, int dst, int* s_src, int* s_dst,
                                                   int* s_rows, float& xsv, float& twv) {
  const int tid = opaque_tid();
  xsv = 0.f;
  twv = 1.f;
  // the last row holding data, per wave: one LDS atomic by lane 0 (a
  // per-thread atomicMax of divergent values compiles to a loop over the
  // wave's lanes)
  const uint64_t have = __ballot(tid < BM + TAIL && dst >= 0);
  if (tid < BM + TAIL) {
    if (dst >= 0) row_scales<ROUTED, DEBUGP>(a, src, dst, xsv, twv);
    s_src[tid] = src;
    s_dst[tid] = dst;
  }
  if (have != 0 && (tid & 63) == 0) atomicMax(s_rows, (tid & ~63) + 64 - __clzll(have));
}

// Body of a 64/128-row tile whose rows are in LDS (c.rows: rows holding
// data): the full-, half- or quarter-height body -- or, for a tile that
// takes the TAIL pairs of its expert's short last block (c.tail), the
// full-height body extended by TAIL rows; symmetric tiles (tsym) run the
// magic-number fold (SYMT).
template <int BM, int WN, int NW, int GS, int KCG, int RD, int ZSG, int RMODE, bool DEBUGP, bool FAST, bool ZSV,
          int TAIL, class Hooks = NoHooks>
__device__ __forceinline__ void prefill_run(const GemmArgs& a, const TileCtx& c, bool tsym, int8_t* s_x,
                                            float* s_scale, int8_t* s_zero, int* s_src, int* s_dst, float* s_xs,
                                            float* s_tw, Hooks* hk = nullptr) {
  constexpr int BMA = BM + TAIL;
  const int rows = c.rows;
  auto run = [&](auto symt_c) __attribute__((always_inline)) {
    constexpr bool SYMT = decltype(symt_c)::value;
    if constexpr (TAIL > 0) {
      if (rows > BM) {
        gemm_body<BMA, BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, SYMT, BMA, Hooks>(
            a, c, s_x, s_scale, s_zero, s_src, s_dst, s_xs, s_tw, hk);
        return;
      }
    }
    // tiles whose valid rows fit in the top quarter (8-wave 128-row tiles:
    // the second block of most DeepSeek-V3 experts) or half
    if constexpr (BM >= 128 && NW == 8) {
      if (rows <= BM / 4) {
        gemm_body<BM / 4, BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, SYMT, BMA, Hooks>(
            a, c, s_x, s_scale, s_zero, s_src, s_dst, s_xs, s_tw, hk);
        return;
      }
    }
    if constexpr (BM >= 64) {
      if (rows <= BM / 2) {
        gemm_body<BM / 2, BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, SYMT, BMA, Hooks>(
            a, c, s_x, s_scale, s_zero, s_src, s_dst, s_xs, s_tw, hk);
        return;
      }
    }
    gemm_body<BM, BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, SYMT, BMA, Hooks>(
        a, c, s_x, s_scale, s_zero, s_src, s_dst, s_xs, s_tw, hk);
  };
  if constexpr (ZSG > 0) {
    if (tsym) run(std::true_type{});
    else run(std::false_type{});
  } else {
    run(std::false_type{});
  }
}

// Entry of a 64/128-row tile of a plain launch (c: its block, expert and
// columns): routing rows and, with an LDS zero/scale block, the tile's
// symmetric check (loads issued together, checked at one barrier), then
// the body.
template <int BM, int WN, int NW, int GS, int KCG, int RD, int ZSG, int RMODE, bool DEBUGP, bool FAST, bool ZSV,
          int TAIL>
__device__ __forceinline__ void prefill_tile_impl(const GemmArgs& a, TileCtx c, int8_t* s_x, float* s_scale,
                                                  int8_t* s_zero, int* s_src, int* s_dst, float* s_xs,
                                                  float* s_tw) {
  constexpr int BN = NW * WN;
  constexpr int NT = NW * 64;
  constexpr bool ROUTED = RMODE != 0;
  const int tid = opaque_tid();
  __shared__ int s_rows;   // rows of the tile holding data
  if (tid == 0) s_rows = 0;
  __syncthreads();
  RowsAhead<zero_check_units<BN, NT, ZSG>()> p;
  prefill_rows_issue<BM, BN, NT, ZSG, TAIL, ROUTED>(a, c, p);
  int zok, src, dst;
  prefill_rows_settle<BM, BN, NT, ZSG, TAIL, ROUTED>(a, c, p, zok, src, dst);
  float xsv, twv;
  prefill_rows_place<BM, TAIL, ROUTED, DEBUGP>(a, src, dst, s_src, s_dst, &s_rows, xsv, twv);
  if (tid < BM + TAIL) {
    s_xs[tid] = xsv;
    s_tw[tid] = twv;
  }
  const bool tsym = ZSG > 0 ? block_and<NW>(zok != 0) : (__syncthreads(), false);
  c.rows = __builtin_amdgcn_readfirstlane(s_rows);
  prefill_run<BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, TAIL>(a, c, tsym, s_x, s_scale, s_zero, s_src,
                                                                          s_dst, s_xs, s_tw);
}

// Reference layout without a block table: the row blocks of expert e are
// ceil((r1 - r0) / BM) blocks of rows [r0, r1) = its offsets clamped to
// [0, M_total], laid out expert after expert -- the table
// csr_block_table_kernel writes, derived by each wave on its own. Lane l of
// chunk k holds expert 64 k + l: its clamped rows and the inclusive prefix
// of the block counts. Returns the block count (wave-uniform).
template <int BM>
__device__ __forceinline__ int csr_scan(const GemmArgs& a, int (&r0)[kCsrScanChunks], int (&r1)[kCsrScanChunks],
                                        int (&incl)[kCsrScanChunks]) {
  const int lane = threadIdx.x & 63;
  int lo[kCsrScanChunks], hi[kCsrScanChunks];
#pragma unroll
  for (int k = 0; k < kCsrScanChunks; ++k) {   // every load before the first use
    const int e = k * 64 + lane;
    lo[k] = hi[k] = 0;
    if (e < a.E) {
      lo[k] = a.offsets[e];
      hi[k] = a.offsets[e + 1];
    }
  }
  int carry = 0;
#pragma unroll
  for (int k = 0; k < kCsrScanChunks; ++k) {
    r0[k] = min(max(lo[k], 0), a.M_total);
    r1[k] = min(max(hi[k], 0), a.M_total);
    int v = r1[k] > r0[k] ? (r1[k] - r0[k] + BM - 1) / BM : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(v, d, 64);
      if (lane >= d) v += o;
    }
    incl[k] = carry + v;
    carry = __builtin_amdgcn_readlane(incl[k], 63);
  }
  return carry;
}

// Block b (< the count csr_scan returned) of that layout: its expert and
// rows [row0, row1). The expert is the first lane whose inclusive prefix
// exceeds b.
template <int BM>
__device__ __forceinline__ void csr_block(int b, const int (&r0)[kCsrScanChunks], const int (&r1)[kCsrScanChunks],
                                          const int (&incl)[kCsrScanChunks], int& e, int& row0, int& row1) {
  e = -1;
  row0 = row1 = 0;
#pragma unroll
  for (int k = 0; k < kCsrScanChunks; ++k) {
    const uint64_t m = __ballot(incl[k] > b);
    if (e < 0 && m != 0) {
      const int l = __builtin_ctzll(m);
      const int lo = __builtin_amdgcn_readlane(r0[k], l);
      const int hi = __builtin_amdgcn_readlane(r1[k], l);
      const int first = __builtin_amdgcn_readlane(incl[k], l) - (hi - lo + BM - 1) / BM;
      e = k * 64 + l;
      row0 = lo + (b - first) * BM;
      row1 = min(row0 + BM, hi);
    }
  }
}

// Inclusive sum / max over the workgroup's threads in thread order; total
// receives the whole workgroup's sum / max. Every thread calls it; s_tmp
// holds NW ints.
template <int NW>
__device__ __forceinline__ int block_scan_add(int v, int* s_tmp, int& total) {
  const int tid = opaque_tid(), lane = tid & 63, w = tid >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  if (lane == 63) s_tmp[w] = v;
  __syncthreads();
  int pre = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    const int y = s_tmp[k];
    if (k < w) pre += y;
    tot += y;
  }
  __syncthreads();
  total = __builtin_amdgcn_readfirstlane(tot);
  return pre + v;
}

template <int NW>
__device__ __forceinline__ int block_scan_max(int v, int* s_tmp, int& top) {
  const int tid = opaque_tid(), lane = tid & 63, w = tid >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v = max(v, o);
  }
  if (lane == 63) s_tmp[w] = v;
  __syncthreads();
  int pre = -1, tot = -1;
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    const int y = s_tmp[k];
    if (k < w) pre = max(pre, y);
    tot = max(tot, y);
  }
  __syncthreads();
  top = __builtin_amdgcn_readfirstlane(tot);
  return max(pre, v);
}

// Hooks of a persistent launch's tile body (see NoHooks).
template <class A, class B, class C>
struct TileHooks {
  static constexpr bool kActive = true;
  A& before;
  B& after;
  C& settle;
  float ep_xs, ep_tw;
  __device__ __forceinline__ void before_barrier() { before(); }
  __device__ __forceinline__ void before_epilogue() { after(); }
  __device__ __forceinline__ void before_stores() { settle(); }
};

// Row blocks the compact block table of a persistent launch holds in the LDS
// left beside a tile's buffers (6 bytes a block; at most 1024).
__host__ __device__ constexpr int compact_blocks(int BMA, int PITCH, int BN, int ZSG) {
  return (163840 - 512 - (2 * BMA * PITCH + (ZSG > 0 ? BN * ZSG * 5 : 20) + 16 * BMA)) / 6 / 64 * 64 > 1024
             ? 1024
             : (163840 - 512 - (2 * BMA * PITCH + (ZSG > 0 ? BN * ZSG * 5 : 20) + 16 * BMA)) / 6 / 64 * 64;
}

// Tile queues of persistent launches: one slot of 256 ints per stream (the
// per-XCD counters 16 ints apart, the finished-workgroup count at [128]).
// Zero at load time; every persistent launch leaves its slot zero.
constexpr int kQueueSlots = 64;
constexpr int kQueueInts = 256;
static __device__ __align__(256) int g_tile_queue[kQueueSlots * kQueueInts];

// ZSG > 0: zero points and scales come from an LDS copy of the tile's
// block; the host launches this only when G <= ZSG (see zs_block_fits).
//
// TAIL > 0 (routed 128-row tiles): an expert's last block that holds at most
// TAIL pairs is computed by the tile of the block before it, as TAIL extra
// rows of that tile, so its weights are streamed once for both; the short
// block's own tiles exit.
//
// PERSIST: one workgroup per CU (the host sizes the grid to the CU count)
// takes tiles from queues instead of one tile per workgroup. The tile list
// is split into 8 equal runs as for the plain grid, one per XCD; workgroup
// L (on XCD L % 8) draws the next tile of its XCD's run from that run's
// counter, so the XCD's CUs still work on adjacent tiles at the same time
// (the row blocks that share a column tile of one expert's weights meet in
// its L2), and once its own run is exhausted it draws from the other XCDs'
// runs. The counter for the next tile is incremented when the current tile
// starts, so its latency hides behind that tile. Compared with one
// workgroup per tile this saves the retire/launch gap between tiles on a
// CU and balances the XCDs, whose runs differ in work (tiles of short
// blocks taken as tails exit at once, and tile heights differ).
template <int BM, int WN, int NW, int GS, int KCG, int RD, int ZSG, int RMODE, bool DEBUGP, bool FAST, bool ZSV,
          int WAVES_PER_EU, int TAIL = 0, bool PERSIST = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WAVES_PER_EU)))
void w4a8_gemm_kernel(const GemmArgs a) {
  constexpr int BN = NW * WN;
  constexpr int PITCH = KCG * GS + 32;
  constexpr bool ZS_LDS = ZSG > 0;
  constexpr bool ROUTED = RMODE != 0;
  constexpr int BMA = BM + TAIL;   // rows staged: the block and a tail
  constexpr int CB = compact_blocks(BMA, PITCH, BN, ZSG);
  static_assert(BM % 16 == 0 && WN % 16 == 0 && GS % 64 == 0 && TAIL % 16 == 0, "tile shape");
  static_assert(TAIL == 0 || (ROUTED && BM >= 128 && NW == 8), "tails are taken by routed 8-wave 128-row tiles");
  static_assert(!PERSIST || (ROUTED && BM >= 64 && CB >= 64), "persistent launches run routed prefill tiles");

  __shared__ __attribute__((aligned(16))) int8_t s_x[2 * BMA * PITCH];
  __shared__ __attribute__((aligned(16))) float s_scale[ZS_LDS ? BN * ZSG : 4];
  __shared__ __attribute__((aligned(16))) int8_t s_zero[ZS_LDS ? BN * ZSG : 16];
  __shared__ int s_src[BMA];
  __shared__ int s_dst[BMA];
  __shared__ float s_xs[BMA];
  __shared__ float s_tw[BMA];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- tile list -----------------------------------------------------------
  // The grid covers the worst-case block count; the actual count is only
  // known here. The actual tiles are split evenly over the 8 XCDs
  // (workgroup L runs on XCD L % 8), each XCD taking a contiguous run of
  // the tile list.
  constexpr bool DECODE_SLOTS = !PERSIST && ROUTED && BM < 64;   // see the routed decode path below
  int nblocks = 0;
  int cs_r0[kCsrScanChunks], cs_r1[kCsrScanChunks], cs_incl[kCsrScanChunks];
  if constexpr (DECODE_SLOTS) {
    // (read there, after the tile's other loads are out)
  } else if constexpr (ROUTED) {
    // blocks past sorted_len / BM would read past sorted_ids / expert_ids
    // (a persistent launch's block table holds at most CB; the host bounds
    // the blocks of such launches by it)
    nblocks = __builtin_amdgcn_readfirstlane(min(a.num_post_pad[0] / BM, a.sorted_len / BM));
    if constexpr (PERSIST) nblocks = min(nblocks, CB);
  } else if (a.offsets != nullptr) {
    nblocks = min(csr_scan<BM>(a, cs_r0, cs_r1, cs_incl), a.max_blocks);
  } else {
    nblocks = a.blk_count[0];
  }
  // routed 64/128-row tiles may run in expert groups (the host decides)
  const bool egroups = ROUTED && BM >= 64 && a.egroups;
  const int span = a.n_tiles * a.R;
  const int tiles = egroups ? nblocks * a.n_tiles : (nblocks + a.R - 1) / a.R * span;
  const int per_xcd = (tiles + 7) >> 3;

  // Tile t of the list -> its context; false for a tile with no work.
  auto tile_ctx = [&](int t, TileCtx& c) __attribute__((always_inline)) -> bool {
    int b, nt, e, row0 = 0, row1 = 0;
    if (egroups) {
      if (!expert_group_tile(t, a.n_tiles, a.R, nblocks, a.expert_ids, a.E, b, nt, e)) return false;
    } else {
      const int chunk_id = t / span;
      const int rem = t - chunk_id * span;
      nt = rem / a.R;
      b = chunk_id * a.R + group_slot(rem - nt * a.R, nt, a.R);
      if (b >= nblocks) return false;
      if constexpr (ROUTED) {
        e = a.expert_ids[b];
        if (e >= a.E) return false;
      } else if (a.offsets != nullptr) {
        csr_block<BM>(b, cs_r0, cs_r1, cs_incl, e, row0, row1);
      } else {
        e = a.blk_expert[b];
        row0 = a.blk_row0[b];
        row1 = a.blk_row1[b];
      }
      if (e < 0) return false;
    }
    int tail = -1;
    if constexpr (TAIL > 0) {
      // block b is its expert's short last block, computed by block b - 1's tile
      if (b > 0 && a.expert_ids[b - 1] == e && short_block<BM, TAIL>(a, b)) return false;
      // this tile computes block b + 1 as its tail
      if (b + 1 < nblocks && a.expert_ids[b + 1] == e && short_block<BM, TAIL>(a, b + 1)) tail = b + 1;
    }
    // Wave-uniform by construction; said so explicitly because the tile
    // tables are read with vector loads once the kernel also writes global
    // memory through atomics, and a descriptor built from a value the
    // compiler takes as divergent costs a waterfall loop per buffer load.
    c.e = __builtin_amdgcn_readfirstlane(e);
    c.blk = __builtin_amdgcn_readfirstlane(b);
    c.tail = __builtin_amdgcn_readfirstlane(tail);
    c.row0 = __builtin_amdgcn_readfirstlane(row0);
    c.row1 = __builtin_amdgcn_readfirstlane(row1);
    c.tile_col0 = __builtin_amdgcn_readfirstlane(nt * BN);
    c.col0 = c.tile_col0 + wave * WN;
    c.nchunks = (a.G + KCG - 1) / KCG;
    c.rows = BM;
    return true;
  };
  auto run_tile = [&](const TileCtx& c) __attribute__((always_inline)) {
    if constexpr (BM < 64) {
      // Decode tiles request their first weight chunks before the routing
      // rows are read (the body loads those itself); they decide the
      // symmetric unpack per group and keep the plain int32 fold -- at these
      // sizes the weight stream, not the fold, sets the time.
      gemm_body<BM, BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, false>(a, c, s_x, s_scale, s_zero, s_src,
                                                                                s_dst, s_xs, s_tw);
    } else {
      prefill_tile_impl<BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, TAIL>(a, c, s_x, s_scale, s_zero, s_src,
                                                                                   s_dst, s_xs, s_tw);
    }
  };

  if constexpr (DECODE_SLOTS) {
    // Routed decode tiles: tile L of the host's worst-case list (tiles past
    // the actual count exit), so that the tile's block -- and with it its
    // expert, its slots and the block count -- is known without a load, and
    // those loads go out together: the weights then follow the expert and the
    // activations the slots one round trip later (instead of the block count,
    // the expert, the slots and, after a barrier, the activations one after
    // the other). Decode blocks share no weights, so the tile order needs no
    // L2 grouping. The reads stay below the routing buffers' extent
    // (max_blocks <= sorted_len / BM; the clamp keeps a grid past it in bounds).
    constexpr int XU = staging_units(BM, KCG, GS, NW);
    constexpr int UPR = KCG * GS / 16;
    const int L = blockIdx.x;
    const int bt = L / a.n_tiles, nt = L - bt * a.n_tiles;
    const int bs = min(bt, a.sorted_len / BM - 1);
    DecodeSlots<XU> pre;
    pre.own = tid < BM ? a.sorted_ids[bs * BM + tid] : -1;
#pragma unroll
    for (int j = 0; j < XU; ++j) pre.unit[j] = a.sorted_ids[bs * BM + row_of_group<UPR>((tid + j * NW * 64) / UPR)];
    const int np = a.num_post_pad[0];
    const int e = __builtin_amdgcn_readfirstlane(a.expert_ids[bs]);
    nblocks = __builtin_amdgcn_readfirstlane(min(np / BM, a.sorted_len / BM));
    if (bt >= nblocks || e < 0 || e >= a.E) return;
    TileCtx c;
    c.e = e;
    c.blk = bt;
    c.tail = -1;
    c.row0 = c.row1 = 0;
    c.tile_col0 = nt * BN;
    c.col0 = c.tile_col0 + wave * WN;
    c.nchunks = (a.G + KCG - 1) / KCG;
    c.rows = BM;
    gemm_body<BM, BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, false, BM, NoHooks, DecodeSlots<XU>>(
        a, c, s_x, s_scale, s_zero, s_src, s_dst, s_xs, s_tw, nullptr, &pre);
  } else if constexpr (!PERSIST) {
    const int L = blockIdx.x;
    if ((L >> 3) >= per_xcd) return;
    const int t = (L & 7) * per_xcd + (L >> 3);
    if (t >= tiles) return;
    TileCtx c;
    if (tile_ctx(t, c)) run_tile(c);
  } else {
    // ---- the launch's row blocks, compacted (LDS) -------------------------
    // Blocks taken as a tail by the block before them are left out, so every
    // index of the tile list [0, ncb * n_tiles) is a tile with work; per
    // compact block: its block (| 0x8000 when it takes the next block as its
    // tail), its expert, and the compact index of the first block of its
    // expert's run (a run: consecutive blocks of one expert).
    constexpr int NT = NW * 64;
    __shared__ uint16_t s_cb_blk[CB], s_cb_e[CB], s_cb_rs[CB];
    __shared__ int s_scan[NW];
    int ncb = 0;
    for (int b0 = 0; b0 < nblocks; b0 += NT) {
      const int b = b0 + tid;
      int e = -1, keep = 0, first = 0, takes = 0;
      if (b < nblocks) {
        e = a.expert_ids[b];
        const int ep = b > 0 ? a.expert_ids[b - 1] : -1;
        keep = e >= 0 && e < a.E;
        first = ep != e;
        if constexpr (TAIL > 0) {
          const int en = b + 1 < nblocks ? a.expert_ids[b + 1] : -1;
          if (!first && short_block<BM, TAIL>(a, b)) keep = 0;
          takes = en == e && short_block<BM, TAIL>(a, b + 1);
        }
      }
      int total;
      const int pos = ncb + block_scan_add<NW>(keep, s_scan, total) - keep;
      if (keep) {
        s_cb_blk[pos] = (uint16_t)(b | (takes ? 0x8000 : 0));
        s_cb_e[pos] = (uint16_t)e;
        s_cb_rs[pos] = (uint16_t)(first ? pos : 0xffff);   // run starts; filled in below
      }
      ncb += total;
    }
    __syncthreads();
    for (int c0 = 0, carry = -1; c0 < ncb; c0 += NT) {
      const int cb = c0 + tid;
      const int v = cb < ncb && s_cb_rs[cb] != 0xffff ? cb : -1;
      int top;
      const int rs = max(block_scan_max<NW>(v, s_scan, top), carry);
      __syncthreads();   // every read of this range's run starts is done
      if (cb < ncb) s_cb_rs[cb] = (uint16_t)rs;
      carry = max(carry, top);
    }
    __syncthreads();
    const int ntiles = ncb * a.n_tiles;
    const int pxcd = (ntiles + 7) >> 3;
    // tile t -> context, from the compact table: t / n_tiles lies in the
    // group of its expert's run (groups of R compact blocks from the run's
    // first), whose tiles take the column tiles in turn, its blocks innermost
    // in the rotated order of group_slot
    auto tile_cb = [&](int t, TileCtx& c) __attribute__((always_inline)) {
      const int R = a.R;
      const int cb = t / a.n_tiles;
      const int rs = s_cb_rs[cb];
      const int g0 = rs + (cb - rs) / R * R;
      int gs = 1;
      while (gs < R && g0 + gs < ncb && s_cb_rs[g0 + gs] == rs) ++gs;
      const int local = t - g0 * a.n_tiles;
      const int nt = local / gs;
      const int k = g0 + group_slot(local - nt * gs, nt, gs);
      const int bi = __builtin_amdgcn_readfirstlane((int)s_cb_blk[k]);
      c.blk = bi & 0x7fff;
      c.tail = (bi & 0x8000) ? c.blk + 1 : -1;
      c.e = __builtin_amdgcn_readfirstlane((int)s_cb_e[k]);
      c.row0 = c.row1 = 0;
      c.tile_col0 = __builtin_amdgcn_readfirstlane(nt * BN);
      c.col0 = c.tile_col0 + wave * WN;
      c.nchunks = (a.G + KCG - 1) / KCG;
      c.rows = BM;
    };

    // ---- tile queues ----------------------------------------------------
    int* const q = a.queue;
    const int x = blockIdx.x & 7;
    // thread 0: the tile of index i drawn from XCD x's counter, or, with
    // that run exhausted, one drawn from another XCD's run; -1 when every
    // run is exhausted
    auto resolve = [&](int i) __attribute__((always_inline)) -> int {
      const int t0 = x * pxcd;
      if (i < pxcd && t0 + i < ntiles) return t0 + i;
      for (int k = 1; k < 8; ++k) {
        const int y = (x + k) & 7;
        const int u0 = y * pxcd, u1 = min(u0 + pxcd, ntiles);
        if (u0 >= u1) continue;
        const int j = __hip_atomic_fetch_add(q + 16 * y, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (u0 + j < u1) return u0 + j;
      }
      return -1;
    };
    // (the counter's address passes through a VGPR: with an address known to
    // be uniform the compiler's atomic optimizer rewrites the add into a
    // wave-aggregated one whose result it consumes at once, which waits for
    // every outstanding load and store -- the previous tile's output stores)
    auto draw = [&]() __attribute__((always_inline)) {
      __attribute__((address_space(1))) int* qx = (__attribute__((address_space(1))) int*)(q + 16 * x);
      asm volatile("" : "+v"(qx));
      return __hip_atomic_fetch_add(qx, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    // ---- tile loop ----------------------------------------------------------
    // Tile i runs with the next tile's work folded in: its index (requested
    // when tile i starts) is resolved once tile i's first loads are out;
    // when tile i's K loop is done every wave decodes it and requests its
    // routing rows and zero points, which arrive during tile i's epilogue.
    // Then they go to LDS, and the next tile's row factors are requested,
    // to be stored just before its own epilogue.
    constexpr int ZCU = zero_check_units<BN, NT, ZSG>();
    __shared__ int s_next[2];
    __shared__ int s_rows[2];
    __shared__ int s_nsym[2];   // nonzero: a zero point of the tile is not 8
    if (tid == 0) {
      s_next[0] = resolve(draw());
      s_rows[0] = 0;
      s_nsym[0] = 0;
    }
    __syncthreads();
    int t = __builtin_amdgcn_readfirstlane(s_next[0]);
    if (t >= 0) {
      TileCtx c, cn;
      // the next tile's rows and zero/scale block in flight (the first
      // tile's before the loop)
      constexpr int SCU = scale_units<BN, NT, ZSG>();
      RowsAhead<ZCU, SCU> p;
      tile_cb(t, c);
      prefill_rows_issue<BM, BN, NT, ZSG, TAIL, ROUTED, DEBUGP, SCU>(a, c, p);
      if constexpr (ZSG > 0) prefill_scales_issue<BN, NT, ZSG, DEBUGP, SCU>(a, c, p);
      int zok, src, dst;   // this tile's row and symmetric check, settled
      prefill_rows_settle<BM, BN, NT, ZSG, TAIL, ROUTED, SCU>(a, c, p, zok, src, dst);
      if (!zok) s_nsym[0] = 1;   // (published with the rows below)
      for (int it = 0;; ++it) {
        const int par = it & 1;
        int pend = 0;
        if (tid == 0) pend = draw();
        float xsv, twv;
        prefill_rows_place<BM, TAIL, ROUTED, DEBUGP>(a, src, dst, s_src, s_dst, &s_rows[par], xsv, twv);
        // one barrier publishes the rows, the row count and the symmetric
        // flag (raised by the previous tile's epilogue, see settle)
        __syncthreads();
        const bool tsym = ZSG > 0 && __builtin_amdgcn_readfirstlane(s_nsym[par]) == 0;
        c.rows = __builtin_amdgcn_readfirstlane(s_rows[par]);
        if constexpr (ZSG > 0) {
          // the tile's zero/scale block (loaded during the previous tile's
          // epilogue) into LDS -- free since the barrier that ended that tile;
          // visible to the body after its first barrier. A symmetric tile
          // stores its scales / 16 and no zero points (see gemm_body).
          const int s_units = BN * a.G / 4, z_units = BN * a.G / 16;
#pragma unroll
          for (int j = 0; j < SCU; ++j) {
            const int u = tid + j * NT;
            if (u < s_units) {
              u32x4 v = p.sq[j];
              if (tsym) {
                v.x = __float_as_uint(__uint_as_float(v.x) * 0.0625f);
                v.y = __float_as_uint(__uint_as_float(v.y) * 0.0625f);
                v.z = __float_as_uint(__uint_as_float(v.z) * 0.0625f);
                v.w = __float_as_uint(__uint_as_float(v.w) * 0.0625f);
              }
              *reinterpret_cast<u32x4*>(s_scale + 4 * u) = v;
            }
          }
#pragma unroll
          for (int j = 0; j < ZCU; ++j) {
            const int u = tid + j * NT;
            if (!tsym && u < z_units) *reinterpret_cast<u32x4*>(s_zero + 16 * u) = p.zq[j];
          }
        }
        int tn = -1;
        auto before = [&]() __attribute__((always_inline)) {
          if (tid == 0) {
            s_next[par ^ 1] = resolve(pend);
            s_rows[par ^ 1] = 0;
            s_nsym[par ^ 1] = 0;
          }
        };
        auto after = [&]() __attribute__((always_inline)) {   // (s_next: written before the K loop's barriers)
          tn = __builtin_amdgcn_readfirstlane(s_next[par ^ 1]);
          if (tn >= 0) {
            tile_cb(tn, cn);
            prefill_rows_issue<BM, BN, NT, ZSG, TAIL, ROUTED, DEBUGP, SCU>(a, cn, p);
          } else {
            // (defined on both paths, so that nothing of the previous tile's
            // loads has to stay live through this tile's K loop)
            p.sid = -1;
#pragma unroll
            for (int j = 0; j < ZCU; ++j) p.zq[j] = u32x4{0u, 0u, 0u, 0u};
          }
        };
        auto settle = [&]() __attribute__((always_inline)) {
          if (tn >= 0) {
            prefill_rows_settle<BM, BN, NT, ZSG, TAIL, ROUTED, SCU>(a, cn, p, zok, src, dst);
            if (!zok) s_nsym[par ^ 1] = 1;   // (reset in before; read after the tile's last barrier)
            // (the scale loads go out here, after the accumulators have left
            // their registers, rather than with the rows before the epilogue)
            if constexpr (ZSG > 0) prefill_scales_issue<BN, NT, ZSG, DEBUGP, SCU>(a, cn, p);
          } else {
            zok = 1;
            src = dst = -1;
#pragma unroll
            for (int j = 0; j < SCU; ++j) p.sq[j] = u32x4{0u, 0u, 0u, 0u};
          }
        };
        TileHooks<decltype(before), decltype(after), decltype(settle)> hk{before, after, settle, xsv, twv};
        prefill_run<BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, TAIL, decltype(hk)>(
            a, c, tsym, s_x, s_scale, s_zero, s_src, s_dst, s_xs, s_tw, &hk);
        __syncthreads();   // every wave is done with the tile's LDS
        if (tn < 0) break;
        c = cn;
      }
    }
    // the launch's last workgroup leaves the queues zero for the next launch
    // on this slot (every workgroup has drawn its last index by now)
    if (tid == 0) {
      const int done = __hip_atomic_fetch_add(q + 128, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      if (done == (int)gridDim.x - 1) {
#pragma unroll
        for (int y = 0; y < 8; ++y) __hip_atomic_store(q + 16 * y, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(q + 128, 0, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
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

// The tile's [BN x G] zero-point/scale block can be copied to an LDS array of
// BN * ZSG entries in whole 16-byte units from 16-byte-aligned addresses.
static bool zs_block_fits(const GemmArgs& a, int BN, int ZSG) {
  return ZSG > 0 && a.G <= ZSG && (BN * a.G) % 16 == 0 && (a.N * a.G) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(a.wz) % 16 == 0 && (a.ws == nullptr || reinterpret_cast<uintptr_t>(a.ws) % 16 == 0);
}

// Persistent launches: the device's CU count and this stream's tile-queue
// slot (its device address in this file's copy of g_tile_queue). Streams
// take slots in order of first use; with more than kQueueSlots streams
// slots are shared, and launches on streams sharing a slot must not run at
// the same time. A graph captured from a stream keeps that stream's slot.
static hipError_t persistent_setup(hipStream_t s, int* ncu, int** slot) {
  constexpr int kDevices = 64;
  static std::mutex mu;
  static int* base[kDevices] = {};
  static int cus[kDevices] = {};
  static int slot_dev[kQueueSlots];
  static hipStream_t slot_stream[kQueueSlots];
  static int n_slots = 0;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (base[dev] == nullptr) {
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_tile_queue));
    if (e != hipSuccess) return e;
    if (p == nullptr || n <= 0) return hipErrorInvalidValue;
    cus[dev] = n;
    base[dev] = static_cast<int*>(p);
  }
  int k = 0;
  while (k < n_slots && k < kQueueSlots && !(slot_dev[k] == dev && slot_stream[k] == s)) ++k;
  if (k == n_slots || k == kQueueSlots) {
    k = n_slots % kQueueSlots;
    slot_dev[k] = dev;
    slot_stream[k] = s;
    ++n_slots;
  }
  *ncu = cus[dev];
  *slot = base[dev] + k * kQueueInts;
  return hipSuccess;
}

template <int BM, int WN, int NW, int GS, int KCG, int RD, int ZSG, int RMODE, bool DEBUGP, int WPE, int TAIL = 0,
          bool PERSIST = false>
static hipError_t launch_one(GemmArgs a, int max_blocks, int R, hipStream_t s) {
  set_grid(a, max_blocks, NW * WN, R);
  // a column's zero points / scales of one window can be read as one aligned
  // run when G is a multiple of the window's groups and both tensors are
  // 16-byte aligned
  a.zs_vec = (a.G % (KCG * zs_window(KCG, RD, BM)) == 0) && (reinterpret_cast<uintptr_t>(a.wz) % 16 == 0) &&
             (reinterpret_cast<uintptr_t>(a.ws) % 16 == 0);
  // output rows can be written in 16-byte pieces
  a.vec_out = (a.N % 8 == 0) && (a.ldo % 8 == 0) && (reinterpret_cast<uintptr_t>(a.out) % 16 == 0);
  // Expert groups pay a short search per tile; they pay off when an expert's
  // weights outgrow one XCD's 4 MB L2 (below that the weights stay cached
  // across row blocks anyway). Groups hold up to 4 blocks (set_grid has
  // sized the grid for any grouping). Measured on MI355X: with 128-row tiles
  // 4 beat 2, 8 and 16 on the skewed DeepSeek-V3 point; with 64-row tiles 4
  // beat 2 by 2.5 % on DeepSeek-V3 down M=4096 (up to 3 blocks an expert).
  a.egroups = RMODE != 0 && BM >= 64 && (int64_t)a.N * (a.K / 2) > (int64_t)4 << 20;
  if (a.egroups) a.R = 4;
  if (a.total_tiles == 0) return hipSuccess;
  // the guard-free body needs whole chunks, a chunk count divisible by the
  // unroll, and (without the LDS zero/scale block) aligned vector runs
  constexpr bool CAN_FAST = BM <= 32;
  constexpr bool RUNS = ZSG == 0;   // vector zero/scale runs apply
  dim3 grid(8 * a.per_xcd), block(NW * 64);
  // Persistent launches pay off from about 8 tiles a CU (worst-case count;
  // measured on MI355X: DeepSeek-V3 up/gate M = 4096, ~32 a CU, 1379 ->
  // 1330 us; Qwen3 M = 2048, ~6 a CU, 108 -> 118 us).
  if constexpr (PERSIST) {
    int ncu = 0;
    const hipError_t e = persistent_setup(s, &ncu, &a.queue);
    if (e != hipSuccess) return e;
    // (the compact block table needs the expert-grouped tile order and
    // room for every block)
    if (a.egroups && max_blocks <= compact_blocks(BM + TAIL, KCG * GS + 32, NW * WN, ZSG) &&
        a.total_tiles >= 8 * ncu) {
      // one workgroup per CU (the tile's LDS allows no second one)
      grid = dim3(ncu);
      if (RUNS && a.zs_vec)
        hipLaunchKernelGGL((w4a8_gemm_kernel<BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, false, RUNS, WPE, TAIL, true>),
                           grid, block, 0, s, a);
      else
        hipLaunchKernelGGL(
            (w4a8_gemm_kernel<BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, false, false, WPE, TAIL, true>), grid,
            block, 0, s, a);
      return hipGetLastError();
    }
  }
  {
    a.queue = nullptr;
    if (CAN_FAST && a.G % (KCG * RD) == 0 && (ZSG > 0 || a.zs_vec))
      hipLaunchKernelGGL((w4a8_gemm_kernel<BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, CAN_FAST, RUNS, WPE, TAIL>),
                         grid, block, 0, s, a);
    else if (RUNS && a.zs_vec)
      hipLaunchKernelGGL((w4a8_gemm_kernel<BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, false, RUNS, WPE, TAIL>), grid,
                         block, 0, s, a);
    else
      hipLaunchKernelGGL((w4a8_gemm_kernel<BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, false, false, WPE, TAIL>), grid,
                         block, 0, s, a);
  }
  return hipGetLastError();
}

// Row-block size -> tile body; instantiated per row source by the gemm_*.hip
// files (declared in mw4a8_internal.h).
template <int GS, int RMODE, bool DEBUGP>
hipError_t dispatch_bm(GemmArgs a, const TileConfig& c, int max_blocks, hipStream_t s) {
  constexpr int K512 = 512 / GS > 0 ? 512 / GS : 1;     // groups per 512 bytes of K
  constexpr int K256 = 256 / GS > 0 ? 256 / GS : 1;
  switch (c.BM) {
    // Decode tiles: 512-byte K chunks (4 groups at group size 128), two in
    // flight per wave, at least two waves per SIMD: measured best or within 2 %
    // on every decode point (M = 1 to 64 of the DeepSeek-V3, Mixtral and Qwen3
    // shapes). The two-wave floor also caps every variant at 256 registers
    // (with a one-wave hint the group-size-64 bodies took 380 and ran one
    // wave per SIMD).
    case 16:
      if (zs_block_fits(a, 64, 64)) return launch_one<16, 16, 4, GS, K512, 2, 64, RMODE, DEBUGP, 2>(a, max_blocks, c.R, s);
      return launch_one<16, 16, 4, GS, K512, 2, 0, RMODE, DEBUGP, 2>(a, max_blocks, c.R, s);
    case 32:
      // (256-byte chunks without the LDS zero/scale block: the 512-byte one
      // spilled at group size 64)
      if (zs_block_fits(a, 64, 64)) return launch_one<32, 16, 4, GS, K512, 2, 64, RMODE, DEBUGP, 2>(a, max_blocks, c.R, s);
      return launch_one<32, 16, 4, GS, K256, 2, 0, RMODE, DEBUGP, 2>(a, max_blocks, c.R, s);
    // three waves per SIMD fit the gs = 128 body without spills; the others keep two
    case 64:
      // G <= 16 (K <= 2048 at group size 128): the tile's [128 x G] zero/scale
      // block in LDS (10 KB; three workgroups per CU still fit)
      if (zs_block_fits(a, 128, 16))
        return launch_one<64, 32, 4, GS, K256, 2, 16, RMODE, DEBUGP, GS == 128 ? 3 : 2>(a, max_blocks, c.R, s);
      return launch_one<64, 32, 4, GS, K256, 2, 0, RMODE, DEBUGP, GS == 128 ? 3 : 2>(a, max_blocks, c.R, s);
    case 128:
      // group sizes 128 and 256: 8 waves x 32 columns, staggered (see
      // STAGGER; the 4-wave 256-row... body spilled at group size 256)
      if constexpr (GS >= 128) {
        // the tile's whole [256 x G] zero-point/scale block in LDS when G <= 64
        // (80 KB beside the 72 KB of activation buffers: one tile per CU).
        // Routed, group size 128, G <= 56: a block of <= 16 pairs (an
        // expert's short last block) rides on the tile before it as 16 extra
        // rows (81 KB of activation buffers beside a 70 KB zero/scale block;
        // at group size 256 that body spilled). DeepSeek-V3 up/gate M = 4096:
        // 1534 -> 1425 us, every expert at 144 pairs 1782 -> 1443 us.
        if constexpr (RMODE != 0 && GS == 128) {
          if (zs_block_fits(a, 256, 56))
            return launch_one<128, 32, 8, GS, K256, 2, 56, RMODE, DEBUGP, 2, 16, true>(a, max_blocks, c.R, s);
        }
        if (zs_block_fits(a, 256, 64))
          return launch_one<128, 32, 8, GS, K256, 2, 64, RMODE, DEBUGP, 2, 0, RMODE != 0 && GS == 128>(a, max_blocks,
                                                                                                   c.R, s);
        return launch_one<128, 32, 8, GS, K256, 2, 0, RMODE, DEBUGP, 2, 0, RMODE != 0 && GS == 128>(a, max_blocks, c.R,
                                                                                                  s);
      } else
        return launch_one<128, 32, 4, GS, K256, 2, 0, RMODE, DEBUGP, 2>(a, max_blocks, c.R, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mw4a8
