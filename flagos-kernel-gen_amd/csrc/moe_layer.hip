// Kernels around the grouped GEMM that complete a W4A8 MoE layer:
//
//   quant_rows      bf16 activations -> per-token int8 + fp32 scale (the
//                   producer of the GEMM's x_q / x_scale)
//   router_topk     router logits -> top-k expert ids + routing weights
//   silu_mul_quant  up/gate GEMM output [gate | up] -> int8 silu(gate)*up +
//                   per-row scale (the down GEMM's activations); the math of
//                   the forward half of reference docs/Task3.md:103-110
//   combine_topk    per-pair down-projection rows -> per-token sum
//
// All four are HBM-bound streaming kernels. Rows are handled by one
// workgroup (quant kernels) or one wave (router) so that reductions stay on
// chip; vector accesses move 16 bytes per lane.
#include "mw4a8_internal.h"
#include "mw4a8_pack.h"

namespace mw4a8 {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace {

constexpr int kRowThreads = 256;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// 8 bf16 values packed in a 16-byte vector -> fp32
__device__ __forceinline__ void unpack8(const u32x4 v, float (&f)[8]) {
  f[0] = __uint_as_float(v.x << 16);
  f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16);
  f[3] = __uint_as_float(v.y & 0xffff0000u);
  f[4] = __uint_as_float(v.z << 16);
  f[5] = __uint_as_float(v.z & 0xffff0000u);
  f[6] = __uint_as_float(v.w << 16);
  f[7] = __uint_as_float(v.w & 0xffff0000u);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// max over the workgroup (kRowThreads threads); every thread gets the result
__device__ __forceinline__ float block_max(float v, float* s_red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();   // s_red may still be read by a previous call
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  float m = s_red[0];
#pragma unroll
  for (int w = 1; w < kRowThreads / 64; ++w) m = fmaxf(m, s_red[w]);
  return m;
}

// Per-token symmetric int8: scale = max(amax, 1e-12) / 127,
// q = clamp(round_half_even(v / scale), -127, 127), bit-identical to the
// same float32 steps on the CPU (IEEE scale division; rint_div below).
__device__ __forceinline__ float row_scale(float amax) { return fmaxf(amax, 1e-12f) / 127.0f; }

// rintf(a / s) for |a / s| <= 128 without dividing in the common case, and
// bit-identical to it: t = a * inv (inv = 1 / s rounded) is within 2e-5 of
// the rounded quotient (two roundings of relative size 2^-24 at |t| <= 128,
// plus the quotient's own half ulp), and t - floor(t) is exact, so when t is
// at least 1e-4 from a half-integer both round to the same integer. Lanes
// closer than that (about 2 in 10^4) take the IEEE division. NaN and inf
// inputs fail the test and give what the division gives.
__device__ __forceinline__ float rint_div(float a, float s, float inv) {
  const float t = a * inv;
  if (fabsf((t - floorf(t)) - 0.5f) < 1e-4f) return rintf(a / s);
  return rintf(t);
}

__device__ __forceinline__ uint32_t quant4(float a, float b, float c, float d, float scale, float inv) {
  const int qa = (int)fminf(fmaxf(rint_div(a, scale, inv), -127.f), 127.f);
  const int qb = (int)fminf(fmaxf(rint_div(b, scale, inv), -127.f), 127.f);
  const int qc = (int)fminf(fmaxf(rint_div(c, scale, inv), -127.f), 127.f);
  const int qd = (int)fminf(fmaxf(rint_div(d, scale, inv), -127.f), 127.f);
  return (uint32_t)(qa & 0xff) | ((uint32_t)(qb & 0xff) << 8) | ((uint32_t)(qc & 0xff) << 16) |
         ((uint32_t)(qd & 0xff) << 24);
}

// One workgroup per row; K % 8 == 0, rows 16-byte aligned (checked on the
// host). CH > 0: the row (at most CH 8-element chunks per thread) is read
// once and kept in registers between the max and the quantization; CH == 0
// reads it twice (any K).
template <int CH>
__global__ __launch_bounds__(kRowThreads) void quant_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                 int K, int8_t* __restrict__ q, int64_t ldq,
                                                                 float* __restrict__ scale) {
  __shared__ float s_red[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  int8_t* qr = q + row * ldq;
  float amax = 0.f;
  if constexpr (CH > 0) {
    u32x4 v[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = (threadIdx.x + j * kRowThreads) * 8;
      v[j] = c < K ? *reinterpret_cast<const u32x4*>(xr + c) : u32x4{0, 0, 0, 0};
      float f[8];
      unpack8(v[j], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    }
    const float s = row_scale(block_max(amax, s_red));
    const float inv = 1.0f / s;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = (threadIdx.x + j * kRowThreads) * 8;
      if (c < K) {
        float f[8];
        unpack8(v[j], f);
        u32x2 o;
        o.x = quant4(f[0], f[1], f[2], f[3], s, inv);
        o.y = quant4(f[4], f[5], f[6], f[7], s, inv);
        *reinterpret_cast<u32x2*>(qr + c) = o;
      }
    }
    if (threadIdx.x == 0) scale[row] = s;
  } else {
    for (int c = threadIdx.x * 8; c < K; c += kRowThreads * 8) {
      float f[8];
      unpack8(*reinterpret_cast<const u32x4*>(xr + c), f);
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    }
    const float s = row_scale(block_max(amax, s_red));
    const float inv = 1.0f / s;
    for (int c = threadIdx.x * 8; c < K; c += kRowThreads * 8) {
      float f[8];
      unpack8(*reinterpret_cast<const u32x4*>(xr + c), f);
      u32x2 o;
      o.x = quant4(f[0], f[1], f[2], f[3], s, inv);
      o.y = quant4(f[4], f[5], f[6], f[7], s, inv);
      *reinterpret_cast<u32x2*>(qr + c) = o;
    }
    if (threadIdx.x == 0) scale[row] = s;
  }
}

// y = silu(gate) * up in fp32 as sigmoid = 1 / (1 + exp(-g)), silu = g *
// sigmoid, y = silu * up (reference docs/Task3.md:103-110 order).
// exp and the reciprocal are the hardware's (v_exp_f32 of -g * log2(e),
// v_rcp_f32): about 1e-6 relative for |g| <= 16, against the ~10 VALU ops
// of a correctly rounded expf that made this kernel ALU-bound; exp overflow
// gives rcp(inf) = 0, as the division does.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-g));
  return (g * sg) * u;
}

// One workgroup per row of h = [gate (I) | up (I)] bf16; I % 8 == 0. CH as
// in quant_rows_kernel (the products y are kept in registers).
template <int CH>
__global__ __launch_bounds__(kRowThreads) void silu_mul_quant_kernel(const uint16_t* __restrict__ h,
                                                                     int64_t ldh, int I, int8_t* __restrict__ q,
                                                                     int64_t ldq, float* __restrict__ scale) {
  __shared__ float s_red[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* hr = h + row * ldh;
  float amax = 0.f;
  if constexpr (CH > 0) {
    float y[CH][8];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = (threadIdx.x + j * kRowThreads) * 8;
      const bool ok = c < I;
      const u32x4 gv = ok ? *reinterpret_cast<const u32x4*>(hr + c) : u32x4{0, 0, 0, 0};
      const u32x4 uv = ok ? *reinterpret_cast<const u32x4*>(hr + I + c) : u32x4{0, 0, 0, 0};
      float g[8], u[8];
      unpack8(gv, g);
      unpack8(uv, u);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y[j][i] = silu_mul(g[i], u[i]);
        amax = fmaxf(amax, fabsf(y[j][i]));
      }
    }
    const float s = row_scale(block_max(amax, s_red));
    const float inv = 1.0f / s;
    int8_t* qr = q + row * ldq;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = (threadIdx.x + j * kRowThreads) * 8;
      if (c < I) {
        u32x2 o;
        o.x = quant4(y[j][0], y[j][1], y[j][2], y[j][3], s, inv);
        o.y = quant4(y[j][4], y[j][5], y[j][6], y[j][7], s, inv);
        *reinterpret_cast<u32x2*>(qr + c) = o;
      }
    }
    if (threadIdx.x == 0) scale[row] = s;
    return;
  }
  for (int c = threadIdx.x * 8; c < I; c += kRowThreads * 8) {
    float g[8], u[8];
    unpack8(*reinterpret_cast<const u32x4*>(hr + c), g);
    unpack8(*reinterpret_cast<const u32x4*>(hr + I + c), u);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(silu_mul(g[i], u[i])));
  }
  const float s = row_scale(block_max(amax, s_red));
    const float inv = 1.0f / s;
  int8_t* qr = q + row * ldq;
  for (int c = threadIdx.x * 8; c < I; c += kRowThreads * 8) {
    float g[8], u[8], y[8];
    unpack8(*reinterpret_cast<const u32x4*>(hr + c), g);
    unpack8(*reinterpret_cast<const u32x4*>(hr + I + c), u);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = silu_mul(g[i], u[i]);
    u32x2 o;
    o.x = quant4(y[0], y[1], y[2], y[3], s, inv);
    o.y = quant4(y[4], y[5], y[6], y[7], s, inv);
    *reinterpret_cast<u32x2*>(qr + c) = o;
  }
  if (threadIdx.x == 0) scale[row] = s;
}

// One wave per token. Each lane holds experts lane, lane + 64, ... (up to
// E = 1024); the k largest logits are picked one at a time by a wave-wide
// (value desc, index asc) reduction. Softmax is monotonic, so these are the
// top-k of the softmax; the weights are exp(l - l_max) normalised over the
// chosen k (renormalize) or over all E.
constexpr int kMaxPerLane = 16;   // E <= 1024

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

// CPL: 64-expert slots per lane, the smallest power of two >= E / 64 (each
// of the k rounds scans only those)
template <int CPL>
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int64_t ld, int M,
                                                          int E, int k, int renormalize, int32_t* __restrict__ ids,
                                                          float* __restrict__ weights) {
  static_assert(CPL >= 1 && CPL <= kMaxPerLane, "experts per lane");
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;   // whole wave leaves together
  const float* lr = logits + m * ld;
  float v[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int e = j * 64 + lane;
    v[j] = e < E ? lr[e] : -INFINITY;
  }
  float top_v = 0.f;      // logit of the largest expert
  float chosen_sum = 0.f;
  float my_w = 0.f;       // lane j < k keeps the j-th pick
  int my_id = 0;
  for (int t = 0; t < k; ++t) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int e = j * 64 + lane;
      if (e < E && better(v[j], e, bv, bi)) {
        bv = v[j];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (t == 0) top_v = bv;
    const float w = expf(bv - top_v);
    chosen_sum += w;
    if (lane == t) {
      my_w = w;
      my_id = bi;
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      if (j * 64 + lane == bi) v[j] = -INFINITY;
  }
  float denom = chosen_sum;
  if (!renormalize) {
    // full softmax denominator over all E experts (the chosen ones were
    // cleared above, so add their terms back from chosen_sum)
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      if (j * 64 + lane < E && v[j] != -INFINITY) s += expf(v[j] - top_v);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    denom = chosen_sum + s;
  }
  if (lane < k) {
    ids[m * k + lane] = my_id;
    weights[m * k + lane] = my_w / denom;
  }
}

// out[m, n] = bf16( sum_j w[m, j] * y[m * topk + j, n] ) with the products
// and sums in fp32 in j order (w = 1 when weights is null). One thread per
// 8 columns; N % 8 == 0. TK > 0: topk known at compile time, and a thread
// issues all TK row loads before the first sum (TK == 0: a run-time loop
// with one load in flight).
template <int TK>
__global__ __launch_bounds__(256) void combine_topk_kernel(const uint16_t* __restrict__ y, int64_t ldy, int topk,
                                                           int N, const float* __restrict__ weights,
                                                           uint16_t* __restrict__ out, int64_t ldo) {
  // separate float32 rounding of each product and sum (no fused multiply-add)
#pragma clang fp contract(off)
  const int64_t m = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= N) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto add = [&](const u32x4 v, int j) {
    float f[8];
    unpack8(v, f);
    if (weights) {
      const float w = weights[m * topk + j];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p = w * f[i];
        acc[i] = acc[i] + p;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = acc[i] + f[i];
    }
  };
  if constexpr (TK > 0) {
    u32x4 v[TK];
#pragma unroll
    for (int j = 0; j < TK; ++j) v[j] = *reinterpret_cast<const u32x4*>(y + (m * TK + j) * ldy + c);
#pragma unroll
    for (int j = 0; j < TK; ++j) add(v[j], j);
  } else {
    for (int j = 0; j < topk; ++j) add(*reinterpret_cast<const u32x4*>(y + (m * topk + j) * ldy + c), j);
  }
  u32x4 o;
  uint32_t b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = bf16_rne_bits(__float_as_uint(acc[i]));
  o.x = b[0] | (b[1] << 16);
  o.y = b[2] | (b[3] << 16);
  o.z = b[4] | (b[5] << 16);
  o.w = b[6] | (b[7] << 16);
  *reinterpret_cast<u32x4*>(out + m * ldo + c) = o;
}

// ---- weight repack ----------------------------------------------------------
// Reference packing: byte j of an 8-element K run holds k = 2j (low nibble)
// and 2j + 1 (high nibble), i.e. nibble k of the run's 32-bit word is
// element k. MFMA order: byte i holds element i (low) and i + 4 (high), each
// nibble XORed with 8. The GEMM's even/odd nibble split then yields elements
// 0-3 and 4-7 in natural order (no activation relabel), and 16*(u - 8) is
// the flipped nibble shifted into the byte's high half.

// 4 nibbles in bits 0-15 -> one per byte (bits 8i .. 8i+3)
__device__ __forceinline__ uint32_t spread4(uint32_t x) {
  x = (x | (x << 8)) & 0x00FF00FFu;
  return (x | (x << 4)) & 0x0F0F0F0Fu;
}

// inverse of spread4
__device__ __forceinline__ uint32_t compact4(uint32_t x) {
  x = (x | (x >> 4)) & 0x00FF00FFu;
  return (x | (x >> 8)) & 0x0000FFFFu;
}

__device__ __forceinline__ uint32_t to_mfma_order(uint32_t w) {
  return (spread4(w & 0xFFFFu) | (spread4(w >> 16) << 4)) ^ 0x88888888u;
}

__device__ __forceinline__ uint32_t to_reference_order(uint32_t v) {
  v ^= 0x88888888u;
  return compact4(v & 0x0F0F0F0Fu) | (compact4((v >> 4) & 0x0F0F0F0Fu) << 16);
}

// grid-stride over 16-byte vectors (16-byte aligned buffers), then the
// n_words % 4 tail words
__global__ __launch_bounds__(256) void repack_weights_kernel(const uint32_t* __restrict__ src,
                                                             uint32_t* __restrict__ dst, int64_t n_words,
                                                             int inverse) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t n_vec = n_words / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n_vec; i += stride) {
    u32x4 v = reinterpret_cast<const u32x4*>(src)[i];
    if (inverse) {
      v.x = to_reference_order(v.x);
      v.y = to_reference_order(v.y);
      v.z = to_reference_order(v.z);
      v.w = to_reference_order(v.w);
    } else {
      v.x = to_mfma_order(v.x);
      v.y = to_mfma_order(v.y);
      v.z = to_mfma_order(v.z);
      v.w = to_mfma_order(v.w);
    }
    reinterpret_cast<u32x4*>(dst)[i] = v;
  }
  const int64_t t = n_vec * 4 + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t < n_words) dst[t] = inverse ? to_reference_order(src[t]) : to_mfma_order(src[t]);
}

// SiLU requant with a row per wave (kWaveRows rows per workgroup), for rows
// of at most 4 eight-element chunks per lane: lane l holds chunks j at
// elements 8 * (64 j + l), so each load instruction reads 1 KB of contiguous
// row and all of a lane's loads are in flight before the row max, which is
// a wave reduction (no LDS, no barrier). Same arithmetic as
// silu_mul_quant_kernel, so the same bits. (For quant_rows the workgroup
// kernel measured faster.)
constexpr int kWaveRows = 4;

template <int CH>
__global__ __launch_bounds__(64 * kWaveRows) void silu_mul_quant_wave_kernel(const uint16_t* __restrict__ h,
                                                                             int64_t ldh, int P, int I,
                                                                             int8_t* __restrict__ q, int64_t ldq,
                                                                             float* __restrict__ scale) {
  const int64_t row = (int64_t)blockIdx.x * kWaveRows + (threadIdx.x >> 6);
  if (row >= P) return;
  const int lane = threadIdx.x & 63;
  const uint16_t* hr = h + row * ldh;
  u32x4 gv[CH], uv[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = (j * 64 + lane) * 8;
    const bool ok = c < I;
    gv[j] = ok ? *reinterpret_cast<const u32x4*>(hr + c) : u32x4{0, 0, 0, 0};
    uv[j] = ok ? *reinterpret_cast<const u32x4*>(hr + I + c) : u32x4{0, 0, 0, 0};
  }
  float y[CH][8];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    float g[8], u[8];
    unpack8(gv[j], g);
    unpack8(uv[j], u);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      y[j][i] = silu_mul(g[i], u[i]);
      amax = fmaxf(amax, fabsf(y[j][i]));
    }
  }
  const float s = row_scale(wave_max(amax));
  const float inv = 1.0f / s;
  int8_t* qr = q + row * ldq;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = (j * 64 + lane) * 8;
    if (c < I) {
      u32x2 o;
      o.x = quant4(y[j][0], y[j][1], y[j][2], y[j][3], s, inv);
      o.y = quant4(y[j][4], y[j][5], y[j][6], y[j][7], s, inv);
      *reinterpret_cast<u32x2*>(qr + c) = o;
    }
  }
  if (lane == 0) scale[row] = s;
}

}  // namespace

hipError_t launch_repack_weights(const uint32_t* src, uint32_t* dst, int64_t n_words, int inverse, hipStream_t s) {
  if (n_words == 0) return hipSuccess;
  int64_t blocks = (n_words / 4 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(repack_weights_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, n_words, inverse);
  return hipGetLastError();
}

// chunks of 8 elements per thread needed to hold a row of n elements
static int row_chunks(int n) { return (n + kRowThreads * 8 - 1) / (kRowThreads * 8); }

hipError_t launch_quant_rows(const uint16_t* x, int64_t ldx, int M, int K, int8_t* q, int64_t ldq, float* scale,
                             hipStream_t s) {
  if (M == 0) return hipSuccess;
  const int ch = row_chunks(K);
  const dim3 g(M), b(kRowThreads);
  if (ch <= 1) hipLaunchKernelGGL(quant_rows_kernel<1>, g, b, 0, s, x, ldx, K, q, ldq, scale);
  else if (ch <= 2) hipLaunchKernelGGL(quant_rows_kernel<2>, g, b, 0, s, x, ldx, K, q, ldq, scale);
  else if (ch <= 4) hipLaunchKernelGGL(quant_rows_kernel<4>, g, b, 0, s, x, ldx, K, q, ldq, scale);
  else if (ch <= 8) hipLaunchKernelGGL(quant_rows_kernel<8>, g, b, 0, s, x, ldx, K, q, ldq, scale);
  else hipLaunchKernelGGL(quant_rows_kernel<0>, g, b, 0, s, x, ldx, K, q, ldq, scale);
  return hipGetLastError();
}

hipError_t launch_silu_mul_quant(const uint16_t* h, int64_t ldh, int P, int I, int8_t* q, int64_t ldq,
                                 float* scale, hipStream_t s) {
  if (P == 0) return hipSuccess;
  const int cw = (I + 511) / 512;   // chunks per lane of a row per wave
  if (cw <= 4) {
    const dim3 g((P + kWaveRows - 1) / kWaveRows), b(64 * kWaveRows);
    if (cw <= 1) hipLaunchKernelGGL(silu_mul_quant_wave_kernel<1>, g, b, 0, s, h, ldh, P, I, q, ldq, scale);
    else if (cw <= 2) hipLaunchKernelGGL(silu_mul_quant_wave_kernel<2>, g, b, 0, s, h, ldh, P, I, q, ldq, scale);
    else hipLaunchKernelGGL(silu_mul_quant_wave_kernel<4>, g, b, 0, s, h, ldh, P, I, q, ldq, scale);
    return hipGetLastError();
  }
  const int ch = row_chunks(I);
  const dim3 g(P), b(kRowThreads);
  if (ch <= 1) hipLaunchKernelGGL(silu_mul_quant_kernel<1>, g, b, 0, s, h, ldh, I, q, ldq, scale);
  else if (ch <= 2) hipLaunchKernelGGL(silu_mul_quant_kernel<2>, g, b, 0, s, h, ldh, I, q, ldq, scale);
  else if (ch <= 4) hipLaunchKernelGGL(silu_mul_quant_kernel<4>, g, b, 0, s, h, ldh, I, q, ldq, scale);
  else hipLaunchKernelGGL(silu_mul_quant_kernel<0>, g, b, 0, s, h, ldh, I, q, ldq, scale);
  return hipGetLastError();
}

hipError_t launch_router_topk(const float* logits, int64_t ld, int M, int E, int k, int renormalize, int32_t* ids,
                              float* weights, hipStream_t s) {
  if (M == 0) return hipSuccess;
  const dim3 g((M + 3) / 4), b(256);
  const int cpl = (E + 63) / 64;
  if (cpl <= 1) hipLaunchKernelGGL(router_topk_kernel<1>, g, b, 0, s, logits, ld, M, E, k, renormalize, ids, weights);
  else if (cpl <= 2) hipLaunchKernelGGL(router_topk_kernel<2>, g, b, 0, s, logits, ld, M, E, k, renormalize, ids, weights);
  else if (cpl <= 4) hipLaunchKernelGGL(router_topk_kernel<4>, g, b, 0, s, logits, ld, M, E, k, renormalize, ids, weights);
  else if (cpl <= 8) hipLaunchKernelGGL(router_topk_kernel<8>, g, b, 0, s, logits, ld, M, E, k, renormalize, ids, weights);
  else hipLaunchKernelGGL(router_topk_kernel<16>, g, b, 0, s, logits, ld, M, E, k, renormalize, ids, weights);
  return hipGetLastError();
}

hipError_t launch_combine_topk(const uint16_t* y, int64_t ldy, int M, int topk, int N, const float* weights,
                               uint16_t* out, int64_t ldo, hipStream_t s) {
  if (M == 0) return hipSuccess;
  dim3 grid((N / 8 + 255) / 256, M);
  const dim3 b(256);
  switch (topk) {
    case 1: hipLaunchKernelGGL(combine_topk_kernel<1>, grid, b, 0, s, y, ldy, topk, N, weights, out, ldo); break;
    case 2: hipLaunchKernelGGL(combine_topk_kernel<2>, grid, b, 0, s, y, ldy, topk, N, weights, out, ldo); break;
    case 4: hipLaunchKernelGGL(combine_topk_kernel<4>, grid, b, 0, s, y, ldy, topk, N, weights, out, ldo); break;
    case 6: hipLaunchKernelGGL(combine_topk_kernel<6>, grid, b, 0, s, y, ldy, topk, N, weights, out, ldo); break;
    case 8: hipLaunchKernelGGL(combine_topk_kernel<8>, grid, b, 0, s, y, ldy, topk, N, weights, out, ldo); break;
    default: hipLaunchKernelGGL(combine_topk_kernel<0>, grid, b, 0, s, y, ldy, topk, N, weights, out, ldo); break;
  }
  return hipGetLastError();
}

}  // namespace mw4a8
