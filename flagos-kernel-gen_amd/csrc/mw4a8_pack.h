// Operand packing helpers shared by the grouped-GEMM kernel and the host
// self-test. Everything here is plain integer arithmetic on 32-bit words so
// the same code runs on the CPU (mw4a8_host_selftest) and on gfx950.
//
// K relabelling. An int8 MFMA sums over its K slots in any order, so the
// activation operand (A) and the weight operand (B) only have to agree on
// which k sits in which byte slot. The packed weight byte p holds k = 2p in
// its low nibble and k = 2p + 1 in its high nibble (docs/Task1.md:78-81).
// Splitting a 32-bit word of packed bytes with a mask and a shift yields the
// even k's of four bytes in one word and the odd k's in another. The
// activations are relabelled to match once, on their way into LDS: every
// 8-byte run x[k0 .. k0+7] is stored as
//     x0 x2 x4 x6 | x1 x3 x5 x7
// so a 16-byte A fragment and the B fragment unpacked from 8 packed bytes
// enumerate the same 16 k's in the same order:
//     0 2 4 6 1 3 5 7 8 10 12 14 9 11 13 15   (relative to k0).
//
// Zero-point fold. The reference computes int8(int16(u) - int16(z)) per
// element, which wraps modulo 256 (docs/Task1.md:83-85). With c = (-z) mod
// 256, the wrapped byte is (u + c) mod 256. For u <= 15 the per-byte sum
// u + (c & 0x7f) never exceeds 0xff, so adding (c & 0x7f) to four bytes at
// once cannot carry between bytes, and adding bit 7 of c modulo 256 is an
// XOR. Two word operations therefore fold four weights exactly, including
// the wrap regime.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define MW4A8_HD __host__ __device__ __forceinline__
#else
#define MW4A8_HD inline
#endif

namespace mw4a8 {

// v_perm_b32: byte i of the result is byte sel[i] (0..7) of the 8-byte value
// {hi, lo} (lo = bytes 0..3, hi = bytes 4..7). On the host this is a plain
// emulation of the same selector semantics, so the CPU self-test checks the
// selector constants the GPU uses.
MW4A8_HD uint32_t byte_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_perm(hi, lo, sel);
#else
  const uint64_t v = ((uint64_t)hi << 32) | lo;
  uint32_t r = 0;
  for (int i = 0; i < 4; ++i) r |= (uint32_t)((v >> (8 * ((sel >> (8 * i)) & 7))) & 0xffu) << (8 * i);
  return r;
#endif
}

// Bytes 0,2 of d0 and 0,2 of d1 -> one word (the even positions of an 8-byte run).
MW4A8_HD uint32_t even_bytes(uint32_t d0, uint32_t d1) { return byte_perm(d1, d0, 0x06040200u); }

// Bytes 1,3 of d0 and 1,3 of d1 -> one word (the odd positions of an 8-byte run).
MW4A8_HD uint32_t odd_bytes(uint32_t d0, uint32_t d1) { return byte_perm(d1, d0, 0x07050301u); }

// Per-(column, group) constants of the zero-point fold.
struct ZeroFold {
  uint32_t lo7;   // (c & 0x7f) in every byte
  uint32_t hi1;   // (c & 0x80) in every byte
};

MW4A8_HD ZeroFold make_zero_fold(int z) {
  const uint32_t c = (uint32_t)(-z) & 0xffu;
  ZeroFold f;
  f.lo7 = (c & 0x7fu) * 0x01010101u;
  f.hi1 = (c & 0x80u) * 0x01010101u;
  return f;
}

// Low nibbles of four packed bytes (even k) -> four int8 weights.
MW4A8_HD uint32_t fold_even(uint32_t packed, ZeroFold f) {
  return ((packed & 0x0f0f0f0fu) + f.lo7) ^ f.hi1;
}

// High nibbles of four packed bytes (odd k) -> four int8 weights.
MW4A8_HD uint32_t fold_odd(uint32_t packed, ZeroFold f) {
  return (((packed >> 4) & 0x0f0f0f0fu) + f.lo7) ^ f.hi1;
}

// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
MW4A8_HD uint16_t bf16_rne_bits(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

}  // namespace mw4a8
