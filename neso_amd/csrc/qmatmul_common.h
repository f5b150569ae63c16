// Helpers shared by the int4 matmul translation units (qmatmul.hip and
// qmatmul_skinny.hip): f16 exponent-trick dequantisation and the 4x4
// transpose across 16-lane rows.
#pragma once

#include "common.h"

namespace neso {
namespace {

__device__ __forceinline__ half2v as_half2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

// 32-bit constants the compiler cannot fold back into literals: gfx9 VOP3
// encodings take no literal and read at most one SGPR, so v_and_or_b32
// needs its two constants as one SGPR and one VGPR.
__device__ __forceinline__ uint32_t sgpr_const(uint32_t v) {
  uint32_t r;
  asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
  return r;
}
__device__ __forceinline__ uint32_t vgpr_const(uint32_t v) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
  return r;
}

// Nibble masks and the f16 exponent patterns, held in registers so that
// (w & mask) | magic is one v_and_or_b32: 0x6400 (f16 1024, ulp 1) turns a
// low nibble c into 1024 + c, 0x5400 (f16 64, ulp 1/16) turns a high
// nibble, which sits at 16 c, into 64 + c.
struct Nibbles {
  uint32_t lo, hi, mag, mag16;
};
__device__ __forceinline__ Nibbles nibble_consts() {
  return Nibbles{sgpr_const(0x000F000Fu), sgpr_const(0x00F000F0u), vgpr_const(0x64006400u),
                 vgpr_const(0x54005400u)};
}

// The zero-point offsets: z1 = 1024 + z for the low nibbles, z64 = 64 + z
// for the high ones, z16 = 1024 + 16 z for high nibbles taken with the 0x6400
// pattern (all exact in f16).
struct ZeroPoint {
  half2v z1, z64, z16;
};
__device__ __forceinline__ ZeroPoint zero_point(int z) {
  const half_t a = (half_t)(1024 + z), b = (half_t)(64 + z), c = (half_t)(1024 + 16 * z);
  return ZeroPoint{{a, a}, {b, b}, {c, c}};
}

// Four f16 pairs of one packed word, shifted by the zero point, all exact:
//   r[0] = (c0 - z, c4 - z)        r[1] = (c1 - z, c5 - z)
//   r[2] = (c2 - z, c6 - z)        r[3] = (c3 - z, c7 - z)
__device__ __forceinline__ void unpack_word(uint32_t w, const Nibbles& k, const ZeroPoint& z,
                                            half2v r[4]) {
  const uint32_t w8 = w >> 8;
  r[0] = as_half2((w & k.lo) | k.mag) - z.z1;
  r[1] = as_half2((w & k.hi) | k.mag16) - z.z64;
  r[2] = as_half2((w8 & k.lo) | k.mag) - z.z1;
  r[3] = as_half2((w8 & k.hi) | k.mag16) - z.z64;
}

// The same with the high nibbles as 16 (c - z), for a scale of s / 16 on
// r[1] and r[3] (the tile GEMM: the form above measured 1.5-2% slower there,
// M = 256 / 512).  Equal results to unpack_word's while s / 16 is a normal
// f16.
__device__ __forceinline__ void unpack_word_x16(uint32_t w, const Nibbles& k, const ZeroPoint& z,
                                                half2v r[4]) {
  const uint32_t w8 = w >> 8;
  r[0] = as_half2((w & k.lo) | k.mag) - z.z1;
  r[1] = as_half2((w & k.hi) | k.mag) - z.z16;
  r[2] = as_half2((w8 & k.lo) | k.mag) - z.z1;
  r[3] = as_half2((w8 & k.hi) | k.mag) - z.z16;
}

// Word j of register w_j in 16-lane row g (chunk g, word j) becomes word g
// of chunk j: a 4x4 transpose between the registers and the four rows.
// v_permlane32_swap exchanges the upper 32 lanes of its first operand with
// the lower 32 lanes of its second; v_permlane16_swap exchanges the odd rows
// of its first operand with the even rows of its second.
__device__ __forceinline__ void transpose_rows4(uint32_t& w0, uint32_t& w1, uint32_t& w2,
                                                uint32_t& w3) {
  const auto a = __builtin_amdgcn_permlane32_swap(w0, w2, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(w1, w3, false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  w0 = c[0];
  w1 = c[1];
  w2 = d[0];
  w3 = d[1];
}

}  // namespace
}  // namespace neso
