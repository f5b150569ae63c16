// Shared device-side helpers for the gfx950 (CDNA4) kernels of neso_amd.
//
// Everything here is written for one target: 64-lane wavefronts, the
// v_mfma_f32_{32x32x16,16x16x32}_f16 matrix instructions and the 160 KiB LDS
// of an MI355X compute unit.  There is no portability layer on purpose.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace neso {

typedef _Float16 half_t;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef int32_t int4v __attribute__((ext_vector_type(4)));
typedef uint32_t uint4v __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// D(32x32,f32) += A(32x16,f16) * B(16x32,f16).
// Lane l supplies A[l%32][8*(l/32) + 0..7] and B[8*(l/32) + 0..7][l%32];
// accumulator register r of lane l is D[8*(r/4) + 4*(l/32) + r%4][l%32].
__device__ __forceinline__ float16v mfma32x32x16(half8v a, half8v b, float16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// D(16x16,f32) += A(16x32,f16) * B(32x16,f16).
// Lane l supplies A[l%16][8*(l/16) + 0..7] and B[8*(l/16) + 0..7][l%16];
// accumulator register r of lane l is D[4*(l/16) + r][l%16].
__device__ __forceinline__ float4v mfma16x16x32(half8v a, half8v b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 2^x on the transcendental unit (v_exp_f32); exp2(-inf) == 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Value held by lane (l ^ 32): the other half of a 64-lane wavefront.
__device__ __forceinline__ float swap_halves(float x) {
  return __shfl_xor(x, 32, kWave);
}

// Wavefront-wide sum; every lane receives the total.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

__device__ __forceinline__ half8v load_half8(const half_t* p) {
  return *reinterpret_cast<const half8v*>(p);
}

// Raw buffer resource over [base, base + bytes).  Buffer loads whose offset
// lies past `bytes` return zeros and such stores are dropped, which gives
// tail handling without per-element compares or clamped addresses.
// dword3 = 0x00020000: 32-bit data format, no swizzle (gfx9 family).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
// Cache-policy operand of the buffer intrinsics: the "nt" (non-temporal,
// streaming) bit of gfx94x/gfx950 memory instructions.
constexpr int kNonTemporal = 2;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
// Byte offset of element idx of a buffer of n elements of `bytes` each, or
// an offset past any buffer when idx is outside [0, n) (the load then
// returns zero).  A negative idx must not reach the load as a wrapped
// offset: the compiler may move a constant part of an offset into the
// instruction's immediate field, and the range check of raw buffer loads
// then sees the register part alone, so an in-range element whose register
// part is a wrapped negative number would read as zero.
__device__ __forceinline__ uint32_t elem_offset(int idx, int n, uint32_t bytes) {
  return (uint32_t)idx < (uint32_t)n ? (uint32_t)idx * bytes : 0xFFFFFFF0u;
}

__device__ __forceinline__ half8v buf_load_half8(rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(half8v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
__device__ __forceinline__ float buf_load_f32(rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
}
// The same as asm, which the compiler's wait-count bookkeeping does not
// see: the caller issues the s_waitcnt that covers it before any use of the
// result, and ties the result to that wait (an empty asm with the value as
// "+v" operand after it).
__device__ __forceinline__ float buf_load_f32_untracked(rsrc_t r, uint32_t byte_off) {
  float v;
  asm volatile("buffer_load_dword %0, %1, %2, 0 offen" : "=v"(v) : "v"(byte_off), "s"(r) : "memory");
  return v;
}
__device__ __forceinline__ void buf_store_f32x4(float4v v, rsrc_t r, uint32_t byte_off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(int4v, v), r, byte_off, 0, 0);
}
__device__ __forceinline__ void buf_store_f16x4(half4v v, rsrc_t r, uint32_t byte_off) {
  typedef int int2v __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(int2v, v), r, byte_off, 0, 0);
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// fences global memory, which makes the compiler drain every outstanding
// global load (s_waitcnt vmcnt(0)) at the barrier and defeats prefetching.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Workgroup index remapped so that consecutive logical indices land on the
// same XCD.  The hardware dispatcher deals workgroups round-robin over the
// 8 XCDs (workgroup i runs on XCD i % 8); each XCD has its own L2, so
// workgroups that share K/V (or weight) tiles should share an XCD.  XCD x
// takes the contiguous logical range of its total / 8 workgroups, one more
// for the first total % 8 XCDs: a bijection of [0, total) for any total.
__device__ __forceinline__ uint32_t xcd_swizzle(uint32_t hw_id, uint32_t total) {
  constexpr uint32_t kXcds = 8;
  const uint32_t q = total / kXcds, r = total % kXcds;
  const uint32_t x = hw_id % kXcds, local = hw_id / kXcds;
  return x < r ? x * (q + 1) + local : r * (q + 1) + (x - r) * q + local;
}

}  // namespace neso
