// Tile-layout helpers shared by the FA2 forward kernels (fa2_fwd.hip,
// fa2_fast.hip).  Both compute the score tile transposed, S^T = K Q^T, with
// v_mfma_f32_32x32x16_f16, so lane l holds the scores of query l % 32 and
// lane l ^ 32 holds the other keys of the same query.
#pragma once

#include "common.h"

namespace neso {

// Row of the 32-key tile loaded into A-operand row rho (= lane % 32) so that
// accumulator register r of lane group g holds key 16*(r/8) + 8*g + r%8.
// Accumulator row rho = 8*(r/4) + 4*g + r%4 (see mfma32x32x16).  With this
// order, 8 consecutive accumulator registers are 8 consecutive keys, which
// is the B-operand fragment of the P V product: P never leaves registers.
__device__ __forceinline__ int kRowPerm(int rho) {
  const int b = rho >> 3, g = (rho >> 2) & 1, j = rho & 3;
  return 16 * (b >> 1) + 8 * g + 4 * (b & 1) + j;
}

// max / sum over lanes l and l ^ 32 (v_permlane32_swap returns the
// lower-half and upper-half values of the lane's position within its half).
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// V tiles live row-major in LDS, [key][D] halves without padding, and the
// P V product reads its V^T operand with gfx950's transposing LDS load.
// 16-byte chunk c of key row r is stored at chunk c ^ vswz<D>(r), which
// makes both the 16-byte stores and the transposed reads below touch every
// LDS bank once per 32-lane pass: a pass reads rows r0..r0+3 (r0 % 4 == 0),
// four chunks each.  D = 32: rows are 16 dwords, four rows fill the banks.
// D = 64: rows r and r+2 share banks unless bit 1 of r flips chunk bit 2.
// D = 128: a row spans all banks, so row r % 4 picks one of four 4-chunk
// sets.
template <int D>
__device__ __forceinline__ int vswz(int r) {
  static_assert(D == 32 || D == 64 || D == 128, "head dim");
  if constexpr (D == 128) return (r & 3) * 4;
  else if constexpr (D == 64) return ((r >> 1) & 1) * 4;
  else return 0;
}

// Position (halves) of the 8-element V piece of key row r, chunk c.
template <int D>
__device__ __forceinline__ int v_store_at(int r, int c) {
  return r * D + 8 * (c ^ vswz<D>(r));
}

// ds_read_b64_tr_b16: in each group of 16 lanes, lane 4e + t passes the
// address of 4 halves (row e, columns 4t..4t+3 of a 4 x 16 tile) and lane j
// receives column j, the 4 rows' element j.
__device__ __forceinline__ half4v lds_read_tr16(const half_t* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(const_cast<half_t*>(p)));
  return __builtin_bit_cast(half4v, r);
}

// This lane's offset (halves) into a V tile for d tile u: key row
// 8 (l / 32) + (l % 16) / 4, columns 32u + 16 ((l / 16) % 2) + 4 (l % 4)
// .. +3, swizzled.  Adding 16 cc or 4 rows leaves the swizzle unchanged
// (it depends on row bits 0 and 1 only).
template <int D>
__device__ __forceinline__ int v_tr_offset(int lane, int u) {
  const int row = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int cu = 32 * u + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  return row * D + 8 * ((cu >> 3) ^ vswz<D>(row)) + (cu & 7);
}

// A operand of O^T += V^T P^T for the 16-key chunk cc (off = v_tr_offset
// of the d tile): lane l gets V[16 cc + 8 (l / 32) + 0..7][32 u + l % 32],
// two 4-key transposed reads.
template <int D>
__device__ __forceinline__ half8v v_frag_tr(const half_t* v_l, int off, int cc) {
  const half_t* pp = v_l + off + 16 * cc * D;
  const half4v a = lds_read_tr16(pp);
  const half4v b = lds_read_tr16(pp + 4 * D);
  return half8v{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Chunk swizzle of the K rows: chunk c of key row r sits at chunk
// c ^ kswz(r).  A K fragment read takes one chunk from each of 16 rows per
// 16-lane pass, rows 0..15 of a 32-row tile in kRowPerm order.  D = 64: a
// 128-byte row covers half the banks, so rows of equal parity need 8
// distinct chunk positions, which bits 1..3 of r give.  D = 128: a row
// covers all banks, so the 16 rows need 16 positions, bits 0..3 of r.
template <int D>
__device__ __forceinline__ int kswz(int r) {
  static_assert(D == 64 || D == 128, "head dim");
  return D == 128 ? (r & 15) : ((r >> 1) & 7);
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// s_waitcnt vmcnt(N): at most the N most recent vector-memory instructions
// of this wave still in flight (gfx9 encoding: vmcnt bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vmem_n() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// 16 bytes per lane from the buffer into LDS (buffer_load_dwordx4 ... lds):
// lane l's bytes land at LDS byte address lds + 16 l.  Written as asm so
// that the compiler does not make the kernel's LDS reads wait for it (it
// cannot tell that they read other slots); the kernel orders these writes
// itself with s_waitcnt vmcnt(0) and a barrier before the slot is read.
// Vector loads only; M0 holds the LDS base (one wait state after writing
// it).  The compiler treats M0 as reserved and ignores the clobber, so
// correctness rests on no compiler-generated instruction using M0 in these
// kernels: neso_amd/build.py checks the assembly of every build for that and
// builds the library without the fast kernel if the check fails.
__device__ __forceinline__ void lds_dma16(rsrc_t r, uint32_t lds, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds), "v"(voff), "s"(r)
      : "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const half_t* p) {
  return (uint32_t)(size_t)(__attribute__((address_space(3))) const half_t*)p;
}

}  // namespace neso
