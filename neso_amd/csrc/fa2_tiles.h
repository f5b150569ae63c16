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

}  // namespace neso
