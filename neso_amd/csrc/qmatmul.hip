// Weight-only quantised matmul for gfx950.
//
// W4A16 (BASELINE format, no reference kernel): Y[M][N] f16 = X[M][K] f16 *
// dequant(W)^T, W packed 8 int4 codes per int32 along K ([N][K/8], code of
// column k is nibble k%8 of word k/8, low nibble first), f16 scales
// [N][K/group], dequant(c) = (c - zero) * scale.  Two regimes:
//   * small M (GEMV): each lane streams one 16-byte word quad = 32 codes = one
//     scale group per load, fully coalesced (a wave reads 1 KiB contiguous),
//     X lives in registers pre-paired for v_dot2_f32_f16;
//   * larger M: the dequantised word is the B operand of
//     v_mfma_f32_32x32x16_f16 directly in registers.
// Dequantisation uses the f16 exponent trick: (w & 0x000F000F) | 0x64006400
// is the f16 pair (1024 + c0, 1024 + c4); subtracting (1024 + zero) is exact.
// Nibbles at bit 4 give 1024 + 16c, handled with a 1/16 factor (exact).
//
// W8A16 (tests/test_quantized_matmul.py:67-167 and :181-283): C[M][N] f32 =
// A[M][K] f16 * f16(B[K][N] int8) [* scale[n] after accumulation].
#include "common.h"
#include "neso_internal.h"

namespace neso {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ half2v as_half2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

// Four f16 pairs of one packed word, shifted by the zero point:
//   r[0] = (c0 - z, c4 - z)        r[1] = 16 * (c1 - z, c5 - z)
//   r[2] = (c2 - z, c6 - z)        r[3] = 16 * (c3 - z, c7 - z)
__device__ __forceinline__ void unpack_word(uint32_t w, half2v z1, half2v z16, half2v r[4]) {
  const uint32_t w8 = w >> 8;
  r[0] = as_half2((w & 0x000F000Fu) | 0x64006400u) - z1;
  r[1] = as_half2((w & 0x00F000F0u) | 0x64006400u) - z16;
  r[2] = as_half2((w8 & 0x000F000Fu) | 0x64006400u) - z1;
  r[3] = as_half2((w8 & 0x00F000F0u) | 0x64006400u) - z16;
}

// ---------------------------------------------------------------------------
// GEMV regime.  MR activation rows, ROWS weight rows per wave, GI 16-byte
// group loads per lane per row (K <= 2048 * GI).
template <int MR, int ROWS, int GI>
__global__ __launch_bounds__(kThreads) void w4a16_gemv_kernel(W4Args a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int G = a.K >> 5;        // 32-code chunks per row
  const int KW = a.K >> 3;       // words per row
  const int SG = a.K / a.group;  // scales per row
  const int n0 = (blockIdx.x * (kThreads / kWave) + wave) * ROWS;
  if (n0 >= a.N) return;

  const half2v z1 = {(half_t)(1024 + a.zero), (half_t)(1024 + a.zero)};
  const half2v z16 = {(half_t)(1024 + 16 * a.zero), (half_t)(1024 + 16 * a.zero)};

  // Weight words and scales first: the HBM stream is what this kernel waits on.
  uint4v wv[ROWS][GI];
  float sc[ROWS][GI];
#pragma unroll
  for (int rr = 0; rr < ROWS; ++rr) {
    const int n = n0 + rr;
#pragma unroll
    for (int gi = 0; gi < GI; ++gi) {
      const int gch = lane + 64 * gi;
      const bool ok = n < a.N && gch < G;
      wv[rr][gi] = ok ? *reinterpret_cast<const uint4v*>(a.W + (int64_t)n * KW + 4 * gch)
                      : uint4v{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
      sc[rr][gi] = ok ? (float)a.S[(int64_t)n * SG + (32 * gch) / a.group] : 0.f;
    }
  }

  // X pairs: for word i of chunk gi, xp[.][gi][4i + e] pairs element e with
  // element e + 4 of that word's eight columns (the order unpack_word gives).
  half2v xp[MR][GI][16];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
#pragma unroll
    for (int gi = 0; gi < GI; ++gi) {
      const int gch = lane + 64 * gi;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half8v x = (m < a.M && gch < G)
                             ? load_half8(a.X + (int64_t)m * a.ldx + 32 * gch + 8 * i)
                             : half8v{};
        xp[m][gi][4 * i + 0] = half2v{x[0], x[4]};
        xp[m][gi][4 * i + 1] = half2v{x[1], x[5]};
        xp[m][gi][4 * i + 2] = half2v{x[2], x[6]};
        xp[m][gi][4 * i + 3] = half2v{x[3], x[7]};
      }
    }
  }

#pragma unroll
  for (int rr = 0; rr < ROWS; ++rr) {
    float y[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) y[m] = 0.f;
#pragma unroll
    for (int gi = 0; gi < GI; ++gi) {
      float a1[MR], a16[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) a1[m] = a16[m] = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        half2v r[4];
        unpack_word(wv[rr][gi][i], z1, z16, r);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          a1[m] = __builtin_amdgcn_fdot2(r[0], xp[m][gi][4 * i + 0], a1[m], false);
          a16[m] = __builtin_amdgcn_fdot2(r[1], xp[m][gi][4 * i + 1], a16[m], false);
          a1[m] = __builtin_amdgcn_fdot2(r[2], xp[m][gi][4 * i + 2], a1[m], false);
          a16[m] = __builtin_amdgcn_fdot2(r[3], xp[m][gi][4 * i + 3], a16[m], false);
        }
      }
#pragma unroll
      for (int m = 0; m < MR; ++m) y[m] += (a1[m] + a16[m] * 0.0625f) * sc[rr][gi];
    }
    const int n = n0 + rr;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float t = wave_sum(y[m]);
      if (lane == 0 && n < a.N && m < a.M) a.Y[(int64_t)m * a.ldy + n] = (half_t)t;
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA regime.  Each wave computes a 32 (m) x 32*TN (n) strip; 4 waves side
// by side along N.  Per 64-column step of K, lane group g owns columns
// [kb + 32g, kb + 32g + 32): one 16-byte word quad and one scale per row.
// MFMA step j uses word j of that quad; the eight codes come out of
// unpack_word in the order {0,4,1,5,2,6,3,7}, and the X fragment is
// permuted the same way, so no register shuffles touch the weights.
template <int TN>
__global__ __launch_bounds__(kThreads) void w4a16_mfma_kernel(W4Args a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 5;
  const int li = lane & 31;
  const int m0 = blockIdx.y * 32;
  const int nw0 = (blockIdx.x * (kThreads / kWave) + wave) * (32 * TN);
  if (nw0 >= a.N) return;
  const int KW = a.K >> 3;
  const int SG = a.K / a.group;
  const half2v z1 = {(half_t)(1024 + a.zero), (half_t)(1024 + a.zero)};
  const half2v z16 = {(half_t)(1024 + 16 * a.zero), (half_t)(1024 + 16 * a.zero)};

  float16v acc[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) acc[t] = float16v{};

  const int m = m0 + li;
  for (int kb = 0; kb < a.K; kb += 64) {
    const int kc = kb + 32 * g;  // this lane group's 32 columns
    const bool kok = kc < a.K;
    half8v xa[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half8v x = (m < a.M && kok) ? load_half8(a.X + (int64_t)m * a.ldx + kc + 8 * j)
                                        : half8v{};
      xa[j] = half8v{x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]};
    }
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int n = nw0 + 32 * t + li;
      const bool ok = n < a.N && kok;
      const uint4v w = ok ? *reinterpret_cast<const uint4v*>(a.W + (int64_t)n * KW + (kc >> 3))
                          : uint4v{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
      const half_t s = ok ? a.S[(int64_t)n * SG + kc / a.group] : (half_t)0;
      const half2v s1 = {s, s};
      const half_t s16v = s * (half_t)0.0625f;
      const half2v s16 = {s16v, s16v};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        half2v r[4];
        unpack_word(w[j], z1, z16, r);
        const half2v d0 = r[0] * s1, d1 = r[1] * s16, d2 = r[2] * s1, d3 = r[3] * s16;
        const half8v b = {d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
        acc[t] = mfma32x32x16(xa[j], b, acc[t]);
      }
    }
  }

  // acc[t] register r: row m0 + 8*(r/4) + 4*g + r%4, column nw0 + 32t + li.
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int n = nw0 + 32 * t + li;
    if (n >= a.N) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mm = m0 + 8 * (r >> 2) + 4 * g + (r & 3);
      if (mm < a.M) a.Y[(int64_t)mm * a.ldy + n] = (half_t)acc[t][r];
    }
  }
}

// ---------------------------------------------------------------------------
// W8A16: one 32x32 output tile per wave, B[K][N] int8 row-major.
__global__ __launch_bounds__(kThreads) void w8a16_kernel(W8Args a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 5;
  const int li = lane & 31;
  const int m0 = blockIdx.y * 32;
  const int n0 = (blockIdx.x * (kThreads / kWave) + wave) * 32;
  if (n0 >= a.N) return;
  const int m = m0 + li;
  const int n = n0 + li;
  float16v acc = float16v{};
  for (int k0 = 0; k0 < a.K; k0 += 16) {
    half8v av, bv;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = k0 + 8 * g + i;
      av[i] = (m < a.M && k < a.K) ? a.A[(int64_t)m * a.lda + k] : (half_t)0;
      bv[i] = (n < a.N && k < a.K) ? (half_t)(float)a.B[(int64_t)k * a.ldb + n] : (half_t)0;
    }
    acc = mfma32x32x16(av, bv, acc);
  }
  if (n >= a.N) return;
  const float s = a.scale ? (float)a.scale[n] : 1.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int mm = m0 + 8 * (r >> 2) + 4 * g + (r & 3);
    if (mm < a.M) a.C[(int64_t)mm * a.ldc + n] = acc[r] * s;
  }
}

template <int MR>
hipError_t launch_gemv_mr(const W4Args& a, hipStream_t s) {
  constexpr int ROWS = 4;
  const int waves = (a.N + ROWS - 1) / ROWS;
  const int blocks = (waves + 3) / 4;
  const int G = a.K / 32;
  if (G <= 64) {
    hipLaunchKernelGGL((w4a16_gemv_kernel<MR, ROWS, 1>), dim3(blocks), dim3(kThreads), 0, s, a);
  } else if (G <= 128) {
    hipLaunchKernelGGL((w4a16_gemv_kernel<MR, ROWS, 2>), dim3(blocks), dim3(kThreads), 0, s, a);
  } else if (G <= 256) {
    hipLaunchKernelGGL((w4a16_gemv_kernel<MR, ROWS, 4>), dim3(blocks), dim3(kThreads), 0, s, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

int w4a16_gemv_max_k() { return 32 * 256; }

hipError_t launch_w4a16(const W4Args& a, hipStream_t s) {
  if (a.M <= 4 && a.K <= w4a16_gemv_max_k()) {
    switch (a.M) {
      case 1: return launch_gemv_mr<1>(a, s);
      case 2: return launch_gemv_mr<2>(a, s);
      case 3: return launch_gemv_mr<3>(a, s);
      default: return launch_gemv_mr<4>(a, s);
    }
  }
  constexpr int TN = 2;
  const dim3 grid((a.N + 4 * 32 * TN - 1) / (4 * 32 * TN), (a.M + 31) / 32);
  hipLaunchKernelGGL((w4a16_mfma_kernel<TN>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_w8a16(const W8Args& a, hipStream_t s) {
  const dim3 grid((a.N + 127) / 128, (a.M + 31) / 32);
  hipLaunchKernelGGL(w8a16_kernel, grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace neso
