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
#include <stdlib.h>

#include "common.h"
#include "neso_internal.h"
#include "qmatmul_common.h"
#include "fa2_tiles.h"

namespace neso {

namespace {

constexpr int kThreads = 256;

// ---------------------------------------------------------------------------
// GEMV regime (M <= 2 by default, up to 4): a persistent stream of weight rows.
//
// Wave w handles rows w, w + T, w + 2T, ... (T = waves in the grid), so at
// any moment the grid streams one contiguous stretch of W.  Lane l owns the
// 32-code chunks l + 64*gi of a row: one 16-byte load per chunk, a wave
// reads 1 KiB contiguous per instruction.  The next row's words and scales
// are loaded while the current row is reduced.  Rows and chunks past the
// end come back as zeros from the buffer bounds check.
//
// Dequantisation without the zero-point subtraction: the exponent trick
// yields (1024 + c) for the low nibble of each byte (OR 0x6400: ulp 1) and
// (64 + c) for the high one (the nibble sits at 16 c in the mantissa; OR
// 0x5400: ulp 1/16), both exact f16.  v_dot2_f32_f16 accumulates them
// against X pairs in one fp32 chain per chunk that starts at
//   corr = -(1024 + z) * S_A - (64 + z) * S_B
// (S_A, S_B = sums of the X elements paired with the two nibble sets), so
// the chain ends at sum((c - z) x) exactly in real arithmetic.  Per 8
// codes: 1 shift, 4 v_and_or_b32, 4 v_dot2.

// Sum over the 64 lanes with DPP row operations; the total lands in lane 63
// and is returned to every lane.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false);
  return v + __int_as_float(s);
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xF>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xF>(v);  // row_mirror
  v = dpp_add<0x142, 0xA>(v);  // row_bcast:15
  v = dpp_add<0x143, 0xC>(v);  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

template <int GI>
struct GemvRow {
  uint4v w[GI];
  float s[GI];
  uint32_t sw;  // GI == 2, group 32: scales 2l and 2l+1 of the row
};

// PS (two chunks per lane, group 32): the scales come as one 4-byte load per
// row and lane.
template <int MR, int GI, int R, bool PS>
__global__ __launch_bounds__(kThreads) void w4a16_gemv_kernel(W4Args a) {
  static_assert(!PS || GI == 2, "paired scales need two chunks per lane");
  const int lane = threadIdx.x & 63;
  const int wid = blockIdx.x * (kThreads / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int T = gridDim.x * (kThreads / kWave);
  const int KW = a.K >> 3;       // words per row
  const int SG = a.K / a.group;  // scales per row
  const uint32_t mlo = sgpr_const(0x000F000Fu);
  const uint32_t mhi = sgpr_const(0x00F000F0u);
  const uint32_t mag = vgpr_const(0x64006400u);    // f16 1024: low nibble -> 1024 + c
  const uint32_t mag16 = vgpr_const(0x54005400u);  // f16 64: nibble at 16 c -> 64 + c

  half2v xp[MR][GI][16];  // X pairs, paired like the nibbles of a word
  float corr[MR][GI];

  auto load_row = [&](GemvRow<GI>& r, int n) {
    // Rows past the end get an empty buffer resource: all loads return 0.
    // Weights and scales are read once per call: non-temporal loads.
    const bool ok = n < a.N;
    const rsrc_t rw = make_rsrc(a.W + (int64_t)(ok ? n : 0) * KW, ok ? (uint32_t)KW * 4 : 0u);
    const rsrc_t rs = make_rsrc(a.S + (int64_t)(ok ? n : 0) * SG, ok ? (uint32_t)SG * 2 : 0u);
#pragma unroll
    for (int gi = 0; gi < GI; ++gi) {
      const int gch = lane + 64 * gi;
      r.w[gi] = __builtin_bit_cast(uint4v, __builtin_amdgcn_raw_buffer_load_b128(
                                               rw, (uint32_t)gch * 16u, 0, kNonTemporal));
      if constexpr (!PS) {
        const uint32_t sidx = (uint32_t)(32 * gch) / (uint32_t)a.group;
        r.s[gi] = (float)__builtin_bit_cast(
            half_t, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, sidx * 2u, 0, kNonTemporal));
      }
    }
    // Two chunks per lane with one scale each: the row's 128 scales in one
    // 4-byte load per lane (half as many load instructions), handed to the
    // lanes that own those chunks in row_dot.
    if constexpr (PS)
      r.sw = __builtin_amdgcn_raw_buffer_load_b32(rs, (uint32_t)lane * 4u, 0, kNonTemporal);
  };

  // Scales of chunks l and l + 64 from lanes l/2 and 32 + l/2 (half l % 2).
  auto pair_scales_of = [&](GemvRow<GI>& r) {
    if constexpr (PS) {
      const int sh = (lane & 1) * 16;
      const uint32_t d0 = (uint32_t)__builtin_amdgcn_ds_bpermute((lane >> 1) * 4, (int)r.sw);
      const uint32_t d1 = (uint32_t)__builtin_amdgcn_ds_bpermute((32 + (lane >> 1)) * 4, (int)r.sw);
      r.s[0] = (float)__builtin_bit_cast(half_t, (uint16_t)(d0 >> sh));
      r.s[1] = (float)__builtin_bit_cast(half_t, (uint16_t)(d1 >> sh));
    }
  };

  auto row_dot = [&](GemvRow<GI>& r, float (&y)[MR]) {
    pair_scales_of(r);
#pragma unroll
    for (int gi = 0; gi < GI; ++gi) {
      // One chain per chunk and X row, started at the correction: the GI
      // chunks, the MR rows and the waves of a SIMD overlap the chains (two
      // or four chains per chunk measured no faster).
      float acc[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[m] = corr[m][gi];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = r.w[gi][i];
        const uint32_t w8 = w >> 8;
        const half2v h0 = as_half2((w & mlo) | mag);     // (1024 + c0, 1024 + c4)
        const half2v h1 = as_half2((w & mhi) | mag16);   // (64 + c1, 64 + c5)
        const half2v h2 = as_half2((w8 & mlo) | mag);    // (1024 + c2, 1024 + c6)
        const half2v h3 = as_half2((w8 & mhi) | mag16);  // (64 + c3, 64 + c7)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          acc[m] = __builtin_amdgcn_fdot2(h0, xp[m][gi][4 * i + 0], acc[m], false);
          acc[m] = __builtin_amdgcn_fdot2(h1, xp[m][gi][4 * i + 1], acc[m], false);
          acc[m] = __builtin_amdgcn_fdot2(h2, xp[m][gi][4 * i + 2], acc[m], false);
          acc[m] = __builtin_amdgcn_fdot2(h3, xp[m][gi][4 * i + 3], acc[m], false);
        }
      }
#pragma unroll
      for (int m = 0; m < MR; ++m) y[m] = gi ? __builtin_fmaf(acc[m], r.s[gi], y[m]) : acc[m] * r.s[gi];
    }
  };

  // X is requested first, then the first EARLY weight rows: loads complete in
  // issue order, so the X pairs and corrections below are computed while
  // the weights are still in flight.  Buffer loads: rows m >= M and chunks
  // past K read as zeros, with no branch around them.
  rsrc_t rx[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m)
    rx[m] = make_rsrc(a.X + (int64_t)(m < a.M ? m : 0) * a.ldx, m < a.M ? (uint32_t)a.K * 2 : 0u);
  half8v xr[MR][GI][4];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int gi = 0; gi < GI; ++gi)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xr[m][gi][i] = buf_load_half8(rx[m], (uint32_t)(32 * (lane + 64 * gi) + 8 * i) * 2u);

  // Wave w handles rows w + k*T, k < R, in straight-line code (a loop
  // back-edge makes the compiler drain every outstanding load).  A ring of
  // PF rows is in flight.  Rows past N read zeros and their (lane-0) stores
  // fall outside ry.
  // The first EARLY rows are requested before the X work below and the rest
  // of the ring after it, pinned there by scheduling barriers (all rows up
  // front only queues behind the first two; this order measured fastest).
  constexpr int PF = R < 4 ? R : 4;
  constexpr int EARLY = PF < 2 ? PF : 2;
  GemvRow<GI> ring[PF];
#pragma unroll
  for (int k = 0; k < EARLY; ++k) load_row(ring[k], wid + k * T);

  // Chunk sums for the corrections with v_dot2 against (1, 1).
  const half2v ones = {(half_t)1, (half_t)1};
#pragma unroll
  for (int m = 0; m < MR; ++m) {
#pragma unroll
    for (int gi = 0; gi < GI; ++gi) {
      float sa = 0.f, sb = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half8v x = xr[m][gi][i];
        xp[m][gi][4 * i + 0] = half2v{x[0], x[4]};
        xp[m][gi][4 * i + 1] = half2v{x[1], x[5]};
        xp[m][gi][4 * i + 2] = half2v{x[2], x[6]};
        xp[m][gi][4 * i + 3] = half2v{x[3], x[7]};
        sa = __builtin_amdgcn_fdot2(xp[m][gi][4 * i + 0], ones, sa, false);
        sa = __builtin_amdgcn_fdot2(xp[m][gi][4 * i + 2], ones, sa, false);
        sb = __builtin_amdgcn_fdot2(xp[m][gi][4 * i + 1], ones, sb, false);
        sb = __builtin_amdgcn_fdot2(xp[m][gi][4 * i + 3], ones, sb, false);
      }
      corr[m][gi] = -(1024.f + a.zero) * sa - (64.f + a.zero) * sb;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = EARLY; k < PF; ++k) load_row(ring[k], wid + k * T);
  __builtin_amdgcn_sched_barrier(0);


  rsrc_t ry[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m)
    ry[m] = make_rsrc(a.Y + (int64_t)(m < a.M ? m : 0) * a.ldy, m < a.M ? (uint32_t)a.N * 2 : 0u);
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int n = wid + k * T;
    float y[MR];
    row_dot(ring[k % PF], y);
    if (k + PF < R) load_row(ring[k % PF], n + PF * T);
    const uint32_t off = lane == 0 ? (uint32_t)n * 2u : 0xFFFFFFF0u;
#pragma unroll
    for (int m = 0; m < MR; ++m)
      __builtin_amdgcn_raw_buffer_store_b16(
          __builtin_bit_cast(uint16_t, (half_t)wave_sum_dpp(y[m])), ry[m], off, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// Skinny-M regime (3 <= M <= 64 by default): split-K MFMA.
//
// A workgroup owns 16*NT rows of W (output columns n) and 16*MT rows of X.
// Its WV waves split K into contiguous ranges of chunk quads (a quad = 4
// chunks = 128 codes) and reduce their partial tiles through LDS, so the
// grid has N / (16*NT) workgroups per 16*MT rows of X and no wave walks all
// of K.
//
// v_mfma_f32_16x16x32_f16, one MFMA per chunk (one scale group when
// group = 32).  Lane (n = l%16, g = l/16) loads the 16-byte word quad of
// chunk 4q + g of row n (coalesced), then a 4x4 transpose across the four
// 16-lane rows (v_permlane32_swap, v_permlane16_swap) leaves register t
// holding word g of chunk 4q + t.  MFMA t takes that word as its B column
// slice, so lane (m, g) supplies X[m][32(4q+t) + 8g + {0,4,1,5,2,6,3,7}]:
// four lanes read 64 contiguous bytes of each X row per load.  Words are
// dequantised and scaled in fp16 before the MFMA: (c - z) * s, one rounding.
// Out-of-range rows and chunks are zero-filled by the buffer bounds check
// (chunks past the wave's range get an out-of-range offset).
template <int MT, int NT, int WV, bool G32>
__global__ __launch_bounds__(WV * kWave) void w4a16_skinny_kernel(W4Args a) {
  constexpr int QB = 2;                   // quads per batch
  constexpr uint32_t kOut = 0x80000000u;  // offset past every buffer
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * (16 * NT);
  const int m0 = blockIdx.y * (16 * MT);
  const int KW = a.K >> 3, SG = a.K / a.group, C = a.K >> 5;
  const int Q = (C + 3) >> 2;
  const int QW = (Q + WV - 1) / WV;
  const int q0 = wave * QW;
  const int q1 = min(q0 + QW, Q);
  const int cend = min(4 * q1, C);
  const int nrows = min(16 * NT, a.N - n0);
  const int mrows = min(16 * MT, a.M - m0);
  const rsrc_t rw = make_rsrc(a.W + (int64_t)n0 * KW, (uint32_t)nrows * (uint32_t)KW * 4u);
  const rsrc_t rs = make_rsrc(a.S + (int64_t)n0 * SG, (uint32_t)nrows * (uint32_t)SG * 2u);
  const rsrc_t rx = make_rsrc(a.X + (int64_t)m0 * a.ldx,
                              (uint32_t)(((int64_t)(mrows - 1) * a.ldx + a.K) * 2));
  const ZeroPoint zp = zero_point(a.zero);
  const Nibbles nib = nibble_consts();
  const uint32_t gm = (uint32_t)a.group >> 5;  // chunks per scale group
  const bool gpow2 = (gm & (gm - 1)) == 0;
  const uint32_t gshift = __builtin_ctz(gm);

  struct Batch {
    half8v x[QB][MT][4];  // [quad][m tile][chunk t]
    uint4v w[QB][NT];     // [quad][n tile]: word quad of chunk 4q + l/16
    half4v s[QB][NT];     // scales of chunks 4q .. 4q+3 of row n
  };
  // Offsets are computed unconditionally and OR-ed with kOut when the chunk
  // is outside the wave's range (in-range offsets are below 2^31), so every
  // load is issued without a branch.
  auto load = [&](Batch& b, int q) {
#pragma unroll
    for (int qi = 0; qi < QB; ++qi) {
      const uint32_t cq = 4 * (q + qi);  // first chunk of the quad
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const uint32_t row = 16 * nt + li;
        // Word quad of chunk cq + lg; the transpose happens at compute time.
        const uint32_t c = cq + lg;
        const uint32_t wo = (row * (uint32_t)KW * 4u + c * 16u) | ((int)c < cend ? 0u : kOut);
        b.w[qi][nt] = __builtin_bit_cast(
            uint4v, __builtin_amdgcn_raw_buffer_load_b128(rw, wo, 0, kNonTemporal));
        if constexpr (G32) {
          // Scales of chunks cq .. cq+3 are contiguous and 8-byte aligned
          // (the launcher picks this path only for group 32 and K % 128 == 0).
          const uint32_t so = ((row * (uint32_t)SG + cq) * 2u) | ((int)cq < cend ? 0u : kOut);
          b.s[qi][nt] = __builtin_bit_cast(
              half4v, __builtin_amdgcn_raw_buffer_load_b64(rs, so, 0, kNonTemporal));
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t ct = cq + t;
            const uint32_t sidx = gpow2 ? ct >> gshift : ct / gm;
            const uint32_t so = ((row * (uint32_t)SG + sidx) * 2u) | ((int)ct < cend ? 0u : kOut);
            b.s[qi][nt][t] = __builtin_bit_cast(
                half_t, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, so, 0, kNonTemporal));
          }
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t ct = cq + t;
          const uint32_t xo = (((16 * mt + li) * (uint32_t)a.ldx + 32u * ct + 8u * lg) * 2u) |
                              ((int)ct < cend ? 0u : kOut);
          b.x[qi][mt][t] = buf_load_half8(rx, xo);
        }
      }
    }
  };

  float4v acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = float4v{};

  auto compute = [&](Batch& b) {
#pragma unroll
    for (int qi = 0; qi < QB; ++qi) {
      half8v xa[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const half8v x = b.x[qi][mt][t];
          xa[mt][t] = half8v{x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]};
        }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        // Word j of chunk cq + l/16  ->  word l/16 of chunk cq + t.
        uint32_t wt[4] = {b.w[qi][nt][0], b.w[qi][nt][1], b.w[qi][nt][2], b.w[qi][nt][3]};
        transpose_rows4(wt[0], wt[1], wt[2], wt[3]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const half_t s = b.s[qi][nt][t];
          const half2v s1 = {s, s};
          half2v r[4];
          unpack_word(wt[t], nib, zp, r);
          const half2v d0 = r[0] * s1, d1 = r[1] * s1, d2 = r[2] * s1, d3 = r[3] * s1;
          const half8v bv = {d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma16x16x32(xa[mt][t], bv, acc[mt][nt]);
        }
      }
    }
  };

  // Two batches in flight; loads past the wave's range read zeros.
  Batch bA, bB;
  load(bA, q0);
  for (int q = q0; q < q1; q += 2 * QB) {
    load(bB, q + QB);
    compute(bA);
    load(bA, q + 2 * QB);
    compute(bB);
  }

  // Reduce the waves' partial tiles.  acc[mt][nt] register r of lane l is
  // D[16mt + 4(l/16) + r][16nt + l%16].
  __shared__ float red[WV][MT * NT * 4][kWave];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][(mt * NT + nt) * 4 + r][lane] = acc[mt][nt][r];
  lds_barrier();
  for (int e = threadIdx.x; e < MT * NT * 4 * kWave; e += WV * kWave) {
    const int slot = e / kWave, ln = e % kWave;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < WV; ++w) v += red[w][slot][ln];
    const int mt = slot / (NT * 4), nt = (slot / 4) % NT, r = slot % 4;
    const int m = m0 + 16 * mt + 4 * (ln >> 4) + r;
    const int n = n0 + 16 * nt + (ln & 15);
    if (m < a.M && n < a.N) a.Y[(int64_t)m * a.ldy + n] = (half_t)v;
  }
}

// ---------------------------------------------------------------------------
// Large-M regime (M > 64): LDS-tiled GEMM.
//
// A workgroup computes a 128 (m) x 128 (n) tile of Y with WM x WN waves
// (2 x 4 by default: 64 x 32 each, two v_mfma_f32_32x32x16_f16 tiles, two
// waves per SIMD so that one wave's dequantisation and LDS reads overlap the
// other's MFMAs).
// Per K-step of 64 codes:
//   * the X tile (128 x 64 fp16) goes through registers into LDS with
//     coalesced 16-byte loads, each 8-element group stored in the order
//     {0,4,1,5,2,6,3,7} of unpack_word; rows padded to 72 halves so the
//     ds_read_b128 fragment reads are conflict-free;
//   * W never touches LDS: lane (n = l%32, h = l/32) of a wave loads the
//     16-byte word quad h (chunk k0/32 + h) of each of its 32-row column
//     tiles and dequantises word ks of it as the B operand of MFMA
//     k-substep ks, so that MFMA's k-block h holds codes
//     k0 + 32h + 8ks + {0,4,1,5,2,6,3,7}.  Each W word is dequantised by
//     the WM waves that share its columns; LDS traffic per step is the X
//     tile once in and one A-fragment read per wave and MFMA row tile.
// W loads run kRingW steps ahead (HBM latency), X loads two steps ahead
// (L2), LDS is double-buffered with one barrier per step.
constexpr int kGBM = 128, kGBK = 64, kGLD = kGBK + 8;
constexpr int kRingW = 8;

template <int WM, int WN, int kGBN>
__global__ __launch_bounds__(WM * WN * kWave) void w4a16_gemm_kernel(W4Args a) {
  constexpr int kT = WM * WN * kWave;       // threads
  constexpr int MI = kGBM / WM / 32;        // 32-row MFMA tiles per wave
  constexpr int NT = kGBN / WN / 32;        // 32-column MFMA tiles per wave
  constexpr int XJ = kGBM * kGBK / 8 / kT;  // 16-byte X pieces per thread per step
  constexpr uint32_t kOut = 0x80000000u;
  __shared__ half8v xs[2][kGBM * kGLD / 8];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 31, lh = lane >> 5;
  const int mtiles = (a.M + kGBM - 1) / kGBM;
  const int ntiles = (a.N + kGBN - 1) / kGBN;
  const int id = (int)xcd_swizzle(blockIdx.x, (uint32_t)(mtiles * ntiles));
  const int m0 = (id % mtiles) * kGBM, n0 = (id / mtiles) * kGBN;
  const int KW = a.K >> 3, SG = a.K / a.group;
  const int mrows = min(kGBM, a.M - m0);
  // This wave's first W row and row count, forced into SGPRs: computed on
  // the VALU, the compiler would otherwise treat the buffer descriptors
  // built from them as divergent and wrap every load in a waterfall loop.
  const int nw0 = __builtin_amdgcn_readfirstlane(n0 + 32 * NT * wn);
  const int nwrows = __builtin_amdgcn_readfirstlane(max(0, min(32 * NT, a.N - nw0)));
  const rsrc_t rx = make_rsrc(a.X + (int64_t)m0 * a.ldx, (uint32_t)(((int64_t)(mrows - 1) * a.ldx + a.K) * 2));
  const rsrc_t rw = make_rsrc(a.W + (int64_t)(nwrows ? nw0 : 0) * KW, (uint32_t)nwrows * KW * 4u);
  const rsrc_t rs = make_rsrc(a.S + (int64_t)(nwrows ? nw0 : 0) * SG, (uint32_t)nwrows * SG * 2u);
  const ZeroPoint zp = zero_point(a.zero);
  const Nibbles nib = nibble_consts();
  const uint32_t gm = (uint32_t)a.group >> 5;
  const bool gpow2 = (gm & (gm - 1)) == 0;
  const uint32_t gshift = __builtin_ctz(gm);

  // X: rows tid/8 + (kT/8)j, 16-byte piece tid%8 of the step.
  const int xr0 = tid >> 3, xp = tid & 7;
  struct XStage {
    half8v v[XJ];
  };
  struct WStage {
    uint4v w[NT];
    half_t s[NT];
  };
  auto load_x = [&](XStage& g, int k0) {
    const uint32_t oob = k0 + 8 * xp < a.K ? 0u : kOut;
#pragma unroll
    for (int j = 0; j < XJ; ++j)
      g.v[j] = buf_load_half8(rx, (((uint32_t)(xr0 + kT / 8 * j) * a.ldx + k0 + 8 * xp) * 2u) | oob);
  };
  auto load_w = [&](WStage& g, int k0) {
    const uint32_t chunk = (uint32_t)(k0 >> 5) + lh;
    const uint32_t oob = (int)(32 * chunk) < a.K ? 0u : kOut;
    const uint32_t sidx = gpow2 ? chunk >> gshift : chunk / gm;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint32_t row = 32 * nt + li;
      g.w[nt] = __builtin_bit_cast(uint4v, __builtin_amdgcn_raw_buffer_load_b128(
                                               rw, (row * KW * 4u + chunk * 16u) | oob, 0, 0));
      g.s[nt] = __builtin_bit_cast(half_t, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(
                                               rs, ((row * SG + sidx) * 2u) | oob, 0, 0));
    }
  };
  auto store_x = [&](const XStage& g, int buf) {
#pragma unroll
    for (int j = 0; j < XJ; ++j) {
      const half8v x = g.v[j];
      xs[buf][((xr0 + kT / 8 * j) * kGLD + 8 * xp) / 8] =
          half8v{x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]};
    }
  };

  float16v acc[MI][NT];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mi][nt] = float16v{};

  auto compute = [&](const WStage& g, int buf) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const half2v s1 = {g.s[nt], g.s[nt]};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        half2v r[4];
        unpack_word(g.w[nt][ks], nib, zp, r);
        const half2v d0 = r[0] * s1, d1 = r[1] * s1, d2 = r[2] * s1, d3 = r[3] * s1;
        const half8v bfr = {d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          const half8v afr =
              xs[buf][((32 * MI * wm + 32 * mi + li) * kGLD + 32 * lh + 8 * ks) / 8];
          acc[mi][nt] = mfma32x32x16(afr, bfr, acc[mi][nt]);
        }
      }
    }
  };

  // Loads past K read zeros; the trailing steps of the last ring turn
  // compute on zeros.
  const int nsteps = (a.K + kGBK - 1) / kGBK;
  XStage xr[2];
  WStage wr[kRingW];
  load_x(xr[0], 0);
  load_x(xr[1], kGBK);
#pragma unroll
  for (int u = 0; u < kRingW; ++u) load_w(wr[u], u * kGBK);
  store_x(xr[0], 0);
  lds_barrier();
  for (int st = 0; st < nsteps; st += kRingW) {
#pragma unroll
    for (int u = 0; u < kRingW; ++u) {
      const int s = st + u;
      load_x(xr[u & 1], (s + 2) * kGBK);
      compute(wr[u], u & 1);
      load_w(wr[u], (s + kRingW) * kGBK);
      store_x(xr[(u + 1) & 1], (u + 1) & 1);
      lds_barrier();
    }
  }

  // acc[mi][nt] register r: row 32(MI wm + mi) + 8(r/4) + 4(lane/32) + r%4,
  // column 32(NT wn + nt) + lane%32.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = nw0 + 32 * nt + li;
    if (n >= a.N) continue;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 32 * MI * wm + 32 * mi + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m < a.M) a.Y[(int64_t)m * a.ldy + n] = (half_t)acc[mi][nt][r];
      }
  }
}

// ---------------------------------------------------------------------------
// Tile GEMM (M > 16, and smaller M past the skinny kernels' K; the
// launcher picks the finest tile whose grid fits on the CUs).
//
// A workgroup computes a 32 MI (m) x 32 WN (n) tile of Y with KG K-groups of
// WN waves; group g takes the contiguous range of K-steps [g T, (g + 1) T)
// (64 codes per step) in its own LDS buffers, and the groups' partial tiles
// are summed through LDS at the end.  Wave w of a group owns columns
// 32 w .. 32 w + 31 of the tile for all its rows (MI x 1
// v_mfma_f32_32x32x16_f16 tiles), so no two waves of a group need the same
// weights and each code is dequantised once per workgroup:
//   * W: lane (n = l%32, h = l/32) loads word quad h (32 codes, 16 bytes,
//     one scale group) of its row's step and its scale, and dequantises
//     (c - z) * s (one fp16 rounding) straight into MFMA B operands: MFMA
//     ks of the step takes word ks, i.e. codes 32 h + 8 ks + {0,4,1,5,2,6,
//     3,7}, the order of unpack_word_x16;
//   * X: the tile (32 MI x 64 fp16 per step) goes through LDS, each
//     8-element group stored in that nibble order, rows padded to 72 halves
//     (no bank conflicts); thread t loads 16-byte piece t%8 of rows
//     t/8 + 8 WN j.  A wave's A fragment for MFMA (mi, ks) is row
//     32 mi + l%32 at codes 32 h + 8 ks of the step, one ds_read_b128.
// Per step and wave: 4 MI MFMAs, 4 MI fragment reads, 4 dequantised words
// and 4 MI / WN X stores.  Only X is stored to LDS; that store stream (LDS
// writes run at about a third of the read rate on gfx950) was the cost of
// the earlier form, which dequantised W into LDS too.  LDS is
// double-buffered per group; X loads run two steps ahead of their store, W
// loads two steps ahead of their use; the next step's X stores are issued
// among the current step's MFMAs.  One sync per step: a workgroup barrier,
// a per-group LDS arrival counter, or for one-wave groups a wave-level
// fence (step_sync below).
constexpr int kTT = 128, kTK = 64, kTLD = kTK + 8;

// K-groups per workgroup, waves (32-column strips) per group, 32-row MFMA
// tiles per wave (tile rows 32 MI).
template <int kTKG, int WN = 4, int MI = 4>
__global__ __launch_bounds__(64 * WN * kTKG) void w4a16_tile_gemm_kernel(W4Args a) {
  static_assert(WN == 1 || WN == 2 || WN == 4, "waves per group");
  static_assert(MI == 1 || MI == 2 || MI == 4, "32-row tiles per wave");
  constexpr uint32_t kOut = 0x80000000u;  // buffer offset past any extent: loads return 0
  constexpr int TM = 32 * MI;             // tile rows
  constexpr int kBuf = TM * kTLD / 8;     // half8v per LDS tile
  constexpr int GT = 64 * WN;             // threads per group
  constexpr int TN = 32 * WN;             // tile columns
  constexpr int XP = 4 * MI / WN;         // X pieces per thread and step
  constexpr int XPK = (XP + 3) / 4;       // X pieces stored per k-slice of a step
  static_assert(XP >= 1 && XP * GT == TM * 8, "X pieces");
  __shared__ half8v lds[kTKG][2][kBuf];   // [group][buffer] X tile
  __shared__ uint32_t arrivals[kTKG];      // per-group arrival counters
  const int tid = threadIdx.x % GT, lane = tid & 63;
  const int kg = __builtin_amdgcn_readfirstlane(threadIdx.x / GT);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 31, lh = lane >> 5;
  const int mtiles = (a.M + TM - 1) / TM;
  const int ntiles = (a.N + TN - 1) / TN;
  const int id = (int)xcd_swizzle(blockIdx.x, (uint32_t)(mtiles * ntiles));
  const int m0 = (id % mtiles) * TM, n0 = (id / mtiles) * TN;
  const int KW = a.K >> 3, SG = a.K / a.group;
  const int mrows = __builtin_amdgcn_readfirstlane(min(TM, a.M - m0));
  const int nrows = __builtin_amdgcn_readfirstlane(min(TN, a.N - n0));
  const rsrc_t rx = make_rsrc(a.X + (int64_t)m0 * a.ldx, (uint32_t)(((int64_t)(mrows - 1) * a.ldx + a.K) * 2));
  const rsrc_t rw = make_rsrc(a.W + (int64_t)n0 * KW, (uint32_t)nrows * KW * 4u);
  const rsrc_t rs = make_rsrc(a.S + (int64_t)n0 * SG, (uint32_t)nrows * SG * 2u);
  const ZeroPoint zp = zero_point(a.zero);
  const Nibbles nib = nibble_consts();
  const uint32_t gm = (uint32_t)a.group >> 5;  // 32-code chunks per scale group
  const bool gpow2 = (gm & (gm - 1)) == 0;
  const uint32_t gshift = __builtin_ctz(gm);
  // Steps per group (every group runs the same count, as the workgroup
  // barriers require); steps past K read zeros.
  const int T = ((a.K + kTK - 1) / kTK + kTKG - 1) / kTKG;

  // X: row tid/8 + 8 WN j, 16-byte piece tid%8 of the step.  W: row
  // 32 wave + li of the tile, word quad lh of the step.
  const int xr0 = tid >> 3, xp = tid & 7;
  const int wrow = 32 * wave + li;
  struct XStage {
    half8v x[XP];
  };
  struct WStage {
    uint4v w;
    half_t s;
  };
  auto xload = [&](XStage& g, int t) {
    const int k = (kg * T + t) * kTK + 8 * xp;
    const uint32_t xoob = k < a.K ? 0u : kOut;
#pragma unroll
    for (int j = 0; j < XP; ++j)
      g.x[j] = buf_load_half8(rx, (((uint32_t)(xr0 + 8 * WN * j) * a.ldx + k) * 2u) | xoob);
  };
  auto wload = [&](WStage& g, int t) {
    const uint32_t chunk = (uint32_t)((kg * T + t) * (kTK / 32)) + lh;
    const uint32_t woob = (int)(32 * chunk) < a.K ? 0u : kOut;
    const uint32_t sidx = gpow2 ? chunk >> gshift : chunk / gm;
    g.w = __builtin_bit_cast(uint4v, __builtin_amdgcn_raw_buffer_load_b128(
                                         rw, ((uint32_t)wrow * KW * 4u + chunk * 16u) | woob, 0, 0));
    g.s = __builtin_bit_cast(half_t, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(
                                         rs, (((uint32_t)wrow * SG + sidx) * 2u) | woob, 0, 0));
  };
  auto xstore = [&](const XStage& g, int buf, int j) {
    const half8v x = g.x[j];
    lds[kg][buf][((xr0 + 8 * WN * j) * kTLD + 8 * xp) / 8] = half8v{x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]};
  };

  float16v acc[MI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) acc[mi] = float16v{};

  // One step: X from LDS buffer buf, W from registers ws; X stage xn (the
  // next step) stored into buffer buf ^ 1 among the MFMAs.  After the last
  // step the stage holds the zeros loaded past K; storing them into the
  // idle buffer is harmless and keeps the step one basic block.
  auto step = [&](int buf, const WStage& ws, const XStage& xn) {
    const half8v* xb = lds[kg][buf];
    auto afrag = [&](int mi, int ks) { return xb[((32 * mi + li) * kTLD + 32 * lh + 8 * ks) / 8]; };
    const half2v s1 = {ws.s, ws.s};
    const half_t s16v = ws.s * (half_t)0.0625f;
    const half2v s16 = {s16v, s16v};
    half8v af[2][MI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) af[0][mi] = afrag(mi, 0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int c = ks & 1;
      if (ks + 1 < 4) {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) af[c ^ 1][mi] = afrag(mi, ks + 1);
      }
      half2v r[4];
      unpack_word_x16(ws.w[ks], nib, zp, r);
      const half2v d0 = r[0] * s1, d1 = r[1] * s16, d2 = r[2] * s1, d3 = r[3] * s16;
      const half8v bop = half8v{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) acc[mi] = mfma32x32x16(af[c][mi], bop, acc[mi]);
#pragma unroll
      for (int j = 0; j < XPK; ++j)
        if (XPK * ks + j < XP) xstore(xn, buf ^ 1, XPK * ks + j);
    }
  };

  // The end of a step: every wave of the group has stored its share of the
  // next X tile and read its last fragment of this one.  Only the group's
  // waves share those buffers, so with a.group_sync each wave counts
  // itself in the group's LDS arrival counter and waits for the group's
  // count (WN per sync), letting the groups drift apart; the two waves
  // that share a SIMD then overlap one's MFMAs with the other's loads and
  // stores.  The wait is bounded: it ends after 2^16 polls whatever it
  // reads (a group's waves are resident together and each adds itself
  // before it waits, so a real wait ends long before).
  // A group of one wave (WN = 1) needs no other wave: LDS executes one
  // wave's instructions in order, so a wave-level fence that keeps the
  // compiler from moving LDS accesses across the step is enough (K = 11008
  // N = 4096 M = 32: 23.8 us against 25.5 with the workgroup barrier and
  // 24.5 with the counter).
  uint32_t syncs = 0;
  auto step_sync = [&]() {
    if constexpr (WN == 1 && kTKG > 1) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      return;
    }
    if (kTKG == 1 || !a.group_sync) {
      lds_barrier();
      return;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    if (lane == 0) __hip_atomic_fetch_add(&arrivals[kg], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const uint32_t target = (uint32_t)WN * ++syncs;
    for (int i = 0; i < (1 << 16); ++i) {
      const uint32_t seen = __builtin_amdgcn_readfirstlane(
          __hip_atomic_load(&arrivals[kg], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
      if (seen >= target) break;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  };

  XStage x0, x1;
  WStage w0, w1;
  xload(x0, 0);
  wload(w0, 0);
  xload(x1, 1);
  wload(w1, 1);
#pragma unroll
  for (int j = 0; j < XP; ++j) xstore(x0, 0, j);
  xload(x0, 2);
  if (threadIdx.x < kTKG) arrivals[threadIdx.x] = 0;
  lds_barrier();
  // Step t: W stage t&1, X buffer t&1; X stage (t+1)&1 stored into buffer
  // (t+1)&1 and reloaded with step t+3; W stage t&1 reloaded with step t+2.
  // Unrolled by two so the stages swap roles without copies.
  for (int t0 = 0; t0 < T; t0 += 2) {
    step(0, w0, x1);
    wload(w0, t0 + 2);
    xload(x1, t0 + 3);
    step_sync();
    if (t0 + 1 < T) {
      step(1, w1, x0);
      wload(w1, t0 + 3);
      xload(x0, t0 + 4);
      step_sync();
    }
  }

  // Sum the groups' partial tiles into group 0, one group at a time in group
  // order.  The partials overwrite every group's X buffers: the first
  // barrier waits for the last group to finish its loop.
  if constexpr (kTKG > 1) {
    lds_barrier();
    static_assert(sizeof(lds) >= (size_t)WN * MI * 16 * 64 * sizeof(float), "reduction buffer");
    float* red = reinterpret_cast<float*>(lds) + (size_t)wave * MI * 16 * 64 + lane;
#pragma unroll
    for (int g = 1; g < kTKG; ++g) {
      if (g > 1) lds_barrier();
      if (kg == g) {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int r = 0; r < 16; ++r) red[(mi * 16 + r) * 64] = acc[mi][r];
      }
      lds_barrier();
      if (kg == 0) {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[mi][r] += red[(mi * 16 + r) * 64];
      }
    }
    if (kg != 0) return;
  }

  // acc[mi] register r: row 32 mi + 8(r/4) + 4 lh + r%4, column
  // 32 wave + li of the tile at (m0, n0).  Rows past M fall outside the
  // buffer resource (ldy >= N >= n0 + nrows); columns past N get an
  // out-of-range offset.
  const rsrc_t ry = make_rsrc(a.Y + (int64_t)m0 * a.ldy + n0, (uint32_t)(((int64_t)(mrows - 1) * a.ldy + nrows) * 2));
  const int nl = 32 * wave + li;
  const uint32_t noob = nl < nrows ? 0u : kOut;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ml = 32 * mi + 8 * (r >> 2) + 4 * lh + (r & 3);
      const uint32_t off = (((uint32_t)ml * a.ldy + (uint32_t)nl) * 2u) | noob;
      __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (half_t)acc[mi][r]), ry, off, 0, 0);
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
  const ZeroPoint zp = zero_point(a.zero);
  const Nibbles nib = nibble_consts();

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
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        half2v r[4];
        unpack_word(w[j], nib, zp, r);
        const half2v d0 = r[0] * s1, d1 = r[1] * s1, d2 = r[2] * s1, d3 = r[3] * s1;
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
// W8A16 GEMM: C[M][N] f32 = A[M][K] f16 * f16(B[K][N] int8) [* scale[n]].
//
// Workgroup tile 128 x 128, four waves of 64 x 64 (2 x 2
// v_mfma_f32_32x32x16_f16 tiles), K-steps of kW8BK.  A goes through LDS in
// unpadded rows with a piece swizzle (w8_a_at: conflict-free 16-byte stores
// and ds_read_b128 fragment reads).  B is N-contiguous
// in memory and stays so in LDS: thread (row, column group) loads 32
// contiguous bytes of one k-row, converts them to f16 exactly (int8 -> f16
// via the exponent trick: 0x6400 | (b ^ 0x80) is 1024 + b + 128) and stores
// them as two 16-byte chunks of Bs[k][n]; the MFMA B operand (8 consecutive
// k of one column per lane) comes from gfx950's transposing LDS read,
// ds_read_b64_tr_b16, two per fragment.  (The earlier layout, transposed on
// the way in as (k, k+1) pairs per column, took 16 ds_write_b32 per thread
// and step and was ~10% slower: 176.8 against 160.9 us at 4096^3.)
// Double-buffered LDS, global loads one step ahead.
// K-step 64: 16 MFMAs per wave between barriers (measured at 4096^3 on one
// box: 179.0 us against 181.9 us with K-steps of 32).
constexpr int kW8BK = 64;
constexpr int kW8AP = kW8BK / 32;  // 16-byte A pieces per thread and row half

// LDS banks as the counters show them on gfx950: a 16-byte read
// (ds_read_b128, and the transposing ds_read_b64_tr_b16 by 32 lanes) is
// served 256 bytes at a time over 64 banks, a 16-byte write 128 bytes (8
// lanes) at a time over 32 banks.  The layouts below keep both passes on
// distinct banks (SQ_LDS_BANK_CONFLICT = 0).
//
// A tile: [m][k] f16 rows of kW8BK = 64 halves without padding (8 pieces of
// 16 bytes, 32 banks), piece p of row r at p ^ fa(r), fa(r) = 4 (r & 1) ^
// ((r >> 1) & 7).  A write pass (rows 2i, 2i + 1, pieces 4 j + 0..3) puts
// the two rows on complementary piece halves; a read pass (16 consecutive
// rows, one piece; even rows on banks 0..31, odd rows on 32..63) maps the 8
// rows of each bank half to 8 distinct pieces.
__device__ __forceinline__ int w8_a_at(int r, int p) {
  return r * kW8BK + 8 * (p ^ (4 * (r & 1)) ^ ((r >> 1) & 7));
}

// B tile: [k][n] f16 in 128-column halves, rows of 128 halves (16 chunks of
// 16 bytes, 64 banks); in half hb, chunk c of row r sits at c ^ 2 (c >> 3)
// ^ 5 (r % 4) ^ hb.  A write pass (one row, chunks 4 j + s of column groups
// j = 0..3 in each half) lands on 8 distinct positions mod 8 (bit 3 of c
// folded into bit 1, the second half one position over); a transposed-read
// pass (4 rows r % 4 = 0..3 x chunks 4 u .. 4 u + 3) covers the four
// aligned groups of four positions once each.
__device__ __forceinline__ int w8_b_at(int hb, int r, int c) {
  return (hb * kW8BK + r) * 128 + 8 * (c ^ (2 * (c >> 3)) ^ (5 * (r & 3)) ^ hb);
}
// This lane's offset for the B fragment of column tile u of half hb
// (v_frag_tr's addressing: row 8 (l / 32) + (l % 16) / 4, columns 32 u + 16
// ((l / 16) % 2) + 4 (l % 4)); adding 4 or 16 rows keeps the swizzle.
__device__ __forceinline__ int w8_b_tr_offset(int lane, int hb, int u) {
  const int row = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int cu = 32 * u + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  return w8_b_at(hb, row, cu >> 3) + (cu & 7);
}

// Workgroup tile T x T (T = 128: four waves of 64 x 64; T = 256: eight
// waves of 64 x 128, a third fewer LDS bytes per MFMA), K-steps of kW8BK.
template <int T>
__global__ __launch_bounds__(2 * T) void w8a16_gemm_kernel(W8Args a) {
  constexpr int NT = 2 * T;          // threads
  constexpr int NI = T / 64;         // 32-column MFMA tiles per wave
  constexpr int NH = T / 128;        // 128-column B halves
  __shared__ half8v as[2][T * kW8BK / 8];
  __shared__ __attribute__((aligned(16))) half_t bs[2][NH * kW8BK * 128];  // [half][k][n]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lh = lane >> 5;
  // Tile order: the dispatch index is remapped so that each XCD takes a
  // contiguous run of logical tiles, and logical tiles go down groups of
  // four m-tiles before moving to the next n-tile, so that the workgroups
  // an XCD runs at once share the A rows and B columns its L2 holds.
  const int mt = (int)gridDim.y, nt = (int)gridDim.x;
  const int lid = (int)xcd_swizzle(blockIdx.y * gridDim.x + blockIdx.x, (uint32_t)(mt * nt));
  constexpr int kGroupM = 4;
  const int grp = lid / (kGroupM * nt), first = grp * kGroupM;
  const int gm = min(mt - first, kGroupM), in = lid % (kGroupM * nt);
  const int m0 = (first + in % gm) * T, n0 = (in / gm) * T;
  const int mrows = min(T, a.M - m0);
  constexpr uint32_t kOut = 0x80000000u;
  const rsrc_t ra = make_rsrc(a.A + (int64_t)m0 * a.lda, (uint32_t)(((int64_t)(mrows - 1) * a.lda + a.K) * 2));
  // K >= 1 (the ABI rejects K = 0 with a non-empty output); the extent is
  // clamped at 0 anyway so a bad call cannot wrap it to ~4 GiB.
  const rsrc_t rb = make_rsrc(
      a.B + n0, (uint32_t)max((int64_t)0, (a.K - 1) * (int64_t)a.ldb + min(T, a.N - n0)));
  // A: rows ar + (T/2) j, 16-byte pieces ap + 4p of the step.
  const int ar = tid >> 2, ap = tid & 3;
  // B: k-row br of the step, columns 32 bc .. 32 bc + 31 (two 16-byte
  // pieces; four or eight lanes read a row's contiguous bytes).
  static_assert(kW8BK * T == 32 * NT, "one 32-byte row piece per thread");
  constexpr int BG = T / 32;  // column groups per row
  const int br = tid / BG, bc = tid % BG;
  const uint32_t nlim = (uint32_t)min(T, a.N - n0);
  struct Stage {
    half8v av[2][kW8AP];
    uint4v b[2];  // 16 int8 of row br, columns 32 bc + 16 h ..
  };
  auto load = [&](Stage& g, int k0) {
#pragma unroll
    for (int p = 0; p < kW8AP; ++p) {
      const int kc = k0 + 8 * (ap + 4 * p);
      const uint32_t aoob = kc < a.K ? 0u : kOut;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        g.av[j][p] = buf_load_half8(ra, (((uint32_t)(ar + (T / 2) * j) * a.lda + kc) * 2u) | aoob);
    }
    // Pieces wholly past N are masked; a piece that straddles N (N % 16 =
    // 8) reads bytes of columns >= N, whose products only reach columns of
    // C that are never stored.  Rows past K fall outside the buffer.
    const int k = k0 + br;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t col = 32u * bc + 16u * h;
      g.b[h] = __builtin_bit_cast(
          uint4v, __builtin_amdgcn_raw_buffer_load_b128(
                      rb, ((uint32_t)k * a.ldb + col) | (k < a.K && col < nlim ? 0u : kOut), 0, 0));
    }
  };
  const uint32_t magic = vgpr_const(0x64006400u);
  const half2v bias = {(half_t)1152, (half_t)1152};
  auto store = [&](const Stage& g, int buf) {
#pragma unroll
    for (int p = 0; p < kW8AP; ++p)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        as[buf][w8_a_at(ar + (T / 2) * j, ap + 4 * p) / 8] = g.av[j][p];
    // Row br as f16 in [k][n] order: bytes (n, n+1) of a word -> one f16
    // pair; chunk c of the row at w8_b_at.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t pr[8];
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        const uint32_t x = g.b[h][wd] ^ 0x80808080u;
        pr[2 * wd] = __builtin_amdgcn_perm(0u, x, 0x0c010c00u) | magic;
        pr[2 * wd + 1] = __builtin_amdgcn_perm(0u, x, 0x0c030c02u) | magic;
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        half8v v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const half2v hp = __builtin_bit_cast(half2v, pr[4 * c + j]) - bias;
          v[2 * j] = hp[0];
          v[2 * j + 1] = hp[1];
        }
        const int chunk = 4 * bc + 2 * h + c;  // of the T-wide row
        *reinterpret_cast<half8v*>(&bs[buf][w8_b_at(chunk >> 4, br, chunk & 15)]) = v;
      }
    }
  };

  float16v acc[2][NI];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = float16v{};
  // Wave (wm, wn) computes rows 64 wm .. and columns (T/2) wn ..: with T =
  // 256 that is half wn of the B tile, with T = 128 tiles 2 wn, 2 wn + 1.
  const int hb = NH == 2 ? wn : 0;
  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < kW8BK / 16; ++ks) {
      half8v bf[NI];
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        bf[ni] = v_frag_tr<128>(bs[buf], w8_b_tr_offset(lane, hb, NH == 2 ? ni : 2 * wn + ni), ks);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const half8v af = as[buf][w8_a_at(64 * wm + 32 * mi + li, 2 * ks + lh) / 8];
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = mfma32x32x16(af, bf[ni], acc[mi][ni]);
      }
    }
  };

  const int nsteps = (a.K + kW8BK - 1) / kW8BK;
  Stage sA, sB;
  load(sA, 0);
  store(sA, 0);
  load(sB, kW8BK);
  lds_barrier();
  for (int st = 0; st < nsteps; st += 2) {
    load(sA, (st + 2) * kW8BK);  // past K: zeros
    compute(0);
    store(sB, 1);
    lds_barrier();
    load(sB, (st + 3) * kW8BK);
    compute(1);
    store(sA, 0);
    lds_barrier();
  }

  // acc[mi][ni] register r: row 64wm + 32mi + 8(r/4) + 4(lane/32) + r%4,
  // column (T/2) wn + 32ni + lane%32.
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int n = n0 + (T / 2) * wn + 32 * ni + li;
    if (n >= a.N) continue;
    const float s = a.scale ? (float)a.scale[n] : 1.f;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 64 * wm + 32 * mi + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m < a.M) a.C[(int64_t)m * a.ldc + n] = acc[mi][ni][r] * s;
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

template <int MR, int R>
hipError_t launch_gemv_r(const W4Args& a, hipStream_t s) {
  const int waves = (a.N + R - 1) / R;
  int blocks = (waves + 3) / 4;
  // Round a grid of more than one workgroup per CU up to whole rounds, so
  // every CU holds the same number of workgroups (the extra waves' rows lie
  // past N and read nothing): N = 11008, 688 -> 768 workgroups, 6.59 ->
  // 6.52 us.
  const int cus = device_cu_count();
  if (blocks > cus) blocks = (blocks + cus - 1) / cus * cus;
  const int G = a.K / 32;
  if (G <= 64)
    return launch<&w4a16_gemv_kernel<MR, 1, R, false>>(
        ktag("w4a16_gemv_kernel", MR, 1, R, false), dim3(blocks), dim3(kThreads), s, a);
  if (G <= 128 && a.group == 32 && G % 2 == 0)  // whole 4-byte scale pairs
    return launch<&w4a16_gemv_kernel<MR, 2, R, true>>(
        ktag("w4a16_gemv_kernel", MR, 2, R, true), dim3(blocks), dim3(kThreads), s, a);
  if (G <= 128)
    return launch<&w4a16_gemv_kernel<MR, 2, R, false>>(
        ktag("w4a16_gemv_kernel", MR, 2, R, false), dim3(blocks), dim3(kThreads), s, a);
  if (G <= 256)
    return launch<&w4a16_gemv_kernel<MR, 4, R, false>>(
        ktag("w4a16_gemv_kernel", MR, 4, R, false), dim3(blocks), dim3(kThreads), s, a);
  return hipErrorInvalidValue;
}

template <int MR>
hipError_t launch_gemv_mr(const W4Args& a, hipStream_t s) {
  // Rows per wave: 4 (all four in flight from the start) unless the grid
  // would then leave SIMDs without a wave; 8 only for very tall matrices.
  // NESO_AMD_GEMV_ROWS_PER_WAVE overrides.
  static const int forced = [] {
    const char* v = getenv("NESO_AMD_GEMV_ROWS_PER_WAVE");
    const int k = v ? atoi(v) : 0;
    return (k == 2 || k == 4 || k == 8) ? k : 0;
  }();
  const int simds = 4 * device_cu_count();
  int r = forced;
  if (!r) r = a.N < 4 * simds ? 2 : (a.N <= 16 * simds ? 4 : 8);
  if (r == 2) return launch_gemv_r<MR, 2>(a, s);
  if (r == 4) return launch_gemv_r<MR, 4>(a, s);
  return launch_gemv_r<MR, 8>(a, s);
}

}  // namespace

int w4a16_gemv_max_k() { return 32 * 256; }

#ifndef NESO_SKINNY_WAVES
#define NESO_SKINNY_WAVES 4
#endif
constexpr int kSkinnyWaves = NESO_SKINNY_WAVES;

hipError_t launch_w4a16(const W4Args& a, hipStream_t s) {
  // GEMV regime up to M = 2.  From M = 3 the skinny MFMA kernel is faster
  // (K = 4096, N = 11008, GEMV / MFMA: M = 1 6.6 / 8.7 us, M = 2 8.6 / 8.7,
  // M = 3 11.1 / 8.7, M = 4 13.8 / 8.7).  NESO_AMD_W4_GEMV_MAX_M = 0..4
  // overrides the largest GEMV M.
  // Values outside 0..4 fall back to the default: the GEMV kernels hold
  // at most four rows of X.
  const char* gemv_env = getenv("NESO_AMD_W4_GEMV_MAX_M");
  const int gemv_env_m = gemv_env ? atoi(gemv_env) : -1;
  const int gemv_max_m = (gemv_env_m >= 0 && gemv_env_m <= 4) ? gemv_env_m : 2;
  if (a.M <= gemv_max_m && a.K <= w4a16_gemv_max_k()) {
    switch (a.M) {
      case 1: return launch_gemv_mr<1>(a, s);
      case 2: return launch_gemv_mr<2>(a, s);
      case 3: return launch_gemv_mr<3>(a, s);
      default: return launch_gemv_mr<4>(a, s);
    }
  }
  // Skinny regime: buffer offsets of one workgroup's X rows and W rows must
  // stay below 2^31 bytes (the out-of-range marker).
  const bool skinny_fits = (int64_t)32 * a.ldx * 2 + (int64_t)a.K * 2 < ((int64_t)1 << 31) &&
                           (int64_t)32 * a.K / 2 < ((int64_t)1 << 31);
  // Tile GEMM: its buffer offsets (one tile's X rows, W rows and scales)
  // must stay below 2^31 bytes.
  const bool tile_fits = (int64_t)kTT * a.ldx * 2 + (int64_t)a.K * 2 < ((int64_t)1 << 31) &&
                         (int64_t)kTT * a.K / 2 < ((int64_t)1 << 31);
  // Its form: the finest of 32 x 32 (eight K-groups of one wave), 32 x 64,
  // 64 x 64 and 128 x 64 tiles (four K-groups of two waves) whose grid fits
  // on the CUs in one round.  Finer tiles put more CUs to work; their extra
  // W and X re-reads mostly hit L2 (K = 4096 unless stated: N = 4096 M = 64
  // 12.5 against 14.5 us for 32 x 64 and 18.6 for 64 x 64, M = 128 15.3
  // against 25.5 for 128 x 64, M = 256 20.2 against 25.8 and 35.5 for
  // 128 x 128; K = 11008 N = 4096 M = 64 26.6 against 33.3, M = 128 36.9
  // against 58.6, M = 256 49.1 against 87.4).  At N = 11008 this gives 32 x 64 tiles for M <= 32,
  // 64 x 64 for M <= 64 and 128 x 64 for M <= 128 (M = 32 17.3, M = 64
  // 22.1, M = 128 31.9 us against 28.1, 34.2 and 35.3 for the kernels they
  // replaced).  When none fits:
  // * M >= 129: 128 x 128 tiles (WN = 4 waves per K-group), two K-groups
  //   while the tiles fit on the CUs (one workgroup each), one K-group and
  //   two workgroups per CU beyond (M = 144 39.2 us against 54.6 for the
  //   128 x 64 kernel; M = 160 36.5 against 49.3 for 128 x 64 tiles in two
  //   rounds);
  // * 65 <= M <= 128: the same 128 x 128 tiles with two K-groups while
  //   they fit (N = 32768 M = 128 52.2 us, N = 24576 M = 100 44.1, against
  //   61.5 and 52.4 for 128 x 64 tiles with two K-groups), else those
  //   128 x 64 tiles;
  // * 33 <= M <= 64: 64 x 64 tiles (N = 32768 M = 64 42.8 against 55.6);
  // * 17 <= M <= 32: 32 x 64 tiles (N = 32768 M = 32 34.4 against 53.6).
  // From M = 17 the tile GEMM is ahead of the split-K skinny kernel on
  // every grid measured (M = 17 N = 1024 10.8 against 13.0 us, N = 4096
  // 11.7 against 13.5; M = 32 K = 11008 N = 4096 25.4 against 39.5).
  // NESO_AMD_W4_TILE_GEMM = 0 turns the tile GEMM off; 1 / 2: 128 x 128
  // tiles with one / two K-groups; 3 / 4: 128 x 64 with two / four; 5:
  // 64 x 64 with four; 6: 32 x 64 with four; 7: 32 x 32 with eight.
  // NESO_AMD_W4_WIDE_TILE_MIN_M (65 by default) is the smallest M for which
  // those 128 x 128 tiles are taken when no fine tile fits.
  const char* tile_env = getenv("NESO_AMD_W4_TILE_GEMM");
  const int tile_mode = tile_env ? atoi(tile_env) : -1;
  const char* wide_env = getenv("NESO_AMD_W4_WIDE_TILE_MIN_M");
  const int wide_min_m = wide_env ? atoi(wide_env) : 65;
  const int cus = device_cu_count();
  auto tiles_of = [&](int tm, int tn) { return ((a.M + tm - 1) / tm) * ((a.N + tn - 1) / tn); };
  const int fine = tiles_of(32, 32) <= cus    ? 7
                   : tiles_of(32, 64) <= cus  ? 6
                   : tiles_of(64, 64) <= cus  ? 5
                   : tiles_of(128, 64) <= cus ? 4
                                              : 0;
  const int mode = tile_mode >= 0      ? tile_mode
                   : fine              ? fine
                   : a.M >= wide_min_m && (a.M > 128 || tiles_of(128, 128) <= cus)
                       ? (tiles_of(128, 128) <= cus ? 2 : 1)
                   : a.M > 64 ? 3
                   : a.M > 32          ? 5
                                       : 6;

  // The skinny kernels: X in LDS up to M = 16 (group 32, K <= 4096), the
  // split-K skinny kernel otherwise up to M = 16 (past that K only where
  // the 32 x 32 tile grid would not fit on the CUs), and up to M = 32 when
  // the tile GEMM is off or its offsets would pass 2^31 bytes.
  // NESO_AMD_W4_SKINNY_MAX_M (at most 64) forces them up to that M.
  const char* skinny_env = getenv("NESO_AMD_W4_SKINNY_MAX_M");
  const int skinny_max_m = skinny_env ? atoi(skinny_env) : 32;
  // Up to M = 16 past the X-in-LDS kernel's K the 32 x 32 tile GEMM beats
  // the split-K skinny kernel when its grid fits (K = 11008 N = 4096:
  // M = 4 20.8, M = 16 22.1 us against 23.9 and 27.3).
  const bool tile_ok = tile_fits && tile_mode != 0;
  const bool skinny_default =
      a.M <= 16 ? !(tile_ok && a.K > w4a16_skinny_lds_max_k() && tiles_of(32, 32) <= cus) : !tile_ok;
  if (a.M <= 16 && a.M <= skinny_max_m && a.group == 32 && a.K % 128 == 0 &&
      a.K <= w4a16_skinny_lds_max_k()) {
    // X in LDS, one persistent workgroup per CU, 8 waves splitting K
    // (qmatmul_skinny.hip).
    return launch_w4a16_skinny_lds(a, s);
  }
  if (a.M <= skinny_max_m && a.M <= 64 && skinny_fits && (skinny_env || skinny_default)) {
    // One 8-byte load fetches the scales of a chunk quad when every chunk
    // has its own scale and rows hold whole quads (8-byte aligned).
    const bool g32 = a.group == 32 && a.K % 128 == 0;
    const dim3 block(kSkinnyWaves * kWave);
    if (a.M <= 16) {
      const dim3 grid((a.N + 31) / 32, 1);
      return g32 ? launch<&w4a16_skinny_kernel<1, 2, kSkinnyWaves, true>>(
          ktag("w4a16_skinny_kernel", 1, 2, kSkinnyWaves, true), grid, block, s, a)
                 : launch<&w4a16_skinny_kernel<1, 2, kSkinnyWaves, false>>(
                     ktag("w4a16_skinny_kernel", 1, 2, kSkinnyWaves, false), grid, block, s, a);
    }
    const dim3 grid((a.N + 31) / 32, (a.M + 31) / 32);
    return g32 ? launch<&w4a16_skinny_kernel<2, 2, kSkinnyWaves, true>>(
        ktag("w4a16_skinny_kernel", 2, 2, kSkinnyWaves, true), grid, block, s, a)
               : launch<&w4a16_skinny_kernel<2, 2, kSkinnyWaves, false>>(
                   ktag("w4a16_skinny_kernel", 2, 2, kSkinnyWaves, false), grid, block, s, a);
  }
#ifndef NESO_GEMM_WN
#define NESO_GEMM_WN 2
#endif
#ifndef NESO_GEMM_BN
#define NESO_GEMM_BN 64
#endif
  if (tile_fits && mode >= 1 && mode <= 7) {
    // Per-group arrival counters instead of workgroup barriers (the
    // kernel's step_sync) pay on long K-loops and on 128-row tiles, where
    // each K-group's step is long (K = 4096, N = 11008: M = 96 29.2 ->
    // 26.4, M = 128 30.2 -> 27.8 us; K = 11008, N = 4096: M = 64 45.7 ->
    // 41.7, M = 128 73.0 -> 58.8, M = 256 94.4 -> 86.6).  Short loops of
    // 32- and 64-row tiles lose 2-4% to the counter round trip.
    // NESO_AMD_W4_TILE_SYNC = 0 / 1 forces barriers / counters (the 32 x 32
    // form's one-wave groups take neither).
    static constexpr int kGroups[8] = {0, 1, 2, 2, 4, 4, 4, 8}, kRowTiles[8] = {0, 4, 4, 4, 4, 2, 1, 1};
    const int kgroups = kGroups[mode], steps = ((a.K + kTK - 1) / kTK + kgroups - 1) / kgroups;
    const char* sync_env = getenv("NESO_AMD_W4_TILE_SYNC");
    W4Args t = a;
    t.group_sync = kgroups > 1 && (sync_env ? atoi(sync_env) != 0
                                            : steps >= (kRowTiles[mode] == 4 ? 16 : 32));
    switch (mode) {
      case 1: return launch<&w4a16_tile_gemm_kernel<1, 4, 4>>(ktag("w4a16_tile_gemm_kernel", 1, 4, 4),
                                                               dim3(tiles_of(128, 128)), dim3(256), s, t);
      case 2: return launch<&w4a16_tile_gemm_kernel<2, 4, 4>>(ktag("w4a16_tile_gemm_kernel", 2, 4, 4),
                                                               dim3(tiles_of(128, 128)), dim3(512), s, t);
      case 3: return launch<&w4a16_tile_gemm_kernel<2, 2, 4>>(ktag("w4a16_tile_gemm_kernel", 2, 2, 4),
                                                               dim3(tiles_of(128, 64)), dim3(256), s, t);
      case 4: return launch<&w4a16_tile_gemm_kernel<4, 2, 4>>(ktag("w4a16_tile_gemm_kernel", 4, 2, 4),
                                                               dim3(tiles_of(128, 64)), dim3(512), s, t);
      case 5: return launch<&w4a16_tile_gemm_kernel<4, 2, 2>>(ktag("w4a16_tile_gemm_kernel", 4, 2, 2),
                                                               dim3(tiles_of(64, 64)), dim3(512), s, t);
      case 6: return launch<&w4a16_tile_gemm_kernel<4, 2, 1>>(ktag("w4a16_tile_gemm_kernel", 4, 2, 1),
                                                               dim3(tiles_of(32, 64)), dim3(512), s, t);
      default: return launch<&w4a16_tile_gemm_kernel<8, 1, 1>>(ktag("w4a16_tile_gemm_kernel", 8, 1, 1),
                                                                dim3(tiles_of(32, 32)), dim3(512), s, t);
    }
  }
  constexpr int WM = 2, WN = NESO_GEMM_WN, BN = NESO_GEMM_BN;
  if ((int64_t)kGBM * a.ldx * 2 + (int64_t)a.K * 2 < ((int64_t)1 << 31) &&
      (int64_t)BN * a.K / 2 < ((int64_t)1 << 31)) {
    const int tiles = ((a.M + kGBM - 1) / kGBM) * ((a.N + BN - 1) / BN);
    return launch<&w4a16_gemm_kernel<WM, WN, BN>>(
        ktag("w4a16_gemm_kernel", WM, WN, BN), dim3(tiles), dim3(WM * WN * kWave), s, a);
  }
  constexpr int TN = 2;
  const dim3 grid((a.N + 4 * 32 * TN - 1) / (4 * 32 * TN), (a.M + 31) / 32);
  return launch<&w4a16_mfma_kernel<TN>>(ktag("w4a16_mfma_kernel", TN), grid, dim3(kThreads), s, a);
}

hipError_t launch_w8a16(const W8Args& a, hipStream_t s) {
  // The tiled kernel reads A and B in 16-byte pieces: A's must be 16-byte
  // aligned and never straddle the end of a row; B's need 8-byte alignment
  // (a piece that straddles N reads columns that are never stored).  Buffer
  // offsets stay below 2^31 bytes.
  const bool tiled = a.K % 8 == 0 && a.lda % 8 == 0 && a.N % 8 == 0 && a.ldb % 8 == 0 &&
                     (reinterpret_cast<uintptr_t>(a.A) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.B) & 7u) == 0 &&
                     (int64_t)256 * a.lda * 2 < ((int64_t)1 << 31) &&
                     (int64_t)a.K * a.ldb < ((int64_t)1 << 31);
  if (tiled) {
    // 256 x 256 tiles (a third fewer LDS bytes per MFMA) when they still
    // give every CU a workgroup; 128 x 128 otherwise.
    const int64_t big = (int64_t)((a.N + 255) / 256) * ((a.M + 255) / 256);
    if (big >= device_cu_count()) {
      const dim3 grid((a.N + 255) / 256, (a.M + 255) / 256);
      return launch<&w8a16_gemm_kernel<256>>(ktag("w8a16_gemm_kernel", 256), grid, dim3(512), s, a);
    }
    const dim3 grid((a.N + 127) / 128, (a.M + 127) / 128);
    return launch<&w8a16_gemm_kernel<128>>(ktag("w8a16_gemm_kernel", 128), grid, dim3(256), s, a);
  }
  const dim3 grid((a.N + 127) / 128, (a.M + 31) / 32);
  return launch<&w8a16_kernel>(ktag("w8a16_kernel"), grid, dim3(kThreads), s, a);
}

}  // namespace neso
