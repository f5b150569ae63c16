// int4 W4A16 skinny-M kernel with X resident in LDS (3 <= M <= 16 by
// default, group 32, K <= 4096, K % 128 == 0): its own translation unit so
// that it can be compiled with its own scheduler options (see build.py).
#include "common.h"
#include "neso_internal.h"
#include "qmatmul_common.h"

namespace neso {

namespace {

// Skinny-M regime with X resident in LDS (M <= 16, K <= 4096, group 32).
//
// The workload is one burst of N*K/2 bytes.  One persistent workgroup per
// CU owns row tiles blockIdx.x + i * gridDim.x (16 rows each, i < T).  Its
// WV waves split K (wave w takes chunk quads [w*QW, (w+1)*QW)) and request
// the weights and scales of tile i + 1 before computing tile i, tile 0
// right after X (plain loads: the non-temporal hint measured slower for
// these 64-byte row pieces).  X is copied
// once per workgroup into LDS, already in MFMA A-fragment order (slot
// (4q + t) * 64 + lane holds X[m][32(4q+t) + 8g + {0,4,1,5,2,6,3,7}] for
// lane = m + 16g), so the per-tile A operand is one conflict-free
// ds_read_b128 per MFMA.  MFMA, transpose and dequantisation are those of
// w4a16_skinny_kernel.  The WV partial tiles are reduced through LDS.
// (The slot's row index is XOR-swizzled; see the X loads below.)
constexpr int kLdsQuads = 32;  // K <= 4096

template <int WV, int T, int QWMAX>
__global__ __launch_bounds__(WV * kWave) void w4a16_skinny_lds_kernel(W4Args a) {
  static_assert(QWMAX <= 4, "a quad's scales come from one of the four lane groups");
  constexpr uint32_t kOut = 0x80000000u;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int KW = a.K >> 3, SG = a.K >> 5, C = a.K >> 5;
  const int Q = (C + 3) >> 2;
  const int QW = (Q + WV - 1) / WV;
  const int q0 = wave * QW;
  const int cend = min(4 * min(q0 + QW, Q), C);
  const int ntiles = (a.N + 15) >> 4;
  const ZeroPoint zp = zero_point(a.zero);
  const Nibbles nib = nibble_consts();

  __shared__ half8v xs[kLdsQuads * 4 * kWave];
  __shared__ float red[T][WV][4][kWave];

  // X first: loads complete in issue order, so X (L2-resident) reaches LDS
  // while the weight burst is still arriving; issued after the weights, it
  // waited behind them (measured: 15.7 -> 14.2 us at M = 16).  Each wave
  // instruction reads 1 KiB of one X row (piece e: row m, pieces pp of 8
  // halves; 16 rows x 64 B per instruction measured 14.2 vs 12.9 us).  Piece
  // (m, chunk ct, quarter g) goes to A-fragment slot ct*64 + 16g + m', with
  // the row index swizzled, m' = m ^ (4 (ct % 4) + g), so that the 64
  // same-row stores of an instruction and the 16-lane fragment reads both
  // spread over all banks.
  constexpr int kXPer = (kLdsQuads * 4 * kWave) / (WV * kWave);
  const rsrc_t rx = make_rsrc(a.X, (uint32_t)(((int64_t)(a.M - 1) * a.ldx + a.K) * 2));
  half8v xv[kXPer];
  uint32_t xslot[kXPer];
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    const uint32_t e = threadIdx.x + i * WV * kWave;
    const uint32_t m = e / (4 * 4 * kLdsQuads), pp = e % (4 * 4 * kLdsQuads);
    const uint32_t ct = pp >> 2, g = pp & 3;
    const uint32_t oob = ((int)ct < C && (int)m < a.M) ? 0u : kOut;
    xv[i] = buf_load_half8(rx, ((m * (uint32_t)a.ldx + 8u * pp) * 2u) | oob);
    xslot[i] = ct * 64 + 16 * g + (m ^ (4 * (ct & 3) + g));
  }

  // Weight and scale loads of this wave for tile i.
  // Scales: one 8-byte load per lane and tile, lane (li, lg) taking quad
  // q0 + lg of row li (32 contiguous bytes per row instead of 8, and no
  // four lanes loading the same bytes); quad qi reaches lane (li, *) from
  // lane (li, qi) by ds_bpermute (measured 12.9 -> 11.7 us at M = 16).
  typedef uint32_t uint2v __attribute__((ext_vector_type(2)));
  uint4v w[T][QWMAX];
  uint2v scw[T];
  auto load_tile = [&](int i) {
    const int tile = blockIdx.x + i * gridDim.x;
    const int n0 = tile * 16;
    const int nrows = tile < ntiles ? min(16, a.N - n0) : 0;
    const rsrc_t rw = make_rsrc(a.W + (int64_t)(nrows ? n0 : 0) * KW, (uint32_t)nrows * KW * 4u);
    const rsrc_t rs = make_rsrc(a.S + (int64_t)(nrows ? n0 : 0) * SG, (uint32_t)nrows * SG * 2u);
#pragma unroll
    for (int qi = 0; qi < QWMAX; ++qi) {
      const uint32_t cq = 4 * (q0 + qi);
      const uint32_t c = cq + lg;
      const bool live = qi < QW;
      const uint32_t wo = (li * (uint32_t)KW * 4u + c * 16u) | (live && (int)c < cend ? 0u : kOut);
      w[i][qi] = __builtin_bit_cast(
          uint4v, __builtin_amdgcn_raw_buffer_load_b128(rw, wo, 0, 0));
    }
    {
      const uint32_t cq = 4 * (q0 + lg);
      const uint32_t so = ((li * (uint32_t)SG + cq) * 2u) | (lg < QW && (int)cq < cend ? 0u : kOut);
      scw[i] = __builtin_bit_cast(uint2v, __builtin_amdgcn_raw_buffer_load_b64(rs, so, 0, 0));
    }
  };
  // Tile 0 now; tile i + 1 is requested when tile i's compute starts.  With
  // every tile requested up front, the wave stalls at the load instructions
  // once the CU's outstanding-request capacity is full, and X, compute and
  // the weight stream run one after another (M = 16: 12.0 -> 9.3 us).
  load_tile(0);

  // X into LDS in A-fragment order.
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    const half8v x = xv[i];
    xs[xslot[i]] = half8v{x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]};
  }
  lds_barrier();

  float4v acc[T];
#pragma unroll
  for (int i = 0; i < T; ++i) {
    if (i + 1 < T) load_tile(i + 1);
    acc[i] = float4v{};
#pragma unroll
    for (int qi = 0; qi < QWMAX; ++qi) {
      if (qi >= QW) break;  // uniform
      const int q = q0 + qi;
      uint32_t wt[4] = {w[i][qi][0], w[i][qi][1], w[i][qi][2], w[i][qi][3]};
      const int src = (li + 16 * qi) * 4;
      const half4v sq = __builtin_bit_cast(
          half4v, uint2v{(uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)scw[i][0]),
                         (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)scw[i][1])});
      transpose_rows4(wt[0], wt[1], wt[2], wt[3]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const half8v xa = xs[(4 * q + t) * kWave + 16 * lg + (li ^ (4 * t + lg))];
        const half_t s = sq[t];
        const half2v s1 = {s, s};
        half2v r[4];
        unpack_word(wt[t], nib, zp, r);
        const half2v d0 = r[0] * s1, d1 = r[1] * s1, d2 = r[2] * s1, d3 = r[3] * s1;
        const half8v bv = {d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
        acc[i] = mfma16x16x32(xa, bv, acc[i]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) red[i][wave][r][lane] = acc[i][r];
  }
  lds_barrier();

  // acc[i] register r of lane l is D[4(l/16) + r][l%16] of tile i.
  for (int e = threadIdx.x; e < T * 4 * kWave; e += WV * kWave) {
    const int i = e / (4 * kWave), r = (e / kWave) & 3, ln = e & 63;
    const int tile = blockIdx.x + i * gridDim.x;
    float v = 0.f;
#pragma unroll
    for (int wv = 0; wv < WV; ++wv) v += red[i][wv][r][ln];
    const int m = 4 * (ln >> 4) + r;
    const int n = tile * 16 + (ln & 15);
    if (tile < ntiles && m < a.M && n < a.N) a.Y[(int64_t)m * a.ldy + n] = (half_t)v;
  }
}

}  // namespace

int w4a16_skinny_lds_max_k() { return 32 * 4 * kLdsQuads; }

hipError_t launch_w4a16_skinny_lds(const W4Args& a, hipStream_t s) {
  const int ntiles = (a.N + 15) / 16;
  const int cus = device_cu_count();
  int T = (ntiles + cus - 1) / cus;
  if (T > 4) T = 4;
  const dim3 grid((ntiles + T - 1) / T);
  constexpr int WV = 8, QWMAX = (kLdsQuads + WV - 1) / WV;
  const dim3 block(WV * kWave);
  switch (T) {
    case 1: return launch<&w4a16_skinny_lds_kernel<WV, 1, QWMAX>>(
        ktag("w4a16_skinny_lds_kernel", WV, 1, QWMAX), grid, block, s, a);
    case 2: return launch<&w4a16_skinny_lds_kernel<WV, 2, QWMAX>>(
        ktag("w4a16_skinny_lds_kernel", WV, 2, QWMAX), grid, block, s, a);
    case 3: return launch<&w4a16_skinny_lds_kernel<WV, 3, QWMAX>>(
        ktag("w4a16_skinny_lds_kernel", WV, 3, QWMAX), grid, block, s, a);
    default: return launch<&w4a16_skinny_lds_kernel<WV, 4, QWMAX>>(
        ktag("w4a16_skinny_lds_kernel", WV, 4, QWMAX), grid, block, s, a);
  }
}

}  // namespace neso
