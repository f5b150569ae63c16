// Relative-position (Transformer-XL) bias precompute for the rel-pos FA2
// kernel, on the GPU.
//
// Reference: precompute_bias_and_qu, tests/test_rel_pos_fa2.py:286-311, run
// on the host there:
//   Q_u[h, i]         = Q[h, i] + bias_u[h]
//   rel_bias[h, i, j] = (Q[h, i] + bias_v[h]) . K_rel[h, T - 1 - i + j]
// (unscaled; the kernel then forms (Q_u K^T + rel_bias) * scale), both
// stored as the fp16 inputs of rel_pos_fa2_fwd (:355-358).
//
// rel_bias is a [T x (2T - 1)] product G = (Q + v) K_rel^T read along
// diagonals, rel_bias[i, j] = G[i, T - 1 - i + j].  A workgroup takes 128
// query rows of one head, one 32-row block per wave, and a group of up to 8
// of the 32-wide tiles of relative positions r0 .. r0 + 31 those rows use
// (grid z picks the group).  Each K_rel tile is read from HBM once per
// workgroup, split and staged in LDS, and used by every wave whose rows
// need it.  Accumulator element (a, c) of a wave's tile is
// rel_bias[i0 + a, r0 + c - (T - 1) + i0 + a]: the tile is a parallelogram
// in (i, j), so every element of G is computed at most once and goes
// straight from the accumulator to its output.
//
// Each fp32 factor x is split into hi = fp16(x) and lo = fp16(x - hi), and a
// tile is hi.hi + hi.lo + lo.hi on v_mfma_f32_32x32x16_f16 with fp32
// accumulation: 3 fp16 MFMAs per 16 features (96 cycles) instead of 8 fp32
// v_mfma_f32_32x32x2f32 (512 cycles).  The dropped lo.lo term and the
// rounding of lo leave about 3 * 2^-22 |q_k k_k| per product, far below the
// fp16 rounding of the output.  Factors must lie in the fp16 range
// (|Q + bias_v|, |K_rel| < 65504), the same limit as fp32-input FA2.
#include "common.h"
#include "neso_internal.h"

namespace neso {

namespace {

constexpr int kPreRows = 128;         // query rows per workgroup, 32 per wave
constexpr int kPreTilesPerGroup = 8;  // relative-position tiles per workgroup

// Eight fp32 values as fp16 hi and lo halves (x ~= hi + lo).
__device__ __forceinline__ void split8(float4v x0, float4v x1, half8v& hi, half8v& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = (half_t)x0[e];
    lo[e] = (half_t)(x0[e] - (float)hi[e]);
    hi[4 + e] = (half_t)x1[e];
    lo[4 + e] = (half_t)(x1[e] - (float)hi[4 + e]);
  }
}

// 16-byte chunk c of staged row n sits at position c ^ (n % (D / 8)): the 32
// lanes that read chunk c of 32 consecutive rows spread over all banks.
template <int D>
__device__ __forceinline__ int chunk_slot(int n, int c) {
  return n * (D / 8) + (c ^ (n & (D / 8 - 1)));
}

// In k-step s, lane l (row l % 32, half g = l / 32) supplies features
// 16 s + 8 g .. + 7 of its query row (A) and of its relative-position row
// (B), the operand layout of v_mfma_f32_32x32x16_f16: chunk 2 s + g.
template <int D>
__global__ __launch_bounds__(256) void relpos_precompute_kernel(RelPreArgs a) {
  constexpr int S = D / 16;
  constexpr int CH = D / 8;  // 16-byte fp16 chunks per staged row
  // [slot][hi, lo][32 rows x CH chunks]: 256 D bytes.
  __shared__ half8v stage[2][2][32 * CH];

  // (row group, head, tile group) from the dispatch index, remapped so that
  // each XCD takes a contiguous run in (head, row group, tile group) order:
  // the workgroups of one head, which read overlapping K_rel rows, share an
  // XCD and its L2.
  const uint32_t gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
  const uint32_t lid = xcd_swizzle(blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z), gx * gy * gz);
  const int bz = (int)(lid % gz), bx = (int)(lid / gz % gx), h = (int)(lid / (gz * gx));
  const int T = a.T;
  const int i0 = bx * kPreRows;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = lane & 31, g = lane >> 5;
  const float* Qh = a.Q + (int64_t)h * T * D;
  const float* Rh = a.K_rel + (int64_t)h * (2 * T - 1) * D;
  const float* bu = a.bias_u + (int64_t)h * D;
  const float* bv = a.bias_v + (int64_t)h * D;

  // Q_u for this workgroup's rows in 4-float pieces, shared out over the
  // grid-z workgroups of the row group.  Q and Q_u are 16-byte aligned.
  {
    constexpr int P4 = D / 4;
    half_t* Qu = a.Q_u + (int64_t)h * T * D;
    for (int e = bz * 256 + tid; e < kPreRows * P4; e += 256 * (int)gz) {
      const int i = i0 + e / P4, f = 4 * (e % P4);
      if (i < T) {
        const float4v x = *reinterpret_cast<const float4v*>(Qh + (int64_t)i * D + f);
        half4v o;
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = (half_t)(x[c] + bu[f + c]);
        *reinterpret_cast<half4v*>(Qu + (int64_t)i * D + f) = o;
      }
    }
  }

  // Relative positions used by the workgroup's rows i0 .. min(i0 + 127,
  // T - 1): r = T - 1 - i + j over j in [0, T).  Uniform over the
  // workgroup, so a workgroup with no tiles leaves before any barrier.
  const int ilast = min(i0 + kPreRows - 1, T - 1);
  const int rlo = T - 1 - ilast;
  const int ntiles = (2 * T - 2 - i0 - rlo) / 32 + 1;
  const int t0 = bz * kPreTilesPerGroup;
  const int t1 = min(ntiles, t0 + kPreTilesPerGroup);
  if (t0 >= t1) return;

  // This wave's rows iw .. iw + 31 and the positions they use.
  const int iw = i0 + 32 * wave;
  const bool rows_ok = iw < T;
  const int w_rlo = T - 1 - min(iw + 31, T - 1);
  const int w_rhi = 2 * T - 2 - iw;

  // (Q + bias_v) of row iw + row, split (rows past T repeat row T - 1;
  // their results are never stored).
  const int qi = min(iw + row, T - 1);
  half8v ahi[S], alo[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int f = 16 * s + 8 * g;
    const float4v x0 = *reinterpret_cast<const float4v*>(Qh + (int64_t)qi * D + f);
    const float4v x1 = *reinterpret_cast<const float4v*>(Qh + (int64_t)qi * D + f + 4);
    const float4v b0 = *reinterpret_cast<const float4v*>(bv + f);
    const float4v b1 = *reinterpret_cast<const float4v*>(bv + f + 4);
    split8(x0 + b0, x1 + b1, ahi[s], alo[s]);
  }

  // Staging: thread e of the 4 D pieces (8 floats each) of a tile takes row
  // e / CH, chunk e % CH; rows past 2T - 2 repeat the last one (their
  // results are never stored).  CH * 32 <= 512 pieces, at most 2 per thread.
  constexpr int PT = (32 * CH + 255) / 256;
  typedef float4v Raw[PT][2];
  auto load_tile = [&](int t, Raw& kr) {
#pragma unroll
    for (int p = 0; p < PT; ++p) {
      const int e = tid + 256 * p;
      if (e < 32 * CH) {
        const int rr = min(rlo + 32 * t + e / CH, 2 * T - 2);
        const float* src = Rh + (int64_t)rr * D + 8 * (e % CH);
        kr[p][0] = *reinterpret_cast<const float4v*>(src);
        kr[p][1] = *reinterpret_cast<const float4v*>(src + 4);
      }
    }
  };
  auto stage_tile = [&](int slot, const Raw& kr) {
#pragma unroll
    for (int p = 0; p < PT; ++p) {
      const int e = tid + 256 * p;
      if (e < 32 * CH) {
        half8v hi, lo;
        split8(kr[p][0], kr[p][1], hi, lo);
        const int at = chunk_slot<D>(e / CH, e % CH);
        stage[slot][0][at] = hi;
        stage[slot][1][at] = lo;
      }
    }
  };

  half_t* Bh = a.rel_bias + (int64_t)h * T * T;
  // Tiles wholly inside the [T x T] output store through a buffer resource:
  // element (q, lane) sits at ia * T + j = lane_base + r0 + dq * (T + 1),
  // dq = 8 (q / 4) + q % 4, so the lane part is one add per tile and the
  // q part a wave-uniform offset.  T^2 * 2 bytes fits 32 bits (T^2 <= 2^31).
  const rsrc_t rb = make_rsrc(Bh, (uint32_t)((int64_t)T * T * 2));
  const int lane_base = (iw + 4 * g) * (T + 1) - (T - 1) + row;
  auto compute = [&](int t, int slot) {
    const int r0 = rlo + 32 * t;
    if (!rows_ok || r0 > w_rhi || r0 + 31 < w_rlo) return;
    float16v acc = float16v{};
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int at = chunk_slot<D>(row, 2 * s + g);
      const half8v bhi = stage[slot][0][at];
      const half8v blo = stage[slot][1][at];
      acc = mfma32x32x16(ahi[s], bhi, acc);
      acc = mfma32x32x16(ahi[s], blo, acc);
      acc = mfma32x32x16(alo[s], bhi, acc);
    }
    // Accumulator register q of lane l: G[iw + a][r0 + c] with
    // a = 8 (q / 4) + 4 g + q % 4, c = l % 32, stored at
    // rel_bias[iw + a][r0 + c - (T - 1) + iw + a].
    const bool inside = iw + 31 < T && r0 - (T - 1) + iw >= 0 && r0 + 62 - (T - 1) + iw < T;
    if (inside) {
      // The empty asm keeps the whole offset in the register: the compiler
      // would otherwise move the tile's part (32 t) into the immediate
      // field, leaving a register part that can be a wrapped negative
      // number, which the range check of raw buffer stores treats as out of
      // range although the whole offset is in range.
      uint32_t voff = (uint32_t)(lane_base + r0) * 2u;
      asm volatile("" : "+v"(voff));
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const uint32_t soff = (uint32_t)((8 * (q >> 2) + (q & 3)) * (T + 1)) * 2u;
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (half_t)acc[q]), rb,
                                              voff, soff, 0);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int ia = iw + 8 * (q >> 2) + 4 * g + (q & 3);
        const int j = r0 + row - (T - 1) + ia;
        if (ia < T && j >= 0 && j < T) Bh[(int64_t)ia * T + j] = (half_t)acc[q];
      }
    }
  };

  // Two LDS slots and two register sets: step t computes tile t from one
  // slot, stages tile t + 1 (loaded a step earlier) into the other, and
  // loads tile t + 2.  The barrier at the top of each step publishes the
  // slot and retires the reads of the step before, which used the slot about
  // to be written.  Unrolled by two so that the register sets have fixed
  // names.
  Raw ka, kb;
  load_tile(t0, ka);
  if (t0 + 1 < t1) load_tile(t0 + 1, kb);
  stage_tile(0, ka);
  for (int t = t0; t < t1; t += 2) {
    lds_barrier();
    if (t + 2 < t1) load_tile(t + 2, ka);
    compute(t, 0);
    if (t + 1 < t1) stage_tile(1, kb);
    if (t + 1 >= t1) break;
    lds_barrier();
    if (t + 3 < t1) load_tile(t + 3, kb);
    compute(t + 1, 1);
    if (t + 2 < t1) stage_tile(0, ka);
  }
}

}  // namespace

// Workgroups along grid z: 8-tile groups of the widest row group's
// relative-position tiles (rows i0 .. i0 + 127 use T + 127 positions, fewer
// when T < 128).
static int relpos_precompute_groups(int T) {
  const int ntiles = (T - 1 + min(kPreRows - 1, T - 1)) / 32 + 1;
  return (ntiles + kPreTilesPerGroup - 1) / kPreTilesPerGroup;
}

hipError_t launch_relpos_precompute(const RelPreArgs& a, int head_dim, hipStream_t s) {
  const dim3 grid((a.T + kPreRows - 1) / kPreRows, a.heads, relpos_precompute_groups(a.T));
  switch (head_dim) {
    case 32:
      return launch<&relpos_precompute_kernel<32>>(ktag("relpos_precompute_kernel", 32), grid,
                                                  dim3(256), s, a);
    case 64:
      return launch<&relpos_precompute_kernel<64>>(ktag("relpos_precompute_kernel", 64), grid,
                                                  dim3(256), s, a);
    case 128:
      return launch<&relpos_precompute_kernel<128>>(ktag("relpos_precompute_kernel", 128), grid,
                                                   dim3(256), s, a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace neso
