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
// diagonals, rel_bias[i, j] = G[i, T - 1 - i + j].  A workgroup takes 32
// query rows i0 .. i0 + 31 of one head; its waves walk the 32-wide tiles of
// relative positions r0 .. r0 + 31 that those rows use.  Each tile is one
// fp32 MFMA product (v_mfma_f32_32x32x2f32, d / 2 k-steps, no fp16 rounding
// of the inputs), and accumulator element (a, c) is rel_bias[i0 + a,
// r0 + c - (T - 1) + i0 + a]: the tile is a parallelogram in (i, j), so
// every element of G is used at most once and goes straight from the
// accumulator to its output without a transpose.
#include "common.h"
#include "neso_internal.h"

namespace neso {

namespace {

__device__ __forceinline__ float16v mfma32x32x2f32(float a, float b, float16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Lane l (row l % 32, k-half g = l / 32) holds features g * D/2 .. +D/2 of
// its row: the MFMA's k-step s pairs feature s with feature D/2 + s, which
// is a reordering of the same dot product.
template <int D>
__global__ __launch_bounds__(256) void relpos_precompute_kernel(RelPreArgs a) {
  constexpr int H = D / 2;
  const int h = blockIdx.y;
  const int T = a.T;
  const int i0 = blockIdx.x * 32;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = lane & 31, g = lane >> 5;
  const float* Qh = a.Q + (int64_t)h * T * D;
  const float* Rh = a.K_rel + (int64_t)h * (2 * T - 1) * D;
  const float* bu = a.bias_u + (int64_t)h * D;
  const float* bv = a.bias_v + (int64_t)h * D;

  // Q_u for this workgroup's rows.
  half_t* Qu = a.Q_u + (int64_t)h * T * D;
  for (int e = tid; e < 32 * D; e += 256) {
    const int i = i0 + e / D, f = e % D;
    if (i < T) Qu[(int64_t)i * D + f] = (half_t)(Qh[(int64_t)i * D + f] + bu[f]);
  }

  // (Q + bias_v) of row i0 + row (rows past T repeat row T - 1; their
  // results are never stored).
  const int qi = min(i0 + row, T - 1);
  float qv[H];
#pragma unroll
  for (int s = 0; s < H; s += 4) {
    const float4v x = *reinterpret_cast<const float4v*>(Qh + (int64_t)qi * D + g * H + s);
    const float4v b = *reinterpret_cast<const float4v*>(bv + g * H + s);
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[s + e] = x[e] + b[e];
  }

  // Relative positions used by rows i0 .. min(i0 + 31, T - 1):
  // r = T - 1 - i + j over j in [0, T).
  const int ilast = min(i0 + 31, T - 1);
  const int rlo = T - 1 - ilast;
  const int rhi = 2 * T - 2 - i0;
  const int ntiles = (rhi - rlo) / 32 + 1;
  half_t* Bh = a.rel_bias + (int64_t)h * T * T;
  for (int t = wave; t < ntiles; t += 4) {
    const int r0 = rlo + 32 * t;
    const int rr = min(r0 + row, 2 * T - 2);
    float16v acc = float16v{};
#pragma unroll
    for (int s = 0; s < H; s += 4) {
      const float4v k = *reinterpret_cast<const float4v*>(Rh + (int64_t)rr * D + g * H + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = mfma32x32x2f32(qv[s + e], k[e], acc);
    }
    // Accumulator register q of lane l: G[i0 + a][r0 + c] with
    // a = 8 (q / 4) + 4 g + q % 4, c = l % 32.
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int ia = i0 + 8 * (q >> 2) + 4 * g + (q & 3);
      const int j = r0 + row - (T - 1) + ia;
      if (ia < T && j >= 0 && j < T) Bh[(int64_t)ia * T + j] = (half_t)acc[q];
    }
  }
}

}  // namespace

hipError_t launch_relpos_precompute(const RelPreArgs& a, int head_dim, hipStream_t s) {
  const dim3 grid((a.T + 31) / 32, a.heads);
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
