// Flash-Attention-2 forward for gfx950, hand-written for 64-lane waves and
// v_mfma_f32_32x32x16_f16.
//
// Algorithm (reference: tests/test_flash_attention.py:79-247, the TTIR loop
// of `flash_attention_fwd`): per query block, m = -inf, l = 0, O = 0; per
// key/value block S = Q K^T * scale, m' = max(m, rowmax S), alpha =
// exp(m - m'), P = exp(S - m'), l = l*alpha + rowsum P, O = O*alpha +
// f16(P) V; finally O /= max(l, 1e-6) (src/neso/backend/codegen/
// lowering.py:4352-4353).  The relative-position variant
// (tests/test_rel_pos_fa2.py:155-253) adds a bias to the logits.
//
// MI355X mapping
// --------------
// * One workgroup = 4 waves = 128 query rows of one (batch, head); each wave
//   owns 32 queries.  Keys/values stream through LDS in blocks of 64,
//   double-buffered with one barrier per block.
// * The score tile is computed transposed, S^T = K Q^T (A = K rows from LDS,
//   B = Q^T from registers), so lane l holds 32 scores of ONE query (l % 32)
//   and the other 32 live in lane l ^ 32: row max / row sum are in-register
//   plus one half-wave exchange, and alpha is a per-lane scalar.
// * The K rows feeding the A operand are permuted (kRowPerm) so that the
//   S^T accumulator registers of lane group g are exactly 8 consecutive keys
//   per 16-key chunk.  exp(S^T) converted to f16 is therefore directly the
//   B operand of O^T = V^T P^T: P never goes through LDS.
// * V is written to LDS transposed ([d][key]) as 32-bit key pairs, which is
//   bank-conflict free, so the A operand V^T is one ds_read_b128 per lane.
// * Softmax runs in the log2 domain: t = s * scale * log2(e), p = 2^(t - m),
//   one FMA + one v_exp_f32 per score.
// * Workgroups of one head are placed on one XCD (xcd_swizzle) so K/V of
//   that head are fetched into a single L2.
#include "common.h"
#include "neso_internal.h"

namespace neso {

namespace {

constexpr int kBM = 128;      // queries per workgroup
constexpr int kKB = 64;       // keys per LDS block
constexpr int kThreads = 256; // 4 waves
constexpr float kLog2e = 1.4426950408889634f;

// Row of the 32-key tile loaded into A-operand row rho (= lane % 32) so that
// accumulator register r of lane group g holds key 16*(r/8) + 8*g + r%8.
// Accumulator row rho = 8*(r/4) + 4*g + r%4 (see mfma32x32x16).
__device__ __forceinline__ int kRowPerm(int rho) {
  const int b = rho >> 3, g = (rho >> 2) & 1, j = rho & 3;
  return 16 * (b >> 1) + 8 * g + 4 * (b & 1) + j;
}

template <int D, bool CAUSAL, int BIAS, bool OUT_F16>
__global__ __launch_bounds__(kThreads) void fa2_fwd_kernel(Fa2Args p) {
  constexpr int KS = D / 16;                   // k-steps of S^T = K Q^T
  constexpr int DT = D / 32;                   // 32-row tiles of O^T
  constexpr int KLD = D + 8;                   // LDS row stride of K (halves)
  constexpr int VLD = kKB + 8;                 // LDS row stride of V^T (halves)
  constexpr int KCH = kKB * D / 8 / kThreads;  // 16-byte K chunks per thread
  constexpr int VJOBS = kKB * D / 16;          // (key pair, 8 columns) jobs
  constexpr int VCH = (VJOBS + kThreads - 1) / kThreads;
  constexpr int BAND = kBM + kKB - 1;          // bias-table entries per block
  static_assert(KCH >= 1 && kKB * D / 8 % kThreads == 0, "K tile split");

  __shared__ __attribute__((aligned(16))) half_t sK[2][kKB * KLD];
  __shared__ __attribute__((aligned(16))) half_t sV[2][D * VLD];
  __shared__ float sBias[2][BIAS == kBiasTableF32 ? BAND + 1 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int ql = lane & 31;

  const uint32_t wg = xcd_swizzle(blockIdx.x, gridDim.x);
  const int bh = wg / p.num_qblocks;
  int qblk = wg % p.num_qblocks;
  if (CAUSAL) qblk = p.num_qblocks - 1 - qblk;  // longest rows first
  const int N = p.N;
  const int q0 = qblk * kBM;
  const int qw0 = q0 + wave * 32;  // first query of this wave
  const int q = qw0 + ql;          // this lane's query

  const half_t* Qh = p.Q + (int64_t)bh * p.bh_stride_q;
  const half_t* Kh = p.K + (int64_t)bh * p.bh_stride_kv;
  const half_t* Vh = p.V + (int64_t)bh * p.bh_stride_kv;

  // Q fragments: B operand of S^T, lane holds Q[q][16*ks + 8*g .. +7].
  half8v qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[ks] = (q < N) ? load_half8(Qh + (int64_t)q * p.stride_q + 16 * ks + 8 * g)
                     : half8v{};
  }

  // Keys this workgroup visits.
  const int kend = CAUSAL ? min(N, q0 + kBM) : N;
  const int nblk = (kend + kKB - 1) / kKB;

  // Global -> register staging of the next K/V block.
  half8v kreg[KCH];
  half8v vreg[VCH][2];
  float breg = 0.f;

  auto gload = [&](int kb0) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + kThreads * i;
      const int key = kb0 + c / (D / 8);
      const int col = 8 * (c % (D / 8));
      kreg[i] = (key < N) ? load_half8(Kh + (int64_t)key * p.stride_kv + col) : half8v{};
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int j = tid + kThreads * i;
      if (j < VJOBS) {
        const int key = kb0 + 2 * (j % (kKB / 2));
        const int col = 8 * (j / (kKB / 2));
        vreg[i][0] = (key < N) ? load_half8(Vh + (int64_t)key * p.stride_kv + col) : half8v{};
        vreg[i][1] = (key + 1 < N) ? load_half8(Vh + (int64_t)(key + 1) * p.stride_kv + col)
                                   : half8v{};
      }
    }
    if (BIAS == kBiasTableF32) {
      // Band of table[h][q - key + N - 1] for q in [q0, q0+BM), key in
      // [kb0, kb0+KB): index base + i with base = q0 - kb0 - (KB-1) + N - 1.
      const int idx = q0 - kb0 - (kKB - 1) + N - 1 + tid;
      const float* tab = static_cast<const float*>(p.bias) + (int64_t)bh * p.bias_stride_h;
      breg = (tid < BAND && idx >= 0 && idx <= 2 * N - 2) ? tab[idx] * kLog2e : 0.f;
    }
  };

  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + kThreads * i;
      *reinterpret_cast<half8v*>(&sK[buf][(c / (D / 8)) * KLD + 8 * (c % (D / 8))]) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int j = tid + kThreads * i;
      if (j < VJOBS) {
        const int kp = 2 * (j % (kKB / 2));
        const int col = 8 * (j / (kKB / 2));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          half2v pr = {vreg[i][0][e], vreg[i][1][e]};
          *reinterpret_cast<half2v*>(&sV[buf][(col + e) * VLD + kp]) = pr;
        }
      }
    }
    if (BIAS == kBiasTableF32) {
      if (tid < BAND) sBias[buf][tid] = breg;
    }
  };

  float m_run = -INFINITY;  // running max (log2 domain), same in lanes l, l^32
  float l_run = 0.f;        // this lane's partial row sum
  float16v o[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) o[u] = float16v{};

  const int krow = kRowPerm(ql);

  if (nblk > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  for (int blk = 0; blk < nblk; ++blk) {
    const int buf = blk & 1;
    const int kb0 = blk * kKB;
    if (blk + 1 < nblk) gload(kb0 + kKB);

    // A wave whose queries all precede this key block has nothing to do.
    const bool active = !CAUSAL || kb0 <= qw0 + 31;
    if (active) {
      // ---- S^T = K Q^T for two 32-key tiles ----
      float16v s[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        s[t] = float16v{};
        const half_t* kp = &sK[buf][(32 * t + krow) * KLD + 8 * g];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s[t] = mfma32x32x16(load_half8(kp + 16 * ks), qf[ks], s[t]);
      }

      // ---- logits in the log2 domain, bias, masks ----
      float x[2][16];
      const bool tail = kb0 + kKB > N;
      const bool diag = CAUSAL && kb0 + kKB - 1 > qw0;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kr = 32 * t + 16 * (r >> 3) + 8 * g + (r & 7);  // key - kb0
          float v;
          if (BIAS == kBiasDenseF16) {
            // Reference semantics: (QK^T + B) * scale, B dense [T, T] f16.
            const int key = kb0 + kr;
            const half_t* bp = static_cast<const half_t*>(p.bias) +
                               (int64_t)bh * p.bias_stride_h;
            const float b = (q < N && key < N) ? (float)bp[(int64_t)q * N + key] : 0.f;
            v = (s[t][r] + b) * p.scale_log2;
          } else if (BIAS == kBiasTableF32) {
            // BASELINE semantics: QK^T * scale + table[h][q - key + N - 1].
            v = s[t][r] * p.scale_log2 + sBias[buf][(q - q0) - kr + (kKB - 1)];
          } else {
            v = s[t][r] * p.scale_log2;
          }
          x[t][r] = v;
        }
      }
      if (tail || diag) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kb0 + 32 * t + 16 * (r >> 3) + 8 * g + (r & 7);
            if (key >= N || (CAUSAL && key > q)) x[t][r] = -INFINITY;
          }
        }
      }

      // ---- online softmax ----
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[t][r]);
      mx = fmaxf(mx, swap_halves(mx));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      m_run = m_new;

      float rs = 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          x[t][r] = fast_exp2(x[t][r] - m_use);
          rs += x[t][r];
        }
      l_run = l_run * alpha + rs;
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[u][r] *= alpha;

      // ---- O^T += V^T P^T, P truncated to f16 (reference :140-145) ----
      half8v pb[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[c][e] = (half_t)x[c >> 1][8 * (c & 1) + e];
#pragma unroll
      for (int u = 0; u < DT; ++u) {
        const half_t* vp = &sV[buf][(32 * u + ql) * VLD + 8 * g];
#pragma unroll
        for (int c = 0; c < 4; ++c) o[u] = mfma32x32x16(load_half8(vp + 16 * c), pb[c], o[u]);
      }
    }

    if (blk + 1 < nblk) sstore(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and store: lane holds O[q][32u + 8b + 4g + 0..3] ----
  // Lanes l and l^32 hold the same query, so the exchange is uniform.
  const float l_tot = l_run + swap_halves(l_run);
  if (q < N) {
    const float inv = 1.f / fmaxf(l_tot, 1e-6f);
#pragma unroll
    for (int u = 0; u < DT; ++u) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int col = 32 * u + 8 * b + 4 * g;
        float4v v = {o[u][4 * b] * inv, o[u][4 * b + 1] * inv, o[u][4 * b + 2] * inv,
                     o[u][4 * b + 3] * inv};
        if (OUT_F16) {
          half_t* op = static_cast<half_t*>(p.O) + (int64_t)bh * p.bh_stride_o +
                       (int64_t)q * p.stride_o + col;
          half4v hv = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
          *reinterpret_cast<half4v*>(op) = hv;
        } else {
          float* op = static_cast<float*>(p.O) + (int64_t)bh * p.bh_stride_o +
                      (int64_t)q * p.stride_o + col;
          *reinterpret_cast<float4v*>(op) = v;
        }
      }
    }
  }
}

template <int D, bool CAUSAL, int BIAS, bool OUT_F16>
hipError_t launch_fa2_t(const Fa2Args& a, hipStream_t stream) {
  const int grid = a.num_qblocks * a.batch_heads;
  hipLaunchKernelGGL((fa2_fwd_kernel<D, CAUSAL, BIAS, OUT_F16>), dim3(grid), dim3(kThreads), 0,
                     stream, a);
  return hipGetLastError();
}

template <int D, int BIAS, bool OUT_F16>
hipError_t launch_fa2_c(const Fa2Args& a, bool causal, hipStream_t s) {
  return causal ? launch_fa2_t<D, true, BIAS, OUT_F16>(a, s)
                : launch_fa2_t<D, false, BIAS, OUT_F16>(a, s);
}

template <int BIAS, bool OUT_F16>
hipError_t launch_fa2_d(const Fa2Args& a, int d, bool causal, hipStream_t s) {
  switch (d) {
    case 32: return launch_fa2_c<32, BIAS, OUT_F16>(a, causal, s);
    case 64: return launch_fa2_c<64, BIAS, OUT_F16>(a, causal, s);
    case 128: return launch_fa2_c<128, BIAS, OUT_F16>(a, causal, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int fa2_query_block() { return kBM; }

hipError_t launch_fa2(Fa2Args a, int head_dim, bool causal, int bias_kind, bool out_f16,
                      hipStream_t stream) {
  a.num_qblocks = (a.N + kBM - 1) / kBM;
  if (bias_kind == kBiasNone) {
    return out_f16 ? launch_fa2_d<kBiasNone, true>(a, head_dim, causal, stream)
                   : launch_fa2_d<kBiasNone, false>(a, head_dim, causal, stream);
  }
  if (bias_kind == kBiasTableF32) {
    return out_f16 ? launch_fa2_d<kBiasTableF32, true>(a, head_dim, causal, stream)
                   : launch_fa2_d<kBiasTableF32, false>(a, head_dim, causal, stream);
  }
  return out_f16 ? launch_fa2_d<kBiasDenseF16, true>(a, head_dim, causal, stream)
                 : launch_fa2_d<kBiasDenseF16, false>(a, head_dim, causal, stream);
}

}  // namespace neso
