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
// * A key group = 4 waves = 128 query rows of one (batch, head); each wave
//   owns 32 queries.  Keys/values stream through LDS in blocks of 64.
//   Global loads run two blocks ahead through registers; the LDS holds two
//   blocks; one barrier per block.
// * KSPLIT key groups per workgroup split the key blocks between them
//   (group g takes blocks g, g+KSPLIT, ...) and merge (m, l, O) through LDS
//   at the end.  KSPLIT = 2 gives every SIMD two waves when the grid alone
//   would leave one, so MFMA work of one wave hides the softmax of the other.
// * The score tile is computed transposed, S^T = K Q^T (A = K rows from LDS,
//   B = Q^T from registers), so lane l holds 32 scores of ONE query (l % 32)
//   and the other 32 live in lane l ^ 32: row max is in-register plus one
//   v_permlane32_swap, and alpha is a per-lane scalar.
// * The K rows feeding the A operand are permuted (kRowPerm) so that the
//   S^T accumulator registers of lane group g are exactly 8 consecutive keys
//   per 16-key chunk.  exp(S^T) converted to f16 is therefore directly the
//   B operand of O^T = V^T P^T: P never goes through LDS.
// * V is stored to LDS row-major ([key][d], 16-byte chunks swizzled) and
//   its V^T operand is read with the transposing LDS load
//   ds_read_b64_tr_b16, two per fragment (v_frag_tr in fa2_tiles.h).
// * Softmax runs in the log2 domain with one FMA + one v_exp_f32 per score:
//   p = 2^(s*c - m), c = |scale| * log2(e).  The running max m is only
//   raised (and O, l rescaled) when a row max exceeds it by more than
//   kLazyLog2, so p <= 2^kLazyLog2 and most blocks skip the O rescale.
//   Row sums use v_dot2_f32_f16 on the fp16 P actually fed to the MFMA.
// * Workgroups of one head are placed on one XCD (xcd_swizzle) so K/V of
//   that head are fetched into a single L2.
#include "common.h"
#include "fa2_tiles.h"
#include "neso_internal.h"

namespace neso {

namespace {

constexpr int kBM = 128;       // queries per workgroup at four query waves
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyLog2 = 8.f;  // rescale threshold (log2 units)

// Keys per LDS block.  64 measured faster than 128 at d = 64 on MI355X
// (fewer live registers; the extra barriers are not the bottleneck).  fp32
// input at d = 128 uses 32: its slots hold the hi and lo halves of K and V,
// and two 32-key slots per key group keep two key groups within the LDS
// (and the fp32 staging registers within the register file).
template <int D, bool F32IN = false>
constexpr int key_block() { return (F32IN && D == 128) ? 32 : 64; }

// One 8-element row piece of K or V in registers: f16, or f32 (two float4).
template <bool F32IN>
struct Piece8 {
  half8v h;
};
template <>
struct Piece8<true> {
  float4v f[2];
};

template <int D, bool F32IN, int GT>
struct Staging {
  static constexpr int kKB = key_block<D, F32IN>();
  static constexpr int KCH = kKB * D / 8 / GT;   // 8-element K (and V) pieces per thread
  Piece8<F32IN> k[KCH];
  Piece8<F32IN> v[KCH];
  float b;
};

// f32 -> (hi, lo) f16 split: x ~= hi + lo to about 2^-22 relative, so the
// three products hi*hi + hi*lo + lo*hi of two split operands reproduce an
// f32 product to that accuracy on the f16 MFMA.
__device__ __forceinline__ void split_f16(const float4v (&f)[2], half8v& hi, half8v& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = f[e >> 2][e & 3];
    hi[e] = (half_t)x;
    lo[e] = (half_t)(x - (float)hi[e]);
  }
}

template <int D, bool CAUSAL, int BIAS, bool OUT_F16, int KSPLIT, bool F32IN, int QW>
__global__ __launch_bounds__(64 * QW * KSPLIT) void fa2_fwd_kernel(Fa2Args p) {
  constexpr int kBM = 32 * QW;      // queries per workgroup (QW waves of 32)
  constexpr int kGroup = 64 * QW;   // threads per key group
  constexpr int kKB = key_block<D, F32IN>();
  constexpr int NT = kKB / 32; // 32-key tiles per block
  constexpr int KS = D / 16;   // k-steps of S^T = K Q^T
  constexpr int DT = D / 32;   // 32-row tiles of O^T
  constexpr int KLD = D + 8;   // LDS row stride of K (halves)
  constexpr int BAND = kBM + kKB - 1;  // bias-table entries per block
  using St = Staging<D, F32IN, kGroup>;
  static_assert(BIAS != kBiasTableF32 || kGroup >= BAND, "one bias-band entry per thread");
  using InT = typename std::conditional<F32IN, float, half_t>::type;
  constexpr int IES = sizeof(InT);  // bytes per input element
  static_assert(St::KCH >= 1 && kKB * D / 8 % kGroup == 0, "K tile split");

  // LDS: per key group two block slots, each K [KB][KLD] then V [KB][D]
  // (halves, swizzled chunks), followed for f32 input by the low halves of
  // both; reused after the loop for the key-group merge.
  constexpr int KHALF = kKB * KLD;
  constexpr int LO = KHALF + kKB * D;  // offset of the low-half tiles
  constexpr int SLOT = F32IN ? 2 * LO : LO;
  __shared__ __attribute__((aligned(16))) half_t smem[KSPLIT * 2 * SLOT];
  __shared__ float sBias[KSPLIT][2][BIAS == kBiasTableF32 ? BAND + 1 : 1];

  const int tid = threadIdx.x;
  // Key group and wave index are wave-uniform; readfirstlane tells the
  // compiler so, which keeps branches on them scalar (not if-converted).
  const int kg = __builtin_amdgcn_readfirstlane(tid / kGroup);  // key group
  const int gtid = tid % kGroup;  // thread index within the key group
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(gtid >> 6);  // query slice (0..3)
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

  const InT* Qh = static_cast<const InT*>(p.Q) + (int64_t)bh * p.bh_stride_q;
  const InT* Kh = static_cast<const InT*>(p.K) + (int64_t)bh * p.bh_stride_kv;
  const InT* Vh = static_cast<const InT*>(p.V) + (int64_t)bh * p.bh_stride_kv;

  // Softmax constant c = |scale| log2(e) > 0; a negative scale flips Q.
  const bool neg = p.scale_log2 < 0.f;
  const float c = fmaxf(fabsf(p.scale_log2), 1.17549435e-38f);

  // Q fragments: B operand of S^T, lane holds Q[q][16*ks + 8*g .. +7].
  // Rows past N read as zeros (buffer bounds check).
  const int qrows = min(N - q0, kBM);
  const rsrc_t rsQ = make_rsrc(Qh + (int64_t)q0 * p.stride_q, (uint32_t)qrows * p.stride_q * IES);
  half8v qf[KS];
  half8v qlo[F32IN ? KS : 1];  // low halves of an f32 Q
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const uint32_t off = ((q - q0) * p.stride_q + 16 * ks + 8 * g) * IES;
    if constexpr (F32IN) {
      float4v f[2] = {__builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(rsQ, off, 0, 0)),
                      __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(rsQ, off + 16, 0, 0))};
      if (neg) { f[0] = -f[0]; f[1] = -f[1]; }
      split_f16(f, qf[ks], qlo[ks]);
    } else {
      half8v t = buf_load_half8(rsQ, off);
      qf[ks] = neg ? -t : t;
    }
  }

  // Key blocks this workgroup visits: [blk0, blk0 + nblk); group kg takes
  // blocks blk0 + kg + KSPLIT*i.  The masked kernels see the keys of the
  // window [q - wl, q + wr] of their queries only.
  const int wl = p.win_left, wr = p.win_right;
  const int kbeg = CAUSAL ? max(0, q0 - wl) : 0;
  const int kend = CAUSAL ? (int)min((int64_t)N, (int64_t)q0 + kBM + wr) : N;
  const int blk0 = kbeg / kKB;
  const int nblk = max(0, (kend + kKB - 1) / kKB - blk0);
  const int my_n = nblk > kg ? (nblk - kg + KSPLIT - 1) / KSPLIT : 0;
  const int iters = (nblk + KSPLIT - 1) / KSPLIT;  // uniform over the workgroup

  // Global -> register staging through per-block buffer resources: the
  // block's base and extent are scalar, each thread's byte offsets are
  // constant, and rows past N read as zeros.  The same number of loads is
  // issued every step (blocks past the end are clamped and never computed)
  // so the compiler's load counter stays exact across the loop.
  uint32_t k_off[St::KCH];
#pragma unroll
  for (int j = 0; j < St::KCH; ++j) {
    const int c8 = gtid + kGroup * j;
    k_off[j] = ((c8 / (D / 8)) * p.stride_kv + 8 * (c8 % (D / 8))) * IES;
  }
  const int kgu = kg;

  auto gload = [&](St& st, int i) {
    const int blk = blk0 + max(0, min(kgu + KSPLIT * i, nblk - 1));
    const int kb0 = blk * kKB;
    const uint32_t bytes = (uint32_t)min(N - kb0, kKB) * p.stride_kv * IES;
    const rsrc_t rk = make_rsrc(Kh + (int64_t)kb0 * p.stride_kv, bytes);
    const rsrc_t rv = make_rsrc(Vh + (int64_t)kb0 * p.stride_kv, bytes);
    auto ld = [&](Piece8<F32IN>& d, rsrc_t r, uint32_t off) {
      if constexpr (F32IN) {
        d.f[0] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
        d.f[1] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0));
      } else {
        d.h = buf_load_half8(r, off);
      }
    };
#pragma unroll
    for (int j = 0; j < St::KCH; ++j) ld(st.k[j], rk, k_off[j]);
#pragma unroll
    for (int j = 0; j < St::KCH; ++j) ld(st.v[j], rv, k_off[j]);
    if (BIAS == kBiasTableF32) {
      // Band of table[h][q - key + N - 1] for q in [q0, q0+BM), key in
      // [kb0, kb0+KB): entry i is index q0 - kb0 - (KB-1) + N - 1 + i;
      // indices outside [0, 2N-2] read as zero.
      const int idx = q0 - kb0 - (kKB - 1) + N - 1 + gtid;
      const rsrc_t rb = make_rsrc(static_cast<const float*>(p.bias) + (int64_t)bh * p.bias_stride_h,
                                  (uint32_t)(2 * N - 1) * 4);
      st.b = buf_load_f32(rb, elem_offset(idx, 2 * N - 1, 4));
    }
  };

  auto sstore = [&](const St& st, int buf) {
    half_t* k_l = &smem[(kg * 2 + buf) * SLOT];
    half_t* v_l = k_l + KHALF;
#pragma unroll
    for (int j = 0; j < St::KCH; ++j) {
      const int c8 = gtid + kGroup * j;
      const int at = (c8 / (D / 8)) * KLD + 8 * (c8 % (D / 8));
      if constexpr (F32IN) {
        half8v hi, lo;
        split_f16(st.k[j].f, hi, lo);
        *reinterpret_cast<half8v*>(&k_l[at]) = hi;
        *reinterpret_cast<half8v*>(&k_l[LO + at]) = lo;
      } else {
        *reinterpret_cast<half8v*>(&k_l[at]) = st.k[j].h;
      }
    }
#pragma unroll
    for (int j = 0; j < St::KCH; ++j) {
      const int c8 = gtid + kGroup * j;
      const int at = v_store_at<D>(c8 / (D / 8), c8 % (D / 8));
      if constexpr (F32IN) {
        half8v hi, lo;
        split_f16(st.v[j].f, hi, lo);
        *reinterpret_cast<half8v*>(&v_l[at]) = hi;
        *reinterpret_cast<half8v*>(&v_l[LO + at]) = lo;
      } else {
        *reinterpret_cast<half8v*>(&v_l[at]) = st.v[j].h;
      }
    }
    if (BIAS == kBiasTableF32) {
      if (gtid < BAND) sBias[kg][buf][gtid] = st.b * kLog2e;
    }
  };

  float m_run = -INFINITY;  // running max (scaled log2 units), same in lanes l, l^32
  float l_run = 0.f;        // this lane's partial row sum
  float16v o[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) o[u] = float16v{};
  const int krow = kRowPerm(ql);
  const half2v ones = {(half_t)1.f, (half_t)1.f};

  // Dense f16 bias (the reference's rel-pos mode) with every row 16-byte
  // aligned (kBiasDenseF16Row16: N, the head stride and the base multiples
  // of 8 halves): lane (ql, g) needs B[q][kb0 + 32 t + 16 h + 8 g + 0..7]
  // for tile t and half h of a block, eight consecutive halves, one 16-byte
  // load.  They are issued one step ahead into a two-block register ring
  // (block i in slot i % 2), so their latency (the bias is read once, from
  // HBM) overlaps the previous block's work.  Block indices are clamped
  // like the K/V loads, so every step issues the same loads.  Rows and keys
  // past N read zeros or the next row's values; every such key is masked.
  // Unaligned rows (kBiasDenseF16) are read element by element when the
  // scores are formed.
  constexpr bool kDense = BIAS == kBiasDenseF16Row16;
  half8v bb[kDense ? 2 : 1][kDense ? 2 * NT : 1];
  const rsrc_t rsB = make_rsrc(
      kDense ? static_cast<const half_t*>(p.bias) + (int64_t)bh * p.bias_stride_h : nullptr,
      kDense ? (uint32_t)((int64_t)N * N * 2) : 0u);
  auto bias_load = [&](int i, int slot) {
    if constexpr (kDense) {
      const int kb0 = (blk0 + max(0, min(kgu + KSPLIT * i, nblk - 1))) * kKB;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          bb[slot][2 * t + h] =
              buf_load_half8(rsB, (uint32_t)(q * N + kb0 + 32 * t + 16 * h + 8 * g) * 2u);
        }
    }
  };

  auto compute = [&](int i, int buf) {
    const int kb0 = (blk0 + kg + KSPLIT * i) * kKB;
    // A wave whose 32 queries all miss this key block has nothing to do.
    if (CAUSAL && (kb0 > qw0 + 31 + wr || kb0 + kKB - 1 < qw0 - wl)) return;
    const half_t* k_l = &smem[(kg * 2 + buf) * SLOT];
    const half_t* v_l = k_l + KHALF;

    // ---- S^T = K Q^T for NT 32-key tiles ----
    float16v s[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      s[t] = float16v{};
      const half_t* kp = &k_l[(32 * t + krow) * KLD + 8 * g];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const half8v kh = load_half8(kp + 16 * ks);
        s[t] = mfma32x32x16(kh, qf[ks], s[t]);
        if constexpr (F32IN) {  // + K_hi Q_lo + K_lo Q_hi
          s[t] = mfma32x32x16(kh, qlo[ks], s[t]);
          s[t] = mfma32x32x16(load_half8(kp + LO + 16 * ks), qf[ks], s[t]);
        }
      }
    }

    // ---- logits x (scaled log2 units for bias modes, raw s otherwise) ----
    // Masked: the block runs past N, or some key of it is outside the
    // window of some query of this wave.
    const bool masked =
        (kb0 + kKB > N) || (CAUSAL && (kb0 + kKB - 1 > qw0 + wr || kb0 < qw0 + 31 - wl));
    if (BIAS != kBiasNone) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kr = 32 * t + 16 * (r >> 3) + 8 * g + (r & 7);  // key - kb0
          if constexpr (kDense) {
            // Reference semantics: (QK^T + B) * scale, B dense [T, T] f16
            // (prefetched by bias_load; keys past N are masked below).
            const float b = (float)(buf ? bb[1][2 * t + (r >> 3)][r & 7] : bb[0][2 * t + (r >> 3)][r & 7]);
            s[t][r] = (s[t][r] + (neg ? -b : b)) * c;
          } else if constexpr (BIAS == kBiasDenseF16) {
            const int key = kb0 + kr;
            const half_t* bp = static_cast<const half_t*>(p.bias) +
                               (int64_t)bh * p.bias_stride_h;
            const float b = (q < N && key < N) ? (float)bp[(int64_t)q * N + key] : 0.f;
            s[t][r] = (s[t][r] + (neg ? -b : b)) * c;
          } else {
            // BASELINE semantics: QK^T * scale + table[h][q - key + N - 1].
            s[t][r] = __builtin_fmaf(s[t][r], c, sBias[kg][buf][(q - q0) - kr + (kKB - 1)]);
          }
        }
      }
    }
    if (masked) {
      // Keeps this a real (scalar) branch: if-converted, the masking would
      // cost 64 VALU ops on every block instead of on the few masked ones.
      asm volatile("");
      // Keys outside [lo, lim) (relative to kb0 + 8g) are invisible to this
      // lane's query.
      const int lim = (CAUSAL ? (int)min((int64_t)N, (int64_t)q + wr + 1) : N) - kb0 - 8 * g;
      const int lo = (CAUSAL ? q - wl : 0) - kb0 - 8 * g;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kr = 32 * t + 16 * (r >> 3) + (r & 7);
          if (kr >= lim || kr < lo) s[t][r] = -INFINITY;
        }
    }

    // ---- online softmax with lazy rescale ----
    // Tree reduction (independent v_max3 chains per 8 values).
    float m8[2 * NT];
#pragma unroll
    for (int cc = 0; cc < 2 * NT; ++cc) {
      const float16v& v = s[cc >> 1];
      const int o8 = 8 * (cc & 1);
      m8[cc] = fmaxf(fmaxf(fmaxf(v[o8], v[o8 + 1]), fmaxf(v[o8 + 2], v[o8 + 3])),
                     fmaxf(fmaxf(v[o8 + 4], v[o8 + 5]), fmaxf(v[o8 + 6], v[o8 + 7])));
    }
#pragma unroll
    for (int w = 1; w < 2 * NT; w *= 2)
#pragma unroll
      for (int cc = 0; cc + w < 2 * NT; cc += 2 * w) m8[cc] = fmaxf(m8[cc], m8[cc + w]);
    const float mx = max_halves(m8[0]);
    // Row max in scaled units (c > 0, so scaling is monotone).
    const float mx_c = (BIAS != kBiasNone || mx == -INFINITY) ? mx : mx * c;
    if (__any(mx_c > m_run + kLazyLog2)) {
      const float m_new = fmaxf(m_run, mx_c);
      // 0 on a row's first visible block; 1 while a row has seen no visible
      // key yet (a windowed row can miss a block its wave still visits).
      const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[u][r] *= alpha;
    }
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run;

    half8v pb[2 * NT];
    half8v pl[F32IN ? 2 * NT : 1];  // low halves of an f32 P
    float ls[2 * NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = (BIAS != kBiasNone) ? s[t][r] - m_use : __builtin_fmaf(s[t][r], c, -m_use);
        const float pv = fast_exp2(e);
        const half_t ph = (half_t)pv;
        pb[2 * t + (r >> 3)][r & 7] = ph;
        if constexpr (F32IN) {
          pl[2 * t + (r >> 3)][r & 7] = (half_t)(pv - (float)ph);
          if ((r & 7) == 0)
            ls[2 * t + (r >> 3)] = pv;
          else
            ls[2 * t + (r >> 3)] += pv;
        }
      }
    }
    // Row sum of the P that feeds the MFMA: the f32 P itself for split
    // input, else the fp16 P (one dot2 chain per chunk).
    if constexpr (!F32IN) {
#pragma unroll
      for (int cc = 0; cc < 2 * NT; ++cc) {
        const half8v& v8 = pb[cc];
        float a = __builtin_amdgcn_fdot2(half2v{v8[0], v8[1]}, ones, 0.f, false);
        a = __builtin_amdgcn_fdot2(half2v{v8[2], v8[3]}, ones, a, false);
        a = __builtin_amdgcn_fdot2(half2v{v8[4], v8[5]}, ones, a, false);
        ls[cc] = __builtin_amdgcn_fdot2(half2v{v8[6], v8[7]}, ones, a, false);
      }
    }
#pragma unroll
    for (int w = 1; w < 2 * NT; w *= 2)
#pragma unroll
      for (int cc = 0; cc + w < 2 * NT; cc += 2 * w) ls[cc] += ls[cc + w];
    l_run += ls[0];

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int u = 0; u < DT; ++u) {
      const int vo = v_tr_offset<D>(lane, u);
#pragma unroll
      for (int cc = 0; cc < 2 * NT; ++cc) {
        const half8v vh = v_frag_tr<D>(v_l, vo, cc);
        o[u] = mfma32x32x16(vh, pb[cc], o[u]);
        if constexpr (F32IN) {  // + V_hi P_lo + V_lo P_hi
          o[u] = mfma32x32x16(vh, pl[cc], o[u]);
          o[u] = mfma32x32x16(v_frag_tr<D>(v_l + LO, vo, cc), pb[cc], o[u]);
        }
      }
    }
  };

  // ---- pipelined main loop: loads two blocks ahead, LDS double buffer ----
  // Loads and LDS stores run unconditionally (blocks past the end are
  // clamped and never computed) so the load counter stays precise.
  St stA, stB;
  gload(stA, 0);
  gload(stB, 1);
  bias_load(0, 0);
  sstore(stA, 0);
  lds_barrier();

  auto step = [&](int i, int buf, St& cur, St& nxt) {
    gload(cur, i + 2);  // cur's block i is already in LDS
    bias_load(i + 1, buf ^ 1);
    if (i < my_n) compute(i, buf);
    sstore(nxt, buf ^ 1);
    lds_barrier();
  };
  // Always run both halves of the pair (the second may compute nothing) so
  // every path into the loop header has the same loads outstanding.
  for (int i = 0; i < iters; i += 2) {
    step(i, 0, stA, stB);
    step(i + 1, 1, stB, stA);
  }

  // ---- merge the key groups ----
  // Groups 1..KSPLIT-1 publish (m, l, O) per lane; group 0 folds them in
  // order.  Lane layout is identical across groups (same query slice).
  if constexpr (KSPLIT > 1) {
    constexpr int SLOTS = 16 * DT + 2;
    constexpr int PART = QW * SLOTS * 64;  // floats per published group
    static_assert(sizeof(smem) >= (size_t)(KSPLIT - 1) * PART * sizeof(float), "merge buffer");
    float* red = reinterpret_cast<float*>(smem) + (size_t)wave * SLOTS * 64 + lane;
    if (kg > 0) {
      float* mine = red + (size_t)(kg - 1) * PART;
      mine[0] = m_run;
      mine[64] = l_run;
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) mine[(2 + 16 * u + r) * 64] = o[u][r];
    }
    lds_barrier();
    if (kg != 0) return;
#pragma unroll
    for (int j = 0; j < KSPLIT - 1; ++j) {
      const float* other = red + (size_t)j * PART;
      const float m1 = other[0];
      const float l1 = other[64];
      const float mm = fmaxf(m_run, m1);
      const float mu = (mm == -INFINITY) ? 0.f : mm;
      const float a0 = fast_exp2(m_run - mu);
      const float a1 = fast_exp2(m1 - mu);
      m_run = mm;
      l_run = l_run * a0 + l1 * a1;
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[u][r] = o[u][r] * a0 + other[(2 + 16 * u + r) * 64] * a1;
    }
  }

  // ---- normalise and store: lane holds O[q][32u + 8b + 4g + 0..3] ----
  // Rows past N fall outside the buffer resource and are dropped.
  const float l_tot = sum_halves(l_run);
  const float inv = 1.f / fmaxf(l_tot, 1e-6f);
  constexpr int ES = OUT_F16 ? 2 : 4;
  const rsrc_t rsO = make_rsrc(static_cast<char*>(p.O) +
                                   ((int64_t)bh * p.bh_stride_o + (int64_t)q0 * p.stride_o) * ES,
                               (uint32_t)qrows * p.stride_o * ES);
#pragma unroll
  for (int u = 0; u < DT; ++u) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int col = 32 * u + 8 * b + 4 * g;
      const uint32_t off = ((q - q0) * p.stride_o + col) * ES;
      float4v v = {o[u][4 * b] * inv, o[u][4 * b + 1] * inv, o[u][4 * b + 2] * inv,
                   o[u][4 * b + 3] * inv};
      if (OUT_F16) {
        buf_store_f16x4(half4v{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]}, rsO, off);
      } else {
        buf_store_f32x4(v, rsO, off);
      }
    }
  }
}

// Static LDS of one workgroup with K key groups.
template <int D, int BIAS, bool F32IN, int QW>
constexpr int fa2_lds_bytes(int K) {
  constexpr int kb = key_block<D, F32IN>();
  const int slot = (kb * (D + 8) + kb * D) * 2 * (F32IN ? 2 : 1);
  const int bias = BIAS == kBiasTableF32 ? (32 * QW + kb) * 4 : 4;
  return K * 2 * (slot + bias);
}

// Launches with K key groups if their LDS fits (returns false otherwise).
template <int D, bool CAUSAL, int BIAS, bool OUT_F16, int K, bool F32IN, int QW>
bool launch_fa2_k(Fa2Args a, hipStream_t stream, hipError_t& err) {
  if constexpr (fa2_lds_bytes<D, BIAS, F32IN, QW>(K) <= 160 * 1024) {
    a.num_qblocks = (a.N + 32 * QW - 1) / (32 * QW);
    err = launch<&fa2_fwd_kernel<D, CAUSAL, BIAS, OUT_F16, K, F32IN, QW>>(
        ktag("fa2_fwd_kernel", D, CAUSAL, BIAS, OUT_F16, K, F32IN, QW),
        dim3(a.num_qblocks * a.batch_heads), dim3(K * 64 * QW), stream, a);
    return true;
  }
  return false;
}

template <int D, bool CAUSAL, int BIAS, bool OUT_F16, bool F32IN, int QW>
hipError_t launch_fa2_q(const Fa2Args& a, int ksplit, hipStream_t stream) {
  // Use the requested key split, or the largest smaller one whose LDS fits.
  hipError_t err = hipSuccess;
  bool done = false;
  if (ksplit >= 4) done = launch_fa2_k<D, CAUSAL, BIAS, OUT_F16, 4, F32IN, QW>(a, stream, err);
  if (!done && ksplit >= 3)
    done = launch_fa2_k<D, CAUSAL, BIAS, OUT_F16, 3, F32IN, QW>(a, stream, err);
  if (!done && ksplit >= 2)
    done = launch_fa2_k<D, CAUSAL, BIAS, OUT_F16, 2, F32IN, QW>(a, stream, err);
  if (!done) launch_fa2_k<D, CAUSAL, BIAS, OUT_F16, 1, F32IN, QW>(a, stream, err);
  return err;
}

// Query waves per key group: 4 (128-query workgroups), or 2 (64-query
// workgroups) when a.qwaves says so (see launch_fa2).
template <int D, bool CAUSAL, int BIAS, bool OUT_F16, bool F32IN = false>
hipError_t launch_fa2_t(const Fa2Args& a, int ksplit, hipStream_t stream) {
  return a.qwaves == 2 ? launch_fa2_q<D, CAUSAL, BIAS, OUT_F16, F32IN, 2>(a, ksplit, stream)
                       : launch_fa2_q<D, CAUSAL, BIAS, OUT_F16, F32IN, 4>(a, ksplit, stream);
}

template <int D, int BIAS, bool OUT_F16>
hipError_t launch_fa2_c(const Fa2Args& a, bool causal, int ksplit, hipStream_t s) {
  if constexpr (BIAS == kBiasNone) {
    if (causal) return launch_fa2_t<D, true, BIAS, OUT_F16>(a, ksplit, s);
  } else {
    if (causal) return hipErrorInvalidValue;  // the biased entry point is never causal
  }
  return launch_fa2_t<D, false, BIAS, OUT_F16>(a, ksplit, s);
}

// f32 Q/K/V (split into f16 hi + lo), no bias, f32 output.
hipError_t launch_fa2_f32in(const Fa2Args& a, int d, bool causal, int ksplit, hipStream_t s) {
  switch (d) {
    case 32:
      return causal ? launch_fa2_t<32, true, kBiasNone, false, true>(a, ksplit, s)
                    : launch_fa2_t<32, false, kBiasNone, false, true>(a, ksplit, s);
    case 64:
      return causal ? launch_fa2_t<64, true, kBiasNone, false, true>(a, ksplit, s)
                    : launch_fa2_t<64, false, kBiasNone, false, true>(a, ksplit, s);
    case 128:
      return causal ? launch_fa2_t<128, true, kBiasNone, false, true>(a, ksplit, s)
                    : launch_fa2_t<128, false, kBiasNone, false, true>(a, ksplit, s);
    default: return hipErrorInvalidValue;
  }
}

template <int BIAS, bool OUT_F16>
hipError_t launch_fa2_d(const Fa2Args& a, int d, bool causal, int ksplit, hipStream_t s) {
  switch (d) {
    case 32: return launch_fa2_c<32, BIAS, OUT_F16>(a, causal, ksplit, s);
    case 64: return launch_fa2_c<64, BIAS, OUT_F16>(a, causal, ksplit, s);
    case 128: return launch_fa2_c<128, BIAS, OUT_F16>(a, causal, ksplit, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int fa2_query_block() { return kBM; }  // the largest query block of any FA2 kernel

hipError_t launch_fa2(Fa2Args a, int head_dim, bool causal, int bias_kind, bool out_f16,
                      hipStream_t stream, bool in_f32) {
  a.num_qblocks = (a.N + kBM - 1) / kBM;
  // Split the keys of a workgroup over two wave groups when the grid alone
  // gives fewer than two workgroups per compute unit.  Causal grids, whose
  // workgroups differ in work by up to N / 128 times, keep the split up to
  // four workgroups per CU: eight-wave workgroups run one per CU and the
  // longest-first order then evens the rounds out (measured, 1 -> 2 key
  // groups: d64 B1 H16 N4096 71.5 -> 51.1 us, d128 B1 H32 N4096 204 ->
  // 174 us, equal or better up to 1024 workgroups; 4-5% worse at 2048).
  const int64_t wgs = (int64_t)a.num_qblocks * a.batch_heads;
  const int64_t cus = device_cu_count();
  const bool full_causal = causal && a.win_left >= a.N && a.win_right == 0;
  int ksplit = (a.ksplit > 0)                             ? a.ksplit
               : (wgs < 2 * cus || (full_causal && wgs <= 4 * cus)) ? 2
                                                                     : 1;
  // Small grid: 128-query workgroups fill at most half the compute units.
  const bool small = 2 * wgs <= cus;
  // The fast kernel carries a bias table in score units (t / |scale|),
  // which needs a scale whose reciprocal stays finite.
  const bool bias = bias_kind != kBiasNone;
  const bool fast_ok = a.allow_fast && fa2_fast_supported(head_dim, bias_kind, in_f32) &&
                       (!bias || fabsf(a.scale_log2) >= 1e-20f);
  if (fast_ok && (a.allow_fast == 2 || fa2_fast_preferred(causal, a.N, head_dim, small, bias))) {
    // Causal grids of at least two workgroups per CU: each workgroup takes a
    // long and a short query block (pair_qblocks), which evens out the work,
    // and the key split then follows the halved grid (fast kernel, measured:
    // d128 B2 H32 N4096 356.6 -> 331.6 us, d64 B1 H32 N4096 102.3 -> 92.1
    // us, d64 B1 H16 N4096 51.7 -> 49.4 us; at 256 workgroups pairing
    // would idle half the CUs).  NESO_AMD_FA2_PAIR = 0 / 1 forces it.
    // Below that, without a window: 64-row halves from opposite ends of the
    // rows, which halve the longest workgroup's work at one workgroup per CU.
    // head_dim 128, full causal, from N = 2048, where the paired 64-row
    // blocks fill at most one round: paired blocks on 64-query workgroups
    // with four key groups instead of 128-row halves, whose long-half waves
    // end up alone on their SIMDs (measured: d128 B1 H8 N4096 53.1 -> 49.1
    // us, B1 H16 N2048 32.1 -> 31.7; at d = 64 the halves stay ahead, H16
    // N2048 19.9 against 21.4).
    const int64_t pairs64 = (int64_t)(((a.N + 63) / 64 + 1) / 2) * a.batch_heads;
    if (head_dim == 128 && full_causal && a.N >= 2048 && pairs64 <= cus && a.pair_qblocks < 0 &&
        a.qwaves != 4 && !bias) {
      a.pair_qblocks = 1;
      a.qwaves = 2;
      if (a.ksplit <= 0) ksplit = 4;
    }
    if (a.pair_qblocks < 0)
      a.pair_qblocks = (full_causal && wgs >= 2 * cus) ? 1 : full_causal ? 2 : 0;
    if (causal && a.pair_qblocks == 1 && a.ksplit <= 0 && a.qwaves != 2) {
      const int64_t pwgs = (int64_t)((a.num_qblocks + 1) / 2) * a.batch_heads;
      ksplit = pwgs < 2 * cus ? 2 : 1;
    }
    // Small grids: 64-query workgroups (two query waves).  Four key groups
    // (eight waves, one workgroup per CU) while those workgroups fit the
    // CUs in one round and each group still sees 4+ key blocks; two
    // otherwise, where shorter rows make the split's prologue and merge
    // cost more (measured, d = 64: H8 N1500 12.7 vs 13.4 us, rel-pos H8
    // N2048 16.7 vs 18.3; H8 N512 7.3 vs 6.9).
    if (a.qwaves != 2 && a.qwaves != 4) a.qwaves = fa2_fast_qwaves(small, a.N, bias);
    if (a.qwaves == 2 && a.ksplit <= 0 && a.pair_qblocks != 1) {
      const int64_t wgs64 = (int64_t)((a.N + 63) / 64) * a.batch_heads;
      ksplit = (wgs64 <= cus && a.N >= 1024) ? 4 : 2;
    }
    return launch_fa2_fast(a, head_dim, causal, bias, out_f16, ksplit, stream);
  }
  // Generic kernel on a small grid: 64-query workgroups (two query waves per
  // key group) and four key groups double the grid, still one round of
  // workgroups, with eight waves each.  With more workgroups the doubled
  // grid takes two rounds (H12 N2048 d64: 34.4 us, the fast kernel 21.5).
  if (a.qwaves != 2 && a.qwaves != 4) a.qwaves = small ? 2 : 4;
  if (a.qwaves == 2 && a.ksplit <= 0) ksplit = 4;
  // head_dim 32: a block is cheap, so more key groups pay off sooner
  // (measured, B1 H16 N4096: causal 58.5 us with two groups, 41.3 with
  // three; non-causal 68.2 with one, 60.9 with two; 1024 causal workgroups
  // stay at two).
  if (head_dim == 32 && a.qwaves == 4 && a.ksplit <= 0)
    ksplit = full_causal ? (wgs <= 2 * cus ? 3 : wgs <= 4 * cus ? 2 : 1) : (wgs <= 2 * cus ? 2 : 1);
  if (in_f32) {
    if (bias_kind != kBiasNone || out_f16) return hipErrorInvalidValue;
    return launch_fa2_f32in(a, head_dim, causal, ksplit, stream);
  }
  if (bias_kind == kBiasNone) {
    return out_f16 ? launch_fa2_d<kBiasNone, true>(a, head_dim, causal, ksplit, stream)
                   : launch_fa2_d<kBiasNone, false>(a, head_dim, causal, ksplit, stream);
  }
  if (bias_kind == kBiasTableF32) {
    return out_f16 ? launch_fa2_d<kBiasTableF32, true>(a, head_dim, causal, ksplit, stream)
                   : launch_fa2_d<kBiasTableF32, false>(a, head_dim, causal, ksplit, stream);
  }
  // Dense bias rows that all start 16-byte aligned take 16-byte loads (the
  // kernel forms 32-bit offsets into one head's N x N bias: N <= 32768).
  if (a.N % 8 == 0 && a.N <= 32768 && a.bias_stride_h % 8 == 0 &&
      (reinterpret_cast<uintptr_t>(a.bias) & 15) == 0)
    return out_f16 ? launch_fa2_d<kBiasDenseF16Row16, true>(a, head_dim, causal, ksplit, stream)
                   : launch_fa2_d<kBiasDenseF16Row16, false>(a, head_dim, causal, ksplit, stream);
  return out_f16 ? launch_fa2_d<kBiasDenseF16, true>(a, head_dim, causal, ksplit, stream)
                 : launch_fa2_d<kBiasDenseF16, false>(a, head_dim, causal, ksplit, stream);
}

}  // namespace neso
