// Flash-Attention-2 forward for fp16 Q/K/V without a bias: the fast path.
//
// Same algorithm and result as fa2_fwd_kernel (reference: the TTIR loop of
// `flash_attention_fwd`, tests/test_flash_attention.py:79-247; final
// O / max(l, 1e-6), src/neso/backend/codegen/lowering.py:4352-4353), with the
// per-score work cut to what the transcendental unit and the P conversion
// need.  Tile layout as in fa2_fwd.hip: a key group is 4 waves and 128
// queries, each wave owns 32 queries, scores are computed transposed
// (S^T = K Q^T, v_mfma_f32_32x32x16_f16) so that lane l holds 32 keys of query
// l % 32 and exp(S^T) in fp16 is directly the B operand of O^T = V^T P^T.
//
// What differs:
// * No row max per block.  The running max m only has to keep p = 2^(c s - m)
//   (c = |scale| log2(e)) in fp16 range, not equal the row max, so each lane
//   compares the sum of its 32 fp16 P values (needed for l anyway, from
//   v_dot2_f32_f16) with 2^12.  A block over the bound, a row's first
//   visible block and every block with masked keys take the slow path:
//   exact row max, m raised to it, O and l rescaled, P redone.  As m only
//   rises and starts at a row's first block max, l >= 1 once a row has seen
//   a key, so p cannot underflow the whole row.  A score then costs one FMA,
//   one v_exp_f32, half a v_cvt_pk_f16_f32 and half a v_dot2_f32_f16.
// * Software pipeline: block i+1's scores (MFMA) are issued in the same
//   straight-line stretch as block i's softmax (VALU), so the matrix unit and
//   the VALU work at the same time inside one wave; two waves per SIMD (two
//   key groups) fill the remaining gaps.  K and V of a block share one
//   slot of a 4-slot LDS ring, which leaves one barrier per block and keeps
//   block i's K in LDS while block i is processed (the slow path recomputes
//   its scores from there).
// * K and V go from global memory straight into LDS (buffer_load_dwordx4
//   ... lds, no staging registers, no LDS stores): step i issues block
//   i+2's loads into its free slot before the fused stretch and waits for
//   them before the step's barrier.  Both tiles are row-major without
//   padding, 16-byte chunks swizzled against bank conflicts, and the V^T
//   operand of P V is read with gfx950's transposing LDS load,
//   ds_read_b64_tr_b16.
#include <type_traits>

#include "common.h"
#include "fa2_tiles.h"
#include "neso_internal.h"

namespace neso {

namespace {

constexpr float kPSumMax = 4096.f;  // fast-path bound on a lane's block sum of P
constexpr float kLog2e = 1.4426950408889634f;

// LDS layout of a key group's K and V tiles, both row-major with 16-byte
// chunks swizzled (no padding: the blocks arrive by LDS-direct loads, which
// fill LDS linearly).
// * Ring: a 4-slot ring, each slot K [KB][D] then V [KB][D].
// * Live: two K slots and two V slots.  The scores of a block stay in
//   registers for its slow path, so a block's K is free once its scores are
//   formed, and its V is loaded one step before its P V.  Used by every
//   two-query-wave kernel, and at head_dim 128 with four query waves
//   (without a bias or 64-row halves), where it fits 64-key blocks; not
//   for paired blocks with one key group, whose 276 registers per wave
//   leave one workgroup per CU (measured, B2 H32 N4096 causal: 360 against
//   341 us in the ring; other d = 128 shapes 2-6% faster in this layout).
template <int D, int QW, bool BIAS, bool HALVES, bool PAIR, int K>
constexpr bool fast_live() {
  return QW == 2 || (D == 128 && !BIAS && !HALVES && !(PAIR && K == 1));
}

// Keys per block: 64 at head_dim 64 and 32 at head_dim 128 in the ring, so
// that a block step carries 16 MFMAs per wave (8 for its scores, 8 for its
// P V); 64 at head_dim 128 in the live layout with four query waves (32
// MFMAs per step: half the steps, and half their barriers and pipeline
// fills); 32 for the bias table with four query waves (whose band of
// 32 + KB - 1 entries is then one per lane).
template <int D, int QW, bool BIAS, bool HALVES, bool PAIR, int K>
constexpr int fast_kb() {
  if (D == 128) return (QW == 4 && fast_live<D, QW, BIAS, HALVES, PAIR, K>()) ? 64 : 32;
  return (BIAS && QW == 4) ? 32 : 64;
}

constexpr int kSlots = 4;
template <int D, int QW, bool BIAS, bool HALVES, bool PAIR, int K>
constexpr int fast_group_lds_halves() {
  return (fast_live<D, QW, BIAS, HALVES, PAIR, K>() ? 4 : kSlots * 2) *
         fast_kb<D, QW, BIAS, HALVES, PAIR, K>() * D;
}

// Bias band slot of one wave: the band's 32 + KB - 1 entries, rounded up.
template <int D, int QW, bool BIAS, bool HALVES, bool PAIR, int K>
constexpr int fast_band_slot() {
  return fast_kb<D, QW, BIAS, HALVES, PAIR, K>() == 64 ? 128 : 64;
}

// Floats past the band slots that reads of masked keys (past N) may touch
// when the slots hold the workgroup's whole table range.
constexpr int kFastTabPad = 64;

// Bytes of LDS of one workgroup: the key groups' tiles, and with a bias two
// band slots per wave (or the table range, in the same space).
template <int D, int QW, bool BIAS, bool HALVES, bool PAIR, int K>
constexpr int fast_lds_bytes() {
  return K * (fast_group_lds_halves<D, QW, BIAS, HALVES, PAIR, K>() * 2 +
              (BIAS ? QW * 2 * fast_band_slot<D, QW, BIAS, HALVES, PAIR, K>() * 4 : 0)) +
         (BIAS ? kFastTabPad * 4 : 0);
}

// Debug build (NESO_FA2_SERIAL_LDS): every LDS phase ends in a full wait and
// a workgroup barrier, so no LDS-DMA write overlaps any LDS read and no wave
// runs ahead of another within a step.  It must give bit-identical results
// to the pipelined ring; a race in the ring's slot bookkeeping would show up
// as a difference.  The pipelined build compiles this to nothing.
__device__ __forceinline__ void serial_lds_point() {
#ifdef NESO_FA2_SERIAL_LDS
  wait_vmem();
  lds_barrier();
#endif
}

// PAIR (causal only): each workgroup takes two query blocks, see below.
// HALVES (full causal only): each workgroup takes two 64-row query blocks
// from opposite ends, see below.
// QW: query waves per key group (4: 128-query workgroups, 2: 64-query
// workgroups, which double a small grid).
// BIAS (unmasked only): logits = Q K^T * scale + table[h][i - j + N - 1]
// (the f32 table of the relative-position entry point).  The table entries
// enter as the initial accumulator of the score MFMAs, in score units
// (t / |scale|), so that c * s is the biased logit in log2 units and the
// softmax is the unbiased one.
template <int D, bool CAUSAL, bool OUT_F16, int KSPLIT, bool PAIR = false, bool HALVES = false,
          int QW = 4, bool BIAS = false, bool TAB = false>
__global__ __launch_bounds__(64 * QW * KSPLIT) void fa2_fast_kernel(Fa2Args p) {
  static_assert(!PAIR || CAUSAL, "paired query blocks are for causal grids");
  static_assert(!HALVES || (CAUSAL && !PAIR), "64-row halves are for full causal grids");
  static_assert(QW == 4 || (QW == 2 && !HALVES), "query waves");
  static_assert(!BIAS || !CAUSAL, "the biased entry point is never masked");
  static_assert(!TAB || BIAS, "the table range is a bias layout");
  constexpr int kBMq = 32 * QW;      // queries per workgroup
  constexpr int kGroup = 64 * QW;    // threads per key group
  constexpr int kKB = fast_kb<D, QW, BIAS, HALVES, PAIR, KSPLIT>();  // keys per block
  constexpr int NT = kKB / 32;  // 32-key tiles per block
  constexpr int KS = D / 16;    // k-steps of S^T = K Q^T
  constexpr int DT = D / 32;    // 32-row tiles of O^T
  constexpr int KSLOT = kKB * D;
  constexpr int VSLOT = kKB * D;
  constexpr int GLDS = fast_group_lds_halves<D, QW, BIAS, HALVES, PAIR, KSPLIT>();
  constexpr int LCH = kKB * D / 8 / 64 / QW;  // 1 KiB load instructions per wave and matrix
  constexpr int CPR = D / 8;      // 16-byte chunks per K/V row
  constexpr int RPI = 64 / CPR;   // rows per 1 KiB load instruction
  static_assert(LCH >= 1 && kKB * D * 2 == QW * LCH * 1024 && RPI * D == 512, "tile split");
  // K and V slots of the live layout, scores kept for the slow path (see
  // fast_live).
  constexpr bool kLive = fast_live<D, QW, BIAS, HALVES, PAIR, KSPLIT>();
  // Ring layout at head_dim 64 without a bias: Q arrives by LDS-DMA into
  // ring slot 3 of key group 0 (free until step 1 loads block 3), so that no
  // load the compiler tracks is in flight and the prologue can wait for Q
  // and the first K tiles alone (counted vmcnt) while the later tiles land
  // under block 0's softmax.
  constexpr bool kQLds = !kLive && !BIAS && D == 64;
  // The same for the live layout with two query waves and 64-key blocks: Q
  // (64 rows) in V slot 1 of key group 0, free until step 1 loads V of
  // block 1.  The bias
  // band's prologue loads are issued untracked (band_load_untracked) for
  // the same reason.
  constexpr bool kQLive = kLive && QW == 2 && !HALVES && 32 * QW <= kKB;
  constexpr bool kQStage = kQLds || kQLive;
  constexpr int BSLOT = fast_band_slot<D, QW, BIAS, HALVES, PAIR, KSPLIT>();
  static_assert(!BIAS || 32 + kKB - 1 <= 2 * 64, "two band entries per lane");
  __shared__ __attribute__((aligned(16))) half_t smem[KSPLIT * GLDS];
  // Bias band: two slots per wave (its own, no barrier); or the whole
  // table range of the workgroup's rows, in the same space (see use_tab).
  constexpr int kTabCap = KSPLIT * QW * 2 * BSLOT;
  __shared__ float sband[BIAS ? kTabCap + kFastTabPad : 1];
  float* const stab = sband;

  const int tid = threadIdx.x;
  const int kg = __builtin_amdgcn_readfirstlane(tid / kGroup);  // key group
  const int gtid = tid % kGroup;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(gtid >> 6);  // query slice (0..QW-1)
  const int g = lane >> 5;
  const int ql = lane & 31;

  // Workgroup x of head bh takes query block nqb - 1 - x (causal: longest
  // rows first) or x.  With PAIR it then also takes block x, so that every
  // workgroup does the work of nqb + 1 blocks' rows.  With HALVES it takes
  // the 64-row blocks x and n64 - 1 - x (n64 = 64-row blocks of N): every
  // workgroup sees about N + 64 keys in total over its 128 rows, half the
  // work of an unmasked block, so causal grids of one workgroup per CU finish
  // in about half the time instead of waiting for the longest block.
  const uint32_t wg = xcd_swizzle(blockIdx.x, gridDim.x);
  const int nqb = p.num_qblocks;
  const int n64 = (p.N + 63) / 64;
  const int wph = PAIR ? (nqb + 1) / 2 : HALVES ? (n64 + 1) / 2 : nqb;  // workgroups per head
  const int bh = wg / wph;
  const int x = wg % wph;

  auto run = [&](const int qblk) {
  const int N = p.N;
  // This wave's 32 query rows start at qw0.  With HALVES, query slice sl of
  // the workgroup's 128 rows is rows 32 (sl % 2) .. of the short block (sl <
  // 2) or of the long block (sl >= 2); with two key groups the second group's
  // waves take the slices two apart (sl = wave ^ 2), so that each SIMD,
  // which holds wave w of both groups, runs one short-block and one
  // long-block wave.  A middle block paired with itself leaves the long
  // half empty (qw0 = N: no rows).
  int q0, qw0, sl = wave;
  if constexpr (HALVES) {
    if (KSPLIT == 2) sl = wave ^ (2 * kg);
    const int hs = qblk, hl = n64 - 1 - qblk;
    q0 = hs * 64;
    qw0 = sl < 2 ? hs * 64 + 32 * sl : (hl == hs ? N : hl * 64 + 32 * (sl - 2));
  } else {
    q0 = qblk * kBMq;
    qw0 = q0 + wave * 32;
  }
  const int q = qw0 + ql;

  const half_t* Qh = static_cast<const half_t*>(p.Q) + (int64_t)bh * p.bh_stride_q;
  const half_t* Kh = static_cast<const half_t*>(p.K) + (int64_t)bh * p.bh_stride_kv;
  const half_t* Vh = static_cast<const half_t*>(p.V) + (int64_t)bh * p.bh_stride_kv;

  // Q fragments (B operand of S^T); a negative scale flips Q so that
  // c = |scale| log2(e) > 0 (kept above 0 so that -inf * c stays -inf).
  // Rows past N read as zeros.
  const bool neg = p.scale_log2 < 0.f;
  const float c = fmaxf(fabsf(p.scale_log2), 1.17549435e-38f);
  // Rows addressed from qb: the workgroup's first row, or with HALVES the
  // wave's own (its two halves are not contiguous).
  const int qb = HALVES ? qw0 : q0;
  const int qrows = HALVES ? max(0, min(N - qw0, 32)) : min(N - q0, kBMq);
  const rsrc_t rsQ = make_rsrc(Qh + (int64_t)qb * p.stride_q, (uint32_t)qrows * p.stride_q * 2);
  half8v qf[KS];
  if constexpr (!kQStage) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const half8v t = buf_load_half8(rsQ, ((q - qb) * p.stride_q + 16 * ks + 8 * g) * 2);
      qf[ks] = neg ? -t : t;
    }
  }

  // Key blocks of this workgroup: [blk0, blk0 + nblk); group kg takes blocks
  // blk0 + kg + KSPLIT*i.  Masked kernels visit the keys of their queries'
  // windows [q - wl, q + wr] only.
  const int wl = p.win_left, wr = p.win_right;
  // With HALVES (full causal, wr = 0) the keys run from 0 to the end of the
  // long block, and each wave stops after the last block any of its rows
  // sees: its first my_nw of the group's my_n blocks (the group's loads go
  // on to my_n).
  const int kbeg = CAUSAL ? max(0, q0 - wl) : 0;
  const int kend = HALVES ? min(N, (n64 - q0 / 64) * 64 + wr)
                 : CAUSAL ? (int)min((int64_t)N, (int64_t)q0 + kBMq + wr) : N;
  const int blk0 = kbeg / kKB;
  const int nblk = max(0, (kend + kKB - 1) / kKB - blk0);
  const int my_n = nblk > kg ? (nblk - kg + KSPLIT - 1) / KSPLIT : 0;
  const int iters = (nblk + KSPLIT - 1) / KSPLIT;  // uniform over the workgroup
  int my_nw = my_n;
  if constexpr (HALVES) {
    const int last = qw0 >= N ? -1 : min(N - 1, qw0 + 31 + wr) / kKB - blk0 - kg;
    my_nw = last < 0 ? 0 : min(my_n, last / KSPLIT + 1);
  }

  half_t* gbase = &smem[kg * GLDS];
  // Four query waves: slot s of the ring holds K then V.  Two: K slots 0
  // and 1, then V slots 0 and 1.
  auto kslot = [&](int s) { return kLive ? gbase + s * KSLOT : gbase + s * (KSLOT + VSLOT); };
  auto vslot = [&](int s) {
    return kLive ? gbase + 2 * KSLOT + s * VSLOT : gbase + s * (KSLOT + VSLOT) + KSLOT;
  };
  // The slots as LDS byte addresses (the M0 operand of the LDS-direct
  // loads), at this wave's first 1 KiB piece (x = LCH wave): a scalar base
  // plus a constant.  The empty asm makes each use re-add the constant to
  // the one base register in the scalar unit, instead of the compiler
  // hoisting every slot's address out of the loop into VGPR lanes (a
  // v_readlane per load).
  const uint32_t wbase_lds = lds_addr(smem) + (uint32_t)(kg * GLDS * 2 + LCH * wave * RPI * D * 2);
  auto lds_base = [&]() {
    uint32_t b = wbase_lds;
    asm volatile("" : "+s"(b));
    return b;
  };
  auto kslot_lds = [&](int s) {
    return lds_base() + (uint32_t)((kLive ? s * KSLOT : s * (KSLOT + VSLOT)) * 2);
  };
  auto vslot_lds = [&](int s) {
    return lds_base() + (uint32_t)((kLive ? 2 * KSLOT + s * VSLOT : s * (KSLOT + VSLOT) + KSLOT) * 2);
  };
  // Bytes of K (or V) from key row kb0 to the end of the block (the
  // descriptor's extent: rows past N read as zeros).  Scalar arithmetic
  // only: a descriptor in VGPRs would wrap every load in a waterfall loop.
  auto block_bytes = [&](int kb0) {
    const int rem = N - kb0;
    return (uint32_t)((rem < kKB ? rem : kKB) * p.stride_kv * 2);
  };

  // Global -> LDS directly (buffer_load_dwordx4 ... lds).  One instruction
  // fills 1 KiB of LDS, lane l's 16 bytes at byte 16 l, i.e. RPI rows of a
  // block; so lane l loads the chunk that the swizzled layout puts at its
  // position: row RPI x + l / CPR (x = instruction of the group), position
  // l % CPR, chunk (l % CPR) ^ swizzle(row).  Rows past N read as zeros.
  uint32_t kgo[LCH], vgo[LCH];
#pragma unroll
  for (int j = 0; j < LCH; ++j) {
    const int row = RPI * (LCH * wave + j) + lane / CPR, pos = lane % CPR;
    kgo[j] = (row * p.stride_kv + 8 * (pos ^ kswz<D>(row))) * 2;
    vgo[j] = (row * p.stride_kv + 8 * (pos ^ vswz<D>(row))) * 2;
  }
  // Block i's K (or V) tile alone into slot s (two query waves; block i
  // lives in slot i % 2).  Only issued for blocks that start before N.
  auto tile_load = [&](int i, bool v, int s) {
    const int kb0 = (blk0 + kg + KSPLIT * i) * kKB;
    const rsrc_t r = make_rsrc((v ? Vh : Kh) + (int64_t)kb0 * p.stride_kv, block_bytes(kb0));
#pragma unroll
    for (int j = 0; j < LCH; ++j)
      lds_dma16(r, (v ? vslot_lds(s) : kslot_lds(s)) + (uint32_t)(j * RPI * D * 2), v ? vgo[j] : kgo[j]);
  };
  auto lds_load = [&](int i, int s) {
    const int kb0 = (blk0 + kg + KSPLIT * i) * kKB;
    const uint32_t bytes = block_bytes(kb0);
    const rsrc_t rk = make_rsrc(Kh + (int64_t)kb0 * p.stride_kv, bytes);
    const rsrc_t rv = make_rsrc(Vh + (int64_t)kb0 * p.stride_kv, bytes);
#pragma unroll
    for (int j = 0; j < LCH; ++j) {
      lds_dma16(rk, kslot_lds(s) + (uint32_t)(j * RPI * D * 2), kgo[j]);
      lds_dma16(rv, vslot_lds(s) + (uint32_t)(j * RPI * D * 2), vgo[j]);
    }
  };

  float m_run = -INFINITY;  // running max (log2 units); -inf: the row has seen no key yet
  float m_use = 0.f;        // value subtracted from c*s (m_run once finite)
  float thr = -1.f;         // fast-path bound on the lane's P sum; -1 forces the slow path
  float l_run = 0.f;        // this lane's partial row sum
  float16v o[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) o[u] = float16v{};
  const int krow = kRowPerm(ql);
  const half2v ones = {(half_t)1.f, (half_t)1.f};

  // Transposed V fragments (A operand of O^T = V^T P^T, d tile u, key
  // chunk cc): this lane's offsets into a V tile.
  int vtr[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) vtr[u] = v_tr_offset<D>(lane, u);
  auto vfrag = [&](const half_t* v_l, int u, int cc) { return v_frag_tr<D>(v_l, vtr[u], cc); };

  // This lane's K fragment offsets (halves) per k-step: row krow (+32 t,
  // which keeps the swizzle), chunk 2 ks + g.
  int koff[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) koff[ks] = krow * D + 8 * ((2 * ks + g) ^ kswz<D>(krow));

  // Bias entries enter the score MFMAs as their initial accumulator, in
  // score units (t / |scale|), from one of two LDS layouts.
  // * Table range (use_tab): the entries q0 .. q0 + kBMq + N - 2, all that
  //   the workgroup's rows meet, loaded once in the prologue when they fit
  //   in the band slots' space (kBMq + N - 1 <= kTabCap), entry q0 + x at
  //   position kTabCap - 1 - x.
  // * Otherwise per-block bands.
  // Bias band of block i (BIAS): entry j < 32 + KB - 1, at position
  // BSLOT - 1 - j of the wave's band slot i % 2, is table[h][qw0 - kb0 -
  // (KB - 1) + N - 1 + j] in score units (t / |scale|), the entries of this
  // wave's 32 queries against the block's keys (indices past the table read
  // as zero; they meet only keys or queries past N).  Lane l loads entries
  // l and l + 64 into registers with the block's K (step i - 2) and stores
  // them after that step's barrier (the slot is the wave's own, and its
  // reads follow the store in program order).  The block's scores (step
  // i - 1) read their 16 NT entries per lane from the slot, and so does its
  // slow path (step i) with four query waves; the slot is rewritten for
  // block i + 2 after the barrier of step i.
  constexpr int BENT = 32 + kKB - 1;  // band entries per block
  const float* Th = BIAS ? static_cast<const float*>(p.bias) + (int64_t)bh * p.bias_stride_h : nullptr;
  const rsrc_t rsT = make_rsrc(Th, BIAS ? (uint32_t)(2 * N - 1) * 4u : 0u);
  const float tscale = kLog2e / c;  // c (s + t tscale) = c s + t log2(e)
  float* const band = &sband[BIAS ? (kg * QW + wave) * 2 * BSLOT : 0];
  constexpr int kThreads = 64 * QW * KSPLIT;
  constexpr int kTL = BIAS ? kTabCap / kThreads : 1;  // table loads per thread (BSLOT / 32)
  static_assert(!BIAS || kTL * kThreads == kTabCap, "table range");
  const int ntab = kBMq + N - 1;  // <= kTabCap (the launcher's choice of TAB)
  constexpr bool use_tab = TAB;
  // The table range's loads, first of all (untracked; tab_store after the
  // prologue's first wait stores them).
  float tabv[kTL];
  if constexpr (use_tab) {
#pragma unroll
    for (int m = 0; m < kTL; ++m) {
      const int x = tid + kThreads * m;
      if (x < ntab) tabv[m] = buf_load_f32_untracked(rsT, elem_offset(q0 + x, 2 * N - 1, 4));
    }
  }
  auto tab_store = [&]() {
    if constexpr (use_tab) {
#pragma unroll
      for (int m = 0; m < kTL; ++m) {
        asm volatile("" : "+v"(tabv[m]));
        const int x = tid + kThreads * m;
        if (x < ntab && x < kTabCap) stab[kTabCap - 1 - x] = tabv[m] * tscale;
      }
    }
  };
  struct BandRegs {
    float t[BENT > 64 ? 2 : 1];
  };
  auto band_load = [&](int i) {
    BandRegs r{};
    if constexpr (BIAS && !use_tab) {
      const int kb0 = (blk0 + kg + KSPLIT * i) * kKB;
      const int j0 = qw0 - kb0 - (kKB - 1) + N - 1 + lane;
      r.t[0] = buf_load_f32(rsT, elem_offset(j0, 2 * N - 1, 4));
      if constexpr (BENT > 64) r.t[1] = buf_load_f32(rsT, elem_offset(j0 + 64, 2 * N - 1, 4));
    }
    return r;
  };
  // band_load through asm buffer loads the compiler does not track (their
  // waits are explicit, band_ready after them).
  auto band_load_untracked = [&](int i) {
    BandRegs r{};
    if constexpr (BIAS && !use_tab) {
      const int kb0 = (blk0 + kg + KSPLIT * i) * kKB;
      const int j0 = qw0 - kb0 - (kKB - 1) + N - 1 + lane;
      r.t[0] = buf_load_f32_untracked(rsT, elem_offset(j0, 2 * N - 1, 4));
      if constexpr (BENT > 64) r.t[1] = buf_load_f32_untracked(rsT, elem_offset(j0 + 64, 2 * N - 1, 4));
    }
    return r;
  };
  // After the explicit wait that covers them: ties the registers to it.
  auto band_ready = [&](BandRegs& r) {
    if constexpr (BIAS) {
#pragma unroll
      for (int e = 0; e < (BENT > 64 ? 2 : 1); ++e) asm volatile("" : "+v"(r.t[e]));
    }
  };
  // Band slots by block parity: block i uses slot i % 2 (par).
  auto band_store = [&](int par, const BandRegs& r) {
    if constexpr (BIAS && !use_tab) {
      float* const slot = band + BSLOT * par + BSLOT - 1;
      slot[-lane] = r.t[0] * tscale;
      if constexpr (BENT > 64) slot[-(lane + 64)] = r.t[1] * tscale;  // within the slot
    }
  };
  // Initial score accumulator of 32-key tile t of the block at key kbb
  // (band slot par): register r of lane (ql, g) is key 32 t + 16 (r / 8) +
  // 8 g + r % 8 of the block, band entry ql - key + KB - 1 at position
  // BSLOT - KB - ql + key, or table entry q - (kbb + key) + N - 1 at
  // position kTabCap - 1 - (q - q0) + kbb + key - (N - 1): either way
  // consecutive registers read consecutive positions (pairs of them per
  // ds_read2_b32, straight into the accumulator registers).
  auto band_acc = [&](int par, int kbb, int t) {
    float16v a;
    if constexpr (BIAS) {
      const float* b;
      if constexpr (use_tab)
        b = stab + (kTabCap - 1) - (qw0 - q0) - (N - 1) - ql + 8 * g + kbb + 32 * t;
      else
        b = band + BSLOT * par + BSLOT - kKB - ql + 8 * g + 32 * t;
#pragma unroll
      for (int r = 0; r < 16; ++r) a[r] = b[16 * (r >> 3) + (r & 7)];
    } else {
      a = float16v{};
    }
    return a;
  };

  // Scores of a block (K tile in k_l, first key kbb), with its bias (band
  // slot par) as initial accumulator.
  auto qk = [&](float16v(&s)[NT], const half_t* k_l, int par, int kbb) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      s[t] = mfma32x32x16(load_half8(k_l + koff[0] + 32 * t * D), qf[0],
                          BIAS ? band_acc(par, kbb, t) : float16v{});
#pragma unroll
      for (int ks = 1; ks < KS; ++ks)
        s[t] = mfma32x32x16(load_half8(k_l + koff[ks] + 32 * t * D), qf[ks], s[t]);
    }
  };

  // P = 2^s in fp16 (the B operand of the P V product) and the lane's sum
  // of that fp16 P.
  auto expsum = [&](const float16v(&s)[NT], half8v(&pb)[2 * NT]) {
    float ls[2 * NT];
#pragma unroll
    for (int cc = 0; cc < 2 * NT; ++cc) {
      const float16v& v = s[cc >> 1];
      const int o8 = 8 * (cc & 1);
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const half2v h = {(half_t)fast_exp2(__builtin_fmaf(v[o8 + e], c, -m_use)),
                          (half_t)fast_exp2(__builtin_fmaf(v[o8 + e + 1], c, -m_use))};
        pb[cc][e] = h[0];
        pb[cc][e + 1] = h[1];
        a = __builtin_amdgcn_fdot2(h, ones, a, false);
      }
      ls[cc] = a;
    }
#pragma unroll
    for (int w = 1; w < 2 * NT; w *= 2)
#pragma unroll
      for (int cc = 0; cc + w < 2 * NT; cc += 2 * w) ls[cc] += ls[cc + w];
    return ls[0];
  };

  // acc += h.x + h.y (v_dot2_f32_f16).
  auto dot2_acc = [&](float& acc, half2v h) { acc = __builtin_amdgcn_fdot2(h, ones, acc, false); };

  // The common step, one straight-line stretch per block i: the scores of
  // block i+1 (KS*NT MFMAs, K from slot k_l), the P V product of block i-1
  // (DT*2NT MFMAs, V^T from slot v_l, P in pprev) and the softmax of block
  // i (scores s -> P in pcur, VALU).  MFMA slots alternate score and P V
  // products, so each accumulator chain has three other MFMAs between its
  // steps; fragments are read AHEAD slots early; every slot carries the
  // VALU work of SPJ scores, staggered (fma of slot j+1, exp of slot j,
  // cvt + dot2 of slot j-1) so that no VALU op waits on the one before it.
  // sched_barrier pins that order.  With one score per slot (head_dim 128)
  // a pair of scores is converted every second slot.  Returns the lane's
  // sum of fp16 pcur.
  auto fused = [&](const float16v(&s)[NT], float16v(&sn)[NT], const half_t* k_l,
                   const half_t* v_l, const half8v(&pprev)[2 * NT], half8v(&pcur)[2 * NT],
                   int npar, int kbn) {
    constexpr int NQ = KS * NT;       // score MFMAs
    constexpr int NP = DT * 2 * NT;   // P V MFMAs
    constexpr int NJ = NQ + NP;       // slots
    constexpr int SPJ = 16 * NT / NJ;  // scores per slot
    constexpr int AHEAD = 4;
    static_assert(NQ == NP && 16 * NT == SPJ * NJ && (SPJ == 1 || SPJ == 2), "slot split");
    // Fragment of slot j: even j -> K (tile q % NT, k-step q / NT),
    // odd j -> V^T (tile q % DT, key chunk q / DT), q = j / 2.
    auto frag = [&](int j) {
      const int q = j / 2;
      return (j % 2 == 0) ? load_half8(k_l + koff[q / NT] + 32 * (q % NT) * D)
                          : vfrag(v_l, q % DT, q / DT);
    };
    auto score = [&](int sc) {  // score sc (0..16 NT - 1) of this lane
      const int cc = sc / 8;
      return s[cc >> 1][8 * (cc & 1) + sc % 8];
    };
    float16v binit[NT];  // bias band of the next block (slot npar), read ahead of the K fragments
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if constexpr (BIAS) binit[t] = band_acc(npar, kbn, t);
    half8v fr[NJ];
#pragma unroll
    for (int j = 0; j < AHEAD; ++j) fr[j] = frag(j);
    // Two sum chains (chunk parity), added at the end.
    float acc[2] = {0.f, 0.f};
    float ev[NJ][SPJ], pv[NJ][SPJ];
    // Scores sc, sc + 1 into pcur (fp16) and the lane's sum.
    auto pack = [&](int sc, float x0, float x1) {
      const int cc = sc / 8, e = sc % 8;
      const half2v h = {(half_t)x0, (half_t)x1};
      pcur[cc][e] = h[0];
      pcur[cc][e + 1] = h[1];
      dot2_acc(acc[cc & 1], h);
    };
#pragma unroll
    for (int e = 0; e < SPJ; ++e) ev[0][e] = __builtin_fmaf(score(e), c, -m_use);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int q = j / 2;
      if (j % 2 == 0) {
        const int t = q % NT, ks = q / NT;
        if constexpr (BIAS)
          sn[t] = mfma32x32x16(fr[j], qf[ks], ks == 0 ? binit[t] : sn[t]);
        else
          sn[t] = mfma32x32x16(fr[j], qf[ks], ks == 0 ? float16v{} : sn[t]);
      } else {
        const int u = q % DT, cc = q / DT;
        o[u] = mfma32x32x16(fr[j], pprev[cc], o[u]);
      }
      if (j + AHEAD < NJ) fr[j + AHEAD] = frag(j + AHEAD);
      if (j + 1 < NJ) {
#pragma unroll
        for (int e = 0; e < SPJ; ++e) ev[j + 1][e] = __builtin_fmaf(score(SPJ * (j + 1) + e), c, -m_use);
      }
#pragma unroll
      for (int e = 0; e < SPJ; ++e) pv[j][e] = fast_exp2(ev[j][e]);
      if (SPJ == 2 && j >= 1) pack(2 * (j - 1), pv[max(j - 1, 0)][0], pv[max(j - 1, 0)][SPJ - 1]);
      if (SPJ == 1 && j >= 2 && j % 2 == 0) pack(j - 2, pv[max(j - 2, 0)][0], pv[max(j - 1, 0)][0]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (SPJ == 2)
      pack(2 * (NJ - 1), pv[NJ - 1][0], pv[NJ - 1][SPJ - 1]);
    else
      pack(NJ - 2, pv[NJ - 2][0], pv[NJ - 1][0]);
    return acc[0] + acc[1];
  };

  // Slow path on the scores s of the block at kb0 (raw Q K^T, modified in
  // place): masked keys set to -inf, the exact row max formed, m raised to
  // it, O and l rescaled, P redone into pb.  Returns the lane's P sum.
  auto slow_scores = [&](float16v(&s)[NT], int kb0, bool masked, half8v(&pb)[2 * NT]) {
    if (masked) {
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
    const float mx = max_halves(m8[0]);                         // raw row max of the block
    const float mx_c = (mx == -INFINITY) ? mx : mx * c;         // c > 0: scaling is monotone
    const float m_new = fmaxf(m_run, mx_c);                     // -inf while nothing seen
    const bool none = (m_new == -INFINITY);
    const float alpha = none ? 1.f : fast_exp2(m_run - m_new);  // 0 on the first visible block
    m_run = m_new;
    m_use = none ? 0.f : m_new;
    thr = none ? -1.f : kPSumMax;
    l_run *= alpha;
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[u][r] *= alpha;
    return expsum(s, pb);
  };

  // Slow path for the block of a step (its K in ring slot ks, its band in
  // slot par): its scores are recomputed from LDS, so the fused step need
  // not keep them live.
  auto slow = [&](int ks, int par, int kb0, bool masked, half8v(&pb)[2 * NT]) {
    float16v s[NT];
    qk(s, kslot(ks), par, kb0);
    return slow_scores(s, kb0, masked, pb);
  };

  // P V of one block on its own (a group's last block, after the loop).
  auto pv_only = [&](const half8v(&pb)[2 * NT], const half_t* v_l) {
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int cc = 0; cc < 2 * NT; ++cc) o[u] = mfma32x32x16(vfrag(v_l, u, cc), pb[cc], o[u]);
  };

  // One block step i: loads straight into LDS slots, then scores of block
  // i+1 into sn, softmax of block i (scores in s, P into pcur) and P V of
  // block i-1 (P in pprev) in the fused stretch, then a wait for the loads
  // and the barrier that publishes them.
  // Four query waves: block j lives in ring slot j % 4 and is loaded in step
  // j - 2, so the four blocks a step touches (i-1, i, i+1, i+2) never share
  // a slot; slot (i+2) % 4 last served block i-2, whose P V ran in step i-1.
  // Two query waves: step i loads K of block i+2 into K slot i % 2, whose
  // block i had its scores formed in step i-1 (the slow path of block i
  // uses those scores, kept in s), and V of block i into V slot i % 2, whose
  // block i-2 had its P V in step i-1.
  // R = i % 4, a compile-time constant: every slot and band address of the
  // step is then a fixed offset from the lane's base address.
  auto body = [&](int i, auto Rc, float16v(&s)[NT], float16v(&sn)[NT], half8v(&pprev)[2 * NT],
                  half8v(&pcur)[2 * NT]) {
    constexpr int R = decltype(Rc)::value;
    constexpr int P0 = R & 1, P1 = (R + 1) & 1;  // slot parity of blocks i (and i+2), i+1
    BandRegs bload{};  // bias band of block i + 2
    if constexpr (kLive) {
#ifdef NESO_FA2_SERIAL_LDS
      // The debug build's barrier must be reached by every wave (my_n
      // differs between key groups), so the loads are issued outside the
      // branch.
      if (i + 2 < my_n) {
        tile_load(i + 2, false, P0);
        bload = band_load(i + 2);
      }
      if (i < my_n) tile_load(i, true, P0);
      serial_lds_point();
      if (i < my_n) {
#else
      if (i < my_n) {
        if (i + 2 < my_n) {
          tile_load(i + 2, false, P0);
          bload = band_load(i + 2);
        }
        tile_load(i, true, P0);
#endif
        const int kb0 = (blk0 + kg + KSPLIT * i) * kKB;
        const bool masked =
            (kb0 + kKB > N) || (CAUSAL && (kb0 + kKB - 1 > qw0 + wr || kb0 < qw0 + 31 - wl));
        float ls = fused(s, sn, kslot(P1), vslot(P1), pprev, pcur, P1, kb0 + KSPLIT * kKB);
        if (__any(masked || !(ls <= thr))) ls = slow_scores(s, kb0, masked, pcur);
        l_run += ls;
      }
    } else {
#ifdef NESO_FA2_SERIAL_LDS
    // The debug build's barrier must be reached by every wave (my_n differs
    // between key groups), so the loads are issued outside the branch.
    if (i + 2 < my_n) {
      lds_load(i + 2, (R + 2) & 3);
      bload = band_load(i + 2);
    }
    serial_lds_point();
    if constexpr (HALVES) {
      if (i == my_nw && i < my_n) pv_only(pprev, vslot((R + 3) & 3));
    }
    if (i < (HALVES ? my_nw : my_n)) {
#else
    if constexpr (HALVES) {
      // The group's loads go on past this wave's last block; the P V of
      // that block comes in the step after it (later loads reuse its slot).
      if (i < my_n) {
        if (i + 2 < my_n) lds_load(i + 2, (R + 2) & 3);
        if (i == my_nw) pv_only(pprev, vslot((R + 3) & 3));
      }
    }
    if (i < (HALVES ? my_nw : my_n)) {
      if (!HALVES && i + 2 < my_n) {
        lds_load(i + 2, (R + 2) & 3);
        bload = band_load(i + 2);
      }
#endif
      const int kb0 = (blk0 + kg + KSPLIT * i) * kKB;
      // Some key of the block is past N or outside some query's window.
      const bool masked =
          (kb0 + kKB > N) || (CAUSAL && (kb0 + kKB - 1 > qw0 + wr || kb0 < qw0 + 31 - wl));
      // After the group's last block the next scores come from a stale
      // slot and are never used.
      float ls = fused(s, sn, kslot((R + 1) & 3), vslot((R + 3) & 3), pprev, pcur, P1,
                       kb0 + KSPLIT * kKB);
      // ls enters the condition so that the softmax cannot sink below it.
      if (__any(masked || !(ls <= thr))) ls = slow(R, P0, kb0, masked, pcur);
      l_run += ls;
    }
    }
    // Steps past the group's last block load nothing: no later step reads
    // those blocks, and the last block's V (read by the P V after the loop)
    // stays in place.
    serial_lds_point();
    wait_vmem();
    lds_barrier();
    // The band slot is this wave's own: its store needs no barrier, and
    // after the barrier its latency overlaps the next step's loads.
    if (BIAS && i + 2 < my_n) band_store(P0, bload);
  };

  // ---- prologue: blocks 0 and 1 into LDS in one round trip ----
  BandRegs bpro[3] = {};  // bias bands of blocks 0..2
  float16v sa[NT], sb[NT];
  half8v pa[2 * NT], pb2[2 * NT];
  if constexpr (kQLds) {
    // The workgroup's 128 query rows (rows past N read as zeros) into ring
    // slot 3 of key group 0, row-major with the K chunk swizzle, staging
    // row 32 sl + ql holding slice sl's row ql: rows q0 .. q0 + 127, or with
    // HALVES the short block's 64 rows then the long block's.  1 KiB
    // instruction x holds staging rows RPI x .., QLC instructions per wave
    // of the workgroup.
    constexpr int QLC = kBMq * D * 2 / 1024 / (QW * KSPLIT);
    static_assert(QLC >= 1 && QLC * QW * KSPLIT * 1024 == kBMq * D * 2 &&
                  kBMq * D <= KSLOT + VSLOT && (!HALVES || 64 % RPI == 0), "Q staging");
    const int wwg = kg * QW + wave;  // wave of the workgroup (scalar)
    const uint32_t qslot_lds = lds_addr(smem) + (uint32_t)(3 * (KSLOT + VSLOT) * 2);
#pragma unroll
    for (int j = 0; j < QLC; ++j) {
      const int x = wwg * QLC + j;
      const int row = RPI * x + lane / CPR, pos = lane % CPR;  // staging row
      rsrc_t rq = rsQ;
      int rr = row;  // row within rq
      if constexpr (HALVES) {
        // Scalar per instruction: the short block (hs = qblk) or the long
        // one (hl = n64 - 1 - qblk, none when it is the short block).
        const bool lng = RPI * x >= 64;
        const int r0 = __builtin_amdgcn_readfirstlane(64 * (lng ? n64 - 1 - qblk : qblk));
        const int nr = __builtin_amdgcn_readfirstlane(
            (lng && n64 - 1 - qblk == qblk) ? 0 : max(0, min(64, N - r0)));
        rq = make_rsrc(Qh + (int64_t)r0 * p.stride_q, (uint32_t)nr * p.stride_q * 2);
        rr = row - (lng ? 64 : 0);
      }
      lds_dma16(rq, qslot_lds + (uint32_t)(x * 1024),
                (uint32_t)((rr * p.stride_q + 8 * (pos ^ kswz<D>(row))) * 2));
    }
    // K of blocks 0 and 1 first, then their V and block 2: the first wait
    // covers Q, K0 and K1 only.
    auto k_load = [&](int i, int s) {
      const int kb0 = (blk0 + kg + KSPLIT * i) * kKB;
      const rsrc_t rk = make_rsrc(Kh + (int64_t)kb0 * p.stride_kv, block_bytes(kb0));
#pragma unroll
      for (int j = 0; j < LCH; ++j) lds_dma16(rk, kslot_lds(s) + (uint32_t)(j * RPI * D * 2), kgo[j]);
    };
    auto v_load = [&](int i, int s) {
      const int kb0 = (blk0 + kg + KSPLIT * i) * kKB;
      const rsrc_t rv = make_rsrc(Vh + (int64_t)kb0 * p.stride_kv, block_bytes(kb0));
#pragma unroll
      for (int j = 0; j < LCH; ++j) lds_dma16(rv, vslot_lds(s) + (uint32_t)(j * RPI * D * 2), vgo[j]);
    };
    if (my_n > 0) k_load(0, 0);
    if (my_n > 1) k_load(1, 1);
    if (my_n > 0) v_load(0, 0);
    if (my_n > 1) v_load(1, 1);
    if (my_n > 2) {
      k_load(2, 2);
      v_load(2, 2);
    }
    serial_lds_point();
    if (my_n > 2)
      wait_vmem_n<4 * LCH>();  // V0, V1, K2, V2 still in flight
    else
      wait_vmem();
    lds_barrier();
    {
      const half_t* qs = smem + 3 * (KSLOT + VSLOT);
      const int row = sl * 32 + ql;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const half8v t = load_half8(qs + row * D + 8 * ((2 * ks + g) ^ kswz<D>(row)));
        qf[ks] = neg ? -t : t;
      }
    }
    // ---- step 0: scores of blocks 0 and 1, block 0's exact softmax ----
    qk(sa, kslot(0), 0, (blk0 + kg) * kKB);
    qk(sb, kslot(1), 1, (blk0 + kg + KSPLIT) * kKB);
    if (HALVES ? my_nw > 0 : my_n > 0) {
      const int kb0 = (blk0 + kg) * kKB;
      const bool masked =
          (kb0 + kKB > N) || (CAUSAL && (kb0 + kKB - 1 > qw0 + wr || kb0 < qw0 + 31 - wl));
      l_run += slow_scores(sa, kb0, masked, pb2);
    }
    serial_lds_point();
    wait_vmem();
    lds_barrier();
  } else if constexpr (kQLive) {
    // Issue order: bands of blocks 0, 1 (untracked), Q, K0, K1, and V0
    // without a bias.  The first wait covers bands, Q and K0; the second K1.
    if (my_n > 0) bpro[0] = band_load_untracked(0);
    if (my_n > 1) bpro[1] = band_load_untracked(1);
    constexpr int QLC = kBMq * D * 2 / 1024 / (QW * KSPLIT);
    static_assert(QLC >= 1 && QLC * QW * KSPLIT * 1024 == kBMq * D * 2 && kBMq * D <= VSLOT,
                  "Q staging");
    const int wwg = kg * QW + wave;
    const uint32_t qslot_lds = lds_addr(smem) + (uint32_t)((2 * KSLOT + VSLOT) * 2);
#pragma unroll
    for (int j = 0; j < QLC; ++j) {
      const int x = wwg * QLC + j;
      const int row = RPI * x + lane / CPR, pos = lane % CPR;
      lds_dma16(rsQ, qslot_lds + (uint32_t)(x * 1024),
                (uint32_t)((row * p.stride_q + 8 * (pos ^ kswz<D>(row))) * 2));
    }
    if (my_n > 0) tile_load(0, false, 0);
    if (my_n > 1) tile_load(1, false, 1);
    if (!BIAS && my_n > 0) tile_load(0, true, 0);
    serial_lds_point();
    if (my_n > 1)
      wait_vmem_n<LCH + (BIAS ? 0 : LCH)>();  // K1 (and V0) still in flight
    else
      wait_vmem();
    band_ready(bpro[0]);
    band_ready(bpro[1]);
    band_store(0, bpro[0]);
    band_store(1, bpro[1]);
    tab_store();
    lds_barrier();
    {
      const half_t* qs = smem + 2 * KSLOT + VSLOT;
      const int row = wave * 32 + ql;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const half8v t = load_half8(qs + row * D + 8 * ((2 * ks + g) ^ kswz<D>(row)));
        qf[ks] = neg ? -t : t;
      }
    }
    // Scores of block 0; then K1 landed and a barrier (every wave done with
    // K slot 0); K of block 2 into that slot while the scores of block 1 are
    // formed.
    qk(sa, kslot(0), 0, (blk0 + kg) * kKB);
    if (my_n > 1) {
      if constexpr (BIAS) wait_vmem(); else wait_vmem_n<LCH>();  // V0 may stay in flight
    }
    lds_barrier();
    if (my_n > 2) {
      tile_load(2, false, 0);
      bpro[2] = band_load_untracked(2);
    }
    qk(sb, kslot(1), 1, (blk0 + kg + KSPLIT) * kKB);
    // ---- step 0: block 0's exact softmax (with the bias, V of block 0) ----
    if (BIAS && my_n > 0) tile_load(0, true, 0);
    serial_lds_point();
    if (my_n > 0) {
      const int kb0 = (blk0 + kg) * kKB;
      const bool masked =
          (kb0 + kKB > N) || (CAUSAL && (kb0 + kKB - 1 > qw0 + wr || kb0 < qw0 + 31 - wl));
      l_run += slow_scores(sa, kb0, masked, pb2);
    }
    wait_vmem();
    band_ready(bpro[2]);
    lds_barrier();
    if (BIAS && my_n > 2) band_store(0, bpro[2]);
  } else {
  if (my_n > 0) {
    if constexpr (kLive) {
      // Without a bias, V of block 0 too: the V slots are free until step
      // 0, and loading it here keeps its latency out of step 0's wait
      // (measured: H16 N1024 d64 10.25 -> 10.05 us; with the bias band the
      // longer prologue cost more, rel-pos 14.21 -> 14.52, so step 0 loads
      // it there).
      tile_load(0, false, 0);
      if constexpr (!BIAS) tile_load(0, true, 0);
    } else {
      lds_load(0, 0);
    }
    bpro[0] = band_load(0);
  }
  if (my_n > 1) {
    if constexpr (kLive)
      tile_load(1, false, 1);
    else
      lds_load(1, 1);
    bpro[1] = band_load(1);
  }
  wait_vmem();
  band_store(0, bpro[0]);
  band_store(1, bpro[1]);
  tab_store();
  lds_barrier();
  if constexpr (kLive) {
    // Scores of block 0, a barrier (every wave done with K slot 0), then K
    // of block 2 into that slot while the scores of block 1 are formed.
    qk(sa, kslot(0), 0, (blk0 + kg) * kKB);
    lds_barrier();
    if (my_n > 2) {
      tile_load(2, false, 0);
      bpro[2] = band_load(2);
    }
    qk(sb, kslot(1), 1, (blk0 + kg + KSPLIT) * kKB);
  }

  // ---- step 0, peeled: block 0 is every row's first visible block, so its
  // softmax is the slow path on its exact scores; scores of block 1; loads
  // of block 2 (two query waves: with the bias, V of block 0).  (Scores of
  // blocks a group does not have come from stale slots and are never
  // used.) ----
  if (!kLive && my_n > 2) {
    lds_load(2, 2);
    bpro[2] = band_load(2);
  }
  if (kLive && BIAS && my_n > 0) tile_load(0, true, 0);
  serial_lds_point();
  if constexpr (!kLive) qk(sa, kslot(0), 0, (blk0 + kg) * kKB);
  if (HALVES ? my_nw > 0 : my_n > 0) {
    const int kb0 = (blk0 + kg) * kKB;
    const bool masked =
        (kb0 + kKB > N) || (CAUSAL && (kb0 + kKB - 1 > qw0 + wr || kb0 < qw0 + 31 - wl));
    if constexpr (!kLive) qk(sb, kslot(1), 1, (blk0 + kg + KSPLIT) * kKB);
    l_run += slow_scores(sa, kb0, masked, pb2);
  }
  wait_vmem();
  lds_barrier();
  if (BIAS && my_n > 2) band_store(0, bpro[2]);
  }  // kQLds

  // Steps 1, 2, ...: unrolled by four, so that the score and P arrays swap
  // roles without copies and each copy knows its ring slots (i % 4).
  using R0 = std::integral_constant<int, 0>;
  using R1 = std::integral_constant<int, 1>;
  using R2 = std::integral_constant<int, 2>;
  using R3 = std::integral_constant<int, 3>;
  for (int i = 1; i < iters; i += 4) {
    body(i, R1{}, sb, sa, pb2, pa);
    body(i + 1, R2{}, sa, sb, pa, pb2);
    body(i + 2, R3{}, sb, sa, pb2, pa);
    body(i + 3, R0{}, sa, sb, pa, pb2);
  }
  // P V of the group's last block.  Step j writes block j's P into pb2
  // when j is even, into pa when j is odd.  (A HALVES wave that stopped
  // before the group's last block has done its last P V in the loop.)
  if (HALVES ? my_nw > 0 && my_nw == my_n : my_n > 0) {
    const int vs = (my_n - 1) & (kLive ? 1 : 3);
    if ((my_n - 1) & 1)
      pv_only(pa, vslot(vs));
    else
      pv_only(pb2, vslot(vs));
  }

  // ---- merge the key groups through LDS ----
  // Split merge (the lane's NV = 16 DT values of O divide into KSPLIT runs
  // of whole float4 pieces): group g finishes values [g VR, g VR + VR).
  // Each group publishes (m, l) and the values the other groups finish, so
  // every group merges and stores 1/KSPLIT of O.  Otherwise group 0 folds
  // the other groups' partials and stores all of O.
  constexpr int NV = 16 * DT;
  constexpr bool kSplitMerge = KSPLIT > 1 && NV % (4 * KSPLIT) == 0;
  constexpr int VR = kSplitMerge ? NV / KSPLIT : NV;
  if constexpr (kSplitMerge) {
    // The partials below overwrite the start of the LDS, where the
    // last-block P V above may still be reading V.
    lds_barrier();
    constexpr int SLOTS = NV - VR + 2;
    static_assert(sizeof(smem) >= (size_t)KSPLIT * QW * SLOTS * 64 * sizeof(float), "merge buffer");
    float* const red = reinterpret_cast<float*>(smem) + lane;
    auto part = [&](int grp) { return red + (size_t)(QW * grp + sl) * SLOTS * 64; };
    // Slot of value v in the list that group grp publishes (all values but
    // its own run).
    auto pos = [](int grp, int v) { return 2 + (v / VR > grp ? v - VR : v); };
#pragma unroll
    for (int me = 0; me < KSPLIT; ++me) {
      if (me != kg) continue;  // kg is wave-uniform: a scalar branch
      float* mine = part(me);
      mine[0] = m_run;
      mine[64] = l_run;
#pragma unroll
      for (int v = 0; v < NV; ++v)
        if (v / VR != me) mine[pos(me, v) * 64] = o[v / 16][v % 16];
    }
    lds_barrier();
#pragma unroll
    for (int me = 0; me < KSPLIT; ++me) {
      if (me != kg) continue;
      float mj[KSPLIT];
      float mm = m_run;
#pragma unroll
      for (int j = 0; j < KSPLIT; ++j) {
        if (j == me) continue;
        mj[j] = part(j)[0];
        mm = fmaxf(mm, mj[j]);
      }
      const float mu = (mm == -INFINITY) ? 0.f : mm;
      const float a0 = fast_exp2(m_run - mu);
      float lsum = l_run * a0;
#pragma unroll
      for (int v = me * VR; v < me * VR + VR; ++v) o[v / 16][v % 16] *= a0;
#pragma unroll
      for (int j = 0; j < KSPLIT; ++j) {
        if (j == me) continue;
        const float* other = part(j);
        const float aj = fast_exp2(mj[j] - mu);
        lsum += other[64] * aj;
#pragma unroll
        for (int v = me * VR; v < me * VR + VR; ++v)
          o[v / 16][v % 16] = __builtin_fmaf(other[pos(j, v) * 64], aj, o[v / 16][v % 16]);
      }
      m_run = mm;
      l_run = lsum;
    }
  } else if constexpr (KSPLIT > 1) {
    // The partials below overwrite the start of the LDS, where group 0's
    // last-block P V above may still be reading V^T.
    lds_barrier();
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
  const float l_tot = sum_halves(l_run);
  const float inv = 1.f / fmaxf(l_tot, 1e-6f);
  constexpr int ES = OUT_F16 ? 2 : 4;
  const rsrc_t rsO = make_rsrc(static_cast<char*>(p.O) +
                                   ((int64_t)bh * p.bh_stride_o + (int64_t)qb * p.stride_o) * ES,
                               (uint32_t)qrows * p.stride_o * ES);
#pragma unroll
  for (int u = 0; u < DT; ++u) {
    if constexpr (kSplitMerge && VR >= 16) {
      if (16 * u / VR != kg) continue;  // scalar branches
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if constexpr (kSplitMerge && VR < 16) {
        if ((16 * u + 4 * b) / VR != kg) continue;
      }
      const int col = 32 * u + 8 * b + 4 * g;
      const uint32_t off = ((q - qb) * p.stride_o + col) * ES;
      float4v v = {o[u][4 * b] * inv, o[u][4 * b + 1] * inv, o[u][4 * b + 2] * inv,
                   o[u][4 * b + 3] * inv};
      if (OUT_F16) {
        buf_store_f16x4(half4v{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]}, rsO, off);
      } else {
        buf_store_f32x4(v, rsO, off);
      }
    }
  }
  };  // run

  if constexpr (PAIR) {
    // One copy of the body: a loop of one or two passes.
    const int npass = x != nqb - 1 - x ? 2 : 1;
#pragma nounroll
    for (int pass = 0; pass < npass; ++pass) {
      if (pass) lds_barrier();  // the merge before read partials that this block's loads overwrite
      run(pass ? x : nqb - 1 - x);
    }
  } else if constexpr (HALVES) {
    run(x);
  } else {
    run(CAUSAL ? nqb - 1 - x : x);
  }
}

// Launches with K key groups if their LDS fits (returns false otherwise).
template <int D, bool CAUSAL, bool OUT_F16, int K, int QW, bool BIAS>
bool launch_fast_k(const Fa2Args& a, hipStream_t stream, hipError_t& err) {
  if constexpr (CAUSAL && !BIAS) {
    if constexpr (fast_lds_bytes<D, QW, BIAS, false, true, K>() <= 160 * 1024) {
      if (a.pair_qblocks == 1) {
        err = launch<&fa2_fast_kernel<D, true, OUT_F16, K, true, false, QW>>(
            ktag("fa2_fast_kernel", D, true, OUT_F16, K, true, false, QW, BIAS),
            dim3((a.num_qblocks + 1) / 2 * a.batch_heads), dim3(K * 64 * QW), stream, a);
        return true;
      }
    }
  }
  if constexpr (CAUSAL && QW == 4) {
    if constexpr (fast_lds_bytes<D, QW, BIAS, true, false, K>() <= 160 * 1024) {
      if (a.pair_qblocks == 2) {
        err = launch<&fa2_fast_kernel<D, true, OUT_F16, K, false, true>>(
            ktag("fa2_fast_kernel", D, true, OUT_F16, K, false, true, QW, BIAS),
            dim3(((a.N + 63) / 64 + 1) / 2 * a.batch_heads), dim3(K * 64 * QW), stream, a);
        return true;
      }
    }
  }
  if constexpr (fast_lds_bytes<D, QW, BIAS, false, false, K>() <= 160 * 1024) {
    if constexpr (BIAS) {
      // The bias table range of a workgroup's rows in the band slots' space
      // when it fits (the plan records BIAS = 2 for it).
      constexpr int cap = K * QW * 2 * fast_band_slot<D, QW, BIAS, false, false, K>();
      if ((int64_t)32 * QW + a.N - 1 <= cap) {
        err = launch<&fa2_fast_kernel<D, CAUSAL, OUT_F16, K, false, false, QW, true, true>>(
            ktag("fa2_fast_kernel", D, CAUSAL, OUT_F16, K, false, false, QW, 2),
            dim3(a.num_qblocks * a.batch_heads), dim3(K * 64 * QW), stream, a);
        return true;
      }
    }
    err = launch<&fa2_fast_kernel<D, CAUSAL, OUT_F16, K, false, false, QW, BIAS>>(
        ktag("fa2_fast_kernel", D, CAUSAL, OUT_F16, K, false, false, QW, BIAS),
        dim3(a.num_qblocks * a.batch_heads), dim3(K * 64 * QW), stream, a);
    return true;
  }
  return false;
}

// The requested key split, or the largest smaller one whose LDS fits: 1
// or 2, and 4 with two query waves.
template <int D, bool CAUSAL, bool OUT_F16, int QW, bool BIAS>
hipError_t launch_fast_t(const Fa2Args& a, int ksplit, hipStream_t stream) {
  hipError_t err = hipSuccess;
  bool done = false;
  if constexpr (QW == 2) {
    if (ksplit >= 4) done = launch_fast_k<D, CAUSAL, OUT_F16, 4, QW, BIAS>(a, stream, err);
  }
  if (!done && ksplit >= 2) done = launch_fast_k<D, CAUSAL, OUT_F16, 2, QW, BIAS>(a, stream, err);
  if (!done) launch_fast_k<D, CAUSAL, OUT_F16, 1, QW, BIAS>(a, stream, err);
  return err;
}

template <int D, bool CAUSAL, bool OUT_F16, bool BIAS>
hipError_t launch_fast_q(const Fa2Args& a, int ksplit, hipStream_t stream) {
  return a.qwaves == 2 ? launch_fast_t<D, CAUSAL, OUT_F16, 2, BIAS>(a, ksplit, stream)
                       : launch_fast_t<D, CAUSAL, OUT_F16, 4, BIAS>(a, ksplit, stream);
}

template <bool OUT_F16>
hipError_t launch_fast_d(const Fa2Args& a, int d, bool causal, bool bias, int ksplit,
                         hipStream_t s) {
  switch (d) {
    case 64:
      return bias     ? launch_fast_q<64, false, OUT_F16, true>(a, ksplit, s)
             : causal ? launch_fast_q<64, true, OUT_F16, false>(a, ksplit, s)
                      : launch_fast_q<64, false, OUT_F16, false>(a, ksplit, s);
    case 128:
      return bias     ? launch_fast_q<128, false, OUT_F16, true>(a, ksplit, s)
             : causal ? launch_fast_q<128, true, OUT_F16, false>(a, ksplit, s)
                      : launch_fast_q<128, false, OUT_F16, false>(a, ksplit, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool fa2_fast_supported(int head_dim, int bias_kind, bool in_f32) {
#ifdef NESO_FA2_FAST_DISABLED
  // Built without the fast kernel (its LDS-DMA M0 check failed at build
  // time): every call takes the generic kernel.
  (void)head_dim, (void)bias_kind, (void)in_f32;
  return false;
#else
  return (head_dim == 64 || head_dim == 128) &&
         (bias_kind == kBiasNone || bias_kind == kBiasTableF32) && !in_f32;
#endif
}

bool fa2_fast_preferred(bool causal, int32_t N, int head_dim, bool small_grid, bool bias) {
  // Measured on MI355X (d = 64, B*H = 8..64): the fast kernel is ahead from
  // N = 128 up without a mask (3-15%) and for causal rows from N = 1024
  // (7-25%, growing with N); for shorter causal rows the generic kernel's
  // per-wave skipping of invisible blocks wins (N = 256: 8.1 vs 8.9 us).
  // On a small grid (128-query workgroups <= half the compute units) from
  // N = 512 it runs 64-query workgroups (two query waves), ahead of the
  // generic kernel's 64-query workgroups by 14-40% (H8 N1500 d64 12.7 vs
  // 15.1 us, H16 N1024 d128 16.5 vs 22.8, H4 N2048 d64 causal 15.0 vs 18.5,
  // rel-pos table H8 N1500 d64 14.1 vs 16.6, d128 21.3 vs 35.8).  With the
  // bias table it is ahead on larger grids too, with 128-query workgroups
  // (H16 N2048 d64: 28.1 vs 29.8 us).
  (void)head_dim;
  if (bias) return true;
  return !causal || N >= 1024;
}

// Query waves of the fast kernel: two on a small grid, from N = 512
// without a bias.
int fa2_fast_qwaves(bool small_grid, int32_t N, bool bias) {
  return small_grid && (bias || N >= 512) ? 2 : 4;
}

hipError_t launch_fa2_fast(Fa2Args a, int head_dim, bool causal, bool bias, bool out_f16,
                           int ksplit, hipStream_t stream) {
#ifdef NESO_FA2_FAST_DISABLED
  (void)a, (void)head_dim, (void)causal, (void)bias, (void)out_f16, (void)ksplit, (void)stream;
  return hipErrorInvalidValue;
#endif
  if (bias && causal) return hipErrorInvalidValue;  // the biased entry point is never masked
  if (a.qwaves != 2) a.qwaves = 4;
  a.num_qblocks = (a.N + 32 * a.qwaves - 1) / (32 * a.qwaves);
  // Paired query blocks (causal kernels, two or four query waves; any
  // window is correct); 64-row halves only with four query waves and
  // without a window (the two halves' key ranges must both start at key 0).
  const bool full_causal = causal && a.win_left >= a.N && a.win_right == 0;
  a.pair_qblocks = (causal && a.pair_qblocks == 1)                          ? 1
                   : (a.qwaves == 4 && full_causal && a.pair_qblocks == 2)  ? 2
                                                                            : 0;
  return out_f16 ? launch_fast_d<true>(a, head_dim, causal, bias, ksplit, stream)
                 : launch_fast_d<false>(a, head_dim, causal, bias, ksplit, stream);
}

}  // namespace neso
