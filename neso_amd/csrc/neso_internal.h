// Internal launch interface between the C-ABI layer (neso_abi.hip) and the
// kernel translation units.  Argument validation happens in the ABI layer;
// the launchers below assume their arguments were checked.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace neso {

// kBiasDenseF16Row16 is internal to the generic FA2 kernel: the dense f16
// bias with every row 16-byte aligned (16-byte bias loads).
enum BiasKind { kBiasNone = 0, kBiasTableF32 = 1, kBiasDenseF16 = 2, kBiasDenseF16Row16 = 3 };

struct Fa2Args {
  const void* Q;        // f16, or f32 for the f32-input kernels
  const void* K;
  const void* V;
  void* O;              // f32 or f16, [batch_heads][N][stride_o]
  const void* bias;     // table f32 [h][2N-1] or dense f16 [h][N][N]
  int32_t N;            // queries == keys per (batch, head)
  int32_t stride_q;     // row stride of Q (elements)
  int32_t stride_kv;    // row stride of K and V (elements)
  int32_t stride_o;     // row stride of O (elements)
  int64_t bh_stride_q;  // (batch, head) strides, elements
  int64_t bh_stride_kv;
  int64_t bh_stride_o;
  int64_t bias_stride_h;
  int32_t batch_heads;
  float scale_log2;     // softmax scale * log2(e)
  int32_t num_qblocks;  // filled in by launch_fa2
  int32_t ksplit;       // key groups per workgroup (1, 2); 0 = chosen from the grid size
  // Window of the masked (causal) kernels: key j is visible to query i iff
  // i - win_left <= j <= i + win_right.  Causal is (N, 0).
  int32_t win_left;
  int32_t win_right;
  // Kernel choice for fp16 calls without a bias or with the f32 bias
  // table: 1 = the fast kernel (fa2_fast.hip) where it is measured faster,
  // 2 = the fast kernel wherever it applies, 0 = always the generic kernel.
  int32_t allow_fast;
  // Query waves per key group (a query block is 32 rows per wave): 4 or 2;
  // 0 = chosen from the grid size.
  int32_t qwaves;
  // Causal fast kernel: 1 = each workgroup takes query blocks nqb-1-x and
  // x; 2 = it takes the 64-row blocks x and n64-1-x (no window); 0 = one
  // block (filled in by launch_fa2; NESO_AMD_FA2_PAIR forces it).
  int32_t pair_qblocks;
};

// Compute units of the current device (cached per device), or the count a
// launch-plan recording stands in for.
int device_cu_count();

// ---- launches ----
// Every kernel of the library is launched through launch<&kernel>(...).
// While a launch plan is being recorded on the calling thread
// (neso_plan_begin / neso_plan_end in the C ABI), the launch is recorded
// instead of issued and no HIP call is made, so the host-side choice of
// kernel, grid and workgroup size can be inspected without a GPU.
bool plan_recording();

// Name and template arguments of a launched kernel, for the plan record.
struct KernelTag {
  const char* name;
  int args[8];
  int nargs;
};
template <typename... T>
KernelTag ktag(const char* name, T... v) {
  static_assert(sizeof...(T) <= 8, "template arguments");
  return KernelTag{name, {static_cast<int>(v)...}, (int)sizeof...(T)};
}
void plan_add(const KernelTag& tag, dim3 grid, dim3 block);

template <auto F, typename... A>
hipError_t launch(const KernelTag& tag, dim3 grid, dim3 block, hipStream_t stream, A... args) {
  if (plan_recording()) {
    plan_add(tag, grid, block);
    return hipSuccess;
  }
  void* argv[] = {static_cast<void*>(&args)...};
  return hipLaunchKernel(reinterpret_cast<const void*>(F), grid, block, argv, 0, stream);
}

int fa2_query_block();
// The fast kernel covers fp16 Q/K/V at head_dim 64 and 128, without a bias
// or with the f32 bias table; fa2_fast_preferred says where it is the
// faster one.  qwaves (2 or 4) picks its query waves per key group.
bool fa2_fast_supported(int head_dim, int bias_kind, bool in_f32);
bool fa2_fast_preferred(bool causal, int32_t N, int head_dim, bool small_grid, bool bias);
int fa2_fast_qwaves(bool small_grid, int32_t N, bool bias);
hipError_t launch_fa2_fast(Fa2Args a, int head_dim, bool causal, bool bias, bool out_f16,
                           int ksplit, hipStream_t stream);
hipError_t launch_fa2(Fa2Args a, int head_dim, bool causal, int bias_kind, bool out_f16,
                      hipStream_t stream, bool in_f32 = false);

// Y[M][N] (f16, row stride ldy) = X[M][K] (f16, row stride ldx) * dequant(W)^T
// with W packed 8 int4 codes per int32 along K ([N][K/8]), scales f16
// [N][K/group], code c -> (c - zero) * scale.
struct W4Args {
  const half_t* X;
  const uint32_t* W;
  const half_t* S;
  half_t* Y;
  int32_t M, N, K;
  int32_t ldx, ldy;
  int32_t group;
  int32_t zero;
  // Tile GEMM only, set by launch_w4a16: nonzero syncs each K-group's
  // waves through an LDS arrival counter instead of the workgroup barrier.
  int32_t group_sync;
};

hipError_t launch_w4a16(const W4Args& a, hipStream_t stream);
// Skinny-M kernel with X in LDS (qmatmul_skinny.hip): M <= 16, group 32,
// K % 128 == 0, K <= w4a16_skinny_lds_max_k().
int w4a16_skinny_lds_max_k();
hipError_t launch_w4a16_skinny_lds(const W4Args& a, hipStream_t stream);

// C[M][N] (f32) = A[M][K] (f16) * f16(B[K][N] int8) [* scale[n]].
struct W8Args {
  const half_t* A;
  const int8_t* B;
  float* C;
  const half_t* scale;  // nullptr: unscaled
  int32_t M, N, K;
  int32_t lda, ldb, ldc;
};

hipError_t launch_w8a16(const W8Args& a, hipStream_t stream);

// Rel-pos bias precompute: Q_u = Q + bias_u and the unscaled dense
// rel_bias[h][i][j] = (Q + bias_v)[h][i] . K_rel[h][T-1-i+j], fp32 in, fp16
// out, all contiguous ([heads][T][d], [heads][2T-1][d], [heads][d],
// [heads][T][T]).
struct RelPreArgs {
  const float* Q;
  const float* K_rel;
  const float* bias_u;
  const float* bias_v;
  half_t* Q_u;
  half_t* rel_bias;
  int32_t T;
  int32_t heads;
};

hipError_t launch_relpos_precompute(const RelPreArgs& a, int head_dim, hipStream_t stream);

}  // namespace neso
