// C ABI of neso_amd: argument validation, status codes and the kernel
// manifest.  Every check below runs before the first HIP call, so invalid
// arguments are reported identically with or without a GPU.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <string>
#include <utility>

#include "../../include/neso_amd.h"
#include "manifest.h"
#include "neso_internal.h"

namespace {

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_last_error[0] = '\0';
  return NESO_OK;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(NESO_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned2(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1u) == 0; }

// Optional override of the FA2 key split, for tuning and for tests that
// exercise every code path: NESO_AMD_FA2_KSPLIT=1..4.
int env_ksplit() {
  const char* v = getenv("NESO_AMD_FA2_KSPLIT");
  if (!v) return 0;
  const int k = atoi(v);
  return (k >= 1 && k <= 4) ? k : 0;
}

// FA2 kernel choice for fp16 calls without a bias or with the f32 bias
// table (tests cover both kernels): NESO_AMD_FA2_FAST=0 always takes the
// generic kernel, =2 the fast kernel wherever it applies; unset or 1
// chooses by shape.
int env_allow_fast() {
  const char* v = getenv("NESO_AMD_FA2_FAST");
  if (!v) return 1;
  if (v[0] == '0') return 0;
  return v[0] == '2' ? 2 : 1;
}

// Query waves per key group of either FA2 kernel (tests cover both):
// NESO_AMD_FA2_QW=2 or 4; unset chooses from the grid size.
int env_qwaves() {
  const char* v = getenv("NESO_AMD_FA2_QW");
  if (!v) return 0;
  const int k = atoi(v);
  return (k == 2 || k == 4) ? k : 0;
}

// Causal work balancing on the fast FA2 kernel: NESO_AMD_FA2_PAIR=1 forces
// paired 128-row query blocks, 2 forces paired 64-row halves (no window
// only), 0 forbids both; unset lets the launcher choose.
int env_pair() {
  const char* v = getenv("NESO_AMD_FA2_PAIR");
  if (!v) return -1;
  const int k = atoi(v);
  return (k == 1 || k == 2) ? k : 0;
}

int check_head_dim(int32_t d) {
  if (d == 32 || d == 64 || d == 128) return NESO_OK;
  return fail(NESO_EUNSUPPORTED, "head_dim %d not supported (32, 64, 128)", d);
}

// Shared by both attention entry points once their layouts are resolved.
int fa2_common(const void* Q, const void* K, const void* V, void* O, const void* bias, int32_t N,
               int32_t stride_q, int32_t stride_kv, int32_t stride_o, float scale,
               int32_t head_dim, int32_t heads, int64_t bh_q, int64_t bh_kv, int64_t bh_o,
               int64_t bias_stride_h, int causal, int bias_kind, bool out_f16, void* stream,
               const char* name, int32_t win_left = -1, int32_t win_right = -1,
               bool in_f32 = false) {
  if (!Q || !K || !V || !O) return fail(NESO_EINVAL, "%s: null tensor pointer", name);
  if (N < 0) return fail(NESO_EINVAL, "%s: N=%d < 0", name, N);
  if (heads < 0) return fail(NESO_EINVAL, "%s: batch_heads=%d < 0", name, heads);
  int st = check_head_dim(head_dim);
  if (st != NESO_OK) return st;
  if (!isfinite(scale)) return fail(NESO_EINVAL, "%s: scale is not finite", name);
  if (causal != 0 && causal != 1) return fail(NESO_EINVAL, "%s: causal=%d", name, causal);
  if (stride_q < head_dim || stride_kv < head_dim || stride_o < head_dim)
    return fail(NESO_EINVAL, "%s: row stride smaller than head_dim %d", name, head_dim);
  // Q/K/V rows are read in 16-byte pieces: 8 f16 or 4 f32 elements.
  const int in_mult = in_f32 ? 4 : 8;
  if (stride_q % in_mult || stride_kv % in_mult || stride_o % 4)
    return fail(NESO_EINVAL, "%s: row strides must be multiples of %d elements", name, in_mult);
  if (bh_q % in_mult || bh_kv % in_mult || bh_o % 4 || bh_q < 0 || bh_kv < 0 || bh_o < 0)
    return fail(NESO_EINVAL, "%s: head strides must be non-negative multiples of %d", name,
                in_mult);
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O))
    return fail(NESO_EINVAL, "%s: Q/K/V/O must be 16-byte aligned", name);
  // A block of 128 rows is addressed with 32-bit byte offsets.
  const int64_t max_stride = std::max({(int64_t)stride_q, (int64_t)stride_kv, (int64_t)stride_o});
  if (max_stride * neso::fa2_query_block() * 4 >= (int64_t)1 << 32)
    return fail(NESO_EUNSUPPORTED, "%s: row stride %lld too large", name, (long long)max_stride);
  if (bias_kind != neso::kBiasNone) {
    if (!bias) return fail(NESO_EINVAL, "%s: null bias pointer", name);
    if (bias_stride_h < 0) return fail(NESO_EINVAL, "%s: bias_stride_h < 0", name);
    if (bias_kind == neso::kBiasTableF32 && (reinterpret_cast<uintptr_t>(bias) & 3u))
      return fail(NESO_EINVAL, "%s: f32 bias table must be 4-byte aligned", name);
    if (bias_kind == neso::kBiasDenseF16 && !aligned2(bias))
      return fail(NESO_EINVAL, "%s: f16 bias must be 2-byte aligned", name);
  }
  if (N == 0 || heads == 0) return ok();
  if ((int64_t)(N + neso::fa2_query_block() - 1) / neso::fa2_query_block() * heads > 0x7fffffff)
    return fail(NESO_EUNSUPPORTED, "%s: grid too large", name);

  neso::Fa2Args a{};
  a.Q = Q;
  a.K = K;
  a.V = V;
  a.O = O;
  a.bias = bias;
  a.N = N;
  a.stride_q = stride_q;
  a.stride_kv = stride_kv;
  a.stride_o = stride_o;
  a.bh_stride_q = bh_q;
  a.bh_stride_kv = bh_kv;
  a.bh_stride_o = bh_o;
  a.bias_stride_h = bias_stride_h;
  a.batch_heads = heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.ksplit = env_ksplit();
  a.allow_fast = env_allow_fast();
  a.qwaves = env_qwaves();
  a.pair_qblocks = env_pair();
  // Causal is the window (N, 0); windows wider than N are clamped to N.
  a.win_left = win_left < 0 ? N : (win_left < N ? win_left : N);
  a.win_right = win_right < 0 ? 0 : (win_right < N ? win_right : N);
  return launched(neso::launch_fa2(a, head_dim, causal != 0, bias_kind, out_f16,
                                   static_cast<hipStream_t>(stream), in_f32),
                  name);
}

// Launch-plan recording state of the calling thread.
struct PlanState {
  bool active = false;
  int cus = 0;  // compute units planned for; 0 = the current device's
  int count = 0;
  std::string json;
};
thread_local PlanState g_plan;

}  // namespace

namespace neso {

bool plan_recording() { return g_plan.active; }

void plan_add(const KernelTag& tag, dim3 grid, dim3 block) {
  std::string targs;
  for (int i = 0; i < tag.nargs; ++i) targs += (i ? ", " : "") + std::to_string(tag.args[i]);
  char buf[320];
  snprintf(buf, sizeof buf,
           "%s{\"device_kernel\": \"%s\", \"template_args\": [%s], \"grid\": [%u, %u, %u], "
           "\"threadgroup_size\": %u, \"num_warps\": %u}",
           g_plan.count ? ", " : "", tag.name, targs.c_str(), grid.x, grid.y, grid.z,
           block.x * block.y * block.z, block.x * block.y * block.z / 64);
  g_plan.json += buf;
  ++g_plan.count;
}

int device_cu_count() {
  if (g_plan.active && g_plan.cus > 0) return g_plan.cus;
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < kMaxDevices) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  if (dev < kMaxDevices) cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// One wave records (shader clock, 100 MHz reference clock) pairs from
// s_memtime and s_memrealtime, one pair every gap_ticks of the reference
// clock.  Each wait ends once the reference clock has advanced, so the
// kernel runs samples * gap_ticks / 100 us and then exits.
__global__ __launch_bounds__(64) void clock_sample_kernel(uint64_t* out, int samples,
                                                          int gap_ticks) {
  for (int i = 0; i < samples; ++i) {
    const uint64_t t = __builtin_amdgcn_s_memtime();
    const uint64_t r = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
      out[2 * i] = t;
      out[2 * i + 1] = r;
    }
    uint64_t now = r;
    while (now < r + (uint64_t)gap_ticks) {
      __builtin_amdgcn_s_sleep(1);
      now = __builtin_amdgcn_s_memrealtime();
    }
  }
}

// Streaming-floor probes (measurement aids): an empty kernel, and a
// read-only stream of 16-byte non-temporal loads in which thread t of the
// grid (T threads) reads pieces t, t + T, ..., t + (NP - 1) T, the layout of
// a persistent grid streaming one contiguous buffer.  Straight-line code
// with a rolling window of DEPTH loads in flight per lane: piece k is folded
// into the lane's XOR as piece k + DEPTH is requested.  The timed form
// (ALL = false) writes a lane's XOR only if it equals `key`, which keeps
// every load live without stores; the checking form (ALL = true) writes
// every lane's XOR to sink[t], so the host can XOR them into the buffer's.
__global__ __launch_bounds__(256) void stream_empty_kernel() {}

template <int NP, int DEPTH, bool ALL>
__global__ __launch_bounds__(256) void stream_read_kernel(const void* src, uint32_t bytes,
                                                          uint32_t key, uint32_t* sink) {
  const rsrc_t r = make_rsrc(src, bytes);
  const uint32_t T = gridDim.x * 256u;
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  uint4v v[NP];
  uint32_t acc = 0;
#pragma unroll
  for (int k = 0; k < NP + DEPTH; ++k) {
    // Pieces past the buffer read as zeros (offsets stay below 2^32: the
    // entry point bounds NP T * 16).
    if (k < NP)
      v[k] = __builtin_bit_cast(uint4v, __builtin_amdgcn_raw_buffer_load_b128(
                                            r, (t + (uint32_t)k * T) * 16u, 0, kNonTemporal));
    if (k >= DEPTH) {
      const uint4v& x = v[k - DEPTH];
      acc ^= x[0] ^ x[1] ^ x[2] ^ x[3];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if (ALL)
    sink[t] = acc;
  else if (acc == key)
    sink[0] = acc;
}

template <int NP>
hipError_t launch_stream_read(bool all, int grid, hipStream_t st, const void* src, uint32_t bytes,
                              uint32_t key, uint32_t* sink) {
  if (all)
    return launch<&stream_read_kernel<NP, 4, true>>(ktag("stream_read_kernel", NP, 4, 1),
                                                    dim3(grid), dim3(256), st, src, bytes, key,
                                                    sink);
  return launch<&stream_read_kernel<NP, 4, false>>(ktag("stream_read_kernel", NP, 4, 0),
                                                   dim3(grid), dim3(256), st, src, bytes, key,
                                                   sink);
}

template <int... NPS>
hipError_t launch_stream_read_np(int np, bool all, int grid, hipStream_t st, const void* src,
                                 uint32_t bytes, uint32_t key, uint32_t* sink,
                                 std::integer_sequence<int, NPS...>) {
  hipError_t err = hipErrorInvalidValue;
  ((np == NPS + 1 ? (err = launch_stream_read<NPS + 1>(all, grid, st, src, bytes, key, sink), 0)
                  : 0),
   ...);
  return err;
}
constexpr int kStreamMaxPieces = 16;  // pieces per thread

}  // namespace neso

extern "C" {

int neso_abi_version(void) { return 2; }

const char* neso_status_string(int status) {
  switch (status) {
    case NESO_OK: return "NESO_OK";
    case NESO_EINVAL: return "NESO_EINVAL: invalid argument";
    case NESO_EUNSUPPORTED: return "NESO_EUNSUPPORTED: unsupported configuration";
    case NESO_ELAUNCH: return "NESO_ELAUNCH: kernel launch failed";
    default: return "NESO_UNKNOWN";
  }
}

const char* neso_last_error(void) { return g_last_error; }

const char* neso_kernel_manifest(void) { return neso::kManifest; }

int neso_plan_begin(int32_t cu_count) {
  if (cu_count < 0) return fail(NESO_EINVAL, "plan_begin: cu_count=%d < 0", cu_count);
  g_plan.active = true;
  g_plan.cus = cu_count;
  g_plan.count = 0;
  g_plan.json.clear();
  return ok();
}

int neso_clock_sample(uint64_t* out, int32_t samples, int32_t gap_ticks, void* stream) {
  if (!out || (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(NESO_EINVAL, "clock_sample: null or misaligned out");
  if (samples < 1 || samples > (1 << 20) || gap_ticks < 1 || gap_ticks > (1 << 20))
    return fail(NESO_EINVAL, "clock_sample: samples=%d, gap_ticks=%d outside [1, 2^20]", samples,
                gap_ticks);
  // The wave spins samples * gap_ticks reference ticks: at most 2^30 (10.7 s).
  if ((int64_t)samples * gap_ticks > (int64_t)1 << 30)
    return fail(NESO_EINVAL, "clock_sample: samples * gap_ticks = %lld above 2^30 (10.7 s)",
                (long long)samples * gap_ticks);
  return launched(neso::launch<&neso::clock_sample_kernel>(
                      neso::ktag("clock_sample_kernel"), dim3(1), dim3(64),
                      static_cast<hipStream_t>(stream), out, (int)samples, (int)gap_ticks),
                  "clock_sample");
}

int neso_stream_probe(const void* src, int64_t bytes, int32_t grid, int32_t mode, uint32_t key,
                      uint32_t* sink, void* stream) {
  if (grid < 1 || grid > (1 << 20))
    return fail(NESO_EINVAL, "stream_probe: grid=%d outside [1, 2^20]", grid);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (mode == 0)
    return launched(neso::launch<&neso::stream_empty_kernel>(neso::ktag("stream_empty_kernel"),
                                                             dim3(grid), dim3(256), st),
                    "stream_probe");
  if (mode != 1 && mode != 2)
    return fail(NESO_EINVAL, "stream_probe: mode=%d not 0, 1 or 2", mode);
  if (!src || !aligned16(src) || !sink || (reinterpret_cast<uintptr_t>(sink) & 3u))
    return fail(NESO_EINVAL, "stream_probe: null or misaligned src/sink");
  const int64_t threads = (int64_t)grid * 256;
  if (bytes <= 0 || bytes % 16)
    return fail(NESO_EINVAL, "stream_probe: bytes=%lld must be a positive multiple of 16",
                (long long)bytes);
  const int64_t np = (bytes / 16 + threads - 1) / threads;  // pieces per thread
  // Every piece offset (np T pieces of 16 bytes) must stay below 2^32.
  if (np > neso::kStreamMaxPieces || np * threads * 16 >= ((int64_t)1 << 32))
    return fail(NESO_EINVAL, "stream_probe: bytes=%lld needs %lld pieces per thread at grid "
                "%d (at most %d, and below 4 GiB)", (long long)bytes, (long long)np, grid,
                neso::kStreamMaxPieces);
  return launched(neso::launch_stream_read_np((int)np, mode == 2, grid, st, src, (uint32_t)bytes,
                                              key, sink,
                                              std::make_integer_sequence<int, neso::kStreamMaxPieces>()),
                  "stream_probe");
}

const char* neso_plan_end(void) {
  static thread_local std::string out;
  out = "{\"launches\": [" + g_plan.json + "]}";
  g_plan = PlanState{};
  return out.c_str();
}

int neso_flash_attention_fwd(const void* Q, const void* K, const void* V, float* O, int32_t N,
                             int32_t stride_qo, int32_t stride_kv, float scale, int32_t head_dim,
                             int32_t batch_heads, int64_t stride_bh_qo, int64_t stride_bh_kv,
                             int32_t causal, void* stream) {
  return fa2_common(Q, K, V, O, nullptr, N, stride_qo, stride_kv, stride_qo, scale, head_dim,
                    batch_heads, stride_bh_qo, stride_bh_kv, stride_bh_qo, 0, causal,
                    neso::kBiasNone, false, stream, "flash_attention_fwd");
}

int neso_flash_attention_f32_fwd(const float* Q, const float* K, const float* V, float* O,
                                 int32_t N, int32_t stride_qo, int32_t stride_kv, float scale,
                                 int32_t head_dim, int32_t batch_heads, int64_t stride_bh_qo,
                                 int64_t stride_bh_kv, int32_t causal, void* stream) {
  return fa2_common(Q, K, V, O, nullptr, N, stride_qo, stride_kv, stride_qo, scale, head_dim,
                    batch_heads, stride_bh_qo, stride_bh_kv, stride_bh_qo, 0, causal,
                    neso::kBiasNone, false, stream, "flash_attention_f32_fwd", -1, -1, true);
}

int neso_flash_attention_io_fwd(const void* Q, const void* K, const void* V, void* O, int32_t N,
                                int32_t d_head, float scale, int32_t io_dtype,
                                int32_t batch_heads, void* stream) {
  const char* name = "flash_attention_io_fwd";
  if (io_dtype != NESO_IO_F16 && io_dtype != NESO_IO_F32)
    return fail(NESO_EINVAL, "%s: io_dtype=%d", name, io_dtype);
  const bool f32 = io_dtype == NESO_IO_F32;
  // Rows are d_head apart and slices N rows apart (the reference's layout).
  const int64_t slice = (int64_t)N * d_head;
  return fa2_common(Q, K, V, O, nullptr, N, d_head, d_head, d_head, scale, d_head, batch_heads,
                    slice, slice, slice, 0, 0, neso::kBiasNone, !f32, stream, name, -1, -1, f32);
}

int neso_flash_attention_window_fwd(const void* Q, const void* K, const void* V, void* O,
                                    int32_t seq_len, int32_t stride_h, int32_t stride_m,
                                    float sm_scale, int32_t window_left, int32_t window_right,
                                    int32_t num_heads, int32_t head_dim, int32_t out_dtype,
                                    void* stream) {
  const char* name = "flash_attention_window_fwd";
  if (window_left < 0 || window_right < 0)
    return fail(NESO_EINVAL, "%s: window (%d, %d) must be non-negative", name, window_left,
                window_right);
  if (out_dtype != NESO_OUT_F16 && out_dtype != NESO_OUT_F32)
    return fail(NESO_EINVAL, "%s: out_dtype=%d", name, out_dtype);
  return fa2_common(Q, K, V, O, nullptr, seq_len, stride_m, stride_m, stride_m, sm_scale,
                    head_dim, num_heads, stride_h, stride_h, stride_h, 0, 1, neso::kBiasNone,
                    out_dtype == NESO_OUT_F16, stream, name, window_left, window_right);
}

int neso_rel_pos_fa2_fwd(const void* Q, const void* K, const void* V, const void* bias, void* O,
                         int32_t T, int32_t stride, float scale, int32_t stride_h,
                         int32_t bias_stride_h, int32_t num_heads, int32_t head_dim,
                         int32_t bias_mode, int32_t out_dtype, void* stream) {
  int kind;
  if (bias_mode == NESO_BIAS_DENSE_SCALED_F16) {
    kind = neso::kBiasDenseF16;
  } else if (bias_mode == NESO_BIAS_TABLE_F32) {
    kind = neso::kBiasTableF32;
  } else {
    return fail(NESO_EINVAL, "rel_pos_fa2_fwd: bias_mode=%d", bias_mode);
  }
  if (out_dtype != NESO_OUT_F16 && out_dtype != NESO_OUT_F32)
    return fail(NESO_EINVAL, "rel_pos_fa2_fwd: out_dtype=%d", out_dtype);
  return fa2_common(Q, K, V, O, bias, T, stride, stride, stride, scale, head_dim, num_heads,
                    stride_h, stride_h, stride_h, bias_stride_h, 0, kind,
                    out_dtype == NESO_OUT_F16, stream, "rel_pos_fa2_fwd");
}

int neso_rel_pos_precompute(const float* Q, const float* K_rel, const float* bias_u,
                            const float* bias_v, int32_t T, int32_t d, int32_t nh, float scale,
                            void* Q_u, void* rel_bias, void* stream) {
  const char* name = "rel_pos_precompute";
  (void)scale;  // the reference's precompute leaves the bias unscaled too
  if (!Q || !K_rel || !bias_u || !bias_v || !Q_u || !rel_bias)
    return fail(NESO_EINVAL, "%s: null tensor pointer", name);
  if (T < 0 || nh < 0) return fail(NESO_EINVAL, "%s: T=%d nh=%d", name, T, nh);
  int st = check_head_dim(d);
  if (st != NESO_OK) return st;
  if (!aligned16(Q) || !aligned16(K_rel) || !aligned16(bias_v) || !aligned16(Q_u) ||
      (reinterpret_cast<uintptr_t>(bias_u) & 3u) || !aligned2(rel_bias))
    return fail(NESO_EINVAL, "%s: Q/K_rel/bias_v/Q_u must be 16-byte aligned", name);
  if (T == 0 || nh == 0) return ok();
  if ((int64_t)T * T > 0x7fffffff || (int64_t)(2 * T - 1) * d > 0x7fffffff)
    return fail(NESO_EUNSUPPORTED, "%s: T=%d too large", name, T);
  neso::RelPreArgs a{};
  a.Q = Q;
  a.K_rel = K_rel;
  a.bias_u = bias_u;
  a.bias_v = bias_v;
  a.Q_u = static_cast<neso::half_t*>(Q_u);
  a.rel_bias = static_cast<neso::half_t*>(rel_bias);
  a.T = T;
  a.heads = nh;
  return launched(neso::launch_relpos_precompute(a, d, static_cast<hipStream_t>(stream)), name);
}

// True when a buffer of `bytes` bytes can be addressed with 32-bit offsets
// (the kernels' buffer resources and per-lane offsets are 32-bit).
static bool extent32(int64_t bytes) { return bytes < ((int64_t)1 << 32); }

int neso_w4a16_matmul(const void* X, const int32_t* W, const void* scales, void* Y, int32_t M,
                      int32_t N, int32_t K, int32_t stride_xm, int32_t stride_ym,
                      int32_t group_size, int32_t zero_point, void* stream) {
  const char* name = "w4a16_matmul";
  if (!X || !W || !scales || !Y) return fail(NESO_EINVAL, "%s: null tensor pointer", name);
  if (M < 0 || N < 0 || K < 0) return fail(NESO_EINVAL, "%s: negative size", name);
  if (K % 32) return fail(NESO_EINVAL, "%s: K=%d must be a multiple of 32", name, K);
  if (group_size <= 0 || group_size % 32 || (K && K % group_size))
    return fail(NESO_EINVAL, "%s: group_size=%d must be a multiple of 32 dividing K", name,
                group_size);
  if (zero_point < 0 || zero_point > 15)
    return fail(NESO_EINVAL, "%s: zero_point=%d outside [0, 15]", name, zero_point);
  if (stride_xm < K || stride_xm % 8)
    return fail(NESO_EINVAL, "%s: stride_xm=%d must be >= K and a multiple of 8", name,
                stride_xm);
  if (stride_ym < N) return fail(NESO_EINVAL, "%s: stride_ym=%d < N", name, stride_ym);
  if (!aligned16(X) || !aligned16(W) || !aligned2(scales) || !aligned2(Y))
    return fail(NESO_EINVAL, "%s: X/W must be 16-byte aligned, scales/Y 2-byte", name);
  if (M == 0 || N == 0) return ok();
  if (K == 0) return fail(NESO_EINVAL, "%s: K=0 with non-empty output", name);
  // The kernels address X and Y with 32-bit buffer offsets.
  if (!extent32(((int64_t)(M - 1) * stride_xm + K) * 2) ||
      !extent32(((int64_t)(M - 1) * stride_ym + N) * 2))
    return fail(NESO_EINVAL, "%s: X or Y spans 4 GiB or more (M=%d, stride_xm=%d, stride_ym=%d)",
                name, M, stride_xm, stride_ym);
  neso::W4Args a{};
  a.X = static_cast<const neso::half_t*>(X);
  a.W = reinterpret_cast<const uint32_t*>(W);
  a.S = static_cast<const neso::half_t*>(scales);
  a.Y = static_cast<neso::half_t*>(Y);
  a.M = M;
  a.N = N;
  a.K = K;
  a.ldx = stride_xm;
  a.ldy = stride_ym;
  a.group = group_size;
  a.zero = zero_point;
  return launched(neso::launch_w4a16(a, static_cast<hipStream_t>(stream)), name);
}

static int w8a16_common(const void* A, const int8_t* B, float* C, const void* scale, int32_t K,
                        int32_t stride_am, int32_t stride_bk, int32_t stride_cm, int32_t M,
                        int32_t N, void* stream, const char* name) {
  if (!A || !B || !C) return fail(NESO_EINVAL, "%s: null tensor pointer", name);
  if (M < 0 || N < 0 || K < 0) return fail(NESO_EINVAL, "%s: negative size", name);
  if (stride_am < K || stride_bk < N || stride_cm < N)
    return fail(NESO_EINVAL, "%s: stride smaller than the row it spans", name);
  if (!aligned2(A) || (scale && !aligned2(scale)) || (reinterpret_cast<uintptr_t>(C) & 3u))
    return fail(NESO_EINVAL, "%s: misaligned A/C/scale", name);
  if (M == 0 || N == 0) return ok();
  if (K == 0) return fail(NESO_EINVAL, "%s: K=0 with non-empty output", name);
  // The kernels address A (fp16) and B (int8) with 32-bit buffer offsets.
  if (!extent32(((int64_t)(M - 1) * stride_am + K) * 2) ||
      !extent32((int64_t)(K - 1) * stride_bk + N))
    return fail(NESO_EINVAL, "%s: A or B spans 4 GiB or more (M=%d, K=%d, stride_am=%d, "
                "stride_bk=%d)", name, M, K, stride_am, stride_bk);
  neso::W8Args a{};
  a.A = static_cast<const neso::half_t*>(A);
  a.B = B;
  a.C = C;
  a.scale = static_cast<const neso::half_t*>(scale);
  a.M = M;
  a.N = N;
  a.K = K;
  a.lda = stride_am;
  a.ldb = stride_bk;
  a.ldc = stride_cm;
  return launched(neso::launch_w8a16(a, static_cast<hipStream_t>(stream)), name);
}

int neso_w8a16_matmul(const void* A, const int8_t* B, float* C, int32_t K, int32_t stride_am,
                      int32_t stride_bk, int32_t stride_cm, int32_t M, int32_t N, void* stream) {
  return w8a16_common(A, B, C, nullptr, K, stride_am, stride_bk, stride_cm, M, N, stream,
                      "w8a16_matmul");
}

int neso_w8a16_scaled_matmul(const void* A, const int8_t* B, float* C, const void* scale,
                             int32_t K, int32_t stride_am, int32_t stride_bk, int32_t stride_cm,
                             int32_t M, int32_t N, void* stream) {
  if (!scale) return fail(NESO_EINVAL, "w8a16_scaled_matmul: null scale pointer");
  return w8a16_common(A, B, C, scale, K, stride_am, stride_bk, stride_cm, M, N, stream,
                      "w8a16_scaled_matmul");
}

}  // extern "C"
