/*
 * neso_amd — C ABI of the MI355X (gfx950) kernels behind neso's hot path.
 *
 * Every entry point takes device pointers the caller owns, sizes and element
 * strides by value, and an optional HIP stream (`void*` = hipStream_t, NULL =
 * the null stream).  Nothing here allocates, copies or synchronises: a call
 * validates its arguments on the host, enqueues one kernel on `stream` and
 * returns.  Validation happens before any HIP call, so argument errors are
 * reported on hosts without a GPU.
 *
 * fp16 buffers are IEEE binary16, passed as `const void*`.
 *
 * Status codes: NESO_OK, NESO_EINVAL (bad argument), NESO_EUNSUPPORTED
 * (valid but not implemented, e.g. head_dim 96), NESO_ELAUNCH (the HIP
 * launch failed; neso_last_error() carries hipGetErrorString).  Calls are
 * thread-safe; neso_last_error() is per thread.
 */
#ifndef NESO_AMD_H_
#define NESO_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NESO_OK 0
#define NESO_EINVAL 1
#define NESO_EUNSUPPORTED 2
#define NESO_ELAUNCH 3

/* rel_pos_fa2_fwd bias_mode */
#define NESO_BIAS_DENSE_SCALED_F16 0 /* bias f16 [h][T][T], logits = (QK^T + B) * scale */
#define NESO_BIAS_TABLE_F32 1        /* bias f32 [h][2T-1], logits = QK^T * scale + B[i-j+T-1] */

/* output dtype selector */
#define NESO_OUT_F16 0
#define NESO_OUT_F32 1

/* element type of Q, K, V and O for neso_flash_attention_io_fwd */
#define NESO_IO_F16 0
#define NESO_IO_F32 1

/* Version of this ABI (bumped on any signature change). */
int neso_abi_version(void);

/* Text of a status code. */
const char* neso_status_string(int status);

/* Detail of the last non-OK status returned on this thread ("" if none). */
const char* neso_last_error(void);

/* JSON manifest of the entry points: name, positional parameters (name,
 * C type, pointer or scalar), reference kernel they replace, constraints.
 * Role of the reference's AOT manifest, src/neso/aot_compile.py:108-117. */
const char* neso_kernel_manifest(void);

/*
 * Launch-plan recording (no GPU needed).  Between neso_plan_begin and
 * neso_plan_end, calls made on this thread validate their arguments and
 * choose their kernels exactly as usual, but record each kernel launch
 * instead of issuing it; no HIP call is made.  cu_count > 0 stands in for
 * the device's compute-unit count (0: the current device's).
 * neso_plan_end returns JSON {"launches": [{"device_kernel", "template_args"
 * (bools as 0/1), "grid": [x, y, z], "threadgroup_size", "num_warps"}]},
 * valid until the next neso_plan_end on this thread.  It is how the
 * manifest's per-variant geometry is checked against the launchers, the
 * role of the reference's AOT metadata (src/neso/aot_compile.py:108-117).
 */
int neso_plan_begin(int32_t cu_count);
const char* neso_plan_end(void);

/*
 * Shader-clock sampler, a measurement aid with no counterpart in the
 * reference.  Launches one wave on `stream` that writes `samples` pairs
 * (shader-clock counter, 100 MHz reference counter) to out[2 i], out[2 i + 1],
 * one pair every `gap_ticks` reference ticks (gap_ticks / 100 us), and then
 * exits.  Launched on a second stream while a workload runs on another, it
 * gives the clock that workload ran at: d(out[2 i]) / d(out[2 i + 1]) * 100
 * MHz.  `out` is device memory of 2 * samples uint64 values, 8-byte aligned;
 * 1 <= samples, gap_ticks <= 2^20, and samples * gap_ticks <= 2^30 (the wave
 * runs at most 10.7 s).
 */
int neso_clock_sample(uint64_t* out, int32_t samples, int32_t gap_ticks, void* stream);

/*
 * Streaming-floor probe, a measurement aid with no counterpart in the
 * reference: what a launch of an HBM-bound kernel costs when it only moves
 * its bytes.  mode 0 launches `grid` workgroups of 256 threads that do
 * nothing (dispatch and the kernel boundary alone); mode 1 reads `bytes`
 * bytes from `src` with 16-byte non-temporal loads, a rolling window of four
 * in flight per lane, thread t of the grid's T threads reading pieces t,
 * t + T, ..., and writes sink[0] only if the XOR of everything that lane
 * read equals `key` (which keeps the loads live without stores); mode 2
 * reads the same way and writes every lane's XOR to sink[t], so that the
 * XOR of sink[0 .. T-1] is the XOR of the buffer (a coverage check).
 * 1 <= grid <= 2^20; modes 1 and 2: src 16-byte aligned, bytes a positive
 * multiple of 16 needing at most 16 pieces per thread
 * (bytes <= 16 * 16 * 256 * grid) and below 4 GiB, sink 4-byte aligned and,
 * for mode 2, holding 256 * grid uint32 values.
 */
int neso_stream_probe(const void* src, int64_t bytes, int32_t grid, int32_t mode, uint32_t key,
                      uint32_t* sink, void* stream);

/*
 * Flash-Attention-2 forward.  Replaces the `flash_attention_fwd` kernel of
 * tests/test_flash_attention.py:149-153 (launched at :287-290 and by
 * macos/harness.rs:149-169 with buffers 0-3 = Q, K, V, O and scalars 4-7 =
 * N, stride_qo, stride_kv, scale).  The first eight parameters keep that
 * order and meaning:
 *   Q, K, V   fp16 [N][d] rows (row stride stride_qo / stride_kv elements)
 *   O         fp32 [N][d] rows, row stride stride_qo (as in the reference)
 *   N         sequence length (queries == keys); no multiple-of-block rule
 *   scale     softmax scale (1/sqrt(d) in the reference)
 * Extensions (the reference bakes d into the kernel and launches one head):
 *   head_dim     32, 64 or 128
 *   batch_heads  number of independent (batch, head) slices, >= 1
 *   stride_bh_qo, stride_bh_kv  element distance between slices of Q/O, K/V
 *   causal       0: full attention; 1: key j visible to query i iff j <= i
 * Strides and pointers must allow 16-byte loads: strides multiple of 8,
 * pointers 16-byte aligned.  O = softmax(Q K^T * scale) V, softmax in fp32,
 * P rounded to fp16 before P V (reference :140-145), fp32 accumulation.
 */
int neso_flash_attention_fwd(const void* Q, const void* K, const void* V, float* O, int32_t N,
                             int32_t stride_qo, int32_t stride_kv, float scale, int32_t head_dim,
                             int32_t batch_heads, int64_t stride_bh_qo, int64_t stride_bh_kv,
                             int32_t causal, void* stream);

/*
 * Flash-Attention-2 forward on fp32 Q, K, V: the reference's default
 * `generate_fa2_ttir(..., qkv_dtype='f32')` kernel of
 * tests/test_flash_attention.py:79-89 (f32 buffers packed at :277-280,
 * same buffer order as above).  Parameters as neso_flash_attention_fwd,
 * except:
 *   Q, K, V   fp32 rows; strides and slice strides multiples of 4 elements
 *   head_dim  32, 64 or 128
 * Each fp32 operand is split into fp16 hi + lo and every product is formed
 * as hi*hi + hi*lo + lo*hi on the fp16 MFMA with fp32 accumulation, as is P
 * for P V, so results track an fp32 computation (about 1e-6 absolute for
 * unit-scale inputs).  Q, K, V elements must lie within the fp16 range
 * (|x| < 65504), and a tensor whose largest |x| is below about 2^-2 loses
 * relative accuracy (its lo parts fall into fp16 subnormals).  A caller
 * brings either case into range exactly with power-of-two factors: Q * 2^a
 * and K * 2^b with scale * 2^-(a+b), V * 2^c with O * 2^-c afterwards (the
 * Python layer, neso_amd.flash_attention_fwd, does this from one device
 * reduction per input).
 */
int neso_flash_attention_f32_fwd(const float* Q, const float* K, const float* V, float* O,
                                 int32_t N, int32_t stride_qo, int32_t stride_kv, float scale,
                                 int32_t head_dim, int32_t batch_heads, int64_t stride_bh_qo,
                                 int64_t stride_bh_kv, int32_t causal, void* stream);

/*
 * Flash-Attention-2 forward with O in the input type.  Replaces the
 * hand-written `flash_attention_fwd(Q, K, V, O, N, d_head, scale)` kernel of
 * bench/bench_flash_attention.py:142-152 (buffers 0-3, scalars 4-6, io_type
 * half or float for all four buffers; O row r at r * d_head, :361).  The
 * first seven parameters keep that order and meaning:
 *   Q, K, V, O  [N][d_head] rows of io_dtype, row stride d_head
 *   N           sequence length; d_head 32, 64 or 128; scale as the reference
 * Appended: io_dtype (NESO_IO_F16: fp16 Q/K/V/O, fp32 softmax and
 * accumulation, O rounded to fp16 once at the end; NESO_IO_F32: fp32
 * Q/K/V/O through the split-precision kernel of neso_flash_attention_f32_fwd),
 * batch_heads (contiguous [batch_heads][N][d_head] slices, >= 1) and stream.
 */
int neso_flash_attention_io_fwd(const void* Q, const void* K, const void* V, void* O, int32_t N,
                                int32_t d_head, float scale, int32_t io_dtype,
                                int32_t batch_heads, void* stream);

/*
 * Sliding-window attention.  Replaces the windowed `flash_attention_fwd`
 * kernel exercised by debug/fa2_correctness_legacy.py:92-102 (buffers
 * Q, K, V, O; scalars seq_len, stride_h, stride_m, sm_scale, window_left,
 * window_right, in that order), whose reference is :53-64: key j is visible
 * to query i iff i - window_left <= j <= i + window_right.  Layout as in the
 * reference: row i of head h starts at element i * stride_m + h * stride_h
 * of Q, K, V and O (e.g. [seq][heads * head_dim] with stride_h = head_dim).
 * Appended: num_heads, head_dim (32, 64, 128), out_dtype (NESO_OUT_F16 as
 * the reference kernel, or NESO_OUT_F32), stream.  Windows are clamped to
 * seq_len; negative windows are NESO_EINVAL.
 */
int neso_flash_attention_window_fwd(const void* Q, const void* K, const void* V, void* O,
                                    int32_t seq_len, int32_t stride_h, int32_t stride_m,
                                    float sm_scale, int32_t window_left, int32_t window_right,
                                    int32_t num_heads, int32_t head_dim, int32_t out_dtype,
                                    void* stream);

/*
 * Relative-position-bias FA2.  Replaces `rel_pos_fa2_fwd` of
 * tests/test_rel_pos_fa2.py:157-163 (grid (T/BM, nh) at :364-368).  The
 * first ten parameters keep the reference order and meaning:
 *   Q, K, V       fp16 [nh][T][d], row stride `stride`, head stride `stride_h`
 *   bias          per bias_mode (head stride bias_stride_h elements):
 *                   NESO_BIAS_DENSE_SCALED_F16 - f16 [nh][T][T] (reference
 *                     kernel: logits = (QK^T + bias) * scale)
 *                   NESO_BIAS_TABLE_F32 - f32 [nh][2T-1] table, logits =
 *                     QK^T * scale + bias[i - j + T - 1]
 *   O             [nh][T][d] (out_dtype NESO_OUT_F16 as the reference, or
 *                 NESO_OUT_F32), row stride `stride`, head stride `stride_h`
 *   T, stride, scale, stride_h, bias_stride_h  as in the reference
 * Extensions: num_heads (the reference's grid y), head_dim (32/64/128),
 * bias_mode, out_dtype.  T needs no multiple-of-block rule (tails masked).
 */
int neso_rel_pos_fa2_fwd(const void* Q, const void* K, const void* V, const void* bias, void* O,
                         int32_t T, int32_t stride, float scale, int32_t stride_h,
                         int32_t bias_stride_h, int32_t num_heads, int32_t head_dim,
                         int32_t bias_mode, int32_t out_dtype, void* stream);

/*
 * Relative-position bias precompute for the reference-signature kernel
 * above.  Replaces the host-side `precompute_bias_and_qu(Q, K_rel, bias_u,
 * bias_v, T, d, nh, scale)` of tests/test_rel_pos_fa2.py:286-311 (same
 * leading arguments and order; `scale` is accepted and unused there too,
 * the bias is returned unscaled).  Inputs fp32, contiguous:
 *   Q [nh][T][d], K_rel [nh][2T-1][d], bias_u, bias_v [nh][d]
 * Outputs fp16, contiguous, ready for neso_rel_pos_fa2_fwd with
 * NESO_BIAS_DENSE_SCALED_F16:
 *   Q_u [nh][T][d]      = Q + bias_u
 *   rel_bias [nh][T][T] = (Q + bias_v)_i . K_rel[T-1-i+j]   rounded to fp16
 *                         once
 * The dot products run on fp16 MFMAs: each fp32 factor x is split into
 * fp16 hi = fp16(x) and lo = fp16(x - hi), and hi*hi + hi*lo + lo*hi is
 * summed in fp32 (lo*lo dropped).  This needs |Q + bias_v| and |K_rel| below
 * 65504, the fp16 limit (larger elements give inf/NaN bias rows); the
 * result is fp32-class for elements above about 2^-10 in magnitude.
 * d 32, 64 or 128; Q, K_rel, bias_v and Q_u 16-byte aligned.
 */
int neso_rel_pos_precompute(const float* Q, const float* K_rel, const float* bias_u,
                            const float* bias_v, int32_t T, int32_t d, int32_t nh, float scale,
                            void* Q_u, void* rel_bias, void* stream);

/*
 * Weight-only int4 matmul, Y[M][N] fp16 = X[M][K] fp16 * dequant(W)^T.
 * No reference kernel packs int4 (the reference's W4A16 stores one int4
 * value per int8, tests/test_quantized_matmul.py:170-178); this is the
 * BASELINE format:
 *   W       int32 [N][K/8]; code of column k = nibble (k % 8) of word k/8,
 *           low nibble first
 *   scales  fp16 [N][K/group_size]
 *   dequant(c) = (c - zero_point) * scale; fp32 accumulation, fp16 output
 * K multiple of 32, group_size a multiple of 32 dividing K, 0 <= zero_point
 * <= 15, X rows 16-byte aligned (stride_xm multiple of 8).
 */
int neso_w4a16_matmul(const void* X, const int32_t* W, const void* scales, void* Y, int32_t M,
                      int32_t N, int32_t K, int32_t stride_xm, int32_t stride_ym,
                      int32_t group_size, int32_t zero_point, void* stream);

/*
 * W8A16 matmul, C[M][N] fp32 = A[M][K] fp16 * f16(B[K][N] int8).  Replaces
 * `w8a16_matmul` of tests/test_quantized_matmul.py:77-80 (positional
 * A, B, C, K, stride_am, stride_bk, stride_cm).  The reference takes M and
 * N from the launch grid; here they are explicit trailing parameters.
 */
int neso_w8a16_matmul(const void* A, const int8_t* B, float* C, int32_t K, int32_t stride_am,
                      int32_t stride_bk, int32_t stride_cm, int32_t M, int32_t N, void* stream);

/*
 * W8A16 with per-output-channel scale applied after accumulation,
 * C = (A * f16(B)) * scale[n], scale fp16 [N].  Replaces
 * `w8a16_scaled_matmul` of tests/test_quantized_matmul.py:189-192
 * (positional A, B, C, scale, K, stride_am, stride_bk, stride_cm).
 */
int neso_w8a16_scaled_matmul(const void* A, const int8_t* B, float* C, const void* scale,
                             int32_t K, int32_t stride_am, int32_t stride_bk, int32_t stride_cm,
                             int32_t M, int32_t N, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NESO_AMD_H_ */
