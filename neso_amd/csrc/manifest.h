// JSON manifest of the C entry points (neso_kernel_manifest()), in the
// shape of the reference's AOT metadata (src/neso/aot_compile.py:108-117:
// kernel_name, params, constants, threadgroup_size, num_warps, grid).  An
// entry point picks one of several device kernels per call, so the fixed
// geometry fields are null and each variant gives its own as expressions
// over its template arguments and the call's sizes; tests/test_abi.py
// evaluates them against what the launchers choose (neso_plan_begin).
#pragma once

namespace neso {

constexpr char kManifest[] = R"JSON({
 "library": "neso_amd",
 "abi_version": 2,
 "target": "gfx950",
 "kernels": [
  {
   "kernel_name": "neso_flash_attention_fwd",
   "replaces": "flash_attention_fwd (tests/test_flash_attention.py:149-153)",
   "params": [
    {
     "index": 0,
     "name": "Q",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 1,
     "name": "K",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 2,
     "name": "V",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 3,
     "name": "O",
     "type": "fp32*",
     "is_pointer": true
    },
    {
     "index": 4,
     "name": "N",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 5,
     "name": "stride_qo",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 6,
     "name": "stride_kv",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 7,
     "name": "scale",
     "type": "fp32",
     "is_pointer": false
    },
    {
     "index": 8,
     "name": "head_dim",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 9,
     "name": "batch_heads",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 10,
     "name": "stride_bh_qo",
     "type": "int64",
     "is_pointer": false
    },
    {
     "index": 11,
     "name": "stride_bh_kv",
     "type": "int64",
     "is_pointer": false
    },
    {
     "index": 12,
     "name": "causal",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 13,
     "name": "stream",
     "type": "hipStream_t",
     "is_pointer": true
    }
   ],
   "constants": {
    "wave_size": 64,
    "head_dim": [
     32,
     64,
     128
    ]
   },
   "threadgroup_size": null,
   "num_warps": null,
   "grid": null,
   "launch": "chosen per call from the sizes below; each variant gives its geometry as expressions over its template arguments and the call's sizes (cdiv = ceiling division, cus = compute units); neso_plan_begin/neso_plan_end report the choice for a given call",
   "size_vars": {
    "N": "N",
    "batch_heads": "batch_heads"
   },
   "variants": [
    {
     "device_kernel": "fa2_fast_kernel",
     "source": "neso_amd/csrc/fa2_fast.hip",
     "template_params": [
      "D",
      "CAUSAL",
      "OUT_F16",
      "KSPLIT",
      "PAIR",
      "HALVES",
      "QW",
      "BIAS"
     ],
     "when": "fp16 Q/K/V at head_dim 64 or 128: without a bias where measured faster than fa2_fwd_kernel (fa2_fast_preferred), and with the f32 bias table whenever |scale| >= 1e-20 (BIAS 2: the table entries of a workgroup's rows, 32 * QW + N - 1, loaded once into the band slots' LDS when they fit, KSPLIT * QW * 2 * 128 or 64 floats; BIAS 1: per-block bands otherwise); KSPLIT key groups of QW query waves (QW = 2 on grids whose 128-query workgroups fill at most half the CUs, from N = 512 without a bias, with KSPLIT = 4 while cdiv(N, 64) * batch_heads <= cus and N >= 1024, else 2); PAIR (causal grids of >= 2 workgroups per CU with QW = 4; head_dim 128 causal without a window from N = 2048 when cdiv(cdiv(N, 64), 2) * batch_heads <= cus with QW = 2, KSPLIT = 4): each workgroup takes query blocks x and nqb-1-x; HALVES (causal without a window, fewer than 2 workgroups per CU, QW = 4): each workgroup takes the 64-row blocks x and cdiv(N, 64)-1-x",
     "threadgroup_size": "64 * QW * KSPLIT",
     "num_warps": "QW * KSPLIT",
     "grid": [
      "cdiv(cdiv(N, 64), 2) * batch_heads if HALVES else (cdiv(cdiv(N, 32 * QW), 2) * batch_heads if PAIR else cdiv(N, 32 * QW) * batch_heads)",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * QW",
      "block_n": "(64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32)",
      "lds_layout": "2 K + 2 V slots (scores kept for the slow path) if (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1))) else a 4-slot ring of K + V",
      "lds_bytes": "KSPLIT * ((4 if (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1))) else 8) * (64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32) * D * 2 + (QW * 2 * (128 if (64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32) == 64 else 64) * 4 if BIAS else 0)) + (256 if BIAS else 0)"
     }
    },
    {
     "device_kernel": "fa2_fwd_kernel",
     "source": "neso_amd/csrc/fa2_fwd.hip",
     "template_params": [
      "D",
      "CAUSAL",
      "BIAS",
      "OUT_F16",
      "KSPLIT",
      "F32IN",
      "QW"
     ],
     "when": "every other FA2 call: the dense f16 bias (BIAS 2), the f32 table (BIAS 1) with |scale| < 1e-20, fp32 input (F32IN), head_dim 32, and unbiased shapes where it is measured faster; QW query waves (2 on grids that fill at most half the CUs) and KSPLIT key groups per workgroup",
     "threadgroup_size": "64 * QW * KSPLIT",
     "num_warps": "QW * KSPLIT",
     "grid": [
      "cdiv(N, 32 * QW) * batch_heads",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * QW",
      "block_n": "32 if (F32IN and D == 128) else 64",
      "lds_double_buffer": "2"
     }
    }
   ]
  },
  {
   "kernel_name": "neso_flash_attention_f32_fwd",
   "replaces": "flash_attention_fwd with qkv_dtype='f32' (tests/test_flash_attention.py:79-89,250-290)",
   "params": [
    {
     "index": 0,
     "name": "Q",
     "type": "const fp32*",
     "is_pointer": true
    },
    {
     "index": 1,
     "name": "K",
     "type": "const fp32*",
     "is_pointer": true
    },
    {
     "index": 2,
     "name": "V",
     "type": "const fp32*",
     "is_pointer": true
    },
    {
     "index": 3,
     "name": "O",
     "type": "fp32*",
     "is_pointer": true
    },
    {
     "index": 4,
     "name": "N",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 5,
     "name": "stride_qo",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 6,
     "name": "stride_kv",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 7,
     "name": "scale",
     "type": "fp32",
     "is_pointer": false
    },
    {
     "index": 8,
     "name": "head_dim",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 9,
     "name": "batch_heads",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 10,
     "name": "stride_bh_qo",
     "type": "int64",
     "is_pointer": false
    },
    {
     "index": 11,
     "name": "stride_bh_kv",
     "type": "int64",
     "is_pointer": false
    },
    {
     "index": 12,
     "name": "causal",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 13,
     "name": "stream",
     "type": "hipStream_t",
     "is_pointer": true
    }
   ],
   "constants": {
    "wave_size": 64,
    "head_dim": [
     32,
     64,
     128
    ],
    "precision": "f32 inputs split into f16 hi + lo, three f16 MFMAs per product, f32 accumulation"
   },
   "threadgroup_size": null,
   "num_warps": null,
   "grid": null,
   "launch": "chosen per call from the sizes below; each variant gives its geometry as expressions over its template arguments and the call's sizes (cdiv = ceiling division, cus = compute units); neso_plan_begin/neso_plan_end report the choice for a given call",
   "size_vars": {
    "N": "N",
    "batch_heads": "batch_heads"
   },
   "variants": [
    {
     "device_kernel": "fa2_fwd_kernel",
     "source": "neso_amd/csrc/fa2_fwd.hip",
     "template_params": [
      "D",
      "CAUSAL",
      "BIAS",
      "OUT_F16",
      "KSPLIT",
      "F32IN",
      "QW"
     ],
     "when": "every other FA2 call: the dense f16 bias (BIAS 2), the f32 table (BIAS 1) with |scale| < 1e-20, fp32 input (F32IN), head_dim 32, and unbiased shapes where it is measured faster; QW query waves (2 on grids that fill at most half the CUs) and KSPLIT key groups per workgroup",
     "threadgroup_size": "64 * QW * KSPLIT",
     "num_warps": "QW * KSPLIT",
     "grid": [
      "cdiv(N, 32 * QW) * batch_heads",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * QW",
      "block_n": "32 if (F32IN and D == 128) else 64",
      "lds_double_buffer": "2"
     }
    }
   ]
  },
  {
   "kernel_name": "neso_flash_attention_io_fwd",
   "replaces": "flash_attention_fwd(Q, K, V, O, N, d_head, scale) (bench/bench_flash_attention.py:142-152)",
   "params": [
    {
     "index": 0,
     "name": "Q",
     "type": "const fp16*|const fp32*",
     "is_pointer": true
    },
    {
     "index": 1,
     "name": "K",
     "type": "const fp16*|const fp32*",
     "is_pointer": true
    },
    {
     "index": 2,
     "name": "V",
     "type": "const fp16*|const fp32*",
     "is_pointer": true
    },
    {
     "index": 3,
     "name": "O",
     "type": "fp16*|fp32*",
     "is_pointer": true
    },
    {
     "index": 4,
     "name": "N",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 5,
     "name": "d_head",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 6,
     "name": "scale",
     "type": "fp32",
     "is_pointer": false
    },
    {
     "index": 7,
     "name": "io_dtype",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 8,
     "name": "batch_heads",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 9,
     "name": "stream",
     "type": "hipStream_t",
     "is_pointer": true
    }
   ],
   "constants": {
    "wave_size": 64,
    "head_dim": [
     32,
     64,
     128
    ],
    "io_dtype": {
     "NESO_IO_F16": 0,
     "NESO_IO_F32": 1
    }
   },
   "threadgroup_size": null,
   "num_warps": null,
   "grid": null,
   "launch": "chosen per call from the sizes below; each variant gives its geometry as expressions over its template arguments and the call's sizes (cdiv = ceiling division, cus = compute units); neso_plan_begin/neso_plan_end report the choice for a given call",
   "size_vars": {
    "N": "N",
    "batch_heads": "batch_heads"
   },
   "variants": [
    {
     "device_kernel": "fa2_fast_kernel",
     "source": "neso_amd/csrc/fa2_fast.hip",
     "template_params": [
      "D",
      "CAUSAL",
      "OUT_F16",
      "KSPLIT",
      "PAIR",
      "HALVES",
      "QW",
      "BIAS"
     ],
     "when": "fp16 Q/K/V at head_dim 64 or 128: without a bias where measured faster than fa2_fwd_kernel (fa2_fast_preferred), and with the f32 bias table whenever |scale| >= 1e-20 (BIAS 2: the table entries of a workgroup's rows, 32 * QW + N - 1, loaded once into the band slots' LDS when they fit, KSPLIT * QW * 2 * 128 or 64 floats; BIAS 1: per-block bands otherwise); KSPLIT key groups of QW query waves (QW = 2 on grids whose 128-query workgroups fill at most half the CUs, from N = 512 without a bias, with KSPLIT = 4 while cdiv(N, 64) * batch_heads <= cus and N >= 1024, else 2); PAIR (causal grids of >= 2 workgroups per CU with QW = 4; head_dim 128 causal without a window from N = 2048 when cdiv(cdiv(N, 64), 2) * batch_heads <= cus with QW = 2, KSPLIT = 4): each workgroup takes query blocks x and nqb-1-x; HALVES (causal without a window, fewer than 2 workgroups per CU, QW = 4): each workgroup takes the 64-row blocks x and cdiv(N, 64)-1-x",
     "threadgroup_size": "64 * QW * KSPLIT",
     "num_warps": "QW * KSPLIT",
     "grid": [
      "cdiv(cdiv(N, 64), 2) * batch_heads if HALVES else (cdiv(cdiv(N, 32 * QW), 2) * batch_heads if PAIR else cdiv(N, 32 * QW) * batch_heads)",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * QW",
      "block_n": "(64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32)",
      "lds_layout": "2 K + 2 V slots (scores kept for the slow path) if (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1))) else a 4-slot ring of K + V",
      "lds_bytes": "KSPLIT * ((4 if (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1))) else 8) * (64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32) * D * 2 + (QW * 2 * (128 if (64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32) == 64 else 64) * 4 if BIAS else 0)) + (256 if BIAS else 0)"
     }
    },
    {
     "device_kernel": "fa2_fwd_kernel",
     "source": "neso_amd/csrc/fa2_fwd.hip",
     "template_params": [
      "D",
      "CAUSAL",
      "BIAS",
      "OUT_F16",
      "KSPLIT",
      "F32IN",
      "QW"
     ],
     "when": "every other FA2 call: the dense f16 bias (BIAS 2), the f32 table (BIAS 1) with |scale| < 1e-20, fp32 input (F32IN), head_dim 32, and unbiased shapes where it is measured faster; QW query waves (2 on grids that fill at most half the CUs) and KSPLIT key groups per workgroup",
     "threadgroup_size": "64 * QW * KSPLIT",
     "num_warps": "QW * KSPLIT",
     "grid": [
      "cdiv(N, 32 * QW) * batch_heads",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * QW",
      "block_n": "32 if (F32IN and D == 128) else 64",
      "lds_double_buffer": "2"
     }
    }
   ]
  },
  {
   "kernel_name": "neso_flash_attention_window_fwd",
   "replaces": "flash_attention_fwd with window_left/right (debug/fa2_correctness_legacy.py:92-102)",
   "params": [
    {
     "index": 0,
     "name": "Q",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 1,
     "name": "K",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 2,
     "name": "V",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 3,
     "name": "O",
     "type": "fp16*|fp32*",
     "is_pointer": true
    },
    {
     "index": 4,
     "name": "seq_len",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 5,
     "name": "stride_h",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 6,
     "name": "stride_m",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 7,
     "name": "sm_scale",
     "type": "fp32",
     "is_pointer": false
    },
    {
     "index": 8,
     "name": "window_left",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 9,
     "name": "window_right",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 10,
     "name": "num_heads",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 11,
     "name": "head_dim",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 12,
     "name": "out_dtype",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 13,
     "name": "stream",
     "type": "hipStream_t",
     "is_pointer": true
    }
   ],
   "constants": {
    "wave_size": 64,
    "head_dim": [
     32,
     64,
     128
    ],
    "out_dtype": {
     "NESO_OUT_F16": 0,
     "NESO_OUT_F32": 1
    }
   },
   "threadgroup_size": null,
   "num_warps": null,
   "grid": null,
   "launch": "chosen per call from the sizes below; each variant gives its geometry as expressions over its template arguments and the call's sizes (cdiv = ceiling division, cus = compute units); neso_plan_begin/neso_plan_end report the choice for a given call",
   "size_vars": {
    "N": "seq_len",
    "batch_heads": "num_heads"
   },
   "variants": [
    {
     "device_kernel": "fa2_fast_kernel",
     "source": "neso_amd/csrc/fa2_fast.hip",
     "template_params": [
      "D",
      "CAUSAL",
      "OUT_F16",
      "KSPLIT",
      "PAIR",
      "HALVES",
      "QW",
      "BIAS"
     ],
     "when": "fp16 Q/K/V at head_dim 64 or 128: without a bias where measured faster than fa2_fwd_kernel (fa2_fast_preferred), and with the f32 bias table whenever |scale| >= 1e-20 (BIAS 2: the table entries of a workgroup's rows, 32 * QW + N - 1, loaded once into the band slots' LDS when they fit, KSPLIT * QW * 2 * 128 or 64 floats; BIAS 1: per-block bands otherwise); KSPLIT key groups of QW query waves (QW = 2 on grids whose 128-query workgroups fill at most half the CUs, from N = 512 without a bias, with KSPLIT = 4 while cdiv(N, 64) * batch_heads <= cus and N >= 1024, else 2); PAIR (causal grids of >= 2 workgroups per CU with QW = 4; head_dim 128 causal without a window from N = 2048 when cdiv(cdiv(N, 64), 2) * batch_heads <= cus with QW = 2, KSPLIT = 4): each workgroup takes query blocks x and nqb-1-x; HALVES (causal without a window, fewer than 2 workgroups per CU, QW = 4): each workgroup takes the 64-row blocks x and cdiv(N, 64)-1-x",
     "threadgroup_size": "64 * QW * KSPLIT",
     "num_warps": "QW * KSPLIT",
     "grid": [
      "cdiv(cdiv(N, 64), 2) * batch_heads if HALVES else (cdiv(cdiv(N, 32 * QW), 2) * batch_heads if PAIR else cdiv(N, 32 * QW) * batch_heads)",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * QW",
      "block_n": "(64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32)",
      "lds_layout": "2 K + 2 V slots (scores kept for the slow path) if (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1))) else a 4-slot ring of K + V",
      "lds_bytes": "KSPLIT * ((4 if (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1))) else 8) * (64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32) * D * 2 + (QW * 2 * (128 if (64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32) == 64 else 64) * 4 if BIAS else 0)) + (256 if BIAS else 0)"
     }
    },
    {
     "device_kernel": "fa2_fwd_kernel",
     "source": "neso_amd/csrc/fa2_fwd.hip",
     "template_params": [
      "D",
      "CAUSAL",
      "BIAS",
      "OUT_F16",
      "KSPLIT",
      "F32IN",
      "QW"
     ],
     "when": "every other FA2 call: the dense f16 bias (BIAS 2), the f32 table (BIAS 1) with |scale| < 1e-20, fp32 input (F32IN), head_dim 32, and unbiased shapes where it is measured faster; QW query waves (2 on grids that fill at most half the CUs) and KSPLIT key groups per workgroup",
     "threadgroup_size": "64 * QW * KSPLIT",
     "num_warps": "QW * KSPLIT",
     "grid": [
      "cdiv(N, 32 * QW) * batch_heads",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * QW",
      "block_n": "32 if (F32IN and D == 128) else 64",
      "lds_double_buffer": "2"
     }
    }
   ]
  },
  {
   "kernel_name": "neso_rel_pos_fa2_fwd",
   "replaces": "rel_pos_fa2_fwd (tests/test_rel_pos_fa2.py:157-163)",
   "params": [
    {
     "index": 0,
     "name": "Q",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 1,
     "name": "K",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 2,
     "name": "V",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 3,
     "name": "bias",
     "type": "const fp16*|const fp32*",
     "is_pointer": true
    },
    {
     "index": 4,
     "name": "O",
     "type": "fp16*|fp32*",
     "is_pointer": true
    },
    {
     "index": 5,
     "name": "T",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 6,
     "name": "stride",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 7,
     "name": "scale",
     "type": "fp32",
     "is_pointer": false
    },
    {
     "index": 8,
     "name": "stride_h",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 9,
     "name": "bias_stride_h",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 10,
     "name": "num_heads",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 11,
     "name": "head_dim",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 12,
     "name": "bias_mode",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 13,
     "name": "out_dtype",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 14,
     "name": "stream",
     "type": "hipStream_t",
     "is_pointer": true
    }
   ],
   "constants": {
    "wave_size": 64,
    "head_dim": [
     32,
     64,
     128
    ],
    "bias_mode": {
     "NESO_BIAS_DENSE_SCALED_F16": 0,
     "NESO_BIAS_TABLE_F32": 1
    },
    "out_dtype": {
     "NESO_OUT_F16": 0,
     "NESO_OUT_F32": 1
    }
   },
   "threadgroup_size": null,
   "num_warps": null,
   "grid": null,
   "launch": "chosen per call from the sizes below; each variant gives its geometry as expressions over its template arguments and the call's sizes (cdiv = ceiling division, cus = compute units); neso_plan_begin/neso_plan_end report the choice for a given call",
   "size_vars": {
    "N": "T",
    "batch_heads": "num_heads"
   },
   "variants": [
    {
     "device_kernel": "fa2_fast_kernel",
     "source": "neso_amd/csrc/fa2_fast.hip",
     "template_params": [
      "D",
      "CAUSAL",
      "OUT_F16",
      "KSPLIT",
      "PAIR",
      "HALVES",
      "QW",
      "BIAS"
     ],
     "when": "fp16 Q/K/V at head_dim 64 or 128: without a bias where measured faster than fa2_fwd_kernel (fa2_fast_preferred), and with the f32 bias table whenever |scale| >= 1e-20 (BIAS 2: the table entries of a workgroup's rows, 32 * QW + N - 1, loaded once into the band slots' LDS when they fit, KSPLIT * QW * 2 * 128 or 64 floats; BIAS 1: per-block bands otherwise); KSPLIT key groups of QW query waves (QW = 2 on grids whose 128-query workgroups fill at most half the CUs, from N = 512 without a bias, with KSPLIT = 4 while cdiv(N, 64) * batch_heads <= cus and N >= 1024, else 2); PAIR (causal grids of >= 2 workgroups per CU with QW = 4; head_dim 128 causal without a window from N = 2048 when cdiv(cdiv(N, 64), 2) * batch_heads <= cus with QW = 2, KSPLIT = 4): each workgroup takes query blocks x and nqb-1-x; HALVES (causal without a window, fewer than 2 workgroups per CU, QW = 4): each workgroup takes the 64-row blocks x and cdiv(N, 64)-1-x",
     "threadgroup_size": "64 * QW * KSPLIT",
     "num_warps": "QW * KSPLIT",
     "grid": [
      "cdiv(cdiv(N, 64), 2) * batch_heads if HALVES else (cdiv(cdiv(N, 32 * QW), 2) * batch_heads if PAIR else cdiv(N, 32 * QW) * batch_heads)",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * QW",
      "block_n": "(64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32)",
      "lds_layout": "2 K + 2 V slots (scores kept for the slow path) if (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1))) else a 4-slot ring of K + V",
      "lds_bytes": "KSPLIT * ((4 if (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1))) else 8) * (64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32) * D * 2 + (QW * 2 * (128 if (64 if (D == 64 and not (BIAS and QW == 4)) or (D == 128 and QW == 4 and (QW == 2 or (D == 128 and not BIAS and not HALVES and not (PAIR and KSPLIT == 1)))) else 32) == 64 else 64) * 4 if BIAS else 0)) + (256 if BIAS else 0)"
     }
    },
    {
     "device_kernel": "fa2_fwd_kernel",
     "source": "neso_amd/csrc/fa2_fwd.hip",
     "template_params": [
      "D",
      "CAUSAL",
      "BIAS",
      "OUT_F16",
      "KSPLIT",
      "F32IN",
      "QW"
     ],
     "when": "every other FA2 call: the dense f16 bias (BIAS 2), the f32 table (BIAS 1) with |scale| < 1e-20, fp32 input (F32IN), head_dim 32, and unbiased shapes where it is measured faster; QW query waves (2 on grids that fill at most half the CUs) and KSPLIT key groups per workgroup",
     "threadgroup_size": "64 * QW * KSPLIT",
     "num_warps": "QW * KSPLIT",
     "grid": [
      "cdiv(N, 32 * QW) * batch_heads",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * QW",
      "block_n": "32 if (F32IN and D == 128) else 64",
      "lds_double_buffer": "2"
     }
    }
   ]
  },
  {
   "kernel_name": "neso_rel_pos_precompute",
   "replaces": "precompute_bias_and_qu(Q, K_rel, bias_u, bias_v, T, d, nh, scale) (tests/test_rel_pos_fa2.py:286-311), host-side in the reference",
   "params": [
    {
     "index": 0,
     "name": "Q",
     "type": "const fp32*",
     "is_pointer": true
    },
    {
     "index": 1,
     "name": "K_rel",
     "type": "const fp32*",
     "is_pointer": true
    },
    {
     "index": 2,
     "name": "bias_u",
     "type": "const fp32*",
     "is_pointer": true
    },
    {
     "index": 3,
     "name": "bias_v",
     "type": "const fp32*",
     "is_pointer": true
    },
    {
     "index": 4,
     "name": "T",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 5,
     "name": "d",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 6,
     "name": "nh",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 7,
     "name": "scale",
     "type": "fp32",
     "is_pointer": false
    },
    {
     "index": 8,
     "name": "Q_u",
     "type": "fp16*",
     "is_pointer": true
    },
    {
     "index": 9,
     "name": "rel_bias",
     "type": "fp16*",
     "is_pointer": true
    },
    {
     "index": 10,
     "name": "stream",
     "type": "hipStream_t",
     "is_pointer": true
    }
   ],
   "constants": {
    "wave_size": 64,
    "head_dim": [
     32,
     64,
     128
    ],
    "rel_bias": "unscaled, (Q + bias_v)_i . K_rel[T - 1 - i + j]"
   },
   "threadgroup_size": null,
   "num_warps": null,
   "grid": null,
   "launch": "one variant per head_dim; geometry below",
   "size_vars": {
    "T": "T",
    "nh": "nh"
   },
   "variants": [
    {
     "device_kernel": "relpos_precompute_kernel",
     "source": "neso_amd/csrc/relpos_pre.hip",
     "template_params": [
      "D"
     ],
     "when": "always",
     "threadgroup_size": "256",
     "num_warps": "4",
     "grid": [
      "cdiv(T, 128)",
      "nh",
      "cdiv((T - 1 + (127 if T > 127 else T - 1)) // 32 + 1, 8)"
     ],
     "constants": {
      "block_m": "32 per wave, 128 per workgroup",
      "relative_positions_per_tile": "32",
      "tiles_per_workgroup": "8",
      "lds_bytes": "256 * D",
      "mfma": "v_mfma_f32_32x32x16_f16 x3 (fp32 split into fp16 hi + lo: hi.hi + hi.lo + lo.hi)"
     }
    }
   ]
  },
  {
   "kernel_name": "neso_w4a16_matmul",
   "replaces": null,
   "params": [
    {
     "index": 0,
     "name": "X",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 1,
     "name": "W",
     "type": "const int32*",
     "is_pointer": true
    },
    {
     "index": 2,
     "name": "scales",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 3,
     "name": "Y",
     "type": "fp16*",
     "is_pointer": true
    },
    {
     "index": 4,
     "name": "M",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 5,
     "name": "N",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 6,
     "name": "K",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 7,
     "name": "stride_xm",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 8,
     "name": "stride_ym",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 9,
     "name": "group_size",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 10,
     "name": "zero_point",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 11,
     "name": "stream",
     "type": "hipStream_t",
     "is_pointer": true
    }
   ],
   "constants": {
    "wave_size": 64,
    "format": "int4 codes packed 8 per int32 along K, low nibble first; fp16 scales per (n, group)"
   },
   "threadgroup_size": null,
   "num_warps": null,
   "grid": null,
   "launch": "chosen per call from M, N, K and the group size; see variants",
   "size_vars": {
    "M": "M",
    "N": "N",
    "K": "K"
   },
   "variants": [
    {
     "device_kernel": "w4a16_gemv_kernel",
     "source": "neso_amd/csrc/qmatmul.hip",
     "template_params": [
      "MR",
      "GI",
      "R",
      "PS"
     ],
     "when": "M <= 2 and K <= 8192: GEMV, one wave per R output rows, MR rows of X",
     "threadgroup_size": "256",
     "num_warps": "4",
     "grid": [
      "cdiv(cdiv(cdiv(N, R), 4), cus) * cus if cdiv(cdiv(N, R), 4) > cus else cdiv(cdiv(N, R), 4)",
      "1",
      "1"
     ],
     "constants": {
      "rows_per_wave": "R",
      "scale_groups_per_load": "GI"
     }
    },
    {
     "device_kernel": "w4a16_skinny_lds_kernel",
     "source": "neso_amd/csrc/qmatmul_skinny.hip",
     "template_params": [
      "WV",
      "T",
      "QWMAX"
     ],
     "when": "3 <= M <= 16, group 32, K % 128 == 0, K <= 4096: X in LDS, WV waves split K, T 16-column tiles per workgroup",
     "threadgroup_size": "64 * WV",
     "num_warps": "WV",
     "grid": [
      "cdiv(cdiv(N, 16), T)",
      "1",
      "1"
     ],
     "constants": {
      "tiles_per_workgroup": "T",
      "block_n": "16"
     }
    },
    {
     "device_kernel": "w4a16_skinny_kernel",
     "source": "neso_amd/csrc/qmatmul.hip",
     "template_params": [
      "MT",
      "NT",
      "WV",
      "G32"
     ],
     "when": "M <= 16 outside the case above (past its K only where the tile GEMM's 32 x 32 grid would not fit on the CUs), and 17 <= M <= 32 when the tile GEMM is off (NESO_AMD_W4_TILE_GEMM = 0) or its offsets pass 2^31 bytes (NESO_AMD_W4_SKINNY_MAX_M forces it up to that M, at most 64)",
     "threadgroup_size": "64 * WV",
     "num_warps": "WV",
     "grid": [
      "cdiv(N, 32)",
      "1 if MT == 1 else cdiv(M, 32)",
      "1"
     ],
     "constants": {
      "block_m": "16 * MT",
      "block_n": "32"
     }
    },
    {
     "device_kernel": "w4a16_tile_gemm_kernel",
     "source": "neso_amd/csrc/qmatmul.hip",
     "template_params": [
      "KG",
      "WN",
      "MI"
     ],
     "when": "M > 16, and M <= 16 past the X-in-LDS kernel's K where the 32 x 32 grid fits on the CUs: 32 MI x 32 WN tiles, each wave a 32 MI x 32 column strip with its weights dequantised once into MFMA registers and X through LDS, KG K-groups of WN waves per workgroup; the finest of 32 x 32 (MI = 1, WN = 1, KG = 8), 32 x 64 (MI = 1), 64 x 64 (MI = 2) and 128 x 64 (MI = 4) tiles (WN = 2, KG = 4) whose cdiv(M, 32 MI) * cdiv(N, 32 WN) <= cus; when none fits: M >= 65 (NESO_AMD_W4_WIDE_TILE_MIN_M overrides): WN = 4, MI = 4, KG = 2 while cdiv(M, 128) * cdiv(N, 128) <= cus, else KG = 1 from M = 129 and WN = 2, MI = 4, KG = 2 below; 33 <= M <= 64: WN = 2, MI = 2, KG = 4; 17 <= M <= 32: WN = 2, MI = 1, KG = 4; KG > 1 steps sync per K-group through LDS arrival counters when MI = 4 and cdiv(cdiv(K, 64), KG) >= 16, or cdiv(cdiv(K, 64), KG) >= 32 (NESO_AMD_W4_TILE_SYNC overrides), else through workgroup barriers; WN = 1 groups (one wave) sync through a wave-level fence only",
     "threadgroup_size": "64 * WN * KG",
     "num_warps": "WN * KG",
     "grid": [
      "cdiv(M, 32 * MI) * cdiv(N, 32 * WN)",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "32 * MI",
      "block_n": "32 * WN",
      "block_k": "64"
     }
    },
    {
     "device_kernel": "w4a16_gemm_kernel",
     "source": "neso_amd/csrc/qmatmul.hip",
     "template_params": [
      "WM",
      "WN",
      "BN"
     ],
     "when": "32 < M: only when the tile GEMM's buffer offsets would pass 2^31 bytes, or NESO_AMD_W4_TILE_GEMM = 0",
     "threadgroup_size": "64 * WM * WN",
     "num_warps": "WM * WN",
     "grid": [
      "cdiv(M, 128) * cdiv(N, BN)",
      "1",
      "1"
     ],
     "constants": {
      "block_m": "128",
      "block_n": "BN",
      "block_k": "64"
     }
    },
    {
     "device_kernel": "w4a16_mfma_kernel",
     "source": "neso_amd/csrc/qmatmul.hip",
     "template_params": [
      "TN"
     ],
     "when": "fallback when the tiled kernels' 32-bit buffer offsets would overflow",
     "threadgroup_size": "256",
     "num_warps": "4",
     "grid": [
      "cdiv(N, 128 * TN)",
      "cdiv(M, 32)",
      "1"
     ],
     "constants": {
      "block_m": "32",
      "block_n": "128 * TN"
     }
    }
   ]
  },
  {
   "kernel_name": "neso_w8a16_matmul",
   "replaces": "w8a16_matmul (tests/test_quantized_matmul.py:77-80)",
   "params": [
    {
     "index": 0,
     "name": "A",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 1,
     "name": "B",
     "type": "const int8*",
     "is_pointer": true
    },
    {
     "index": 2,
     "name": "C",
     "type": "fp32*",
     "is_pointer": true
    },
    {
     "index": 3,
     "name": "K",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 4,
     "name": "stride_am",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 5,
     "name": "stride_bk",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 6,
     "name": "stride_cm",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 7,
     "name": "M",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 8,
     "name": "N",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 9,
     "name": "stream",
     "type": "hipStream_t",
     "is_pointer": true
    }
   ],
   "constants": {
    "wave_size": 64,
    "b_layout": "int8 [K][N] row-major (stride_bk)",
    "c_dtype": "fp32"
   },
   "threadgroup_size": null,
   "num_warps": null,
   "grid": null,
   "launch": "chosen per call from the shape and alignment; see variants",
   "size_vars": {
    "M": "M",
    "N": "N",
    "K": "K"
   },
   "variants": [
    {
     "device_kernel": "w8a16_gemm_kernel",
     "source": "neso_amd/csrc/qmatmul.hip",
     "template_params": [
      "T"
     ],
     "when": "K, N, lda, ldb multiples of 8 and A 16-byte / B 8-byte aligned: T x T MFMA tiles, B dequantised into LDS as [k][n] f16 and read transposed; T = 256 (eight waves of 64 x 128) when cdiv(M, 256) * cdiv(N, 256) >= cus, else T = 128 (four waves of 64 x 64)",
     "threadgroup_size": "2 * T",
     "num_warps": "T // 32",
     "grid": [
      "cdiv(N, T)",
      "cdiv(M, T)",
      "1"
     ],
     "constants": {
      "block_m": "T",
      "block_n": "T",
      "block_k": "64"
     }
    },
    {
     "device_kernel": "w8a16_kernel",
     "source": "neso_amd/csrc/qmatmul.hip",
     "template_params": [],
     "when": "any other shape or alignment",
     "threadgroup_size": "256",
     "num_warps": "4",
     "grid": [
      "cdiv(N, 128)",
      "cdiv(M, 32)",
      "1"
     ],
     "constants": {
      "block_m": "32",
      "block_n": "128"
     }
    }
   ]
  },
  {
   "kernel_name": "neso_w8a16_scaled_matmul",
   "replaces": "w8a16_scaled_matmul (tests/test_quantized_matmul.py:189-192)",
   "params": [
    {
     "index": 0,
     "name": "A",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 1,
     "name": "B",
     "type": "const int8*",
     "is_pointer": true
    },
    {
     "index": 2,
     "name": "C",
     "type": "fp32*",
     "is_pointer": true
    },
    {
     "index": 3,
     "name": "scale",
     "type": "const fp16*",
     "is_pointer": true
    },
    {
     "index": 4,
     "name": "K",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 5,
     "name": "stride_am",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 6,
     "name": "stride_bk",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 7,
     "name": "stride_cm",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 8,
     "name": "M",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 9,
     "name": "N",
     "type": "int32",
     "is_pointer": false
    },
    {
     "index": 10,
     "name": "stream",
     "type": "hipStream_t",
     "is_pointer": true
    }
   ],
   "constants": {
    "wave_size": 64,
    "b_layout": "int8 [K][N] row-major (stride_bk)",
    "c_dtype": "fp32"
   },
   "threadgroup_size": null,
   "num_warps": null,
   "grid": null,
   "launch": "chosen per call from the shape and alignment; see variants",
   "size_vars": {
    "M": "M",
    "N": "N",
    "K": "K"
   },
   "variants": [
    {
     "device_kernel": "w8a16_gemm_kernel",
     "source": "neso_amd/csrc/qmatmul.hip",
     "template_params": [
      "T"
     ],
     "when": "K, N, lda, ldb multiples of 8 and A 16-byte / B 8-byte aligned: T x T MFMA tiles, B dequantised into LDS as [k][n] f16 and read transposed; T = 256 (eight waves of 64 x 128) when cdiv(M, 256) * cdiv(N, 256) >= cus, else T = 128 (four waves of 64 x 64)",
     "threadgroup_size": "2 * T",
     "num_warps": "T // 32",
     "grid": [
      "cdiv(N, T)",
      "cdiv(M, T)",
      "1"
     ],
     "constants": {
      "block_m": "T",
      "block_n": "T",
      "block_k": "64"
     }
    },
    {
     "device_kernel": "w8a16_kernel",
     "source": "neso_amd/csrc/qmatmul.hip",
     "template_params": [],
     "when": "any other shape or alignment",
     "threadgroup_size": "256",
     "num_warps": "4",
     "grid": [
      "cdiv(N, 128)",
      "cdiv(M, 32)",
      "1"
     ],
     "constants": {
      "block_m": "32",
      "block_n": "128"
     }
    }
   ]
  }
 ]
})JSON";

}  // namespace neso
