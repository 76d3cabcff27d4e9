#pragma once
/// @file gemm.h
/// C++ GEMM entry points of the gfx950 implementation.
///
/// Every declaration keeps the signature of the reference header
/// (include/dnnopt/gemm/gemm.h:14-58 and :97-100) so existing callers
/// recompile and relink unchanged.  Semantics shared with the reference:
///   * all matrices are row-major and ld* are row strides in elements;
///   * M<=0, N<=0 or K<=0 returns without touching C (gemm.cpp:180);
///   * beta==0 never reads C (gemm_tiny_fp32.cpp:202-203);
///   * every call is synchronous: C holds the result when the call returns.
///
/// A, B and C may be host or device memory.  Device (or managed) pointers
/// are used in place; host pointers are staged through library-owned device
/// buffers.  The calls return void like the reference; a failure leaves C
/// unmodified, is recorded in a thread-local status readable through
/// dnnopt_hip_last_status() (dnnopt_hip.h) and is reported once on stderr.

#include <cstdint>

#include "dnnopt/gemm/gemm_types.h"

namespace dnnopt {

/// C = alpha * A * B + beta * C with A: M x K, B: K x N, C: M x N (fp32).
/// Reference: src/gemm/gemm.cpp:168-173.
void gemm_fp32(int M, int N, int K,
               float alpha, const float* A, int lda,
               const float* B, int ldb,
               float beta, float* C, int ldc);

/// fp32 GEMM with an explicit algorithm request.
/// Reference: src/gemm/gemm.cpp:175-377.
void gemm_fp32(int M, int N, int K,
               float alpha, const float* A, int lda,
               const float* B, int ldb,
               float beta, float* C, int ldc,
               GemmAlgo algo);

/// bf16 GEMM on fp32 storage: A and B are rounded to bf16 (round to nearest
/// even) inside the kernel, products accumulate in fp32, C is fp32.
/// Reference: src/gemm/gemm.cpp:379-416.
void gemm_bf16(int M, int N, int K,
               float alpha, const float* A, int lda,
               const float* B, int ldb,
               float beta, float* C, int ldc);

/// bf16 GEMM on bf16 storage with fp32 accumulation and fp32 C.
/// Reference: src/gemm/gemm_driver_bf16.cpp:134-218.
void gemm_bf16_bf16bf16f32(int M, int N, int K,
                           float alpha, const bfloat16_t* A, int lda,
                           const bfloat16_t* B, int ldb,
                           float beta, float* C, int ldc);

/// int8 GEMM on fp32 storage with dynamic symmetric per-tensor quantization
/// (scale = max|X| / 127, round to nearest even, clamp to [-128, 127]), exact
/// int32 accumulation, then C = alpha * sA * sB * acc + beta * C.
/// Reference: src/gemm/gemm.cpp:418-455, src/gemm/gemm_pack_int8.cpp:29-71.
void gemm_int8(int M, int N, int K,
               float alpha, const float* A, int lda,
               const float* B, int ldb,
               float beta, float* C, int ldc);

/// Exact int8 x int8 -> int32 GEMM, C overwritten (no alpha/beta).
/// B is stored N x K (K contiguous, row stride ldb), which is the layout the
/// reference code reads (src/gemm/gemm_int8_native.cpp:206, 217, 228, 243)
/// although its header comment says K x N.
/// Reference: src/gemm/gemm_int8_native.cpp:189-248.
void gemm_int8_int8int8int32(int M, int N, int K,
                             const int8_t* A, int lda,
                             const int8_t* B, int ldb,
                             int32_t* C, int ldc);

/// Thread-count control kept for ABI compatibility
/// (src/gemm/gemm_threading.cpp:19-32).  The value is recorded and returned
/// but does not change the device launch.
void gemm_set_num_threads(int n);
int gemm_get_num_threads();

}  // namespace dnnopt
