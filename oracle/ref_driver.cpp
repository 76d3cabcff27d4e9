// ref_driver.cpp -- C entry points into the reference's own sources, for
// pinning the oracle.  TEST INFRASTRUCTURE ONLY: built into oracle/_ref from
// /root/reference (which exists only in the development container) and loaded
// by tests/test_oracle.py.  It calls the reference functions unchanged:
//   dnnopt::bfloat16_t            include/dnnopt/gemm/gemm_types.h:18-24
//   dnnopt::gemm_fp32(..., kNaive) src/gemm/gemm.cpp:88-100, 175-185
//   dnnopt::gemm_int8_int8int8int32 src/gemm/gemm_int8_native.cpp:189-248
//   cblas_saxpy                   src/blas/cblas_saxpy.cpp:13-51
// Only these paths are compiled for x86 without the reference's missing
// AArch64 pieces; other paths of gemm.cpp are left unresolved and never
// called (the library is linked and loaded with lazy binding).
#include <stdint.h>

#include "dnnopt/blas/cblas.h"
#include "dnnopt/gemm/gemm.h"
#include "dnnopt/gemm/gemm_types.h"

extern "C" {

uint16_t ref_bf16_round(float f) { return dnnopt::bfloat16_t(f).raw_bits; }

float ref_bf16_widen(uint16_t b) { return (float)dnnopt::bfloat16_t(b, true); }

void ref_gemm_naive_f32(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc) {
    dnnopt::gemm_fp32(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, dnnopt::GemmAlgo::kNaive);
}

void ref_gemm_s8s8s32(int M, int N, int K, const int8_t* A, int lda, const int8_t* B, int ldb, int32_t* C,
                      int ldc) {
    dnnopt::gemm_int8_int8int8int32(M, N, K, A, lda, B, ldb, C, ldc);
}

void ref_saxpy(int N, float alpha, const float* X, int incX, float* Y, int incY) {
    cblas_saxpy(N, alpha, X, incX, Y, incY);
}

}  // extern "C"
