#pragma once
/// @file cblas.h
/// CBLAS / Fortran-BLAS single-precision entry points backed by the gfx950
/// GEMM path.  Names, enumerator values and signatures follow the reference
/// (include/dnnopt/blas/cblas.h:14-50, src/blas/blas_fortran.cpp:12-42) so the
/// library can be linked or LD_PRELOADed in place of libdnnopt_blas.so.
///
/// Differences from the reference, by design:
///   * transposed operands are read in place by the kernels; no transposed
///     temporary is materialized (reference: cblas_sgemm.cpp:80-98);
///   * host or device pointers are accepted (see dnnopt/gemm/gemm.h).

#ifdef __cplusplus
extern "C" {
#endif

enum CBLAS_ORDER {
    CblasRowMajor = 101,
    CblasColMajor = 102
};

enum CBLAS_TRANSPOSE {
    CblasNoTrans   = 111,
    CblasTrans     = 112,
    CblasConjTrans = 113
};

/// C = alpha * op(A) * op(B) + beta * C.  Returns at once when M, N or K is
/// not positive, or when alpha == 0 and beta == 1 (cblas_sgemm.cpp:114-115).
/// ConjTrans is Trans for real data.
void cblas_sgemm(enum CBLAS_ORDER Order,
                 enum CBLAS_TRANSPOSE TransA,
                 enum CBLAS_TRANSPOSE TransB,
                 int M, int N, int K,
                 float alpha,
                 const float *A, int lda,
                 const float *B, int ldb,
                 float beta,
                 float *C, int ldc);

/// Y = alpha * X + Y.  Returns at once when N <= 0 or alpha == 0
/// (cblas_saxpy.cpp:15).  Increments of 0 follow the reference's strided
/// loop (X[0] broadcast; every update on Y[0], in order); negative ones are
/// rejected (dnnopt_hip_last_status() reports DNNOPT_ERR_INVALID_ARG).
void cblas_saxpy(int N, float alpha, const float *X, int incX,
                 float *Y, int incY);

/// Fortran SGEMM (column-major, arguments by pointer).
/// Reference: src/blas/blas_fortran.cpp:12-42.
void sgemm_(const char *transa, const char *transb,
            const int *m, const int *n, const int *k,
            const float *alpha,
            const float *a, const int *lda,
            const float *b, const int *ldb,
            const float *beta,
            float *c, const int *ldc);
void SGEMM(const char *transa, const char *transb,
           const int *m, const int *n, const int *k,
           const float *alpha,
           const float *a, const int *lda,
           const float *b, const int *ldb,
           const float *beta,
           float *c, const int *ldc);

/// Thread control under the names other BLAS libraries export
/// (src/blas/blas_utils.cpp:10-24).  Recorded, no effect on the device.
void openblas_set_num_threads(int num_threads);
int  openblas_get_num_threads(void);
void blas_set_num_threads(int num_threads);
void omp_set_num_threads_blas(int num_threads);

#ifdef __cplusplus
}
#endif
