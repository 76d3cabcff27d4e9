// blas.cpp -- CBLAS / Fortran BLAS entry points (include/dnnopt/blas/cblas.h).
//
// Order and transpose handling follows the reference (src/blas/cblas_sgemm.cpp:
// 105-143): a column-major product is the row-major product of the swapped
// operands, C^T = op(B)^T op(A)^T, so ColMajor(TransA, TransB, M, N, A, B)
// becomes RowMajor(TransB, TransA, N, M, B, A).  Unlike the reference, a
// transposed operand is never copied: the kernels read it in place.
#include <hip/hip_runtime.h>

#include "api_internal.h"
#include "dnnopt/blas/cblas.h"
#include "dnnopt/gemm/gemm.h"
#include "dnnopt_hip.h"

using namespace dnnopt_api;

namespace {

int trans_flag(enum CBLAS_TRANSPOSE t) { return t == CblasNoTrans ? 0 : 1; }

bool valid_trans(enum CBLAS_TRANSPOSE t) { return t == CblasNoTrans || t == CblasTrans || t == CblasConjTrans; }

enum CBLAS_TRANSPOSE fortran_trans(const char* c) {
    if (*c == 'T' || *c == 't') return CblasTrans;
    if (*c == 'C' || *c == 'c') return CblasConjTrans;
    return CblasNoTrans;
}

}  // namespace

extern "C" {

void cblas_sgemm(enum CBLAS_ORDER Order, enum CBLAS_TRANSPOSE TransA, enum CBLAS_TRANSPOSE TransB, int M, int N,
                 int K, float alpha, const float* A, int lda, const float* B, int ldb, float beta, float* C,
                 int ldc) {
    if (M <= 0 || N <= 0 || K <= 0) return;
    if (alpha == 0.0f && beta == 1.0f) return;
    if ((Order != CblasRowMajor && Order != CblasColMajor) || !valid_trans(TransA) || !valid_trans(TransB)) {
        record(DNNOPT_ERR_INVALID_ARG, "cblas_sgemm");
        return;
    }
    int st;
    if (Order == CblasRowMajor)
        st = sgemm_any(trans_flag(TransA), trans_flag(TransB), M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, false);
    else
        st = sgemm_any(trans_flag(TransB), trans_flag(TransA), N, M, K, alpha, B, ldb, A, lda, beta, C, ldc, false);
    record(st, "cblas_sgemm");
}

void cblas_saxpy(int N, float alpha, const float* X, int incX, float* Y, int incY) {
    if (N <= 0 || alpha == 0.0f) return;
    int st = DNNOPT_OK;
    if (!X || !Y || incX < 0 || incY < 0) {
        st = DNNOPT_ERR_INVALID_ARG;
    } else if (dnnopt_hip_device_count() == 0) {
        st = DNNOPT_ERR_NO_DEVICE;
    } else {
        void* s = api_stream(&st);
        DrainGuard drain(s);
        Operand x = stage_in(X, ((size_t)(N - 1) * incX + 1) * 4, 0, true, s, &st);
        Operand y = stage_in(Y, ((size_t)(N - 1) * incY + 1) * 4, 2, true, s, &st);
        if (st == DNNOPT_OK) st = dnnopt_hip_saxpy(N, alpha, (const float*)x.dev, incX, (float*)y.dev, incY, s);
        if (st == DNNOPT_OK) st = sync_stream(s);
        if (st == DNNOPT_OK) st = stage_out(y, s);
        if (st == DNNOPT_OK) drain.release();
    }
    record(st, "cblas_saxpy");
}

void sgemm_(const char* transa, const char* transb, const int* m, const int* n, const int* k, const float* alpha,
            const float* a, const int* lda, const float* b, const int* ldb, const float* beta, float* c,
            const int* ldc) {
    cblas_sgemm(CblasColMajor, fortran_trans(transa), fortran_trans(transb), *m, *n, *k, *alpha, a, *lda, b, *ldb,
                *beta, c, *ldc);
}

void SGEMM(const char* transa, const char* transb, const int* m, const int* n, const int* k, const float* alpha,
           const float* a, const int* lda, const float* b, const int* ldb, const float* beta, float* c,
           const int* ldc) {
    sgemm_(transa, transb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc);
}

void openblas_set_num_threads(int num_threads) { dnnopt::gemm_set_num_threads(num_threads); }
int openblas_get_num_threads(void) { return dnnopt::gemm_get_num_threads(); }
void blas_set_num_threads(int num_threads) { dnnopt::gemm_set_num_threads(num_threads); }
void omp_set_num_threads_blas(int num_threads) { dnnopt::gemm_set_num_threads(num_threads); }

}  // extern "C"
