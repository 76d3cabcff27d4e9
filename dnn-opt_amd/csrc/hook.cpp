// hook.cpp -- the oneDNN integration entry points: column-major GEMMs with
// the semantics of the reference's hook into oneDNN's extended_sgemm and
// gemm_bf16bf16f32 (integration/onednn/0001-dnnopt-integration.patch:279-370
// and 573-630).
//
// What the hook does, and how it is done here:
//   * 'P'/'p' (packed) operands are not handled (fp32 only): status
//     DNNOPT_ERR_UNSUPPORTED, which the oneDNN side maps to
//     status::unimplemented so that its own fallback runs (patch:285-287).
//     Any other letter than 'T'/'t' means "not transposed" (patch:309-310).
//   * M == 0 or N == 0: nothing (patch:289).
//   * K == 0: C = 0 if beta == 0 (C not read), C *= beta if beta != 1, then
//     the bias (fp32 only) -- alpha is not used (patch:290-305).
//   * otherwise the column-major product is the row-major product of the
//     swapped operands, C^T = op(B)^T op(A)^T with C^T an N x M row-major
//     matrix of row stride ldc (patch:308-329).  The reference transposes
//     'T' operands into temporaries (patch:243-268, 536-560); the kernels
//     here read fp32 operands and a bf16 B in place (a bf16 A stored K x M is
//     transposed on the device when M > 8).
//   * ldc < M: the product goes to a temporary of row stride M, which is then
//     written back row by row (patch:330-352); see k_colmajor.hip for the
//     result this gives where columns overlap.
//   * bias (fp32 only): C[j * ldc + i] += bias[i] after the product
//     (patch:355-362), rounded as a separate addition.
//
// The dnnopt_hip_ext_* functions take device pointers and enqueue on a
// stream; dnnopt_onednn_* take the hook's own argument list (pointers to the
// scalars, host or device memory) and return when C is final.
#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdint.h>

#include "api_internal.h"
#include "dnnopt_hip.h"
#include "host.h"

using namespace dnnopt_hip;

namespace {

bool is_t(char c) { return c == 'T' || c == 't'; }
bool is_p(char c) { return c == 'P' || c == 'p'; }

int launch_status(hipError_t e) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return to_status(e);
    }
    return DNNOPT_OK;
}

int ext_common(bool bf16, char transa, char transb, int64_t M, int64_t N, int64_t K, float alpha, const void* A,
               int64_t lda, const void* B, int64_t ldb, float beta, float* C, int64_t ldc, const float* bias,
               void* stream) {
    if (!bf16 && (is_p(transa) || is_p(transb))) return DNNOPT_ERR_UNSUPPORTED;
    if (M == 0 || N == 0) return DNNOPT_OK;
    if (M < 0 || N < 0 || K < 0 || ldc < 1 || !C) return DNNOPT_ERR_INVALID_ARG;
    if (M > INT_MAX || N > INT_MAX || K > INT_MAX || lda > INT_MAX || ldb > INT_MAX || ldc > INT_MAX)
        return DNNOPT_ERR_UNSUPPORTED;
    const int tA = is_t(transa) ? 1 : 0, tB = is_t(transb) ? 1 : 0;
    // Leading dimensions of column-major op(A) (M x K) and op(B) (K x N).
    if (K > 0 && (!A || !B || lda < (tA ? K : M) || ldb < (tB ? N : K))) return DNNOPT_ERR_INVALID_ARG;
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    StreamLock lock(s);
    const int m = (int)M, n = (int)N, k = (int)K;
    if (k == 0) {
        const int op = beta == 0.0f ? kCmZero : (beta != 1.0f ? kCmScale : kCmNone);
        if (op == kCmNone && !bias) return DNNOPT_OK;
        return launch_status(launch_cm_fixup(C, m, n, ldc, op, beta, bias, s));
    }

    // Row-major view: C^T (N x M, row stride ldc) = op(B)^T (N x K) op(A)^T (K x M).
    float* Cw = C;
    int ldw = (int)ldc;
    if (ldc < M) {
        void* tmp = nullptr;
        unsigned* unused = nullptr;
        int st = get_workspace(s, (size_t)M * (size_t)N * sizeof(float), &tmp, &unused, kSlotHookC);
        if (st != DNNOPT_OK) return st;
        Cw = static_cast<float*>(tmp);
        ldw = m;
        if (beta != 0.0f) {
            st = launch_status(launch_cm_gather(C, ldc, Cw, m, n, s));
            if (st != DNNOPT_OK) return st;
        }
    }
    // The bias is one addition after each output's epilogue: fused into the
    // GEMM when C is written in place (bias[i] is column i of C^T); after the
    // write-back when columns overlap (the bias loop then runs per covering
    // column, as the reference's does).
    const float* fused_bias = Cw == C ? bias : nullptr;
    int st = bf16 ? dnnopt_hip_gemm_bf16_ex(tB, tA, n, m, k, alpha, static_cast<const uint16_t*>(B), (int)ldb,
                                            static_cast<const uint16_t*>(A), (int)lda, beta, Cw, ldw, stream)
                  : sgemm_bias(tB, tA, n, m, k, alpha, static_cast<const float*>(B), (int)ldb,
                               static_cast<const float*>(A), (int)lda, beta, Cw, ldw, fused_bias, s);
    if (st != DNNOPT_OK) return st;
    if (Cw != C) {
        st = launch_status(launch_cm_scatter(Cw, m, n, ldc, C, s));
        if (st != DNNOPT_OK) return st;
    }
    if (bias && !fused_bias) return launch_status(launch_cm_fixup(C, m, n, ldc, kCmNone, 0.0f, bias, s));
    return DNNOPT_OK;
}

// Elements spanned by a column-major rows x cols block with column stride ld.
size_t cm_extent(int64_t rows, int64_t cols, int64_t ld) {
    if (rows <= 0 || cols <= 0) return 0;
    return (size_t)(cols - 1) * (size_t)ld + (size_t)rows;
}

int onednn_common(bool bf16, const char* transa, const char* transb, const int64_t* M, const int64_t* N,
                  const int64_t* K, const float* alpha, const void* A, const int64_t* lda, const void* B,
                  const int64_t* ldb, const float* beta, float* C, const int64_t* ldc, const float* bias) {
    using namespace dnnopt_api;
    if (!transa || !transb || !M || !N || !K || !alpha || !lda || !ldb || !beta || !ldc)
        return DNNOPT_ERR_INVALID_ARG;
    if (!bf16 && (is_p(*transa) || is_p(*transb))) return DNNOPT_ERR_UNSUPPORTED;
    if (*M == 0 || *N == 0) return DNNOPT_OK;
    if (*M < 0 || *N < 0 || *K < 0 || *ldc < 1 || !C) return DNNOPT_ERR_INVALID_ARG;
    if (*M > INT_MAX || *N > INT_MAX || *K > INT_MAX || *lda > INT_MAX || *ldb > INT_MAX || *ldc > INT_MAX)
        return DNNOPT_ERR_UNSUPPORTED;
    const bool tA = is_t(*transa), tB = is_t(*transb);
    // Checked before any staging: the extents below assume valid strides.
    if (*K > 0 && (!A || !B || *lda < (tA ? *K : *M) || *ldb < (tB ? *N : *K))) return DNNOPT_ERR_INVALID_ARG;
    if (*K == 0 && *beta == 1.0f && !bias) return DNNOPT_OK;
    if (dnnopt_hip_device_count() == 0) return DNNOPT_ERR_NO_DEVICE;
    const size_t es = bf16 ? 2 : 4;
    int st = DNNOPT_OK;
    void* s = api_stream(&st);
    DrainGuard drain(s);
    Operand a, b;
    if (*K > 0) {
        a = stage_in(A, (tA ? cm_extent(*K, *M, *lda) : cm_extent(*M, *K, *lda)) * es, 0, true, s, &st);
        b = stage_in(B, (tB ? cm_extent(*N, *K, *ldb) : cm_extent(*K, *N, *ldb)) * es, 1, true, s, &st);
    }
    // C is uploaded unless every element of its extent is overwritten
    // without being read (beta == 0 and no gaps between columns).
    Operand c = stage_in(C, cm_extent(*M, *N, *ldc) * 4, 2, *beta != 0.0f || *ldc > *M, s, &st);
    Operand bs = bias ? stage_in(bias, (size_t)*M * 4, 3, true, s, &st) : Operand{};
    if (st != DNNOPT_OK) return st;
    st = ext_common(bf16, *transa, *transb, *M, *N, *K, *alpha, a.dev, *lda, b.dev, *ldb, *beta,
                    static_cast<float*>(c.dev), *ldc, static_cast<const float*>(bs.dev), s);
    if (st != DNNOPT_OK) return st;
    st = sync_stream(s);
    if (st != DNNOPT_OK) return st;
    st = stage_out(c, s);
    if (st == DNNOPT_OK) drain.release();
    return st;
}

}  // namespace

extern "C" {

int dnnopt_hip_ext_sgemm(char transa, char transb, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
                         int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc,
                         const float* bias, void* stream) {
    return ext_common(false, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias, stream);
}

int dnnopt_hip_ext_gemm_bf16bf16f32(char transa, char transb, int64_t M, int64_t N, int64_t K, float alpha,
                                    const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, float beta,
                                    float* C, int64_t ldc, void* stream) {
    return ext_common(true, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, nullptr, stream);
}

int dnnopt_onednn_sgemm(const char* transa, const char* transb, const int64_t* M, const int64_t* N,
                        const int64_t* K, const float* alpha, const float* A, const int64_t* lda, const float* B,
                        const int64_t* ldb, const float* beta, float* C, const int64_t* ldc, const float* bias) {
    const int st = onednn_common(false, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias);
    dnnopt_api::record(st == DNNOPT_ERR_UNSUPPORTED ? DNNOPT_OK : st, "dnnopt_onednn_sgemm");
    return st;
}

int dnnopt_onednn_gemm_bf16bf16f32(const char* transa, const char* transb, const int64_t* M, const int64_t* N,
                                   const int64_t* K, const float* alpha, const uint16_t* A, const int64_t* lda,
                                   const uint16_t* B, const int64_t* ldb, const float* beta, float* C,
                                   const int64_t* ldc) {
    const int st = onednn_common(true, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, nullptr);
    dnnopt_api::record(st, "dnnopt_onednn_gemm_bf16bf16f32");
    return st;
}

}  // extern "C"
