#ifndef DNNOPT_HIP_H
#define DNNOPT_HIP_H
/*
 * dnnopt_hip.h -- C-ABI boundary of the gfx950 small/irregular-shape GEMM path.
 *
 * These are the entry points a foreign-function binding (ctypes, cgo, JNI,
 * a oneDNN hook) calls.  Every function takes plain pointers and sizes and
 * returns a status code; nothing in a signature is a HIP or PyTorch type.
 *
 * Conventions shared by every GEMM entry point:
 *   - row-major storage, ld* = row stride in elements;
 *   - A, B, C (and col_scale) are DEVICE pointers; the work is enqueued on
 *     `stream` (a hipStream_t passed as void*, NULL = the null stream) and
 *     the call returns without waiting;
 *   - M <= 0, N <= 0 or K <= 0 is a successful no-op that does not touch C
 *     (reference: src/gemm/gemm.cpp:180);
 *   - beta == 0 never reads C;
 *   - a non-zero status means nothing was enqueued and C is untouched;
 *   - results are deterministic: the same call on the same inputs gives the
 *     same bits every time (fixed reduction order, no floating atomics).
 *
 * The synchronous host-pointer API of the reference (dnnopt::gemm_* in
 * dnnopt/gemm/gemm.h, cblas_sgemm in dnnopt/blas/cblas.h) is implemented on
 * top of these functions in the same shared library.
 */

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define DNNOPT_OK                0
#define DNNOPT_ERR_INVALID_ARG   1  /* bad size, stride, flag or NULL pointer */
#define DNNOPT_ERR_NO_DEVICE     2  /* no HIP device visible                  */
#define DNNOPT_ERR_HIP           3  /* a HIP runtime call failed               */
#define DNNOPT_ERR_UNSUPPORTED   4  /* shape/option outside what is built      */
#define DNNOPT_ERR_OUT_OF_MEMORY 5  /* workspace or staging allocation failed  */
#define DNNOPT_ERR_SCRATCH_LIMIT 6  /* needs more scratch than the no-allocation */
                                    /* entry point holds (DNNOPT_NOALLOC_SCRATCH_BYTES) */

/* operand transpose flags for dnnopt_hip_sgemm */
#define DNNOPT_OP_N 0
#define DNNOPT_OP_T 1

/* ---- GEMM entry points (device pointers, stream-ordered) --------------- */

/* fp32: C = alpha * op(A) * op(B) + beta * C.  op(A) is M x K, op(B) is K x N.
 * With transA, A is stored K x M (lda >= M); with transB, B is stored N x K
 * (ldb >= K).  Epilogue as the reference kernels: beta == 0 gives
 * alpha*acc, otherwise fma(alpha, acc, beta*C).
 * Replaces dnnopt::gemm_fp32 (src/gemm/gemm.cpp:168-377) and the transposed
 * cases of cblas_sgemm (src/blas/cblas_sgemm.cpp:67-99), which the
 * reference materializes as temporaries. */
int dnnopt_hip_sgemm(int transA, int transB, int M, int N, int K,
                     float alpha, const float* A, int lda,
                     const float* B, int ldb,
                     float beta, float* C, int ldc, void* stream);

/* fp32 GEMM exactly as dnnopt_hip_sgemm (same plan, same kernels, same
 * bits), for callers that cannot allocate device memory: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  It
 * calls no hipMalloc/hipFree or other allocating routine: split-k partial
 * sums and tickets live in a fixed device array of the library,
 * DNNOPT_NOALLOC_SCRATCH_BYTES per GPU, held from the library's load until
 * the process ends.  A call whose plan needs more scratch than that returns
 * DNNOPT_ERR_SCRATCH_LIMIT before any of its GEMM work is enqueued and
 * leaves C untouched.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (concurrent
 * streams, or host threads) race and must be serialised by the caller.  The
 * first call on each device also enqueues one small kernel that clears the
 * array's ticket counters.
 * No counterpart in the reference (whose calls allocate per call); it exists
 * for the callers that cannot allocate. */
#define DNNOPT_NOALLOC_SCRATCH_BYTES (16u << 20)
int dnnopt_hip_sgemm_noalloc(int transA, int transB, int M, int N, int K,
                             float alpha, const float* A, int lda,
                             const float* B, int ldb,
                             float beta, float* C, int ldc, void* stream);

/* fp32 scalar reference: one output per thread, k ascending, separate
 * multiply and add roundings, then alpha*acc + beta*C -- bit-identical to
 * the reference's naive loop.  Serves GemmAlgo::kNaive
 * (src/gemm/gemm.cpp:88-100, 182-185). */
int dnnopt_hip_sgemm_naive(int M, int N, int K,
                           float alpha, const float* A, int lda,
                           const float* B, int ldb,
                           float beta, float* C, int ldc, void* stream);

/* bf16 storage (raw bf16 bit patterns), fp32 accumulation, fp32 C.
 * Replaces dnnopt::gemm_bf16_bf16bf16f32 (src/gemm/gemm_driver_bf16.cpp:134). */
int dnnopt_hip_gemm_bf16(int M, int N, int K,
                         float alpha, const uint16_t* A, int lda,
                         const uint16_t* B, int ldb,
                         float beta, float* C, int ldc, void* stream);

/* bf16 storage with operand transposes: with transA, A is stored K x M
 * (lda >= M); with transB, B is stored N x K (ldb >= K).  Otherwise as
 * dnnopt_hip_gemm_bf16.  Replaces the oneDNN hook's row-major bf16 helper
 * dnnopt_gemm_bf16_row_major (integration/onednn/0001-dnnopt-integration.patch:
 * 536-560), which copies transposed operands into temporaries: here B is read
 * in place and a K x M A is read in place (M <= 8) or transposed on the
 * device into library workspace. */
int dnnopt_hip_gemm_bf16_ex(int transA, int transB, int M, int N, int K,
                            float alpha, const uint16_t* A, int lda,
                            const uint16_t* B, int ldb,
                            float beta, float* C, int ldc, void* stream);

/* fp32 storage, both operands rounded to bf16 (nearest even) in registers,
 * fp32 accumulation.  Replaces dnnopt::gemm_bf16 (src/gemm/gemm.cpp:379-416). */
int dnnopt_hip_gemm_bf16_f32in(int M, int N, int K,
                               float alpha, const float* A, int lda,
                               const float* B, int ldb,
                               float beta, float* C, int ldc, void* stream);

/* Exact int8 x int8 -> int32, C overwritten.  B is N x K (K contiguous).
 * Replaces dnnopt::gemm_int8_int8int8int32
 * (src/gemm/gemm_int8_native.cpp:189-248). */
int dnnopt_hip_gemm_s8s8s32(int M, int N, int K,
                            const int8_t* A, int lda,
                            const int8_t* B, int ldb,
                            int32_t* C, int ldc, void* stream);

/* Same contraction with a per-column dequantization epilogue:
 * C[i][j] = (float)acc[i][j] * col_scale[j] (one rounding for the int->float
 * conversion, one for the multiply).  The reference has no per-column scale;
 * its caller applies a per-tensor scale the same way
 * (src/conv/conv3d.cpp:511-514). */
int dnnopt_hip_gemm_s8s8f32_colscale(int M, int N, int K,
                                     const int8_t* A, int lda,
                                     const int8_t* B, int ldb,
                                     const float* col_scale,
                                     float* C, int ldc, void* stream);

/* fp32 storage, dynamic symmetric per-tensor int8 quantization (scale s_X =
 * max|X|/127, or 1 for an all-zero operand; round to nearest even; clamp to
 * [-128, 127]) and an exact int32 contraction, routed by M as the reference
 * routes it on a CPU with I8MM (src/gemm/gemm.cpp:418-455):
 *   M <= 8  gemm_smallm_int8 (src/gemm/gemm_smallm_int8.cpp:126-511):
 *           q = rint(x / s_X) (true division), t = alpha*(sA*sB);
 *           M == 1: C = t*acc (beta == 0) or fma(beta, C, t*acc);
 *           M >= 2: C = (beta == 0 ? 0 : beta*C) + t*acc, two roundings;
 *           DNNOPT_ERR_UNSUPPORTED when a row of B spans 2 GiB or more.
 *   M > 8   the packed path (src/gemm/gemm_driver_generic.cpp:49-67,
 *           src/gemm/gemm_pack_int8.cpp:29-71): q = rint(x * (1/s_X)),
 *           C = alpha*sA*sB*acc (beta == 0) or fma(alpha*sA*sB, acc, beta*C). */
int dnnopt_hip_gemm_int8_f32(int M, int N, int K,
                             float alpha, const float* A, int lda,
                             const float* B, int ldb,
                             float beta, float* C, int ldc, void* stream);

/* Y = alpha * X + Y (strided).  Replaces cblas_saxpy
 * (src/blas/cblas_saxpy.cpp:13-51): N <= 0 or alpha == 0 is a no-op;
 * incX = 0 adds alpha*X[0] to every element, incY = 0 applies all N updates
 * to Y[0] in order (the reference's strided loop, :45-49).  Negative
 * increments are DNNOPT_ERR_INVALID_ARG (the reference would index before
 * the start of X or Y). */
int dnnopt_hip_saxpy(int N, float alpha, const float* X, int incX,
                     float* Y, int incY, void* stream);

/* ---- oneDNN hook: column-major GEMMs ------------------------------------
 * C (M x N, column-major: C(i,j) at C[j*ldc + i]) = alpha * op(A) * op(B)
 * + beta * C, then C(i,j) += bias[i] when bias != NULL (fp32 only); op(A) is
 * M x K, op(B) is K x N, column-major.  transa/transb are the BLAS letters:
 * 'T'/'t' transposed, 'P'/'p' (packed, fp32 only) -> DNNOPT_ERR_UNSUPPORTED,
 * anything else not transposed.  M == 0 or N == 0: nothing.  K == 0: C = 0
 * (beta == 0, C not read) or C *= beta (beta != 1), then the bias.  ldc < M is
 * accepted and gives the reference's result for overlapping columns.  Sizes
 * are 64-bit as oneDNN's dim_t; values above INT_MAX ->
 * DNNOPT_ERR_UNSUPPORTED.
 * Replace the hook functions dnnopt_sgemm and dnnopt_gemm_bf16bf16f32 that
 * the reference adds to oneDNN
 * (integration/onednn/0001-dnnopt-integration.patch:279-370, 573-630). */

/* Device pointers, enqueued on `stream` (as the GEMM entry points above). */
int dnnopt_hip_ext_sgemm(char transa, char transb, int64_t M, int64_t N,
                         int64_t K, float alpha, const float* A, int64_t lda,
                         const float* B, int64_t ldb, float beta, float* C,
                         int64_t ldc, const float* bias, void* stream);
int dnnopt_hip_ext_gemm_bf16bf16f32(char transa, char transb, int64_t M,
                                    int64_t N, int64_t K, float alpha,
                                    const uint16_t* A, int64_t lda,
                                    const uint16_t* B, int64_t ldb,
                                    float beta, float* C, int64_t ldc,
                                    void* stream);

/* The hook's own argument list (every scalar by pointer, as oneDNN's
 * extended_sgemm passes them), host or device memory, synchronous: returns
 * when C holds the result.  A oneDNN build maps DNNOPT_OK to
 * dnnl_success, DNNOPT_ERR_UNSUPPORTED to dnnl_unimplemented (its own
 * fallback then runs) and other codes to dnnl_runtime_error. */
int dnnopt_onednn_sgemm(const char* transa, const char* transb,
                        const int64_t* M, const int64_t* N, const int64_t* K,
                        const float* alpha, const float* A, const int64_t* lda,
                        const float* B, const int64_t* ldb, const float* beta,
                        float* C, const int64_t* ldc, const float* bias);
int dnnopt_onednn_gemm_bf16bf16f32(const char* transa, const char* transb,
                                   const int64_t* M, const int64_t* N,
                                   const int64_t* K, const float* alpha,
                                   const uint16_t* A, const int64_t* lda,
                                   const uint16_t* B, const int64_t* ldb,
                                   const float* beta, float* C,
                                   const int64_t* ldc);

/* ---- planning (host only; needs no device) ----------------------------- */

/* Kernel families chosen by the dispatcher. */
#define DNNOPT_K_NONE        0
#define DNNOPT_K_SKINNY_F32  1  /* M <= 8, fp32 B streamed once             */
#define DNNOPT_K_SKINNY_BF16 2  /* M <= 8, bf16 B streamed once             */
#define DNNOPT_K_SKINNY_F2B  3  /* M <= 8, fp32 B rounded to bf16 in regs   */
#define DNNOPT_K_MFMA_S8     4  /* int8 MFMA tiles, B as N x K              */
#define DNNOPT_K_TILE_F32    5  /* fp32 MFMA tiles (tall-skinny, split-K;   */
                                /* name dnnopt_kouter_f32: k-major TransA) */
#define DNNOPT_K_TILE_BF16   6  /* bf16 MFMA tiles                          */
#define DNNOPT_K_NAIVE_F32   7  /* scalar reference kernel                  */
#define DNNOPT_K_ROWDOT_F32  8  /* M <= 8, fp32 B stored N x K, rows once   */
#define DNNOPT_K_ROWDOT_BF16 9  /* M <= 8, bf16 B stored N x K, rows once   */
#define DNNOPT_K_TALL_F32   10  /* large M, N <= 64, fp32 B resident in LDS  */
#define DNNOPT_K_ROWDOT_S8  11  /* M <= 8, int8 B stored N x K, rows once   */
#define DNNOPT_K_SKINNY_Q8  12  /* M <= 8, fp32-API int8: fp32 B quantized  */
                                /* as it is streamed (no int8 copy of B)   */
#define DNNOPT_K_WIDE       13  /* any layout, 64-bit addressing: operands  */
                                /* whose spans exceed the other kernels'   */
                                /* 32-bit offsets (rows of gigabytes)      */

typedef struct dnnopt_plan {
    int kernel;             /* DNNOPT_K_* */
    int rows;               /* M rows handled per workgroup tile          */
    int cols;               /* N columns handled per workgroup tile       */
    int splits;             /* split-K factor (1 = none)                  */
    int grid_x, grid_y, grid_z;
    int block;              /* threads per workgroup                      */
    size_t workspace_bytes; /* device scratch needed (partials+tickets)   */
    char name[64];          /* kernel symbol prefix, as rocprof lists it  */
} dnnopt_plan;

int dnnopt_hip_plan_sgemm(int transA, int transB, int M, int N, int K,
                          dnnopt_plan* out);
/* As dnnopt_hip_plan_sgemm for the given row strides (the plan of
 * dnnopt_hip_sgemm with these lda, ldb, ldc): kernels that address an
 * operand with 32-bit offsets are only chosen when its strides allow. */
int dnnopt_hip_plan_sgemm_ex(int transA, int transB, int M, int N, int K,
                             int lda, int ldb, int ldc, dnnopt_plan* out);
int dnnopt_hip_plan_gemm_bf16(int fp32_inputs, int M, int N, int K,
                              dnnopt_plan* out);
int dnnopt_hip_plan_gemm_bf16_ex(int transA, int transB, int M, int N, int K,
                                 dnnopt_plan* out);
int dnnopt_hip_plan_gemm_s8(int with_scale, int M, int N, int K,
                            dnnopt_plan* out);
/* The GEMM launch of dnnopt_hip_gemm_int8_f32 with unpadded strides: after
 * its maxima pass, for M <= 8 the skinny kernel that quantizes B as it
 * streams it (DNNOPT_K_SKINNY_Q8), else (after A's quantization pass) the
 * int8 tiles that quantize the fp32 B while staging it. */
int dnnopt_hip_plan_gemm_int8_f32(int M, int N, int K, dnnopt_plan* out);

/* ---- synthetic inputs on the device ------------------------------------
 * Counter-based SplitMix64: element i of tensor `tensor_id` under `seed`
 * is a pure function of (seed, tensor_id, i), so any slice can be
 * regenerated on the host.
 *   dtype: 0 = fp32, 1 = bf16 (fp32 value rounded to nearest even), 2 = int8
 *   dist : 0 = uniform [p0, p1), 1 = normal(mean p0, sigma p1),
 *          2 = uniform integers in [p0, p1] (int8 only)                   */
int dnnopt_hip_fill(void* dst, size_t n, int dtype, int dist,
                    uint64_t seed, uint32_t tensor_id,
                    double p0, double p1, void* stream);

/* ---- status and device queries ---------------------------------------- */
const char* dnnopt_hip_status_string(int status);
int dnnopt_hip_last_status(void);     /* last failure of the C++/cblas API on
                                         this thread, DNNOPT_OK if none      */
int dnnopt_hip_device_count(void);    /* 0 when no device is visible        */

/* ---- tunable parameters of the shape dispatcher -------------------------
 * No counterpart in the reference (its tile choice is an autotuned cache,
 * src/gemm/gemm_autotune.cpp, outside this path).  Every routing or
 * launch-shape choice the dispatcher can be steered in has a key; the
 * library starts from built-in defaults and changes one only when a caller
 * sets it here (process-wide, effective from the next planning call).  The
 * default build never reads the environment; a build with -DDNNOPT_TUNING=1
 * seeds the table once from DNNOPT_<NAME> variables (whole integers from 1,
 * from 0 for SPLIT_REDUCE and S8_CFG; others are ignored).  Switches take 1 / 0;
 * forcing keys take 0 (-1 for DNNOPT_TUNE_S8_CFG) to let the planner decide.
 * *previous (if not NULL) receives the old value.                        */
#define DNNOPT_TUNE_Q8B              0  /* 1: int8 tiles quantize the fp32 B while staging it */
#define DNNOPT_TUNE_KOUTER           1  /* 1: k-outer kernel for A stored K x M, large K */
#define DNNOPT_TUNE_KOUTER_WGS_PER_CU 2
#define DNNOPT_TUNE_WAVES_PER_CU     3
#define DNNOPT_TUNE_SKINNY_NW        4  /* 4, 8 or 16 waves; 0 = by problem size */
#define DNNOPT_TUNE_SKINNY_WGS_PER_CU 5
#define DNNOPT_TUNE_MAX_SPLITS       6
#define DNNOPT_TUNE_SPLIT_REDUCE     7  /* split-k sums: 1 (default) the planners' choice (the
                                           last-arriving workgroup for small skinny combines and
                                           fp32 tiles of at most 8 splits), 2 the reduce kernel,
                                           0 the last-arriving workgroup */
#define DNNOPT_TUNE_SKINNY_WGS       8
#define DNNOPT_TUNE_TILE_SPLITS      9  /* force the k-splits of a tile launch */
#define DNNOPT_TUNE_TILE_CFG        10  /* force a tile configuration (bf16 LDS-staged: 5 and up;
                                           fp32 register tiles: 1-4, 35, 36; fp32 LDS-DMA tiles,
                                           A stored M x K: 41-47, and 48-50 with B stored N x K) */
#define DNNOPT_TUNE_TILE_TICKET     11
#define DNNOPT_TUNE_S8_CFG          12
#define DNNOPT_TUNE_S8_ROWDOT       13
#define DNNOPT_TUNE_S8_SPLITS       14
#define DNNOPT_TUNE_ROWDOT_KW       15
#define DNNOPT_TUNE_TALL_RT         16
#define DNNOPT_TUNE_TALL_WGS_PER_CU 17
#define DNNOPT_TUNE_TALL            18
#define DNNOPT_TUNE_WIDE            19  /* 1: every GEMM on the last-resort kernel (tests) */
#define DNNOPT_TUNE_COUNT           20
int dnnopt_hip_set_tunable(int key, int value, int* previous);
int dnnopt_hip_get_tunable(int key, int* value);

#define DNNOPT_HIP_ABI_VERSION 4
int dnnopt_hip_abi_version(void);     /* DNNOPT_HIP_ABI_VERSION; bumped on any signature change */

#ifdef __cplusplus
}
#endif

#endif /* DNNOPT_HIP_H */
