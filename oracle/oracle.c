/*
 * oracle.c -- CPU restatement of DNN-Opt's small/irregular-shape GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the gfx950 library
 * and the CPU baseline that bench.py reports beside it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the
 * library never links, calls or falls back to it.
 *
 * Each function restates one reference routine on the host, in the same
 * operation order where the reference's order is fixed by its code (the fp32
 * kernels use fused multiply-adds in k order), so that its outputs are the
 * reference's outputs for the same inputs.  Compile with -ffp-contract=off:
 * every fused operation below is an explicit fmaf().
 *
 * How each function is pinned (tests/test_oracle.py):
 *   orc_gemm_naive_f32    bit-exact vs the reference's own gemm.cpp built in
 *                         oracle/_ref (GemmAlgo::kNaive); fp64 closed form.
 *   orc_gemm_s8s8s32      bit-exact vs the reference's gemm_int8_native.cpp
 *                         built in oracle/_ref; int64 numpy brute force.
 *   orc_bf16_rne          bit-exact vs the reference's bfloat16_t (header
 *                         built in oracle/_ref); closed-form tie cases.
 *   orc_saxpy             bit-exact vs the reference's cblas_saxpy.cpp built
 *                         in oracle/_ref for the scalar (x86) build.
 *   orc_gemm_int8_dynq    closed forms with scales 1 and 2 whose quantized
 *                         values include exact ties (0.5, 1.5, 2.5, -0.5,
 *                         -2.5) and fractions (63.7): only round-to-nearest-
 *                         even passes (copies built with truncf or roundf
 *                         are compiled and rejected by the tests).
 *   orc_gemm_int8_smallm  (and orc_gemm_int8, its M <= 8 / M > 8 routing)
 *                         closed forms: max|X| = 128, x = 88.18897247 has
 *                         x / s = 87.5 exactly (quantized 88) but
 *                         x * (1 / s) = 87.49999 (87); the epilogues' roundings
 *                         (M = 1: fma(beta, C, t acc); M >= 2: beta C and
 *                         t acc rounded, then their rounded sum) by exact
 *                         integer cases with 2^24-scale C; ties with scales
 *                         1 and 2; copies built with the reciprocal or with
 *                         one fused epilogue are compiled and rejected.
 *   orc_gemv_1xn_f32, orc_smallm_wide_f32, orc_adaptive_f32, orc_gemm_bf16,
 *   orc_cblas_sgemm, orc_onednn_sgemm,
 *   orc_onednn_gemm_bf16bf16f32:
 *                         the reference's NEON kernels cannot run here (no
 *                         AArch64 toolchain or emulator); pinned by exact
 *                         small-integer inputs (every rounding exact, so the
 *                         result must equal the integer product), by the
 *                         fp64 error bound gamma_K * sum|a||b|, by special
 *                         cases that reduce to another pinned function, and
 *                         by planted-mistake checks.
 *   generator             SplitMix64 published test vector.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------
 * Synthetic inputs (same definition as the library's device generator).
 * ---------------------------------------------------------------------- */
static const uint64_t kGamma = 0x9E3779B97F4A7C15ull;

uint64_t orc_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* SplitMix64 stream: state += gamma; output mix64(state). */
void orc_splitmix64(uint64_t state, uint64_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        state += kGamma;
        out[i] = orc_mix64(state);
    }
}

uint64_t orc_tensor_key(uint64_t seed, uint32_t tensor_id) {
    return orc_mix64(seed ^ (0xD1B54A32D192ED03ull * ((uint64_t)tensor_id + 1)));
}

static uint64_t draw(uint64_t key, uint64_t i) { return orc_mix64(key + (i + 1) * kGamma); }

void orc_fill_uniform_f32(float* out, size_t n, uint64_t seed, uint32_t tid, double lo, double hi) {
    const uint64_t key = orc_tensor_key(seed, tid);
    for (size_t i = 0; i < n; ++i) {
        const double u = (double)(draw(key, i) >> 40) * (1.0 / 16777216.0);
        const double scaled = (hi - lo) * u;
        out[i] = (float)(lo + scaled);
    }
}

void orc_fill_normal_f32(float* out, size_t n, uint64_t seed, uint32_t tid, double mu, double sigma) {
    const uint64_t key = orc_tensor_key(seed, tid);
    for (size_t i = 0; i < n; ++i) {
        const double u1 = (double)((draw(key, 2 * i) >> 40) + 1) * (1.0 / 16777216.0);
        const double u2 = (double)(draw(key, 2 * i + 1) >> 40) * (1.0 / 16777216.0);
        const double rad = sqrt(-2.0 * log(u1));
        const double ang = 6.283185307179586476925286766559 * u2;
        const double z = rad * cos(ang);
        const double scaled = sigma * z;
        out[i] = (float)(mu + scaled);
    }
}

void orc_fill_int8(int8_t* out, size_t n, uint64_t seed, uint32_t tid, int lo, int hi) {
    const uint64_t key = orc_tensor_key(seed, tid);
    const uint64_t range = (uint64_t)(hi - lo + 1);
    for (size_t i = 0; i < n; ++i) out[i] = (int8_t)(lo + (int)(((draw(key, i) >> 32) * range) >> 32));
}

/* ------------------------------------------------------------------------
 * bfloat16 rounding: include/dnnopt/gemm/gemm_types.h:18-24 (reference).
 * Round to nearest, ties to even, by adding 0x7FFF + lsb; no NaN case.
 * ---------------------------------------------------------------------- */
uint16_t orc_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float orc_bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_round_bf16(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_bf16_rne(in[i]);
}

/* ------------------------------------------------------------------------
 * Scalar fallback: src/gemm/gemm.cpp:88-100 (gemm_naive_fp32), as built for
 * a target without FMA contraction: product and sum rounded separately,
 * C always read.
 * ---------------------------------------------------------------------- */
void orc_gemm_naive_f32(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc) {
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float p = A[(size_t)i * lda + k] * B[(size_t)k * ldb + j];
                acc = acc + p;
            }
            const float t0 = alpha * acc;
            const float t1 = beta * C[(size_t)i * ldc + j];
            C[(size_t)i * ldc + j] = t0 + t1;
        }
}

/* Reference kernel epilogue, NEON store paths:
 * beta == 0: alpha*acc;  else fma(alpha, acc, beta*C)
 * (gemm_tiny_fp32.cpp:200-207, gemm_smallm_wide_fp32.cpp:47-59). */
static float epi_fused(float acc, float alpha, float beta, float c) {
    if (beta == 0.0f) return alpha * acc;
    return fmaf(alpha, acc, beta * c);
}

/* Partial-tile epilogue: round alpha*acc first, then fma(beta, C, .)
 * (gemm_smallm_wide_fp32.cpp:63-76 store_tail; gemm_adaptive_tile_fp32.cpp
 * gemm_tile_tail; gemm_ukernel_fp32_npo2.cpp:181-191; gemm_kernel_asm_fp32.cpp
 * 6x16 epilogue fmul then fmla). */
static float epi_tail(float acc, float alpha, float beta, float c) {
    const float t = alpha * acc;
    if (beta == 0.0f) return t;
    return fmaf(beta, c, t);
}

/* Per-column fused dot product in ascending k (NEON FMLA lanes). */
static float dot_fma(const float* a, int a_stride, const float* b, size_t b_stride, int k0, int k1) {
    float acc = 0.0f;
    for (int k = k0; k < k1; ++k) acc = fmaf(a[(size_t)k * a_stride], b[(size_t)k * b_stride], acc);
    return acc;
}

/* ------------------------------------------------------------------------
 * M = 1 GEMV: src/gemm/gemm_tiny_fp32.cpp:167-218 (gemm_1xn_fp32).
 * 64-column panels; full 4-column quads accumulate with FMLA in k order and
 * store with epi_fused; the N % 4 columns of a panel use the scalar loop
 * (contracted to fma by the compiler) and alpha*sum + beta*C, taken here as
 * fma(alpha, sum, beta*C).
 * ---------------------------------------------------------------------- */
void orc_gemv_1xn_f32(int N, int K, float alpha, const float* A, const float* B, int ldb, float beta, float* C) {
    for (int j0 = 0; j0 < N; j0 += 64) {
        const int jlen = N - j0 < 64 ? N - j0 : 64;
        for (int j = 0; j < jlen; ++j) {
            const float acc = dot_fma(A, 1, B + j0 + j, (size_t)ldb, 0, K);
            C[j0 + j] = epi_fused(acc, alpha, beta, C[j0 + j]);
        }
    }
}

/* ------------------------------------------------------------------------
 * M = 2..7 wide driver: src/gemm/gemm_smallm_wide_fp32.cpp:412-490.
 * Rows in groups of 4, then 2, then a single leftover row; 48-column panels
 * in 16-column sub-blocks; Kc = 256 blocks keep the accumulators, so every
 * output is one fused dot product in k order.  Full 16-column sub-blocks
 * store with epi_fused, partial ones with epi_tail (store_tail).  The
 * leftover row is the 64-column GEMV with epi_fused on full quads and the
 * scalar loop on the N % 4 columns of each panel.
 * ---------------------------------------------------------------------- */
void orc_smallm_wide_f32(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                         float beta, float* C, int ldc) {
    int i = 0;
    const int group[2] = {4, 2};
    for (int gi = 0; gi < 2; ++gi) {
        const int g = group[gi];
        for (; i + g - 1 < M; i += g) {
            for (int j0 = 0; j0 < N; j0 += 48) {
                const int jlen = N - j0 < 48 ? N - j0 : 48;
                for (int js = 0; js < jlen; js += 16) {
                    const int sub = jlen - js < 16 ? jlen - js : 16;
                    for (int r = i; r < i + g; ++r)
                        for (int j = 0; j < sub; ++j) {
                            const int col = j0 + js + j;
                            const float acc = dot_fma(A + (size_t)r * lda, 1, B + col, (size_t)ldb, 0, K);
                            float* c = C + (size_t)r * ldc + col;
                            *c = sub == 16 ? epi_fused(acc, alpha, beta, *c) : epi_tail(acc, alpha, beta, *c);
                        }
                }
            }
        }
    }
    if (i < M) {
        for (int j0 = 0; j0 < N; j0 += 64) {
            const int jlen = N - j0 < 64 ? N - j0 : 64;
            for (int j = 0; j < jlen; ++j) {
                const int col = j0 + j;
                const float acc = dot_fma(A + (size_t)i * lda, 1, B + col, (size_t)ldb, 0, K);
                float* c = C + (size_t)i * ldc + col;
                *c = epi_fused(acc, alpha, beta, *c);
            }
        }
    }
}

/* ------------------------------------------------------------------------
 * Adaptive register tiles: src/gemm/gemm_adaptive_tile_fp32.cpp:664-780
 * (tile choice :34-78, tail kernel :577-658).  Used by the reference for
 * M = 5 and M = 7 when N*K > 4Mi.  The k range is cut into Kc blocks,
 * Kc = floor((L1D*4/5) / ((Mr + 16) * 4)); block b accumulates a fused dot
 * product over its k and updates C with epi_tail using beta for b = 0 and
 * 1 afterwards, so C is re-rounded after every block.  Panels of 16
 * columns run in parallel (OpenMP) above 50 MiFLOP, as in the reference.
 * mr is the row tile the reference picks (5 for M = 5, 6 for M = 7); the
 * result does not depend on it, only Kc does.
 * ---------------------------------------------------------------------- */
void orc_adaptive_f32(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                      float beta, float* C, int ldc, int mr, int l1d_bytes, int nthreads) {
    int Kc = (int)((unsigned)l1d_bytes * 4u / 5u) / ((mr + 16) * 4);
    if (Kc < 1) Kc = 1;
    if (Kc > K) Kc = K;
    const int jfull = (N / 16) * 16;
    const int panels = jfull / 16;
    const long long flops = 2ll * M * N * K;
    const int threaded = panels >= 2 && flops > 50ll * 1024 * 1024 && nthreads > 1;
    (void)threaded;
#ifdef _OPENMP
#pragma omp parallel for num_threads(nthreads) schedule(static) if (threaded)
#endif
    for (int p = 0; p < panels + (jfull < N ? 1 : 0); ++p) {
        const int j0 = p * 16;
        const int jlen = N - j0 < 16 ? N - j0 : 16;
        for (int r = 0; r < M; ++r)
            for (int j = 0; j < jlen; ++j) {
                float* c = C + (size_t)r * ldc + j0 + j;
                for (int pc = 0; pc < K; pc += Kc) {
                    const int k1 = pc + Kc < K ? pc + Kc : K;
                    const float acc = dot_fma(A + (size_t)r * lda, 1, B + j0 + j, (size_t)ldb, pc, k1);
                    *c = epi_tail(acc, alpha, pc == 0 ? beta : 1.0f, *c);
                }
            }
    }
}

/* Reference fp32 routing for the small-M shapes (src/gemm/gemm.cpp:175-329,
 * default thresholds, Neoverse N2 L1D = 64 KiB): M == 1 -> GEMV; M = 2, 3 ->
 * wide driver; M = 5, 7 -> adaptive tiles when N*K > 4Mi, else wide driver;
 * M = 4, 6 with N*K > 4Mi go to the packed path, which is not restated here
 * (returns -1).  Returns 0 when computed. */
int orc_gemm_f32_smallm(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc, int nthreads) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const long long nk = (long long)N * K;
    if (M == 1) {
        orc_gemv_1xn_f32(N, K, alpha, A, B, ldb, beta, C);
        return 0;
    }
    if ((M == 4 || M == 6) && nk > 4ll * 1024 * 1024) return -1;
    if ((M == 5 || M == 7) && nk > 4ll * 1024 * 1024) {
        orc_adaptive_f32(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, M == 5 ? 5 : 6, 64 * 1024, nthreads);
        return 0;
    }
    if (M >= 2 && M < 8 && (M < 4 || N >= 48)) {
        orc_smallm_wide_f32(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
        return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------------
 * Native int8: src/gemm/gemm_int8_native.cpp:238-247 (the scalar loop; the
 * SMMLA tiles compute the same exact integer sums).  B is N x K.
 * ---------------------------------------------------------------------- */
void orc_gemm_s8s8s32(int M, int N, int K, const int8_t* A, int lda, const int8_t* B, int ldb, int32_t* C,
                      int ldc) {
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            int32_t s = 0;
            for (int k = 0; k < K; ++k) s += (int32_t)A[(size_t)i * lda + k] * (int32_t)B[(size_t)j * ldb + k];
            C[(size_t)i * ldc + j] = s;
        }
}

/* Per-column dequantization: C = (float)acc * scale[j]; the per-tensor form
 * of the reference's caller is src/conv/conv3d.cpp:511-514. */
void orc_gemm_s8_colscale(int M, int N, int K, const int8_t* A, int lda, const int8_t* B, int ldb,
                          const float* scale, float* C, int ldc) {
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            int32_t s = 0;
            for (int k = 0; k < K; ++k) s += (int32_t)A[(size_t)i * lda + k] * (int32_t)B[(size_t)j * ldb + k];
            C[(size_t)i * ldc + j] = (float)s * scale[j];
        }
}

/* ------------------------------------------------------------------------
 * bf16 GEMM on bf16 operands with fp32 accumulation
 * (src/gemm/gemm_driver_bf16.cpp:134-218; src/gemm/gemm_smallm_bf16.cpp:73-247).
 * A product of two bf16 values is exact in fp32, so the only roundings are
 * the fp32 sums; the reference's BFMMLA accumulates in groups of 4 k whose
 * internal order is hardware-defined, so this restatement fixes the order as
 * fused ascending k and the kernels are compared to it by tolerance.
 * Epilogue epi_fused.
 * ---------------------------------------------------------------------- */
void orc_gemm_bf16(int M, int N, int K, float alpha, const uint16_t* A, int lda, const uint16_t* B, int ldb,
                   float beta, float* C, int ldc) {
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k)
                acc = fmaf(orc_bf16_to_f32(A[(size_t)i * lda + k]), orc_bf16_to_f32(B[(size_t)k * ldb + j]), acc);
            float* c = C + (size_t)i * ldc + j;
            *c = epi_fused(acc, alpha, beta, *c);
        }
}

/* ------------------------------------------------------------------------
 * fp32-API int8 with dynamic per-tensor quantization: the reference's packed
 * path (src/gemm/gemm_driver_generic.cpp:49-67 scales,
 * src/gemm/gemm_pack_int8.cpp:29-71 quantization,
 * src/gemm/gemm_ukernel_int8_neon.cpp:87-131 epilogue):
 *   s_X = max|X| / 127 (1 if max|X| == 0), q = clamp(rint(x * (1/s_X))),
 *   C = (sA*sB*alpha) * acc  or  fma(sA*sB*alpha, acc, beta*C).
 * The int32 sum is exact.  (The reference re-rounds C per Kc block on its
 * packed path; this restatement and the library take the single-pass form.)
 * ---------------------------------------------------------------------- */
static float quant_scale(float amax) { return amax == 0.0f ? 1.0f : amax / 127.0f; }

/* The reference rounds with lrintf (nearest, ties to even, in the default
 * rounding mode).  ORC_QUANT_ROUND exists only so that tests can build
 * deliberately wrong copies of this oracle (truncf, roundf) and show that the
 * tie/fraction closed-form test rejects them. */
#ifndef ORC_QUANT_ROUND
#define ORC_QUANT_ROUND rintf
#endif

static int8_t quant_s8(float v, float inv) {
    float q = ORC_QUANT_ROUND(v * inv);
    if (q > 127.0f) q = 127.0f;
    if (q < -128.0f) q = -128.0f;
    return (int8_t)(int)q;
}

void orc_gemm_int8_dynq(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc) {
    float amax_a = 0.0f, amax_b = 0.0f;
    for (int i = 0; i < M; ++i)
        for (int k = 0; k < K; ++k) amax_a = fmaxf(amax_a, fabsf(A[(size_t)i * lda + k]));
    for (int k = 0; k < K; ++k)
        for (int j = 0; j < N; ++j) amax_b = fmaxf(amax_b, fabsf(B[(size_t)k * ldb + j]));
    const float sa = quant_scale(amax_a), sb = quant_scale(amax_b);
    const float ia = 1.0f / sa, ib = 1.0f / sb;
    const float s = (sa * sb) * alpha;
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            int32_t acc = 0;
            for (int k = 0; k < K; ++k)
                acc += (int32_t)quant_s8(A[(size_t)i * lda + k], ia) * (int32_t)quant_s8(B[(size_t)k * ldb + j], ib);
            float* c = C + (size_t)i * ldc + j;
            *c = beta == 0.0f ? s * (float)acc : fmaf(s, (float)acc, beta * *c);
        }
}

/* ------------------------------------------------------------------------
 * fp32-API int8 for M <= 8: the reference's gemm_smallm_int8 route, taken by
 * gemm_int8 whenever M <= 8 on a CPU with I8MM (src/gemm/gemm.cpp:431-434).
 *   M == 1     gemm_mx1_int8 (src/gemm/gemm_smallm_int8.cpp:126-189)
 *   M == 2..8  gemm_smallm_int8_smmla (src/gemm/gemm_smallm_int8.cpp:198-488)
 * Both take per-tensor scales s_X = max|X| / 127 (1 if max|X| == 0) and
 * quantize with a true division, q = clamp(lrintf(x / s_X), -128, 127)
 * (:151, :159, :233, :280-281) -- not the packed path's x * (1 / s_X), which
 * rounds differently when x / s_X lies within an ulp of a half-integer.
 * The int32 sums are exact; t = alpha * (sA * sB) (:146, :170, :223, :356).
 *   M == 1: C = t * acc                          (beta == 0, C not read)
 *           C = fma(beta, C, t * acc)            (beta != 0)
 *     (:170-175: `result + beta * C[j]`, where `result` = t * acc also
 *     feeds the beta == 0 store, so a contracting compiler -- GCC's
 *     -ffp-contract=fast default, or clang's per-expression contraction --
 *     can fuse only the beta * C[j] product into the addition.)
 *   M >= 2: C is first set to 0 (beta == 0) or beta * C (beta != 1)
 *     (:243-250), then C + t * acc is stored, two roundings (:356-383,
 *     store_edge_tile_row :38-50; vfmaq_f32 with the factor 1.0 is the
 *     rounded sum).
 * Two defects of the reference's store code are fixed here, as in the
 * library: for M = 3 the reference never stores row 2 (its second row pair
 * is stored only when m_tile >= 4, :391), and for M = 7 it adds zeros to a
 * row 7 past the end of C (:445); this restatement stores rows 0..M-1.
 *
 * ORC_SMALLM_RECIP / ORC_SMALLM_FUSED exist only so that tests can build
 * deliberately wrong copies (reciprocal quantization; one fused epilogue)
 * and show that the closed-form tests reject them.
 * ---------------------------------------------------------------------- */
static int8_t quant_div(float v, float s) {
#ifdef ORC_SMALLM_RECIP
    float q = rintf(v * (1.0f / s));
#else
    float q = rintf(v / s);
#endif
    if (q > 127.0f) q = 127.0f;
    if (q < -128.0f) q = -128.0f;
    return (int8_t)(int)q;
}

void orc_gemm_int8_smallm(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                          float beta, float* C, int ldc) {
    if (M < 1 || M > 8 || N <= 0 || K <= 0) return;
    float amax_a = 0.0f, amax_b = 0.0f;
    for (int i = 0; i < M; ++i)
        for (int k = 0; k < K; ++k) {
            const float av = fabsf(A[(size_t)i * lda + k]);
            if (av > amax_a) amax_a = av;
        }
    for (int k = 0; k < K; ++k)
        for (int j = 0; j < N; ++j) {
            const float bv = fabsf(B[(size_t)k * ldb + j]);
            if (bv > amax_b) amax_b = bv;
        }
    const float sa = quant_scale(amax_a), sb = quant_scale(amax_b);
    const float t = alpha * (sa * sb);
    int8_t* qa = (int8_t*)malloc((size_t)M * K);
    int8_t* qb = (int8_t*)malloc((size_t)K * N);
    for (int i = 0; i < M; ++i)
        for (int k = 0; k < K; ++k) qa[(size_t)i * K + k] = quant_div(A[(size_t)i * lda + k], sa);
    for (int k = 0; k < K; ++k)
        for (int j = 0; j < N; ++j) qb[(size_t)k * N + j] = quant_div(B[(size_t)k * ldb + j], sb);
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            int32_t acc = 0;
            for (int k = 0; k < K; ++k) acc += (int32_t)qa[(size_t)i * K + k] * (int32_t)qb[(size_t)k * N + j];
            float* c = C + (size_t)i * ldc + j;
            const float r = t * (float)acc;
#ifdef ORC_SMALLM_FUSED
            *c = beta == 0.0f ? r : fmaf(t, (float)acc, beta * *c);
#else
            if (M == 1) {
                *c = beta == 0.0f ? r : fmaf(beta, *c, r);
            } else {
                const float c0 = beta == 0.0f ? 0.0f : (beta == 1.0f ? *c : *c * beta);
                *c = c0 + r;
            }
#endif
        }
    free(qa);
    free(qb);
}

/* gemm_int8's routing on the reference's target (I8MM present): M <= 8 the
 * small-M route above, otherwise the packed path (src/gemm/gemm.cpp:431-449). */
void orc_gemm_int8(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb, float beta,
                   float* C, int ldc) {
    if (M <= 0 || N <= 0 || K <= 0) return;
    if (M <= 8)
        orc_gemm_int8_smallm(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    else
        orc_gemm_int8_dynq(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
}

/* ------------------------------------------------------------------------
 * CBLAS: src/blas/cblas_sgemm.cpp:67-143.  Early exits, the column-major
 * duality (swap A<->B, M<->N, TransA<->TransB) and the explicit transposes of
 * the reference, then the scalar GEMM on the row-major no-transpose problem.
 * ---------------------------------------------------------------------- */
static void transpose_f32(const float* src, float* dst, int rows, int cols, int ld_src, int ld_dst) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) dst[(size_t)c * ld_dst + r] = src[(size_t)r * ld_src + c];
}

static void row_major(int ta, int tb, int M, int N, int K, float alpha, const float* A, int lda, const float* B,
                      int ldb, float beta, float* C, int ldc) {
    float* at = NULL;
    float* bt = NULL;
    if (ta) {
        at = (float*)malloc((size_t)M * K * sizeof(float));
        transpose_f32(A, at, K, M, lda, K);
        A = at;
        lda = K;
    }
    if (tb) {
        bt = (float*)malloc((size_t)K * N * sizeof(float));
        transpose_f32(B, bt, N, K, ldb, N);
        B = bt;
        ldb = N;
    }
    if (beta != 0.0f) {
        orc_gemm_naive_f32(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    } else {
        /* beta == 0: the production kernels store alpha*acc and never read C
         * (gemm_tiny_fp32.cpp:200-207, gemm_smallm_wide_fp32.cpp:47-59), so
         * C may hold NaN or, for the oneDNN hook's small-ldc temporary,
         * uninitialised memory.  Same k order as the naive loops. */
        for (int i = 0; i < M; ++i)
            for (int j = 0; j < N; ++j) {
                float acc = 0.0f;
                for (int k = 0; k < K; ++k) {
                    const float p = A[(size_t)i * lda + k] * B[(size_t)k * ldb + j];
                    acc = acc + p;
                }
                C[(size_t)i * ldc + j] = alpha * acc;
            }
    }
    free(at);
    free(bt);
}

/* order: 101 row-major, 102 column-major; trans: 111 N, 112 T, 113 C. */
void orc_cblas_sgemm(int order, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, int lda,
                     const float* B, int ldb, float beta, float* C, int ldc) {
    if (M <= 0 || N <= 0 || K <= 0) return;
    if (alpha == 0.0f && beta == 1.0f) return;
    const int ta = trans_a != 111, tb = trans_b != 111;
    if (order == 101)
        row_major(ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    else
        row_major(tb, ta, N, M, K, alpha, B, ldb, A, lda, beta, C, ldc);
}

/* ------------------------------------------------------------------------
 * oneDNN hook: integration/onednn/0001-dnnopt-integration.patch:279-370
 * (dnnopt_sgemm, fp32 with bias) and 573-630 (dnnopt_gemm_bf16bf16f32).
 * Column-major C (element (i, j) at C[j*ldc + i]).  The reference's steps, in
 * its order: 'P'/'p' -> unimplemented (fp32 only); M or N zero -> nothing;
 * K == 0 -> per column memset (beta == 0) or C *= beta (beta != 1), then the
 * bias loop; otherwise the row-major problem of the swapped operands
 * (patch:316-329) with transposed operands copied out first
 * (patch:243-268, 536-560), through a temporary of row stride M when
 * ldc < M (patch:330-352), then the bias loop (patch:355-362).  The
 * row-major product is the scalar orc_gemm_naive_f32 / orc_gemm_bf16 (the
 * reference calls its dispatcher there; kernels are compared to this by
 * tolerance).  Returns 0, or 1 for "unimplemented".
 * ---------------------------------------------------------------------- */
static void transpose_u16(const uint16_t* src, uint16_t* dst, int rows, int cols, int ld_src, int ld_dst) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) dst[(size_t)c * ld_dst + r] = src[(size_t)r * ld_src + c];
}

static void row_major_bf16(int ta, int tb, int M, int N, int K, float alpha, const uint16_t* A, int lda,
                           const uint16_t* B, int ldb, float beta, float* C, int ldc) {
    uint16_t* at = NULL;
    uint16_t* bt = NULL;
    if (ta) {
        at = (uint16_t*)malloc((size_t)M * K * sizeof(uint16_t));
        transpose_u16(A, at, K, M, lda, K);
        A = at;
        lda = K;
    }
    if (tb) {
        bt = (uint16_t*)malloc((size_t)K * N * sizeof(uint16_t));
        transpose_u16(B, bt, N, K, ldb, N);
        B = bt;
        ldb = N;
    }
    orc_gemm_bf16(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    free(at);
    free(bt);
}

static int onednn_hook(int bf16, char transa, char transb, int64_t M, int64_t N, int64_t K, float alpha,
                       const void* A, int64_t lda, const void* B, int64_t ldb, float beta, float* C, int64_t ldc,
                       const float* bias) {
    if (!bf16 && (transa == 'P' || transa == 'p' || transb == 'P' || transb == 'p')) return 1;
    if (M == 0 || N == 0) return 0;
    if (K == 0) {
        if (beta == 0.0f) {
            for (int64_t j = 0; j < N; ++j) memset(C + j * ldc, 0, (size_t)M * sizeof(float));
        } else if (beta != 1.0f) {
            for (int64_t j = 0; j < N; ++j)
                for (int64_t i = 0; i < M; ++i) C[j * ldc + i] *= beta;
        }
        if (bias)
            for (int64_t j = 0; j < N; ++j)
                for (int64_t i = 0; i < M; ++i) C[j * ldc + i] += bias[i];
        return 0;
    }
    const int tA = transa == 'T' || transa == 't';
    const int tB = transb == 'T' || transb == 't';
    const int rm_M = (int)N, rm_N = (int)M, rm_K = (int)K;
    float* out = C;
    int ld_out = (int)ldc;
    float* tmp = NULL;
    if ((int)ldc < rm_N) {
        tmp = (float*)malloc((size_t)rm_M * rm_N * sizeof(float));
        if (beta != 0.0f)
            for (int r = 0; r < rm_M; ++r)
                for (int c = 0; c < rm_N; ++c) tmp[(size_t)r * rm_N + c] = C[(size_t)r * ldc + c];
        out = tmp;
        ld_out = rm_N;
    }
    if (bf16)
        row_major_bf16(tB, tA, rm_M, rm_N, rm_K, alpha, (const uint16_t*)B, (int)ldb, (const uint16_t*)A, (int)lda,
                       beta, out, ld_out);
    else
        row_major(tB, tA, rm_M, rm_N, rm_K, alpha, (const float*)B, (int)ldb, (const float*)A, (int)lda, beta, out,
                  ld_out);
    if (tmp) {
        for (int r = 0; r < rm_M; ++r)
            for (int c = 0; c < rm_N; ++c) C[(size_t)r * ldc + c] = tmp[(size_t)r * rm_N + c];
        free(tmp);
    }
    if (bias)
        for (int64_t j = 0; j < N; ++j)
            for (int64_t i = 0; i < M; ++i) C[j * ldc + i] += bias[i];
    return 0;
}

int orc_onednn_sgemm(char transa, char transb, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
                     int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc,
                     const float* bias) {
    return onednn_hook(0, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias);
}

int orc_onednn_gemm_bf16bf16f32(char transa, char transb, int64_t M, int64_t N, int64_t K, float alpha,
                                const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, float beta, float* C,
                                int64_t ldc) {
    return onednn_hook(1, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, NULL);
}

/* cblas_saxpy: src/blas/cblas_saxpy.cpp:13-51 (fused update on the NEON
 * path; the x86 scalar build rounds the product separately: fused = 0). */
void orc_saxpy(int N, float alpha, const float* X, int incX, float* Y, int incY, int fused) {
    if (N <= 0 || alpha == 0.0f) return;
    for (int i = 0; i < N; ++i) {
        float* y = Y + (size_t)i * incY;
        const float x = X[(size_t)i * incX];
        if (fused) {
            *y = fmaf(alpha, x, *y);
        } else {
            const float p = alpha * x;
            *y = *y + p;
        }
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
