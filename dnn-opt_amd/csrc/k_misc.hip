// k_misc.hip -- scalar-reference GEMM, saxpy and synthetic-input kernels (gfx950).
#include "device_common.h"
#include "kernels.h"
#include "synth.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

// One thread per output, k ascending, product and sum rounded separately
// (no fused multiply-add), then alpha*acc + beta*C with C always read: the
// reference's scalar loop (src/gemm/gemm.cpp:88-100) as compiled for a target
// without FMA contraction.  Used for GemmAlgo::kNaive.
#pragma clang fp contract(off)
__global__ __launch_bounds__(256) void dnnopt_naive_f32(int M, int N, int K, float alpha, const float* A,
                                                       int lda, const float* B, int ldb, float beta, float* C,
                                                       int ldc, int row0) {
    const int j = blockIdx.x * 64 + (threadIdx.x & 63);
    const int i = row0 + blockIdx.y * 4 + (threadIdx.x >> 6);
    if (i >= M || j >= N) return;
    const float* a = A + (size_t)i * lda;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) {
        const float prod = a[k] * B[(size_t)k * ldb + j];
        acc = acc + prod;
    }
    float* c = C + (size_t)i * ldc + j;
    const float t0 = alpha * acc;
    const float t1 = beta * *c;
    *c = t0 + t1;
}
#pragma clang fp contract(on)

// Y[i*incy] = fma(alpha, X[i*incx], Y[i*incy])  (src/blas/cblas_saxpy.cpp:17-49
// computes the same fused update on its NEON path).  incx = 0 broadcasts
// X[0] (cblas_saxpy.cpp:45-49 indexes X[i * incX]); incy > 0 gives every i
// its own element of Y.
__global__ __launch_bounds__(256) void dnnopt_saxpy(int n, float alpha, const float* x, int incx, float* y,
                                                   int incy) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (size_t)n; i += stride) {
        float* yp = y + i * (size_t)incy;
        *yp = __builtin_fmaf(alpha, x[i * (size_t)incx], *yp);
    }
}

// incy = 0: every update lands on Y[0], in i order (the reference's strided
// loop, cblas_saxpy.cpp:45-49), so one thread applies them one after another.
__global__ __launch_bounds__(64) void dnnopt_saxpy_one(int n, float alpha, const float* x, int incx, float* y) {
    if (threadIdx.x != 0) return;
    float acc = *y;
    for (int i = 0; i < n; ++i) acc = __builtin_fmaf(alpha, x[(size_t)i * incx], acc);
    *y = acc;
}

#pragma clang fp contract(off)
__global__ __launch_bounds__(256) void dnnopt_fill(void* dst, size_t n, int dtype, int dist, uint64_t key,
                                                  double p0, double p1) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        if (dtype == 2) {
            static_cast<int8_t*>(dst)[i] = dnnopt_synth::int_value(key, i, (int)p0, (int)p1);
            continue;
        }
        const float v = dist == 1 ? dnnopt_synth::normal_value(key, i, p0, p1)
                                  : dnnopt_synth::uniform_value(key, i, p0, p1);
        if (dtype == 0) {
            static_cast<float*>(dst)[i] = v;
        } else {
            static_cast<uint16_t*>(dst)[i] = f32_to_bf16_bits(v);
        }
    }
}
#pragma clang fp contract(on)

hipError_t launch_naive_f32(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                            float beta, float* C, int ldc, hipStream_t s) {
    // Rows in launches of at most 65535 * 4 (the grid's y limit).
    constexpr int kRowsPerLaunch = 65535 * 4;
    for (int row0 = 0; row0 < M; row0 += kRowsPerLaunch) {
        const int rows = M - row0 < kRowsPerLaunch ? M - row0 : kRowsPerLaunch;
        dim3 grid((N + 63) / 64, (rows + 3) / 4);
        hipLaunchKernelGGL(dnnopt_naive_f32, grid, dim3(256), 0, s, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc,
                           row0);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_saxpy(int n, float alpha, const float* x, int incx, float* y, int incy, hipStream_t s) {
    if (incy == 0) {
        hipLaunchKernelGGL(dnnopt_saxpy_one, dim3(1), dim3(64), 0, s, n, alpha, x, incx, y);
        return hipGetLastError();
    }
    int blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(dnnopt_saxpy, dim3(blocks), dim3(256), 0, s, n, alpha, x, incx, y, incy);
    return hipGetLastError();
}

hipError_t launch_fill(void* dst, size_t n, int dtype, int dist, uint64_t seed, uint32_t tensor_id, double p0,
                       double p1, hipStream_t s) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(dnnopt_fill, dim3((unsigned)blocks), dim3(256), 0, s, dst, n, dtype, dist,
                       dnnopt_synth::tensor_key(seed, tensor_id), p0, p1);
    return hipGetLastError();
}

}  // namespace dnnopt_hip

namespace dnnopt_hip {

// Sum k-split partial tiles [split][tile][bm*bn] (tile = tile_m * tiles_n +
// tile_n, row-major inside a tile) into C with the reference epilogue.  One
// thread per 4 consecutive columns of a tile row: the partial reads of a
// wave are contiguous and C (for beta != 0) is requested with the partials.
// Q = 1 (up to 16 splits): splits are added in ascending order -- the order
// of the last-arriving-workgroup reduction, so both give the same bits.
// Q > 1 (many splits): Q threads per output each add an ascending range of
// splits, and the Q range sums are added in ascending order through LDS; the
// order is fixed, so the result is still reproducible.  SB loads (the
// smallest of 2, 4, 8, 16 that covers a thread's splits) are issued per batch,
// so a 2-way split issues 2 loads per output group, not 16.
template <int Q, int SB = 16>
__global__ __launch_bounds__(256) void dnnopt_splitk_reduce(const float* __restrict__ part, int splits,
                                                           int tiles_n, int tiles, int bm, int bn, int M, int N,
                                                           float alpha, float beta, float* C, int ldc,
                                                           const float* bias) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int OUTS = 256 / Q;
    __shared__ f4 red[Q > 1 ? Q * OUTS : 1];
    const int o = threadIdx.x % OUTS, q = threadIdx.x / OUTS;
    const int per_tile = bm * bn / 4;
    const long long idx = (long long)blockIdx.x * OUTS + o;
    const bool valid = idx < (long long)tiles * per_tile;
    const int tile = valid ? (int)(idx / per_tile) : 0;
    const int loc = valid ? (int)(idx % per_tile) * 4 : 0;
    const int m = (tile / tiles_n) * bm + loc / bn;
    const int n = (tile % tiles_n) * bn + loc % bn;
    const bool live = valid && m < M && n < N;
    float* c = C + (size_t)m * ldc + n;
    float c_old[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live && q == 0 && beta != 0.0f) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (n + e < N) c_old[e] = c[e];
    }
    const int s_lo = (int)((long long)splits * q / Q), s_hi = (int)((long long)splits * (q + 1) / Q);
    f4 s = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live && s_lo < s_hi) {
        // One batch of unconditional 16-byte loads per kSplitBatch splits
        // (offsets past s_hi are out of range and read zero), then the adds
        // in ascending split order, predicated on the range.
        constexpr int kSplitBatch = SB;
        const uint32_t stride = (uint32_t)tiles * (uint32_t)per_tile * 16u;
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, range31((size_t)splits * tiles * per_tile * 16));
        const uint32_t base = (uint32_t)idx * 16u;
        for (int sp0 = s_lo; sp0 < s_hi; sp0 += kSplitBatch) {
            f4 v[kSplitBatch];
#pragma unroll
            for (int u = 0; u < kSplitBatch; ++u)
                v[u] = __builtin_bit_cast(f4, buf_load_x4(rp, sp0 + u < s_hi ? base + (uint32_t)(sp0 + u) * stride : kOobOffset));
#pragma unroll
            for (int u = 0; u < kSplitBatch; ++u) {
                if (sp0 + u < s_hi) s = sp0 + u == s_lo ? v[u] : s + v[u];
            }
        }
    }
    if constexpr (Q > 1) {
        red[q * OUTS + o] = s;
        __syncthreads();
        if (q != 0) return;
        s = red[o];
        for (int qq = 1; qq < Q; ++qq)
            if ((long long)splits * qq / Q < (long long)splits * (qq + 1) / Q) s += red[qq * OUTS + o];
    }
    if (!live) return;
    f4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        out[e] = n + e < N ? add_bias(beta == 0.0f ? alpha * s[e] : __builtin_fmaf(alpha, s[e], beta * c_old[e]), bias, n + e)
                           : 0.0f;
    // Four whole columns on a 16-byte boundary: one 16-byte store.
    if (n + 4 <= N && (reinterpret_cast<uintptr_t>(c) & 15) == 0) {
        *reinterpret_cast<f4*>(c) = out;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (n + e < N) c[e] = out[e];
    }
}

hipError_t launch_splitk_reduce(const float* part, int splits, int tiles_n, int tiles_m, int bm, int bn, int M,
                                int N, float alpha, float beta, float* C, int ldc, const float* bias,
                                hipStream_t s) {
    const long long quads = (long long)tiles_n * tiles_m * bm * bn / 4;
    // The kernel addresses the partials with 32-bit buffer offsets.
    if (splits < 1 || (long long)splits * quads * 16 > 0x7FFFFFFFll) return hipErrorInvalidValue;
    if (splits <= 16) {
        const dim3 grid((unsigned)((quads + 255) / 256));
        const int tiles = tiles_n * tiles_m;
        if (splits <= 2)
            hipLaunchKernelGGL((dnnopt_splitk_reduce<1, 2>), grid, dim3(256), 0, s, part, splits, tiles_n, tiles, bm,
                               bn, M, N, alpha, beta, C, ldc, bias);
        else if (splits <= 4)
            hipLaunchKernelGGL((dnnopt_splitk_reduce<1, 4>), grid, dim3(256), 0, s, part, splits, tiles_n, tiles, bm,
                               bn, M, N, alpha, beta, C, ldc, bias);
        else if (splits <= 8)
            hipLaunchKernelGGL((dnnopt_splitk_reduce<1, 8>), grid, dim3(256), 0, s, part, splits, tiles_n, tiles, bm,
                               bn, M, N, alpha, beta, C, ldc, bias);
        else
            hipLaunchKernelGGL((dnnopt_splitk_reduce<1, 16>), grid, dim3(256), 0, s, part, splits, tiles_n, tiles,
                               bm, bn, M, N, alpha, beta, C, ldc, bias);
    } else {
        hipLaunchKernelGGL(dnnopt_splitk_reduce<16>, dim3((unsigned)((quads + 15) / 16)), dim3(256), 0, s, part,
                           splits, tiles_n, tiles_n * tiles_m, bm, bn, M, N, alpha, beta, C, ldc, bias);
    }
    return hipGetLastError();
}

// Sum the k-split partials of the skinny kernel, [split][M][ncols_pad], in
// ascending split order and apply the reference epilogue.  Column tile t of T
// (width tw, a multiple of the 256-thread block) has splits_of_tile(t, G, T)
// partials.  The loads of a batch of kRedBatch partials (all of them for up
// to kRedBatch splits) are issued unconditionally -- offsets past the tile's
// splits are out of range and read zero -- before the first add, so the
// reduction costs one memory round trip; the adds are predicated on the
// split count, so the sum is exactly the ordered sum of the real partials.
// The batch is the smallest of 8, 16, 32, 64 that holds every split of a
// tile (at most 64), so a tile of 5 splits issues 8 loads per output, not
// 32, and one of 64 splits needs one round trip, not two.
template <int kRedBatch>
__global__ __launch_bounds__(256) void dnnopt_skinny_reduce(const float* __restrict__ part, int G, int T, int tw,
                                                           int M, int N, int ncols_pad, float alpha, float beta,
                                                           float* C, int ldc, const float* bias) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int m = blockIdx.y;
    if (n >= N) return;
    const int splits = splits_of_tile(n / tw, G, T);
    const int max_splits = G / T + (G % T ? 1 : 0);
    const uint32_t stride = (uint32_t)M * (uint32_t)ncols_pad * 4u;  // bytes between splits
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, range31((size_t)max_splits * M * ncols_pad * 4));
    const uint32_t base = ((uint32_t)m * (uint32_t)ncols_pad + (uint32_t)n) * 4u;
    float* c = C + (size_t)m * ldc + n;
    // C is requested together with the partials (one memory round trip).
    const float c_old = beta != 0.0f ? *c : 0.0f;
    float s = 0.0f;
    for (int sp0 = 0; sp0 < splits; sp0 += kRedBatch) {
        float v[kRedBatch];
#pragma unroll
        for (int u = 0; u < kRedBatch; ++u)
            v[u] = as_f32(buf_load_x1(rp, sp0 + u < splits ? base + (uint32_t)(sp0 + u) * stride : kOobOffset));
#pragma unroll
        for (int u = 0; u < kRedBatch; ++u) {
            if (sp0 + u < splits) s = sp0 + u == 0 ? v[u] : s + v[u];
        }
    }
    *c = add_bias(beta == 0.0f ? alpha * s : __builtin_fmaf(alpha, s, beta * c_old), bias, n);
}

// Sum exact int32 partial tiles [split][tile][bm*bn] and store C.
__global__ __launch_bounds__(256) void dnnopt_s8_reduce(const int32_t* __restrict__ part, int splits, int tiles_n,
                                                       int tiles, int bm, int bn, int M, int N, int epi,
                                                       const float* scale, const unsigned* amax, float alpha,
                                                       float beta, void* C, int ldc) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long long)M * N) return;
    const int m = (int)(idx / N), n = (int)(idx % N);
    const int tile_id = (m / bm) * tiles_n + n / bn;
    const int32_t* src = part + (size_t)tile_id * bm * bn + (size_t)(m % bm) * bn + (n % bn);
    const size_t stride = (size_t)tiles * bm * bn;
    int32_t s = 0;
    int sp = 0;
    for (; sp + 8 <= splits; sp += 8) {
        int32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = src[(size_t)(sp + u) * stride];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; sp < splits; ++sp) s += src[sp * stride];
    if (epi) {
        float* c = static_cast<float*>(C) + (size_t)m * ldc + n;
        *c = s8_out(s, n, scale, amax, amax ? dyn_dequant_scale(amax, alpha) : 0.0f, beta, c);
    } else {
        static_cast<int32_t*>(C)[(size_t)m * ldc + n] = s;
    }
}

hipError_t launch_skinny_reduce(const float* part, int G, int T, int tw, int M, int N, int ncols_pad,
                                float alpha, float beta, float* C, int ldc, const float* bias, hipStream_t s) {
    // The kernel addresses the partials with 32-bit buffer offsets.
    if (G < 1 || T < 1 || (long long)(G / T + (G % T ? 1 : 0)) * M * ncols_pad * 4 > 0x7FFFFFFFll)
        return hipErrorInvalidValue;
    const int max_splits = G / T + (G % T ? 1 : 0);
    const dim3 grid((N + 255) / 256, M);
    if (max_splits <= 8)
        hipLaunchKernelGGL(dnnopt_skinny_reduce<8>, grid, dim3(256), 0, s, part, G, T, tw, M, N, ncols_pad, alpha, beta,
                           C, ldc, bias);
    else if (max_splits <= 16)
        hipLaunchKernelGGL(dnnopt_skinny_reduce<16>, grid, dim3(256), 0, s, part, G, T, tw, M, N, ncols_pad, alpha,
                           beta, C, ldc, bias);
    else if (max_splits <= 32)
        hipLaunchKernelGGL(dnnopt_skinny_reduce<32>, grid, dim3(256), 0, s, part, G, T, tw, M, N, ncols_pad, alpha,
                           beta, C, ldc, bias);
    else
        hipLaunchKernelGGL(dnnopt_skinny_reduce<64>, grid, dim3(256), 0, s, part, G, T, tw, M, N, ncols_pad, alpha,
                           beta, C, ldc, bias);
    return hipGetLastError();
}

hipError_t launch_s8_reduce(const int32_t* part, int splits, int tiles_n, int tiles_m, int bm, int bn, int M,
                            int N, int epi, const float* scale, const unsigned* amax, float alpha, float beta,
                            void* C, int ldc, hipStream_t s) {
    const long long outs = (long long)M * N;
    hipLaunchKernelGGL(dnnopt_s8_reduce, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, s, part, splits,
                       tiles_n, tiles_n * tiles_m, bm, bn, M, N, epi, scale, amax, alpha, beta, C, ldc);
    return hipGetLastError();
}

}  // namespace dnnopt_hip
