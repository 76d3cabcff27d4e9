// k_quant.hip -- dynamic per-tensor int8 quantization for the fp32 gemm_int8 API.
//
// Semantics of the reference's packed int8 path (src/gemm/gemm_driver_generic.cpp:
// 49-67, src/gemm/gemm_pack_int8.cpp:29-71):
//   scale_X = max|X| / 127, or 1 when max|X| == 0;
//   q = clamp(round_to_nearest_even(x * (1 / scale_X)), -128, 127);
//   C = alpha*scale_A*scale_B * acc  (beta == 0)  or
//       fma(alpha*scale_A*scale_B, acc, beta*C)   (ukernel_int8_neon.cpp:87-131).
//
// The pipeline is three launches: dnnopt_absmax_part (per-workgroup maxima of
// both operands), dnnopt_quantize_pair (every workgroup reduces those maxima,
// then quantizes its share of A, or of B straight into the N x K layout the
// int8 kernels read), and the int8 GEMM, whose epilogue dequantizes into the
// fp32 C (s8_out in device_common.h) -- no int32 copy of C exists.
#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

namespace {

// |x| as an orderable bit pattern; NaN contributes nothing (the reference's
// `if (av > max) max = av` never takes a NaN).
__device__ __forceinline__ unsigned abs_bits(float x) {
    const unsigned b = as_u32(x) & 0x7FFFFFFFu;
    return b > 0x7F800000u ? 0u : b;
}

__device__ __forceinline__ unsigned block_max(unsigned m, unsigned* lds) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned o = (unsigned)__shfl_xor((int)m, off, 64);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = m;
    __syncthreads();
    m = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) m = lds[w] > m ? lds[w] : m;
    return m;
}

__device__ __forceinline__ int8_t quantize(float x, float inv) {
    float v = __builtin_rintf(x * inv);
    v = v > 127.0f ? 127.0f : (v < -128.0f ? -128.0f : v);
    return (int8_t)(int)v;
}

constexpr int kTK = 128;  // B tile (k rows) quantized and transposed through LDS
constexpr int kTN = 64;   // B tile (n columns)

// Four consecutive floats of a row starting at column c (VEC: one 16-byte
// load; else element loads), zero past `cols`.
template <int VEC>
__device__ __forceinline__ f32x4 load4(const float* row, int c, int cols) {
    if constexpr (VEC) {
        if (c + 4 <= cols) return *reinterpret_cast<const f32x4*>(row + c);
    }
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = c + e < cols ? row[c + e] : 0.0f;
    return v;
}

}  // namespace

// Blocks [0, ga) take rows of A (M x K, stride lda), blocks [ga, grid) rows of
// B (K x N, stride ldb); each stores the max |x| bits of its rows to part.
// VEC: rows start on 16-byte boundaries (16-byte loads, four in flight per
// thread).
template <int VEC>
__global__ __launch_bounds__(256) void dnnopt_absmax_part(const float* __restrict__ A, int M, int K, int lda,
                                                         int ga, const float* __restrict__ B, int N, int ldb,
                                                         unsigned* part) {
    __shared__ unsigned red[4];
    const bool is_a = (int)blockIdx.x < ga;
    const float* x = is_a ? A : B;
    const int rows = is_a ? M : K, cols = is_a ? K : N, ld = is_a ? lda : ldb;
    const int g = is_a ? (int)blockIdx.x : (int)blockIdx.x - ga;
    const int G = is_a ? ga : (int)gridDim.x - ga;
    unsigned m = 0;
    for (int r = g; r < rows; r += G) {
        const float* row = x + (size_t)r * ld;
        for (int c0 = 0; c0 < cols; c0 += 256 * 16) {
            f32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = c0 + (u * 256 + (int)threadIdx.x) * 4;
                v[u] = c < cols ? load4<VEC>(row, c, cols) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const unsigned b = abs_bits(v[u][e]);
                    m = b > m ? b : m;
                }
        }
    }
    m = block_max(m, red);
    if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// Every block first reduces the partial maxima (ga of A, gb of B); block 0
// also stores them to amax[0..1] for the GEMM's epilogue.  Blocks [0, qa)
// quantize rows of A into qA (M x ldq); the others quantize 128 x 64 (k x n)
// tiles of B into qB (N x ldq, i.e. transposed) through LDS: a wave reads 4
// rows of 64 floats per instruction, and each row of the tile is written as
// 128 contiguous bytes of k.  Bytes of a row between K and ldq are zero.
template <int VEC>
__global__ __launch_bounds__(256) void dnnopt_quantize_pair(const float* __restrict__ A, int M, int K, int lda,
                                                           const float* __restrict__ B, int N, int ldb,
                                                           const unsigned* part, int ga, int gb, unsigned* amax,
                                                           int qa, int8_t* qA, int8_t* qB, int ldq) {
    __shared__ unsigned red[4];
    __shared__ __attribute__((aligned(16))) int8_t tile[kTN][kTK + 16];
    unsigned ma = 0, mb = 0;
    for (int i = (int)threadIdx.x; i < ga; i += 256) ma = part[i] > ma ? part[i] : ma;
    for (int i = (int)threadIdx.x; i < gb; i += 256) mb = part[ga + i] > mb ? part[ga + i] : mb;
    ma = block_max(ma, red);
    __syncthreads();
    mb = block_max(mb, red);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        amax[0] = ma;
        amax[1] = mb;
    }
    if ((int)blockIdx.x < qa) {
        const float inv = 1.0f / quant_scale_bits(ma);
        for (int r = (int)blockIdx.x; r < M; r += qa) {
            const float* row = A + (size_t)r * lda;
            int8_t* q = qA + (size_t)r * ldq;
            for (int c = (int)threadIdx.x * 4; c < ldq; c += 256 * 4) {
                const f32x4 v = c < K ? load4<VEC>(row, c, K) : f32x4{0.f, 0.f, 0.f, 0.f};
                char4 o;
                o.x = quantize(v[0], inv);
                o.y = quantize(v[1], inv);
                o.z = quantize(v[2], inv);
                o.w = quantize(v[3], inv);
                *reinterpret_cast<char4*>(q + c) = o;  // ldq is a multiple of 16, so c + 4 <= ldq
            }
        }
        return;
    }
    const float inv = 1.0f / quant_scale_bits(mb);
    const int tiles_k = (ldq + kTK - 1) / kTK;
    const int tb = (int)blockIdx.x - qa;
    const int k0 = (tb % tiles_k) * kTK, n0 = (tb / tiles_k) * kTN;
    // Load: lanes 16 apart take rows 4 apart; 16 lanes cover 64 floats of a row.
    {
        const int nc = ((int)threadIdx.x & 15) * 4;
        const int kr0 = (int)threadIdx.x >> 4;  // 0..15
        f32x4 v[kTK / 16];
#pragma unroll
        for (int j = 0; j < kTK / 16; ++j) {
            const int k = k0 + kr0 + 16 * j;
            v[j] = (k < K && n0 + nc < N) ? load4<VEC>(B + (size_t)k * ldb + n0, nc, N - n0)
                                          : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < kTK / 16; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) tile[nc + e][kr0 + 16 * j] = quantize(v[j][e], inv);
    }
    __syncthreads();
    // Store: 8 threads per row of the tile, 16 bytes of k each.
    {
        const int kc = ((int)threadIdx.x & 7) * 16;
#pragma unroll
        for (int j = 0; j < kTN / 32; ++j) {
            const int nr = ((int)threadIdx.x >> 3) + 32 * j;
            const int n = n0 + nr, k = k0 + kc;
            if (n < N && k < ldq) *reinterpret_cast<int4*>(qB + (size_t)n * ldq + k) =
                *reinterpret_cast<const int4*>(&tile[nr][kc]);
        }
    }
}

// Blocks for the maxima of the two operands: about one per 64 KiB of input,
// at most 1024 in all, shared out by size.
void absmax_blocks(int M, int N, int K, int* ga, int* gb) {
    const double a = (double)M * K, b = (double)K * N;
    long long total = (long long)((a + b) * 4 / 65536) + 2;
    if (total > 1024) total = 1024;
    long long x = (long long)(total * a / (a + b));
    if (x < 1) x = 1;
    if (x > M) x = M;
    long long y = total - x;
    if (y < 1) y = 1;
    if (y > K) y = K;
    *ga = (int)x;
    *gb = (int)y;
}

hipError_t launch_quant_pair(const float* A, int lda, const float* B, int ldb, int M, int N, int K, int ldq,
                             unsigned* part, unsigned* amax, int8_t* qA, int8_t* qB, hipStream_t s) {
    if (ldq % 16 != 0) return hipErrorInvalidValue;
    int ga = 1, gb = 1;
    absmax_blocks(M, N, K, &ga, &gb);
    // 16-byte loads when every row of both operands starts on a 16-byte boundary.
    const bool vec = ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15u) == 0 &&
                     (lda & 3) == 0 && (ldb & 3) == 0;
    if (vec)
        hipLaunchKernelGGL(dnnopt_absmax_part<1>, dim3(ga + gb), dim3(256), 0, s, A, M, K, lda, ga, B, N, ldb, part);
    else
        hipLaunchKernelGGL(dnnopt_absmax_part<0>, dim3(ga + gb), dim3(256), 0, s, A, M, K, lda, ga, B, N, ldb, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int qa = M < 256 ? M : 256;
    const long long qb = (long long)((ldq + kTK - 1) / kTK) * ((N + kTN - 1) / kTN);
    if (qa + qb > 0x7FFFFFFFll) return hipErrorInvalidValue;
    if (vec)
        hipLaunchKernelGGL(dnnopt_quantize_pair<1>, dim3((unsigned)(qa + qb)), dim3(256), 0, s, A, M, K, lda, B, N,
                           ldb, part, ga, gb, amax, qa, qA, qB, ldq);
    else
        hipLaunchKernelGGL(dnnopt_quantize_pair<0>, dim3((unsigned)(qa + qb)), dim3(256), 0, s, A, M, K, lda, B, N,
                           ldb, part, ga, gb, amax, qa, qA, qB, ldq);
    return hipGetLastError();
}

}  // namespace dnnopt_hip
