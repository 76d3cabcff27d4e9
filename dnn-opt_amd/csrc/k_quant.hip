// k_quant.hip -- dynamic per-tensor int8 quantization for the fp32 gemm_int8 API.
//
// Semantics of the reference's packed int8 path (src/gemm/gemm_driver_generic.cpp:
// 49-67, src/gemm/gemm_pack_int8.cpp:29-71):
//   scale_X = max|X| / 127, or 1 when max|X| == 0;
//   q = clamp(round_to_nearest_even(x * (1 / scale_X)), -128, 127);
//   C = alpha*scale_A*scale_B * acc  (beta == 0)  or
//       fma(alpha*scale_A*scale_B, acc, beta*C)   (ukernel_int8_neon.cpp:87-131).
// B (K x N, fp32) is quantized straight into the N x K int8 layout that the
// int8 MFMA kernel reads, so no separate transpose pass exists.
#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

__global__ __launch_bounds__(64) void dnnopt_zero_u32(unsigned* p, int n) {
    const int i = threadIdx.x;
    if (i < n) p[i] = 0u;
}

// max|x| of a rows x cols row-major block (row stride ld) into *out.  The
// bit patterns of non-negative floats order like the floats, so an integer
// atomic max is exact and independent of arrival order.
__global__ __launch_bounds__(256) void dnnopt_absmax(const float* __restrict__ x, int rows, int cols, int ld,
                                                    unsigned* out) {
    const long long total = (long long)rows * cols;
    const long long stride = (long long)gridDim.x * blockDim.x;
    unsigned m = 0;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int r = (int)(i / cols), c = (int)(i % cols);
        const unsigned b = as_u32(x[(size_t)r * ld + c]) & 0x7FFFFFFFu;
        m = b > m ? b : m;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned o = (unsigned)__shfl_xor((int)m, off, 64);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0 && m != 0) atomicMax(out, m);
}

__device__ __forceinline__ float quant_scale(unsigned amax_bits) {
    const float amax = as_f32(amax_bits);
    return amax == 0.0f ? 1.0f : amax / 127.0f;
}

// Quantize x (rows x cols, stride ld) into q.  transpose = 0: q[r][c] with
// row stride ldq; transpose = 1: q[c][r] (row stride ldq), which turns a
// K x N operand into the N x K layout.
__global__ __launch_bounds__(256) void dnnopt_quantize(const float* __restrict__ x, int rows, int cols, int ld,
                                                      int transpose, const unsigned* amax, int8_t* q, int ldq) {
    const float inv = 1.0f / quant_scale(*amax);
    const long long total = (long long)rows * cols;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        int r, c;
        if (transpose) {  // consecutive threads walk q's rows (x's columns) for coalesced stores
            c = (int)(i / rows);
            r = (int)(i % rows);
        } else {
            r = (int)(i / cols);
            c = (int)(i % cols);
        }
        float v = __builtin_rintf(x[(size_t)r * ld + c] * inv);
        v = v > 127.0f ? 127.0f : (v < -128.0f ? -128.0f : v);
        const int8_t s = (int8_t)(int)v;
        if (transpose) q[(size_t)c * ldq + r] = s;
        else q[(size_t)r * ldq + c] = s;
    }
}

// C = alpha*sA*sB*acc (+ beta*C), acc exact int32 (see header comment).
__global__ __launch_bounds__(256) void dnnopt_dequant(const int32_t* __restrict__ acc, int M, int N,
                                                     const unsigned* amax, float alpha, float beta, float* C,
                                                     int ldc) {
    const float s = (quant_scale(amax[0]) * quant_scale(amax[1])) * alpha;
    const long long total = (long long)M * N;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int m = (int)(i / N), n = (int)(i % N);
        float* c = C + (size_t)m * ldc + n;
        const float a = (float)acc[i];
        *c = beta == 0.0f ? s * a : __builtin_fmaf(s, a, beta * (*c));
    }
}

static unsigned grid_for(long long total) {
    long long b = (total + 255) / 256;
    if (b < 1) b = 1;
    if (b > 8192) b = 8192;
    return (unsigned)b;
}

hipError_t launch_quant_prepare(const float* A, int lda, const float* B, int ldb, int M, int N, int K, int ldq,
                                unsigned* amax, int8_t* qA, int8_t* qB, hipStream_t s) {
    hipLaunchKernelGGL(dnnopt_zero_u32, dim3(1), dim3(64), 0, s, amax, 2);
    hipLaunchKernelGGL(dnnopt_absmax, dim3(grid_for((long long)M * K)), dim3(256), 0, s, A, M, K, lda, amax);
    hipLaunchKernelGGL(dnnopt_absmax, dim3(grid_for((long long)K * N)), dim3(256), 0, s, B, K, N, ldb, amax + 1);
    hipLaunchKernelGGL(dnnopt_quantize, dim3(grid_for((long long)M * K)), dim3(256), 0, s, A, M, K, lda, 0, amax,
                       qA, ldq);
    hipLaunchKernelGGL(dnnopt_quantize, dim3(grid_for((long long)K * N)), dim3(256), 0, s, B, K, N, ldb, 1,
                       amax + 1, qB, ldq);
    return hipGetLastError();
}

hipError_t launch_dequant(const int32_t* acc, int M, int N, const unsigned* amax, float alpha, float beta,
                          float* C, int ldc, hipStream_t s) {
    hipLaunchKernelGGL(dnnopt_dequant, dim3(grid_for((long long)M * N)), dim3(256), 0, s, acc, M, N, amax, alpha,
                       beta, C, ldc);
    return hipGetLastError();
}

}  // namespace dnnopt_hip
