// k_colmajor.hip -- column-major helpers of the oneDNN-hook entry points
// (gfx950): the K == 0 / bias epilogue, the temporary row stride used when
// ldc < M, and a bf16 transpose.
//
// The hook these serve (integration/onednn/0001-dnnopt-integration.patch:
// 279-370 for fp32, 573-630 for bf16) works on a column-major C whose
// element (i, j) lives at C[j * ldc + i].  With ldc < M consecutive columns
// overlap; the reference then applies its loops in a fixed order and the
// result at an address is decided by that order.  Every kernel here computes,
// for each address, the value those loops leave there:
//   * scaling (`C *= beta`, all columns, j ascending) multiplies an address
//     once per column that covers it;
//   * the bias loop adds bias[i] once per covering column, j ascending;
//   * the copy-back of a temporary with row stride M (rows r = 0..N-1, each
//     written in full in turn) leaves the element of the LAST row r that
//     covers the address.
// For ldc >= M columns are disjoint and each address is covered once.
#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

namespace {

constexpr int kThreads = 256;
constexpr long long kMaxBlocks = 16384;

__device__ __forceinline__ long long gtid() { return (long long)blockIdx.x * kThreads + threadIdx.x; }
__device__ __forceinline__ long long gstride() { return (long long)gridDim.x * kThreads; }

// Columns j (ascending) whose span [j*ldc, j*ldc + M) covers address e.
__device__ __forceinline__ void covering(long long e, int M, int N, long long ldc, long long* jlo, long long* jhi) {
    const long long hi = e / ldc;
    *jhi = hi < N - 1 ? hi : N - 1;
    const long long lo_num = e - M + 1;
    *jlo = lo_num <= 0 ? 0 : (lo_num + ldc - 1) / ldc;
}

// op: kCmNone (leave), kCmZero (C = 0, not read), kCmScale (C *= beta per
// covering column); then C += bias[i] per covering column.  Products and sums
// are rounded separately (no contraction), as the reference's loops are.
__global__ __launch_bounds__(kThreads) void dnnopt_cm_fixup(float* C, int M, int N, long long ldc, int op, float beta,
                                                           const float* bias) {
    if (ldc >= M) {
        const long long total = (long long)M * N;
        for (long long e = gtid(); e < total; e += gstride()) {
            const long long j = e / M;
            const int i = (int)(e - j * M);
            float* c = C + j * ldc + i;
            float v = op == kCmZero ? 0.0f : *c;
            if (op == kCmScale) v = mul_rn(v, beta);
            if (bias) v = add_rn(v, bias[i]);
            *c = v;
        }
        return;
    }
    const long long total = (long long)(N - 1) * ldc + M;
    for (long long e = gtid(); e < total; e += gstride()) {
        long long jlo, jhi;
        covering(e, M, N, ldc, &jlo, &jhi);
        float v = op == kCmZero ? 0.0f : C[e];
        if (op == kCmScale)
            for (long long j = jlo; j <= jhi; ++j) v = mul_rn(v, beta);
        if (bias)
            for (long long j = jlo; j <= jhi; ++j) v = add_rn(v, bias[e - j * ldc]);
        C[e] = v;
    }
}

// T (N rows x M, row stride M) <- C viewed as N rows of M at stride ldc.
__global__ __launch_bounds__(kThreads) void dnnopt_cm_gather(const float* C, long long ldc, float* T, int M, int N) {
    const long long total = (long long)M * N;
    for (long long e = gtid(); e < total; e += gstride()) {
        const long long r = e / M;
        const long long c = e - r * M;
        T[e] = C[r * ldc + c];
    }
}

// C <- rows of T written back at stride ldc < M, the last covering row wins.
__global__ __launch_bounds__(kThreads) void dnnopt_cm_scatter(const float* T, int M, int N, long long ldc, float* C) {
    const long long total = (long long)(N - 1) * ldc + M;
    for (long long e = gtid(); e < total; e += gstride()) {
        long long r = e / ldc;
        if (r > N - 1) r = N - 1;
        C[e] = T[r * M + (e - r * ldc)];
    }
}

// dst (cols x rows, stride ldd) = transpose of src (rows x cols, stride lds),
// 2-byte elements, 64 x 64 tiles through LDS (padded row: no bank conflicts
// on the transposed read).
constexpr int kTT = 64;
__global__ __launch_bounds__(kThreads) void dnnopt_transpose_u16(const uint16_t* src, int rows, int cols,
                                                                long long lds, uint16_t* dst, long long ldd) {
    __shared__ uint16_t tile[kTT][kTT + 2];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4 threads
    const long long r0 = (long long)blockIdx.y * kTT, c0 = (long long)blockIdx.x * kTT;
    for (int y = ty; y < kTT; y += 4) {
        const long long r = r0 + y, c = c0 + tx;
        if (r < rows && c < cols) tile[y][tx] = src[r * lds + c];
    }
    __syncthreads();
    for (int y = ty; y < kTT; y += 4) {
        const long long c = c0 + y, r = r0 + tx;
        if (c < cols && r < rows) dst[c * ldd + r] = tile[tx][y];
    }
}

unsigned blocks_for(long long n) {
    const long long b = (n + kThreads - 1) / kThreads;
    return (unsigned)(b < 1 ? 1 : (b > kMaxBlocks ? kMaxBlocks : b));
}

}  // namespace

hipError_t launch_cm_fixup(float* C, int M, int N, long long ldc, int op, float beta, const float* bias,
                           hipStream_t s) {
    if (M <= 0 || N <= 0 || ldc < 1) return hipErrorInvalidValue;
    const long long total = ldc >= M ? (long long)M * N : (long long)(N - 1) * ldc + M;
    hipLaunchKernelGGL(dnnopt_cm_fixup, dim3(blocks_for(total)), dim3(kThreads), 0, s, C, M, N, ldc, op, beta, bias);
    return hipGetLastError();
}

hipError_t launch_cm_gather(const float* C, long long ldc, float* T, int M, int N, hipStream_t s) {
    if (M <= 0 || N <= 0 || ldc < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dnnopt_cm_gather, dim3(blocks_for((long long)M * N)), dim3(kThreads), 0, s, C, ldc, T, M, N);
    return hipGetLastError();
}

hipError_t launch_cm_scatter(const float* T, int M, int N, long long ldc, float* C, hipStream_t s) {
    if (M <= 0 || N <= 0 || ldc < 1 || ldc >= M) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dnnopt_cm_scatter, dim3(blocks_for((long long)(N - 1) * ldc + M)), dim3(kThreads), 0, s, T, M,
                       N, ldc, C);
    return hipGetLastError();
}

hipError_t launch_transpose_u16(const uint16_t* src, int rows, int cols, long long lds, uint16_t* dst,
                                long long ldd, hipStream_t s) {
    if (rows <= 0 || cols <= 0 || lds < cols || ldd < rows) return hipErrorInvalidValue;
    const long long gx = (cols + kTT - 1) / kTT, gy = (rows + kTT - 1) / kTT;
    if (gx > 0x7FFFFFFFll || gy > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dnnopt_transpose_u16, dim3((unsigned)gx, (unsigned)gy), dim3(kThreads), 0, s, src, rows, cols,
                       lds, dst, ldd);
    return hipGetLastError();
}

}  // namespace dnnopt_hip
