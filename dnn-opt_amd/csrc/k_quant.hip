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
// both operands), dnnopt_quantize_pair (every wave reduces those maxima, then
// quantizes its share of A, or of B straight into the N x K layout the int8
// kernels read), and the int8 GEMM, whose epilogue dequantizes into the fp32
// C (s8_out in device_common.h) -- no int32 copy of C exists.
#include "device_common.h"
#include "kernels.h"

#include <algorithm>

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

// Four quantized values as the bytes of one dword, the first in the low byte.
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | (uint32_t)(b & 0xFF) << 8 | (uint32_t)(c & 0xFF) << 16 | (uint32_t)d << 24;
}

constexpr int kQK = 64;   // k rows of a B block (16 per lane, 4 lanes)
constexpr int kQN = 256;  // n columns of a B block (64 per wave, 4 per lane)

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

// Blocks [0, qa) quantize rows of A into qA (M x ldq); blocks [qa, grid)
// quantize 64 (k) x 256 (n) tiles of B into qB (N x ldq, i.e. transposed)
// without LDS: lane (kq, ng) of wave w loads rows k0 + 16 kq .. + 15 of
// columns n0 + 64 w + 4 ng .. + 3 (per load, 4 rows x 256 contiguous bytes
// per wave), quantizes them and stores each column's 16 k as one 16-byte
// store (64 contiguous bytes of a qB row per 4 lanes).  B's loads are issued
// before the maxima are read, and every wave reduces the block maxima itself,
// so the loads stay in flight through the reduction.  Wave 0 of block 0
// stores max|A|, max|B| to amax[0..1] for the GEMM's epilogue.  Bytes of a
// row between K and ldq are zero.
template <int VEC>
__global__ __launch_bounds__(256) void dnnopt_quantize_pair(const float* __restrict__ A, int M, int K, int lda,
                                                           const float* __restrict__ B, int N, int ldb,
                                                           const unsigned* part, int ga, int gb, unsigned* amax,
                                                           int qa, int8_t* qA, int8_t* qB, int ldq) {
    if ((int)blockIdx.x < qa) {
        unsigned ma, mb;
        wave_maxima(part, ga, gb, &ma, &mb);
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            amax[0] = ma;
            amax[1] = mb;
        }
        const float inv = 1.0f / quant_scale_bits(ma);
        for (int r = (int)blockIdx.x; r < M; r += qa) {
            const float* row = A + (size_t)r * lda;
            int8_t* q = qA + (size_t)r * ldq;
            for (int c = (int)threadIdx.x * 4; c < ldq; c += 256 * 4) {
                const f32x4 v = c < K ? load4<VEC>(row, c, K) : f32x4{0.f, 0.f, 0.f, 0.f};
                // ldq is a multiple of 16, so c + 4 <= ldq
                *reinterpret_cast<uint32_t*>(q + c) =
                    pack4(quant_s8(v[0], inv), quant_s8(v[1], inv), quant_s8(v[2], inv), quant_s8(v[3], inv));
            }
        }
        return;
    }
    // The B blocks stride over the tiles (two per block at 4096 x 4096), so
    // one tile's stores overlap the next tile's loads.
    const int tiles_n = (N + kQN - 1) / kQN;
    const int ntiles = tiles_n * ((ldq + kQK - 1) / kQK);
    const int lane = lane_id();
    const int kq = lane & 3, ng = lane >> 2;
    float inv = 0.0f;
    bool first = true;
    for (int tb = (int)blockIdx.x - qa; tb < ntiles; tb += (int)gridDim.x - qa) {
        const int kr = (tb / tiles_n) * kQK + 16 * kq;                   // first of this lane's 16 rows
        const int n = (tb % tiles_n) * kQN + 64 * wave_id() + 4 * ng;  // first of its 4 columns
        f32x4 v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
            v[r] = (kr + r < K && n < N) ? load4<VEC>(B + (size_t)(kr + r) * ldb, n, N) : f32x4{0.f, 0.f, 0.f, 0.f};
        if (first) {
            unsigned ma, mb;
            wave_maxima(part, ga, gb, &ma, &mb);
            inv = 1.0f / quant_scale_bits(mb);
            first = false;
        }
        if (kr >= ldq) continue;  // ldq is a multiple of 16: a lane's 16 rows are all below it or all past it
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (n + e >= N) break;
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = pack4(quant_s8(v[4 * j][e], inv), quant_s8(v[4 * j + 1][e], inv),
                             quant_s8(v[4 * j + 2][e], inv), quant_s8(v[4 * j + 3][e], inv));
            *reinterpret_cast<u32x4*>(qB + (size_t)(n + e) * ldq + kr) = o;
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

// 16-byte loads when every row of both operands starts on a 16-byte boundary.
static bool quant_vec(const float* A, int lda, const float* B, int ldb) {
    return ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15u) == 0 && (lda & 3) == 0 &&
           (ldb & 3) == 0;
}

hipError_t launch_absmax(const float* A, int lda, const float* B, int ldb, int M, int N, int K, unsigned* part,
                         hipStream_t s) {
    int ga = 1, gb = 1;
    absmax_blocks(M, N, K, &ga, &gb);
    if (quant_vec(A, lda, B, ldb))
        hipLaunchKernelGGL(dnnopt_absmax_part<1>, dim3(ga + gb), dim3(256), 0, s, A, M, K, lda, ga, B, N, ldb, part);
    else
        hipLaunchKernelGGL(dnnopt_absmax_part<0>, dim3(ga + gb), dim3(256), 0, s, A, M, K, lda, ga, B, N, ldb, part);
    return hipGetLastError();
}

// A alone: one thread per 4 consecutive elements of qA (M x ldq), so a call
// is one memory round trip (its load goes out before the maxima are read).
template <int VEC>
__global__ __launch_bounds__(256) void dnnopt_quantize_a(const float* __restrict__ A, int M, int K, int lda,
                                                        const unsigned* part, int ga, int gb, unsigned* amax,
                                                        int8_t* qA, int ldq) {
    const long long e = ((long long)blockIdx.x * 256 + threadIdx.x) * 4;
    const int r = (int)(e / ldq), c = (int)(e % ldq);
    const bool live = r < M;
    const f32x4 v = live && c < K ? load4<VEC>(A + (size_t)r * lda, c, K) : f32x4{0.f, 0.f, 0.f, 0.f};
    unsigned ma, mb;
    wave_maxima(part, ga, gb, &ma, &mb);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        amax[0] = ma;
        amax[1] = mb;
    }
    if (!live) return;
    const float inv = 1.0f / quant_scale_bits(ma);
    // ldq is a multiple of 16, so c + 4 <= ldq
    *reinterpret_cast<uint32_t*>(qA + (size_t)r * ldq + c) =
        pack4(quant_s8(v[0], inv), quant_s8(v[1], inv), quant_s8(v[2], inv), quant_s8(v[3], inv));
}

hipError_t launch_quant_a(const float* A, int lda, int M, int K, int ldq, const unsigned* part, int ga, int gb,
                          unsigned* amax, int8_t* qA, hipStream_t s) {
    if (ldq % 16 != 0 || ga + gb > 1024) return hipErrorInvalidValue;
    const long long blocks = ((long long)M * ldq / 4 + 255) / 256;
    if (blocks > 0x7FFFFFFFll) return hipErrorInvalidValue;
    if (quant_vec(A, lda, A, lda))
        hipLaunchKernelGGL(dnnopt_quantize_a<1>, dim3((unsigned)blocks), dim3(256), 0, s, A, M, K, lda, part, ga, gb,
                           amax, qA, ldq);
    else
        hipLaunchKernelGGL(dnnopt_quantize_a<0>, dim3((unsigned)blocks), dim3(256), 0, s, A, M, K, lda, part, ga, gb,
                           amax, qA, ldq);
    return hipGetLastError();
}

hipError_t launch_quant_pair(const float* A, int lda, const float* B, int ldb, int M, int N, int K, int ldq,
                             unsigned* part, unsigned* amax, int8_t* qA, int8_t* qB, hipStream_t s) {
    if (ldq % 16 != 0) return hipErrorInvalidValue;
    int ga = 1, gb = 1;
    absmax_blocks(M, N, K, &ga, &gb);
    const bool vec = quant_vec(A, lda, B, ldb);
    hipError_t e = launch_absmax(A, lda, B, ldb, M, N, K, part, s);
    if (e != hipSuccess) return e;
    const int qa = M < 256 ? M : 256;
    if (ga + gb > 1024) return hipErrorInvalidValue;  // one wave reduces the maxima
    // Tiles of B; above 1024 of them each block takes two, else at most 512
    // blocks (MI355X, 4096 x 4096: 1024 blocks of one tile 16.5 us, 512 of
    // two 15 us).
    const long long tiles = (long long)((ldq + kQK - 1) / kQK) * ((N + kQN - 1) / kQN);
    const long long qb = tiles > 1024 ? (tiles + 1) / 2 : std::min<long long>(tiles, 512);
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
