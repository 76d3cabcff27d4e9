// k_kouter.hip -- fp32 C = A^T B for k-major operands with at most 64 rows
// and columns of C and a long k (gfx950).
//
// Shape: A stored K x M (TransA, lda >= M), B stored K x N (lda, ldb
// multiples of 4, both 16-byte aligned), 32 < M, N <= 64, K large: the
// reference's "transpose case" of cblas_sgemm (RowMajor, Trans, NoTrans;
// src/blas/cblas_sgemm.cpp:80-85 materialises A^T before its packed BLIS
// path, src/gemm/gemm_driver_generic.cpp:27-248).  Every k-row of A and B is
// one contiguous run of M (N) floats, so the GEMM is a sum over k of outer
// products and the whole job is streaming the two K x 64 panels once.
//
//   * Lane l = 16 g + q loads floats 4q .. 4q+3 of row k + g of A and of B
//     (one 16-byte load each): a wave load covers 4 rows x 64 columns of a
//     panel.  Every byte is read once, so the loads carry the non-temporal
//     hint (MI355X, 64 x 64 x 262144: 25.6-26.1 -> 23.6 us for the kernel).
//   * v_mfma_f32_16x16x4_f32 (i, j), i, j = 0..3, takes component i of the
//     lane's A floats as A-operand row q and component j of its B floats as
//     B-operand column q, so MFMA tile (i, j) holds the outputs
//     C[4 r + i][4 c + j] (r, c = 0..15): 16 MFMAs per 4 rows of k, every
//     loaded float used by 4 of them.
//   * A workgroup (4 waves) owns a contiguous range of 4-row steps; wave w
//     takes steps w, w + 4, w + 8, ... with a register ring of D steps in
//     flight.  Steps past the wave's last read zero from out-of-range
//     offsets; rows past K and columns past M / N are out of range or only
//     reach outputs outside C.
//   * The 4 waves' 64 x 64 sums are added in wave order through LDS and
//     stored as the workgroup's partial tile [split][64 * 64]; the split-K
//     reduce kernel adds the partials in split order and applies
//     alpha / beta / bias.
// Accumulation: fp32, k in MFMA order within a step (4 k), steps in
// ascending order per wave, then waves, then splits in fixed order -- the
// result is the same for every run of a given launch shape.
#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

namespace {

constexpr int kKOuterThreads = 256;  // 4 waves

template <int D>
__global__ __launch_bounds__(kKOuterThreads) void dnnopt_kouter_f32(TileArgs p) {
    __shared__ __attribute__((aligned(16))) float red[4][64 * 64];
    const int lane = lane_id(), q = lane & 15, g = lane >> 4;
    const int w = wave_id();
    const int t = (int)threadIdx.x;
    const int split = (int)blockIdx.z;

    const long long nsteps = ((long long)p.K + 3) / 4;
    const int lo = (int)(nsteps * split / p.splits);
    const int hi = (int)(nsteps * (split + 1) / p.splits);
    const int n = hi - lo;
    const int cnt = n > w ? (n - w + 3) >> 2 : 0;

    // Operand windows start at this workgroup's first row and end at the
    // last float of the operand (rows >= K read zero).
    const long long r0 = (long long)lo * 4;
    const bool any = n > 0 && r0 < p.K;
    const float* A = static_cast<const float*>(p.A);
    const float* B = static_cast<const float*>(p.B);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(
        any ? A + r0 * p.lda : A, any ? range31((size_t)((p.K - 1 - r0) * p.lda + p.M) * 4) : 0u);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(
        any ? B + r0 * p.ldb : B, any ? range31((size_t)((p.K - 1 - r0) * p.ldb + p.N) * 4) : 0u);
    const uint32_t a_lane = ((uint32_t)(4 * w + g) * (uint32_t)p.lda + 4u * q) * 4u;
    const uint32_t b_lane = ((uint32_t)(4 * w + g) * (uint32_t)p.ldb + 4u * q) * 4u;
    const uint32_t a_step = 64u * (uint32_t)p.lda, b_step = 64u * (uint32_t)p.ldb;  // 16 rows

    f32x4 av[D], bv[D];
    auto load = [&](int i, int slot) {
        const bool ok = i < cnt;
        av[slot] = __builtin_bit_cast(f32x4, buf_load_x4_stream(ra, ok ? a_lane + (uint32_t)i * a_step : kOobOffset));
        bv[slot] = __builtin_bit_cast(f32x4, buf_load_x4_stream(rb, ok ? b_lane + (uint32_t)i * b_step : kOobOffset));
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int slot) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[slot][i], bv[slot][j], acc[i][j], 0, 0, 0);
    };

#pragma unroll
    for (int d = 0; d < D; ++d) load(d, d);
    int i0 = 0;
    for (; i0 + D <= cnt; i0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            compute(d);
            load(i0 + d + D, d);
            // Keep each refill right after the MFMAs that free its slot (the
            // scheduler would otherwise sink the loads to the end of the
            // group and drain the ring).
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (i0 + d < cnt) compute(d);

    // MFMA tile (i, j), lane (g, q), element e holds C[16 g + 4 e + i][4 q + j].
    float* mine = red[w];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<f32x4*>(&mine[(16 * g + 4 * e + i) * 64 + 4 * q]) =
                f32x4{acc[i][0][e], acc[i][1][e], acc[i][2][e], acc[i][3][e]};
    __syncthreads();
    // The partial tile is written through to memory (sc0 sc1): the reduce
    // kernel reads it from there, and the launch ends with no dirty L2 lines
    // to write back (MI355X, 64 x 64 x 262144: 30.6 -> 30.2 us).
    const __amdgpu_buffer_rsrc_t rpart = make_rsrc(p.part + (size_t)split * (64 * 64), 64 * 64 * 4);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int f = 4 * (t + u * kKOuterThreads);
        f32x4 v = *reinterpret_cast<const f32x4*>(&red[0][f]);
        v += *reinterpret_cast<const f32x4*>(&red[1][f]);
        v += *reinterpret_cast<const f32x4*>(&red[2][f]);
        v += *reinterpret_cast<const f32x4*>(&red[3][f]);
        buf_store_x4_coherent(rpart, (uint32_t)f * 4u, v);
    }
}

// Steps in flight per wave (measured at 64 x 64 x 262144: 2 -> 42, 3 -> 33.7,
// 4 -> 32.5, 6 -> 31.9, 8 -> 32.0 us with the reduce).
#ifndef DNNOPT_KOUTER_D
#define DNNOPT_KOUTER_D 6
#endif

}  // namespace

hipError_t launch_kouter_f32(dim3 grid, const TileArgs& a, hipStream_t s) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(a.A) | reinterpret_cast<uintptr_t>(a.B);
    if (!a.transA || a.transB || a.M < 1 || a.M > 64 || a.N < 1 || a.N > 64 || a.K < 1 || a.lda < a.M ||
        a.ldb < a.N || (a.lda & 3) || (a.ldb & 3) || (al & 15) || a.part == nullptr || a.splits < 1 ||
        grid.x != 1 || grid.y != 1 || (int)grid.z != a.splits)
        return hipErrorInvalidValue;
    // Per-workgroup offsets: the rows of one split plus one step of 16 rows.
    const long long nsteps = ((long long)a.K + 3) / 4;
    const long long rows = ((nsteps + a.splits - 1) / a.splits) * 4 + 16;
    if (rows * (a.lda > a.ldb ? a.lda : a.ldb) * 4 >= 0x7FFFFFFFll) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dnnopt_kouter_f32<DNNOPT_KOUTER_D>, grid, dim3(kKOuterThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dnnopt_hip
