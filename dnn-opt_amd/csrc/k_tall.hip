// k_tall.hip -- fp32 tall-skinny GEMM with B resident in LDS (gfx950).
//
// Shapes: M large, N <= 64 (the dispatcher sends 16 < N <= 64), K small
// enough that all of B (K x N, fp32) fits
// in 64 KiB of LDS -- the tall-skinny case of the reference's packed BLIS
// path (src/gemm/gemm_driver_generic.cpp:27-248), where every row block of A
// meets the same small B.  The register-only MFMA tiles re-read B through L1
// for every k-step; here each workgroup stages B once, in MFMA fragment
// order, and its waves stream A:
//   * v_mfma_f32_16x16x4_f32: lane l supplies A[row l % 16][k] and
//     B[k][col l % 16] for the 4 k of its quad, k = k0 + 4 * (l / 16) + c --
//     one 16-byte load of A and one 16-byte LDS read of B per 4 MFMAs;
//   * B in LDS as [K/4][NP][4] floats (NP = 16 * NT columns, zero beyond K
//     and N), so the 16 lanes of a quarter-wave read 16 consecutive 16-byte
//     chunks;
//   * each wave owns RT x 16 rows at a time and walks (row tile, 16-k chunk)
//     pairs in one flattened sequence with a register ring of D chunks of A
//     in flight, so the stream does not stop at row-tile boundaries;
//   * workgroups are persistent (a few per CU) and take row tiles in a
//     strided order.
// Accumulation is fp32 in ascending k within a lane quad (MFMA order), C =
// alpha*acc (beta == 0, C unread) or fma(alpha, acc, beta*C), then the
// optional column bias.  A's elements past K in the last chunk are masked
// (they belong to the next row).
//
// The loop body issues no memory operation other than the ring's loads (the
// bias is read before the loop, outputs outside C go to out-of-range buffer
// offsets instead of being branched around, and the beta == 0 variant never
// reads C), so every wait on a chunk is exact and the ring stays full across
// row tiles.
#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

namespace {

#ifndef DNNOPT_TALL_WAVES
#define DNNOPT_TALL_WAVES 8
#endif
#ifndef DNNOPT_TALL_D
#define DNNOPT_TALL_D 4
#endif
constexpr int kTallWaves = DNNOPT_TALL_WAVES;
constexpr int kTallD = DNNOPT_TALL_D;

__device__ __forceinline__ u32x4 keep_first(u32x4 v, int valid) {
    u32x4 r;
#pragma unroll
    for (int d = 0; d < 4; ++d) r[d] = d < valid ? v[d] : 0u;
    return r;
}

}  // namespace

// NT column tiles of 16 (N <= 16 * NT), RT row tiles of 16 per wave, D
// chunks of A in flight, TB: B stored N x K, BETA: C is read (beta != 0).
template <int NT, int RT, int D, int TB, int BETA>
__global__ __launch_bounds__(kTallWaves * 64) void dnnopt_tall_f32(TallArgs p) {
    constexpr int NP = 16 * NT;
    extern __shared__ __attribute__((aligned(16))) float bsm[];

    const int lane = lane_id(), w = wave_id();
    const int r = lane & 15, g = lane >> 4;
    const int KC = (p.K + 15) / 16;           // 16-k chunks
    const int tiles = (p.M + 16 * RT - 1) / (16 * RT);
    const int gw = (int)blockIdx.x * kTallWaves + w, GW = (int)gridDim.x * kTallWaves;
    const int my_tiles = gw < tiles ? (tiles - 1 - gw) / GW + 1 : 0;
    const int total = my_tiles * KC;

    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc(p.A, range31(((size_t)(p.M - 1) * p.lda + p.K) * 4));

    // A chunk `i` of this wave: row tile gw + (i / KC) * GW, k = 16 * (i % KC).
    u32x4 ring[D][RT];
    auto load = [&](int i, int slot) {
        const int ic = i < total ? i : total - 1;  // past the end: re-read the last chunk (unused)
        const int ti = gw + (ic / KC) * GW, kc = ic % KC;
        const int kq = kc * 16 + 4 * g;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int row = ti * 16 * RT + rt * 16 + r;
            const uint32_t off = (row < p.M && kq < p.K) ? ((uint32_t)row * p.lda + kq) * 4u : kOobOffset;
            ring[slot][rt] = buf_load_x4(ra, off);
        }
    };
    // First chunks of A go out before B is staged.
    if (total > 0) {
#pragma unroll
        for (int d = 0; d < D; ++d) load(d, d);
    }

    // Stage B: unit u = (k quad kq, column n) -> 4 floats at bsm[(kq * NP + n) * 4].
    {
        const int KQ = KC * 4;
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(
            p.B, range31((TB ? (size_t)(p.N - 1) * p.ldb + p.K : (size_t)(p.K - 1) * p.ldb + p.N) * 4));
        for (int u = (int)threadIdx.x; u < KQ * NP; u += kTallWaves * 64) {
            const int kq = u / NP, n = u % NP;
            const int k0 = 4 * kq;
            if constexpr (TB) {
                const uint32_t off = (n < p.N && k0 < p.K) ? ((uint32_t)n * p.ldb + k0) * 4u : kOobOffset;
                *reinterpret_cast<u32x4*>(&bsm[(size_t)u * 4]) = keep_first(buf_load_x4(rb, off), p.K - k0);
            }
        }
        if constexpr (!TB) {
            // B stored K x N: unit = (k, 4 columns), one 16-byte load spread
            // over the 4 column slots of quad k / 4.  Columns past N (in the
            // last partial group, or past the padded width) are zero.
            const int NQ = NP / 4;
            for (int u = (int)threadIdx.x; u < KQ * 4 * NQ; u += kTallWaves * 64) {
                const int k = u / NQ, n0 = (u % NQ) * 4;
                u32x4 v = {0u, 0u, 0u, 0u};
                if (k < p.K) {
                    if (n0 + 4 <= p.N && ((p.ldb & 3) == 0)) {
                        v = buf_load_x4(rb, ((uint32_t)k * p.ldb + n0) * 4u);
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            v[c] = n0 + c < p.N ? buf_load_x1(rb, ((uint32_t)k * p.ldb + n0 + c) * 4u) : 0u;
                    }
                }
#pragma unroll
                for (int c = 0; c < 4; ++c) bsm[((size_t)(k >> 2) * NP + n0 + c) * 4 + (k & 3)] = as_f32(v[c]);
            }
        }
    }
    __syncthreads();
    if (total == 0) return;

    // Column bias of this lane's NT columns (read once).
    const bool has_bias = p.bias != nullptr;
    float biasv[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) biasv[nt] = (has_bias && nt * 16 + r < p.N) ? p.bias[nt * 16 + r] : 0.0f;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.C, range31(((size_t)(p.M - 1) * p.ldc + p.N) * 4));

    f32x4 acc[RT][NT];
    const int ktail = p.K - (KC - 1) * 16;  // k of the last chunk (1..16)

    auto step = [&](int i, const u32x4 (&a)[RT]) {
        const int kc = i % KC;
        if (kc == 0) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        u32x4 av[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) av[rt] = (kc == KC - 1 && ktail < 16) ? keep_first(a[rt], ktail - 4 * g) : a[rt];
        u32x4 bv[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            bv[nt] = *reinterpret_cast<const u32x4*>(&bsm[((size_t)(kc * 4 + g) * NP + nt * 16 + r) * 4]);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(as_f32(av[rt][c]), as_f32(bv[nt][c]),
                                                                      acc[rt][nt], 0, 0, 0);
        if (kc == KC - 1) {
            const int ti = gw + (i / KC) * GW;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int m = ti * 16 * RT + rt * 16 + 4 * g + e;
                        const int n = nt * 16 + r;
                        const uint32_t off = (m < p.M && n < p.N) ? ((uint32_t)m * p.ldc + n) * 4u : kOobOffset;
                        float v;
                        if constexpr (BETA) v = __builtin_fmaf(p.alpha, acc[rt][nt][e], p.beta * as_f32(buf_load_x1(rc, off)));
                        else v = p.alpha * acc[rt][nt][e];
                        if (has_bias) v = __fadd_rn(v, biasv[nt]);
                        buf_store_x1(rc, off, as_u32(v));
                    }
        }
    };

    // Chunk i lives in slot i % D from its load until its MFMAs; full groups
    // of D run without conditionals so the waits stay exact.
    int i0 = 0;
    for (; i0 + D <= total; i0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            u32x4 a[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) a[rt] = ring[d][rt];
            load(i0 + d + D, d);
            step(i0 + d, a);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (i0 + d < total) {
            u32x4 a[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) a[rt] = ring[d][rt];
            step(i0 + d, a);
        }
    }
}

int tall_waves() { return kTallWaves; }

template <int BETA>
static hipError_t launch_tall_beta(int nt, int tb, dim3 grid, size_t lds_bytes, const TallArgs& a, hipStream_t s) {
    const dim3 blk(kTallWaves * 64);
    switch (nt * 2 + (tb ? 1 : 0)) {
        case 2: hipLaunchKernelGGL((dnnopt_tall_f32<1, 2, kTallD, 0, BETA>), grid, blk, lds_bytes, s, a); break;
        case 3: hipLaunchKernelGGL((dnnopt_tall_f32<1, 2, kTallD, 1, BETA>), grid, blk, lds_bytes, s, a); break;
        case 4: hipLaunchKernelGGL((dnnopt_tall_f32<2, 2, kTallD, 0, BETA>), grid, blk, lds_bytes, s, a); break;
        case 5: hipLaunchKernelGGL((dnnopt_tall_f32<2, 2, kTallD, 1, BETA>), grid, blk, lds_bytes, s, a); break;
        case 6: hipLaunchKernelGGL((dnnopt_tall_f32<3, 2, kTallD, 0, BETA>), grid, blk, lds_bytes, s, a); break;
        case 7: hipLaunchKernelGGL((dnnopt_tall_f32<3, 2, kTallD, 1, BETA>), grid, blk, lds_bytes, s, a); break;
        case 8: hipLaunchKernelGGL((dnnopt_tall_f32<4, 2, kTallD, 0, BETA>), grid, blk, lds_bytes, s, a); break;
        case 9: hipLaunchKernelGGL((dnnopt_tall_f32<4, 2, kTallD, 1, BETA>), grid, blk, lds_bytes, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_tall_f32(int nt, int tb, dim3 grid, size_t lds_bytes, const TallArgs& a, hipStream_t s) {
    if (lds_bytes > 65536) return hipErrorInvalidValue;
    return a.beta == 0.0f ? launch_tall_beta<0>(nt, tb, grid, lds_bytes, a, s)
                          : launch_tall_beta<1>(nt, tb, grid, lds_bytes, a, s);
}

}  // namespace dnnopt_hip
