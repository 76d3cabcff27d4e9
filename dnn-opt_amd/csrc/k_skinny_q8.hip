// k_skinny_q8.hip -- fp32-API gemm_int8 for M <= 8 in one pass over B (gfx950).
//
// With M <= 8 the reference's fp32 gemm_int8 (src/gemm/gemm.cpp:431-434)
// takes its small-M route, gemm_smallm_int8 (src/gemm/gemm_smallm_int8.cpp):
// per-tensor scales s_X = max|X| / 127 (1 if zero), quantization by a true
// division, q = clamp(lrintf(x / s_X), -128, 127) (:151, :159, :233,
// :280-281), exact int32 sums, and its own epilogues -- M = 1:
// t acc or fma(beta, C, t acc) (:170-175); M = 2..8: C set to 0 or beta C
// first (:243-250), then C + t acc (:356-383), with t = alpha (sA sB).
// (The reference's M = 3 store skips row 2 and its M = 7 store touches a row
// 7 past C, :391, :445; every row 0..M-1 is stored here, nothing else.)
//
// The product is a stream over B, so this kernel reads the fp32 B (K x N,
// row-major) once, after the maxima pass (dnnopt_absmax_part), quantizes
// every element as it arrives (A's values of each block are quantized by
// the wave's lanes into LDS bytes), and adds exact int32 products with
// v_dot4_i32_i8: no int8 copy of B is written or read.  The division is the
// reciprocal product plus one fused correction (quant_s8_div), which gives
// the correctly rounded quotient.
//
// Lane layout and k-split follow dnnopt_skinny: a wave covers 256 columns (16
// bytes of a row per lane), the 8 waves of a workgroup and the workgroups of
// a column tile take contiguous k-ranges, waves are combined through LDS and
// workgroups through int32 partial sums that dnnopt_skinny_q8_reduce adds up.
// Integer sums are exact, so the order of the combine does not matter.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

namespace {

constexpr int kQ8Waves = 8;
constexpr int kQ8Unroll = 16;  // rows of B in flight per wave
constexpr int kQ8Cols = 256;   // columns per wave (4 per lane)

// Four values in [-128, 127] as the bytes of one dword, the first in the low
// byte (the operand layout of v_dot4_i32_i8): each value's low byte, picked
// by three byte permutes.
__device__ __forceinline__ uint32_t pack_q4(int a, int b, int c, int d) {
    const uint32_t ab = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);  // [a0 b0 0 0]
    const uint32_t cd = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);  // [c0 d0 0 0]
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);                                  // [a0 b0 c0 d0]
}

// B is read exactly once: streaming loads.
__device__ __forceinline__ u32x4 load_row(__amdgpu_buffer_rsrc_t r, uint32_t off) { return buf_load_x4_stream(r, off); }


}  // namespace

template <int MR>
__global__ __launch_bounds__(kQ8Waves * 64) void dnnopt_skinny_q8(SkinnyQ8Args p) {
    constexpr int NW = kQ8Waves, U = kQ8Unroll, TW = kQ8Cols;
    // LDS combine of the waves in passes of G rows (G * 8 KB).
    constexpr int G = MR < 4 ? MR : 4;
    constexpr int P = (MR + G - 1) / G;
    __shared__ i32x4 red[NW * G * (TW / 4)];
    // A's values of a block, quantized by the wave's lanes (lane l takes
    // entries l, l + 64, ...: row e / U, k e % U) into bytes, read back as
    // broadcasts of 16 k per row.
    constexpr int QA = MR * U;
    constexpr int QL = (QA + 63) / 64;
    static_assert(U == 16, "one 16-byte broadcast per row of A per block");
    __shared__ u32x4 qa_lds[NW][MR];

    const int lane = lane_id(), w = wave_id();
    const SplitPos sp = split_pos((int)blockIdx.x, (int)gridDim.x, p.tiles);
    const int col0 = sp.tile * TW;
    // With a reduce kernel to follow every tile publishes partial sums, also
    // a tile of one k-split (the reduce kernel covers every column of C).
    const bool direct = !p.defer;
    const long long nblk = (p.K + U - 1) / U;
    const long long chunks = (long long)sp.nsplit * NW;
    const long long cw = (long long)sp.split * NW + w;
    const int k_lo = (int)((nblk * cw) / chunks) * U;
    const int k_hi = min(p.K, (int)((nblk * (cw + 1)) / chunks) * U);
    const int kb = (int)((nblk * ((long long)sp.split * NW)) / chunks) * U;

    // Buffer range from row kb, column col0 to the last element of B; lanes
    // whose four columns all lie past N read nothing.  Columns past N inside
    // a lane's group read the next row's values, which are never stored.
    const float* bbase = p.B + (size_t)kb * p.ldb + col0;
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(bbase, range31(((size_t)(p.K - 1 - kb) * p.ldb + (size_t)(p.N - col0)) * 4));
    const uint32_t rowbytes = (uint32_t)p.ldb * 4u;
    const uint32_t lane_off = col0 + lane * 4 < p.N ? (uint32_t)lane * 16u : kOobOffset;

    // A: lane l of a block takes entries l, l + 64, ... (row e / U, k e % U)
    // through a 64-bit pointer (A's rows may lie further apart than a
    // buffer's 31-bit offsets reach); lanes past the block's MR x U entries
    // load nothing.
    const float* a_lane[QL];
#pragma unroll
    for (int j = 0; j < QL; ++j) {
        const int e = lane + 64 * j;
        a_lane[j] = e < QA ? p.A + (size_t)(e / U) * p.lda + e % U : nullptr;
    }
    auto load_block = [&](u32x4 (&raw)[U], float (&av)[QL], int k0) {
#pragma unroll
        for (int u = 0; u < U; ++u) raw[u] = load_row(rs, (uint32_t)(k0 + u - kb) * rowbytes + lane_off);
#pragma unroll
        for (int j = 0; j < QL; ++j) av[j] = (QA % 64 == 0 || lane + 64 * j < QA) ? a_lane[j][k0] : 0.0f;
    };

    // The first block goes out before the maxima are read.
    u32x4 raw0[U], raw1[U];
    float av0[QL], av1[QL];
    int k = k_lo;
    if (k + U <= k_hi) load_block(raw0, av0, k);
    unsigned ma, mb;
    wave_maxima(p.qpart, p.ga, p.gb, &ma, &mb);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        p.amax[0] = ma;
        p.amax[1] = mb;
    }
    const QuantDiv qd_a = quant_div_of(ma), qd_b = quant_div_of(mb);
    // Either scale outside the fast division's range: both take the exact
    // division (the two forms agree wherever the fast one applies).
    const bool exact = qd_a.exact || qd_b.exact;

    int acc[MR][4];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[m][e] = 0;

    // One whole block: A's MR x 16 values are quantized by the wave's lanes
    // into LDS bytes and read back as one 16-byte broadcast per row; per 4
    // rows of B a lane packs each of its columns' 4 quantized k into one
    // dword and adds 4 products per v_dot4_i32_i8.  |x| <= max|X| bounds
    // |x / s| by 127 (plus rounding), so the values need no clamp here.
    int8_t* const qw = reinterpret_cast<int8_t*>(qa_lds[w]);
    auto compute_block = [&](const u32x4 (&raw)[U], const float (&av)[QL]) {
#pragma unroll
        for (int j = 0; j < QL; ++j)
            if (lane + 64 * j < QA) qw[lane + 64 * j] = (int8_t)quant_s8_div<false, false>(av[j], qd_a);
        u32x4 a16[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) a16[m] = qa_lds[w][m];
#pragma unroll
        for (int q = 0; q < U / 4; ++q) {
            uint32_t b4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                b4[e] = pack_q4(quant_s8_div<false, false>(as_f32(raw[4 * q][e]), qd_b),
                                quant_s8_div<false, false>(as_f32(raw[4 * q + 1][e]), qd_b),
                                quant_s8_div<false, false>(as_f32(raw[4 * q + 2][e]), qd_b),
                                quant_s8_div<false, false>(as_f32(raw[4 * q + 3][e]), qd_b));
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[m][e] = __builtin_amdgcn_sdot4((int)a16[m][q], (int)b4[e], acc[m][e], false);
        }
    };
    // Whole blocks, two register sets alternating (the next block's loads
    // are in flight while one is consumed, with no copies between sets).
    // Only with both scales in the fast division's range; otherwise
    // (wave-uniform) the whole range goes through the row-at-a-time loop
    // below with the exact division.
    if (!exact) {
        while (k + U <= k_hi) {
            if (k + 2 * U <= k_hi) load_block(raw1, av1, k + U);
            compute_block(raw0, av0);
            k += U;
            if (k + U > k_hi) break;
            if (k + 2 * U <= k_hi) load_block(raw0, av0, k + U);
            compute_block(raw1, av1);
            k += U;
        }
    }
    // The last k % 16 rows of the range (all of it with the exact division),
    // one at a time.
    auto rows = [&](auto ex) {
        constexpr bool EX = decltype(ex)::value;
        for (; k < k_hi; ++k) {
            const u32x4 v = load_row(rs, (uint32_t)(k - kb) * rowbytes + lane_off);
            int qb[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) qb[e] = quant_s8_div<EX, true>(as_f32(v[e]), qd_b);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const int qa = quant_s8_div<EX, true>(p.A[(size_t)m * p.lda + k], qd_a);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[m][e] += qa * qb[e];
            }
        }
    };
    if (exact)
        rows(std::true_type{});
    else
        rows(std::false_type{});

    // Combine the waves: thread t owns 4-column group t % 64 of row t / 64
    // within a pass of G rows.
    const float t_dq = mul_rn(p.alpha, mul_rn(qd_a.s, qd_b.s));
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.part, range31((size_t)p.splits * MR * p.ncols_pad * 4));
#pragma unroll
    for (int pass = 0; pass < P; ++pass) {
        if (pass) __syncthreads();
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int m = pass * G + g;
            if (m < MR) red[(w * G + g) * (TW / 4) + lane] = i32x4{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
        }
        __syncthreads();
        const int t = (int)threadIdx.x;
        const int g = t / (TW / 4), c4 = t % (TW / 4);
        const int m = pass * G + g;
        if (t < G * (TW / 4) && m < MR) {
            i32x4 s = red[g * (TW / 4) + c4];
#pragma unroll
            for (int w2 = 1; w2 < NW; ++w2) s += red[(w2 * G + g) * (TW / 4) + c4];
            const int n = col0 + 4 * c4;
            if (direct) {
                float* c = p.C + (size_t)m * p.ldc + n;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n + e < p.N) c[e] = smallm_out(s[e], MR == 1, t_dq, p.beta, p.beta != 0.0f ? c[e] : 0.0f);
            } else {
                const uint32_t off = (uint32_t)((((size_t)sp.split * MR + m) * p.ncols_pad + n) * 4);
                buf_store_x4_coherent(rp, off, __builtin_bit_cast(f32x4, s));
            }
        }
    }
}

// Sum the int32 partials [split][M][ncols_pad] of a tile's splits (exact) and
// store C with the small-M epilogue (smallm_out).  All partial loads of an output (a batch of SB,
// the smallest of 8, 16, 32, 64 that holds the largest split count) are
// issued before the first add -- offsets past the tile's splits are out of
// range and read zero -- so the sum costs one memory round trip.
template <int SB>
__global__ __launch_bounds__(256) void dnnopt_skinny_q8_reduce(const int32_t* __restrict__ part, int G, int T, int M,
                                                              int N, int ncols_pad, const unsigned* amax, float alpha,
                                                              float beta, float* C, int ldc) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int m = blockIdx.y;
    if (n >= N) return;
    const int splits = splits_of_tile(n / kQ8Cols, G, T);
    const int max_splits = G / T + (G % T ? 1 : 0);
    const uint32_t stride = (uint32_t)M * (uint32_t)ncols_pad * 4u;
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, range31((size_t)max_splits * M * ncols_pad * 4));
    const uint32_t base = ((uint32_t)m * (uint32_t)ncols_pad + (uint32_t)n) * 4u;
    float* c = C + (size_t)m * ldc + n;
    const float c_old = beta != 0.0f ? *c : 0.0f;
    int32_t s = 0;
    for (int sp0 = 0; sp0 < splits; sp0 += SB) {
        uint32_t v[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u) v[u] = buf_load_x1(rp, sp0 + u < splits ? base + (uint32_t)(sp0 + u) * stride : kOobOffset);
#pragma unroll
        for (int u = 0; u < SB; ++u) s += (int32_t)v[u];  // out-of-range loads read 0
    }
    const float t = mul_rn(alpha, mul_rn(quant_scale_bits(amax[0]), quant_scale_bits(amax[1])));
    *c = smallm_out(s, M == 1, t, beta, c_old);
}

hipError_t launch_skinny_q8(int mr, dim3 grid, const SkinnyQ8Args& a, hipStream_t s) {
    const dim3 blk(kQ8Waves * 64);
    switch (mr) {
        case 1: hipLaunchKernelGGL(dnnopt_skinny_q8<1>, grid, blk, 0, s, a); break;
        case 2: hipLaunchKernelGGL(dnnopt_skinny_q8<2>, grid, blk, 0, s, a); break;
        case 3: hipLaunchKernelGGL(dnnopt_skinny_q8<3>, grid, blk, 0, s, a); break;
        case 4: hipLaunchKernelGGL(dnnopt_skinny_q8<4>, grid, blk, 0, s, a); break;
        case 5: hipLaunchKernelGGL(dnnopt_skinny_q8<5>, grid, blk, 0, s, a); break;
        case 6: hipLaunchKernelGGL(dnnopt_skinny_q8<6>, grid, blk, 0, s, a); break;
        case 7: hipLaunchKernelGGL(dnnopt_skinny_q8<7>, grid, blk, 0, s, a); break;
        case 8: hipLaunchKernelGGL(dnnopt_skinny_q8<8>, grid, blk, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    if (!a.defer) return hipGetLastError();
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 rg((a.N + 255) / 256, a.M);
    const int G = (int)grid.x, T = a.tiles, ms = G / T + (G % T ? 1 : 0);
#define DNNOPT_Q8_REDUCE(SB)                                                                                   \
    hipLaunchKernelGGL(dnnopt_skinny_q8_reduce<SB>, rg, dim3(256), 0, s, a.part, G, T, a.M, a.N, a.ncols_pad, \
                       a.amax, a.alpha, a.beta, a.C, a.ldc)
    if (ms <= 8) DNNOPT_Q8_REDUCE(8);
    else if (ms <= 16) DNNOPT_Q8_REDUCE(16);
    else if (ms <= 32) DNNOPT_Q8_REDUCE(32);
    else DNNOPT_Q8_REDUCE(64);
#undef DNNOPT_Q8_REDUCE
    return hipGetLastError();
}

int skinny_q8_waves() { return kQ8Waves; }

}  // namespace dnnopt_hip
