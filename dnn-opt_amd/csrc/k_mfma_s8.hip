// k_mfma_s8.hip -- exact int8 x int8 -> int32 GEMM with B stored N x K (gfx950).
//
// Replaces the reference's native int8 GEMM (src/gemm/gemm_int8_native.cpp:
// 37-248: SMMLA 8x8 tiles plus scalar tails).  Both operands are K-contiguous,
// which is exactly the per-lane packing of v_mfma_i32_16x16x64_i8: lane l
// supplies 16 consecutive bytes of row (l % 16) of its operand, so A rows and
// B rows feed the matrix cores straight from 128-bit loads with no transpose.
//
// Per 256-byte k block, lane l (r = l % 16, g = l / 16) loads the 16-byte
// chunks at byte 64*j + 16*g (j = 0..3) of its row; MFMA j consumes chunk j.
// The same chunk-to-k assignment is used for A and B, so every k of the block
// meets its partner exactly once.  Integer accumulation is exact, so the
// reduction order across waves and workgroups does not affect the result.
//
// Tails: rows of A past M and rows of B past N read as zero (out-of-range
// buffer offset); bytes of A past K are masked to zero inside the last chunk,
// which zeroes their products whatever B holds there.
#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

namespace {

// Zero the bytes of a 16-byte chunk at or beyond `valid` (0..16).
__device__ __forceinline__ i32x4 mask_chunk(i32x4 v, int valid) {
    if (valid >= 16) return v;
    i32x4 r;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const int keep = valid - 4 * d;  // bytes of this dword to keep
        uint32_t m = keep >= 4 ? 0xFFFFFFFFu : (keep <= 0 ? 0u : ((1u << (8 * keep)) - 1u));
        r[d] = (int32_t)((uint32_t)v[d] & m);
    }
    return r;
}

}  // namespace

// AL = 1: all rows of A and B start on 4-byte boundaries; AL = 0: rows are
// read with funnel-shifted loads.
template <int AL>
__device__ __forceinline__ i32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (AL) return __builtin_bit_cast(i32x4, buf_load_x4(r, off));
    return __builtin_bit_cast(i32x4, buf_load_x4_unaligned(r, off));
}

template <int MT, int NT, int WM, int WN, int KW, int EPI, int AL>
__global__ __launch_bounds__(WM* WN* KW * 64) void dnnopt_mfma_s8(S8Args p) {
    constexpr int BM = WM * MT * 16;
    constexpr int BN = WN * NT * 16;
    constexpr int SUB = MT * NT * 4;  // accumulator dwords per lane

    __shared__ int32_t red[(KW > 1 ? (KW - 1) : 1) * WM * WN * SUB * 64];
    __shared__ int last_flag;

    const int lane = lane_id();
    const int r = lane & 15;
    const int g = lane >> 4;
    const int w = wave_id();
    const int wn = w % WN;
    const int wm = (w / WN) % WM;
    const int wk = w / (WN * WM);

    const int tile_n = blockIdx.x, tile_m = blockIdx.y, split = blockIdx.z;
    const int m0 = tile_m * BM, n0 = tile_n * BN;

    // Buffer descriptors start at this workgroup's first row of A and B.
    const int8_t* abase = p.A + (size_t)m0 * p.lda;
    const int8_t* bbase = p.B + (size_t)n0 * p.ldb;
    const size_t arem = (size_t)(p.M - 1 - m0) * p.lda + p.K;
    const size_t brem = (size_t)(p.N - 1 - n0) * p.ldb + p.K;
    uint32_t alo = 0, blo = 0;
    const __amdgpu_buffer_rsrc_t ra = rsrc_aligned(abase, arem, &alo);
    const __amdgpu_buffer_rsrc_t rb = rsrc_aligned(bbase, brem, &blo);

    uint32_t arow[MT], brow[NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int ml = (wm * MT + mt) * 16 + r;
        arow[mt] = (m0 + ml < p.M) ? (uint32_t)ml * p.lda + alo : kOobOffset;
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int nl = (wn * NT + nt) * 16 + r;
        brow[nt] = (n0 + nl < p.N) ? (uint32_t)nl * p.ldb + blo : kOobOffset;
    }

    const int nblk = (p.K + 255) / 256;
    const long long chunks = (long long)p.splits * KW;
    const long long cw = (long long)split * KW + wk;
    const int b_lo = (int)(((long long)nblk * cw) / chunks);
    const int b_hi = (int)(((long long)nblk * (cw + 1)) / chunks);

    i32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = i32x4{0, 0, 0, 0};

    for (int blk = b_lo; blk < b_hi; ++blk) {
        i32x4 a[MT][4], b[NT][4];
        const int kbase = blk * 256 + 16 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kc = kbase + 64 * j;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const uint32_t off = (kc < p.K && arow[mt] != kOobOffset) ? arow[mt] + kc : kOobOffset;
                a[mt][j] = load16<AL>(ra, off);
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t off = (brow[nt] != kOobOffset) ? brow[nt] + kc : kOobOffset;
                b[nt][j] = load16<AL>(rb, off);
            }
        }
        if (blk * 256 + 256 > p.K) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) a[mt][j] = mask_chunk(a[mt][j], p.K - (kbase + 64 * j));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mt][j], b[nt][j], acc[mt][nt], 0, 0, 0);
    }

    // Waves that split k inside the workgroup: add into the wk == 0 wave.
    if constexpr (KW > 1) {
        const int slot = wm * WN + wn;
        if (wk > 0) {
            int32_t* dst = &red[(((wk - 1) * WM * WN + slot) * SUB) * 64];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) dst[((mt * NT + nt) * 4 + i) * 64 + lane] = acc[mt][nt][i];
        }
        __syncthreads();
        if (wk == 0) {
#pragma unroll
            for (int q = 1; q < KW; ++q) {
                const int32_t* src = &red[(((q - 1) * WM * WN + slot) * SUB) * 64];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[mt][nt][i] += src[((mt * NT + nt) * 4 + i) * 64 + lane];
            }
        }
    }

    // Output element (mt, nt, i) of this lane: row 4*g + i, column r of the
    // 16 x 16 tile (v_mfma_*_16x16x* accumulator layout).
    const int tiles = gridDim.x * gridDim.y;
    const int tile_id = tile_m * gridDim.x + tile_n;
    if (p.splits > 1) {
        // Partials are written through to memory (coherent stores) so the
        // reducing workgroup can read them without cache maintenance.
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(
            p.part, (uint32_t)min<size_t>((size_t)p.splits * tiles * BM * BN * 4, 0x7FFFFFFFull));
        if (wk == 0) {
            const size_t base = ((size_t)split * tiles + tile_id) * (BM * BN);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int ml = (wm * MT + mt) * 16 + 4 * g + i;
                        const int nl = (wn * NT + nt) * 16 + r;
                        buf_store_x1_coherent(rp, (uint32_t)((base + ml * BN + nl) * 4), (uint32_t)acc[mt][nt][i]);
                    }
        }
        if (p.defer_reduce) return;
        if (!split_ticket(&p.tickets[tile_id], (unsigned)p.splits, &last_flag)) return;
        if (wk != 0) return;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int ml = (wm * MT + mt) * 16 + 4 * g + i;
                    const int nl = (wn * NT + nt) * 16 + r;
                    int32_t s = 0;
                    for (int sp = 0; sp < p.splits; ++sp)
                        s += (int32_t)buf_load_x1_coherent(
                            rp, (uint32_t)((((size_t)sp * tiles + tile_id) * (BM * BN) + ml * BN + nl) * 4));
                    acc[mt][nt][i] = s;
                }
    } else if (wk != 0) {
        return;
    }

#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + (wm * MT + mt) * 16 + 4 * g + i;
                const int n = n0 + (wn * NT + nt) * 16 + r;
                if (m < p.M && n < p.N) {
                    if constexpr (EPI == 0) {
                        static_cast<int32_t*>(p.C)[(size_t)m * p.ldc + n] = acc[mt][nt][i];
                    } else {
                        static_cast<float*>(p.C)[(size_t)m * p.ldc + n] = (float)acc[mt][nt][i] * p.scale[n];
                    }
                }
            }
}

// ---------------------------------------------------------------- launch table
// {MT, NT, WM, WN, KW}
static const S8Config kS8Configs[] = {
    {1, 1, 1, 4, 2},  // 0: M <= 16, 16 x 64 tiles, 8 waves
    {1, 2, 1, 2, 4},  // 1: M <= 16, 16 x 64 tiles, k split over 4 waves
    {2, 2, 2, 2, 1},  // 2: 64 x 64 tiles
    {2, 2, 4, 2, 1},  // 3: 128 x 64 tiles
    {2, 4, 4, 1, 1},  // 4: 128 x 64 tiles, 4 waves
};

int s8_config_count() { return (int)(sizeof(kS8Configs) / sizeof(kS8Configs[0])); }
S8Config s8_config(int idx) { return kS8Configs[idx]; }

template <int EPI, int AL>
static hipError_t launch_s8_cfg(int cfg, dim3 grid, const S8Args& a, hipStream_t s) {
    switch (cfg) {
        case 0: hipLaunchKernelGGL((dnnopt_mfma_s8<1, 1, 1, 4, 2, EPI, AL>), grid, dim3(512), 0, s, a); break;
        case 1: hipLaunchKernelGGL((dnnopt_mfma_s8<1, 2, 1, 2, 4, EPI, AL>), grid, dim3(512), 0, s, a); break;
        case 2: hipLaunchKernelGGL((dnnopt_mfma_s8<2, 2, 2, 2, 1, EPI, AL>), grid, dim3(256), 0, s, a); break;
        case 3: hipLaunchKernelGGL((dnnopt_mfma_s8<2, 2, 4, 2, 1, EPI, AL>), grid, dim3(512), 0, s, a); break;
        case 4: hipLaunchKernelGGL((dnnopt_mfma_s8<2, 4, 4, 1, 1, EPI, AL>), grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_mfma_s8(int cfg_idx, int epi, int aligned, dim3 grid, const S8Args& a, hipStream_t s) {
    if (epi) return aligned ? launch_s8_cfg<1, 1>(cfg_idx, grid, a, s) : launch_s8_cfg<1, 0>(cfg_idx, grid, a, s);
    return aligned ? launch_s8_cfg<0, 1>(cfg_idx, grid, a, s) : launch_s8_cfg<0, 0>(cfg_idx, grid, a, s);
}

}  // namespace dnnopt_hip
