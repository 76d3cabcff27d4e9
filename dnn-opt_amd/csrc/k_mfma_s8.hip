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
#include <type_traits>

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
// STREAM: rows read once (B), aligned loads carry the non-temporal hint.
template <int AL, bool STREAM = false>
__device__ __forceinline__ i32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (AL && STREAM) return __builtin_bit_cast(i32x4, buf_load_x4_stream(r, off));
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

    // Operands of one 256-byte k block, loaded one block ahead of the MFMAs
    // that consume them (two register sets, alternating).
    // blk >= b_hi: a block past this wave's range, loaded only to keep the
    // loop free of conditional loads -- every offset is out of range, so it
    // reads nothing from memory.
    auto load_blk = [&](int blk, i32x4 (&a)[MT][4], i32x4 (&b)[NT][4]) {
        const bool live = blk < b_hi;
        const int kbase = blk * 256 + 16 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kc = kbase + 64 * j;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const uint32_t off = (live && kc < p.K && arow[mt] != kOobOffset) ? arow[mt] + kc : kOobOffset;
                a[mt][j] = load16<AL>(ra, off);
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t off = (live && brow[nt] != kOobOffset) ? brow[nt] + kc : kOobOffset;
                b[nt][j] = load16<AL, true>(rb, off);
            }
        }
    };
    auto compute_blk = [&](int blk, i32x4 (&a)[MT][4], i32x4 (&b)[NT][4]) {
        if (blk * 256 + 256 > p.K) {
            const int kbase = blk * 256 + 16 * g;
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
    };
    i32x4 a0[MT][4], b0[NT][4], a1[MT][4], b1[NT][4];
    if (b_lo < b_hi) load_blk(b_lo, a0, b0);
    int blk = b_lo;
    for (; blk + 2 <= b_hi; blk += 2) {
        load_blk(blk + 1, a1, b1);
        compute_blk(blk, a0, b0);
        // The block after this pair (out of range at the end: no traffic).
        load_blk(blk + 2, a0, b0);
        compute_blk(blk + 1, a1, b1);
    }
    if (blk < b_hi) compute_blk(blk, a0, b0);

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
            p.part, range31((size_t)p.splits * tiles * BM * BN * 4));
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
        if (!split_ticket(&p.tickets[(size_t)tile_id * kTicketStride], (unsigned)p.splits, &last_flag)) return;
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

    const float dq = EPI == 1 && p.amax ? dyn_dequant_scale(p.amax, p.alpha) : 0.0f;
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
                        float* c = static_cast<float*>(p.C) + (size_t)m * p.ldc + n;
                        *c = s8_out(acc[mt][nt][i], n, p.scale, p.amax, dq, p.beta, c);
                    }
                }
            }
}

// ---------------------------------------------------------------- LDS-staged
// Both operands are k-contiguous, so A and B tiles are staged in LDS the same
// way: k-blocks of 128 bytes, one LDS row of 128 bytes per operand row, the
// 16-byte chunks of a row XOR-swizzled by the row index so that the 16 rows
// read by one MFMA operand fall in different banks.  Each operand row is
// read from global memory once per workgroup (the register kernel reads it
// once per wave), the next D - 1 blocks are in flight while one is consumed,
// and C is written through LDS in whole rows.
namespace {
__device__ __forceinline__ int swz16(int row, int c) { return c ^ (row & 7); }
}  // namespace

// QB = 1 (fp32-API gemm_int8; 32 x 128 B blocks, 256 threads): B is the
// fp32 K x N matrix p.Bf.  Thread t loads 4 columns (4 cg .. 4 cg + 3, cg = t
// mod 8) of 4 consecutive k rows (4 kq .. 4 kq + 3, kq = t / 8) with four
// 16-byte loads (a wave's load covers 8 rows x 128 bytes), quantizes them
// when the stage is written, and stores each column's 4 k bytes as one dword
// of that column's LDS row: the LDS layout and the MFMAs are those of int8
// B.  Columns past N hold whatever the loads return; their outputs are not
// stored.
template <int MT, int NT, int WM, int WN, int D, int EPI, int BK = 128, int QB = 0>
__global__ __launch_bounds__(WM* WN * 64) void dnnopt_s8_lds(S8Args p) {
    constexpr int BM = WM * MT * 16, BN = WN * NT * 16;  // BK: bytes (= k) per block
    constexpr int NTH = WM * WN * 64;
    constexpr int ROWB = BK;
    constexpr int CPR = ROWB / 16;  // 16-byte chunks per LDS row
    constexpr int KK = BK / 64;     // MFMA k-steps per block
    constexpr int A_BYTES = BM * ROWB, STAGE = (BM + BN) * ROWB;
    constexpr int ACH = BM * CPR, BCH = BN * CPR;  // 16-byte chunks per block
    constexpr int AU = (ACH + NTH - 1) / NTH, BU = (BCH + NTH - 1) / NTH;
    constexpr int CROW = BN + 4;
    constexpr int LDS_BYTES = 2 * STAGE > BM * CROW * 4 ? 2 * STAGE : BM * CROW * 4;
    __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];

    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
    const int w = wave_id();
    const int wn = w % WN, wm = w / WN;
    const int t = (int)threadIdx.x;
    const TileXY tile = xcd_tile((int)blockIdx.x, p.tiles_n, p.tiles_m);
    if (!tile.ok) return;
    const int tile_n = tile.n, tile_m = tile.m, split = blockIdx.z;
    const int m0 = tile_m * BM, n0 = tile_n * BN;

    const int nblk = (p.K + BK - 1) / BK;
    const int b_lo = (int)(((long long)nblk * split) / p.splits);
    const int b_hi = (int)(((long long)nblk * (split + 1)) / p.splits);

    // Ranges end at the last byte of each operand, rounded up to a dword.
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc(p.A + (size_t)m0 * p.lda,
                  range31(((size_t)(p.M - 1 - m0) * p.lda + p.K + 3) & ~(size_t)3));
    const __amdgpu_buffer_rsrc_t rb =
        QB ? make_rsrc(p.Bf + n0, range31(((size_t)(p.K - 1) * p.ldb + (p.N - n0)) * 4))
           : make_rsrc(p.B + (size_t)n0 * p.ldb, range31(((size_t)(p.N - 1 - n0) * p.ldb + p.K + 3) & ~(size_t)3));
    float inv_b = 0.0f;
    if constexpr (QB) {
        unsigned ma, mb;
        wave_maxima(p.qpart, p.ga, p.gb, &ma, &mb);
        inv_b = 1.0f / quant_scale_bits(mb);
    }

    uint32_t a_off[AU], b_off[BU];
    int a_lds[AU], b_lds[BU], a_c[AU];
#pragma unroll
    for (int i = 0; i < AU; ++i) {
        const int idx = t + i * NTH, row = idx / CPR, c = idx % CPR;
        const bool ok = (ACH % NTH == 0 || idx < ACH) && m0 + row < p.M;
        a_off[i] = ok ? (uint32_t)row * p.lda + 16 * c : kOobOffset;
        a_lds[i] = row * ROWB + swz16(row, c) * 16;
        a_c[i] = 16 * c;
    }
#pragma unroll
    for (int i = 0; i < BU; ++i) {
        const int idx = t + i * NTH;
        // QB: consecutive threads take consecutive columns of one k-chunk.
        const int row = QB ? idx % BN : idx / CPR, c = QB ? idx / BN : idx % CPR;
        const bool ok = (BCH % NTH == 0 || idx < BCH) && n0 + row < p.N;
        b_off[i] = ok ? (uint32_t)row * p.ldb + 16 * c : kOobOffset;
        b_lds[i] = A_BYTES + row * ROWB + swz16(row, c) * 16;
    }
    static_assert(!QB || (BN == 32 && BK == 128 && NTH == 256), "fp32 B staging: 32 x 128 blocks, 256 threads");
    const int q_cg = t % 8, q_kq = t / 8;
    const uint32_t q_off = ((uint32_t)(4 * q_kq) * (uint32_t)p.ldb + 4 * q_cg) * 4u;
    int q_lds[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int row = 4 * q_cg + e, c = q_kq / 4;
        q_lds[e] = A_BYTES + row * ROWB + swz16(row, c) * 16 + 4 * (q_kq % 4);
    }

    i32x4 sa[D][AU], sb[D][BU];
    f32x4 sbq[D][QB ? 4 : 1];
    auto load_stage = [&](int blk, int slot) {
        const uint32_t k0 = (uint32_t)(blk < b_hi ? blk : b_hi - 1) * BK;
#pragma unroll
        for (int i = 0; i < AU; ++i) sa[slot][i] = __builtin_bit_cast(i32x4, buf_load_x4(ra, a_off[i] + k0));
        if constexpr (QB) {
            const uint32_t kb = k0 * (uint32_t)p.ldb * 4u + q_off;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                sbq[slot][j] = __builtin_bit_cast(f32x4, buf_load_x4(rb, kb + (uint32_t)j * (uint32_t)p.ldb * 4u));
        } else {
#pragma unroll
            for (int i = 0; i < BU; ++i) sb[slot][i] = __builtin_bit_cast(i32x4, buf_load_x4(rb, b_off[i] + k0));
        }
    };
    auto write_stage = [&](int slot, int buf, int blk) {
        char* St = lds + buf * STAGE;
        // Bytes of A past K (the next row's data) are zeroed in the block
        // that holds k = K - 1, which zeroes their products whatever B holds.
        const bool tail = (blk + 1) * BK > p.K;
#pragma unroll
        for (int i = 0; i < AU; ++i) {
            i32x4 v = sa[slot][i];
            if (tail) v = mask_chunk(v, p.K - (blk * BK + a_c[i]));
            if (ACH % NTH == 0 || t + i * NTH < ACH) *reinterpret_cast<i32x4*>(St + a_lds[i]) = v;
        }
        if constexpr (QB) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                *reinterpret_cast<uint32_t*>(St + q_lds[e]) =
                    (uint32_t)(quant_s8(sbq[slot][0][e], inv_b) & 0xFF) |
                    (uint32_t)(quant_s8(sbq[slot][1][e], inv_b) & 0xFF) << 8 |
                    (uint32_t)(quant_s8(sbq[slot][2][e], inv_b) & 0xFF) << 16 |
                    (uint32_t)quant_s8(sbq[slot][3][e], inv_b) << 24;
        } else {
#pragma unroll
            for (int i = 0; i < BU; ++i)
                if (BCH % NTH == 0 || t + i * NTH < BCH) *reinterpret_cast<i32x4*>(St + b_lds[i]) = sb[slot][i];
        }
    };

    int a_rd[KK][MT], b_rd[KK][NT];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        const int c = kk * 4 + g;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int row = (wm * MT + mt) * 16 + r;
            a_rd[kk][mt] = row * ROWB + swz16(row, c) * 16;
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int row = (wn * NT + nt) * 16 + r;
            b_rd[kk][nt] = A_BYTES + row * ROWB + swz16(row, c) * 16;
        }
    }
    i32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = i32x4{0, 0, 0, 0};
    auto compute = [&](int buf) {
        const char* St = lds + buf * STAGE;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            i32x4 af[MT], bfr[NT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) af[mt] = *reinterpret_cast<const i32x4*>(St + a_rd[kk][mt]);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) bfr[nt] = *reinterpret_cast<const i32x4*>(St + b_rd[kk][nt]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[mt], bfr[nt], acc[mt][nt], 0, 0, 0);
        }
    };

    const int nb = b_hi - b_lo;
    if (nb > 0) {
#pragma unroll
        for (int d = 0; d < D; ++d) load_stage(b_lo + d, d);
        write_stage(0, 0, b_lo);
    }
    __syncthreads();
    int i0 = 0;
    for (; i0 + D <= nb; i0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int i = i0 + d;
            load_stage(b_lo + i + D, d);
            compute(i & 1);
            write_stage((d + 1) % D, (i + 1) & 1, b_lo + i + 1);
            __syncthreads();
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const int i = i0 + d;
        if (i < nb) {
            compute(i & 1);
            write_stage((d + 1) % D, (i + 1) & 1, b_lo + i + 1);
            __syncthreads();
        }
    }

    // Stage the accumulators in LDS (row-major tile), then write whole rows.
    int32_t* Cs = reinterpret_cast<int32_t*>(lds);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                Cs[((wm * MT + mt) * 16 + 4 * g + i) * CROW + (wn * NT + nt) * 16 + r] = acc[mt][nt][i];
    __syncthreads();
    constexpr int Q4 = BN / 4;
    if (p.splits > 1) {
        // Exact int32 partial tile [split][tile][BM * BN], summed by the
        // reduce kernel that follows.
        const int tiles = p.tiles_n * p.tiles_m;
        const int tile_id = tile_m * p.tiles_n + tile_n;
        int32_t* part = p.part + ((size_t)split * tiles + tile_id) * (BM * BN);
        for (int e = t; e < BM * Q4; e += NTH) {
            const int row = e / Q4, q = e % Q4;
            *reinterpret_cast<i32x4*>(part + row * BN + 4 * q) = *reinterpret_cast<const i32x4*>(&Cs[row * CROW + 4 * q]);
        }
        return;
    }
    const size_t esz = EPI == 0 ? 4 : 4;
    const float dq = EPI == 1 && p.amax ? dyn_dequant_scale(p.amax, p.alpha) : 0.0f;
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(static_cast<char*>(p.C) + ((size_t)m0 * p.ldc + n0) * esz,
                  range31(((size_t)(p.M - 1 - m0) * p.ldc + (p.N - n0)) * esz));
    for (int e = t; e < BM * Q4; e += NTH) {
        const int row = e / Q4, q = e % Q4;
        const int m = m0 + row, n = n0 + 4 * q;
        if (m >= p.M || n >= p.N) continue;
        const i32x4 v = *reinterpret_cast<const i32x4*>(&Cs[row * CROW + 4 * q]);
        const uint32_t off = ((uint32_t)row * p.ldc + 4 * q) * 4u;
        if (n + 4 <= p.N) {
            u32x4 out;
            if constexpr (EPI == 0) {
                out = __builtin_bit_cast(u32x4, v);
            } else {
                float* c = static_cast<float*>(p.C) + (size_t)m * p.ldc + n;
#pragma unroll
                for (int k = 0; k < 4; ++k) out[k] = as_u32(s8_out(v[k], n + k, p.scale, p.amax, dq, p.beta, c + k));
            }
            __builtin_amdgcn_raw_buffer_store_b128(out, rc, off, 0, 0);
        } else {
            for (int k = 0; k < p.N - n; ++k) {
                if constexpr (EPI == 0) {
                    static_cast<int32_t*>(p.C)[(size_t)m * p.ldc + n + k] = v[k];
                } else {
                    float* c = static_cast<float*>(p.C) + (size_t)m * p.ldc + n + k;
                    *c = s8_out(v[k], n + k, p.scale, p.amax, dq, p.beta, c);
                }
            }
        }
    }
}

// ---------------------------------------------------------------- LDS DMA
// The LDS-staged tile of above with both operands copied into LDS by the
// vector memory unit itself (buffer_load_dwordx4 ... lds: lane l of a wave
// load writes its 16 bytes at the wave's LDS address + 16 l), so no block
// passes through registers and no LDS store waits on them.  S stages, one
// __shared__ array each, blocks S - 1 ahead; per block one wait for this
// wave's own copies of the next block, one barrier, the copy of block
// i + S - 1 into the stage block i - 1 left, then block i's fragments.
// LDS rows are BK bytes, chunk c of row r at slot c ^ (r mod 16) (mod 8 for
// 8-chunk rows): the wave load that fills a 1 KB span of a stage reads, for
// its lane at slot s of row r, global chunk s ^ swz(r) of that row, so its
// lanes still read whole rows of 128 / 256 bytes, and the 16 rows an MFMA
// operand reads fall in 16 different bank groups.  Bytes of A past K are
// zeroed in registers after the fragment read.
template <int CPR>
__device__ __forceinline__ int dma_swz(int row, int c) { return c ^ (row & (CPR >= 16 ? 15 : CPR - 1)); }

template <int MT, int NT, int WM, int WN, int NS, int EPI, int BK>
__global__ __launch_bounds__(WM* WN * 64) void dnnopt_s8_dma(S8Args p) {
    constexpr int BM = WM * MT * 16, BN = WN * NT * 16;
    constexpr int NW = WM * WN;
    constexpr int CPR = BK / 16;  // 16-byte chunks per LDS row
    constexpr int KK = BK / 64;   // MFMA k-steps per block
    constexpr int A_BYTES = BM * BK, STAGE = (BM + BN) * BK;
    static_assert(NS >= 2 && NS <= 4, "2 to 4 stages");
    static_assert(A_BYTES % 1024 == 0 && STAGE % (NW * 1024) == 0, "whole 1 KB wave loads, as many per wave");
    constexpr int IPW = STAGE / 1024 / NW;  // wave loads per wave and block
    __shared__ __attribute__((aligned(1024))) char st0[STAGE];
    __shared__ __attribute__((aligned(1024))) char st1[STAGE];
    __shared__ __attribute__((aligned(1024))) char st2[NS > 2 ? STAGE : 16];
    __shared__ __attribute__((aligned(1024))) char st3[NS > 3 ? STAGE : 16];
    auto stage = [&](int i) -> char* { return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : st3; };

    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
    const int w = wave_id();
    const int wn = w % WN, wm = w / WN;
    const TileXY tile = xcd_tile((int)blockIdx.x, p.tiles_n, p.tiles_m);
    if (!tile.ok) return;
    const int tile_n = tile.n, tile_m = tile.m, split = blockIdx.z;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int nblk = (p.K + BK - 1) / BK;
    const int b_lo = (int)(((long long)nblk * split) / p.splits);
    const int b_hi = (int)(((long long)nblk * (split + 1)) / p.splits);
    const int nb = b_hi - b_lo;

    // Ranges end at the last byte of each operand, rounded up to a dword;
    // rows past M / N start at kOobOffset and read zero.
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc(p.A + (size_t)m0 * p.lda, range31(((size_t)(p.M - 1 - m0) * p.lda + p.K + 3) & ~(size_t)3));
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(p.B + (size_t)n0 * p.ldb, range31(((size_t)(p.N - 1 - n0) * p.ldb + p.K + 3) & ~(size_t)3));
    uint32_t goff[IPW];
    bool gb[IPW];
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
        const int q = (w * IPW + j) * 1024 + 16 * lane;  // byte of the stage this lane fills
        const bool isb = (w * IPW + j) * 1024 >= A_BYTES;
        const int qq = isb ? q - A_BYTES : q;
        const int row = qq / BK, c = dma_swz<CPR>(row, (qq % BK) / 16);
        const bool ok = isb ? n0 + row < p.N : m0 + row < p.M;
        goff[j] = ok ? (uint32_t)row * (uint32_t)(isb ? p.ldb : p.lda) + 16u * c : kOobOffset;
        gb[j] = isb;
    }
    // Block `blk` of this split into stage `st`; blocks past the split read
    // nothing (out-of-range offsets) but are issued, so every wave's count of
    // outstanding loads per block is the same.
    auto dma = [&](int st, int blk) {
        const uint32_t k0 = blk < b_hi ? (uint32_t)blk * BK : kOobOffset;
        char* base = stage(st) + w * IPW * 1024;
#pragma unroll
        for (int j = 0; j < IPW; ++j)
            lds_dma16(gb[j] ? rb : ra, base + j * 1024, goff[j] + k0);
    };

    int a_rd[KK][MT], b_rd[KK][NT];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        const int c = kk * 4 + g;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int row = (wm * MT + mt) * 16 + r;
            a_rd[kk][mt] = row * BK + dma_swz<CPR>(row, c) * 16;
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int row = (wn * NT + nt) * 16 + r;
            b_rd[kk][nt] = A_BYTES + row * BK + dma_swz<CPR>(row, c) * 16;
        }
    }
    // Two accumulator sets (even and odd k-steps) halve the dependent MFMA
    // chain of a block; integer sums, so the split does not change C.
    constexpr int AS = KK >= 2 ? 2 : 1;
    i32x4 acc[AS][MT][NT];
#pragma unroll
    for (int a = 0; a < AS; ++a)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[a][mt][nt] = i32x4{0, 0, 0, 0};
    // TAIL: the block holds k = K - 1 (compiled separately, so the common
    // block has no branch between its fragment reads).
    auto compute_blk = [&](int st, int blk, auto tail_tag) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        const char* St = stage(st);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            i32x4 af[MT], bfr[NT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) af[mt] = *reinterpret_cast<const i32x4*>(St + a_rd[kk][mt]);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) bfr[nt] = *reinterpret_cast<const i32x4*>(St + b_rd[kk][nt]);
            if constexpr (TAIL) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) af[mt] = mask_chunk(af[mt], p.K - (blk * BK + kk * 64 + 16 * g));
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[kk % AS][mt][nt] =
                        __builtin_amdgcn_mfma_i32_16x16x64_i8(af[mt], bfr[nt], acc[kk % AS][mt][nt], 0, 0, 0);
        }
    };
    auto compute = [&](int st, int blk) {
        if ((blk + 1) * BK > p.K) compute_blk(st, blk, std::true_type{});
        else compute_blk(st, blk, std::false_type{});
    };
    auto iter = [&](int i, int st) {
        // This wave's copies of block i are done (the NS - 2 later blocks'
        // may still be in flight); after the barrier every wave's are, and
        // every wave has consumed block i - 1's fragments.
        wait_vmcnt<(NS - 2) * IPW>();
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        dma((st + NS - 1) % NS, b_lo + i + NS - 1);
        compute(st, b_lo + i);
    };

    if (nb > 0) {
#pragma unroll
        for (int s = 0; s < NS - 1; ++s) dma(s, b_lo + s);
    }
    int i0 = 0;
    for (; i0 + NS <= nb; i0 += NS) {
#pragma unroll
        for (int s = 0; s < NS; ++s) iter(i0 + s, s);
    }
#pragma unroll
    for (int s = 0; s < NS; ++s)
        if (i0 + s < nb) iter(i0 + s, s);
    // Every copy has landed before the workgroup ends (the last ones read
    // nothing but still write their stage).
    wait_vmcnt<0>();

    i32x4 res[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            res[mt][nt] = acc[0][mt][nt];
            if constexpr (AS > 1) res[mt][nt] += acc[1][mt][nt];
        }
    // Lane element i of sub-tile (mt, nt): row 4g + i, column r.
    const int tiles = p.tiles_n * p.tiles_m;
    const int tile_id = tile_m * p.tiles_n + tile_n;
    const float dq = EPI == 1 && p.amax ? dyn_dequant_scale(p.amax, p.alpha) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int nl = (wn * NT + nt) * 16 + r, n = n0 + nl;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ml = (wm * MT + mt) * 16 + 4 * g + i, m = m0 + ml;
                if (p.splits > 1) {
                    // Exact int32 partial tile [split][tile][BM * BN], summed
                    // by the reduce kernel that follows.
                    p.part[((size_t)split * tiles + tile_id) * (BM * BN) + ml * BN + nl] = res[mt][nt][i];
                } else if (m < p.M && n < p.N) {
                    if constexpr (EPI == 0) {
                        static_cast<int32_t*>(p.C)[(size_t)m * p.ldc + n] = res[mt][nt][i];
                    } else {
                        float* c = static_cast<float*>(p.C) + (size_t)m * p.ldc + n;
                        *c = s8_out(res[mt][nt][i], n, p.scale, p.amax, dq, p.beta, c);
                    }
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
    {1, 1, 1, 1, 8},  // 5: M <= 16, 16 x 16 tiles, k split over 8 waves
    {2, 1, 2, 2, 2},  // 6: 64 x 32 tiles, k split over 2 waves
    {2, 1, 4, 2, 1},  // 7: 128 x 32 tiles, 8 waves
    {1, 1, 4, 2, 1},  // 8: 64 x 32 tiles, 8 waves
    {1, 1, 1, 2, 4},  // 9: M <= 16, 16 x 32 tiles, k split over 4 waves
    {2, 2, 2, 2, 1, 2},  // 10: 64 x 64 through LDS
    {2, 1, 2, 2, 1, 2},  // 11: 64 x 32 through LDS
    {2, 2, 4, 2, 1, 2},  // 12: 128 x 64 through LDS, 8 waves
    {1, 1, 2, 2, 1, 3},  // 13: 32 x 32 through LDS, 3 blocks ahead
    {2, 1, 2, 4, 1, 2},  // 14: 64 x 64 through LDS, 8 waves
    {1, 1, 1, 4, 1, 3},  // 15: 16 x 64 through LDS (M <= 16)
    {2, 1, 2, 2, 1, 2, 512},  // 16: 64 x 32 through LDS, 512-byte k blocks
    {1, 1, 2, 2, 1, 2, 512},  // 17: 32 x 32 through LDS, 512-byte k blocks
    {2, 2, 2, 2, 1, 2, 512},  // 18: 64 x 64 through LDS, 512-byte k blocks
    {1, 1, 1, 4, 1, 2, 512},  // 19: 16 x 64 through LDS, 512-byte k blocks (M <= 16)
    {1, 1, 2, 2, 1, 2, 256},  // 20: 32 x 32 through LDS, 256-byte k blocks
    // LDS DMA: {MT, NT, WM, WN, 1, stages, k bytes per block}
    {1, 1, 2, 2, 1, 3, 256},  // 21: 32 x 32, 3 stages
    {1, 1, 2, 2, 1, 4, 256},  // 22: 32 x 32, 4 stages
    {2, 1, 2, 2, 1, 3, 256},  // 23: 64 x 32, 3 stages
    {1, 1, 2, 2, 1, 4, 128},  // 24: 32 x 32, 4 stages of 128-byte blocks
    {2, 2, 2, 2, 1, 3, 256},  // 25: 64 x 64, 3 stages
    {1, 1, 1, 4, 1, 4, 256},  // 26: 16 x 64, 4 stages (M <= 16)
    {2, 1, 2, 2, 1, 4, 256},  // 27: 64 x 32, 4 stages
    {2, 1, 2, 2, 1, 4, 128},  // 28: 64 x 32, 4 stages of 128-byte blocks
    {2, 2, 2, 2, 1, 4, 128},  // 29: 64 x 64, 4 stages of 128-byte blocks
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
        case 5: hipLaunchKernelGGL((dnnopt_mfma_s8<1, 1, 1, 1, 8, EPI, AL>), grid, dim3(512), 0, s, a); break;
        case 6: hipLaunchKernelGGL((dnnopt_mfma_s8<2, 1, 2, 2, 2, EPI, AL>), grid, dim3(512), 0, s, a); break;
        case 7: hipLaunchKernelGGL((dnnopt_mfma_s8<2, 1, 4, 2, 1, EPI, AL>), grid, dim3(512), 0, s, a); break;
        case 8: hipLaunchKernelGGL((dnnopt_mfma_s8<1, 1, 4, 2, 1, EPI, AL>), grid, dim3(512), 0, s, a); break;
        case 9: hipLaunchKernelGGL((dnnopt_mfma_s8<1, 1, 1, 2, 4, EPI, AL>), grid, dim3(512), 0, s, a); break;
        case 10: hipLaunchKernelGGL((dnnopt_s8_lds<2, 2, 2, 2, 2, EPI>), grid, dim3(256), 0, s, a); break;
        case 11: hipLaunchKernelGGL((dnnopt_s8_lds<2, 1, 2, 2, 2, EPI>), grid, dim3(256), 0, s, a); break;
        case 12: hipLaunchKernelGGL((dnnopt_s8_lds<2, 2, 4, 2, 2, EPI>), grid, dim3(512), 0, s, a); break;
        case 13: hipLaunchKernelGGL((dnnopt_s8_lds<1, 1, 2, 2, 3, EPI>), grid, dim3(256), 0, s, a); break;
        case 14: hipLaunchKernelGGL((dnnopt_s8_lds<2, 1, 2, 4, 2, EPI>), grid, dim3(512), 0, s, a); break;
        case 15: hipLaunchKernelGGL((dnnopt_s8_lds<1, 1, 1, 4, 3, EPI>), grid, dim3(256), 0, s, a); break;
        case 16: hipLaunchKernelGGL((dnnopt_s8_lds<2, 1, 2, 2, 2, EPI, 512>), grid, dim3(256), 0, s, a); break;
        case 17: hipLaunchKernelGGL((dnnopt_s8_lds<1, 1, 2, 2, 2, EPI, 512>), grid, dim3(256), 0, s, a); break;
        case 18: hipLaunchKernelGGL((dnnopt_s8_lds<2, 2, 2, 2, 2, EPI, 512>), grid, dim3(256), 0, s, a); break;
        case 19: hipLaunchKernelGGL((dnnopt_s8_lds<1, 1, 1, 4, 2, EPI, 512>), grid, dim3(256), 0, s, a); break;
        case 20: hipLaunchKernelGGL((dnnopt_s8_lds<1, 1, 2, 2, 2, EPI, 256>), grid, dim3(256), 0, s, a); break;
        case 21: hipLaunchKernelGGL((dnnopt_s8_dma<1, 1, 2, 2, 3, EPI, 256>), grid, dim3(256), 0, s, a); break;
        case 22: hipLaunchKernelGGL((dnnopt_s8_dma<1, 1, 2, 2, 4, EPI, 256>), grid, dim3(256), 0, s, a); break;
        case 23: hipLaunchKernelGGL((dnnopt_s8_dma<2, 1, 2, 2, 3, EPI, 256>), grid, dim3(256), 0, s, a); break;
        case 24: hipLaunchKernelGGL((dnnopt_s8_dma<1, 1, 2, 2, 4, EPI, 128>), grid, dim3(256), 0, s, a); break;
        case 25: hipLaunchKernelGGL((dnnopt_s8_dma<2, 2, 2, 2, 3, EPI, 256>), grid, dim3(256), 0, s, a); break;
        case 26: hipLaunchKernelGGL((dnnopt_s8_dma<1, 1, 1, 4, 4, EPI, 256>), grid, dim3(256), 0, s, a); break;
        case 27: hipLaunchKernelGGL((dnnopt_s8_dma<2, 1, 2, 2, 4, EPI, 256>), grid, dim3(256), 0, s, a); break;
        case 28: hipLaunchKernelGGL((dnnopt_s8_dma<2, 1, 2, 2, 4, EPI, 128>), grid, dim3(256), 0, s, a); break;
        case 29: hipLaunchKernelGGL((dnnopt_s8_dma<2, 2, 2, 2, 4, EPI, 128>), grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// 64 x 32 tiles, 3 blocks of 128 k in flight (MI355X, 128 x 4096 x 4096
// call: 2 / 3 / 4 / 6 blocks 38.6 / 38.4 / 38.8 / 39.6 us).
hipError_t launch_s8_q8b(dim3 grid, const S8Args& a, hipStream_t s) {
    hipLaunchKernelGGL((dnnopt_s8_lds<2, 1, 2, 2, 3, 1, 128, 1>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_mfma_s8(int cfg_idx, int epi, int aligned, dim3 grid, const S8Args& a, hipStream_t s) {
    if (cfg_idx < 0 || cfg_idx >= s8_config_count()) return hipErrorInvalidValue;
    if (cfg_idx >= kS8FirstLds && !aligned) return hipErrorInvalidValue;
    if (epi) return aligned ? launch_s8_cfg<1, 1>(cfg_idx, grid, a, s) : launch_s8_cfg<1, 0>(cfg_idx, grid, a, s);
    return aligned ? launch_s8_cfg<0, 1>(cfg_idx, grid, a, s) : launch_s8_cfg<0, 0>(cfg_idx, grid, a, s);
}

}  // namespace dnnopt_hip
