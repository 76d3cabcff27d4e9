// k_skinny.hip -- M = 1..8 rows against a row-major K x N operand (gfx950).
//
// Replaces the reference's M=1 GEMV (src/gemm/gemm_tiny_fp32.cpp:167-218), the
// M=2..7 wide driver (src/gemm/gemm_smallm_wide_fp32.cpp:412-490), the M=5/7
// adaptive tiles (src/gemm/gemm_adaptive_tile_fp32.cpp:664-780) and the small-M
// bf16 kernels (src/gemm/gemm_smallm_bf16.cpp:73-270).  These shapes are
// HBM-bound: the kernel reads every byte of B exactly once, with 128-bit
// loads, and keeps all M rows of a column in the registers of one lane.
//
// Lane layout: a wave covers TW = 64*VEC consecutive columns (VEC = 4 fp32 or
// 8 bf16, i.e. 16 bytes per lane per row).  The NW waves of a workgroup and
// the grid.y workgroups of a column tile each take a contiguous slice of k;
// within a lane the k of its slice are accumulated in ascending order with
// fused multiply-adds.  Slices are combined in ascending order: waves through
// LDS, workgroups through a workspace (by a separate reduce kernel, or by the
// last workgroup to arrive).  The summation order is therefore fixed for a
// given launch shape and the result is bit-reproducible.
//
// Ragged tails: B is read through a buffer descriptor whose range ends at the
// last element of B, so the loads of the last row past column N return zero;
// columns >= N of earlier rows are read (they are the next row's data) but
// never stored.  No padded copy of any operand is made.
#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

template <int MODE>
struct SkinnyTraits;
template <>
struct SkinnyTraits<kSkinnyF32> {
    static constexpr int VEC = 4, ES = 4;
};
template <>
struct SkinnyTraits<kSkinnyBF16> {
    static constexpr int VEC = 8, ES = 2;
};
template <>
struct SkinnyTraits<kSkinnyF2B> {
    static constexpr int VEC = 4, ES = 4;
};

template <int MODE>
__device__ __forceinline__ void unpack_b(const u32x4& raw, float* out) {
    if constexpr (MODE == kSkinnyBF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = bf16_lo(raw[i]);
            out[2 * i + 1] = bf16_hi(raw[i]);
        }
    } else if constexpr (MODE == kSkinnyF2B) {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = round_bf16(as_f32(raw[i]));
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = as_f32(raw[i]);
    }
}

// B is read exactly once: non-temporal loads keep it from displacing data
// that is reused (A, partial sums) in the caches.
template <int AL>
__device__ __forceinline__ u32x4 load_row(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (AL) return buf_load_x4_stream(r, off);
    return buf_load_x4_unaligned(r, off);
}

// A is only read by these kernels.  Its loads go through the constant
// address space, which tells the compiler that nothing the kernel stores
// can change them: wave-uniform A loads then stay scalar loads (s_load)
// however many stores the kernel makes elsewhere.
template <typename T>
using const_ptr = const __attribute__((address_space(4))) T*;
template <typename T>
__device__ __forceinline__ const_ptr<T> as_const(const void* p) {
    return reinterpret_cast<const_ptr<T>>(reinterpret_cast<uintptr_t>(p));
}

template <int MODE>
__device__ __forceinline__ float load_a(const void* A, size_t idx) {
    if constexpr (MODE == kSkinnyBF16) {
        return bf16_to_f32(as_const<uint16_t>(A)[idx]);
    } else if constexpr (MODE == kSkinnyF2B) {
        return round_bf16(as_const<float>(A)[idx]);
    } else {
        return as_const<float>(A)[idx];
    }
}

// A values of rows m < MR at k, k+1, ..., k+UG-1 into av[m][u].  A is tiny
// and uniform across the wave, so these are scalar loads; the layouts give
// the compiler constant offsets from one base so it merges them into wide
// s_load_dwordxN that are issued together with the B loads.
//   AK = 0: A row-major (k contiguous), 4-byte aligned rows
//   AK = 1: A stored K x M (m contiguous), fp32
//   AK = 2: any layout, element by element (bf16 rows off 4-byte alignment)
template <int MR, int UG, int MODE, int AK>
__device__ __forceinline__ void load_a_block(const SkinnyArgs& p, int k, float (&av)[MR][UG]) {
    if constexpr (AK == 0 && MODE == kSkinnyBF16) {
        static_assert(UG % 2 == 0, "bf16 A groups load whole dwords");
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const_ptr<uint32_t> ap = as_const<uint32_t>(static_cast<const uint16_t*>(p.A) + (size_t)m * p.a_sm + k);
#pragma unroll
            for (int d = 0; d < UG / 2; ++d) {
                const uint32_t w2 = ap[d];
                av[m][2 * d] = bf16_lo(w2);
                av[m][2 * d + 1] = bf16_hi(w2);
            }
        }
    } else if constexpr (AK == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const_ptr<float> ap = as_const<float>(static_cast<const float*>(p.A) + (size_t)m * p.a_sm + k);
#pragma unroll
            for (int u = 0; u < UG; ++u) av[m][u] = MODE == kSkinnyF2B ? round_bf16(ap[u]) : ap[u];
        }
    } else if constexpr (AK == 1) {
#pragma unroll
        for (int u = 0; u < UG; ++u) {
            const_ptr<float> ap = as_const<float>(static_cast<const float*>(p.A) + (size_t)(k + u) * p.a_sk);
#pragma unroll
            for (int m = 0; m < MR; ++m) av[m][u] = MODE == kSkinnyF2B ? round_bf16(ap[m]) : ap[m];
        }
    } else {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int u = 0; u < UG; ++u) av[m][u] = load_a<MODE>(p.A, (size_t)m * p.a_sm + (size_t)(k + u) * p.a_sk);
    }
}

// AL = 1: every row of B starts on a 4-byte boundary (always true for fp32);
// AL = 0: bf16 rows may start on a 2-byte boundary and are funnel-shifted.
// AK: layout of A, see load_a_block.
// U: rows of B per load block of a wave (16, or 4: on MI355X the 4-row
// blocks stream the fp32 C1 / C2 shapes 0.5-0.7 us faster with 8-wave
// workgroups, the 16-row ones suit the 4-wave groups of small problems).
template <int MR, int NW, int MODE, int AL, int AK, int U>
__global__ __launch_bounds__(NW * 64) void dnnopt_skinny(SkinnyArgs p) {
    constexpr int VEC = SkinnyTraits<MODE>::VEC;
    constexpr int ES = SkinnyTraits<MODE>::ES;
    constexpr int TW = 64 * VEC;
    constexpr int UG = U < 8 ? U : 8;  // rows per group of A values
    constexpr int NT = NW * 64;
    // LDS reduction in passes of G rows, at most 32 KiB of LDS per pass.
    constexpr int GMAX = 32768 / (NW * TW * 4) > 0 ? 32768 / (NW * TW * 4) : 1;
    constexpr int G = MR < GMAX ? MR : GMAX;
    constexpr int P = (MR + G - 1) / G;

    __shared__ float red[NW * G * TW];
    __shared__ int last_flag;

    const int lane = lane_id();
    const int w = wave_id();
    // Workgroup -> (column tile, k-split): the grid has G = gridDim.x
    // workgroups for T column tiles, and every tile gets G/T or G/T + 1
    // k-splits, so each workgroup streams (nearly) the same number of bytes
    // whatever T is.
    const SplitPos sp = split_pos((int)blockIdx.x, (int)gridDim.x, p.tiles);
    const int tile = sp.tile;
    const int split = sp.split;
    const int nsplit = sp.nsplit;
    // A tile with one k-split stores C itself, unless a reduce kernel follows:
    // that kernel then covers every column of C, so a one-split tile (G / T
    // == 1 with a remainder gives tiles of one and two splits) publishes its
    // sums like the others.
    const bool direct = nsplit == 1 && !p.defer_reduce;
    const int col0 = tile * TW;
    // k is cut into blocks of U rows; chunk cw (wave w of split `split`)
    // owns a contiguous run of blocks, so every chunk but the last starts and
    // ends on a multiple of U.
    const long long nblk = (p.K + U - 1) / U;
    const long long chunks = (long long)nsplit * NW;
    const long long cw = (long long)split * NW + w;
    const int k_lo = (int)((nblk * cw) / chunks) * U;
    const int k_hi = min(p.K, (int)((nblk * (cw + 1)) / chunks) * U);
    const int kb = (int)((nblk * ((long long)split * NW)) / chunks) * U;

    // Buffer range: from row kb, column col0 to the last element of B.
    const char* bbase = static_cast<const char*>(p.B) + ((size_t)kb * p.ldb + col0) * ES;
    const size_t remain = ((size_t)(p.K - 1 - kb) * p.ldb + (size_t)(p.N - col0)) * ES;
    uint32_t base_lo = 0;
    const __amdgpu_buffer_rsrc_t rs = rsrc_aligned(bbase, remain, &base_lo);
    const uint32_t rowbytes = (uint32_t)p.ldb * ES;
    // Lanes whose columns all lie past N read nothing (out-of-range offset)
    // instead of the next row's data.
    const uint32_t lane_off = col0 + lane * VEC < p.N ? (uint32_t)lane * VEC * ES + base_lo : kOobOffset;

    // Unsplit tiles store C directly: fetch the C values of this thread's
    // outputs now so that the read overlaps the main loop.  Output group gi
    // of a reduction pass is (row gi / QG, float4 group gi % QG).
    constexpr int QG = TW / 4;                  // float4 groups per row of the tile
    constexpr int OG = G * QG;                  // output groups per reduction pass
    constexpr int I4 = (OG + NT - 1) / NT;      // groups per thread per reduction pass
    auto group_row = [](int gi) { return gi / QG; };
    auto group_col = [](int gi) { return (gi % QG) * 4; };
    float c_pre[P][I4][4];
#pragma unroll
    for (int pass = 0; pass < P; ++pass)
#pragma unroll
        for (int i = 0; i < I4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                c_pre[pass][i][e] = 0.0f;
                const int gi = (int)threadIdx.x + i * NT;
                const int m = pass * G + group_row(gi);
                const int n = col0 + group_col(gi) + e;
                if (direct && p.beta != 0.0f && gi < OG && m < MR && n < p.N)
                    c_pre[pass][i][e] = p.C[(size_t)m * p.ldc + n];
            }

    float acc[MR][VEC];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[m][v] = 0.0f;

    auto load_block = [&](u32x4 (&raw)[U], int k0) {
#pragma unroll
        for (int u = 0; u < U; ++u) raw[u] = load_row<AL>(rs, (uint32_t)(k0 + u - kb) * rowbytes + lane_off);
    };
    auto compute_block = [&](const u32x4 (&raw)[U], int k0) {
#pragma unroll
        for (int g0 = 0; g0 < U; g0 += UG) {
            float av[MR][UG];
            load_a_block<MR, UG, MODE, AK>(p, k0 + g0, av);
#pragma unroll
            for (int u = 0; u < UG; ++u) {
                float bv[VEC];
                unpack_b<MODE>(raw[g0 + u], bv);
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int v = 0; v < VEC; ++v) acc[m][v] = __builtin_fmaf(av[m][u], bv[v], acc[m][v]);
            }
        }
    };

    int k = k_lo;
    for (; k + U <= k_hi; k += U) {
        u32x4 raw[U];
        load_block(raw, k);
        compute_block(raw, k);
    }
    for (; k < k_hi; ++k) {
        const u32x4 raw = load_row<AL>(rs, (uint32_t)(k - kb) * rowbytes + lane_off);
        float bv[VEC];
        unpack_b<MODE>(raw, bv);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float a = load_a<MODE>(p.A, (size_t)m * p.a_sm + (size_t)k * p.a_sk);
#pragma unroll
            for (int v = 0; v < VEC; ++v) acc[m][v] = __builtin_fmaf(a, bv[v], acc[m][v]);
        }
    }

    // Reduce the NW waves of this workgroup, waves in ascending order.  Each
    // thread owns float4 groups of 4 consecutive columns of one row; LDS is
    // used in passes of G rows.
    f32x4 out[P][I4];
#pragma unroll
    for (int pass = 0; pass < P; ++pass) {
        if (pass) __syncthreads();
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int m = pass * G + g;
            if (m < MR) {
                float* dst = &red[(w * G + g) * TW + lane * VEC];
#pragma unroll
                for (int v = 0; v < VEC; v += 4)
                    *reinterpret_cast<f32x4*>(dst + v) =
                        f32x4{acc[m][v], acc[m][v + 1], acc[m][v + 2], acc[m][v + 3]};
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < I4; ++i) {
            const int gi = (int)threadIdx.x + i * NT;
            const int g = group_row(gi), c4 = gi % QG;
            f32x4 sum = {0.f, 0.f, 0.f, 0.f};
            if (gi < OG && pass * G + g < MR) {
                sum = *reinterpret_cast<const f32x4*>(&red[g * TW + c4 * 4]);
#pragma unroll
                for (int w2 = 1; w2 < NW; ++w2) sum += *reinterpret_cast<const f32x4*>(&red[(w2 * G + g) * TW + c4 * 4]);
            }
            out[pass][i] = sum;
        }
    }

    if (direct) {
#pragma unroll
        for (int pass = 0; pass < P; ++pass)
#pragma unroll
            for (int i = 0; i < I4; ++i) {
                const int gi = (int)threadIdx.x + i * NT;
                const int m = pass * G + group_row(gi);
                if (gi < OG && m < MR) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int n = col0 + group_col(gi) + e;
                        if (n < p.N)
                            p.C[(size_t)m * p.ldc + n] =
                                add_bias(p.beta == 0.0f ? p.alpha * out[pass][i][e]
                                                        : __builtin_fmaf(p.alpha, out[pass][i][e],
                                                                         p.beta * c_pre[pass][i][e]),
                                         p.bias, n);
                    }
                }
            }
        return;
    }

    // Split-k: publish this workgroup's partial sums [split][MR][ncols_pad],
    // written through to memory (sc0 sc1).  The last-arriving workgroup reads
    // them without cache maintenance; for the reduce kernel that follows they
    // leave no dirty L2 lines to write back at the end of the launch (MI355X,
    // C2 step 3243 -> 3267 GB/s against plain stores).
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(p.part, range31((size_t)p.splits * MR * p.ncols_pad * 4));
#pragma unroll
    for (int pass = 0; pass < P; ++pass)
#pragma unroll
        for (int i = 0; i < I4; ++i) {
            const int gi = (int)threadIdx.x + i * NT;
            const int m = pass * G + group_row(gi);
            if (gi < OG && m < MR) {
                const uint32_t off =
                    (uint32_t)((((size_t)split * MR + m) * p.ncols_pad + col0 + group_col(gi)) * 4);
                buf_store_x4_coherent(rp, off, out[pass][i]);
            }
        }
    if (p.defer_reduce) return;
    if (!split_ticket(&p.tickets[(size_t)tile * kTicketStride], (unsigned)nsplit, &last_flag)) return;

    // Last workgroup of the tile: add the partials in split order.  Each
    // thread owns float4 outputs of the whole tile; C (for beta != 0) and a
    // chunk of CH partials per output are requested before any is used, so
    // the tail costs one memory round trip per CH splits.
    constexpr int QT = QG;
    constexpr int OUTS = MR * QT;
    constexpr int OPT = (OUTS + NT - 1) / NT;
    constexpr int CH = OPT == 1 ? 16 : 8;
    const uint32_t stride = (uint32_t)((size_t)MR * p.ncols_pad * 4);
    uint32_t off0[OPT];
    float c_old[OPT][4];
#pragma unroll
    for (int o = 0; o < OPT; ++o) {
        const int idx = (int)threadIdx.x + o * NT;
        const int m = idx / QT, n0 = col0 + (idx % QT) * 4;
        off0[o] = idx < OUTS ? (uint32_t)(((size_t)m * p.ncols_pad + n0) * 4) : kOobOffset;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            c_old[o][e] = (idx < OUTS && p.beta != 0.0f && n0 + e < p.N) ? p.C[(size_t)m * p.ldc + n0 + e] : 0.0f;
    }
    auto chunk = [&](int j, f32x4 (&v)[OPT][CH]) {
#pragma unroll
        for (int o = 0; o < OPT; ++o)
#pragma unroll
            for (int u = 0; u < CH; ++u)
                v[o][u] = buf_load_x4_coherent(rp, j + u < nsplit && off0[o] != kOobOffset
                                                       ? off0[o] + (uint32_t)(j + u) * stride
                                                       : kOobOffset);
    };
    f32x4 sum[OPT];
    {
        f32x4 v[OPT][CH];
        chunk(0, v);
#pragma unroll
        for (int o = 0; o < OPT; ++o) {
            sum[o] = v[o][0];
#pragma unroll
            for (int u = 1; u < CH; ++u)
                if (u < nsplit) sum[o] += v[o][u];
        }
    }
    for (int j = CH; j < nsplit; j += CH) {
        f32x4 v[OPT][CH];
        chunk(j, v);
#pragma unroll
        for (int o = 0; o < OPT; ++o)
#pragma unroll
            for (int u = 0; u < CH; ++u)
                if (j + u < nsplit) sum[o] += v[o][u];
    }
#pragma unroll
    for (int o = 0; o < OPT; ++o) {
        const int idx = (int)threadIdx.x + o * NT;
        const int m = idx / QT, n0 = col0 + (idx % QT) * 4;
        if (idx < OUTS) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n0 + e < p.N)
                    p.C[(size_t)m * p.ldc + n0 + e] =
                        add_bias(p.beta == 0.0f ? p.alpha * sum[o][e]
                                                : __builtin_fmaf(p.alpha, sum[o][e], p.beta * c_old[o][e]),
                                 p.bias, n0 + e);
        }
    }
}

// ---------------------------------------------------------------- launch table
template <int MODE, int NW, int AL, int AK, int U>
static hipError_t launch_mr(int mr, dim3 grid, const SkinnyArgs& a, hipStream_t s) {
    dim3 block(NW * 64);
    switch (mr) {
        case 1: hipLaunchKernelGGL((dnnopt_skinny<1, NW, MODE, AL, AK, U>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((dnnopt_skinny<2, NW, MODE, AL, AK, U>), grid, block, 0, s, a); break;
        case 3: hipLaunchKernelGGL((dnnopt_skinny<3, NW, MODE, AL, AK, U>), grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL((dnnopt_skinny<4, NW, MODE, AL, AK, U>), grid, block, 0, s, a); break;
        case 5: hipLaunchKernelGGL((dnnopt_skinny<5, NW, MODE, AL, AK, U>), grid, block, 0, s, a); break;
        case 6: hipLaunchKernelGGL((dnnopt_skinny<6, NW, MODE, AL, AK, U>), grid, block, 0, s, a); break;
        case 7: hipLaunchKernelGGL((dnnopt_skinny<7, NW, MODE, AL, AK, U>), grid, block, 0, s, a); break;
        case 8: hipLaunchKernelGGL((dnnopt_skinny<8, NW, MODE, AL, AK, U>), grid, block, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int MODE, int AL, int AK>
static hipError_t launch_nw(int mr, int nw, int unroll, dim3 grid, const SkinnyArgs& a, hipStream_t s) {
    if constexpr (MODE == kSkinnyF32) {
        if (unroll == 4) return nw == 8 ? launch_mr<MODE, 8, AL, AK, 4>(mr, grid, a, s) : hipErrorInvalidValue;
    }
    if (unroll != 16) return hipErrorInvalidValue;
    switch (nw) {
        case 4: return launch_mr<MODE, 4, AL, AK, 16>(mr, grid, a, s);
        case 8: return launch_mr<MODE, 8, AL, AK, 16>(mr, grid, a, s);
        case 16: return launch_mr<MODE, 16, AL, AK, 16>(mr, grid, a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_skinny(int mode, int mr, int nw, int unroll, int b_aligned, int a_layout, dim3 grid,
                         const SkinnyArgs& a, hipStream_t s) {
    switch (mode) {
        case kSkinnyF32:
            return a_layout == 1 ? launch_nw<kSkinnyF32, 1, 1>(mr, nw, unroll, grid, a, s)
                                 : launch_nw<kSkinnyF32, 1, 0>(mr, nw, unroll, grid, a, s);
        case kSkinnyBF16:
            if (b_aligned)
                return a_layout == 2 ? launch_nw<kSkinnyBF16, 1, 2>(mr, nw, unroll, grid, a, s)
                                     : launch_nw<kSkinnyBF16, 1, 0>(mr, nw, unroll, grid, a, s);
            return a_layout == 2 ? launch_nw<kSkinnyBF16, 0, 2>(mr, nw, unroll, grid, a, s)
                                 : launch_nw<kSkinnyBF16, 0, 0>(mr, nw, unroll, grid, a, s);
        case kSkinnyF2B: return launch_nw<kSkinnyF2B, 1, 0>(mr, nw, unroll, grid, a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dnnopt_hip
