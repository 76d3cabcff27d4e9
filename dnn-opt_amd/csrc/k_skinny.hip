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
// LDS, workgroups through a workspace by the last workgroup to arrive.  The
// summation order is therefore fixed for a given launch shape and the result
// is bit-reproducible.
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

template <int MODE>
__device__ __forceinline__ float load_a(const void* A, size_t idx) {
    if constexpr (MODE == kSkinnyBF16) {
        return bf16_to_f32(static_cast<const uint16_t*>(A)[idx]);
    } else if constexpr (MODE == kSkinnyF2B) {
        return round_bf16(static_cast<const float*>(A)[idx]);
    } else {
        return static_cast<const float*>(A)[idx];
    }
}

template <int MR, int NW, int MODE>
__global__ __launch_bounds__(NW * 64) void dnnopt_skinny(SkinnyArgs p) {
    constexpr int VEC = SkinnyTraits<MODE>::VEC;
    constexpr int ES = SkinnyTraits<MODE>::ES;
    constexpr int TW = 64 * VEC;
    constexpr int U = kSkinnyUnroll;
    constexpr int NT = NW * 64;
    // LDS reduction in passes of G rows, at most 32 KiB of LDS per pass.
    constexpr int GMAX = 32768 / (NW * TW * 4) > 0 ? 32768 / (NW * TW * 4) : 1;
    constexpr int G = MR < GMAX ? MR : GMAX;
    constexpr int P = (MR + G - 1) / G;
    constexpr int I = (G * TW + NT - 1) / NT;

    __shared__ float red[NW * G * TW];
    __shared__ int last_flag;

    const int lane = lane_id();
    const int w = wave_id();
    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int col0 = tile * TW;
    const long long chunks = (long long)p.splits * NW;
    const long long cw = (long long)split * NW + w;
    const int k_lo = (int)(((long long)p.K * cw) / chunks);
    const int k_hi = (int)(((long long)p.K * (cw + 1)) / chunks);
    const int kb = (int)(((long long)p.K * ((long long)split * NW)) / chunks);

    // Buffer range: from row kb, column col0 to the last element of B.
    const char* bbase = static_cast<const char*>(p.B) + ((size_t)kb * p.ldb + col0) * ES;
    const size_t remain = ((size_t)(p.K - 1 - kb) * p.ldb + (size_t)(p.N - col0)) * ES;
    const uint32_t nrec = remain > 0x7FFFFFFFull ? 0x7FFFFFFFu : (uint32_t)remain;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(bbase, nrec);
    const uint32_t rowbytes = (uint32_t)p.ldb * ES;
    const uint32_t lane_off = (uint32_t)lane * VEC * ES;

    float acc[MR][VEC];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[m][v] = 0.0f;

    int k = k_lo;
    for (; k + U <= k_hi; k += U) {
        u32x4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) raw[u] = buf_load_x4(rs, (uint32_t)(k + u - kb) * rowbytes + lane_off);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float bv[VEC];
            unpack_b<MODE>(raw[u], bv);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float a = load_a<MODE>(p.A, (size_t)m * p.a_sm + (size_t)(k + u) * p.a_sk);
#pragma unroll
                for (int v = 0; v < VEC; ++v) acc[m][v] = __builtin_fmaf(a, bv[v], acc[m][v]);
            }
        }
    }
    for (; k < k_hi; ++k) {
        const u32x4 raw = buf_load_x4(rs, (uint32_t)(k - kb) * rowbytes + lane_off);
        float bv[VEC];
        unpack_b<MODE>(raw, bv);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float a = load_a<MODE>(p.A, (size_t)m * p.a_sm + (size_t)k * p.a_sk);
#pragma unroll
            for (int v = 0; v < VEC; ++v) acc[m][v] = __builtin_fmaf(a, bv[v], acc[m][v]);
        }
    }

    // Reduce the NW waves of this workgroup, waves in ascending order.
    float out[P][I];
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
        for (int i = 0; i < I; ++i) {
            const int idx = (int)threadIdx.x + i * NT;
            const int g = idx / TW;
            const int col = idx % TW;
            float s = 0.0f;
            if (idx < G * TW && pass * G + g < MR) {
                s = red[g * TW + col];
#pragma unroll
                for (int w2 = 1; w2 < NW; ++w2) s += red[(w2 * G + g) * TW + col];
            }
            out[pass][i] = s;
        }
    }

    if (p.splits == 1) {
#pragma unroll
        for (int pass = 0; pass < P; ++pass)
#pragma unroll
            for (int i = 0; i < I; ++i) {
                const int idx = (int)threadIdx.x + i * NT;
                const int m = pass * G + idx / TW;
                const int n = col0 + idx % TW;
                if (idx < G * TW && m < MR && n < p.N) {
                    float* c = p.C + (size_t)m * p.ldc + n;
                    *c = epilogue(out[pass][i], p.alpha, p.beta, c);
                }
            }
        return;
    }

    // Split-k: publish this workgroup's partial sums, last arrival reduces.
    float* mine = p.part + (size_t)split * MR * p.ncols_pad;
#pragma unroll
    for (int pass = 0; pass < P; ++pass)
#pragma unroll
        for (int i = 0; i < I; ++i) {
            const int idx = (int)threadIdx.x + i * NT;
            const int m = pass * G + idx / TW;
            if (idx < G * TW && m < MR) mine[(size_t)m * p.ncols_pad + col0 + idx % TW] = out[pass][i];
        }
    if (!split_ticket(&p.tickets[tile], (unsigned)p.splits, &last_flag)) return;

#pragma unroll
    for (int pass = 0; pass < P; ++pass)
#pragma unroll
        for (int i = 0; i < I; ++i) {
            const int idx = (int)threadIdx.x + i * NT;
            const int m = pass * G + idx / TW;
            const int n = col0 + idx % TW;
            if (idx < G * TW && m < MR && n < p.N) {
                const float* src = p.part + (size_t)m * p.ncols_pad + n;
                const size_t stride = (size_t)MR * p.ncols_pad;
                float s = src[0];
                for (int sp = 1; sp < p.splits; ++sp) s += src[sp * stride];
                float* c = p.C + (size_t)m * p.ldc + n;
                *c = epilogue(s, p.alpha, p.beta, c);
            }
        }
}

// ---------------------------------------------------------------- launch table
template <int MODE, int NW>
static hipError_t launch_mr(int mr, dim3 grid, const SkinnyArgs& a, hipStream_t s) {
    dim3 block(NW * 64);
    switch (mr) {
        case 1: hipLaunchKernelGGL((dnnopt_skinny<1, NW, MODE>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((dnnopt_skinny<2, NW, MODE>), grid, block, 0, s, a); break;
        case 3: hipLaunchKernelGGL((dnnopt_skinny<3, NW, MODE>), grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL((dnnopt_skinny<4, NW, MODE>), grid, block, 0, s, a); break;
        case 5: hipLaunchKernelGGL((dnnopt_skinny<5, NW, MODE>), grid, block, 0, s, a); break;
        case 6: hipLaunchKernelGGL((dnnopt_skinny<6, NW, MODE>), grid, block, 0, s, a); break;
        case 7: hipLaunchKernelGGL((dnnopt_skinny<7, NW, MODE>), grid, block, 0, s, a); break;
        case 8: hipLaunchKernelGGL((dnnopt_skinny<8, NW, MODE>), grid, block, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int MODE>
static hipError_t launch_nw(int mr, int nw, dim3 grid, const SkinnyArgs& a, hipStream_t s) {
    switch (nw) {
        case 4: return launch_mr<MODE, 4>(mr, grid, a, s);
        case 8: return launch_mr<MODE, 8>(mr, grid, a, s);
        case 16: return launch_mr<MODE, 16>(mr, grid, a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_skinny(int mode, int mr, int nw, dim3 grid, const SkinnyArgs& a, hipStream_t s) {
    switch (mode) {
        case kSkinnyF32: return launch_nw<kSkinnyF32>(mr, nw, grid, a, s);
        case kSkinnyBF16: return launch_nw<kSkinnyBF16>(mr, nw, grid, a, s);
        case kSkinnyF2B: return launch_nw<kSkinnyF2B>(mr, nw, grid, a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dnnopt_hip
