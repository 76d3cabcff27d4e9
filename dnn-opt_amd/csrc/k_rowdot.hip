// k_rowdot.hip -- M <= 8 rows against a B stored N x K (gfx950).
//
// C[m][n] = alpha * sum_k A[m][k] * B[n][k] (+ beta * C[m][n]): every output
// is the dot product of two k-contiguous rows.  This is the layout of an
// inner product whose weights are kept output-major (oneDNN's extended_sgemm
// with transa = 'T', integration/onednn/0001-dnnopt-integration.patch:
// 316-329, and cblas_sgemm(RowMajor, NoTrans, Trans), src/blas/cblas_sgemm.cpp:
// 86-91), which the reference serves by copying B into a transposed
// temporary first.  Here B is streamed once, in place:
//   * a wave owns R consecutive rows of B; its 64 lanes cover 64 consecutive
//     16-byte chunks of a row per load (1 KiB per row and instruction), all R
//     rows' loads of U steps are issued before their FMAs;
//   * A (at most 8 short rows, re-read by every wave) is read through the
//     vector L1/L2 caches with the same chunking;
//   * the KW waves of a workgroup that share rows split the chunks of a row
//     into KW contiguous ranges;
//   * each lane accumulates its chunks in ascending k with fused
//     multiply-adds, the 64 lanes are combined by a fixed butterfly, the KW
//     waves in ascending k order through LDS -- bit-reproducible;
//   * epilogue as the reference kernels: alpha * acc (beta == 0, C not read)
//     or fma(alpha, acc, beta * C).
// Tails: elements past the end of a row (of A and of B) are masked in the
// only loop step that can hold them (the last); rows past N read as zero
// (out-of-range buffer offsets) and are not stored.
//
// int8 (MODE 2: int32 C, MODE 3: fp32 C = (float)acc * scale[n], the
// reference's s8s8s32 and column-scaled paths for M <= 4 with B stored
// N x K, src/gemm/gemm_int8_native.cpp): 16 int8 per chunk, exact int32
// accumulation with v_dot4_i32_i8 (four products per instruction, wrapping
// like the int32 accumulators of the MFMA path), the lanes and waves combined
// with integer adds.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

namespace {

constexpr int kWaves = kRowdotWaves;
constexpr int kU = 2;  // load steps in flight per wave

__device__ __forceinline__ uint32_t rec_bytes(size_t bytes) {
    bytes = (bytes + 3) & ~(size_t)3;
    return bytes > 0x7FFFFFFFull ? 0x7FFFFFFFu : (uint32_t)bytes;
}

// Element size and accumulator type per mode: 0 fp32, 1 bf16, 2 / 3 int8.
template <int MODE>
struct RowdotMode {
    static constexpr int ES = MODE >= 2 ? 1 : (MODE ? 2 : 4);
    using Acc = std::conditional_t<(MODE >= 2), int32_t, float>;
};

// Values of one 16-byte chunk as fp32: 4 floats, or 8 bf16 (MODE 1).
template <int MODE>
__device__ __forceinline__ void widen(const u32x4& v, float (&out)[MODE ? 8 : 4]) {
    if constexpr (MODE == 0) {
#pragma unroll
        for (int d = 0; d < 4; ++d) out[d] = as_f32(v[d]);
    } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            out[2 * d] = bf16_lo(v[d]);
            out[2 * d + 1] = bf16_hi(v[d]);
        }
    }
}

// Zero the elements of a chunk at or past `valid` (elements, may be <= 0).
template <int MODE>
__device__ __forceinline__ u32x4 keep_elems(u32x4 v, int valid) {
    u32x4 r;
    if constexpr (MODE >= 2) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int keep = valid - 4 * d;
            r[d] = keep >= 4 ? v[d] : (keep <= 0 ? 0u : (v[d] & ((1u << (8 * keep)) - 1u)));
        }
    } else if constexpr (MODE == 0) {
#pragma unroll
        for (int d = 0; d < 4; ++d) r[d] = d < valid ? v[d] : 0u;
    } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int keep = valid - 2 * d;
            r[d] = keep >= 2 ? v[d] : (keep == 1 ? (v[d] & 0xFFFFu) : 0u);
        }
    }
    return r;
}

// STREAM: rows read once (B), aligned loads carry the non-temporal hint.
template <int AL, bool STREAM = false>
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (AL && STREAM) return buf_load_x4_stream(r, off);
    else if constexpr (AL) return buf_load_x4(r, off);
    else return buf_load_x4_unaligned(r, off);
}

// MR rows of A, R rows of B per wave, KW waves per row group (8 / KW row
// groups per workgroup); MODE 0 fp32, 1 bf16 storage; AL: rows start on
// 4-byte boundaries.
template <int MR, int R, int KW, int MODE, int AL>
__global__ __launch_bounds__(kWaves * 64) void dnnopt_rowdot(RowdotArgs p) {
    constexpr int ES = RowdotMode<MODE>::ES;
    using Acc = typename RowdotMode<MODE>::Acc;
    constexpr int VEC = 16 / ES;  // elements per chunk
    constexpr int RG = kWaves / KW;
    __shared__ Acc red[kWaves][MR * R];

    const int lane = lane_id(), w = wave_id();
    const int wr = w / KW, kw = w % KW;
    const int n0 = ((int)blockIdx.x * RG + wr) * R;

    const char* B = static_cast<const char*>(p.B);
    const char* A = static_cast<const char*>(p.A);
    const int nrows = n0 < p.N ? p.N - n0 : 0;
    uint32_t blo = 0, alo = 0;
    // B range: rows n0 .. N-1 of this wave's group; A range: all M rows.
    const __amdgpu_buffer_rsrc_t rb =
        nrows > 0 ? (AL ? make_rsrc(B + (size_t)n0 * p.ldb * ES, rec_bytes(((size_t)(nrows - 1) * p.ldb + p.K) * ES))
                        : rsrc_aligned(B + (size_t)n0 * p.ldb * ES, ((size_t)(nrows - 1) * p.ldb + p.K) * ES, &blo))
                  : make_rsrc(B, 0);
    const __amdgpu_buffer_rsrc_t ra =
        AL ? make_rsrc(A, rec_bytes(((size_t)(p.M - 1) * p.lda + p.K) * ES))
           : rsrc_aligned(A, ((size_t)(p.M - 1) * p.lda + p.K) * ES, &alo);

    // Chunks of a row, load steps of 64 chunks, this wave's step range.
    const int nch = (p.K + VEC - 1) / VEC;
    const int J = (nch + 63) / 64;
    const int j_lo = (int)(((long long)J * kw) / KW), j_hi = (int)(((long long)J * (kw + 1)) / KW);

    uint32_t b_row[R];
#pragma unroll
    for (int r = 0; r < R; ++r) b_row[r] = r < nrows ? (uint32_t)r * p.ldb * ES + blo : kOobOffset;
    uint32_t a_row[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) a_row[m] = (uint32_t)m * p.lda * ES + alo;

    Acc acc[MR][R];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = Acc(0);

    auto step = [&](const u32x4 (&bv)[R], const u32x4 (&av)[MR]) {
        if constexpr (MODE >= 2) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int d = 0; d < 4; ++d)
                        acc[m][r] = __builtin_amdgcn_sdot4((int)av[m][d], (int)bv[r][d], acc[m][r], false);
        } else {
            float b[R][VEC];
#pragma unroll
            for (int r = 0; r < R; ++r) widen<MODE>(bv[r], b[r]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float a[VEC];
                widen<MODE>(av[m], a);
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int e = 0; e < VEC; ++e) acc[m][r] = __builtin_fmaf(a[e], b[r][e], acc[m][r]);
            }
        }
    };

    // Steps before the last one of the row hold only whole, valid chunks.
    const int j_full = j_hi < J ? j_hi : J - 1;
    int j = j_lo;
    for (; j + kU <= j_full; j += kU) {
        u32x4 bv[kU][R], av[kU][MR];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const uint32_t ko = (uint32_t)((j + u) * 64 + lane) * 16u;
#pragma unroll
            for (int r = 0; r < R; ++r) bv[u][r] = load16<AL, true>(rb, b_row[r] + ko);
#pragma unroll
            for (int m = 0; m < MR; ++m) av[u][m] = load16<AL>(ra, a_row[m] + ko);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) step(bv[u], av[u]);
    }
    for (; j < j_hi; ++j) {
        const int c = j * 64 + lane;
        const uint32_t ko = (uint32_t)c * 16u;
        const int valid = p.K - c * VEC;  // elements of this chunk inside the row
        u32x4 bv[R], av[MR];
#pragma unroll
        for (int r = 0; r < R; ++r) bv[r] = load16<AL, true>(rb, valid > 0 ? b_row[r] + ko : kOobOffset);
#pragma unroll
        for (int m = 0; m < MR; ++m) av[m] = load16<AL>(ra, valid > 0 ? a_row[m] + ko : kOobOffset);
        if (valid < VEC) {
            // Both operands: past K lies the next row, whose values (even
            // non-finite ones) must not reach a product.
#pragma unroll
            for (int r = 0; r < R; ++r) bv[r] = keep_elems<MODE>(bv[r], valid);
#pragma unroll
            for (int m = 0; m < MR; ++m) av[m] = keep_elems<MODE>(av[m], valid);
        }
        step(bv, av);
    }

    // Lanes: fixed butterfly, every lane ends with the wave's sums.
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            Acc v = acc[m][r];
#pragma unroll
            for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s, 64);
            acc[m][r] = v;
        }
    if constexpr (KW > 1) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) red[w][m * R + r] = acc[m][r];
        }
        __syncthreads();
        if (kw != 0) return;
    }
    // Lane i < MR * R stores output (m, r) = (i / R, i % R).
    if (lane >= MR * R) return;
    const int m = lane / R, r = lane % R;
    if (r >= nrows) return;
    Acc v = Acc(0);
    if constexpr (KW > 1) {
#pragma unroll
        for (int q = 0; q < KW; ++q) v += red[w + q][lane];
    } else {
#pragma unroll
        for (int mm = 0; mm < MR; ++mm)
#pragma unroll
            for (int rr = 0; rr < R; ++rr)
                if (mm * R + rr == lane) v = acc[mm][rr];
    }
    if constexpr (MODE == 2) {
        p.Ci[(size_t)m * p.ldc + n0 + r] = v;
    } else if constexpr (MODE == 3) {
        float* c = p.C + (size_t)m * p.ldc + n0 + r;
        const float dq = p.amax ? dyn_dequant_scale(p.amax, p.alpha) : 0.0f;
        *c = s8_out(v, n0 + r, p.scale, p.amax, dq, p.beta, c);
    } else {
        float* c = p.C + (size_t)m * p.ldc + n0 + r;
        *c = add_bias(epilogue(v, p.alpha, p.beta, c), p.bias, n0 + r);
    }
}

}  // namespace

#define DNNOPT_ROWDOT_KW(MR, R, MODE, AL)                                                                    \
    switch (kw) {                                                                                            \
        case 1: hipLaunchKernelGGL((dnnopt_rowdot<MR, R, 1, MODE, AL>), grid, dim3(kWaves * 64), 0, s, a); break; \
        case 2: hipLaunchKernelGGL((dnnopt_rowdot<MR, R, 2, MODE, AL>), grid, dim3(kWaves * 64), 0, s, a); break; \
        case 4: hipLaunchKernelGGL((dnnopt_rowdot<MR, R, 4, MODE, AL>), grid, dim3(kWaves * 64), 0, s, a); break; \
        case 8: hipLaunchKernelGGL((dnnopt_rowdot<MR, R, 8, MODE, AL>), grid, dim3(kWaves * 64), 0, s, a); break; \
        default: return hipErrorInvalidValue;                                                                \
    }

template <int MODE, int AL>
static hipError_t launch_rowdot_mode(int mr, int kw, dim3 grid, const RowdotArgs& a, hipStream_t s) {
    // int8 modes are built for M <= kRowdotS8MaxM only.
    if (MODE >= 2 && mr > kRowdotS8MaxM) return hipErrorInvalidValue;
    switch (mr) {
        case 1: DNNOPT_ROWDOT_KW(1, rowdot_rows(MODE, 1), MODE, AL) break;
        case 2: DNNOPT_ROWDOT_KW(2, rowdot_rows(MODE, 2), MODE, AL) break;
        case 3: DNNOPT_ROWDOT_KW(3, rowdot_rows(MODE, 3), MODE, AL) break;
        case 4: DNNOPT_ROWDOT_KW(4, rowdot_rows(MODE, 4), MODE, AL) break;
        default:
            if constexpr (MODE < 2) {
                switch (mr) {
                    case 5: DNNOPT_ROWDOT_KW(5, rowdot_rows(MODE, 5), MODE, AL) break;
                    case 6: DNNOPT_ROWDOT_KW(6, rowdot_rows(MODE, 6), MODE, AL) break;
                    case 7: DNNOPT_ROWDOT_KW(7, rowdot_rows(MODE, 7), MODE, AL) break;
                    case 8: DNNOPT_ROWDOT_KW(8, rowdot_rows(MODE, 8), MODE, AL) break;
                    default: return hipErrorInvalidValue;
                }
            } else {
                return hipErrorInvalidValue;
            }
    }
    return hipGetLastError();
}

hipError_t launch_rowdot(int mode, int mr, int kw, int aligned, dim3 grid, const RowdotArgs& a, hipStream_t s) {
    if (mr < 1 || mr > 8 || mr != a.M) return hipErrorInvalidValue;
    switch (mode) {
        case 0: return launch_rowdot_mode<0, 1>(mr, kw, grid, a, s);
        case 1: return aligned ? launch_rowdot_mode<1, 1>(mr, kw, grid, a, s) : launch_rowdot_mode<1, 0>(mr, kw, grid, a, s);
        case 2:
            if (!a.Ci) return hipErrorInvalidValue;
            return aligned ? launch_rowdot_mode<2, 1>(mr, kw, grid, a, s) : launch_rowdot_mode<2, 0>(mr, kw, grid, a, s);
        case 3:
            if (!a.C || (!a.scale && !a.amax)) return hipErrorInvalidValue;
            return aligned ? launch_rowdot_mode<3, 1>(mr, kw, grid, a, s) : launch_rowdot_mode<3, 0>(mr, kw, grid, a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dnnopt_hip
