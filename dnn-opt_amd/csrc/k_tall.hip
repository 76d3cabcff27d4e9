// k_tall.hip -- fp32 tall-skinny GEMM with B resident in LDS (gfx950).
//
// Shapes: M large, N <= 64 (the dispatcher sends 12 < N <= 64), K small
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
#define DNNOPT_TALL_D 2
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
// chunks of A in flight, TB: B stored N x K, BETA: C is read (beta != 0),
// KFULL: K % 16 == 0 (no partial chunk to mask).
template <int NT, int RT, int D, int TB, int BETA, int KFULL>
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

    // A's range ends at the last element of row M - 1, so every row >= M
    // (a partial last tile, chunks past this wave's last tile) reads zero:
    // row * lda + k >= M * lda >= (M - 1) * lda + K.  Offsets are split into a
    // per-lane constant and a wave-uniform part kept in scalar registers.
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc(p.A, range31(((size_t)(p.M - 1) * p.lda + p.K) * 4));
    uint32_t lane_a[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) lane_a[rt] = ((uint32_t)(rt * 16 + r) * p.lda + 4 * g) * 4u;
    const uint32_t tile_step = (uint32_t)(16 * RT) * (uint32_t)GW * (uint32_t)p.lda * 4u;  // next tile of this wave
    // Load cursor: byte offset of (row tile, chunk) for the next load, and its
    // chunk number.  Past the wave's last chunk it runs on into rows that are
    // out of range or unused; no load faults and no such chunk is consumed.
    uint32_t l_off = (uint32_t)gw * (uint32_t)(16 * RT) * (uint32_t)p.lda * 4u;
    int l_kc = 0;

    // D chunks in flight need D + 1 slots: chunk i + D is loaded into the
    // slot chunk i - 1 left before chunk i's MFMAs are issued.
    constexpr int S = D + 1;
    u32x4 ring[S][RT];
    auto load = [&](int slot) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) ring[slot][rt] = buf_load_x4(ra, lane_a[rt] + l_off);
        l_off += 64u;
        if (++l_kc == KC) {
            l_kc = 0;
            l_off += tile_step - (uint32_t)KC * 64u;
        }
    };
    // First chunks of A go out before B is staged.
    if (total > 0) {
#pragma unroll
        for (int d = 0; d < D; ++d) load(d);
    }

    // Stage B.  Unit u = (k quad kq = u / NP, column n = u % NP) is the
    // 16-byte chunk at bsm[u * 4], so consecutive threads write consecutive
    // chunks (no LDS bank conflicts).  There are KC * 4 * NP units, at
    // most kStageU per thread (the host caps B's image at 64 KiB); every
    // thread issues all its loads before its first LDS write, so staging
    // costs one L2 round trip rather than one per unit.
    {
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(
            p.B, range31((TB ? (size_t)(p.N - 1) * p.ldb + p.K : (size_t)(p.K - 1) * p.ldb + p.N) * 4));
        constexpr int kStageU = 65536 / 16 / (kTallWaves * 64);
        const int units = KC * 4 * NP;
        u32x4 v[kStageU];
#pragma unroll
        for (int j = 0; j < kStageU; ++j) {
            const int u = (int)threadIdx.x + j * kTallWaves * 64;
            const int kq = u / NP, n = u % NP, k0 = 4 * kq;
            const bool ok = u < units && n < p.N;
            if constexpr (TB) {
                // B stored N x K: the chunk is one 16-byte load from row n
                // (its elements past K, in the row's padding or the next
                // row, are masked when written).
                v[j] = buf_load_x4(rb, ok && k0 < p.K ? ((uint32_t)n * p.ldb + k0) * 4u : kOobOffset);
            } else {
                // B stored K x N: four loads from rows k0..k0+3, column n;
                // a wave's loads of one row are contiguous.  Rows past K
                // read zero.
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    v[j][c] = buf_load_x1(rb, ok && k0 + c < p.K ? ((uint32_t)(k0 + c) * p.ldb + n) * 4u : kOobOffset);
            }
        }
#pragma unroll
        for (int j = 0; j < kStageU; ++j) {
            const int u = (int)threadIdx.x + j * kTallWaves * 64;
            if (u < units) {
                u32x4 w = v[j];
                if constexpr (TB) w = keep_first(w, p.K - 4 * (u / NP));
                *reinterpret_cast<u32x4*>(&bsm[(size_t)u * 4]) = w;
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
    // C's range ends at the last element of row M - 1: rows >= M of a partial
    // tile fall outside it (m * ldc + n >= M * ldc), columns >= N are masked
    // explicitly (they may lie inside the range, in C's padding).
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.C, range31(((size_t)(p.M - 1) * p.ldc + p.N) * 4));
    uint32_t lane_c[RT * 4];
#pragma unroll
    for (int q = 0; q < RT * 4; ++q)
        lane_c[q] = ((uint32_t)((q >> 2) * 16 + 4 * g + (q & 3)) * (uint32_t)p.ldc + (uint32_t)r) * 4u;
    bool col_ok[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) col_ok[nt] = nt * 16 + r < p.N;

    f32x4 acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int ktail = p.K - (KC - 1) * 16;  // k of the last chunk (1..16)
    // LDS byte offset of this lane's B fragment in chunk 0; chunk kc adds
    // kc * 4 * NP * 16 bytes, column tile nt adds nt * 256.
    const uint32_t lane_b = (uint32_t)(g * NP + r) * 16u;
    // Compute cursor: chunk number and first row of the tile in progress.
    int c_kc = 0;
    int c_row0 = gw * 16 * RT;

    auto step = [&](const u32x4 (&a)[RT]) {
        u32x4 av[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if constexpr (KFULL) av[rt] = a[rt];
            else av[rt] = c_kc == KC - 1 ? keep_first(a[rt], ktail - 4 * g) : a[rt];
        }
        const char* bp = reinterpret_cast<const char*>(bsm) + lane_b + (uint32_t)c_kc * (uint32_t)(NP * 64);
        u32x4 bv[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) bv[nt] = *reinterpret_cast<const u32x4*>(bp + nt * 256);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(as_f32(av[rt][c]), as_f32(bv[nt][c]),
                                                                      acc[rt][nt], 0, 0, 0);
        if (c_kc == KC - 1) {
            const uint32_t s_c = (uint32_t)c_row0 * (uint32_t)p.ldc * 4u;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t row_off = s_c + lane_c[rt * 4 + e];
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const uint32_t off = col_ok[nt] ? row_off + nt * 64u : kOobOffset;
                        float v;
                        if constexpr (BETA) v = __builtin_fmaf(p.alpha, acc[rt][nt][e], p.beta * as_f32(buf_load_x1(rc, off)));
                        else v = p.alpha * acc[rt][nt][e];
                        if (has_bias) v = add_rn(v, biasv[nt]);
                        buf_store_x1(rc, off, as_u32(v));
                        acc[rt][nt][e] = 0.0f;
                    }
                }
            c_kc = 0;
            c_row0 += 16 * RT * GW;
        } else {
            ++c_kc;
        }
    };

    // Chunk i lives in slot i % S from its load until its MFMAs.  Unrolled
    // over the S slots, every slot keeps its registers around the loop (no
    // copy at the back edge, whose wait would drain every load in flight),
    // and the wait for chunk i leaves the D later chunks' loads in flight.
    int i0 = 0;
    for (; i0 + S <= total; i0 += S) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            load((s + D) % S);
            // Keep the loads ahead of this chunk's wait and MFMAs.
            __builtin_amdgcn_sched_barrier(0);
            step(ring[s]);
        }
    }
    // The last total - i0 < S chunks are in slots 0, 1, ... already.
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (i0 + s < total) step(ring[s]);
}

int tall_waves() { return kTallWaves; }

template <int RT, int BETA, int KFULL>
static hipError_t launch_tall_beta(int nt, int tb, dim3 grid, size_t lds_bytes, const TallArgs& a, hipStream_t s) {
    const dim3 blk(kTallWaves * 64);
#define DNNOPT_TALL_CASE(NT, TB)                                                                           \
    case NT * 2 + TB:                                                                                      \
        hipLaunchKernelGGL((dnnopt_tall_f32<NT, RT, kTallD, TB, BETA, KFULL>), grid, blk, lds_bytes, s, a); \
        break;
    switch (nt * 2 + (tb ? 1 : 0)) {
        DNNOPT_TALL_CASE(1, 0)
        DNNOPT_TALL_CASE(1, 1)
        DNNOPT_TALL_CASE(2, 0)
        DNNOPT_TALL_CASE(2, 1)
        DNNOPT_TALL_CASE(3, 0)
        DNNOPT_TALL_CASE(3, 1)
        DNNOPT_TALL_CASE(4, 0)
        DNNOPT_TALL_CASE(4, 1)
        default: return hipErrorInvalidValue;
    }
#undef DNNOPT_TALL_CASE
    return hipGetLastError();
}

template <int RT>
static hipError_t launch_tall_rt(int nt, int tb, dim3 grid, size_t lds_bytes, const TallArgs& a, hipStream_t s) {
    const bool kfull = a.K % 16 == 0;
    if (a.beta == 0.0f)
        return kfull ? launch_tall_beta<RT, 0, 1>(nt, tb, grid, lds_bytes, a, s)
                     : launch_tall_beta<RT, 0, 0>(nt, tb, grid, lds_bytes, a, s);
    return kfull ? launch_tall_beta<RT, 1, 1>(nt, tb, grid, lds_bytes, a, s)
                 : launch_tall_beta<RT, 1, 0>(nt, tb, grid, lds_bytes, a, s);
}

hipError_t launch_tall_f32(int nt, int tb, int rt, dim3 grid, size_t lds_bytes, const TallArgs& a, hipStream_t s) {
    // The kernel stages all of B: the image must fit the 64 KiB its staging
    // loop is sized for, and the launch must provide it.
    const size_t need = tall_lds_bytes(nt, a.K);
    if (need > 65536 || lds_bytes < need) return hipErrorInvalidValue;
    if (rt == 1) return launch_tall_rt<1>(nt, tb, grid, lds_bytes, a, s);
    if (rt == 2) return launch_tall_rt<2>(nt, tb, grid, lds_bytes, a, s);
    return hipErrorInvalidValue;
}

}  // namespace dnnopt_hip
