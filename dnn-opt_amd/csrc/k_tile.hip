// k_tile.hip -- fp32 and bf16 MFMA tile kernels for M > 8 (gfx950).
//
// Replaces the reference's packed BLIS path for these shapes
// (src/gemm/gemm_driver_generic.cpp:27-248 with the fp32 8x12/8x16 and bf16
// BFMMLA 8x8 micro-kernels, src/gemm/gemm_driver_bf16.cpp:134-218) and the
// materialized transposes of cblas_sgemm (src/blas/cblas_sgemm.cpp:80-98):
// transposed operands are read in place.
//
// Matrix-core operand packing (16 x 16 output tile, wave64):
//   fp32  v_mfma_f32_16x16x4_f32 : lane l gives 1 value,  k = 4*(l/16) + c
//   bf16  v_mfma_f32_16x16x32_bf16: lane l gives 8 values, k = 8*(l/16) + e
// with row (A) or column (B) = l % 16.  A loop step covers 64 k (fp32: four
// groups j of 16 k, each four MFMAs c) or 128 k (bf16: four groups of 32 k).
// The k assigned to a (lane, register) slot is the same for A and B, so each
// k meets its partner once.  Output register i of lane l holds row
// 4*(l/16) + i, column l % 16 of the tile.
//
// Accumulation is fp32.  Waves that split k inside a workgroup are combined
// in ascending k order through LDS, k-split workgroups in ascending split
// order by the last workgroup to arrive; the result is bit-reproducible.
//
// Tails: operand rows/columns outside M/N and k outside K read as zero
// (out-of-range buffer offsets, and masking inside a partially valid 128-bit
// chunk), so garbage past an edge never reaches an accumulator.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

using namespace dnnopt_dev;

namespace dnnopt_hip {

namespace {

__device__ __forceinline__ uint32_t clamp_rec(size_t bytes) {
    return bytes > 0x7FFFFFFFull ? 0x7FFFFFFFu : (uint32_t)bytes;
}

// Keep the first `valid` 32-bit lanes of v (0..4).
__device__ __forceinline__ u32x4 keep_dwords(u32x4 v, int valid) {
    u32x4 r;
#pragma unroll
    for (int d = 0; d < 4; ++d) r[d] = d < valid ? v[d] : 0u;
    return r;
}

// Keep the first `valid` 16-bit halves of v (0..8).
__device__ __forceinline__ u32x4 keep_halves(u32x4 v, int valid) {
    u32x4 r;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const int keep = valid - 2 * d;
        r[d] = keep >= 2 ? v[d] : (keep == 1 ? (v[d] & 0xFFFFu) : 0u);
    }
    return r;
}

template <int MT, int NT, int WM, int WN, int KW>
struct TileShape {
    static constexpr int BM = WM * MT * 16;
    static constexpr int BN = WN * NT * 16;
    static constexpr int SUB = MT * NT * 4;
    static constexpr int RED = KW > 1 ? (KW - 1) * WM * WN * SUB * 64 : 1;
};

// Column (within the tile) of lane column r of accumulator sub-tile nt of
// wave column wn: 16 consecutive columns per sub-tile, or (ILV) sub-tiles in
// groups of 4 whose columns interleave over 64: 4 r + nt mod 4.
template <int NT, bool ILV>
__device__ __forceinline__ int tile_col(int wn, int nt, int r) {
    if constexpr (ILV) return ((wn * NT + nt) / 4) * 64 + 4 * r + (nt & 3);
    return (wn * NT + nt) * 16 + r;
}

// Combine k-split waves (LDS) and k-split workgroups (ticket), then apply the
// epilogue.  Shared by the fp32 and bf16 kernels.
template <int MT, int NT, int WM, int WN, int KW, bool ILV = false>
__device__ __forceinline__ void tile_finish(const TileArgs& p, f32x4 (&acc)[MT][NT], float* red,
                                            int* last_flag, int w, int lane, int tile_n, int tile_m, int tiles_n,
                                            int tiles) {
    using S = TileShape<MT, NT, WM, WN, KW>;
    const int r = lane & 15, g = lane >> 4;
    const int wn = w % WN, wm = (w / WN) % WM, wk = w / (WN * WM);
    if constexpr (KW > 1) {
        const int slot = wm * WN + wn;
        if (wk > 0) {
            float* dst = &red[(((wk - 1) * WM * WN + slot) * S::SUB) * 64];
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
                const float* src = &red[(((q - 1) * WM * WN + slot) * S::SUB) * 64];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[mt][nt][i] += src[((mt * NT + nt) * 4 + i) * 64 + lane];
            }
        }
    }

    const int split = blockIdx.z;
    const int tile_id = tile_m * tiles_n + tile_n;
    if (p.splits > 1) {
        // Partials are written through to memory (coherent stores) so the
        // reducing workgroup can read them without cache maintenance.
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(
            p.part, range31((size_t)p.splits * tiles * S::BM * S::BN * 4));
        if (wk == 0) {
            const size_t base = ((size_t)split * tiles + tile_id) * (S::BM * S::BN);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int ml = (wm * MT + mt) * 16 + 4 * g + i;
                        const int nl = tile_col<NT, ILV>(wn, nt, r);
                        buf_store_x1_coherent(rp, (uint32_t)((base + ml * S::BN + nl) * 4), as_u32(acc[mt][nt][i]));
                    }
        }
        if (p.defer_reduce) return;
        if (!split_ticket(&p.tickets[(size_t)tile_id * kTicketStride], (unsigned)p.splits, last_flag)) return;
        // Last workgroup of the tile: every thread sums 16-byte pieces of the
        // tile's row-major partial block over the splits in ascending split
        // order (as dnnopt_splitk_reduce, so the same bits), CH splits' loads
        // in flight at a time, and stores C with the epilogue.  Its own
        // partial is read back from memory like the others.
        constexpr int NTH = WM * WN * KW * 64;
        constexpr int Q4 = S::BM * S::BN / 4;      // 16-byte pieces of the tile
        constexpr int QT = (Q4 + NTH - 1) / NTH;   // pieces per thread
        constexpr int CH = QT >= 8 ? 1 : 8 / QT;  // splits per batch of loads (8 pieces in flight)
        const uint32_t stride = (uint32_t)tiles * (uint32_t)(S::BM * S::BN) * 4u;
        const uint32_t tbase = (uint32_t)tile_id * (uint32_t)(S::BM * S::BN) * 4u;
        f32x4 sum[QT];
        for (int sp0 = 0; sp0 < p.splits; sp0 += CH) {
            f32x4 v[CH][QT];
#pragma unroll
            for (int u = 0; u < CH; ++u)
#pragma unroll
                for (int j = 0; j < QT; ++j) {
                    const int q = (int)threadIdx.x + j * NTH;
                    v[u][j] = buf_load_x4_coherent(
                        rp, sp0 + u < p.splits && q < Q4 ? tbase + (uint32_t)(sp0 + u) * stride + (uint32_t)q * 16u
                                                         : kOobOffset);
                }
#pragma unroll
            for (int u = 0; u < CH; ++u)
#pragma unroll
                for (int j = 0; j < QT; ++j)
                    if (sp0 + u < p.splits) sum[j] = sp0 + u == 0 ? v[u][j] : sum[j] + v[u][j];
        }
        const int m0 = tile_m * S::BM, n0 = tile_n * S::BN;
#pragma unroll
        for (int j = 0; j < QT; ++j) {
            const int q = (int)threadIdx.x + j * NTH;
            const int m = m0 + (4 * q) / S::BN, n1 = n0 + (4 * q) % S::BN;
            if (q < Q4 && m < p.M) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int n = n1 + e;
                    if (n < p.N) {
                        float* c = p.C + (size_t)m * p.ldc + n;
                        *c = add_bias(epilogue(sum[j][e], p.alpha, p.beta, c), p.bias, n);
                    }
                }
            }
        }
        return;
    } else if (wk != 0) {
        return;
    }

    const int m0 = tile_m * S::BM, n0 = tile_n * S::BN;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + (wm * MT + mt) * 16 + 4 * g + i;
                const int n = n0 + tile_col<NT, ILV>(wn, nt, r);
                if (m < p.M && n < p.N) {
                    float* c = p.C + (size_t)m * p.ldc + n;
                    *c = add_bias(epilogue(acc[mt][nt][i], p.alpha, p.beta, c), p.bias, n);
                }
            }
}

}  // namespace

// ---------------------------------------------------------------- fp32
template <int MT, int NT, int WM, int WN, int KW, int TA, int TB>
__global__ __launch_bounds__(WM* WN* KW * 64) void dnnopt_tile_f32(TileArgs p) {
    using S = TileShape<MT, NT, WM, WN, KW>;
    constexpr int KB = 64;
    __shared__ float red[S::RED];
    __shared__ int last_flag;

    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
    const int w = wave_id();
    const int wn = w % WN, wm = (w / WN) % WM, wk = w / (WN * WM);
    // 16-row tiles (one row of waves) are launched as one XCD-ordered row of
    // workgroups: the row tiles of a column strip run on one XCD, close in
    // time, and share B in its L2.
    constexpr bool XCD = MT == 1 && WM == 1;
    int tn_ = (int)blockIdx.x, tm_ = (int)blockIdx.y, tiles_n = (int)gridDim.x;
    if constexpr (XCD) {
        const TileXY t = xcd_tile((int)blockIdx.x, p.tiles_n, p.tiles_m);
        if (!t.ok) return;
        tn_ = t.n;
        tm_ = t.m;
        tiles_n = p.tiles_n;
    }
    const int m0 = tm_ * S::BM, n0 = tn_ * S::BN;

    const int nblk = (p.K + KB - 1) / KB;
    const long long chunks = (long long)p.splits * KW;
    const long long cw = (long long)blockIdx.z * KW + wk;
    const int b_lo = (int)(((long long)nblk * cw) / chunks);
    const int b_hi = (int)(((long long)nblk * (cw + 1)) / chunks);
    const int ks = (int)(((long long)nblk * ((long long)blockIdx.z * KW)) / chunks) * KB;

    const float* A = static_cast<const float*>(p.A);
    const float* B = static_cast<const float*>(p.B);
    // Descriptors start at (m0 or n0, ks) of each operand.
    const float* abase = TA ? A + (size_t)ks * p.lda + m0 : A + (size_t)m0 * p.lda + ks;
    const size_t arem = TA ? (size_t)(p.K - 1 - ks) * p.lda + (p.M - m0) : (size_t)(p.M - 1 - m0) * p.lda + (p.K - ks);
    const float* bbase = TB ? B + (size_t)n0 * p.ldb + ks : B + (size_t)ks * p.ldb + n0;
    const size_t brem = TB ? (size_t)(p.N - 1 - n0) * p.ldb + (p.K - ks) : (size_t)(p.K - 1 - ks) * p.ldb + (p.N - n0);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(abase, clamp_rec(arem * 4));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bbase, clamp_rec(brem * 4));

    int mloc[MT], nloc[NT];
    bool mval[MT], nval[NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        mloc[mt] = (wm * MT + mt) * 16 + r;
        mval[mt] = m0 + mloc[mt] < p.M;
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        nloc[nt] = (wn * NT + nt) * 16 + r;
        nval[nt] = n0 + nloc[nt] < p.N;
    }
    // B stored K x N, 16-row tiles with whole groups of 4 sub-tiles: one
    // 16-byte load of columns 4 r .. 4 r + 3 of a 64-column group per k
    // (instead of four 4-byte loads of one column); component e feeds
    // sub-tile 4 q + e, whose lane column r is column 4 r + e of the group.
    // (MI355X, us, 16 x 128 tiles: 32 x 4096 x 4096 29.3 -> 25.1, 32 x 11003
    // x 2048 52.8 -> 45.7; the 64 x 128 tiles at M >= 128 were slower with it,
    // 65.2 -> 79.8 at 128 x 4096 x 4096, and keep the column loads.)
    constexpr bool ILV = TB == 0 && NT % 4 == 0 && WM == 1 && MT == 1;
    constexpr int NG = ILV ? NT / 4 : 1;
    int gloc[NG];
    bool gval[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        gloc[q] = (wn * NG + q) * 64 + 4 * r;
        gval[q] = n0 + gloc[q] < p.N;
    }

    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int blk = b_lo; blk < b_hi; ++blk) {
        const int kl0 = blk * KB - ks;  // k of this block relative to ks
        u32x4 a[MT][4], b[NT][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kq = kl0 + 16 * j + 4 * g;  // first k of this lane's quad (relative)
            const int kvalid = p.K - (ks + kq);   // how many of the 4 k are < K
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                if constexpr (TA == 0) {
                    const uint32_t off = (mval[mt] && kvalid > 0) ? ((uint32_t)mloc[mt] * p.lda + kq) * 4u : kOobOffset;
                    a[mt][j] = buf_load_x4(ra, off);
                    if (kvalid < 4) a[mt][j] = keep_dwords(a[mt][j], kvalid);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const uint32_t off = (mval[mt] && c < kvalid) ? ((uint32_t)(kq + c) * p.lda + mloc[mt]) * 4u : kOobOffset;
                        a[mt][j][c] = buf_load_x1(ra, off);
                    }
                }
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                if constexpr (ILV) {
                    // b[4 q + c][j] holds row kq + c, columns 4 r .. + 3 of group q;
                    // sub-tile 4 q + e takes its component e below.
                    if (nt % 4 == 0) {
                        const int q = nt / 4;
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const uint32_t off = (gval[q] && c < kvalid) ? ((uint32_t)(kq + c) * p.ldb + gloc[q]) * 4u : kOobOffset;
                            b[nt + c][j] = buf_load_x4(rb, off);
                        }
                    }
                } else if constexpr (TB == 1) {
                    const uint32_t off = (nval[nt] && kvalid > 0) ? ((uint32_t)nloc[nt] * p.ldb + kq) * 4u : kOobOffset;
                    b[nt][j] = buf_load_x4(rb, off);
                    if (kvalid < 4) b[nt][j] = keep_dwords(b[nt][j], kvalid);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const uint32_t off = (nval[nt] && c < kvalid) ? ((uint32_t)(kq + c) * p.ldb + nloc[nt]) * 4u : kOobOffset;
                        b[nt][j][c] = buf_load_x1(rb, off);
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        // ILV: the B value of k = kq + c for sub-tile nt = 4 q + e is
                        // component e of the load of row kq + c of group q.
                        const uint32_t bv = ILV ? b[(nt & ~3) + c][j][nt & 3] : b[nt][j][c];
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(as_f32(a[mt][j][c]), as_f32(bv),
                                                                          acc[mt][nt], 0, 0, 0);
                    }
    }

    tile_finish<MT, NT, WM, WN, KW, ILV>(p, acc, red, &last_flag, w, lane, tn_, tm_, tiles_n,
                                         XCD ? p.tiles_n * p.tiles_m : (int)(gridDim.x * gridDim.y));
}

// ---------------------------------------------------------------- bf16
// MODE kTileBF16: A, B hold bf16 bit patterns.  MODE kTileF2B: A, B are fp32
// and are rounded to bf16 (nearest even, reference formula) on load.
// AL = 0: rows of a bf16-storage A may start on a 2-byte boundary and are
// read with funnel-shifted loads.
// TB = 1: B is stored N x K (k contiguous, bf16 storage only) and each
// lane's 8 k of a column are one 16-byte load, like A's.
template <int MT, int NT, int WM, int WN, int KW, int MODE, int AL, int TB = 0>
__global__ __launch_bounds__(WM* WN* KW * 64) void dnnopt_tile_bf16(TileArgs p) {
    static_assert(!TB || MODE == kTileBF16, "B stored N x K needs bf16 storage");
    using S = TileShape<MT, NT, WM, WN, KW>;
    constexpr int KB = 128;
    constexpr int ES = MODE == kTileBF16 ? 2 : 4;
    __shared__ float red[S::RED];
    __shared__ int last_flag;

    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
    const int w = wave_id();
    const int wn = w % WN, wm = (w / WN) % WM, wk = w / (WN * WM);
    const int m0 = blockIdx.y * S::BM, n0 = blockIdx.x * S::BN;

    const int nblk = (p.K + KB - 1) / KB;
    const long long chunks = (long long)p.splits * KW;
    const long long cw = (long long)blockIdx.z * KW + wk;
    const int b_lo = (int)(((long long)nblk * cw) / chunks);
    const int b_hi = (int)(((long long)nblk * (cw + 1)) / chunks);
    const int ks = (int)(((long long)nblk * ((long long)blockIdx.z * KW)) / chunks) * KB;

    const char* A = static_cast<const char*>(p.A);
    const char* B = static_cast<const char*>(p.B);
    const char* abase = A + ((size_t)m0 * p.lda + ks) * ES;
    const size_t arem = (size_t)(p.M - 1 - m0) * p.lda + (p.K - ks);
    const char* bbase = TB ? B + ((size_t)n0 * p.ldb + ks) * ES : B + ((size_t)ks * p.ldb + n0) * ES;
    const size_t brem = TB ? (size_t)(p.N - 1 - n0) * p.ldb + (p.K - ks) : (size_t)(p.K - 1 - ks) * p.ldb + (p.N - n0);
    uint32_t alo = 0, blo = 0;
    const __amdgpu_buffer_rsrc_t ra = rsrc_aligned(abase, arem * ES, &alo);
    const __amdgpu_buffer_rsrc_t rb = TB ? rsrc_aligned(bbase, brem * ES, &blo) : make_rsrc(bbase, clamp_rec(brem * ES));

    int mloc[MT], nloc[NT];
    bool mval[MT], nval[NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        mloc[mt] = (wm * MT + mt) * 16 + r;
        mval[mt] = m0 + mloc[mt] < p.M;
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        nloc[nt] = (wn * NT + nt) * 16 + r;
        nval[nt] = n0 + nloc[nt] < p.N;
    }
    // B stored K x N, 16-row tiles with whole groups of 4 sub-tiles: one
    // 16-byte load of columns 4 r .. 4 r + 3 of a 64-column group per k
    // (instead of four 4-byte loads of one column); component e feeds
    // sub-tile 4 q + e, whose lane column r is column 4 r + e of the group.
    // (MI355X, us, 16 x 128 tiles: 32 x 4096 x 4096 29.3 -> 25.1, 32 x 11003
    // x 2048 52.8 -> 45.7; the 64 x 128 tiles at M >= 128 were slower with it,
    // 65.2 -> 79.8 at 128 x 4096 x 4096, and keep the column loads.)
    constexpr bool ILV = TB == 0 && NT % 4 == 0 && WM == 1 && MT == 1;
    constexpr int NG = ILV ? NT / 4 : 1;
    int gloc[NG];
    bool gval[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        gloc[q] = (wn * NG + q) * 64 + 4 * r;
        gval[q] = n0 + gloc[q] < p.N;
    }

    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int blk = b_lo; blk < b_hi; ++blk) {
        const int kl0 = blk * KB - ks;
        u32x4 a[MT][4], b[NT][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ko = kl0 + 32 * j + 8 * g;  // first of this lane's 8 k (relative)
            const int kvalid = p.K - (ks + ko);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                if constexpr (MODE == kTileBF16) {
                    const uint32_t off =
                        (mval[mt] && kvalid > 0) ? ((uint32_t)mloc[mt] * p.lda + ko) * 2u + alo : kOobOffset;
                    if constexpr (AL) a[mt][j] = buf_load_x4(ra, off);
                    else a[mt][j] = buf_load_x4_unaligned(ra, off);
                    if (kvalid < 8) a[mt][j] = keep_halves(a[mt][j], kvalid);
                } else {
                    const uint32_t off =
                        (mval[mt] && kvalid > 0) ? ((uint32_t)mloc[mt] * p.lda + ko) * 4u + alo : kOobOffset;
                    u32x4 lo = buf_load_x4(ra, off);
                    u32x4 hi = buf_load_x4(ra, (mval[mt] && kvalid > 4) ? off + 16u : kOobOffset);
                    (void)AL;
                    if (kvalid < 4) lo = keep_dwords(lo, kvalid);
                    if (kvalid < 8) hi = keep_dwords(hi, kvalid - 4);
#pragma unroll
                    for (int d = 0; d < 2; ++d) {
                        a[mt][j][d] = (uint32_t)f32_to_bf16_bits(as_f32(lo[2 * d])) |
                                      ((uint32_t)f32_to_bf16_bits(as_f32(lo[2 * d + 1])) << 16);
                        a[mt][j][d + 2] = (uint32_t)f32_to_bf16_bits(as_f32(hi[2 * d])) |
                                          ((uint32_t)f32_to_bf16_bits(as_f32(hi[2 * d + 1])) << 16);
                    }
                }
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                if constexpr (TB) {
                    const uint32_t off =
                        (nval[nt] && kvalid > 0) ? ((uint32_t)nloc[nt] * p.ldb + ko) * 2u + blo : kOobOffset;
                    if constexpr (AL) b[nt][j] = buf_load_x4(rb, off);
                    else b[nt][j] = buf_load_x4_unaligned(rb, off);
                    if (kvalid < 8) b[nt][j] = keep_halves(b[nt][j], kvalid);
                } else {
                    uint32_t h[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint32_t off =
                            (nval[nt] && e < kvalid) ? ((uint32_t)(ko + e) * p.ldb + nloc[nt]) * ES : kOobOffset;
                        if constexpr (MODE == kTileBF16) {
                            h[e] = buf_load_u16(rb, off);
                        } else {
                            h[e] = f32_to_bf16_bits(as_f32(buf_load_x1(rb, off)));
                        }
                    }
#pragma unroll
                    for (int d = 0; d < 4; ++d) b[nt][j][d] = h[2 * d] | (h[2 * d + 1] << 16);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[mt][j]),
                                                                         __builtin_bit_cast(bf16x8, b[nt][j]),
                                                                         acc[mt][nt], 0, 0, 0);
    }

    tile_finish<MT, NT, WM, WN, KW>(p, acc, red, &last_flag, w, lane, blockIdx.x, blockIdx.y, gridDim.x,
                                    gridDim.x * gridDim.y);
}

// ---------------------------------------------------------------- bf16, LDS-staged
// Row-major A (M x K) and B (K x N) through LDS, double-buffered in k-blocks
// of 64.  Per block a workgroup stages A as BM rows x 64 k (k-contiguous, so
// an A operand is one 16-byte LDS read) and B as it lies in memory, BK rows
// of k x BN columns, written with 16-byte stores.  A B operand (8 k of one
// column per lane) is gathered by two ds_read_b64_tr_b16: in each group of
// 16 lanes, lane p points at row k0 + p / 4, columns 4 (p % 4) .. + 3 of the
// 16-column tile, and lane r receives B[k0 + 0..3][column r] -- four
// consecutive k of its column.  B rows are padded by 32 bytes so that the
// four rows of one read fall in different banks.  16-byte chunks of an A row
// are XOR-swizzled by the row index so that the 16 rows read by one MFMA
// operand fall in different banks.  The next block's global loads are issued
// before the current block's MFMAs.
//
// TB = 1 (bf16 storage only): B is stored N x K.  Its rows are then staged
// exactly like A's -- 16-byte chunks of 8 k, no transpose.
//
// Requirements (checked by the host): rows of A and B start on 4-byte
// boundaries (even lda, ldb and 4-byte aligned pointers for bf16 storage).
namespace {

// 8 fp32 values (two 16-byte loads) rounded to bf16 (reference formula) and
// packed as 8 bf16 bit patterns.
__device__ __forceinline__ u32x4 pack_bf16x8(const u32x4& lo, const u32x4& hi) {
    u32x4 out;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        out[d] = (uint32_t)f32_to_bf16_bits(as_f32(lo[2 * d])) | ((uint32_t)f32_to_bf16_bits(as_f32(lo[2 * d + 1])) << 16);
        out[d + 2] =
            (uint32_t)f32_to_bf16_bits(as_f32(hi[2 * d])) | ((uint32_t)f32_to_bf16_bits(as_f32(hi[2 * d + 1])) << 16);
    }
    return out;
}

// Physical 16-byte chunk of logical chunk c (0..7) in LDS row `row`.
__device__ __forceinline__ int swz_a(int row, int c) { return c ^ (row & 7); }

// 32-byte segment swizzle of LDS row k of a K x N B tile (LDS DMA kernel).
__device__ __forceinline__ int bseg_swz(int k) { return (k & 3) | (((k >> 3) & 1) << 2); }

}  // namespace

// KW: waves that split each k-block's MFMA k-steps for the same output
// sub-tile (the WM x WN output waves are replicated KW times); their sums
// are added in ascending order through LDS after the loop.  Fewer, larger
// per-wave sub-tiles read fewer operand bytes from LDS per MFMA.
template <int MT, int NT, int WM, int WN, int D, int MODE, int TB = 0, int KB0 = 0, int KW = 1>
__global__ __launch_bounds__(WM* WN * KW * 64) void dnnopt_tile_bf16_lds(TileArgs p) {
    static_assert(!TB || MODE == kTileBF16, "B stored N x K needs bf16 storage");
    using S = TileShape<MT, NT, WM, WN, 1>;
    constexpr int BM = S::BM, BN = S::BN;
    // k per block: DNNOPT_LDS_KB when both stages fit in 128 KiB of LDS.
    constexpr int BK = tile_lds_bk(BM, BN, KB0);
    constexpr int NTH = WM * WN * KW * 64;
    constexpr int ROWB = BK * 2;  // bytes of one LDS row (BK bf16)
    constexpr int CPR = ROWB / 16;  // 16-byte chunks per LDS row
    constexpr int KK = BK / 32;     // MFMA k-steps per block
    static_assert(KK % KW == 0, "the k-steps of a block split evenly over the KW waves");
    constexpr int KKW = KK / KW;    // k-steps per wave per block
    // B in LDS: stored N x K, BN rows of BK k (like A); stored K x N, BK rows
    // of BN columns padded by 32 bytes.
    constexpr int BROW = TB ? ROWB : BN * 2 + 32;
    constexpr int A_BYTES = BM * ROWB, B_BYTES = TB ? BN * ROWB : BK * BROW, STAGE = A_BYTES + B_BYTES;
    constexpr int ACH = BM * CPR;              // A chunks (8 k) per block
    // B units per block: one 16-byte chunk, 8 n of one k row (stored K x N)
    // or 8 k of one column (stored N x K).
    constexpr int BUN = TB ? BN * CPR : (BN / 8) * BK;
    constexpr int AU = (ACH + NTH - 1) / NTH;  // per thread
    constexpr int BU = (BUN + NTH - 1) / NTH;
    // The two k-block stages, reused after the main loop to add the KW waves'
    // sums and to stage C rows.
    constexpr int CROW = BN + 4;  // floats per staged C row (padding spreads the banks)
    constexpr int RED_BYTES = (KW - 1) * WM * WN * S::SUB * 64 * 4;
    constexpr int LDS_0 = 2 * STAGE > BM * CROW * 4 ? 2 * STAGE : BM * CROW * 4;
    constexpr int LDS_BYTES = LDS_0 > RED_BYTES ? LDS_0 : RED_BYTES;
    __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
    __shared__ float red_unused[1];
    __shared__ int last_flag;

    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
    const int w = wave_id();
    const int wn = w % WN, wm = (w / WN) % WM, wk = w / (WN * WM);
    const int t = (int)threadIdx.x;
    const TileXY tile = xcd_tile((int)blockIdx.x, p.tiles_n, p.tiles_m);
    if (!tile.ok) return;
    const int m0 = tile.m * BM, n0 = tile.n * BN;

    const int nblk = (p.K + BK - 1) / BK;
    const int b_lo = (int)(((long long)nblk * blockIdx.z) / p.splits);
    const int b_hi = (int)(((long long)nblk * (blockIdx.z + 1)) / p.splits);

    constexpr int ES = MODE == kTileBF16 ? 2 : 4;
    const char* abase = static_cast<const char*>(p.A) + (size_t)m0 * p.lda * ES;
    const char* bbase = static_cast<const char*>(p.B) + (TB ? (size_t)n0 * p.ldb : (size_t)n0) * ES;
    // Ranges end at the last element of each operand, rounded up to a whole
    // dword: the range check of a dword load drops a dword that extends past
    // the range, and the last element may share its dword with the next.
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc(abase, clamp_rec((((size_t)(p.M - 1 - m0) * p.lda + p.K) * ES + 3) & ~(size_t)3));
    const size_t b_last = TB ? (size_t)(p.N - 1 - n0) * p.ldb + p.K : (size_t)(p.K - 1) * p.ldb + (p.N - n0);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bbase, clamp_rec((b_last * ES + 3) & ~(size_t)3));

    // Per-thread offsets that do not change from block to block are computed
    // once: global element offsets of this thread's A chunks and B rows (an
    // out-of-range offset for rows past M), LDS byte offsets of its stores
    // and of the wave's operand reads.
    uint32_t a_off[AU], b_off[BU];
    int a_lds[AU], b_lds[BU];
    int a_c[AU], b_c[BU];
#pragma unroll
    for (int i = 0; i < AU; ++i) {
        const int idx = t + i * NTH, row = idx / CPR, c = idx % CPR;
        const bool ok = (ACH % NTH == 0 || idx < ACH) && m0 + row < p.M;
        a_off[i] = ok ? ((uint32_t)row * p.lda + 8 * c) * ES : kOobOffset;
        a_lds[i] = row * ROWB + swz_a(row, c) * 16;
        a_c[i] = 8 * c;
    }
#pragma unroll
    for (int i = 0; i < BU; ++i) {
        if constexpr (TB) {
            const int idx = t + i * NTH, row = idx / CPR, c = idx % CPR;
            const bool ok = (BUN % NTH == 0 || idx < BUN) && n0 + row < p.N;
            b_off[i] = ok ? ((uint32_t)row * p.ldb + 8 * c) * ES : kOobOffset;
            b_lds[i] = row * ROWB + swz_a(row, c) * 16;
            b_c[i] = 8 * c;
        } else {
            const int u = t + i * NTH, cg = u % (BN / 8), kr = u / (BN / 8);
            const bool ok = BUN % NTH == 0 || u < BUN;
            b_c[i] = 0;
            b_off[i] = ok ? ((uint32_t)kr * p.ldb + 8 * cg) * ES : kOobOffset;
            b_lds[i] = ok ? kr * BROW + cg * 16 : -1;
        }
    }

    // Register ring of D k-blocks: block i of this workgroup lives in slot
    // i % D from its load until it is written to LDS.  Loads run ahead of the
    // range by up to D - 1 blocks; those re-read the last block (never used),
    // so every load is unconditional and the compiler waits for exactly the
    // loads each LDS store needs.
    u32x4 sa[D][AU], sb[D][BU];
    auto load_stage = [&](int blk, int slot) {
        const int bc = blk < b_hi ? blk : b_hi - 1;
        const uint32_t ka = (uint32_t)bc * BK * ES;
        const uint32_t kb = TB ? ka : (uint32_t)bc * BK * p.ldb * ES;
#pragma unroll
        for (int i = 0; i < AU; ++i) {
            if constexpr (MODE == kTileBF16) {
                sa[slot][i] = buf_load_x4(ra, a_off[i] + ka);
            } else {
                const u32x4 lo = buf_load_x4(ra, a_off[i] + ka);
                const u32x4 hi = buf_load_x4(ra, a_off[i] + ka + 16u);
                sa[slot][i] = pack_bf16x8(lo, hi);
            }
        }
#pragma unroll
        for (int i = 0; i < BU; ++i) {
            if constexpr (MODE == kTileBF16) {
                sb[slot][i] = buf_load_x4(rb, b_off[i] + kb);
            } else {
                const u32x4 lo = buf_load_x4(rb, b_off[i] + kb);
                const u32x4 hi = buf_load_x4(rb, b_off[i] + kb + 16u);
                sb[slot][i] = pack_bf16x8(lo, hi);
            }
        }
    };
    auto write_stage = [&](int slot, int buf, int blk) {
        char* As = lds + buf * STAGE;
        char* Bs = As + A_BYTES;
        if ((blk + 1) * BK > p.K) {
            // Only the block holding k = K - 1 has elements of k-contiguous
            // rows past K (the next row's data): zero them.  Rows of a K x N
            // B past K read as zero (out of range).  A separate, rarely taken
            // path: computed on every block, the masks cost ~50 vector
            // instructions per block and wave.
            const int kv = p.K - blk * BK;
            auto keep_k = [&](u32x4 v, int kvalid) {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int keep = kvalid - 2 * d;
                    v[d] = keep >= 2 ? v[d] : (keep == 1 ? (v[d] & 0xFFFFu) : 0u);
                }
                return v;
            };
#pragma unroll
            for (int i = 0; i < AU; ++i)
                if (ACH % NTH == 0 || t + i * NTH < ACH)
                    *reinterpret_cast<u32x4*>(As + a_lds[i]) = keep_k(sa[slot][i], kv - a_c[i]);
#pragma unroll
            for (int i = 0; i < BU; ++i) {
                if (BUN % NTH != 0 && t + i * NTH >= BUN) continue;
                *reinterpret_cast<u32x4*>(Bs + b_lds[i]) = TB ? keep_k(sb[slot][i], kv - b_c[i]) : sb[slot][i];
            }
            // Keeps the masked stores in this branch: merged with the plain
            // path they would become per-element selects on every block.
            asm volatile("" ::: "memory");
            return;
        }
#pragma unroll
        for (int i = 0; i < AU; ++i)
            if (ACH % NTH == 0 || t + i * NTH < ACH) *reinterpret_cast<u32x4*>(As + a_lds[i]) = sa[slot][i];
#pragma unroll
        for (int i = 0; i < BU; ++i) {
            if (BUN % NTH != 0 && t + i * NTH >= BUN) continue;
            *reinterpret_cast<u32x4*>(Bs + b_lds[i]) = sb[slot][i];
        }
    };

    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // LDS offsets of this wave's operand reads for its k-steps kk = j * KW + wk.
    int a_rd[KKW][MT], b_rd[KKW][NT];
#pragma unroll
    for (int j = 0; j < KKW; ++j) {
        const int kk = j * KW + wk;
        const int c = kk * 4 + g;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int row = (wm * MT + mt) * 16 + r;
            a_rd[j][mt] = row * ROWB + swz_a(row, c) * 16;
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            if constexpr (TB) {
                const int n = (wn * NT + nt) * 16 + r;
                b_rd[j][nt] = A_BYTES + n * ROWB + swz_a(n, c) * 16;
            } else {
                // first transposing read: row kk * 32 + 8 g + r / 4, columns 4 (r % 4) of the tile
                b_rd[j][nt] = A_BYTES + (kk * 32 + 8 * g + (r >> 2)) * BROW + ((wn * NT + nt) * 16 + 4 * (r & 3)) * 2;
            }
        }
    }
    auto compute = [&](int buf) {
        const char* St = lds + buf * STAGE;
#pragma unroll
        for (int kk = 0; kk < KKW; ++kk) {
            u32x4 af[MT], bfr[NT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) af[mt] = *reinterpret_cast<const u32x4*>(St + a_rd[kk][mt]);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                if constexpr (TB) {
                    bfr[nt] = *reinterpret_cast<const u32x4*>(St + b_rd[kk][nt]);
                } else {
                    typedef short s16x4 __attribute__((ext_vector_type(4)));
                    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
                    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(St + b_rd[kk][nt]));
                    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(St + b_rd[kk][nt] + 4 * BROW));
                    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
                    bfr[nt] = u32x4{l2[0], l2[1], h2[0], h2[1]};
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[mt]),
                                                                         __builtin_bit_cast(bf16x8, bfr[nt]),
                                                                         acc[mt][nt], 0, 0, 0);
        }
    };

    // Block i (relative to b_lo) is loaded D iterations ahead, written to LDS
    // buffer i & 1 at the end of iteration i - 1 and consumed in iteration i.
    // Full groups of D iterations run without conditionals, so the compiler
    // can wait for exactly the loads each LDS write needs.
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

    if constexpr (KW > 1) {
        // Add the KW waves of each output sub-tile in ascending k order (the
        // main loop ended with a barrier, so the stages are free).
        float* red = reinterpret_cast<float*>(lds);
        const int slot = wm * WN + wn;
        if (wk > 0) {
            float* dst = &red[(((wk - 1) * WM * WN + slot) * S::SUB) * 64];
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
                const float* src = &red[(((q - 1) * WM * WN + slot) * S::SUB) * 64];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[mt][nt][i] += src[((mt * NT + nt) * 4 + i) * 64 + lane];
            }
        }
        __syncthreads();
    }
    if (p.splits > 1) {
        // Waves of k-slot wk > 0 store nothing (tile_finish keys on it).
        tile_finish<MT, NT, WM, WN, 1>(p, acc, red_unused, &last_flag, w, lane, tile.n, tile.m, p.tiles_n,
                                       p.tiles_n * p.tiles_m);
        return;
    }
    // Unsplit tile: stage the BM x BN accumulators in LDS (the stages are
    // free), then write C row by row with 16-byte accesses -- the MFMA layout
    // would store 4 rows x 16 columns per instruction.
    float* Cs = reinterpret_cast<float*>(lds);
    if (wk == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    Cs[((wm * MT + mt) * 16 + 4 * g + i) * CROW + (wn * NT + nt) * 16 + r] = acc[mt][nt][i];
    }
    __syncthreads();
    constexpr int Q4 = BN / 4;  // float4 groups per row
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(
        p.C + (size_t)m0 * p.ldc + n0, clamp_rec(((size_t)(p.M - 1 - m0) * p.ldc + (p.N - n0)) * 4));
    for (int e = t; e < BM * Q4; e += NTH) {
        const int row = e / Q4, q = e % Q4;
        const int m = m0 + row, n = n0 + 4 * q;
        if (m >= p.M || n >= p.N) continue;
        const f32x4 v = *reinterpret_cast<const f32x4*>(&Cs[row * CROW + 4 * q]);
        const uint32_t off = ((uint32_t)row * p.ldc + 4 * q) * 4u;
        if (n + 4 <= p.N) {
            f32x4 out;
            if (p.beta == 0.0f) {
                out = p.alpha * v;
            } else {
                const f32x4 c_old = __builtin_bit_cast(f32x4, buf_load_x4(rc, off));
#pragma unroll
                for (int k = 0; k < 4; ++k) out[k] = __builtin_fmaf(p.alpha, v[k], p.beta * c_old[k]);
            }
            if (p.bias) {
#pragma unroll
                for (int k = 0; k < 4; ++k) out[k] = add_rn(out[k], p.bias[n + k]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, out), rc, off, 0, 0);
        } else {
            float* c = p.C + (size_t)m * p.ldc + n;
            for (int k = 0; k < p.N - n; ++k) c[k] = add_bias(epilogue(v[k], p.alpha, p.beta, c + k), p.bias, n + k);
        }
    }
}

// ---------------------------------------------------------------- bf16, LDS DMA
// bf16 storage: the tile above with both operands copied into LDS by the
// vector memory unit (buffer_load_dwordx4 ... lds: a wave load fills 1 KB of
// a stage, lane l's 16 bytes at +16 l), so no block passes through registers
// and no LDS store waits on them.  The stage layout is the one the
// register-staged kernel builds for A (rows of BK bf16 with XOR-swizzled
// 16-byte chunks) and for B stored N x K (like A); B stored K x N is kept as
// BK rows of 256 bytes (BN <= 128 columns) whose 32-byte segments are
// XOR-swizzled by f(k) = (k mod 4) + 4 ((k / 8) mod 2), so that the 8 rows
// {k0..k0+3, k0+8..k0+11} one half of a ds_read_b64_tr_b16 gathers from
// land in 8 different bank groups (the register-staged kernel's 32-byte
// padding leaves rows k and k + 8 on the same banks).  The lane that fills
// stage byte q loads the global chunk that belongs there (a padding slot
// loads nothing).
// The stage's 1 KB units are dealt round robin over the waves; a wave with
// one unit fewer issues one load into a spare 1 KB so that every wave waits
// on the same count.  S stages (one __shared__ array each), blocks S - 1
// ahead; per block one wait for this wave's own copies of the next block, one
// barrier, the copy of block i + S - 1 into the stage block i - 1 left, then
// block i's MFMAs.  Elements past K of k-contiguous rows (A, and B stored
// N x K) are zeroed in registers after the fragment read, in a separately
// compiled tail block; rows of a K x N B past K are out of range (zero).
template <int MT, int NT, int WM, int WN, int NS, int TB, int BK>
__global__ __launch_bounds__(WM* WN * 64) void dnnopt_tile_bf16_dma(TileArgs p) {
    using SH = TileShape<MT, NT, WM, WN, 1>;
    constexpr int BM = SH::BM, BN = SH::BN;
    constexpr int NW = WM * WN;
    constexpr int ROWB = BK * 2;  // bytes of one A row (BK bf16)
    constexpr int KK = BK / 32;   // MFMA k-steps per block
    constexpr int BROW = TB ? ROWB : 256;
    static_assert(TB || BN <= 128, "a K x N B row of the tile fits 256 bytes");
    constexpr int A_BYTES = BM * ROWB, B_BYTES = TB ? BN * ROWB : BK * BROW, STAGE = A_BYTES + B_BYTES;
    static_assert(NS >= 2 && NS <= 4, "2 to 4 stages");
    static_assert(A_BYTES % 1024 == 0 && B_BYTES % 1024 == 0, "whole 1 KB wave loads per operand");
    constexpr int UNITS = STAGE / 1024;
    constexpr int IPW = (UNITS + NW - 1) / NW;  // wave loads per wave and block
    __shared__ __attribute__((aligned(1024))) char st0[STAGE];
    __shared__ __attribute__((aligned(1024))) char st1[STAGE];
    __shared__ __attribute__((aligned(1024))) char st2[NS > 2 ? STAGE : 16];
    __shared__ __attribute__((aligned(1024))) char st3[NS > 3 ? STAGE : 16];
    __shared__ __attribute__((aligned(1024))) char spare[UNITS % NW ? 1024 : 16];
    __shared__ float red_unused[1];
    __shared__ int last_flag;
    auto stage = [&](int i) -> char* { return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : st3; };

    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
    const int w = wave_id();
    const int wn = w % WN, wm = w / WN;
    const TileXY tile = xcd_tile((int)blockIdx.x, p.tiles_n, p.tiles_m);
    if (!tile.ok) return;
    const int m0 = tile.m * BM, n0 = tile.n * BN;
    const int nblk = (p.K + BK - 1) / BK;
    const int b_lo = (int)(((long long)nblk * blockIdx.z) / p.splits);
    const int b_hi = (int)(((long long)nblk * (blockIdx.z + 1)) / p.splits);
    const int nb = b_hi - b_lo;

    const char* abase = static_cast<const char*>(p.A) + (size_t)m0 * p.lda * 2;
    const char* bbase = static_cast<const char*>(p.B) + (TB ? (size_t)n0 * p.ldb : (size_t)n0) * 2;
    // Ranges end at the last element of each operand, rounded up to a dword.
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc(abase, clamp_rec((((size_t)(p.M - 1 - m0) * p.lda + p.K) * 2 + 3) & ~(size_t)3));
    const size_t b_last = TB ? (size_t)(p.N - 1 - n0) * p.ldb + p.K : (size_t)(p.K - 1) * p.ldb + (p.N - n0);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bbase, clamp_rec((b_last * 2 + 3) & ~(size_t)3));

    // This lane's global byte offset (block 0) for each of its wave's loads;
    // rows past M / N and padding slots start at kOobOffset (read zero).
    uint32_t goff[IPW];
    bool gb[IPW];
    int unit[IPW];
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
        const int u = j * NW + w;
        unit[j] = u < UNITS ? u : -1;
        gb[j] = u * 1024 >= A_BYTES;
        goff[j] = kOobOffset;
        if (u >= UNITS) continue;
        const int q = u * 1024 + 16 * lane;
        if (q < A_BYTES) {
            const int row = q / ROWB, c = swz_a(row, (q % ROWB) / 16);
            if (m0 + row < p.M) goff[j] = ((uint32_t)row * p.lda + 8 * c) * 2u;
        } else if constexpr (TB) {
            const int qq = q - A_BYTES, row = qq / ROWB, c = swz_a(row, (qq % ROWB) / 16);
            if (n0 + row < p.N) goff[j] = ((uint32_t)row * p.ldb + 8 * c) * 2u;
        } else {
            const int qq = q - A_BYTES, kr = qq / BROW, b = qq % BROW;
            const int cb = (((b >> 5) ^ bseg_swz(kr)) << 5) | (b & 31);  // column byte held by slot byte b
            if (cb < 2 * BN) goff[j] = (uint32_t)kr * p.ldb * 2u + (uint32_t)cb;
        }
    }
    // Block `blk` into stage `st`; blocks past the split read nothing
    // (out-of-range offsets) but are issued, so every wave's count of
    // outstanding loads per block is the same.
    auto dma = [&](int st, int blk) {
        const bool live = blk < b_hi;
        const uint32_t ka = live ? (uint32_t)blk * BK * 2u : kOobOffset;
        const uint32_t kb = TB ? ka : (live ? (uint32_t)blk * BK * (uint32_t)p.ldb * 2u : kOobOffset);
        char* base = stage(st);
#pragma unroll
        for (int j = 0; j < IPW; ++j)
            lds_dma16(gb[j] ? rb : ra, unit[j] >= 0 ? base + unit[j] * 1024 : spare, goff[j] + (gb[j] ? kb : ka));
    };

    int a_rd[KK][MT], b_rd[KK][NT], b_rd2[KK][NT];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        const int c = kk * 4 + g;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int row = (wm * MT + mt) * 16 + r;
            a_rd[kk][mt] = row * ROWB + swz_a(row, c) * 16;
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            if constexpr (TB) {
                const int n = (wn * NT + nt) * 16 + r;
                b_rd[kk][nt] = A_BYTES + n * ROWB + swz_a(n, c) * 16;
                b_rd2[kk][nt] = 0;
            } else {
                // transposing reads: rows kk * 32 + 8 g + r / 4 and that + 4,
                // columns 4 (r % 4) .. + 3 of the 16-column tile
                const int cb = ((wn * NT + nt) * 16 + 4 * (r & 3)) * 2;
                const int k1 = kk * 32 + 8 * g + (r >> 2), k2 = k1 + 4;
                b_rd[kk][nt] = A_BYTES + k1 * BROW + ((((cb >> 5) ^ bseg_swz(k1)) << 5) | (cb & 31));
                b_rd2[kk][nt] = A_BYTES + k2 * BROW + ((((cb >> 5) ^ bseg_swz(k2)) << 5) | (cb & 31));
            }
        }
    }
    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto keep_k = [](u32x4 v, int kvalid) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int keep = kvalid - 2 * d;
            v[d] = keep >= 2 ? v[d] : (keep == 1 ? (v[d] & 0xFFFFu) : 0u);
        }
        return v;
    };
    auto compute_blk = [&](int st, int blk, auto tail_tag) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        const char* St = stage(st);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            u32x4 af[MT], bfr[NT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) af[mt] = *reinterpret_cast<const u32x4*>(St + a_rd[kk][mt]);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                if constexpr (TB) {
                    bfr[nt] = *reinterpret_cast<const u32x4*>(St + b_rd[kk][nt]);
                } else {
                    typedef short s16x4 __attribute__((ext_vector_type(4)));
                    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
                    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(St + b_rd[kk][nt]));
                    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(St + b_rd2[kk][nt]));
                    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
                    bfr[nt] = u32x4{l2[0], l2[1], h2[0], h2[1]};
                }
            }
            if constexpr (TAIL) {
                const int kv = p.K - (blk * BK + kk * 32 + 8 * g);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) af[mt] = keep_k(af[mt], kv);
                if constexpr (TB) {
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) bfr[nt] = keep_k(bfr[nt], kv);
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[mt]),
                                                                         __builtin_bit_cast(bf16x8, bfr[nt]),
                                                                         acc[mt][nt], 0, 0, 0);
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
    // Every copy has landed before the workgroup ends (the run-on copies
    // read nothing but still write their stage).
    wait_vmcnt<0>();
    tile_finish<MT, NT, WM, WN, 1>(p, acc, red_unused, &last_flag, w, lane, tile.n, tile.m, p.tiles_n,
                                   p.tiles_n * p.tiles_m);
}

// ---------------------------------------------------------------- fp32, LDS DMA
// fp32 tiles with both operands copied into LDS by the memory unit, as the
// bf16 LDS-DMA tiles above: 32 k per block (128-byte rows of A, and of B
// stored N x K, with the same chunk swizzle), NS stages, blocks NS - 1 ahead,
// one barrier per block.  v_mfma_f32_16x16x4_f32 takes one fp32 of A and one
// of B per lane: a lane's 16-byte fragment read (k = 16 kk + 4 g .. + 3 of
// its row) feeds four MFMAs, k-slot g of MFMA c holding k = 16 kk + 4 g + c
// for A and B alike.  B stored K x N is staged as 32 rows of BN floats and
// read 16 bytes of one k row at a time (columns 4 r .. 4 r + 3 of a
// 64-column group), whose components feed the four sub-tiles of the group
// (their columns interleave over 64, as in the 16-row register tiles), so
// that layout needs wave tiles of whole 64-column groups.
// Bytes of A (and of B stored N x K) past K are zeroed in registers in the
// last block; rows of B stored K x N past K read zero.  A stored M x K only.
template <int MT, int NT, int WM, int WN, int NS, int TB>
__global__ __launch_bounds__(WM* WN * 64) void dnnopt_tile_f32_dma(TileArgs p) {
    static_assert(TB || NT % 4 == 0, "B stored K x N: whole 64-column groups per wave");
    using SH = TileShape<MT, NT, WM, WN, 1>;
    constexpr int BM = SH::BM, BN = SH::BN;
    constexpr int NW = WM * WN;
    constexpr int BK = 32;
    constexpr int ROWB = BK * 4;  // 128 bytes: one row of A (or of B stored N x K) per block
    constexpr int BROW = BN * 4;  // one k row of B stored K x N
    constexpr int KK = BK / 16;   // fragment reads per row and block
    constexpr int NG = NT / 4;    // 64-column groups per wave (B stored K x N)
    constexpr bool ILV = TB == 0;
    constexpr int A_BYTES = BM * ROWB, B_BYTES = TB ? BN * ROWB : BK * BROW, STAGE = A_BYTES + B_BYTES;
    static_assert(NS >= 2 && NS <= 4, "2 to 4 stages");
    static_assert(A_BYTES % 1024 == 0 && B_BYTES % 1024 == 0, "whole 1 KB wave loads per operand");
    constexpr int UNITS = STAGE / 1024;
    constexpr int IPW = (UNITS + NW - 1) / NW;  // wave loads per wave and block
    __shared__ __attribute__((aligned(1024))) char st0[STAGE];
    __shared__ __attribute__((aligned(1024))) char st1[STAGE];
    __shared__ __attribute__((aligned(1024))) char st2[NS > 2 ? STAGE : 16];
    __shared__ __attribute__((aligned(1024))) char st3[NS > 3 ? STAGE : 16];
    __shared__ __attribute__((aligned(1024))) char spare[UNITS % NW ? 1024 : 16];
    __shared__ float red_unused[1];
    __shared__ int last_flag;
    auto stage = [&](int i) -> char* { return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : st3; };

    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
    const int w = wave_id();
    const int wn = w % WN, wm = w / WN;
    const TileXY tile = xcd_tile((int)blockIdx.x, p.tiles_n, p.tiles_m);
    if (!tile.ok) return;
    const int m0 = tile.m * BM, n0 = tile.n * BN;
    const int nblk = (p.K + BK - 1) / BK;
    const int b_lo = (int)(((long long)nblk * blockIdx.z) / p.splits);
    const int b_hi = (int)(((long long)nblk * (blockIdx.z + 1)) / p.splits);
    const int nb = b_hi - b_lo;

    const char* abase = static_cast<const char*>(p.A) + (size_t)m0 * p.lda * 4;
    const char* bbase = static_cast<const char*>(p.B) + (TB ? (size_t)n0 * p.ldb : (size_t)n0) * 4;
    // Ranges end at the last element of each operand.
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(abase, clamp_rec(((size_t)(p.M - 1 - m0) * p.lda + p.K) * 4));
    const size_t b_last = TB ? (size_t)(p.N - 1 - n0) * p.ldb + p.K : (size_t)(p.K - 1) * p.ldb + (p.N - n0);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bbase, clamp_rec(b_last * 4));

    // This lane's global byte offset (block 0) for each of its wave's loads;
    // rows past M / N, columns past N and padding slots start at kOobOffset
    // (read zero).
    uint32_t goff[IPW];
    bool gb[IPW];
    int unit[IPW];
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
        const int u = j * NW + w;
        unit[j] = u < UNITS ? u : -1;
        gb[j] = u * 1024 >= A_BYTES;
        goff[j] = kOobOffset;
        if (u >= UNITS) continue;
        const int q = u * 1024 + 16 * lane;
        if (q < A_BYTES) {
            const int row = q / ROWB, c = swz_a(row, (q % ROWB) / 16);
            if (m0 + row < p.M) goff[j] = ((uint32_t)row * p.lda + 4 * c) * 4u;
        } else if constexpr (TB) {
            const int qq = q - A_BYTES, row = qq / ROWB, c = swz_a(row, (qq % ROWB) / 16);
            if (n0 + row < p.N) goff[j] = ((uint32_t)row * p.ldb + 4 * c) * 4u;
        } else {
            const int qq = q - A_BYTES, kr = qq / BROW, cb = qq % BROW;
            if (n0 + cb / 4 < p.N) goff[j] = (uint32_t)kr * p.ldb * 4u + (uint32_t)cb;
        }
    }
    // Block `blk` into stage `st`; blocks past the split read nothing
    // (out-of-range offsets) but are issued, so every wave's count of
    // outstanding loads per block is the same.
    auto dma = [&](int st, int blk) {
        const bool live = blk < b_hi;
        const uint32_t ka = live ? (uint32_t)blk * BK * 4u : kOobOffset;
        const uint32_t kb = TB ? ka : (live ? (uint32_t)blk * BK * (uint32_t)p.ldb * 4u : kOobOffset);
        char* base = stage(st);
#pragma unroll
        for (int j = 0; j < IPW; ++j)
            lds_dma16(gb[j] ? rb : ra, unit[j] >= 0 ? base + unit[j] * 1024 : spare, goff[j] + (gb[j] ? kb : ka));
    };

    // LDS byte offsets of this lane's fragment reads.
    int a_rd[KK][MT], b_rd[KK][TB ? NT : 1], b_rdk[KK][4][TB ? 1 : NG];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        const int c = kk * 4 + g;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int row = (wm * MT + mt) * 16 + r;
            a_rd[kk][mt] = row * ROWB + swz_a(row, c) * 16;
        }
        if constexpr (TB) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int n = (wn * NT + nt) * 16 + r;
                b_rd[kk][nt] = A_BYTES + n * ROWB + swz_a(n, c) * 16;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int q = 0; q < NG; ++q)
                    b_rdk[kk][e][q] = A_BYTES + (16 * kk + 4 * g + e) * BROW + ((wn * NG + q) * 64 + 4 * r) * 4;
        }
    }
    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute_blk = [&](int st, int blk, auto tail_tag) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        const char* St = stage(st);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            u32x4 af[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) af[mt] = *reinterpret_cast<const u32x4*>(St + a_rd[kk][mt]);
            const int kv = p.K - (blk * BK + 16 * kk + 4 * g);  // valid k of this lane's chunk
            if constexpr (TAIL) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) af[mt] = keep_dwords(af[mt], kv);
            }
            if constexpr (TB) {
                u32x4 bf[NT];
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    bf[nt] = *reinterpret_cast<const u32x4*>(St + b_rd[kk][nt]);
                    if constexpr (TAIL) bf[nt] = keep_dwords(bf[nt], kv);
                }
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int nt = 0; nt < NT; ++nt)
                            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(as_f32(af[mt][c]), as_f32(bf[nt][c]),
                                                                              acc[mt][nt], 0, 0, 0);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    u32x4 bv[NG];
#pragma unroll
                    for (int q = 0; q < NG; ++q) bv[q] = *reinterpret_cast<const u32x4*>(St + b_rdk[kk][c][q]);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int nt = 0; nt < NT; ++nt)
                            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                                as_f32(af[mt][c]), as_f32(bv[nt / 4][nt & 3]), acc[mt][nt], 0, 0, 0);
                }
            }
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
    // Every copy has landed before the workgroup ends.
    wait_vmcnt<0>();
    tile_finish<MT, NT, WM, WN, 1, ILV>(p, acc, red_unused, &last_flag, w, lane, tile.n, tile.m, p.tiles_n,
                                        p.tiles_n * p.tiles_m);
}

// ---------------------------------------------------------------- launch table
// {MT, NT, WM, WN, KW}
static const TileConfig kTileConfigs[] = {
    {1, 1, 4, 1, 1},  // 0: 64 x 16   tall-skinny, narrow N
    {1, 4, 4, 1, 1},  // 1: 64 x 64   tall-skinny, N = 64
    {2, 2, 2, 2, 1},  // 2: 64 x 64   general / split-k
    {2, 2, 2, 2, 2},  // 3: 64 x 64   k split over 2 waves
    {2, 4, 2, 2, 1},  // 4: 64 x 128
    {4, 4, 2, 2, 1, 2},  // 5: 128 x 128  bf16 through LDS
    {2, 2, 1, 4, 1, 2},  // 6: 32 x 128   bf16 through LDS, small M
    {2, 4, 2, 2, 1, 2},  // 7: 64 x 128   bf16 through LDS
    {4, 4, 2, 2, 1, 3},  // 8: 128 x 128  bf16 through LDS, 3 blocks ahead
    {4, 4, 2, 2, 1, 4},  // 9: 128 x 128  bf16 through LDS, 4 blocks ahead
    {2, 2, 1, 4, 1, 4},  // 10: 32 x 128  bf16 through LDS, 4 blocks ahead
    {2, 4, 2, 2, 1, 4},  // 11: 64 x 128  bf16 through LDS, 4 blocks ahead
    {4, 2, 2, 4, 1, 3},  // 12: 128 x 128 bf16 through LDS, 8 waves, 3 blocks ahead
    {2, 3, 4, 2, 1, 3},  // 13: 128 x 96  bf16 through LDS, 8 waves, 3 blocks ahead
    {2, 3, 4, 2, 1, 2},  // 14: 128 x 96  bf16 through LDS, 8 waves
    {4, 2, 2, 4, 1, 2},  // 15: 128 x 128 bf16 through LDS, 8 waves
    {2, 1, 1, 4, 1, 2, 256},  // 16: 32 x 64  bf16 through LDS, 256 k per block
    {2, 2, 1, 2, 1, 2, 256},  // 17: 32 x 64  bf16 through LDS, 2 waves, 256 k per block
    {2, 2, 1, 4, 1, 2, 128},  // 18: 32 x 128 bf16 through LDS, 128 k per block
    {2, 1, 1, 4, 1, 3, 128},  // 19: 32 x 64  bf16 through LDS, 128 k per block, 3 ahead
    {2, 3, 4, 2, 1, 2, 128},  // 20: 128 x 96 bf16 through LDS, 8 waves, 128 k per block
    {2, 2, 2, 2, 1, 3, 128},  // 21: 64 x 64  bf16 through LDS, 128 k per block, 3 ahead
    {2, 4, 2, 2, 1, 2, 128},  // 22: 64 x 128 bf16 through LDS, 128 k per block
    {2, 2, 2, 4, 1, 2, 128},  // 23: 64 x 128 bf16 through LDS, 8 waves, 128 k per block
    {4, 3, 2, 2, 2, 3},       // 24: 128 x 96  bf16 through LDS, 4 x 2 waves (k-steps split), 3 ahead
    {4, 3, 2, 2, 2, 6},       // 25: 128 x 96  bf16 through LDS, 4 x 2 waves, 6 ahead
    // bf16 storage, LDS DMA: {MT, NT, WM, WN, 1, stages, k per block}
    {2, 3, 4, 2, 1, 3, 64},   // 26: 128 x 96, 3 stages
    {2, 3, 4, 2, 1, 4, 64},   // 27: 128 x 96, 4 stages
    {2, 1, 1, 4, 1, 3, 128},  // 28: 32 x 64, 3 stages of 128 k
    {2, 2, 2, 2, 1, 3, 128},  // 29: 64 x 64, 3 stages of 128 k
    {2, 2, 2, 4, 1, 3, 128},  // 30: 64 x 128, 8 waves, 3 stages of 128 k
    {4, 3, 2, 2, 1, 3, 64},   // 31: 128 x 96, 4 waves, 3 stages
    {2, 4, 4, 2, 1, 3, 64},   // 32: 128 x 128, 8 waves, 3 stages
    {4, 3, 4, 2, 1, 3, 64},   // 33: 256 x 96, 8 waves (64 x 48 each), 3 stages
    {4, 4, 4, 2, 1, 3, 64},   // 34: 256 x 128, 8 waves (64 x 64 each), 3 stages
    // fp32 register tiles for few rows
    {1, 1, 1, 1, 8},          // 35: 16 x 16, k over the 8 waves of a workgroup
    {1, 4, 1, 2, 2},          // 36: 16 x 128, 2 column waves x 2 k-groups
    // bf16 storage through LDS, B stored N x K, few rows
    {2, 1, 1, 3, 1, 3, 128},  // 37: 32 x 48, 3 waves, 128 k per block, 3 ahead
    {1, 1, 1, 3, 1, 3, 128},  // 38: 16 x 48, 3 waves, 128 k per block, 3 ahead
    // bf16 storage, LDS DMA (continued)
    {4, 4, 2, 2, 1, 3, 64},   // 39: 128 x 128, 4 waves of 64 x 64, 3 stages
    // LDS-staged (continued)
    {4, 3, 4, 2, 1, 2, 64},   // 40: 256 x 96, 8 waves of 64 x 48, 64 k per block
    // fp32, LDS DMA: {MT, NT, WM, WN, 1, stages, k per block}
    {2, 4, 2, 2, 1, 3, 32},   // 41: 64 x 128, 4 waves of 32 x 64
    {4, 4, 2, 2, 1, 3, 32},   // 42: 128 x 128, 4 waves of 64 x 64
    {1, 4, 4, 1, 1, 3, 32},   // 43: 64 x 64, 4 waves of 16 x 64
    {2, 4, 4, 1, 1, 3, 32},   // 44: 128 x 64, 4 waves of 32 x 64
    {2, 4, 4, 2, 1, 3, 32},   // 45: 128 x 128, 8 waves of 32 x 64
    {1, 4, 2, 1, 1, 3, 32},   // 46: 32 x 64, 2 waves of 16 x 64
    {1, 4, 4, 2, 1, 3, 32},   // 47: 64 x 128, 8 waves of 16 x 64
    // fp32, LDS DMA, B stored N x K only (wave tiles of 32 columns)
    {1, 2, 2, 1, 1, 3, 32},   // 48: 32 x 32, 2 waves of 16 x 32
    {2, 2, 2, 2, 1, 3, 32},   // 49: 64 x 64, 4 waves of 32 x 32
    {1, 2, 2, 2, 1, 3, 32},   // 50: 32 x 64, 4 waves of 16 x 32
};

int tile_config_count() { return (int)(sizeof(kTileConfigs) / sizeof(kTileConfigs[0])); }
TileConfig tile_config(int idx) { return kTileConfigs[idx]; }

#define DNNOPT_TILE_CASE(IDX, MT, NT, WM, WN, KW)                                                        \
    case IDX:                                                                                            \
        if (mode == kTileF32) {                                                                          \
            if (!ta && !tb) hipLaunchKernelGGL((dnnopt_tile_f32<MT, NT, WM, WN, KW, 0, 0>), grid, blk, 0, s, a); \
            else if (ta && !tb) hipLaunchKernelGGL((dnnopt_tile_f32<MT, NT, WM, WN, KW, 1, 0>), grid, blk, 0, s, a); \
            else if (!ta && tb) hipLaunchKernelGGL((dnnopt_tile_f32<MT, NT, WM, WN, KW, 0, 1>), grid, blk, 0, s, a); \
            else hipLaunchKernelGGL((dnnopt_tile_f32<MT, NT, WM, WN, KW, 1, 1>), grid, blk, 0, s, a);    \
        } else if (mode == kTileBF16 && tb) {                                                            \
            if (al) hipLaunchKernelGGL((dnnopt_tile_bf16<MT, NT, WM, WN, KW, kTileBF16, 1, 1>), grid, blk, 0, s, a); \
            else hipLaunchKernelGGL((dnnopt_tile_bf16<MT, NT, WM, WN, KW, kTileBF16, 0, 1>), grid, blk, 0, s, a);    \
        } else if (mode == kTileBF16) {                                                                  \
            if (al) hipLaunchKernelGGL((dnnopt_tile_bf16<MT, NT, WM, WN, KW, kTileBF16, 1>), grid, blk, 0, s, a); \
            else hipLaunchKernelGGL((dnnopt_tile_bf16<MT, NT, WM, WN, KW, kTileBF16, 0>), grid, blk, 0, s, a);    \
        } else {                                                                                         \
            hipLaunchKernelGGL((dnnopt_tile_bf16<MT, NT, WM, WN, KW, kTileF2B, 1>), grid, blk, 0, s, a);  \
        }                                                                                                \
        break;

#define DNNOPT_TILE_DMA_CASE(IDX, MT, NT, WM, WN, NS, BK)                                                  \
    case IDX:                                                                                              \
        if (mode == kTileBF16 && tb) hipLaunchKernelGGL((dnnopt_tile_bf16_dma<MT, NT, WM, WN, NS, 1, BK>), grid, blk, 0, s, a); \
        else if (mode == kTileBF16) hipLaunchKernelGGL((dnnopt_tile_bf16_dma<MT, NT, WM, WN, NS, 0, BK>), grid, blk, 0, s, a); \
        else return hipErrorInvalidValue;                                                                  \
        break;

#define DNNOPT_TILE_F32DMA_CASE(IDX, MT, NT, WM, WN, NS)                                                 \
    case IDX:                                                                                              \
        if (mode != kTileF32 || ta) return hipErrorInvalidValue;                                           \
        if (tb) hipLaunchKernelGGL((dnnopt_tile_f32_dma<MT, NT, WM, WN, NS, 1>), grid, blk, 0, s, a);       \
        else hipLaunchKernelGGL((dnnopt_tile_f32_dma<MT, NT, WM, WN, NS, 0>), grid, blk, 0, s, a);          \
        break;

#define DNNOPT_TILE_F32DMA_TB_CASE(IDX, MT, NT, WM, WN, NS)                                              \
    case IDX:                                                                                              \
        if (mode != kTileF32 || ta || !tb) return hipErrorInvalidValue;                                    \
        hipLaunchKernelGGL((dnnopt_tile_f32_dma<MT, NT, WM, WN, NS, 1>), grid, blk, 0, s, a);               \
        break;

#define DNNOPT_TILE_LDS_CASE(IDX, MT, NT, WM, WN, D, KB, KW)                                              \
    case IDX:                                                                                              \
        if (mode == kTileBF16 && tb) hipLaunchKernelGGL((dnnopt_tile_bf16_lds<MT, NT, WM, WN, D, kTileBF16, 1, KB, KW>), grid, blk, 0, s, a); \
        else if (mode == kTileBF16) hipLaunchKernelGGL((dnnopt_tile_bf16_lds<MT, NT, WM, WN, D, kTileBF16, 0, KB, KW>), grid, blk, 0, s, a); \
        else if (mode == kTileF2B) hipLaunchKernelGGL((dnnopt_tile_bf16_lds<MT, NT, WM, WN, D, kTileF2B, 0, KB, KW>), grid, blk, 0, s, a); \
        else return hipErrorInvalidValue;                                                                  \
        break;

hipError_t launch_tile(int mode, int cfg_idx, int ta, int tb, int al, dim3 grid, const TileArgs& a, hipStream_t s) {
    // Transposed operands: fp32 both, bf16 storage B only (stored N x K).
    if (mode != kTileF32 && (ta || (tb && mode != kTileBF16))) return hipErrorInvalidValue;
    if (cfg_idx == kTileKOuter) return mode == kTileF32 && ta && !tb ? launch_kouter_f32(grid, a, s) : hipErrorInvalidValue;
    if (cfg_idx < 0 || cfg_idx >= tile_config_count()) return hipErrorInvalidValue;
    const TileConfig c = kTileConfigs[cfg_idx];
    const dim3 blk(c.wm * c.wn * c.kw * 64);
    if (cfg_idx >= kTileFirstLds && !al) return hipErrorInvalidValue;
    switch (cfg_idx) {
        DNNOPT_TILE_CASE(0, 1, 1, 4, 1, 1)
        DNNOPT_TILE_CASE(1, 1, 4, 4, 1, 1)
        DNNOPT_TILE_CASE(2, 2, 2, 2, 2, 1)
        DNNOPT_TILE_CASE(3, 2, 2, 2, 2, 2)
        DNNOPT_TILE_CASE(4, 2, 4, 2, 2, 1)
        DNNOPT_TILE_LDS_CASE(5, 4, 4, 2, 2, 2, 0, 1)
        DNNOPT_TILE_LDS_CASE(6, 2, 2, 1, 4, 2, 0, 1)
        DNNOPT_TILE_LDS_CASE(7, 2, 4, 2, 2, 2, 0, 1)
        DNNOPT_TILE_LDS_CASE(8, 4, 4, 2, 2, 3, 0, 1)
        DNNOPT_TILE_LDS_CASE(9, 4, 4, 2, 2, 4, 0, 1)
        DNNOPT_TILE_LDS_CASE(10, 2, 2, 1, 4, 4, 0, 1)
        DNNOPT_TILE_LDS_CASE(11, 2, 4, 2, 2, 4, 0, 1)
        DNNOPT_TILE_LDS_CASE(12, 4, 2, 2, 4, 3, 0, 1)
        DNNOPT_TILE_LDS_CASE(13, 2, 3, 4, 2, 3, 0, 1)
        DNNOPT_TILE_LDS_CASE(14, 2, 3, 4, 2, 2, 0, 1)
        DNNOPT_TILE_LDS_CASE(15, 4, 2, 2, 4, 2, 0, 1)
        DNNOPT_TILE_LDS_CASE(16, 2, 1, 1, 4, 2, 256, 1)
        DNNOPT_TILE_LDS_CASE(17, 2, 2, 1, 2, 2, 256, 1)
        DNNOPT_TILE_LDS_CASE(18, 2, 2, 1, 4, 2, 128, 1)
        DNNOPT_TILE_LDS_CASE(19, 2, 1, 1, 4, 3, 128, 1)
        DNNOPT_TILE_LDS_CASE(20, 2, 3, 4, 2, 2, 128, 1)
        DNNOPT_TILE_LDS_CASE(21, 2, 2, 2, 2, 3, 128, 1)
        DNNOPT_TILE_LDS_CASE(22, 2, 4, 2, 2, 2, 128, 1)
        DNNOPT_TILE_LDS_CASE(23, 2, 2, 2, 4, 2, 128, 1)
        DNNOPT_TILE_LDS_CASE(24, 4, 3, 2, 2, 3, 0, 2)
        DNNOPT_TILE_LDS_CASE(25, 4, 3, 2, 2, 6, 0, 2)
        DNNOPT_TILE_DMA_CASE(26, 2, 3, 4, 2, 3, 64)
        DNNOPT_TILE_DMA_CASE(27, 2, 3, 4, 2, 4, 64)
        DNNOPT_TILE_DMA_CASE(28, 2, 1, 1, 4, 3, 128)
        DNNOPT_TILE_DMA_CASE(29, 2, 2, 2, 2, 3, 128)
        DNNOPT_TILE_DMA_CASE(30, 2, 2, 2, 4, 3, 128)
        DNNOPT_TILE_DMA_CASE(31, 4, 3, 2, 2, 3, 64)
        DNNOPT_TILE_DMA_CASE(32, 2, 4, 4, 2, 3, 64)
        DNNOPT_TILE_DMA_CASE(33, 4, 3, 4, 2, 3, 64)
        DNNOPT_TILE_DMA_CASE(34, 4, 4, 4, 2, 3, 64)
        DNNOPT_TILE_CASE(35, 1, 1, 1, 1, 8)
        DNNOPT_TILE_CASE(36, 1, 4, 1, 2, 2)
        DNNOPT_TILE_LDS_CASE(37, 2, 1, 1, 3, 3, 128, 1)
        DNNOPT_TILE_LDS_CASE(38, 1, 1, 1, 3, 3, 128, 1)
        DNNOPT_TILE_DMA_CASE(39, 4, 4, 2, 2, 3, 64)
        DNNOPT_TILE_LDS_CASE(40, 4, 3, 4, 2, 2, 64, 1)
        DNNOPT_TILE_F32DMA_CASE(41, 2, 4, 2, 2, 3)
        DNNOPT_TILE_F32DMA_CASE(42, 4, 4, 2, 2, 3)
        DNNOPT_TILE_F32DMA_CASE(43, 1, 4, 4, 1, 3)
        DNNOPT_TILE_F32DMA_CASE(44, 2, 4, 4, 1, 3)
        DNNOPT_TILE_F32DMA_CASE(45, 2, 4, 4, 2, 3)
        DNNOPT_TILE_F32DMA_CASE(46, 1, 4, 2, 1, 3)
        DNNOPT_TILE_F32DMA_CASE(47, 1, 4, 4, 2, 3)
        DNNOPT_TILE_F32DMA_TB_CASE(48, 1, 2, 2, 1, 3)
        DNNOPT_TILE_F32DMA_TB_CASE(49, 2, 2, 2, 2, 3)
        DNNOPT_TILE_F32DMA_TB_CASE(50, 1, 2, 2, 2, 3)
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dnnopt_hip
