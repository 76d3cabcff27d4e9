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

// ---------------------------------------------------------------- A by LDS-DMA
// fp32 tall-skinny GEMM for N <= 16 NT (NT = 1..4) and K = 64 KQ (KQ =
// 1..4), A stored M x K with 16-byte aligned rows.  B is staged once into
// LDS as above; A is copied into LDS by the memory unit (buffer_load ...
// lds) in pieces of 16 rows x PK k, the largest of K, K / 2 and 64 whose
// two slots per wave fit beside B's image.  Each copy instruction moves 64
// lanes x 16 bytes of whole row segments (PK = 256: one 1 KiB row per
// instruction), so HBM sees contiguous row reads where the register-ring
// kernel reads 16 rows x 64 bytes per load, and a wave keeps a whole piece
// in flight without spending registers on it.
//   * 8 waves per workgroup (two per SIMD), each with a private ring of two
//     piece slots, walking its (16-row tile, piece) pairs as one flat
//     sequence: piece i + 1 is copied into the slot piece i - 1 left while
//     piece i's MFMAs run; the wave waits only for its own copies (vmcnt),
//     no barrier after B's staging;
//   * within a slot, row r's 16-byte chunk c sits at physical chunk
//     (c + r) mod (PK / 4) of the row segment (a multiple of 256 bytes), so
//     the 16 rows a quarter-wave reads at one chunk fall in 16 different
//     16-byte bank groups;
//   * MFMA operands as in dnnopt_tall_f32 (lane (r, g) reads k = 16 kc + 4 g
//     .. + 3 of row r, component c feeding MFMA c), in the same k order, so
//     both kernels add the same products in the same order.
//   * with one or two column tiles, where the stream of A bounds the kernel,
//     its copies carry the non-temporal hint (A is read once): MI355X,
//     65536 x 16 x 256 15.9 -> 14.7 us, N = 8 / 12 / 24 / 32 4-9% faster;
//     from three column tiles the MFMAs bound it and the hint measured
//     1-5% slower (N = 48 / 64), so those copies stay plain.
// Measured at 65536 rows against 4 waves with two whole-tile slots, 4 waves
// with 3 / 4 slots, 2 and 3 waves, and 8 waves with one slot: this layout
// is the fastest at K = 192 / 256 for every N and level elsewhere.
constexpr int kTallDmaWaves = 8;
constexpr int kTallDmaSlots = 2;
constexpr int kTallDmaLds = 163840;  // LDS bytes of one workgroup at most

// k per piece for K = 64 kq and nt column tiles (see above).
constexpr bool tall_dma_pk_fits(int kq, int nt, int pk) {
    return kq * 64 * 64 * nt + kTallDmaWaves * kTallDmaSlots * 16 * pk * 4 <= kTallDmaLds;
}
constexpr int tall_dma_pk(int kq, int nt) {
    return tall_dma_pk_fits(kq, nt, kq * 64)                      ? kq * 64
           : (kq % 2 == 0 && tall_dma_pk_fits(kq, nt, kq * 32)) ? kq * 32
                                                                  : 64;
}

template <int KQ, int NT, int TB, int BETA>
__global__ __launch_bounds__(kTallDmaWaves * 64) void dnnopt_tall_dma_f32(TallArgs p) {
    constexpr int W = kTallDmaWaves;
    constexpr int S = kTallDmaSlots;
    constexpr int K = 64 * KQ;
    constexpr int NP = 16 * NT;              // columns of B's image
    constexpr int PK = tall_dma_pk(KQ, NT);  // k per piece
    constexpr int PPT = K / PK;              // pieces per tile
    constexpr int CPR = PK / 4;              // 16-byte chunks per row segment
    constexpr int SEGB = PK * 4;             // bytes per row segment
    constexpr int PIECEB = 16 * SEGB;        // bytes per piece
    constexpr int NI = PIECEB / 1024;        // copy instructions per piece
    constexpr int KCP = PK / 16;             // 16-k chunks per piece (4 MFMAs per column tile each)
    constexpr int BBYTES = K * NP * 4;       // B image, [K/4][NP][4] floats
    static_assert(K % PK == 0 && PK % 64 == 0, "pieces of whole 64-k blocks");
    static_assert((S - 1) * NI < 64, "vmcnt range");
    static_assert(BBYTES + W * S * PIECEB <= kTallDmaLds, "LDS");
    __shared__ __attribute__((aligned(1024))) char lds[BBYTES + W * S * PIECEB];

    const int lane = lane_id(), w = wave_id();
    const int r = lane & 15, g = lane >> 4;
    const int tiles = (p.M + 15) / 16;
    const int gw = (int)blockIdx.x * W + w, GW = (int)gridDim.x * W;
    const int my_tiles = gw < tiles ? (tiles - 1 - gw) / GW + 1 : 0;
    const int total = my_tiles * PPT;  // pieces of this wave
    // The column bias is read with B, before the copies of A.
    const bool has_bias = p.bias != nullptr;
    float biasv[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) biasv[nt] = (has_bias && nt * 16 + r < p.N) ? p.bias[nt * 16 + r] : 0.0f;

    // A's range ends at the last element of row M - 1: rows >= M of the last
    // tile read zero.
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, range31(((size_t)(p.M - 1) * p.lda + K) * 4));
    // Copy instruction j of a piece: lane l fills physical chunk q = 64 j + l
    // of the slot, row q / CPR, with that row segment's chunk
    // (q mod CPR - row) mod CPR.
    uint32_t src[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int q = 64 * j + lane, row = q / CPR, pc = q % CPR;
        const int lc = (pc - row % CPR + CPR) % CPR;
        src[j] = ((uint32_t)row * (uint32_t)p.lda + (uint32_t)lc * 4u) * 4u;
    }
    char* ring = lds + BBYTES + w * S * PIECEB;
    const uint32_t tile_step = 16u * (uint32_t)GW * (uint32_t)p.lda * 4u;
    // Copy cursor: byte offset of the next piece's tile and its piece number.
    uint32_t l_tile = (uint32_t)gw * 16u * (uint32_t)p.lda * 4u;
    int l_p = 0;
    auto copy_piece = [&](int slot) {
        char* dst = ring + slot * PIECEB;
        const uint32_t base = l_tile + (uint32_t)l_p * (uint32_t)SEGB;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            if constexpr (NT <= 2) lds_dma16_stream(ra, dst + j * 1024, src[j] + base);
            else lds_dma16(ra, dst + j * 1024, src[j] + base);
        }
        if (++l_p == PPT) {
            l_p = 0;
            l_tile += tile_step;
        }
    };

    // Stage B (as dnnopt_tall_f32): unit u = (k quad u / NP, column u % NP)
    // is the 16-byte chunk at byte 16 u.
    {
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(
            p.B, range31((TB ? (size_t)(p.N - 1) * p.ldb + K : (size_t)(K - 1) * p.ldb + p.N) * 4));
        constexpr int UNITS = K / 4 * NP;
        constexpr int SU = (UNITS + W * 64 - 1) / (W * 64);  // units per thread
        u32x4 v[SU];
#pragma unroll
        for (int j = 0; j < SU; ++j) {
            const int u = (int)threadIdx.x + j * W * 64;
            const int k0 = 4 * (u / NP), n = u % NP;
            const bool ok = u < UNITS && n < p.N;
            if constexpr (TB) {
                v[j] = buf_load_x4(rb, ok ? ((uint32_t)n * p.ldb + k0) * 4u : kOobOffset);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) v[j][c] = buf_load_x1(rb, ok ? ((uint32_t)(k0 + c) * p.ldb + n) * 4u : kOobOffset);
            }
        }
        // B (and the bias) arrive before the first copies of A go out, so
        // no register the loop uses is still loading when it starts (the
        // compiler would otherwise wait for every copy before the loop).
        // Always S - 1 copies, a fixed sequence the compiler's wait counts
        // see through: past this wave's last piece they read rows of later
        // tiles or out-of-range zeros into its own slots, never consumed.
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) asm volatile("" ::"v"(biasv[nt]));
        wait_vmcnt<0>();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < S - 1; ++i) copy_piece(i);
#pragma unroll
        for (int j = 0; j < SU; ++j) {
            const int u = (int)threadIdx.x + j * W * 64;
            if (u < UNITS) *reinterpret_cast<u32x4*>(lds + (size_t)u * 16) = v[j];
        }
    }
    // B's LDS writes are all the barrier publishes: no wait on the copies of
    // A in flight (each wave waits for its own before reading them).
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    if (total == 0) {
        wait_vmcnt<0>();  // the copies land before the wave ends
        return;
    }

    const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.C, range31(((size_t)(p.M - 1) * p.ldc + p.N) * 4));
    uint32_t lane_c[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) lane_c[e] = ((uint32_t)(4 * g + e) * (uint32_t)p.ldc + (uint32_t)r) * 4u;
    bool col_ok[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) col_ok[nt] = nt * 16 + r < p.N;
    const uint32_t c_step = 16u * (uint32_t)GW * (uint32_t)p.ldc * 4u;
    uint32_t c_off = (uint32_t)gw * 16u * (uint32_t)p.ldc * 4u;
    // This lane's B fragment of 16-k chunk 0, column tile 0; chunk kc adds
    // kc * NP * 64 bytes, column tile nt adds nt * 256.
    const char* b_lane = lds + (g * NP + r) * 16;

    f32x4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float c_old[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) c_old[nt][e] = 0.0f;
    int c_p = 0;  // piece number within the current tile
    for (int i = 0; i < total; ++i) {
        if constexpr (BETA) {
            if (c_p == 0) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        c_old[nt][e] = as_f32(buf_load_x1(rc, col_ok[nt] ? c_off + lane_c[e] + nt * 64u : kOobOffset));
            }
        }
        if (i + S - 1 < total) {
            // The slot piece i - 1 used is refilled once its reads are done;
            // then wait for piece i, leaving the next piece's copies in
            // flight (vector memory operations complete in order; C loads
            // and stores issued meanwhile only make the wait stricter).
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            copy_piece((i + S - 1) % S);
            wait_vmcnt<(S - 1) * NI>();
        } else {
            wait_vmcnt<0>();
        }
        const char* a_row = ring + (i % S) * PIECEB + r * SEGB;
        const char* b_piece = b_lane + c_p * (KCP * NP * 64);
#pragma unroll
        for (int kc = 0; kc < KCP; ++kc) {
            int pc = 4 * kc + g + r;
            if (pc >= CPR) pc -= CPR;
            const u32x4 av = *reinterpret_cast<const u32x4*>(a_row + pc * 16);
            u32x4 bv[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) bv[nt] = *reinterpret_cast<const u32x4*>(b_piece + kc * (NP * 64) + nt * 256);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(as_f32(av[c]), as_f32(bv[nt][c]), acc[nt], 0, 0, 0);
        }
        if (++c_p == PPT) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    float v;
                    if constexpr (BETA) v = __builtin_fmaf(p.alpha, acc[nt][e], p.beta * c_old[nt][e]);
                    else v = p.alpha * acc[nt][e];
                    if (has_bias) v = add_rn(v, biasv[nt]);
                    buf_store_x1(rc, col_ok[nt] ? c_off + lane_c[e] + nt * 64u : kOobOffset, as_u32(v));
                }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
            c_p = 0;
            c_off += c_step;
        }
    }
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

bool tall_dma_fits(int N, int K, int lda) { return N >= 1 && N <= 64 && K % 64 == 0 && K >= 64 && K <= 256 && lda % 4 == 0; }

size_t tall_dma_lds_bytes(int nt, int K) {
    return (size_t)K * 64 * nt + (size_t)kTallDmaWaves * kTallDmaSlots * 16 * tall_dma_pk(K / 64, nt) * 4;
}

int tall_dma_waves() { return kTallDmaWaves; }

template <int KQ, int NT>
static void launch_tall_dma_kq(int tb, dim3 grid, const TallArgs& a, hipStream_t s) {
    const dim3 blk(kTallDmaWaves * 64);
    if (tb) {
        if (a.beta == 0.0f) hipLaunchKernelGGL((dnnopt_tall_dma_f32<KQ, NT, 1, 0>), grid, blk, 0, s, a);
        else hipLaunchKernelGGL((dnnopt_tall_dma_f32<KQ, NT, 1, 1>), grid, blk, 0, s, a);
    } else {
        if (a.beta == 0.0f) hipLaunchKernelGGL((dnnopt_tall_dma_f32<KQ, NT, 0, 0>), grid, blk, 0, s, a);
        else hipLaunchKernelGGL((dnnopt_tall_dma_f32<KQ, NT, 0, 1>), grid, blk, 0, s, a);
    }
}

template <int NT>
static hipError_t launch_tall_dma_nt(int tb, dim3 grid, const TallArgs& a, hipStream_t s) {
    switch (a.K / 64) {
        case 1: launch_tall_dma_kq<1, NT>(tb, grid, a, s); break;
        case 2: launch_tall_dma_kq<2, NT>(tb, grid, a, s); break;
        case 3: launch_tall_dma_kq<3, NT>(tb, grid, a, s); break;
        case 4: launch_tall_dma_kq<4, NT>(tb, grid, a, s); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_tall_dma_f32(int tb, dim3 grid, const TallArgs& a, hipStream_t s) {
    // The kernel's LDS-DMA copies need 16-byte aligned rows of A.
    if (!tall_dma_fits(a.N, a.K, a.lda) || (reinterpret_cast<uintptr_t>(a.A) & 15u) != 0) return hipErrorInvalidValue;
    switch ((a.N + 15) / 16) {
        case 1: return launch_tall_dma_nt<1>(tb, grid, a, s);
        case 2: return launch_tall_dma_nt<2>(tb, grid, a, s);
        case 3: return launch_tall_dma_nt<3>(tb, grid, a, s);
        case 4: return launch_tall_dma_nt<4>(tb, grid, a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dnnopt_hip
