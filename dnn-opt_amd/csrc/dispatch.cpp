// dispatch.cpp -- shape dispatcher for the gfx950 GEMM path.
//
// Replaces the reference's routing (src/gemm/gemm.cpp:175-455), which is
// tuned for Neoverse caches: tiny/GEMV kernels, the small-M wide driver below
// M=8, adaptive register tiles, and a packed BLIS driver with cache-derived
// blocking (src/gemm/gemm_config.h:43-145) and OpenMP decomposition.
//
// On MI355X the questions are different: a launch must put enough bytes in
// flight to cover HBM latency on every compute unit, and the shapes of this
// path are almost all HBM-bound.  The rules:
//   * M <= 8 with B stored N x K (fp32, bf16): the row-dot kernel streams the
//     rows of B once; waves of a workgroup split k when there are too few
//     rows to give every CU two workgroups.
//   * M <= 8 (fp32, bf16): the skinny kernel streams B once.  Work is split
//     over column tiles, over the waves of a workgroup and, when there are too
//     few column tiles to occupy the chip, over k across workgroups (split-k,
//     partials summed in split order by a reduce kernel) -- one 8-wave
//     workgroup per CU.
//   * M > 8 bf16 with 4-byte aligned rows: LDS-staged MFMA tiles (128 x 96
//     with 8 waves above M = 128; 64 x 128, 64 x 64 and 32 x 64 tiles with
//     128-k blocks below), split-k only when the tiles leave more than half
//     of the CUs idle.
//   * fp32 with 12 < N <= 64 (K >= 128 for N <= 16), B small enough for LDS and at least a row
//     tile for most waves of one workgroup per CU (32-row tiles from ~48K
//     rows, 16-row tiles from ~16K rows with K >= 256): B resident in LDS,
//     persistent workgroups stream A (k_tall.hip).
//   * fp32 with A stored K x M and B stored K x N (TransA, NoTrans), 32 < M,
//     N <= 64, K >= 32768, row strides multiples of 4 floats: the k-major
//     outer-product kernel (k_kouter.hip), one workgroup per CU, each a
//     contiguous k-range, partials summed by the split-K reduce kernel.
//   * other M > 8 (fp32, bf16): MFMA tiles sized to the shape (64 x 16 for
//     N <= 16, 64 x 64 otherwise); split-k when the tile count cannot occupy
//     the CUs, with a separate reduce kernel once the split count is large.
//   * int8 (B as N x K): the row-dot kernel (v_dot4) for M <= 4; 16 x 16
//     MFMA tiles with k split over the waves of a workgroup for M <= 16;
//     32 x 32 tiles staged through LDS (256-byte k-blocks) above that (4-byte
//     aligned rows), split-k only when the tiles leave more than half of the
//     CUs idle.
//   The LDS-staged tile and k-split of bf16 storage above M = 128, and of
//   fp32 inputs above M = 64, come from a fitted cost model (pick_tile) when
//   it beats the rule by 5%; the fp32 register tile and k-split (A stored
//   M x K, M >= 12, N >= 64) from another (pick_f32_tile) when it beats the
//   rule by 10%; and, from M = 12, every LDS-staged and LDS-DMA tile and
//   k-split from a third (pick_lds_tile, one parameter set for bf16
//   storage and one for fp32 inputs) when it beats the choice above by 10%
//   (bf16 storage) or 5% (fp32 inputs); fp32 with A stored M x K also
//   prices the fp32 LDS-DMA tiles (the same model form) and takes one where
//   it is 10% ahead of the register tiles' choice, or beyond 10^10 MACs.
//   * any shape whose operand spans none of these kernels can address with
//     32-bit offsets: the 64-bit last-resort kernel (k_wide.hip).
// Tunables (dnnopt_hip_set_tunable; a DNNOPT_TUNING build seeds them from
// these environment variables):
//   DNNOPT_WAVES_PER_CU (default 8), DNNOPT_SKINNY_NW (4, 8 or 16; default 8),
//   DNNOPT_SKINNY_WGS_PER_CU (default 1), DNNOPT_SKINNY_WGS (force G),
//   DNNOPT_MAX_SPLITS (default 256), DNNOPT_SPLIT_REDUCE (0 ticket, 1 the
//   planners' choice, 2 reduce kernel),
//   DNNOPT_TILE_SPLITS (force the k-splits of a tile launch), DNNOPT_TILE_CFG
//   (force a tile configuration: an LDS-staged bf16 one, index 5 and up, or
//   an fp32 register tile, 1-4, 35 or 36; either turns the cost models off),
//   DNNOPT_S8_CFG / DNNOPT_S8_SPLITS (force the int8 configuration / splits),
//   DNNOPT_TALL=0 (keep tall-skinny fp32 GEMMs on the register-only tiles),
//   DNNOPT_TALL_WGS_PER_CU (default 1), DNNOPT_TALL_RT (force 16- or 32-row
//   tall tiles: 1 or 2), DNNOPT_ROWDOT_KW (force the row-dot k-split: 1, 2,
//   4 or 8 waves), DNNOPT_S8_ROWDOT=0 (int8 M <= 4 on
//   the MFMA tiles), DNNOPT_KOUTER=0 (k-major fp32 operands on the register
//   tiles), DNNOPT_KOUTER_WGS_PER_CU (default 1), DNNOPT_WIDE=1 (every
//   fp32 / bf16 / int8 GEMM on the last-resort kernel, for its tests).
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cstdio>

#include "host.h"

namespace dnnopt_hip {

namespace {

// k-major outer-product kernel: k-extent from which it replaces the
// register tiles, and workgroups per CU.
constexpr int kKOuterMinK = 32768;
bool kouter_enabled() { return tunable(kTuneKOuter) != 0; }
int kouter_wgs_per_cu() { return std::max(1, tunable(kTuneKOuterWgsPerCu)); }

int waves_per_cu() { return std::max(1, tunable(kTuneWavesPerCu)); }
// Forced skinny waves per workgroup, or 0 when the planner chooses.
int skinny_nw_forced() {
    const int x = tunable(kTuneSkinnyNW);
    return (x == 4 || x == 8 || x == 16) ? x : 0;
}
int skinny_wgs_per_cu() { return std::max(1, tunable(kTuneSkinnyWgsPerCu)); }
int max_splits() { return std::max(1, tunable(kTuneMaxSplits)); }

}  // namespace

int split_reduce_mode() { return tunable(kTuneSplitReduce) != 0 ? 1 : 0; }

namespace {

// Splits beyond this are reduced by a separate kernel rather than by the
// last-arriving workgroup.
constexpr int kTicketSplitLimit = 16;
constexpr int kTileTicketSplits = 8;  // fp32 tiles: last-workgroup split sums up to this many splits

long long ceil_div(long long a, long long b) { return (a + b - 1) / b; }

void fill_pub(Launch* L, int kernel, const char* name, int rows, int cols, int splits, int block) {
    L->pub.kernel = kernel;
    L->pub.rows = rows;
    L->pub.cols = cols;
    L->pub.splits = splits;
    L->pub.grid_x = (int)L->grid.x;
    L->pub.grid_y = (int)L->grid.y;
    L->pub.grid_z = (int)L->grid.z;
    L->pub.block = block;
    L->pub.workspace_bytes = L->part_bytes + (L->tickets ? kTicketBytes : 0);
    snprintf(L->pub.name, sizeof L->pub.name, "%s", name);
    L->family = kernel;
}

}  // namespace

int plan_skinny(int mode, int M, int N, int K, int ldb, Launch* L) {
    if (M < 1 || M > 8) return DNNOPT_ERR_UNSUPPORTED;
    *L = Launch{};
    const int tw = skinny_tile_cols(mode);
    const int es = skinny_elem_bytes(mode);
    const long long T = ceil_div(N, tw);
    const long long cus = num_cus();
    // Every wave should own at least one unrolled step of rows; problems too
    // small to give every CU a workgroup of 8 such waves use 4-wave groups.
    int nw = skinny_nw_forced();
    if (nw == 0) nw = T * std::max<long long>(1, K / (8ll * kSkinnyUnroll)) < cus ? 4 : 8;
    const long long smax = std::max<long long>(1, K / ((long long)nw * kSkinnyUnroll));
    // G workgroups, about skinny_wgs_per_cu() per CU, shared by the T column
    // tiles as G/T or G/T + 1 k-splits each (balanced work per workgroup).
    // When there is more than one CU's worth of work, G is a whole multiple
    // of the CU count so that no CU runs one workgroup more than the others
    // (then adjusted to whole splits per tile, below).
    const long long g_target = cus * skinny_wgs_per_cu();
    long long G;
    if (T >= g_target) {
        G = T;
    } else {
        G = std::min<long long>(g_target, T * smax);
        if (G >= cus) G = std::max<long long>(T, G / cus * cus);
    }
    // Whole splits per column tile: the workgroups of a tile with one split
    // fewer run longer and set the kernel's time, so an uneven share is
    // rounded -- up when the last tile is at most a quarter wide (its
    // workgroups finish early and the extra ones take over their CUs; N = 4099:
    // 272 instead of 256 workgroups, 1-3% faster), else down when that idles
    // at most a fifth of the CUs (N = 11003: 215, 4% faster; bf16 N = 11008:
    // 242, 4% faster).
    if (G > T && G % T != 0) {
        if (N - (T - 1) * tw <= tw / 4)
            G = std::min<long long>(ceil_div(G, T) * T, T * smax);
        else if (G % T * 5 <= G)
            G = G / T * T;
    }
    const int forced = tunable(kTuneSkinnyWgs);
    if (forced > 0) G = std::min<long long>(std::max<long long>(forced, T), T * smax);
    G = std::max<long long>(G, T);
    // Keep per-workgroup buffer offsets inside 31 bits: more splits shorten
    // the k-range of a workgroup.
    auto span_ok = [&](long long g) { return ceil_div(K, g / T) * (long long)ldb * es + (long long)tw * es < 0x7FFFFFFFll; };
    while (!span_ok(G) && G / T < K) G += T;
    if (!span_ok(G) || G > 0x7FFFFFFFll) return DNNOPT_ERR_UNSUPPORTED;
    if (G > T && T > kMaxTickets && tunable(kTuneSplitReduce) == 0) return DNNOPT_ERR_UNSUPPORTED;
    const long long smax_tile = ceil_div(G, T);
    L->mode = mode;
    L->mr = M;
    L->nw = nw;
    // fp32 with 8-wave groups streams 4-row load blocks (MI355X, us, 16 -> 4
    // rows: C1 15.2 -> 14.5; C2 N = 4099 / 11003 about 0.6 us less per GEMM);
    // the split points stay those of 16-row units (the planner's unit).
    L->unroll = (mode == kSkinnyF32 && nw == 8) ? 4 : 16;
    L->tiles = (int)T;
    L->grid = dim3((unsigned)G, 1, 1);
    // Split-k sums: the last-arriving workgroup of a tile adds the partials
    // itself (one kernel) when they are few rows and few bytes, else the
    // reduce kernel (MI355X, graph replays, us: C1 14.57 -> 14.23, bf16 1 x
    // 11008 x 4096 18.77 -> 18.05, M = 2 / 3 x 4099 / 11003 0.1 less; but M
    // = 5 x 11003 (25 KiB) +0.43, M = 2 x 1009 (64 KiB) +0.30, M = 7 x 1009
    // (224 KiB) +2.6).
    const int srm = tunable(kTuneSplitReduce);
    const bool ticket = srm == 0 || (srm == 1 && M <= 3 && T <= kMaxTickets &&
                                     smax_tile * M * tw * 4 <= kSkinnyTicketBytes);
    L->defer_reduce = (G > T && !ticket) ? 1 : 0;
    L->part_bytes = G > T ? (size_t)smax_tile * M * T * tw * sizeof(float) : 0;
    L->tickets = (G > T && !L->defer_reduce) ? (int)T : 0;
    const int kernel = mode == kSkinnyF32 ? DNNOPT_K_SKINNY_F32
                       : mode == kSkinnyBF16 ? DNNOPT_K_SKINNY_BF16
                                             : DNNOPT_K_SKINNY_F2B;
    fill_pub(L, kernel, "dnnopt_skinny", M, tw, (int)smax_tile, nw * 64);
    return DNNOPT_OK;
}

// k-major fp32 operands (A stored K x M, B stored K x N) with 32 < M, N <= 64
// and a long k: the outer-product kernel streams both panels with 16-byte
// loads, one 4-wave workgroup per CU, each summing a contiguous k-range.
int plan_kouter(int M, int N, int K, int lda, int ldb, Launch* L) {
    const long long cus = num_cus();
    const long long nsteps = ((long long)K + 3) / 4;
    const int forced_splits = tunable(kTuneTileSplits);
    long long s = forced_splits > 0 ? forced_splits : cus * kouter_wgs_per_cu();
    s = std::min<long long>(s, std::max<long long>(1, nsteps / 16));
    // 32-bit offsets within one split's rows (plus one 16-row step).
    const long long ld = std::max(lda, ldb);
    while ((((nsteps + s - 1) / s) * 4 + 16) * ld * 4 >= 0x7FFFFFFFll && s < nsteps) s *= 2;
    s = std::min(s, nsteps);
    if ((((nsteps + s - 1) / s) * 4 + 16) * ld * 4 >= 0x7FFFFFFFll || s > 65535) return DNNOPT_ERR_UNSUPPORTED;
    L->mode = kTileF32;
    L->cfg = kTileKOuter;
    L->bm = 64;
    L->bn = 64;
    L->tn = 1;
    L->tm = 1;
    L->grid = dim3(1, 1, (unsigned)s);
    L->defer_reduce = 1;
    L->part_bytes = (size_t)s * 64 * 64 * sizeof(float);
    L->tickets = 0;
    (void)M;
    (void)N;
    fill_pub(L, DNNOPT_K_TILE_F32, "dnnopt_kouter_f32", 64, 64, (int)s, 256);
    return DNNOPT_OK;
}

// The LDS-staged tile and k-split count from a cost model fitted on MI355X.
// Every workgroup owns one CU, so a launch of W workgroups takes ceil(W /
// CUs) rounds of one workgroup's time: the MACs of its tile and k-range at a
// per-configuration rate, plus a fixed cost per round; a k-split adds its
// fp32 partial tiles, written and read at 5 TB/s, and 3 us for the reduce
// launch.  Rates (us per MAC) and fixed costs (us per round):
//   bf16 storage (LDS DMA; M = 96..512, N = 2048..11008, K = 1024 and 4096,
//   B stored K x N and N x K, within about 10% of every point measured):
//   128 x 96 on 8 waves of 32 x 48 0.83e-6, 256 x 96 on 8 waves of 64 x 48
//   0.57e-6, 128 x 128 on 4 waves of 64 x 64 0.715e-6, no fixed cost;
//   fp32 inputs rounded in registers (M = 96..512, N = 4096 and 11008, K =
//   1024 and 4096; the pick is within 1% of the best of 6 measured choices
//   on 21 of 24 shapes): 128 x 96 1.35e-6 + 3 us, 256 x 96 1.15e-6 + 9 us.
struct TilePick {
    int cfg;
    long long s;
    double us;
};

static double tile_cost(int mode, int cfg, long long s, int M, int N, int K, long long cus) {
    const TileConfig c = tile_config(cfg);
    const int bm = c.wm * c.mt * 16, bn = c.wn * c.nt * 16;
    const int kb = tile_lds_bk(bm, bn, c.kblk);
    const long long tiles = ceil_div(M, bm) * ceil_div(N, bn), nblk = ceil_div(K, kb);
    double rate, fixed = 0.0;
    if (mode == kTileF2B) {
        rate = cfg == kTileF2BTall ? 1.15e-6 : 1.35e-6;
        fixed = cfg == kTileF2BTall ? 9.0 : 3.0;
    } else {
        rate = cfg == 33 ? 0.57e-6 : (cfg == kTileBF16Dma4w ? 0.715e-6 : 0.83e-6);
    }
    const double macs = (double)bm * bn * (double)ceil_div(nblk, s) * kb;
    double us = (double)ceil_div(tiles * s, cus) * (macs * rate + fixed);
    if (s > 1) us += 2.0 * (double)s * tiles * bm * bn * 4 / 5e6 + 3.0;
    return us;
}

// k-splits of an LDS-staged tile launch by the occupancy rule: one workgroup
// per CU is the unit of work, so split k only when the tiles leave more than
// half of the CUs idle.
static long long lds_rule_splits(int cfg, int M, int N, int K) {
    const TileConfig c = tile_config(cfg);
    const int bm = c.wm * c.mt * 16, bn = c.wn * c.nt * 16;
    const long long tiles = ceil_div(M, bm) * ceil_div(N, bn), nblk = ceil_div(K, tile_lds_bk(bm, bn, c.kblk));
    const long long cus = num_cus();
    if (tiles * 2 >= cus) return 1;
    return std::min<long long>({ceil_div(cus, tiles), std::max<long long>(1, nblk / 2), (long long)max_splits()});
}

// The measured default (def_cfg, split by the LDS rule) unless the model puts
// another candidate at least 5% ahead.
static TilePick pick_tile(int mode, int M, int N, int K, int def_cfg, bool tall_ok) {
    const long long cus = num_cus();
    const long long s_def = lds_rule_splits(def_cfg, M, N, K);
    TilePick best{def_cfg, s_def, tile_cost(mode, def_cfg, s_def, M, N, K, cus)};
    const double def_us = best.us;
    static const int kBf16[] = {26, 33, kTileBF16Dma4w};
    static const int kF2B[] = {20, kTileF2BTall};
    const int* cand = mode == kTileF2B ? kF2B : kBf16;
    const int ncand = mode == kTileF2B ? (tall_ok ? 2 : 1) : 3;
    for (int i = 0; i < ncand; ++i) {
        const int cfg = cand[i];
        const TileConfig c = tile_config(cfg);
        const long long nblk = ceil_div(K, tile_lds_bk(c.wm * c.mt * 16, c.wn * c.nt * 16, c.kblk));
        const long long smax = std::min<long long>({16, std::max<long long>(1, nblk / 2), (long long)max_splits()});
        for (long long s = 1; s <= smax; ++s) {
            const double us = tile_cost(mode, cfg, s, M, N, K, cus);
            if (us < best.us) best = TilePick{cfg, s, us};
        }
    }
    if (best.us > 0.95 * def_us) return TilePick{def_cfg, s_def, def_us};
    return best;
}

// LDS-staged tiles (bf16 storage from M = 12, fp32 inputs from M = 12; N >=
// 64): every LDS-staged and LDS-DMA tile and k-split priced by models fitted
// on MI355X.  A launch of W workgroups gives each CU ceil(W / CUs) of them,
// occ at a time (the configuration's workgroups per CU, from its LDS and
// register use); a workgroup fills its pipeline once (fill) and then takes
// max(m, c) per k-block times the workgroups sharing its CU, m being the
// block's MFMAs per SIMD (16 cycles each at 2.4 GHz, times a fitted factor)
// and c the copy of its A and B block at a fitted cost per byte; the whole
// launch takes at least its operands' and C's bytes at the fitted HBM rate;
// a fixed cost per launch, and a k-split adds a fixed cost plus its fp32
// partials written and read at the fitted rate.
//   bf16 storage: 248 measured cases (M = 12..4096, N = 64..11008, K =
//   64..4608, both B layouts; 14 configurations, 1 to 16 splits; median
//   error 7%, 90% of the cases within 19%); 2.72 us per launch, 3.3 TB/s;
//   a split 1.83 us plus its partials at 6.8 TB/s.
//   fp32 inputs rounded in registers: 124 measured cases (same shapes, B
//   stored K x N; 9 configurations; median error 6%, 90% within 17%); 1.99 us
//   per launch, 3.3 TB/s; a split 2.73 us plus its partials at 6.6 TB/s.
struct LdsFit {
    int cfg, tb, occ;
    double fill, mfma, ps_per_byte;
};
struct LdsModel {
    const LdsFit* fits;
    int n;
    int es;              // operand bytes per element
    double mfma_cyc_k;   // MFMA cycles per k of one 16 x 16 tile (bf16 16x16x32: 0.5, fp32 16x16x4: 8)
    double launch_us, split_us, partial_ps, hbm_ps;
};
static const LdsFit kBf16Fit[] = {
    {19, 0, 2, 1.554, 7.035, 12.05}, {19, 1, 2, 1.754, 3.739, 14.44}, {21, 0, 2, 2.192, 3.347, 16.11},
    {21, 1, 1, 2.300, 2.732, 17.49}, {22, 0, 1, 2.550, 1.912, 20.50}, {22, 1, 1, 2.924, 2.862, 18.74},
    {23, 0, 1, 2.333, 0.400, 17.36}, {23, 1, 1, 2.396, 0.353, 16.76}, {26, 0, 1, 2.293, 3.010, 16.87},
    {26, 1, 1, 2.139, 0.636, 15.85}, {28, 0, 1, 1.974, 1.334, 20.25}, {28, 1, 2, 1.632, 0.602, 12.84},
    {29, 0, 1, 2.686, 1.010, 19.61}, {29, 1, 1, 2.165, 1.259, 16.65}, {30, 0, 1, 2.417, 0.847, 15.05},
    {30, 1, 1, 2.482, 2.219, 14.83}, {31, 0, 1, 2.905, 0.051, 19.32}, {31, 1, 1, 2.678, 0.893, 18.93},
    {32, 0, 1, 2.479, 1.655, 15.85}, {32, 1, 1, 2.427, 0.941, 15.87}, {33, 0, 1, 2.957, 0.035, 16.75},
    {33, 1, 1, 2.869, 2.173, 15.43}, {37, 1, 2, 1.792, 1.107, 14.87}, {38, 1, 2, 1.478, 0.319, 15.10},
    {39, 0, 1, 3.676, 1.549, 18.18}, {39, 1, 2, 3.846, 0.005, 19.16},
};
static const LdsFit kF2BFit[] = {
    {14, 0, 1, 2.250, 7.797, 21.59}, {16, 0, 1, 2.357, 1.674, 22.14}, {18, 0, 1, 2.400, 2.607, 20.58},
    {19, 0, 2, 2.255, 1.381, 16.62}, {20, 0, 1, 3.124, 6.880, 6.68}, {21, 0, 1, 2.956, 5.461, 19.89},
    {22, 0, 1, 3.047, 0.031, 22.17}, {23, 0, 1, 2.674, 0.063, 19.12}, {40, 0, 1, 3.112, 5.685, 17.17},
};
// fp32 LDS-DMA tiles (A stored M x K; the 32-column wave tiles with B
// stored N x K only): 320 measured cases (M = 10..12544, N = 64..11008, K =
// 64..4608; 10 configurations, 1 to 16 splits; median error 5%, 90% within
// 19%); 4.72 us per launch, 3.5 TB/s; a split 1.25 us plus its partials at
// 4.6 TB/s.
static const LdsFit kF32DmaFit[] = {
    {41, 0, 2, 2.274, 1.228, 0.26}, {41, 1, 2, 0.261, 1.185, 19.57}, {42, 0, 1, 4.514, 1.193, 8.00},
    {42, 1, 1, 1.171, 1.155, 34.31}, {43, 0, 3, 1.236, 1.247, 11.13}, {43, 1, 3, 0.000, 1.186, 11.69},
    {44, 0, 2, 2.429, 1.212, 17.13}, {44, 1, 2, 0.217, 1.184, 41.16}, {45, 0, 1, 3.863, 1.126, 7.86},
    {45, 1, 1, 0.237, 1.148, 2.48}, {46, 0, 4, 1.143, 1.949, 31.79}, {46, 1, 4, 0.083, 1.846, 15.47},
    {47, 0, 2, 2.006, 1.152, 9.30}, {47, 1, 2, 0.074, 1.122, 19.73}, {48, 1, 6, 0.000, 1.683, 3.93},
    {49, 1, 3, 0.000, 1.171, 20.76}, {50, 1, 4, 0.000, 1.212, 12.92},
};
static const LdsModel kBf16Model{kBf16Fit, (int)(sizeof kBf16Fit / sizeof kBf16Fit[0]), 2, 0.5, 2.72, 1.83, 0.1467, 0.2994};
static const LdsModel kF32DmaModel{kF32DmaFit, (int)(sizeof kF32DmaFit / sizeof kF32DmaFit[0]), 4, 8.0, 4.72, 1.25, 0.2168, 0.2869};
static const LdsModel kF2BModel{kF2BFit, (int)(sizeof kF2BFit / sizeof kF2BFit[0]), 4, 0.5, 1.99, 2.73, 0.1509, 0.3039};

static double lds_tile_cost(const LdsModel& md, const LdsFit& f, long long s, int M, int N, int K, long long cus) {
    const TileConfig c = tile_config(f.cfg);
    const int bm = c.wm * c.mt * 16, bn = c.wn * c.nt * 16, kb = tile_lds_bk(bm, bn, c.kblk);
    const long long tiles = ceil_div(M, bm) * ceil_div(N, bn), nblk = ceil_div(K, kb);
    s = std::min(s, nblk);
    const long long per_cu = ceil_div(tiles * s, cus), resident = std::min<long long>(f.occ, per_cu);
    const double m = c.wm * c.wn * c.kw / 4.0 * c.mt * c.nt * kb * md.mfma_cyc_k / 2400.0 * f.mfma;
    const double copy = (double)(bm + bn) * kb * md.es * f.ps_per_byte * 1e-6;
    const double core =
        (double)ceil_div(per_cu, f.occ) * (f.fill + (double)ceil_div(nblk, s) * resident * std::max(m, copy));
    const double hbm = ((double)md.es * ((double)M * K + (double)K * N) + 4.0 * M * N) * md.hbm_ps * 1e-6;
    double us = md.launch_us + std::max(core, hbm);
    if (s > 1) us += md.split_us + 2.0 * (double)s * tiles * bm * bn * 4 * md.partial_ps * 1e-6;
    return us;
}

// The model's best configuration and split count of layout tb among those
// `usable` accepts (s = 0 when there is none).
template <class Usable>
static TilePick best_lds_tile(const LdsModel& md, int tb, int M, int N, int K, Usable usable) {
    const long long cus = num_cus();
    TilePick best{0, 0, 0.0};
    for (int i = 0; i < md.n; ++i) {
        const LdsFit& f = md.fits[i];
        if (f.tb != tb || !usable(f.cfg)) continue;
        const TileConfig c = tile_config(f.cfg);
        const long long nblk = ceil_div(K, tile_lds_bk(c.wm * c.mt * 16, c.wn * c.nt * 16, c.kblk));
        for (long long s : {1, 2, 4, 8, 16}) {
            if (s > nblk || s > max_splits()) break;
            const double us = lds_tile_cost(md, f, s, M, N, K, cus);
            if (best.s == 0 || us < best.us) best = TilePick{f.cfg, s, us};
        }
    }
    return best;
}

// The given default (configuration, k-splits) unless the model puts another
// choice at least `margin` ahead (s = 0 in the result: keep the default).
// tall_ok: 256-row register-ring tiles may be used (C offsets fit).
static TilePick pick_lds_tile(const LdsModel& md, int tb, int M, int N, int K, int def_cfg, long long def_s,
                              double margin, bool tall_ok) {
    const long long cus = num_cus();
    const LdsFit* d = nullptr;
    for (int i = 0; i < md.n; ++i)
        if (md.fits[i].cfg == def_cfg && md.fits[i].tb == tb) d = &md.fits[i];
    if (!d) return TilePick{def_cfg, 0, 0.0};
    const double def_us = lds_tile_cost(md, *d, def_s, M, N, K, cus);
    TilePick best{def_cfg, 0, def_us};
    for (int i = 0; i < md.n; ++i) {
        const LdsFit& f = md.fits[i];
        if (f.tb != tb || (f.cfg == kTileF2BTall && !tall_ok)) continue;
        const TileConfig c = tile_config(f.cfg);
        const long long nblk = ceil_div(K, tile_lds_bk(c.wm * c.mt * 16, c.wn * c.nt * 16, c.kblk));
        for (long long s : {1, 2, 4, 8, 16}) {
            if (s > nblk || s > max_splits()) break;
            const double us = lds_tile_cost(md, f, s, M, N, K, cus);
            if (us < best.us) best = TilePick{f.cfg, s, us};
        }
    }
    if (best.us > (1.0 - margin) * def_us) return TilePick{def_cfg, 0, def_us};
    return best;
}

// k-splits of an fp32 register-tile launch by the occupancy rule: split k
// when the tiles give fewer workgroups than waves_per_cu() waves on every CU.
static long long reg_tile_splits(int cfg, int M, int N, int K) {
    const TileConfig c = tile_config(cfg);
    const int bm = c.wm * c.mt * 16, bn = c.wn * c.nt * 16;
    const long long tiles = ceil_div(M, bm) * ceil_div(N, bn), nblk = ceil_div(K, 64);
    const long long target_wgs = num_cus() * waves_per_cu() / (c.wm * c.wn * c.kw);
    if (tiles >= target_wgs) return 1;
    return std::max<long long>(1, std::min<long long>({ceil_div(target_wgs, tiles),
                                                      std::max<long long>(1, nblk / (2 * c.kw)),
                                                      (long long)max_splits()}));
}

// fp32 register tiles (A stored M x K, M >= 12, N >= 64, at most 10^10
// MACs): the configuration and k-split from a cost model fitted on MI355X
// (320 measured cases: M = 10..12544, N = 64..11008, K = 64..4608, B stored
// K x N and N x K; six configurations, 1 to 16 splits; median error 5%, 90%
// of the cases within 13%).  A launch of W waves gives each SIMD ceil(W / (4
// CUs)) waves, occ of them resident at a time (the configuration's
// occupancy, from its register use); each of a wave's 64-k blocks takes
// max(lat + m, r m), m being the block's 16 MT NT MFMAs (32 cycles at 2.4
// GHz, times a fitted factor) and r the waves resident on its SIMD; every CU
// also reads its workgroups' A and B tiles (at a fitted cost per byte);
// 3.23 us per launch, and a k-split adds 2.22 us plus its fp32 partials
// written and read at 6.4 TB/s.
struct F32Fit {
    int cfg, tb, occ;
    double lat, mfma, ps_per_byte;
};
static const F32Fit kF32Fit[] = {
    {1, 0, 4, 0.394, 0.140, 45.3}, {1, 1, 4, 0.762, 0.297, 55.9}, {2, 0, 4, 0.502, 0.185, 41.9},
    {2, 1, 8, 1.130, 0.189, 46.6}, {3, 0, 4, 0.558, 0.371, 39.3}, {3, 1, 8, 0.978, 0.163, 48.8},
    {4, 0, 3, 0.638, 0.119, 50.6}, {4, 1, 4, 2.089, 0.406, 45.1}, {35, 0, 8, 0.457, 1.144, 15.0},
    {35, 1, 8, 0.248, 0.785, 20.7}, {36, 0, 4, 0.707, 0.251, 14.5}, {36, 1, 4, 0.952, 0.249, 25.5},
};

static double f32_tile_cost(const F32Fit& f, long long s, int M, int N, int K, long long cus) {
    const TileConfig c = tile_config(f.cfg);
    const int bm = c.wm * c.mt * 16, bn = c.wn * c.nt * 16;
    const long long tiles = ceil_div(M, bm) * ceil_div(N, bn), nblk = ceil_div(K, 64);
    s = std::min(s, nblk);
    const long long blocks = ceil_div(nblk, s * c.kw);  // k-blocks of one wave
    const long long per_simd = ceil_div(tiles * s * c.wm * c.wn * c.kw, cus * 4);
    const long long resident = std::min<long long>(f.occ, per_simd);
    const double m = 16.0 * c.mt * c.nt * 32 / 2400.0 * f.mfma;
    double us = 3.23 + (double)ceil_div(per_simd, f.occ) * (double)blocks * std::max(f.lat + m, (double)resident * m);
    us += (double)ceil_div(tiles * s, cus) * (bm + bn) * (double)(ceil_div(nblk, s) * 64) * 4 * f.ps_per_byte * 1e-6;
    if (s > 1) us += 2.22 + 2.0 * (double)s * tiles * bm * bn * 4 * 0.1574e-6;
    return us;
}

// The rule's configuration and split count unless the model puts another
// choice at least 10% ahead.
static TilePick pick_f32_tile(int tb, int M, int N, int K, int def_cfg) {
    const long long cus = num_cus(), def_s = reg_tile_splits(def_cfg, M, N, K);
    const F32Fit* d = nullptr;
    for (const F32Fit& f : kF32Fit)
        if (f.cfg == def_cfg && f.tb == tb) d = &f;
    if (!d) return TilePick{def_cfg, 0, 0.0};
    const double def_us = f32_tile_cost(*d, def_s, M, N, K, cus);
    TilePick best{def_cfg, def_s, def_us};
    const long long nblk = ceil_div(K, 64);
    for (const F32Fit& f : kF32Fit) {
        if (f.tb != tb) continue;
        for (long long s : {1, 2, 3, 4, 6, 8, 12, 16}) {
            if (s > nblk || s > max_splits()) break;
            const double us = f32_tile_cost(f, s, M, N, K, cus);
            if (us < best.us) best = TilePick{f.cfg, s, us};
        }
    }
    if (best.us > 0.9 * def_us) return TilePick{def_cfg, 0, def_us};
    return best;
}

// fp32 LDS-DMA tiles address A from the tile's first row and B from its
// first row (N x K) or column (K x N) with 32-bit offsets over all of k; the
// 32-column wave tiles need B stored N x K.
static bool f32_dma_fits(int cfg, int transA, int transB, int M, int K, int lda, int ldb) {
    (void)M;
    if (transA || (!transB && cfg >= kTileF32DmaTbFirst)) return false;
    const TileConfig c = tile_config(cfg);
    const long long bm = c.wm * c.mt * 16, bn = c.wn * c.nt * 16;
    return (bm * lda + K) * 4 < 0x7FFFFFFFll &&
           (transB ? (bn * ldb + K) : ((long long)K * ldb + bn)) * 4 < 0x7FFFFFFFll;
}

int plan_tile(int mode, int transA, int transB, int M, int N, int K, int lda, int ldb, Launch* L, bool lds_ok,
              int ldc) {
    *L = Launch{};
    if (ldc <= 0) ldc = N;
    if (mode == kTileF32 && transA && !transB && lds_ok && kouter_enabled() && M > 32 && M <= 64 && N > 32 &&
        N <= 64 && K >= kKOuterMinK && (lda & 3) == 0 && (ldb & 3) == 0 &&
        plan_kouter(M, N, K, lda, ldb, L) == DNNOPT_OK)
        return DNNOPT_OK;
    *L = Launch{};
    const long long es = mode == kTileBF16 ? 2 : 4;
    // bf16 GEMMs with 4-byte aligned rows go through the LDS-staged kernel
    // (B stored N x K too, for bf16 storage).
    const bool lds = mode != kTileF32 && lds_ok && !transA && (!transB || mode == kTileBF16) &&
                     (mode == kTileF2B || ((lda & 1) == 0 && (ldb & 1) == 0)) &&
                     ((long long)(M + 128) * lda + K) * es < 0x7FFFFFFFll &&
                     (transB ? ((long long)(N + 128) * ldb + K) : ((long long)K * ldb + N)) * es < 0x7FFFFFFFll &&
                     (long long)128 * ldc * 4 < 0x7FFFFFFFll;
    int cfg;
    long long model_splits = 0;  // the cost model's split count
    const int forced_cfg = tunable(kTuneTileCfg);
    if (lds) {
        // 128 k per LDS block below M = 128 (fewer barriers, more bytes per
        // block in flight); measured on MI355X at N = 11008, K = 4096.
        cfg = M > 128 ? 13 : (M > 64 ? 23 : (M > 32 ? 21 : 19));
        // B stored N x K (bf16 storage), M <= 32: 48-column tiles, more of
        // them over the CUs (MI355X, us, 32 x 64 -> 32 x 48 / 16 x 48, N =
        // 11008, K = 4096: M=32 25.8 -> 24.6, M=24 24.8 -> 23.6, M=16 23.9 ->
        // 22.7 (16 x 48), M=8 21.2 -> 20.4 (16 x 48)).  A K x N B keeps the
        // 64-column tiles (48 columns: 34 vs 26 us at M=32).
        if (transB && mode == kTileBF16 && M <= 32) cfg = M <= 16 ? kTileBF16Tb48Few : kTileBF16Tb48;
        // fp32 inputs rounded in registers, M > 64: 128 x 96 tiles with 128 k
        // per block (MI355X, us, N = 11008, K = 4096: M = 72 / 96 / 128 / 256
        // / 512 72.7 / 75.4 / 79.8 / 97.1 / 174.8 -> 67.1 / 69.3 / 73.6 / 84.5
        // / 162.3; 1024 x 4096 x 4096 156.1 -> 144.6).  The cost model may
        // pick another split count or 256 x 96 tiles (register ring, 64 k
        // per block; measured, us, default -> picked: 128 x 11008 x 1024 32.4
        // -> 23.4 (2 splits instead of 3), 256 x 4096 x 4096 62.1 -> 47.1 (2
        // instead of 3), 512 x 11008 x 4096 145.7 -> 121.5 (256 x 96)).
        if (mode == kTileF2B && M > 64) cfg = 20;
        // bf16 storage above M = 128: the same 128 x 96 tile with the
        // operands copied into LDS by the memory unit (C4 M=256 43.1 vs 45.4
        // us; no gain measured at M = 32).  When 128-row tiles would take more
        // than one round over the CUs, 256 x 96 tiles (64 x 48 per wave: 30%
        // fewer LDS bytes read per MFMA) in fewer rounds: 512 x 11008 x 4096
        // 67 vs 86 us, 1024 x 4096 x 4096 58 vs 77 us, 384 x 11008 x 4096 66
        // vs 82 us; 512 x 4096 x 4096 (one round of 128-row tiles) keeps the
        // 128-row tile, 42 vs 51 us.  Where the cost model above puts another
        // tile or split count at least 5% ahead, that one (measured, us,
        // default -> picked: 256 x 4096 x 4096 35.7 -> 22.2 on 128 x 128 with
        // 4 splits, 192 x 8192 x 4096 38.4 -> 31.5 (128 x 128, 2 splits),
        // 384 x 8192 x 4096 53.2 -> 47.0 (128 x 128), 512 x 2048 x 4096 30.8
        // -> 22.1; C4's 256 x 11008 x 4096 keeps 128 x 96).
        if (M > 128 && mode == kTileBF16) {
            cfg = 26;
            if (ceil_div(M, 128) * ceil_div(N, 96) > num_cus()) cfg = 33;
        }
        // 256-row register-staged tiles: 32-bit C offsets over 256 rows.
        const bool tall_ok = 256LL * ldc * 4 < 0x7FFFFFFFll;
        const bool nothing_forced = forced_cfg < kTileFirstLds && tunable(kTuneTileSplits) <= 0;
        if (nothing_forced && ((M > 128 && mode == kTileBF16) || (M > 64 && mode == kTileF2B))) {
            const TilePick pick = pick_tile(mode, M, N, K, cfg, tall_ok);
            cfg = pick.cfg;
            model_splits = pick.s;
        }
        // From M = 12: every LDS-staged tile and split priced by the second
        // models, against that choice (bf16 storage: 10% margin, fp32
        // inputs: 5%).
        if (nothing_forced && M >= 12 && N >= 64) {
            const long long def_s = model_splits > 0 ? model_splits : lds_rule_splits(cfg, M, N, K);
            const TilePick pick = mode == kTileBF16
                                      ? pick_lds_tile(kBf16Model, transB ? 1 : 0, M, N, K, cfg, def_s, 0.10, false)
                                      : pick_lds_tile(kF2BModel, 0, M, N, K, cfg, def_s, 0.05, tall_ok);
            if (pick.s > 0) {
                cfg = pick.cfg;
                model_splits = pick.s;
            }
        }
        const bool forced_dma = forced_cfg >= kTileFirstDma && forced_cfg < kTileF32Few;
        if (((forced_cfg >= kTileFirstLds && forced_cfg < kTileF32Few) || forced_cfg == kTileBF16Tb48 ||
             forced_cfg == kTileBF16Tb48Few || forced_cfg == kTileBF16Dma4w ||
             (forced_cfg == kTileF2BTall && tall_ok)) &&
            ((!forced_dma && forced_cfg != kTileBF16Dma4w) || mode == kTileBF16))
            cfg = forced_cfg;
    } else if (mode == kTileF32 && N <= 16) {
        cfg = 0;
    } else if (mode == kTileF32 && (transA ? M <= (transB ? 16 : 32) : (M <= 32 || (!transB && M <= 512)))) {
        // Few rows: 16-row tiles instead of 64-row tiles that are mostly
        // padding.  MI355X, us (64 x 64 tiles -> 16 x 16 with k over 8 waves
        // / 16 x 128 with two k-groups): B stored N x K 12 x 11003 x 2048
        // 71.1 -> 30.9 / 34.7, 16 x 4096 x 4096 46.7 -> 23.2 / 24.3, 24 x 4096
        // x 4096 -> 34.6 / 32.3, 32 x 4096 x 4096 47.5 -> 37.1 / 32.8; B stored
        // K x N 12 x 11003 x 2048 60.4 -> 40.4 / 37.0, 16 x 4096 x 4096 36.5 ->
        // 29.6 / 21.5, 32 x 4096 x 4096 38.8 -> 46.5 / 28.9.  With B stored
        // K x N the 16 x 128 tile (its 16-byte column loads, and the row tiles
        // of a column strip sharing one XCD's L2) also wins up to M = 512
        // (measured): 48 / 64 x 4096 x 4096 40.4 / 42.8 -> 32.5 / 34.6, 128 /
        // 256 / 512 x 4096 x 4096 67.0 / 109.6 / 189.0 -> 61.8 / 96.8 / 175.6,
        // 128 x 11003 x 2048 108.9 -> 89.2.  With B stored N x K it loses above
        // M = 32 (128 x 4096 x 4096 77.7 -> 90.0).  A stored K x M (64 x 64
        // tiles -> 16-row tiles): B stored K x N 16 / 32 x 4096 x 4096 35.6 /
        // 35.8 -> 23.3 / 31.2, but 64 / 128 x 4096 x 4096 39.8 / 61.0 -> 48.2 /
        // 82.9; B stored N x K 8 / 16 x 4096 x 4096 39.1 / 39.5 -> 22.8 / 24.5,
        // 7 x 11003 x 2048 62.4 -> 32.5, but 32 x 4096 x 4096 40.2 -> 43.4.
        cfg = transB && M <= 16 ? kTileF32Few : kTileF32Few128;
    } else if (mode == kTileF32 && N <= 64 && M >= 4096) {
        cfg = 1;
    } else if (M >= 128 && N >= 128) {
        cfg = 4;
    } else {
        cfg = 2;
    }
    // fp32 register tiles: the cost model's choice when nothing is forced, or
    // a forced configuration (tunable TILE_CFG).
    if (!lds && mode == kTileF32 && !transA && M >= 12 && N >= 64 && forced_cfg <= 0 &&
        tunable(kTuneTileSplits) <= 0) {
        // The 32-column wave tiles only while 64 x 128 tiles would fill the
        // chip fewer than 4 times: beyond that their extra re-reads of A and
        // B, which the model does not price, cost more than they save
        // (measured 10-16% slower at 1200-1600 such tiles).
        const bool small_grid = ceil_div(M, 64) * ceil_div(N, 128) < 4 * num_cus();
        auto dma_ok = [&](int k) {
            return (k < kTileF32DmaTbFirst || small_grid) && f32_dma_fits(k, transA, transB, M, K, lda, ldb);
        };
        const TilePick dma = best_lds_tile(kF32DmaModel, transB ? 1 : 0, M, N, K, dma_ok);
        if ((double)M * N * K <= 1e10) {
            // the register tiles' model, then the LDS-DMA tiles where their
            // model puts them 10% ahead of that choice
            const TilePick pick = pick_f32_tile(transB ? 1 : 0, M, N, K, cfg);
            cfg = pick.cfg;
            model_splits = pick.s;
            if (dma.s > 0 && pick.us > 0.0 && dma.us < 0.9 * pick.us) {
                cfg = dma.cfg;
                model_splits = dma.s;
            }
        } else if (dma.s > 0) {
            // beyond the fitted range (MFMA-bound): the LDS-DMA tiles
            cfg = dma.cfg;
            model_splits = dma.s;
        }
    }
    if (!lds && mode == kTileF32 &&
        ((forced_cfg >= 1 && forced_cfg <= 4) || forced_cfg == kTileF32Few || forced_cfg == kTileF32Few128 ||
         (tile_f32_dma(forced_cfg) && f32_dma_fits(forced_cfg, transA, transB, M, K, lda, ldb))))
        cfg = forced_cfg;
    const bool f32dma = mode == kTileF32 && tile_f32_dma(cfg);
    const TileConfig c = tile_config(cfg);
    const int bm = c.wm * c.mt * 16, bn = c.wn * c.nt * 16;
    const int kb = lds || f32dma ? tile_lds_bk(bm, bn, c.kblk) : (mode == kTileF32 ? 64 : 128);
    const long long tn = ceil_div(N, bn), tm = ceil_div(M, bm), tiles = tn * tm;
    const long long nblk = ceil_div(K, kb);
    const int waves_per_wg = c.wm * c.wn * c.kw;
    const long long cus = num_cus();
    long long s = 1;
    const int forced_splits = tunable(kTuneTileSplits);
    if (lds) {
        // One LDS-staged workgroup per CU is the unit of work; split k only
        // when the tiles leave more than half of the CUs idle.
        if (tiles * 2 < cus) s = std::min<long long>({ceil_div(cus, tiles), std::max<long long>(1, nblk / 2),
                                                      (long long)max_splits()});
        if (model_splits > 0) s = model_splits;
    } else if (mode == kTileF32) {
        s = model_splits > 0 ? model_splits : (f32dma ? lds_rule_splits(cfg, M, N, K) : reg_tile_splits(cfg, M, N, K));
    } else {
        const long long target_wgs = cus * waves_per_cu() / waves_per_wg;
        if (tiles < target_wgs) {
            s = ceil_div(target_wgs, tiles);
            s = std::min<long long>({s, std::max<long long>(1, nblk / (2 * c.kw)), (long long)max_splits()});
            s = std::max<long long>(1, s);
        }
    }
    if (forced_splits > 0) s = std::min<long long>(forced_splits, nblk);
    // Per-workgroup buffer offsets must fit in 31 bits: an operand read along
    // its rows spans one tile of rows, one read along k spans the k-range of
    // one workgroup.  More splits shorten that range.  (The LDS kernel
    // addresses k from 0; its spans were checked above.)
    auto span_ok = [&](long long splits) {
        if (lds || f32dma) return true;  // checked above, over all of k
        const long long kext = ceil_div(nblk, splits) * kb;
        const long long a = transA ? kext * lda : (long long)bm * lda;
        const long long b = transB ? (long long)bn * ldb : kext * ldb;
        return (a + kext + bm) * es < 0x7FFFFFFFll && (b + kext + bn) * es < 0x7FFFFFFFll;
    };
    while (!span_ok(s) && s < nblk) s *= 2;
    if (s > nblk) s = nblk;
    if (!span_ok(s)) return DNNOPT_ERR_UNSUPPORTED;
    if (tm > 65535 || s > 65535 || tn * tm > 0x7FFFFFF0ll) return DNNOPT_ERR_UNSUPPORTED;
    L->mode = mode;
    L->cfg = cfg;
    L->bm = bm;
    L->bn = bn;
    L->tn = (int)tn;
    L->tm = (int)tm;
    // LDS-staged tiles and the 16-row fp32 tiles are launched as one
    // XCD-ordered row of workgroups.
    const bool xcd = lds || f32dma || (mode == kTileF32 && c.mt == 1 && c.wm == 1);
    L->grid = xcd ? dim3((unsigned)xcd_grid((int)tn, (int)tm), 1, (unsigned)s) : dim3((unsigned)tn, (unsigned)tm, (unsigned)s);
    // k-splits of the LDS-staged kernels are summed by a reduce kernel, except
    // for the LDS-DMA tiles (tunable TILE_TICKET = 1): the last workgroup to
    // finish a tile adds the others' partials.
    const bool dma_ticket = tunable(kTuneTileTicket) == 1;
    const bool dma = (cfg >= kTileFirstDma && cfg < kTileF32Few) || cfg == kTileBF16Dma4w;  // LDS-DMA tiles
    const bool ticket_ok = !lds || (dma_ticket && dma);
    // Split sums: fp32 tiles (register and LDS-DMA) let the tile's
    // last-arriving workgroup add up to 8 splits' partials (one kernel; its
    // threads read the partial block in 16-byte pieces, 8 in flight each),
    // the reduce kernel beyond (MI355X, 36 split shapes, us, reduce ->
    // last workgroup: 2-6 splits 1.01-1.11x faster, e.g. 784 x 128 x 1152
    // 9.35 -> 8.42, 384 x 768 x 768 12.78 -> 11.73; 8 splits level to 1.03x;
    // 16 splits 0.85-0.96x).  Tunable SPLIT_REDUCE: 0 the last workgroup up
    // to 16 splits, 2 the reduce kernel.
    const int srm = tunable(kTuneSplitReduce);
    const bool want_ticket = srm == 0 || (srm == 1 && s <= kTileTicketSplits);
    L->defer_reduce =
        (s > 1 && (!want_ticket || s > kTicketSplitLimit || tiles > kMaxTickets || !ticket_ok)) ? 1 : 0;
    L->part_bytes = s > 1 ? (size_t)s * tiles * bm * bn * sizeof(float) : 0;
    L->tickets = (s > 1 && !L->defer_reduce) ? (int)tiles : 0;
    const int kernel = mode == kTileF32 ? DNNOPT_K_TILE_F32 : DNNOPT_K_TILE_BF16;
    fill_pub(L, kernel,
             mode == kTileF32 ? (f32dma ? "dnnopt_tile_f32_dma" : "dnnopt_tile_f32")
                              : (dma ? "dnnopt_tile_bf16_dma" : (lds ? "dnnopt_tile_bf16_lds" : "dnnopt_tile_bf16")),
             bm, bn, (int)s, waves_per_wg * 64);
    return DNNOPT_OK;
}

static int plan_s8_kernels(int epi, int M, int N, int K, Launch* L, bool lds_ok, int lda, int ldb, int ldc) {
    *L = Launch{};
    if (ldc <= 0) ldc = N;
    // The LDS-staged kernel addresses a C tile with 32-bit offsets.
    if ((long long)128 * ldc * 4 >= 0x7FFFFFFFll) lds_ok = false;
    const int forced_cfg = tunable(kTuneS8Cfg);
    // M <= 4 (B is stored N x K): the row-dot kernel streams every row of B
    // once in 1 KiB steps with exact int32 dot products and needs no partial
    // sums; the kTuneS8Rowdot switch keeps the MFMA tiles when off.
    const bool rowdot_ok = tunable(kTuneS8Rowdot) != 0;
    if (M <= kRowdotS8MaxM && rowdot_ok && forced_cfg < 0 &&
        plan_rowdot(2 + (epi ? 1 : 0), M, N, K, lda > 0 ? lda : K, ldb > 0 ? ldb : K, L) == DNNOPT_OK)
        return DNNOPT_OK;
    *L = Launch{};
    const int forced_splits = tunable(kTuneS8Splits);
    // M <= 16: 16 x 16 tiles with k split over the 8 waves of a workgroup
    // (one launch, no partial sums).  Larger M: operands copied into LDS by
    // the memory unit (LDS DMA), the largest of 64 x 64 (4 stages of
    // 128-byte blocks), 64 x 32 (3 stages of 256 bytes) and 32 x 32 (4
    // stages of 256 bytes) that still gives every CU a tile.  Measured (us,
    // against the register-staged 32 x 32 LDS kernel): 128 x 4096 x 4096
    // 11.2 vs 12.6, 128 x 2048 x 4096 7.9 vs 9.6, 64 x 4096 x 4096 8.8 vs
    // 10.2, 256 x 4096 x 4096 13.9 vs 21.7, 128 x 8192 x 4096 16.1 vs 22.5.
    int cfg = 5;
    if (M > 16) {
        const long long cus_ = num_cus();
        if (ceil_div(M, 64) * ceil_div(N, 64) >= cus_) cfg = 29;
        else if (ceil_div(M, 64) * ceil_div(N, 32) >= cus_) cfg = 23;
        else cfg = 22;
    }
    if (forced_cfg >= 0 && forced_cfg < s8_config_count()) cfg = forced_cfg;
    if (cfg >= kS8FirstLds && !lds_ok) cfg = M <= 16 ? 5 : (M >= 128 ? 3 : 2);
    const bool lds = cfg >= kS8FirstLds;
    const bool dma = cfg >= kS8FirstDma;
    const S8Config c = s8_config(cfg);
    const int bm = c.wm * c.mt * 16, bn = c.wn * c.nt * 16;
    const long long tn = ceil_div(N, bn), tm = ceil_div(M, bm), tiles = tn * tm;
    const int kb = lds ? (c.kblk > 0 ? c.kblk : 128) : 256;
    const long long nblk = ceil_div(K, kb);
    const int waves_per_wg = c.wm * c.wn * c.kw;
    const long long cus = num_cus();
    long long s = 1;
    if (lds) {
        if (tiles * 2 < cus) s = std::min<long long>({ceil_div(cus, tiles), std::max<long long>(1, nblk / 2),
                                                      (long long)max_splits()});
    } else {
        const long long target_wgs = cus * waves_per_cu() / waves_per_wg;
        if (tiles < target_wgs) {
            s = ceil_div(target_wgs, tiles);
            s = std::min<long long>({s, std::max<long long>(1, nblk / c.kw), (long long)kTicketSplitLimit});
            s = std::max<long long>(1, s);
        }
    }
    if (forced_splits > 0) s = std::min<long long>(forced_splits, std::max<long long>(1, nblk / c.kw));
    if (s > 1 && tiles > kMaxTickets && !split_reduce_mode() && !lds) s = 1;
    // The tiles address A and B from their first row with 32-bit offsets.
    if ((long long)bm * (lda > 0 ? lda : K) + K >= 0x7FFFFFFFll || (long long)bn * (ldb > 0 ? ldb : K) + K >= 0x7FFFFFFFll)
        return DNNOPT_ERR_UNSUPPORTED;
    if (tm > 65535 || s > 65535 || tn * tm > 0x7FFFFFF0ll) return DNNOPT_ERR_UNSUPPORTED;
    // The LDS-staged kernel always hands its k-splits to the reduce kernel.
    L->defer_reduce = (s > 1 && (split_reduce_mode() || lds)) ? 1 : 0;
    L->mode = epi;
    L->cfg = cfg;
    L->bm = bm;
    L->bn = bn;
    L->tn = (int)tn;
    L->tm = (int)tm;
    L->grid = lds ? dim3((unsigned)xcd_grid((int)tn, (int)tm), 1, (unsigned)s) : dim3((unsigned)tn, (unsigned)tm, (unsigned)s);
    L->part_bytes = s > 1 ? (size_t)s * tiles * bm * bn * sizeof(int32_t) : 0;
    L->tickets = (s > 1 && !L->defer_reduce) ? (int)tiles : 0;
    fill_pub(L, DNNOPT_K_MFMA_S8, dma ? "dnnopt_s8_dma" : (lds ? "dnnopt_s8_lds" : "dnnopt_mfma_s8"), bm, bn, (int)s,
             waves_per_wg * 64);
    return DNNOPT_OK;
}

int plan_s8(int epi, int M, int N, int K, Launch* L, bool lds_ok, int lda, int ldb, int ldc) {
    if (tunable(kTuneWide)) {
        plan_wide(M, N, L);
        return DNNOPT_OK;
    }
    const int st = plan_s8_kernels(epi, M, N, K, L, lds_ok, lda, ldb, ldc);
    if (st == DNNOPT_ERR_UNSUPPORTED) plan_wide(M, N, L);
    return st == DNNOPT_ERR_UNSUPPORTED ? DNNOPT_OK : st;
}

int plan_rowdot(int mode, int M, int N, int K, int lda, int ldb, Launch* L) {
    if (M < 1 || M > 8) return DNNOPT_ERR_UNSUPPORTED;
    *L = Launch{};
    const long long es = mode >= 2 ? 1 : (mode ? 2 : 4), R = rowdot_rows(mode, M);
    // Buffer offsets are 32-bit from the first row of a wave (B) and of A.
    if ((R * ldb + K) * es >= 0x7FFFFFFFll || ((long long)(M - 1) * lda + K) * es >= 0x7FFFFFFFll)
        return DNNOPT_ERR_UNSUPPORTED;
    constexpr long long kSteps = 2;  // load steps a wave issues at once
    const long long steps = ceil_div(ceil_div(K, 16 / es), 64);  // 1 KiB row steps
    const long long cus = num_cus();
    // Waves of a workgroup split k (kw ways) until there are two workgroups
    // per CU, as long as each wave keeps whole multi-step k-ranges.
    int kw = 1;
    while (kw < 8 && ceil_div(N, (kRowdotWaves / kw) * R) < 2 * cus && steps / (2 * kw) >= kSteps) kw *= 2;
    const int forced_kw = tunable(kTuneRowdotKW);
    if (forced_kw == 1 || forced_kw == 2 || forced_kw == 4 || forced_kw == 8) kw = forced_kw;
    const long long rows_per_wg = (kRowdotWaves / kw) * R;
    const long long G = ceil_div(N, rows_per_wg);
    if (G > 0x7FFFFFFFll) return DNNOPT_ERR_UNSUPPORTED;
    L->mode = mode;
    L->mr = M;
    L->nw = kw;
    L->grid = dim3((unsigned)G, 1, 1);
    fill_pub(L, mode >= 2 ? DNNOPT_K_ROWDOT_S8 : (mode ? DNNOPT_K_ROWDOT_BF16 : DNNOPT_K_ROWDOT_F32), "dnnopt_rowdot", M,
             (int)rows_per_wg, 1, kRowdotWaves * 64);
    return DNNOPT_OK;
}

int plan_tall(int transB, int M, int N, int K, int lda, int ldb, Launch* L, int ldc) {
    *L = Launch{};
    if (ldc <= 0) ldc = N;
    // N <= 12 (a quarter or more of the padded 16-column MFMA tile wasted)
    // and N <= 16 with short K stream faster through the register tiles
    // (64 x 16) than through the register-ring kernel here (65536 x 12 x
    // 256: 20.4 vs 19.5 us, 262144 x 16 x 64: 20.9 vs 19.9), but slower than
    // through the LDS-DMA kernel below where it fits (MI355X, us, register
    // tiles -> LDS-DMA: 65536 x 12 x 256 17.7 -> 16.8, 65536 x 1 x 256 23.3
    // -> 16.4, 262144 x 16 x 64 20.0 -> 17.6, 131072 x 8 x 128 18.7 -> 16.2).
    if ((N <= 12 || (N <= 16 && K < 128)) && !tall_dma_fits(N, K, lda)) return DNNOPT_ERR_UNSUPPORTED;
    if (N > 64 || M < 4096) return DNNOPT_ERR_UNSUPPORTED;
    const int nt = (N + 15) / 16;
    const size_t lds = tall_lds_bytes(nt, K);
    if (lds > 65536) return DNNOPT_ERR_UNSUPPORTED;
    if (((long long)(M - 1) * lda + K) * 4 >= 0x7FFFFFFFll) return DNNOPT_ERR_UNSUPPORTED;
    // B is read through one descriptor with 32-bit offsets.
    if ((transB ? (long long)(N - 1) * ldb + K : (long long)(K - 1) * ldb + N) * 4 >= 0x7FFFFFFFll)
        return DNNOPT_ERR_UNSUPPORTED;
    // C is stored through one descriptor from its first element.
    if (((long long)(M - 1) * ldc + N) * 4 >= 0x7FFFFFFFll) return DNNOPT_ERR_UNSUPPORTED;
    // Each wave runs its row tiles as one serial chain of MFMAs, so the kernel
    // needs about one tile for every wave of one workgroup per CU: 16-row
    // tiles from ~48K rows, and from ~16K rows when K >= 256; below that the
    // register tiles, which spread the same work over more waves, are faster.
    // Measured at N = 64, K = 256: 16K rows 15.0 vs 17.8 us (register tiles),
    // 32K rows 17.2 vs 23.0.  16-row tiles beat 32-row tiles from 48K rows
    // too (two tiles per wave, so one tile's C stores overlap the next
    // tile's loads): 65536 x 16 x 256 17.6 vs 19.0 us, 131072 x 16 x 256 32.1
    // vs 33.6, 65536 x 64 x 256 27.4 vs 28.6, 65536 x 48 x 128 14.3 vs 15.1.
    const long long waves = num_cus() * tall_waves();
    int rt = 1;
    // K = 64 .. 256 (a multiple of 64) with 16-byte rows of A: A copied
    // into LDS by the memory unit (dnnopt_tall_dma_f32), except K = 128 with
    // N > 32, where the register-ring kernel is faster (65536 x 48 / 64 x
    // 128: 15.0 / 16.4 vs 15.4 / 17.5 us).  For N <= 16 it needs no row
    // count either: it beats the register tiles from 4K rows (MI355X, us:
    // 4096 x 16 x 256 6.7 -> 4.7, 8192 x 16 x 256 7.9 -> 5.8, 12288 x 16 x
    // 128 4.8 -> 4.2, 8192 x 8 x 128 4.4 -> 3.7, 24576 x 16 x 64 4.6 -> 4.2).
    const bool dma = tall_dma_fits(N, K, lda) && !(K == 128 && N > 32);
    if (!(dma && nt == 1) && ceil_div(M, 32) * 4 < 3 * waves && (K < 256 || ceil_div(M, 16) * 2 < waves))
        return DNNOPT_ERR_UNSUPPORTED;
    const int forced_rt = tunable(kTuneTallRT);
    if (forced_rt == 1 || forced_rt == 2) rt = forced_rt;
    // The LDS-DMA kernel: persistent 8-wave workgroups, as many per CU as
    // their LDS allows (at most 4).  Against the register-ring kernel
    // (MI355X, us, 65536 rows): N = 16 x K = 256 16.9 -> 16.2, N = 32 x 192
    // 17.1 -> 14.7, N = 32 x 256 21.2 -> 19.5, N = 48 x 256 22.9 -> 21.1,
    // N = 64 x 256 27.4 -> 26.2 (B stored N x K 30.3 -> 28.6), N = 64 x 64
    // 11.3 -> 11.1, 65536 x 13 x 128 11.3 -> 9.8, 16384 x 16 x 256 9.0 -> 7.1.
    if (dma && forced_rt <= 0) {
        const size_t dlds = tall_dma_lds_bytes(nt, K);
        const long long per_cu_d = std::max<long long>(1, std::min<long long>(4, 160 * 1024 / (long long)dlds));
        const long long Gd = std::max<long long>(
            1, std::min<long long>(num_cus() * per_cu_d, ceil_div(ceil_div(M, 16), tall_dma_waves())));
        L->cfg = nt;
        L->mr = 0;
        L->lds = dlds;
        L->mode = transB;
        L->grid = dim3((unsigned)Gd, 1, 1);
        fill_pub(L, DNNOPT_K_TALL_F32, "dnnopt_tall_dma_f32", 16, 16 * nt, 1, tall_dma_waves() * 64);
        return DNNOPT_OK;
    }
    const long long tiles = ceil_div(M, 16 * rt);
    // Persistent: one workgroup per CU by default, no more than there are row
    // tiles for their waves.  More row tiles per wave keep loads, MFMAs and
    // stores of different tiles overlapped; a second workgroup per CU (more
    // waves, one tile each) measured slower at every K.
    const long long per_cu = std::max<long long>(1, std::min<long long>(4, 160 * 1024 / (long long)lds));
    const int wgs_per_cu = tunable(kTuneTallWgsPerCu);
    const long long want = num_cus() * std::min<long long>(std::max(wgs_per_cu, 1), per_cu);
    const long long G = std::max<long long>(1, std::min<long long>(want, ceil_div(tiles, tall_waves())));
    L->cfg = nt;
    L->mr = rt;
    L->lds = lds;
    L->mode = transB;
    L->grid = dim3((unsigned)G, 1, 1);
    fill_pub(L, DNNOPT_K_TALL_F32, "dnnopt_tall_f32", 16 * rt, 16 * nt, 1, tall_waves() * 64);
    return DNNOPT_OK;
}

void plan_wide(int M, int N, Launch* L) {
    *L = Launch{};
    L->grid = wide_grid(M, N);
    fill_pub(L, DNNOPT_K_WIDE, "dnnopt_wide", 1, 64, 1, wide_threads());
}

namespace {

int plan_sgemm_kernels(int transA, int transB, int M, int N, int K, int lda, int ldb, Launch* L, int ldc) {
    // The skinny kernel for M <= 8 unless its spans exceed 32-bit offsets
    // (then the tiles, which split k into shorter ranges).
    if (M <= 8 && !transB && plan_skinny(kSkinnyF32, M, N, K, ldb, L) == DNNOPT_OK) return DNNOPT_OK;
    *L = Launch{};
    // B stored N x K: the row-dot kernel up to M = 4 and for narrow N; from
    // M = 5 at N >= 2048 the 16-row MFMA tiles (us, row-dot -> tiles: M=5 / 6
    // / 8 x 11003 x 2048 27.6 / 29.8 / 32.4 -> 26.1 / 26.5 / 28.1, x 4096 x
    // 4096 21.5 / 21.2 / 25.5 -> 17.3 / 17.9 / 19.0, M=7 x 4099 x 2048 15.9
    // -> 13.8; N = 1009 and M <= 4 favour the row-dot kernel).
    const bool few_rows_tile = transB && M >= 5 && N >= 2048;
    // (The row-dot kernel reads B as N x K rows: never for a K x N B.)
    if (transB && M <= 8 && !transA && !few_rows_tile && plan_rowdot(0, M, N, K, lda, ldb, L) == DNNOPT_OK)
        return DNNOPT_OK;
    const bool tall_ok = tunable(kTuneTall) != 0;
    if (tall_ok && !transA && plan_tall(transB, M, N, K, lda, ldb, L, ldc) == DNNOPT_OK) return DNNOPT_OK;
    return plan_tile(kTileF32, transA, transB, M, N, K, lda, ldb, L, true, ldc);
}

int plan_bf16_kernels(int fp32_inputs, int M, int N, int K, int lda, int ldb, Launch* L, int transB, int ldc) {
    // B stored N x K has k-contiguous columns: MFMA tiles read it in place
    // for every M (the skinny kernel streams rows of a K x N B).  bf16
    // storage with a K x N B and 4-byte aligned rows: the skinny kernel up to
    // M = 5, the LDS-staged 32 x 64 tiles from M = 6 (MI355X, us, skinny ->
    // tiles, N = 11008, K = 4096: M=6 24.8 -> 22.6, M=7 27.9 -> 22.6, M=8
    // 31.0 -> 22.4; 8 x 4096 x 4096 16.2 -> 13.5; M=5 22.6 vs 22.4, M=4 21.0
    // vs 22.2, 5 x 4096 x 4096 13.6 vs 13.8).
    const bool tile_kn = !transB && !fp32_inputs && M >= 6 && (lda & 1) == 0 && (ldb & 1) == 0;
    if (M <= 8 && !transB && !tile_kn &&
        plan_skinny(fp32_inputs ? kSkinnyF2B : kSkinnyBF16, M, N, K, ldb, L) == DNNOPT_OK)
        return DNNOPT_OK;
    *L = Launch{};
    if (transB && fp32_inputs) return DNNOPT_ERR_UNSUPPORTED;
    // B stored N x K: the row-dot kernel up to M = 4 and for rows off 4-byte
    // boundaries; from M = 5 the LDS-staged tiles (us, row-dot -> 32 x 64
    // tiles, N = 11008, K = 4096: M=5 26.5 -> 23.3, M=7 31.6 -> 23.5, M=8 34.0
    // -> 24.1; 8 x 4096 x 4096 15.7 -> 12.4; M=4 24.1 vs 23.8, M=1 19.1 vs
    // 22.6).
    const bool tile_tb = transB && M >= 5 && (lda & 1) == 0 && (ldb & 1) == 0;
    if (transB && M <= 8 && !tile_tb && plan_rowdot(1, M, N, K, lda, ldb, L) == DNNOPT_OK) return DNNOPT_OK;
    return plan_tile(fp32_inputs ? kTileF2B : kTileBF16, 0, transB, M, N, K, lda, ldb, L, true, ldc);
}

}  // namespace

// Shapes no tiled kernel can address (operand spans past 32-bit offsets)
// run on the 64-bit last-resort kernel.
int plan_sgemm(int transA, int transB, int M, int N, int K, int lda, int ldb, Launch* L, int ldc) {
    if (tunable(kTuneWide)) {
        plan_wide(M, N, L);
        return DNNOPT_OK;
    }
    const int st = plan_sgemm_kernels(transA, transB, M, N, K, lda, ldb, L, ldc);
    if (st == DNNOPT_ERR_UNSUPPORTED) plan_wide(M, N, L);
    return st == DNNOPT_ERR_UNSUPPORTED ? DNNOPT_OK : st;
}

int plan_bf16(int fp32_inputs, int M, int N, int K, int lda, int ldb, Launch* L, int transB, int ldc) {
    if (transB && fp32_inputs) return DNNOPT_ERR_UNSUPPORTED;  // no entry point takes this combination
    if (tunable(kTuneWide)) {
        plan_wide(M, N, L);
        return DNNOPT_OK;
    }
    const int st = plan_bf16_kernels(fp32_inputs, M, N, K, lda, ldb, L, transB, ldc);
    if (st == DNNOPT_ERR_UNSUPPORTED) plan_wide(M, N, L);
    return st == DNNOPT_ERR_UNSUPPORTED ? DNNOPT_OK : st;
}

}  // namespace dnnopt_hip
