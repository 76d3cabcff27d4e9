// kernels.h -- argument blocks and launch wrappers of the gfx950 kernels.
//
// Host code (dispatch.cpp, capi.cpp) fills these structs and calls the
// launch_* wrappers; each wrapper maps its configuration onto one template
// instantiation and enqueues it on the given stream.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dnnopt_hip {

// Split-k tickets (one arrival counter per output tile) lie 256 bytes apart:
// atomics on one cache line are serialised (MI355X: 256 workgroups counting
// on one line, +2.4 us per launch; 256 bytes apart, no measurable cost).
constexpr int kTicketStride = 64;  // words

// ---------------------------------------------------------------- skinny
// M <= 8 rows against a row-major K x N operand B that is streamed once.
// Workgroup (x, y) = (column tile, k-split); its NW waves split the k-range
// of the workgroup and are reduced through LDS; split groups are reduced by
// the last workgroup to arrive (ticket) in split order.
enum SkinnyMode {
    kSkinnyF32 = 0,   // A, B fp32
    kSkinnyBF16 = 1,  // A, B bf16 storage
    kSkinnyF2B = 2,   // A, B fp32 rounded to bf16 in registers
};

struct SkinnyArgs {
    const void* A;
    const void* B;
    float* C;
    float* part;        // [splits][M][ncols_pad] partial sums (splits > 1)
    unsigned* tickets;  // one per column tile (splits > 1)
    int a_sm, a_sk;     // element strides of A over m and over k (lda,1 or 1,lda)
    int ldb, ldc;
    int M, N, K;
    float alpha, beta;
    int splits;         // most k-splits of any tile (partial buffer rows)
    int ncols_pad;
    int defer_reduce;   // splits > 1: 1 = only store partials (a reduce kernel follows)
    int tiles;          // column tiles T; the grid has G >= T workgroups
    const float* bias;  // per-column bias added after the epilogue (or null)
};

// Rows of B per k-split unit of the planner; the kernel's load block (rows
// of B in flight per wave) is 16 or 4 (launch_skinny's `unroll`).
constexpr int kSkinnyUnroll = 16;
inline int skinny_tile_cols(int mode) { return mode == kSkinnyBF16 ? 512 : 256; }
inline int skinny_elem_bytes(int mode) { return mode == kSkinnyBF16 ? 2 : 4; }

// b_aligned: every row of B starts on a 4-byte boundary (checked by the host).
// a_layout: 0 = A row-major with 4-byte aligned rows, 1 = A stored K x M (fp32),
// 2 = bf16 A rows off 4-byte alignment (element loads).
// unroll: rows of B per load block of a wave, 16 or 4 (4 only for fp32 with
// 8-wave workgroups).
hipError_t launch_skinny(int mode, int mr, int nw, int unroll, int b_aligned, int a_layout, dim3 grid,
                         const SkinnyArgs& a, hipStream_t s);

// ---------------------------------------------------------------- row dot (B stored N x K)
// M <= 8 rows of a row-major A against B stored N x K (k contiguous): each
// output is a dot product of two rows.  Workgroups of kRowdotWaves waves;
// rowdot_rows(M) rows of B per wave; KW waves of a workgroup split k.
struct RowdotArgs {
    const void* A;
    const void* B;
    float* C;           // fp32 output (modes 0, 1, 3)
    int lda, ldb, ldc;
    int M, N, K;
    float alpha, beta;
    const float* bias;  // per-column bias added after the epilogue (or null)
    int32_t* Ci;        // int32 output (mode 2)
    const float* scale; // per-column scale of mode 3
    // Mode 3 with amax != nullptr: the fp32-API gemm_int8's dynamic
    // dequantization instead of the column scale (s8_out in device_common.h;
    // amax[0..1] = bits of max|A|, max|B|; alpha, beta as above).
    const unsigned* amax;
};
constexpr int kRowdotWaves = 8;
#ifndef DNNOPT_ROWDOT_R58
#define DNNOPT_ROWDOT_R58 2  // rows of B per wave for 4 < M <= 8
#endif
constexpr int rowdot_rows(int mr) { return mr <= 2 ? 8 : (mr <= 4 ? 4 : DNNOPT_ROWDOT_R58); }
// Rows of B per wave for a mode (0 fp32, 1 bf16, 2 / 3 int8).  An int8 row
// of B is a quarter of an fp32 one, so more waves with 2 rows each keep more
// of it in flight (measured at K = 4096: 1 / 2 / 4 rows per wave 5.9 / 5.5
// / 6.3 us at M = 1).
constexpr int rowdot_rows(int mode, int mr) { return mode >= 2 ? 2 : rowdot_rows(mr); }
// The int8 modes serve M <= kRowdotS8MaxM (beyond it the MFMA tiles are
// faster: M = 5 ties, M = 8 is 1.2 us slower on the row-dot kernel).
constexpr int kRowdotS8MaxM = 4;
// mode 0 fp32, 1 bf16 storage, 2 int8 -> int32 C, 3 int8 -> fp32 C scaled
// per column; kw in {1, 2, 4, 8}; aligned: every row of A and B starts on a
// 4-byte boundary (bf16, int8).  grid.x = workgroups, each
// covering (kRowdotWaves / kw) * rowdot_rows(M) rows of B.
hipError_t launch_rowdot(int mode, int mr, int kw, int aligned, dim3 grid, const RowdotArgs& a, hipStream_t s);

// ---------------------------------------------------------------- tall-skinny fp32, B in LDS
// Large M, N <= 16 * nt (nt in {1, 2, 3, 4}), all of B staged in LDS
// (ceil(K / 16) * 16 * 16 * nt * 4 bytes <= 64 KiB); persistent workgroups
// of 4 waves stream row tiles of A (32 rows per wave).  A rows must fit
// 32-bit buffer offsets: ((M - 1) * lda + K) * 4 < 2^31.
struct TallArgs {
    const float* A;
    const float* B;
    float* C;
    int lda, ldb, ldc;
    int M, N, K;
    float alpha, beta;
    const float* bias;  // per-column bias added after the epilogue (or null)
};
inline size_t tall_lds_bytes(int nt, int K) { return (size_t)((K + 15) / 16) * 16 * 16 * nt * 4; }
int tall_waves();  // waves per workgroup of the tall kernel
// rt: row tiles of 16 a wave takes at a time (1 or 2).
hipError_t launch_tall_f32(int nt, int tb, int rt, dim3 grid, size_t lds_bytes, const TallArgs& a, hipStream_t s);
// A copied into LDS by the memory unit (N <= 64, K = 64, 128, 192 or 256,
// lda % 4 == 0, A 16-byte aligned): persistent workgroups of tall_dma_waves()
// waves, each with a ring of two 16-row pieces of A, tall_dma_lds_bytes(nt,
// K) of LDS per workgroup for nt = ceil(N / 16) column tiles.
bool tall_dma_fits(int N, int K, int lda);
size_t tall_dma_lds_bytes(int nt, int K);
int tall_dma_waves();
hipError_t launch_tall_dma_f32(int tb, dim3 grid, const TallArgs& a, hipStream_t s);

// ---------------------------------------------------------------- int8 MFMA
// Exact s8 x s8 -> s32 with B stored N x K.  Each wave owns MT x NT tiles of
// 16 x 16 outputs (v_mfma_i32_16x16x64_i8); a workgroup is WM x WN x KW waves
// (KW waves split k and are reduced through LDS); grid.z splits k across
// workgroups with a ticket reduction.
struct S8Args {
    const int8_t* A;
    const int8_t* B;
    void* C;             // int32_t* (EPI 0) or float* (EPI 1)
    const float* scale;  // per-column scale (EPI 1)
    int32_t* part;       // [splits][tiles][BM*BN]
    unsigned* tickets;   // one per output tile
    int lda, ldb, ldc;
    int M, N, K;
    int splits;
    int defer_reduce;    // splits > 1: 1 = only store partials (a reduce kernel follows)
    int tiles_n, tiles_m;  // LDS-staged kernel: tile grid (blockIdx.x is XCD-ordered, see xcd_tile)
    // EPI 1 with amax != nullptr: the fp32-API gemm_int8's dynamic
    // dequantization instead of the column scale (s8_out in device_common.h).
    const unsigned* amax;
    float alpha, beta;
    // fp32-API gemm_int8, M > 8 (launch_s8_q8b): B is the fp32 K x N matrix
    // (row stride ldb floats), quantized while it is staged with the scale
    // from the maxima partials qpart[ga, ga + gb); A is already quantized.
    const float* Bf;
    const unsigned* qpart;
    int ga, gb;
};

struct S8Config {
    int mt, nt, wm, wn, kw;
    int depth;  // LDS-staged configurations: k-blocks loaded ahead
    int kblk;   // LDS-staged configurations: bytes of k per block (0 = 128)
};
// Configurations from this index on stage both operands through LDS; they
// need 4-byte aligned rows and reduce k-splits with the reduce kernel only.
constexpr int kS8FirstLds = 10;
// Configurations from this index on copy both operands into LDS with the
// vector memory unit's LDS path (no register staging); same requirements
// and tile order as the LDS-staged ones, depth = stages.
constexpr int kS8FirstDma = 21;
// Index into the table of built int8 configurations.
int s8_config_count();
S8Config s8_config(int idx);
// aligned: all rows of A and B start on 4-byte boundaries (checked by the host).
hipError_t launch_mfma_s8(int cfg_idx, int epi, int aligned, dim3 grid, const S8Args& a, hipStream_t s);

// ---------------------------------------------------------------- fp32 / bf16 tiles
// Row-major C (M x N) = alpha * op(A) op(B) + beta * C with MFMA tiles.
// Operand element type per mode: fp32 (v_mfma_f32_16x16x4_f32), bf16 storage
// or fp32 rounded to bf16 (v_mfma_f32_16x16x32_bf16).
enum TileMode {
    kTileF32 = 0,
    kTileBF16 = 1,
    kTileF2B = 2,
};

struct TileArgs {
    const void* A;
    const void* B;
    float* C;
    float* part;        // [splits][tiles][BM*BN]
    unsigned* tickets;  // one per output tile
    int lda, ldb, ldc;
    int M, N, K;
    float alpha, beta;
    int transA, transB;
    int splits;
    int defer_reduce;   // splits > 1: 1 = only store partials (a reduce kernel follows)
    int tiles_n, tiles_m;  // LDS-staged kernels: tile grid (blockIdx.x is a linear, XCD-ordered index)
    const float* bias;     // per-column bias added after the epilogue (or null)
};

// LDS-staged kernels walk the tiles in an XCD-aware order: workgroup L runs on
// XCD L % 8 (the hardware dispatches workgroups to XCDs round robin).  The
// tiles are numbered strip by strip (t = n tm + m) and XCD x takes the run
// t = x P .. x P + P - 1, P = ceil(tn tm / 8), in order, so the row tiles that
// share a strip of B run together on one XCD and share its L2, and every XCD
// gets P tiles (the last one fewer) however few column strips there are.
// Workgroups past the last tile exit.  The order affects speed only, never
// which tiles exist.  The host keeps tn tm below 2^31 - 8.
struct TileXY {
    int n, m;
    bool ok;
};
__host__ __device__ inline TileXY xcd_tile(int L, int tn, int tm) {
    const int per = (tn * tm + 7) >> 3, j = L >> 3, t = (L & 7) * per + j;
    if (j >= per || t >= tn * tm) return TileXY{0, 0, false};
    return TileXY{t / tm, t % tm, true};
}
// Workgroups to launch for a tn x tm tile grid in that order.
inline int xcd_grid(int tn, int tm) { return 8 * ((tn * tm + 7) / 8); }

struct TileConfig {
    int mt, nt, wm, wn, kw;
    int depth;  // LDS-staged kernels: k-blocks loaded ahead (register ring)
    int kblk;   // LDS-staged kernels: k per block (0 = DNNOPT_LDS_KB)
};
int tile_config_count();
TileConfig tile_config(int idx);
#ifndef DNNOPT_LDS_KB
#define DNNOPT_LDS_KB 64  // k per LDS stage of the bf16 tile kernel (64 or 128)
#endif
// Configurations from this index on are the LDS-staged bf16 kernels: bf16 or
// fp32-rounded modes only, rows of A and B 4-byte aligned, no transposed A
// (B stored N x K with bf16 storage).
constexpr int kTileFirstLds = 5;
// Configurations from this index on copy the operands into LDS with the
// memory unit's LDS path (bf16 storage only; the fp32-input mode keeps the
// register-staged kernel).
constexpr int kTileFirstDma = 26;
// fp32 register tiles for few rows (after the LDS-staged entries; fp32
// only): 16 x 16 with k split over the 8 waves of a workgroup, and 16 x 128
// with two column waves and two k-groups.
constexpr int kTileF32Few = 35;
constexpr int kTileF32Few128 = 36;
// bf16 storage, B stored N x K, M <= 32: LDS-staged tiles 48 columns wide
// (16 x 48 up to M = 16, 32 x 48 above), 230 tiles at N = 11008 instead of 172.
constexpr int kTileBF16Tb48 = 37, kTileBF16Tb48Few = 38;
// bf16 storage, LDS DMA: 128 x 128 tiles on 4 waves of 64 x 64 (bf16
// storage only, like the LDS-DMA entries from kTileFirstDma).
constexpr int kTileBF16Dma4w = 39;
// LDS-staged (register ring), 256 x 96 on 8 waves of 64 x 48, 64 k per
// block: fp32 inputs rounded in registers, many tiles.  Its unsplit epilogue
// addresses C with 32-bit offsets from the tile's first row, so it needs
// 256 * ldc * 4 < 2^31.
constexpr int kTileF2BTall = 40;
// fp32, both operands copied into LDS by the memory unit (A stored M x K):
// configurations kTileF32DmaFirst..Last, 32 k per block; wave tiles of 16,
// 32 or 64 rows by 64 columns (B stored K x N or N x K), and from
// kTileF32DmaTbFirst by 32 columns (B stored N x K only).
constexpr int kTileF32DmaFirst = 41, kTileF32DmaTbFirst = 48, kTileF32DmaLast = 50;
constexpr bool tile_f32_dma(int cfg) { return cfg >= kTileF32DmaFirst && cfg <= kTileF32DmaLast; }
// k per LDS block of an LDS-staged configuration: its kblk (or
// DNNOPT_LDS_KB) when both stages fit in 128 KiB of LDS, else 64.
constexpr int tile_lds_bk(int bm, int bn, int kblk) {
    return (bm + bn) * (kblk > 0 ? kblk : DNNOPT_LDS_KB) * 2 * 2 <= 131072 ? (kblk > 0 ? kblk : DNNOPT_LDS_KB) : 64;
}
// Tile "configuration" of the k-major outer-product kernel (k_kouter.hip):
// fp32, A stored K x M and B stored K x N, 32 < M, N <= 64, a long k; one
// 64 x 64 partial tile per k-split (grid = (1, 1, splits), 256 threads),
// always followed by the split-K reduce kernel.
constexpr int kTileKOuter = 64;
hipError_t launch_kouter_f32(dim3 grid, const TileArgs& a, hipStream_t s);
// transA: fp32 only; transB: fp32, or bf16 storage with B stored N x K.
// aligned: all k-contiguous rows (A; B stored N x K) start on 4-byte
// boundaries (matters for bf16 storage).
hipError_t launch_tile(int mode, int cfg_idx, int transA, int transB, int aligned, dim3 grid,
                       const TileArgs& a, hipStream_t s);

// ---------------------------------------------------------------- last resort
// dnnopt_wide (k_wide.hip): any layout and size with 64-bit addressing, for
// shapes whose operand spans the tiled kernels' 32-bit offsets cannot reach.
enum WideMode { kWideF32 = 0, kWideBF16 = 1, kWideF2B = 2, kWideS8 = 3 };
struct WideArgs {
    const void* A;  // fp32, bf16 bits (kWideBF16), fp32 rounded to bf16 (kWideF2B) or int8
    const void* B;
    void* C;        // fp32, or int32 for kWideS8 with epi 0
    long long lda, ldb, ldc;
    int M, N, K;
    int transA, transB;  // A stored K x M / B stored N x K
    float alpha, beta;
    const float* bias;   // fp32 modes: per-column bias after the epilogue (or null)
    int epi;             // kWideS8: 0 int32 C, 1 fp32 C through s8_out (scale or amax)
    const float* scale;
    const unsigned* amax;
};
hipError_t launch_wide(int mode, const WideArgs& a, hipStream_t s);
dim3 wide_grid(int M, int N);
int wide_threads();

// ---------------------------------------------------------------- small kernels
hipError_t launch_naive_f32(int M, int N, int K, float alpha, const float* A, int lda,
                            const float* B, int ldb, float beta, float* C, int ldc,
                            hipStream_t s);
hipError_t launch_saxpy(int n, float alpha, const float* x, int incx, float* y, int incy,
                        hipStream_t s);
hipError_t launch_fill(void* dst, size_t n, int dtype, int dist, uint64_t seed,
                       uint32_t tensor_id, double p0, double p1, hipStream_t s);
// fp32-API int8, before the GEMM: two launches.  The first stores per-block
// maxima of |A| and |B| in part (absmax_blocks() words); the second reduces
// them, stores the bits of max|A| and max|B| in amax[0..1], and quantizes
// A (M x K) into qA (M x ldq) and B (K x N) into qB transposed (N x ldq).
// The GEMM then dequantizes in its epilogue (EPI 1 / mode 3 with amax).
void absmax_blocks(int M, int N, int K, int* ga, int* gb);
hipError_t launch_quant_pair(const float* A, int lda, const float* B, int ldb, int M, int N, int K, int ldq,
                             unsigned* part, unsigned* amax, int8_t* qA, int8_t* qB, hipStream_t s);
// fp32-API gemm_int8 for M <= 8 in one pass over the fp32 B (K x N): the
// elements are quantized as they are read, with the scales taken from the
// maxima partials qpart[0, ga) (A) and qpart[ga, ga + gb) (B) of
// dnnopt_absmax_part; exact int32 sums, dequantized into C.  The grid and the
// partial buffer are those of the fp32 skinny plan (256 columns per wave);
// defer = 1 (more workgroups than column tiles): every workgroup stores int32
// partials [split][M][ncols_pad] and a reduce kernel, launched by
// launch_skinny_q8, sums them.  amax[0..1] receive max|A|, max|B| bits.
struct SkinnyQ8Args {
    const float* A;
    const float* B;
    float* C;
    int32_t* part;
    const unsigned* qpart;
    unsigned* amax;
    int lda, ldb, ldc;
    int M, N, K;
    int ga, gb;
    float alpha, beta;
    int tiles, splits, ncols_pad, defer;
};
hipError_t launch_skinny_q8(int mr, dim3 grid, const SkinnyQ8Args& a, hipStream_t s);
int skinny_q8_waves();  // waves per workgroup of dnnopt_skinny_q8 (256 columns each)
// Maxima partials only (the first launch of the fp32-API int8 pipeline).
hipError_t launch_absmax(const float* A, int lda, const float* B, int ldb, int M, int N, int K, unsigned* part,
                         hipStream_t s);
// Quantize A only (M x K fp32 -> qA, M x ldq int8) and store max|A|, max|B|
// to amax[0..1] (maxima from launch_absmax's partials).
hipError_t launch_quant_a(const float* A, int lda, int M, int K, int ldq, const unsigned* part, int ga, int gb,
                          unsigned* amax, int8_t* qA, hipStream_t s);
// fp32-API int8 GEMM, M > 8: int8 A (qA) x fp32 K x N B quantized while it is
// staged (64 x 32 tiles through LDS), dequantizing epilogue.  grid.x =
// xcd_grid(ceil(N / 32), ceil(M / 64)).
hipError_t launch_s8_q8b(dim3 grid, const S8Args& a, hipStream_t s);
// Reduce skinny partials [split][M][ncols_pad] into C (epilogue applied);
// tile t (of T, tile width tw) has splits_of_tile(t, G, T) partials.
hipError_t launch_skinny_reduce(const float* part, int G, int T, int tw, int M, int N, int ncols_pad,
                                float alpha, float beta, float* C, int ldc, const float* bias, hipStream_t s);
// Reduce int8 partial tiles [splits][tiles][bm*bn] (exact int32) into C:
// epi 0 stores int32, epi 1 stores s8_out(acc) (column scale, or the dynamic
// dequantization when amax != nullptr).
hipError_t launch_s8_reduce(const int32_t* part, int splits, int tiles_n, int tiles_m, int bm, int bn, int M,
                            int N, int epi, const float* scale, const unsigned* amax, float alpha, float beta,
                            void* C, int ldc, hipStream_t s);
// Reduce partial tiles [splits][tiles_m*tiles_n][bm*bn] into C (epilogue applied).
hipError_t launch_splitk_reduce(const float* part, int splits, int tiles_n, int tiles_m, int bm,
                                int bn, int M, int N, float alpha, float beta, float* C, int ldc,
                                const float* bias, hipStream_t s);

// Column-major helpers of the oneDNN-hook entry points.  C(i, j) is at
// C[j * ldc + i]; ldc < M means overlapping columns (see k_colmajor.hip).
enum CmOp { kCmNone = 0, kCmZero = 1, kCmScale = 2 };
// op on the M x N column-major C, then C += bias[i] (bias may be null).
hipError_t launch_cm_fixup(float* C, int M, int N, long long ldc, int op, float beta, const float* bias,
                           hipStream_t s);
// T (N x M, row stride M) <- the N strided rows of C.
hipError_t launch_cm_gather(const float* C, long long ldc, float* T, int M, int N, hipStream_t s);
// Rows of T back into C at stride ldc < M, in row order (the last row wins).
hipError_t launch_cm_scatter(const float* T, int M, int N, long long ldc, float* C, hipStream_t s);
// dst (cols x rows, row stride ldd) = transpose of src (rows x cols, stride lds).
hipError_t launch_transpose_u16(const uint16_t* src, int rows, int cols, long long lds, uint16_t* dst,
                                long long ldd, hipStream_t s);

}  // namespace dnnopt_hip
