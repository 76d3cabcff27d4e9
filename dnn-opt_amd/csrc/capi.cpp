// capi.cpp -- the extern "C" boundary declared in include/dnnopt_hip.h.
//
// Each entry point validates its arguments, asks the dispatcher for a launch,
// takes the stream's workspace when the launch needs one, and enqueues the
// kernel.  Nothing here falls back to the host: a failure is a status code.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "dnnopt_hip.h"
#include "host.h"

using namespace dnnopt_hip;

namespace {

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

int finish_launch(hipError_t e) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return to_status(e);
    }
    return DNNOPT_OK;
}

// The 64-bit last-resort kernel (DNNOPT_K_WIDE) for an fp32 / bf16 GEMM;
// `mode` is a TileMode (the WideMode of the same number).
int run_wide(int mode, int ta, int tb, const void* A, int lda, const void* B, int ldb, float* C, int ldc, int M,
             int N, int K, float alpha, float beta, hipStream_t s, const float* bias = nullptr) {
    WideArgs w{};
    w.A = A;
    w.B = B;
    w.C = C;
    w.lda = lda;
    w.ldb = ldb;
    w.ldc = ldc;
    w.M = M;
    w.N = N;
    w.K = K;
    w.transA = ta;
    w.transB = tb;
    w.alpha = alpha;
    w.beta = beta;
    w.bias = bias;
    return finish_launch(launch_wide(mode, w, s));
}

// Partial-sum space and tickets of a split-k launch: the stream's workspace,
// or the caller's scratch when one is given.
int take_workspace(hipStream_t s, size_t part_bytes, const ExtScratch* ext, void** part, unsigned** tickets) {
    if (!ext) return get_workspace(s, part_bytes, part, tickets);
    if (ext->bytes < kTicketBytes || part_bytes > ext->bytes - kTicketBytes) return DNNOPT_ERR_SCRATCH_LIMIT;
    *tickets = static_cast<unsigned*>(ext->base);
    *part = static_cast<char*>(ext->base) + kTicketBytes;
    return DNNOPT_OK;
}

int run_skinny(const Launch& L, const void* A, int a_sm, int a_sk, const void* B, int ldb, float* C, int ldc,
               int M, int N, int K, float alpha, float beta, hipStream_t s, const float* bias = nullptr,
               const ExtScratch* ext = nullptr) {
    SkinnyArgs a{};
    a.bias = bias;
    a.A = A;
    a.B = B;
    a.C = C;
    a.a_sm = a_sm;
    a.a_sk = a_sk;
    a.ldb = ldb;
    a.ldc = ldc;
    a.M = M;
    a.N = N;
    a.K = K;
    a.alpha = alpha;
    a.beta = beta;
    const int T = L.tiles;
    const int G = (int)L.grid.x;
    a.tiles = T;
    a.splits = (G + T - 1) / T;
    a.ncols_pad = T * skinny_tile_cols(L.mode);
    a.defer_reduce = L.defer_reduce;
    if (a.splits > 1) {
        void* part = nullptr;
        unsigned* tickets = nullptr;
        int st = take_workspace(s, L.part_bytes, ext, &part, &tickets);
        if (st != DNNOPT_OK) return st;
        a.part = static_cast<float*>(part);
        a.tickets = tickets;
    }
    // bf16 rows start on 4-byte boundaries only when the matrix does and its
    // row stride is even.  bf16 A stored K x M is read element by element.
    const bool bf16 = L.mode == kSkinnyBF16;
    const int b_aligned = !bf16 || ((reinterpret_cast<uintptr_t>(B) & 3u) == 0 && (ldb & 1) == 0);
    int a_layout = a_sk == 1 ? 0 : 1;
    if (bf16 && (a_sk != 1 || (reinterpret_cast<uintptr_t>(A) & 3u) != 0 || (a_sm & 1) != 0)) a_layout = 2;
    int st = finish_launch(launch_skinny(L.mode, L.mr, L.nw, L.unroll, b_aligned, a_layout, L.grid, a, s));
    if (st != DNNOPT_OK || !L.defer_reduce) return st;
    return finish_launch(launch_skinny_reduce(a.part, G, T, skinny_tile_cols(L.mode), M, N, a.ncols_pad, alpha,
                                              beta, C, ldc, bias, s));
}

int run_tile(const Launch& L0, int ta, int tb, const void* A, int lda, const void* B, int ldb, float* C, int ldc,
             int M, int N, int K, float alpha, float beta, hipStream_t s, const float* bias = nullptr,
             const ExtScratch* ext = nullptr) {
    Launch L = L0;
    // The LDS-staged bf16 kernel reads whole dwords: bf16 operands must start
    // on 4-byte boundaries, else the register-only kernel serves the call.
    // The k-major outer-product kernel reads 16-byte chunks: its operands must
    // start on 16-byte boundaries, else the register tiles serve the call.
    if ((L.cfg >= kTileFirstLds && L.cfg != kTileKOuter && L.mode == kTileBF16 &&
         ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 3u) != 0) ||
        (L.cfg == kTileKOuter && ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15u) != 0)) {
        const int st = plan_tile(L.mode, ta, tb, M, N, K, lda, ldb, &L, false, ldc);
        if (st == DNNOPT_ERR_UNSUPPORTED)
            return run_wide(L0.mode, ta, tb, A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s, bias);
        if (st != DNNOPT_OK) return st;
    }
    TileArgs a{};
    a.bias = bias;
    a.A = A;
    a.B = B;
    a.C = C;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.M = M;
    a.N = N;
    a.K = K;
    a.alpha = alpha;
    a.beta = beta;
    a.transA = ta;
    a.transB = tb;
    a.tiles_n = L.tn;
    a.tiles_m = L.tm;
    a.splits = (int)L.grid.z;
    a.defer_reduce = L.defer_reduce;
    if (a.splits > 1) {
        void* part = nullptr;
        unsigned* tickets = nullptr;
        int st = take_workspace(s, L.part_bytes, ext, &part, &tickets);
        if (st != DNNOPT_OK) return st;
        a.part = static_cast<float*>(part);
        a.tickets = tickets;
    }
    // Register bf16 kernel: k-contiguous rows (A, and B stored N x K) that do
    // not start on 4-byte boundaries are read with shifted loads.
    const int aligned = L.cfg >= kTileFirstLds || L.mode != kTileBF16 ||
                        ((reinterpret_cast<uintptr_t>(A) & 3u) == 0 && (lda & 1) == 0 &&
                         (!tb || ((reinterpret_cast<uintptr_t>(B) & 3u) == 0 && (ldb & 1) == 0)));
    int st = finish_launch(launch_tile(L.mode, L.cfg, ta, tb, aligned, L.grid, a, s));
    if (st != DNNOPT_OK || !L.defer_reduce) return st;
    return finish_launch(
        launch_splitk_reduce(a.part, a.splits, L.tn, L.tm, L.bm, L.bn, M, N, alpha, beta, C, ldc, bias, s));
}

int run_rowdot(const Launch& L, const void* A, int lda, const void* B, int ldb, float* C, int ldc, int M, int N,
               int K, float alpha, float beta, hipStream_t s, const float* bias = nullptr) {
    RowdotArgs a{};
    a.bias = bias;
    a.A = A;
    a.B = B;
    a.C = C;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.M = M;
    a.N = N;
    a.K = K;
    a.alpha = alpha;
    a.beta = beta;
    // bf16 rows start on 4-byte boundaries only when the matrix does and its
    // row stride is even.
    const int aligned = L.mode == 0 || (((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 3u) == 0 &&
                                        (lda & 1) == 0 && (ldb & 1) == 0);
    return finish_launch(launch_rowdot(L.mode, L.mr, L.nw, aligned, L.grid, a, s));
}

bool dims_ok(int M, int N, int K) { return M > 0 && N > 0 && K > 0; }

}  // namespace

namespace dnnopt_hip {

static int sgemm_planned(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda,
                         const float* B, int ldb, float beta, float* C, int ldc, const float* bias, hipStream_t s,
                         const ExtScratch* ext) {
    Launch L;
    int st = plan_sgemm(transA, transB, M, N, K, lda, ldb, &L, ldc);
    if (st != DNNOPT_OK) return st;
    if (L.family == DNNOPT_K_WIDE)
        return run_wide(kTileF32, transA, transB, A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s, bias);
    if (L.family == DNNOPT_K_SKINNY_F32)
        return run_skinny(L, A, transA ? 1 : lda, transA ? lda : 1, B, ldb, C, ldc, M, N, K, alpha, beta, s, bias,
                          ext);
    if (L.family == DNNOPT_K_ROWDOT_F32)
        return run_rowdot(L, A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s, bias);
    if (L.family == DNNOPT_K_TALL_F32) {
        TallArgs a{A, B, C, lda, ldb, ldc, M, N, K, alpha, beta, bias};
        if (L.mr == 0) {
            // A copied by LDS-DMA needs 16-byte aligned rows; otherwise the
            // register-ring kernel takes the same grid.
            if ((reinterpret_cast<uintptr_t>(A) & 15u) == 0)
                return finish_launch(launch_tall_dma_f32(L.mode, L.grid, a, s));
            return finish_launch(launch_tall_f32(L.cfg, L.mode, 1, L.grid, tall_lds_bytes(L.cfg, K), a, s));
        }
        return finish_launch(launch_tall_f32(L.cfg, L.mode, L.mr, L.grid, L.lds, a, s));
    }
    return run_tile(L, transA, transB, A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s, bias, ext);
}

int sgemm_bias(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda, const float* B,
               int ldb, float beta, float* C, int ldc, const float* bias, hipStream_t s, const ExtScratch* ext) {
    if ((transA != 0 && transA != 1) || (transB != 0 && transB != 1)) return DNNOPT_ERR_INVALID_ARG;
    if (!dims_ok(M, N, K)) return DNNOPT_OK;
    if (!A || !B || !C) return DNNOPT_ERR_INVALID_ARG;
    if (lda < (transA ? M : K) || ldb < (transB ? K : N) || ldc < N) return DNNOPT_ERR_INVALID_ARG;
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    if (ext) return sgemm_planned(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias, s, ext);
    StreamLock lock(s);
    return sgemm_planned(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias, s, nullptr);
}

}  // namespace dnnopt_hip

extern "C" {

int dnnopt_hip_abi_version(void) { return DNNOPT_HIP_ABI_VERSION; }

int dnnopt_hip_device_count(void) { return visible_devices(); }

const char* dnnopt_hip_status_string(int status) {
    switch (status) {
        case DNNOPT_OK: return "ok";
        case DNNOPT_ERR_INVALID_ARG: return "invalid argument";
        case DNNOPT_ERR_NO_DEVICE: return "no HIP device visible";
        case DNNOPT_ERR_HIP: return "HIP runtime error";
        case DNNOPT_ERR_UNSUPPORTED: return "unsupported shape or option";
        case DNNOPT_ERR_OUT_OF_MEMORY: return "device memory allocation failed";
        case DNNOPT_ERR_SCRATCH_LIMIT:
            return "the call needs more device scratch than the no-allocation entry point holds";
        default: return "unknown status";
    }
}

int dnnopt_hip_plan_sgemm(int transA, int transB, int M, int N, int K, dnnopt_plan* out) {
    if (!out || (transA != 0 && transA != 1) || (transB != 0 && transB != 1)) return DNNOPT_ERR_INVALID_ARG;
    if (!dims_ok(M, N, K)) return DNNOPT_ERR_INVALID_ARG;
    Launch L;
    int st = plan_sgemm(transA, transB, M, N, K, transA ? M : K, transB ? K : N, &L);
    if (st == DNNOPT_OK) *out = L.pub;
    return st;
}

int dnnopt_hip_plan_sgemm_ex(int transA, int transB, int M, int N, int K, int lda, int ldb, int ldc,
                             dnnopt_plan* out) {
    if (!out || (transA != 0 && transA != 1) || (transB != 0 && transB != 1)) return DNNOPT_ERR_INVALID_ARG;
    if (!dims_ok(M, N, K)) return DNNOPT_ERR_INVALID_ARG;
    if (lda < (transA ? M : K) || ldb < (transB ? K : N) || ldc < N) return DNNOPT_ERR_INVALID_ARG;
    Launch L;
    int st = plan_sgemm(transA, transB, M, N, K, lda, ldb, &L, ldc);
    if (st == DNNOPT_OK) *out = L.pub;
    return st;
}

int dnnopt_hip_plan_gemm_bf16(int fp32_inputs, int M, int N, int K, dnnopt_plan* out) {
    if (!out || !dims_ok(M, N, K)) return DNNOPT_ERR_INVALID_ARG;
    Launch L;
    int st = plan_bf16(fp32_inputs ? 1 : 0, M, N, K, K, N, &L);
    if (st == DNNOPT_OK) *out = L.pub;
    return st;
}

int dnnopt_hip_plan_gemm_bf16_ex(int transA, int transB, int M, int N, int K, dnnopt_plan* out) {
    if (!out || !dims_ok(M, N, K) || (transA != 0 && transA != 1) || (transB != 0 && transB != 1))
        return DNNOPT_ERR_INVALID_ARG;
    // As dnnopt_hip_gemm_bf16_ex with unpadded strides (a transposed A is
    // read in place by the skinny kernel up to M = 8 with B stored K x N, else
    // first copied to an even row stride).
    const int lda = transA ? (K + 1) & ~1 : K;
    Launch L;
    if (transA && !transB && M <= 8 && !tunable(kTuneWide) && plan_skinny(kSkinnyBF16, M, N, K, N, &L) == DNNOPT_OK) {
        *out = L.pub;
        return DNNOPT_OK;
    }
    int st = plan_bf16(0, M, N, K, lda, transB ? K : N, &L, transB);
    if (st == DNNOPT_OK) *out = L.pub;
    return st;
}

int dnnopt_hip_plan_gemm_s8(int with_scale, int M, int N, int K, dnnopt_plan* out) {
    if (!out || !dims_ok(M, N, K)) return DNNOPT_ERR_INVALID_ARG;
    Launch L;
    int st = plan_s8(with_scale ? 1 : 0, M, N, K, &L);
    if (st == DNNOPT_OK) *out = L.pub;
    return st;
}

int dnnopt_hip_plan_gemm_int8_f32(int M, int N, int K, dnnopt_plan* out) {
    if (!out || !dims_ok(M, N, K)) return DNNOPT_ERR_INVALID_ARG;
    Launch L;
    if (M <= 8 && plan_skinny(kSkinnyF32, M, N, K, N, &L) == DNNOPT_OK) {
        // dnnopt_skinny_q8 runs on the fp32 skinny plan's grid and partials,
        // summed by its own reduce kernel (no ticket slots).
        *out = L.pub;
        out->workspace_bytes = L.part_bytes;
        out->kernel = DNNOPT_K_SKINNY_Q8;
        out->block = skinny_q8_waves() * 64;
        snprintf(out->name, sizeof out->name, "%s", "dnnopt_skinny_q8");
        return DNNOPT_OK;
    }
    // M > 8: the int8 tiles that quantize the fp32 B while staging it (as
    // dnnopt_hip_gemm_int8_f32 with unpadded strides and DNNOPT_Q8B unset).
    const int ldq = (K + 15) & ~15;
    if (((long long)K * N + N) * 4 < 0x7FFFFFFFll && ((long long)M + 64) * ldq < 0x7FFFFFFFll &&
        (long long)((N + 31) / 32) * ((M + 63) / 64) <= 0x7FFFFFF0ll) {
        *out = dnnopt_plan{};
        out->kernel = DNNOPT_K_MFMA_S8;
        out->rows = 64;
        out->cols = 32;
        out->splits = 1;
        out->grid_x = xcd_grid((N + 31) / 32, (M + 63) / 64);
        out->grid_y = out->grid_z = 1;
        out->block = 256;
        snprintf(out->name, sizeof out->name, "%s", "dnnopt_s8_lds_q8b");
        return DNNOPT_OK;
    }
    int st = plan_s8(1, M, N, K, &L, true, ldq, ldq, N);
    if (st == DNNOPT_OK) *out = L.pub;
    return st;
}

int dnnopt_hip_sgemm(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda,
                     const float* B, int ldb, float beta, float* C, int ldc, void* stream) {
    return sgemm_bias(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, nullptr, as_stream(stream));
}

int dnnopt_hip_sgemm_naive(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                           float beta, float* C, int ldc, void* stream) {
    if (!dims_ok(M, N, K)) return DNNOPT_OK;
    if (!A || !B || !C) return DNNOPT_ERR_INVALID_ARG;
    if (lda < K || ldb < N || ldc < N) return DNNOPT_ERR_INVALID_ARG;
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    return finish_launch(launch_naive_f32(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, as_stream(stream)));
}

static int gemm_bf16_common(int fp32_inputs, int M, int N, int K, float alpha, const void* A, int lda,
                            const void* B, int ldb, float beta, float* C, int ldc, void* stream) {
    if (!dims_ok(M, N, K)) return DNNOPT_OK;
    if (!A || !B || !C) return DNNOPT_ERR_INVALID_ARG;
    if (lda < K || ldb < N || ldc < N) return DNNOPT_ERR_INVALID_ARG;
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    hipStream_t s = as_stream(stream);
    StreamLock lock(s);
    Launch L;
    int st = plan_bf16(fp32_inputs, M, N, K, lda, ldb, &L, 0, ldc);
    if (st != DNNOPT_OK) return st;
    if (L.family == DNNOPT_K_WIDE)
        return run_wide(fp32_inputs ? kTileF2B : kTileBF16, 0, 0, A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s);
    if (L.family == DNNOPT_K_SKINNY_BF16 || L.family == DNNOPT_K_SKINNY_F2B)
        return run_skinny(L, A, lda, 1, B, ldb, C, ldc, M, N, K, alpha, beta, s);
    return run_tile(L, 0, 0, A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s);
}

int dnnopt_hip_gemm_bf16(int M, int N, int K, float alpha, const uint16_t* A, int lda, const uint16_t* B, int ldb,
                         float beta, float* C, int ldc, void* stream) {
    return gemm_bf16_common(0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream);
}

int dnnopt_hip_gemm_bf16_ex(int transA, int transB, int M, int N, int K, float alpha, const uint16_t* A, int lda,
                            const uint16_t* B, int ldb, float beta, float* C, int ldc, void* stream) {
    if ((transA != 0 && transA != 1) || (transB != 0 && transB != 1)) return DNNOPT_ERR_INVALID_ARG;
    if (!dims_ok(M, N, K)) return DNNOPT_OK;
    if (!A || !B || !C) return DNNOPT_ERR_INVALID_ARG;
    if (lda < (transA ? M : K) || ldb < (transB ? K : N) || ldc < N) return DNNOPT_ERR_INVALID_ARG;
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    hipStream_t s = as_stream(stream);
    StreamLock lock(s);
    Launch L;
    if (transA && !transB && M <= 8 && !tunable(kTuneWide)) {
        // The skinny kernel reads a K x M A in place (A is M*K elements).
        if (plan_skinny(kSkinnyBF16, M, N, K, ldb, &L) == DNNOPT_OK)
            return run_skinny(L, A, 1, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s);
    }
    // MFMA tiles read k-contiguous rows of A: a K x M A is first transposed
    // into workspace (M x K, even row stride so rows stay 4-byte aligned),
    // unless no tile can take the shape (then the last-resort kernel reads
    // it in place).
    const int ldt = transA ? (K + 1) & ~1 : lda;
    int st = plan_bf16(0, M, N, K, ldt, ldb, &L, transB, ldc);
    if (st != DNNOPT_OK) return st;
    if (L.family == DNNOPT_K_WIDE)
        return run_wide(kTileBF16, transA, transB, A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s);
    if (transA) {
        void* ws = nullptr;
        unsigned* unused = nullptr;
        st = get_workspace(s, (size_t)M * ldt * sizeof(uint16_t), &ws, &unused, kSlotTransA);
        if (st != DNNOPT_OK) return st;
        st = finish_launch(launch_transpose_u16(A, K, M, lda, static_cast<uint16_t*>(ws), ldt, s));
        if (st != DNNOPT_OK) return st;
        A = static_cast<const uint16_t*>(ws);
        lda = ldt;
    }
    if (L.family == DNNOPT_K_SKINNY_BF16) return run_skinny(L, A, lda, 1, B, ldb, C, ldc, M, N, K, alpha, beta, s);
    if (L.family == DNNOPT_K_ROWDOT_BF16) return run_rowdot(L, A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s);
    return run_tile(L, 0, transB, A, lda, B, ldb, C, ldc, M, N, K, alpha, beta, s);
}

int dnnopt_hip_gemm_bf16_f32in(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                               float beta, float* C, int ldc, void* stream) {
    return gemm_bf16_common(1, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream);
}

// Dynamic dequantization of the fp32-API gemm_int8 (EPI 1 with amax): C =
// (sA sB alpha) acc (+ beta C), sA, sB from the bits of max|A|, max|B|.
struct DynDequant {
    const unsigned* amax;
    float alpha, beta;
};

static int gemm_s8_common(int epi, int M, int N, int K, const int8_t* A, int lda, const int8_t* B, int ldb,
                          const float* scale, void* C, int ldc, void* stream, const DynDequant* dyn = nullptr) {
    if (!dims_ok(M, N, K)) return DNNOPT_OK;
    if (!A || !B || !C || (epi && !scale && !dyn)) return DNNOPT_ERR_INVALID_ARG;
    if (lda < K || ldb < K || ldc < N) return DNNOPT_ERR_INVALID_ARG;
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    const int aligned = ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 3u) == 0 &&
                        (lda & 3) == 0 && (ldb & 3) == 0;
    hipStream_t s = as_stream(stream);
    StreamLock lock(s);
    Launch L;
    int st = plan_s8(epi, M, N, K, &L, aligned != 0, lda, ldb, ldc);
    if (st != DNNOPT_OK) return st;
    if (L.family == DNNOPT_K_WIDE) {
        WideArgs w{};
        w.A = A;
        w.B = B;
        w.C = C;
        w.lda = lda;
        w.ldb = ldb;
        w.ldc = ldc;
        w.M = M;
        w.N = N;
        w.K = K;
        w.transB = 1;  // int8 B is stored N x K
        w.epi = epi;
        w.scale = scale;
        w.amax = dyn ? dyn->amax : nullptr;
        w.alpha = dyn ? dyn->alpha : 1.0f;
        w.beta = dyn ? dyn->beta : 0.0f;
        return finish_launch(launch_wide(kWideS8, w, s));
    }
    if (L.family == DNNOPT_K_ROWDOT_S8) {
        RowdotArgs r{};
        r.A = A;
        r.B = B;
        r.C = epi ? static_cast<float*>(C) : nullptr;
        r.Ci = epi ? nullptr : static_cast<int32_t*>(C);
        r.scale = scale;
        r.amax = dyn ? dyn->amax : nullptr;
        r.alpha = dyn ? dyn->alpha : 1.0f;
        r.beta = dyn ? dyn->beta : 0.0f;
        r.lda = lda;
        r.ldb = ldb;
        r.ldc = ldc;
        r.M = M;
        r.N = N;
        r.K = K;
        return finish_launch(launch_rowdot(L.mode, L.mr, L.nw, aligned, L.grid, r, s));
    }
    S8Args a{};
    a.A = A;
    a.B = B;
    a.C = C;
    a.scale = scale;
    a.amax = dyn ? dyn->amax : nullptr;
    a.alpha = dyn ? dyn->alpha : 1.0f;
    a.beta = dyn ? dyn->beta : 0.0f;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.M = M;
    a.N = N;
    a.K = K;
    a.splits = (int)L.grid.z;
    a.defer_reduce = L.defer_reduce;
    a.tiles_n = L.tn;
    a.tiles_m = L.tm;
    if (a.splits > 1) {
        void* part = nullptr;
        unsigned* tickets = nullptr;
        st = get_workspace(s, L.part_bytes, &part, &tickets);
        if (st != DNNOPT_OK) return st;
        a.part = static_cast<int32_t*>(part);
        a.tickets = tickets;
    }
    st = finish_launch(launch_mfma_s8(L.cfg, epi, aligned, L.grid, a, s));
    if (st != DNNOPT_OK || !L.defer_reduce) return st;
    return finish_launch(launch_s8_reduce(a.part, a.splits, L.tn, L.tm, L.bm, L.bn, M, N, epi, scale, a.amax, a.alpha,
                                          a.beta, C, ldc, s));
}

int dnnopt_hip_gemm_s8s8s32(int M, int N, int K, const int8_t* A, int lda, const int8_t* B, int ldb, int32_t* C,
                            int ldc, void* stream) {
    return gemm_s8_common(0, M, N, K, A, lda, B, ldb, nullptr, C, ldc, stream);
}

int dnnopt_hip_gemm_s8s8f32_colscale(int M, int N, int K, const int8_t* A, int lda, const int8_t* B, int ldb,
                                     const float* col_scale, float* C, int ldc, void* stream) {
    return gemm_s8_common(1, M, N, K, A, lda, B, ldb, col_scale, C, ldc, stream);
}

int dnnopt_hip_gemm_int8_f32(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                             float beta, float* C, int ldc, void* stream) {
    if (!dims_ok(M, N, K)) return DNNOPT_OK;
    if (!A || !B || !C) return DNNOPT_ERR_INVALID_ARG;
    if (lda < K || ldb < N || ldc < N) return DNNOPT_ERR_INVALID_ARG;
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    hipStream_t s = as_stream(stream);
    StreamLock lock(s);
    if (M <= 8) {
        // The reference's small-M route (division quantizer, its own
        // epilogues), only in dnnopt_skinny_q8.  Two passes over the fp32 B:
        // the maxima, then dnnopt_skinny_q8, which quantizes B as it streams
        // it (plus its reduce kernel when k is split over workgroups).
        // Staging (slot 1): [absmax partials][max|A|, max|B|].
        Launch L;
        if (plan_skinny(kSkinnyF32, M, N, K, ldb, &L) != DNNOPT_OK) return DNNOPT_ERR_UNSUPPORTED;
        {
            int ga = 1, gb = 1;
            absmax_blocks(M, N, K, &ga, &gb);
            const size_t part_bytes = ((size_t)(ga + gb) * 4 + 255) & ~(size_t)255;
            void* stage = nullptr;
            unsigned* unused = nullptr;
            int st = get_workspace(s, part_bytes + 256, &stage, &unused, kSlotQuant);
            if (st != DNNOPT_OK) return st;
            SkinnyQ8Args a{};
            a.A = A;
            a.B = B;
            a.C = C;
            unsigned* qpart = static_cast<unsigned*>(stage);
            a.qpart = qpart;
            a.amax = reinterpret_cast<unsigned*>(static_cast<char*>(stage) + part_bytes);
            a.lda = lda;
            a.ldb = ldb;
            a.ldc = ldc;
            a.M = M;
            a.N = N;
            a.K = K;
            a.ga = ga;
            a.gb = gb;
            a.alpha = alpha;
            a.beta = beta;
            a.tiles = L.tiles;
            a.splits = ((int)L.grid.x + L.tiles - 1) / L.tiles;
            a.ncols_pad = L.tiles * skinny_tile_cols(kSkinnyF32);
            a.defer = (int)L.grid.x > L.tiles ? 1 : 0;
            if (a.defer) {
                void* part = nullptr;
                unsigned* tickets = nullptr;
                st = get_workspace(s, L.part_bytes, &part, &tickets);
                if (st != DNNOPT_OK) return st;
                a.part = static_cast<int32_t*>(part);
            }
            st = finish_launch(launch_absmax(A, lda, B, ldb, M, N, K, qpart, s));
            if (st != DNNOPT_OK) return st;
            return finish_launch(launch_skinny_q8(M, L.grid, a, s));
        }
    }
    const bool q8b_ok = tunable(kTuneQ8B) != 0;
    const int ldq = (K + 15) & ~15;
    // The q8b tiles address B, their quantized A and their 64-row block of C
    // with 31-bit buffer offsets; larger strides take the quantization pass
    // and gemm_s8_common, whose planner checks its own ranges.
    if (q8b_ok && ((long long)K * ldb + N) * 4 < 0x7FFFFFFFll && ((long long)M + 64) * ldq < 0x7FFFFFFFll &&
        ((long long)64 * ldc + N) * 4 < 0x7FFFFFFFll && (long long)((N + 31) / 32) * ((M + 63) / 64) <= 0x7FFFFFF0ll) {
        // Maxima, A quantized (M x ldq), then 64 x 32 int8 tiles that quantize
        // the fp32 B while staging it: no int8 copy of B.  Staging (slot 1):
        // [qA M x ldq][absmax partials][max|A|, max|B|].
        int ga = 1, gb = 1;
        absmax_blocks(M, N, K, &ga, &gb);
        const size_t qa_bytes = ((size_t)M * ldq + 255) & ~(size_t)255;
        const size_t part_bytes = ((size_t)(ga + gb) * 4 + 255) & ~(size_t)255;
        void* stage = nullptr;
        unsigned* unused = nullptr;
        int st = get_workspace(s, qa_bytes + part_bytes + 256, &stage, &unused, kSlotQuant);
        if (st != DNNOPT_OK) return st;
        char* base = static_cast<char*>(stage);
        int8_t* qa = reinterpret_cast<int8_t*>(base);
        unsigned* part = reinterpret_cast<unsigned*>(base + qa_bytes);
        unsigned* amax = reinterpret_cast<unsigned*>(base + qa_bytes + part_bytes);
        st = finish_launch(launch_absmax(A, lda, B, ldb, M, N, K, part, s));
        if (st != DNNOPT_OK) return st;
        st = finish_launch(launch_quant_a(A, lda, M, K, ldq, part, ga, gb, amax, qa, s));
        if (st != DNNOPT_OK) return st;
        S8Args a{};
        a.A = qa;
        a.Bf = B;
        a.C = C;
        a.lda = ldq;
        a.ldb = ldb;
        a.ldc = ldc;
        a.M = M;
        a.N = N;
        a.K = K;
        a.splits = 1;
        a.tiles_n = (N + 31) / 32;
        a.tiles_m = (M + 63) / 64;
        a.amax = amax;
        a.alpha = alpha;
        a.beta = beta;
        a.qpart = part;
        a.ga = ga;
        a.gb = gb;
        return finish_launch(launch_s8_q8b(dim3((unsigned)xcd_grid(a.tiles_n, a.tiles_m)), a, s));
    }
    if (N > 0x7FFFFFFF / 2 || (long long)N * ((K + 15) & ~15) > 0x7FFFFFFFll) return DNNOPT_ERR_UNSUPPORTED;
    // Staging (slot 1): [qA M x ldq][qB N x ldq][absmax partials][max|A|, max|B|];
    // ldq pads K to 16 bytes so every quantized row is 16-byte aligned.
    // Three launches: maxima, quantization, and the int8 GEMM whose epilogue
    // dequantizes straight into C.
    int ga = 1, gb = 1;
    absmax_blocks(M, N, K, &ga, &gb);
    const size_t qa_bytes = ((size_t)M * ldq + 255) & ~(size_t)255;
    const size_t qb_bytes = ((size_t)N * ldq + 255) & ~(size_t)255;
    const size_t part_bytes = ((size_t)(ga + gb) * 4 + 255) & ~(size_t)255;
    void* stage = nullptr;
    unsigned* unused = nullptr;
    int st = get_workspace(s, qa_bytes + qb_bytes + part_bytes + 256, &stage, &unused, kSlotQuant);
    if (st != DNNOPT_OK) return st;
    char* base = static_cast<char*>(stage);
    int8_t* qa = reinterpret_cast<int8_t*>(base);
    int8_t* qb = reinterpret_cast<int8_t*>(base + qa_bytes);
    unsigned* part = reinterpret_cast<unsigned*>(base + qa_bytes + qb_bytes);
    unsigned* amax = reinterpret_cast<unsigned*>(base + qa_bytes + qb_bytes + part_bytes);
    st = finish_launch(launch_quant_pair(A, lda, B, ldb, M, N, K, ldq, part, amax, qa, qb, s));
    if (st != DNNOPT_OK) return st;
    const DynDequant dyn{amax, alpha, beta};
    return gemm_s8_common(1, M, N, K, qa, ldq, qb, ldq, nullptr, C, ldc, stream, &dyn);
}

int dnnopt_hip_saxpy(int N, float alpha, const float* X, int incX, float* Y, int incY, void* stream) {
    if (N <= 0 || alpha == 0.0f) return DNNOPT_OK;
    if (!X || !Y || incX < 0 || incY < 0) return DNNOPT_ERR_INVALID_ARG;
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    return finish_launch(launch_saxpy(N, alpha, X, incX, Y, incY, as_stream(stream)));
}

int dnnopt_hip_fill(void* dst, size_t n, int dtype, int dist, uint64_t seed, uint32_t tensor_id, double p0,
                    double p1, void* stream) {
    if (n == 0) return DNNOPT_OK;
    if (!dst || dtype < 0 || dtype > 2 || dist < 0 || dist > 2) return DNNOPT_ERR_INVALID_ARG;
    if ((dtype == 2) != (dist == 2)) return DNNOPT_ERR_INVALID_ARG;
    if (dtype == 2 && (p0 < -128 || p1 > 127 || p0 > p1)) return DNNOPT_ERR_INVALID_ARG;
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    return finish_launch(launch_fill(dst, n, dtype, dist, seed, tensor_id, p0, p1, as_stream(stream)));
}

}  // extern "C"
