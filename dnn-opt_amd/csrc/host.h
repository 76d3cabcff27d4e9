// host.h -- internal host-side interfaces: device state, workspace, dispatch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "dnnopt_hip.h"
#include "kernels.h"

namespace dnnopt_hip {

// ---------------------------------------------------------------- runtime
// Compute units of the current device, or 256 (MI355X) when no device is
// visible, so that plans can be computed and tested without a GPU.
int num_cus();
int visible_devices();
int to_status(hipError_t e);

// Per-(device, stream, slot) scratch: `tickets` (kMaxTickets counters, zero
// between launches) followed by `part_bytes` of partial-sum space.  Launches
// on one stream are ordered, so they can share it; the buffer only grows.
// Slot 0 serves the GEMM kernels, slot 1 the int8 quantization staging.
// The caller must hold a StreamLock for `s` from this call until its last
// launch that uses the buffer is enqueued.
constexpr int kMaxTickets = 4096;  // ticket slots, kTicketStride words each
constexpr size_t kTicketBytes = (size_t)kMaxTickets * kTicketStride * sizeof(unsigned);
int get_workspace(hipStream_t s, size_t part_bytes, void** part, unsigned** tickets, int slot = 0);

// Serialises the calls that enqueue work on one stream of one device (the
// current device).  Every entry point that may take workspace holds it from
// planning until its last launch is enqueued, so that
//   * the launches of two calls sharing a stream never interleave (a split-k
//     kernel and its reduce kernel communicate through the stream's
//     workspace, which the other call would overwrite), and
//   * a workspace buffer is only freed (when it grows) by the holder of the
//     lock, after synchronising the stream: no other call can still hold a
//     pointer into it.
// Recursive: entry points call one another on the same thread.
class StreamLock {
public:
    explicit StreamLock(hipStream_t s);
    ~StreamLock();
    StreamLock(const StreamLock&) = delete;
    StreamLock& operator=(const StreamLock&) = delete;

private:
    void* mu_;
};

// The calling thread's own stream on the current device, for the synchronous
// host APIs (gemm.h, cblas.h, the oneDNN hook): each host thread gets a
// distinct stream, hence distinct workspace, so that concurrent synchronous
// calls from several threads neither share buffers nor wait on each other.
// Streams are created with default flags and priority (ordered with the null
// stream, like the null-stream launches they replace), taken from a pool of
// the process and returned to it when the thread ends; they are never
// destroyed.  nullptr (with *status set) if no stream could be created.
hipStream_t thread_stream(int* status);

// ---------------------------------------------------------------- dispatch
struct Launch {
    dnnopt_plan pub;
    int family = DNNOPT_K_NONE;
    int mode = 0;        // SkinnyMode / TileMode / int8 epilogue
    int mr = 0, nw = 0;  // skinny (rowdot: nw = waves splitting k)
    int unroll = 16;     // skinny: rows of B per load block of a wave
    int cfg = 0;         // tile / int8 configuration index (tall: column tiles nt)
    size_t lds = 0;      // dynamic LDS bytes (tall)
    int bm = 0, bn = 0;  // tile shape
    int tn = 0, tm = 0;  // tile grid (column tiles, row tiles)
    int tiles = 0;       // skinny: column tiles T (the grid has G >= T workgroups)
    dim3 grid;
    size_t part_bytes = 0;
    int tickets = 0;
    int defer_reduce = 0;
};

// Split-k reduction strategy (tunable SPLIT_REDUCE): 0 = last-arriving
// workgroup (ticket) wherever the kernel has one; 1 (default) = the
// planners' choice: the separate reduce kernel, except skinny launches of at
// most 3 rows whose last workgroup reads at most kSkinnyTicketBytes of
// partials and fp32 tile launches of at most 8 splits; 2 = the reduce kernel
// everywhere.  split_reduce_mode() is 0 for
// the ticket, 1 for the reduce kernel (the planners' default).
constexpr long long kSkinnyTicketBytes = 48 * 1024;
int split_reduce_mode();

// Tunable parameters of the planners (tune.cpp), in the order of the
// DNNOPT_TUNE_* keys of dnnopt_hip.h.  Switches are 1 (on) / 0 (off);
// forcing values are 0 (or -1 for kTuneS8Cfg) when the planner decides.
enum Tunable {
    kTuneQ8B = 0,           // fp32-API int8 M > 8: int8 tiles quantizing B while staging it
    kTuneKOuter,            // k-outer kernel for TransA split-k shapes
    kTuneKOuterWgsPerCu,    // its workgroups per CU
    kTuneWavesPerCu,        // register tiles: waves per CU for the split count
    kTuneSkinnyNW,          // skinny waves per workgroup (4, 8, 16; 0 = by size)
    kTuneSkinnyWgsPerCu,    // skinny workgroups per CU
    kTuneMaxSplits,         // register tiles: most k-splits
    kTuneSplitReduce,       // split-k sums: 0 last workgroup, 1 planners' choice, 2 reduce kernel
    kTuneSkinnyWgs,         // forced skinny workgroup count
    kTuneTileSplits,        // forced tile k-splits
    kTuneTileCfg,           // forced tile configuration
    kTuneTileTicket,        // LDS-DMA tiles: last-workgroup sum of their splits
    kTuneS8Cfg,             // forced int8 tile configuration
    kTuneS8Rowdot,          // int8 M <= 4 on the row-dot kernel
    kTuneS8Splits,          // forced int8 k-splits
    kTuneRowdotKW,          // forced row-dot k-split waves (1, 2, 4, 8)
    kTuneTallRT,            // forced tall-kernel row tiles per wave (1, 2)
    kTuneTallWgsPerCu,      // tall-kernel workgroups per CU
    kTuneTall,              // tall-skinny kernel with B resident in LDS
    kTuneWide,              // 1: every fp32 / bf16 / int8 GEMM on the last-resort kernel (tests)
    kTuneCount
};
int tunable(Tunable t);
int tunable_default(Tunable t);

int plan_skinny(int mode, int M, int N, int K, int ldb, Launch* L);
// fp32, large M, N <= 64, B small enough to stay in LDS (no transposed A).
// ldc: row stride of C (0 = N); C is addressed with 32-bit offsets from its
// first element, so ((M - 1) * ldc + N) * 4 must stay below 2^31.
int plan_tall(int transB, int M, int N, int K, int lda, int ldb, Launch* L, int ldc = 0);
// M <= 8 against B stored N x K; mode 0 fp32, 1 bf16 storage.
int plan_rowdot(int mode, int M, int N, int K, int lda, int ldb, Launch* L);
// lds_ok = false keeps bf16 GEMMs off the LDS-staged kernel (operands whose
// rows do not start on 4-byte boundaries).
// ldc: row stride of C (0 = N); the LDS-staged kernels address a C tile with
// 32-bit offsets from its first element.
int plan_tile(int mode, int transA, int transB, int M, int N, int K, int lda, int ldb, Launch* L,
              bool lds_ok = true, int ldc = 0);
// lds_ok = false keeps int8 GEMMs off the LDS-staged kernel (rows of A or B
// not on 4-byte boundaries).
// lda, ldb: row strides of A and B (0 = packed, K).
int plan_s8(int epi, int M, int N, int K, Launch* L, bool lds_ok = true, int lda = 0, int ldb = 0, int ldc = 0);

// Caller-provided device scratch in place of the stream's workspace: the
// first kMaxTickets * 4 bytes are the ticket counters (zero between
// launches), the rest holds partial sums.  A launch that needs more than
// `bytes` fails with DNNOPT_ERR_SCRATCH_LIMIT; nothing is allocated.
struct ExtScratch {
    void* base;
    size_t bytes;
};

// fp32 GEMM of dnnopt_hip_sgemm with an optional per-column bias added to
// each finished output (one more rounding): C = epilogue + bias[n].  With
// `ext`, split-k partials and tickets live in that scratch (no workspace is
// taken and no stream lock is held).
int sgemm_bias(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda, const float* B,
               int ldb, float beta, float* C, int ldc, const float* bias, hipStream_t s,
               const ExtScratch* ext = nullptr);

// The 64-bit last-resort kernel (dnnopt_wide) for an M x N output.
void plan_wide(int M, int N, Launch* L);
// Route an fp32 GEMM to a kernel family (skinny, row-dot, tall, tile; the
// last-resort kernel when no other one can address the operands).
int plan_sgemm(int transA, int transB, int M, int N, int K, int lda, int ldb, Launch* L, int ldc = 0);
// Route a bf16 GEMM (fp32_inputs: operands are fp32 and rounded in registers;
// transB: B stored N x K, bf16 storage only).
int plan_bf16(int fp32_inputs, int M, int N, int K, int lda, int ldb, Launch* L, int transB = 0, int ldc = 0);

// Workspace slots (get_workspace): 0 GEMM partials and tickets, 1 int8
// quantization staging, 2 the column-major hook's temporary C, 3 transposed
// bf16 A operands.
constexpr int kSlotGemm = 0, kSlotQuant = 1, kSlotHookC = 2, kSlotTransA = 3;

}  // namespace dnnopt_hip
