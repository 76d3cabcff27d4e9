// api_internal.h -- helpers shared by the host-pointer APIs (gemm.h, cblas.h).
#pragma once

#include <stddef.h>

namespace dnnopt_api {

// A device view of one operand: `dev` is what the kernel reads or writes;
// when the caller passed host memory, `host`/`bytes` say where to copy back.
struct Operand {
    void* dev = nullptr;
    void* host = nullptr;
    size_t bytes = 0;
};

void record(int status, const char* what);
int last_status();
void set_threads(int n);
int get_threads();

bool is_device_pointer(const void* p);
// The calling thread's stream on the current device (a hipStream_t), or
// nullptr with *status set; nothing is done when *status is already an error.
void* api_stream(int* status);
// Stage `bytes` of `host` into this thread's staging slot `slot` (0..3) unless
// it already is device memory; `copy` = false skips the upload (output-only
// operand).  The upload is enqueued on `stream`.
Operand stage_in(const void* host, size_t bytes, int slot, bool copy, void* stream, int* status);
// Copy a staged operand back to host memory and wait for `stream`.
int stage_out(const Operand& o, void* stream);
int sync_stream(void* stream);
// Ends a synchronous call that stages operands: unless released once the
// results are back, it waits for `stream` (status ignored) when the call
// returns, so that an error return never leaves an upload from, or a copy
// into, the caller's host buffers in flight (pinned host memory is staged
// asynchronously).
struct DrainGuard {
    void* stream;
    explicit DrainGuard(void* s) : stream(s) {}
    ~DrainGuard() {
        if (stream) (void)sync_stream(stream);
    }
    DrainGuard(const DrainGuard&) = delete;
    DrainGuard& operator=(const DrainGuard&) = delete;
    void release() { stream = nullptr; }
};

// Bytes spanned by a rows x cols row-major block with row stride ld.
size_t extent(int rows, int cols, int ld, size_t esize);

// fp32 GEMM with row-major transpose flags, host or device pointers,
// synchronous.  naive = the scalar reference kernel (no transposes).
int sgemm_any(int ta, int tb, int M, int N, int K, float alpha, const float* A, int lda, const float* B,
              int ldb, float beta, float* C, int ldc, bool naive);

}  // namespace dnnopt_api
