// api.cpp -- the reference's synchronous C++ API (include/dnnopt/gemm/gemm.h)
// on top of the C-ABI entry points.
//
// Pointer residency: device and managed pointers are used in place; any other
// pointer is host memory and is staged through per-thread device buffers
// (host -> device before the launch, C back after it).  The call waits for
// the launch before returning, as the reference's calls are synchronous.
// There is no host compute path: if no device is visible or a launch fails,
// C is left unmodified and the failure is recorded (dnnopt_hip_last_status)
// and reported once on stderr.
//
// Threads: every host thread enqueues on its own stream (thread_stream) and
// stages through its own buffers, so concurrent calls from several threads
// share no device memory and run side by side, as the reference's calls are
// reentrant.  The streams are ordered with the null stream, so device
// operands written by earlier null-stream work are read after it.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <map>

#include "api_internal.h"
#include "dnnopt/gemm/gemm.h"
#include "dnnopt_hip.h"
#include "host.h"

namespace dnnopt_api {

namespace {

thread_local int t_last_status = DNNOPT_OK;
std::atomic<int> g_num_threads{0};

struct StageBuf {
    void* ptr = nullptr;
    size_t cap = 0;
    ~StageBuf() {
        if (ptr) (void)hipFree(ptr);
    }
    void* get(size_t bytes, int* st) {
        if (cap >= bytes && ptr) return ptr;
        if (ptr) {
            (void)hipFree(ptr);
            ptr = nullptr;
            cap = 0;
        }
        if (hipMalloc(&ptr, bytes) != hipSuccess) {
            (void)hipGetLastError();
            ptr = nullptr;
            *st = DNNOPT_ERR_OUT_OF_MEMORY;
            return nullptr;
        }
        cap = bytes;
        return ptr;
    }
};

// Staging buffers of this thread, per device.
struct StageSet {
    StageBuf slot[4];
};
thread_local std::map<int, StageSet> t_stage;

StageBuf& stage_buf(int slot, int* st) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        *st = DNNOPT_ERR_NO_DEVICE;
    }
    return t_stage[dev].slot[slot];
}

}  // namespace

void* api_stream(int* st) {
    if (*st != DNNOPT_OK) return nullptr;
    return dnnopt_hip::thread_stream(st);
}

void record(int status, const char* what) {
    t_last_status = status;
    if (status == DNNOPT_OK) return;
    static std::atomic<int> reported{0};
    if (reported.fetch_add(1) == 0)
        fprintf(stderr, "dnnopt: %s failed: %s (further failures are not reported)\n", what,
                dnnopt_hip_status_string(status));
}

int last_status() { return t_last_status; }
void set_threads(int n) { g_num_threads.store(n < 0 ? 0 : n); }
int get_threads() { return g_num_threads.load(); }

bool is_device_pointer(const void* p) {
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

Operand stage_in(const void* host, size_t bytes, int slot, bool copy, void* stream, int* st) {
    Operand o;
    if (*st != DNNOPT_OK || bytes == 0) return o;
    if (is_device_pointer(host)) {
        o.dev = const_cast<void*>(host);
        return o;
    }
    StageBuf& buf = stage_buf(slot, st);
    if (*st != DNNOPT_OK) return o;
    void* d = buf.get(bytes, st);
    if (!d) return o;
    if (copy) {
        // Ordered before the launch on the same stream; the host memory is
        // pageable, so the copy has read it when the call returns.
        hipError_t e = hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) {
            (void)hipGetLastError();
            *st = DNNOPT_ERR_HIP;
            return o;
        }
    }
    o.dev = d;
    o.host = const_cast<void*>(host);
    o.bytes = bytes;
    return o;
}

int stage_out(const Operand& o, void* stream) {
    if (!o.host) return DNNOPT_OK;
    hipError_t e = hipMemcpyAsync(o.host, o.dev, o.bytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return DNNOPT_ERR_HIP;
    }
    return DNNOPT_OK;
}

int sync_stream(void* stream) {
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return DNNOPT_ERR_HIP;
    }
    return DNNOPT_OK;
}

size_t extent(int rows, int cols, int ld, size_t esize) {
    if (rows <= 0 || cols <= 0) return 0;
    return ((size_t)(rows - 1) * (size_t)ld + (size_t)cols) * esize;
}

// C has to be uploaded when the kernel reads it (beta != 0) or when its
// extent has elements the GEMM does not write (row padding, ldc > N): the
// whole extent is copied back.
bool c_read_or_kept(float beta, int ldc, int N) { return beta != 0.0f || ldc != N; }

int sgemm_any(int ta, int tb, int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
              float beta, float* C, int ldc, bool naive) {
    if (M <= 0 || N <= 0 || K <= 0) return DNNOPT_OK;
    if (!A || !B || !C) return DNNOPT_ERR_INVALID_ARG;
    if (dnnopt_hip_device_count() == 0) return DNNOPT_ERR_NO_DEVICE;
    int st = DNNOPT_OK;
    void* s = api_stream(&st);
    DrainGuard drain(s);
    Operand a = stage_in(A, ta ? extent(K, M, lda, 4) : extent(M, K, lda, 4), 0, true, s, &st);
    Operand b = stage_in(B, tb ? extent(N, K, ldb, 4) : extent(K, N, ldb, 4), 1, true, s, &st);
    Operand c = stage_in(C, extent(M, N, ldc, 4), 2, naive || c_read_or_kept(beta, ldc, N), s, &st);
    if (st != DNNOPT_OK) return st;
    if (naive)
        st = dnnopt_hip_sgemm_naive(M, N, K, alpha, (const float*)a.dev, lda, (const float*)b.dev, ldb, beta,
                                    (float*)c.dev, ldc, s);
    else
        st = dnnopt_hip_sgemm(ta, tb, M, N, K, alpha, (const float*)a.dev, lda, (const float*)b.dev, ldb, beta,
                              (float*)c.dev, ldc, s);
    if (st != DNNOPT_OK) return st;
    st = sync_stream(s);
    if (st != DNNOPT_OK) return st;
    st = stage_out(c, s);
    if (st == DNNOPT_OK) drain.release();
    return st;
}

}  // namespace dnnopt_api

// ---------------------------------------------------------------- dnnopt::
namespace dnnopt {

using namespace dnnopt_api;

void gemm_fp32(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb, float beta,
               float* C, int ldc) {
    gemm_fp32(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, GemmAlgo::kAuto);
}

void gemm_fp32(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb, float beta,
               float* C, int ldc, GemmAlgo algo) {
    record(sgemm_any(0, 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, algo == GemmAlgo::kNaive), "gemm_fp32");
}

void gemm_bf16(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb, float beta,
               float* C, int ldc) {
    int st = DNNOPT_OK;
    if (M > 0 && N > 0 && K > 0) {
        if (!A || !B || !C) {
            st = DNNOPT_ERR_INVALID_ARG;
        } else if (dnnopt_hip_device_count() == 0) {
            st = DNNOPT_ERR_NO_DEVICE;
        } else {
            void* s = api_stream(&st);
            DrainGuard drain(s);
            Operand a = stage_in(A, extent(M, K, lda, 4), 0, true, s, &st);
            Operand b = stage_in(B, extent(K, N, ldb, 4), 1, true, s, &st);
            Operand c = stage_in(C, extent(M, N, ldc, 4), 2, c_read_or_kept(beta, ldc, N), s, &st);
            if (st == DNNOPT_OK)
                st = dnnopt_hip_gemm_bf16_f32in(M, N, K, alpha, (const float*)a.dev, lda, (const float*)b.dev, ldb,
                                                beta, (float*)c.dev, ldc, s);
            if (st == DNNOPT_OK) st = sync_stream(s);
            if (st == DNNOPT_OK) st = stage_out(c, s);
            if (st == DNNOPT_OK) drain.release();
        }
    }
    record(st, "gemm_bf16");
}

void gemm_bf16_bf16bf16f32(int M, int N, int K, float alpha, const bfloat16_t* A, int lda, const bfloat16_t* B,
                           int ldb, float beta, float* C, int ldc) {
    int st = DNNOPT_OK;
    if (M > 0 && N > 0 && K > 0) {
        if (!A || !B || !C) {
            st = DNNOPT_ERR_INVALID_ARG;
        } else if (dnnopt_hip_device_count() == 0) {
            st = DNNOPT_ERR_NO_DEVICE;
        } else {
            void* s = api_stream(&st);
            DrainGuard drain(s);
            Operand a = stage_in(A, extent(M, K, lda, 2), 0, true, s, &st);
            Operand b = stage_in(B, extent(K, N, ldb, 2), 1, true, s, &st);
            Operand c = stage_in(C, extent(M, N, ldc, 4), 2, c_read_or_kept(beta, ldc, N), s, &st);
            if (st == DNNOPT_OK)
                st = dnnopt_hip_gemm_bf16(M, N, K, alpha, (const uint16_t*)a.dev, lda, (const uint16_t*)b.dev, ldb,
                                          beta, (float*)c.dev, ldc, s);
            if (st == DNNOPT_OK) st = sync_stream(s);
            if (st == DNNOPT_OK) st = stage_out(c, s);
            if (st == DNNOPT_OK) drain.release();
        }
    }
    record(st, "gemm_bf16_bf16bf16f32");
}

void gemm_int8(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb, float beta,
               float* C, int ldc) {
    int st = DNNOPT_OK;
    if (M > 0 && N > 0 && K > 0) {
        if (!A || !B || !C) {
            st = DNNOPT_ERR_INVALID_ARG;
        } else if (dnnopt_hip_device_count() == 0) {
            st = DNNOPT_ERR_NO_DEVICE;
        } else {
            void* s = api_stream(&st);
            DrainGuard drain(s);
            Operand a = stage_in(A, extent(M, K, lda, 4), 0, true, s, &st);
            Operand b = stage_in(B, extent(K, N, ldb, 4), 1, true, s, &st);
            Operand c = stage_in(C, extent(M, N, ldc, 4), 2, c_read_or_kept(beta, ldc, N), s, &st);
            if (st == DNNOPT_OK)
                st = dnnopt_hip_gemm_int8_f32(M, N, K, alpha, (const float*)a.dev, lda, (const float*)b.dev, ldb,
                                              beta, (float*)c.dev, ldc, s);
            if (st == DNNOPT_OK) st = sync_stream(s);
            if (st == DNNOPT_OK) st = stage_out(c, s);
            if (st == DNNOPT_OK) drain.release();
        }
    }
    record(st, "gemm_int8");
}

void gemm_int8_int8int8int32(int M, int N, int K, const int8_t* A, int lda, const int8_t* B, int ldb, int32_t* C,
                             int ldc) {
    int st = DNNOPT_OK;
    if (M > 0 && N > 0 && K > 0) {
        if (!A || !B || !C) {
            st = DNNOPT_ERR_INVALID_ARG;
        } else if (dnnopt_hip_device_count() == 0) {
            st = DNNOPT_ERR_NO_DEVICE;
        } else {
            void* s = api_stream(&st);
            DrainGuard drain(s);
            Operand a = stage_in(A, extent(M, K, lda, 1), 0, true, s, &st);
            Operand b = stage_in(B, extent(N, K, ldb, 1), 1, true, s, &st);
            Operand c = stage_in(C, extent(M, N, ldc, 4), 2, ldc != N, s, &st);
            if (st == DNNOPT_OK)
                st = dnnopt_hip_gemm_s8s8s32(M, N, K, (const int8_t*)a.dev, lda, (const int8_t*)b.dev, ldb,
                                             (int32_t*)c.dev, ldc, s);
            if (st == DNNOPT_OK) st = sync_stream(s);
            if (st == DNNOPT_OK) st = stage_out(c, s);
            if (st == DNNOPT_OK) drain.release();
        }
    }
    record(st, "gemm_int8_int8int8int32");
}

void gemm_set_num_threads(int n) { set_threads(n); }
int gemm_get_num_threads() { return get_threads(); }

}  // namespace dnnopt

extern "C" int dnnopt_hip_last_status(void) { return dnnopt_api::last_status(); }
