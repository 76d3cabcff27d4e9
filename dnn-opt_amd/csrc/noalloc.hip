// noalloc.hip -- dnnopt_hip_sgemm_noalloc: the fp32 GEMM entry point for
// callers that cannot allocate device memory (graph capture, serving loops).
//
// Split-k launches need device scratch (partial sums and ticket counters).
// dnnopt_hip_sgemm takes it from a per-stream workspace that grows with
// hipMalloc; this entry point instead uses `scratch`, a fixed array of
// DNNOPT_NOALLOC_SCRATCH_BYTES in the library's code object.  Each GPU that
// loads the library holds its own copy for the life of the process, at its
// own address: the host-side name `scratch` is only a stand-in, so the
// device address is looked up once per device with hipGetSymbolAddress and
// only that address is ever passed to kernels.
//
// The ticket counters must be zero before a launch takes one, and every
// kernel that takes a ticket leaves it at zero again.  The array is zero when
// the code object is loaded; the first call on a device also clears the
// ticket block with a fill kernel (not hipMemsetAsync, which must not be
// recorded into a captured graph).
#include <hip/hip_runtime.h>

#include <mutex>

#include "dnnopt_hip.h"
#include "host.h"

namespace {

constexpr size_t kScratchBytes = DNNOPT_NOALLOC_SCRATCH_BYTES;
constexpr int kTicketWords = (int)(dnnopt_hip::kTicketBytes / 4);
static_assert(kScratchBytes > (size_t)kTicketWords * 4, "scratch holds the ticket block and partials");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ __launch_bounds__(256) void dnnopt_zero_tickets(unsigned* p, int n) {
    for (int i = (int)(blockIdx.x * blockDim.x + threadIdx.x); i < n; i += (int)(gridDim.x * blockDim.x)) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];  // device address of `scratch` per device (null until set up)

// Device address of this device's scratch array; the first call on a device
// looks it up and enqueues the clearing of its tickets on `s`.
int scratch_address(hipStream_t s, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return dnnopt_hip::to_status(e);
    }
    if (dev < 0 || dev >= kMaxDevices) return DNNOPT_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            return e != hipSuccess ? dnnopt_hip::to_status(e) : DNNOPT_ERR_HIP;
        }
        hipLaunchKernelGGL(dnnopt_zero_tickets, dim3((kTicketWords + 255) / 256), dim3(256), 0, s,
                           static_cast<unsigned*>(p), kTicketWords);
        e = hipGetLastError();
        if (e != hipSuccess) return dnnopt_hip::to_status(e);
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return DNNOPT_OK;
}

}  // namespace

extern "C" int dnnopt_hip_sgemm_noalloc(int transA, int transB, int M, int N, int K, float alpha, const float* A,
                                        int lda, const float* B, int ldb, float beta, float* C, int ldc,
                                        void* stream) {
    if ((transA != 0 && transA != 1) || (transB != 0 && transB != 1)) return DNNOPT_ERR_INVALID_ARG;
    if (M <= 0 || N <= 0 || K <= 0) return DNNOPT_OK;
    if (!A || !B || !C) return DNNOPT_ERR_INVALID_ARG;
    if (lda < (transA ? M : K) || ldb < (transB ? K : N) || ldc < N) return DNNOPT_ERR_INVALID_ARG;
    if (dnnopt_hip::visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    void* base = nullptr;
    int st = scratch_address(s, &base);
    if (st != DNNOPT_OK) return st;
    const dnnopt_hip::ExtScratch ext{base, kScratchBytes};
    return dnnopt_hip::sgemm_bias(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, nullptr, s, &ext);
}
