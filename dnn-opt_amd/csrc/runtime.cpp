// runtime.cpp -- device queries, status mapping and the per-stream workspace.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <utility>

#include "host.h"

namespace dnnopt_hip {

int visible_devices() {
    static int count = [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void)hipGetLastError();
            n = 0;
        }
        return n;
    }();
    return count;
}

int num_cus() {
    if (visible_devices() == 0) return 256;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    static std::mutex mu;
    static std::map<int, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev] = cus;
    return cus;
}

int to_status(hipError_t e) {
    if (e == hipSuccess) return DNNOPT_OK;
    if (e == hipErrorOutOfMemory) return DNNOPT_ERR_OUT_OF_MEMORY;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) return DNNOPT_ERR_NO_DEVICE;
    return DNNOPT_ERR_HIP;
}

namespace {

struct Scratch {
    void* ptr = nullptr;
    size_t cap = 0;  // bytes after the ticket block
};

std::mutex g_ws_mu;
std::map<std::pair<std::pair<int, int>, hipStream_t>, Scratch> g_ws;

constexpr size_t kTicketBytes = (size_t)kMaxTickets * sizeof(unsigned);

}  // namespace

int get_workspace(hipStream_t s, size_t part_bytes, void** part, unsigned** tickets, int slot) {
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return to_status(e);
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Scratch& w = g_ws[{{dev, slot}, s}];
    if (w.ptr == nullptr || w.cap < part_bytes) {
        size_t want = part_bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : part_bytes;
        if (w.ptr) {
            // Launches already queued on this stream may still use the old buffer.
            e = hipStreamSynchronize(s);
            if (e != hipSuccess) return to_status(e);
            (void)hipFree(w.ptr);
            w.ptr = nullptr;
            w.cap = 0;
        }
        void* p = nullptr;
        e = hipMalloc(&p, kTicketBytes + want);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return DNNOPT_ERR_OUT_OF_MEMORY;
        }
        // Tickets start at zero; every kernel that takes one leaves it at zero.
        e = hipMemset(p, 0, kTicketBytes);
        if (e != hipSuccess) {
            (void)hipFree(p);
            return to_status(e);
        }
        w.ptr = p;
        w.cap = want;
    }
    *tickets = static_cast<unsigned*>(w.ptr);
    *part = static_cast<char*>(w.ptr) + kTicketBytes;
    return DNNOPT_OK;
}

}  // namespace dnnopt_hip
