// runtime.cpp -- device queries, status mapping and the per-stream workspace.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

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

// Locks of StreamLock, per (device, stream).  Never destroyed: calls may
// still run while the process's static objects are being torn down.
std::mutex& lock_table_mu() {
    static std::mutex* m = new std::mutex;
    return *m;
}
std::map<std::pair<int, hipStream_t>, std::recursive_mutex*>& lock_table() {
    static auto* t = new std::map<std::pair<int, hipStream_t>, std::recursive_mutex*>;
    return *t;
}

// Streams of finished threads, per device, for reuse by new threads.
struct StreamPool {
    std::mutex mu;
    std::map<int, std::vector<hipStream_t>> idle;
};
StreamPool& stream_pool() {
    static StreamPool* p = new StreamPool;
    return *p;
}

// A thread's streams; returned to the pool (no HIP call) when it ends.
struct ThreadStreams {
    std::map<int, hipStream_t> by_dev;
    ~ThreadStreams() {
        StreamPool& p = stream_pool();
        std::lock_guard<std::mutex> g(p.mu);
        for (auto& kv : by_dev) p.idle[kv.first].push_back(kv.second);
    }
};
thread_local ThreadStreams t_streams;

}  // namespace

StreamLock::StreamLock(hipStream_t s) : mu_(nullptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        dev = -1;
    }
    std::recursive_mutex* m;
    {
        std::lock_guard<std::mutex> g(lock_table_mu());
        std::recursive_mutex*& slot = lock_table()[{dev, s}];
        if (!slot) slot = new std::recursive_mutex;
        m = slot;
    }
    m->lock();
    mu_ = m;
}

StreamLock::~StreamLock() { static_cast<std::recursive_mutex*>(mu_)->unlock(); }

hipStream_t thread_stream(int* status) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *status = to_status(e);
        return nullptr;
    }
    auto it = t_streams.by_dev.find(dev);
    if (it != t_streams.by_dev.end()) return it->second;
    hipStream_t s = nullptr;
    {
        StreamPool& p = stream_pool();
        std::lock_guard<std::mutex> g(p.mu);
        std::vector<hipStream_t>& v = p.idle[dev];
        if (!v.empty()) {
            s = v.back();
            v.pop_back();
        }
    }
    if (!s) {
        e = hipStreamCreate(&s);  // default flags and priority
        if (e != hipSuccess) {
            (void)hipGetLastError();
            *status = to_status(e);
            return nullptr;
        }
    }
    t_streams.by_dev[dev] = s;
    return s;
}

int get_workspace(hipStream_t s, size_t part_bytes, void** part, unsigned** tickets, int slot) {
    if (visible_devices() == 0) return DNNOPT_ERR_NO_DEVICE;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return to_status(e);
    // g_ws_mu guards only the map (entries are never erased, so a reference
    // stays valid).  The entry of (device, stream) is used only under that
    // stream's StreamLock, which the caller holds, so it is grown outside
    // g_ws_mu: one stream's synchronize never stalls another's lookup.
    Scratch* w = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_ws_mu);
        w = &g_ws[{{dev, slot}, s}];
    }
    if (w->ptr == nullptr || w->cap < part_bytes) {
        size_t want = part_bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : part_bytes;
        if (w->ptr) {
            // Launches already queued on this stream may still use the old buffer.
            e = hipStreamSynchronize(s);
            if (e != hipSuccess) return to_status(e);
            (void)hipFree(w->ptr);
            w->ptr = nullptr;
            w->cap = 0;
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
        w->ptr = p;
        w->cap = want;
    }
    *tickets = static_cast<unsigned*>(w->ptr);
    *part = static_cast<char*>(w->ptr) + kTicketBytes;
    return DNNOPT_OK;
}

}  // namespace dnnopt_hip
