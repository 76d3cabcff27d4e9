#pragma once
/// @file aligned_alloc.h
/// Aligned host allocation helpers.  Kept because the oneDNN integration
/// wrapper allocates its temporaries with dnnopt::aligned_array
/// (reference: include/dnnopt/aligned_alloc.h:19-67,
/// integration/onednn/0001-dnnopt-integration.patch:164, 224, 251).

#include <cstddef>
#include <cstdlib>
#include <memory>

namespace dnnopt {

constexpr size_t kCacheLineSize = 64;
constexpr size_t kHugePageThreshold = 2 * 1024 * 1024;

/// Returns nullptr on failure; free with aligned_free().
void* aligned_malloc(size_t size, size_t alignment = kCacheLineSize);

/// Large buffers are rounded to 2 MiB and advised for transparent huge
/// pages; free with aligned_free_huge().
void* aligned_malloc_huge(size_t size, size_t alignment = kCacheLineSize);

void aligned_free(void* ptr);
void aligned_free_huge(void* ptr, size_t size);

template <typename T>
struct AlignedDeleter {
    void operator()(T* ptr) const { aligned_free(ptr); }
};

template <typename T>
using AlignedPtr = std::unique_ptr<T[], AlignedDeleter<T>>;

template <typename T>
AlignedPtr<T> aligned_array(size_t count, size_t alignment = kCacheLineSize) {
    return AlignedPtr<T>(static_cast<T*>(aligned_malloc(count * sizeof(T), alignment)));
}

template <typename T>
struct HugePageDeleter {
    size_t size_bytes = 0;
    void operator()(T* ptr) const { aligned_free_huge(ptr, size_bytes); }
};

template <typename T>
using HugePagePtr = std::unique_ptr<T[], HugePageDeleter<T>>;

template <typename T>
HugePagePtr<T> aligned_array_huge(size_t count, size_t alignment = kCacheLineSize) {
    const size_t bytes = count * sizeof(T);
    HugePageDeleter<T> d;
    d.size_bytes = bytes;
    return HugePagePtr<T>(static_cast<T*>(aligned_malloc_huge(bytes, alignment)), d);
}

}  // namespace dnnopt
