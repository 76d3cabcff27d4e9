// aligned_alloc.cpp -- host allocation helpers of include/dnnopt/aligned_alloc.h.
#include "dnnopt/aligned_alloc.h"

#include <stdint.h>
#include <stdlib.h>
#include <sys/mman.h>

namespace dnnopt {

void* aligned_malloc(size_t size, size_t alignment) {
    if (size == 0) return nullptr;  // as the reference (src/utils/aligned_alloc.cpp:16)
    if (alignment < sizeof(void*)) alignment = sizeof(void*);
    void* p = nullptr;
    if (posix_memalign(&p, alignment, size) != 0) return nullptr;
    return p;
}

void aligned_free(void* ptr) { free(ptr); }

void* aligned_malloc_huge(size_t size, size_t alignment) {
    if (size < kHugePageThreshold) return aligned_malloc(size, alignment);
    const size_t rounded = (size + kHugePageThreshold - 1) & ~(kHugePageThreshold - 1);
    void* p = aligned_malloc(rounded, kHugePageThreshold);
    if (p) (void)madvise(p, rounded, MADV_HUGEPAGE);
    return p;
}

void aligned_free_huge(void* ptr, size_t /*size*/) { free(ptr); }

}  // namespace dnnopt
