// hostcopy.cpp -- a multi-threaded host memcpy for large downloads: the
// engine stages device data in pinned host memory and moves it on to the
// caller's (pageable) buffer with this, block-parallel under OpenMP, while
// the next chunk's DMA is in flight.
#include <omp.h>

#include <algorithm>
#include <cstddef>
#include <cstring>

void ms_parallel_memcpy(void *dst, const void *src, size_t bytes) {
    constexpr size_t kBlock = size_t(1) << 20;
    const long long nblocks = (long long)((bytes + kBlock - 1) / kBlock);
    if (nblocks <= 1) {
        std::memcpy(dst, src, bytes);
        return;
    }
    const int threads = (int)std::min<long long>(nblocks, std::min(8, omp_get_max_threads()));
#pragma omp parallel for num_threads(threads) schedule(static)
    for (long long b = 0; b < nblocks; ++b) {
        const size_t off = (size_t)b * kBlock, len = std::min(kBlock, bytes - off);
        std::memcpy(static_cast<char *>(dst) + off, static_cast<const char *>(src) + off, len);
    }
}
