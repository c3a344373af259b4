/** @file mi355x_allocator.hpp
 *  @brief The device-memory cache behind MI355XBackend::allocate(): freed blocks are kept per size
 *         class and handed to later requests of that class instead of going back to hipMalloc.
 *
 *  Same contract as Pulsatrix's CachingAllocator (include/pulsatrix/caching_allocator.hpp,
 *  src/hip_backend.hip:36-54, tests/caching_allocator_test.cpp:44-127):
 *    * size classes: 512-byte steps below 1 MiB, then steps of an eighth of the power of two at or
 *      below the size (at most 12.5% rounding waste);
 *    * allocate(0) returns nullptr, free(nullptr) is a no-op;
 *    * a request that would take in-use + cached bytes over the budget releases the cache first;
 *      a request that still does not fit throws std::bad_alloc and changes nothing;
 *    * a failed device allocation (the raw allocator throws std::bad_alloc or returns nullptr)
 *      releases the cache and retries once, then throws std::bad_alloc;
 *    * memory goes back to the device only after the synchronize callback has run (empty_cache(),
 *      the destructor, the release before a retry, a free whose block cannot be cached), since
 *      queued kernels may still read a block;
 *    * when host memory for the bookkeeping runs out, allocate() throws std::bad_alloc with the block
 *      returned (to the cache, or to the device if it was fresh) and free() hands the block to the
 *      device after the synchronize.
 *  Device-independent: the raw operations are injected, so the logic runs in CPU-only tests.
 *  Safe on one in-order stream: a block freed by the host was last used by work already queued on
 *  that stream, and its next user's work is queued after it.
 */
#pragma once

#include <cstddef>
#include <functional>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace pulsatrix {
namespace mi355x {

class CachingAllocator {
public:
    using RawAlloc = std::function<void*(size_t bytes)>;  ///< nullptr or std::bad_alloc on failure
    using RawFree = std::function<void(void* ptr)>;
    using Synchronize = std::function<void()>;  ///< waits for queued device work

    struct Stats {
        size_t in_use_bytes = 0;
        size_t cached_bytes = 0;
        size_t peak_in_use_bytes = 0;
        size_t raw_allocs = 0;
        size_t raw_frees = 0;
        size_t cache_hits = 0;
    };

    /** @param budget_bytes most memory held, in use plus cached; 0 = no limit but the device's. */
    CachingAllocator(RawAlloc raw_alloc, RawFree raw_free, Synchronize synchronize, size_t budget_bytes = 0);
    /** @brief Synchronizes, then returns every block, cached or still in use, to the device. */
    ~CachingAllocator();
    CachingAllocator(const CachingAllocator&) = delete;
    CachingAllocator& operator=(const CachingAllocator&) = delete;

    [[nodiscard]] void* allocate(size_t bytes);
    void free(void* ptr) noexcept;
    /** @brief Synchronizes, then returns every cached (not in-use) block to the device. */
    void empty_cache();
    /** @brief 0 = unlimited; applies from the next allocation. */
    void set_budget(size_t budget_bytes);
    [[nodiscard]] size_t budget() const;
    [[nodiscard]] Stats stats() const;
    [[nodiscard]] static size_t round_size(size_t bytes);

private:
    void drop_cache_locked(bool sync);  // (synchronize,) raw_free every cached block; mutex held
    void* raw_try(size_t size);  // nullptr when the device refuses
    bool mark_live_locked(void* p, size_t size) noexcept;  // false when the bookkeeping cannot grow

    RawAlloc raw_alloc_;
    RawFree raw_free_;
    Synchronize synchronize_;
    size_t budget_;
    mutable std::mutex mu_;
    std::unordered_map<size_t, std::vector<void*>> cached_;  // size class -> free blocks
    std::unordered_map<void*, size_t> live_;                 // block in use -> size class
    Stats stats_;
};

}  // namespace mi355x
}  // namespace pulsatrix
