// The size-class device-memory cache of MI355XBackend (no HIP dependency: the raw operations are
// injected). Contract: include/pulsatrix/caching_allocator.hpp and src/hip_backend.hip:36-54 of
// the reference.
#include "pulsatrix/mi355x_allocator.hpp"

#include <new>
#include <utility>

namespace pulsatrix {
namespace mi355x {

CachingAllocator::CachingAllocator(RawAlloc raw_alloc, RawFree raw_free, Synchronize synchronize,
                                   size_t budget_bytes)
    : raw_alloc_(std::move(raw_alloc)),
      raw_free_(std::move(raw_free)),
      synchronize_(std::move(synchronize)),
      budget_(budget_bytes) {}

CachingAllocator::~CachingAllocator() {
    std::lock_guard<std::mutex> lock(mu_);
    if (synchronize_) {
        try {
            synchronize_();
        } catch (...) {  // a destructor cannot throw; the blocks are released regardless
        }
    }
    for (auto& [size, blocks] : cached_)
        for (void* p : blocks) raw_free_(p);
    cached_.clear();
    for (auto& [p, size] : live_) raw_free_(p);
    live_.clear();
}

size_t CachingAllocator::round_size(size_t bytes) {
    constexpr size_t kSmall = 512, kMiB = size_t{1} << 20;
    if (bytes < kMiB) return bytes == 0 ? kSmall : (bytes + kSmall - 1) / kSmall * kSmall;
    size_t top = kMiB;  // largest power of two <= bytes
    while (top <= bytes / 2) top *= 2;
    const size_t step = top / 8;
    return (bytes + step - 1) / step * step;
}

void* CachingAllocator::raw_try(size_t size) {
    try {
        void* p = raw_alloc_(size);
        if (p != nullptr) ++stats_.raw_allocs;
        return p;
    } catch (const std::bad_alloc&) {
        return nullptr;
    }
}

void CachingAllocator::drop_cache_locked(bool sync) {
    if (stats_.cached_bytes == 0) return;
    if (sync && synchronize_) synchronize_();
    for (auto& [size, blocks] : cached_) {
        for (void* p : blocks) {
            raw_free_(p);
            ++stats_.raw_frees;
        }
    }
    cached_.clear();
    stats_.cached_bytes = 0;
}

void* CachingAllocator::allocate(size_t bytes) {
    if (bytes == 0) return nullptr;
    const size_t size = round_size(bytes);
    std::lock_guard<std::mutex> lock(mu_);
    auto hit = cached_.find(size);
    if (hit != cached_.end() && !hit->second.empty()) {
        void* p = hit->second.back();
        hit->second.pop_back();
        if (!mark_live_locked(p, size)) {
            hit->second.push_back(p);  // back where it was (the vector still has the capacity)
            throw std::bad_alloc();
        }
        stats_.cached_bytes -= size;
        ++stats_.cache_hits;
        stats_.in_use_bytes += size;
        if (stats_.in_use_bytes > stats_.peak_in_use_bytes) stats_.peak_in_use_bytes = stats_.in_use_bytes;
        return p;
    }
    if (budget_ > 0) {
        if (stats_.in_use_bytes + size > budget_) throw std::bad_alloc();  // cannot fit even with no cache
        if (stats_.in_use_bytes + stats_.cached_bytes + size > budget_) drop_cache_locked(true);
    }
    void* p = raw_try(size);
    if (p == nullptr) {  // the device said no: give the cache back and try once more
        drop_cache_locked(true);
        p = raw_try(size);
        if (p == nullptr) throw std::bad_alloc();
    }
    if (!mark_live_locked(p, size)) {  // no host memory to record it: the fresh block goes straight back
        raw_free_(p);
        ++stats_.raw_frees;
        throw std::bad_alloc();
    }
    stats_.in_use_bytes += size;
    if (stats_.in_use_bytes > stats_.peak_in_use_bytes) stats_.peak_in_use_bytes = stats_.in_use_bytes;
    return p;
}

void CachingAllocator::free(void* ptr) noexcept {
    if (ptr == nullptr) return;
    std::lock_guard<std::mutex> lock(mu_);
    auto it = live_.find(ptr);
    if (it == live_.end()) return;  // not ours: ignored, as a double free must not corrupt the cache
    const size_t size = it->second;
    live_.erase(it);
    stats_.in_use_bytes -= size;
    try {
        cached_[size].push_back(ptr);
        stats_.cached_bytes += size;
    } catch (...) {
        // No host memory to cache it: the block goes back to the device, after the synchronize
        // (queued work may still read it). If even that fails, it is leaked rather than freed early.
        try {
            if (synchronize_) synchronize_();
            raw_free_(ptr);
            ++stats_.raw_frees;
        } catch (...) {
        }
    }
}

bool CachingAllocator::mark_live_locked(void* p, size_t size) noexcept {
    try {
        live_.emplace(p, size);
        return true;
    } catch (...) {
        return false;
    }
}

void CachingAllocator::empty_cache() {
    std::lock_guard<std::mutex> lock(mu_);
    if (synchronize_) synchronize_();
    drop_cache_locked(false);
}

void CachingAllocator::set_budget(size_t budget_bytes) {
    std::lock_guard<std::mutex> lock(mu_);
    budget_ = budget_bytes;
}

size_t CachingAllocator::budget() const {
    std::lock_guard<std::mutex> lock(mu_);
    return budget_;
}

CachingAllocator::Stats CachingAllocator::stats() const {
    std::lock_guard<std::mutex> lock(mu_);
    return stats_;
}

}  // namespace mi355x
}  // namespace pulsatrix
