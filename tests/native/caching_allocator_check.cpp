// CPU contract checks of MI355XBackend's device-memory cache (pulsatrix::mi355x::CachingAllocator),
// driven through a fake device made of host memory: the cases of the reference's
// tests/caching_allocator_test.cpp:44-127 plus the budget read from PULSATRIX_HIP_MEMORY_BUDGET_MB.
// Built and run by tests/test_allocator_cpu.py; prints one line per failed check and exits 1.
#include <cstdio>
#include <cstdlib>
#include <new>

#include "pulsatrix/mi355x_allocator.hpp"

using pulsatrix::mi355x::CachingAllocator;

// The next operator new throws std::bad_alloc while g_fail_next_new is set (and clears it): host
// memory for the allocator's own bookkeeping running out at that point.
bool g_fail_next_new = false;

void* operator new(size_t n) {
    if (g_fail_next_new) {
        g_fail_next_new = false;
        throw std::bad_alloc();
    }
    if (void* p = std::malloc(n == 0 ? 1 : n)) return p;
    throw std::bad_alloc();
}
void* operator new[](size_t n) { return operator new(n); }
void operator delete(void* p) noexcept { std::free(p); }
void operator delete[](void* p) noexcept { std::free(p); }
void operator delete(void* p, size_t) noexcept { std::free(p); }
void operator delete[](void* p, size_t) noexcept { std::free(p); }

namespace {

int g_failed = 0;
#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            std::printf("FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);        \
            ++g_failed;                                                          \
        }                                                                        \
    } while (0)

template <class F>
bool throws_bad_alloc(F f) {
    try {
        f();
    } catch (const std::bad_alloc&) {
        return true;
    }
    return false;
}

// A pretend HBM for the allocator's injected callbacks: up to 64 blocks of host memory in fixed
// slots (so the callbacks themselves never call operator new), a byte limit (0 = none) past which
// it refuses the way hipMalloc does when HBM is full (by throwing, or by returning nullptr when
// `null_on_full`), and counters of raw allocations, frees and synchronizations.
struct HostHbm {
    struct Slot {
        void* p = nullptr;
        size_t bytes = 0;
    };
    Slot slot[64];
    size_t limit = 0, held = 0;
    int mallocs = 0, frees = 0, syncs = 0;
    bool null_on_full = false;

    [[nodiscard]] bool holds(const void* p) const {
        for (const Slot& s : slot)
            if (s.p == p && p != nullptr) return true;
        return false;
    }
    [[nodiscard]] int blocks() const {
        int k = 0;
        for (const Slot& s : slot) k += s.p != nullptr;
        return k;
    }
    void* take(size_t bytes) {
        if (limit != 0 && held + bytes > limit) {
            if (null_on_full) return nullptr;
            throw std::bad_alloc();
        }
        for (Slot& s : slot) {
            if (s.p != nullptr) continue;
            s.p = std::malloc(bytes);
            s.bytes = bytes;
            held += bytes;
            ++mallocs;
            return s.p;
        }
        throw std::bad_alloc();  // out of slots
    }
    void give(void* p) {
        for (Slot& s : slot) {
            if (s.p != p) continue;
            std::free(s.p);
            held -= s.bytes;
            s = Slot{};
            ++frees;
            return;
        }
    }
    CachingAllocator make(size_t budget = 0) {
        return CachingAllocator([this](size_t b) { return take(b); }, [this](void* p) { give(p); },
                                [this] { ++syncs; }, budget);
    }
};

void size_classes() {
    CHECK(CachingAllocator::round_size(1) == 512u);
    CHECK(CachingAllocator::round_size(512) == 512u);
    CHECK(CachingAllocator::round_size(513) == 1024u);
    CHECK(CachingAllocator::round_size((1u << 20) - 1) == 1u << 20);
    CHECK(CachingAllocator::round_size(1u << 20) == 1u << 20);
    CHECK(CachingAllocator::round_size((1u << 20) + 1) == (1u << 20) + (1u << 17));
    CHECK(CachingAllocator::round_size(3u << 20) == 3u << 20);
    CHECK(CachingAllocator::round_size((3u << 20) + 1) == (3u << 20) + (1u << 18));
    // waste stays under 12.5% everywhere from 1 MiB up
    for (size_t b = (1u << 20) + 7; b < (size_t{1} << 34); b = b * 3 / 2 + 13) {
        const size_t r = CachingAllocator::round_size(b);
        CHECK(r >= b && r - b < b / 8 + 1);
    }
}

void freed_block_is_reused_for_its_class() {
    HostHbm dev;
    CachingAllocator a = dev.make();
    void* p = a.allocate(100);
    a.free(p);
    CHECK(a.allocate(400) == p);  // 100 and 400 bytes share the 512-byte class
    CHECK(dev.mallocs == 1);
    CHECK(a.stats().cache_hits == 1u);
    void* q = a.allocate(600);  // another class: a new block
    CHECK(q != p);
    CHECK(dev.mallocs == 2);
}

void tracks_in_use_cached_and_peak() {
    HostHbm dev;
    CachingAllocator a = dev.make();
    void* p = a.allocate(1000);
    void* q = a.allocate(2000);
    CHECK(a.stats().in_use_bytes == 3072u);
    a.free(p);
    CHECK(a.stats().in_use_bytes == 2048u);
    CHECK(a.stats().cached_bytes == 1024u);
    CHECK(a.stats().peak_in_use_bytes == 3072u);
    a.free(q);
    CHECK(a.stats().cached_bytes == 3072u);
    CHECK(a.stats().raw_allocs == 2u);
}

void empty_cache_synchronizes_then_releases_only_cached() {
    HostHbm dev;
    CachingAllocator a = dev.make();
    void* kept = a.allocate(512);
    a.free(a.allocate(1024));
    const int syncs = dev.syncs;
    a.empty_cache();
    CHECK(dev.syncs > syncs);  // never hand back memory a queued kernel may still read
    CHECK(dev.frees == 1);
    CHECK(a.stats().cached_bytes == 0u);
    CHECK(dev.holds(kept));
}

void over_budget_releases_the_cache_first() {
    HostHbm dev;
    CachingAllocator a = dev.make(4096);
    a.free(a.allocate(2048));
    const int syncs = dev.syncs;
    void* big = a.allocate(3000);  // class 3072: 2048 cached + 3072 > 4096, so the cache goes first
    CHECK(big != nullptr);
    CHECK(dev.frees == 1);
    CHECK(dev.syncs > syncs);
    CHECK(a.stats().cached_bytes == 0u);
    CHECK(a.stats().in_use_bytes == 3072u);
}

void request_beyond_budget_throws_and_changes_nothing() {
    HostHbm dev;
    CachingAllocator a = dev.make(4096);
    void* p = a.allocate(3000);
    CHECK(throws_bad_alloc([&] { (void)a.allocate(2000); }));
    CHECK(a.stats().in_use_bytes == 3072u);
    CHECK(dev.mallocs == 1);
    a.free(p);
    a.set_budget(0);  // unlimited from the next allocation
    void* q = a.allocate(8000);
    CHECK(q != nullptr);
    a.free(q);
}

void device_failure_releases_the_cache_and_retries() {
    for (int null_mode = 0; null_mode < 2; ++null_mode) {
        HostHbm dev;
        dev.limit = 4096;
        dev.null_on_full = null_mode == 1;
        CachingAllocator a = dev.make();  // no budget: only the device refuses
        a.free(a.allocate(2048));
        void* p = a.allocate(3000);  // fails once (2048 held + 3072 > 4096), succeeds after the release
        CHECK(p != nullptr);
        CHECK(dev.frees == 1);
        dev.limit = 1;
        CHECK(throws_bad_alloc([&] { (void)a.allocate(8000); }));  // nothing left to release
        CHECK(a.stats().in_use_bytes == 3072u);
        a.free(p);
    }
}

void zero_bytes_and_null() {
    HostHbm dev;
    CachingAllocator a = dev.make();
    CHECK(a.allocate(0) == nullptr);
    a.free(nullptr);
    int local = 0;
    a.free(&local);  // not a block of this cache: ignored
    CHECK(dev.mallocs == 0);
    CHECK(a.stats().cached_bytes == 0u);
}

void destruction_releases_everything() {
    HostHbm dev;
    {
        CachingAllocator a = dev.make();
        (void)a.allocate(100);  // still in use: released too, the device goes away
        a.free(a.allocate(5000));
    }
    CHECK(dev.blocks() == 0);
    CHECK(dev.mallocs == dev.frees);
    CHECK(dev.syncs >= 1);
}

void budget_from_environment() {
    // MI355XBackend reads PULSATRIX_HIP_MEMORY_BUDGET_MB as megabytes (hip_backend.hip:38-41).
    const char* mb = std::getenv("PULSATRIX_HIP_MEMORY_BUDGET_MB");
    if (mb == nullptr) return;
    const size_t budget = static_cast<size_t>(std::strtoull(mb, nullptr, 10)) << 20;
    HostHbm dev;
    CachingAllocator a = dev.make(budget);
    void* p = a.allocate(budget - (size_t{1} << 20));
    CHECK(p != nullptr);
    CHECK(throws_bad_alloc([&] { (void)a.allocate(size_t{2} << 20); }));
    a.free(p);
}

void bookkeeping_failure_returns_the_block() {
    HostHbm dev;
    CachingAllocator a = dev.make();
    // a fresh block whose entry cannot be recorded goes straight back to the device
    g_fail_next_new = true;
    CHECK(throws_bad_alloc([&] { (void)a.allocate(700); }));
    g_fail_next_new = false;
    CHECK(dev.blocks() == 0 && dev.mallocs == 1 && dev.frees == 1);
    CHECK(a.stats().in_use_bytes == 0u);
    // a cached block whose entry cannot be recorded stays cached
    void* p = a.allocate(700);
    a.free(p);
    const size_t cached = a.stats().cached_bytes;
    g_fail_next_new = true;
    CHECK(throws_bad_alloc([&] { (void)a.allocate(700); }));
    g_fail_next_new = false;
    CHECK(a.stats().cached_bytes == cached && a.stats().in_use_bytes == 0u);
    CHECK(a.allocate(700) == p);  // and is handed out by the next request of its class
}

void free_without_cache_room_synchronizes_before_releasing() {
    HostHbm dev;
    CachingAllocator a = dev.make();
    void* p = a.allocate(3000);  // a size class with no cache entry yet: caching it needs a new node
    const int syncs = dev.syncs;
    g_fail_next_new = true;
    a.free(p);
    g_fail_next_new = false;
    CHECK(!dev.holds(p) && dev.frees == 1);
    CHECK(dev.syncs > syncs);  // queued work may still read it
    CHECK(a.stats().in_use_bytes == 0u && a.stats().cached_bytes == 0u);
}

}  // namespace

int main() {
    size_classes();
    freed_block_is_reused_for_its_class();
    tracks_in_use_cached_and_peak();
    empty_cache_synchronizes_then_releases_only_cached();
    over_budget_releases_the_cache_first();
    request_beyond_budget_throws_and_changes_nothing();
    device_failure_releases_the_cache_and_retries();
    zero_bytes_and_null();
    destruction_releases_everything();
    budget_from_environment();
    bookkeeping_failure_returns_the_block();
    free_without_cache_room_synchronizes_before_releasing();
    std::printf("%s\n", g_failed == 0 ? "all allocator checks passed" : "allocator checks failed");
    return g_failed == 0 ? 0 : 1;
}
