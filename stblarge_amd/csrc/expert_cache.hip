// HBM expert cache with LRU replacement, refilled from a pinned host pool on a side stream.
//
// Reference: ExpertCache and its use in stbl/model.cu:99-106, :347-422, :497-507. The reference
// reads misses from SSD with pread into pinned stages and copies them on reader streams, waiting on
// the host; here the experts live in a pinned host pool (the next tier down), every miss is one
// hipMemcpyAsync on the cache's own copy stream, and the caller's compute stream waits on an event,
// so no host thread blocks on a copy. Bookkeeping follows the reference:
//   * key = layer << 32 | expert; a hit moves the entry to the most-recently-used end;
//   * before any miss of a lookup is served, every cached expert of that lookup is touched, so a
//     miss never evicts an expert the same lookup needs (stbl/model.cu:497-502);
//   * a miss takes a never-used slot (lowest first) or evicts the least recently used entry
//     (stbl/model.cu:347-371); with every slot held by the current lookup it fails;
//   * a failed refill leaves the slot unmapped, so the next lookup misses it again.
// A slot may still be read by kernels queued before it is evicted. stbl_amd_cache_mark_used records
// an event on the compute stream after those kernels; a later refill of the slot waits for it on the
// copy stream. Events come from a ring, so a recycled event only makes a refill wait longer.
// One host thread drives a cache; lookups of different caches may run on different threads.
#include <list>
#include <unordered_map>
#include <vector>

#include "abi_util.hpp"

namespace stbl {

struct ExpertCache {
    int device = 0;
    int slots = 0;
    uint64_t slot_bytes = 0;
    uint8_t *mem = nullptr;
    const uint8_t *host = nullptr;
    uint64_t host_stride = 0;
    int n_experts = 0, n_layers = 0;
    hipStream_t copy = nullptr;
    hipEvent_t ready = nullptr;
    static constexpr int kRing = 64;
    hipEvent_t ring[kRing] = {};
    int ring_next = 0;
    std::vector<int> slot_use;  // ring index of the last use of each slot, -1 if none
    std::unordered_map<uint64_t, std::pair<int, std::list<uint64_t>::iterator>> where;
    std::list<uint64_t> lru;  // front = most recently used
    std::vector<int> free_slots;
    int next_slot = 0;
    std::vector<int> touched;  // slots of the last lookup
    uint64_t hits = 0, misses = 0, refill_bytes = 0, lookups = 0;
    int fail_in = -1;  // test hook: the refill after this many more fails (host side, nothing copied)
};

static int take_slot(ExpertCache &c) {
    if (!c.free_slots.empty()) {
        const int s = c.free_slots.back();
        c.free_slots.pop_back();
        return s;
    }
    if (c.next_slot < c.slots) return c.next_slot++;
    return -1;  // caller evicts
}

// Teardown is best effort: a failure here cannot be reported to anyone who could act on it.
static void destroy(ExpertCache *c) {
    if (!c) return;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(c->device);
    if (c->copy) (void)hipStreamSynchronize(c->copy);
    for (auto &e : c->ring)
        if (e) (void)hipEventDestroy(e);
    if (c->ready) (void)hipEventDestroy(c->ready);
    if (c->copy) (void)hipStreamDestroy(c->copy);
    if (c->mem) (void)hipFree(c->mem);
    (void)hipSetDevice(prev);
    delete c;
}

}  // namespace stbl

using namespace stbl;

extern "C" {

// Creates a cache of `slots` slots of slot_bytes each on the current device (allocates slots *
// slot_bytes of device memory, a copy stream and events). host_pool holds n_layers * n_experts
// experts, host_stride bytes apart, in pinned host memory that outlives the cache. NULL on failure.
void *stbl_amd_cache_create(int slots, uint64_t slot_bytes, const void *host_pool, uint64_t host_stride, int n_experts,
                            int n_layers) {
    if (slots < 1 || slot_bytes == 0 || !host_pool || host_stride < slot_bytes || n_experts < 1 || n_layers < 1) {
        abi_fail(hipErrorInvalidValue, "cache_create: bad arguments");
        return nullptr;
    }
    ExpertCache *c = new ExpertCache();
    c->slots = slots;
    c->slot_bytes = slot_bytes;
    c->host = (const uint8_t *)host_pool;
    c->host_stride = host_stride;
    c->n_experts = n_experts;
    c->n_layers = n_layers;
    c->slot_use.assign(slots, -1);
    hipError_t e = hipGetDevice(&c->device);
    if (e == hipSuccess) e = hipMalloc(&c->mem, (size_t)slots * slot_bytes);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->ready, hipEventDisableTiming);
    for (int i = 0; i < ExpertCache::kRing && e == hipSuccess; i++) e = hipEventCreateWithFlags(&c->ring[i], hipEventDisableTiming);
    if (e != hipSuccess) {
        abi_status(e, "cache_create");
        destroy(c);
        return nullptr;
    }
    return c;
}

void stbl_amd_cache_destroy(void *cache) { destroy((ExpertCache *)cache); }

// Looks up n expert ids (HOST array) of one layer, in order. slot_ptrs (HOST, n entries) receives
// each expert's slot; hit (HOST, optional) 1/0 per id. Misses are copied from the host pool on the
// copy stream and `compute` is made to wait for them. Returns the number of misses, or a negative
// hipError_t (then nothing of this lookup is mapped that was not before, apart from completed
// refills, and the caller must not use slot_ptrs).
int stbl_amd_cache_lookup(void *cache, const int *ids, int n, int layer, void **slot_ptrs, int *hit,
                          hipStream_t compute) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || !ids || !slot_ptrs || n < 0 || layer < 0 || layer >= c->n_layers)
        return abi_fail(hipErrorInvalidValue, "cache_lookup: bad arguments");
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= c->n_experts) return abi_fail(hipErrorInvalidValue, "cache_lookup: expert id %d out of range", ids[i]);
    c->lookups++;
    auto key = [&](int e) { return (uint64_t)layer << 32 | (uint32_t)e; };
    // 1. touch every cached expert of this lookup first
    for (int i = 0; i < n; i++) {
        auto it = c->where.find(key(ids[i]));
        if (it != c->where.end()) c->lru.splice(c->lru.begin(), c->lru, it->second.second);
    }
    c->touched.clear();
    int nmiss = 0;
    for (int i = 0; i < n; i++) {
        const uint64_t k = key(ids[i]);
        auto it = c->where.find(k);
        if (it != c->where.end()) {
            c->lru.splice(c->lru.begin(), c->lru, it->second.second);
            slot_ptrs[i] = c->mem + (uint64_t)it->second.first * c->slot_bytes;
            if (hit) hit[i] = 1;
            c->hits++;
            c->touched.push_back(it->second.first);
            continue;
        }
        // 2. miss: a free slot, or the least recently used entry not needed by this lookup
        int s = take_slot(*c);
        if (s < 0) {
            const uint64_t victim = c->lru.back();
            bool needed = false;
            for (int j = 0; j < n; j++) needed |= key(ids[j]) == victim;
            if (needed) return abi_fail(hipErrorOutOfMemory, "cache_lookup: every slot is held by this lookup (%d slots)", c->slots);
            s = c->where[victim].first;
            c->where.erase(victim);
            c->lru.pop_back();
        }
        uint8_t *dst = c->mem + (uint64_t)s * c->slot_bytes;
        const uint8_t *src = c->host + ((uint64_t)layer * c->n_experts + ids[i]) * c->host_stride;
        hipError_t e = hipSuccess;
        if (c->slot_use[s] >= 0) e = hipStreamWaitEvent(c->copy, c->ring[c->slot_use[s]], 0);
        if (e == hipSuccess) {
            if (c->fail_in == 0) e = hipErrorUnknown;
            else e = hipMemcpyAsync(dst, src, c->slot_bytes, hipMemcpyHostToDevice, c->copy);
            if (c->fail_in >= 0) c->fail_in--;
        }
        if (e != hipSuccess) {
            c->free_slots.push_back(s);  // slot stays unmapped: the next lookup misses again
            return abi_fail(e, "cache_lookup: refill of expert %d failed: %s", ids[i], hipGetErrorString(e));
        }
        c->lru.push_front(k);
        c->where[k] = {s, c->lru.begin()};
        slot_ptrs[i] = dst;
        if (hit) hit[i] = 0;
        c->misses++;
        c->refill_bytes += c->slot_bytes;
        c->touched.push_back(s);
        nmiss++;
    }
    if (nmiss > 0) {
        hipError_t e = hipEventRecord(c->ready, c->copy);
        if (e == hipSuccess) e = hipStreamWaitEvent(compute, c->ready, 0);
        if (e != hipSuccess) return abi_status(e, "cache_lookup: ordering the compute stream after the refills");
    }
    return nmiss;
}

// Marks every slot of the last lookup as read by the work queued so far on `compute`: a later
// refill of one of those slots waits until that work is done.
int stbl_amd_cache_mark_used(void *cache, hipStream_t compute) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c) return abi_fail(hipErrorInvalidValue, "cache_mark_used: null cache");
    if (c->touched.empty()) return 0;
    const int r = c->ring_next;
    c->ring_next = (r + 1) % ExpertCache::kRing;
    const hipError_t e = hipEventRecord(c->ring[r], compute);
    if (e != hipSuccess) return abi_status(e, "cache_mark_used");
    for (int s : c->touched) c->slot_use[s] = r;
    return 0;
}

// out[0..5] = hits, misses, refill bytes, lookups, slots in use, slots.
int stbl_amd_cache_stats(void *cache, uint64_t *out) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || !out) return abi_fail(hipErrorInvalidValue, "cache_stats: bad arguments");
    out[0] = c->hits;
    out[1] = c->misses;
    out[2] = c->refill_bytes;
    out[3] = c->lookups;
    out[4] = c->where.size();
    out[5] = (uint64_t)c->slots;
    return 0;
}

// Slot of a cached expert (no LRU update), or NULL.
void *stbl_amd_cache_peek(void *cache, int layer, int expert) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c) return nullptr;
    auto it = c->where.find((uint64_t)layer << 32 | (uint32_t)expert);
    return it == c->where.end() ? nullptr : c->mem + (uint64_t)it->second.first * c->slot_bytes;
}

// Test hook: the refill after `n` more refills fails on the host (no copy is issued); -1 disables.
int stbl_amd_cache_fail_refill_after(void *cache, int n) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c) return abi_fail(hipErrorInvalidValue, "cache_fail_refill_after: null cache");
    c->fail_in = n;
    return 0;
}

}  // extern "C"
