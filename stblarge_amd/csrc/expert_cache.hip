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
//
// File tier (stbl_amd_cache_create_gguf): the experts come from a GGUF file instead of a host pool,
// as in the reference engine (stbl/model.cu:283-308, :383-422): each expert's gate, up and down MXFP4
// blocks are read in 2 MiB pieces by reader threads (O_DIRECT where the file system allows it, at
// 4 KiB-aligned offsets) into per-reader pinned stages and copied on per-reader streams into a device
// staging area; a repack kernel on the copy stream then turns the 17-byte GGUF blocks into the slot's
// OCP layout (codes, then scales), so the routed-expert kernels read file-refilled and pool-refilled
// slots alike. The misses of one lookup are read together, up to kStageExperts at a time; the host
// thread returns once the reads have landed in pinned memory and every copy and repack is queued.
#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <list>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "abi_util.hpp"
#include "expert_layout.hpp"
#include "gemv_core.hpp"

extern "C" {
void *stbl_amd_gguf_open(const char *path);
void stbl_amd_gguf_close(void *g);
int stbl_amd_gguf_tensor(void *g, const char *name, uint32_t *type, uint64_t *dims, int *ndims, uint64_t *offset,
                         uint64_t *nbytes);
}

namespace stbl {

constexpr uint64_t kPiece = 2u << 20, kAlign = 4096;
constexpr int kStageExperts = 8, kMaxReaders = 16;

// The file tier's state: the expert tensors of each layer and the read path.
struct FileTier {
    int fd = -1, dfd = -1;      // buffered and O_DIRECT descriptors (dfd -1: buffered reads only)
    std::vector<uint64_t> part_off;  // [layer][gate, up, down]: file offset of the layer's expert tensor
    uint64_t part_bytes = 0;     // bytes of one expert's part (the three are equal: inter * dim / 32 * 17)
    int dim = 0, inter = 0;
    uint8_t *dstage = nullptr;   // device: kStageExperts experts of 3 parts
    std::vector<uint8_t *> pinned;       // per reader: two halves of kPiece bytes
    std::vector<uint8_t *> bounce;       // per reader, O_DIRECT only: kPiece + 2 kAlign page-aligned bytes
    std::vector<hipStream_t> rstream;    // per reader
    std::vector<hipEvent_t> half_done;   // per reader and half: the copy out of it
    std::vector<int> half_used;          // whether half_done was recorded
    std::vector<hipEvent_t> rdone;       // per reader: its copies of a batch
    hipEvent_t repacked = nullptr;       // the repacks of the last batch (dstage free again)
    bool repack_pending = false;
    uint64_t bytes_read = 0, read_ns = 0, experts_read = 0;
};

struct Piece {
    uint8_t *dst;  // device
    uint64_t off, bytes;
};

// Background reads of guessed experts (stbl_amd_cache_prefetch; the reference's STBL_PREFETCH jobs,
// stbl/model.cu:88-97, :310-345, :478-496). A job owns a slot, mapped as soon as it is queued, and a
// staging area; prefetch readers take its pieces from a queue, waiting while a demand read runs, and
// the reader that lands the last piece queues the repack into the slot on its own stream.
enum PfState { PF_QUEUED, PF_READING, PF_LANDED, PF_CANCELLED, PF_FAILED, PF_TAKEN };
constexpr int kPfStages = 16;  // prefetch jobs in flight at most

struct PfJob {
    int layer = 0, expert = 0, slot = 0, stage = 0;
    std::vector<Piece> ps;
    std::atomic<int> state{PF_QUEUED};
    std::atomic<int> done{0};  // pieces landed
    std::atomic<int> busy{0};  // readers inside a piece of this job
};

struct Prefetcher {
    std::vector<std::thread> threads;
    std::vector<uint8_t *> pinned, bounce;  // per reader: kPiece pinned bytes; O_DIRECT bounce buffer
    std::vector<hipStream_t> stream;        // per reader
    uint8_t *stage_mem = nullptr;           // device: kPfStages experts of 3 parts
    hipEvent_t ready[kPfStages] = {};       // per stage: the repack of its last job
    hipEvent_t slot_free[kPfStages] = {};   // per stage: recorded on the copy stream after its job's slot was free
    std::vector<int> free_stages;
    std::unordered_map<uint64_t, std::shared_ptr<PfJob>> jobs;  // the lookup thread's
    std::deque<std::pair<std::shared_ptr<PfJob>, int>> queue;   // (job, piece) under mu, best guesses first
    std::mutex mu;
    std::condition_variable cv;
    std::atomic<bool> stop{false};
    std::atomic<int> demand{0};  // demand reads in flight: readers wait before starting a piece
    std::atomic<bool> paused{false};  // test hook: readers start no job (pieces of started jobs go on)
    std::atomic<uint64_t> bytes_read{0};
    // issued, routed and landed, routed while still reading, cancelled, taken over by a demand read
    uint64_t stat[5] = {};
};

struct PendingRead {
    int expert, slot;
};

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
    FileTier *file = nullptr;
    Prefetcher *pf = nullptr;
    // A lookup between stbl_amd_cache_lookup_begin and _end: its file misses (mapped, not yet read),
    // routed prefetch jobs still being read when it began, and whether the copy stream holds work
    // the compute stream must be ordered after.
    struct Open {
        bool open = false, order = false;
        int layer = 0;
        std::vector<PendingRead> pend;
        std::vector<uint64_t> reading;
    } op;
    // Per layer, the guesses noted for it before the lookups that may evict them, and whether each
    // was uncached then; the lookahead counters (the reference's stbl_lookahead, stbl/model.cu:452-460).
    struct Guess {
        std::vector<int> ids;
        std::vector<char> cold;
    };
    std::unordered_map<int, Guess> guesses;
    uint64_t la[4] = {};
};

// GGUF MXFP4 blocks (byte 0: E8M0 scale; byte 1+i: element i in the low nibble, element 16+i in the
// high one) to the OCP slot layout (codes: element 2j in the low nibble of byte j, 2j+1 in the high
// one; scales: one byte per 32). Block g of a part is row g / (k/32), column g % (k/32), so its codes
// go to byte 16 g of the part's codes and its scale to byte g of its scales, whatever the shape.
// One thread per block; the three parts are numbered gate, up, down, n_blocks each.
__global__ void k_gguf17_to_ocp(const uint8_t *src, uint8_t *slot, uint64_t n_blocks, uint64_t c0, uint64_t s0,
                                uint64_t c1, uint64_t s1, uint64_t c2, uint64_t s2) {
    const uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= 3 * n_blocks) return;
    const int p = (int)(g / n_blocks);
    const uint64_t b = g - (uint64_t)p * n_blocks;
    uint32_t sc;
    u32x4 c;
    load_gguf_block(src + g * 17, sc, c);
    // 4 bytes holding one nibble each -> 2 bytes of nibble pairs
    auto pk = [](uint32_t w) { return (w & 0xfu) | ((w >> 4) & 0xf0u) | ((w >> 8) & 0xf00u) | ((w >> 12) & 0xf000u); };
    u32x4 o;
    o[0] = pk(c[0] & 0x0f0f0f0fu) | pk(c[1] & 0x0f0f0f0fu) << 16;
    o[1] = pk(c[2] & 0x0f0f0f0fu) | pk(c[3] & 0x0f0f0f0fu) << 16;
    o[2] = pk((c[0] >> 4) & 0x0f0f0f0fu) | pk((c[1] >> 4) & 0x0f0f0f0fu) << 16;
    o[3] = pk((c[2] >> 4) & 0x0f0f0f0fu) | pk((c[3] >> 4) & 0x0f0f0f0fu) << 16;
    const uint64_t co = p == 0 ? c0 : p == 1 ? c1 : c2, so = p == 0 ? s0 : p == 1 ? s1 : s2;
    *(u32x4 *)(slot + co + 16 * b) = o;
    slot[so + b] = (uint8_t)sc;
}

static int take_slot(ExpertCache &c) {
    if (!c.free_slots.empty()) {
        const int s = c.free_slots.back();
        c.free_slots.pop_back();
        return s;
    }
    if (c.next_slot < c.slots) return c.next_slot++;
    return -1;  // caller evicts
}

// Stops the prefetch readers (each finishes the piece it is in) and frees their resources.
static void destroy_pf(Prefetcher *P) {
    if (!P) return;
    {
        std::lock_guard<std::mutex> lk(P->mu);
        P->stop = true;
    }
    P->cv.notify_all();
    for (auto &t : P->threads) t.join();
    for (auto st : P->stream)
        if (st) (void)hipStreamSynchronize(st);
    for (auto st : P->stream)
        if (st) (void)hipStreamDestroy(st);
    for (int i = 0; i < kPfStages; i++) {
        if (P->ready[i]) (void)hipEventDestroy(P->ready[i]);
        if (P->slot_free[i]) (void)hipEventDestroy(P->slot_free[i]);
    }
    for (auto p : P->pinned)
        if (p) (void)hipHostFree(p);
    for (auto p : P->bounce) free(p);
    if (P->stage_mem) (void)hipFree(P->stage_mem);
    delete P;
}

static void destroy_file(FileTier *f) {
    if (!f) return;
    for (auto s : f->rstream)
        if (s) (void)hipStreamSynchronize(s);
    for (auto s : f->rstream)
        if (s) (void)hipStreamDestroy(s);
    for (auto e : f->half_done)
        if (e) (void)hipEventDestroy(e);
    for (auto e : f->rdone)
        if (e) (void)hipEventDestroy(e);
    if (f->repacked) (void)hipEventDestroy(f->repacked);
    for (auto p : f->pinned)
        if (p) (void)hipHostFree(p);
    for (auto p : f->bounce) free(p);
    if (f->dstage) (void)hipFree(f->dstage);
    if (f->fd >= 0) close(f->fd);
    if (f->dfd >= 0) close(f->dfd);
    delete f;
}

// Teardown is best effort: a failure here cannot be reported to anyone who could act on it.
static void destroy(ExpertCache *c) {
    if (!c) return;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(c->device);
    destroy_pf(c->pf);  // before the file tier: its readers read the file
    if (c->copy) (void)hipStreamSynchronize(c->copy);
    destroy_file(c->file);
    for (auto &e : c->ring)
        if (e) (void)hipEventDestroy(e);
    if (c->ready) (void)hipEventDestroy(c->ready);
    if (c->copy) (void)hipStreamDestroy(c->copy);
    if (c->mem) (void)hipFree(c->mem);
    (void)hipSetDevice(prev);
    delete c;
}

// Reads `bytes` at file offset `off` into `dst` (a pinned half). Buffered reads go straight into it.
// An O_DIRECT read covers the enclosing 4 KiB-aligned range (it may run past the end of the file,
// which ends it short) and must land in pageable memory: the kernel refuses to pin pages of
// hipHostMalloc memory for direct I/O (EFAULT), so it lands in the reader's page-aligned bounce
// buffer and the payload is copied into dst. A direct read that returns short of a 4 KiB boundary
// is finished with buffered reads (O_DIRECT needs aligned offsets). Returns 0 or an errno value
// (-1: end of file).
static int read_range(const FileTier &f, uint8_t *bounce, uint8_t *dst, uint64_t off, uint64_t bytes) {
    const bool direct = f.dfd >= 0;
    const uint64_t start = direct ? off & ~(kAlign - 1) : off;
    const uint64_t need = off - start + bytes, len = direct ? (need + kAlign - 1) & ~(kAlign - 1) : need;
    uint8_t *buf = direct ? bounce : dst;
    for (uint64_t got = 0; got < need;) {
        const bool dio = direct && (got & (kAlign - 1)) == 0;
        const ssize_t r = pread(dio ? f.dfd : f.fd, buf + got, (dio ? len : need) - got, (off_t)(start + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return r == 0 ? -1 : (errno ? errno : EIO);
        got += (uint64_t)r;
    }
    if (direct) memcpy(dst, bounce + (off - start), bytes);
    return 0;
}

// Reads the pieces with every reader thread and queues their copies into device staging; `copy`
// is then made to wait for the copies. Each reader alternates between the two halves of its pinned
// stage and waits for the copy out of a half before reading into it again.
static hipError_t read_pieces(ExpertCache &c, const std::vector<Piece> &ps, std::string &err) {
    FileTier &f = *c.file;
    const int nr = (int)std::min<size_t>(f.pinned.size(), ps.size());
    for (int w = 0; w < nr && f.repack_pending; w++) {
        const hipError_t e = hipStreamWaitEvent(f.rstream[w], f.repacked, 0);  // staging still read by repacks
        if (e != hipSuccess) return err = "ordering reads after repacks", e;
    }
    std::atomic<size_t> next{0};
    std::atomic<int> failed{0};  // 0, or 1 + the failing piece's index
    std::atomic<int> status{(int)hipSuccess}, read_errno{0};
    auto work = [&](int w) {
        hipError_t e = w > 0 ? hipSetDevice(c.device) : hipSuccess;  // new threads start on device 0
        int half = 0;
        for (size_t j; e == hipSuccess && !failed && (j = next++) < ps.size(); half ^= 1) {
            const int h = 2 * w + half;
            uint8_t *stage = f.pinned[w] + (uint64_t)half * kPiece;
            if (f.half_used[h]) e = hipEventSynchronize(f.half_done[h]);
            if (e != hipSuccess) break;
            const int rc = read_range(f, f.bounce.empty() ? nullptr : f.bounce[w], stage, ps[j].off, ps[j].bytes);
            if (rc) {
                read_errno = rc;
                failed = 1 + (int)j;
                break;
            }
            e = hipMemcpyAsync(ps[j].dst, stage, ps[j].bytes, hipMemcpyHostToDevice, f.rstream[w]);
            if (e == hipSuccess) e = hipEventRecord(f.half_done[h], f.rstream[w]);
            if (e == hipSuccess) f.half_used[h] = 1;
        }
        if (e != hipSuccess) status = (int)e, failed = 1;
    };
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<std::thread> pool;
    for (int w = 1; w < nr; w++) pool.emplace_back(work, w);
    work(0);
    for (auto &t : pool) t.join();
    f.read_ns += (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0).count();
    if (failed) {
        if (status != (int)hipSuccess) return err = "copying a piece", (hipError_t)status.load();
        const Piece &p = ps[failed - 1];
        err = "reading " + std::to_string(p.bytes) + " bytes at file offset " + std::to_string(p.off) + ": " +
              (read_errno == -1 ? std::string("end of file") : std::string(strerror(read_errno)));
        return hipErrorFileNotFound;
    }
    for (int w = 0; w < nr; w++) {
        hipError_t e = hipEventRecord(f.rdone[w], f.rstream[w]);
        if (e == hipSuccess) e = hipStreamWaitEvent(c.copy, f.rdone[w], 0);
        if (e != hipSuccess) return err = "ordering the repacks after the copies", e;
    }
    for (const Piece &p : ps) f.bytes_read += p.bytes;
    return hipSuccess;
}

// Serves the file misses of one lookup: reads them in batches of kStageExperts, then repacks each
// into its slot on the copy stream after the slot's last use. Returns how many were served (a prefix
// of `pend`); on failure `err` says why.
static size_t serve_file_misses(ExpertCache &c, int layer, const std::vector<PendingRead> &pend, hipError_t &status,
                                std::string &err) {
    FileTier &f = *c.file;
    const ExpertLayout L = expert_layout(EXPERT_FP4, f.dim, f.inter);
    const uint64_t n_blocks = f.part_bytes / 17;
    size_t done = 0;
    status = hipSuccess;
    while (done < pend.size()) {
        const size_t n = std::min<size_t>(kStageExperts, pend.size() - done);
        std::vector<Piece> ps;
        for (size_t i = 0; i < n; i++) {
            if (c.fail_in >= 0 && c.fail_in-- == 0) {
                status = hipErrorUnknown;
                err = "injected refill failure";
                return done;
            }
            for (int p = 0; p < 3; p++) {
                const uint64_t off = f.part_off[3 * layer + p] + (uint64_t)pend[done + i].expert * f.part_bytes;
                uint8_t *dst = f.dstage + (3 * i + p) * f.part_bytes;
                for (uint64_t at = 0; at < f.part_bytes; at += kPiece)
                    ps.push_back({dst + at, off + at, std::min<uint64_t>(kPiece, f.part_bytes - at)});
            }
        }
        if (c.pf) c.pf->demand++;
        status = read_pieces(c, ps, err);
        if (c.pf) c.pf->demand--;
        if (status != hipSuccess) return done;
        for (size_t i = 0; i < n && status == hipSuccess; i++) {
            const int s = pend[done + i].slot;
            if (c.slot_use[s] >= 0) status = hipStreamWaitEvent(c.copy, c.ring[c.slot_use[s]], 0);
            if (status != hipSuccess) break;
            hipLaunchKernelGGL(k_gguf17_to_ocp, dim3((unsigned)((3 * n_blocks + 255) / 256)), dim3(256), 0, c.copy,
                               f.dstage + 3 * i * f.part_bytes, c.mem + (uint64_t)s * c.slot_bytes, n_blocks, L.off[0],
                               L.off[1], L.off[2], L.off[3], L.off[4], L.off[5]);
            status = hipGetLastError();
        }
        if (status == hipSuccess) status = hipEventRecord(f.repacked, c.copy);
        if (status != hipSuccess) {
            err = "queueing the repacks";
            return done;
        }
        f.repack_pending = true;
        f.experts_read += n;
        done += n;
    }
    return done;
}

// ---- prefetch ------------------------------------------------------------------------------------------

static void launch_repack(const ExpertCache &c, const uint8_t *src, int slot, hipStream_t st) {
    const FileTier &f = *c.file;
    const ExpertLayout L = expert_layout(EXPERT_FP4, f.dim, f.inter);
    const uint64_t n_blocks = f.part_bytes / 17;
    hipLaunchKernelGGL(k_gguf17_to_ocp, dim3((unsigned)((3 * n_blocks + 255) / 256)), dim3(256), 0, st, src,
                       c.mem + (uint64_t)slot * c.slot_bytes, n_blocks, L.off[0], L.off[1], L.off[2], L.off[3], L.off[4],
                       L.off[5]);
}

// A prefetch reader: takes (job, piece) from the queue, skips pieces of jobs no longer wanted, reads
// the piece into its pinned stage and copies it into the job's staging (waiting for the stage's
// previous repack first). The reader that lands a job's last piece queues the repack into the slot
// after the slot is free, records the stage's `ready` event and marks the job landed.
static void pf_reader(ExpertCache *c, int w) {
    Prefetcher &P = *c->pf;
    const FileTier &f = *c->file;
    hipError_t e = hipSetDevice(c->device);
    for (;;) {
        std::shared_ptr<PfJob> job;
        int piece = 0;
        {
            std::unique_lock<std::mutex> lk(P.mu);
            P.cv.wait(lk, [&] { return P.stop.load() || !P.queue.empty(); });
            if (P.stop) return;
            std::tie(job, piece) = P.queue.front();
            P.queue.pop_front();
        }
        while ((P.demand.load() > 0 || (P.paused.load() && job->state.load() == PF_QUEUED)) && !P.stop.load())
            std::this_thread::sleep_for(std::chrono::microseconds(20));
        job->busy++;
        int st = PF_QUEUED;
        if (!job->state.compare_exchange_strong(st, PF_READING) && st != PF_READING) {
            job->busy--;  // cancelled, taken over or failed
            continue;
        }
        const Piece &pc = job->ps[piece];
        bool ok = e == hipSuccess && hipStreamWaitEvent(P.stream[w], P.ready[job->stage], 0) == hipSuccess;
        ok = ok && read_range(f, P.bounce.empty() ? nullptr : P.bounce[w], P.pinned[w], pc.off, pc.bytes) == 0;
        ok = ok && hipMemcpyAsync(pc.dst, P.pinned[w], pc.bytes, hipMemcpyHostToDevice, P.stream[w]) == hipSuccess;
        ok = ok && hipStreamSynchronize(P.stream[w]) == hipSuccess;  // the pinned stage is reused next
        if (ok) {
            P.bytes_read += pc.bytes;
            if (++job->done == (int)job->ps.size()) {
                ok = hipStreamWaitEvent(P.stream[w], P.slot_free[job->stage], 0) == hipSuccess;
                if (ok) {
                    launch_repack(*c, P.stage_mem + (uint64_t)job->stage * 3 * f.part_bytes, job->slot, P.stream[w]);
                    ok = hipGetLastError() == hipSuccess && hipEventRecord(P.ready[job->stage], P.stream[w]) == hipSuccess;
                }
                if (ok) job->state = PF_LANDED;
            }
        }
        if (!ok) job->state = PF_FAILED;
        job->busy--;
    }
}

static void pf_release(ExpertCache &c, const std::shared_ptr<PfJob> &j) {
    while (j->busy.load() > 0) std::this_thread::yield();  // a reader still inside a piece of it
    c.pf->free_stages.push_back(j->stage);
}

// A landed job becomes an ordinary cache entry: the copy stream (and through it the compute stream,
// see order_compute) waits for its repack.
static hipError_t pf_retire_landed(ExpertCache &c, std::unordered_map<uint64_t, std::shared_ptr<PfJob>>::iterator jt) {
    const hipError_t e = hipStreamWaitEvent(c.copy, c.pf->ready[jt->second->stage], 0);
    pf_release(c, jt->second);
    c.pf->jobs.erase(jt);
    return e;
}

// Before a lookup of `layer` (stbl/model.cu:478-496): queued guesses of this layer that were not
// routed are cancelled and their slots freed; landed jobs of earlier layers and failed jobs that are
// not routed now become ordinary entries or free slots.
static hipError_t pf_settle(ExpertCache &c, int layer, const int *ids, int n) {
    Prefetcher &P = *c.pf;
    hipError_t e = hipSuccess;
    for (auto it = P.jobs.begin(); it != P.jobs.end() && e == hipSuccess;) {
        PfJob &j = *it->second;
        bool routed = false;
        for (int i = 0; i < n && j.layer == layer; i++) routed |= ids[i] == j.expert;
        int st = PF_QUEUED;
        const bool cancel = j.layer == layer && !routed && j.state.compare_exchange_strong(st, PF_CANCELLED);
        const bool drop_failed = !routed && j.state.load() == PF_FAILED;
        if (cancel || drop_failed) {
            auto w = c.where.find(it->first);
            c.lru.erase(w->second.second);
            c.where.erase(w);
            c.free_slots.push_back(j.slot);
            pf_release(c, it->second);
            if (cancel) P.stat[3]++;
            it = P.jobs.erase(it);
        } else if (j.layer < layer && j.state.load() == PF_LANDED) {
            auto next = std::next(it);
            e = pf_retire_landed(c, it);
            it = next;
        } else {
            ++it;
        }
    }
    return e;
}

// A routed expert that a prefetch job holds (stbl/model.cu:478-496, 550-553): 0 when it landed (its
// repack is then ordered on the copy stream); 1 when it is still being read (the lookup's end waits
// for it, as the reference waits after queueing the cached experts' kernels); 2 when the caller
// must read it on demand (the job had not started, or failed); <0 on a runtime error.
static int pf_claim(ExpertCache &c, std::unordered_map<uint64_t, std::shared_ptr<PfJob>>::iterator jt) {
    std::shared_ptr<PfJob> j = jt->second;
    int st = PF_QUEUED;
    if (!j->state.compare_exchange_strong(st, PF_TAKEN)) {
        if (st == PF_READING) return 1;
        if (st == PF_LANDED) {
            c.pf->stat[1]++;
            return pf_retire_landed(c, jt) == hipSuccess ? 0 : -1;
        }
    }
    c.pf->stat[4]++;  // not started (now taken) or failed
    pf_release(c, j);
    c.pf->jobs.erase(jt);
    return 2;
}

// The least recently used entry that may be evicted, skipping prefetch jobs still queued or reading
// and entries `keep` names; a landed prefetch evicted unused is retired first. Slot, -1 if none, -2 on
// a runtime error.
template <class Keep>
static int evict_lru(ExpertCache &c, Keep keep) {
    for (auto it = c.lru.end(); it != c.lru.begin();) {
        --it;
        const uint64_t key = *it;
        const int slot = c.where[key].first;
        if (keep(key, slot)) continue;
        if (c.pf) {
            auto jt = c.pf->jobs.find(key);
            if (jt != c.pf->jobs.end()) {
                if (jt->second->state.load() != PF_LANDED) continue;
                if (pf_retire_landed(c, jt) != hipSuccess) return -2;
            }
        }
        c.where.erase(key);
        c.lru.erase(it);
        return slot;
    }
    return -1;
}

static ExpertCache *new_cache(int slots, uint64_t slot_bytes, int n_experts, int n_layers) {
    ExpertCache *c = new ExpertCache();
    c->slots = slots;
    c->slot_bytes = slot_bytes;
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

// The open lookup's file misses from `from` on leave the map again (their slots are free; they
// count as neither misses nor refills), so the next lookup misses them again.
static void unmap_pending(ExpertCache &c, size_t from) {
    auto &pend = c.op.pend;
    for (size_t j = from; j < pend.size(); j++) {
        auto it = c.where.find((uint64_t)c.op.layer << 32 | (uint32_t)pend[j].expert);
        c.lru.erase(it->second.second);
        c.where.erase(it);
        c.free_slots.push_back(pend[j].slot);
        c.misses--;
        c.refill_bytes -= c.slot_bytes;
    }
    pend.resize(from);
}

// Makes `compute` wait for the work queued so far on the copy stream.
static hipError_t order_compute(ExpertCache &c, hipStream_t compute) {
    hipError_t e = hipEventRecord(c.ready, c.copy);
    if (e == hipSuccess) e = hipStreamWaitEvent(compute, c.ready, 0);
    return e;
}

// Lookahead counters at the lookup of the guessed layer (stbl/model.cu:452-460): the guesses that
// were uncached when noted and how many of them are routed; the routed experts not mapped now
// (counted before the lookup maps them) and how many of them were guessed.
static void count_lookahead(ExpertCache &c, const int *ids, int n, int layer) {
    auto g = c.guesses.find(layer);
    if (g == c.guesses.end()) return;
    const std::vector<int> &guess = g->second.ids;
    auto routed = [&](int e) { return std::find(ids, ids + n, e) != ids + n; };
    for (size_t i = 0; i < guess.size(); i++)
        if (g->second.cold[i]) c.la[0]++, c.la[1] += routed(guess[i]);
    for (int i = 0; i < n; i++)
        if (!c.where.count((uint64_t)layer << 32 | (uint32_t)ids[i]))
            c.la[2]++, c.la[3] += std::find(guess.begin(), guess.end(), ids[i]) != guess.end();
    c.guesses.erase(g);
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
    ExpertCache *c = new_cache(slots, slot_bytes, n_experts, n_layers);
    if (c) {
        c->host = (const uint8_t *)host_pool;
        c->host_stride = host_stride;
    }
    return c;
}

// File-backed cache: the routed experts of GGUF blocks first_layer .. first_layer + n_layers - 1
// (tensors blk.N.ffn_{gate,up,down}_exps.weight, MXFP4, dims [dim, inter, experts] for gate and up and
// [inter, dim, experts] for down, as the reference's converter writes them) are read from `path` on
// misses by `readers` threads (1..16) into FP4 (OCP) slots. direct = 1 reads with O_DIRECT where the
// file system supports it (falling back to buffered reads where it does not), 0 always buffered.
// Cache layer l is GGUF block first_layer + l. NULL on failure.
void *stbl_amd_cache_create_gguf(int slots, const char *path, int first_layer, int n_layers, int readers, int direct) {
    if (slots < 1 || !path || first_layer < 0 || n_layers < 1 || readers < 1 || readers > kMaxReaders) {
        abi_fail(hipErrorInvalidValue, "cache_create_gguf: bad arguments");
        return nullptr;
    }
    void *g = stbl_amd_gguf_open(path);
    if (!g) return nullptr;  // the reader recorded why
    FileTier *f = new FileTier();
    int n_experts = 0;
    std::string err;
    static const char *kParts[3] = {"gate", "up", "down"};
    for (int l = 0; l < n_layers && err.empty(); l++)
        for (int p = 0; p < 3 && err.empty(); p++) {
            const std::string name = "blk." + std::to_string(first_layer + l) + ".ffn_" + kParts[p] + "_exps.weight";
            uint32_t type = 0;
            uint64_t dims[4] = {}, off = 0, nbytes = 0;
            int nd = 0;
            if (stbl_amd_gguf_tensor(g, name.c_str(), &type, dims, &nd, &off, &nbytes) != 0) {
                err = "no tensor " + name;
                break;
            }
            const uint64_t k = dims[0], rows = dims[1], e = dims[2];
            if (type != 39 || nd != 3 || k % 32 || !rows || !e || k > (1u << 20) || rows > (1u << 20) || e > (1u << 16)) {
                err = name + ": want MXFP4 [k, rows, experts] with k % 32 == 0";
                break;
            }
            if (l == 0 && p == 0) f->dim = (int)k, f->inter = (int)rows, n_experts = (int)e;
            const bool down = p == 2;
            if (f->dim % 32 || f->inter % 32) {
                err = name + ": dim and inter must be multiples of 32";
                break;
            }
            if ((int)k != (down ? f->inter : f->dim) || (int)rows != (down ? f->dim : f->inter) || (int)e != n_experts) {
                err = name + ": shape differs from the first layer's gate";
                break;
            }
            f->part_bytes = rows * k / 32 * 17;
            f->part_off.push_back(off);
        }
    stbl_amd_gguf_close(g);
    ExpertCache *c = nullptr;
    if (err.empty()) c = new_cache(slots, expert_layout(EXPERT_FP4, f->dim, f->inter).bytes, n_experts, n_layers);
    if (!c) {
        if (!err.empty()) abi_fail(hipErrorInvalidValue, "cache_create_gguf: %s: %s", path, err.c_str());
        destroy_file(f);
        return nullptr;
    }
    c->file = f;
    f->fd = open(path, O_RDONLY);
    if (direct) f->dfd = open(path, O_RDONLY | O_DIRECT);  // -1 where the file system refuses it
    hipError_t e = f->fd >= 0 ? hipSuccess : hipErrorFileNotFound;
    if (e == hipSuccess) e = hipMalloc(&f->dstage, (size_t)kStageExperts * 3 * f->part_bytes);
    if (e == hipSuccess) e = hipMemsetAsync(c->mem, 0, (size_t)c->slots * c->slot_bytes, c->copy);  // padding reads as 0
    f->pinned.assign(readers, nullptr);
    f->rstream.assign(readers, nullptr);
    f->rdone.assign(readers, nullptr);
    f->half_done.assign(2 * readers, nullptr);
    f->half_used.assign(2 * readers, 0);
    for (int w = 0; w < readers && e == hipSuccess; w++) {
        e = hipHostMalloc((void **)&f->pinned[w], 2 * kPiece, hipHostMallocDefault);
        if (e == hipSuccess && f->dfd >= 0) {
            void *b = nullptr;
            if (posix_memalign(&b, kAlign, kPiece + 2 * kAlign)) e = hipErrorOutOfMemory;
            f->bounce.push_back((uint8_t *)b);
        }
        if (e == hipSuccess) e = hipStreamCreateWithFlags(&f->rstream[w], hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&f->rdone[w], hipEventDisableTiming);
        for (int h = 0; h < 2 && e == hipSuccess; h++) e = hipEventCreateWithFlags(&f->half_done[2 * w + h], hipEventDisableTiming);
    }
    if (e == hipSuccess) e = hipEventCreateWithFlags(&f->repacked, hipEventDisableTiming);
    if (e != hipSuccess) {
        abi_status(e, "cache_create_gguf");
        destroy(c);
        return nullptr;
    }
    return c;
}

// File tier facts: out[0..7] = dim, inter, experts, slot bytes, 1 if reads use O_DIRECT, bytes read
// from the file, nanoseconds spent reading (wall time of the reader threads), experts read.
int stbl_amd_cache_file_info(void *cache, uint64_t *out) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || !out || !c->file) return abi_fail(hipErrorInvalidValue, "cache_file_info: not a file-backed cache");
    const FileTier &f = *c->file;
    const uint64_t v[8] = {(uint64_t)f.dim, (uint64_t)f.inter, (uint64_t)c->n_experts, c->slot_bytes, f.dfd >= 0 ? 1u : 0u,
                           f.bytes_read, f.read_ns, f.experts_read};
    for (int i = 0; i < 8; i++) out[i] = v[i];
    return 0;
}

void stbl_amd_cache_destroy(void *cache) { destroy((ExpertCache *)cache); }

// Looks up n expert ids (HOST array) of one layer, in order, and maps every miss to a slot.
// slot_ptrs (HOST, n entries) receives each expert's slot; hit (HOST, optional) 1/0 per id; ready
// (HOST, optional) 1 where `compute` may read the slot at once, 0 where it must first pass
// stbl_amd_cache_lookup_end (a refill, a landed or still-reading prefetch). Pool misses are queued on
// the copy stream here; file misses are read by _end. Every begin must be followed by an end before
// the next lookup or prefetch of the cache: in between, the caller may queue kernels that read the
// ready slots, which then run while the misses are copied or read (stbl/model.cu:541-549, 588).
// Returns the number of misses, or a negative hipError_t (then nothing of this lookup is mapped that
// was not before, apart from completed refills; the lookup is not open and slot_ptrs must not be used).
int stbl_amd_cache_lookup_begin(void *cache, const int *ids, int n, int layer, void **slot_ptrs, int *hit, int *ready,
                                hipStream_t compute) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || !ids || !slot_ptrs || n < 0 || layer < 0 || layer >= c->n_layers)
        return abi_fail(hipErrorInvalidValue, "cache_lookup: bad arguments");
    if (c->op.open) return abi_fail(hipErrorInvalidValue, "cache_lookup: the previous lookup was not ended");
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= c->n_experts) return abi_fail(hipErrorInvalidValue, "cache_lookup: expert id %d out of range", ids[i]);
    c->lookups++;
    count_lookahead(*c, ids, n, layer);
    auto key = [&](int e) { return (uint64_t)layer << 32 | (uint32_t)e; };
    ExpertCache::Open &op = c->op;
    op.order = false;
    op.layer = layer;
    op.pend.clear();
    op.reading.clear();
    // A lookup that fails after queueing refills still orders `compute` after them: the refilled
    // experts stay mapped, and a later lookup that hits them queues no wait of its own.
    auto fail = [&](hipError_t e, const std::string &msg) {
        unmap_pending(*c, 0);
        op.reading.clear();
        if (op.order) (void)order_compute(*c, compute);
        return abi_fail(e, "cache_lookup: %s", msg.c_str());
    };
    if (c->pf) {
        const hipError_t e = pf_settle(*c, layer, ids, n);
        op.order = true;  // retired prefetches made the copy stream wait
        if (e != hipSuccess) return fail(e, std::string("settling prefetches: ") + hipGetErrorString(e));
    }
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
        int s = -1;
        if (it != c->where.end()) {
            c->lru.splice(c->lru.begin(), c->lru, it->second.second);
            s = it->second.first;
            int claim = -3;  // a plain entry
            if (c->pf) {
                auto jt = c->pf->jobs.find(k);
                if (jt != c->pf->jobs.end()) claim = pf_claim(*c, jt);
            }
            if (claim == -1) return fail(hipErrorUnknown, "expert " + std::to_string(ids[i]) + ": retiring its prefetch failed");
            if (claim != 2) {
                slot_ptrs[i] = c->mem + (uint64_t)s * c->slot_bytes;
                if (hit) hit[i] = 1;
                if (ready) ready[i] = claim == -3;
                if (claim == 0) op.order = true;
                if (claim == 1) op.reading.push_back(k);
                c->hits++;
                c->touched.push_back(s);
                continue;
            }
            op.pend.push_back({ids[i], s});  // a prefetch that had not started or failed: read it on demand
        } else {
            // 2. miss: a free slot, or the least recently used entry not needed by this lookup
            s = take_slot(*c);
            if (s < 0)
                s = evict_lru(*c, [&](uint64_t key_, int) {
                    for (int j = 0; j < n; j++)
                        if (key(ids[j]) == key_) return true;
                    return false;
                });
            if (s == -2) return fail(hipErrorUnknown, "expert " + std::to_string(ids[i]) + ": retiring a prefetch failed");
            if (s < 0)
                return fail(hipErrorOutOfMemory,
                            "every slot is held by this lookup or a prefetch (" + std::to_string(c->slots) + " slots)");
            if (!c->file) {
                const uint8_t *src = c->host + ((uint64_t)layer * c->n_experts + ids[i]) * c->host_stride;
                hipError_t e = hipSuccess;
                if (c->slot_use[s] >= 0) e = hipStreamWaitEvent(c->copy, c->ring[c->slot_use[s]], 0);
                if (e == hipSuccess) {
                    if (c->fail_in == 0) e = hipErrorUnknown;
                    else e = hipMemcpyAsync(c->mem + (uint64_t)s * c->slot_bytes, src, c->slot_bytes, hipMemcpyHostToDevice, c->copy);
                    if (c->fail_in >= 0) c->fail_in--;
                }
                if (e != hipSuccess) {
                    c->free_slots.push_back(s);  // slot stays unmapped: the next lookup misses again
                    return fail(e, "refill of expert " + std::to_string(ids[i]) + " failed: " + hipGetErrorString(e));
                }
                op.order = true;
            } else {
                op.pend.push_back({ids[i], s});
            }
            c->lru.push_front(k);
            c->where[k] = {s, c->lru.begin()};
        }
        slot_ptrs[i] = c->mem + (uint64_t)s * c->slot_bytes;
        if (hit) hit[i] = 0;
        if (ready) ready[i] = 0;
        c->misses++;
        c->refill_bytes += c->slot_bytes;
        c->touched.push_back(s);
        nmiss++;
    }
    op.open = true;
    return nmiss;
}

// Ends the open lookup (a no-op when none is open): reads its file misses (the host thread waits
// for the reads; the kernels queued meanwhile run on), waits for routed prefetches still being
// read (one that failed is read on demand), and makes `compute` wait for every copy and repack of
// the lookup. Returns 0 or a negative hipError_t; on failure the experts not yet read stay unmapped
// and the caller must not queue kernels on the slots begin reported not ready.
int stbl_amd_cache_lookup_end(void *cache, hipStream_t compute) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c) return abi_fail(hipErrorInvalidValue, "cache_lookup_end: null cache");
    ExpertCache::Open &op = c->op;
    if (!op.open) return 0;
    op.open = false;
    auto serve = [&]() -> int {
        if (op.pend.empty()) return 0;
        hipError_t e;
        std::string err;
        const size_t served = serve_file_misses(*c, op.layer, op.pend, e, err);
        op.order |= served > 0;
        if (served == op.pend.size()) {
            op.pend.clear();
            return 0;
        }
        const int first = op.pend[served].expert;
        unmap_pending(*c, served);
        if (op.order) (void)order_compute(*c, compute);
        return abi_fail(e == hipSuccess ? hipErrorUnknown : e, "cache_lookup: reading expert %d of layer %d failed: %s",
                        first, op.layer, err.c_str());
    };
    // 1. demand reads (stbl/model.cu:550)
    if (int r = serve()) return r;
    // 2. routed prefetches that were being read (stbl/model.cu:551-553)
    for (uint64_t k : op.reading) {
        auto jt = c->pf->jobs.find(k);
        if (jt == c->pf->jobs.end()) continue;
        const std::shared_ptr<PfJob> j = jt->second;
        int st;
        while ((st = j->state.load()) == PF_READING) std::this_thread::yield();
        if (st == PF_LANDED) {
            c->pf->stat[2]++;
            op.order = true;
            if (pf_retire_landed(*c, jt) != hipSuccess) {
                (void)order_compute(*c, compute);
                return abi_fail(hipErrorUnknown, "cache_lookup: retiring the prefetch of expert %d failed", j->expert);
            }
        } else {  // it failed: read it on demand, as a miss
            c->pf->stat[4]++;
            pf_release(*c, j);
            c->pf->jobs.erase(jt);
            op.pend.push_back({j->expert, j->slot});
            c->hits--, c->misses++, c->refill_bytes += c->slot_bytes;
        }
    }
    op.reading.clear();
    if (int r = serve()) return r;
    if (op.order) {
        const hipError_t e = order_compute(*c, compute);
        if (e != hipSuccess) return abi_status(e, "cache_lookup: ordering the compute stream after the refills");
    }
    return 0;
}

// Looks up n expert ids of one layer and makes `compute` wait for every refill: begin, then end.
// Returns the number of misses, or a negative hipError_t (then nothing of this lookup is mapped that
// was not before, apart from completed refills, and the caller must not use slot_ptrs).
int stbl_amd_cache_lookup(void *cache, const int *ids, int n, int layer, void **slot_ptrs, int *hit,
                          hipStream_t compute) {
    const int nmiss = stbl_amd_cache_lookup_begin(cache, ids, n, layer, slot_ptrs, hit, nullptr, compute);
    if (nmiss < 0) return nmiss;
    const int r = stbl_amd_cache_lookup_end(cache, compute);
    return r < 0 ? r : nmiss;
}

// Notes the guesses for `layer` (best first; the reference's STBL_LOOKAHEAD guesses: the next
// layer's router on this layer's input, stbl/model.cu:461-474) before the lookups that could evict
// them, with whether each is uncached now. The next lookup of `layer` then updates the lookahead
// counters with them. A later note for the same layer replaces an unused one.
int stbl_amd_cache_note_guesses(void *cache, const int *ids, int n, int layer) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || (!ids && n > 0) || n < 0 || layer < 0 || layer >= c->n_layers)
        return abi_fail(hipErrorInvalidValue, "cache_note_guesses: bad arguments");
    ExpertCache::Guess &g = c->guesses[layer];
    g.ids.assign(ids, ids + n);
    g.cold.assign(n, 0);
    for (int i = 0; i < n; i++) g.cold[i] = !c->where.count((uint64_t)layer << 32 | (uint32_t)ids[i]);
    return 0;
}

// out[0..3] = guesses that were uncached when noted, of those how many the lookup of their layer
// routed; routed experts that were not mapped at their lookup, of those how many were guessed (the
// reference's stbl_lookahead counters, stbl/model.cu:452-460, 1107-1109).
int stbl_amd_cache_lookahead(void *cache, uint64_t *out) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || !out) return abi_fail(hipErrorInvalidValue, "cache_lookahead: bad arguments");
    for (int i = 0; i < 4; i++) out[i] = c->la[i];
    return 0;
}

// Starts `readers` (1..16) background prefetch readers on a file-backed cache, with staging for
// kPfStages experts in flight. Once per cache.
int stbl_amd_cache_enable_prefetch(void *cache, int readers) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || !c->file || readers < 1 || readers > kMaxReaders)
        return abi_fail(hipErrorInvalidValue, "cache_enable_prefetch: needs a file-backed cache and 1..%d readers", kMaxReaders);
    if (c->pf) return abi_fail(hipErrorInvalidValue, "cache_enable_prefetch: already enabled");
    Prefetcher *P = new Prefetcher();
    const FileTier &f = *c->file;
    hipError_t e = hipMalloc(&P->stage_mem, (size_t)kPfStages * 3 * f.part_bytes);
    for (int i = 0; i < kPfStages && e == hipSuccess; i++) {
        e = hipEventCreateWithFlags(&P->ready[i], hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&P->slot_free[i], hipEventDisableTiming);
        P->free_stages.push_back(kPfStages - 1 - i);
    }
    P->pinned.assign(readers, nullptr);
    P->stream.assign(readers, nullptr);
    for (int w = 0; w < readers && e == hipSuccess; w++) {
        e = hipHostMalloc((void **)&P->pinned[w], kPiece, hipHostMallocDefault);
        if (e == hipSuccess) e = hipStreamCreateWithFlags(&P->stream[w], hipStreamNonBlocking);
        if (e == hipSuccess && f.dfd >= 0) {
            void *b = nullptr;
            if (posix_memalign(&b, kAlign, kPiece + 2 * kAlign)) e = hipErrorOutOfMemory;
            P->bounce.push_back((uint8_t *)b);
        }
    }
    if (e != hipSuccess) {
        destroy_pf(P);
        return abi_status(e, "cache_enable_prefetch");
    }
    c->pf = P;
    for (int w = 0; w < readers; w++) P->threads.emplace_back(pf_reader, c, w);
    return 0;
}

// Queues background reads of the given experts of `layer` (HOST array, best guess first; the
// reference's stale-router guesses, stbl/model.cu:555-586) that are not cached. Each gets a slot
// (never one of the last lookup's, so the kernels queued for it keep their weights) and is mapped at
// once; a later lookup that routes it waits for it, reads it itself if it had not started, and the
// lookup of its layer cancels it if it is not routed and has not started. Stops early when kPfStages
// jobs are in flight or no slot can be taken. Returns the number queued or a negative hipError_t.
int stbl_amd_cache_prefetch(void *cache, const int *ids, int n, int layer) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || !c->pf || !ids || n < 0 || layer < 0 || layer >= c->n_layers)
        return abi_fail(hipErrorInvalidValue, "cache_prefetch: bad arguments or prefetch not enabled");
    if (c->op.open) return abi_fail(hipErrorInvalidValue, "cache_prefetch: a lookup is open (end it first)");
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= c->n_experts) return abi_fail(hipErrorInvalidValue, "cache_prefetch: expert id %d out of range", ids[i]);
    Prefetcher &P = *c->pf;
    const FileTier &f = *c->file;
    std::vector<std::shared_ptr<PfJob>> fresh;
    hipError_t e = hipSuccess;
    for (int i = 0; i < n && !P.free_stages.empty(); i++) {
        const uint64_t key = (uint64_t)layer << 32 | (uint32_t)ids[i];
        if (c->where.count(key)) continue;
        int s = take_slot(*c);
        if (s < 0)
            s = evict_lru(*c, [&](uint64_t, int slot) {
                return std::find(c->touched.begin(), c->touched.end(), slot) != c->touched.end();
            });
        if (s == -2) {
            e = hipErrorUnknown;
            break;
        }
        if (s < 0) break;
        auto j = std::make_shared<PfJob>();
        j->layer = layer, j->expert = ids[i], j->slot = s, j->stage = P.free_stages.back();
        // the slot is free once the compute stream's last use of it is done
        if (c->slot_use[s] >= 0) e = hipStreamWaitEvent(c->copy, c->ring[c->slot_use[s]], 0);
        if (e == hipSuccess) e = hipEventRecord(P.slot_free[j->stage], c->copy);
        if (e != hipSuccess) {
            c->free_slots.push_back(s);
            break;
        }
        P.free_stages.pop_back();
        uint8_t *stage = P.stage_mem + (uint64_t)j->stage * 3 * f.part_bytes;
        for (int p = 0; p < 3; p++) {
            const uint64_t off = f.part_off[3 * layer + p] + (uint64_t)ids[i] * f.part_bytes;
            for (uint64_t at = 0; at < f.part_bytes; at += kPiece)
                j->ps.push_back({stage + p * f.part_bytes + at, off + at, std::min<uint64_t>(kPiece, f.part_bytes - at)});
        }
        c->lru.push_front(key);
        c->where[key] = {s, c->lru.begin()};
        P.jobs[key] = j;
        fresh.push_back(j);
        P.stat[0]++;
    }
    if (!fresh.empty()) {
        {
            std::lock_guard<std::mutex> lk(P.mu);
            for (auto &j : fresh)
                for (int pc = 0; pc < (int)j->ps.size(); pc++) P.queue.emplace_back(j, pc);
        }
        P.cv.notify_all();
    }
    if (e != hipSuccess) return abi_status(e, "cache_prefetch");
    return (int)fresh.size();
}

// Test hook: while paused, prefetch readers start no queued job (a started one is finished).
int stbl_amd_cache_prefetch_pause(void *cache, int paused) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || !c->pf) return abi_fail(hipErrorInvalidValue, "cache_prefetch_pause: prefetch not enabled");
    c->pf->paused = paused != 0;
    return 0;
}

// out[0..5] = prefetches issued, routed after landing, routed while still reading (the lookup
// waited), cancelled unrouted, taken over by a demand read (not started or failed), bytes read by
// the prefetch readers (the reference's stbl_prefetch counters, stbl/model.cu:1103-1105).
int stbl_amd_cache_prefetch_stats(void *cache, uint64_t *out) {
    ExpertCache *c = (ExpertCache *)cache;
    if (!c || !c->pf || !out) return abi_fail(hipErrorInvalidValue, "cache_prefetch_stats: prefetch not enabled");
    for (int i = 0; i < 5; i++) out[i] = c->pf->stat[i];
    out[5] = c->pf->bytes_read.load();
    return 0;
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
