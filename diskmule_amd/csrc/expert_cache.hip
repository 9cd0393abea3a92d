// expert_cache.hip -- routed-expert residency and the MoE decode layer.
//
// ExpertCache of src/expert.rs:64-229 with HBM slots: the LRU bookkeeping is
// the reference's (clock per layer, hit updates last_used, a miss evicts the
// unpinned slot with the smallest (is_some, last_used, index)), and the
// positional reads become asynchronous host->HBM copies on the context's
// two upload streams (alternating by expert).  The expert bytes come from
// host memory the caller provides (ideally pinned), or from a file: then a
// miss reads gate_up and down with two parallel positional reads into one
// entry of a small pinned staging ring (src/expert.rs:203-215, :241-256), and
// the ring bounds the host memory the cache uses.
//
// Ordering is by events, never by device-wide waits:
//   * before an upload into a slot is issued, the host waits for the
//     `released` event recorded after the last compute work that read the
//     slot, and for the `ready` event of the slot's previous upload (the
//     upload streams themselves never wait on another queue's event);
//   * compute work that uses a freshly loaded slot waits for its `ready`
//     event (the end of its upload);
//   * a staging entry is refilled only after the host has waited for the
//     copy out of it (`done`).
#include "runtime.h"

#include <errno.h>
#include <string.h>
#include <unistd.h>

#include <chrono>
#include <thread>
#include <vector>

#include "dm_qmv.h"

namespace dm {

// Host-to-HBM copy of one expert's two byte ranges (gate_up, then down) by a
// kernel that reads the pinned source over PCIe: each thread keeps four
// 16-byte loads in flight before it stores them.  Measured on MI355X with
// 3 MB experts on two upload streams: 54-55 GB/s against 42.6 GB/s for
// hipMemcpyAsync (the DMA engines), 16 to 32 workgroups per copy.
constexpr uint32_t kUploadCopyGroups = 32;
typedef uint32_t c16 __attribute__((ext_vector_type(4)));  // 16-byte aligned
__global__ void __launch_bounds__(256) upload_copy_kernel(const c16 *__restrict__ a_src, c16 *__restrict__ a_dst,
                                                          size_t a16, const c16 *__restrict__ b_src,
                                                          c16 *__restrict__ b_dst, size_t b16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x, n = a16 + b16;
    auto at = [&](size_t i) -> const c16 & { return i < a16 ? a_src[i] : b_src[i - a16]; };
    auto put = [&](size_t i, const c16 &v) {
        if (i < a16) a_dst[i] = v; else b_dst[i - a16] = v;
    };
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n; i += 4 * stride) {
        const c16 v0 = at(i), v1 = at(i + stride), v2 = at(i + 2 * stride), v3 = at(i + 3 * stride);
        put(i, v0);
        put(i + stride, v1);
        put(i + 2 * stride, v2);
        put(i + 3 * stride, v3);
    }
    for (; i < n; i += stride) put(i, at(i));
}

__global__ void gather_rows_kernel(const float *__restrict__ x, const uint32_t *__restrict__ rows,
                                   uint32_t count, uint32_t width, float *__restrict__ out) {
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < (size_t)count * width;
         e += (size_t)gridDim.x * blockDim.x) {
        uint32_t p = (uint32_t)(e / width), i = (uint32_t)(e - (size_t)p * width);
        out[e] = x[(size_t)rows[p] * width + i];
    }
}

// y[t] = fold over the k selections in order of fma(out[pos[t][j]], p[t][j], y)
// (src/gemma4/cpu.rs:608-611); without `pos` selection t * k + j is row
// t * k + j of expert_out.
__global__ void moe_combine_pos_kernel(const float *__restrict__ expert_out,
                                       const uint32_t *__restrict__ pos, const float *__restrict__ p,
                                       uint32_t batch, uint32_t k, uint32_t hidden,
                                       float *__restrict__ y, const uint32_t *__restrict__ go) {
    // the device-side lookup found a slot missing (go: one word per token)
    if (go)
        for (uint32_t t = 0; t < batch; t++)
            if (go[t] == 0) return;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < (size_t)batch * hidden;
         e += (size_t)gridDim.x * blockDim.x) {
        uint32_t t = (uint32_t)(e / hidden), i = (uint32_t)(e - (size_t)t * hidden);
        float acc = 0.0f;
        for (uint32_t j = 0; j < k; j++) {
            const size_t row = pos ? pos[t * k + j] : t * k + j;
            acc = __builtin_fmaf(expert_out[row * hidden + i], p[t * k + j], acc);
        }
        y[e] = acc;
    }
}

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_expert() { return (const void *)gather_rows_kernel; }

struct Slot {
    bool has = false;
    size_t expert = 0;
    uint64_t last_used = 0;
    // Holders through dmhip_expert_acquire; a slot with pins is never a
    // victim.  (The MoE layer's own acquires do not pin: it never evicts a
    // slot its open phase uses.)
    uint32_t pins = 0;
    dmhip_buf *gate_up_buf = nullptr;  // cache-owned, len = gate_up_bytes
    dmhip_buf *down_buf = nullptr;     // cache-owned, len = down_bytes
    void *gate_up = nullptr;           // their device addresses
    void *down = nullptr;
    hipEvent_t ready = nullptr;  // end of the last upload into the slot
    bool uploaded = false;       // ready has been recorded
    // The compute stream has not been made to wait for `ready` yet (the MoE
    // layer defers that wait to the launch that first reads the slot).
    bool ready_pending = false;
    // End of the last compute that read it: an event of the cache's ring,
    // shared by the slots released together.  Once the ring wraps the event
    // may be recorded again later on the same stream, which only makes a
    // wait on it later, never earlier.
    hipEvent_t released = nullptr;
    bool released_recorded = false;
};

struct Layer {
    dmhip_expert_layer_layout layout;
    std::vector<Slot> slots;
    uint64_t clock = 0;
    // This layer's residency table: the device addresses of each expert's
    // slot bytes (gate_up at [0, expert_count), down after them; 0 when not
    // resident).  The host keeps the master copy in pinned memory and
    // copies it to the device copy before a call that looks experts up,
    // when it changed since.
    uint64_t *table = nullptr;       // device copy
    uint64_t *host_table = nullptr;  // pinned master
    bool table_dirty = false;
    // Whether the next one-token MoE call tries the device-side lookup: set
    // after a call whose experts were all resident, cleared by one that
    // found a slot missing.
    bool try_lookup = true;
};

// Memory source: the device time of one upload, a (start, end) pair of
// timing events from a ring.  io_wait adds the durations of finished
// uploads; nothing on the acquire path waits for an upload to finish.
struct TimedUpload {
    hipEvent_t start = nullptr, end = nullptr;
    bool pending = false;  // recorded, not yet added to io_wait
};

// One pinned host buffer of the file source's staging ring.
struct Staging {
    uint8_t *host = nullptr;
    uint8_t *host_dev = nullptr;  // its device address (pinned memory)
    hipEvent_t done = nullptr;  // end of the copies out of it
    bool busy = false;          // done has been recorded
};

}  // namespace dm

struct dmhip_expert_cache {
    dmhip_ctx *ctx = nullptr;
    int device = 0;
    // Memory source (fd < 0) or file source.
    const uint8_t *source = nullptr;
    size_t source_len = 0;
    // The source's address on the device when it is pinned host memory
    // (uploads then run as copy kernels), else null (hipMemcpyAsync).
    const uint8_t *source_dev = nullptr;
    int fd = -1;
    std::vector<dm::Staging> staging;
    size_t next_staging = 0;
    std::vector<dm::TimedUpload> timed;  // memory source
    size_t next_timed = 0;
    std::vector<dm::Layer> layers;
    dmhip_expert_cache_stats stats = {};
    // MoE workspace (device): grows on demand.
    dm::Scratch work;
    // Pinned host copy of the router's selection (ids, then probabilities;
    // kSelectionPairs pairs, then one non-finite flag per token), written by
    // the router kernel itself.
    uint8_t *host_selection = nullptr;
    // Release events, used round-robin: one record per released group.
    std::vector<hipEvent_t> release_events;
    size_t next_release = 0;
    // Device memory: every layer's residency table, then the lookup's
    // outputs (gate_up and down addresses per selection, a go word per token); the
    // tables' pinned host masters.
    uint64_t *tables = nullptr;
    uint64_t *host_tables = nullptr;
    uint64_t *lookup_gate_up = nullptr, *lookup_down = nullptr;
    uint32_t *lookup_go = nullptr;
    uint32_t *combine_tickets = nullptr;  // kCombineTickets, zero between calls
};

namespace {
constexpr size_t kSelectionPairs = 16 * dm::kMaxTopK;  // batch <= 16
constexpr size_t kSelectionBytes = kSelectionPairs * 8 + 16 * 4 + 16 * 4;  // ids, probabilities, per-token flags, go
constexpr size_t kReleaseEvents = 64;
constexpr size_t kCombineTickets = 4096;  // row-tile workgroups of a fused down + combine launch
constexpr size_t kStagingEntries = 4;  // file source: experts in flight from storage
// Memory source: uploads whose timing is kept until it is read.  The ring is
// reused oldest first, so a wait at reuse only ever meets an upload issued
// 64 uploads earlier.
constexpr size_t kTimedUploads = 64;
}

using namespace dm;

namespace {

// read_exact_at (src/expert.rs:241-256): the whole range or an error; an
// interrupted read is retried, a zero-byte read is an unexpected end of
// file (error 0).
int read_exact_at(int fd, uint64_t offset, uint8_t *dst, size_t n) {
    while (n > 0) {
        const ssize_t got = pread(fd, dst, n, (off_t)offset);
        if (got == 0) return 0;
        if (got < 0) {
            if (errno == EINTR) continue;
            return errno ? errno : EIO;
        }
        dst += got;
        n -= (size_t)got;
        offset += (uint64_t)got;
    }
    return -1;  // complete
}

// Adds the device-measured duration of a finished upload into io_wait (the
// memory source: the host never waits for its asynchronous copies, so the
// time the bytes took to arrive is what io_wait reports).  `wait` waits for
// an upload still in flight; otherwise one in flight is left for later.
void account_upload(dmhip_expert_cache *c, TimedUpload &t, bool wait) {
    if (!t.pending) return;
    if (!wait && hipEventQuery(t.end) != hipSuccess) return;
    float ms = 0.0f;
    if (hipEventSynchronize(t.end) == hipSuccess && hipEventElapsedTime(&ms, t.start, t.end) == hipSuccess)
        c->stats.io_wait_ns += (uint64_t)((double)ms * 1e6);
    t.pending = false;
}

void account_uploads(dmhip_expert_cache *c, bool wait) {
    for (TimedUpload &t : c->timed) account_upload(c, t, wait);
}

// Copies expert `expert` of the layer into slot s on an upload stream that
// first waits for the slot's last readers and its previous upload.  With
// wait_now the compute stream waits for the copy at once; otherwise the
// slot is marked ready_pending and the caller enqueues that wait
// (wait_ready) before the first work that reads the slot.
int upload_expert(dmhip_expert_cache *c, const dmhip_expert_layer_layout &L, size_t expert, Slot &s,
                  bool wait_now) {
    const size_t gu_bytes = L.gate_up_bytes, dn_bytes = L.down_bytes;
    const uint64_t gu_off = L.gate_up_offset + (uint64_t)expert * gu_bytes;
    const uint64_t dn_off = L.down_offset + (uint64_t)expert * dn_bytes;
    const auto started = std::chrono::steady_clock::now();
    const uint8_t *gu_src, *dn_src;
    Staging *entry = nullptr;
    if (c->fd >= 0) {
        entry = &c->staging[c->next_staging++ % c->staging.size()];
        if (entry->busy) DM_HIP(hipEventSynchronize(entry->done));
        entry->busy = false;
        // the two reads in parallel, as rayon::join does (src/expert.rs:209-212)
        int gu_err = -1, dn_err = -1;
        std::thread reader([&] { gu_err = read_exact_at(c->fd, gu_off, entry->host, gu_bytes); });
        dn_err = read_exact_at(c->fd, dn_off, entry->host + gu_bytes, dn_bytes);
        reader.join();
        if (gu_err >= 0) return fail_io(gu_err);
        if (dn_err >= 0) return fail_io(dn_err);
        gu_src = entry->host;
        dn_src = entry->host + gu_bytes;
    } else {
        gu_src = c->source + gu_off;
        dn_src = c->source + dn_off;
    }
    // the source's device addresses, when the copy can run as a kernel
    const uint8_t *gu_dev = nullptr, *dn_dev = nullptr;
    if (entry && entry->host_dev) {
        gu_dev = entry->host_dev;
        dn_dev = entry->host_dev + gu_bytes;
    } else if (!entry && c->source_dev) {
        gu_dev = c->source_dev + gu_off;
        dn_dev = c->source_dev + dn_off;
    }
    const bool by_kernel = gu_dev && ((uintptr_t)gu_dev % 16 | (uintptr_t)dn_dev % 16 | gu_bytes % 16 |
                                      dn_bytes % 16 | (uintptr_t)s.gate_up % 16 | (uintptr_t)s.down % 16) == 0;
    // experts alternate between the two upload streams
    hipStream_t up = (c->ctx->upload_next++ & 1u) ? c->ctx->upload2 : c->ctx->upload;
    // The slot's last readers and its previous upload are waited for here,
    // on the host, not by the upload stream: a copy queued behind a wait on
    // an event of another queue that has not completed yet moved expert
    // bytes at 26 GB/s against 42 GB/s for free copies (MI355X, the MoE
    // layer at 4 tokens: 3.6-4.3 against 2.2 ms per call).  Both events are
    // usually complete by the time a slot is reused.
    if (s.released_recorded) DM_HIP(hipEventSynchronize(s.released));
    if (s.uploaded) DM_HIP(hipEventSynchronize(s.ready));
    TimedUpload *timer = nullptr;
    if (c->fd < 0) {
        timer = &c->timed[c->next_timed++ % c->timed.size()];
        account_upload(c, *timer, true);  // the oldest pair of the ring
        DM_HIP(hipEventRecord(timer->start, up));
    }
    if (by_kernel) {
        hipLaunchKernelGGL(upload_copy_kernel, dim3(kUploadCopyGroups), dim3(256), 0, up, (const c16 *)gu_dev,
                           (c16 *)s.gate_up, gu_bytes / 16, (const c16 *)dn_dev, (c16 *)s.down, dn_bytes / 16);
        DM_HIP(hipGetLastError());
    } else {
        DM_HIP(hipMemcpyAsync(s.gate_up, gu_src, gu_bytes, hipMemcpyHostToDevice, up));
        DM_HIP(hipMemcpyAsync(s.down, dn_src, dn_bytes, hipMemcpyHostToDevice, up));
    }
    DM_HIP(hipEventRecord(s.ready, up));
    s.uploaded = true;
    if (timer) {
        DM_HIP(hipEventRecord(timer->end, up));
        timer->pending = true;
    }
    if (entry) {
        DM_HIP(hipEventRecord(entry->done, up));
        entry->busy = true;
        c->stats.io_wait_ns += (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                                   std::chrono::steady_clock::now() - started).count();
    }
    if (wait_now) {
        DM_HIP(hipStreamWaitEvent(c->ctx->stream, s.ready, 0));
        s.ready_pending = false;
    } else {
        s.ready_pending = true;
    }
    return DMHIP_OK;
}

// Makes the compute stream wait for a deferred upload into the slot.
int wait_ready(dmhip_expert_cache *c, Slot &s) {
    if (s.ready_pending) {
        DM_HIP(hipStreamWaitEvent(c->ctx->stream, s.ready, 0));
        s.ready_pending = false;
    }
    return DMHIP_OK;
}

int wait_all_ready(dmhip_expert_cache *c, size_t layer) {
    for (Slot &s : c->layers[layer].slots) DM_CHECK_STATUS(wait_ready(c, s));
    return DMHIP_OK;
}

// ExpertCache::acquire (src/expert.rs:166-229): the slot holding `expert`,
// or the victim it is loaded into.  Counters as in the reference: a miss
// counts before its reads, so a failed read leaves misses (and evictions)
// counted but no reads; the slot then keeps its previous expert.
int acquire(dmhip_expert_cache *c, size_t layer_index, size_t expert, size_t *slot_out, bool wait_now = true) {
    if (layer_index >= c->layers.size()) return fail_layer(layer_index, c->layers.size());
    Layer &layer = c->layers[layer_index];
    if (expert >= layer.layout.expert_count) return fail_expert(layer_index, expert, layer.layout.expert_count);
    layer.clock += 1;
    for (size_t i = 0; i < layer.slots.size(); i++) {
        Slot &s = layer.slots[i];
        if (s.has && s.expert == expert) {
            s.last_used = layer.clock;
            c->stats.hits += 1;
            *slot_out = i;
            return DMHIP_OK;
        }
    }
    c->stats.misses += 1;
    size_t victim = SIZE_MAX;
    for (size_t i = 0; i < layer.slots.size(); i++) {
        const Slot &s = layer.slots[i];
        if (s.pins) continue;
        if (victim == SIZE_MAX) { victim = i; continue; }
        const Slot &v = layer.slots[victim];
        if (s.has < v.has || (s.has == v.has && s.last_used < v.last_used)) victim = i;
    }
    if (victim == SIZE_MAX) return fail_pinned(layer_index);
    Slot &s = layer.slots[victim];
    if (s.has) c->stats.evictions += 1;
    DM_CHECK_STATUS(upload_expert(c, layer.layout, expert, s, wait_now));
    // the residency table's master (no device reads it until it is copied,
    // and every call that copies it has ended with a synchronisation)
    const size_t n = layer.layout.expert_count;
    if (s.has) layer.host_table[s.expert] = layer.host_table[n + s.expert] = 0;
    layer.host_table[expert] = (uint64_t)(uintptr_t)s.gate_up;
    layer.host_table[n + expert] = (uint64_t)(uintptr_t)s.down;
    layer.table_dirty = true;
    c->stats.reads += 2;
    c->stats.bytes_read += layer.layout.gate_up_bytes + layer.layout.down_bytes;
    s.has = true;
    s.expert = expert;
    s.last_used = layer.clock;
    *slot_out = victim;
    return DMHIP_OK;
}

// Records one event after the compute work enqueued so far and makes it the
// `released` event of `count` slots of a layer (their last readers).
int record_release(dmhip_expert_cache *c, size_t layer, const size_t *slots, size_t count) {
    hipEvent_t ev = c->release_events[c->next_release++ % kReleaseEvents];
    DM_HIP(hipEventRecord(ev, c->ctx->stream));
    for (size_t i = 0; i < count; i++) {
        Slot &s = c->layers[layer].slots[slots[i]];
        s.released = ev;
        s.released_recorded = true;
    }
    return DMHIP_OK;
}

dmhip_buf *new_slot_buffer(dmhip_ctx *ctx, size_t bytes) {
    dmhip_buf *b = new dmhip_buf();
    b->ctx = ctx;
    b->device = ctx->device;
    b->len = bytes;
    b->cache_owned = true;
    // 256 spare bytes: vector loads of a row's end may read a few bytes past it
    if (hipMalloc(&b->dev, bytes + 256) != hipSuccess || hipMemset(b->dev, 0, bytes + 256) != hipSuccess) {
        if (b->dev) (void)hipFree(b->dev);
        delete b;
        return nullptr;
    }
    return b;
}

void free_slot_buffer(dmhip_buf *b) {
    if (!b) return;
    if (b->dev) (void)hipFree(b->dev);
    delete b;
}

void destroy(dmhip_expert_cache *c) {
    (void)hipSetDevice(c->device);
    // Wait for the cache's own work: uploads into the slots, the copies out
    // of the staging ring and the compute released last from each slot.
    for (Layer &layer : c->layers)
        for (Slot &s : layer.slots) {
            if (s.uploaded) (void)hipEventSynchronize(s.ready);
            if (s.released_recorded) (void)hipEventSynchronize(s.released);
        }
    for (Staging &e : c->staging)
        if (e.busy) (void)hipEventSynchronize(e.done);
    for (Layer &layer : c->layers)
        for (Slot &s : layer.slots) {
            free_slot_buffer(s.gate_up_buf);
            free_slot_buffer(s.down_buf);
            if (s.ready) (void)hipEventDestroy(s.ready);
        }
    for (TimedUpload &t : c->timed) {
        if (t.pending) (void)hipEventSynchronize(t.end);
        if (t.start) (void)hipEventDestroy(t.start);
        if (t.end) (void)hipEventDestroy(t.end);
    }
    for (hipEvent_t ev : c->release_events)
        if (ev) (void)hipEventDestroy(ev);
    for (Staging &e : c->staging) {
        if (e.host) (void)hipHostFree(e.host);
        if (e.done) (void)hipEventDestroy(e.done);
    }
    // the work area's readers were released above; the context (and its
    // stream) may already be gone
    c->work.stream = nullptr;
    c->work.release();
    if (c->tables) (void)hipFree(c->tables);
    if (c->host_tables) (void)hipHostFree(c->host_tables);
    if (c->host_selection) (void)hipHostFree(c->host_selection);
    delete c;
}

// The shared part of both constructors: slots, events, selection buffer.
int build_cache(dmhip_ctx *ctx, const dmhip_expert_layer_layout *layouts, size_t layer_count,
                size_t slots_per_layer, dmhip_expert_cache *c) {
    c->ctx = ctx;
    c->device = ctx->device;
    c->work.stream = ctx->stream;
    c->layers.resize(layer_count);
    uint64_t resident = 0;
    for (size_t l = 0; l < layer_count; l++) {
        Layer &layer = c->layers[l];
        layer.layout = layouts[l];
        layer.slots.resize(slots_per_layer);
        for (Slot &s : layer.slots) {
            s.gate_up_buf = new_slot_buffer(ctx, layer.layout.gate_up_bytes);
            s.down_buf = new_slot_buffer(ctx, layer.layout.down_bytes);
            if (!s.gate_up_buf || !s.down_buf)
                return fail_alloc(!s.gate_up_buf ? layer.layout.gate_up_bytes : layer.layout.down_bytes);
            s.gate_up = s.gate_up_buf->dev;
            s.down = s.down_buf->dev;
            if (hipEventCreate(&s.ready) != hipSuccess)
                return fail(DMHIP_ERR_COMMAND, "could not create the expert slot events");
            resident += layer.layout.gate_up_bytes + layer.layout.down_bytes;
        }
    }
    c->stats.resident_bytes = resident;
    c->timed.resize(kTimedUploads);
    for (TimedUpload &t : c->timed)
        if (hipEventCreate(&t.start) != hipSuccess || hipEventCreate(&t.end) != hipSuccess)
            return fail(DMHIP_ERR_COMMAND, "could not create the upload timing events");
    c->release_events.assign(kReleaseEvents, nullptr);
    for (hipEvent_t &ev : c->release_events)
        if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
            ev = nullptr;
            return fail(DMHIP_ERR_COMMAND, "could not create the slot release events");
        }
    if (hipHostMalloc((void **)&c->host_selection, kSelectionBytes, hipHostMallocDefault) != hipSuccess) {
        c->host_selection = nullptr;
        return fail_alloc(kSelectionBytes);
    }
    // residency tables (all zero: nothing resident) and the lookup outputs
    size_t entries = 0;
    for (const Layer &layer : c->layers) entries += 2 * layer.layout.expert_count;
    const size_t table_bytes = (entries + 2 * kMaxTopK + 8) * sizeof(uint64_t) + kCombineTickets * sizeof(uint32_t);
    if (hipMalloc((void **)&c->tables, table_bytes) != hipSuccess) {
        c->tables = nullptr;
        return fail_alloc(table_bytes);
    }
    if (hipMemset(c->tables, 0, table_bytes) != hipSuccess)
        return fail(DMHIP_ERR_COMMAND, "could not clear the expert residency tables");
    if (entries && hipHostMalloc((void **)&c->host_tables, entries * sizeof(uint64_t), hipHostMallocDefault) != hipSuccess) {
        c->host_tables = nullptr;
        return fail_alloc(entries * sizeof(uint64_t));
    }
    if (entries) memset(c->host_tables, 0, entries * sizeof(uint64_t));
    size_t at = 0;
    for (Layer &layer : c->layers) {
        layer.table = c->tables + at;
        layer.host_table = c->host_tables + at;
        at += 2 * layer.layout.expert_count;
    }
    c->lookup_gate_up = c->tables + at;
    c->lookup_down = c->lookup_gate_up + kMaxTopK;
    c->lookup_go = (uint32_t *)(c->lookup_down + kMaxTopK);  // 16 words: one per token
    c->combine_tickets = (uint32_t *)(c->lookup_down + kMaxTopK + 8);
    return DMHIP_OK;
}

int check_layouts(const dmhip_expert_layer_layout *layouts, size_t layer_count, size_t slots_per_layer) {
    if (slots_per_layer == 0)
        return fail(DMHIP_ERR_NO_SLOTS, "expert cache requires at least one slot per layer");
    if (layer_count && !layouts) return fail(DMHIP_ERR_INVALID_ARGUMENT, "layouts must not be null");
    for (size_t l = 0; l < layer_count; l++)
        if (layouts[l].gate_up_bytes == 0 || layouts[l].down_bytes == 0) return fail_alloc(0);
    return DMHIP_OK;
}

}  // namespace

extern "C" {

int dmhip_expert_cache_new(dmhip_ctx *ctx, const void *source, size_t source_len,
                           const dmhip_expert_layer_layout *layouts, size_t layer_count,
                           size_t slots_per_layer, dmhip_expert_cache **out) {
    if (!ctx || !out) return fail(DMHIP_ERR_INVALID_ARGUMENT, "context and out must not be null");
    *out = nullptr;
    DM_CHECK_STATUS(check_layouts(layouts, layer_count, slots_per_layer));
    if (layer_count && !source) return fail(DMHIP_ERR_INVALID_ARGUMENT, "source must not be null");
    for (size_t l = 0; l < layer_count; l++) {
        const dmhip_expert_layer_layout &L = layouts[l];
        unsigned __int128 gu_end = (unsigned __int128)L.gate_up_offset +
                                   (unsigned __int128)L.expert_count * L.gate_up_bytes;
        unsigned __int128 dn_end = (unsigned __int128)L.down_offset +
                                   (unsigned __int128)L.expert_count * L.down_bytes;
        if (gu_end > source_len || dn_end > source_len)
            return fail(DMHIP_ERR_INVALID_LAYOUT, "layer %zu expert ranges exceed the %zu-byte source", l,
                        source_len);
    }
    DM_CHECK_STATUS(set_device(ctx));
    dmhip_expert_cache *c = new dmhip_expert_cache();
    c->source = (const uint8_t *)source;
    c->source_len = source_len;
    // Pinned host memory (hipHostMalloc, dmhip_host_alloc_pinned) has a
    // device address: uploads from it run as copy kernels.
    if (source_len) {
        hipPointerAttribute_t attr;
        void *dev = nullptr;
        if (hipPointerGetAttributes(&attr, source) == hipSuccess && attr.type == hipMemoryTypeHost &&
            hipHostGetDevicePointer(&dev, const_cast<void *>(source), 0) == hipSuccess)
            c->source_dev = (const uint8_t *)dev;
        (void)hipGetLastError();  // a pageable source leaves an error behind
    }
    const int st = build_cache(ctx, layouts, layer_count, slots_per_layer, c);
    if (st != DMHIP_OK) {
        destroy(c);
        return st;
    }
    *out = c;
    return DMHIP_OK;
}

int dmhip_expert_cache_new_file(dmhip_ctx *ctx, int fd, const dmhip_expert_layer_layout *layouts,
                                size_t layer_count, size_t slots_per_layer, dmhip_expert_cache **out) {
    if (!ctx || !out) return fail(DMHIP_ERR_INVALID_ARGUMENT, "context and out must not be null");
    *out = nullptr;
    if (fd < 0) return fail(DMHIP_ERR_INVALID_ARGUMENT, "file descriptor %d is not open", fd);
    DM_CHECK_STATUS(check_layouts(layouts, layer_count, slots_per_layer));
    for (size_t l = 0; l < layer_count; l++) {
        const dmhip_expert_layer_layout &L = layouts[l];
        // expert_offset's overflow checks (src/expert.rs:231-239), up front
        const unsigned __int128 gu_end = (unsigned __int128)L.gate_up_offset +
                                         (unsigned __int128)L.expert_count * L.gate_up_bytes;
        const unsigned __int128 dn_end = (unsigned __int128)L.down_offset +
                                         (unsigned __int128)L.expert_count * L.down_bytes;
        if (gu_end > (unsigned __int128)UINT64_MAX || dn_end > (unsigned __int128)UINT64_MAX)
            return fail(DMHIP_ERR_INVALID_LAYOUT, "layer %zu expert file offsets overflow", l);
    }
    DM_CHECK_STATUS(set_device(ctx));
    dmhip_expert_cache *c = new dmhip_expert_cache();
    c->fd = fd;
    int st = build_cache(ctx, layouts, layer_count, slots_per_layer, c);
    size_t entry_bytes = 0;
    for (size_t l = 0; l < layer_count; l++) {
        const size_t b = layouts[l].gate_up_bytes + layouts[l].down_bytes;
        entry_bytes = b > entry_bytes ? b : entry_bytes;
    }
    if (st == DMHIP_OK && layer_count) {
        c->staging.resize(kStagingEntries);
        for (Staging &e : c->staging) {
            if (hipHostMalloc((void **)&e.host, entry_bytes, hipHostMallocDefault) != hipSuccess) {
                e.host = nullptr;
                st = fail_alloc(entry_bytes);
                break;
            }
            void *dev = nullptr;
            if (hipHostGetDevicePointer(&dev, e.host, 0) == hipSuccess) e.host_dev = (uint8_t *)dev;
            (void)hipGetLastError();
            if (hipEventCreateWithFlags(&e.done, hipEventDisableTiming) != hipSuccess) {
                e.done = nullptr;
                st = fail(DMHIP_ERR_COMMAND, "could not create the staging events");
                break;
            }
        }
    }
    if (st != DMHIP_OK) {
        destroy(c);
        return st;
    }
    *out = c;
    return DMHIP_OK;
}

void dmhip_expert_cache_free(dmhip_expert_cache *c) {
    if (c) destroy(c);
}

int dmhip_expert_cache_stats_get(dmhip_expert_cache *c, dmhip_expert_cache_stats *stats) {
    if (!c || !stats) return fail(DMHIP_ERR_INVALID_ARGUMENT, "cache and stats must not be null");
    DM_CHECK_STATUS(set_device(c->ctx));
    account_uploads(c, true);
    *stats = c->stats;
    return DMHIP_OK;
}

size_t dmhip_expert_cache_slots_per_layer(const dmhip_expert_cache *c) {
    return (c && !c->layers.empty()) ? c->layers[0].slots.size() : 0;
}

int dmhip_expert_acquire(dmhip_expert_cache *c, size_t layer, size_t expert,
                         const volatile int *cancelled, size_t *slot, const dmhip_buf **gate_up,
                         const dmhip_buf **down) {
    if (!c || !slot || !gate_up || !down)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "cache and outputs must not be null");
    if (cancelled && *cancelled) return fail(DMHIP_ERR_CANCELLED, "expert loading was cancelled");
    DM_CHECK_STATUS(set_device(c->ctx));
    size_t s;
    DM_CHECK_STATUS(acquire(c, layer, expert, &s));
    if (cancelled && *cancelled) return fail(DMHIP_ERR_CANCELLED, "expert loading was cancelled");
    Slot &slot_ref = c->layers[layer].slots[s];
    slot_ref.pins += 1;
    *slot = s;
    *gate_up = slot_ref.gate_up_buf;
    *down = slot_ref.down_buf;
    return DMHIP_OK;
}

int dmhip_expert_release(dmhip_expert_cache *c, size_t layer, size_t slot) {
    if (!c) return fail(DMHIP_ERR_INVALID_ARGUMENT, "cache must not be null");
    if (layer >= c->layers.size()) return fail_layer(layer, c->layers.size());
    if (slot >= c->layers[layer].slots.size())
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "slot %zu of layer %zu does not exist", slot, layer);
    Slot &s = c->layers[layer].slots[slot];
    if (s.pins == 0) return fail(DMHIP_ERR_INVALID_ARGUMENT, "slot %zu of layer %zu is not acquired", slot, layer);
    DM_CHECK_STATUS(set_device(c->ctx));
    DM_CHECK_STATUS(record_release(c, layer, &slot, 1));
    s.pins -= 1;
    return DMHIP_OK;
}

int dmhip_moe_layer(dmhip_ctx *ctx, dmhip_expert_cache *c, size_t layer, size_t batch,
                    size_t hidden, size_t width, size_t experts, size_t k,
                    const uint16_t *router_bf16, uint32_t gate_up_type, uint32_t down_type,
                    const float *x, float *y, uint32_t *ids, float *probabilities) {
    if (!ctx || !c || !router_bf16 || !x || !y || !ids || !probabilities)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "moe_layer arguments must not be null");
    if (c->ctx != ctx) return fail(DMHIP_ERR_INVALID_ARGUMENT, "the cache belongs to another context");
    if (batch < 1 || batch > 16) return fail(DMHIP_ERR_INVALID_ARGUMENT, "batch %zu is outside 1..=16", batch);
    if (k == 0 || k > experts)
        return fail_top_k(k, experts);
    if (k > kMaxTopK || experts > 16384)
        return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "router with %zu experts, top-%zu exceeds the kernel limits",
                    experts, k);
    if (hidden == 0 || width == 0) return fail_empty("MoE layer");
    if (layer >= c->layers.size())
        return fail_layer(layer, c->layers.size());
    const dmhip_expert_layer_layout &L = c->layers[layer].layout;
    uint64_t gu_row, dn_row;
    if (!row_byte_len(gate_up_type, hidden, &gu_row) || !row_byte_len(down_type, width, &dn_row))
        return fail_element_count(row_byte_len(gate_up_type, hidden, &gu_row) ? down_type : gate_up_type,
                                  row_byte_len(gate_up_type, hidden, &gu_row) ? width : hidden);
    if (L.gate_up_bytes != 2 * width * gu_row || L.down_bytes != hidden * dn_row)
        return fail(DMHIP_ERR_INVALID_LAYOUT,
                    "layer %zu slots hold %zu + %zu bytes; the expert shape needs %llu + %llu", layer,
                    L.gate_up_bytes, L.down_bytes, (unsigned long long)(2 * width * gu_row),
                    (unsigned long long)(hidden * dn_row));
    if (L.expert_count < experts)
        return fail(DMHIP_ERR_INVALID_LAYOUT, "layer %zu holds %zu experts; the router has %zu", layer,
                    L.expert_count, experts);
    DM_CHECK_STATUS(set_device(ctx));

    // Workspace: logits | ids | probs | pos | pair tokens | xg | gate_up | act | expert_out
    const size_t pairs = batch * k;
    const size_t a_logits = 0;
    const size_t a_ids = a_logits + ((batch * experts * 8 + 255) & ~(size_t)255);  // the certified router's (L, rho)
    const size_t a_probs = a_ids + ((pairs * 4 + 255) & ~(size_t)255);
    const size_t a_pos = a_probs + ((pairs * 4 + 255) & ~(size_t)255);
    const size_t a_tok = a_pos + ((pairs * 4 + 255) & ~(size_t)255);
    const size_t a_xg = a_tok + ((pairs * 4 + 255) & ~(size_t)255);
    const size_t a_gu = a_xg + ((pairs * hidden * 4 + 255) & ~(size_t)255);
    const size_t a_act = a_gu + ((pairs * 2 * width * 4 + 255) & ~(size_t)255);
    const size_t a_eo = a_act + ((pairs * width * 4 + 255) & ~(size_t)255);
    const size_t total = a_eo + ((pairs * hidden * 4 + 255) & ~(size_t)255);
    DM_CHECK_STATUS(c->work.ensure(total));
    char *w = (char *)c->work.ptr;
    float *d_logits = (float *)(w + a_logits);
    uint32_t *d_ids = (uint32_t *)(w + a_ids);
    float *d_probs = (float *)(w + a_probs);
    uint32_t *d_pos = (uint32_t *)(w + a_pos);
    uint32_t *d_tok = (uint32_t *)(w + a_tok);
    float *d_xg = (float *)(w + a_xg);
    float *d_gu = (float *)(w + a_gu);
    float *d_act = (float *)(w + a_act);
    float *d_eo = (float *)(w + a_eo);

    // Grouped int8 path: one launch applies every slot of a phase, with the
    // gate/up activation in its epilogue; act and expert-output rows are
    // indexed by pair.  Slot buffers come from hipMalloc (256-byte aligned).
    const uint64_t up_offset = (uint64_t)width * gu_row;
    const bool grouped = qmv8_grouped_supported(gate_up_type, width, hidden, 2) &&
                         qmv8_grouped_supported(down_type, hidden, width, 1) &&
                         up_offset % (gate_up_type == 12 ? 16 : 4) == 0 &&  // 12: Q4_K
                         (uint64_t)pairs * (hidden > width ? hidden : width) < (1ull << 31);

    // 1. Router logits and top-k softmax on the GPU (the certified router:
    //    the exact fold's ids and order).
    uint32_t *sel_ids = (uint32_t *)c->host_selection;
    float *sel_probs = (float *)(c->host_selection + kSelectionPairs * 4);
    uint32_t *sel_bad = (uint32_t *)(c->host_selection + kSelectionPairs * 8);
    volatile uint32_t *sel_go = (volatile uint32_t *)(c->host_selection + kSelectionPairs * 8 + 16 * 4);
    // The previous call has finished (it ends with a synchronisation): the
    // per-token words can be cleared from here.
    memset(sel_bad, 0, 16 * 4);
    Layer &Lay = c->layers[layer];
    // Up to kMaxLookupTokens tokens whose experts are likely resident: each
    // token's last router workgroup looks its selected experts up in the
    // layer's residency table, and the expert launches (one job per token
    // and selection) and the combine are queued right behind the router,
    // reading the slot addresses it found; when a slot is missing (or a
    // token's logits are not finite) they do nothing and the host takes the
    // path below with the selection in hand.  Every earlier upload is
    // already waited for on the compute stream, before the table copy and
    // the router.
    const bool lookup = Lay.try_lookup && grouped && pairs <= kMaxGroupedJobs &&
                        router_takes_lookup((uint32_t)hidden, (uint32_t)experts, (uint32_t)batch, router_bf16, x);
    if (lookup) {
        for (size_t t = 0; t < batch; t++) sel_go[t] = 0;
        DM_CHECK_STATUS(wait_all_ready(c, layer));  // none pending after a completed call
        if (Lay.table_dirty) {
            DM_HIP(hipMemcpyAsync(Lay.table, Lay.host_table, 2 * L.expert_count * sizeof(uint64_t),
                                  hipMemcpyHostToDevice, ctx->stream));
            Lay.table_dirty = false;
        }
        const ExpertLookup el{Lay.table, Lay.table + L.expert_count, c->lookup_gate_up, c->lookup_down,
                              c->lookup_go, (uint32_t *)sel_go};
        DM_HIP(launch_router_top_k(ctx->stream, router_bf16, (uint32_t)hidden, (uint32_t)experts, (uint32_t)k,
                                   (uint32_t)batch, x, d_logits, d_ids, d_probs, BadFlag{ctx->flags + kMoeFlagWord, 1},
                                   sel_ids, sel_probs, ctx->router_tickets, sel_bad, &el, true));
        // job p: selection p % k of token p / k
        std::vector<QmvJob> gu_jobs(pairs), dn_jobs(pairs);
        for (size_t p = 0; p < pairs; p++) {
            gu_jobs[p] = QmvJob{nullptr, 1u, (uint32_t)(p / k * hidden), (uint32_t)(p * width), 0, 0};
            dn_jobs[p] = QmvJob{nullptr, 1u, (uint32_t)(p * width), (uint32_t)(p * hidden), 0, 0};
        }
        const uint32_t tokens = (uint32_t)batch;
        DM_HIP(launch_qmv8_grouped(ctx, gate_up_type, (uint32_t)width, (uint32_t)hidden, 1, up_offset,
                                   gu_jobs.data(), pairs, x, d_act, c->lookup_gate_up, c->lookup_go, nullptr, tokens));
        // the down launch also makes the ordered combine when its split
        // allows (every workgroup holds whole row tiles of every expert)
        const QmvCombine cmb{c->combine_tickets, kCombineTickets, d_probs, y, (uint32_t)k, (uint32_t)hidden};
        if (launch_qmv8_grouped(ctx, down_type, (uint32_t)hidden, (uint32_t)width, 0, 0, dn_jobs.data(), pairs,
                                d_act, d_eo, c->lookup_down, c->lookup_go, &cmb, tokens) != hipSuccess) {
            (void)hipGetLastError();
            DM_HIP(launch_qmv8_grouped(ctx, down_type, (uint32_t)hidden, (uint32_t)width, 0, 0, dn_jobs.data(), pairs,
                                       d_act, d_eo, c->lookup_down, c->lookup_go, nullptr, tokens));
            hipLaunchKernelGGL(moe_combine_pos_kernel, dim3((uint32_t)((batch * hidden + 255) / 256)), dim3(256), 0,
                               ctx->stream, d_eo, nullptr, d_probs, tokens, (uint32_t)k, (uint32_t)hidden, y,
                               c->lookup_go);
            DM_HIP(hipGetLastError());
        }
    } else {
        DM_HIP(launch_router_top_k(ctx->stream, router_bf16, (uint32_t)hidden, (uint32_t)experts,
                                   (uint32_t)k, (uint32_t)batch, x, d_logits, d_ids, d_probs,
                                   BadFlag{ctx->flags + kMoeFlagWord, 1}, sel_ids, sel_probs,
                                   batch <= kRouterTickets ? ctx->router_tickets : nullptr, sel_bad, nullptr, true));
    }
    DM_CHECK_STATUS(stream_wait(ctx));
    // top_k_softmax rejects non-finite logits (src/cpu.rs:240-245); nothing
    // has been acquired yet.
    for (size_t t = 0; t < batch; t++)
        if (sel_bad[t]) return fail_non_finite("top-k softmax");
    memcpy(ids, sel_ids, pairs * 4);
    memcpy(probabilities, sel_probs, pairs * 4);
    bool all_go = lookup;
    for (size_t t = 0; all_go && t < batch; t++) all_go = sel_go[t] != 0;
    if (all_go) {
        // Done on the device: the cache's bookkeeping is the reference's
        // acquire sequence (token by token, selection order), every one a
        // hit.  The work that read the slots has finished (the
        // synchronisation above), so a later upload into them has nothing to
        // wait for.
        size_t slot;
        for (size_t p = 0; p < pairs; p++) DM_CHECK_STATUS(acquire(c, layer, ids[p], &slot));
        for (size_t p = 0; p < pairs; p++)
            for (Slot &sl : Lay.slots)
                if (sl.has && sl.expert == ids[p]) sl.released_recorded = false;
        return DMHIP_OK;
    }
    if (lookup) Lay.try_lookup = false;
    const uint64_t misses_before = c->stats.misses;

    // 2. Acquire in the reference's order (token by token, selection order)
    //    and cut the pairs into phases: a phase ends before an acquire whose
    //    slot is already used by the phase (it would overwrite its bytes).
    std::vector<uint32_t> pos(pairs);
    std::vector<size_t> slot_of(pairs);
    size_t begin = 0;
    // More pairs than slots can need more than one phase: then the compute
    // stream's waits for uploads are deferred to the launches that read the
    // slots, and phases that more acquires follow run as two halves (below).
    // Otherwise (one token's experts, say) each upload is waited for as it
    // is issued and the phase is one launch: measured faster there (the
    // 8-slot one-token layer 0.555 against 0.57 ms with the deferred waits).
    const bool split_phases = pairs > Lay.slots.size();
    // Host sources of the per-phase token lists stay alive until the final
    // synchronisation below.
    std::vector<std::vector<uint32_t>> phase_tokens;
    std::vector<QmvJob> gu_jobs, dn_jobs;
    auto run_phase = [&](size_t p0, size_t p1, bool more) -> int {
        if (p0 == p1) return DMHIP_OK;
        // Group the phase's pairs by slot: sorted order = pair index order
        // within each slot, slots in first-use order.
        std::vector<size_t> order;
        std::vector<size_t> group_start, group_slot;
        std::vector<char> done(p1 - p0, 0);
        for (size_t i = p0; i < p1; i++) {
            if (done[i - p0]) continue;
            group_start.push_back(order.size());
            group_slot.push_back(slot_of[i]);
            for (size_t j = i; j < p1; j++)
                if (!done[j - p0] && slot_of[j] == slot_of[i]) {
                    done[j - p0] = 1;
                    order.push_back(j);
                }
        }
        group_start.push_back(order.size());
        const size_t groups = group_start.size() - 1;
        if (grouped) {
            // When more acquires follow (`more`), two halves of the phase's
            // slots in first-use order, each launched once its own uploads
            // have landed and released after its own launches: the first
            // half computes while the second half's experts are still
            // crossing PCIe, and the next phase's first uploads (into the
            // first half's slots) need not wait for the second half.  The
            // last phase of a call is one launch.  One job per one or two
            // pairs of a slot (two tokens share the slot's weight stream).
            const size_t halves = split_phases && more && groups >= 2 ? 2 : 1;
            for (size_t hv = 0; hv < halves; hv++) {
                const size_t g0 = groups * hv / halves, g1 = groups * (hv + 1) / halves;
                gu_jobs.clear();
                dn_jobs.clear();
                for (size_t g = g0; g < g1; g++) {
                    Slot &s = c->layers[layer].slots[group_slot[g]];
                    DM_CHECK_STATUS(wait_ready(c, s));
                    for (size_t q = group_start[g]; q < group_start[g + 1]; q += 2) {
                        const size_t a = order[q];
                        const bool two = q + 1 < group_start[g + 1];
                        const size_t b = two ? order[q + 1] : a;
                        const int32_t tok_step = (int32_t)(b / k - a / k), pair_step = (int32_t)(b - a);
                        gu_jobs.push_back(QmvJob{s.gate_up, two ? 2u : 1u, (uint32_t)((a / k) * hidden),
                                                 (uint32_t)(a * width), tok_step * (int32_t)hidden,
                                                 pair_step * (int32_t)width});
                        dn_jobs.push_back(QmvJob{s.down, two ? 2u : 1u, (uint32_t)(a * width),
                                                 (uint32_t)(a * hidden), pair_step * (int32_t)width,
                                                 pair_step * (int32_t)hidden});
                    }
                }
                DM_HIP(launch_qmv8_grouped(ctx, gate_up_type, (uint32_t)width, (uint32_t)hidden, 1, up_offset,
                                           gu_jobs.data(), gu_jobs.size(), x, d_act));
                DM_HIP(launch_qmv8_grouped(ctx, down_type, (uint32_t)hidden, (uint32_t)width, 0, 0,
                                           dn_jobs.data(), dn_jobs.size(), d_act, d_eo));
                DM_CHECK_STATUS(record_release(c, layer, group_slot.data() + g0, g1 - g0));
            }
            return DMHIP_OK;
        }
        phase_tokens.emplace_back(order.size());
        std::vector<uint32_t> &tokens = phase_tokens.back();
        for (size_t q = 0; q < order.size(); q++) {
            tokens[q] = (uint32_t)(order[q] / k);
            pos[order[q]] = (uint32_t)(p0 + q);  // row in the expert-output buffer
        }
        DM_HIP(hipMemcpyAsync(d_tok, tokens.data(), tokens.size() * 4, hipMemcpyHostToDevice, ctx->stream));
        hipLaunchKernelGGL(gather_rows_kernel, dim3(64), dim3(256), 0, ctx->stream, x, d_tok,
                           (uint32_t)tokens.size(), (uint32_t)hidden, d_xg + p0 * hidden);
        DM_HIP(hipGetLastError());
        for (size_t g = 0; g < groups; g++) {
            const size_t q0 = group_start[g], q1 = group_start[g + 1];
            Slot &s = c->layers[layer].slots[group_slot[g]];
            DM_CHECK_STATUS(wait_ready(c, s));
            const size_t cnt = q1 - q0;
            const float *xin = d_xg + (p0 + q0) * hidden;
            float *gu = d_gu + (p0 + q0) * 2 * width;
            DM_CHECK_STATUS(enqueue_matvec(ctx, gate_up_type, 2 * width, hidden, s.gate_up, cnt, xin, gu));
            DM_HIP(launch_silu_mul_glm_pairs(ctx->stream, gu, (uint32_t)cnt, (uint32_t)width,
                                             d_act + (p0 + q0) * width));
            DM_CHECK_STATUS(enqueue_matvec(ctx, down_type, hidden, width, s.down, cnt,
                                           d_act + (p0 + q0) * width, d_eo + (p0 + q0) * hidden));
        }
        return record_release(c, layer, group_slot.data(), group_slot.size());
    };
    // A failure after slots of the open phase were acquired still records
    // their release after whatever was enqueued, so that a later upload into
    // one of them waits for that work.
    auto fail_phase = [&](size_t p0, size_t p1, int status) -> int {
        // later work on the compute stream stays behind every upload issued
        (void)wait_all_ready(c, layer);
        if (p1 > p0) (void)record_release(c, layer, slot_of.data() + p0, p1 - p0);
        return status;
    };
    for (size_t p = 0; p < pairs; p++) {
        // Would this acquire evict a slot the open phase still needs?  Check
        // with the reference's victim rule before touching any state.
        Layer &Ly = c->layers[layer];
        const size_t e = ids[p];
        bool hit = false;
        for (const Slot &s : Ly.slots)
            if (s.has && s.expert == e) hit = true;
        if (!hit) {
            size_t victim = SIZE_MAX;
            for (size_t i = 0; i < Ly.slots.size(); i++) {
                const Slot &s = Ly.slots[i];
                if (s.pins) continue;
                if (victim == SIZE_MAX) { victim = i; continue; }
                const Slot &v = Ly.slots[victim];
                if (s.has < v.has || (s.has == v.has && s.last_used < v.last_used)) victim = i;
            }
            bool used = false;
            for (size_t q = begin; q < p; q++)
                if (slot_of[q] == victim) used = true;
            if (used) {
                const int st = run_phase(begin, p, true);
                if (st != DMHIP_OK) return fail_phase(begin, p, st);
                begin = p;
            }
        }
        const int st = acquire(c, layer, e, &slot_of[p], !split_phases);
        if (st != DMHIP_OK) return fail_phase(begin, p, st);
    }
    {
        const int st = run_phase(begin, pairs, false);
        if (st != DMHIP_OK) return fail_phase(begin, pairs, st);
    }

    // 3. Ordered combine and copy out.
    if (!grouped) DM_HIP(hipMemcpyAsync(d_pos, pos.data(), pairs * 4, hipMemcpyHostToDevice, ctx->stream));
    hipLaunchKernelGGL(moe_combine_pos_kernel, dim3((uint32_t)((batch * hidden + 255) / 256)), dim3(256), 0,
                       ctx->stream, d_eo, grouped ? nullptr : d_pos, d_probs, (uint32_t)batch, (uint32_t)k,
                       (uint32_t)hidden, y, nullptr);
    DM_HIP(hipGetLastError());
    DM_CHECK_STATUS(stream_wait(ctx));
    // a call whose experts were all resident lets the next one-token call
    // try the device-side lookup again
    if (c->stats.misses == misses_before) Lay.try_lookup = true;
    return DMHIP_OK;
}

}  // extern "C"
