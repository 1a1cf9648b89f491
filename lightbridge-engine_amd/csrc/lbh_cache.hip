// lbh_cache.hip — the HBM expert cache behind lbh_expert_cache_* (declared in
// include/lightbridge_hip.h).
//
// The reference keeps routed experts' compressed bytes in a byte-ceiling cache
// (CompressedCache, crates/bridge-cache/src/lib.rs) keyed by (layer, expert),
// filled from an expert-major sidecar record (crates/bridge-format/src/lib.rs:
// 63-100, 309-329) through a loader closure (crates/bridge-runtime/src/
// hy3_scalar.rs:575-604).  Here the entries live in HBM, already in the
// backend's device layout, so a hit costs nothing but a pin:
//
//   * one slab of fixed-size slots (every entry of a cache has the same shape);
//   * a miss reserves a slot under the cache's byte ceiling (evicting the
//     least recently used unpinned entries, lib.rs:560-595), calls the loader,
//     which writes the tight record (gate | up | down GGML bytes) straight into
//     one of two pinned staging buffers, checks every f16 d / dmin on the host,
//     then DMAs the record and repacks it into the slot on a copy stream of its
//     own; an event marks the upload so the compute stream waits for it only
//     when it reads the entry;
//   * releasing a lease records an event on the context's stream, and a slot
//     is refilled only after the copy stream has waited for it, so an upload
//     never overwrites planes a queued kernel still reads;
//   * admission, pins, ephemeral entries and the counters follow
//     get_or_try_insert / CacheLease::drop (lib.rs:129-265, 419-443).
#include <hip/hip_runtime.h>

#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <new>
#include <unordered_map>
#include <vector>

#include "lbh_cache.h"
#include "lbh_host.h"

using namespace lbh;

namespace {

constexpr int N_STAGE = 2;                 // pinned staging buffers: fill one while the other is DMA'd
constexpr int32_t LEASE_LIVE = 0x4c454153;  // lbh_expert_lease::reserved of a pinned lease

enum class State { Loading, Ready };

struct Entry {
    State state;
    int slot;
    size_t pins;
    uint64_t last_used;
    bool resident;
};

struct Slot {
    uint8_t *base;
    hipEvent_t ready;      // recorded on the copy stream after the entry's upload
    hipEvent_t last_use;   // recorded on the reading stream by every forward that reads the slot
    hipStream_t use_stream;  // the stream last_use was last recorded on
    bool used;             // last_use has been recorded at least once
};

struct Stage {
    uint8_t *host;         // pinned
    uint8_t *dev;
    hipEvent_t done;       // the DMA out of `host` has finished
    bool pending;
};

uint64_t key_of(uint32_t layer, uint32_t expert) { return ((uint64_t)layer << 32) | expert; }
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

struct lbh_expert_cache {
    lbh_ctx *ctx;
    int device;
    uint64_t capacity, admit_after;
    CacheShape shape;
    size_t bytes_gu, bytes_d, entry_bytes;   // tight record: gate | up | down
    size_t off_up, off_down, slot_stride;    // device slot: 256-byte aligned planes
    uint8_t *slab = nullptr;
    std::vector<Slot> slots;
    std::vector<int> free_slots;
    std::unordered_map<uint64_t, Entry> entries;
    std::unordered_map<uint64_t, uint64_t> heat;
    uint64_t used = 0, reserved = 0, tick = 0, hits = 0, misses = 0, loads = 0, waits = 0, evictions = 0;
    uint64_t uploaded = 0;
    std::mutex mu;
    std::condition_variable changed;
    hipStream_t copy = nullptr;
    Stage stage[N_STAGE] = {};
    int next_stage = 0;
    std::mutex stage_mu;
};

namespace {

void free_cache(lbh_expert_cache *c) {
    if (!c) return;
    DeviceGuard g(c->device);
    if (c->copy) (void)hipStreamSynchronize(c->copy);
    if (c->ctx) (void)hipStreamSynchronize(c->ctx->stream);
    for (Slot &s : c->slots) {
        if (s.ready) (void)hipEventDestroy(s.ready);
        if (s.last_use) (void)hipEventDestroy(s.last_use);
    }
    for (Stage &s : c->stage) {
        if (s.host) (void)hipHostFree(s.host);
        if (s.dev) (void)hipFree(s.dev);
        if (s.done) (void)hipEventDestroy(s.done);
    }
    if (c->slab) (void)hipFree(c->slab);
    if (c->copy) (void)hipStreamDestroy(c->copy);
    delete c;
}

// reserve_capacity (lib.rs:560-595): evict least recently used unpinned ready
// entries until the request fits under the ceiling.  Caller holds mu.
lbh_status reserve(lbh_expert_cache *c, lbh_error *err) {
    for (;;) {
        if (c->used + c->reserved + c->entry_bytes <= c->capacity) return LBH_OK;
        uint64_t victim = 0, oldest = UINT64_MAX;
        bool found = false;
        for (const auto &kv : c->entries) {
            const Entry &e = kv.second;
            if (e.state == State::Ready && e.pins == 0 && e.last_used < oldest) {
                oldest = e.last_used;
                victim = kv.first;
                found = true;
            }
        }
        if (!found) return fail(err, (lbh_status)LBH_CACHE_CAPACITY_PINNED, 0, 0, c->entry_bytes);
        c->free_slots.push_back(c->entries[victim].slot);
        c->entries.erase(victim);
        c->used -= c->entry_bytes;
        c->evictions += 1;
    }
}

// First non-finite f16 d (then dmin, for K-quants) in block order of one
// matrix of the record (validate_scales, crates/bridge-quant-layout/src/k_quants.rs:178-208):
// NonFiniteScale { ty, block_index, field, bits } with the row and the segment.
lbh_status check_scales(int ty, const uint8_t *p, long long units, int nb, int segment, lbh_error *err) {
    const size_t bb = (size_t)layout_of(ty).block_bytes;
    const bool kq = ty == LBH_Q4_K || ty == LBH_Q5_K;
    for (long long u = 0; u < units; ++u) {
        const uint8_t *b = p + (size_t)u * bb;
        for (int f = 0; f < (kq ? 2 : 1); ++f) {
            const uint32_t h = b[2 * f] | ((uint32_t)b[2 * f + 1] << 8);
            if ((h & 0x7c00u) == 0x7c00u)
                return fail(err, LBH_NON_FINITE_SCALE, ty, (uint64_t)(u % nb), (uint64_t)segment, 0, h, (uint32_t)f,
                            (uint64_t)(u / nb));
        }
    }
    return LBH_OK;
}

// Loader call, host checks and the upload of one record into `slot`.  No
// cache lock is held (the loader may be slow); the staging lock serializes
// uploads, which share one PCIe link anyway.
lbh_status load_into(lbh_expert_cache *c, int slot, uint32_t layer, uint32_t expert, lbh_expert_loader loader,
                     void *user, lbh_error *err) {
    std::lock_guard<std::mutex> sg(c->stage_mu);
    DeviceGuard g(c->device);
    Stage &s = c->stage[c->next_stage];
    c->next_stage = (c->next_stage + 1) % N_STAGE;
    if (s.pending) {
        HIP_TRY(hipEventSynchronize(s.done));
        s.pending = false;
    }
    size_t written = 0;
    const int32_t code = loader(user, layer, expert, s.host, c->entry_bytes, &written);
    if (code != 0) return fail(err, (lbh_status)LBH_CACHE_LOADER_FAILED, 0, expert, 0, (uint64_t)(int64_t)code);
    if (written != c->entry_bytes)
        return fail(err, (lbh_status)LBH_CACHE_LOADED_SIZE_MISMATCH, 0, expert, c->entry_bytes, written);
    const CacheShape &sh = c->shape;
    const long long ugu = sh.views.gate.units, ud = sh.views.down.units;
    lbh_status st = check_scales(sh.type_gate_up, s.host, ugu, sh.views.gate.nb, 0, err);
    if (st == LBH_OK) st = check_scales(sh.type_gate_up, s.host + c->bytes_gu, ugu, sh.views.up.nb, 1, err);
    if (st == LBH_OK) st = check_scales(sh.type_down, s.host + 2 * c->bytes_gu, ud, sh.views.down.nb, 2, err);
    if (st != LBH_OK) return st;
    Slot &sl = c->slots[slot];
    bool wait_last_use;
    {
        std::lock_guard<std::mutex> lk(c->mu);
        wait_last_use = sl.used;
    }
    if (wait_last_use) HIP_TRY(hipStreamWaitEvent(c->copy, sl.last_use, 0));
    HIP_TRY(hipMemcpyAsync(s.dev, s.host, c->entry_bytes, hipMemcpyHostToDevice, c->copy));
    HIP_TRY(launch_repack(sh.type_gate_up, s.dev, sl.base, ugu, 1, c->copy));
    HIP_TRY(launch_repack(sh.type_gate_up, s.dev + c->bytes_gu, sl.base + c->off_up, ugu, 1, c->copy));
    HIP_TRY(launch_repack(sh.type_down, s.dev + 2 * c->bytes_gu, sl.base + c->off_down, ud, 1, c->copy));
    HIP_TRY(hipEventRecord(s.done, c->copy));
    s.pending = true;
    HIP_TRY(hipEventRecord(sl.ready, c->copy));
    return LBH_OK;
}

void fill_lease(lbh_expert_lease *out, uint32_t layer, uint32_t expert, int slot) {
    out->layer = layer;
    out->expert = expert;
    out->slot = slot;
    out->reserved = LEASE_LIVE;
}

MatView shape_view(int ty, size_t rows, size_t k) {
    MatView v{};
    v.planes = nullptr;
    v.type = ty;
    v.nb = (int32_t)(k / 256);
    v.rows = (int32_t)rows;
    v.units = (long long)(rows * (k / 256));
    v.bytes = (long long)(rows * (k / 256) * (size_t)layout_of(ty).block_bytes);
    return v;
}

}  // namespace

namespace lbh {

bool cache_shape(const lbh_expert_cache *c, CacheShape *out) {
    if (!c || !out) return false;
    *out = c->shape;
    return true;
}

bool cache_lease_planes(lbh_expert_cache *c, const lbh_expert_lease *lease, const uint8_t *planes[3],
                        hipEvent_t *ready) {
    if (!c || !lease || lease->reserved != LEASE_LIVE) return false;
    std::lock_guard<std::mutex> lk(c->mu);
    const auto it = c->entries.find(key_of(lease->layer, lease->expert));
    if (it == c->entries.end() || it->second.state != State::Ready || it->second.slot != lease->slot ||
        it->second.pins == 0)
        return false;
    const Slot &s = c->slots[lease->slot];
    planes[0] = s.base;
    planes[1] = s.base + c->off_up;
    planes[2] = s.base + c->off_down;
    *ready = s.ready;
    return true;
}

bool cache_note_use(lbh_expert_cache *c, const lbh_expert_lease *lease, hipStream_t stream) {
    if (!c || !lease || lease->reserved != LEASE_LIVE) return false;
    std::lock_guard<std::mutex> lk(c->mu);
    const auto it = c->entries.find(key_of(lease->layer, lease->expert));
    if (it == c->entries.end() || it->second.state != State::Ready || it->second.slot != lease->slot ||
        it->second.pins == 0)
        return false;
    Slot &s = c->slots[lease->slot];
    DeviceGuard g(c->device);
    // One event per slot: a use on a second stream first waits for the use
    // recorded on the other one, so the new record covers both readers.
    if (s.used && s.use_stream != stream && hipStreamWaitEvent(stream, s.last_use, 0) != hipSuccess) return false;
    if (hipEventRecord(s.last_use, stream) != hipSuccess) return false;
    s.used = true;
    s.use_stream = stream;
    return true;
}

}  // namespace lbh

extern "C" {

lbh_status lbh_expert_cache_create(lbh_ctx *ctx, const lbh_expert_cache_config *config, uint32_t hidden, uint32_t ffn,
                                   int32_t gate_up_type, int32_t down_type, lbh_expert_cache **out, lbh_error *err) {
    if (!ctx || !config || !out) return fail(err, LBH_NULL_ARGUMENT);
    *out = nullptr;
    // CacheConfig::validate (lib.rs:19-29)
    if (config->capacity_bytes == 0) return fail(err, (lbh_status)LBH_CACHE_ZERO_CAPACITY);
    if (config->admit_after_requests == 0) return fail(err, (lbh_status)LBH_CACHE_ZERO_ADMISSION_THRESHOLD);
    const auto dot_type = [](int t) { return t == LBH_IQ2_S || t == LBH_IQ3_S || t == LBH_Q4_K || t == LBH_Q5_K; };
    if (!dot_type(gate_up_type)) return fail(err, LBH_UNSUPPORTED_TYPE, gate_up_type);
    if (!dot_type(down_type)) return fail(err, LBH_UNSUPPORTED_TYPE, down_type);
    if (hidden == 0 || ffn == 0) return fail(err, LBH_ZERO_LOGICAL_ELEMENTS);
    if (hidden % 256 || ffn % 256) return fail(err, LBH_LOGICAL_ELEMENTS_NOT_DIVISIBLE, 0, 0, 256, hidden % 256 ? hidden : ffn);
    if (hidden / 256 > 64 || ffn / 256 > 64) return fail(err, LBH_UNSUPPORTED_SHAPE, 0, 0, 64 * 256);

    lbh_expert_cache *c = new (std::nothrow) lbh_expert_cache();
    if (!c) return fail(err, LBH_HIP_ERROR);
    c->ctx = ctx;
    c->device = ctx->device;
    c->capacity = config->capacity_bytes;
    c->admit_after = config->admit_after_requests;
    c->shape.views.gate = shape_view(gate_up_type, ffn, hidden);
    c->shape.views.up = c->shape.views.gate;
    c->shape.views.down = shape_view(down_type, hidden, ffn);
    c->shape.hidden = hidden;
    c->shape.ffn = ffn;
    c->shape.type_gate_up = gate_up_type;
    c->shape.type_down = down_type;
    c->shape.device = ctx->device;
    c->bytes_gu = (size_t)c->shape.views.gate.bytes;
    c->bytes_d = (size_t)c->shape.views.down.bytes;
    c->entry_bytes = 2 * c->bytes_gu + c->bytes_d;
    c->off_up = align256(c->bytes_gu);
    c->off_down = c->off_up + align256(c->bytes_gu);
    c->slot_stride = align256(c->off_down + c->bytes_d);
    // EntryTooLarge (lib.rs:139-145): every entry has this size, so no slot at all.
    if (c->entry_bytes > c->capacity) {
        const uint64_t need = c->entry_bytes;
        delete c;
        return fail(err, (lbh_status)LBH_CACHE_ENTRY_TOO_LARGE, 0, 0, need, config->capacity_bytes);
    }
    const size_t n_slots = (size_t)(c->capacity / c->entry_bytes);
    DeviceGuard g(c->device);
    hipError_t e = hipMalloc(&c->slab, n_slots * c->slot_stride);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking);
    c->slots.resize(n_slots);
    for (size_t i = 0; i < n_slots && e == hipSuccess; ++i) {
        Slot &s = c->slots[i];
        s.base = c->slab + i * c->slot_stride;
        s.used = false;
        s.ready = s.last_use = nullptr;
        s.use_stream = nullptr;
        e = hipEventCreateWithFlags(&s.ready, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&s.last_use, hipEventDisableTiming);
    }
    for (int i = 0; i < N_STAGE && e == hipSuccess; ++i) {
        e = hipHostMalloc(&c->stage[i].host, c->entry_bytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipMalloc(&c->stage[i].dev, c->entry_bytes);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&c->stage[i].done, hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        free_cache(c);
        return hip_fail(err, e);
    }
    c->free_slots.reserve(n_slots);
    for (size_t i = n_slots; i-- > 0;) c->free_slots.push_back((int)i);
    *out = c;
    return ok(err);
}

lbh_status lbh_expert_cache_destroy(lbh_expert_cache *cache) {
    if (!cache) return LBH_NULL_ARGUMENT;
    free_cache(cache);
    return LBH_OK;
}

uint64_t lbh_expert_cache_entry_bytes(const lbh_expert_cache *cache) { return cache ? cache->entry_bytes : 0; }

lbh_status lbh_expert_cache_get_or_load(lbh_expert_cache *c, uint32_t layer, uint32_t expert, lbh_expert_loader loader,
                                        void *user, lbh_expert_lease *out, lbh_error *err) {
    if (!c || !out) return fail(err, LBH_NULL_ARGUMENT);
    const uint64_t key = key_of(layer, expert);
    std::unique_lock<std::mutex> lk(c->mu);
    for (;;) {
        const uint64_t tick = ++c->tick;
        auto it = c->entries.find(key);
        if (it != c->entries.end()) {
            if (it->second.state == State::Ready) {   // hit (lib.rs:152-170)
                it->second.pins += 1;
                it->second.last_used = tick;
                c->hits += 1;
                fill_lease(out, layer, expert, it->second.slot);
                return ok(err);
            }
            c->waits += 1;                            // another caller is loading it (lib.rs:171-180)
            c->changed.wait(lk);
            continue;
        }
        if (!loader) return fail(err, LBH_NULL_ARGUMENT);
        // miss: heat, admission, reservation (lib.rs:181-210)
        c->misses += 1;
        const uint64_t requests = ++c->heat[key];
        const bool resident = requests >= c->admit_after;
        lbh_status st = reserve(c, err);
        if (st != LBH_OK) return st;
        c->reserved += c->entry_bytes;
        c->loads += 1;
        const int slot = c->free_slots.back();
        c->free_slots.pop_back();
        c->entries[key] = Entry{State::Loading, slot, 0, tick, resident};
        lk.unlock();
        st = load_into(c, slot, layer, expert, loader, user, err);
        lk.lock();
        c->reserved -= c->entry_bytes;
        if (st != LBH_OK) {   // LoadReservation::drop (lib.rs:446-472): nothing inserted
            c->entries.erase(key);
            c->free_slots.push_back(slot);
            c->changed.notify_all();
            return st;
        }
        c->used += c->entry_bytes;
        c->uploaded += c->entry_bytes;
        c->entries[key] = Entry{State::Ready, slot, 1, ++c->tick, resident};
        c->changed.notify_all();
        fill_lease(out, layer, expert, slot);
        return ok(err);
    }
}

lbh_status lbh_expert_cache_get(lbh_expert_cache *c, uint32_t layer, uint32_t expert, lbh_expert_lease *out,
                                int32_t *found) {
    if (!c || !out || !found) return LBH_NULL_ARGUMENT;
    std::lock_guard<std::mutex> lk(c->mu);
    const uint64_t tick = ++c->tick;
    *found = 0;
    auto it = c->entries.find(key_of(layer, expert));
    if (it == c->entries.end()) {
        c->misses += 1;
        return LBH_OK;
    }
    if (it->second.state != State::Ready) return LBH_OK;
    it->second.pins += 1;
    it->second.last_used = tick;
    c->hits += 1;
    fill_lease(out, layer, expert, it->second.slot);
    *found = 1;
    return LBH_OK;
}

lbh_status lbh_expert_cache_release(lbh_expert_cache *c, lbh_expert_lease *lease) {
    if (!c || !lease) return LBH_NULL_ARGUMENT;
    if (lease->reserved != LEASE_LIVE) return LBH_INVALID_PARAMETER;
    std::lock_guard<std::mutex> lk(c->mu);
    auto it = c->entries.find(key_of(lease->layer, lease->expert));
    if (it == c->entries.end() || it->second.state != State::Ready || it->second.slot != lease->slot ||
        it->second.pins == 0)
        return LBH_INVALID_PARAMETER;
    // Every kernel that reads the slot recorded its use when it was enqueued
    // (cache_note_use, on the stream it runs on), so a later upload into the
    // slot waits for it whichever stream it was: nothing to record here.
    it->second.pins -= 1;
    if (it->second.pins == 0 && !it->second.resident) {   // ephemeral entry (lib.rs:429-440)
        c->free_slots.push_back(it->second.slot);
        c->entries.erase(it);
        c->used -= c->entry_bytes;
    }
    lease->reserved = 0;
    c->changed.notify_all();
    return LBH_OK;
}

lbh_status lbh_expert_cache_stats(lbh_expert_cache *c, lbh_cache_stats *out) {
    if (!c || !out) return LBH_NULL_ARGUMENT;
    std::lock_guard<std::mutex> lk(c->mu);
    std::memset(out, 0, sizeof(*out));
    for (const auto &kv : c->entries) {
        const Entry &e = kv.second;
        if (e.state == State::Loading) {
            out->loading_entries += 1;
        } else {
            if (e.pins > 0) out->pinned_entries += 1;
            if (e.resident) out->resident_entries += 1;
        }
    }
    out->capacity_bytes = c->capacity;
    out->used_bytes = c->used;
    out->reserved_bytes = c->reserved;
    out->heat_entries = c->heat.size();
    out->hits = c->hits;
    out->misses = c->misses;
    out->loads = c->loads;
    out->waits = c->waits;
    out->evictions = c->evictions;
    out->entry_bytes = c->entry_bytes;
    out->slots = c->slots.size();
    out->bytes_uploaded = c->uploaded;
    return LBH_OK;
}

lbh_status lbh_expert_cache_clear_unpinned(lbh_expert_cache *c, uint64_t *removed) {
    if (!c) return LBH_NULL_ARGUMENT;
    std::lock_guard<std::mutex> lk(c->mu);
    uint64_t n = 0;
    for (auto it = c->entries.begin(); it != c->entries.end();) {
        if (it->second.state == State::Ready && it->second.pins == 0) {
            c->free_slots.push_back(it->second.slot);
            c->used -= c->entry_bytes;
            it = c->entries.erase(it);
            n += 1;
        } else {
            ++it;
        }
    }
    if (removed) *removed = n;
    return LBH_OK;
}

lbh_status lbh_expert_cache_read_record(lbh_expert_cache *c, const lbh_expert_lease *lease, void *host_out,
                                        size_t bytes, lbh_error *err) {
    if (!c || !lease || !host_out) return fail(err, LBH_NULL_ARGUMENT);
    if (bytes != c->entry_bytes) return fail(err, LBH_ENCODED_LENGTH_MISMATCH, 0, 0, c->entry_bytes, bytes);
    const uint8_t *planes[3];
    hipEvent_t ready;
    if (!cache_lease_planes(c, lease, planes, &ready)) return fail(err, LBH_INVALID_PARAMETER);
    DeviceGuard g(c->device);
    hipStream_t s = c->ctx->stream;
    uint8_t *tmp = nullptr;
    HIP_TRY(hipMalloc(&tmp, c->entry_bytes));
    const CacheShape &sh = c->shape;
    hipError_t e = hipStreamWaitEvent(s, ready, 0);
    if (e == hipSuccess) e = launch_repack(sh.type_gate_up, planes[0], tmp, sh.views.gate.units, 0, s);
    if (e == hipSuccess) e = launch_repack(sh.type_gate_up, planes[1], tmp + c->bytes_gu, sh.views.up.units, 0, s);
    if (e == hipSuccess) e = launch_repack(sh.type_down, planes[2], tmp + 2 * c->bytes_gu, sh.views.down.units, 0, s);
    if (e == hipSuccess) e = hipMemcpyAsync(host_out, tmp, c->entry_bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail(err, e);
    return ok(err);
}

}  // extern "C"
