// cache.hip -- experts kept in host memory behind a fixed set of HBM slots.
//
// The policy is the reference's ExpertCache (spm-granite-moe/src/
// expert_cache.rs:20-90): every lookup ages the cache; a hit refreshes the
// entry's age; a miss counts an observation of the expert, and on its second
// observation the expert is admitted, room being made by evicting the least
// recently used resident expert.  Layer-aware eviction (tools/llama-logits/
// mmid-cache.hpp:134-173) prefers a victim of the incoming expert's own layer,
// least recently used among those.  An expert not admitted is streamed
// through: uploaded into a transient slot for this one use.  The experts of
// the call in progress are never evicted by it (mmid-cache's `active`), since
// the call's kernels read them after every upload has been issued.
//
// Device side: n_slots resident and n_transient transient slots of
// expert_bytes each, one HBM allocation.  Uploads are hipMemcpyAsync from the
// caller's host bytes (pinned: emu_host_alloc) on the context stream, so the
// kernels launched after them see the bytes, and a later upload into a slot
// cannot overtake an earlier kernel that reads it.
#include "internal.hpp"

#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <unordered_map>
#include <vector>

int emu_moe_ffn_table(emu_ctx *ctx, const emu_moe_desc *d, const uint8_t *const *d_table, const float *d_x,
                      uint32_t n_tok, const int32_t *d_ids, const float *d_weights, void *d_workspace,
                      size_t workspace_bytes, float *d_out);

namespace {

// Lookup outcomes.
enum { kHit = 0, kAdmitted = 1, kStreamed = 2 };

struct CachePolicy {
    struct Entry {
        uint32_t seen = 0;
        int32_t slot = -1;
        uint64_t age = 0;
        bool active = false;
    };
    uint32_t n_slots = 0;
    bool layer_aware = false;
    uint64_t age = 0;
    std::unordered_map<uint64_t, Entry> entries;
    std::vector<uint64_t> owner; // slot -> key + 1 (0: free)
    std::vector<uint64_t> active;
    uint64_t hits = 0, misses = 0, loads = 0, evictions = 0, streamed = 0;

    static uint64_t key(uint32_t layer, uint32_t expert) { return ((uint64_t)layer << 32) | expert; }

    void init(uint32_t slots, bool aware)
    {
        n_slots = slots;
        layer_aware = aware;
        owner.assign(slots, 0);
    }

    // Every expert of a call is in use from the call's start to its end
    // (mmid-cache.hpp's acquire/release): none of them is a victim for
    // another of the call's admissions, whatever order they are looked up in.
    void begin_call(uint32_t layer, const uint32_t *experts, size_t n)
    {
        for (size_t i = 0; i < n; ++i) {
            const uint64_t k = key(layer, experts[i]);
            Entry &en = entries[k];
            if (!en.active) {
                en.active = true;
                active.push_back(k);
            }
        }
    }

    // expert_cache.rs:36-72 (get) with the slot it lands in (-1: streamed).
    int access(uint32_t layer, uint32_t expert, int32_t *slot)
    {
        const uint64_t k = key(layer, expert);
        ++age;
        Entry &en = entries[k];
        if (en.slot >= 0) {
            ++hits;
            en.age = age;
            *slot = en.slot;
            return kHit;
        }
        ++misses;
        ++en.seen;
        if (en.seen >= 2) {
            int32_t s = free_slot();
            if (s < 0) s = evict(layer);
            if (s >= 0) {
                en.slot = s;
                en.age = age;
                owner[s] = k + 1;
                ++loads;
                *slot = s;
                return kAdmitted;
            }
        }
        ++streamed;
        *slot = -1;
        return kStreamed;
    }

    int32_t free_slot() const
    {
        for (uint32_t s = 0; s < n_slots; ++s)
            if (owner[s] == 0) return (int32_t)s;
        return -1;
    }

    // expert_cache.rs:74-90 (evict: least age), mmid-cache.hpp:134-160
    // (layer-aware: the incoming expert's layer first).  Experts of the call
    // in progress are skipped; -1 when every resident expert is in use.
    int32_t evict(uint32_t layer)
    {
        int32_t best = -1;
        uint64_t best_age = 0;
        bool best_same = false;
        for (uint32_t s = 0; s < n_slots; ++s) {
            if (!owner[s]) continue;
            const uint64_t k = owner[s] - 1;
            const Entry &c = entries[k];
            if (c.active) continue;
            const bool same = (uint32_t)(k >> 32) == layer;
            const bool better = best < 0 || (!layer_aware && c.age < best_age) ||
                                (layer_aware && ((same && !best_same) || (same == best_same && c.age < best_age)));
            if (better) {
                best = (int32_t)s;
                best_age = c.age;
                best_same = same;
            }
        }
        if (best >= 0) {
            entries[owner[best] - 1].slot = -1;
            owner[best] = 0;
            ++evictions;
        }
        return best;
    }

    void end_call()
    {
        for (uint64_t k : active) entries[k].active = false;
        active.clear();
    }

    uint32_t resident() const
    {
        uint32_t n = 0;
        for (uint64_t o : owner) n += o != 0;
        return n;
    }
};

constexpr int kTableRing = 8;

// ---------------------------------------------------------- device policy --
// The same policy run on the device, per mixture-of-experts layer of a
// decode step (emu_session_attach_expert_cache), over the routes the step's
// gate wrote: no host round trip, so the cached step is captured into the
// step's graph like the resident one.  An admission is copied from its pinned
// host bytes into its HBM slot by a copy kernel right after the plan, and the
// layer's experts read it from there; a miss that is not admitted is read by
// the expert kernels straight from its host bytes (zero-copy over PCIe,
// overlapped with the resident experts' arithmetic in the same launch).  So
// every missed byte crosses PCIe once.
struct DevSlot {
    uint64_t owner; // key + 1 (0: free)
    uint64_t age;   // the owning expert's age
};
struct DevEntry {
    int32_t seen, slot;
    uint64_t age;
};
struct DevState {
    uint64_t age, hits, misses, loads, evictions, streamed, bytes_uploaded, bytes_streamed;
};
struct CopyJob {
    const uint8_t *src;
    uint8_t *dst;
};

constexpr int kPlanThreads = 256;
constexpr int kMaxDevSlots = 2048;   // slot metadata held in LDS by the plan kernel
constexpr int kMaxCallExperts = 64;  // 8 tokens x 8 routes
constexpr int kMaxDevExperts = 256;  // the call's experts as a 256-bit mask
constexpr size_t kCopyChunk = 64 << 10;

struct PlanArgs {
    DevEntry *entries;         // [layers][E]
    DevSlot *meta;             // [n_slots]
    DevState *state;
    CopyJob *jobs;             // [layers][kMaxCallExperts]
    uint32_t *njobs;           // [layers]
    const uint8_t *const *src; // [layers][E] device addresses of the pinned host bytes
    uint8_t *slots;
    size_t stride;             // bytes between slots
    size_t expert_bytes;
    const uint8_t **tables;    // [layers][E]
    const int32_t *ids;        // the layer's routes
    int nk, layer, E, n_slots, layer_aware;
};

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v)
{
    for (int o = 32; o >= 1; o >>= 1) {
        const uint64_t w = __shfl_xor(v, o, 64);
        v = w < v ? w : v;
    }
    return v;
}

// One workgroup.  The call's distinct experts, ascending (the order the host
// policy looks them up in), are marked in use first; then thread 0 ages,
// hits, misses and admits one after another while every thread takes part
// in each admission's victim search over the slots held in LDS: the least
// key of (free slot: its index) < (occupied: 1, layer-aware and another
// layer, the owner's age, index) -- the lowest free slot, else the least
// recently used (own layer first when layer-aware), the lowest index among
// equals, experts of the call never.  Victim choice and counters are those of
// CachePolicy step for step.
__global__ __launch_bounds__(kPlanThreads) void cache_plan_kernel(PlanArgs a)
{
    __shared__ uint64_t skey[kMaxDevSlots], sage[kMaxDevSlots];
    __shared__ uint32_t mask[kMaxDevExperts / 32];
    __shared__ int32_t list[kMaxCallExperts];
    __shared__ DevEntry ent[kMaxCallExperts];
    __shared__ uint64_t red[kPlanThreads / 64];
    __shared__ int count, need;
    const int tid = threadIdx.x;
    for (int i = tid; i < a.n_slots; i += kPlanThreads) {
        skey[i] = a.meta[i].owner;
        sage[i] = a.meta[i].age;
    }
    if (tid < kMaxDevExperts / 32) mask[tid] = 0;
    __syncthreads();
    if (tid < a.nk) {
        const int e = a.ids[tid];
        if (e >= 0 && e < a.E) atomicOr(&mask[e >> 5], 1u << (e & 31));
    }
    const uint8_t **table = a.tables + (size_t)a.layer * a.E;
    for (int e = tid; e < a.E; e += kPlanThreads) table[e] = nullptr;
    __syncthreads();
    if (tid == 0) {
        int n = 0;
        for (int w = 0; w < kMaxDevExperts / 32; ++w)
            for (uint32_t m = mask[w]; m; m &= m - 1) list[n++] = 32 * w + (__ffs(m) - 1);
        count = n;
    }
    __syncthreads();
    const int n = count;
    if (tid < n) ent[tid] = a.entries[(size_t)a.layer * a.E + list[tid]];
    DevState st{};
    if (tid == 0) st = *a.state;
    uint32_t jobs = 0;
    __syncthreads();
    for (int i = 0; i < n; ++i) {
        const int e = list[i];
        const uint64_t key = ((uint64_t)(uint32_t)a.layer << 32) | (uint32_t)e;
        const uint8_t *src = a.src[(size_t)a.layer * a.E + e];
        if (tid == 0) {
            DevEntry &en = ent[i];
            ++st.age;
            need = 0;
            if (en.slot >= 0) {
                ++st.hits;
                en.age = st.age;
                sage[en.slot] = st.age;
                table[e] = a.slots + (size_t)en.slot * a.stride;
            } else {
                ++st.misses;
                ++en.seen;
                table[e] = src;
                if (en.seen >= 2) {
                    need = 1;
                } else {
                    ++st.streamed;
                    st.bytes_streamed += a.expert_bytes;
                }
            }
        }
        __syncthreads();
        if (need) { // uniform: every thread searches its slots
            uint64_t best = ~0ull;
            for (int t = tid; t < a.n_slots; t += kPlanThreads) {
                const uint64_t o = skey[t];
                uint64_t k;
                if (o == 0) {
                    k = (uint64_t)t;
                } else {
                    const uint64_t ok = o - 1;
                    const int kl = (int)(ok >> 32), ke = (int)(ok & 0xffffffffu);
                    const bool same = kl == a.layer;
                    const bool busy = same && ke < kMaxDevExperts && ((mask[ke >> 5] >> (ke & 31)) & 1u);
                    k = busy ? ~0ull
                             : (1ull << 63) | ((uint64_t)(a.layer_aware && !same) << 62) |
                                   ((sage[t] & ((1ull << 46) - 1)) << 16) | (uint64_t)t;
                }
                best = k < best ? k : best;
            }
            best = wave_min_u64(best);
            if ((tid & 63) == 0) red[tid >> 6] = best;
            __syncthreads();
            if (tid == 0) {
                uint64_t b = red[0];
                for (int w = 1; w < kPlanThreads / 64; ++w) b = red[w] < b ? red[w] : b;
                DevEntry &en = ent[i];
                if (b != ~0ull) {
                    const int sl = (int)(b & 0xffffu);
                    if (skey[sl] != 0) { // the victim leaves its slot (its own entry keeps its count)
                        const uint64_t vk = skey[sl] - 1;
                        a.entries[(size_t)(vk >> 32) * a.E + (vk & 0xffffffffu)].slot = -1;
                        ++st.evictions;
                    }
                    en.slot = sl;
                    en.age = st.age;
                    skey[sl] = key + 1;
                    sage[sl] = st.age;
                    ++st.loads;
                    a.jobs[(size_t)a.layer * kMaxCallExperts + jobs] = CopyJob{src, a.slots + (size_t)sl * a.stride};
                    ++jobs;
                    st.bytes_uploaded += a.expert_bytes;
                    table[e] = a.slots + (size_t)sl * a.stride; // read from its slot once copied
                } else {
                    ++st.streamed;
                    st.bytes_streamed += a.expert_bytes;
                }
            }
        }
        __syncthreads();
    }
    if (tid < n) a.entries[(size_t)a.layer * a.E + list[tid]] = ent[tid];
    for (int t = tid; t < a.n_slots; t += kPlanThreads) a.meta[t] = DevSlot{skey[t], sage[t]};
    if (tid == 0) {
        *a.state = st;
        a.njobs[a.layer] = jobs;
    }
}

// The admissions' copies, host bytes into HBM slots: grid (chunk, job); a
// job past the layer's count exits.  Pointers and lengths are multiples of
// 16 bytes (the slot stride and the host layout are 256-aligned).
__global__ __launch_bounds__(256) void cache_copy_kernel(const CopyJob *jobs, const uint32_t *njobs, size_t bytes)
{
    if (blockIdx.y >= *njobs) return;
    const CopyJob j = jobs[blockIdx.y];
    const size_t lo = (size_t)blockIdx.x * kCopyChunk;
    const size_t hi = lo + kCopyChunk < bytes ? lo + kCopyChunk : bytes;
    for (size_t o = lo + 16 * (size_t)threadIdx.x; o < hi; o += 16 * 256)
        *reinterpret_cast<uint4 *>(j.dst + o) = *reinterpret_cast<const uint4 *>(j.src + o);
}

size_t round16(size_t n) { return (n + 15) & ~(size_t)15; }

} // namespace

struct emu_expert_cache {
    emu_ctx *ctx = nullptr;
    uint32_t layers = 0, n_experts = 0, n_slots = 0, n_transient = 0;
    size_t expert_bytes = 0;
    uint8_t *slots = nullptr; // (n_slots + n_transient) * expert_bytes
    std::vector<const void *> src;
    CachePolicy pol;
    uint32_t next_transient = 0;
    const uint8_t **d_tables = nullptr;  // kTableRing tables of n_experts device pointers
    const uint8_t **h_tables = nullptr;  // their pinned host staging
    hipEvent_t table_ev[kTableRing] = {};
    bool table_used[kTableRing] = {};
    int ring = 0;
    uint64_t bytes_uploaded = 0;
    size_t stride = 0; // bytes between slots (expert_bytes rounded up to 256)
    // device policy (emu_session_attach_expert_cache)
    bool device_policy = false;
    DevEntry *d_entries = nullptr;
    DevSlot *d_meta = nullptr;
    DevState *d_state = nullptr;
    CopyJob *d_jobs = nullptr;
    uint32_t *d_njobs = nullptr;
    const uint8_t **d_src = nullptr;    // [layers][E] device addresses of the sources
    const uint8_t **d_ltables = nullptr; // [layers][E] per-layer tables of the decode step
};

extern "C" int emu_host_alloc(emu_ctx *ctx, size_t bytes, void **h_out)
{
    if (!ctx || !h_out) return EMU_E_ARG;
    *h_out = nullptr;
    EMU_HIP(ctx, hipSetDevice(ctx->device));
    EMU_HIP(ctx, hipHostMalloc(h_out, bytes ? bytes : 1, hipHostMallocDefault));
    return EMU_OK;
}

extern "C" int emu_host_device_pointer(emu_ctx *ctx, void *h, void **d_out)
{
    if (!ctx || !h || !d_out) return EMU_E_ARG;
    *d_out = nullptr;
    EMU_HIP(ctx, hipHostGetDevicePointer(d_out, h, 0));
    return EMU_OK;
}

extern "C" int emu_host_free(emu_ctx *ctx, void *h)
{
    if (!ctx) return EMU_E_ARG;
    if (h) EMU_HIP(ctx, hipHostFree(h));
    return EMU_OK;
}

extern "C" int emu_expert_cache_destroy(emu_expert_cache *c)
{
    if (!c) return EMU_E_ARG;
    emu_ctx *ctx = c->ctx;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto &ev : c->table_ev)
        if (ev) (void)hipEventDestroy(ev);
    void *dev[] = {c->d_entries, c->d_meta, c->d_state, c->d_jobs, c->d_njobs, c->d_src, c->d_ltables};
    for (void *p : dev) emu_free(ctx, p);
    if (c->h_tables) (void)hipHostFree(c->h_tables);
    emu_free(ctx, c->d_tables);
    emu_free(ctx, c->slots);
    delete c;
    return EMU_OK;
}

extern "C" int emu_expert_cache_create(emu_ctx *ctx, uint32_t layers, uint32_t n_experts, size_t expert_bytes,
                                       uint32_t n_slots, uint32_t n_transient, int layer_aware,
                                       emu_expert_cache **out)
{
    if (!ctx || !out || layers == 0 || n_experts == 0 || expert_bytes == 0 || n_transient == 0) return EMU_E_ARG;
    *out = nullptr;
    emu_expert_cache *c = new (std::nothrow) emu_expert_cache();
    if (!c) return EMU_E_NOMEM;
    c->ctx = ctx;
    c->layers = layers;
    c->n_experts = n_experts;
    c->expert_bytes = expert_bytes;
    c->n_slots = n_slots;
    c->n_transient = n_transient;
    c->src.assign((size_t)layers * n_experts, nullptr);
    c->pol.init(n_slots, layer_aware != 0);
    c->stride = (expert_bytes + 255) & ~(size_t)255;
    int st = emu_malloc(ctx, (size_t)(n_slots + n_transient) * c->stride, (void **)&c->slots);
    if (st == EMU_OK) st = emu_malloc(ctx, sizeof(void *) * kTableRing * n_experts, (void **)&c->d_tables);
    if (st == EMU_OK && hipHostMalloc((void **)&c->h_tables, sizeof(void *) * kTableRing * n_experts,
                                      hipHostMallocDefault) != hipSuccess)
        st = EMU_E_HIP;
    for (int i = 0; st == EMU_OK && i < kTableRing; ++i)
        if (hipEventCreateWithFlags(&c->table_ev[i], hipEventDisableTiming) != hipSuccess) st = EMU_E_HIP;
    if (st != EMU_OK) {
        emu_expert_cache_destroy(c);
        return st;
    }
    *out = c;
    return EMU_OK;
}

extern "C" int emu_expert_cache_set_source(emu_expert_cache *c, uint32_t layer, uint32_t expert, const void *h_bytes)
{
    if (!c || !h_bytes || layer >= c->layers || expert >= c->n_experts) return EMU_E_ARG;
    c->src[(size_t)layer * c->n_experts + expert] = h_bytes;
    return EMU_OK;
}

extern "C" int emu_expert_cache_stats(const emu_expert_cache *c, emu_cache_stats *out)
{
    if (!c || !out) return EMU_E_ARG;
    if (c->device_policy) {
        DevState ds{};
        EMU_HIP(c->ctx, hipStreamSynchronize(c->ctx->stream));
        EMU_HIP(c->ctx, hipMemcpy(&ds, c->d_state, sizeof ds, hipMemcpyDeviceToHost));
        std::vector<DevSlot> meta(c->n_slots);
        if (c->n_slots)
            EMU_HIP(c->ctx, hipMemcpy(meta.data(), c->d_meta, sizeof(DevSlot) * c->n_slots, hipMemcpyDeviceToHost));
        out->hits = ds.hits;
        out->misses = ds.misses;
        out->loads = ds.loads;
        out->evictions = ds.evictions;
        out->streamed = ds.streamed;
        out->bytes_uploaded = ds.bytes_uploaded;
        out->bytes_streamed = ds.bytes_streamed;
        uint32_t r = 0;
        for (const DevSlot &m : meta) r += m.owner != 0;
        out->resident = r;
        return EMU_OK;
    }
    out->hits = c->pol.hits;
    out->misses = c->pol.misses;
    out->loads = c->pol.loads;
    out->evictions = c->pol.evictions;
    out->streamed = c->pol.streamed;
    out->bytes_uploaded = c->bytes_uploaded;
    out->bytes_streamed = 0;
    out->resident = c->pol.resident();
    return EMU_OK;
}

extern "C" int emu_expert_cache_slot(const emu_expert_cache *c, uint32_t layer, uint32_t expert, int32_t *slot)
{
    if (!c || !slot || layer >= c->layers || expert >= c->n_experts) return EMU_E_ARG;
    if (c->device_policy) {
        DevEntry en{};
        EMU_HIP(c->ctx, hipStreamSynchronize(c->ctx->stream));
        EMU_HIP(c->ctx, hipMemcpy(&en, c->d_entries + (size_t)layer * c->n_experts + expert, sizeof en,
                                  hipMemcpyDeviceToHost));
        *slot = en.slot;
        return EMU_OK;
    }
    auto it = c->pol.entries.find(CachePolicy::key(layer, expert));
    *slot = it == c->pol.entries.end() ? -1 : it->second.slot;
    return EMU_OK;
}

extern "C" int emu_moe_ffn_cached(emu_ctx *ctx, const emu_moe_desc *d, emu_expert_cache *c, uint32_t layer,
                                  const float *d_x, uint32_t n_tok, const int32_t *h_ids, const int32_t *d_ids,
                                  const float *d_weights, void *d_workspace, size_t workspace_bytes, float *d_out)
{
    if (!ctx || !d || !c || !h_ids || c->ctx != ctx || layer >= c->layers || d->n_experts != c->n_experts)
        return EMU_E_ARG;
    if (c->device_policy) return EMU_E_CONFIG; // its policy state lives on the device, for a session
    if (n_tok == 0) return EMU_OK;
    if (n_tok > 8 || d->k == 0 || d->k > 8) return EMU_E_ARG;
    uint32_t be_in = 0, bb_in = 0, be_ff = 0, bb_ff = 0;
    int st = emu_block_layout(d->enc_gate_up, &be_in, &bb_in);
    if (st == EMU_OK) st = emu_block_layout(d->enc_down, &be_ff, &bb_ff);
    if (st != EMU_OK) return st;
    if (d->width % be_in || d->ff % be_ff) return EMU_E_SHORT;
    const size_t need = 2 * (size_t)d->ff * (d->width / be_in) * bb_in + (size_t)d->width * (d->ff / be_ff) * bb_ff;
    if (need != c->expert_bytes) return EMU_E_SHAPE;
    // The distinct experts of the call, ascending.
    std::vector<int32_t> ids(h_ids, h_ids + (size_t)n_tok * d->k);
    std::sort(ids.begin(), ids.end());
    ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
    for (int32_t e : ids)
        if (e < 0 || (uint32_t)e >= c->n_experts || !c->src[(size_t)layer * c->n_experts + e]) return EMU_E_ARG;
    size_t streamed = 0;
    for (int32_t e : ids) {
        auto it = c->pol.entries.find(CachePolicy::key(layer, (uint32_t)e));
        const bool resident = it != c->pol.entries.end() && it->second.slot >= 0;
        streamed += resident ? 0 : 1;
    }
    if (streamed > c->n_transient) {
        snprintf(ctx->last_error, sizeof ctx->last_error,
                 "expert cache: %zu experts to stream through, %u transient slots", streamed, c->n_transient);
        return EMU_E_CONFIG;
    }
    // The table ring slot: its previous host-to-device copy has finished.
    const int r = c->ring;
    c->ring = (c->ring + 1) % kTableRing;
    if (c->table_used[r]) EMU_HIP(ctx, hipEventSynchronize(c->table_ev[r]));
    const uint8_t **ht = c->h_tables + (size_t)r * c->n_experts;
    for (uint32_t e = 0; e < c->n_experts; ++e) ht[e] = nullptr;
    {
        std::vector<uint32_t> call(ids.begin(), ids.end());
        c->pol.begin_call(layer, call.data(), call.size());
    }
    for (int32_t e : ids) {
        int32_t slot = -1;
        const int how = c->pol.access(layer, (uint32_t)e, &slot);
        uint8_t *dst;
        if (how == kStreamed) {
            dst = c->slots + (size_t)(c->n_slots + c->next_transient) * c->stride;
            c->next_transient = (c->next_transient + 1) % c->n_transient;
        } else {
            dst = c->slots + (size_t)slot * c->stride;
        }
        if (how != kHit) {
            EMU_HIP(ctx, hipMemcpyAsync(dst, c->src[(size_t)layer * c->n_experts + e], c->expert_bytes,
                                        hipMemcpyHostToDevice, ctx->stream));
            c->bytes_uploaded += c->expert_bytes;
        }
        ht[e] = dst;
    }
    c->pol.end_call();
    const uint8_t **dt = c->d_tables + (size_t)r * c->n_experts;
    EMU_HIP(ctx, hipMemcpyAsync(dt, ht, sizeof(void *) * c->n_experts, hipMemcpyHostToDevice, ctx->stream));
    EMU_HIP(ctx, hipEventRecord(c->table_ev[r], ctx->stream));
    c->table_used[r] = true;
    return emu_moe_ffn_table(ctx, d, dt, d_x, n_tok, d_ids, d_weights, d_workspace, workspace_bytes, d_out);
}

extern "C" int emu_expert_cache_policy_trace(uint32_t n_slots, int layer_aware, const uint32_t *calls,
                                             const uint32_t *layers, const uint32_t *experts, uint32_t n,
                                             int32_t *outcome, int32_t *slot)
{
    if (n && (!calls || !layers || !experts || !outcome || !slot)) return EMU_E_ARG;
    CachePolicy pol;
    pol.init(n_slots, layer_aware != 0);
    for (uint32_t i = 0; i < n;) {
        uint32_t j = i;
        while (j < n && calls[j] == calls[i]) ++j;
        for (uint32_t t = i; t < j; ++t) pol.begin_call(layers[t], &experts[t], 1);
        for (uint32_t t = i; t < j; ++t) outcome[t] = pol.access(layers[t], experts[t], &slot[t]);
        pol.end_call();
        i = j;
    }
    return EMU_OK;
}

// ------------------------------------------------ device policy: set-up --

size_t emu_cache_expert_bytes(const emu_expert_cache *c) { return c->expert_bytes; }
uint32_t emu_cache_layers(const emu_expert_cache *c) { return c->layers; }
uint32_t emu_cache_experts(const emu_expert_cache *c) { return c->n_experts; }

int emu_cache_device_enable(emu_expert_cache *c)
{
    emu_ctx *ctx = c->ctx;
    if (c->n_slots > (uint32_t)kMaxDevSlots || c->n_experts > (uint32_t)kMaxDevExperts) return EMU_E_CONFIG;
    const size_t le = (size_t)c->layers * c->n_experts;
    // every source pinned (device-addressable), 16-byte aligned for the copies
    std::vector<const uint8_t *> dev(le);
    for (size_t i = 0; i < le; ++i) {
        if (!c->src[i]) {
            snprintf(ctx->last_error, sizeof ctx->last_error, "expert cache: no source for (layer %zu, expert %zu)",
                     i / c->n_experts, i % c->n_experts);
            return EMU_E_ARG;
        }
        void *d = nullptr;
        if (hipHostGetDevicePointer(&d, const_cast<void *>(c->src[i]), 0) != hipSuccess || !d ||
            ((uintptr_t)d & 15u) != 0) {
            (void)hipGetLastError();
            snprintf(ctx->last_error, sizeof ctx->last_error,
                     "expert cache: the source of (layer %zu, expert %zu) is not 16-byte aligned pinned memory "
                     "(emu_host_alloc)", i / c->n_experts, i % c->n_experts);
            return EMU_E_ARG;
        }
        dev[i] = static_cast<const uint8_t *>(d);
    }
    if (c->device_policy) { // already set up: refresh the sources only
        EMU_HIP(ctx, hipMemcpy(c->d_src, dev.data(), sizeof(void *) * le, hipMemcpyHostToDevice));
        return EMU_OK;
    }
    int st = EMU_OK;
    auto alloc = [&](void **p, size_t bytes) {
        if (st == EMU_OK) st = emu_malloc(ctx, bytes, p);
    };
    alloc((void **)&c->d_entries, sizeof(DevEntry) * le);
    alloc((void **)&c->d_meta, sizeof(DevSlot) * (c->n_slots ? c->n_slots : 1));
    alloc((void **)&c->d_state, sizeof(DevState));
    alloc((void **)&c->d_jobs, sizeof(CopyJob) * c->layers * kMaxCallExperts);
    alloc((void **)&c->d_njobs, sizeof(uint32_t) * c->layers);
    alloc((void **)&c->d_src, sizeof(void *) * le);
    alloc((void **)&c->d_ltables, sizeof(void *) * le);
    if (st != EMU_OK) return st;
    std::vector<DevEntry> ent(le, DevEntry{0, -1, 0});
    std::vector<DevSlot> meta(c->n_slots ? c->n_slots : 1, DevSlot{0, 0});
    const DevState zero{};
    EMU_HIP(ctx, hipMemcpy(c->d_entries, ent.data(), sizeof(DevEntry) * le, hipMemcpyHostToDevice));
    EMU_HIP(ctx, hipMemcpy(c->d_meta, meta.data(), sizeof(DevSlot) * meta.size(), hipMemcpyHostToDevice));
    EMU_HIP(ctx, hipMemcpy(c->d_state, &zero, sizeof zero, hipMemcpyHostToDevice));
    EMU_HIP(ctx, hipMemset(c->d_njobs, 0, sizeof(uint32_t) * c->layers));
    EMU_HIP(ctx, hipMemcpy(c->d_src, dev.data(), sizeof(void *) * le, hipMemcpyHostToDevice));
    EMU_HIP(ctx, hipMemset(c->d_ltables, 0, sizeof(void *) * le));
    c->device_policy = true;
    return EMU_OK;
}

int emu_cache_plan(emu_expert_cache *c, uint32_t layer, const int32_t *d_ids, int nk, const uint8_t *const **table)
{
    emu_ctx *ctx = c->ctx;
    if (!c->device_policy || layer >= c->layers || nk < 0 || nk > kMaxCallExperts) return EMU_E_CONFIG;
    PlanArgs a{};
    a.entries = c->d_entries;
    a.meta = c->d_meta;
    a.state = c->d_state;
    a.jobs = c->d_jobs;
    a.njobs = c->d_njobs;
    a.src = c->d_src;
    a.slots = c->slots;
    a.stride = c->stride;
    a.expert_bytes = c->expert_bytes;
    a.tables = c->d_ltables;
    a.ids = d_ids;
    a.nk = nk;
    a.layer = (int)layer;
    a.E = (int)c->n_experts;
    a.n_slots = (int)c->n_slots;
    a.layer_aware = c->pol.layer_aware ? 1 : 0;
    hipLaunchKernelGGL(cache_plan_kernel, dim3(1), dim3(kPlanThreads), 0, ctx->stream, a);
    EMU_LAUNCH_CHECK(ctx);
    // the admissions' copies, before the experts that read them
    const unsigned chunks = (unsigned)((round16(c->expert_bytes) + kCopyChunk - 1) / kCopyChunk);
    hipLaunchKernelGGL(cache_copy_kernel, dim3(chunks, kMaxCallExperts), dim3(256), 0, ctx->stream,
                       c->d_jobs + (size_t)layer * kMaxCallExperts, c->d_njobs + layer, round16(c->expert_bytes));
    EMU_LAUNCH_CHECK(ctx);
    *table = c->d_ltables + (size_t)layer * c->n_experts;
    return EMU_OK;
}
