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

    // expert_cache.rs:36-72 (get) with the slot it lands in (-1: streamed).
    int access(uint32_t layer, uint32_t expert, int32_t *slot)
    {
        const uint64_t k = key(layer, expert);
        ++age;
        Entry &en = entries[k];
        if (!en.active) {
            en.active = true;
            active.push_back(k);
        }
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
};

extern "C" int emu_host_alloc(emu_ctx *ctx, size_t bytes, void **h_out)
{
    if (!ctx || !h_out) return EMU_E_ARG;
    *h_out = nullptr;
    EMU_HIP(ctx, hipSetDevice(ctx->device));
    EMU_HIP(ctx, hipHostMalloc(h_out, bytes ? bytes : 1, hipHostMallocDefault));
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
    int st = emu_malloc(ctx, (size_t)(n_slots + n_transient) * expert_bytes, (void **)&c->slots);
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
    out->hits = c->pol.hits;
    out->misses = c->pol.misses;
    out->loads = c->pol.loads;
    out->evictions = c->pol.evictions;
    out->streamed = c->pol.streamed;
    out->bytes_uploaded = c->bytes_uploaded;
    out->resident = c->pol.resident();
    return EMU_OK;
}

extern "C" int emu_expert_cache_slot(const emu_expert_cache *c, uint32_t layer, uint32_t expert, int32_t *slot)
{
    if (!c || !slot || layer >= c->layers || expert >= c->n_experts) return EMU_E_ARG;
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
    for (int32_t e : ids) {
        int32_t slot = -1;
        const int how = c->pol.access(layer, (uint32_t)e, &slot);
        uint8_t *dst;
        if (how == kStreamed) {
            dst = c->slots + (size_t)(c->n_slots + c->next_transient) * c->expert_bytes;
            c->next_transient = (c->next_transient + 1) % c->n_transient;
        } else {
            dst = c->slots + (size_t)slot * c->expert_bytes;
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
    for (uint32_t i = 0; i < n; ++i) {
        if (i > 0 && calls[i] != calls[i - 1]) pol.end_call();
        outcome[i] = pol.access(layers[i], experts[i], &slot[i]);
    }
    return EMU_OK;
}
