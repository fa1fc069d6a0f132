// attn.hip -- fused decode attention for the decode step.
//
// One workgroup per (context chunk, kv head, client).  Each workgroup
//   1. rebuilds the rotated queries of its GQ = heads/kv_heads query heads from
//      the projection output (per-head RMSNorm when the model has QK-norm, then
//      RoPE from the host-built table: spm-qwen3-slice/src/attention.rs:27-34);
//   2. if its chunk holds the new position, rotates the new key, rounds key and
//      value to the cache type and appends them (KvCache::append,
//      spm-kv/src/cache.rs:49-58) -- the same values it then attends with;
//   3. scores its chunk's positions (one position per thread, the query heads
//      broadcast from LDS), takes the chunk max and exp-sum, and accumulates
//      the un-normalised weighted values (head lanes x position halves);
//   4. writes (max, sum, partial) per query head; the last workgroup of the
//      (client, kv head) to finish merges every chunk (flash-decoding) and
//      resets the arrival counter for the next step.
// Cache layout: [client][layer][kv_head][context][head_dim], f16 or f32.
#include "internal.hpp"

#include <math.h>

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 256; // positions per workgroup: one per thread

struct AttnArgs {
    const float *qkv;       // [client][q_width + 2*kv_width]
    void *k_cache, *v_cache;
    const uint32_t *positions;
    const float2 *rope;     // [context][hd/2] (cos, sin)
    const float *q_norm, *k_norm; // per-layer gains or null
    float eps;
    float score_mul;        // score = dot * score_mul (or / score_div)
    float score_div;        // > 0 selects division
    int rope_fma;           // spm-ops form: fma(x, cos, -(y*sin))
    int heads, kv_heads, layers, layer, context;
    float *partial;         // [client][head][max_chunks][hd + 2]
    uint32_t *counters;     // [client][kv_head]
    int max_chunks;
    float *out;             // [client][heads * hd]
};

template <int HD> __device__ __forceinline__ float rotate_pair_first(float l, float r, float2 cs, int fma_form)
{
#pragma clang fp contract(off)
    if (fma_form) return __builtin_fmaf(l, cs.x, -(r * cs.y));
    return l * cs.x - r * cs.y;
}
template <int HD> __device__ __forceinline__ float rotate_pair_second(float l, float r, float2 cs, int fma_form)
{
#pragma clang fp contract(off)
    if (fma_form) return __builtin_fmaf(l, cs.y, r * cs.x);
    return r * cs.x + l * cs.y;
}

// Norm + rotate one head of HD values held in LDS by the first HD/2 threads of
// a wave-aligned group.  src/dst may alias.
template <int HD>
__device__ void prep_head(const float *src, float *dst, const float *gain, float eps, float2 const *rope_row,
                          int fma_form, int tid, float *red)
{
    // Sum of squares over the head (threads 0..HD-1 of this call each own one).
    float v = tid < HD ? src[tid] : 0.0f;
    float s = v * v;
    s = wave_sum(s);
    if (HD > 64) {
        if ((tid & 63) == 0 && tid < HD) red[tid >> 6] = s;
        __syncthreads();
        s = 0.0f;
#pragma unroll
        for (int i = 0; i < HD / 64; ++i) s += red[i];
        __syncthreads();
    }
    float scale = 1.0f;
    if (gain) scale = 1.0f / sqrtf(s / (float)HD + eps);
    const float nv = gain && tid < HD ? __fmul_rn(__fmul_rn(v, scale), gain[tid]) : v;
    __syncthreads();
    if (tid < HD) dst[tid] = nv;
    __syncthreads();
    if (tid < HD / 2) {
        const float2 cs = rope_row[tid];
        const float l = dst[tid], r = dst[tid + HD / 2];
        const float a = rotate_pair_first<HD>(l, r, cs, fma_form);
        const float b = rotate_pair_second<HD>(l, r, cs, fma_form);
        dst[tid] = a;
        dst[tid + HD / 2] = b;
    }
    __syncthreads();
}

template <int HD, bool F16>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(AttnArgs a)
{
    using kv_t = typename std::conditional<F16, __half, float>::type;
    const int chunk = blockIdx.x, kvh = blockIdx.y, client = blockIdx.z;
    const int tid = threadIdx.x;
    const int pos = (int)a.positions[client];
    const int n = pos + 1;
    const int n_chunks = (n + kChunk - 1) / kChunk;
    if (chunk >= n_chunks) return; // uniform per workgroup
    const int GQ = a.heads / a.kv_heads;

    __shared__ float q_s[8][HD];      // GQ <= 8
    __shared__ float knew[HD], vnew[HD];
    __shared__ float sc[8][kChunk];
    __shared__ float red[8];
    __shared__ float accs[2][8][HD];

    const int qw = a.heads * HD, kw = a.kv_heads * HD;
    const float *row = a.qkv + (size_t)client * (qw + 2 * kw);
    const float2 *rope_row = a.rope + (size_t)pos * (HD / 2);
    const float *qn = a.q_norm ? a.q_norm + (size_t)a.layer * HD : nullptr;
    const float *kn = a.k_norm ? a.k_norm + (size_t)a.layer * HD : nullptr;

    for (int g = 0; g < GQ; ++g) {
        const int head = kvh * GQ + g;
        if (tid < HD) q_s[g][tid] = row[head * HD + tid];
        __syncthreads();
        prep_head<HD>(q_s[g], q_s[g], qn, a.eps, rope_row, a.rope_fma, tid, red);
    }

    const size_t cache_base = (((size_t)client * a.layers + a.layer) * a.kv_heads + kvh) * (size_t)a.context * HD;
    kv_t *kc = static_cast<kv_t *>(a.k_cache) + cache_base;
    kv_t *vc = static_cast<kv_t *>(a.v_cache) + cache_base;
    const int p0 = chunk * kChunk;
    const bool owner = pos >= p0 && pos < p0 + kChunk;
    if (owner) {
        if (tid < HD) knew[tid] = row[qw + kvh * HD + tid];
        __syncthreads();
        prep_head<HD>(knew, knew, kn, a.eps, rope_row, a.rope_fma, tid, red);
        if (tid < HD) {
            const float kv = knew[tid];
            const float vv = row[qw + kw + kvh * HD + tid];
            kv_t kq, vq;
            if constexpr (F16) {
                kq = (kv_t)__float2half_rn(kv);
                vq = (kv_t)__float2half_rn(vv);
            } else {
                kq = (kv_t)kv;
                vq = (kv_t)vv;
            }
            kc[(size_t)pos * HD + tid] = kq;
            vc[(size_t)pos * HD + tid] = vq;
            knew[tid] = (float)kq; // attend with the cached (rounded) values
            vnew[tid] = (float)vq;
        }
        __syncthreads();
    }

    // Scores: thread per position.
    const int p = p0 + tid;
    const bool live = p < n;
    float s[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) s[g] = -INFINITY;
    if (live) {
        float dot[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) dot[g] = 0.0f;
        if (p == pos) {
            for (int i = 0; i < HD; ++i) {
                const float kv = knew[i];
#pragma unroll
                for (int g = 0; g < 8; ++g)
                    if (g < GQ) dot[g] = __builtin_fmaf(q_s[g][i], kv, dot[g]);
            }
        } else {
            const kv_t *kr = kc + (size_t)p * HD;
            for (int i = 0; i < HD; i += 8) {
                float kv[8];
                if constexpr (F16) {
                    const uint4 raw = *reinterpret_cast<const uint4 *>(kr + i);
                    const __half2 *h2 = reinterpret_cast<const __half2 *>(&raw);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float2 f = __half22float2(h2[j]);
                        kv[2 * j] = f.x;
                        kv[2 * j + 1] = f.y;
                    }
                } else {
                    const float4 x0 = *reinterpret_cast<const float4 *>(kr + i);
                    const float4 x1 = *reinterpret_cast<const float4 *>(kr + i + 4);
                    kv[0] = x0.x; kv[1] = x0.y; kv[2] = x0.z; kv[3] = x0.w;
                    kv[4] = x1.x; kv[5] = x1.y; kv[6] = x1.z; kv[7] = x1.w;
                }
#pragma unroll
                for (int g = 0; g < 8; ++g)
                    if (g < GQ)
#pragma unroll
                        for (int j = 0; j < 8; ++j) dot[g] = __builtin_fmaf(q_s[g][i + j], kv[j], dot[g]);
            }
        }
#pragma unroll
        for (int g = 0; g < 8; ++g)
            if (g < GQ) s[g] = a.score_div > 0.0f ? dot[g] / a.score_div : dot[g] * a.score_mul;
    }
    // Chunk max and exp per head.
    float m[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        if (g >= GQ) break;
        float v = s[g];
        for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
        if ((tid & 63) == 0) red[tid >> 6] = v;
        __syncthreads();
        m[g] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        sc[g][tid] = live ? expf(s[g] - m[g]) : 0.0f;
    }
    __syncthreads();
    float l[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        if (g >= GQ) break;
        float v = wave_sum(sc[g][tid]);
        if ((tid & 63) == 0) red[tid >> 6] = v;
        __syncthreads();
        l[g] = (red[0] + red[1]) + (red[2] + red[3]);
        __syncthreads();
    }

    // Weighted values: thread = (lane d, half of the chunk's positions).
    const int cnt = min(kChunk, n - p0);
    for (int d0 = 0; d0 < HD; d0 += kThreads / 2) {
        const int d = d0 + (tid % (kThreads / 2));
        const int halfsel = tid / (kThreads / 2);
        float acc[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) acc[g] = 0.0f;
        if (d < HD) {
            for (int i = halfsel; i < cnt; i += 2) {
                const int pp = p0 + i;
                const float vv = pp == pos ? vnew[d] : (float)vc[(size_t)pp * HD + d];
#pragma unroll
                for (int g = 0; g < 8; ++g)
                    if (g < GQ) acc[g] = __builtin_fmaf(sc[g][i], vv, acc[g]);
            }
#pragma unroll
            for (int g = 0; g < 8; ++g)
                if (g < GQ) accs[halfsel][g][d] = acc[g];
        }
        __syncthreads();
        if (halfsel == 0 && d < HD) {
#pragma unroll
            for (int g = 0; g < 8; ++g)
                if (g < GQ) accs[0][g][d] = accs[0][g][d] + accs[1][g][d];
        }
        __syncthreads();
    }

    float *outp = a.out + (size_t)client * qw;
    if (n_chunks == 1) {
        for (int idx = tid; idx < GQ * HD; idx += kThreads) {
            const int g = idx / HD, d = idx % HD;
            outp[(kvh * GQ + g) * HD + d] = accs[0][g][d] / l[g];
        }
        return;
    }
    // Partial for the merge.
    for (int idx = tid; idx < GQ * (HD + 2); idx += kThreads) {
        const int g = idx / (HD + 2), j = idx % (HD + 2);
        const int head = kvh * GQ + g;
        float *pp = a.partial + (((size_t)client * a.heads + head) * a.max_chunks + chunk) * (HD + 2);
        pp[j] = j < HD ? accs[0][g][j] : (j == HD ? m[g] : l[g]);
    }
    __threadfence();
    __syncthreads();
    __shared__ uint32_t arrived;
    if (tid == 0) arrived = atomicAdd(a.counters + (size_t)client * a.kv_heads + kvh, 1u);
    __syncthreads();
    if (arrived != (uint32_t)(n_chunks - 1)) return;
    __threadfence();
    for (int idx = tid; idx < GQ * HD; idx += kThreads) {
        const int g = idx / HD, d = idx % HD;
        const int head = kvh * GQ + g;
        const float *pb = a.partial + ((size_t)client * a.heads + head) * a.max_chunks * (HD + 2);
        float M = -INFINITY;
        for (int c = 0; c < n_chunks; ++c) M = fmaxf(M, __builtin_nontemporal_load(pb + c * (HD + 2) + HD));
        float L = 0.0f, O = 0.0f;
        for (int c = 0; c < n_chunks; ++c) {
            const float *pc = pb + c * (HD + 2);
            const float f = expf(__builtin_nontemporal_load(pc + HD) - M);
            L = __builtin_fmaf(__builtin_nontemporal_load(pc + HD + 1), f, L);
            O = __builtin_fmaf(__builtin_nontemporal_load(pc + d), f, O);
        }
        outp[head * HD + d] = O / L;
    }
    if (tid == 0) atomicExch(a.counters + (size_t)client * a.kv_heads + kvh, 0u);
}

} // namespace


int emu_attn_max_chunks(int context) { return (context + kChunk - 1) / kChunk; }

int emu_launch_attn(emu_ctx *ctx, const EmuAttnLaunch &l)
{
    if (l.heads % l.kv_heads != 0 || l.heads / l.kv_heads > 8) return EMU_E_CONFIG;
    AttnArgs a{};
    a.qkv = l.qkv;
    a.k_cache = l.k_cache;
    a.v_cache = l.v_cache;
    a.positions = l.positions;
    a.rope = reinterpret_cast<const float2 *>(l.rope);
    a.q_norm = l.q_norm;
    a.k_norm = l.k_norm;
    a.eps = l.eps;
    a.score_mul = l.score_mul;
    a.score_div = l.score_div;
    a.rope_fma = l.rope_fma;
    a.heads = l.heads;
    a.kv_heads = l.kv_heads;
    a.layers = l.layers;
    a.layer = l.layer;
    a.context = l.context;
    a.partial = l.partial;
    a.counters = l.counters;
    a.max_chunks = emu_attn_max_chunks(l.context);
    a.out = l.out;
    dim3 grid(a.max_chunks, l.kv_heads, l.clients);
#define EMU_ATTN_CASE(HD)                                                                              \
    case HD:                                                                                           \
        if (l.kv_f16)                                                                                  \
            hipLaunchKernelGGL((attn_decode_kernel<HD, true>), grid, dim3(kThreads), 0, ctx->stream, a); \
        else                                                                                           \
            hipLaunchKernelGGL((attn_decode_kernel<HD, false>), grid, dim3(kThreads), 0, ctx->stream, a); \
        break;
    switch (l.head_dim) {
        EMU_ATTN_CASE(64)
        EMU_ATTN_CASE(128)
        EMU_ATTN_CASE(256)
    default: return EMU_E_CONFIG;
    }
#undef EMU_ATTN_CASE
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}
