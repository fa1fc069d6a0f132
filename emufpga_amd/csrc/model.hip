// model.hip -- dense decoder resident in HBM, client sessions, and the
// decode step (serve API: spm-batch/src/step.rs:19-39).
//
// HBM residency: one allocation per model.  Each layer's seven matrices sit
// back to back in the reference's consume order q, k, v, o, gate, up, down
// (layouts/smollm2-135m.order:3-8), each as GGUF row-major blocks, so q|k|v
// is one (q_width + 2*kv_width) x hidden matrix and gate|up a pair of
// equal-shaped matrices.  Then the embedding, the output matrix (unless
// tied) and the f32 norm gains.
//
// One decode step is a fixed launch sequence that reads every input from
// device memory (tokens, positions), so it is captured once into a HIP graph
// and replayed per step:
//   embed -> per layer { qkv matvec (RMSNorm fused) -> attention (QK-norm,
//   RoPE, KV append, split-context softmax) -> o matvec (+residual) ->
//   gate|up matvec (RMSNorm + SwiGLU fused) -> down matvec (+residual) }
//   -> output matvec (final RMSNorm fused) -> greedy select + advance.
#include "internal.hpp"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <stdio.h>

#include <algorithm>
#include <initializer_list>
#include <vector>

int emu_build_rope_table(uint32_t positions, uint32_t head_dim, float theta, int fma_form,
                         std::vector<float> &table);

namespace {

constexpr int kThreads = 256;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

} // namespace

struct emu_model {
    emu_ctx *ctx = nullptr;
    emu_model_config cfg{};
    uint8_t *base = nullptr;
    size_t total = 0;
    size_t rb_h = 0, rb_q = 0, rb_f = 0; // row bytes for cols = hidden, q_width, ffn
    size_t layer_bytes = 0;
    size_t off_q = 0, off_k = 0, off_v = 0, off_o = 0, off_g = 0, off_u = 0, off_d = 0;
    size_t off_layers = 0, off_embed = 0, off_output = 0, off_attn_norm = 0, off_ffn_norm = 0,
           off_q_norm = 0, off_k_norm = 0, off_out_norm = 0;
    size_t embed_bytes = 0;
    // Mixture-of-experts layers: router (f32) and gate/up/down experts,
    // expert-major (spm-granite-moe/src/weights.rs:57-73), after q, k, v, o.
    size_t off_r = 0, off_ge = 0, off_ue = 0, off_de = 0, rb_he = 0, rb_fe = 0;
    // Gemma-4 form: router and down scales, the shared FFN (off_ge holds the
    // fused gate|up experts), and the experts' input gains.
    size_t off_rs = 0, off_ds = 0, off_sg = 0, off_su = 0, off_sd = 0, rb_sf = 0, off_ffn_norm2 = 0;
    bool gemma() const { return moe() && cfg.gemma; }
    // Lane-major copy (emu_lane_major_q6k) of the Q6_K matrices the batch-1
    // limb matvec reads, at the same offsets as in `base` for the layers and
    // at off_embed for the output matrix (tied or not).  Rebuilt before the
    // next decode launch whenever the weights may have changed.
    uint8_t *lm = nullptr;
    size_t lm_bytes = 0, mm_bytes = 0; // the two derived copies' allocations
    bool lm_dirty = true;
    bool moe() const { return cfg.style == EMU_STYLE_GRANITE; }
    bool lm_takes(uint32_t cols) const { return lm && emu_limb_supports(cfg.encoding, (int)cols); }
    // The matrix a batch-1 matvec over `cols` columns reads, and whether it
    // is the lane-major copy (never with f32 activations, whose kernels read
    // GGUF order).
    const uint8_t *lm_or(const uint8_t *w, uint32_t cols, uint32_t n, int *lane_major, bool f32 = false) const
    {
        *lane_major = !f32 && n == 1 && lm_takes(cols);
        return *lane_major ? lm + (w - base) : w;
    }
    // Matrix-core operand copy (emu_mfma_major_q6k) of the Q6_K matrices the
    // chained matrix-core matvecs read: each listed matrix (its offset in
    // `base`, rows, cols) has its copy at `dst` in `mm`, rows padded to whole
    // 32-row tiles.  Rebuilt with the lane-major copy.
    struct MmEntry {
        size_t src, dst;
        uint32_t rows, cols;
    };
    uint8_t *mm = nullptr;
    std::vector<MmEntry> mm_map;
    // The matrix a chained matvec reads, and whether it is the operand copy.
    const uint8_t *mm_or(const uint8_t *w, int *mfma_major) const
    {
        const size_t off = (size_t)(w - base);
        for (const MmEntry &e : mm_map)
            if (e.src == off) {
                *mfma_major = 1;
                return mm + e.dst;
            }
        *mfma_major = 0;
        return w;
    }
};

struct emu_session {
    emu_model *m = nullptr;
    uint32_t n = 0, context = 0;
    int kv_f16 = 1;
    uint32_t flags = 0; // EMU_SESSION_*
    bool f32() const { return (flags & EMU_SESSION_F32_ACT) != 0; }
    void *k_cache = nullptr, *v_cache = nullptr;
    size_t kv_bytes = 0;
    uint32_t *positions = nullptr, *tokens = nullptr, *steps = nullptr, *prompt = nullptr,
             *hist = nullptr, *ctrl = nullptr, *last = nullptr, *counters = nullptr;
    uint64_t *keys = nullptr; // per-client greedy-selection keys written by the output matvec
    uint32_t key_stride = 0;
    float *state = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr,
          *partial = nullptr, *rope = nullptr;
    // mixture-of-experts scratch: normalised input, router logits, routes,
    // expert output, and the selected-expert FFN's workspace
    float *xn = nullptr, *rlog = nullptr, *rwts = nullptr, *rwts_s = nullptr;
    // Gemma form: the router's input and the global layers' RoPE table
    float *rope2 = nullptr;
    uint32_t *gate_counters = nullptr; // [client] arrivals at the MoE gate
    uint32_t *span_counters = nullptr; // arrivals per (expert, span) at the experts' gate|up
    // Zipf routing for throughput runs and the device route trace
    // ([capacity][layer][client][k] ids and weights, slot = step % capacity)
    float zipf_s = 0.0f;
    uint64_t zipf_seed = 0;
    int32_t *trace_ids = nullptr;
    float *trace_w = nullptr;
    uint32_t trace_cap = 0;
    int32_t *rids = nullptr, *rids_s = nullptr; // routes in top-k order (traced) and in ascending id (used)
    void *moe_ws = nullptr;
    size_t moe_ws_bytes = 0;
    std::vector<uint32_t> host_pos;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // emu_session_time_layers: events after the embedding, after each layer
    // and after the selection, recorded only while `marking`
    std::vector<hipEvent_t> marks;
    bool marking = false;
    // experts behind the expert cache's HBM slots (emu_session_attach_expert_cache)
    emu_expert_cache *cache = nullptr;
};

namespace {

// ------------------------------------------------------------ synthesis --
// Counter-based N(0, std): splitmix64 of (seed, stream, element) -> Box-Muller.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Box-Muller, r * cos(2 pi u2) with r = sqrt(-2 ln u1), evaluated in double
// precision by additions, multiplications and one division per logarithm
// (every one correctly rounded, none contracted), then rounded once to
// float: the same bits on any IEEE-754 machine, so a CPU can synthesise the
// same weights.  u1 = k / 2^24 (k = 1 .. 2^24) and u2 = j / 2^24 are exact.
//   ln k = e ln 2 + ln m, k = 2^e m, m in [sqrt(1/2), sqrt(2)), by
//          2 atanh(s) = 2 (s + s^3/3 + ... + s^23/23), s = (m - 1) / (m + 1);
//   cos(2 pi j / 2^24) by the quadrant of j and a Taylor polynomial of sin or
//          cos on [0, pi/4] (terms to x^17 / x^18);
//   sqrt(y) = y / sqrt(y) from six Newton steps of 1/sqrt(y) started at a
//          guess built from y's exponent.
__device__ __forceinline__ double synth_ln_int(uint32_t k) // ln k, k >= 1
{
#pragma clang fp contract(off)
    int e = 31 - __builtin_clz(k);
    double m = (double)k * __longlong_as_double((long long)(1023 - e) << 52); // k / 2^e, exact
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        e += 1;
    }
    const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    double p = 1.0 / 23.0;
    p = p * s2 + 1.0 / 21.0;
    p = p * s2 + 1.0 / 19.0;
    p = p * s2 + 1.0 / 17.0;
    p = p * s2 + 1.0 / 15.0;
    p = p * s2 + 1.0 / 13.0;
    p = p * s2 + 1.0 / 11.0;
    p = p * s2 + 1.0 / 9.0;
    p = p * s2 + 1.0 / 7.0;
    p = p * s2 + 1.0 / 5.0;
    p = p * s2 + 1.0 / 3.0;
    p = p * s2 + 1.0;
    return (double)e * 0.6931471805599453 + 2.0 * (s * p);
}

__device__ __forceinline__ double synth_sin_poly(double x) // x in [0, pi/4]
{
#pragma clang fp contract(off)
    const double x2 = x * x;
    double p = 1.0 / 355687428096000.0; // 1/17!
    p = p * x2 - 1.0 / 1307674368000.0; // 1/15!
    p = p * x2 + 1.0 / 6227020800.0;
    p = p * x2 - 1.0 / 39916800.0;
    p = p * x2 + 1.0 / 362880.0;
    p = p * x2 - 1.0 / 5040.0;
    p = p * x2 + 1.0 / 120.0;
    p = p * x2 - 1.0 / 6.0;
    p = p * x2 + 1.0;
    return x * p;
}

__device__ __forceinline__ double synth_cos_poly(double x) // x in [0, pi/4]
{
#pragma clang fp contract(off)
    const double x2 = x * x;
    double p = 1.0 / 6402373705728000.0; // 1/18!
    p = p * x2 - 1.0 / 20922789888000.0; // 1/16!
    p = p * x2 + 1.0 / 87178291200.0;
    p = p * x2 - 1.0 / 479001600.0;
    p = p * x2 + 1.0 / 3628800.0;
    p = p * x2 - 1.0 / 40320.0;
    p = p * x2 + 1.0 / 720.0;
    p = p * x2 - 1.0 / 24.0;
    p = p * x2 + 1.0 / 2.0;
    return 1.0 - x2 * p;
}

__device__ __forceinline__ double synth_cos_turn(uint32_t j) // cos(2 pi j / 2^24), j < 2^24
{
#pragma clang fp contract(off)
    const uint32_t q = j >> 22, f = j & 0x3fffffu; // angle = pi/2 (q + f / 2^22)
    const bool hi = f > 0x200000u;                 // past pi/4 in the quadrant: the co-function
    const double g = (double)(hi ? 0x400000u - f : f) * (1.0 / 4194304.0);
    const double x = g * 1.5707963267948966;
    const double cg = synth_cos_poly(x), sg = synth_sin_poly(x);
    const double c = hi ? sg : cg, sn = hi ? cg : sg; // cos and sin of pi/2 * f / 2^22
    return q == 0 ? c : q == 1 ? -sn : q == 2 ? -c : sn;
}

__device__ __forceinline__ double synth_sqrt(double y) // y >= 0
{
#pragma clang fp contract(off)
    if (y == 0.0) return 0.0;
    const long long b = __double_as_longlong(y);
    double r = __longlong_as_double(0x5fe6eb50c7b537a9ll - (b >> 1)); // ~1/sqrt(y)
    for (int i = 0; i < 6; ++i) r = r * (1.5 - (0.5 * y) * (r * r));
    return y * r;
}

__device__ __forceinline__ float gauss(uint64_t seed, uint64_t stream, uint64_t idx, float sd)
{
#pragma clang fp contract(off)
    const uint64_t h = splitmix64(seed ^ splitmix64(stream * 0x632be59bd9b4e019ull + idx));
    const uint32_t k = (uint32_t)(h >> 40) + 1u; // u1 = k / 2^24 in (0, 1]
    const uint32_t j = (uint32_t)(h & 0xffffffu); // u2 = j / 2^24 in [0, 1)
    const double ln_u1 = synth_ln_int(k) - 24.0 * 0.6931471805599453;
    const double r = synth_sqrt(-2.0 * ln_u1);
    return (float)(((double)sd * r) * synth_cos_turn(j));
}

// Zipf(s) routing for throughput runs: expert e (Zipf rank e + 1) gets the
// logit -s * ln(e + 1) + G with G a Gumbel draw keyed by (seed, client,
// position, layer, expert).  The top k of these are a sample without
// replacement with probabilities proportional to (e + 1)^-s (Gumbel-top-k).
struct ZipfRoute {
    float s;           // 0: the model's own router
    uint64_t seed;
    const uint32_t *positions;
    int layer;
};

__device__ __forceinline__ float zipf_logit(const ZipfRoute &z, int client, int e)
{
    const uint64_t key = ((uint64_t)(uint32_t)client << 48) ^ ((uint64_t)z.positions[client] << 24) ^
                         ((uint64_t)(uint32_t)z.layer << 12) ^ (uint64_t)(uint32_t)e;
    const uint64_t h = splitmix64(z.seed ^ splitmix64(key));
    const float u = (float)((h >> 40) + 1) * (1.0f / 16777217.0f); // (0, 1)
    return -z.s * logf((float)(e + 1)) - logf(-logf(u));
}

__device__ __forceinline__ uint16_t f2h(float x) { return __half_as_ushort(__float2half_rn(x)); }

__device__ __forceinline__ float clampf(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

// One thread per block; the block is assembled in private memory then stored.
// No contraction, so the bits are those of the same arithmetic on a CPU.
template <int ENC>
__global__ __launch_bounds__(kThreads) void synth_kernel(uint8_t *dst, size_t nblocks, uint64_t seed,
                                                         uint64_t stream, float sd)
{
#pragma clang fp contract(off)
    const size_t b = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (b >= nblocks) return;
    if constexpr (ENC == EMU_ENC_Q8_0) {
        uint8_t out[34];
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(gauss(seed, stream, b * 32 + i, sd)));
        const uint16_t d16 = f2h(amax / 127.0f);
        const float dd = h2f(d16);
        out[0] = (uint8_t)d16;
        out[1] = (uint8_t)(d16 >> 8);
        for (int i = 0; i < 32; ++i) {
            const float v = gauss(seed, stream, b * 32 + i, sd);
            const float q = dd > 0.0f ? clampf(rintf(v / dd), -127.0f, 127.0f) : 0.0f;
            out[2 + i] = (uint8_t)(int8_t)q;
        }
        for (int i = 0; i < 34; ++i) dst[b * 34 + i] = out[i];
    } else if constexpr (ENC == EMU_ENC_Q6_K) {
        uint8_t out[210];
        for (int i = 0; i < 210; ++i) out[i] = 0;
        float scale[16];
        float mx = 0.0f;
        for (int s = 0; s < 16; ++s) {
            float amax = 0.0f;
            for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(gauss(seed, stream, b * 256 + s * 16 + i, sd)));
            scale[s] = amax / 31.0f;
            mx = fmaxf(mx, scale[s]);
        }
        const uint16_t d16 = f2h(mx / 127.0f);
        const float dd = h2f(d16);
        int sc[16];
        for (int s = 0; s < 16; ++s) {
            sc[s] = dd > 0.0f ? (int)clampf(rintf(scale[s] / dd), -128.0f, 127.0f) : 0;
            out[192 + s] = (uint8_t)(int8_t)sc[s];
        }
        out[208] = (uint8_t)d16;
        out[209] = (uint8_t)(d16 >> 8);
        for (int e = 0; e < 256; ++e) {
            const float v = gauss(seed, stream, b * 256 + e, sd);
            const float m = dd * (float)sc[e / 16];
            const int q = m > 0.0f ? (int)clampf(rintf(v / m) + 32.0f, 0.0f, 63.0f) : 32;
            const int h = e / 128, r = e % 128, j = r / 32, l = r % 32;
            out[64 * h + l + 32 * (j & 1)] |= (uint8_t)((q & 15) << (4 * (j >> 1)));
            out[128 + 32 * h + l] |= (uint8_t)((q >> 4) << (2 * j));
        }
        for (int i = 0; i < 210; ++i) dst[b * 210 + i] = out[i];
    } else if constexpr (ENC == EMU_ENC_Q5_K) {
        uint8_t out[176];
        for (int i = 0; i < 176; ++i) out[i] = 0;
        float scale[8], mneg[8];
        float ms = 0.0f, mm = 0.0f;
        for (int s = 0; s < 8; ++s) {
            float lo = 0.0f, hi = -INFINITY;
            for (int i = 0; i < 32; ++i) {
                const float v = gauss(seed, stream, b * 256 + s * 32 + i, sd);
                lo = fminf(lo, v);
                hi = fmaxf(hi, v);
            }
            scale[s] = (hi - lo) / 31.0f;
            mneg[s] = -lo;
            ms = fmaxf(ms, scale[s]);
            mm = fmaxf(mm, mneg[s]);
        }
        const uint16_t d16 = f2h(ms / 63.0f), m16 = f2h(mm / 63.0f);
        const float dd = h2f(d16), dm = h2f(m16);
        int sc[8], mi[8];
        for (int s = 0; s < 8; ++s) {
            sc[s] = dd > 0.0f ? (int)clampf(rintf(scale[s] / dd), 0.0f, 63.0f) : 0;
            mi[s] = dm > 0.0f ? (int)clampf(rintf(mneg[s] / dm), 0.0f, 63.0f) : 0;
        }
        out[0] = (uint8_t)d16;
        out[1] = (uint8_t)(d16 >> 8);
        out[2] = (uint8_t)m16;
        out[3] = (uint8_t)(m16 >> 8);
        uint8_t *packed = out + 4;
        for (int j = 0; j < 4; ++j) {
            packed[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            packed[j + 4] = (uint8_t)((mi[j] & 63) | ((mi[j + 4] >> 4) << 6));
            packed[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mi[j + 4] & 15) << 4));
        }
        for (int e = 0; e < 256; ++e) {
            const int s = e / 32, g = e / 64, half = (e / 32) & 1, l = e % 32;
            const float v = gauss(seed, stream, b * 256 + e, sd);
            const float scl = dd * (float)sc[s];
            const int q = scl > 0.0f ? (int)clampf(rintf((v + dm * (float)mi[s]) / scl), 0.0f, 31.0f) : 0;
            out[48 + 32 * g + l] |= (uint8_t)((q & 15) << (4 * half));
            out[16 + l] |= (uint8_t)((q >> 4) << (2 * g + half));
        }
        for (int i = 0; i < 176; ++i) dst[b * 176 + i] = out[i];
    } else { // Q2_K
        uint8_t out[84];
        for (int i = 0; i < 84; ++i) out[i] = 0;
        float scale[16], mneg[16];
        float ms = 0.0f, mm = 0.0f;
        for (int s = 0; s < 16; ++s) {
            float lo = 0.0f, hi = -INFINITY;
            for (int i = 0; i < 16; ++i) {
                const float v = gauss(seed, stream, b * 256 + s * 16 + i, sd);
                lo = fminf(lo, v);
                hi = fmaxf(hi, v);
            }
            scale[s] = (hi - lo) / 3.0f;
            mneg[s] = -lo;
            ms = fmaxf(ms, scale[s]);
            mm = fmaxf(mm, mneg[s]);
        }
        const uint16_t d16 = f2h(ms / 15.0f), m16 = f2h(mm / 15.0f);
        const float dd = h2f(d16), dm = h2f(m16);
        int sc[16], mi[16];
        for (int s = 0; s < 16; ++s) {
            sc[s] = dd > 0.0f ? (int)clampf(rintf(scale[s] / dd), 0.0f, 15.0f) : 0;
            mi[s] = dm > 0.0f ? (int)clampf(rintf(mneg[s] / dm), 0.0f, 15.0f) : 0;
            out[s] = (uint8_t)(sc[s] | (mi[s] << 4));
        }
        out[80] = (uint8_t)d16;
        out[81] = (uint8_t)(d16 >> 8);
        out[82] = (uint8_t)m16;
        out[83] = (uint8_t)(m16 >> 8);
        for (int e = 0; e < 256; ++e) {
            const int N = e / 128, j = (e / 32) & 3, s = (e / 16) & 1, l = e % 16;
            const int si = e / 16;
            const float v = gauss(seed, stream, b * 256 + e, sd);
            const float scl = dd * (float)sc[si];
            const int q = scl > 0.0f ? (int)clampf(rintf((v + dm * (float)mi[si]) / scl), 0.0f, 3.0f) : 0;
            out[16 + 32 * N + 16 * s + l] |= (uint8_t)(q << (2 * j));
        }
        for (int i = 0; i < 84; ++i) dst[b * 84 + i] = out[i];
    }
}

__global__ void fill_kernel(float *p, size_t n, float v)
{
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) p[i] = v;
}

int synth_tensor(emu_ctx *ctx, int enc, uint8_t *dst, size_t bytes, uint64_t seed, uint64_t stream)
{
    uint32_t be = 0, bb = 0;
    int st = emu_block_layout(enc, &be, &bb);
    if (st != EMU_OK) return st;
    const size_t nblocks = bytes / bb;
    if (nblocks == 0) return EMU_OK;
    const dim3 grid((unsigned)((nblocks + kThreads - 1) / kThreads));
    const float sd = 0.02f;
    switch (enc) {
    case EMU_ENC_Q8_0: hipLaunchKernelGGL(synth_kernel<EMU_ENC_Q8_0>, grid, dim3(kThreads), 0, ctx->stream, dst, nblocks, seed, stream, sd); break;
    case EMU_ENC_Q6_K: hipLaunchKernelGGL(synth_kernel<EMU_ENC_Q6_K>, grid, dim3(kThreads), 0, ctx->stream, dst, nblocks, seed, stream, sd); break;
    case EMU_ENC_Q5_K: hipLaunchKernelGGL(synth_kernel<EMU_ENC_Q5_K>, grid, dim3(kThreads), 0, ctx->stream, dst, nblocks, seed, stream, sd); break;
    case EMU_ENC_Q2_K: hipLaunchKernelGGL(synth_kernel<EMU_ENC_Q2_K>, grid, dim3(kThreads), 0, ctx->stream, dst, nblocks, seed, stream, sd); break;
    default: return EMU_E_UNSUPPORTED;
    }
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

__global__ __launch_bounds__(kThreads) void synth_f32_kernel(float *dst, size_t n, uint64_t seed, uint64_t stream,
                                                             float sd)
{
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) dst[i] = gauss(seed, stream, i, sd);
}

// --------------------------------------------------------- step kernels --
// Tokens per partial-sum block of the multi-token matvec ([slice][matrix]
// [8 tokens][rows]).
constexpr int kMaxTokChain = 8;

// The MoE layer's gate (moe.rs:17-35, 132-138), in both forms:
//   Granite / OLMoE  router input = expert input = RMSNorm(r) * ffn_norm
//   Gemma            router input = (r * rscale) * (q / sqrt(W)),
//                    expert input = (r * q) * pre_ffw_norm_2,
//                    q = 1 / sqrt(sum r^2 / W + 1e-6)   (gemma_smoke.rs:57-86)
struct GateArgs {
    const float *state;  // [client][width] residual
    const float *gain;   // ffn_norm (Gemma: pre_ffw_norm_2)
    const float *rscale; // Gemma: the router input scale; else null
    const float *router; // [experts][width] f32
    const float *opart;  // chained: the o projection's partial sums; else null
    int o_nks;
    float o_scale;
    int width, experts, k;
    float eps;
    float *xn;           // [client][width] expert input
    EmuLimbPlanes xp;    // and, when xp.q is set, as the experts' limb planes
    // Gemma form, chained: the shared FFN's input rms(r) * ffn_gain as the
    // gate|up matvec's A operands (null: none)
    uint8_t *ffn_xa;
    float *ffn_xs;
    const float *ffn_gain;
    float ffn_eps;
    float *state_out;    // chained: r + o * o_scale
    float *logits;       // [client][experts] hand-off between workgroups
    uint32_t *counters;  // [client] arrivals, zero between launches
    int32_t *ids;
    float *weights;
    int32_t *ids_sorted; // and again in ascending expert id (null: not wanted)
    float *weights_sorted;
    ZipfRoute z;
};

// Grid (expert groups of four, clients), one wavefront per (expert, client).
// Lane l works on columns 4l + 256q of a row.  First the workgroup forms the
// client's row once, wavefront w taking the column groups q = w, w + 4, ...:
// the residual (chained: with the o projection's partial sums added), its
// sum of squares (folded per lane in column order, a butterfly per
// wavefront, the four wavefront sums added in order) and the router input,
// both into LDS -- every workgroup of a client forms the same row, the same
// instructions on the same data.  Then each wavefront dots its expert's
// router row (loaded at the start, with the row's operands) with the router
// input (fma per lane in column order, then a butterfly).  The logit goes to
// the device-coherent level by an agent-scope store, every store completes
// before the arrival counter moves, and the client's last workgroup to
// arrive routes (wavefront 0: softmax and top-k over the logits read back by
// agent-scope loads) while its wavefronts 1-3 write, chained, the updated
// residual and reset the counter.  No other workgroup of the client writes
// the residual, so all of them read it whole.  After arriving, wavefronts 1-3
// of every workgroup write the expert input (also as the experts' limb
// planes, one 256-column span per wavefront, and in the Gemma form the
// shared FFN's input as its matvec's operands), the spans dealt one per
// wavefront across the workgroups.
template <int NQ, bool GEMMA>
__global__ __launch_bounds__(kThreads) void moe_gate_kernel(GateArgs a)
{
    constexpr int NW = kThreads / EMU_WAVE;
    constexpr int QW = (NQ + NW - 1) / NW; // column groups per wavefront in the row phase
    __shared__ float p[256];
    __shared__ float red[NW];
    __shared__ uint32_t arrived;
    __shared__ __align__(16) float xrow[NQ * 4 * EMU_WAVE]; // the residual (chained: with o added)
    __shared__ __align__(16) float rrow[NQ * 4 * EMU_WAVE]; // the router input
    const int c = blockIdx.y, tid = threadIdx.x, lane = tid & (EMU_WAVE - 1), w = tid / EMU_WAVE;
    const int W = a.width, E = a.experts;
    const int e = NW * blockIdx.x + w;
    const float *xr = a.state + (size_t)c * W;
    const float *rr = a.router + (size_t)(e < E ? e : E - 1) * W; // a valid row; its result is dropped
    auto ld = [&](const float *base, int q) {
        const int i = 4 * lane + 4 * EMU_WAVE * q;
        return i < W ? *reinterpret_cast<const float4 *>(base + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    const bool chained = a.opart != nullptr;
    // The o projection's slices 1..kGateSlices-1 load with the first loads
    // (a slot past o_nks reads slice 0 and is not added): a loop over the
    // slices would wait a round trip per slice.
    constexpr int kGateSlices = 4;
    const size_t stride = (size_t)kMaxTokChain * W; // floats between slices
    float4 xv[QW], ov[QW], sv[QW], rw[NQ], os[kGateSlices - 1][QW];
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        const int q = w + NW * j;
        const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        xv[j] = q < NQ ? ld(xr, q) : z;
        ov[j] = q < NQ && chained ? ld(a.opart + (size_t)c * W, q) : z;
#pragma unroll
        for (int s = 1; s < kGateSlices; ++s)
            os[s - 1][j] = q < NQ && chained ? ld(a.opart + (s < a.o_nks ? s : 0) * stride + (size_t)c * W, q) : z;
        sv[j] = q < NQ ? ld(GEMMA ? a.rscale : a.gain, q) : z;
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) rw[q] = ld(rr, q);
    // this wavefront's first expert-input column group (wavefronts 1..NW-1)
    // and, in the Gemma form, its gains
    const int nq = (W + 4 * EMU_WAVE - 1) / (4 * EMU_WAVE);
    const int q0 = w > 0 ? (w - 1) * (int)gridDim.x + (int)blockIdx.x : nq;
    float4 g2 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), fg = g2;
    if (GEMMA && q0 < nq && 4 * lane + 4 * EMU_WAVE * q0 < W) {
        g2 = *reinterpret_cast<const float4 *>(a.gain + 4 * lane + 4 * EMU_WAVE * q0);
        if (a.ffn_xa) fg = *reinterpret_cast<const float4 *>(a.ffn_gain + 4 * lane + 4 * EMU_WAVE * q0);
    }
    if (chained) {
        // the o projection's slices added in order, then r + v * o_scale
        // (what the matvec's finishing pass would do)
#pragma unroll
        for (int s = 1; s < kGateSlices; ++s) {
            if (s >= a.o_nks) break; // uniform
#pragma unroll
            for (int j = 0; j < QW; ++j) {
                ov[j].x += os[s - 1][j].x;
                ov[j].y += os[s - 1][j].y;
                ov[j].z += os[s - 1][j].z;
                ov[j].w += os[s - 1][j].w;
            }
        }
        for (int s = kGateSlices; s < a.o_nks; ++s) { // wider o projections
#pragma unroll
            for (int j = 0; j < QW; ++j) {
                const int q = w + NW * j;
                if (q >= NQ) continue;
                const float4 t = ld(a.opart + s * stride + (size_t)c * W, q);
                ov[j].x += t.x;
                ov[j].y += t.y;
                ov[j].z += t.z;
                ov[j].w += t.w;
            }
        }
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            xv[j].x = emu_resid_add(xv[j].x, ov[j].x, a.o_scale);
            xv[j].y = emu_resid_add(xv[j].y, ov[j].y, a.o_scale);
            xv[j].z = emu_resid_add(xv[j].z, ov[j].z, a.o_scale);
            xv[j].w = emu_resid_add(xv[j].w, ov[j].w, a.o_scale);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        ss = __builtin_fmaf(xv[j].x, xv[j].x, ss);
        ss = __builtin_fmaf(xv[j].y, xv[j].y, ss);
        ss = __builtin_fmaf(xv[j].z, xv[j].z, ss);
        ss = __builtin_fmaf(xv[j].w, xv[j].w, ss);
    }
    ss = wave_sum(ss);
    if (lane == 0) red[w] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int k = 0; k < NW; ++k) tot += red[k];
    const float scale = 1.0f / sqrtf(tot / (float)W + (GEMMA ? 1e-6f : a.eps));
    const float qr = GEMMA ? scale / sqrtf((float)W) : scale;
    // router input: Gemma (r * rscale) * qr, else (r * scale) * gain
    auto rin = [&](float v, float s) { return GEMMA ? __fmul_rn(__fmul_rn(v, s), qr) : __fmul_rn(__fmul_rn(v, scale), s); };
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        const int q = w + NW * j;
        if (q >= NQ) continue;
        const int i = 4 * lane + 4 * EMU_WAVE * q; // zeros past the row
        *reinterpret_cast<float4 *>(xrow + i) = xv[j];
        *reinterpret_cast<float4 *>(rrow + i) = make_float4(rin(xv[j].x, sv[j].x), rin(xv[j].y, sv[j].y),
                                                            rin(xv[j].z, sv[j].z), rin(xv[j].w, sv[j].w));
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const float4 in = *reinterpret_cast<const float4 *>(rrow + 4 * lane + 4 * EMU_WAVE * q);
        acc = __builtin_fmaf(rw[q].x, in.x, acc);
        acc = __builtin_fmaf(rw[q].y, in.y, acc);
        acc = __builtin_fmaf(rw[q].z, in.z, acc);
        acc = __builtin_fmaf(rw[q].w, in.w, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0 && e < E) {
        // throughput runs: Zipf routing in place of the router's logit
        const float lg = a.z.s > 0.0f ? zipf_logit(a.z, c, e) : acc;
        __hip_atomic_store(a.logits + (size_t)c * E + e, lg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t *counter = a.counters + c;
    if (tid == 0) arrived = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const bool last = arrived == gridDim.x - 1; // uniform: from LDS
    if (last) {
        for (int j = tid; j < E; j += kThreads)
            p[j] = __hip_atomic_load(a.logits + (size_t)c * E + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (w == 0) {
            emu_route_token(p, E, a.k, a.ids + (size_t)c * a.k, a.weights + (size_t)c * a.k,
                            a.ids_sorted ? a.ids_sorted + (size_t)c * a.k : nullptr,
                            a.weights_sorted ? a.weights_sorted + (size_t)c * a.k : nullptr);
            return;
        }
        if (tid == EMU_WAVE) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (chained) { // the updated residual, once every workgroup has read it
            for (int q = w - 1; q < nq; q += NW - 1) {
                const int i = 4 * lane + 4 * EMU_WAVE * q;
                if (i < W) *reinterpret_cast<float4 *>(a.state_out + (size_t)c * W + i) = *reinterpret_cast<const float4 *>(xrow + i);
            }
        }
    } else if (w == 0) {
        return;
    }
    // Wavefronts 1..NW-1 of every workgroup of the client: the expert input
    // (and in the Gemma form the shared FFN's operands), one column group
    // each, groups dealt across the workgroups first.  It does not depend on
    // the routes, so only the routing waits for the last arrival.
    for (int q = q0, j = 0; q < nq; q += (NW - 1) * gridDim.x, ++j) {
        const int i = 4 * lane + 4 * EMU_WAVE * q;
        const bool live = i < W;
        if (GEMMA && j > 0 && live) { // further groups (narrow grids): gains loaded here
            g2 = *reinterpret_cast<const float4 *>(a.gain + i);
            if (a.ffn_xa) fg = *reinterpret_cast<const float4 *>(a.ffn_gain + i);
        }
        const float4 x4 = *reinterpret_cast<const float4 *>(xrow + i);
        float4 v;
        if constexpr (GEMMA) { // (r * q) * gain2
            v = make_float4(__fmul_rn(__fmul_rn(x4.x, scale), g2.x), __fmul_rn(__fmul_rn(x4.y, scale), g2.y),
                            __fmul_rn(__fmul_rn(x4.z, scale), g2.z), __fmul_rn(__fmul_rn(x4.w, scale), g2.w));
        } else { // the router input is the expert input
            v = *reinterpret_cast<const float4 *>(rrow + i);
        }
        if (live) *reinterpret_cast<float4 *>(a.xn + (size_t)c * W + i) = v;
        if (a.xp.q) emu_span_limbs_wave(v, live, c, q, a.xp); // span q of the experts' limb planes
        if (GEMMA && a.ffn_xa) { // the shared FFN's input, as the link kernel would form it
            const float s2 = 1.0f / sqrtf(tot / (float)W + a.ffn_eps);
            const float4 u = make_float4(__fmul_rn(__fmul_rn(x4.x, s2), fg.x), __fmul_rn(__fmul_rn(x4.y, s2), fg.y),
                                         __fmul_rn(__fmul_rn(x4.z, s2), fg.z), __fmul_rn(__fmul_rn(x4.w, s2), fg.w));
            emu_emit_limbs4(u, live, i, c, a.ffn_xa, a.ffn_xs);
        }
    }
}

// Launch of the gate: NQ = 256-column groups per row, up to 16 (width 4096).
template <bool GEMMA> int launch_gate(emu_ctx *ctx, const GateArgs &a, int n)
{
    const dim3 grid((unsigned)((a.experts + 3) / 4), (unsigned)n);
    const int nq = (a.width + 255) / 256;
    if (nq <= 1) hipLaunchKernelGGL((moe_gate_kernel<1, GEMMA>), grid, dim3(kThreads), 0, ctx->stream, a);
    else if (nq <= 2) hipLaunchKernelGGL((moe_gate_kernel<2, GEMMA>), grid, dim3(kThreads), 0, ctx->stream, a);
    else if (nq <= 4) hipLaunchKernelGGL((moe_gate_kernel<4, GEMMA>), grid, dim3(kThreads), 0, ctx->stream, a);
    else if (nq <= 8) hipLaunchKernelGGL((moe_gate_kernel<8, GEMMA>), grid, dim3(kThreads), 0, ctx->stream, a);
    else if (nq <= 12) hipLaunchKernelGGL((moe_gate_kernel<12, GEMMA>), grid, dim3(kThreads), 0, ctx->stream, a);
    else if (nq <= 16) hipLaunchKernelGGL((moe_gate_kernel<16, GEMMA>), grid, dim3(kThreads), 0, ctx->stream, a);
    else return EMU_E_CONFIG;
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

// Copy of one layer's routes into the session's route trace, slot
// steps[c] % capacity (one thread per (client, slot)).
__global__ void trace_routes_kernel(const int32_t *ids, const float *weights, int n, int k, int layer, int layers,
                                    const uint32_t *steps, int capacity, int32_t *t_ids, float *t_w)
{
    const int i = threadIdx.x;
    if (i >= n * k) return;
    const int c = i / k, r = i % k;
    const size_t slot = steps[c] % (uint32_t)capacity;
    const size_t at = ((slot * layers + layer) * n + c) * k + r;
    t_ids[at] = ids[i];
    t_w[at] = weights[i];
}

// Embedding row of tokens[c]: a unit-per-thread decode of one row.
template <class F>
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint8_t *embed, size_t row_bytes, int hidden,
                                                         const uint32_t *tokens, float *state, float scale)
{
    const int c = blockIdx.y;
    const int u = blockIdx.x * kThreads + threadIdx.x;
    const int units = hidden / F::BE * F::UPB;
    if (u >= units) return;
    const int blk = u / F::UPB, sub = u % F::UPB;
    const uint8_t *row = embed + (size_t)tokens[c] * row_bytes;
    typename F::Raw raw;
    F::load(row + (size_t)blk * F::BB, sub, raw);
    float *out = state + (size_t)c * hidden + blk * F::BE;
#pragma unroll
    for (int g = 0; g < F::G; ++g) {
        const Grp gp = F::group(raw, sub, g);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float v = grp_weight_exact<F::BIAS>(gp, i);
            out[F::col(sub, g) + i] = scale != 0.0f ? v * scale : v; // model.rs:196-213: value * 12.0
        }
    }
}

// Greedy select + advance, one workgroup per client, over the selection keys
// the output matvec left per wavefront (key_slots of them per client).
// ctrl[0] = prompt length (0: every step is a free-running decode step),
// ctrl[1] = capacity of the generated-token history per client.
__global__ __launch_bounds__(1024) void finalize_kernel(const uint64_t *keys, int key_stride, int key_slots,
                                                        int tie_last, const uint32_t *prompt, int prompt_stride,
                                                        uint32_t *hist, const uint32_t *ctrl,
                                                        uint32_t *tokens, uint32_t *positions,
                                                        uint32_t *steps, uint32_t *last)
{
    __shared__ uint64_t red[16];
    const int c = blockIdx.x;
    const uint64_t *kr = keys + (size_t)c * key_stride;
    uint64_t best = 0;
    for (int i = threadIdx.x; i < key_slots; i += blockDim.x) {
        const uint64_t k = kr[i];
        best = k > best ? k : best;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off, 64);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) best = red[i] > best ? red[i] : best;
    const uint32_t lo = (uint32_t)best;
    const uint32_t am = tie_last ? lo : 0xffffffffu - lo;
    const uint32_t plen = ctrl[0], cap = ctrl[1];
    const uint32_t s = steps[c];
    uint32_t next = am;
    if (s + 1 < plen) next = prompt[(size_t)c * prompt_stride + s + 1];
    if (s + 1 >= plen) {
        const uint32_t gi = s + 1 - plen;
        if (gi < cap) hist[(size_t)c * cap + gi] = am;
    }
    tokens[c] = next;
    last[c] = am;
    positions[c] = positions[c] + 1;
    steps[c] = s + 1;
}

template <class F>
int launch_embed(emu_ctx *ctx, const emu_model *m, const uint32_t *tokens, float *state, uint32_t n)
{
    const int units = (int)(m->cfg.hidden / F::BE * F::UPB);
    dim3 grid((units + kThreads - 1) / kThreads, n);
    hipLaunchKernelGGL(embed_kernel<F>, grid, dim3(kThreads), 0, ctx->stream, m->base + m->off_embed,
                       m->rb_h, (int)m->cfg.hidden, tokens, state, m->cfg.embed_scale);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

EmuAttnLaunch layer_attn(emu_session *s, uint32_t layer)
{
    const emu_model *m = s->m;
    const emu_model_config &c = m->cfg;
    const uint32_t hd = c.head_dim;
    const int smol = c.style == EMU_STYLE_SMOL;
    EmuAttnLaunch al{};
    al.qkv = s->qkv;
    al.k_cache = s->k_cache;
    al.v_cache = s->v_cache;
    al.positions = s->positions;
    al.rope = s->rope;
    al.q_norm = c.qk_norm ? reinterpret_cast<const float *>(m->base + m->off_q_norm) : nullptr;
    al.k_norm = c.qk_norm ? reinterpret_cast<const float *>(m->base + m->off_k_norm) : nullptr;
    al.eps = c.eps;
    al.score_mul = smol ? 1.0f / sqrtf((float)hd) : 0.0f;
    al.score_div = smol ? 0.0f : sqrtf((float)hd);
    al.rope_fma = smol;
    al.interleaved = 0;
    if (m->moe()) { // spm-granite-moe/src/attention.rs:12-26, 40-46
        al.score_mul = c.score_mul != 0.0f ? c.score_mul : 1.0f / sqrtf((float)hd);
        al.score_div = 0.0f;
        al.interleaved = c.rope_neox ? 0 : 1;
        if (m->gemma() && c.window) { // local layers: the last `window` positions, the local RoPE base
            const bool global = (layer + 1) % c.global_every == 0;
            al.window = global ? 0 : (int)c.window;
            al.rope = global ? s->rope2 : s->rope;
        }
    }
    al.heads = (int)c.heads;
    al.kv_heads = (int)c.kv_heads;
    al.head_dim = (int)hd;
    al.layers = (int)c.layers;
    al.layer = (int)layer;
    al.context = (int)s->context;
    al.clients = (int)s->n;
    al.kv_f16 = s->kv_f16;
    al.partial = s->partial;
    al.counters = s->counters;
    al.out = s->attn;
    return al;
}

// The step's interval marks (emu_session_time_layers), a no-op otherwise.
int mark(emu_session *s, size_t i)
{
    if (!s->marking) return EMU_OK;
    if (i >= s->marks.size()) return EMU_E_CONFIG;
    EMU_HIP(s->m->ctx, hipEventRecord(s->marks[i], s->m->ctx->stream));
    return EMU_OK;
}

int launch_finalize(emu_session *s, int slots)
{
    emu_ctx *ctx = s->m->ctx;
    const int smol = s->m->cfg.style == EMU_STYLE_SMOL;
    if (slots <= 0 || slots > (int)s->key_stride) return EMU_E_CONFIG;
    hipLaunchKernelGGL(finalize_kernel, dim3(s->n), dim3(1024), 0, ctx->stream, s->keys, (int)s->key_stride, slots,
                       smol ? 1 : 0, s->prompt, (int)s->context, s->hist, s->ctrl, s->tokens, s->positions,
                       s->steps, s->last);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

// Whether the step's matvecs take the chained multi-token form (mfma.hip):
// several clients, Q6_K, and every matvec's columns a multiple of its slice.
bool mfma_chain(const emu_model *m, uint32_t n)
{
    const emu_model_config &c = m->cfg;
    const int QW = (int)(c.heads * c.head_dim), KW = (int)(c.kv_heads * c.head_dim);
    return !m->moe() && n >= 2 && emu_mfma_supports(c.encoding, (int)c.hidden, (int)n) &&
           emu_mfma_supports(c.encoding, QW, (int)n) && emu_mfma_supports(c.encoding, (int)c.ffn, (int)n) &&
           (QW + 2 * KW) % 16 == 0 && (QW + 2 * KW) <= (int)c.ffn;
}

// Workspace of the chained form: operands of up to the widest input, and the
// largest matvec's partial sums.
size_t mfma_chain_bytes(const emu_model *m)
{
    const emu_model_config &c = m->cfg;
    const int H = (int)c.hidden, QW = (int)(c.heads * c.head_dim), KW = (int)(c.kv_heads * c.head_dim),
              F = (int)c.ffn;
    const int cap = std::max(H, std::max(QW, F));
    size_t part = emu_mfma_part_bytes(QW + 2 * KW, H, 1);
    part = std::max(part, emu_mfma_part_bytes(H, QW, 1));
    part = std::max(part, emu_mfma_part_bytes(F, H, 2));
    part = std::max(part, emu_mfma_part_bytes(H, F, 1));
    part = std::max(part, emu_mfma_part_bytes((int)c.vocab, H, 1));
    return emu_mfma_chain_bytes(cap, part);
}

// The layers, output matvec and selection of a multi-token step, chained:
// each link kernel finishes the previous matvec (residual add / SwiGLU /
// q|k|v sums) and prepares the next one's operands, RMS norm included.
int run_chain(emu_session *s)
{
    emu_model *m = s->m;
    emu_ctx *ctx = m->ctx;
    const emu_model_config &c = m->cfg;
    const int H = (int)c.hidden, QW = (int)(c.heads * c.head_dim), KW = (int)(c.kv_heads * c.head_dim),
              F = (int)c.ffn;
    const int n = (int)s->n, cap = std::max(H, std::max(QW, F));
    uint32_t be = 0, bb = 0;
    emu_block_layout(c.encoding, &be, &bb);
    const float *attn_norm = reinterpret_cast<const float *>(m->base + m->off_attn_norm);
    const float *ffn_norm = reinterpret_cast<const float *>(m->base + m->off_ffn_norm);
    const float *out_norm = reinterpret_cast<const float *>(m->base + m->off_out_norm);
    int st = EMU_OK;
    auto link = [&](int mode, int nks, int nmat, float *h, const float *x, int cols, const float *gain, bool limbs) {
        EmuMfmaLink l{};
        l.mode = mode;
        l.from_part = mode != 0;
        l.part_nks = nks;
        l.part_nmat = nmat;
        l.h = h;
        l.x = x;
        l.cols = cols;
        l.cols_cap = cap;
        l.n_tok = n;
        l.gain = gain;
        l.eps = c.eps;
        l.limbs = limbs;
        l.span = 1;
        l.defer_norm = gain ? 1 : 0; // the consuming span matvec applies the RMS factor
        return emu_mfma_link(ctx, l);
    };
    // span: the operands come from a link (one scale per 256-column span);
    // the o projection's come from the attention, per 16-column sub-block.
    // norm: that link normalised, its RMS factor left to this matvec.
    auto matvec = [&](const uint8_t *w, const uint8_t *w_up, size_t rb, int rows, int cols, int *nks, bool span,
                      bool norm) {
        QmvArgs q{};
        q.span_norm = norm ? 1 : 0;
        q.eps = c.eps;
        q.w = m->mm_or(w, &q.mfma_major);
        q.w_up = w_up ? m->mm_or(w_up, &q.mfma_major) : nullptr;
        q.row_bytes = rb;
        q.rows = rows;
        q.cols = cols;
        q.nb = cols / (int)be;
        q.span_scales = span ? 1 : 0;
        return emu_mfma_matvec(ctx, q, n, cap, nks);
    };
    uint8_t *xa = nullptr;
    float *xs = nullptr, *part = nullptr;
    emu_mfma_buffers(ctx, cap, &xa, &xs, &part);
    // the first layer's q|k|v input: the embeddings, normalised
    if ((st = link(0, 0, 1, nullptr, s->state, H, attn_norm, true)) != EMU_OK) return st;
    for (uint32_t layer = 0; layer < c.layers; ++layer) {
        const uint8_t *lw = m->base + m->off_layers + (size_t)layer * m->layer_bytes;
        int nks = 0;
        if ((st = matvec(lw + m->off_q, nullptr, m->rb_h, QW + 2 * KW, H, &nks, true, true)) != EMU_OK) return st;
        // Attention adds the q|k|v slices itself and writes the o
        // projection's operands: no link kernel on either side of it.
        EmuAttnLaunch al = layer_attn(s, layer);
        al.qkv = part;
        al.qkv_slices = nks;
        al.qkv_client_stride = QW + 2 * KW;
        al.qkv_slice_stride = (size_t)8 * (QW + 2 * KW);
        al.xa = xa;
        al.xs = xs;
        if ((st = emu_launch_attn(ctx, al)) != EMU_OK) return st;
        if ((st = matvec(lw + m->off_o, nullptr, m->rb_q, H, QW, &nks, false, false)) != EMU_OK) return st;
        if ((st = link(1, nks, 1, s->state, nullptr, H, ffn_norm + (size_t)layer * H, true)) != EMU_OK) return st;
        if ((st = matvec(lw + m->off_g, lw + m->off_u, m->rb_h, F, H, &nks, true, true)) != EMU_OK) return st;
        if ((st = link(2, nks, 2, nullptr, nullptr, F, nullptr, true)) != EMU_OK) return st;
        if ((st = matvec(lw + m->off_d, nullptr, m->rb_f, H, F, &nks, true, false)) != EMU_OK) return st;
        const float *next = layer + 1 < c.layers ? attn_norm + (size_t)(layer + 1) * H : out_norm;
        if ((st = link(1, nks, 1, s->state, nullptr, H, next, true)) != EMU_OK) return st;
        if ((st = mark(s, layer + 1)) != EMU_OK) return st;
    }
    QmvArgs out{};
    out.w = m->mm_or(m->base + (c.tied ? m->off_embed : m->off_output), &out.mfma_major);
    out.row_bytes = m->rb_h;
    out.rows = (int)c.vocab;
    out.cols = H;
    out.nb = H / (int)be;
    out.y = s->logits;
    out.keys = s->keys;
    out.key_stride = (int)s->key_stride;
    out.tie_last = c.style == EMU_STYLE_SMOL ? 1 : 0;
    out.span_scales = 1;
    out.span_norm = 1;
    out.eps = c.eps;
    if ((st = emu_mfma_matvec(ctx, out, n, cap, nullptr)) != EMU_OK) return st;
    int slots = 0;
    if ((st = emu_mfma_finish(ctx, out, n, cap, &slots)) != EMU_OK) return st;
    if ((st = launch_finalize(s, slots)) != EMU_OK) return st;
    return mark(s, c.layers + 1);
}

// The layers, output matvec and selection of a mixture-of-experts step
// (spm-granite-moe/src/model.rs:330-411): attention as in the dense step but
// with adjacent-pair RoPE and score * score_mul, residual adds r + v * 0.22,
// then per layer RMSNorm, the f32 router, top-k routing and the selected
// experts, and logits from the tied embedding divided by logit_div.
// The chained step: every projection on the matrix cores (the gate adds
// the o projection's partial sums to the residual; the Gemma form's shared
// FFN chains link -> gate|up -> link -> down, its down projection's partial
// sums joining the residual in the next layer's link).
bool moe_chain(const emu_model *m, uint32_t n)
{
    const emu_model_config &c = m->cfg;
    const int QW = (int)(c.heads * c.head_dim);
    const bool shared = !m->gemma() || c.shared_ff == 0 ||
                        (emu_mfma_shape_ok(c.encoding, (int)c.shared_ff) && c.shared_ff <= std::max(c.hidden, (uint32_t)QW));
    return m->moe() && n >= 1 && n <= 8 && shared && emu_mfma_shape_ok(c.encoding, (int)c.hidden) &&
           emu_mfma_shape_ok(c.encoding, QW) && QW % 16 == 0;
}

size_t moe_chain_bytes(const emu_model *m)
{
    const emu_model_config &c = m->cfg;
    const int H = (int)c.hidden, QW = (int)(c.heads * c.head_dim), KW = (int)(c.kv_heads * c.head_dim);
    size_t part = std::max(emu_mfma_part_bytes(QW + 2 * KW, H, 1), emu_mfma_part_bytes(H, QW, 1));
    if (m->gemma() && c.shared_ff) {
        part = std::max(part, emu_mfma_part_bytes((int)c.shared_ff, H, 2));
        part = std::max(part, emu_mfma_part_bytes(H, (int)c.shared_ff, 1));
    }
    return emu_mfma_chain_bytes(std::max(H, QW), part);
}

int run_moe(emu_session *s)
{
    emu_model *m = s->m;
    emu_ctx *ctx = m->ctx;
    const emu_model_config &c = m->cfg;
    const uint32_t H = c.hidden, QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim;
    const uint32_t E = c.n_experts, K = c.experts_used;
    const int n = (int)s->n;
    uint32_t be = 0, bb = 0;
    emu_block_layout(c.encoding, &be, &bb);
    const float *attn_norm = reinterpret_cast<const float *>(m->base + m->off_attn_norm);
    const float *ffn_norm = reinterpret_cast<const float *>(m->base + m->off_ffn_norm);
    int st = EMU_OK;
    // Chained at 2-8 clients: the q|k|v and o projections on the matrix
    // cores with the attention adding q|k|v's partial sums and writing o's
    // operands, and the gate kernel adding o's partial sums to the residual
    // (no finishing or link launch around the attention).
    const bool chain = !s->f32() && moe_chain(m, s->n);
    const int cap = (int)std::max(H, QW);
    uint8_t *xa = nullptr;
    float *xs = nullptr, *part = nullptr;
    if (chain) emu_mfma_buffers(ctx, cap, &xa, &xs, &part);
    int sd_nks = 0; // chained Gemma form: the previous layer's shared down projection, as partial sums
    for (uint32_t layer = 0; layer < c.layers; ++layer) {
        const uint8_t *lw = m->base + m->off_layers + (size_t)layer * m->layer_bytes;
        const float *opart = nullptr;
        int o_nks = 0;
        const ZipfRoute zr{s->zipf_s, s->zipf_seed, s->positions, (int)layer};
        if (chain) {
            EmuMfmaLink l{};
            l.mode = 0; // input: the residual, normalised, as operands
            l.x = s->state;
            l.cols = (int)H;
            l.cols_cap = cap;
            l.n_tok = n;
            l.gain = attn_norm + (size_t)layer * H;
            l.eps = c.eps;
            l.limbs = true;
            l.span = 1;
            l.defer_norm = 1; // the q|k|v matvec applies the RMS factor
            if (layer > 0) { // the previous layer's (shared down and) expert sum join the residual here
                l.h = s->state;
                l.d_part = sd_nks > 0;
                l.d_nks = sd_nks;
                l.d_scale = c.residual_scale;
                l.m_contrib = emu_moe_contrib(s->moe_ws, (uint32_t)n, K, c.expert_ff);
                l.m_ids = s->rids_s;
                l.m_wts = s->rwts_s;
                l.m_sorted = 1;
                l.m_k = (int)K;
                l.m_experts = (int)E;
                l.m_scale = c.residual_scale;
            }
            if ((st = emu_mfma_link(ctx, l)) != EMU_OK) return st;
            QmvArgs q{};
            q.w = m->mm_or(lw + m->off_q, &q.mfma_major);
            q.row_bytes = m->rb_h;
            q.rows = (int)(QW + 2 * KW);
            q.cols = (int)H;
            q.nb = (int)(H / be);
            q.span_scales = 1; // the link's operands
            q.span_norm = l.defer_norm;
            q.eps = c.eps;
            int nks = 0;
            if ((st = emu_mfma_matvec(ctx, q, n, cap, &nks)) != EMU_OK) return st;
            EmuAttnLaunch al = layer_attn(s, layer);
            al.qkv = part;
            al.qkv_slices = nks;
            al.qkv_client_stride = (int)(QW + 2 * KW);
            al.qkv_slice_stride = (size_t)kMaxTokChain * (QW + 2 * KW);
            al.xa = xa;
            al.xs = xs;
            if ((st = emu_launch_attn(ctx, al)) != EMU_OK) return st;
            QmvArgs o{};
            o.w = m->mm_or(lw + m->off_o, &o.mfma_major);
            o.row_bytes = m->rb_q;
            o.rows = (int)H;
            o.cols = (int)QW;
            o.nb = (int)(QW / be);
            if ((st = emu_mfma_matvec(ctx, o, n, cap, &o_nks)) != EMU_OK) return st;
            opart = part;
        } else {
        QmvArgs a{};
        a.w = lw + m->off_q;
        a.row_bytes = m->rb_h;
        a.rows = (int)(QW + 2 * KW);
        a.cols = (int)H;
        a.nb = (int)(H / be);
        a.x = s->state;
        a.gain = attn_norm + (size_t)layer * H;
        a.eps = c.eps;
        a.y = s->qkv;
        a.f32_act = s->f32();
        if ((st = emu_launch_qmv(ctx, c.encoding, a, n)) != EMU_OK) return st;
        if ((st = emu_launch_attn(ctx, layer_attn(s, layer))) != EMU_OK) return st;
        QmvArgs o{};
        o.f32_act = s->f32();
        o.w = lw + m->off_o;
        o.row_bytes = m->rb_q;
        o.rows = (int)H;
        o.cols = (int)QW;
        o.nb = (int)(QW / be);
        o.x = s->attn;
        o.y = s->state;
        o.accumulate = 1;
        o.acc_scale = c.residual_scale;
        if ((st = emu_launch_qmv(ctx, c.encoding, o, n)) != EMU_OK) return st;
        }
        emu_moe_desc d{};
        d.enc_gate_up = c.expert_encoding;
        d.enc_down = m->gemma() ? c.expert_down_encoding : c.expert_encoding;
        d.d_gate = lw + m->off_ge;
        d.d_up = m->gemma() ? nullptr : lw + m->off_ue; // gemma: fused gate|up rows per expert
        d.d_down = lw + m->off_de;
        d.d_down_scale = m->gemma() ? reinterpret_cast<const float *>(lw + m->off_ds) : nullptr;
        d.n_experts = E;
        d.width = H;
        d.ff = c.expert_ff;
        d.k = K;
        d.act = m->gemma() ? EMU_ACT_GELU_TANH : EMU_ACT_SILU;
        d.flags = s->f32() ? EMU_MOE_F32_ACT : 0u;
        // the gate writes the experts' limb planes of the expert input
        const bool planes = emu_moe_mma_form(&d);
        GateArgs ga{};
        if (planes) ga.xp = emu_moe_x_planes(s->moe_ws, (uint32_t)n, K, H, c.expert_ff);
        ga.state = s->state;
        ga.router = reinterpret_cast<const float *>(lw + m->off_r);
        ga.width = (int)H;
        ga.experts = (int)E;
        ga.k = (int)K;
        ga.eps = c.eps;
        ga.xn = s->xn;
        ga.logits = s->rlog;
        ga.counters = s->gate_counters;
        ga.ids = s->rids;
        ga.weights = s->rwts;
        ga.ids_sorted = s->rids_s;
        ga.weights_sorted = s->rwts_s;
        ga.z = zr;
        if (m->gemma()) {
            // router and expert inputs from the residual before the shared FFN
            ga.gain = reinterpret_cast<const float *>(m->base + m->off_ffn_norm2) + (size_t)layer * H;
            ga.rscale = reinterpret_cast<const float *>(lw + m->off_rs);
            ga.opart = opart;
            ga.o_nks = o_nks;
            ga.o_scale = c.residual_scale;
            ga.state_out = s->state;
            if (c.shared_ff && chain) { // the gate writes the shared FFN's operands
                ga.ffn_xa = xa;
                ga.ffn_xs = xs;
                ga.ffn_gain = ffn_norm + (size_t)layer * H;
                ga.ffn_eps = c.eps;
            }
            if ((st = launch_gate<true>(ctx, ga, n)) != EMU_OK) return st;
            if (c.shared_ff && chain) {
                // (gate's operands) -> gate|up -> link (GeGLU) -> down; the
                // down's partial sums join the residual in the next layer's
                // link (the last layer's here, before the expert sum)
                QmvArgs g{};
                g.w = m->mm_or(lw + m->off_sg, &g.mfma_major);
                g.w_up = m->mm_or(lw + m->off_su, &g.mfma_major);
                g.row_bytes = m->rb_h;
                g.rows = (int)c.shared_ff;
                g.cols = (int)H;
                g.nb = (int)(H / be);
                int gu_nks = 0;
                if ((st = emu_mfma_matvec(ctx, g, n, cap, &gu_nks)) != EMU_OK) return st;
                EmuMfmaLink la{};
                la.mode = 2; // the gate/up pair's activation
                la.from_part = true;
                la.part_nks = gu_nks;
                la.part_nmat = 2;
                la.cols = (int)c.shared_ff;
                la.cols_cap = cap;
                la.n_tok = n;
                la.limbs = true;
                la.span = 1;
                la.act = EMU_ACT_GELU_TANH;
                if ((st = emu_mfma_link(ctx, la)) != EMU_OK) return st;
                QmvArgs dq{};
                dq.w = m->mm_or(lw + m->off_sd, &dq.mfma_major);
                dq.row_bytes = m->rb_sf;
                dq.rows = (int)H;
                dq.cols = (int)c.shared_ff;
                dq.nb = (int)(c.shared_ff / be);
                dq.y = s->state;
                dq.accumulate = 1;
                dq.acc_scale = c.residual_scale;
                dq.span_scales = 1; // the link's operands
                if ((st = emu_mfma_matvec(ctx, dq, n, cap, &sd_nks)) != EMU_OK) return st;
                if (layer + 1 == c.layers && (st = emu_mfma_finish(ctx, dq, n, cap, nullptr)) != EMU_OK) return st;
            } else if (c.shared_ff) {
                QmvArgs g{};
                g.w = lw + m->off_sg;
                g.w_up = lw + m->off_su;
                g.row_bytes = m->rb_h;
                g.rows = (int)c.shared_ff;
                g.cols = (int)H;
                g.nb = (int)(H / be);
                g.x = s->state;
                g.gain = ffn_norm + (size_t)layer * H;
                ga.eps = c.eps;
                g.y = s->act;
                g.act = EMU_ACT_GELU_TANH;
                if ((st = emu_launch_qmv(ctx, c.encoding, g, n)) != EMU_OK) return st;
                QmvArgs d{};
                d.w = lw + m->off_sd;
                d.row_bytes = m->rb_sf;
                d.rows = (int)H;
                d.cols = (int)c.shared_ff;
                d.nb = (int)(c.shared_ff / be);
                d.x = s->act;
                d.y = s->state;
                d.accumulate = 1;
                d.acc_scale = c.residual_scale;
                if ((st = emu_launch_qmv(ctx, c.encoding, d, n)) != EMU_OK) return st;
            }
        } else {
            ga.gain = ffn_norm + (size_t)layer * H;
            ga.opart = opart;
            ga.o_nks = o_nks;
            ga.o_scale = c.residual_scale;
            ga.state_out = s->state;
            if ((st = launch_gate<false>(ctx, ga, n)) != EMU_OK) return st;
        }
        if (s->trace_cap) {
            hipLaunchKernelGGL(trace_routes_kernel, dim3(1), dim3(64), 0, ctx->stream, s->rids, s->rwts, n, (int)K,
                               (int)layer, (int)c.layers, s->steps, (int)s->trace_cap, s->trace_ids, s->trace_w);
            EMU_LAUNCH_CHECK(ctx);
        }
        // the weighted expert sum lands on the residual stream as add_scaled does
        // chained: the next layer's link adds the expert sum (the last layer's
        // is combined here, for the output matvec)
        const bool combine = !chain || layer + 1 == c.layers;
        // with the expert cache: this layer's expert addresses from the
        // device policy over the routes just written
        const uint8_t *const *table = nullptr;
        if (s->cache && (st = emu_cache_plan(s->cache, layer, s->rids_s, n * (int)K, &table)) != EMU_OK) return st;
        if ((st = emu_moe_ffn_resid(ctx, &d, s->xn, (uint32_t)n, s->rids_s, s->rwts_s, s->moe_ws, s->moe_ws_bytes,
                                    s->state, c.residual_scale, combine, planes, s->span_counters, table)) != EMU_OK)
            return st;
        if ((st = mark(s, layer + 1)) != EMU_OK) return st;
    }
    QmvArgs out{};
    out.w = m->base + (c.tied ? m->off_embed : m->off_output); // Granite: tied (model.rs:403-407)
    if (chain) out.w = m->mm_or(out.w, &out.mfma_major); // the matrix-core launch below reads either order
    out.row_bytes = m->rb_h;
    out.rows = (int)c.vocab;
    out.cols = (int)H;
    out.nb = (int)(H / be);
    out.x = s->state;
    out.gain = reinterpret_cast<const float *>(m->base + m->off_out_norm);
    out.eps = c.eps;
    out.y = s->logits;
    out.keys = s->keys;
    out.key_stride = (int)s->key_stride;
    out.tie_last = 0; // top_k: ties to the lowest index (math.rs:35-40)
    out.out_div = c.logit_div;
    out.softcap = c.logit_softcap;
    out.f32_act = s->f32();
    out.span_scales = chain ? 1 : 0;
    int slots = 0;
    // chained: the output on the matrix cores at any client count, as the
    // projections before it (a client's logits do not depend on the batch)
    if ((st = chain ? emu_launch_mfma(ctx, c.encoding, out, n, &slots) : emu_launch_qmv(ctx, c.encoding, out, n, &slots)) !=
        EMU_OK)
        return st;
    if ((st = launch_finalize(s, slots)) != EMU_OK) return st;
    return mark(s, c.layers + 1);
}

int run_step(emu_session *s)
{
    emu_model *m = s->m;
    emu_ctx *ctx = m->ctx;
    const emu_model_config &c = m->cfg;
    const uint32_t H = c.hidden, hd = c.head_dim, QW = c.heads * hd, KW = c.kv_heads * hd, F = c.ffn;
    const int n = (int)s->n;
    int st = EMU_OK;
    switch (c.encoding) {
    case EMU_ENC_Q6_K: st = launch_embed<FmtQ6K>(ctx, m, s->tokens, s->state, s->n); break;
    case EMU_ENC_Q8_0: st = launch_embed<FmtQ8_0>(ctx, m, s->tokens, s->state, s->n); break;
    case EMU_ENC_Q5_K: st = launch_embed<FmtQ5K>(ctx, m, s->tokens, s->state, s->n); break;
    case EMU_ENC_Q2_K: st = launch_embed<FmtQ2K>(ctx, m, s->tokens, s->state, s->n); break;
    default: return EMU_E_UNSUPPORTED;
    }
    if (st != EMU_OK) return st;
    if ((st = mark(s, 0)) != EMU_OK) return st;
    if (m->moe()) return run_moe(s);
    const bool f32 = s->f32();
    if (!f32 && mfma_chain(m, s->n)) return run_chain(s);
    uint32_t be = 0, bb = 0;
    emu_block_layout(c.encoding, &be, &bb);
    const int smol = c.style == EMU_STYLE_SMOL;
    for (uint32_t layer = 0; layer < c.layers; ++layer) {
        const uint8_t *lw = m->base + m->off_layers + (size_t)layer * m->layer_bytes;
        QmvArgs a{};
        // q|k|v with the attention RMSNorm fused.
        a.f32_act = f32;
        a.w = m->lm_or(lw + m->off_q, H, s->n, &a.lane_major, f32);
        a.row_bytes = m->rb_h;
        a.rows = (int)(QW + 2 * KW);
        a.cols = (int)H;
        a.nb = (int)(H / be);
        a.x = s->state;
        a.gain = reinterpret_cast<const float *>(m->base + m->off_attn_norm) + (size_t)layer * H;
        a.eps = c.eps;
        a.y = s->qkv;
        if ((st = emu_launch_qmv(ctx, c.encoding, a, n)) != EMU_OK) return st;
        if ((st = emu_launch_attn(ctx, layer_attn(s, layer))) != EMU_OK) return st;
        // o projection + residual.
        QmvArgs o{};
        o.f32_act = f32;
        o.w = m->lm_or(lw + m->off_o, QW, s->n, &o.lane_major, f32);
        o.row_bytes = m->rb_q;
        o.rows = (int)H;
        o.cols = (int)QW;
        o.nb = (int)(QW / be);
        o.x = s->attn;
        o.y = s->state;
        o.accumulate = 1;
        if ((st = emu_launch_qmv(ctx, c.encoding, o, n)) != EMU_OK) return st;
        // gate|up with the FFN RMSNorm and SwiGLU fused.
        QmvArgs g{};
        g.f32_act = f32;
        g.w = m->lm_or(lw + m->off_g, H, s->n, &g.lane_major, f32);
        g.w_up = m->lm_or(lw + m->off_u, H, s->n, &g.lane_major, f32);
        g.row_bytes = m->rb_h;
        g.rows = (int)F;
        g.cols = (int)H;
        g.nb = (int)(H / be);
        g.x = s->state;
        g.gain = reinterpret_cast<const float *>(m->base + m->off_ffn_norm) + (size_t)layer * H;
        g.eps = c.eps;
        g.y = s->act;
        if ((st = emu_launch_qmv(ctx, c.encoding, g, n)) != EMU_OK) return st;
        // down projection + residual.
        QmvArgs d{};
        d.f32_act = f32;
        d.w = m->lm_or(lw + m->off_d, F, s->n, &d.lane_major, f32);
        d.row_bytes = m->rb_f;
        d.rows = (int)H;
        d.cols = (int)F;
        d.nb = (int)(F / be);
        d.x = s->act;
        d.y = s->state;
        d.accumulate = 1;
        if ((st = emu_launch_qmv(ctx, c.encoding, d, n)) != EMU_OK) return st;
        if ((st = mark(s, layer + 1)) != EMU_OK) return st;
    }
    QmvArgs out{};
    out.w = m->base + (c.tied ? m->off_embed : m->off_output);
    out.f32_act = f32;
    if (!f32 && n == 1 && m->lm_takes(H)) {
        out.w = m->lm + m->off_embed;
        out.lane_major = 1;
    }
    out.row_bytes = m->rb_h;
    out.rows = (int)c.vocab;
    out.cols = (int)H;
    out.nb = (int)(H / be);
    out.x = s->state;
    out.gain = reinterpret_cast<const float *>(m->base + m->off_out_norm);
    out.eps = c.eps;
    out.y = s->logits;
    out.keys = s->keys;
    out.key_stride = (int)s->key_stride;
    out.tie_last = smol ? 1 : 0;
    int slots = 0;
    if ((st = emu_launch_qmv(ctx, c.encoding, out, n, &slots)) != EMU_OK) return st;
    if ((st = launch_finalize(s, slots)) != EMU_OK) return st;
    return mark(s, c.layers + 1);
}

// Rebuild the lane-major copy (outside any graph capture).
int model_sync(emu_model *m)
{
    if ((!m->lm && !m->mm) || !m->lm_dirty) return EMU_OK;
    emu_ctx *ctx = m->ctx;
    const emu_model_config &c = m->cfg;
    const uint32_t QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim;
    int st;
    for (const emu_model::MmEntry &e : m->mm_map)
        if ((st = emu_mfma_major_q6k(ctx, m->base + e.src, e.rows, e.cols, m->mm + e.dst)) != EMU_OK) return st;
    auto put = [&](size_t off, uint32_t rows, uint32_t cols, size_t rb) -> int {
        if (!m->lm_takes(cols)) return EMU_OK;
        return emu_lane_major_q6k(ctx, m->base + off, (size_t)rows * rb / 210, m->lm + off);
    };
    for (uint32_t l = 0; l < c.layers; ++l) {
        const size_t lo = m->off_layers + (size_t)l * m->layer_bytes;
        if ((st = put(lo + m->off_q, QW + 2 * KW, c.hidden, m->rb_h)) != EMU_OK ||
            (st = put(lo + m->off_o, c.hidden, QW, m->rb_q)) != EMU_OK ||
            (st = put(lo + m->off_g, c.ffn, c.hidden, m->rb_h)) != EMU_OK ||
            (st = put(lo + m->off_u, c.ffn, c.hidden, m->rb_h)) != EMU_OK ||
            (st = put(lo + m->off_d, c.hidden, c.ffn, m->rb_f)) != EMU_OK)
            return st;
    }
    const size_t out_src = c.tied ? m->off_embed : m->off_output;
    if (m->lm_takes(c.hidden)) {
        if ((st = emu_lane_major_q6k(ctx, m->base + out_src, m->embed_bytes / 210, m->lm + m->off_embed)) != EMU_OK)
            return st;
    }
    if ((st = emu_ctx_sync(ctx)) != EMU_OK) return st;
    m->lm_dirty = false;
    return EMU_OK;
}

int ensure_graph(emu_session *s)
{
    if (s->exec) return EMU_OK;
    int st0 = model_sync(s->m);
    if (st0 != EMU_OK) return st0;
    emu_ctx *ctx = s->m->ctx;
    EMU_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    int st = run_step(s);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (st != EMU_OK) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    if (e != hipSuccess) return emu_hip_fail(ctx, e, "hipStreamEndCapture");
    e = hipGraphInstantiate(&s->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return emu_hip_fail(ctx, e, "hipGraphInstantiate");
    }
    s->graph = g;
    return EMU_OK;
}

// EMU_SESSION_DIRECT launches the step's kernels directly instead of
// replaying the captured graph (same kernels, same order; for profilers, and
// to measure what the graph saves).
bool graphs_enabled(const emu_session *s) { return !(s->flags & EMU_SESSION_DIRECT); }

int launch_steps(emu_session *s, uint32_t count)
{
    emu_ctx *ctx = s->m->ctx;
    if (int st = model_sync(s->m); st != EMU_OK) return st;
    if (!graphs_enabled(s)) {
        for (uint32_t i = 0; i < count; ++i) {
            const int st = run_step(s);
            if (st != EMU_OK) return st;
        }
    } else {
        int st = ensure_graph(s);
        if (st != EMU_OK) return st;
        for (uint32_t i = 0; i < count; ++i) EMU_HIP(ctx, hipGraphLaunch(s->exec, ctx->stream));
    }
    for (auto &p : s->host_pos) p += count;
    return EMU_OK;
}

int check_room(emu_session *s, uint64_t steps)
{
    for (uint32_t p : s->host_pos)
        if ((uint64_t)p + steps > s->context) return EMU_E_CONTEXT_FULL;
    return EMU_OK;
}

int set_ctrl(emu_session *s, uint32_t prompt_len, uint32_t cap)
{
    const uint32_t ctrl[2] = {prompt_len, cap};
    return emu_memcpy_htod(s->m->ctx, s->ctrl, ctrl, sizeof ctrl);
}

} // namespace

// ------------------------------------------------------------------ API --

extern "C" int emu_model_create(emu_ctx *ctx, const emu_model_config *cfg, emu_model **out)
{
    if (!ctx || !cfg || !out) return EMU_E_ARG;
    *out = nullptr;
    const emu_model_config &c = *cfg;
    const bool moe = c.style == EMU_STYLE_GRANITE;
    if (c.hidden == 0 || c.heads == 0 || c.kv_heads == 0 || c.head_dim == 0 || (c.ffn == 0 && !moe) ||
        c.vocab == 0 || c.layers == 0)
        return EMU_E_CONFIG;
    // MoE: routes of up to 8 experts per token for up to 8 clients (the
    // selected-expert FFN's limits), the router's rows float4-loadable, the
    // output tied to the embedding (model.rs:403-407).
    if (moe && (c.n_experts == 0 || c.experts_used == 0 || c.experts_used > c.n_experts || c.experts_used > 8 ||
                c.n_experts > 256 || c.expert_ff == 0 || c.hidden % 8 != 0 || c.hidden > 4096))
        return EMU_E_CONFIG;
    if (!moe && (c.gemma || c.rope_neox)) return EMU_E_CONFIG;
    if (c.gemma && c.window && c.global_every == 0) return EMU_E_CONFIG;
    if (c.heads % c.kv_heads != 0 || c.heads / c.kv_heads > 8) return EMU_E_CONFIG;
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256) return EMU_E_CONFIG;
    if (c.style != EMU_STYLE_QWEN3 && c.style != EMU_STYLE_SMOL && c.style != EMU_STYLE_GRANITE)
        return EMU_E_CONFIG;
    emu_model *m = new (std::nothrow) emu_model();
    if (!m) return EMU_E_NOMEM;
    m->ctx = ctx;
    m->cfg = c;
    const uint32_t QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim;
    int st;
    if ((st = emu_row_bytes(c.encoding, c.hidden, &m->rb_h)) != EMU_OK ||
        (st = emu_row_bytes(c.encoding, QW, &m->rb_q)) != EMU_OK ||
        (!moe && (st = emu_row_bytes(c.encoding, c.ffn, &m->rb_f)) != EMU_OK) ||
        (moe && (st = emu_row_bytes(c.expert_encoding, c.hidden, &m->rb_he)) != EMU_OK) ||
        (moe && (st = emu_row_bytes(c.gemma ? c.expert_down_encoding : c.expert_encoding, c.expert_ff, &m->rb_fe)) !=
                    EMU_OK) ||
        (c.gemma && c.shared_ff && (st = emu_row_bytes(c.encoding, c.shared_ff, &m->rb_sf)) != EMU_OK)) {
        delete m;
        return st == EMU_E_SHORT ? EMU_E_CONFIG : st;
    }
    m->off_q = 0;
    m->off_k = m->off_q + (size_t)QW * m->rb_h;
    m->off_v = m->off_k + (size_t)KW * m->rb_h;
    m->off_o = m->off_v + (size_t)KW * m->rb_h;
    if (moe && c.gemma) {
        // q k v o | router | router scale | down scales | shared gate, up,
        // down | fused gate|up experts | down experts
        m->off_r = align_up(m->off_o + (size_t)c.hidden * m->rb_q, 16);
        m->off_rs = m->off_r + sizeof(float) * c.n_experts * c.hidden;
        m->off_ds = align_up(m->off_rs + sizeof(float) * c.hidden, 16);
        m->off_sg = align_up(m->off_ds + sizeof(float) * c.n_experts, 16);
        m->off_su = m->off_sg + (size_t)c.shared_ff * m->rb_h;
        m->off_sd = m->off_su + (size_t)c.shared_ff * m->rb_h;
        m->off_ge = m->off_sd + (size_t)c.hidden * m->rb_sf;
        m->off_ue = m->off_ge;
        m->off_de = m->off_ge + (size_t)c.n_experts * 2 * c.expert_ff * m->rb_he;
        m->layer_bytes = align_up(m->off_de + (size_t)c.n_experts * c.hidden * m->rb_fe, 16);
    } else if (moe) {
        m->off_r = align_up(m->off_o + (size_t)c.hidden * m->rb_q, 16);
        m->off_ge = m->off_r + sizeof(float) * c.n_experts * c.hidden;
        m->off_ue = m->off_ge + (size_t)c.n_experts * c.expert_ff * m->rb_he;
        m->off_de = m->off_ue + (size_t)c.n_experts * c.expert_ff * m->rb_he;
        m->layer_bytes = align_up(m->off_de + (size_t)c.n_experts * c.hidden * m->rb_fe, 16);
    } else {
        m->off_g = m->off_o + (size_t)c.hidden * m->rb_q;
        m->off_u = m->off_g + (size_t)c.ffn * m->rb_h;
        m->off_d = m->off_u + (size_t)c.ffn * m->rb_h;
        m->layer_bytes = m->off_d + (size_t)c.hidden * m->rb_f;
    }
    m->embed_bytes = (size_t)c.vocab * m->rb_h;
    size_t off = 0;
    m->off_layers = off;
    off = align_up(off + m->layer_bytes * c.layers, 256);
    m->off_embed = off;
    off = align_up(off + m->embed_bytes, 256);
    m->off_output = off;
    if (!c.tied) off = align_up(off + m->embed_bytes, 256);
    m->off_attn_norm = off;
    off = align_up(off + sizeof(float) * c.layers * c.hidden, 256);
    m->off_ffn_norm = off;
    off = align_up(off + sizeof(float) * c.layers * c.hidden, 256);
    m->off_q_norm = off;
    off = align_up(off + sizeof(float) * c.layers * c.head_dim, 256);
    m->off_k_norm = off;
    off = align_up(off + sizeof(float) * c.layers * c.head_dim, 256);
    m->off_out_norm = off;
    off = align_up(off + sizeof(float) * c.hidden, 256);
    m->off_ffn_norm2 = off;
    if (c.gemma) off = align_up(off + sizeof(float) * c.layers * c.hidden, 256);
    m->total = off;
    void *p = nullptr;
    if ((st = emu_malloc(ctx, m->total, &p)) != EMU_OK) {
        delete m;
        return st;
    }
    m->base = static_cast<uint8_t *>(p);
    // The lane-major copy: dense Q6_K models with a width the batch-1 limb
    // matvec takes (the layers' region plus one output matrix).
    const bool lm_any = !moe && (emu_limb_supports(c.encoding, (int)c.hidden) ||
                                 emu_limb_supports(c.encoding, (int)QW) || emu_limb_supports(c.encoding, (int)c.ffn));
    if (lm_any) {
        void *q = nullptr;
        if ((st = emu_malloc(ctx, m->off_embed + m->embed_bytes, &q)) != EMU_OK) {
            emu_free(ctx, m->base);
            delete m;
            return st;
        }
        m->lm = static_cast<uint8_t *>(q);
        m->lm_bytes = m->off_embed + m->embed_bytes;
    }
    // The matrix-core operand copy: every Q6_K matrix that a chained
    // matrix-core matvec reads (a width it takes, whole 32-row tiles but for
    // the output): q|k|v and o, the dense FFN or the Gemma shared FFN, and
    // the output.
    if (c.encoding == EMU_ENC_Q6_K) {
        size_t mm_off = 0;
        auto add = [&](size_t src, uint32_t rows, uint32_t cols, bool any_rows) {
            if (!emu_mfma_shape_ok(c.encoding, (int)cols) || (!any_rows && rows % 32 != 0)) return;
            m->mm_map.push_back({src, mm_off, rows, cols});
            mm_off = align_up(mm_off + emu_mfma_major_bytes(rows, cols), 256);
        };
        for (uint32_t l = 0; l < c.layers; ++l) {
            const size_t lo = m->off_layers + (size_t)l * m->layer_bytes;
            add(lo + m->off_q, QW + 2 * KW, c.hidden, false);
            add(lo + m->off_o, c.hidden, QW, false);
            if (!moe) {
                add(lo + m->off_g, c.ffn, c.hidden, false);
                add(lo + m->off_u, c.ffn, c.hidden, false);
                add(lo + m->off_d, c.hidden, c.ffn, false);
            } else if (c.gemma && c.shared_ff) {
                add(lo + m->off_sg, c.shared_ff, c.hidden, false);
                add(lo + m->off_su, c.shared_ff, c.hidden, false);
                add(lo + m->off_sd, c.hidden, c.shared_ff, false);
            }
        }
        add(c.tied ? m->off_embed : m->off_output, c.vocab, c.hidden, true);
        if (mm_off) {
            void *q = nullptr;
            if ((st = emu_malloc(ctx, mm_off, &q)) != EMU_OK) {
                if (m->lm) emu_free(ctx, m->lm);
                emu_free(ctx, m->base);
                delete m;
                return st;
            }
            m->mm = static_cast<uint8_t *>(q);
            m->mm_bytes = mm_off;
        } else {
            m->mm_map.clear();
        }
    }
    *out = m;
    return EMU_OK;
}

extern "C" int emu_model_destroy(emu_model *m)
{
    if (!m) return EMU_E_ARG;
    emu_free(m->ctx, m->base);
    if (m->lm) emu_free(m->ctx, m->lm);
    if (m->mm) emu_free(m->ctx, m->mm);
    delete m;
    return EMU_OK;
}

extern "C" int emu_model_tensor(emu_model *m, int kind, uint32_t layer, void **d_ptr, size_t *bytes)
{
    if (!m || !d_ptr || !bytes) return EMU_E_ARG;
    const emu_model_config &c = m->cfg;
    if ((kind == EMU_T_LAYER) && layer >= c.layers) return EMU_E_ARG;
    size_t off = 0, len = 0;
    switch (kind) {
    case EMU_T_LAYER: off = m->off_layers + (size_t)layer * m->layer_bytes; len = m->layer_bytes; break;
    case EMU_T_EMBED: off = m->off_embed; len = m->embed_bytes; break;
    case EMU_T_OUTPUT:
        if (c.tied) return EMU_E_ARG;
        off = m->off_output; len = m->embed_bytes; break;
    case EMU_T_ATTN_NORM: off = m->off_attn_norm; len = sizeof(float) * c.layers * c.hidden; break;
    case EMU_T_FFN_NORM: off = m->off_ffn_norm; len = sizeof(float) * c.layers * c.hidden; break;
    case EMU_T_Q_NORM: off = m->off_q_norm; len = sizeof(float) * c.layers * c.head_dim; break;
    case EMU_T_K_NORM: off = m->off_k_norm; len = sizeof(float) * c.layers * c.head_dim; break;
    case EMU_T_OUT_NORM: off = m->off_out_norm; len = sizeof(float) * c.hidden; break;
    case EMU_T_FFN_NORM2:
        if (!m->gemma()) return EMU_E_ARG;
        off = m->off_ffn_norm2; len = sizeof(float) * c.layers * c.hidden; break;
    default: return EMU_E_ARG;
    }
    *d_ptr = m->base + off;
    *bytes = len;
    m->lm_dirty = true; // the caller may write through the pointer
    return EMU_OK;
}

extern "C" int emu_model_sync(emu_model *m)
{
    if (!m) return EMU_E_ARG;
    m->lm_dirty = true;
    return model_sync(m);
}

extern "C" int emu_model_tensor_lane_major(emu_model *m, int kind, uint32_t layer, void **d_ptr, size_t *bytes)
{
    if (!m || !d_ptr || !bytes) return EMU_E_ARG;
    if (!m->lm) return EMU_E_UNSUPPORTED;
    const emu_model_config &c = m->cfg;
    size_t off = 0, len = 0;
    switch (kind) {
    case EMU_T_LAYER:
        if (layer >= c.layers) return EMU_E_ARG;
        off = m->off_layers + (size_t)layer * m->layer_bytes;
        len = m->layer_bytes;
        break;
    case EMU_T_OUTPUT:
        if (!m->lm_takes(c.hidden)) return EMU_E_UNSUPPORTED;
        off = m->off_embed;
        len = m->embed_bytes;
        break;
    default: return EMU_E_ARG;
    }
    const int st = model_sync(m);
    if (st != EMU_OK) return st;
    *d_ptr = m->lm + off;
    *bytes = len;
    return EMU_OK;
}

extern "C" int emu_model_synth(emu_model *m, uint64_t seed)
{
    if (!m) return EMU_E_ARG;
    m->lm_dirty = true;
    emu_ctx *ctx = m->ctx;
    const emu_model_config &c = m->cfg;
    const uint32_t QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim;
    int st;
    for (uint32_t l = 0; l < c.layers; ++l) {
        uint8_t *lw = m->base + m->off_layers + (size_t)l * m->layer_bytes;
        if (m->gemma()) {
            const size_t sz[4] = {(size_t)QW * m->rb_h, (size_t)KW * m->rb_h, (size_t)KW * m->rb_h,
                                  (size_t)c.hidden * m->rb_q};
            const size_t of[4] = {m->off_q, m->off_k, m->off_v, m->off_o};
            for (int t = 0; t < 4; ++t)
                if ((st = synth_tensor(ctx, c.encoding, lw + of[t], sz[t], seed, 16ull * (l + 1) + t)) != EMU_OK)
                    return st;
            const size_t nr = (size_t)c.n_experts * c.hidden;
            hipLaunchKernelGGL(synth_f32_kernel, dim3((unsigned)((nr + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                               ctx->stream, reinterpret_cast<float *>(lw + m->off_r), nr, seed, 16ull * (l + 1) + 4,
                               0.02f);
            EMU_LAUNCH_CHECK(ctx);
            // router and down scales: 1.0
            hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((c.hidden + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                               ctx->stream, reinterpret_cast<float *>(lw + m->off_rs), (size_t)c.hidden, 1.0f);
            hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((c.n_experts + kThreads - 1) / kThreads)), dim3(kThreads),
                               0, ctx->stream, reinterpret_cast<float *>(lw + m->off_ds), (size_t)c.n_experts, 1.0f);
            EMU_LAUNCH_CHECK(ctx);
            const size_t ssz = (size_t)c.shared_ff * m->rb_h;
            const size_t ge = (size_t)c.n_experts * 2 * c.expert_ff * m->rb_he, de = (size_t)c.n_experts * c.hidden * m->rb_fe;
            if ((c.shared_ff &&
                 ((st = synth_tensor(ctx, c.encoding, lw + m->off_sg, ssz, seed, 16ull * (l + 1) + 8)) != EMU_OK ||
                  (st = synth_tensor(ctx, c.encoding, lw + m->off_su, ssz, seed, 16ull * (l + 1) + 9)) != EMU_OK ||
                  (st = synth_tensor(ctx, c.encoding, lw + m->off_sd, (size_t)c.hidden * m->rb_sf, seed,
                                     16ull * (l + 1) + 10)) != EMU_OK)) ||
                (st = synth_tensor(ctx, c.expert_encoding, lw + m->off_ge, ge, seed, 16ull * (l + 1) + 5)) != EMU_OK ||
                (st = synth_tensor(ctx, c.expert_down_encoding, lw + m->off_de, de, seed, 16ull * (l + 1) + 7)) != EMU_OK)
                return st;
            continue;
        }
        if (m->moe()) {
            const size_t sz[6] = {(size_t)QW * m->rb_h, (size_t)KW * m->rb_h, (size_t)KW * m->rb_h,
                                  (size_t)c.hidden * m->rb_q, 0, 0};
            const size_t of[4] = {m->off_q, m->off_k, m->off_v, m->off_o};
            for (int t = 0; t < 4; ++t)
                if ((st = synth_tensor(ctx, c.encoding, lw + of[t], sz[t], seed, 16ull * (l + 1) + t)) != EMU_OK)
                    return st;
            const size_t nr = (size_t)c.n_experts * c.hidden;
            hipLaunchKernelGGL(synth_f32_kernel, dim3((unsigned)((nr + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                               ctx->stream, reinterpret_cast<float *>(lw + m->off_r), nr, seed, 16ull * (l + 1) + 4,
                               0.02f);
            EMU_LAUNCH_CHECK(ctx);
            const size_t ge = (size_t)c.n_experts * c.expert_ff * m->rb_he, de = (size_t)c.n_experts * c.hidden * m->rb_fe;
            if ((st = synth_tensor(ctx, c.expert_encoding, lw + m->off_ge, ge, seed, 16ull * (l + 1) + 5)) != EMU_OK ||
                (st = synth_tensor(ctx, c.expert_encoding, lw + m->off_ue, ge, seed, 16ull * (l + 1) + 6)) != EMU_OK ||
                (st = synth_tensor(ctx, c.expert_encoding, lw + m->off_de, de, seed, 16ull * (l + 1) + 7)) != EMU_OK)
                return st;
            continue;
        }
        const size_t sizes[7] = {(size_t)QW * m->rb_h, (size_t)KW * m->rb_h, (size_t)KW * m->rb_h,
                                 (size_t)c.hidden * m->rb_q, (size_t)c.ffn * m->rb_h, (size_t)c.ffn * m->rb_h,
                                 (size_t)c.hidden * m->rb_f};
        const size_t offs[7] = {m->off_q, m->off_k, m->off_v, m->off_o, m->off_g, m->off_u, m->off_d};
        for (int t = 0; t < 7; ++t)
            if ((st = synth_tensor(ctx, c.encoding, lw + offs[t], sizes[t], seed, 16ull * (l + 1) + t)) != EMU_OK)
                return st;
    }
    if ((st = synth_tensor(ctx, c.encoding, m->base + m->off_embed, m->embed_bytes, seed, 1)) != EMU_OK) return st;
    if (!c.tied &&
        (st = synth_tensor(ctx, c.encoding, m->base + m->off_output, m->embed_bytes, seed, 2)) != EMU_OK)
        return st;
    const size_t nf = (m->total - m->off_attn_norm) / sizeof(float);
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((nf + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                       ctx->stream, reinterpret_cast<float *>(m->base + m->off_attn_norm), nf, 1.0f);
    EMU_LAUNCH_CHECK(ctx);
    return emu_ctx_sync(ctx);
}

namespace {

// One tensor of the file and where it lands in the model's residency.
struct Placement {
    char name[96];
    uint32_t dtype;
    uint32_t n_dims;
    uint64_t dims[3]; // GGML order: dims[0] is the row length
    uint8_t *dst;
    size_t bytes;
};

int place(emu_model *m, emu_gguf *g, const Placement &p)
{
    emu_ctx *ctx = m->ctx;
    uint64_t idx;
    if (emu_gguf_find(g, p.name, &idx) != EMU_OK) {
        snprintf(ctx->last_error, sizeof ctx->last_error, "%s", emu_gguf_error(g));
        return EMU_E_FORMAT;
    }
    emu_gguf_tensor_info t;
    emu_gguf_tensor_at(g, idx, &t);
    bool shape = t.n_dims == p.n_dims;
    for (uint32_t d = 0; shape && d < p.n_dims; ++d) shape = t.dims[d] == p.dims[d];
    if (t.dtype != p.dtype || !shape || t.len != p.bytes) {
        snprintf(ctx->last_error, sizeof ctx->last_error,
                 "tensor %s: dtype %u, %u dims [%llu, %llu, %llu], %llu bytes; the model expects dtype %u, "
                 "[%llu, %llu, %llu], %zu bytes",
                 p.name, t.dtype, t.n_dims, (unsigned long long)t.dims[0], (unsigned long long)t.dims[1],
                 (unsigned long long)t.dims[2], (unsigned long long)t.len, p.dtype, (unsigned long long)p.dims[0],
                 (unsigned long long)p.dims[1], (unsigned long long)p.dims[2], p.bytes);
        return EMU_E_FORMAT;
    }
    const int st = emu_gguf_upload(ctx, g, idx, 0, p.bytes, p.dst);
    if (st != EMU_OK && st != EMU_E_HIP)
        snprintf(ctx->last_error, sizeof ctx->last_error, "%s: %s", p.name, emu_gguf_error(g));
    return st;
}

Placement mk(const char *name, uint32_t dtype, std::initializer_list<uint64_t> dims, uint8_t *dst, size_t bytes)
{
    Placement p{};
    snprintf(p.name, sizeof p.name, "%s", name);
    p.dtype = dtype;
    p.n_dims = (uint32_t)dims.size();
    uint32_t i = 0;
    for (uint64_t d : dims) p.dims[i++] = d;
    p.dst = dst;
    p.bytes = bytes;
    return p;
}

} // namespace

extern "C" int emu_model_load_gguf(emu_model *m, emu_gguf *g)
{
    if (!m || !g) return EMU_E_ARG;
    if (m->gemma()) return EMU_E_UNSUPPORTED; // the Gemma form's tensors are placed through emu_model_tensor
    m->lm_dirty = true;
    const emu_model_config &c = m->cfg;
    const uint32_t QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim;
    const uint32_t enc = (uint32_t)c.encoding, F32 = EMU_ENC_F32;
    std::vector<Placement> ps;
    ps.push_back(mk("token_embd.weight", enc, {c.hidden, c.vocab}, m->base + m->off_embed, m->embed_bytes));
    if (!c.tied)
        ps.push_back(mk("output.weight", enc, {c.hidden, c.vocab}, m->base + m->off_output, m->embed_bytes));
    ps.push_back(mk("output_norm.weight", F32, {c.hidden}, m->base + m->off_out_norm, sizeof(float) * c.hidden));
    char nm[96];
    for (uint32_t l = 0; l < c.layers; ++l) {
        uint8_t *lw = m->base + m->off_layers + (size_t)l * m->layer_bytes;
        auto add = [&](const char *suffix, uint32_t dt, std::initializer_list<uint64_t> dims, uint8_t *dst,
                       size_t bytes) {
            snprintf(nm, sizeof nm, "blk.%u.%s.weight", l, suffix);
            ps.push_back(mk(nm, dt, dims, dst, bytes));
        };
        add("attn_norm", F32, {c.hidden}, m->base + m->off_attn_norm + sizeof(float) * l * c.hidden,
            sizeof(float) * c.hidden);
        add("ffn_norm", F32, {c.hidden}, m->base + m->off_ffn_norm + sizeof(float) * l * c.hidden,
            sizeof(float) * c.hidden);
        if (c.qk_norm) {
            add("attn_q_norm", F32, {c.head_dim}, m->base + m->off_q_norm + sizeof(float) * l * c.head_dim,
                sizeof(float) * c.head_dim);
            add("attn_k_norm", F32, {c.head_dim}, m->base + m->off_k_norm + sizeof(float) * l * c.head_dim,
                sizeof(float) * c.head_dim);
        }
        add("attn_q", enc, {c.hidden, QW}, lw + m->off_q, (size_t)QW * m->rb_h);
        add("attn_k", enc, {c.hidden, KW}, lw + m->off_k, (size_t)KW * m->rb_h);
        add("attn_v", enc, {c.hidden, KW}, lw + m->off_v, (size_t)KW * m->rb_h);
        add("attn_output", enc, {QW, c.hidden}, lw + m->off_o, (size_t)c.hidden * m->rb_q);
        if (m->moe()) {
            const uint32_t xe = (uint32_t)c.expert_encoding;
            add("ffn_gate_inp", F32, {c.hidden, c.n_experts}, lw + m->off_r, sizeof(float) * c.n_experts * c.hidden);
            add("ffn_gate_exps", xe, {c.hidden, c.expert_ff, c.n_experts}, lw + m->off_ge,
                (size_t)c.n_experts * c.expert_ff * m->rb_he);
            add("ffn_up_exps", xe, {c.hidden, c.expert_ff, c.n_experts}, lw + m->off_ue,
                (size_t)c.n_experts * c.expert_ff * m->rb_he);
            add("ffn_down_exps", xe, {c.expert_ff, c.hidden, c.n_experts}, lw + m->off_de,
                (size_t)c.n_experts * c.hidden * m->rb_fe);
        } else {
            add("ffn_gate", enc, {c.hidden, c.ffn}, lw + m->off_g, (size_t)c.ffn * m->rb_h);
            add("ffn_up", enc, {c.hidden, c.ffn}, lw + m->off_u, (size_t)c.ffn * m->rb_h);
            add("ffn_down", enc, {c.ffn, c.hidden}, lw + m->off_d, (size_t)c.hidden * m->rb_f);
        }
    }
    for (const Placement &p : ps) {
        const int st = place(m, g, p);
        if (st != EMU_OK) return st;
    }
    return EMU_OK;
}

extern "C" int emu_model_resident_bytes(const emu_model *m, uint64_t *bytes)
{
    if (!m || !bytes) return EMU_E_ARG;
    *bytes = (uint64_t)m->total + m->lm_bytes + m->mm_bytes;
    return EMU_OK;
}

extern "C" int emu_model_weight_bytes(const emu_model *m, uint64_t *bytes)
{
    if (!m || !bytes) return EMU_E_ARG;
    const emu_model_config &c = m->cfg;
    if (m->moe()) {
        // attention + router + the experts one token routes to, per layer
        const uint64_t per_expert = (uint64_t)2 * c.expert_ff * m->rb_he + (uint64_t)c.hidden * m->rb_fe;
        *bytes = ((uint64_t)m->off_ge + (uint64_t)c.experts_used * per_expert) * c.layers + m->embed_bytes;
        return EMU_OK;
    }
    *bytes = (uint64_t)m->layer_bytes * m->cfg.layers + m->embed_bytes;
    return EMU_OK;
}

extern "C" int emu_session_create(emu_model *m, uint32_t n_clients, uint32_t context, int kv_f16,
                                  emu_session **out)
{
    if (!m || !out || n_clients == 0 || n_clients > 8 || context == 0) return EMU_E_ARG;
    if (context > 65536) return EMU_E_CONFIG; // positions fit u16 (spm-qwen3-slice/src/attention.rs:14-16)
    *out = nullptr;
    emu_ctx *ctx = m->ctx;
    const emu_model_config &c = m->cfg;
    emu_session *s = new (std::nothrow) emu_session();
    if (!s) return EMU_E_NOMEM;
    s->m = m;
    s->n = n_clients;
    s->context = context;
    s->kv_f16 = kv_f16 ? 1 : 0;
    s->host_pos.assign(n_clients, 0);
    const uint32_t QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim;
    s->kv_bytes = (size_t)n_clients * c.layers * KW * context * (s->kv_f16 ? 2 : 4);
    const int chunks = emu_attn_max_chunks((int)context);
    int st = EMU_OK;
    auto alloc = [&](void **p, size_t bytes) {
        if (st == EMU_OK) st = emu_malloc(ctx, bytes, p);
    };
    alloc(&s->k_cache, s->kv_bytes);
    alloc(&s->v_cache, s->kv_bytes);
    alloc((void **)&s->positions, sizeof(uint32_t) * n_clients);
    alloc((void **)&s->tokens, sizeof(uint32_t) * n_clients);
    alloc((void **)&s->steps, sizeof(uint32_t) * n_clients);
    alloc((void **)&s->last, sizeof(uint32_t) * n_clients);
    alloc((void **)&s->prompt, sizeof(uint32_t) * n_clients * context);
    alloc((void **)&s->hist, sizeof(uint32_t) * n_clients * context);
    alloc((void **)&s->ctrl, sizeof(uint32_t) * 4);
    alloc((void **)&s->counters, sizeof(uint32_t) * n_clients * c.kv_heads);
    alloc((void **)&s->state, sizeof(float) * n_clients * c.hidden);
    alloc((void **)&s->qkv, sizeof(float) * n_clients * (QW + 2 * KW));
    alloc((void **)&s->attn, sizeof(float) * n_clients * QW);
    alloc((void **)&s->act, sizeof(float) * n_clients * std::max(std::max(c.ffn, c.gemma ? c.shared_ff : 0u), 1u));
    if (m->moe()) {
        alloc((void **)&s->xn, sizeof(float) * n_clients * c.hidden);
        alloc((void **)&s->gate_counters, sizeof(uint32_t) * n_clients);
        alloc((void **)&s->span_counters, sizeof(uint32_t) * emu_moe_span_counters());
        alloc((void **)&s->rlog, sizeof(float) * n_clients * c.n_experts);
        alloc((void **)&s->rids, sizeof(int32_t) * n_clients * c.experts_used);
        alloc((void **)&s->rwts, sizeof(float) * n_clients * c.experts_used);
        alloc((void **)&s->rids_s, sizeof(int32_t) * n_clients * c.experts_used);
        alloc((void **)&s->rwts_s, sizeof(float) * n_clients * c.experts_used);
        s->moe_ws_bytes = emu_moe_workspace_bytes(n_clients, c.experts_used, c.hidden, c.expert_ff);
        alloc(&s->moe_ws, s->moe_ws_bytes);
    }
    alloc((void **)&s->logits, sizeof(float) * n_clients * c.vocab);
    s->key_stride = c.vocab + 8; // >= key slots of any output-matvec launch shape
    alloc((void **)&s->keys, sizeof(uint64_t) * n_clients * s->key_stride);
    alloc((void **)&s->partial, sizeof(float) * n_clients * c.heads * chunks * (c.head_dim + 2));
    alloc((void **)&s->rope, sizeof(float) * (size_t)context * c.head_dim);
    if (st == EMU_OK) {
        std::vector<float> table;
        emu_build_rope_table(context, c.head_dim, c.rope_theta, c.style == EMU_STYLE_SMOL, table);
        st = emu_memcpy_htod(ctx, s->rope, table.data(), table.size() * sizeof(float));
    }
    if (m->gemma() && c.window) {
        alloc((void **)&s->rope2, sizeof(float) * (size_t)context * c.head_dim);
        if (st == EMU_OK) {
            std::vector<float> table;
            emu_build_rope_table(context, c.head_dim, c.rope_theta_global, 0, table);
            st = emu_memcpy_htod(ctx, s->rope2, table.data(), table.size() * sizeof(float));
        }
    }
    if (st == EMU_OK) st = emu_memset(ctx, s->counters, 0, sizeof(uint32_t) * n_clients * c.kv_heads);
    if (st == EMU_OK && s->gate_counters) st = emu_memset(ctx, s->gate_counters, 0, sizeof(uint32_t) * n_clients);
    if (st == EMU_OK && s->span_counters)
        st = emu_memset(ctx, s->span_counters, 0, sizeof(uint32_t) * emu_moe_span_counters());
    if (st == EMU_OK) {
        // The multi-token matvec's workspace must exist before the step is
        // captured into a graph: size it for every matvec of the step.
        const int shapes[5][3] = {{(int)(QW + 2 * KW), (int)c.hidden, 1},
                                  {(int)c.hidden, (int)QW, 1},
                                  {(int)c.ffn, (int)c.hidden, 2},
                                  {(int)c.hidden, (int)c.ffn, 1},
                                  {(int)c.vocab, (int)c.hidden, 1}};
        size_t ws = mfma_chain(m, n_clients) ? mfma_chain_bytes(m) : moe_chain(m, n_clients) ? moe_chain_bytes(m) : 0;
        for (const auto &sh : shapes)
            if (emu_mfma_supports(c.encoding, sh[1], (int)n_clients)) {
                const size_t b = emu_mfma_workspace_bytes(sh[0], sh[1], sh[2]);
                ws = b > ws ? b : ws;
            }
        if (moe_chain(m, n_clients)) { // the output matvec runs on the matrix cores at any client count
            const size_t b = emu_mfma_workspace_bytes((int)c.vocab, (int)c.hidden, 1);
            ws = b > ws ? b : ws;
        }
        if (ws) st = emu_mfma_reserve(ctx, ws);
    }
    if (st == EMU_OK) st = emu_session_reset(s);
    if (st != EMU_OK) {
        emu_session_destroy(s);
        return st;
    }
    *out = s;
    return EMU_OK;
}

extern "C" int emu_session_destroy(emu_session *s)
{
    if (!s) return EMU_E_ARG;
    emu_ctx *ctx = s->m->ctx;
    if (s->exec) (void)hipGraphExecDestroy(s->exec);
    if (s->graph) (void)hipGraphDestroy(s->graph);
    for (hipEvent_t e : s->marks) (void)hipEventDestroy(e);
    void *ptrs[] = {s->k_cache, s->v_cache, s->positions, s->tokens, s->steps, s->last, s->prompt, s->hist,
                    s->ctrl, s->counters, s->state, s->qkv, s->attn, s->act, s->logits, s->keys, s->partial,
                    s->rope, s->xn, s->rlog, s->rids, s->rwts, s->rids_s, s->rwts_s, s->moe_ws, s->gate_counters,
                    s->span_counters, s->rope2, s->trace_ids, s->trace_w};
    for (void *p : ptrs) emu_free(ctx, p);
    delete s;
    return EMU_OK;
}

extern "C" int emu_session_reset_client(emu_session *s, uint32_t client)
{
    if (!s || client >= s->n) return EMU_E_ARG;
    emu_ctx *ctx = s->m->ctx;
    int st;
    // Position and step count back to 0: attention reads only the positions
    // below the client's own, so its old cache rows are never seen again.
    if ((st = emu_memset(ctx, s->positions + client, 0, sizeof(uint32_t))) != EMU_OK) return st;
    if ((st = emu_memset(ctx, s->steps + client, 0, sizeof(uint32_t))) != EMU_OK) return st;
    s->host_pos[client] = 0;
    return emu_ctx_sync(ctx);
}

extern "C" int emu_session_reset(emu_session *s)
{
    if (!s) return EMU_E_ARG;
    emu_ctx *ctx = s->m->ctx;
    int st;
    if ((st = emu_memset(ctx, s->positions, 0, sizeof(uint32_t) * s->n)) != EMU_OK) return st;
    if ((st = emu_memset(ctx, s->steps, 0, sizeof(uint32_t) * s->n)) != EMU_OK) return st;
    if ((st = emu_memset(ctx, s->k_cache, 0, s->kv_bytes)) != EMU_OK) return st;
    if ((st = emu_memset(ctx, s->v_cache, 0, s->kv_bytes)) != EMU_OK) return st;
    for (auto &p : s->host_pos) p = 0;
    return emu_ctx_sync(ctx);
}

extern "C" int emu_decode_step(emu_session *s, const uint32_t *h_tokens, uint32_t *h_next, float *d_logits)
{
    if (!s || !h_tokens) return EMU_E_ARG;
    for (uint32_t i = 0; i < s->n; ++i)
        if (h_tokens[i] >= s->m->cfg.vocab) return EMU_E_ARG;
    int st = check_room(s, 1);
    if (st != EMU_OK) return st;
    emu_ctx *ctx = s->m->ctx;
    if ((st = emu_memcpy_htod(ctx, s->tokens, h_tokens, sizeof(uint32_t) * s->n)) != EMU_OK) return st;
    if ((st = set_ctrl(s, 0, 0)) != EMU_OK) return st;
    if ((st = launch_steps(s, 1)) != EMU_OK) return st;
    if (d_logits &&
        (st = emu_memcpy_dtod(ctx, d_logits, s->logits, sizeof(float) * s->n * s->m->cfg.vocab)) != EMU_OK)
        return st;
    if (h_next) return emu_memcpy_dtoh(ctx, h_next, s->last, sizeof(uint32_t) * s->n);
    return emu_ctx_sync(ctx);
}

extern "C" int emu_generate(emu_session *s, const uint32_t *h_prompt, uint32_t prompt_len, uint32_t steps,
                            uint32_t *h_out)
{
    if (!s || !h_prompt || prompt_len == 0 || (steps && !h_out)) return EMU_E_ARG;
    if (steps == 0) return EMU_OK;
    for (size_t i = 0; i < (size_t)s->n * prompt_len; ++i)
        if (h_prompt[i] >= s->m->cfg.vocab) return EMU_E_ARG;
    const uint64_t total = (uint64_t)prompt_len + steps - 1;
    int st = check_room(s, total);
    if (st != EMU_OK) return st;
    emu_ctx *ctx = s->m->ctx;
    // prompt buffer rows are `context` long
    std::vector<uint32_t> buf((size_t)s->n * s->context, 0);
    for (uint32_t c = 0; c < s->n; ++c)
        memcpy(&buf[(size_t)c * s->context], h_prompt + (size_t)c * prompt_len, sizeof(uint32_t) * prompt_len);
    if ((st = emu_memcpy_htod(ctx, s->prompt, buf.data(), buf.size() * sizeof(uint32_t))) != EMU_OK) return st;
    std::vector<uint32_t> first(s->n);
    for (uint32_t c = 0; c < s->n; ++c) first[c] = h_prompt[(size_t)c * prompt_len];
    if ((st = emu_memcpy_htod(ctx, s->tokens, first.data(), sizeof(uint32_t) * s->n)) != EMU_OK) return st;
    if ((st = emu_memset(ctx, s->steps, 0, sizeof(uint32_t) * s->n)) != EMU_OK) return st;
    if ((st = set_ctrl(s, prompt_len, steps)) != EMU_OK) return st;
    if ((st = launch_steps(s, (uint32_t)total)) != EMU_OK) return st;
    std::vector<uint32_t> hist((size_t)s->n * steps);
    if ((st = emu_memcpy_dtoh(ctx, hist.data(), s->hist, hist.size() * sizeof(uint32_t))) != EMU_OK) return st;
    memcpy(h_out, hist.data(), hist.size() * sizeof(uint32_t));
    return EMU_OK;
}

extern "C" int emu_time_decode(emu_session *s, uint32_t steps, float *ms)
{
    if (!s || !ms) return EMU_E_ARG;
    int st = check_room(s, steps);
    if (st != EMU_OK) return st;
    emu_ctx *ctx = s->m->ctx;
    if ((st = set_ctrl(s, 0, 0)) != EMU_OK) return st;
    if (graphs_enabled(s) && (st = ensure_graph(s)) != EMU_OK) return st;
    if ((st = emu_ctx_sync(ctx)) != EMU_OK) return st;
    if ((st = emu_event_record(ctx, 14)) != EMU_OK) return st;
    if ((st = launch_steps(s, steps)) != EMU_OK) return st;
    if ((st = emu_event_record(ctx, 15)) != EMU_OK) return st;
    return emu_event_elapsed(ctx, 14, 15, ms);
}

extern "C" int emu_session_time_layers(emu_session *s, float *h_us, uint32_t n)
{
    if (!s || !h_us) return EMU_E_ARG;
    const uint32_t L = s->m->cfg.layers;
    if (n < L + 2) return EMU_E_ARG;
    int st = check_room(s, 1);
    if (st != EMU_OK) return st;
    emu_ctx *ctx = s->m->ctx;
    if ((st = model_sync(s->m)) != EMU_OK) return st;
    while (s->marks.size() < L + 2) {
        hipEvent_t e = nullptr;
        EMU_HIP(ctx, hipEventCreate(&e));
        s->marks.push_back(e);
    }
    if ((st = set_ctrl(s, 0, 0)) != EMU_OK) return st;
    if ((st = emu_ctx_sync(ctx)) != EMU_OK) return st;
    if ((st = emu_event_record(ctx, 13)) != EMU_OK) return st;
    s->marking = true; // direct launches: a replayed graph would not record the marks
    st = run_step(s);
    s->marking = false;
    if (st != EMU_OK) return st;
    for (auto &p : s->host_pos) p += 1;
    EMU_HIP(ctx, hipEventSynchronize(s->marks[L + 1]));
    hipEvent_t prev = ctx->events[13];
    for (uint32_t i = 0; i < L + 2; ++i) {
        float ms = 0.0f;
        EMU_HIP(ctx, hipEventElapsedTime(&ms, prev, s->marks[i]));
        h_us[i] = ms * 1e3f;
        prev = s->marks[i];
    }
    return EMU_OK;
}

namespace {
// The captured step bakes in launch arguments: drop it so the next step
// captures the new routing settings.
void drop_graph(emu_session *s)
{
    if (s->exec) (void)hipGraphExecDestroy(s->exec);
    if (s->graph) (void)hipGraphDestroy(s->graph);
    s->exec = nullptr;
    s->graph = nullptr;
}
} // namespace

extern "C" int emu_session_set_options(emu_session *s, uint32_t flags)
{
    if (!s) return EMU_E_ARG;
    if (flags & ~(uint32_t)(EMU_SESSION_F32_ACT | EMU_SESSION_DIRECT)) return EMU_E_ARG;
    s->flags = flags;
    drop_graph(s);
    return EMU_OK;
}

extern "C" int emu_session_attach_expert_cache(emu_session *s, emu_expert_cache *c)
{
    if (!s) return EMU_E_ARG;
    drop_graph(s);
    if (!c) {
        s->cache = nullptr;
        return EMU_OK;
    }
    const emu_model *m = s->m;
    const emu_model_config &cf = m->cfg;
    if (!m->moe()) return EMU_E_UNSUPPORTED;
    const size_t gate = (size_t)cf.expert_ff * m->rb_he, down = (size_t)cf.hidden * m->rb_fe;
    if (emu_cache_layers(c) != cf.layers || emu_cache_experts(c) != cf.n_experts ||
        emu_cache_expert_bytes(c) != 2 * gate + down)
        return EMU_E_SHAPE;
    int st = emu_cache_device_enable(c);
    if (st != EMU_OK) return st;
    s->cache = c;
    return EMU_OK;
}

extern "C" int emu_expert_cache_load_model(emu_expert_cache *c, emu_model *m, void *h_buf, size_t h_len)
{
    if (!c || !m || !h_buf) return EMU_E_ARG;
    if (!m->moe()) return EMU_E_UNSUPPORTED;
    const emu_model_config &cf = m->cfg;
    const size_t gate = (size_t)cf.expert_ff * m->rb_he, down = (size_t)cf.hidden * m->rb_fe, eb = 2 * gate + down;
    if (emu_cache_layers(c) != cf.layers || emu_cache_experts(c) != cf.n_experts || emu_cache_expert_bytes(c) != eb)
        return EMU_E_SHAPE;
    const size_t stride = (eb + 255) & ~(size_t)255;
    if (h_len < (size_t)cf.layers * cf.n_experts * stride) return EMU_E_ARG;
    emu_ctx *ctx = m->ctx;
    int st = emu_ctx_sync(ctx);
    if (st != EMU_OK) return st;
    uint8_t *h = static_cast<uint8_t *>(h_buf);
    for (uint32_t l = 0; l < cf.layers; ++l) {
        const uint8_t *lw = m->base + m->off_layers + (size_t)l * m->layer_bytes;
        for (uint32_t e = 0; e < cf.n_experts; ++e) {
            uint8_t *dst = h + ((size_t)l * cf.n_experts + e) * stride;
            if (m->gemma()) { // fused gate|up rows: 2 ff rows per expert
                EMU_HIP(ctx, hipMemcpy(dst, lw + m->off_ge + (size_t)e * 2 * gate, 2 * gate, hipMemcpyDeviceToHost));
            } else {
                EMU_HIP(ctx, hipMemcpy(dst, lw + m->off_ge + (size_t)e * gate, gate, hipMemcpyDeviceToHost));
                EMU_HIP(ctx, hipMemcpy(dst + gate, lw + m->off_ue + (size_t)e * gate, gate, hipMemcpyDeviceToHost));
            }
            EMU_HIP(ctx, hipMemcpy(dst + 2 * gate, lw + m->off_de + (size_t)e * down, down, hipMemcpyDeviceToHost));
            if ((st = emu_expert_cache_set_source(c, l, e, dst)) != EMU_OK) return st;
        }
    }
    return EMU_OK;
}

extern "C" int emu_session_route_zipf(emu_session *s, float zipf_s, uint64_t seed)
{
    if (!s || !(zipf_s >= 0.0f)) return EMU_E_ARG;
    if (!s->m->moe()) return EMU_E_UNSUPPORTED;
    s->zipf_s = zipf_s;
    s->zipf_seed = seed;
    drop_graph(s);
    return EMU_OK;
}

extern "C" int emu_session_route_trace(emu_session *s, uint32_t capacity)
{
    if (!s) return EMU_E_ARG;
    if (!s->m->moe()) return EMU_E_UNSUPPORTED;
    emu_ctx *ctx = s->m->ctx;
    const emu_model_config &c = s->m->cfg;
    emu_free(ctx, s->trace_ids);
    emu_free(ctx, s->trace_w);
    s->trace_ids = nullptr;
    s->trace_w = nullptr;
    s->trace_cap = 0;
    drop_graph(s);
    if (capacity == 0) return EMU_OK;
    const size_t n = (size_t)capacity * c.layers * s->n * c.experts_used;
    int st = emu_malloc(ctx, sizeof(int32_t) * n, (void **)&s->trace_ids);
    if (st == EMU_OK) st = emu_malloc(ctx, sizeof(float) * n, (void **)&s->trace_w);
    if (st == EMU_OK) st = emu_memset(ctx, s->trace_ids, 0xff, sizeof(int32_t) * n); // -1: no step yet
    if (st != EMU_OK) {
        emu_free(ctx, s->trace_ids);
        emu_free(ctx, s->trace_w);
        s->trace_ids = nullptr;
        s->trace_w = nullptr;
        return st;
    }
    s->trace_cap = capacity;
    return EMU_OK;
}

extern "C" int emu_session_read_routes(emu_session *s, uint32_t slot, int32_t *h_ids, float *h_weights)
{
    if (!s || !h_ids) return EMU_E_ARG;
    if (!s->trace_cap) return EMU_E_UNSUPPORTED;
    if (slot >= s->trace_cap) return EMU_E_ARG;
    const emu_model_config &c = s->m->cfg;
    const size_t per = (size_t)c.layers * s->n * c.experts_used;
    int st = emu_memcpy_dtoh(s->m->ctx, h_ids, s->trace_ids + per * slot, sizeof(int32_t) * per);
    if (st == EMU_OK && h_weights)
        st = emu_memcpy_dtoh(s->m->ctx, h_weights, s->trace_w + per * slot, sizeof(float) * per);
    return st;
}

extern "C" int emu_session_positions(emu_session *s, uint32_t *h_positions)
{
    if (!s || !h_positions) return EMU_E_ARG;
    return emu_memcpy_dtoh(s->m->ctx, h_positions, s->positions, sizeof(uint32_t) * s->n);
}

extern "C" int emu_session_read_kv(emu_session *s, uint32_t client, uint32_t layer, int which_v, float *h_out,
                                   uint32_t positions)
{
    if (!s || !h_out || client >= s->n || layer >= s->m->cfg.layers || positions > s->context) return EMU_E_ARG;
    const emu_model_config &c = s->m->cfg;
    const uint32_t hd = c.head_dim, nkv = c.kv_heads, kw = nkv * hd;
    const size_t esz = s->kv_f16 ? 2 : 4;
    const uint8_t *base = static_cast<const uint8_t *>(which_v ? s->v_cache : s->k_cache);
    std::vector<uint8_t> tmp((size_t)nkv * s->context * hd * esz);
    const size_t off = ((size_t)client * c.layers + layer) * nkv * s->context * hd * esz;
    int st = emu_memcpy_dtoh(s->m->ctx, tmp.data(), base + off, tmp.size());
    if (st != EMU_OK) return st;
    for (uint32_t p = 0; p < positions; ++p)
        for (uint32_t h = 0; h < nkv; ++h)
            for (uint32_t d = 0; d < hd; ++d) {
                const size_t src = ((size_t)h * s->context + p) * hd + d;
                float v;
                if (s->kv_f16) {
                    uint16_t bits;
                    memcpy(&bits, &tmp[src * 2], 2);
                    v = __half2float(__ushort_as_half(bits));
                } else {
                    memcpy(&v, &tmp[src * 4], 4);
                }
                h_out[(size_t)p * kw + h * hd + d] = v;
            }
    return EMU_OK;
}
