// attn.hip -- fused decode attention for the decode step.
//
// One workgroup (4 wavefronts) per (64-position context chunk, kv head,
// client).  Each workgroup
//   1. rebuilds the rotated queries of its GQ = heads/kv_heads query heads
//      from the projection output, one head per wavefront: per-head RMSNorm
//      when the model has QK-norm, then RoPE from the host-built table
//      (spm-qwen3-slice/src/attention.rs:27-34, spm-kv/src/attend.rs:13-19);
//   2. if its chunk holds the new position, also rotates the new key, rounds
//      key and value to the cache type and appends them (KvCache::append,
//      spm-kv/src/cache.rs:49-58) -- and attends with exactly those values;
//   3. scores its 64 positions: wavefront w takes 16 of them, lanes split the
//      head dimension, so every K and V row is one coalesced load per lane and
//      all 32 of a lane's loads are in flight at once; the per-lane partial
//      dots of (position, head) pairs are combined by a butterfly
//      reduce-scatter across the wavefront (DPP and permlane swaps, one
//      exchange per pair);
//   4. softmax per head over the chunk (max, exp, sum), weighted values,
//      wavefronts merged through LDS;
//   5. writes (max, sum, unnormalised output) per query head; the last
//      workgroup of the (client, kv head) to finish merges all chunks
//      (flash-decoding) and resets the arrival counter for the next step.
//      The hand-off uses agent-scope atomic stores/loads and a relaxed
//      counter rather than an L2 write-back fence.
// Load order matters: vector loads complete in issue order, so the query
// values, gains and rotation rows are issued before the K/V rows (which come
// from HBM), and nothing that the preparation needs sits behind them.
// Cache layout: [client][layer][kv_head][context][head_dim], f16 or f32.
#include "internal.hpp"

#include <math.h>
#include <type_traits>

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * EMU_WAVE;
constexpr int kPP = 16;              // positions per wavefront
constexpr int kChunk = kWaves * kPP; // positions per workgroup
constexpr int kMergeBatch = 16;      // chunks whose partials the merge loads at once

struct AttnArgs {
    const float *qkv;       // [client][q_width + 2*kv_width], or the sum of qkv_slices such arrays
    int qkv_slices;         // partial-sum slices to add (>= 1)
    int qkv_client_stride;  // floats between clients
    size_t qkv_slice_stride; // floats between slices
    void *k_cache, *v_cache;
    const uint32_t *positions;
    const float2 *rope;     // [context][hd/2] (cos, sin)
    const float *q_norm, *k_norm; // per-layer gains or null
    float eps;
    float score_mul;        // score = dot * score_mul, or dot / score_div when score_div > 0
    float score_div;
    int rope_fma;           // spm-ops form: fma(x, cos, -(y*sin))
    int interleaved;        // adjacent-pair RoPE (spm-granite-moe/src/attention.rs:12-26)
    int heads, kv_heads, layers, layer, context;
    float *partial;         // [client][head][max_chunks][hd + 2]
    uint32_t *counters;     // [client][kv_head]
    int max_chunks;
    float *out;             // [client][heads * hd]
    uint8_t *xa;            // optional: the output as the multi-token matvec's A operands
    float *xs;              //           and their scales (token = client)
    int window;             // attend to the last `window` positions only (0: all)
};

// A value of q|k|v: one plain load (MS 1), or the sum of its ns <= MS
// partial-sum slices (as many as the multi-token matvec makes) in slice
// order, MS being 4 or 12 (the launch takes the smaller that holds ns).
// Straight-line code either way: slots past ns load slice 0 and are not
// added, so all of a thread's q|k|v loads go out before the first wait (a
// branch on ns between two values' loads would put a full memory round trip
// between them).
constexpr int kMaxSlices = 12;
template <int MS> __device__ __forceinline__ float qkv_at(const float *p, int ns, size_t stride)
{
    if constexpr (MS == 1) {
        return p[0];
    } else {
        float q[MS];
#pragma unroll
        for (int s = 0; s < MS; ++s) q[s] = p[(s < ns ? s : 0) * stride];
        float v = q[0];
#pragma unroll
        for (int s = 1; s < MS; ++s) v = s < ns ? v + q[s] : v;
        return v;
    }
}

// One column of the output written as the multi-token matvec's A operands:
// three 7-bit limbs under the 16-column sub-block's power-of-two scale (the
// link kernel's split, bit for bit).  The 16 lanes of a sub-block are
// neighbours and all call this together.
__device__ __forceinline__ void emit_limbs(float v, int col, int t, uint8_t *xa, float *xs)
{
    float amax = fabsf(v);
    int bad = !(fabsf(v) <= 3.402823466e38f);
    float fb = __int_as_float(bad); // the flag rides the float exchange bit for bit
    amax = fmaxf(amax, emu_xor_lane<1>(amax));
    fb = __int_as_float(__float_as_int(fb) | __float_as_int(emu_xor_lane<1>(fb)));
    amax = fmaxf(amax, emu_xor_lane<2>(amax));
    fb = __int_as_float(__float_as_int(fb) | __float_as_int(emu_xor_lane<2>(fb)));
    amax = fmaxf(amax, emu_xor_lane<4>(amax));
    fb = __int_as_float(__float_as_int(fb) | __float_as_int(emu_xor_lane<4>(fb)));
    amax = fmaxf(amax, emu_xor_lane<8>(amax));
    fb = __int_as_float(__float_as_int(fb) | __float_as_int(emu_xor_lane<8>(fb)));
    bad = __float_as_int(fb);
    const bool finite = !bad;
    int e = 0;
    (void)frexpf(finite ? amax : 0.0f, &e);
    const float s = finite ? ldexpf(v, 6 - e) : 0.0f;
    const float f0 = rintf(s);
    const float r1 = (s - f0) * 128.0f;
    const float f1 = rintf(r1);
    const float f2 = rintf((r1 - f1) * 128.0f);
    const int sb = col >> 4, kh = (col >> 3) & 1;
    uint8_t *dst = xa + (size_t)sb * 384 + (size_t)(kh * 24 + t) * 8 + (col & 7);
    dst[0] = (uint8_t)(int)f0;
    dst[64] = (uint8_t)(int)f1;
    dst[128] = (uint8_t)(int)f2;
    if ((col & 15) == 0) xs[(size_t)sb * 8 + t] = finite ? ldexpf(1.0f, e - 20) : __int_as_float(0x7fc00000);
}

__device__ __forceinline__ float wave_max(float v)
{
    return emu_wave_reduce(v, [](float x, float y) { return fmaxf(x, y); });
}

// Rotation of one pair, with the reference's roundings: separate products and
// sum (spm-qwen3-slice/src/attention.rs:22-23) or the fma form of
// spm-ops/src/attention.rs:29-30.
__device__ __forceinline__ void rotate(float &l, float &r, float2 cs, int fma_form)
{
#pragma clang fp contract(off)
    float a, b;
    if (fma_form) {
        a = __builtin_fmaf(l, cs.x, -(r * cs.y));
        b = __builtin_fmaf(l, cs.y, r * cs.x);
    } else {
        a = l * cs.x - r * cs.y;
        b = r * cs.x + l * cs.y;
    }
    l = a;
    r = b;
}

// One wavefront: RMSNorm (optional) + RoPE of one head of HD values from
// global memory into dst (LDS).  Lanes own rotation pairs.  load() issues
// every load of the head (values, gains, rotation table), finish() does the
// arithmetic, so a wavefront with several heads has all of their loads in
// flight before the first one is used.
template <int HD, int MS> struct HeadPrep {
    static constexpr int NP = HD / 2;
    static constexpr int PPL = (NP + EMU_WAVE - 1) / EMU_WAVE;
    float a[PPL], b[PPL], ga[PPL], gb[PPL];
    float2 cs[PPL];
    int ia[PPL], ib[PPL];

    __device__ __forceinline__ void load(const float *src, int ns, size_t sstride, const float *gain,
                                         const float2 *rope_row, int interleaved, int lane)
    {
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            const int i = lane + EMU_WAVE * j;
            const int ic = i < NP ? i : NP - 1; // in-bounds stand-in for idle lanes
            ia[j] = interleaved ? 2 * ic : ic;
            ib[j] = interleaved ? 2 * ic + 1 : ic + NP;
            a[j] = qkv_at<MS>(src + ia[j], ns, sstride);
            b[j] = qkv_at<MS>(src + ib[j], ns, sstride);
            cs[j] = rope_row[ic];
            const float *g = gain ? gain : src; // unconditional loads; unused without gains
            ga[j] = g[ia[j]];
            gb[j] = g[ib[j]];
        }
    }

    __device__ __forceinline__ void finish(float *dst, bool has_gain, float eps, int fma_form, int lane)
    {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            if (lane + EMU_WAVE * j < NP) {
                ss = __builtin_fmaf(a[j], a[j], ss);
                ss = __builtin_fmaf(b[j], b[j], ss);
            }
        }
        // selects, not a branch: the gain loads stay where load() put them
        const float scale = 1.0f / sqrtf(wave_sum(ss) / (float)HD + eps);
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            const float na = __fmul_rn(__fmul_rn(a[j], scale), ga[j]);
            const float nb = __fmul_rn(__fmul_rn(b[j], scale), gb[j]);
            a[j] = has_gain ? na : a[j];
            b[j] = has_gain ? nb : b[j];
        }
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            rotate(a[j], b[j], cs[j], fma_form);
            if (lane + EMU_WAVE * j < NP) {
                dst[ia[j]] = a[j];
                dst[ib[j]] = b[j];
            }
        }
    }
};

// Butterfly reduce-scatter of N (<= 64, power of two) per-lane values:
// afterwards lane l holds the wavefront-wide sum of value (l >> log2(64/N)).
// Each step halves the values a lane keeps (the lower half where the lane's
// bit OFF is clear), adding the partner lane's copy of it; once one value is
// left, plain xor-sums finish.  Offsets 32 and 16 use the permlane swaps, the
// others DPP, so no step goes through the LDS crossbar.
template <int N, int OFF>
__device__ __forceinline__ void reduce_scatter_step(float *v, int lane)
{
    if constexpr (OFF >= 16) {
        constexpr int H = N > 1 ? N / 2 : 1;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            float a = v[i], b = N > 1 ? v[i + H] : v[i];
            emu_swap_halves<OFF>(a, b);
            v[i] = a + b;
        }
        reduce_scatter_step<H, OFF / 2>(v, lane);
    } else if constexpr (OFF > 0) {
        if constexpr (N > 1) {
            constexpr int H = N / 2;
            const bool up = (lane & OFF) != 0;
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float keep = up ? v[i + H] : v[i];
                const float send = up ? v[i] : v[i + H];
                v[i] = keep + emu_xor_lane<OFF>(send);
            }
            reduce_scatter_step<H, OFF / 2>(v, lane);
        } else {
            v[0] += emu_xor_lane<OFF>(v[0]);
            reduce_scatter_step<1, OFF / 2>(v, lane);
        }
    }
}

template <int NV>
__device__ __forceinline__ float reduce_scatter(float (&v)[NV], int lane)
{
    reduce_scatter_step<NV, 32>(v, lane);
    return v[0];
}

template <class T, int N> struct VecLoad;
template <> struct VecLoad<__half, 1> { using type = uint16_t; };
template <> struct VecLoad<__half, 2> { using type = uint32_t; };
template <> struct VecLoad<__half, 4> { using type = uint2; };
template <> struct VecLoad<float, 1> { using type = float; };
template <> struct VecLoad<float, 2> { using type = float2; };
template <> struct VecLoad<float, 4> { using type = float4; };

template <int EPL, bool F16, class V>
__device__ __forceinline__ void unpack_row(const V &raw, float (&out)[EPL])
{
    if constexpr (F16) {
        const uint16_t *h = reinterpret_cast<const uint16_t *>(&raw);
#pragma unroll
        for (int e = 0; e < EPL; ++e) out[e] = __half2float(__ushort_as_half(h[e]));
    } else {
        const float *f = reinterpret_cast<const float *>(&raw);
#pragma unroll
        for (int e = 0; e < EPL; ++e) out[e] = f[e];
    }
}

// One query head per kv head (head dim 128, f16 K/V) fits in 80 registers
// (83 with twelve q|k|v slices), so six (five) workgroups share a CU instead
// of four: at eight clients and 1k positions (2,176 workgroups) the chunks
// run in fewer rounds.
constexpr int attn_per_cu(int hd, bool f16, int gqp, int ms)
{
    return gqp == 1 && hd == 128 && f16 ? (ms <= 4 ? 6 : 5) : 1;
}

template <int HD, bool F16, int GQP, int MS>
__global__ __launch_bounds__(kThreads, attn_per_cu(HD, F16, GQP, MS)) void attn_decode_kernel(AttnArgs a)
{
    using kv_t = typename std::conditional<F16, __half, float>::type;
    constexpr int EPL = HD / EMU_WAVE;          // head elements per lane
    constexpr int GH = GQP < 4 ? GQP : 4;       // heads per scoring pass
    constexpr int NV = kPP * GH;                // values per reduce-scatter
    using vec_t = typename VecLoad<kv_t, EPL>::type;

    // Grid: x = (kv head, client), y = chunk.  Workgroups are dispatched x
    // first, so every client's low chunks (the ones a context uses) go out
    // before the idle high chunks, which exit at once.
    const int kvh = blockIdx.x % a.kv_heads, client = blockIdx.x / a.kv_heads, chunk = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & (EMU_WAVE - 1), w = tid / EMU_WAVE;
    const int pos = (int)a.positions[client];
    const int n = pos + 1;
    const int n_chunks = (n + kChunk - 1) / kChunk;
    // Positions lo..pos are attended: all of them, or the last `window`.
    const int lo = a.window > 0 && n > a.window ? n - a.window : 0;
    const int c_lo = lo / kChunk;
    if (chunk >= n_chunks || chunk < c_lo) return; // uniform per workgroup
    const int live_chunks = n_chunks - c_lo;
    const int GQ = a.heads / a.kv_heads;

    __shared__ float q_s[GQP][HD];
    __shared__ float knew[HD], vnew[HD], junk[HD];
    __shared__ __align__(16) float sc[GQP][kChunk];
    __shared__ float mh[GQP], lh[GQP];
    __shared__ float accs[kWaves][GQP][HD];
    __shared__ uint32_t arrived;

    const int qw = a.heads * HD, kw = a.kv_heads * HD;
    const float *row = a.qkv + (size_t)client * a.qkv_client_stride;
    const float2 *rope_row = a.rope + (size_t)pos * (HD / 2);
    const float *qn = a.q_norm ? a.q_norm + (size_t)a.layer * HD : nullptr;
    const float *kn = a.k_norm ? a.k_norm + (size_t)a.layer * HD : nullptr;
    const size_t cache_base =
        (((size_t)client * a.layers + a.layer) * a.kv_heads + kvh) * (size_t)a.context * HD;
    kv_t *kc = static_cast<kv_t *>(a.k_cache) + cache_base;
    kv_t *vc = static_cast<kv_t *>(a.v_cache) + cache_base;
    const int p0 = chunk * kChunk;
    const bool owner = pos >= p0 && pos < p0 + kChunk;

    // 1-2. Rotated queries (and the new key) into LDS: item i on wavefront
    // i % 4.  A wavefront issues the loads of all its items (and every
    // thread its element of the new value) before any arithmetic; idle item
    // slots load item 0 and are not finished.
    const int items = GQ + (owner ? 1 : 0);
    constexpr int IPW = (GQP + 1 + kWaves - 1) / kWaves; // items per wavefront at most
    HeadPrep<HD, MS> hp[IPW];
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
        const int it = w + i * kWaves < items ? w + i * kWaves : 0;
        const bool key = it == GQ;
        hp[i].load(key ? row + qw + kvh * HD : row + (kvh * GQ + it) * HD, a.qkv_slices, a.qkv_slice_stride,
                   key ? kn : qn, rope_row, a.interleaved, lane);
    }
    const float vv = qkv_at<MS>(row + qw + kw + kvh * HD + (tid % HD), a.qkv_slices, a.qkv_slice_stride);
    // Keep those loads ahead of the K/V loads below: loads complete in issue
    // order, so anything issued after the K/V rows waits for them.
    __builtin_amdgcn_sched_barrier(0);
    // This wavefront's 16 positions: issue every K and V row load after the
    // queries' (which the preparation below waits for first), with no
    // branch around them (a branch per load serialises them behind waits).
    // Positions past the context read row `pos - 1` or row 0 (always inside
    // the cache) and are masked after the loads; the new position's row is
    // being written by its owner and is replaced by the owner's values.
    const int pw = p0 + w * kPP;
    const int safe_row = pos > 0 ? pos - 1 : 0;
    vec_t kr[kPP], vr[kPP];
#pragma unroll
    for (int pp = 0; pp < kPP; ++pp) {
        const int p = pw + pp;
        const int r = (p >= lo && p < n && p != pos) ? p : safe_row;
        kr[pp] = *reinterpret_cast<const vec_t *>(kc + (size_t)r * HD + lane * EPL);
        vr[pp] = *reinterpret_cast<const vec_t *>(vc + (size_t)r * HD + lane * EPL);
    }

    // Every slot is finished, idle ones into a junk row: with no branch
    // around the arithmetic the compiler cannot sink the item loads behind
    // the K/V loads (whose in-order completion would then gate them).
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
        const int it = w + i * kWaves;
        const bool key = it == GQ;
        float *dst = it < items ? (key ? knew : q_s[it < GQ ? it : 0]) : junk;
        hp[i].finish(dst, (key ? kn : qn) != nullptr, a.eps, a.rope_fma, lane);
    }
    for (int g = GQ + w; g < GQP; g += kWaves)
        for (int e = lane; e < HD; e += EMU_WAVE) q_s[g][e] = 0.0f;
    __syncthreads();
    if (owner && tid < HD) {
        const float kv = knew[tid];
        kv_t kq, vq;
        if constexpr (F16) {
            kq = __float2half_rn(kv);
            vq = __float2half_rn(vv);
        } else {
            kq = kv;
            vq = vv;
        }
        kc[(size_t)pos * HD + tid] = kq;
        vc[(size_t)pos * HD + tid] = vq;
        knew[tid] = (float)kq; // attend with the cached (rounded) values
        vnew[tid] = (float)vq;
    }
    __syncthreads();

    // 3. Scores.
    float qreg[GQP][EPL];
#pragma unroll
    for (int g = 0; g < GQP; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) qreg[g][e] = q_s[g][lane * EPL + e];
    // Branch-free: a branch per position puts each LDS read behind its own
    // wait.  The new key is read once and selected where its position is.
    float kfresh[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) kfresh[e] = knew[lane * EPL + e];
    float kf[kPP][EPL];
#pragma unroll
    for (int pp = 0; pp < kPP; ++pp) {
        unpack_row<EPL, F16>(kr[pp], kf[pp]);
        const bool is_new = pw + pp == pos;
#pragma unroll
        for (int e = 0; e < EPL; ++e) kf[pp][e] = is_new ? kfresh[e] : kf[pp][e];
    }
    constexpr int SHIFT = NV >= 64 ? 0 : (NV == 32 ? 1 : 2);
#pragma unroll
    for (int pass = 0; pass < GQP / GH; ++pass) {
        float v[NV];
#pragma unroll
        for (int pp = 0; pp < kPP; ++pp)
#pragma unroll
            for (int gh = 0; gh < GH; ++gh) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) d = __builtin_fmaf(qreg[pass * GH + gh][e], kf[pp][e], d);
                v[pp * GH + gh] = d;
            }
        const float dot = reduce_scatter<NV>(v, lane);
        if ((lane & ((1 << SHIFT) - 1)) == 0) {
            const int idx = lane >> SHIFT;
            const int pp = idx / GH, g = pass * GH + idx % GH;
            const int p = pw + pp;
            const float s = a.score_div > 0.0f ? dot / a.score_div : dot * a.score_mul;
            sc[g][w * kPP + pp] = p < n && p >= lo ? s : -INFINITY;
        }
    }
    __syncthreads();

    // 4. Softmax over the chunk, one head per wavefront.
    for (int g = w; g < GQ; g += kWaves) {
        const float s = sc[g][lane];
        const float m = wave_max(s);
        const float e = s == -INFINITY ? 0.0f : expf(s - m);
        const float l = wave_sum(e);
        sc[g][lane] = e;
        if (lane == 0) {
            mh[g] = m;
            lh[g] = l;
        }
    }
    __syncthreads();

    // Weighted values, branch-free: every head's 16 weights of this
    // wavefront's positions come in with four 16-byte LDS reads, the new value
    // is read once and selected, and all GQP heads accumulate (the rows past
    // GQ hold zero queries' scores and are never written out).
    float wgt[GQP][kPP];
#pragma unroll
    for (int g = 0; g < GQP; ++g)
#pragma unroll
        for (int q4 = 0; q4 < kPP / 4; ++q4) {
            const float4 v4 = *reinterpret_cast<const float4 *>(&sc[g][w * kPP + 4 * q4]);
            wgt[g][4 * q4] = v4.x; wgt[g][4 * q4 + 1] = v4.y; wgt[g][4 * q4 + 2] = v4.z; wgt[g][4 * q4 + 3] = v4.w;
        }
    float vn[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) vn[e] = vnew[lane * EPL + e];
    float acc[GQP][EPL];
#pragma unroll
    for (int g = 0; g < GQP; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = 0.0f;
#pragma unroll
    for (int pp = 0; pp < kPP; ++pp) {
        const int p = pw + pp;
        float vf[EPL];
        unpack_row<EPL, F16>(vr[pp], vf);
        // the new position takes the appended value; stand-in rows past the
        // context are zeroed so that their zero weight cannot meet a NaN
#pragma unroll
        for (int e = 0; e < EPL; ++e) vf[e] = p == pos ? vn[e] : (p >= n || p < lo ? 0.0f : vf[e]);
#pragma unroll
        for (int g = 0; g < GQP; ++g)
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[g][e] = __builtin_fmaf(wgt[g][pp], vf[e], acc[g][e]);
    }
#pragma unroll
    for (int g = 0; g < GQP; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) accs[w][g][lane * EPL + e] = acc[g][e];
    __syncthreads();

    float *outp = a.out + (size_t)client * qw;
    if (live_chunks == 1) {
        for (int idx = tid; idx < GQ * HD; idx += kThreads) {
            const int g = idx / HD, d = idx % HD;
            const float o = (accs[0][g][d] + accs[1][g][d]) + (accs[2][g][d] + accs[3][g][d]);
            const float r = o / lh[g];
            outp[(kvh * GQ + g) * HD + d] = r;
            if (a.xa) emit_limbs(r, (kvh * GQ + g) * HD + d, client, a.xa, a.xs);
        }
        return;
    }
    // 5. Partial for the merge.  The hand-off between workgroups uses
    // agent-scope atomic stores and loads (written through to, and read from,
    // the device-coherent level) and a relaxed arrival counter, with every
    // store completed (s_waitcnt) before the counter moves: no L2 write-back
    // fence, which costs several microseconds per workgroup on this part.
    constexpr int PS = HD + 2; // floats per (head, chunk) partial: output, max, exp sum
    for (int idx = tid; idx < GQ * PS; idx += kThreads) {
        const int g = idx / PS, j = idx % PS;
        const int head = kvh * GQ + g;
        float *pp = a.partial + (((size_t)client * a.heads + head) * a.max_chunks + chunk) * PS;
        float val;
        if (j < HD)
            val = (accs[0][g][j] + accs[1][g][j]) + (accs[2][g][j] + accs[3][g][j]);
        else
            val = j == HD ? mh[g] : lh[g];
        __hip_atomic_store(pp + j, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t *counter = a.counters + (size_t)client * a.kv_heads + kvh;
    if (tid == 0) arrived = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != (uint32_t)(live_chunks - 1)) return;
    // Merge (last workgroup to arrive), MB chunks per batch.  The chunk
    // weights depend only on the head, so they are formed once: thread
    // t < GQ * MB owns (head t / MB, chunk t % MB) and the MB lanes of a head
    // take the batch's max and exp sum by DPP butterflies, one expf per lane.
    // Each item thread (NI (head, dim) outputs) loads its output values of
    // the whole batch at once and folds them with the weights from LDS:
    //   O = O * exp(M_old - M) + sum_j o_j * exp(m_j - M), in chunk order.
    constexpr int NI = (GQP * HD + kThreads - 1) / kThreads;
    constexpr int MB = NI <= 2 ? kMergeBatch : 32 / NI;
    static_assert(GQP * MB <= kThreads && MB <= 16, "one 16-lane row per head and batch");
    __shared__ float wt[GQP][MB];
    __shared__ float rs[GQP];
    const int pg = tid / MB, pj = tid % MB;
    const bool pair = pg < GQ;
    const float *pm = a.partial + ((size_t)client * a.heads + kvh * GQ + (pair ? pg : 0)) * a.max_chunks * PS;
    float Mrun = -INFINITY, Lrun = 0.0f; // per head, the same in its MB lanes
    float O[NI];
    const float *pb[NI];
    int head_of[NI], dim_of[NI];
    bool live[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int idx = tid + i * kThreads;
        live[i] = idx < GQ * HD;
        const int ic = live[i] ? idx : 0; // in-bounds stand-in
        head_of[i] = ic / HD;             // within the kv head's group
        dim_of[i] = ic % HD;
        pb[i] = a.partial + ((size_t)client * a.heads + kvh * GQ + head_of[i]) * a.max_chunks * PS;
        O[i] = 0.0f;
    }
    for (int c0 = c_lo; c0 < n_chunks; c0 += MB) {
        const int cp = c0 + pj < n_chunks ? c0 + pj : n_chunks - 1;
        const float mj = __hip_atomic_load(pm + (size_t)cp * PS + HD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float lj = __hip_atomic_load(pm + (size_t)cp * PS + HD + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        float o[NI][MB];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < MB; ++j) {
                const int c = c0 + j < n_chunks ? c0 + j : n_chunks - 1;
                o[i][j] = __hip_atomic_load(pb[i] + (size_t)c * PS + dim_of[i], __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
            }
        const bool valid = c0 + pj < n_chunks;
        float bm = valid ? mj : -INFINITY;
        if constexpr (MB > 8) bm = fmaxf(bm, emu_xor_lane<8>(bm));
        if constexpr (MB > 4) bm = fmaxf(bm, emu_xor_lane<4>(bm));
        if constexpr (MB > 2) bm = fmaxf(bm, emu_xor_lane<2>(bm));
        if constexpr (MB > 1) bm = fmaxf(bm, emu_xor_lane<1>(bm));
        bm = fmaxf(bm, Mrun);
        const float f = valid ? expf(mj - bm) : 0.0f;
        const float r = expf(Mrun - bm); // 0 on the first batch (M = -inf)
        const float lsum = emu_group_sum<MB>(lj * f);
        Lrun = __builtin_fmaf(Lrun, r, lsum);
        Mrun = bm;
        if (pair) {
            wt[pg][pj] = f;
            if (pj == 0) rs[pg] = r;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int g = head_of[i];
            O[i] *= rs[g];
#pragma unroll
            for (int j = 0; j < MB; ++j) O[i] = __builtin_fmaf(o[i][j], wt[g][j], O[i]);
        }
        __syncthreads(); // the next batch rewrites wt and rs
    }
    if (pair && pj == 0) lh[pg] = Lrun;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NI; ++i)
        if (live[i]) {
            const int head = kvh * GQ + head_of[i];
            const float r = O[i] / lh[head_of[i]];
            outp[head * HD + dim_of[i]] = r;
            if (a.xa) emit_limbs(r, head * HD + dim_of[i], client, a.xa, a.xs); // whole 16-lane groups
        }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HD, bool F16, int MS>
void launch_ms(const AttnArgs &a, dim3 grid, hipStream_t stream, int gq)
{
    if (gq <= 1)
        hipLaunchKernelGGL((attn_decode_kernel<HD, F16, 1, MS>), grid, dim3(kThreads), 0, stream, a);
    else if (gq <= 2)
        hipLaunchKernelGGL((attn_decode_kernel<HD, F16, 2, MS>), grid, dim3(kThreads), 0, stream, a);
    else if (gq <= 4)
        hipLaunchKernelGGL((attn_decode_kernel<HD, F16, 4, MS>), grid, dim3(kThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((attn_decode_kernel<HD, F16, 8, MS>), grid, dim3(kThreads), 0, stream, a);
}

template <int HD, bool F16>
void launch_hd(const AttnArgs &a, dim3 grid, hipStream_t stream, int gq)
{
    if (a.qkv_slices > 4) launch_ms<HD, F16, kMaxSlices>(a, grid, stream, gq);
    else if (a.qkv_slices > 1) launch_ms<HD, F16, 4>(a, grid, stream, gq);
    else launch_ms<HD, F16, 1>(a, grid, stream, gq);
}

} // namespace

int emu_attn_max_chunks(int context) { return (context + kChunk - 1) / kChunk; }

int emu_launch_attn(emu_ctx *ctx, const EmuAttnLaunch &l)
{
    if (l.kv_heads <= 0 || l.heads % l.kv_heads != 0 || l.heads / l.kv_heads > 8) return EMU_E_CONFIG;
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
    a.interleaved = l.interleaved;
    a.heads = l.heads;
    a.kv_heads = l.kv_heads;
    a.layers = l.layers;
    a.layer = l.layer;
    a.context = l.context;
    a.partial = l.partial;
    a.counters = l.counters;
    a.max_chunks = emu_attn_max_chunks(l.context);
    a.out = l.out;
    a.qkv_slices = l.qkv_slices > 0 ? l.qkv_slices : 1;
    a.qkv_client_stride = l.qkv_client_stride > 0 ? l.qkv_client_stride : (l.heads + 2 * l.kv_heads) * l.head_dim;
    a.qkv_slice_stride = l.qkv_slice_stride;
    a.xa = l.xa;
    a.xs = l.xs;
    a.window = l.window > 0 ? l.window : 0;
    if (a.qkv_slices > kMaxSlices) return EMU_E_CONFIG;
    if (a.xa && (l.clients > 8 || (l.heads * l.head_dim) % 16 != 0)) return EMU_E_CONFIG;
    const dim3 grid(l.kv_heads * l.clients, a.max_chunks);
    const int gq = l.heads / l.kv_heads;
    switch (l.head_dim * 2 + (l.kv_f16 ? 1 : 0)) {
    case 128: launch_hd<64, false>(a, grid, ctx->stream, gq); break;
    case 129: launch_hd<64, true>(a, grid, ctx->stream, gq); break;
    case 256: launch_hd<128, false>(a, grid, ctx->stream, gq); break;
    case 257: launch_hd<128, true>(a, grid, ctx->stream, gq); break;
    case 512: launch_hd<256, false>(a, grid, ctx->stream, gq); break;
    case 513: launch_hd<256, true>(a, grid, ctx->stream, gq); break;
    default: return EMU_E_CONFIG;
    }
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}
