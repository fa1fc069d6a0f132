// ops.hip -- RMSNorm, RoPE, cached attention, MoE router and greedy selection
// as standalone entry points.  The decode step uses fused versions of the
// same arithmetic (attn.hip, qmv.hip); these are the per-function parity
// hooks and the building blocks of the MoE path.
#include "internal.hpp"

#include <mutex>

#include <math.h>
#include <vector>

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float block_sum(float v, float *red)
{
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = 0.0f;
    const int nw = (blockDim.x + 63) >> 6;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

// One workgroup per row.
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const float *x, const float *gain,
                                                            int width, float eps, float *out)
{
    __shared__ float red[4];
    const float *xr = x + (size_t)blockIdx.x * width;
    float *yr = out + (size_t)blockIdx.x * width;
    float s = 0.0f;
    for (int i = threadIdx.x; i < width; i += kThreads) s = __builtin_fmaf(xr[i], xr[i], s);
    s = block_sum(s, red);
    const float scale = 1.0f / sqrtf(s / (float)width + eps);
    for (int i = threadIdx.x; i < width; i += kThreads) yr[i] = __fmul_rn(__fmul_rn(xr[i], scale), gain[i]);
}

// Thread per (token, head, pair).  Arithmetic kept uncontracted so a table
// built with the reference's libm gives the reference's bits:
// NEOX x' = x*cos - y*sin, y' = y*cos + x*sin (spm-qwen3-slice/src/attention.rs:22-23);
// interleaved pairs (spm-granite-moe/src/attention.rs:20-23).
__global__ __launch_bounds__(kThreads) void rope_kernel(float *x, int n_tok, int heads, int hd,
                                                        const uint32_t *positions, const float2 *table,
                                                        int table_positions, int style)
{
#pragma clang fp contract(off)
    const int half = hd / 2;
    const size_t id = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (id >= (size_t)n_tok * heads * half) return;
    const int i = (int)(id % half);
    const int h = (int)((id / half) % heads);
    const int t = (int)(id / ((size_t)half * heads));
    uint32_t pos = positions[t];
    if (pos >= (uint32_t)table_positions) pos = table_positions - 1; // host validated
    const float2 cs = table[(size_t)pos * half + i];
    float *head = x + ((size_t)t * heads + h) * hd;
    const bool halves = style != EMU_ROPE_INTERLEAVED; // NEOX and its fma form pair i with i + hd/2
    const int a = halves ? i : 2 * i;
    const int b = halves ? i + half : 2 * i + 1;
    const float l = head[a], r = head[b];
    if (style == EMU_ROPE_NEOX_FMA) {
        // spm-ops/src/attention.rs:28-30: fma(x, cos, -(y*sin)), fma(x, sin, y*cos)
        head[a] = __builtin_fmaf(l, cs.x, -(r * cs.y));
        head[b] = __builtin_fmaf(l, cs.y, r * cs.x);
    } else {
        head[a] = l * cs.x - r * cs.y;
        head[b] = r * cs.x + l * cs.y;
    }
}

// attend_cached (spm-kv/src/attend.rs:37-94): one workgroup per query head.
// Threads own positions for the scores, then head lanes for the weighted sum.
__global__ __launch_bounds__(kThreads) void attend_kernel(const float *q, const void *keys,
                                                          const void *values, int kv_f16,
                                                          int positions, int heads, int kv_heads,
                                                          int hd, float scale, float *scores_ws,
                                                          float *out)
{
    __shared__ float red[4];
    const int head = blockIdx.x;
    const int group = heads / kv_heads;
    const int kvh = head / group;
    const int stride = kv_heads * hd;
    const float *qh = q + (size_t)head * hd;
    float *sc = scores_ws + (size_t)head * positions;
    auto kv_at = [&](const void *base, size_t idx) -> float {
        return kv_f16 ? __half2float(static_cast<const __half *>(base)[idx])
                      : static_cast<const float *>(base)[idx];
    };
    float m = -INFINITY;
    for (int p = threadIdx.x; p < positions; p += kThreads) {
        float dot = 0.0f;
        for (int i = 0; i < hd; ++i) dot = __builtin_fmaf(qh[i], kv_at(keys, (size_t)p * stride + kvh * hd + i), dot);
        const float s = dot * scale;
        sc[p] = s;
        m = fmaxf(m, s);
    }
    // block max
    m = emu_wave_reduce(m, [](float x, float y) { return fmaxf(x, y); });
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float l = 0.0f;
    for (int p = threadIdx.x; p < positions; p += kThreads) {
        const float e = expf(sc[p] - m);
        sc[p] = e;
        l += e;
    }
    l = block_sum(l, red);
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += kThreads) {
        float acc = 0.0f;
        for (int p = 0; p < positions; ++p)
            acc = __builtin_fmaf(sc[p] / l, kv_at(values, (size_t)p * stride + kvh * hd + d), acc);
        out[(size_t)head * hd + d] = acc;
    }
}

// Rust f32::total_cmp key, as an order-preserving unsigned.
__device__ __forceinline__ uint32_t total_key_u(float f)
{
    int32_t i = __float_as_int(f);
    i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
    return (uint32_t)i ^ 0x80000000u;
}

// Reduction key: tie_last == 0 -> greatest total-order value, lowest index;
// tie_last == 1 -> greatest value with -0 == +0, highest index.
__device__ __forceinline__ uint64_t select_key(float v, uint32_t idx, int tie_last)
{
    if (tie_last) {
        if (v == 0.0f) v = 0.0f;
        return ((uint64_t)total_key_u(v) << 32) | idx;
    }
    return ((uint64_t)total_key_u(v) << 32) | (0xffffffffu - idx);
}

__device__ __forceinline__ uint32_t key_index(uint64_t k, int tie_last)
{
    const uint32_t lo = (uint32_t)k;
    return tie_last ? lo : 0xffffffffu - lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(k, off, 64);
        k = o > k ? o : k;
    }
    return k;
}

// One workgroup per row.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *x, int width, int tie_last, int32_t *out)
{
    __shared__ uint64_t red[16];
    const float *xr = x + (size_t)blockIdx.x * width;
    uint64_t best = 0;
    for (int i = threadIdx.x; i < width; i += blockDim.x) {
        const uint64_t k = select_key(xr[i], (uint32_t)i, tie_last);
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = red[0];
        for (int i = 1; i < (int)(blockDim.x >> 6); ++i) b = red[i] > b ? red[i] : b;
        out[blockIdx.x] = (int32_t)key_index(b, tie_last);
    }
}

// moe::route: one wavefront per token; n_experts <= 256, k <= 64.
__global__ __launch_bounds__(64) void route_kernel(const float *logits, int n_experts, int k,
                                                   int32_t *ids, float *weights)
{
    const int t = blockIdx.x;
    emu_route_token(logits + (size_t)t * n_experts, n_experts, k, ids + (size_t)t * k, weights + (size_t)t * k);
}

} // namespace

extern "C" int emu_rms_norm(emu_ctx *ctx, const float *d_x, const float *d_gain, uint32_t n_rows,
                            uint32_t width, float eps, float *d_out)
{
    if (!ctx || !d_x || !d_gain || !d_out || width == 0) return EMU_E_ARG;
    if (n_rows == 0) return EMU_OK;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(n_rows), dim3(kThreads), 0, ctx->stream, d_x, d_gain,
                       (int)width, eps, d_out);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

// Angles as spm-qwen3-slice/src/attention.rs:14-19 computes them:
// angle = pos / theta^(2i/d), in f32 with the host libm.
int emu_build_rope_table(uint32_t positions, uint32_t head_dim, float theta, int fma_form,
                         std::vector<float> &table)
{
    const uint32_t half = head_dim / 2;
    table.resize((size_t)positions * half * 2);
    for (uint32_t pos = 0; pos < positions; ++pos) {
        for (uint32_t i = 0; i < half; ++i) {
            float angle;
            if (fma_form) {
                // spm-ops/src/attention.rs:24-27: base^(-2i/d) * pos
                volatile float e = -2.0f * (float)i;
                volatile float ex = e / (float)head_dim;
                volatile float pw = powf(theta, ex);
                angle = pw * (float)pos;
            } else {
                volatile float e = 2.0f * (float)i;
                volatile float ex = e / (float)head_dim;
                volatile float pw = powf(theta, ex);
                angle = (float)pos / pw;
            }
            table[((size_t)pos * half + i) * 2] = cosf(angle);
            table[((size_t)pos * half + i) * 2 + 1] = sinf(angle);
        }
    }
    return EMU_OK;
}

extern "C" int emu_rope_table(emu_ctx *ctx, uint32_t positions, uint32_t head_dim, float theta,
                              float *d_table)
{
    if (!ctx || !d_table || head_dim == 0 || head_dim % 2) return EMU_E_ARG;
    if (positions > 65536) return EMU_E_CONFIG; // positions fit u16 (attention.rs:14-16)
    std::vector<float> t;
    emu_build_rope_table(positions, head_dim, theta, 0, t);
    return emu_memcpy_htod(ctx, d_table, t.data(), t.size() * sizeof(float));
}

extern "C" int emu_rope_table_style(emu_ctx *ctx, int style, uint32_t positions, uint32_t head_dim, float theta,
                                    float *d_table)
{
    if (!ctx || !d_table || head_dim == 0 || head_dim % 2) return EMU_E_ARG;
    if (style != EMU_ROPE_NEOX && style != EMU_ROPE_INTERLEAVED && style != EMU_ROPE_NEOX_FMA) return EMU_E_ARG;
    if (positions > 65536) return EMU_E_CONFIG;
    std::vector<float> t;
    emu_build_rope_table(positions, head_dim, theta, style == EMU_ROPE_NEOX_FMA, t);
    return emu_memcpy_htod(ctx, d_table, t.data(), t.size() * sizeof(float));
}

extern "C" int emu_rope(emu_ctx *ctx, float *d_x, uint32_t n_tok, uint32_t heads, uint32_t head_dim,
                        const uint32_t *d_positions, const float *d_table, uint32_t table_positions,
                        int style)
{
    if (!ctx || !d_x || !d_positions || !d_table || head_dim % 2 || table_positions == 0) return EMU_E_ARG;
    if (style != EMU_ROPE_NEOX && style != EMU_ROPE_INTERLEAVED && style != EMU_ROPE_NEOX_FMA) return EMU_E_ARG;
    const size_t n = (size_t)n_tok * heads * (head_dim / 2);
    if (n == 0) return EMU_OK;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                       ctx->stream, d_x, (int)n_tok, (int)heads, (int)head_dim, d_positions,
                       reinterpret_cast<const float2 *>(d_table), (int)table_positions, style);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

extern "C" int emu_attend_cached(emu_ctx *ctx, const float *d_q, const void *d_keys, const void *d_values,
                                 int kv_f16, uint32_t positions, uint32_t heads, uint32_t kv_heads,
                                 uint32_t head_dim, float scale, float *d_out)
{
    if (!ctx || !d_q || !d_keys || !d_values || !d_out || head_dim == 0) return EMU_E_ARG;
    if (kv_heads == 0 || heads % kv_heads != 0) return EMU_E_CONFIG; // attend.rs:82-85
    if (positions == 0 || heads == 0) return EMU_OK;
    void *ws = nullptr;
    int st = emu_malloc(ctx, sizeof(float) * (size_t)heads * positions, &ws);
    if (st != EMU_OK) return st;
    hipLaunchKernelGGL(attend_kernel, dim3(heads), dim3(kThreads), 0, ctx->stream, d_q, d_keys, d_values,
                       kv_f16, (int)positions, (int)heads, (int)kv_heads, (int)head_dim, scale,
                       static_cast<float *>(ws), d_out);
    hipError_t e = hipGetLastError();
    emu_free(ctx, ws);
    if (e != hipSuccess) return emu_hip_fail(ctx, e, "attend_kernel");
    return EMU_OK;
}

// ---- attend_cached without allocation -------------------------------------
// The scores of emu_attend_cached_noalloc live in this file-scope device
// array: heads * positions floats at most.  Each device holds its own copy,
// at its own address, for the life of the process; host code reaches it only
// through that address (the array's name is not a device address on the
// host).  Every call on a device shares the device's copy, so calls that
// overlap on one device race; the kernel writes every score it reads, so
// nothing needs clearing between calls.
constexpr size_t kAttendScratchFloats = (size_t)1 << 20; // 4 MiB
static __device__ __align__(256) float scratch[kAttendScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch[kMaxDevices] = {};
} // namespace

int emu_ops_device_init(emu_ctx *ctx)
{
    if (ctx->device < 0 || ctx->device >= kMaxDevices) return EMU_E_ARG;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[ctx->device]) return EMU_OK;
    // the context's device is current (emu_ctx_create set it)
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return emu_hip_fail(ctx, e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                     "hipGetSymbolAddress(scratch)");
    g_scratch[ctx->device] = static_cast<float *>(ptr);
    return EMU_OK;
}

extern "C" int emu_attend_cached_noalloc(emu_ctx *ctx, const float *d_q, const void *d_keys, const void *d_values,
                                         int kv_f16, uint32_t positions, uint32_t heads, uint32_t kv_heads,
                                         uint32_t head_dim, float scale, float *d_out)
{
    if (!ctx || !d_q || !d_keys || !d_values || !d_out || head_dim == 0) return EMU_E_ARG;
    if (kv_heads == 0 || heads % kv_heads != 0) return EMU_E_CONFIG; // attend.rs:82-85
    if (positions == 0 || heads == 0) return EMU_OK;
    if ((uint64_t)heads * positions > kAttendScratchFloats) {
        snprintf(ctx->last_error, sizeof ctx->last_error,
                 "emu_attend_cached_noalloc: heads * positions = %llu exceeds its scratch of %zu scores",
                 (unsigned long long)heads * positions, kAttendScratchFloats);
        return EMU_E_CONFIG;
    }
    float *ws = ctx->device >= 0 && ctx->device < kMaxDevices ? g_scratch[ctx->device] : nullptr;
    if (!ws) return EMU_E_ARG; // no context set this device up
    hipLaunchKernelGGL(attend_kernel, dim3(heads), dim3(kThreads), 0, ctx->stream, d_q, d_keys, d_values, kv_f16,
                       (int)positions, (int)heads, (int)kv_heads, (int)head_dim, scale, ws, d_out);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

extern "C" int emu_route(emu_ctx *ctx, const float *d_logits, uint32_t n_tok, uint32_t n_experts,
                         uint32_t k, int32_t *d_ids, float *d_weights)
{
    if (!ctx || !d_logits || !d_ids || !d_weights) return EMU_E_ARG;
    if (n_experts == 0 || n_experts > 256 || k == 0 || k > n_experts || k > 64) return EMU_E_CONFIG;
    if (n_tok == 0) return EMU_OK;
    hipLaunchKernelGGL(route_kernel, dim3(n_tok), dim3(64), 0, ctx->stream, d_logits, (int)n_experts,
                       (int)k, d_ids, d_weights);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

extern "C" int emu_argmax(emu_ctx *ctx, const float *d_x, uint32_t n_rows, uint32_t width, int tie_last,
                          int32_t *d_out)
{
    if (!ctx || !d_x || !d_out || width == 0) return EMU_E_ARG;
    if (n_rows == 0) return EMU_OK;
    hipLaunchKernelGGL(argmax_kernel, dim3(n_rows), dim3(1024), 0, ctx->stream, d_x, (int)width,
                       tie_last ? 1 : 0, d_out);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

namespace {

// Reads every 16-byte word of the buffer once (non-temporal, as the decode
// step's weight loads), grid-stride with one load in flight per lane, so the
// grid's front is one contiguous region moving through the buffer: on this
// part that reads a 2 GiB buffer at 7.2 TB/s, against 6.0 TB/s with four
// loads per lane a grid-stride apart (four pages open per lane).  The xor of
// the words is stored only if it equals a value no input makes likely, so
// the loads are not dropped.
__global__ __launch_bounds__(256) void hbm_read_kernel(const uint8_t *buf, size_t words, uint32_t *sink)
{
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < words; i += stride) {
        const uint4 a = ldnt16(buf + 16 * i);
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

} // namespace

extern "C" int emu_hbm_read_rate(emu_ctx *ctx, const void *d_buf, size_t bytes, uint32_t passes, float *gbs)
{
    if (!ctx || !d_buf || !gbs || passes == 0 || bytes < 16) return EMU_E_ARG;
    const size_t words = bytes / 16;
    const unsigned grid = (unsigned)(ctx->cus > 0 ? ctx->cus * 8 : 2048);
    uint32_t *sink = const_cast<uint32_t *>(static_cast<const uint32_t *>(d_buf));
    const uint8_t *buf = static_cast<const uint8_t *>(d_buf);
    hipLaunchKernelGGL(hbm_read_kernel, dim3(grid), dim3(256), 0, ctx->stream, buf, words, sink); // warm
    EMU_LAUNCH_CHECK(ctx);
    int st;
    if ((st = emu_event_record(ctx, 11)) != EMU_OK) return st;
    for (uint32_t p = 0; p < passes; ++p)
        hipLaunchKernelGGL(hbm_read_kernel, dim3(grid), dim3(256), 0, ctx->stream, buf, words, sink);
    EMU_LAUNCH_CHECK(ctx);
    if ((st = emu_event_record(ctx, 12)) != EMU_OK) return st;
    float ms = 0.0f;
    if ((st = emu_event_elapsed(ctx, 11, 12, &ms)) != EMU_OK) return st;
    *gbs = ms > 0.0f ? (float)((double)words * 16.0 * passes / (ms * 1e-3) / 1e9) : 0.0f;
    return EMU_OK;
}
