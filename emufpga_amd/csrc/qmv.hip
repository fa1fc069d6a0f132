// qmv.hip -- GGUF block dequant, quantized matvec and integer block dots.
//
// Matvec layout: one wavefront owns R consecutive rows (2R for the SwiGLU
// pair).  Lane l walks the row's units u = l, l+64, ... (a unit is the
// 32-weight slice of a block described in internal.hpp), so one wave-wide
// load instruction reads 8 neighbouring blocks' bytes: every byte of the row
// is fetched exactly once, with dwordx2/x4 loads at the blocks' natural
// (2-byte) alignment.  The R rows share each activation load.  Per-lane
// partial sums are reduced across the wave at the end.  Optional prologue:
// RMSNorm of x (sum of squares accumulated from the same activation loads,
// scale applied to the finished dot).  Optional epilogues: residual
// accumulate, SwiGLU of a gate/up row pair.
#include "internal.hpp"

#include <math.h>
#include <stdlib.h>

namespace {

constexpr int kThreads = 256;

// Output rows per wavefront: the rows (or gate/up row pairs) that share each
// activation load.  Four matrix rows in flight per lane at batch 1.
template <int NT, bool DUAL> constexpr int rows_per_wave()
{
    return DUAL ? (NT == 1 ? 2 : 1) : (NT == 1 ? 4 : (NT <= 4 ? 2 : 1));
}

__device__ __forceinline__ void load8f(const float *p, float v[8])
{
    const float4 a = *reinterpret_cast<const float4 *>(p);
    const float4 b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <class F, int NT, bool DUAL, bool NORM>
__global__ __launch_bounds__(kThreads) void qmv_kernel(QmvArgs a)
{
    constexpr int R = rows_per_wave<NT, DUAL>();
    constexpr int NR = DUAL ? 2 * R : R;
    constexpr int G = F::G;
    const int lane = threadIdx.x & (EMU_WAVE - 1);
    const int wave = (blockIdx.x * kThreads + threadIdx.x) / EMU_WAVE;
    const int r0 = wave * R;
    if (r0 >= a.rows) return; // uniform per wave; no barriers below

    float acc[NR][NT];
    float ss[NT];
#pragma unroll
    for (int k = 0; k < NR; ++k)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[k][t] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) ss[t] = 0.0f;

    const uint8_t *rowp[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
        int row = r0 + (k % R);
        row = row < a.rows ? row : a.rows - 1; // duplicate a valid row; never stored
        const uint8_t *base = (DUAL && k >= R) ? a.w_up : a.w;
        rowp[k] = base + (size_t)row * a.row_bytes;
    }

    const int U = a.nb * F::UPB;
    for (int u = lane; u < U; u += EMU_WAVE) {
        const int blk = u / F::UPB, sub = u % F::UPB;
        typename F::Raw raw[NR];
#pragma unroll
        for (int k = 0; k < NR; ++k) F::load(rowp[k] + (size_t)blk * F::BB, sub, raw[k]);
        const int c0 = blk * F::BE;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int col = c0 + F::col(sub, g);
            float xv[NT][8];
            float gn[8];
            if (NORM) load8f(a.gain + col, gn);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                load8f(a.x + (size_t)t * a.cols + col, xv[t]);
                if (NORM) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        ss[t] = __builtin_fmaf(xv[t][i], xv[t][i], ss[t]);
                        xv[t][i] = xv[t][i] * gn[i];
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < NR; ++k) {
                const Grp gp = F::group(raw[k], sub, g);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float w = grp_weight(gp, i);
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[k][t] = __builtin_fmaf(w, xv[t][i], acc[k][t]);
                }
            }
        }
    }

    float scale[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        scale[t] = 1.0f;
        if (NORM) {
            const float mean = wave_sum(ss[t]) / (float)a.cols;
            scale[t] = 1.0f / sqrtf(mean + a.eps);
        }
    }
#pragma unroll
    for (int k = 0; k < NR; ++k)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[k][t] = wave_sum(acc[k][t]) * scale[t];
    if (!DUAL) {
#pragma unroll
        for (int k = 0; k < NR; ++k)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[k][t] = emu_out_epi(acc[k][t], a.out_div, a.softcap);
    }

    if (!DUAL && a.keys && lane == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            uint64_t best = 0;
#pragma unroll
            for (int k = 0; k < R; ++k) {
                if (r0 + k < a.rows) {
                    const uint64_t key = emu_select_key(acc[k][t], (uint32_t)(r0 + k), a.tie_last);
                    best = key > best ? key : best;
                }
            }
            a.keys[(size_t)t * a.key_stride + wave] = best;
        }
    }

#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int row = r0 + k;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (lane == k * NT + t && row < a.rows) {
                float v = acc[k][t];
                if (DUAL) v = emu_glu(v, acc[k + R][t], a.act);
                float *dst = a.y + (size_t)t * a.rows + row;
                if (DUAL) v = emu_out_epi(v, a.out_div, a.softcap);
                *dst = a.accumulate ? emu_resid_add(*dst, v, a.acc_scale) : v;
            }
        }
    }
}

template <class F, int NT>
int launch_nt(emu_ctx *ctx, const QmvArgs &a)
{
    const bool dual = a.w_up != nullptr, norm = a.gain != nullptr;
    const int R = dual ? rows_per_wave<NT, true>() : rows_per_wave<NT, false>();
    const int waves = (a.rows + R - 1) / R;
    const int blocks = (waves * EMU_WAVE + kThreads - 1) / kThreads;
    if (dual && norm)
        hipLaunchKernelGGL((qmv_kernel<F, NT, true, true>), dim3(blocks), dim3(kThreads), 0, ctx->stream, a);
    else if (dual)
        hipLaunchKernelGGL((qmv_kernel<F, NT, true, false>), dim3(blocks), dim3(kThreads), 0, ctx->stream, a);
    else if (norm)
        hipLaunchKernelGGL((qmv_kernel<F, NT, false, true>), dim3(blocks), dim3(kThreads), 0, ctx->stream, a);
    else
        hipLaunchKernelGGL((qmv_kernel<F, NT, false, false>), dim3(blocks), dim3(kThreads), 0, ctx->stream, a);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

// ---- batch-1 matvec: persistent, software-pipelined, activations in LDS ----
// LDS slot of column c (4 pad floats per 128 columns) and of 8-column group
// q's sum (4 pad floats per 32 groups); 16-byte alignment of 4-column runs
// is kept.
__host__ __device__ constexpr int px(int c) { return c + 4 * (c >> 7); }
__host__ __device__ constexpr int pg(int q) { return q + 4 * (q >> 5); }
__host__ __device__ constexpr int lds_x_floats(int cols) { return px(cols) + 4; }
__host__ __device__ constexpr int lds_g_floats(int cols) { return pg(cols / 8) + 4; }

// The workgroup stages x (RMS-normalised as (x*s)*gain when requested, the
// reference's order) in LDS once.  Each wavefront then walks its row groups
// (R rows, or R gate/up row pairs) as a flat list of items (row group x unit
// iteration) and issues the next item's block loads before the current
// item's arithmetic, so two items of loads are in flight per wave.  R is
// chosen per launch: large for tall matrices (fewer activation reads per
// weight), small for short ones (enough wavefronts to fill every CU).  With a
// key buffer the epilogue also tracks the wave's greedy-selection key.
template <class F, int R, bool DUAL, bool NORM>
__global__ __launch_bounds__(kThreads) void qmv_pipe_kernel(QmvArgs a, int total_waves)
{
    constexpr int NR = DUAL ? 2 * R : R;
    constexpr int G = F::G;
    extern __shared__ float xs[];
    __shared__ float red[kThreads / EMU_WAVE];
    const int tid = threadIdx.x, lane = tid & (EMU_WAVE - 1), wv = tid / EMU_WAVE;

    const int gw = blockIdx.x * (kThreads / EMU_WAVE) + wv;
    const int n_rg = (a.rows + R - 1) / R;
    const int U = a.nb * F::UPB;
    const int iters = (U + EMU_WAVE - 1) / EMU_WAVE;
    const int my_rg = gw < n_rg ? (n_rg - 1 - gw) / total_waves + 1 : 0;
    const int items = my_rg * iters;

    // One item's loads: the R (or 2R) rows' unit bytes and, for the first item
    // of a row group, the residual the epilogue adds to (so the epilogue never
    // waits on a load issued behind the prefetch).  Row bases are
    // wave-uniform: they stay in scalar registers and each lane addresses its
    // unit with a 32-bit offset.
    struct Buf {
        typename F::Raw raw[NR];
        float resid;
    };
    auto load_item = [&](int it, Buf &dst) {
        const int rg = gw + (it / iters) * total_waves;
        const int ui = it % iters;
        int u = lane + EMU_WAVE * ui;
        u = u < U ? u : U - 1; // in-bounds duplicate; its contribution is masked
        const int blk = u / F::UPB, sub = u % F::UPB;
        const uint32_t off = (uint32_t)blk * F::BB;
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            int row = rg * R + (k % R);
            row = row < a.rows ? row : a.rows - 1;
            const uint8_t *base = (DUAL && k >= R) ? a.w_up : a.w;
            row = __builtin_amdgcn_readfirstlane(row);
            F::load(base + (size_t)row * a.row_bytes, off, sub, dst.raw[k]);
        }
        if (a.accumulate && ui == 0) {
            int row = rg * R + (lane < R ? lane : R - 1);
            row = row < a.rows ? row : a.rows - 1;
            dst.resid = a.y[row];
        }
    };

    // Padded LDS layout: column c lives at px(c), 8-column group q's sum at
    // xg[pg(q)].  Lane units sit 32 columns apart except for their 8-column
    // slot, so without padding 16 lanes would share each bank group.
    float *xg = xs + lds_x_floats(a.cols);
    // The first 2 * kThreads * 4 columns of x load into registers, then the
    // first item's weight loads go out, then x is staged and normalised:
    // loads complete in issue order, so the prologue waits only for x while
    // the weights' round trip runs.
    float4 xr[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = tid * 4 + i * kThreads * 4;
        xr[i] = *reinterpret_cast<const float4 *>(a.x + (c < a.cols ? c : 0)); // in-bounds stand-in
    }
    __builtin_amdgcn_sched_barrier(0);
    Buf b0, b1;
    load_item(0, b0); // clamped to valid rows even when this wave has no item
    __builtin_amdgcn_sched_barrier(0);
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = tid * 4 + i * kThreads * 4;
        if (c < a.cols) {
            const float4 v = xr[i];
            if (NORM) ss = __builtin_fmaf(v.w, v.w, __builtin_fmaf(v.z, v.z, __builtin_fmaf(v.y, v.y, __builtin_fmaf(v.x, v.x, ss))));
            *reinterpret_cast<float4 *>(xs + px(c)) = v;
        }
    }
    for (int c = tid * 4 + 2 * kThreads * 4; c < a.cols; c += kThreads * 4) {
        const float4 v = *reinterpret_cast<const float4 *>(a.x + c);
        if (NORM) ss = __builtin_fmaf(v.w, v.w, __builtin_fmaf(v.z, v.z, __builtin_fmaf(v.y, v.y, __builtin_fmaf(v.x, v.x, ss))));
        *reinterpret_cast<float4 *>(xs + px(c)) = v;
    }
    if (NORM) {
        ss = wave_sum(ss);
        if (lane == 0) red[wv] = ss;
        __syncthreads();
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float scale = 1.0f / sqrtf(tot / (float)a.cols + a.eps);
        for (int c = tid * 4; c < a.cols; c += kThreads * 4) {
            float4 v = *reinterpret_cast<float4 *>(xs + px(c));
            const float4 g = *reinterpret_cast<const float4 *>(a.gain + c);
            v.x = __fmul_rn(__fmul_rn(v.x, scale), g.x);
            v.y = __fmul_rn(__fmul_rn(v.y, scale), g.y);
            v.z = __fmul_rn(__fmul_rn(v.z, scale), g.z);
            v.w = __fmul_rn(__fmul_rn(v.w, scale), g.w);
            *reinterpret_cast<float4 *>(xs + px(c)) = v;
        }
    }
    __syncthreads();
    for (int q = tid; q < a.cols / 8; q += kThreads) {
        const float *p = xs + px(8 * q);
        xg[pg(q)] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    }
    __syncthreads();

    float acc[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) acc[k] = 0.0f;
    uint64_t best = 0;
    float resid = 0.0f;

    // w_i = code_i * mul + add, so a group adds mul * sum(code_i x_i) + add * sum(x_i).
    auto process = [&](int it, const Buf &buf) {
        const typename F::Raw(&cur)[NR] = buf.raw;
        const int ui = it % iters;
        if (a.accumulate && ui == 0) resid = buf.resid;
        const int u = lane + EMU_WAVE * ui;
        if (u < U) {
            const int blk = u / F::UPB, sub = u % F::UPB;
            const int c0 = blk * F::BE;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const int col = c0 + F::col(sub, g);
                const float4 x0 = *reinterpret_cast<const float4 *>(xs + px(col));
                const float4 x1 = *reinterpret_cast<const float4 *>(xs + px(col) + 4);
                const float xsum = xg[pg(col / 8)];
                const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int k = 0; k < NR; ++k) {
                    const Grp gp = F::group(cur[k], sub, g);
                    float t = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; ++i) t = __builtin_fmaf(byte_f(i < 4 ? gp.q0 : gp.q1, i & 3), xv[i], t);
                    if (F::BIAS) // add == -BIAS * mul: mul * (t - BIAS * xsum)
                        acc[k] = __builtin_fmaf(gp.mul, __builtin_fmaf(-(float)F::BIAS, xsum, t), acc[k]);
                    else
                        acc[k] = __builtin_fmaf(gp.add, xsum, __builtin_fmaf(gp.mul, t, acc[k]));
                }
            }
        }
        if (ui == iters - 1) {
            const int rg = gw + (it / iters) * total_waves;
            float v[NR];
#pragma unroll
            for (int k = 0; k < NR; ++k) {
                v[k] = wave_sum(acc[k]);
                acc[k] = 0.0f;
            }
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const int row = rg * R + k;
                float val = v[k];
                if (DUAL) val = emu_glu(val, v[k + R], a.act);
                val = emu_out_epi(val, a.out_div, a.softcap);
                if (row < a.rows) {
                    if (lane == k) a.y[row] = a.accumulate ? emu_resid_add(resid, val, a.acc_scale) : val;
                    if (a.keys) {
                        const uint64_t key = emu_select_key(val, (uint32_t)row, a.tie_last);
                        best = key > best ? key : best;
                    }
                }
            }
        }
    };

    // Two buffers in turn: item it+1's loads are in flight during item it.
    // The prefetch is unconditional (clamped to the last item) so the
    // compiler's wait counts never have to cover a maybe-issued load.
    if (items > 0) {
        const int last = items - 1;
        for (int it = 0; it < items; it += 2) {
            load_item(it + 1 < last ? it + 1 : last, b1);
            process(it, b0);
            load_item(it + 2 < last ? it + 2 : last, b0);
            if (it + 1 < items) process(it + 1, b1);
        }
    }
    if (a.keys && lane == 0) a.keys[gw] = best;
}

template <class F, int R>
void launch_pipe_r(emu_ctx *ctx, const QmvArgs &a, int blocks, int total_waves, size_t lds)
{
    const bool dual = a.w_up != nullptr, norm = a.gain != nullptr;
    if (dual && norm)
        hipLaunchKernelGGL((qmv_pipe_kernel<F, R, true, true>), dim3(blocks), dim3(kThreads), lds, ctx->stream, a, total_waves);
    else if (dual)
        hipLaunchKernelGGL((qmv_pipe_kernel<F, R, true, false>), dim3(blocks), dim3(kThreads), lds, ctx->stream, a, total_waves);
    else if (norm)
        hipLaunchKernelGGL((qmv_pipe_kernel<F, R, false, true>), dim3(blocks), dim3(kThreads), lds, ctx->stream, a, total_waves);
    else
        hipLaunchKernelGGL((qmv_pipe_kernel<F, R, false, false>), dim3(blocks), dim3(kThreads), lds, ctx->stream, a, total_waves);
}

template <class F>
int launch_pipe(emu_ctx *ctx, const QmvArgs &a, int *key_slots)
{
    const bool dual = a.w_up != nullptr;
    const int waves_per_block = kThreads / EMU_WAVE;
    const int cus = ctx->cus > 0 ? ctx->cus : 256;
    const int max_blocks = cus * 4;               // 16 wavefronts per CU resident
    const int want_waves = max_blocks * waves_per_block;
    // Largest R (rows sharing each activation read) that still gives every
    // CU its full complement of wavefronts; gate/up pairs count double.
    int R = dual ? 2 : 4;
    while (R > 1 && (a.rows + R - 1) / R < want_waves) R /= 2;
    const int n_rg = (a.rows + R - 1) / R;
    int blocks = (n_rg + waves_per_block - 1) / waves_per_block;
    blocks = blocks < max_blocks ? blocks : max_blocks;
    const int total_waves = blocks * waves_per_block;
    if (a.keys && total_waves > a.key_stride) return EMU_E_CONFIG; // key slot per wave
    const size_t lds = sizeof(float) * (size_t)(lds_x_floats(a.cols) + lds_g_floats(a.cols));
    switch (R) {
    case 4: launch_pipe_r<F, 4>(ctx, a, blocks, total_waves, lds); break;
    case 2: launch_pipe_r<F, 2>(ctx, a, blocks, total_waves, lds); break;
    default: launch_pipe_r<F, 1>(ctx, a, blocks, total_waves, lds); break;
    }
    EMU_LAUNCH_CHECK(ctx);
    if (key_slots) *key_slots = total_waves;
    return EMU_OK;
}

constexpr int kPipeMaxCols = 12288; // padded activations + group sums fit in 58 KB of LDS

template <class F>
int launch_fmt(emu_ctx *ctx, const QmvArgs &a, int n_tok, int *key_slots)
{
    if (n_tok == 1 && a.cols <= kPipeMaxCols && a.cols % 4 == 0)
        return launch_pipe<F>(ctx, a, key_slots);
    if (a.keys && a.w_up) return EMU_E_ARG; // keys select among plain matvec rows
    if (key_slots) {
        const bool dual = a.w_up != nullptr;
        int R = 1;
        switch (n_tok) {
        case 1: R = dual ? rows_per_wave<1, true>() : rows_per_wave<1, false>(); break;
        case 2: case 3: case 4: R = rows_per_wave<2, false>(); break;
        default: R = rows_per_wave<8, false>(); break;
        }
        *key_slots = (a.rows + R - 1) / R;
        if (a.keys && *key_slots > a.key_stride) return EMU_E_CONFIG;
    }
    switch (n_tok) {
    case 1: return launch_nt<F, 1>(ctx, a);
    case 2: return launch_nt<F, 2>(ctx, a);
    case 3: return launch_nt<F, 3>(ctx, a);
    case 4: return launch_nt<F, 4>(ctx, a);
    case 5: return launch_nt<F, 5>(ctx, a);
    case 6: return launch_nt<F, 6>(ctx, a);
    case 7: return launch_nt<F, 7>(ctx, a);
    case 8: return launch_nt<F, 8>(ctx, a);
    default: return EMU_E_ARG;
    }
}

// ---- dequant: one thread per unit, 32 exact weights out -------------------
template <class F>
__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint8_t *src, size_t nblocks,
                                                           float *out)
{
    const size_t u = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (u >= nblocks * F::UPB) return;
    const size_t blk = u / F::UPB;
    const int sub = (int)(u % F::UPB);
    typename F::Raw raw;
    F::load(src + blk * F::BB, sub, raw);
#pragma unroll
    for (int g = 0; g < F::G; ++g) {
        const Grp gp = F::group(raw, sub, g);
        float w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = grp_weight_exact<F::BIAS>(gp, i);
        float4 *dst = reinterpret_cast<float4 *>(out + blk * F::BE + F::col(sub, g));
        dst[0] = make_float4(w[0], w[1], w[2], w[3]);
        dst[1] = make_float4(w[4], w[5], w[6], w[7]);
    }
}

template <class F>
int launch_dequant(emu_ctx *ctx, const uint8_t *src, size_t nblocks, float *out)
{
    const size_t units = nblocks * F::UPB;
    if (units == 0) return EMU_OK;
    const size_t blocks = (units + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(dequant_kernel<F>, dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream, src,
                       nblocks, out);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

// ---- integer block dots: thread per (token, row, unit) --------------------
// The code of weight i is its unsigned byte minus the format's bias; each
// group's 8-column partial is added into its sub-block's int32 sum.
template <class F>
__global__ __launch_bounds__(kThreads) void block_dots_kernel(const uint8_t *w, size_t row_bytes,
                                                              int rows, int cols, int nb,
                                                              const int8_t *xq, int n_tok,
                                                              int32_t *out)
{
    const size_t id = (size_t)blockIdx.x * kThreads + threadIdx.x;
    const size_t units = (size_t)nb * F::UPB;
    if (id >= units * rows * n_tok) return;
    const int t = (int)(id / (units * rows));
    const int r = (int)((id / units) % rows);
    const int u = (int)(id % units);
    const int blk = u / F::UPB, sub = u % F::UPB;
    typename F::Raw raw;
    F::load(w + (size_t)r * row_bytes + (size_t)blk * F::BB, sub, raw);
    const int nsub = cols / F::SUB;
#pragma unroll
    for (int g = 0; g < F::G; ++g) {
        const Grp gp = F::group(raw, sub, g);
        const int col = blk * F::BE + F::col(sub, g);
        int32_t s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s += grp_code<F::BIAS>(gp, i) * (int32_t)xq[(size_t)t * cols + col + i];
        atomicAdd(out + ((size_t)t * rows + r) * nsub + col / F::SUB, s);
    }
}

template <class F>
int launch_block_dots(emu_ctx *ctx, const uint8_t *w, size_t row_bytes, int rows, int cols,
                      const int8_t *xq, int n_tok, int32_t *out)
{
    const int nb = cols / F::BE;
    const size_t total = (size_t)nb * F::UPB * rows * n_tok;
    EMU_HIP(ctx, hipMemsetAsync(out, 0, sizeof(int32_t) * (size_t)n_tok * rows * (cols / F::SUB),
                                ctx->stream));
    if (total == 0) return EMU_OK;
    hipLaunchKernelGGL(block_dots_kernel<F>, dim3((unsigned)((total + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, ctx->stream, w, row_bytes, rows, cols, nb, xq, n_tok, out);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

// ---- int8-activation matvec ----------------------------------------------
// Same row-per-wave walk; per group the integer dot of 8 codes with 8 int8
// activations is exact, scaled by (mul * s_x); the min term of Q5_K / Q2_K
// uses the integer activation sum.  y = sum over groups of
//   s_x * (mul * (sum code*q) + add_part) with add = -(dmin*m) per weight.
template <class F>
__global__ __launch_bounds__(kThreads) void qmv_i8_kernel(const uint8_t *w, size_t row_bytes,
                                                          int rows, int cols, int nb,
                                                          const int8_t *xq, const float *xs,
                                                          int n_tok, float *y)
{
    const int lane = threadIdx.x & (EMU_WAVE - 1);
    const int wave = (blockIdx.x * kThreads + threadIdx.x) / EMU_WAVE;
    const int row = wave;
    if (row >= rows * n_tok) return;
    const int t = row / rows, r = row % rows;
    const uint8_t *rp = w + (size_t)r * row_bytes;
    float acc = 0.0f;
    const int U = nb * F::UPB;
    for (int u = lane; u < U; u += EMU_WAVE) {
        const int blk = u / F::UPB, sub = u % F::UPB;
        typename F::Raw raw;
        F::load(rp + (size_t)blk * F::BB, sub, raw);
#pragma unroll
        for (int g = 0; g < F::G; ++g) {
            const Grp gp = F::group(raw, sub, g);
            const int col = blk * F::BE + F::col(sub, g);
            const int8_t *xp = xq + (size_t)t * cols + col;
            const uint2 xv = *reinterpret_cast<const uint2 *>(xp);
            int32_t dot = 0, xsum = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int code = grp_code<F::BIAS>(gp, i);
                const int xi = (int)(int8_t)((i < 4 ? xv.x : xv.y) >> (8 * (i & 3)));
                dot += code * xi;
                xsum += xi;
            }
            // exact weight = code*mul + (add + BIAS*mul)
            const float base = __builtin_fmaf((float)F::BIAS, gp.mul, gp.add);
            const float s = xs[((size_t)t * cols + col) / 32];
            acc = __builtin_fmaf(s, __builtin_fmaf(gp.mul, (float)dot, base * (float)xsum), acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[(size_t)t * rows + r] = acc;
}

template <class F>
int launch_qmv_i8(emu_ctx *ctx, const uint8_t *w, size_t row_bytes, int rows, int cols,
                  const int8_t *xq, const float *xs, int n_tok, float *y)
{
    const int nb = cols / F::BE;
    const size_t waves = (size_t)rows * n_tok;
    if (waves == 0) return EMU_OK;
    const size_t blocks = (waves * EMU_WAVE + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(qmv_i8_kernel<F>, dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream, w,
                       row_bytes, rows, cols, nb, xq, xs, n_tok, y);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

// ---- activation quantizer: one thread per 32-column block ----------------
__global__ __launch_bounds__(kThreads) void quantize_act_kernel(const float *x, size_t nblk,
                                                                int8_t *q, float *scales)
{
    const size_t b = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (b >= nblk) return;
    const float *xp = x + b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const float v = fabsf(xp[i]);
        amax = v > amax ? v : amax;
    }
    const float s = amax / 127.0f;
    const float id = s != 0.0f ? 1.0f / s : 0.0f;
    scales[b] = s;
    for (int i = 0; i < 32; ++i) {
        float v = roundf(xp[i] * id);
        v = v > 127.0f ? 127.0f : (v < -127.0f ? -127.0f : v);
        q[b * 32 + i] = (int8_t)v;
    }
}

int check_matrix(int encoding, size_t w_len, uint32_t rows, uint32_t cols, size_t *row_bytes)
{
    int st = emu_row_bytes(encoding, cols, row_bytes);
    if (st != EMU_OK) return st;
    if ((size_t)rows * *row_bytes != w_len) return EMU_E_SHAPE;
    return EMU_OK;
}

} // namespace

int emu_row_bytes(int encoding, uint32_t cols, size_t *row_bytes)
{
    uint32_t be = 0, bb = 0;
    int st = emu_block_layout(encoding, &be, &bb);
    if (st != EMU_OK) return st;
    if (encoding == EMU_ENC_F32 || encoding == EMU_ENC_F16) return EMU_E_UNSUPPORTED;
    if (cols % be != 0) return EMU_E_SHORT;
    *row_bytes = (size_t)(cols / be) * bb;
    return EMU_OK;
}

int emu_launch_qmv(emu_ctx *ctx, int encoding, const QmvArgs &a, int n_tok, int *key_slots)
{
    if (a.rows == 0 || n_tok == 0) return EMU_OK;
    if (a.f32_act && (a.mfma_major || a.lane_major)) return EMU_E_UNSUPPORTED; // int8-limb layouts
    if (a.mfma_major) { // only the multi-token matrix-core kernel reads that layout
        if (!emu_mfma_supports(encoding, a.cols, n_tok) || (a.w_up && a.accumulate)) return EMU_E_UNSUPPORTED;
        return emu_launch_mfma(ctx, encoding, a, n_tok, key_slots);
    }
    if (!a.f32_act && n_tok == 1 && emu_limb_supports(encoding, a.cols) && !(a.w_up && a.accumulate))
        return emu_launch_limb(ctx, encoding, a, key_slots);
    if (a.lane_major) return EMU_E_UNSUPPORTED; // only the batch-1 limb kernel reads that layout
    if (!a.f32_act && emu_mfma_supports(encoding, a.cols, n_tok) && !(a.w_up && a.accumulate))
        return emu_launch_mfma(ctx, encoding, a, n_tok, key_slots);
    switch (encoding) {
    case EMU_ENC_Q6_K: return launch_fmt<FmtQ6K>(ctx, a, n_tok, key_slots);
    case EMU_ENC_Q8_0: return launch_fmt<FmtQ8_0>(ctx, a, n_tok, key_slots);
    case EMU_ENC_Q5_K: return launch_fmt<FmtQ5K>(ctx, a, n_tok, key_slots);
    case EMU_ENC_Q2_K: return launch_fmt<FmtQ2K>(ctx, a, n_tok, key_slots);
    default: return EMU_E_UNSUPPORTED;
    }
}

extern "C" int emu_dequant(emu_ctx *ctx, int encoding, const void *d_src, size_t src_len, float *d_out)
{
    if (!ctx || (!d_src && src_len) || (!d_out && src_len)) return EMU_E_ARG;
    uint32_t be = 0, bb = 0;
    int st = emu_block_layout(encoding, &be, &bb);
    if (st != EMU_OK) return st;
    if (src_len % bb != 0) return EMU_E_SHORT;
    const size_t nblocks = src_len / bb;
    const uint8_t *src = static_cast<const uint8_t *>(d_src);
    switch (encoding) {
    case EMU_ENC_Q6_K: return launch_dequant<FmtQ6K>(ctx, src, nblocks, d_out);
    case EMU_ENC_Q8_0: return launch_dequant<FmtQ8_0>(ctx, src, nblocks, d_out);
    case EMU_ENC_Q5_K: return launch_dequant<FmtQ5K>(ctx, src, nblocks, d_out);
    case EMU_ENC_Q2_K: return launch_dequant<FmtQ2K>(ctx, src, nblocks, d_out);
    default: return EMU_E_UNSUPPORTED;
    }
}

extern "C" int emu_qmatvec(emu_ctx *ctx, int encoding, const void *d_w, size_t w_len, uint32_t rows,
                           uint32_t cols, const float *d_x, size_t x_len, uint32_t n_tok, float *d_y,
                           uint32_t flags)
{
    if (!ctx || !d_w || !d_x || !d_y) return EMU_E_ARG;
    if (n_tok < 1 || n_tok > 8) return EMU_E_ARG;
    const bool mm = (flags & EMU_MV_MFMA_MAJOR) != 0;
    if (mm && (flags & EMU_MV_LANE_MAJOR)) return EMU_E_ARG;
    size_t rb = 0;
    int st = mm ? emu_row_bytes(encoding, cols, &rb) : check_matrix(encoding, w_len, rows, cols, &rb);
    if (st != EMU_OK) return st;
    if (mm && w_len != emu_mfma_major_bytes(rows, cols)) return EMU_E_SHAPE;
    if (x_len < (size_t)n_tok * cols) return EMU_E_ACTIVATION_LEN;
    QmvArgs a{};
    a.w = static_cast<const uint8_t *>(d_w);
    a.row_bytes = rb;
    a.rows = (int)rows;
    a.cols = (int)cols;
    uint32_t be = 0, bb = 0;
    emu_block_layout(encoding, &be, &bb);
    a.nb = (int)(cols / be);
    a.x = d_x;
    a.y = d_y;
    a.accumulate = (flags & EMU_MV_ACCUMULATE) ? 1 : 0;
    a.lane_major = (flags & EMU_MV_LANE_MAJOR) ? 1 : 0;
    a.mfma_major = mm ? 1 : 0;
    a.f32_act = (flags & EMU_MV_F32_ACT) ? 1 : 0;
    return emu_launch_qmv(ctx, encoding, a, (int)n_tok);
}

extern "C" int emu_qmatvec_fused(emu_ctx *ctx, int encoding, const void *d_w, const void *d_w_up,
                                 uint32_t rows, uint32_t cols, const float *d_x, uint32_t n_tok,
                                 const float *d_gain, float eps, float *d_y, uint32_t flags)
{
    if (!ctx || !d_w || !d_x || !d_y) return EMU_E_ARG;
    if (n_tok < 1 || n_tok > 8) return EMU_E_ARG;
    size_t rb = 0;
    int st = emu_row_bytes(encoding, cols, &rb);
    if (st != EMU_OK) return st;
    uint32_t be = 0, bb = 0;
    emu_block_layout(encoding, &be, &bb);
    QmvArgs a{};
    a.w = static_cast<const uint8_t *>(d_w);
    a.w_up = static_cast<const uint8_t *>(d_w_up);
    a.row_bytes = rb;
    a.rows = (int)rows;
    a.cols = (int)cols;
    a.nb = (int)(cols / be);
    a.x = d_x;
    a.gain = d_gain;
    a.eps = eps;
    a.y = d_y;
    a.accumulate = (flags & EMU_MV_ACCUMULATE) ? 1 : 0;
    a.lane_major = (flags & EMU_MV_LANE_MAJOR) ? 1 : 0;
    a.mfma_major = (flags & EMU_MV_MFMA_MAJOR) ? 1 : 0;
    a.f32_act = (flags & EMU_MV_F32_ACT) ? 1 : 0;
    if (a.lane_major && a.mfma_major) return EMU_E_ARG;
    return emu_launch_qmv(ctx, encoding, a, (int)n_tok);
}

extern "C" int emu_quantize_act(emu_ctx *ctx, const float *d_x, uint32_t n_tok, uint32_t cols,
                                int8_t *d_q, float *d_scales)
{
    if (!ctx || !d_x || !d_q || !d_scales) return EMU_E_ARG;
    if (cols % 32 != 0) return EMU_E_SHORT;
    const size_t nblk = (size_t)n_tok * cols / 32;
    if (nblk == 0) return EMU_OK;
    hipLaunchKernelGGL(quantize_act_kernel, dim3((unsigned)((nblk + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, ctx->stream, d_x, nblk, d_q, d_scales);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

extern "C" int emu_block_dots(emu_ctx *ctx, int encoding, const void *d_w, size_t w_len, uint32_t rows,
                              uint32_t cols, const int8_t *d_q, uint32_t n_tok, int32_t *d_out)
{
    if (!ctx || !d_w || !d_q || !d_out) return EMU_E_ARG;
    size_t rb = 0;
    int st = check_matrix(encoding, w_len, rows, cols, &rb);
    if (st != EMU_OK) return st;
    const uint8_t *w = static_cast<const uint8_t *>(d_w);
    switch (encoding) {
    case EMU_ENC_Q6_K: return launch_block_dots<FmtQ6K>(ctx, w, rb, rows, cols, d_q, n_tok, d_out);
    case EMU_ENC_Q8_0: return launch_block_dots<FmtQ8_0>(ctx, w, rb, rows, cols, d_q, n_tok, d_out);
    case EMU_ENC_Q5_K: return launch_block_dots<FmtQ5K>(ctx, w, rb, rows, cols, d_q, n_tok, d_out);
    case EMU_ENC_Q2_K: return launch_block_dots<FmtQ2K>(ctx, w, rb, rows, cols, d_q, n_tok, d_out);
    default: return EMU_E_UNSUPPORTED;
    }
}

extern "C" int emu_qmatvec_i8(emu_ctx *ctx, int encoding, const void *d_w, size_t w_len, uint32_t rows,
                              uint32_t cols, const int8_t *d_q, const float *d_scales, uint32_t n_tok,
                              float *d_y)
{
    if (!ctx || !d_w || !d_q || !d_scales || !d_y) return EMU_E_ARG;
    size_t rb = 0;
    int st = check_matrix(encoding, w_len, rows, cols, &rb);
    if (st != EMU_OK) return st;
    if (cols % 32 != 0) return EMU_E_SHORT;
    const uint8_t *w = static_cast<const uint8_t *>(d_w);
    switch (encoding) {
    case EMU_ENC_Q6_K: return launch_qmv_i8<FmtQ6K>(ctx, w, rb, rows, cols, d_q, d_scales, n_tok, d_y);
    case EMU_ENC_Q8_0: return launch_qmv_i8<FmtQ8_0>(ctx, w, rb, rows, cols, d_q, d_scales, n_tok, d_y);
    case EMU_ENC_Q5_K: return launch_qmv_i8<FmtQ5K>(ctx, w, rb, rows, cols, d_q, d_scales, n_tok, d_y);
    case EMU_ENC_Q2_K: return launch_qmv_i8<FmtQ2K>(ctx, w, rb, rows, cols, d_q, d_scales, n_tok, d_y);
    default: return EMU_E_UNSUPPORTED;
    }
}
