// moe.hip -- selected-expert FFN of one MoE layer (moe::run,
// spm-granite-moe/src/moe.rs:37-159; the Gemma expert form of
// gemma_smoke.rs:92-139).
//
// After routing (emu_route: ids and weights, n_tok x k), three launches:
//   1. gate|up: grid (expert, row tile).  A wavefront finds the tokens routed
//      to its expert with one ballot over the n_tok*k routing table (token
//      order, as expert_tokens does), streams gate and up rows once for all of
//      them, and writes act(gate) * up per (token, slot);
//   2. down: grid (expert, row tile) over the hidden rows, reading the
//      activations of the expert's tokens, times the expert's optional output
//      scale, into a per-(token, slot) contribution;
//   3. combine: per token and column, output = +0.0 plus contribution * weight
//      added in ascending expert id (accumulate, moe.rs:58-75, with the experts
//      visited in BTreeSet order), each product rounded before the add.
// Expert rows are short (a 1024-column Q6_K row is 32 units of 32 weights),
// so a row takes L = 16, 32 or 64 lanes (the unit count rounded up to a power
// of two) and a wavefront works 64/L rows at once: every lane loads, and a
// wavefront's rows cost one memory round trip.  With L <= 32 the gate and up
// rows of one hidden unit sit in neighbouring lane groups and meet by one
// cross-group shuffle.
// Experts nobody chose cost one ballot per wavefront.  Weights are read once
// per step however many tokens share an expert (the reference's batch reuse).
#include "internal.hpp"

#include <math.h>
#include <stdlib.h>

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / EMU_WAVE;
constexpr int kMaxTok = 8;

struct MoeArgs {
    const uint8_t *gate, *up, *down; // up == nullptr: gate holds 2*ff rows per expert (gate, then up)
    const float *down_scale;         // per expert, or null
    size_t rb_in, rb_ff;             // row bytes of gate/up rows (width cols) and down rows (ff cols)
    int nb_in, nb_ff;                // blocks per row
    int n_experts, width, ff, k, n_tok, act;
    const float *x;                  // n_tok x width
    const int32_t *ids;              // n_tok x k
    const float *weights;            // n_tok x k
    float *act_buf;                  // (n_tok*k) x ff
    float *contrib;                  // (n_tok*k) x width
    float *out;                      // n_tok x width, or
    float *resid;                    // the residual stream it is added to (r + sum * resid_scale)
    float resid_scale;
    // Experts in cache slots instead of expert-major tensors: table[e] holds
    // expert e's gate rows, up rows and down rows back to back (null for an
    // expert no token routes to).
    const uint8_t *const *table;
};

// Rows of expert e: gate row r, up row r (hidden unit r), down row r.
__device__ __forceinline__ const uint8_t *gate_row(const MoeArgs &a, int e, int r)
{
    if (a.table) return a.table[e] + (size_t)r * a.rb_in;
    const size_t per = (size_t)(a.up ? 1 : 2) * a.ff;
    return a.gate + ((size_t)e * per + r) * a.rb_in;
}
__device__ __forceinline__ const uint8_t *up_row(const MoeArgs &a, int e, int r)
{
    if (a.table) return a.table[e] + ((size_t)a.ff + r) * a.rb_in;
    if (a.up) return a.up + ((size_t)e * a.ff + r) * a.rb_in;
    return a.gate + ((size_t)e * 2 * a.ff + a.ff + r) * a.rb_in;
}
__device__ __forceinline__ const uint8_t *down_row(const MoeArgs &a, int e, int r)
{
    if (a.table) return a.table[e] + 2 * (size_t)a.ff * a.rb_in + (size_t)r * a.rb_ff;
    return a.down + ((size_t)e * a.width + r) * a.rb_ff;
}

__device__ __forceinline__ void load8(const float *p, float v[8])
{
    const float4 a = *reinterpret_cast<const float4 *>(p);
    const float4 b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// The routing-table entries (t*k + slot) that chose expert e, ascending
// (token order); at most kMaxTok of them, since a token picks an expert once.
__device__ __forceinline__ int expert_slots(const MoeArgs &a, int e, int lane, int (&slot)[kMaxTok])
{
    const int nk = a.n_tok * a.k;
    const bool hit = lane < nk && a.ids[lane] == e;
    uint64_t m = __ballot(hit);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < kMaxTok; ++i) {
        slot[i] = m ? __ffsll((unsigned long long)m) - 1 : 0;
        cnt += m ? 1 : 0;
        m &= m - 1;
    }
    return cnt;
}

template <int ACT> __device__ __forceinline__ float activate(float g, float u)
{
#pragma clang fp contract(off)
    if (ACT == EMU_ACT_GELU_TANH) return emu_gelu_tanh(g) * u;
    return (g / (1.0f + expf(-g))) * u; // moe.rs:46-56
}

// One row of one expert matrix against the cnt routed input vectors
// (in[slot[t] * in_stride + c]), worked by the L lanes q = 0..L-1 of a lane
// group; per-lane partial sums, not yet reduced.
template <class F, int L>
__device__ __forceinline__ void row_dots(const uint8_t *row, int nb, const float *in, int in_stride,
                                         const int (&slot)[kMaxTok], int cnt, int q, float (&acc)[kMaxTok])
{
    const int U = nb * F::UPB;
    for (int u = q; u < U; u += L) {
        const int blk = u / F::UPB, sub = u % F::UPB;
        typename F::Raw raw;
        F::load(row, (uint32_t)blk * F::BB, sub, raw);
        const int c0 = blk * F::BE;
#pragma unroll
        for (int g = 0; g < F::G; ++g) {
            const Grp gp = F::group(raw, sub, g);
            float w[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i] = grp_weight(gp, i);
            const int col = c0 + F::col(sub, g);
#pragma unroll
            for (int t = 0; t < kMaxTok; ++t) {
                if (t < cnt) {
                    float xv[8];
                    load8(in + (size_t)slot[t] * in_stride + col, xv);
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[t] = __builtin_fmaf(w[i], xv[i], acc[t]);
                }
            }
        }
    }
}

// The dots of one unit (lane q's unit q of a row of U <= L units) against
// the cnt routed vectors, from the unit's raw bytes.
template <class F>
__device__ __forceinline__ void unit_dots(const typename F::Raw &raw, int u, const float *in, int in_stride,
                                          const int (&slot)[kMaxTok], int cnt, float (&acc)[kMaxTok])
{
    const int blk = u / F::UPB, sub = u % F::UPB;
    const int c0 = blk * F::BE;
#pragma unroll
    for (int g = 0; g < F::G; ++g) {
        const Grp gp = F::group(raw, sub, g);
        float w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = grp_weight(gp, i);
        const int col = c0 + F::col(sub, g);
#pragma unroll
        for (int t = 0; t < kMaxTok; ++t) {
            if (t < cnt) {
                float xv[8];
                load8(in + (size_t)slot[t] * in_stride + col, xv);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[t] = __builtin_fmaf(w[i], xv[i], acc[t]);
            }
        }
    }
}

// The same unit u of R rows (so the same columns) against CNT routed
// vectors (the expert's token count rounded up to 1, 2, 4 or 8; slots past
// the real count read slot 0 and their sums are never used): a group's 8
// activations per token are loaded once for all R rows, every token's loads
// of a group issued together with no branch around them.
template <class F, int R, int CNT>
__device__ __forceinline__ void units_dots(const typename F::Raw (&raw)[R], int u, const float *in, int in_stride,
                                           const int (&slot)[kMaxTok], float (&acc)[R][kMaxTok])
{
    const int blk = u / F::UPB, sub = u % F::UPB;
    const int c0 = blk * F::BE;
#pragma unroll
    for (int g = 0; g < F::G; ++g) {
        const int col = c0 + F::col(sub, g);
        float xv[CNT][8];
#pragma unroll
        for (int t = 0; t < CNT; ++t) load8(in + (size_t)slot[t] * in_stride + col, xv[t]);
        float w[R][8];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const Grp gp = F::group(raw[r], sub, g);
#pragma unroll
            for (int i = 0; i < 8; ++i) w[r][i] = grp_weight(gp, i);
        }
#pragma unroll
        for (int t = 0; t < CNT; ++t)
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[r][t] = __builtin_fmaf(w[r][i], xv[t][i], acc[r][t]);
    }
}

// units_dots with the token count bucketed at run time (uniform per wavefront).
template <class F, int R>
__device__ __forceinline__ void units_dots_any(const typename F::Raw (&raw)[R], int u, const float *in,
                                               int in_stride, const int (&slot)[kMaxTok], int cnt,
                                               float (&acc)[R][kMaxTok])
{
    if (cnt <= 1) units_dots<F, R, 1>(raw, u, in, in_stride, slot, acc);
    else if (cnt <= 2) units_dots<F, R, 2>(raw, u, in, in_stride, slot, acc);
    else if (cnt <= 4) units_dots<F, R, 4>(raw, u, in, in_stride, slot, acc);
    else units_dots<F, R, 8>(raw, u, in, in_stride, slot, acc);
}

template <class F> __device__ __forceinline__ void unit_load(const uint8_t *row, int u, typename F::Raw &raw)
{
    F::load(row, (uint32_t)(u / F::UPB) * F::BB, u % F::UPB, raw);
}

// Sum over the L lanes of a lane group (L a power of two, <= 64).
template <int L> __device__ __forceinline__ float group_sum(float v)
{
    return emu_group_sum<L>(v);
}

// Hidden units per wavefront of the gate|up kernel with L lanes per row.
template <int L> constexpr int up_rows_per_wave() { return L >= EMU_WAVE ? 1 : EMU_WAVE / L / 2; }

template <class F, int ACT, int L>
__global__ __launch_bounds__(kThreads) void moe_up_kernel(MoeArgs a)
{
    constexpr int S = EMU_WAVE / L; // rows a wavefront works at once
    const int e = blockIdx.x;
    const int lane = threadIdx.x & (EMU_WAVE - 1), wv = threadIdx.x / EMU_WAVE;
    int slot[kMaxTok];
    const int cnt = expert_slots(a, e, lane, slot);
    if (cnt == 0) return; // uniform: the ballot is the same in every wavefront
    // Token rows of x: slot / k is the token.
    int tok[kMaxTok];
#pragma unroll
    for (int t = 0; t < kMaxTok; ++t) tok[t] = slot[t] / a.k;
    const int j = lane / L, q = lane % L;
    // Lane groups 2i and 2i+1 take the gate and up rows of hidden unit r; the
    // groups of one unit (and every lane a shuffle below reads) share r, so
    // they leave together.
    const int r = (blockIdx.y * kWaves + wv) * up_rows_per_wave<L>() + (S >= 2 ? j >> 1 : 0);
    if (r >= a.ff) return;
    const uint8_t *grow = gate_row(a, e, r);
    const uint8_t *urow = up_row(a, e, r);
    float ag[kMaxTok], au[kMaxTok];
#pragma unroll
    for (int t = 0; t < kMaxTok; ++t) ag[t] = au[t] = 0.0f;
    if constexpr (S >= 2) {
        const bool is_up = j & 1;
        row_dots<F, L>(is_up ? urow : grow, a.nb_in, a.x, a.width, tok, cnt, q, ag);
#pragma unroll
        for (int t = 0; t < kMaxTok; ++t) {
            if (t < cnt) {
                ag[t] = group_sum<L>(ag[t]);
                au[t] = emu_xor_get<L>(ag[t]);
            }
        }
        if (is_up || q != 0) return;
    } else {
        row_dots<F, L>(grow, a.nb_in, a.x, a.width, tok, cnt, q, ag);
        row_dots<F, L>(urow, a.nb_in, a.x, a.width, tok, cnt, q, au);
#pragma unroll
        for (int t = 0; t < kMaxTok; ++t) {
            if (t < cnt) {
                ag[t] = group_sum<L>(ag[t]);
                au[t] = group_sum<L>(au[t]);
            }
        }
        if (q != 0) return;
    }
#pragma unroll
    for (int t = 0; t < kMaxTok; ++t)
        if (t < cnt) a.act_buf[(size_t)slot[t] * a.ff + r] = activate<ACT>(ag[t], au[t]);
}

// Rows of at most L units (one per lane): a wavefront works P row sets, every
// set's unit loads issued before the first dot, so one memory round trip
// serves P times the rows.  Rows past the matrix are computed on a valid row
// and not stored.
constexpr int kPasses = 4;
template <int L> constexpr int up_passes() { return L >= EMU_WAVE ? kPasses / 2 : kPasses; }
constexpr int kUpRounds = 2;

template <class F, int ACT, int L>
__global__ __launch_bounds__(kThreads) void moe_up_p_kernel(MoeArgs a)
{
    constexpr int S = EMU_WAVE / L, RPW = up_rows_per_wave<L>();
    constexpr int NR = S >= 2 ? 1 : 2;         // rows a lane loads per pass (L = 64: gate and up)
    constexpr int P = up_passes<L>();           // four rows per lane in all
    const int e = blockIdx.x;
    const int lane = threadIdx.x & (EMU_WAVE - 1), wv = threadIdx.x / EMU_WAVE;
    int slot[kMaxTok];
    const int cnt = expert_slots(a, e, lane, slot);
    if (cnt == 0) return;
    int tok[kMaxTok];
#pragma unroll
    for (int t = 0; t < kMaxTok; ++t) tok[t] = slot[t] / a.k;
    const int j = lane / L, q = lane % L;
    const int U = a.nb_in * F::UPB;
    const bool has_unit = q < U;
    const int u = has_unit ? q : 0;
    // kUpRounds row sets per wavefront, one after another: half the
    // workgroups, so the routed experts' waves fit the CUs in one round.
    for (int round = 0; round < kUpRounds; ++round) {
        const int r0 = ((blockIdx.y * kWaves + wv) * kUpRounds + round) * P * RPW + (S >= 2 ? j >> 1 : 0);
        typename F::Raw raw[P * NR];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            int r = r0 + p * RPW;
            r = r < a.ff ? r : a.ff - 1;
            const uint8_t *grow = gate_row(a, e, r);
            const uint8_t *urow = up_row(a, e, r);
            if (NR == 1) unit_load<F>((j & 1) ? urow : grow, u, raw[p]);
            else {
                unit_load<F>(grow, u, raw[NR * p]);
                unit_load<F>(urow, u, raw[NR * p + 1]);
            }
        }
        float accs[P * NR][kMaxTok];
#pragma unroll
        for (int i = 0; i < P * NR; ++i)
#pragma unroll
            for (int t = 0; t < kMaxTok; ++t) accs[i][t] = 0.0f;
        if (has_unit) units_dots_any<F, P * NR>(raw, u, a.x, a.width, tok, cnt, accs);
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int r = r0 + p * RPW;
            float ag[kMaxTok], au[kMaxTok];
#pragma unroll
            for (int t = 0; t < kMaxTok; ++t) {
                ag[t] = au[t] = 0.0f;
                if (t < cnt) {
                    ag[t] = group_sum<L>(accs[NR * p][t]);
                    au[t] = NR == 2 ? group_sum<L>(accs[NR * p + 1][t]) : emu_xor_get<L>(ag[t]);
                }
            }
            const bool writer = q == 0 && (NR == 2 || !(j & 1));
            if (writer && r < a.ff) {
#pragma unroll
                for (int t = 0; t < kMaxTok; ++t)
                    if (t < cnt) a.act_buf[(size_t)slot[t] * a.ff + r] = activate<ACT>(ag[t], au[t]);
            }
        }
    }
}

template <class F, int L>
__global__ __launch_bounds__(kThreads) void moe_down_p_kernel(MoeArgs a)
{
    constexpr int S = EMU_WAVE / L;
    const int e = blockIdx.x;
    const int lane = threadIdx.x & (EMU_WAVE - 1), wv = threadIdx.x / EMU_WAVE;
    int slot[kMaxTok];
    const int cnt = expert_slots(a, e, lane, slot);
    if (cnt == 0) return;
    const int j = lane / L, q = lane % L;
    const int U = a.nb_ff * F::UPB;
    const bool has_unit = q < U;
    const int u = has_unit ? q : 0;
    const int r0 = (blockIdx.y * kWaves + wv) * kPasses * S + j;
    typename F::Raw raw[kPasses];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        int r = r0 + p * S;
        r = r < a.width ? r : a.width - 1;
        unit_load<F>(down_row(a, e, r), u, raw[p]);
    }
    const float scale = a.down_scale ? a.down_scale[e] : 1.0f;
    float accs[kPasses][kMaxTok];
#pragma unroll
    for (int p = 0; p < kPasses; ++p)
#pragma unroll
        for (int t = 0; t < kMaxTok; ++t) accs[p][t] = 0.0f;
    if (has_unit) units_dots_any<F, kPasses>(raw, u, a.act_buf, a.ff, slot, cnt, accs);
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int r = r0 + p * S;
#pragma unroll
        for (int t = 0; t < kMaxTok; ++t) {
            if (t < cnt) {
                float v = group_sum<L>(accs[p][t]);
                if (a.down_scale) v = __fmul_rn(v, scale); // gemma_smoke.rs:129-137
                if (q == 0 && r < a.width) a.contrib[(size_t)slot[t] * a.width + r] = v;
            }
        }
    }
}

template <class F, int L>
__global__ __launch_bounds__(kThreads) void moe_down_kernel(MoeArgs a)
{
    constexpr int S = EMU_WAVE / L;
    const int e = blockIdx.x;
    const int lane = threadIdx.x & (EMU_WAVE - 1), wv = threadIdx.x / EMU_WAVE;
    int slot[kMaxTok];
    const int cnt = expert_slots(a, e, lane, slot);
    if (cnt == 0) return;
    const int j = lane / L, q = lane % L;
    const int r = (blockIdx.y * kWaves + wv) * S + j; // a lane group's row; the group leaves together
    if (r >= a.width) return;
    const float scale = a.down_scale ? a.down_scale[e] : 1.0f;
    const uint8_t *row = down_row(a, e, r);
    float acc[kMaxTok];
#pragma unroll
    for (int t = 0; t < kMaxTok; ++t) acc[t] = 0.0f;
    row_dots<F, L>(row, a.nb_ff, a.act_buf, a.ff, slot, cnt, q, acc);
#pragma unroll
    for (int t = 0; t < kMaxTok; ++t) {
        if (t < cnt) {
            float v = group_sum<L>(acc[t]);
            if (a.down_scale) v = __fmul_rn(v, scale); // gemma_smoke.rs:129-137
            if (q == 0) a.contrib[(size_t)slot[t] * a.width + r] = v;
        }
    }
}

// Per token (blockIdx.x) and column: sum over its slots in ascending expert
// id, from +0.0.
__global__ __launch_bounds__(kThreads) void moe_combine_kernel(MoeArgs a)
{
    const int t = blockIdx.x;
    const int c = blockIdx.y * kThreads + threadIdx.x;
    if (c >= a.width) return;
    int order[8];
    float w[8];
    const int n = emu_route_order(a.ids + t * a.k, a.weights + t * a.k, a.k, a.n_experts, order, w);
    float v[kMaxTok];
#pragma unroll
    for (int i = 0; i < kMaxTok; ++i) v[i] = i < n ? a.contrib[((size_t)t * a.k + order[i]) * a.width + c] : 0.0f;
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxTok; ++i)
        if (i < n) sum = __fadd_rn(sum, __fmul_rn(v[i], w[i]));
    if (a.resid) {
        float *r = a.resid + (size_t)t * a.width + c;
        *r = emu_resid_add(*r, sum, a.resid_scale);
    } else {
        a.out[(size_t)t * a.width + c] = sum;
    }
}

// Lanes per row for a row of U units: the power of two in {16, 32, 64} that
// covers it (longer rows loop).
int lanes_for(int units) { return units > 32 ? 64 : units > 16 ? 32 : 16; }

template <class F, int ACT, int L> void launch_up_l(emu_ctx *ctx, const MoeArgs &a)
{
    if (a.nb_in * F::UPB <= L) { // one unit per lane: the multi-row form
        constexpr int per_block = kWaves * up_rows_per_wave<L>() * up_passes<L>() * kUpRounds;
        const dim3 grid(a.n_experts, (a.ff + per_block - 1) / per_block);
        hipLaunchKernelGGL((moe_up_p_kernel<F, ACT, L>), grid, dim3(kThreads), 0, ctx->stream, a);
        return;
    }
    constexpr int per_block = kWaves * up_rows_per_wave<L>();
    const dim3 grid(a.n_experts, (a.ff + per_block - 1) / per_block);
    hipLaunchKernelGGL((moe_up_kernel<F, ACT, L>), grid, dim3(kThreads), 0, ctx->stream, a);
}

template <class F, int ACT> void launch_up_a(emu_ctx *ctx, const MoeArgs &a)
{
    switch (lanes_for(a.nb_in * F::UPB)) {
    case 16: launch_up_l<F, ACT, 16>(ctx, a); break;
    case 32: launch_up_l<F, ACT, 32>(ctx, a); break;
    default: launch_up_l<F, ACT, 64>(ctx, a); break;
    }
}

template <class F> void launch_up(emu_ctx *ctx, const MoeArgs &a)
{
    if (a.act == EMU_ACT_GELU_TANH)
        launch_up_a<F, EMU_ACT_GELU_TANH>(ctx, a);
    else
        launch_up_a<F, EMU_ACT_SILU>(ctx, a);
}

template <class F, int L> void launch_down_l(emu_ctx *ctx, const MoeArgs &a)
{
    if (a.nb_ff * F::UPB <= L) {
        constexpr int per_block = kWaves * (EMU_WAVE / L) * kPasses;
        const dim3 grid(a.n_experts, (a.width + per_block - 1) / per_block);
        hipLaunchKernelGGL((moe_down_p_kernel<F, L>), grid, dim3(kThreads), 0, ctx->stream, a);
        return;
    }
    constexpr int per_block = kWaves * (EMU_WAVE / L);
    const dim3 grid(a.n_experts, (a.width + per_block - 1) / per_block);
    hipLaunchKernelGGL((moe_down_kernel<F, L>), grid, dim3(kThreads), 0, ctx->stream, a);
}

template <class F> void launch_down(emu_ctx *ctx, const MoeArgs &a)
{
    switch (lanes_for(a.nb_ff * F::UPB)) {
    case 16: launch_down_l<F, 16>(ctx, a); break;
    case 32: launch_down_l<F, 32>(ctx, a); break;
    default: launch_down_l<F, 64>(ctx, a); break;
    }
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

} // namespace

extern "C" size_t emu_moe_workspace_bytes(uint32_t n_tok, uint32_t k, uint32_t width, uint32_t ff)
{
    const size_t slots = (size_t)n_tok * k;
    return align256(sizeof(float) * slots * ff) + align256(sizeof(float) * slots * width);
}

namespace {

int moe_ffn(emu_ctx *ctx, const emu_moe_desc *d, const float *d_x, uint32_t n_tok, const int32_t *d_ids,
            const float *d_weights, void *d_workspace, size_t workspace_bytes, float *d_out, float *d_resid,
            float resid_scale, bool combine = true, const uint8_t *const *d_table = nullptr)
{
    if (!ctx || !d || !d_x || !d_ids || !d_weights || !(d_out || d_resid) || (!d_table && (!d->d_gate || !d->d_down)))
        return EMU_E_ARG;
    if (n_tok == 0) return EMU_OK;
    if (n_tok > kMaxTok || d->k == 0 || d->k > 8 || d->n_experts == 0 || d->k > d->n_experts) return EMU_E_ARG;
    if (d->act != EMU_ACT_SILU && d->act != EMU_ACT_GELU_TANH) return EMU_E_ARG;
    uint32_t be_in = 0, bb_in = 0, be_ff = 0, bb_ff = 0;
    int st = emu_block_layout(d->enc_gate_up, &be_in, &bb_in);
    if (st == EMU_OK) st = emu_block_layout(d->enc_down, &be_ff, &bb_ff);
    if (st != EMU_OK) return st;
    if (d->width == 0 || d->ff == 0 || d->width % be_in != 0 || d->ff % be_ff != 0) return EMU_E_SHORT;
    if (d->width % 8 != 0 || d->ff % 8 != 0) return EMU_E_SHAPE; // 8-column activation groups
    if (!d_workspace || workspace_bytes < emu_moe_workspace_bytes(n_tok, d->k, d->width, d->ff)) return EMU_E_ARG;
    MoeArgs a{};
    a.gate = static_cast<const uint8_t *>(d->d_gate);
    a.up = static_cast<const uint8_t *>(d->d_up);
    a.down = static_cast<const uint8_t *>(d->d_down);
    a.down_scale = d->d_down_scale;
    a.nb_in = (int)(d->width / be_in);
    a.nb_ff = (int)(d->ff / be_ff);
    a.rb_in = (size_t)a.nb_in * bb_in;
    a.rb_ff = (size_t)a.nb_ff * bb_ff;
    a.n_experts = (int)d->n_experts;
    a.width = (int)d->width;
    a.ff = (int)d->ff;
    a.k = (int)d->k;
    a.n_tok = (int)n_tok;
    a.act = d->act;
    a.x = d_x;
    a.ids = d_ids;
    a.weights = d_weights;
    a.act_buf = static_cast<float *>(d_workspace);
    a.contrib = const_cast<float *>(emu_moe_contrib(d_workspace, n_tok, d->k, d->ff));
    a.out = d_out;
    a.resid = d_resid;
    a.resid_scale = resid_scale;
    a.table = d_table;
    switch (d->enc_gate_up) {
    case EMU_ENC_Q6_K: launch_up<FmtQ6K>(ctx, a); break;
    case EMU_ENC_Q8_0: launch_up<FmtQ8_0>(ctx, a); break;
    case EMU_ENC_Q5_K: launch_up<FmtQ5K>(ctx, a); break;
    case EMU_ENC_Q2_K: launch_up<FmtQ2K>(ctx, a); break;
    default: return EMU_E_UNSUPPORTED;
    }
    EMU_LAUNCH_CHECK(ctx);
    switch (d->enc_down) {
    case EMU_ENC_Q6_K: launch_down<FmtQ6K>(ctx, a); break;
    case EMU_ENC_Q8_0: launch_down<FmtQ8_0>(ctx, a); break;
    case EMU_ENC_Q5_K: launch_down<FmtQ5K>(ctx, a); break;
    case EMU_ENC_Q2_K: launch_down<FmtQ2K>(ctx, a); break;
    default: return EMU_E_UNSUPPORTED;
    }
    EMU_LAUNCH_CHECK(ctx);
    if (!combine) return EMU_OK;
    hipLaunchKernelGGL(moe_combine_kernel, dim3(n_tok, (d->width + kThreads - 1) / kThreads), dim3(kThreads), 0,
                       ctx->stream, a);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

} // namespace

extern "C" int emu_moe_ffn(emu_ctx *ctx, const emu_moe_desc *d, const float *d_x, uint32_t n_tok,
                           const int32_t *d_ids, const float *d_weights, void *d_workspace, size_t workspace_bytes,
                           float *d_out)
{
    if (!d_out) return EMU_E_ARG;
    return moe_ffn(ctx, d, d_x, n_tok, d_ids, d_weights, d_workspace, workspace_bytes, d_out, nullptr, 0.0f);
}

// The selected-expert FFN with expert e's gate, up and down rows at
// d_table[e] (cache.hip).
int emu_moe_ffn_table(emu_ctx *ctx, const emu_moe_desc *d, const uint8_t *const *d_table, const float *d_x,
                      uint32_t n_tok, const int32_t *d_ids, const float *d_weights, void *d_workspace,
                      size_t workspace_bytes, float *d_out)
{
    if (!d_out || !d_table) return EMU_E_ARG;
    return moe_ffn(ctx, d, d_x, n_tok, d_ids, d_weights, d_workspace, workspace_bytes, d_out, nullptr, 0.0f, true,
                   d_table);
}

int emu_moe_ffn_resid(emu_ctx *ctx, const emu_moe_desc *d, const float *d_x, uint32_t n_tok, const int32_t *d_ids,
                      const float *d_weights, void *d_workspace, size_t workspace_bytes, float *d_state,
                      float scale, bool combine)
{
    if (!d_state) return EMU_E_ARG;
    return moe_ffn(ctx, d, d_x, n_tok, d_ids, d_weights, d_workspace, workspace_bytes, nullptr, d_state, scale,
                   combine);
}

const float *emu_moe_contrib(const void *d_workspace, uint32_t n_tok, uint32_t k, uint32_t ff)
{
    return reinterpret_cast<const float *>(static_cast<const uint8_t *>(d_workspace) +
                                           align256(sizeof(float) * (size_t)n_tok * k * ff));
}
