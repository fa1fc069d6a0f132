// moe.hip -- selected-expert FFN of one MoE layer (moe::run,
// spm-granite-moe/src/moe.rs:37-159; the Gemma expert form of
// gemma_smoke.rs:92-139).
//
// After routing (emu_route: ids and weights, n_tok x k), inputs of up to 4096
// columns take the matrix-core form (the section "matrix-core form" below):
//   1. limbs: the tokens' x as int8 limb planes (or the decode step's gate
//      kernel writes them);
//   2. gate|up on v_mfma_i32_32x32x16_i8, one grid row per routed expert
//      (each workgroup reads its expert off the routing table), writing
//      act(gate) * up per (token, slot);
//   3. limbs: the activations as limb planes;
//   4. down on the matrix cores into a per-(token, slot) contribution;
//   5. combine, as below.
// Wider inputs (and EMU_MOE_MMA=0) take the direct form, three launches:
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
#include <type_traits>

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

// ---- matrix-core form ---------------------------------------------------------
// The batch-1 limb idea on v_mfma_i32_32x32x16_i8, for every expert format.
// Each routed input vector (a token's x for gate|up, a route's activation for
// down) is carried as three signed 7-bit limbs per column with one
// power-of-two scale per 256-column span, x ~= s * (16384*L0 + 128*L1 + L2),
// exact to 2^-20 of the span's largest |x|.  One MFMA takes one 16-column
// chunk: A (32 x 16) holds M row 8*limb + position (an expert's routed vectors
// are its positions 0..7; rows 24..31 and positions past its count are zero),
// B (16 x 32) the codes of 32 weight rows.  Lane l, register r of the result
// holds limb r/4 of position 4*(l/32) + r%4 for weight row l%32.
//
// Within a span the sums stay integers and the span's d (and dmin) and the
// activation scale apply once per span:
//   Q2_K  a code times its 4-bit sub-block scale fits a byte, so B carries
//         the scaled codes and the chunks chain on the matrix pipe;
//   Q6_K  each chunk's limb sums times the chunk's int8 scale, added into a
//         32-bit integer per limb;
//   Q5_K  a sub-block's two chunks chain, times its 6-bit scale, likewise;
//   Q8_0  a block's two chunks chain, times its d, in float.
// The per-chunk terms that do not depend on the codes -- Q6_K's code bias
// (-32 * sc * sum x) and the K-quant mins (dmin * m * sum x) -- are one more
// product per span: each vector's per-chunk limb sums S (|S| <= 1024) are kept
// as two int8 digits, S = 64 h + l, and two MFMAs take them against the
// chunks' coefficients (K = the span's 16 chunks).
//
// A workgroup's wavefronts each own a 32-row tile (gate|up: 16 gate rows and
// the 16 matching up rows, so the activation meets its pair in a lane
// shuffle) and a share of its spans; the shares meet in LDS in a fixed order.
// A wavefront stages each span's 32 rows through its own LDS rows, and a
// chunk's A operand register is refilled with the next span's chunk as soon
// as its MFMA has issued.  Three forms of the span loop:
//   one span per wavefront (the shares equal the spans): the rows come in by
//         coalesced 16-byte loads into registers and are stored to LDS;
//         nothing is prefetched, so the kernel holds 104-111 registers and
//         four workgroups fit a CU;
//   direct (Q5_K, Q2_K: 4-byte aligned spans): the rows go from memory
//         straight into LDS (global_load_lds_dword, one instruction per
//         row), and the next span's rows are requested as soon as the
//         current span's operand words have been read out of LDS, so the
//         prefetch holds no registers;
//   loop (Q6_K and Q8_0 spans start 2-byte aligned): the next span's rows
//         are in flight in registers while the current span computes.
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kChunkBytes = kEmuChunkBytes; // three int8 limbs of 16 columns
constexpr int kSpanChunks = kEmuSpanChunks; // 16-column chunks per 256-column span
constexpr int kSpanMeta = kEmuSpanMeta;     // per vector and span: digits [h, l][limb][16 chunks] int8, then the scale
constexpr int kMmaMaxCols = 4096;
constexpr int kMmaMaxSpans = kMmaMaxCols / 256;

// Limb planes of n vectors of C chunks (EmuLimbPlanes).
using LimbPlanes = EmuLimbPlanes;
int spans_of(int C) { return (C + kSpanChunks - 1) / kSpanChunks; }
size_t limb_plane_bytes(size_t n_vec, int C)
{
    return n_vec * ((size_t)C * kChunkBytes + (size_t)spans_of(C) * kSpanMeta);
}
LimbPlanes limb_planes(void *base, size_t n_vec, int C)
{
    LimbPlanes p;
    p.C = C;
    p.ns = spans_of(C);
    p.q = static_cast<uint8_t *>(base);
    p.dg = p.q + n_vec * C * kChunkBytes;
    return p;
}

// OR of a 64-bit value over the wavefront, every lane getting it.
__device__ __forceinline__ uint64_t wave_or_u64(uint64_t v)
{
    auto step = [](uint64_t x, auto off) {
        constexpr int OFF = decltype(off)::value;
        const uint32_t lo = __float_as_uint(emu_xor_get<OFF>(__uint_as_float((uint32_t)x)));
        const uint32_t hi = __float_as_uint(emu_xor_get<OFF>(__uint_as_float((uint32_t)(x >> 32))));
        return x | ((uint64_t)hi << 32) | lo;
    };
    v = step(v, std::integral_constant<int, 32>{});
    v = step(v, std::integral_constant<int, 16>{});
    v = step(v, std::integral_constant<int, 8>{});
    v = step(v, std::integral_constant<int, 4>{});
    v = step(v, std::integral_constant<int, 2>{});
    v = step(v, std::integral_constant<int, 1>{});
    return v;
}

// Entry y of the call's routed experts in ascending id, read off the
// routing table itself (ids[t], t < nk <= 64; a token's ids are distinct, so
// an expert has at most kMaxTok entries): the expert, its entry count and its
// entries t in ascending order (0 past the count); false past the last
// expert.  The matrix-core launches take one grid row per routed expert, so
// no workgroup slot is spent on experts nobody chose.  Every wavefront forms
// the same (uniform) result: the present experts as a 256-bit mask (an OR
// butterfly per 64-bit word), its y-th set bit, one ballot for the entries.
__device__ __forceinline__ bool list_entry(const int32_t *ids, int nk, int n_experts, int y, int &e, int &cnt,
                                           int (&slot)[kMaxTok])
{
    const int lane = threadIdx.x & (EMU_WAVE - 1);
    const int my = lane < nk ? ids[lane] : -1;
    const bool ok = my >= 0 && my < n_experts;
    int base = 0;
    e = -1;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint64_t b = wave_or_u64(ok && (my >> 6) == w ? 1ull << (my & 63) : 0ull);
        const int pc = __popcll(b);
        if (e < 0 && y < base + pc) { // uniform
            const int want = y - base; // lane l tests bit l
            const bool hit = ((b >> lane) & 1ull) && __popcll(b & ((1ull << lane) - 1ull)) == want;
            e = 64 * w + __ffsll((unsigned long long)__ballot(hit)) - 1;
        }
        base += pc;
    }
    if (e < 0) return false;
    uint64_t m = __ballot(my == e);
    const int c = __popcll(m);
    cnt = c < kMaxTok ? c : kMaxTok;
#pragma unroll
    for (int i = 0; i < kMaxTok; ++i) {
        slot[i] = m ? __ffsll((unsigned long long)m) - 1 : 0;
        m &= m - 1ull;
    }
    return true;
}

// n_vec vectors of cols floats (row stride cols) into limb planes: sixteen
// threads per span, one 16-column chunk each.
__global__ __launch_bounds__(kThreads) void moe_limbs_kernel(const float *x, int n_vec, int cols, LimbPlanes P)
{
    const int idx = blockIdx.x * kThreads + threadIdx.x;
    const int total = n_vec * P.ns * kSpanChunks; // whole groups of 16 lanes
    const int i = idx < total ? idx : total - 1;
    const int m = i % kSpanChunks, vs = i / kSpanChunks;
    const int vec = vs / P.ns, c = (vs % P.ns) * kSpanChunks + m;
    const bool col = c < P.C;
    float w[16];
#pragma unroll
    for (int k = 0; k < 2; ++k) load8(x + (size_t)vec * cols + 16 * (col ? c : 0) + 8 * k, w + 8 * k);
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const float a = col ? fabsf(w[e]) : 0.0f;
        amax = fmaxf(amax, a);
        bad |= !(a <= 3.402823466e38f);
    }
#pragma unroll
    for (int o = 1; o < kSpanChunks; o <<= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o, EMU_WAVE));
        bad |= __shfl_xor(bad, o, EMU_WAVE);
    }
    const bool finite = !bad;
    int e2 = 0;
    (void)frexpf(finite ? amax : 0.0f, &e2);
    if (idx >= total) return;
    uint32_t q[3][4] = {};
    int S[3] = {0, 0, 0};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        int L[3];
        emu_limb3(finite && col ? w[e] : 0.0f, e2, L);
#pragma unroll
        for (int l = 0; l < 3; ++l) {
            q[l][e >> 2] |= ((uint32_t)L[l] & 0xffu) << (8 * (e & 3));
            S[l] += L[l];
        }
    }
    // the digits, also for chunks past the columns (zero), so the span's
    // digit block is whole
    uint8_t *dg = P.dg + (size_t)vs * kSpanMeta + m;
#pragma unroll
    for (int l = 0; l < 3; ++l) {
        const int h = (S[l] + 32) >> 6; // |S| <= 1024: h in [-16, 16], S - 64h in [-32, 31]
        dg[16 * l] = (uint8_t)h;
        dg[48 + 16 * l] = (uint8_t)(S[l] - 64 * h);
    }
    if (col) {
        uint8_t *dst = P.q + ((size_t)vec * P.C + c) * kChunkBytes;
#pragma unroll
        for (int l = 0; l < 3; ++l)
            *reinterpret_cast<uint4 *>(dst + 16 * l) = make_uint4(q[l][0], q[l][1], q[l][2], q[l][3]);
    }
    if (m == 0)
        *reinterpret_cast<float *>(P.dg + (size_t)vs * kSpanMeta + 96) = finite ? ldexpf(1.0f, e2 - 20) : __int_as_float(0x7fc00000);
}

__device__ __forceinline__ double limb_combine(int d0, int d1, int d2)
{
    return (double)d0 * 16384.0 + (double)d1 * 128.0 + (double)d2; // exact
}

// Byte b of the eight packed bytes (b < 8).
__device__ __forceinline__ uint32_t byte8(uint2 v, int b) { return ((b < 4 ? v.x : v.y) >> (8 * (b & 3))) & 0xffu; }

__device__ __forceinline__ long pack8(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

// a * b + c for |a|, |b| < 2^23 (both sign-extended from 24 bits, which the
// compiler folds into v_mad_i32_i24, a full-rate instruction; a 32-bit
// integer multiply is quarter rate).  A chunk's limb sums are below 2^17
// and the scales below 2^7.
__device__ __forceinline__ int mad24(int a, int b, int c) { return ((a << 8) >> 8) * ((b << 8) >> 8) + c; }

// Pins twelve running sums at this point of the program: without it the
// compiler reassociates a span's sixteen chunk products into a tree at the
// end, which keeps every chunk's 16-register MFMA result alive at once.
__device__ __forceinline__ void pin12(int (&I)[12])
{
    asm volatile(""
                 : "+v"(I[0]), "+v"(I[1]), "+v"(I[2]), "+v"(I[3]), "+v"(I[4]), "+v"(I[5]), "+v"(I[6]), "+v"(I[7]),
                   "+v"(I[8]), "+v"(I[9]), "+v"(I[10]), "+v"(I[11]));
}

// The A operands of one span: the 16 chunks' limbs and the two limb sum
// digits, refilled chunk by chunk with the next span's; and the lane's
// position's span scale.
struct SpanA {
    long av[kSpanChunks];
    long ad[2];
    float sc;
};

// Where a lane's A operands come from: M row j = limb j/8 of position j%8,
// column half kh; zero for rows 24..31, positions past the count and chunks
// past the columns.
struct ASource {
    const uint8_t *q, *dg, *meta;
    int C, ns;
    bool live, pos;
    __device__ long chunk(int span, int m) const
    {
        const int c = kSpanChunks * span + m;
        return live && c < C ? *reinterpret_cast<const long *>(q + (size_t)c * kChunkBytes) : 0;
    }
    __device__ long digit(int span, int d) const
    {
        return live ? *reinterpret_cast<const long *>(dg + (size_t)span * kSpanMeta + 48 * d) : 0;
    }
    __device__ float scale(int span) const
    {
        return pos ? *reinterpret_cast<const float *>(meta + (size_t)span * kSpanMeta + 96) : 0.0f;
    }
};

// The span's sum-times-coefficient term: per position 4*kh + r (r < 4) and
// the lane's row, sum over chunks m of coef_m * (16384 S0 + 128 S1 + S2)_m,
// coef in the B bytes (chunks 8*kh .. 8*kh + 7).
__device__ __forceinline__ void digit_sums(const long (&ad)[2], long coef, double (&t)[4])
{
    v16i Dh = {}, Dl = {};
    Dh = __builtin_amdgcn_mfma_i32_32x32x16_i8(ad[0], coef, Dh, 0, 0, 0);
    Dl = __builtin_amdgcn_mfma_i32_32x32x16_i8(ad[1], coef, Dl, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r)
        t[r] = limb_combine(64 * Dh[r] + Dl[r], 64 * Dh[r + 4] + Dl[r + 4], 64 * Dh[r + 8] + Dl[r + 8]);
}

// Per format: a 256-column span of a row (SPAN bytes) is staged into an LDS
// row of STRIDE bytes as NP 16-byte pieces and NT tails of TB bytes, and
// span_dots() gives, for the lane's weight row and positions 4*kh + r, the
// span's dot of the weights with the positions' combined limb integers (the
// span's share of the matvec before the activation scale), refilling each A
// register through refill() once its MFMA has issued.
template <class F> struct Mma;

// Q6_K, 210 bytes: ql[128], qh[64], sc[16] (int8), d.  Chunk m = 8h + 2q + p
// holds elements 128h + 32q + 16p + l (l < 16) with scale sc[m]:
// |sc * (A x codes)| < 2^23 per chunk, sixteen chunks < 2^27.
template <> struct Mma<FmtQ6K> {
    static constexpr int SPAN = 210, STRIDE = 232, NP = 13, NT = 1, TB = 2;
    static constexpr bool DIGITS = true;
    __device__ static int gp(int k) { return 16 * k; }
    __device__ static int lp(int k) { return 16 * k; }
    __device__ static int gt(int) { return 208; }
    __device__ static int lt(int) { return 208; }
    __device__ static bool live_p(int, int) { return true; }
    __device__ static bool live_t(int, int) { return true; }
    template <class Refill, class Issue>
    __device__ static void span_dots(const uint8_t *rp, SpanA &A, int, int kh, float (&v)[4], const Refill &refill,
                                     const Issue &issue)
    {
        // The span's operand words, read once: ql of (h, q&1, p) and qh of (h, p).
        uint2 ql[8], qh[4];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            ql[i] = *reinterpret_cast<const uint2 *>(rp + 64 * (i >> 2) + 32 * ((i >> 1) & 1) + 16 * (i & 1) + 8 * kh);
#pragma unroll
        for (int i = 0; i < 4; ++i) qh[i] = *reinterpret_cast<const uint2 *>(rp + 128 + 32 * (i >> 1) + 16 * (i & 1) + 8 * kh);
        const uint2 s0 = *reinterpret_cast<const uint2 *>(rp + 192), s1 = *reinterpret_cast<const uint2 *>(rp + 200);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(rp + 208));
        issue();
        int I[12];
#pragma unroll
        for (int i = 0; i < 12; ++i) I[i] = 0;
#pragma unroll
        for (int m = 0; m < kSpanChunks; ++m) {
            // chunk m = 8h + 2q + p: elements 128h + 32q + 16p + l
            const int h = m >> 3, q = (m >> 1) & 3, p = m & 1;
            const uint2 lo = ql[4 * h + 2 * (q & 1) + p], hi = qh[2 * h + p];
            const int ns = 4 * (q >> 1), hs = 2 * q;
            const long b = pack8(((lo.x >> ns) & 0x0f0f0f0fu) | (((hi.x >> hs) & 0x03030303u) << 4),
                                 ((lo.y >> ns) & 0x0f0f0f0fu) | (((hi.y >> hs) & 0x03030303u) << 4));
            v16i D = {};
            D = __builtin_amdgcn_mfma_i32_32x32x16_i8(A.av[m], b, D, 0, 0, 0);
            refill(m);
            const int sc = (int)(int8_t)byte8(m < 8 ? s0 : s1, m & 7);
#pragma unroll
            for (int i = 0; i < 12; ++i) I[i] = mad24(sc, D[i], I[i]);
            pin12(I);
        }
        double ts[4];
        const uint2 sk = kh ? s1 : s0; // the int8 scales of chunks 8kh .. 8kh + 7
        digit_sums(A.ad, pack8(sk.x, sk.y), ts);
        refill(kSpanChunks);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = (float)((double)d * (limb_combine(I[r], I[r + 4], I[r + 8]) - 32.0 * ts[r]));
    }
};

// Q5_K, 176 bytes: d, dmin, 12 scale bytes, qh[32], qs[128].  Chunk m: group
// g = m/4, nibble half = (m/2)&1, l in 16(m&1) + [0, 16); sub-block m/2 (32
// columns, two chunks) has scale sc and min mn: |sc * D| < 2^22 per
// sub-block, eight < 2^25.
template <> struct Mma<FmtQ5K> {
    static constexpr int SPAN = 176, STRIDE = 184, NP = 11, NT = 0, TB = 2;
    static constexpr bool DIGITS = true;
    __device__ static int bytes(int) { return SPAN; }
    __device__ static int gp(int k) { return 16 * k; }
    __device__ static int lp(int k) { return 16 * k; }
    __device__ static int gt(int) { return 0; }
    __device__ static int lt(int) { return 0; }
    __device__ static bool live_p(int, int) { return true; }
    __device__ static bool live_t(int, int) { return true; }
    template <class Refill, class Issue>
    __device__ static void span_dots(const uint8_t *rp, SpanA &A, int, int kh, float (&v)[4], const Refill &refill,
                                     const Issue &issue)
    {
        FmtQ5K::Raw r;
        const uint2 a = *reinterpret_cast<const uint2 *>(rp), b = *reinterpret_cast<const uint2 *>(rp + 8);
        r.dd = a.x;
        r.s0 = a.y;
        r.s1 = b.x;
        r.s2 = b.y;
        // The span's operand words, read once: qs of (g, m&1) and qh of m&1.
        uint2 qs[8], qh[2];
#pragma unroll
        for (int i = 0; i < 8; ++i) qs[i] = *reinterpret_cast<const uint2 *>(rp + 48 + 32 * (i >> 1) + 16 * (i & 1) + 8 * kh);
#pragma unroll
        for (int i = 0; i < 2; ++i) qh[i] = *reinterpret_cast<const uint2 *>(rp + 16 + 16 * i + 8 * kh);
        issue();
        auto codes = [&](int m) {
            // chunk m: group g = m/4, nibble half = (m/2)&1, l in 16(m&1) + [0, 16)
            const int g = m >> 2, half = (m >> 1) & 1;
            const uint2 w = qs[2 * g + (m & 1)], h = qh[m & 1];
            const int ns = 4 * half, hs = 2 * g + half;
            return pack8(((w.x >> ns) & 0x0f0f0f0fu) | (((h.x >> hs) & 0x01010101u) << 4),
                         ((w.y >> ns) & 0x0f0f0f0fu) | (((h.y >> hs) & 0x01010101u) << 4));
        };
        int I[12];
#pragma unroll
        for (int i = 0; i < 12; ++i) I[i] = 0;
#pragma unroll
        for (int sb = 0; sb < kSpanChunks / 2; ++sb) {
            v16i D = {};
            D = __builtin_amdgcn_mfma_i32_32x32x16_i8(A.av[2 * sb], codes(2 * sb), D, 0, 0, 0);
            D = __builtin_amdgcn_mfma_i32_32x32x16_i8(A.av[2 * sb + 1], codes(2 * sb + 1), D, 0, 0, 0);
            refill(2 * sb);
            refill(2 * sb + 1);
            uint32_t sc, mn;
            FmtQ5K::scale_min(r, sb, sc, mn);
#pragma unroll
            for (int i = 0; i < 12; ++i) I[i] = mad24((int)sc, D[i], I[i]);
            pin12(I);
        }
        // the mins of chunks 8kh .. 8kh + 7: sub-blocks 4kh .. 4kh + 3, two chunks each
        uint32_t mb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) { // constant indices, then a select: no per-lane index into the scale words
            uint32_t sc0, mn0, sc1, mn1;
            FmtQ5K::scale_min(r, k, sc0, mn0);
            FmtQ5K::scale_min(r, 4 + k, sc1, mn1);
            mb[k] = (kh ? mn1 : mn0) * 0x0101u;
        }
        double ts[4];
        digit_sums(A.ad, pack8(mb[0] | (mb[1] << 16), mb[2] | (mb[3] << 16)), ts);
        refill(kSpanChunks);
        const double d = h2f((uint16_t)(r.dd & 0xffffu)), dmin = h2f((uint16_t)(r.dd >> 16));
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (float)(d * limb_combine(I[q], I[q + 4], I[q + 8]) - dmin * ts[q]);
    }
};

// Q2_K, 84 bytes: sc[16] (scale low nibble, min high nibble), qs[64], d,
// dmin.  Chunk m = 8N + 2j + s: codes (qs[32N + 16s + l] >> 2j) & 3, scale
// byte sc[m].  The scaled codes (<= 45) chain over the span on the matrix
// pipe (< 2^20 per limb).
template <> struct Mma<FmtQ2K> {
    static constexpr int SPAN = 84, STRIDE = 88, NP = 5, NT = 1, TB = 4;
    static constexpr bool DIGITS = true;
    __device__ static int bytes(int) { return SPAN; }
    __device__ static int gp(int k) { return 16 * k; }
    __device__ static int lp(int k) { return 16 * k; }
    __device__ static int gt(int) { return 80; }
    __device__ static int lt(int) { return 80; }
    __device__ static bool live_p(int, int) { return true; }
    __device__ static bool live_t(int, int) { return true; }
    template <class Refill, class Issue>
    __device__ static void span_dots(const uint8_t *rp, SpanA &A, int, int kh, float (&v)[4], const Refill &refill,
                                     const Issue &issue)
    {
        const uint2 s0 = *reinterpret_cast<const uint2 *>(rp), s1 = *reinterpret_cast<const uint2 *>(rp + 8);
        const uint32_t dd = *reinterpret_cast<const uint32_t *>(rp + 80);
        // The span's code words, read once: qs of (N, s); chunk 8N + 2j + s shifts them by 2j.
        uint2 qs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qs[i] = *reinterpret_cast<const uint2 *>(rp + 16 + 32 * (i >> 1) + 16 * (i & 1) + 8 * kh);
        issue();
        v16i Dq = {};
#pragma unroll
        for (int m = 0; m < kSpanChunks; ++m) {
            const int N = m >> 3, j = (m >> 1) & 3, sh = m & 1;
            const uint2 w = qs[2 * N + sh];
            const uint32_t sc = byte8(m < 8 ? s0 : s1, m & 7) & 15u;
            Dq = __builtin_amdgcn_mfma_i32_32x32x16_i8(
                A.av[m], pack8(((w.x >> (2 * j)) & 0x03030303u) * sc, ((w.y >> (2 * j)) & 0x03030303u) * sc), Dq, 0,
                0, 0);
            refill(m);
        }
        const uint2 sk = kh ? s1 : s0; // min nibbles of chunks 8kh .. 8kh + 7
        double ts[4];
        digit_sums(A.ad, pack8((sk.x >> 4) & 0x0f0f0f0fu, (sk.y >> 4) & 0x0f0f0f0fu), ts);
        refill(kSpanChunks);
        const double d = h2f((uint16_t)(dd & 0xffffu)), dmin = h2f((uint16_t)(dd >> 16));
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (float)(d * limb_combine(Dq[q], Dq[q + 4], Dq[q + 8]) - dmin * ts[q]);
    }
};

// Q8_0: a span is eight 34-byte blocks (d, 32 int8 codes).  The LDS row holds
// the 256 codes first (block b at 32b) and the eight d values at 256 + 2b, so
// every operand read is 8-byte aligned.  A row's last span may be partial.
// A block's two chunks chain in one accumulator; its d scales the limb sums
// in float.
template <> struct Mma<FmtQ8_0> {
    static constexpr int SPAN = 272, STRIDE = 280, NP = 16, NT = 8, TB = 2;
    static constexpr bool DIGITS = false;
    __device__ static int gp(int k) { return 34 * (k >> 1) + 2 + 16 * (k & 1); }
    __device__ static int lp(int k) { return 16 * k; }
    __device__ static int gt(int k) { return 34 * k; }
    __device__ static int lt(int k) { return 256 + 2 * k; }
    // nch chunks of the span are present: blocks below nch / 2
    __device__ static bool live_p(int k, int nch) { return (k >> 1) < (nch >> 1); }
    __device__ static bool live_t(int k, int nch) { return k < (nch >> 1); }
    template <class Refill, class Issue>
    __device__ static void span_dots(const uint8_t *rp, SpanA &A, int nch, int kh, float (&v)[4],
                                     const Refill &refill, const Issue &issue)
    {
        const uint2 d0 = *reinterpret_cast<const uint2 *>(rp + 256), d1 = *reinterpret_cast<const uint2 *>(rp + 264);
        float acc[12];
#pragma unroll
        for (int i = 0; i < 12; ++i) acc[i] = 0.0f;
        long cw[kSpanChunks]; // the span's codes, read once
#pragma unroll
        for (int m = 0; m < kSpanChunks; ++m) cw[m] = *reinterpret_cast<const long *>(rp + 16 * m + 8 * kh);
        issue();
#pragma unroll
        for (int b = 0; b < kSpanChunks / 2; ++b) {
            v16i D = {};
            D = __builtin_amdgcn_mfma_i32_32x32x16_i8(A.av[2 * b], cw[2 * b], D, 0, 0, 0);
            D = __builtin_amdgcn_mfma_i32_32x32x16_i8(A.av[2 * b + 1], cw[2 * b + 1], D, 0, 0, 0);
            refill(2 * b);
            refill(2 * b + 1);
            if (2 * b < nch) { // uniform
                const uint2 dv = b < 4 ? d0 : d1;
                const float db = h2f((uint16_t)(((b & 3) < 2 ? dv.x : dv.y) >> (16 * (b & 1))));
#pragma unroll
                for (int i = 0; i < 12; ++i) acc[i] = __builtin_fmaf((float)D[i], db, acc[i]);
            }
        }
        refill(kSpanChunks);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = __builtin_fmaf(acc[q], 16384.0f, __builtin_fmaf(acc[q + 4], 128.0f, acc[q + 8]));
    }
};

// Q8_0 rows as stored (the direct form's LDS rows): block b at 34b, its d
// then its 32 codes.  The codes of even blocks start 2 bytes past a dword
// boundary: their 8-byte operands are assembled from three dword reads by
// v_alignbyte; odd blocks' start on one.  The same products, in the same
// order, as Mma<FmtQ8_0>.
struct MmaQ8Raw {
    static constexpr int SPAN = 272, STRIDE = 280;
    static constexpr bool DIGITS = false;
    __device__ static int bytes(int nch) { return 17 * nch; } // nch / 2 blocks of 34 bytes
    template <class Refill, class Issue>
    __device__ static void span_dots(const uint8_t *rp, SpanA &A, int nch, int kh, float (&v)[4],
                                     const Refill &refill, const Issue &issue)
    {
        auto rd = [&](int off) { return *reinterpret_cast<const uint32_t *>(rp + off); }; // off % 4 == 0
        long cw[kSpanChunks];
        uint32_t dd[kSpanChunks / 2];
#pragma unroll
        for (int b = 0; b < kSpanChunks / 2; ++b) {
            const int base = 34 * b;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int o = base + 16 * p + 8 * kh; // the operand's bytes start at o + 2
                uint32_t lo, hi;
                if (b % 2 == 0) {
                    const uint32_t x0 = rd(o), x1 = rd(o + 4), x2 = rd(o + 8);
                    lo = __builtin_amdgcn_alignbyte(x1, x0, 2);
                    hi = __builtin_amdgcn_alignbyte(x2, x1, 2);
                } else {
                    lo = rd(o + 2);
                    hi = rd(o + 6);
                }
                cw[2 * b + p] = (long)(((uint64_t)hi << 32) | lo);
            }
            dd[b] = b % 2 == 0 ? rd(base) & 0xffffu : rd(base - 2) >> 16;
        }
        issue();
        float acc[12];
#pragma unroll
        for (int i = 0; i < 12; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int b = 0; b < kSpanChunks / 2; ++b) {
            v16i D = {};
            D = __builtin_amdgcn_mfma_i32_32x32x16_i8(A.av[2 * b], cw[2 * b], D, 0, 0, 0);
            D = __builtin_amdgcn_mfma_i32_32x32x16_i8(A.av[2 * b + 1], cw[2 * b + 1], D, 0, 0, 0);
            refill(2 * b);
            refill(2 * b + 1);
            if (2 * b < nch) { // uniform
                const float db = h2f((uint16_t)dd[b]);
#pragma unroll
                for (int i = 0; i < 12; ++i) acc[i] = __builtin_fmaf((float)D[i], db, acc[i]);
            }
        }
        refill(kSpanChunks);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = __builtin_fmaf(acc[q], 16384.0f, __builtin_fmaf(acc[q + 4], 128.0f, acc[q + 8]));
    }
};

template <class M> constexpr int mma_piece_iters() { return (32 * M::NP + EMU_WAVE - 1) / EMU_WAVE; }
template <class M> constexpr int mma_tail_iters() { return (32 * M::NT + EMU_WAVE - 1) / EMU_WAVE; }

// One span's weight pieces, in flight.
template <class M> struct SpanW {
    uint4 p[mma_piece_iters<M>()];
    uint32_t t[mma_tail_iters<M>() > 0 ? mma_tail_iters<M>() : 1];
};

enum { kMmaUp = 0, kMmaDown = 1 };

struct MmaArgs {
    MoeArgs a;
    LimbPlanes in;       // the input vectors: tokens (gate|up) or routes (down)
    int ks;        // wavefronts sharing a tile's spans (1, 2 or 4)
    int tiles;     // tiles per expert
    // gate|up with counters set: the routes' limb planes, written by the
    // last tile of each 256-column span to arrive (counters [expert slot]
    // [span], zero between launches)
    LimbPlanes out;
    uint32_t *counters;
};

// Global-memory views of the weight rows.  The rows are reached through
// the expert table or the layer's tensors; loading through a global pointer
// keeps the loads off the flat path (whose completions also count against
// the LDS counter, so every LDS wait would wait for the next span's rows).
typedef __attribute__((address_space(1))) const uint8_t gbyte;
struct __attribute__((packed)) Pk16 {
    uint32_t x, y, z, w;
};
struct __attribute__((packed)) Pk4 {
    uint32_t v;
};
struct __attribute__((packed)) Pk2 {
    uint16_t v;
};
__device__ __forceinline__ uint4 gld16(gbyte *p)
{
    const __attribute__((address_space(1))) Pk16 *q = (const __attribute__((address_space(1))) Pk16 *)p;
    return make_uint4(q->x, q->y, q->z, q->w);
}
__device__ __forceinline__ uint32_t gld4(gbyte *p) { return ((const __attribute__((address_space(1))) Pk4 *)p)->v; }
__device__ __forceinline__ uint32_t gld2(gbyte *p) { return ((const __attribute__((address_space(1))) Pk2 *)p)->v; }

// Expert e's row bases (wave-uniform): gate|up: its gate rows and up rows;
// down: its down rows (in lo).
template <int KIND> struct RowBases {
    gbyte *lo, *hi;
    size_t rb;
};
template <int KIND> __device__ __forceinline__ RowBases<KIND> row_bases(const MoeArgs &a, int e)
{
    RowBases<KIND> b;
    if (KIND == kMmaUp) {
        b.lo = (gbyte *)gate_row(a, e, 0);
        b.hi = (gbyte *)up_row(a, e, 0);
        b.rb = a.rb_in;
    } else {
        b.lo = b.hi = (gbyte *)down_row(a, e, 0);
        b.rb = a.rb_ff;
    }
    return b;
}

// Row rr (0..31) of tile `tile`: gate|up rows 16*tile + rr (gate) and
// 16*tile + rr - 16 (up); down rows 32*tile + rr (clamped to a valid row;
// rows past the matrix are never stored).
template <int KIND>
__device__ __forceinline__ gbyte *tile_row(const MoeArgs &a, const RowBases<KIND> &b, int tile, int rr)
{
    if (KIND == kMmaUp) return (rr < 16 ? b.lo : b.hi) + (size_t)(uint32_t)(16 * tile + (rr & 15)) * b.rb;
    const int r = 32 * tile + rr;
    return b.lo + (size_t)(uint32_t)(r < a.width ? r : a.width - 1) * b.rb;
}

template <class F, int KIND>
__device__ __forceinline__ void span_wload(const MoeArgs &a, const RowBases<KIND> &rbs, int C, int tile, int span,
                                           int lane, SpanW<Mma<F>> &sw)
{
    using M = Mma<F>;
    const int nch = C - kSpanChunks * span < kSpanChunks ? C - kSpanChunks * span : kSpanChunks;
    const size_t so = (size_t)span * M::SPAN;
#pragma unroll
    for (int i = 0; i < mma_piece_iters<M>(); ++i) {
        const int item = i * EMU_WAVE + lane;
        const int rr = item / M::NP, k = item % M::NP;
        if (item < 32 * M::NP && M::live_p(k, nch)) sw.p[i] = gld16(tile_row<KIND>(a, rbs, tile, rr) + so + M::gp(k));
    }
#pragma unroll
    for (int i = 0; i < mma_tail_iters<M>(); ++i) {
        const int item = i * EMU_WAVE + lane;
        const int rr = item / (M::NT > 0 ? M::NT : 1), k = item % (M::NT > 0 ? M::NT : 1);
        if (item < 32 * M::NT && M::live_t(k, nch)) {
            gbyte *src = tile_row<KIND>(a, rbs, tile, rr) + so + M::gt(k);
            sw.t[i] = M::TB == 4 ? gld4(src) : gld2(src);
        }
    }
}

template <class F>
__device__ __forceinline__ void span_stage(const SpanW<Mma<F>> &sw, uint8_t *stage, int lane, int nch)
{
    using M = Mma<F>;
#pragma unroll
    for (int i = 0; i < mma_piece_iters<M>(); ++i) {
        const int item = i * EMU_WAVE + lane;
        const int rr = item / M::NP, k = item % M::NP;
        if (item < 32 * M::NP && M::live_p(k, nch)) {
            uint8_t *d = stage + rr * M::STRIDE + M::lp(k);
            *reinterpret_cast<uint2 *>(d) = make_uint2(sw.p[i].x, sw.p[i].y);
            *reinterpret_cast<uint2 *>(d + 8) = make_uint2(sw.p[i].z, sw.p[i].w);
        }
    }
#pragma unroll
    for (int i = 0; i < mma_tail_iters<M>(); ++i) {
        const int item = i * EMU_WAVE + lane;
        const int rr = item / (M::NT > 0 ? M::NT : 1), k = item % (M::NT > 0 ? M::NT : 1);
        if (item < 32 * M::NT && M::live_t(k, nch)) {
            uint8_t *d = stage + rr * M::STRIDE + M::lt(k);
            if (M::TB == 4) *reinterpret_cast<uint32_t *>(d) = sw.t[i];
            else *reinterpret_cast<uint16_t *>(d) = (uint16_t)sw.t[i];
        }
    }
}

// One span of the tile's 32 rows straight into this wavefront's LDS rows:
// one instruction per row, lane l bringing the row's dword l (the rows are
// the layout span_stage writes; the rows tile_row names).  The row
// addresses are formed per call in scalar registers from wave-uniform bases
// (gate|up: the tile's first gate and up rows; down: its first row) behind
// an empty asm statement: left free, the compiler hoists all 32 out of the
// span loop into 64 vector registers.
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void gvoid;
template <class M, int KIND>
__device__ __forceinline__ void span_dma(const MoeArgs &a, const RowBases<KIND> &rbs, int tile, int span, int nbytes,
                                         int lane, uint8_t *stage)
{
    static_assert(M::SPAN % 4 == 0 && M::STRIDE % 4 == 0 && M::SPAN <= 8 * EMU_WAVE, "dword rows");
    const int W = nbytes / 4; // the span's bytes in the row (a multiple of 4)
    const uint64_t so = (uint64_t)span * M::SPAN;
    uint64_t b0, b1, rb = rbs.rb;
    int last = 31; // down: the last row inside the matrix, relative to the tile (rows past it read it again)
    if (KIND == kMmaUp) {
        b0 = (uint64_t)(rbs.lo + (size_t)(uint32_t)(16 * tile) * rbs.rb) + so;
        b1 = (uint64_t)(rbs.hi + (size_t)(uint32_t)(16 * tile) * rbs.rb) + so;
    } else {
        b0 = (uint64_t)(rbs.lo + (size_t)(uint32_t)(32 * tile) * rbs.rb) + so;
        b1 = b0;
        last = a.width - 1 - 32 * tile; // tile < ceil(width / 32): last >= 0
    }
    auto sgpr = [](uint64_t v) {
        return (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v) |
               ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32)) << 32);
    };
    b0 = sgpr(b0);
    b1 = sgpr(b1);
    rb = sgpr(rb);
    last = __builtin_amdgcn_readfirstlane(last);
    asm volatile("" : "+s"(b0), "+s"(b1), "+s"(rb), "+s"(last));
#pragma unroll
    for (int rr = 0; rr < 32; ++rr) {
        // gate|up: gate row rr or up row rr - 16; down: row min(rr, last) (0 <= last)
        const int r = KIND == kMmaUp ? (rr & 15) : (rr < last ? rr : last);
        const uint64_t row = (KIND == kMmaUp && rr >= 16 ? b1 : b0) + (uint64_t)(uint32_t)r * rb;
        if (lane < W)
            __builtin_amdgcn_global_load_lds((gvoid *)(row + 4 * (uint32_t)lane), (lds_void *)(stage + rr * M::STRIDE),
                                             4, 0, 0);
        if (M::SPAN > 4 * EMU_WAVE && lane + EMU_WAVE < W) // rows of more than 64 dwords: the rest
            __builtin_amdgcn_global_load_lds((gvoid *)(row + 4 * (uint32_t)(lane + EMU_WAVE)),
                                             (lds_void *)(stage + rr * M::STRIDE + 4 * EMU_WAVE), 4, 0, 0);
    }
}

// The span arithmetic of each form: the direct form reads Q8_0 rows as stored.
enum { kFormLoop = 0, kFormOne = 1, kFormDirect = 2 };
template <class F, int FORM> struct MmaSel {
    using type = Mma<F>;
};
template <> struct MmaSel<FmtQ8_0, kFormDirect> {
    using type = MmaQ8Raw;
};


// The routed position p's vector: the token (gate|up) or the route (down).
template <int KIND> __device__ __forceinline__ int position_vec(const MoeArgs &a, const int (&slot)[kMaxTok], int p)
{
    int v = 0;
#pragma unroll
    for (int t = 0; t < kMaxTok; ++t) v = t == p ? slot[t] : v;
    return KIND == kMmaUp ? v / a.k : v;
}

template <class F, int KIND, int ACT, int FORM>
__global__ __launch_bounds__(kThreads, FORM == kFormLoop ? 2 : 3) void moe_mma_kernel(MmaArgs g)
{
    using M = typename MmaSel<F, FORM>::type;
    const MoeArgs &a = g.a;
    extern __shared__ __align__(16) uint8_t smem[];
    const int C = g.in.C, ns = g.in.ns, ks = g.ks;
    float *red = reinterpret_cast<float *>(smem); // [kWaves][8][32]
    const int tid = threadIdx.x, lane = tid & (EMU_WAVE - 1);
    // wave-uniform (the direct form's row addresses are scalar)
    const int w = FORM == kFormDirect ? __builtin_amdgcn_readfirstlane(tid / EMU_WAVE) : tid / EMU_WAVE;
    float *wsc = red + kWaves * kMaxTok * 32 + w * kMaxTok; // this wavefront's positions' span scales
    uint8_t *stage = reinterpret_cast<uint8_t *>(red + kWaves * kMaxTok * 32 + kWaves * kMaxTok) + w * 32 * M::STRIDE;
    // Grid: x = tile group, fastest, so that consecutive workgroups -- which
    // the dispatcher deals round-robin to the XCDs -- are one expert's tiles
    // and every routed expert's work spreads over all XCDs; y = the expert's
    // place among the routed experts.
    int e = 0, cnt = 0, slot[kMaxTok];
    if (!list_entry(a.ids, a.n_tok * a.k, a.n_experts, (int)blockIdx.y, e, cnt, slot)) return; // uniform
    const int tl = w / ks, kp = w % ks;
    const int tile_raw = blockIdx.x * (kWaves / ks) + tl;
    const int tile = tile_raw < g.tiles ? tile_raw : g.tiles - 1;
    const int s0 = kp * ns / ks, s1 = FORM == kFormOne ? s0 + 1 : (kp + 1) * ns / ks;
    // The first span's rows go out first: they do not depend on the routes.
    const RowBases<KIND> rbs = row_bases<KIND>(a, e);
    SpanW<Mma<F>> sw; // the register forms' rows in flight
    if (s0 < s1) {
        if constexpr (FORM == kFormDirect)
            span_dma<M, KIND>(a, rbs, tile, s0, M::bytes(C - kSpanChunks * s0 < kSpanChunks ? C - kSpanChunks * s0 : kSpanChunks), lane, stage);
        else span_wload<F, KIND>(a, rbs, C, tile, s0, lane, sw);
    }
    const int j = lane & 31, kh = lane >> 5;
    ASource src;
    src.live = j < 24 && (j & 7) < cnt;
    src.pos = lane < kMaxTok && lane < cnt; // lane p reads position p's scales
    src.C = C;
    src.ns = ns;
    const int myvec = position_vec<KIND>(a, slot, j & 7);
    src.q = g.in.q + (size_t)myvec * C * kChunkBytes + 16 * (j >> 3) + 8 * kh;
    src.meta = g.in.dg + (size_t)myvec * ns * kSpanMeta;
    src.dg = src.meta + 16 * (j >> 3) + 8 * kh;
    SpanA A;
    if (s0 < s1) {
#pragma unroll
        for (int m = 0; m < kSpanChunks; ++m) A.av[m] = src.chunk(s0, m);
        A.ad[0] = M::DIGITS ? src.digit(s0, 0) : 0;
        A.ad[1] = M::DIGITS ? src.digit(s0, 1) : 0;
        A.sc = src.scale(s0);
    }
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = s0; s < s1; ++s) {
        const int nch = C - kSpanChunks * s < kSpanChunks ? C - kSpanChunks * s : kSpanChunks;
        if constexpr (FORM == kFormDirect) {
            __builtin_amdgcn_s_waitcnt(0); // the span's rows are in LDS, its A operands in registers
        } else {
            span_stage<F>(sw, stage, lane, nch);
            if (FORM == kFormLoop && s + 1 < s1) span_wload<F, KIND>(a, rbs, C, tile, s + 1, lane, sw); // in flight
        }
        __builtin_amdgcn_wave_barrier(); // LDS accesses of one wavefront complete in order
        const bool more = FORM != kFormOne && s + 1 < s1;
        // The next span's A operands go into each register as soon as its
        // MFMA has issued (lanes outside the positions keep their zeros).
        const int nchn = more ? (C - kSpanChunks * (s + 1) < kSpanChunks ? C - kSpanChunks * (s + 1) : kSpanChunks) : 0;
        const uint8_t *an = src.q + (size_t)kSpanChunks * (s + 1) * kChunkBytes;
        const uint8_t *dn = src.dg + (size_t)(s + 1) * kSpanMeta;
        auto refill = [&](int m) {
            if (m < kSpanChunks) {
                if (m >= nchn) A.av[m] = 0; // uniform: no next span, or past its columns
                else if (src.live) A.av[m] = *reinterpret_cast<const long *>(an + m * kChunkBytes);
            } else if (M::DIGITS && more && src.live) {
                A.ad[0] = *reinterpret_cast<const long *>(dn);
                A.ad[1] = *reinterpret_cast<const long *>(dn + 48);
            }
        };
        if (lane < kMaxTok) wsc[lane] = A.sc; // positions past the count: 0
        if (more) A.sc = src.scale(s + 1);
        // Direct form: once the span's operand words are in registers (the
        // LDS reads complete: lgkmcnt 0), the next span's rows replace them.
        auto issue = [&]() {
            if constexpr (FORM == kFormDirect) {
                if (more) {
                    __builtin_amdgcn_s_waitcnt(0xc07f);
                    span_dma<M, KIND>(a, rbs, tile, s + 1, M::bytes(nchn), lane, stage);
                }
            }
        };
        float v[4];
        M::span_dots(stage + j * M::STRIDE, A, nch, kh, v, refill, issue);
        const float4 s4 = *reinterpret_cast<const float4 *>(wsc + 4 * kh);
        acc[0] = __builtin_fmaf(v[0], s4.x, acc[0]);
        acc[1] = __builtin_fmaf(v[1], s4.y, acc[1]);
        acc[2] = __builtin_fmaf(v[2], s4.z, acc[2]);
        acc[3] = __builtin_fmaf(v[3], s4.w, acc[3]);
        __builtin_amdgcn_wave_barrier();
    }
    // The tile's span shares meet in LDS, added in share order.
    float v[4] = {acc[0], acc[1], acc[2], acc[3]};
    if (ks > 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(w * kMaxTok + 4 * kh + r) * 32 + j] = acc[r];
        __syncthreads();
        if (kp == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float sum = red[(w * kMaxTok + 4 * kh + r) * 32 + j];
                for (int k = 1; k < ks; ++k) sum += red[((w + k) * kMaxTok + 4 * kh + r) * 32 + j];
                v[r] = sum;
            }
        }
    }
    if (kp != 0 || tile_raw >= g.tiles) return; // uniform per wavefront
    if (KIND == kMmaDown) {
        const int row = 32 * tile + j;
        const float scale = a.down_scale ? a.down_scale[e] : 1.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = 4 * kh + r;
            float o = v[r];
            if (a.down_scale) o = __fmul_rn(o, scale); // gemma_smoke.rs:129-137
            if (p < cnt && row < a.width) a.contrib[(size_t)position_vec<KIND>(a, slot, p) * a.width + row] = o;
        }
        return;
    }
    // gate|up: lanes j < 16 hold gate row 16*tile + j, lanes j + 16 its up row.
    const bool handoff = g.counters != nullptr;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float u = __shfl_xor(v[r], 16, EMU_WAVE);
        const int p = 4 * kh + r;
        if (j < 16 && p < cnt) {
            float *dst = a.act_buf + (size_t)position_vec<kMmaDown>(a, slot, p) * a.ff + 16 * tile + j;
            const float o = activate<ACT>(v[r], u);
            if (handoff) __hip_atomic_store(dst, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else *dst = o;
        }
    }
    if (!handoff) return;
    // The routes' limb planes, in place of a launch of the limb kernel: the
    // activations went to the device-coherent level, every store completes
    // before the span's arrival counter moves, and the last of the span's
    // tiles to arrive reads the span back (agent-scope loads) and splits it
    // for each position, as the limb kernel would, then resets the counter.
    __builtin_amdgcn_s_waitcnt(0);
    const int span = tile / kSpanChunks;
    const int need = g.tiles - kSpanChunks * span < kSpanChunks ? g.tiles - kSpanChunks * span : kSpanChunks;
    uint32_t *counter = g.counters + (size_t)blockIdx.y * kMmaMaxSpans + span;
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = (uint32_t)__shfl((int)old, 0, EMU_WAVE);
    if ((int)old != need - 1) return; // uniform
    if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int col = kSpanChunks * 16 * span + 4 * lane;
    const bool live = col < a.ff;
    float4 xv[kMaxTok];
#pragma unroll
    for (int p = 0; p < kMaxTok; ++p) {
        xv[p] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (p < cnt && live) {
            const float *src = a.act_buf + (size_t)position_vec<kMmaDown>(a, slot, p) * a.ff + col;
            xv[p].x = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            xv[p].y = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            xv[p].z = __hip_atomic_load(src + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            xv[p].w = __hip_atomic_load(src + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
#pragma unroll
    for (int p = 0; p < kMaxTok; ++p)
        if (p < cnt) emu_span_limbs_wave(xv[p], live, position_vec<kMmaDown>(a, slot, p), span, g.out); // uniform
}

// Wavefronts per tile.  A matrix of 1, 2 or 4 spans gets a share per span
// (the one-span form, whose wavefronts hold no prefetch: four workgroups a
// CU).  Otherwise enough shares for about `budget` wavefronts
// over the experts eight tokens can route to -- 16384 for gate|up, 2048 for
// down -- as measured in the decode steps (with every layer's experts coming
// from HBM, gate|up gains from more rows in flight; the downs lose with more
// shares).  The shares depend on the layer's shape only, not on the token
// count, so that a token's sums are added in the same order whichever tokens
// share the call.
int mma_shares(const MoeArgs &a, int tiles, int spans, int budget)
{
    if (spans <= kWaves && (spans & (spans - 1)) == 0) return spans;
    int ks = 1;
    const int active = kMaxTok * a.k < a.n_experts ? kMaxTok * a.k : a.n_experts;
    while (ks < kWaves && 2 * ks <= spans && active * tiles * ks < budget) ks *= 2;
    return ks;
}

template <class F, int KIND, int ACT>
int launch_mma(emu_ctx *ctx, const MoeArgs &a, const LimbPlanes &in, const LimbPlanes &out = LimbPlanes{},
               uint32_t *counters = nullptr)
{
    using M = Mma<F>;
    MmaArgs g;
    g.a = a;
    g.in = in;
    g.out = out;
    g.counters = KIND == kMmaUp ? counters : nullptr;
    g.tiles = KIND == kMmaUp ? a.ff / 16 : (a.width + 31) / 32;
    g.ks = mma_shares(a, g.tiles, in.ns, KIND == kMmaUp ? 16384 : 2048);
    const int tpw = kWaves / g.ks;
    const size_t lds = kWaves * kMaxTok * 32 * 4 + kWaves * kMaxTok * 4 + kWaves * 32 * M::STRIDE;
    const int routed = a.n_tok * a.k < a.n_experts ? a.n_tok * a.k : a.n_experts; // grid rows: at most this many experts
    const dim3 grid((g.tiles + tpw - 1) / tpw, routed);
    // The direct form for device-resident rows whose spans start and end on
    // 4-byte boundaries (an expert table may point some experts at pinned
    // host memory; those launches keep the register form).  Q5_K and Q2_K
    // spans are 176 and 84 bytes; Q8_0 spans are 272 bytes, the last one
    // (C % 16) / 2 blocks of 34 bytes.
    constexpr bool direct = std::is_same<F, FmtQ5K>::value || std::is_same<F, FmtQ2K>::value ||
                            std::is_same<F, FmtQ8_0>::value;
    const size_t rb = KIND == kMmaUp ? a.rb_in : a.rb_ff;
    const uintptr_t p0 = (uintptr_t)(KIND == kMmaUp ? a.gate : a.down), p1 = (uintptr_t)(KIND == kMmaUp ? a.up : a.down);
    const bool aligned = rb % 4 == 0 && p0 % 4 == 0 && p1 % 4 == 0 &&
                         (!std::is_same<F, FmtQ8_0>::value || (in.C % kSpanChunks) % 4 == 0);
    if (g.ks == in.ns)
        hipLaunchKernelGGL((moe_mma_kernel<F, KIND, ACT, kFormOne>), grid, dim3(kThreads), lds, ctx->stream, g);
    else if (direct && !a.table && aligned)
        hipLaunchKernelGGL((moe_mma_kernel<F, KIND, ACT, direct ? kFormDirect : kFormLoop>), grid, dim3(kThreads),
                           lds, ctx->stream, g);
    else
        hipLaunchKernelGGL((moe_mma_kernel<F, KIND, ACT, kFormLoop>), grid, dim3(kThreads), lds, ctx->stream, g);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

template <class F>
int launch_mma_up(emu_ctx *ctx, const MoeArgs &a, const LimbPlanes &in, const LimbPlanes &out, uint32_t *counters)
{
    if (a.act == EMU_ACT_GELU_TANH) return launch_mma<F, kMmaUp, EMU_ACT_GELU_TANH>(ctx, a, in, out, counters);
    return launch_mma<F, kMmaUp, EMU_ACT_SILU>(ctx, a, in, out, counters);
}

int launch_limbs(emu_ctx *ctx, const float *x, int n_vec, int cols, const LimbPlanes &L)
{
    const int total = n_vec * L.ns * kSpanChunks;
    hipLaunchKernelGGL(moe_limbs_kernel, dim3((total + kThreads - 1) / kThreads), dim3(kThreads), 0, ctx->stream, x,
                       n_vec, cols, L);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

} // namespace

extern "C" size_t emu_moe_workspace_bytes(uint32_t n_tok, uint32_t k, uint32_t width, uint32_t ff)
{
    const size_t slots = (size_t)n_tok * k;
    return align256(sizeof(float) * slots * ff) + align256(sizeof(float) * slots * width) +
           align256(limb_plane_bytes(n_tok, (int)((width + 15) / 16))) +
           align256(limb_plane_bytes(slots, (int)((ff + 15) / 16)));
}

namespace {

// The matrix-core form finds a workgroup's expert in a 256-bit mask of the
// routed experts, so it takes layers of up to 256 experts; wider layers, and
// calls that ask for f32 activations, take the vector form.
constexpr uint32_t kMmaMaxExperts = 256;

bool mma_form(const emu_moe_desc *d)
{
    return !(d->flags & EMU_MOE_F32_ACT) && d->n_experts <= kMmaMaxExperts && d->width <= kMmaMaxCols && d->ff <= kMmaMaxCols && d->width % 16 == 0 && d->ff % 16 == 0;
}

// The workspace: activations, contributions, the tokens' limb planes, the
// routes' limb planes.
uint8_t *x_plane_base(void *ws, size_t slots, uint32_t width, uint32_t ff)
{
    return static_cast<uint8_t *>(ws) + align256(sizeof(float) * slots * ff) + align256(sizeof(float) * slots * width);
}

int moe_ffn(emu_ctx *ctx, const emu_moe_desc *d, const float *d_x, uint32_t n_tok, const int32_t *d_ids,
            const float *d_weights, void *d_workspace, size_t workspace_bytes, float *d_out, float *d_resid,
            float resid_scale, bool combine = true, const uint8_t *const *d_table = nullptr,
            bool x_planes_ready = false, uint32_t *span_counters = nullptr)
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
    if (mma_form(d)) {
        // matrix-core form: the tokens' limb planes (unless the caller wrote
        // them), gate|up into the activations, the routes' limb planes (by
        // the gate|up launch when the caller keeps span counters), down into
        // the contributions
        const int c_in = (int)(d->width / 16), c_ff = (int)(d->ff / 16);
        const size_t slots = (size_t)n_tok * d->k;
        uint8_t *xp = x_plane_base(d_workspace, slots, d->width, d->ff);
        uint8_t *fp = xp + align256(limb_plane_bytes(n_tok, c_in));
        const LimbPlanes lx = limb_planes(xp, n_tok, c_in), lf = limb_planes(fp, slots, c_ff);
        if (!x_planes_ready && (st = launch_limbs(ctx, d_x, (int)n_tok, (int)d->width, lx)) != EMU_OK) return st;
        switch (d->enc_gate_up) {
        case EMU_ENC_Q6_K: st = launch_mma_up<FmtQ6K>(ctx, a, lx, lf, span_counters); break;
        case EMU_ENC_Q8_0: st = launch_mma_up<FmtQ8_0>(ctx, a, lx, lf, span_counters); break;
        case EMU_ENC_Q5_K: st = launch_mma_up<FmtQ5K>(ctx, a, lx, lf, span_counters); break;
        case EMU_ENC_Q2_K: st = launch_mma_up<FmtQ2K>(ctx, a, lx, lf, span_counters); break;
        default: return EMU_E_UNSUPPORTED;
        }
        if (st != EMU_OK) return st;
        if (!span_counters && (st = launch_limbs(ctx, a.act_buf, (int)slots, (int)d->ff, lf)) != EMU_OK) return st;
        switch (d->enc_down) {
        case EMU_ENC_Q6_K: st = launch_mma<FmtQ6K, kMmaDown, 0>(ctx, a, lf); break;
        case EMU_ENC_Q8_0: st = launch_mma<FmtQ8_0, kMmaDown, 0>(ctx, a, lf); break;
        case EMU_ENC_Q5_K: st = launch_mma<FmtQ5K, kMmaDown, 0>(ctx, a, lf); break;
        case EMU_ENC_Q2_K: st = launch_mma<FmtQ2K, kMmaDown, 0>(ctx, a, lf); break;
        default: return EMU_E_UNSUPPORTED;
        }
        if (st != EMU_OK) return st;
    } else {
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
    }
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
                      float scale, bool combine, bool x_planes_ready, uint32_t *span_counters,
                      const uint8_t *const *d_table)
{
    if (!d_state) return EMU_E_ARG;
    return moe_ffn(ctx, d, d_x, n_tok, d_ids, d_weights, d_workspace, workspace_bytes, nullptr, d_state, scale,
                   combine, d_table, x_planes_ready && mma_form(d), span_counters);
}

size_t emu_moe_span_counters() { return (size_t)kMaxTok * 8 * kMmaMaxSpans; }

bool emu_moe_mma_form(const emu_moe_desc *d) { return d && mma_form(d); }

EmuLimbPlanes emu_moe_x_planes(void *d_workspace, uint32_t n_tok, uint32_t k, uint32_t width, uint32_t ff)
{
    return limb_planes(x_plane_base(d_workspace, (size_t)n_tok * k, width, ff), n_tok, (int)((width + 15) / 16));
}

const float *emu_moe_contrib(const void *d_workspace, uint32_t n_tok, uint32_t k, uint32_t ff)
{
    return reinterpret_cast<const float *>(static_cast<const uint8_t *>(d_workspace) +
                                           align256(sizeof(float) * (size_t)n_tok * k * ff));
}
