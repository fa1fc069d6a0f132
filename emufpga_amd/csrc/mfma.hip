// mfma.hip -- quantized matvec for 2..8 tokens on the int8 matrix cores.
//
// The activations are carried as in the batch-1 limb kernel: per token and
// 16-column sub-block, x ~= s * (16384*L0 + 128*L1 + L2) with |L| <= 64 and
// s a power of two (exact to 2^-20 of the sub-block's largest |x|).  A Q6_K
// sub-block is 16 columns, which is exactly the K of v_mfma_i32_32x32x16_i8,
// so one instruction forms every (token, limb) x (weight row) integer dot of
// one sub-block for 32 weight rows:
//
//     A (32 x 16, int8) = the limbs: M row i = 8 * limb + token (rows 24..31 zero)
//     B (16 x 32, int8) = the weight codes minus 32 of 32 consecutive rows
//     D (32 x 32, int32): lane l, register r holds row i = 8*(r/4) + 4*(l/32) + r%4
//                         of weight row l % 32, i.e. limb r/4 of token 4*(l/32) + r%4
//
// so each lane finds the three limb sums of its (row, token) pairs in its own
// registers and combines them exactly, t = (D0 << 14) + (D1 << 7) + D2, before
// the one float step per sub-block, acc = fma(t, (sc * d) * s, acc), the same
// step as the batch-1 kernel.
//
// Work split: a workgroup owns 32 weight rows of one matrix and a 1024-column
// slice (four 256-column blocks, one per wavefront); the four wavefronts'
// sums meet in LDS in a fixed order and the slice's partial sum is written to
// a workspace.  A finishing pass adds the slices' partials in slice order and
// applies the epilogue (residual accumulate, SwiGLU of a gate/up pair, greedy
// selection keys).  Everything is deterministic.
//
// Kernels:
//   mfma_link_kernel   the producing matvec's partial sums (or a given x) ->
//                      its epilogue (residual add, SwiGLU) -> optional RMS
//                      norm -> the next matvec's A operands and scales
//   qmv_mfma_kernel    A operands x weight codes -> per-slice partial sums
//   mfma_finish_kernel partial sums -> y (residual accumulate, SwiGLU, keys)
// A decode step chains them as link, matvec, link, matvec, ... so each
// matvec costs one small kernel besides its own.
#include "internal.hpp"

#include <math.h>
#include <stdlib.h>

namespace {

typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ void ld8f(const float *p, float (&v)[8])
{
    const float4 a = *reinterpret_cast<const float4 *>(p);
    const float4 b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

constexpr int kMaxTok = 8;          // tokens per tile (A rows 8 * limb + token)
constexpr int kTileRows = 32;       // weight rows per tile (MFMA N)
constexpr int kWaves = 4;           // wavefronts per workgroup, one 256-column block each
constexpr int kSlice = kWaves * 256; // columns per workgroup
constexpr int kSbBytes = 2 * 24 * 8; // A-operand bytes per 16-column sub-block
constexpr int kRowStride = 232;      // LDS bytes per staged weight row: 58 dwords, so 32 rows hit distinct banks
constexpr int kFinishThreads = 256;

// One token's activation vector, finished from the producing matvec's
// partial sums (or taken as given) and turned into the next matvec's A
// operands.  Modes: the producing matvec's epilogue.
enum LinkMode { kLinkInput = 0, kLinkResid = 1, kLinkSwiglu = 2, kLinkPlain = 3 };

struct LinkArgs {
    const float *part; // [nks][nmat][kMaxTok][cols] partial sums, or null (kLinkInput)
    int nks, nmat, mode;
    float *h;       // kLinkResid: residual stream, updated in place; kLinkPlain: output
    const float *x; // kLinkInput: the activations
    int cols, n_tok;
    const float *gain; // RMS gain of the next matvec's input, or null
    float eps;
    uint8_t *xa; // A operands (null: none wanted)
    float *xs;
    // kLinkInput, optional: a MoE layer's expert sum joins x first (h gets
    // the result): x + sum * m_scale, the sum over the token's routes in
    // expert-id order from +0.0 (the combining pass's arithmetic).
    const float *m_contrib;
    const int32_t *m_ids;
    const float *m_wts;
    int m_k, m_experts;
    float m_scale;
    int m_sorted; // the routes come in ascending expert id (no reordering)
    // kLinkInput, optional, before the expert sum: a dense FFN's down
    // projection (part, d_nks slices of one matrix) joins x as x + v * d_scale.
    const float *d_part;
    int d_nks;
    float d_scale;
    int act; // kLinkSwiglu: EMU_ACT_SILU or EMU_ACT_GELU_TANH
    int span; // one limb scale per 256-column span (xs: [span][8]) instead of per sub-block
    // With gain, optional: the RMS factor is left to the consuming matvec.
    // The limbs are of x * gain; each (one-wavefront) workgroup writes the
    // sum of squares of its columns to ssp[token * kSsGroups + blockIdx.y].
    float *ssp;
};

// A-operand layout: sub-block sb, half kh (columns 8kh..8kh+7 of the
// sub-block), limb, token -> 8 bytes at xa + sb*kSbBytes + (kh*24 + 8*limb + token)*8.
// Thread pair (2m, 2m+1) holds the two 8-column halves of one sub-block;
// a thread owns up to kLinkPairs such 8-column pieces.  With an RMS norm one
// workgroup covers a token's row (the norm needs its sum of squares);
// without one, gridDim.y workgroups share it.
constexpr int kMaxSlices = 12; // input columns / slice width, at most

// Sum of n (<= MAXS) slices' 8 partial sums, in slice order: slice_load
// issues the loads (slices past n read slice 0 and are dropped), slice_add
// adds them.  Every load of a column pair goes out before its first add, so
// a pair costs one memory round trip.
template <int MAXS>
__device__ __forceinline__ void slice_load(const float *p, size_t stride, int n, float (&q)[MAXS][8])
{
#pragma unroll
    for (int s = 0; s < MAXS; ++s) ld8f(p + (s < n ? s : 0) * stride, q[s]);
}
template <int MAXS> __device__ __forceinline__ void slice_add(const float (&q)[MAXS][8], int n, float (&v)[8])
{
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = q[0][e];
#pragma unroll
    for (int s = 1; s < MAXS; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = s < n ? v[e] + q[s][e] : v[e];
}

constexpr int kLinkThreads = 512;
constexpr int kLinkPairs = 3; // columns per token up to 8 * kLinkThreads * kLinkPairs = 12288
// Without a norm nothing spans the row, so the link runs as many small
// workgroups (one 8-column piece per thread): the partial sums it reads are
// spread over the CUs instead of queueing at a few.
constexpr int kLinkSmall = 64;
constexpr int kSsGroups = kLinkThreads * kLinkPairs / kLinkSmall; // small workgroups per token, at most
constexpr size_t kSsBytes = (size_t)kMaxTok * kSsGroups * sizeof(float);
constexpr size_t kSsRegion = (kSsBytes + 255) & ~(size_t)255; // just ahead of the A operands

template <int MAXS, int MODE, int TH>
__global__ __launch_bounds__(TH) void mfma_link_kernel(LinkArgs a)
{
    const int t = blockIdx.x, tid = threadIdx.x;
    const int npairs = a.cols / 8;
    float v[kLinkPairs][8], gn[kLinkPairs][8];
    float ss = 0.0f;
    // The gain goes out with the first loads (it does not depend on them).
    if (a.gain && a.xa) {
#pragma unroll
        for (int k = 0; k < kLinkPairs; ++k) {
            const int p = (blockIdx.y + k * gridDim.y) * TH + tid;
            if (p < npairs) ld8f(a.gain + 8 * p, gn[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < kLinkPairs; ++k) {
        const int p = (blockIdx.y + k * gridDim.y) * TH + tid;
        if (p >= npairs) break;
        const int c0 = 8 * p;
        if constexpr (MODE == kLinkInput) {
            // Every load first: x, the dense FFN's slices, and (routes in
            // ascending id) the routes' ids, weights and contributions, whose
            // addresses depend on no load.
            float dq[MAXS][8], cv[8][8], w[8];
            int order[8], ids[8], n = 0;
            ld8f(a.x + (size_t)t * a.cols + c0, v[k]);
            if (a.d_part) slice_load<MAXS>(a.d_part + (size_t)t * a.cols + c0, (size_t)kMaxTok * a.cols, a.d_nks, dq);
            if (a.m_contrib) {
                if (a.m_sorted) {
                    const int32_t *ip = a.m_ids + t * a.m_k;
                    const float *wp = a.m_wts + t * a.m_k;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const bool in = i < a.m_k;
                        ids[i] = in ? ip[i] : -1;
                        order[i] = in ? i : 0;
                        w[i] = in ? wp[i] : 0.0f;
                    }
                } else { // the order needs the ids first: a second round trip
                    n = emu_route_order(a.m_ids + t * a.m_k, a.m_wts + t * a.m_k, a.m_k, a.m_experts, order, w);
                }
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    ld8f(a.m_contrib + ((size_t)t * a.m_k + order[i]) * a.cols + c0, cv[i]); // slot 0 past n
            }
            __builtin_amdgcn_sched_barrier(0);
            if (a.d_part) {
                float dv[8];
                slice_add<MAXS>(dq, a.d_nks, dv);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[k][e] = emu_resid_add(v[k][e], dv[e], a.d_scale);
            }
            if (a.d_part && !a.m_contrib) {
                float *hp = a.h + (size_t)t * a.cols + c0;
                *reinterpret_cast<float4 *>(hp) = make_float4(v[k][0], v[k][1], v[k][2], v[k][3]);
                *reinterpret_cast<float4 *>(hp + 4) = make_float4(v[k][4], v[k][5], v[k][6], v[k][7]);
            }
            if (a.m_contrib) {
                if (a.m_sorted) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) // ascending: the valid ones lead
                        n += i < a.m_k && ids[i] >= 0 && ids[i] < a.m_experts ? 1 : 0;
                }
                float *hp = a.h + (size_t)t * a.cols + c0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float sum = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (i < n) sum = __fadd_rn(sum, __fmul_rn(cv[i][e], w[i]));
                    v[k][e] = emu_resid_add(v[k][e], sum, a.m_scale);
                }
                *reinterpret_cast<float4 *>(hp) = make_float4(v[k][0], v[k][1], v[k][2], v[k][3]);
                *reinterpret_cast<float4 *>(hp + 4) = make_float4(v[k][4], v[k][5], v[k][6], v[k][7]);
            }
        } else {
            // Slices added in slice order (the finishing pass's order); the
            // up slices and the residual go out with the first slices' loads.
            const size_t stride = (size_t)a.nmat * kMaxTok * a.cols;
            const float *pp = a.part + (size_t)t * a.cols + c0;
            float *hp = a.h + (size_t)t * a.cols + c0;
            float q[MAXS][8], qu[MAXS][8], hv[8];
            (void)qu;
            (void)hv;
            slice_load<MAXS>(pp, stride, a.nks, q);
            if constexpr (MODE == kLinkSwiglu) slice_load<MAXS>(pp + (size_t)kMaxTok * a.cols, stride, a.nks, qu);
            if constexpr (MODE == kLinkResid) ld8f(hp, hv);
            __builtin_amdgcn_sched_barrier(0);
            slice_add<MAXS>(q, a.nks, v[k]);
            if constexpr (MODE == kLinkSwiglu) {
                float u[8];
                slice_add<MAXS>(qu, a.nks, u);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[k][e] = emu_glu(v[k][e], u[e], a.act);
            }
            if constexpr (MODE == kLinkResid || MODE == kLinkPlain) {
                if constexpr (MODE == kLinkResid) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[k][e] = hv[e] + v[k][e];
                }
                *reinterpret_cast<float4 *>(hp) = make_float4(v[k][0], v[k][1], v[k][2], v[k][3]);
                *reinterpret_cast<float4 *>(hp + 4) = make_float4(v[k][4], v[k][5], v[k][6], v[k][7]);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[k][e], v[k][e], ss);
    }
    if (!a.xa) return; // uniform
    float scale = 1.0f;
    if (a.gain && a.ssp) { // the factor comes later: this workgroup's share of the sum of squares
        ss = wave_sum(ss);
        if (tid == 0) a.ssp[t * kSsGroups + blockIdx.y] = ss;
    } else if (a.gain) {
        __shared__ float red[TH / EMU_WAVE];
        ss = wave_sum(ss);
        if ((tid & (EMU_WAVE - 1)) == 0) red[tid / EMU_WAVE] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int k = 0; k < TH / EMU_WAVE; ++k) tot += red[k];
        scale = 1.0f / sqrtf(tot / (float)a.cols + a.eps);
    }
#pragma unroll
    for (int k = 0; k < kLinkPairs; ++k) {
        const int p = (blockIdx.y + k * gridDim.y) * TH + tid;
        if (p >= npairs) break; // pairs (2m, 2m+1) stop together: npairs is even
        const int sb = p >> 1, kh = p & 1;
        float w[8];
        if (a.gain) {
#pragma unroll
            for (int e = 0; e < 8; ++e) w[e] = __fmul_rn(__fmul_rn(v[k][e], scale), gn[k][e]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) w[e] = v[k][e];
        }
        float amax = 0.0f;
        int bad = 0; // an inf or NaN (fmaxf alone would drop a NaN)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            amax = fmaxf(amax, fabsf(w[e]));
            bad |= !(fabsf(w[e]) <= 3.402823466e38f);
        }
        // One exchange chain carries both: a non-finite piece enters as +inf,
        // which every max keeps.  DPP and permlane moves, no LDS round trips.
        amax = bad ? __int_as_float(0x7f800000) : amax;
        amax = fmaxf(amax, emu_xor_get<1>(amax));
        if (a.span) { // the span's 32 pairs are 32 neighbouring lanes (npairs is whole spans)
            amax = fmaxf(amax, emu_xor_get<2>(amax));
            amax = fmaxf(amax, emu_xor_get<4>(amax));
            amax = fmaxf(amax, emu_xor_get<8>(amax));
            amax = fmaxf(amax, emu_xor_get<16>(amax));
        }
        const bool finite = amax <= 3.402823466e38f;
        int e2 = 0;
        (void)frexpf(finite ? amax : 0.0f, &e2); // amax < 2^e2, so |x| * 2^(6-e2) < 64
        uint32_t lo[3] = {0u, 0u, 0u}, hi[3] = {0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float s = finite ? ldexpf(w[e], 6 - e2) : 0.0f; // exact
            const float f0 = rintf(s);
            const float r1 = (s - f0) * 128.0f; // exact
            const float f1 = rintf(r1);
            const float f2 = rintf((r1 - f1) * 128.0f);
            const uint32_t b[3] = {(uint32_t)(int)f0 & 0xffu, (uint32_t)(int)f1 & 0xffu, (uint32_t)(int)f2 & 0xffu};
#pragma unroll
            for (int l = 0; l < 3; ++l) {
                if (e < 4) lo[l] |= b[l] << (8 * e);
                else hi[l] |= b[l] << (8 * (e - 4));
            }
        }
        uint8_t *dst = a.xa + (size_t)sb * kSbBytes + (size_t)(kh * 24 + t) * 8;
#pragma unroll
        for (int l = 0; l < 3; ++l) *reinterpret_cast<uint2 *>(dst + 64 * l) = make_uint2(lo[l], hi[l]);
        const float scale = finite ? ldexpf(1.0f, e2 - 20) : __int_as_float(0x7fc00000);
        if (!a.span && kh == 0) a.xs[(size_t)sb * kMaxTok + t] = scale;
        if (a.span && (p & 31) == 0) a.xs[(size_t)(p >> 5) * kMaxTok + t] = scale;
    }
}

struct MfmaArgs {
    const uint8_t *w[2]; // one matrix, or the gate/up pair
    int nmat;
    size_t row_bytes;
    int rows, cols, n_tok;
    const uint8_t *xa;
    const float *xs;
    float *part; // [slices][nmat][kMaxTok][rows], slices = ceil(cols / kSlice)
    float eps; // NORM: each token's RMS factor 1 / sqrt(sum / cols + eps)
};

// Q6_K codes (0..63) of 8 columns, two dwords: sub-block (h, q, p) takes
// the nibble q>>1 of the ql bytes and bits 2q..2q+1 of the qh bytes.
__device__ __forceinline__ uint32_t code8(uint32_t ql, uint32_t qh, int q)
{
    switch (q) {
    case 0: return (ql & 0x0f0f0f0fu) | ((qh << 4) & 0x30303030u);
    case 1: return (ql & 0x0f0f0f0fu) | ((qh << 2) & 0x30303030u);
    case 2: return ((ql >> 4) & 0x0f0f0f0fu) | (qh & 0x30303030u);
    default: return ((ql >> 4) & 0x0f0f0f0fu) | ((qh >> 2) & 0x30303030u);
    }
}

// The operand-order copy: per 32-row tile and 256-column block one chunk of
// kMmChunk bytes -- six 1 KB code segments (lane l's 16 bytes at 16 l of
// each), the 32 rows' 16 scale bytes, their 32 d.  Lane l = 32 kh + j holds
// row j's codes for columns 8 kh .. 8 kh + 7 of each 16-column sub-block sb
// in 24 words: for the sub-block group g = sb / 4 and half p (columns
// 8 kh + 4 p .. + 3), word 6 g + 3 p + w, w = 0..2, has in byte b the code of
// sub-block 4 g + w in its low six bits and two bits of sub-block 4 g + 3's
// code in its top two (bits 0-1 in w = 0, 2-3 in w = 1, 4-5 in w = 2).
constexpr int kMmChunk = 6720;

// Four codes (one word of the MFMA B operand) of sub-block 4 g + jj.
__device__ __forceinline__ uint32_t mm_code4(const uint32_t *w, int jj)
{
    switch (jj) {
    case 0: return w[0] & 0x3f3f3f3fu;
    case 1: return w[1] & 0x3f3f3f3fu;
    case 2: return w[2] & 0x3f3f3f3fu;
    default: return ((w[0] >> 6) & 0x03030303u) | ((w[1] >> 4) & 0x0c0c0c0cu) | ((w[2] >> 2) & 0x30303030u);
    }
}

// One unit of work: 32 weight rows of one matrix x one 1024-column slice.
// A lane holds, for its row (lane % 32) and column half kh = lane / 32 of
// each 16-column sub-block of its wavefront's 256-column block, the weight
// bytes and the A operands (limbs of M row lane % 32).
struct Unit {
    uint2 ql[2][2][2], qh[2][2];
    uint32_t cw[24]; // the operand-order copy's code words (MM)
    uint4 sc;
    uint32_t d;
    long av[16];
    int ks, rt, mat;
};

// One unit per workgroup (four fit per CU; they drift out of step, so one
// loads while another computes).  The weight bytes are fetched coalesced --
// four rows per instruction, 16 bytes per lane -- into the wavefront's own
// LDS rows and read back in the MFMA operand layout (fetching that layout
// directly, 8 bytes from each of 32 rows per instruction, streams at about
// two thirds of the rate).  The unit's per-token scales are staged in LDS
// while the weights load.
// MM: the weights come from the operand-order copy (emu_mfma_major_q6k):
// each 32-row x 256-column tile block is one 6720-byte chunk whose code words
// are already in each lane's operand order, so six 1 KB loads per wavefront
// bring them straight into registers (no LDS round trip), and its scales and
// d follow, all with the non-temporal hint (each weight byte is read once per
// step; batch 8 measured 0.7% faster than with plain loads).  The codes are
// the same, so the results are bit for bit those of the GGUF-order path.
// NORM (span form only): the operands come from a link that left its RMS
// factor to this matvec; the link's sums of squares sit kSsRegion bytes
// ahead of xa.
template <bool MM, bool SPAN, bool NORM>
__global__ __launch_bounds__(EMU_WAVE * kWaves, 4) void qmv_mfma_kernel(MfmaArgs a, int units)
{
    const int nks = (a.cols + kSlice - 1) / kSlice, nrt = (a.rows + kTileRows - 1) / kTileRows;
    const int tid = threadIdx.x, lane = tid & (EMU_WAVE - 1), w = tid / EMU_WAVE;
    const int j = lane & 31, kh = lane >> 5;
    // A row j: limb j / 8 of token j % 8.  Rows 24..31 and the rows of tokens
    // past n_tok hold whatever the operand area holds: an MFMA output row
    // depends on its own A row only, and those rows' outputs are never stored.
    const int arow = j < 24 ? j : 0;
    __shared__ __align__(16) float xs[kSlice / 16 * kMaxTok];
    __shared__ float red[kWaves][kMaxTok][kTileRows];

    Unit b;
    float4 xsv;
    float sq[3];
    __shared__ __align__(16) uint8_t wl[kWaves][kTileRows * kRowStride];
    {
        const int u = blockIdx.x;
        b.ks = u % nks;
        const int v = u / nks;
        b.rt = v % nrt;
        b.mat = v / nrt;
        const int cb = b.ks * kWaves + w; // this wavefront's 256-column block
        // The last slice of a row whose width is not a multiple of the slice
        // has wavefronts past the row: they read the row's last block and
        // add zeros (d = 0, and every sum is a finite integer).
        const bool has = cb < a.cols / 256;
        const int cbl = has ? cb : a.cols / 256 - 1; // a block of the row: past it, scaled by zero
        // The A operands (activation limbs, from L2) load before the weights
        // (from HBM): loads complete in issue order, so the other way round
        // their round trip would follow the weights' instead of overlapping it.
        const uint8_t *ap = a.xa + (size_t)cbl * 16 * kSbBytes + (size_t)(kh * 24 + arow) * 8;
#pragma unroll
        for (int sb = 0; sb < 16; ++sb) b.av[sb] = *reinterpret_cast<const long *>(ap + sb * kSbBytes);
        if constexpr (NORM) { // the link's sums of squares: lane 8 t + i, token t's sums i, i + 8, i + 16
            const float *ssp = reinterpret_cast<const float *>(a.xa - kSsRegion);
            const int tt = lane >> 3, g = lane & 7, groups = (a.cols / 8 + kLinkSmall - 1) / kLinkSmall;
#pragma unroll
            for (int k = 0; k < 3; ++k) sq[k] = g + 8 * k < groups ? ssp[tt * kSsGroups + g + 8 * k] : 0.0f;
        }
        // and so do the slice's activation scales (one float4 per thread:
        // half a sub-block's eight tokens; zero past the row)
        static_assert(kSlice / 16 * kMaxTok / 4 <= EMU_WAVE * kWaves, "one scale load per thread");
        if constexpr (SPAN) { // the block's span scale for this lane's four tokens
            xsv = *reinterpret_cast<const float4 *>(a.xs + (size_t)cbl * kMaxTok + 4 * kh);
            if (!has) xsv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        } else {
            const float4 *xsrc = reinterpret_cast<const float4 *>(a.xs + (size_t)b.ks * (kSlice / 16) * kMaxTok);
            const int t4 = tid < kSlice / 16 * kMaxTok / 4 ? tid : 0;
            xsv = b.ks * (kSlice / 16) + t4 / 2 < a.cols / 16 ? xsrc[t4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        __builtin_amdgcn_sched_barrier(0);
        // Coalesced: instruction k covers rows 4k..4k+3 of the tile, 16 lanes
        // per row (13 x 16 bytes + the 2-byte d), into this wavefront's LDS rows.
        const int r4 = lane >> 4, c16 = lane & 15;
        if (MM) {
            const uint8_t *cp = a.w[b.mat] + ((size_t)b.rt * (a.cols / 256) + cbl) * kMmChunk;
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                const uint4 q4 = ldnt16(cp + 1024 * i + 16 * lane);
                b.cw[4 * i] = q4.x;
                b.cw[4 * i + 1] = q4.y;
                b.cw[4 * i + 2] = q4.z;
                b.cw[4 * i + 3] = q4.w;
            }
            b.sc = ldnt16(cp + 6144 + 16 * j);
            b.d = ldnt2(cp + 6656 + 2 * j);
            // Every load goes out before anything waits on one: without this
            // barrier the scheduler put the last two code loads behind the
            // conversion of d, whose wait then took the whole first batch (a
            // second HBM round trip per workgroup; batch 8 2,500 -> 2,590 tok/s).
            __builtin_amdgcn_sched_barrier(0);
        } else {
            uint4 raw[8];
            uint16_t dd[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                int row = b.rt * kTileRows + 4 * k + r4;
                row = row < a.rows ? row : a.rows - 1; // a valid row; never stored
                const uint8_t *bp = a.w[b.mat] + (size_t)row * a.row_bytes + (size_t)cbl * 210;
                if (c16 < 13) raw[k] = ld16(bp + 16 * c16);
                else if (c16 == 13) dd[k] = ld2(bp + 208);
            }
            uint8_t *mine = wl[w];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                uint8_t *rp = mine + (4 * k + r4) * kRowStride;
                if (c16 < 13) {
                    *reinterpret_cast<uint2 *>(rp + 16 * c16) = make_uint2(raw[k].x, raw[k].y);
                    *reinterpret_cast<uint2 *>(rp + 16 * c16 + 8) = make_uint2(raw[k].z, raw[k].w);
                } else if (c16 == 13) {
                    *reinterpret_cast<uint16_t *>(rp + 208) = dd[k];
                }
            }
            __builtin_amdgcn_wave_barrier(); // LDS accesses of one wavefront complete in order
            const uint8_t *bp = mine + j * kRowStride;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    b.ql[h][0][p] = *reinterpret_cast<const uint2 *>(bp + 64 * h + 16 * p + 8 * kh);
                    b.ql[h][1][p] = *reinterpret_cast<const uint2 *>(bp + 64 * h + 32 + 16 * p + 8 * kh);
                    b.qh[h][p] = *reinterpret_cast<const uint2 *>(bp + 128 + 32 * h + 16 * p + 8 * kh);
                }
            const uint2 s0 = *reinterpret_cast<const uint2 *>(bp + 192), s1 = *reinterpret_cast<const uint2 *>(bp + 200);
            b.sc = make_uint4(s0.x, s0.y, s1.x, s1.y);
            b.d = *reinterpret_cast<const uint16_t *>(bp + 208);
        }
        if (!has) b.d = 0; // d = 0: the block's (finite, integer) sums add exact zeros
    }
    static_assert(SPAN || !NORM, "the deferred norm comes with span scales");
    if constexpr (NORM) {
        // The factor, formed while the weights are in flight: the sums in a
        // fixed order (the same in every workgroup), token t's in lane 8 t.
        // Tokens past n_tok take whatever their slots hold; their outputs
        // are never stored.
        float tot = (sq[0] + sq[1]) + sq[2];
        tot += emu_xor_lane<1>(tot);
        tot += emu_xor_lane<2>(tot);
        tot += emu_xor_lane<4>(tot);
        const int rb = __float_as_int(1.0f / sqrtf(tot / (float)a.cols + a.eps));
        float rs[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) rs[t] = __int_as_float(__builtin_amdgcn_readlane(rb, 8 * t));
        xsv.x *= kh ? rs[4] : rs[0]; // a power of two times the factor: exact
        xsv.y *= kh ? rs[5] : rs[1];
        xsv.z *= kh ? rs[6] : rs[2];
        xsv.w *= kh ? rs[7] : rs[3];
    }
    if constexpr (!SPAN) { // the slice's scales, shared by the workgroup
        if (tid < kSlice / 16 * kMaxTok / 4) reinterpret_cast<float4 *>(xs)[tid] = xsv;
        __syncthreads();
    }

    // Sub-block sb = 8h + 2q + p: D = A x codes + A x (-32), then the float
    // step.  Software-pipelined by hand (the next sub-block's MFMAs go out
    // before this one's float step) with a scheduling barrier per step, so
    // only two accumulator tiles are live.
    const long neg32 = (long)0xe0e0e0e0e0e0e0e0ull;
    const float d = h2f((uint16_t)b.d);
    const float *sp = xs + (size_t)w * 16 * kMaxTok + 4 * kh;
    auto mma = [&](int sb) {
        long bv;
        if constexpr (MM) {
            const int g = sb >> 2, jj = sb & 3;
            const uint32_t lo = mm_code4(b.cw + 6 * g, jj), hi = mm_code4(b.cw + 6 * g + 3, jj);
            bv = (long)(((uint64_t)hi << 32) | lo);
        } else {
            const int h = sb >> 3, q = (sb >> 1) & 3, p = sb & 1;
            const uint2 lq = b.ql[h][q & 1][p], hq = b.qh[h][p];
            bv = (long)(((uint64_t)code8(lq.y, hq.y, q) << 32) | code8(lq.x, hq.x, q));
        }
        v16i D = {};
        D = __builtin_amdgcn_mfma_i32_32x32x16_i8(b.av[sb], bv, D, 0, 0, 0);
        return __builtin_amdgcn_mfma_i32_32x32x16_i8(b.av[sb], neg32, D, 0, 0, 0);
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // Span scales: the block is one span, so the limb sums stay integers
    // across its sixteen sub-blocks, each times its 8-bit scale
    // (|D| <= 16 * 32 * 64 = 2^15, |sc| <= 2^7, sixteen of them < 2^27; the
    // operands sign-extended from 24 bits, which the compiler folds into
    // the full-rate v_mad_i32_i24), and one float step per block forms
    // (16384 S0 + 128 S1 + S2) * d * s in double, rounded once.
    int acci[3][4] = {};
    auto epi = [&](int sb, const v16i &D) {
        const uint32_t sw = sb < 4 ? b.sc.x : sb < 8 ? b.sc.y : sb < 12 ? b.sc.z : b.sc.w;
        if constexpr (SPAN) {
            const int sc = (int)__builtin_amdgcn_sbfe(sw, 8u * (uint32_t)(sb & 3), 8u);
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int l = 0; l < 3; ++l) acci[l][r] = ((D[r + 4 * l] << 8) >> 8) * ((sc << 8) >> 8) + acci[l][r];
            // The running sums are pinned here: left free, the compiler
            // pairs two sub-blocks' products into v_mul_i32_i24 + v_add3_u32
            // (263 VALU instructions per block instead of 192 multiply-adds).
            asm volatile(""
                         : "+v"(acci[0][0]), "+v"(acci[0][1]), "+v"(acci[0][2]), "+v"(acci[0][3]), "+v"(acci[1][0]),
                           "+v"(acci[1][1]), "+v"(acci[1][2]), "+v"(acci[1][3]), "+v"(acci[2][0]), "+v"(acci[2][1]),
                           "+v"(acci[2][2]), "+v"(acci[2][3]));
        } else {
            const float scd = (float)(int)__builtin_amdgcn_sbfe(sw, 8u * (uint32_t)(sb & 3), 8u) * d;
            const float4 s4 = *reinterpret_cast<const float4 *>(sp + sb * kMaxTok);
            const float s[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // |t| < 2^30 by the limb bounds; unsigned arithmetic keeps the
                // intermediate sums well defined.
                const uint32_t t1 = ((uint32_t)D[r] << 7) + (uint32_t)D[r + 4];
                const int t = (int)((t1 << 7) + (uint32_t)D[r + 8]);
                acc[r] = __builtin_fmaf((float)t, scd * s[r], acc[r]);
            }
        }
    };
    v16i cur = mma(0);
#pragma unroll
    for (int sb = 0; sb < 16; ++sb) {
        v16i next;
        if (sb + 1 < 16) next = mma(sb + 1);
        epi(sb, cur);
        __builtin_amdgcn_sched_barrier(0);
        if (sb + 1 < 16) cur = next;
    }
    if constexpr (SPAN) {
        const float s[4] = {xsv.x, xsv.y, xsv.z, xsv.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const double t = (double)acci[0][r] * 16384.0 + (double)acci[1][r] * 128.0 + (double)acci[2][r]; // exact
            acc[r] = (float)(t * ((double)d * (double)s[r]));
        }
    }

    // The four wavefronts' sums meet in LDS in a fixed order.
#pragma unroll
    for (int r = 0; r < 4; ++r) red[w][4 * kh + r][j] = acc[r];
    __syncthreads();
    if (tid < kMaxTok * kTileRows) {
        const int t = tid / kTileRows, jj = tid % kTileRows, orow = b.rt * kTileRows + jj;
        if (t < a.n_tok && orow < a.rows) {
            float v = red[0][t][jj];
#pragma unroll
            for (int k = 1; k < kWaves; ++k) v += red[k][t][jj];
            a.part[(((size_t)b.ks * a.nmat + b.mat) * kMaxTok + t) * a.rows + orow] = v;
        }
    }
}

struct FinishArgs {
    const float *part;
    int nks, nmat, rows;
    float *y; // n_tok x rows
    int accumulate;
    float acc_scale, out_div, softcap;
    int act;
    uint64_t *keys;
    int key_stride, tie_last;
};

// A row's slices added in slice order, every load issued before the first
// add (slots past n read slice 0 and are dropped): one memory round trip.
template <int MAXS> __device__ __forceinline__ float slice_sum1(const float *p, size_t stride, int n)
{
    float q[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; ++s) q[s] = p[(s < n ? s : 0) * stride];
    float v = q[0];
#pragma unroll
    for (int s = 1; s < MAXS; ++s) v = s < n ? v + q[s] : v;
    return v;
}

template <int MAXS>
__global__ __launch_bounds__(kFinishThreads) void mfma_finish_kernel(FinishArgs a)
{
    const int t = blockIdx.y, row = blockIdx.x * kFinishThreads + threadIdx.x;
    const bool ok = row < a.rows;
    float v = 0.0f;
    if (ok) {
        const size_t stride = (size_t)a.nmat * kMaxTok * a.rows;
        const float *p = a.part + (size_t)t * a.rows + row;
        v = slice_sum1<MAXS>(p, stride, a.nks);
        if (a.nmat == 2) {
            const float up = slice_sum1<MAXS>(p + (size_t)kMaxTok * a.rows, stride, a.nks);
            v = emu_glu(v, up, a.act);
        }
        v = emu_out_epi(v, a.out_div, a.softcap);
        float *dst = a.y + (size_t)t * a.rows + row;
        *dst = a.accumulate ? emu_resid_add(*dst, v, a.acc_scale) : v;
    }
    if (a.keys) {
        __shared__ uint64_t best[kFinishThreads / EMU_WAVE];
        uint64_t k = ok ? emu_select_key(v, (uint32_t)row, a.tie_last) : 0;
#pragma unroll
        for (int o = EMU_WAVE / 2; o >= 1; o >>= 1) {
            const uint64_t other = __shfl_xor(k, o, EMU_WAVE);
            k = other > k ? other : k;
        }
        if ((threadIdx.x & (EMU_WAVE - 1)) == 0) best[threadIdx.x / EMU_WAVE] = k;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t m = best[0];
#pragma unroll
            for (int w = 1; w < kFinishThreads / EMU_WAVE; ++w) m = best[w] > m ? best[w] : m;
            a.keys[(size_t)t * a.key_stride + blockIdx.x] = m;
        }
    }
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Workspace: the deferred norms' sums of squares (kSsRegion bytes, so a
// matvec finds them just ahead of its A operands), the A operands and
// scales for up to cols_cap columns, then the partial sums.
struct Ws {
    uint8_t *xa;
    float *xs, *part, *ss;
    size_t part_bytes;
};
size_t operand_bytes(int cols_cap)
{
    const size_t nsb = (size_t)cols_cap / 16;
    return kSsRegion + align256(nsb * kSbBytes) + align256(nsb * kMaxTok * sizeof(float));
}
Ws workspace(emu_ctx *ctx, int cols_cap)
{
    const size_t nsb = (size_t)cols_cap / 16;
    uint8_t *base = static_cast<uint8_t *>(ctx->mfma_ws);
    Ws w;
    w.ss = reinterpret_cast<float *>(base);
    w.xa = base + kSsRegion;
    w.xs = reinterpret_cast<float *>(w.xa + align256(nsb * kSbBytes));
    w.part = reinterpret_cast<float *>(base + operand_bytes(cols_cap));
    w.part_bytes = ctx->mfma_ws_bytes > operand_bytes(cols_cap) ? ctx->mfma_ws_bytes - operand_bytes(cols_cap) : 0;
    return w;
}
size_t part_bytes(int rows, int cols, int nmat)
{
    return (size_t)((cols + kSlice - 1) / kSlice) * nmat * kMaxTok * (size_t)rows * sizeof(float);
}

} // namespace

size_t emu_mfma_workspace_bytes(int rows, int cols, int nmat)
{
    return operand_bytes(cols) + align256(part_bytes(rows, cols, nmat));
}

size_t emu_mfma_chain_bytes(int cols_cap, size_t max_part_bytes)
{
    return operand_bytes(cols_cap) + align256(max_part_bytes);
}

size_t emu_mfma_part_bytes(int rows, int cols, int nmat) { return part_bytes(rows, cols, nmat); }

int emu_mfma_reserve(emu_ctx *ctx, size_t bytes)
{
    if (bytes <= ctx->mfma_ws_bytes) return EMU_OK;
    if (ctx->mfma_ws) {
        EMU_HIP(ctx, hipStreamSynchronize(ctx->stream));
        EMU_HIP(ctx, hipFree(ctx->mfma_ws));
        ctx->mfma_ws = nullptr;
        ctx->mfma_ws_bytes = 0;
    }
    EMU_HIP(ctx, hipMalloc(&ctx->mfma_ws, bytes));
    ctx->mfma_ws_bytes = bytes;
    return EMU_OK;
}

bool emu_mfma_shape_ok(int encoding, int cols)
{
    return encoding == EMU_ENC_Q6_K && cols > 0 && (cols % kSlice == 0 || (cols % 256 == 0 && cols >= 2048)) &&
           (cols + kSlice - 1) / kSlice <= kMaxSlices && cols <= 8 * kLinkThreads * kLinkPairs;
}

bool emu_mfma_supports(int encoding, int cols, int n_tok)
{
    // Widths that are not whole slices (a multiple of 256 columns, the last
    // slice partly empty) only from 2048 columns: below that the single-launch
    // vector kernel costs less than link, matvec and finish.
    return encoding == EMU_ENC_Q6_K && n_tok >= 2 && n_tok <= kMaxTok && cols > 0 &&
           (cols % kSlice == 0 || (cols % 256 == 0 && cols >= 2048)) && (cols + kSlice - 1) / kSlice <= kMaxSlices &&
           cols <= 8 * kLinkThreads * kLinkPairs;
}

template <int MODE> static void launch_link(bool narrow, dim3 grid, hipStream_t stream, const LinkArgs &a)
{
    if (a.gain && !a.ssp) { // the row's sum of squares in one workgroup
        if (narrow)
            hipLaunchKernelGGL((mfma_link_kernel<4, MODE, kLinkThreads>), grid, dim3(kLinkThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((mfma_link_kernel<kMaxSlices, MODE, kLinkThreads>), grid, dim3(kLinkThreads), 0, stream,
                               a);
    } else {
        if (narrow)
            hipLaunchKernelGGL((mfma_link_kernel<4, MODE, kLinkSmall>), grid, dim3(kLinkSmall), 0, stream, a);
        else
            hipLaunchKernelGGL((mfma_link_kernel<kMaxSlices, MODE, kLinkSmall>), grid, dim3(kLinkSmall), 0, stream, a);
    }
}

int emu_mfma_link(emu_ctx *ctx, const EmuMfmaLink &l)
{
    if (l.n_tok < 1 || l.n_tok > kMaxTok || l.cols <= 0 || l.cols % 16 != 0 || l.cols > l.cols_cap ||
        l.cols > 8 * kLinkThreads * kLinkPairs)
        return EMU_E_CONFIG;
    const Ws w = workspace(ctx, l.cols_cap);
    if (!ctx->mfma_ws || (l.limbs && ctx->mfma_ws_bytes < operand_bytes(l.cols_cap))) return EMU_E_CONFIG;
    LinkArgs a{};
    a.part = l.from_part ? w.part : nullptr;
    a.nks = l.from_part ? l.part_nks : 0;
    a.nmat = l.part_nmat;
    a.mode = l.mode;
    a.h = l.h;
    a.x = l.x;
    a.cols = l.cols;
    a.n_tok = l.n_tok;
    a.gain = l.gain;
    a.eps = l.eps;
    a.xa = l.limbs ? w.xa : nullptr;
    a.xs = l.limbs ? w.xs : nullptr;
    a.m_contrib = l.mode == kLinkInput ? l.m_contrib : nullptr;
    a.m_sorted = l.m_sorted;
    a.m_ids = l.m_ids;
    a.m_wts = l.m_wts;
    a.m_k = l.m_k;
    a.m_experts = l.m_experts;
    a.m_scale = l.m_scale;
    a.d_part = l.mode == kLinkInput && l.d_part ? w.part : nullptr;
    a.d_nks = l.d_nks;
    a.d_scale = l.d_scale;
    a.act = l.act;
    a.span = l.span;
    a.ssp = l.defer_norm && a.gain && a.xa ? w.ss : nullptr;
    if (a.span && (l.cols % 256 != 0 || !a.xa)) return EMU_E_CONFIG;
    if (l.defer_norm && (!a.gain || !a.span || !a.xa)) return EMU_E_CONFIG; // only before a span matvec
    if (a.m_contrib && (!a.h || !a.m_ids || !a.m_wts || a.m_k < 1 || a.m_k > 8)) return EMU_E_CONFIG;
    if (a.d_part && (!a.h || a.d_nks < 1 || a.d_nks > kMaxSlices ||
                     (size_t)a.d_nks * kMaxTok * (size_t)l.cols * sizeof(float) > w.part_bytes))
        return EMU_E_CONFIG;
    if (l.from_part && (size_t)a.nks * a.nmat * kMaxTok * (size_t)l.cols * sizeof(float) > w.part_bytes)
        return EMU_E_CONFIG;
    // Without a norm (or with it deferred) there is no row-wide sum: one
    // small workgroup per 512 columns.
    const int gy = a.gain && !a.ssp ? 1 : (l.cols / 8 + kLinkSmall - 1) / kLinkSmall;
    const bool narrow = a.nks <= 4 && a.d_nks <= 4;
    const dim3 grid(l.n_tok, gy);
    switch (a.mode) {
    case kLinkInput: launch_link<kLinkInput>(narrow, grid, ctx->stream, a); break;
    case kLinkResid: launch_link<kLinkResid>(narrow, grid, ctx->stream, a); break;
    case kLinkSwiglu: launch_link<kLinkSwiglu>(narrow, grid, ctx->stream, a); break;
    case kLinkPlain: launch_link<kLinkPlain>(narrow, grid, ctx->stream, a); break;
    default: return EMU_E_CONFIG;
    }
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

int emu_mfma_matvec(emu_ctx *ctx, const QmvArgs &q, int n_tok, int cols_cap, int *part_nks)
{
    if (n_tok < 1 || n_tok > kMaxTok || !emu_mfma_shape_ok(EMU_ENC_Q6_K, q.cols) || q.cols > cols_cap || q.rows <= 0)
        return EMU_E_CONFIG;
    const int nmat = q.w_up ? 2 : 1;
    const Ws w = workspace(ctx, cols_cap);
    if (!ctx->mfma_ws || part_bytes(q.rows, q.cols, nmat) > w.part_bytes) return EMU_E_CONFIG;
    MfmaArgs ma{};
    ma.w[0] = q.w;
    ma.w[1] = q.w_up;
    ma.nmat = nmat;
    ma.row_bytes = q.row_bytes;
    ma.rows = q.rows;
    ma.cols = q.cols;
    ma.n_tok = n_tok;
    ma.xa = w.xa;
    ma.xs = w.xs;
    ma.part = w.part;
    if (q.span_norm && !q.span_scales) return EMU_E_CONFIG;
    ma.eps = q.eps;
    const int nks = (q.cols + kSlice - 1) / kSlice, nrt = (q.rows + kTileRows - 1) / kTileRows;
    const int units = nks * nrt * nmat;
    const dim3 grid((unsigned)units), block(EMU_WAVE * kWaves);
    if (q.mfma_major && q.span_norm)
        hipLaunchKernelGGL((qmv_mfma_kernel<true, true, true>), grid, block, 0, ctx->stream, ma, units);
    else if (q.mfma_major && q.span_scales)
        hipLaunchKernelGGL((qmv_mfma_kernel<true, true, false>), grid, block, 0, ctx->stream, ma, units);
    else if (q.mfma_major)
        hipLaunchKernelGGL((qmv_mfma_kernel<true, false, false>), grid, block, 0, ctx->stream, ma, units);
    else if (q.span_norm)
        hipLaunchKernelGGL((qmv_mfma_kernel<false, true, true>), grid, block, 0, ctx->stream, ma, units);
    else if (q.span_scales)
        hipLaunchKernelGGL((qmv_mfma_kernel<false, true, false>), grid, block, 0, ctx->stream, ma, units);
    else
        hipLaunchKernelGGL((qmv_mfma_kernel<false, false, false>), grid, block, 0, ctx->stream, ma, units);
    EMU_LAUNCH_CHECK(ctx);
    if (part_nks) *part_nks = nks;
    return EMU_OK;
}

int emu_mfma_finish(emu_ctx *ctx, const QmvArgs &q, int n_tok, int cols_cap, int *key_slots)
{
    const int nmat = q.w_up ? 2 : 1;
    const int gx = (q.rows + kFinishThreads - 1) / kFinishThreads;
    if (q.keys && gx > q.key_stride) return EMU_E_CONFIG;
    const Ws w = workspace(ctx, cols_cap);
    FinishArgs fa{};
    fa.part = w.part;
    fa.nks = (q.cols + kSlice - 1) / kSlice;
    fa.nmat = nmat;
    fa.rows = q.rows;
    fa.y = q.y;
    fa.accumulate = q.accumulate;
    fa.acc_scale = q.acc_scale;
    fa.out_div = q.out_div;
    fa.softcap = q.softcap;
    fa.act = q.act;
    fa.keys = q.keys;
    fa.key_stride = q.key_stride;
    fa.tie_last = q.tie_last;
    if (fa.nks <= 4)
        hipLaunchKernelGGL(mfma_finish_kernel<4>, dim3((unsigned)gx, (unsigned)n_tok), dim3(kFinishThreads), 0,
                           ctx->stream, fa);
    else
        hipLaunchKernelGGL(mfma_finish_kernel<kMaxSlices>, dim3((unsigned)gx, (unsigned)n_tok), dim3(kFinishThreads),
                           0, ctx->stream, fa);
    EMU_LAUNCH_CHECK(ctx);
    if (key_slots) *key_slots = gx;
    return EMU_OK;
}

void emu_mfma_buffers(emu_ctx *ctx, int cols_cap, uint8_t **xa, float **xs, float **part)
{
    const Ws w = workspace(ctx, cols_cap);
    *xa = w.xa;
    *xs = w.xs;
    *part = w.part;
}

int emu_launch_mfma(emu_ctx *ctx, int encoding, const QmvArgs &a, int n_tok, int *key_slots)
{
    if (n_tok < 1 || n_tok > kMaxTok || !emu_mfma_shape_ok(encoding, a.cols)) return EMU_E_UNSUPPORTED;
    if (a.rows <= 0) return EMU_E_ARG;
    const int nmat = a.w_up ? 2 : 1;
    if (nmat == 2 && a.accumulate) return EMU_E_ARG; // the fused entry point never asks for this
    const int gx = (a.rows + kFinishThreads - 1) / kFinishThreads;
    if (a.keys && gx > a.key_stride) return EMU_E_CONFIG;
    int st = emu_mfma_reserve(ctx, emu_mfma_workspace_bytes(a.rows, a.cols, nmat));
    if (st != EMU_OK) return st;
    EmuMfmaLink l{};
    l.mode = kLinkInput;
    l.x = a.x;
    l.cols = a.cols;
    l.cols_cap = a.cols;
    l.n_tok = n_tok;
    l.gain = a.gain;
    l.eps = a.eps;
    l.limbs = true;
    l.span = a.span_scales; // the chained steps' output matvec; the C ABI's calls keep per-sub-block scales
    l.defer_norm = a.span_scales && a.gain; // the matvec takes the RMS factor
    if ((st = emu_mfma_link(ctx, l)) != EMU_OK) return st;
    QmvArgs q = a;
    q.span_norm = l.defer_norm;
    if ((st = emu_mfma_matvec(ctx, q, n_tok, a.cols, nullptr)) != EMU_OK) return st;
    return emu_mfma_finish(ctx, a, n_tok, a.cols, key_slots);
}

namespace {

// Code (0..63) of column c of a Q6_K block held at in[0..209]: column
// 128h + 32q + 16m + i takes the nibble q >> 1 of ql[64h + 32(q & 1) + 16m + i]
// and bits 2q..2q+1 of qh[32h + 16m + i].
__device__ __forceinline__ uint32_t q6k_code(const uint8_t *in, uint32_t c)
{
    const uint32_t h = c >> 7, q = (c >> 5) & 3u, m = (c >> 4) & 1u, i = c & 15u;
    const uint32_t lo = (uint32_t)in[64u * h + 32u * (q & 1u) + 16u * m + i] >> (4u * (q >> 1)) & 15u;
    const uint32_t hi = (uint32_t)in[128u + 32u * h + 16u * m + i] >> (2u * q) & 3u;
    return lo | hi << 4;
}

// One workgroup per (32-row tile, 256-column block) chunk, grid-stride: the
// chunk's 32 blocks come into LDS (rows past the matrix repeat its last row)
// and each destination byte is formed from there.
__global__ __launch_bounds__(256) void mfma_major_kernel(const uint8_t *src, uint32_t rows, uint32_t nblk,
                                                         size_t row_bytes, uint8_t *dst, size_t chunks)
{
    __shared__ uint8_t in[kTileRows][210];
    for (size_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const uint32_t rt = (uint32_t)(c / nblk), cb = (uint32_t)(c % nblk);
        for (uint32_t o = threadIdx.x; o < kTileRows * 210u; o += 256u) {
            const uint32_t r = o / 210u, k = o % 210u;
            const uint32_t row = rt * kTileRows + r < rows ? rt * kTileRows + r : rows - 1;
            in[r][k] = src[(size_t)row * row_bytes + (size_t)cb * 210u + k];
        }
        __syncthreads();
        uint8_t *d = dst + c * kMmChunk;
        for (uint32_t o = threadIdx.x; o < (uint32_t)kMmChunk; o += 256u) {
            uint8_t v;
            if (o < 6144u) { // code word 6g + 3p + w of lane 32 kh + j, byte b
                const uint32_t within = o & 1023u, lane = within >> 4, q = within & 15u;
                const uint32_t k = 4u * (o >> 10) + (q >> 2), b = q & 3u;
                const uint32_t g = k / 6u, p = (k % 6u) / 3u, w = k % 3u;
                const uint32_t col = 8u * (lane >> 5) + 4u * p + b;
                const uint8_t *r = in[lane & 31u];
                const uint32_t cw = q6k_code(r, 16u * (4u * g + w) + col);
                const uint32_t c3 = q6k_code(r, 16u * (4u * g + 3u) + col);
                v = (uint8_t)(cw | ((c3 >> (2u * w)) & 3u) << 6);
            } else if (o < 6656u) { // the 32 rows' scale bytes
                const uint32_t r = o - 6144u;
                v = in[r >> 4][192u + (r & 15u)];
            } else { // and their d
                const uint32_t r = o - 6656u;
                v = in[r >> 1][208u + (r & 1u)];
            }
            d[o] = v;
        }
        __syncthreads();
    }
}

} // namespace

size_t emu_mfma_major_bytes(uint32_t rows, uint32_t cols)
{
    return (size_t)((rows + kTileRows - 1) / kTileRows) * (cols / 256) * kMmChunk;
}

int emu_mfma_major_q6k(emu_ctx *ctx, const uint8_t *src, uint32_t rows, uint32_t cols, uint8_t *dst)
{
    if (rows == 0 || cols == 0) return EMU_OK;
    if (cols % 256 != 0) return EMU_E_SHORT;
    const uint32_t nblk = cols / 256;
    const size_t chunks = (size_t)((rows + kTileRows - 1) / kTileRows) * nblk;
    const unsigned grid = (unsigned)(chunks < 65536 ? chunks : 65536);
    hipLaunchKernelGGL(mfma_major_kernel, dim3(grid), dim3(256), 0, ctx->stream, src, rows, nblk, (size_t)nblk * 210,
                       dst, chunks);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

extern "C" size_t emu_weights_mfma_major_bytes(uint32_t rows, uint32_t cols)
{
    return cols % 256 == 0 ? emu_mfma_major_bytes(rows, cols) : 0;
}

extern "C" int emu_weights_mfma_major(emu_ctx *ctx, int encoding, const void *d_src, size_t len, uint32_t rows,
                                      uint32_t cols, void *d_dst)
{
    if (!ctx || !d_src || !d_dst) return EMU_E_ARG;
    if (encoding != EMU_ENC_Q6_K) return EMU_E_UNSUPPORTED;
    if (rows == 0 || cols == 0 || cols % 256 != 0) return EMU_E_SHORT;
    if (len != (size_t)rows * (cols / 256) * 210) return EMU_E_SHAPE;
    const uint8_t *s = static_cast<const uint8_t *>(d_src);
    uint8_t *d = static_cast<uint8_t *>(d_dst);
    const size_t out = emu_mfma_major_bytes(rows, cols);
    if (s < d + out && d < s + len) return EMU_E_ARG; // not in place
    return emu_mfma_major_q6k(ctx, s, rows, cols, d);
}
