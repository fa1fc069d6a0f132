// limb.hip -- batch-1 quantized matvec on integer dot products.
//
// The weight codes of a GGUF K-quant are small integers; the activations are
// f32.  Instead of converting every code to float (one convert and one fma
// per weight), the activation vector is re-expressed once per launch as
// integers: each 16-column sub-block gets a power-of-two scale s and three
// signed 7-bit limbs per column,
//
//     x ~= s * (16384 * L0 + 128 * L1 + L2),    |L0|, |L1|, |L2| <= 64,
//
// exact to 2^-20 of the sub-block's largest |x| (the residual of the third
// limb), i.e. as fine as the rounding of an f32 dot over a few thousand
// terms.  A sub-block's dot with the codes is then three v_dot4_i32_i8 chains
// (four weights per instruction) combined exactly in int32, so the float work
// is one convert and one fma per 16 weights.
//
// Layout of the work: a wavefront covers 4096 columns of a row, lane l owning
// the 64 columns of unit l (for Q6_K: the (half, 16-column slot) quarter of a
// 256-column block, i.e. 16 bytes of ql low nibbles, 16 of ql high nibbles,
// 16 of qh and the block's scales -- three dwordx4 loads per row).  The lane
// keeps its 64 columns' limbs in registers for the whole launch, so a row
// costs only its weight bytes.  Waves are persistent: row-group g handles rows
// g, g + G, g + 2G, ... (G row-groups in the grid) with the next D rows'
// loads in flight while the current ones are reduced (DPP wave sums, two
// values per reduction).  A wavefront's rows are finished (activation,
// residual, store) a window of up to 64 at a time, one row per lane, not
// once per row by a single lane.  Rows of 4096*S columns use S wavefronts
// per row-group, whose partial sums meet in LDS in a fixed order
// (deterministic results).
//
// Prologue (per workgroup, overlapped with the first rows' loads, which are
// issued right after x's): x is read,
// optionally RMS-normalised as (x * scale) * gain with
// scale = 1 / sqrt(mean(x^2) + eps), and split into limbs in LDS.  A
// sub-block holding an inf or NaN gets a NaN scale, so every row it meets
// comes out NaN; sub-blocks whose largest |x| is below 2^-107 have subnormal
// scales and lose precision (as f32 products of such values do).
#include "internal.hpp"

#include <type_traits>

#include <math.h>
#include <stdlib.h>

namespace {

struct LimbRec { // one 16-column sub-block, 64 bytes
    uint4 l0, l1, l2; // limbs, one byte per column
    float s;          // power-of-two scale (NaN when the sub-block holds a non-finite value)
    int sum;          // sum over the columns of 16384*L0 + 128*L1 + L2
    int pad[2];
};
static_assert(sizeof(LimbRec) == 64, "LimbRec layout");

// A lane's four sub-blocks: limbs, scales and the format's bias term.
struct Limbs {
    uint4 l[4][3];
    float s[4];
    int c[4];
};

__device__ __forceinline__ int comp(const uint4 &v, int i)
{
    return (int)(i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w);
}

// Wave-wide sum by DPP row operations; the total is valid in lane 63.
#define EMU_DPP(v, ctrl, rm) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, rm, 0xf, false))
__device__ __forceinline__ float wave_sum63(float v)
{
    v += EMU_DPP(v, 0xb1, 0xf);  // quad_perm [1,0,3,2]
    v += EMU_DPP(v, 0x4e, 0xf);  // quad_perm [2,3,0,1]
    v += EMU_DPP(v, 0x141, 0xf); // row_half_mirror
    v += EMU_DPP(v, 0x140, 0xf); // row_mirror
    v += EMU_DPP(v, 0x142, 0xa); // row_bcast:15 into rows 1 and 3
    v += EMU_DPP(v, 0x143, 0xc); // row_bcast:31 into rows 2 and 3
    return v;
}

// Wave-wide sums of two values at once, bit for bit those of wave_sum63:
// lanes 0..15 and 32..47 get a's total, lanes 16..31 and 48..63 b's.  Both
// get their 16-lane row sums by DPP, a permlane16 swap adds row pairs of a
// into rows 0 and 2 and of b into rows 1 and 3, and a permlane32 swap adds
// the two halves: (r0 + r1) + (r2 + r3) per value, the same sum in the same
// order as wave_sum63's (r3 + r2) + (r1 + r0).  12 instructions for both
// totals, against 20 for two wave_sum63.
__device__ __forceinline__ float row_sum(float v)
{
    v += EMU_DPP(v, 0xb1, 0xf);  // quad_perm [1,0,3,2]
    v += EMU_DPP(v, 0x4e, 0xf);  // quad_perm [2,3,0,1]
    v += EMU_DPP(v, 0x141, 0xf); // row_half_mirror
    v += EMU_DPP(v, 0x140, 0xf); // row_mirror: every lane holds its row's sum
    return v;
}

__device__ __forceinline__ float pair_sum(float a, float b)
{
    a = row_sum(a);
    b = row_sum(b);
    emu_swap_halves<16>(a, b); // rows: a = [a0 b0 a2 b2], b = [a1 b1 a3 b3]
    const float v = a + b;
    float x = v, y = v;
    emu_swap_halves<32>(x, y);
    return x + y;
}

// The same for one value: its total in every lane.
__device__ __forceinline__ float wave_total(float v)
{
    v = row_sum(v);
    float x = v, y = v;
    emu_swap_halves<16>(x, y);
    v = x + y;
    x = v;
    y = v;
    emu_swap_halves<32>(x, y);
    return x + y;
}

__device__ __forceinline__ float lane_value(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// v with lane l's value replaced by the wave-uniform s.
__device__ __forceinline__ float set_lane(float v, float s, int l)
{
    return (int)__lane_id() == l ? s : v;
}

// Q6_K (210-byte blocks of 256: ql[128], qh[64], int8 scales[16], f16 d).
// Column 128h + 32j + 16m + i of a block has code
//   (ql[64h + 32(j&1) + 16m + i] >> 4(j>>1) & 15) | (qh[32h + 16m + i] >> 2j & 3) << 4
// and weight d * scales[8h + 2j + m] * (code - 32).  Unit (blk, h, m) owns
// the four sub-blocks j = 0..3.
struct LimbQ6K {
    struct Raw {
        uint4 a, b, q; // ql[64h+16m..], ql[64h+32+16m..], qh[32h+16m..]
        uint2 sc;      // scales[8h .. 8h+8]
        uint32_t d;
    };
    __device__ static __forceinline__ void load(const uint8_t *row, int unit, Raw &r)
    {
        const uint32_t blk = (uint32_t)unit >> 2, h = ((uint32_t)unit >> 1) & 1u, m = (uint32_t)unit & 1u;
        const uint32_t off = blk * 210u;
        r.a = ld16(row + (off + 64u * h + 16u * m));
        r.b = ld16(row + (off + 64u * h + 32u + 16u * m));
        r.q = ld16(row + (off + 128u + 32u * h + 16u * m));
        r.sc = ld8(row + (off + 192u + 8u * h));
        r.d = ld2(row + (off + 208u));
    }
    __device__ static __forceinline__ int sub_block(int unit, int j)
    {
        return 16 * (unit >> 2) + 8 * ((unit >> 1) & 1) + 2 * j + (unit & 1);
    }
    // The codes are biased by 32: start each sub-block's last chain at -32 * sum.
    __device__ static __forceinline__ int bias(int sum) { return (int)(0u - 32u * (uint32_t)sum); }
    __device__ static __forceinline__ uint32_t code(const Raw &r, int j, int i)
    {
        const uint32_t A = (uint32_t)comp(r.a, i), B = (uint32_t)comp(r.b, i), Q = (uint32_t)comp(r.q, i);
        switch (j) {
        case 0: return (A & 0x0f0f0f0fu) | ((Q << 4) & 0x30303030u);
        case 1: return (B & 0x0f0f0f0fu) | ((Q << 2) & 0x30303030u);
        case 2: return ((A >> 4) & 0x0f0f0f0fu) | (Q & 0x30303030u);
        default: return ((B >> 4) & 0x0f0f0f0fu) | ((Q >> 2) & 0x30303030u);
        }
    }
    __device__ static __forceinline__ float dot(const Raw &r, const Limbs &L, int unit)
    {
        return q6k_dot<LimbQ6K>(r, L, unit);
    }
    // The staged dot's pieces: sub-block j's chains combined into
    // t = 16384 s0 + 128 s1 + s2 (as in q6k_dot), and its float factor.
    template <class CODES> __device__ static __forceinline__ int q6k_chain(const Raw &r, const Limbs &L, int j)
    {
        // Each chain starts with the three-operand form, its accumulator
        // (0, or the bias term, which later rows reuse) read in place: the
        // accumulate-in-place form the compiler picks would need a register
        // copy of it first.
        int a0, a1, a2;
        {
            const int q = (int)CODES::code(r, j, 0);
            asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(a0) : "v"(q), "v"(comp(L.l[j][0], 0)));
            asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(a1) : "v"(q), "v"(comp(L.l[j][1], 0)));
            asm("v_dot4_i32_i8 %0, %1, %2, %3" : "=v"(a2) : "v"(q), "v"(comp(L.l[j][2], 0)), "v"(L.c[j]));
        }
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            const int q = (int)CODES::code(r, j, i);
            a0 = __builtin_amdgcn_sdot4(q, comp(L.l[j][0], i), a0, false);
            a1 = __builtin_amdgcn_sdot4(q, comp(L.l[j][1], i), a1, false);
            a2 = __builtin_amdgcn_sdot4(q, comp(L.l[j][2], i), a2, false);
        }
        // |result| < 2^31 by the limb bounds; unsigned arithmetic keeps the
        // intermediate sums well defined.
        return (int)(((uint32_t)a0 << 14) + ((uint32_t)a1 << 7) + (uint32_t)a2);
    }
    // Sub-block j's float factor: d folded in before t, since t * s alone
    // (a sum of codes times x) can overflow where the dot itself does not.
    __device__ static __forceinline__ float q6k_factor(const Raw &r, const Limbs &L, int unit, int j, float d)
    {
        const uint32_t sw = j < 2 ? r.sc.x : r.sc.y;
        const float sc = (float)(int)__builtin_amdgcn_sbfe(sw, 8u * (uint32_t)((unit & 1) + 2 * (j & 1)), 8u);
        return (sc * d) * L.s[j];
    }
    // The limb dots of one unit: per sub-block three v_dot4_i32_i8 chains
    // over its four code words, combined exactly, then one float step.
    template <class CODES>
    __device__ static __forceinline__ float q6k_dot(const Raw &r, const Limbs &L, int unit)
    {
        const int m = unit & 1;
        const float d = h2f((uint16_t)r.d);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // Each chain starts with the three-operand form, its accumulator
            // (0, or the bias term, which later rows reuse) read in place:
            // the accumulate-in-place form the compiler picks would need a
            // register copy of it first.
            int a0, a1, a2;
            {
                const int q = (int)CODES::code(r, j, 0);
                asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(a0) : "v"(q), "v"(comp(L.l[j][0], 0)));
                asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(a1) : "v"(q), "v"(comp(L.l[j][1], 0)));
                asm("v_dot4_i32_i8 %0, %1, %2, %3" : "=v"(a2) : "v"(q), "v"(comp(L.l[j][2], 0)), "v"(L.c[j]));
            }
#pragma unroll
            for (int i = 1; i < 4; ++i) {
                const int q = (int)CODES::code(r, j, i);
                a0 = __builtin_amdgcn_sdot4(q, comp(L.l[j][0], i), a0, false);
                a1 = __builtin_amdgcn_sdot4(q, comp(L.l[j][1], i), a1, false);
                a2 = __builtin_amdgcn_sdot4(q, comp(L.l[j][2], i), a2, false);
            }
            // |result| < 2^31 by the limb bounds; unsigned arithmetic keeps the
            // intermediate sums well defined.
            const int t = (int)(((uint32_t)a0 << 14) + ((uint32_t)a1 << 7) + (uint32_t)a2);
            const uint32_t sw = j < 2 ? r.sc.x : r.sc.y;
            const float sc = (float)(int)__builtin_amdgcn_sbfe(sw, 8u * (uint32_t)(m + 2 * (j & 1)), 8u);
            // d folded in before t: t * s alone (a sum of codes times x) can
            // overflow where the dot itself does not.
            acc = __builtin_fmaf((float)t, (sc * d) * L.s[j], acc);
        }
        return acc;
    }
};

// The same units read from the lane-major layout: a 4096-column stretch of a
// row (16 blocks) is one chunk, so each load instruction of a wavefront
// covers one contiguous kilobyte (three of them), then 256 bytes of scales
// and 32 of d, all with the non-temporal hint (a step reads each weight byte
// once; measured 3-6% faster over the batch-1 decode step than plain loads).  The three code words of a column quad are re-packed so that
// three of its four sub-blocks' codes are one mask each: byte b of
//   W0 = c0 | (c3 & 3) << 6,  W1 = c1 | (c3 >> 2 & 3) << 6,
//   W2 = c2 | (c3 >> 4) << 6
// for the 6-bit codes c0..c3 of sub-blocks j = 0..3 (the GGUF form takes
// three or four operations per code word).  Same codes, so the arithmetic
// and its results are identical to the GGUF-order kernel's.
// An ordering point for the staged dot: t (a finished chain) is computed
// before it, no memory access crosses it, and w reads as written by it.
__device__ __forceinline__ void pin_word(uint4 &w, int t)
{
    asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w) : "v"(t) : "memory");
}

struct LimbQ6KLM : LimbQ6K {
    __device__ static __forceinline__ uint32_t code(const Raw &r, int j, int i)
    {
        const uint32_t W0 = (uint32_t)comp(r.a, i), W1 = (uint32_t)comp(r.b, i), W2 = (uint32_t)comp(r.q, i);
        switch (j) {
        case 0: return W0 & 0x3f3f3f3fu;
        case 1: return W1 & 0x3f3f3f3fu;
        case 2: return W2 & 0x3f3f3f3fu;
        default: return ((W0 >> 6) & 0x03030303u) | ((W1 >> 4) & 0x0c0c0c0cu) | ((W2 >> 2) & 0x30303030u);
        }
    }
    __device__ static __forceinline__ float dot(const Raw &r, const Limbs &L, int unit)
    {
        return q6k_dot<LimbQ6KLM>(r, L, unit);
    }
    __device__ static __forceinline__ void load(const uint8_t *row, int unit, Raw &r)
    {
        const uint32_t L = (uint32_t)unit & 63u;
        const uint8_t *c = row + 3360u * ((uint32_t)unit >> 6);
        r.a = ldnt16(c + 16u * L);
        r.b = ldnt16(c + 1024u + 16u * L);
        r.q = ldnt16(c + 2048u + 16u * L);
        r.sc = ldnt8(c + 3072u + 8u * (L >> 1));
        r.d = ldnt2(c + 3328u + 2u * (L >> 2));
    }
    // The dot with the next row's loads (next: that row's start) staged
    // into the same registers as each code word's last use passes.  Sub-blocks 0,
    // 1 and 2 read one word each (a, b, q) and sub-block 3 reads all three,
    // so sub-block 3's chains go first, then 0 and a's refill, 1 and b's, 2
    // and q's with the scales and d (the float factors are formed before).
    // The float steps then run in sub-block order, as in q6k_dot: the same
    // bits, with the next row's first loads out about three quarters of the
    // dots earlier than a refill after the whole dot.
    static constexpr bool kStaged = true;
    __device__ static __forceinline__ float dot_staged(Raw &r, const Limbs &L, int unit, const uint8_t *next)
    {
        const float d = h2f((uint16_t)r.d);
        float f[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) f[j] = q6k_factor(r, L, unit, j, d);
        const uint32_t Lu = (uint32_t)unit & 63u;
        const uint8_t *c = next + 3360u * ((uint32_t)unit >> 6);
        int t[4];
        // Each chain is pinned before the refill that follows it ("memory":
        // no load moves above the pin), and the pin nominally rewrites the
        // word the next chain reads, so no chain moves above it either: a
        // word's old and new values are never both live.
        t[3] = q6k_chain<LimbQ6KLM>(r, L, 3);
        pin_word(r.a, t[3]);
        t[0] = q6k_chain<LimbQ6KLM>(r, L, 0);
        pin_word(r.b, t[0]);
        r.a = ldnt16(c + 16u * Lu);
        t[1] = q6k_chain<LimbQ6KLM>(r, L, 1);
        pin_word(r.q, t[1]);
        r.b = ldnt16(c + 1024u + 16u * Lu);
        t[2] = q6k_chain<LimbQ6KLM>(r, L, 2);
        asm volatile("" ::"v"(t[2]), "v"(f[0]), "v"(f[1]), "v"(f[2]), "v"(f[3]) : "memory");
        r.q = ldnt16(c + 2048u + 16u * Lu);
        r.sc = ldnt8(c + 3072u + 8u * (Lu >> 1));
        r.d = ldnt2(c + 3328u + 2u * (Lu >> 2));
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_fmaf((float)t[j], f[j], acc);
        return acc;
    }
};

// Whether a format stages the next row's loads inside its dot, and the call
// to that dot (named only where a format has it).
template <class LF, class = void> struct StagedDot {
    static constexpr bool value = false;
};
template <class LF> struct StagedDot<LF, decltype((void)LF::kStaged)> {
    static constexpr bool value = LF::kStaged;
};
template <bool STAGED> struct StagedCall {
    template <class LF, class R> __device__ static float dot(R &, const Limbs &, int, const uint8_t *) { return 0.0f; }
};
template <> struct StagedCall<true> {
    template <class LF, class R>
    __device__ static __forceinline__ float dot(R &r, const Limbs &L, int unit, const uint8_t *next)
    {
        return LF::dot_staged(r, L, unit, next);
    }
};

template <int S, int WV = 0> struct LimbShape {
    static constexpr int W = WV ? WV : S == 1 ? 8 : 4 * S; // wavefronts per workgroup
    static constexpr int RG = W / S;             // row-groups per workgroup
    static constexpr int T = EMU_WAVE * W;
    static constexpr int NSB = 256 * S;          // 16-column sub-blocks per row
    static constexpr int G = T / NSB;            // prologue threads per sub-block
    static constexpr int CPT = 16 / G;           // prologue columns per thread
    static_assert(G * NSB == T && (G == 1 || G == 2 || G == 4), "prologue mapping");
};

// The low bytes of four words, in order, as one word: three v_perm_b32
// (selector bytes 0..3 pick the second operand's bytes, 4..7 the first's,
// 0x0c gives zero).
__device__ __forceinline__ uint32_t pack_low_bytes(const uint32_t (&w)[4])
{
    const uint32_t lo = __builtin_amdgcn_perm(w[1], w[0], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(w[3], w[2], 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Split this thread's CPT columns (already normalised) into limbs; the G
// threads of a sub-block are neighbouring lanes.
template <int G, int CPT>
__device__ __forceinline__ void make_limbs(const float (&xv)[CPT], LimbRec *rec, int sb, int part)
{
    float amax = 0.0f;
    int bad = 0; // an inf or NaN in the sub-block (fmaxf alone would drop a NaN)
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        amax = fmaxf(amax, fabsf(xv[k]));
        bad |= !(fabsf(xv[k]) <= 3.402823466e38f);
    }
    // The G threads' exchanges by DPP (no LDS round trips); a non-finite
    // value enters the max as +inf, which every max keeps.
    amax = bad ? __int_as_float(0x7f800000) : amax;
    if (G >= 2) amax = fmaxf(amax, emu_xor_lane<1>(amax));
    if (G >= 4) amax = fmaxf(amax, emu_xor_lane<2>(amax));
    const bool finite = amax <= 3.402823466e38f;
    int e = 0;
    (void)frexpf(finite ? amax : 0.0f, &e);      // amax < 2^e, so |x| * 2^(6-e) < 64
    // Digits by the float recurrence f0 = rint(v), r1 = (v - f0) * 128,
    // f1 = rint(r1), f2 = rint((r1 - f1) * 128), each rint as an add of
    // 1.5 * 2^23 (whose ulp is 1, so the add rounds to the nearest integer,
    // ties to even, for |value| < 2^22) that leaves the integer in the sum's
    // low mantissa bits: its low byte is the limb's int8, no convert needed.
    // The limbs' sum, sum_c (16384 L0 + 128 L1 + L2), comes from the packed
    // bytes by dot products with ones.
    constexpr float kRound = 12582912.0f;
    uint32_t p0[CPT / 4], p1[CPT / 4], p2[CPT / 4];
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int q = 0; q < CPT / 4; ++q) {
        uint32_t t[3][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // exact; in a sub-block holding an inf or NaN the digits are
            // garbage, and the NaN scale makes every dot with it NaN anyway
            const float v = ldexpf(xv[4 * q + u], 6 - e);
            const float t0 = v + kRound;
            const float r1 = (v - (t0 - kRound)) * 128.0f; // exact
            const float t1 = r1 + kRound;
            const float t2 = (r1 - (t1 - kRound)) * 128.0f + kRound;
            t[0][u] = __float_as_uint(t0);
            t[1][u] = __float_as_uint(t1);
            t[2][u] = __float_as_uint(t2);
        }
        const uint32_t b0 = pack_low_bytes(t[0]), b1 = pack_low_bytes(t[1]), b2 = pack_low_bytes(t[2]);
        p0[q] = b0;
        p1[q] = b1;
        p2[q] = b2;
        s0 = __builtin_amdgcn_sdot4((int)b0, 0x01010101, s0, false);
        s1 = __builtin_amdgcn_sdot4((int)b1, 0x01010101, s1, false);
        s2 = __builtin_amdgcn_sdot4((int)b2, 0x01010101, s2, false);
    }
    int sum = s0 * 16384 + s1 * 128 + s2;
    if (G >= 2) sum += __float_as_int(emu_xor_lane<1>(__int_as_float(sum)));
    if (G >= 4) sum += __float_as_int(emu_xor_lane<2>(__int_as_float(sum)));
    uint32_t *d0 = reinterpret_cast<uint32_t *>(&rec[sb].l0);
    uint32_t *d1 = reinterpret_cast<uint32_t *>(&rec[sb].l1);
    uint32_t *d2 = reinterpret_cast<uint32_t *>(&rec[sb].l2);
#pragma unroll
    for (int k = 0; k < CPT / 4; ++k) {
        d0[part * (CPT / 4) + k] = p0[k];
        d1[part * (CPT / 4) + k] = p1[k];
        d2[part * (CPT / 4) + k] = p2[k];
    }
    if (part == 0) {
        rec[sb].s = finite ? ldexpf(1.0f, e - 20) : __int_as_float(0x7fc00000);
        rec[sb].sum = sum;
    }
}

template <class LF, int S, int D, bool DUAL, bool NORM, bool ACC, int WV>
__global__ __launch_bounds__((EMU_WAVE * LimbShape<S, WV>::W)) void qmv_limb_kernel(QmvArgs a, int rounds)
{
    using SH = LimbShape<S, WV>;
    constexpr int NR = DUAL ? 2 : 1;
    __shared__ LimbRec rec[SH::NSB];
    __shared__ float red[SH::W];
    __shared__ float part[2][SH::RG][S][D][NR];

    const int tid = threadIdx.x, lane = tid & (EMU_WAVE - 1), wv = tid / EMU_WAVE;
    const int rg = wv / S, sl = wv % S;
    const int grg = blockIdx.x * SH::RG + rg, total_rg = gridDim.x * SH::RG;
    const int unit = sl * EMU_WAVE + lane;

    struct Slot {
        typename LF::Raw raw[NR];
        float resid;
    };
    auto row_of = [&](int k, int d) {
        const int row = grg + (k * D + d) * total_rg;
        return __builtin_amdgcn_readfirstlane(row < a.rows ? row : a.rows - 1);
    };
    auto load_slot = [&](int k, int d, Slot &s) {
        const int row = row_of(k, d);
#pragma unroll
        for (int n = 0; n < NR; ++n) LF::load((n ? a.w_up : a.w) + (size_t)row * a.row_bytes, unit, s.raw[n]);
        if (ACC) s.resid = a.y[row];
    };

    // The activation (and gain) loads go out first, then the first rows'
    // weight loads, and the prologue's arithmetic hides under the latter:
    // loads complete in issue order, so a prologue value loaded after the
    // weights would wait for their HBM round trip.
    Slot buf[D];
    {
        const int sb = tid / SH::G, pi = tid % SH::G;
        const int c0 = 16 * sb + SH::CPT * pi;
        float xv[SH::CPT], gv[SH::CPT];
#pragma unroll
        for (int k = 0; k < SH::CPT; k += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(a.x + c0 + k);
            xv[k] = v.x; xv[k + 1] = v.y; xv[k + 2] = v.z; xv[k + 3] = v.w;
            if (NORM) {
                const float4 g = *reinterpret_cast<const float4 *>(a.gain + c0 + k);
                gv[k] = g.x; gv[k + 1] = g.y; gv[k + 2] = g.z; gv[k + 3] = g.w;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < D; ++d) load_slot(0, d, buf[d]);
        __builtin_amdgcn_sched_barrier(0);
        if (NORM) {
            // The limbs are of x * gain and the RMS factor multiplies each
            // row's dot, so the row's sum of squares is needed only after
            // the limb records' barrier, not before the limbs: one barrier.
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < SH::CPT; ++k) ss = __builtin_fmaf(xv[k], xv[k], ss);
            ss = wave_sum63(ss);
            if (lane == EMU_WAVE - 1) red[wv] = ss;
#pragma unroll
            for (int k = 0; k < SH::CPT; ++k) xv[k] = __fmul_rn(xv[k], gv[k]);
        }
        make_limbs<SH::G, SH::CPT>(xv, rec, sb, pi);
    }
    __syncthreads();
    float rscale = 1.0f;
    if (NORM) {
        float tot = 0.0f;
#pragma unroll
        for (int k = 0; k < SH::W; ++k) tot += red[k];
        rscale = 1.0f / sqrtf(tot / (float)a.cols + a.eps);
    }
    Limbs L;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const LimbRec &r = rec[LF::sub_block(unit, j)];
        L.l[j][0] = r.l0;
        L.l[j][1] = r.l1;
        L.l[j][2] = r.l2;
        L.s[j] = r.s;
        L.c[j] = LF::bias(r.sum);
    }

    uint64_t best = 0;
    auto finish = [&](int row, const float (&p)[NR], float resid) {
        float val = NORM ? __fmul_rn(p[0], rscale) : p[0];
        if (DUAL) val = emu_glu(val, NORM ? __fmul_rn(p[1], rscale) : p[1], a.act);
        val = emu_out_epi(val, a.out_div, a.softcap);
        if (row < a.rows) {
            a.y[row] = ACC ? emu_resid_add(resid, val, a.acc_scale) : val;
            if (a.keys) {
                const uint64_t key = emu_select_key(val, (uint32_t)row, a.tie_last);
                best = key > best ? key : best;
            }
        }
    };

    // A round's NV = D * NR dot sums, in (d, n) order, are reduced two at a
    // time (pair i: value 2i in lane 0, value 2i + 1 in lane 16).
    // With one wavefront per row (S == 1) the rows' epilogues are deferred:
    // lane j of dv / dr holds the sums and residual of the j-th row of a
    // window of 64, and the window's rows are finished together, one per
    // lane, so the activation and store run once per window, not per row.
    constexpr int NV = D * NR, NP = (NV + 1) / 2;
    float dv[NR], dr = 0.0f;
#pragma unroll
    for (int n = 0; n < NR; ++n) dv[n] = 0.0f;
    // One round: the D slots' dots (with the next round's loads staged into
    // them when `staged`), their reductions and the epilogue.  The gate|up
    // pair of a format with a staged dot runs every round but the last
    // staged, so the staged loads need no branch around them and each round
    // waits only for the loads of the row it starts on (gate|up 16.7 ->
    // 16.4 us back to back; the single matrices measured no better staged).
    auto round = [&](int k, auto staged) {
        float resid[D]; // this round's residuals (the slots are refilled below)
        float v[NV];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if constexpr (decltype(staged)::value) {
                // the next round's row loads go out inside the dots (every
                // round but the last, which the caller runs unstaged)
                const int nrow = row_of(k + 1, d);
#pragma unroll
                for (int n = 0; n < NR; ++n)
                    v[d * NR + n] = StagedCall<StagedDot<LF>::value>::template dot<LF>(
                        buf[d].raw[n], L, unit, (n ? a.w_up : a.w) + (size_t)nrow * a.row_bytes);
                resid[d] = ACC ? buf[d].resid : 0.0f;
                if (ACC) buf[d].resid = a.y[nrow];
            } else {
#pragma unroll
                for (int n = 0; n < NR; ++n) {
                    v[d * NR + n] = LF::dot(buf[d].raw[n], L, unit);
                    // The dot is finished here, above the refill: sunk below
                    // it (its sums are not used before the reduction), it
                    // would keep the slot's old words alive beside the new
                    // ones, a register copy per word and a wavefront per
                    // SIMD lost.
                    asm volatile("" ::"v"(v[d * NR + n]));
                }
                resid[d] = ACC ? buf[d].resid : 0.0f;
                if (k + 1 < rounds) load_slot(k + 1, d, buf[d]);
            }
        }
        float tot[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) tot[i] = 2 * i + 1 < NV ? pair_sum(v[2 * i], v[2 * i + 1]) : wave_total(v[2 * i]);
        if constexpr (S == 1) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int slot = k * D + d, pos = slot & (EMU_WAVE - 1);
#pragma unroll
                for (int n = 0; n < NR; ++n) {
                    const int i = d * NR + n;
                    dv[n] = set_lane(dv[n], lane_value(tot[i / 2], (i & 1) * 16), pos);
                }
                if (ACC) dr = set_lane(dr, lane_value(resid[d], 0), pos);
                if (pos == EMU_WAVE - 1 || slot == rounds * D - 1) {
                    if (lane <= pos) finish(grg + (slot - pos + lane) * total_rg, dv, dr);
                }
            }
        } else {
            // Double-buffered by round parity: one barrier per round suffices.
            float *pk = &part[k & 1][rg][sl][0][0];
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int idx = 2 * i + ((lane >> 4) & 1);
                if ((lane & 47) == 0 && idx < NV) pk[idx] = tot[i]; // lanes 0 and 16
            }
            __syncthreads();
            if (sl == 0 && lane < D) { // lane d finishes the round's row d
                const int d = lane;
                float p[NR];
#pragma unroll
                for (int n = 0; n < NR; ++n) {
                    float t = part[k & 1][rg][0][d][n];
#pragma unroll
                    for (int s2 = 1; s2 < S; ++s2) t += part[k & 1][rg][s2][d][n];
                    p[n] = t;
                }
                float r = resid[0];
#pragma unroll
                for (int e = 1; e < D; ++e) r = d == e ? resid[e] : r;
                finish(grg + (k * D + d) * total_rg, p, r);
            }
        }
    };
    if constexpr (StagedDot<LF>::value && S == 1 && DUAL) {
        for (int k = 0; k + 1 < rounds; ++k) round(k, std::true_type{});
        round(rounds - 1, std::false_type{});
    } else {
        (void)round;
        for (int k = 0; k < rounds; ++k) {
            float resid[D]; // this round's residuals (the slots are refilled below)
            float v[NV];
#pragma unroll
            for (int d = 0; d < D; ++d) {
#pragma unroll
                for (int n = 0; n < NR; ++n) {
                    v[d * NR + n] = LF::dot(buf[d].raw[n], L, unit);
                    // The dot is finished here, above the refill: sunk below it
                    // (its sums are not used before the reduction), it would
                    // keep the slot's old words alive beside the new ones, a
                    // register copy per word and a wavefront per SIMD lost.
                    asm volatile("" ::"v"(v[d * NR + n]));
                }
                resid[d] = ACC ? buf[d].resid : 0.0f;
                if (k + 1 < rounds) load_slot(k + 1, d, buf[d]);
            }
            float tot[NP];
#pragma unroll
            for (int i = 0; i < NP; ++i) tot[i] = 2 * i + 1 < NV ? pair_sum(v[2 * i], v[2 * i + 1]) : wave_total(v[2 * i]);
            if constexpr (S == 1) {
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    const int slot = k * D + d, pos = slot & (EMU_WAVE - 1);
#pragma unroll
                    for (int n = 0; n < NR; ++n) {
                        const int i = d * NR + n;
                        dv[n] = set_lane(dv[n], lane_value(tot[i / 2], (i & 1) * 16), pos);
                    }
                    if (ACC) dr = set_lane(dr, lane_value(resid[d], 0), pos);
                    if (pos == EMU_WAVE - 1 || slot == rounds * D - 1) {
                        if (lane <= pos) finish(grg + (slot - pos + lane) * total_rg, dv, dr);
                    }
                }
            } else {
                // Double-buffered by round parity: one barrier per round suffices.
                float *pk = &part[k & 1][rg][sl][0][0];
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int idx = 2 * i + ((lane >> 4) & 1);
                    if ((lane & 47) == 0 && idx < NV) pk[idx] = tot[i]; // lanes 0 and 16
                }
                __syncthreads();
                if (sl == 0 && lane < D) { // lane d finishes the round's row d
                    const int d = lane;
                    float p[NR];
#pragma unroll
                    for (int n = 0; n < NR; ++n) {
                        float t = part[k & 1][rg][0][d][n];
#pragma unroll
                        for (int s2 = 1; s2 < S; ++s2) t += part[k & 1][rg][s2][d][n];
                        p[n] = t;
                    }
                    float r = resid[0];
#pragma unroll
                    for (int e = 1; e < D; ++e) r = d == e ? resid[e] : r;
                    finish(grg + (k * D + d) * total_rg, p, r);
                }
            }
        }
    }
    if (a.keys) {
        best = emu_wave_max_u64(best);
        if (sl == 0 && lane == 0) a.keys[grg] = best;
    }
}

// Rows in flight per wavefront and workgroups per CU, measured per shape on
// weights streamed from HBM: one row in flight with two workgroups per CU for
// the gate|up pair (four waves per SIMD hide the latency better than deeper
// prefetch in fewer waves: 18.0 us against 21.2 us with two rows and one
// workgroup), one row and one workgroup for the other 4096-column matvecs
// (q|k|v 7.6 against 8.7 us, o 6.2 against 6.5, the 151936-row output 92.8
// against 95.8), and two rows for the 12288-column down projection.
template <int S, bool DUAL> struct LimbTune {
    static constexpr int D = S == 1 ? 1 : 2;
    static constexpr int PER_CU = DUAL ? 2 : 1;
};

template <class LF, int S, int D, bool DUAL, bool NORM, bool ACC>
void launch_limb_d(emu_ctx *ctx, const QmvArgs &a, int blocks)
{
    using SH = LimbShape<S>;
    const int total_rg = blocks * SH::RG;
    const int rounds = (a.rows + total_rg * D - 1) / (total_rg * D);
    hipLaunchKernelGGL((qmv_limb_kernel<LF, S, D, DUAL, NORM, ACC, 0>), dim3(blocks), dim3(SH::T), 0, ctx->stream,
                       a, rounds);
}

template <class LF, int S, bool DUAL, bool NORM, bool ACC>
void launch_limb_cfg(emu_ctx *ctx, const QmvArgs &a, int blocks)
{
    launch_limb_d<LF, S, LimbTune<S, DUAL>::D, DUAL, NORM, ACC>(ctx, a, blocks);
}

template <class LF, int S>
int launch_limb_s(emu_ctx *ctx, const QmvArgs &a, int *key_slots)
{
    const bool dual = a.w_up != nullptr, norm = a.gain != nullptr, acc = a.accumulate != 0;
    if (dual && acc) return EMU_E_ARG; // the fused entry point never asks for this
    const int cus = ctx->cus > 0 ? ctx->cus : 256;
    const int per_cu = dual ? LimbTune<S, true>::PER_CU : LimbTune<S, false>::PER_CU;
    // No more row-groups than rows (a key slot per row-group must fit the
    // caller's key stride, which holds rows + 8).
    const int need = (a.rows + LimbShape<S>::RG - 1) / LimbShape<S>::RG;
    const int blocks = cus * per_cu < need ? cus * per_cu : need;
    // key slots the launch writes: one per row-group of the grid it takes
    const int slots = blocks * LimbShape<S>::RG;
    if (a.keys && slots > a.key_stride) return EMU_E_CONFIG;
    if (dual) {
        if (norm) launch_limb_cfg<LF, S, true, true, false>(ctx, a, blocks);
        else launch_limb_cfg<LF, S, true, false, false>(ctx, a, blocks);
    } else if (acc) {
        if (norm) launch_limb_cfg<LF, S, false, true, true>(ctx, a, blocks);
        else launch_limb_cfg<LF, S, false, false, true>(ctx, a, blocks);
    } else {
        if (norm) launch_limb_cfg<LF, S, false, true, false>(ctx, a, blocks);
        else launch_limb_cfg<LF, S, false, false, false>(ctx, a, blocks);
    }
    EMU_LAUNCH_CHECK(ctx);
    if (key_slots) *key_slots = slots;
    return EMU_OK;
}

} // namespace

bool emu_limb_supports(int encoding, int cols)
{
    if (encoding != EMU_ENC_Q6_K) return false;
    return cols == 4096 || cols == 12288;
}

int emu_launch_limb(emu_ctx *ctx, int encoding, const QmvArgs &a, int *key_slots)
{
    if (!emu_limb_supports(encoding, a.cols)) return EMU_E_UNSUPPORTED;
    if (a.rows <= 0) return EMU_E_ARG;
    switch (a.cols) {
    case 4096:
        return a.lane_major ? launch_limb_s<LimbQ6KLM, 1>(ctx, a, key_slots)
                            : launch_limb_s<LimbQ6K, 1>(ctx, a, key_slots);
    case 12288:
        return a.lane_major ? launch_limb_s<LimbQ6KLM, 3>(ctx, a, key_slots)
                            : launch_limb_s<LimbQ6K, 3>(ctx, a, key_slots);
    default: return EMU_E_UNSUPPORTED;
    }
}

namespace {

// Byte offset, inside a chunk of n blocks in GGUF order, of the byte that the
// lane-major layout puts at offset o.
__device__ __forceinline__ uint32_t lane_major_source(uint32_t o, uint32_t n)
{
    if (o < 192u * n) {
        const uint32_t region = o / (64u * n), r = o % (64u * n);
        const uint32_t L = r >> 4, i = r & 15u;
        const uint32_t j = L >> 2, h = (L >> 1) & 1u, m = L & 1u;
        if (region == 0) return 210u * j + 64u * h + 16u * m + i;
        if (region == 1) return 210u * j + 64u * h + 32u + 16u * m + i;
        return 210u * j + 128u + 32u * h + 16u * m + i;
    }
    if (o < 208u * n) {
        const uint32_t r = o - 192u * n, k = r >> 3, t = r & 7u;
        return 210u * (k >> 1) + 192u + 8u * (k & 1u) + t;
    }
    const uint32_t r = o - 208u * n;
    return 210u * (r >> 1) + 208u + (r & 1u);
}

// One workgroup per chunk (grid-stride): the chunk's bytes come into LDS,
// and each destination byte is gathered from there.
__global__ __launch_bounds__(256) void lane_major_kernel(const uint8_t *src, size_t nblocks, uint8_t *dst)
{
    __shared__ uint8_t in[16 * 210];
    const size_t chunks = (nblocks + 15) / 16;
    for (size_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const size_t b0 = 16 * c;
        const uint32_t n = (uint32_t)(nblocks - b0 < 16 ? nblocks - b0 : 16);
        const uint8_t *s = src + 210 * b0;
        uint8_t *d = dst + 210 * b0;
        for (uint32_t o = threadIdx.x; o < 210u * n; o += 256u) in[o] = s[o];
        __syncthreads();
        for (uint32_t o = threadIdx.x; o < 210u * n; o += 256u) {
            uint8_t v;
            if (o < 192u * n) { // a code byte: re-packed from its column's ql-low, ql-high and qh bytes
                const uint32_t r = o % (64u * n);
                const uint32_t A = in[lane_major_source(r, n)], B = in[lane_major_source(64u * n + r, n)],
                               Q = in[lane_major_source(128u * n + r, n)];
                const uint32_t region = o / (64u * n);
                v = (uint8_t)(region == 0   ? (A & 15u) | (Q & 3u) << 4 | (B >> 4 & 3u) << 6
                              : region == 1 ? (B & 15u) | (Q >> 2 & 3u) << 4 | (B >> 6) << 6
                                            : (A >> 4) | (Q & 0xf0u));
            } else {
                v = in[lane_major_source(o, n)];
            }
            d[o] = v;
        }
        __syncthreads();
    }
}

} // namespace

int emu_lane_major_q6k(emu_ctx *ctx, const uint8_t *src, size_t nblocks, uint8_t *dst)
{
    if (nblocks == 0) return EMU_OK;
    const size_t chunks = (nblocks + 15) / 16;
    const unsigned grid = (unsigned)(chunks < 65536 ? chunks : 65536);
    hipLaunchKernelGGL(lane_major_kernel, dim3(grid), dim3(256), 0, ctx->stream, src, nblocks, dst);
    EMU_LAUNCH_CHECK(ctx);
    return EMU_OK;
}

extern "C" int emu_weights_lane_major(emu_ctx *ctx, int encoding, const void *d_src, size_t len, void *d_dst)
{
    if (!ctx || (!d_src && len) || (!d_dst && len)) return EMU_E_ARG;
    if (encoding != EMU_ENC_Q6_K) return EMU_E_UNSUPPORTED;
    if (len % 210 != 0) return EMU_E_SHORT;
    const uint8_t *s = static_cast<const uint8_t *>(d_src);
    uint8_t *d = static_cast<uint8_t *>(d_dst);
    if (len && s < d + len && d < s + len) return EMU_E_ARG; // the permutation is not in place
    return emu_lane_major_q6k(ctx, s, len / 210, d);
}
