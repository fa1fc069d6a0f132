// internal.hpp -- shared host/device definitions of libemuhip.
//
// Quantized formats are read through one abstraction: a *unit* is the
// 32-weight slice of a GGUF block that one lane owns.  A unit is G groups of 8
// consecutive columns; for each group the lane holds 8 unsigned codes (two
// packed dwords), a multiplier and an addend, and weight i of the group is
//     w = fma(code_i, mul, add)
// which is exact: every format's weight is d*sc*q (exact in f32) minus an
// exact d_min*m term, so the single rounding of the fma is the single rounding
// the reference performs (components/cli/crates/spm-gguf/src/tensor.rs:103-210).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>
#include <type_traits>

#include "../../include/emuhip.h"

#define EMU_WAVE 64

struct emu_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t events[16] = {};
    int cus = 0;
    char arch[64] = {0};
    char last_error[256] = {0};
    void *mfma_ws = nullptr; // multi-token matvec workspace (mfma.hip), grown on demand
    size_t mfma_ws_bytes = 0;
    void *stage[2] = {};         // pinned host staging for file -> HBM uploads (files.hip)
    hipEvent_t stage_ev[2] = {}; // the copy out of each staging buffer
    size_t stage_bytes = 0;
};

// Per-device set-up of ops.hip's no-allocation scratch (the device address of
// its file-scope array on the context's device); called by emu_ctx_create.
int emu_ops_device_init(emu_ctx *ctx);

int emu_hip_fail(emu_ctx *ctx, hipError_t e, const char *what);

#define EMU_HIP(ctx, call)                                                   \
    do {                                                                     \
        hipError_t emu_e_ = (call);                                          \
        if (emu_e_ != hipSuccess) return emu_hip_fail((ctx), emu_e_, #call); \
    } while (0)

#define EMU_LAUNCH_CHECK(ctx) EMU_HIP(ctx, hipGetLastError())

// ---------------------------------------------------------------- device --

__device__ __forceinline__ uint2 ld8(const uint8_t *p)
{
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
__device__ __forceinline__ uint4 ld16(const uint8_t *p)
{
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
__device__ __forceinline__ uint32_t ld4(const uint8_t *p)
{
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
__device__ __forceinline__ uint16_t ld2(const uint8_t *p)
{
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

// Loads with the non-temporal hint, for weight bytes that a decode step reads
// once: their cache lines are marked for early eviction instead of displacing
// lines that are read again (activations, the KV cache, partial sums).  Like
// ld16, these compile to single dwordx4 (dwordx2, ushort) loads, which the
// hardware takes at any address.
__device__ __forceinline__ uint4 ldnt16(const uint8_t *p)
{
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldnt8(const uint8_t *p)
{
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint16_t ldnt2(const uint8_t *p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
}

// f16 -> f32 is exact (hardware conversion handles subnormal halves), the same
// value as f16_to_f32 of spm-gguf/src/tensor.rs:82-98.
__device__ __forceinline__ float h2f(uint16_t bits)
{
    return __half2float(__ushort_as_half(bits));
}

// A pointer every lane of the wavefront holds: read into scalar registers so
// memory instructions take it as their scalar base.
__device__ __forceinline__ const uint8_t *uniform_ptr(const uint8_t *p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const uint8_t *>(((uint64_t)hi << 32) | lo);
}

// Byte i of w as a float: the backend selects v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ float byte_f(uint32_t w, int i)
{
    return (float)((w >> (8 * i)) & 0xffu);
}

// Byte k (0..7) of an 8-byte pair.
__device__ __forceinline__ uint32_t byte_of(uint2 v, int k)
{
    uint32_t w = k < 4 ? v.x : v.y;
    return (w >> (8 * (k & 3))) & 0xffu;
}

// One decoded group: 8 unsigned codes (two packed dwords) and the group's
// multiplier / addend.  Weight i of the group is fma(code_i, mul, add).
struct Grp {
    uint32_t q0, q1;
    float mul, add;
};

// Weight i (0..7) of a group for the matvec: one fma, exact value.  For the
// biased formats (Q6_K, Q8_0) a zero weight comes out +0.0 where the
// reference's d*sc*(q-32) may give -0.0; the sign of a zero weight cannot
// change a dot product, so the matvec keeps the single instruction.
__device__ __forceinline__ float grp_weight(const Grp &g, int i)
{
    return __builtin_fmaf(byte_f(i < 4 ? g.q0 : g.q1, i & 3), g.mul, g.add);
}

// Weight i with the reference's exact bits, signed zeros included:
// Q6_K d*sc*(q-32) and Q8_0 d*i8 as (code - BIAS) * mul; Q5_K / Q2_K
// d*sc*q - dmin*m as one fma of the exact product and the exact min term.
template <int BIAS> __device__ __forceinline__ float grp_weight_exact(const Grp &g, int i)
{
    const float b = byte_f(i < 4 ? g.q0 : g.q1, i & 3);
    if (BIAS) return __fmul_rn(__fsub_rn(b, (float)BIAS), g.mul);
    return __builtin_fmaf(b, g.mul, g.add);
}

// Code i (0..7) of a group minus the format's bias: the signed integer the
// format multiplies by its sub-block scale.
template <int BIAS> __device__ __forceinline__ int grp_code(const Grp &g, int i)
{
    return (int)(((i < 4 ? g.q0 : g.q1) >> (8 * (i & 3))) & 0xffu) - BIAS;
}

// ---- Q6_K: 210-byte blocks, 256 weights (spm-gguf/src/tensor.rs:103-139) --
// Unit (h, l8): h = half (0/1), l8 = 0..3 picks l in [8*l8, 8*l8+8).
// Group j (0..3) covers elements 128h + 32j + 8*l8 + i with code
//   j0: ql[l] & 15 | (qh[l] & 3) << 4        j1: ql[l+32] & 15 | (qh[l]>>2 & 3) << 4
//   j2: ql[l] >> 4 | (qh[l]>>4 & 3) << 4     j3: ql[l+32] >> 4 | (qh[l]>>6 & 3) << 4
// and scale sc[8h + l/16 + 2j]; weight = d*sc*(q-32) = fma(q, d*sc, -32*d*sc).
struct FmtQ6K {
    static constexpr int BB = 210, BE = 256, UPB = 8, G = 4, SUB = 16, BIAS = 32;
    struct Raw {
        uint2 a, b, c, s;
        uint32_t d;
    };
    // Block at base + off; unsigned 32-bit offsets let a wave-uniform base
    // stay in scalar registers.
    __device__ __forceinline__ static void load(const uint8_t *base, uint32_t off, int sub, Raw &r)
    {
        const uint32_t h = (uint32_t)sub >> 2, l8 = (uint32_t)sub & 3u;
        r.a = ld8(base + (off + 64u * h + 8u * l8));
        r.b = ld8(base + (off + 64u * h + 32u + 8u * l8));
        r.c = ld8(base + (off + 128u + 32u * h + 8u * l8));
        r.s = ld8(base + (off + 192u + 8u * h));
        r.d = ld2(base + (off + 208u));
    }
    __device__ __forceinline__ static void load(const uint8_t *blk, int sub, Raw &r) { load(blk, 0u, sub, r); }
    __device__ __forceinline__ static int col(int sub, int g)
    {
        return 128 * (sub >> 2) + 32 * g + 8 * (sub & 3);
    }
    __device__ __forceinline__ static Grp group(const Raw &r, int sub, int j)
    {
        const uint32_t lo = 0x0f0f0f0fu, hi = 0x30303030u;
        const uint2 src = (j & 1) ? r.b : r.a;
        const int ns = 4 * (j >> 1);
        const uint32_t h0 = j < 2 ? (r.c.x << (4 - 2 * j)) : (r.c.x >> (2 * j - 4));
        const uint32_t h1 = j < 2 ? (r.c.y << (4 - 2 * j)) : (r.c.y >> (2 * j - 4));
        Grp g;
        g.q0 = ((src.x >> ns) & lo) | (h0 & hi);
        g.q1 = ((src.y >> ns) & lo) | (h1 & hi);
        const float d = h2f((uint16_t)r.d);
        const float sc = (float)(int8_t)byte_of(r.s, ((sub & 3) >> 1) + 2 * j);
        g.mul = d * sc;
        g.add = -32.0f * g.mul;
        return g;
    }
};

// ---- Q8_0: 34-byte blocks, 32 weights (spm-gguf/src/tensor.rs:193-210) ----
// Unit (half): 16 weights, 2 groups of 8.  Codes are the int8 values with the
// sign bit flipped (i8 + 128 as u8); weight = d*i8 = fma(u8, d, -128*d).
struct FmtQ8_0 {
    static constexpr int BB = 34, BE = 32, UPB = 2, G = 2, SUB = 32, BIAS = 128;
    struct Raw {
        uint4 v;
        uint32_t d;
    };
    __device__ __forceinline__ static void load(const uint8_t *base, uint32_t off, int sub, Raw &r)
    {
        r.v = ld16(base + (off + 2u + 16u * (uint32_t)sub));
        r.d = ld2(base + off);
    }
    __device__ __forceinline__ static void load(const uint8_t *blk, int sub, Raw &r) { load(blk, 0u, sub, r); }
    __device__ __forceinline__ static int col(int sub, int g) { return 16 * sub + 8 * g; }
    __device__ __forceinline__ static Grp group(const Raw &r, int, int gi)
    {
        const uint32_t f = 0x80808080u;
        Grp g;
        g.q0 = (gi ? r.v.z : r.v.x) ^ f;
        g.q1 = (gi ? r.v.w : r.v.y) ^ f;
        g.mul = h2f((uint16_t)r.d);
        g.add = -128.0f * g.mul;
        return g;
    }
};

// ---- Q5_K: 176-byte blocks, 256 weights (spm-gguf/src/tensor.rs:144-188) --
// Element 64g + 32*half + l: low = qs[32g+l] nibble `half`, high bit
// qh[l] >> (2g+half), scale/min from scale_min_q5(2g+half).
// Unit (g, l16): l in [16*l16, 16*l16+16), both halves: 32 weights, groups
// gi = 2*half + k for k = 0,1 covering l = 16*l16 + 8k + i.
// weight = d*sc*q - dmin*m = fma(q, d*sc, -(dmin*m)), one rounding.
struct FmtQ5K {
    static constexpr int BB = 176, BE = 256, UPB = 8, G = 4, SUB = 32, BIAS = 0;
    struct Raw {
        uint4 qs, qh;
        uint32_t s0, s1, s2, dd;
    };
    __device__ __forceinline__ static void load(const uint8_t *base, uint32_t off, int sub, Raw &r)
    {
        const uint32_t g = (uint32_t)sub >> 1, l16 = (uint32_t)sub & 1u;
        r.qs = ld16(base + (off + 48u + 32u * g + 16u * l16));
        r.qh = ld16(base + (off + 16u + 16u * l16));
        r.dd = ld4(base + off);
        r.s0 = ld4(base + (off + 4u));
        r.s1 = ld4(base + (off + 8u));
        r.s2 = ld4(base + (off + 12u));
    }
    __device__ __forceinline__ static void load(const uint8_t *blk, int sub, Raw &r) { load(blk, 0u, sub, r); }
    __device__ __forceinline__ static int col(int sub, int gi)
    {
        return 64 * (sub >> 1) + 32 * (gi >> 1) + 16 * (sub & 1) + 8 * (gi & 1);
    }
    // scale_min_q5 (spm-gguf/src/tensor.rs:179-188) over the 12 packed bytes.
    __device__ __forceinline__ static void scale_min(const Raw &r, int index, uint32_t &sc,
                                                     uint32_t &m)
    {
        const uint32_t s[3] = {r.s0, r.s1, r.s2};
        auto byte = [&](int i) -> uint32_t { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; };
        if (index < 4) {
            sc = byte(index) & 63u;
            m = byte(index + 4) & 63u;
        } else {
            sc = (byte(index + 4) & 0x0fu) | ((byte(index - 4) >> 6) << 4);
            m = (byte(index + 4) >> 4) | ((byte(index) >> 6) << 4);
        }
    }
    __device__ __forceinline__ static Grp group(const Raw &r, int sub, int gi)
    {
        const int half = gi >> 1, k = gi & 1;
        const int index = 2 * (sub >> 1) + half;
        const uint32_t w0 = k ? r.qs.z : r.qs.x, w1 = k ? r.qs.w : r.qs.y;
        const uint32_t h0 = k ? r.qh.z : r.qh.x, h1 = k ? r.qh.w : r.qh.y;
        const uint32_t lo = 0x0f0f0f0fu;
        Grp g;
        g.q0 = (half ? ((w0 >> 4) & lo) : (w0 & lo)) | (((h0 >> index) & 0x01010101u) << 4);
        g.q1 = (half ? ((w1 >> 4) & lo) : (w1 & lo)) | (((h1 >> index) & 0x01010101u) << 4);
        uint32_t sc, m;
        scale_min(r, index, sc, m);
        g.mul = h2f((uint16_t)(r.dd & 0xffffu)) * (float)sc;
        g.add = -(h2f((uint16_t)(r.dd >> 16)) * (float)m);
        return g;
    }
};

// ---- Q2_K: 84-byte blocks, 256 weights (published GGML block_q2_K) --------
// Element 128N + 32j + 16s + l: code (qs[32N+16s+l] >> 2j) & 3, scale byte
// sc[8N+2j+s] (low nibble scale, high nibble min), d at 80, dmin at 82.
// Unit (N, s, l8): 8 bytes qs[32N+16s+8*l8 ..], group j = 0..3.
// weight = d*(sc&15)*code - dmin*(sc>>4) = fma(code, d*(sc&15), -(dmin*(sc>>4))).
struct FmtQ2K {
    static constexpr int BB = 84, BE = 256, UPB = 8, G = 4, SUB = 16, BIAS = 0;
    struct Raw {
        uint2 qs, sc;
        uint32_t dd;
    };
    __device__ __forceinline__ static void load(const uint8_t *base, uint32_t off, int sub, Raw &r)
    {
        const uint32_t N = (uint32_t)sub >> 2, s = ((uint32_t)sub >> 1) & 1u, l8 = (uint32_t)sub & 1u;
        r.qs = ld8(base + (off + 16u + 32u * N + 16u * s + 8u * l8));
        r.sc = ld8(base + (off + 8u * N));
        r.dd = ld4(base + (off + 80u));
    }
    __device__ __forceinline__ static void load(const uint8_t *blk, int sub, Raw &r) { load(blk, 0u, sub, r); }
    __device__ __forceinline__ static int col(int sub, int j)
    {
        return 128 * (sub >> 2) + 32 * j + 16 * ((sub >> 1) & 1) + 8 * (sub & 1);
    }
    __device__ __forceinline__ static Grp group(const Raw &r, int sub, int j)
    {
        Grp g;
        g.q0 = (r.qs.x >> (2 * j)) & 0x03030303u;
        g.q1 = (r.qs.y >> (2 * j)) & 0x03030303u;
        const uint32_t packed = byte_of(r.sc, 2 * j + ((sub >> 1) & 1));
        g.mul = h2f((uint16_t)(r.dd & 0xffffu)) * (float)(packed & 15u);
        g.add = -(h2f((uint16_t)(r.dd >> 16)) * (float)(packed >> 4));
        return g;
    }
};

// ------------------------------------------------------ greedy selection --
// Rust f32::total_cmp as an order-preserving unsigned key.
__device__ __forceinline__ uint32_t emu_total_key(float f)
{
    int32_t i = __float_as_int(f);
    i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
    return (uint32_t)i ^ 0x80000000u;
}

// 64-bit selection key, larger is better.  tie_last == 0: greatest value in
// total order, lowest index on ties (top_k, spm-qwen3-slice/src/math.rs:38-48);
// tie_last == 1: greatest value with -0 == +0, last index on ties
// (max_by(partial_cmp), spm-batch/tests/batching.rs:111-123).  Key 0 is
// below every real key.
__device__ __forceinline__ uint64_t emu_select_key(float v, uint32_t idx, int tie_last)
{
    if (tie_last) {
        if (v == 0.0f) v = 0.0f;
        return ((uint64_t)emu_total_key(v) << 32) | idx;
    }
    return ((uint64_t)emu_total_key(v) << 32) | (0xffffffffu - idx);
}

__device__ __forceinline__ uint32_t emu_key_index(uint64_t k, int tie_last)
{
    const uint32_t lo = (uint32_t)k;
    return tie_last ? lo : 0xffffffffu - lo;
}

// ------------------------------------------------------------ reductions --

// The value that lane (lane ^ OFF) holds, for OFF = 1, 2, 4 or 8, by DPP row
// operations (no trip through the LDS crossbar): quad_perm for 1 and 2,
// row_half_mirror then quad_perm [3,2,1,0] for 4 (7 - (i ^ 3) = i ^ 4 within
// eight lanes), row_ror:8 for 8.
template <int OFF> __device__ __forceinline__ float emu_xor_lane(float v)
{
    int x = __float_as_int(v);
    if constexpr (OFF == 1) {
        x = __builtin_amdgcn_update_dpp(0, x, 0xb1, 0xf, 0xf, false);
    } else if constexpr (OFF == 2) {
        x = __builtin_amdgcn_update_dpp(0, x, 0x4e, 0xf, 0xf, false);
    } else if constexpr (OFF == 4) {
        x = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xf, 0xf, false);
        x = __builtin_amdgcn_update_dpp(0, x, 0x1b, 0xf, 0xf, false);
    } else {
        static_assert(OFF == 8, "DPP exchange within a 16-lane row");
        x = __builtin_amdgcn_update_dpp(0, x, 0x128, 0xf, 0xf, false);
    }
    return __int_as_float(x);
}

// Exchange across 32 or 16 lanes with v_permlane32_swap / v_permlane16_swap:
// for the pair (a, b) the results (a', b') hold, in every lane l, a' = the
// operand of the lane with bit OFF clear and b' = that of the lane with it
// set, of a where l has the bit clear and of b where it is set.  So
// a' + b' is, in every lane, "own + partner's" of the value the lane keeps in
// a butterfly that keeps a in the lower and b in the upper half.
template <int OFF> __device__ __forceinline__ void emu_swap_halves(float &a, float &b)
{
    static_assert(OFF == 16 || OFF == 32, "permlane swap distance");
    if constexpr (OFF == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        a = __uint_as_float(r[0]);
        b = __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        a = __uint_as_float(r[0]);
        b = __uint_as_float(r[1]);
    }
}

// The value that lane (lane ^ OFF) holds, for any power of two OFF below 64
// (OFF >= 64 names no other lane of the wavefront: the lane's own value, as
// __shfl_xor gives).
template <int OFF> __device__ __forceinline__ float emu_xor_get(float v)
{
    if constexpr (OFF >= 64) {
        return v;
    } else if constexpr (OFF >= 16) {
        float a = v, b = v;
        emu_swap_halves<OFF>(a, b);
        return (__lane_id() & OFF) ? a : b;
    } else {
        return emu_xor_lane<OFF>(v);
    }
}

// Sum over aligned groups of L lanes (L a power of two, <= 64), every lane
// getting its group's sum: a xor butterfly from offset L / 2 down to 1.
template <int L> __device__ __forceinline__ float emu_group_sum(float v)
{
    if constexpr (L > 32) {
        float a = v, b = v;
        emu_swap_halves<32>(a, b);
        v = a + b;
    }
    if constexpr (L > 16) {
        float a = v, b = v;
        emu_swap_halves<16>(a, b);
        v = a + b;
    }
    if constexpr (L > 8) v += emu_xor_lane<8>(v);
    if constexpr (L > 4) v += emu_xor_lane<4>(v);
    if constexpr (L > 2) v += emu_xor_lane<2>(v);
    if constexpr (L > 1) v += emu_xor_lane<1>(v);
    return v;
}

// Wavefront all-reduce by a xor butterfly (offsets 32, 16, ..., 1) of a
// commutative op: every lane gets the same value, in the same association
// order as __shfl_xor butterflies give.
template <class Op> __device__ __forceinline__ float emu_wave_reduce(float v, Op op)
{
    float a = v, b = v;
    emu_swap_halves<32>(a, b);
    v = op(a, b);
    a = v;
    b = v;
    emu_swap_halves<16>(a, b);
    v = op(a, b);
    v = op(v, emu_xor_lane<8>(v));
    v = op(v, emu_xor_lane<4>(v));
    v = op(v, emu_xor_lane<2>(v));
    v = op(v, emu_xor_lane<1>(v));
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
    return emu_wave_reduce(v, [](float x, float y) { return x + y; });
}

// Workgroup sum: wavefront butterflies, then the wavefront totals in order.
__device__ __forceinline__ float emu_block_sum(float v, float *red)
{
    v = wave_sum(v);
    const int lane = threadIdx.x & (EMU_WAVE - 1), w = threadIdx.x / EMU_WAVE;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = 0.0f;
    const int nw = (blockDim.x + EMU_WAVE - 1) / EMU_WAVE;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

__device__ __forceinline__ uint64_t emu_wave_max_u64(uint64_t k)
{
    auto step = [](uint64_t v, auto off) {
        constexpr int OFF = decltype(off)::value;
        const uint32_t lo = __float_as_uint(emu_xor_get<OFF>(__uint_as_float((uint32_t)v)));
        const uint32_t hi = __float_as_uint(emu_xor_get<OFF>(__uint_as_float((uint32_t)(v >> 32))));
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        return o > v ? o : v;
    };
    k = step(k, std::integral_constant<int, 32>{});
    k = step(k, std::integral_constant<int, 16>{});
    k = step(k, std::integral_constant<int, 8>{});
    k = step(k, std::integral_constant<int, 4>{});
    k = step(k, std::integral_constant<int, 2>{});
    k = step(k, std::integral_constant<int, 1>{});
    return k;
}

// v[j] of a four-entry register array at a wavefront-uniform j (selects, so
// the array stays in registers).
__device__ __forceinline__ float emu_pick4(const float (&v)[4], int j)
{
    return j == 0 ? v[0] : j == 1 ? v[1] : j == 2 ? v[2] : v[3];
}

// Router softmax and top-k of one token (moe::route, spm-granite-moe/src/moe.rs:17-35),
// by one wavefront (threads past the first wavefront return at once; no
// barrier inside): p[0..n_experts) holds the logits (n_experts <= 256,
// k <= 64), lane l keeping experts l, l + 64, ... in registers.  Softmax with
// the max subtracted, the sum a left fold in expert order (lane by lane,
// v_readlane); then k rounds of argmax in total order, lower id first on
// ties, with the winner removed; weights are the selected probabilities
// over their left-fold total, in selection order.
// ids_sorted / weights_sorted (optional): the same k routes again, in
// ascending expert id.
__device__ __forceinline__ void emu_route_token(const float *p, int n_experts, int k, int32_t *ids, float *weights,
                                                int32_t *ids_sorted = nullptr, float *weights_sorted = nullptr)
{
    if (threadIdx.x >= EMU_WAVE) return;
    const int lane = threadIdx.x;
    float v[4];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + EMU_WAVE * j;
        v[j] = e < n_experts ? p[e] : -INFINITY;
        m = fmaxf(m, v[j]);
    }
    m = emu_wave_reduce(m, [](float x, float y) { return fmaxf(x, y); });
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = lane + EMU_WAVE * j < n_experts ? expf(v[j] - m) : 0.0f;
    // the fold over experts 0, 1, ...: entries past n_experts are +0.0 and
    // leave the (non-negative) sum unchanged
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (EMU_WAVE * j >= n_experts) break; // uniform
        const int bits = __float_as_int(v[j]);
#pragma unroll
        for (int l = 0; l < EMU_WAVE; ++l) sum = __fadd_rn(sum, __int_as_float(__builtin_amdgcn_readlane(bits, l)));
    }
    uint64_t key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + EMU_WAVE * j;
        v[j] = v[j] / sum;
        key[j] = e < n_experts ? emu_select_key(v[j], (uint32_t)e, 0) : 0; // every live key is > 0
    }
    float my_sel = 0.0f;
    int my_id = 0;
    for (int r = 0; r < k; ++r) {
        uint64_t best = key[0];
#pragma unroll
        for (int j = 1; j < 4; ++j) best = key[j] > best ? key[j] : best;
        best = emu_wave_max_u64(best);
        const int e = __builtin_amdgcn_readfirstlane((int)emu_key_index(best, 0));
        const int wl = e & (EMU_WAVE - 1), wj = e / EMU_WAVE;
        const float pe = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(emu_pick4(v, wj)), wl));
        if (lane == wl) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (j == wj) key[j] = 0;
        }
        if (lane == r) {
            my_sel = pe;
            my_id = e;
        }
    }
    float total = 0.0f;
    for (int r = 0; r < k; ++r) total = __fadd_rn(total, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_sel), r)));
    if (lane < k) {
        ids[lane] = my_id;
        weights[lane] = my_sel / total;
    }
    if (ids_sorted) { // the ids are distinct: a route's place is the count of smaller ids
        int rank = 0;
        for (int r = 0; r < k; ++r) rank += __builtin_amdgcn_readlane(my_id, r) < my_id ? 1 : 0;
        if (lane < k) {
            ids_sorted[rank] = my_id;
            weights_sorted[rank] = my_sel / total;
        }
    }
}

// The MoE matrix-core form's limb planes (moe.hip) of n vectors of C
// 16-column chunks: limbs [vec][C][3][16] int8, then per vector and
// 256-column span kEmuSpanMeta bytes: the limb sum digits [h, l][limb][16
// chunks] int8 and, at byte 96, the span's scale (NaN: the span holds an inf
// or NaN).  A vector v ~= scale * (16384 L0 + 128 L1 + L2) per span.
constexpr int kEmuChunkBytes = 48;  // three int8 limbs of 16 columns
constexpr int kEmuSpanChunks = 16;  // 16-column chunks per 256-column span
constexpr int kEmuSpanMeta = 112;
struct EmuLimbPlanes {
    uint8_t *q;
    uint8_t *dg;
    int C, ns;
};

// v * 2^(20 - e2) as three signed 7-bit limbs (|v| < 2^e2).
__device__ __forceinline__ void emu_limb3(float v, int e2, int (&L)[3])
{
    const float s = ldexpf(v, 6 - e2); // exact, |s| < 64
    const float f0 = rintf(s);
    const float r1 = (s - f0) * 128.0f; // exact
    const float f1 = rintf(r1);
    const float f2 = rintf((r1 - f1) * 128.0f);
    L[0] = (int)f0;
    L[1] = (int)f1;
    L[2] = (int)f2;
}

// Span `span` of vector `vec` into limb planes by one wavefront whose lane l
// holds the span's columns 4l..4l+3 (live: inside the row; zero otherwise):
// the span's largest |v| sets the power-of-two scale, each value splits into
// three limbs, and each 16-column chunk's limb sums go in as two digits
// S = 64 h + l (|S| <= 1024).
__device__ __forceinline__ void emu_span_limbs_wave(float4 v4, bool live, int vec, int span, const EmuLimbPlanes &P)
{
    const int lane = threadIdx.x & (EMU_WAVE - 1);
    const float x[4] = {v4.x, v4.y, v4.z, v4.w};
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = live ? fabsf(x[i]) : 0.0f;
        amax = fmaxf(amax, a);
        bad |= !(a <= 3.402823466e38f);
    }
    amax = emu_wave_reduce(amax, [](float p, float q) { return fmaxf(p, q); });
    const bool finite = __ballot(bad) == 0;
    int e2 = 0;
    (void)frexpf(finite ? amax : 0.0f, &e2);
    uint32_t q[3] = {0u, 0u, 0u};
    int S[3] = {0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int L[3];
        emu_limb3(finite && live ? x[i] : 0.0f, e2, L);
#pragma unroll
        for (int l = 0; l < 3; ++l) {
            q[l] |= ((uint32_t)L[l] & 0xffu) << (8 * i);
            S[l] += L[l];
        }
    }
#pragma unroll
    for (int l = 0; l < 3; ++l) { // the chunk's 16 columns: lanes 4m..4m+3
        S[l] += __shfl_xor(S[l], 1, EMU_WAVE);
        S[l] += __shfl_xor(S[l], 2, EMU_WAVE);
    }
    const int m = lane >> 2, c = kEmuSpanChunks * span + m;
    uint8_t *meta = P.dg + ((size_t)vec * P.ns + span) * kEmuSpanMeta;
    if ((lane & 3) == 0) {
#pragma unroll
        for (int l = 0; l < 3; ++l) {
            const int h = (S[l] + 32) >> 6; // h in [-16, 16], S - 64h in [-32, 31]
            meta[16 * l + m] = (uint8_t)h;
            meta[48 + 16 * l + m] = (uint8_t)(S[l] - 64 * h);
        }
    }
    if (c < P.C) {
        uint8_t *dst = P.q + ((size_t)vec * P.C + c) * kEmuChunkBytes + 4 * (lane & 3);
#pragma unroll
        for (int l = 0; l < 3; ++l) *reinterpret_cast<uint32_t *>(dst + 16 * l) = q[l];
    }
    if (lane == 0)
        *reinterpret_cast<float *>(meta + 96) = finite ? ldexpf(1.0f, e2 - 20) : __int_as_float(0x7fc00000);
}

// Columns col..col+3 (col a multiple of 4) of token t as the multi-token
// matvec's A operands (mfma.hip layout: 16-column sub-block sb, 8-column half
// kh, limb l, token t -> 8 bytes at xa + 384 sb + (24 kh + 8 l + t) 8, the
// scale at xs[8 sb + t]), by the four neighbouring lanes that hold the
// sub-block (live: inside the row, the same for all four): three 7-bit limbs
// under the sub-block's power-of-two scale, the link kernel's split.
__device__ __forceinline__ void emu_emit_limbs4(float4 v4, bool live, int col, int t, uint8_t *xa, float *xs)
{
    const float x[4] = {v4.x, v4.y, v4.z, v4.w};
    float amax = 0.0f;
    int bad = 0; // an inf or NaN (fmaxf alone would drop a NaN)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = live ? fabsf(x[i]) : 0.0f;
        amax = fmaxf(amax, a);
        bad |= !(a <= 3.402823466e38f);
    }
    amax = fmaxf(amax, emu_xor_lane<1>(amax));
    amax = fmaxf(amax, emu_xor_lane<2>(amax));
    bad |= __shfl_xor(bad, 1, EMU_WAVE);
    bad |= __shfl_xor(bad, 2, EMU_WAVE);
    const bool finite = !bad;
    int e2 = 0;
    (void)frexpf(finite ? amax : 0.0f, &e2); // amax < 2^e2, so |x| * 2^(6-e2) < 64
    uint32_t b[3] = {0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float s = finite && live ? ldexpf(x[i], 6 - e2) : 0.0f; // exact
        const float f0 = rintf(s);
        const float r1 = (s - f0) * 128.0f; // exact
        const float f1 = rintf(r1);
        const float f2 = rintf((r1 - f1) * 128.0f);
        b[0] |= ((uint32_t)(int)f0 & 0xffu) << (8 * i);
        b[1] |= ((uint32_t)(int)f1 & 0xffu) << (8 * i);
        b[2] |= ((uint32_t)(int)f2 & 0xffu) << (8 * i);
    }
    if (!live) return;
    const int sb = col >> 4, kh = (col >> 3) & 1;
    uint8_t *dst = xa + (size_t)sb * 384 + (size_t)(kh * 24 + t) * 8 + (col & 7);
#pragma unroll
    for (int l = 0; l < 3; ++l) *reinterpret_cast<uint32_t *>(dst + 64 * l) = b[l];
    if ((col & 15) == 0) xs[(size_t)sb * 8 + t] = finite ? ldexpf(1.0f, e2 - 20) : __int_as_float(0x7fc00000);
}

// One token's k (<= 8) routes in ascending expert id (ids are distinct;
// entries past k or outside the expert range are skipped): order[i] is the
// slot and w[i] its weight; returns how many (moe.rs:37-159 combines in that
// order, from +0.0).
__device__ __forceinline__ int emu_route_order(const int32_t *ids, const float *wts, int k, int n_experts,
                                               int (&order)[8], float (&w)[8])
{
    int idv[8];
    float wv[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        idv[s] = s < k ? ids[s] : 0x7fffffff;
        wv[s] = s < k ? wts[s] : 0.0f;
    }
    int n = 0, prev = -1;
    for (int i = 0; i < k; ++i) {
        int best = -1, best_id = 0x7fffffff;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int id = idv[s];
            if (id > prev && id < best_id && id < n_experts) {
                best = s;
                best_id = id;
            }
        }
        if (best < 0) break;
        order[n++] = best;
        prev = best_id;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int o = i < n ? order[i] : 0;
        order[i] = o;
        float wi = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; ++s) wi = s == o ? wv[s] : wi;
        w[i] = wi;
    }
    return n;
}

// ------------------------------------------------------------- launchers --
// Implemented per translation unit; declared here for the model code.
struct QmvArgs {
    const uint8_t *w;      // rows x row_bytes
    const uint8_t *w_up;   // SwiGLU partner matrix or null
    size_t row_bytes;
    int rows, cols, nb;    // nb = blocks per row
    const float *x;        // n_tok x cols
    const float *gain;     // RMS gain or null
    float eps;
    float *y;              // n_tok x rows
    int accumulate;
    uint64_t *keys;        // optional greedy-selection keys: keys[t * key_stride + wave]
    int key_stride;
    int tie_last;
    float acc_scale;       // accumulate as y + v * acc_scale (0: y + v)
    float out_div;         // results divided by this before store and keys (0: none)
    int lane_major;        // w / w_up in the Q6_K lane-major layout (emu_lane_major_q6k)
    int mfma_major;        // w / w_up in the Q6_K matrix-core operand layout (emu_mfma_major_q6k)
    int act;               // gate|up pair: EMU_ACT_SILU (SwiGLU) or EMU_ACT_GELU_TANH (GeGLU)
    float softcap;         // results -> softcap * tanh(v / softcap) after out_div (0: none)
    int f32_act;           // f32 activations: the dequant + f32 FMA kernels, not the int8-limb ones
    int span_scales;       // multi-token chain: the A operands carry one scale per 256-column span
    int span_norm;         // with span_scales: apply the deferring link's RMS factor (with eps)
};

// A matvec result's epilogue: divided by out_div (when set), then added to
// the residual as r + v * s with two roundings (the reference's add_scaled,
// spm-granite-moe/src/math.rs:31-33), or r + v when s is 0.
__device__ __forceinline__ float emu_out_div(float v, float d) { return d != 0.0f ? v / d : v; }
// The output epilogue: divided by d (when set), then soft-capped as
// cap * tanh(v / cap) (when cap is set).
__device__ __forceinline__ float emu_out_epi(float v, float d, float cap)
{
    v = emu_out_div(v, d);
    return cap != 0.0f ? cap * tanhf(v / cap) : v;
}
// gelu, tanh form (spm-granite-moe/src/gemma_smoke.rs:88-90), left to right,
// no contraction.
__device__ __forceinline__ float emu_gelu_tanh(float v)
{
#pragma clang fp contract(off)
    float inner = 0.044715f * v;
    inner = inner * v;
    inner = 1.0f + inner;
    float arg = 0.7978846f * v;
    arg = arg * inner;
    const float t = tanhf(arg);
    const float half = 0.5f * v;
    return half * (1.0f + t);
}
// A gate|up pair's activation: silu(g) * u (spm-ops/src/nonlinear.rs:5-7) or
// gelu(g) * u (gemma_smoke.rs:111-120).
__device__ __forceinline__ float emu_glu(float g, float u, int act)
{
#pragma clang fp contract(off)
    return act == 1 ? emu_gelu_tanh(g) * u : (g / (1.0f + expf(-g))) * u;
}
__device__ __forceinline__ float emu_resid_add(float r, float v, float s)
{
    return s != 0.0f ? r + __fmul_rn(v, s) : r + v;
}

// Launch a quantized matvec; *key_slots (optional) receives how many key
// slots per token the launch writes when a.keys is set.
int emu_launch_qmv(emu_ctx *ctx, int encoding, const QmvArgs &a, int n_tok, int *key_slots = nullptr);
int emu_row_bytes(int encoding, uint32_t cols, size_t *row_bytes);
// Batch-1 integer-limb matvec (limb.hip): shapes and formats it covers, and
// its launcher (EMU_E_UNSUPPORTED for anything else).
bool emu_limb_supports(int encoding, int cols);
int emu_launch_limb(emu_ctx *ctx, int encoding, const QmvArgs &a, int *key_slots);
// Q6_K lane-major layout (limb.hip): the block stream cut into chunks of 16
// blocks (the last may hold fewer, n), each chunk permuted so that unit L =
// 4*(block) + 2*h + m finds its ql-low 16 bytes at 16L, ql-high at 64n + 16L,
// qh at 128n + 16L, the 8 scale bytes of (block, h) at 192n + 8*(L/2) and the
// block's d at 208n + 2*(L/4).  A pure byte permutation of each chunk: sizes
// and chunk offsets are unchanged.  src and dst must not overlap.
int emu_lane_major_q6k(emu_ctx *ctx, const uint8_t *src, size_t nblocks, uint8_t *dst);
// The Q6_K matrix-core operand copy of a rows x cols matrix (mfma.hip):
// emu_mfma_major_bytes(rows, cols) bytes, rows rounded up to whole 32-row
// tiles (the padding rows repeat the last row).
size_t emu_mfma_major_bytes(uint32_t rows, uint32_t cols);
int emu_mfma_major_q6k(emu_ctx *ctx, const uint8_t *src, uint32_t rows, uint32_t cols, uint8_t *dst);
// Multi-token (2..8) matvec on the int8 matrix cores (mfma.hip).  Its
// workspace lives in the context and grows on demand (hipMalloc); callers
// that capture graphs reserve it beforehand with emu_mfma_reserve.
bool emu_mfma_supports(int encoding, int cols, int n_tok);
// The same shapes at any token count 1..8 (the chained MoE step runs a single
// client on the matrix cores too, so that a client's bits do not depend on
// how many share the step).
bool emu_mfma_shape_ok(int encoding, int cols);
size_t emu_mfma_workspace_bytes(int rows, int cols, int nmat);
int emu_mfma_reserve(emu_ctx *ctx, size_t bytes);
int emu_launch_mfma(emu_ctx *ctx, int encoding, const QmvArgs &a, int n_tok, int *key_slots);
// The chained form used by the decode step: link (the producing matvec's
// partial sums -> its epilogue -> the next matvec's A operands), matvec
// (A operands -> partial sums), ... with one workspace sized for operands of
// up to cols_cap columns plus the largest partial-sum set
// (emu_mfma_chain_bytes).  Modes of the link: 0 input x, 1 residual add into
// h, 2 SwiGLU of a gate/up pair, 3 plain sums written to h.
struct EmuMfmaLink {
    int mode;
    bool from_part; // the partial sums of the last matvec (modes 1-3)
    int part_nks, part_nmat;
    float *h;
    const float *x;
    int cols, cols_cap, n_tok;
    const float *gain;
    float eps;
    bool limbs; // write the next matvec's A operands
    // Mode 0 only, optional: before the norm, add a MoE layer's expert sum
    // to x (its k routes' contributions, weighted, in expert-id order), as
    // x + sum * m_scale, and write the result back to h.
    const float *m_contrib;
    const int32_t *m_ids;
    const float *m_wts;
    int m_k, m_experts;
    float m_scale;
    int m_sorted; // the routes come in ascending expert id (no reordering)
    // Mode 0 only, optional, before the expert sum: a dense FFN's down
    // projection, as the last matvec's d_nks partial-sum slices (one
    // matrix), joins x as x + v * d_scale.
    bool d_part;
    int d_nks;
    float d_scale;
    // Mode 2: the gate/up pair's activation (EMU_ACT_SILU or EMU_ACT_GELU_TANH).
    int act;
    // The limbs under one power-of-two scale per 256-column span (xs holds
    // [span][8 tokens]) instead of per 16-column sub-block: exact to 2^-20 of
    // the span's largest |x|, as the expert kernels' limb planes.  Only for a
    // matvec launched with QmvArgs::span_scales.
    int span;
    // With gain and span: the row's RMS factor is left to the consuming
    // matvec (QmvArgs::span_norm), so no workgroup needs the whole row and
    // the link runs as many small ones.  The limbs are of x * gain.
    int defer_norm;
};
size_t emu_mfma_chain_bytes(int cols_cap, size_t max_part_bytes);
size_t emu_mfma_part_bytes(int rows, int cols, int nmat);
int emu_mfma_link(emu_ctx *ctx, const EmuMfmaLink &l);
int emu_mfma_matvec(emu_ctx *ctx, const QmvArgs &q, int n_tok, int cols_cap, int *part_nks);
int emu_mfma_finish(emu_ctx *ctx, const QmvArgs &q, int n_tok, int cols_cap, int *key_slots);
// The chained form's buffers: A operands + scales, and the partial sums
// (layout [slice][matrix][8 tokens][rows]).
void emu_mfma_buffers(emu_ctx *ctx, int cols_cap, uint8_t **xa, float **xs, float **part);

// Fused decode attention of one layer for every client (attn.hip).
struct EmuAttnLaunch {
    const float *qkv;
    void *k_cache, *v_cache;
    const uint32_t *positions;
    const float *rope;
    const float *q_norm, *k_norm;
    float eps, score_mul, score_div;
    int rope_fma, interleaved, heads, kv_heads, head_dim, layers, layer, context, clients, kv_f16;
    float *partial;
    uint32_t *counters;
    float *out;
    // Optional: q|k|v as the sum of qkv_slices partial-sum arrays (client
    // stride and slice stride in floats; 0 = one plain array), and the output
    // also written as the multi-token matvec's A operands (mfma.hip layout).
    int qkv_slices, qkv_client_stride;
    size_t qkv_slice_stride;
    uint8_t *xa;
    float *xs;
    // Sliding window: attend to the last `window` positions only (0: all).
    int window;
};
int emu_launch_attn(emu_ctx *ctx, const EmuAttnLaunch &l);
// emu_moe_ffn whose weighted expert sum is added to the residual stream,
// state = state + sum * scale with two roundings (moe.hip).
// With combine false the weighted sum is left for the caller: the expert
// outputs stay at emu_moe_contrib(workspace, ...) ([token][slot][width]).
// With x_planes_ready the tokens' limb planes (emu_moe_x_planes) already
// hold x (the matrix-core form only: see emu_moe_mma_form).  With
// span_counters (emu_moe_span_counters() entries, zero before the first
// call; every call leaves them zero) the gate|up launch also writes the
// routes' limb planes, one launch fewer; calls sharing them must not overlap.
int emu_moe_ffn_resid(emu_ctx *ctx, const emu_moe_desc *d, const float *d_x, uint32_t n_tok, const int32_t *d_ids,
                      const float *d_weights, void *d_workspace, size_t workspace_bytes, float *d_state,
                      float scale, bool combine = true, bool x_planes_ready = false,
                      uint32_t *span_counters = nullptr, const uint8_t *const *d_table = nullptr);
size_t emu_moe_span_counters();
const float *emu_moe_contrib(const void *d_workspace, uint32_t n_tok, uint32_t k, uint32_t ff);
// Whether the layer takes the matrix-core form, and where its workspace
// keeps the tokens' limb planes.
bool emu_moe_mma_form(const emu_moe_desc *d);
// The expert cache's device policy (cache.hip), for the decode step: set-up
// and one layer's plan (its table of expert addresses, then the admissions'
// copies into their slots).
size_t emu_cache_expert_bytes(const emu_expert_cache *c);
uint32_t emu_cache_layers(const emu_expert_cache *c);
uint32_t emu_cache_experts(const emu_expert_cache *c);
int emu_cache_device_enable(emu_expert_cache *c);
int emu_cache_plan(emu_expert_cache *c, uint32_t layer, const int32_t *d_ids, int nk, const uint8_t *const **table);
EmuLimbPlanes emu_moe_x_planes(void *d_workspace, uint32_t n_tok, uint32_t k, uint32_t width, uint32_t ff);
int emu_attn_max_chunks(int context);
