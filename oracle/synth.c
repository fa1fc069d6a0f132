/*
 * synth.c -- the seeded synthetic weights, computed on the CPU.
 *
 * TEST INFRASTRUCTURE ONLY: lets the checker build, without a GPU, the same
 * model bytes that the library's device synthesis (emu_model_synth) writes,
 * so that oracle runs too long for a GPU test (the full 36-layer Qwen3-8B
 * shape over hundreds of steps) can be done here and committed as golden
 * tokens.  No reference counterpart: the reference has no synthetic weights.
 *
 * Every tensor element is a N(0, sd) draw keyed by (seed, stream, index):
 * splitmix64 gives two exact 24-bit uniforms, and Box-Muller is evaluated in
 * double precision with additions, multiplications and correctly rounded
 * divisions only (compiled without contraction), then rounded once to float,
 * so the bits do not depend on any math library.  Blocks are then quantized
 * by the GGML-format rules below (scales from the block's own maxima, codes
 * by round-half-even of v / scale).
 *
 * Pinned by: a GPU test that the device synthesis writes these bytes, every
 * format, sampled tensors (tests/test_gpu_synth.py); CPU tests of the draws'
 * moments and of the logarithm, cosine and square root pieces against libm
 * (tests/test_synth.py).
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

static uint64_t splitmix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static double bits_to_double(uint64_t b)
{
    double d;
    memcpy(&d, &b, 8);
    return d;
}

static uint64_t double_to_bits(double d)
{
    uint64_t b;
    memcpy(&b, &d, 8);
    return b;
}

/* ln k for an integer k >= 1: k = 2^e m with m in [sqrt(1/2), sqrt(2)),
 * ln m = 2 atanh(s) = 2 (s + s^3/3 + ... + s^23/23), s = (m - 1) / (m + 1). */
double or_synth_ln_int(uint32_t k)
{
    int e = 31 - __builtin_clz(k);
    double m = (double)k * bits_to_double((uint64_t)(1023 - e) << 52);
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

/* Taylor polynomials of sin and cos on [0, pi/4] (to x^17 and x^18). */
static double sin_poly(double x)
{
    const double x2 = x * x;
    double p = 1.0 / 355687428096000.0;
    p = p * x2 - 1.0 / 1307674368000.0;
    p = p * x2 + 1.0 / 6227020800.0;
    p = p * x2 - 1.0 / 39916800.0;
    p = p * x2 + 1.0 / 362880.0;
    p = p * x2 - 1.0 / 5040.0;
    p = p * x2 + 1.0 / 120.0;
    p = p * x2 - 1.0 / 6.0;
    p = p * x2 + 1.0;
    return x * p;
}

static double cos_poly(double x)
{
    const double x2 = x * x;
    double p = 1.0 / 6402373705728000.0;
    p = p * x2 - 1.0 / 20922789888000.0;
    p = p * x2 + 1.0 / 87178291200.0;
    p = p * x2 - 1.0 / 479001600.0;
    p = p * x2 + 1.0 / 3628800.0;
    p = p * x2 - 1.0 / 40320.0;
    p = p * x2 + 1.0 / 720.0;
    p = p * x2 - 1.0 / 24.0;
    p = p * x2 + 1.0 / 2.0;
    return 1.0 - x2 * p;
}

/* cos(2 pi j / 2^24) for j < 2^24: the angle is pi/2 (q + f / 2^22); past
 * pi/4 within the quadrant the co-function of the complement is taken. */
double or_synth_cos_turn(uint32_t j)
{
    const uint32_t q = j >> 22, f = j & 0x3fffffu;
    const int hi = f > 0x200000u;
    const double g = (double)(hi ? 0x400000u - f : f) * (1.0 / 4194304.0);
    const double x = g * 1.5707963267948966;
    const double cg = cos_poly(x), sg = sin_poly(x);
    const double c = hi ? sg : cg, sn = hi ? cg : sg;
    return q == 0 ? c : q == 1 ? -sn : q == 2 ? -c : sn;
}

/* sqrt(y) = y * (1/sqrt(y)), six Newton steps from an exponent-based guess. */
double or_synth_sqrt(double y)
{
    if (y == 0.0) return 0.0;
    const int64_t b = (int64_t)double_to_bits(y);
    double r = bits_to_double((uint64_t)(0x5fe6eb50c7b537a9ll - (b >> 1)));
    for (int i = 0; i < 6; ++i) r = r * (1.5 - (0.5 * y) * (r * r));
    return y * r;
}

float or_synth_gauss(uint64_t seed, uint64_t stream, uint64_t idx, float sd)
{
    const uint64_t h = splitmix64(seed ^ splitmix64(stream * 0x632be59bd9b4e019ull + idx));
    const uint32_t k = (uint32_t)(h >> 40) + 1u;
    const uint32_t j = (uint32_t)(h & 0xffffffu);
    const double ln_u1 = or_synth_ln_int(k) - 24.0 * 0.6931471805599453;
    const double r = or_synth_sqrt(-2.0 * ln_u1);
    return (float)(((double)sd * r) * or_synth_cos_turn(j));
}

static float clampf(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

static void synth_q8_0(uint8_t *out, size_t b, uint64_t seed, uint64_t stream, float sd)
{
    float v[32], amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        v[i] = or_synth_gauss(seed, stream, b * 32 + (uint64_t)i, sd);
        amax = fmaxf(amax, fabsf(v[i]));
    }
    const uint16_t d16 = or_f32_to_f16(amax / 127.0f);
    const float dd = or_f16_to_f32(d16);
    out[0] = (uint8_t)d16;
    out[1] = (uint8_t)(d16 >> 8);
    for (int i = 0; i < 32; ++i) {
        const float q = dd > 0.0f ? clampf(rintf(v[i] / dd), -127.0f, 127.0f) : 0.0f;
        out[2 + i] = (uint8_t)(int8_t)q;
    }
}

static void synth_q6_k(uint8_t *out, size_t b, uint64_t seed, uint64_t stream, float sd)
{
    float v[256], scale[16], mx = 0.0f;
    memset(out, 0, 210);
    for (int s = 0; s < 16; ++s) {
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) {
            v[16 * s + i] = or_synth_gauss(seed, stream, b * 256 + (uint64_t)(16 * s + i), sd);
            amax = fmaxf(amax, fabsf(v[16 * s + i]));
        }
        scale[s] = amax / 31.0f;
        mx = fmaxf(mx, scale[s]);
    }
    const uint16_t d16 = or_f32_to_f16(mx / 127.0f);
    const float dd = or_f16_to_f32(d16);
    int sc[16];
    for (int s = 0; s < 16; ++s) {
        sc[s] = dd > 0.0f ? (int)clampf(rintf(scale[s] / dd), -128.0f, 127.0f) : 0;
        out[192 + s] = (uint8_t)(int8_t)sc[s];
    }
    out[208] = (uint8_t)d16;
    out[209] = (uint8_t)(d16 >> 8);
    for (int e = 0; e < 256; ++e) {
        const float m = dd * (float)sc[e / 16];
        const int q = m > 0.0f ? (int)clampf(rintf(v[e] / m) + 32.0f, 0.0f, 63.0f) : 32;
        const int h = e / 128, r = e % 128, j = r / 32, l = r % 32;
        out[64 * h + l + 32 * (j & 1)] |= (uint8_t)((q & 15) << (4 * (j >> 1)));
        out[128 + 32 * h + l] |= (uint8_t)((q >> 4) << (2 * j));
    }
}

static void synth_q5_k(uint8_t *out, size_t b, uint64_t seed, uint64_t stream, float sd)
{
    float v[256], scale[8], mneg[8], ms = 0.0f, mm = 0.0f;
    memset(out, 0, 176);
    for (int s = 0; s < 8; ++s) {
        float lo = 0.0f, hi = -INFINITY;
        for (int i = 0; i < 32; ++i) {
            const float x = or_synth_gauss(seed, stream, b * 256 + (uint64_t)(32 * s + i), sd);
            v[32 * s + i] = x;
            lo = fminf(lo, x);
            hi = fmaxf(hi, x);
        }
        scale[s] = (hi - lo) / 31.0f;
        mneg[s] = -lo;
        ms = fmaxf(ms, scale[s]);
        mm = fmaxf(mm, mneg[s]);
    }
    const uint16_t d16 = or_f32_to_f16(ms / 63.0f), m16 = or_f32_to_f16(mm / 63.0f);
    const float dd = or_f16_to_f32(d16), dm = or_f16_to_f32(m16);
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
        const float scl = dd * (float)sc[s];
        const int q = scl > 0.0f ? (int)clampf(rintf((v[e] + dm * (float)mi[s]) / scl), 0.0f, 31.0f) : 0;
        out[48 + 32 * g + l] |= (uint8_t)((q & 15) << (4 * half));
        out[16 + l] |= (uint8_t)((q >> 4) << (2 * g + half));
    }
}

static void synth_q2_k(uint8_t *out, size_t b, uint64_t seed, uint64_t stream, float sd)
{
    float v[256], scale[16], mneg[16], ms = 0.0f, mm = 0.0f;
    memset(out, 0, 84);
    for (int s = 0; s < 16; ++s) {
        float lo = 0.0f, hi = -INFINITY;
        for (int i = 0; i < 16; ++i) {
            const float x = or_synth_gauss(seed, stream, b * 256 + (uint64_t)(16 * s + i), sd);
            v[16 * s + i] = x;
            lo = fminf(lo, x);
            hi = fmaxf(hi, x);
        }
        scale[s] = (hi - lo) / 3.0f;
        mneg[s] = -lo;
        ms = fmaxf(ms, scale[s]);
        mm = fmaxf(mm, mneg[s]);
    }
    const uint16_t d16 = or_f32_to_f16(ms / 15.0f), m16 = or_f32_to_f16(mm / 15.0f);
    const float dd = or_f16_to_f32(d16), dm = or_f16_to_f32(m16);
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
        const int N = e / 128, j = (e / 32) & 3, s = (e / 16) & 1, l = e % 16, si = e / 16;
        const float scl = dd * (float)sc[si];
        const int q = scl > 0.0f ? (int)clampf(rintf((v[e] + dm * (float)mi[si]) / scl), 0.0f, 3.0f) : 0;
        out[16 + 32 * N + 16 * s + l] |= (uint8_t)(q << (2 * j));
    }
}

int or_synth_blocks(int dtype, uint8_t *dst, size_t nblocks, uint64_t seed, uint64_t stream, float sd)
{
    size_t bb;
    switch (dtype) {
    case OR_Q8_0: bb = 34; break;
    case OR_Q6_K: bb = 210; break;
    case OR_Q5_K: bb = 176; break;
    case OR_Q2_K: bb = 84; break;
    default: return -1;
    }
#pragma omp parallel for schedule(static)
    for (long long b = 0; b < (long long)nblocks; ++b) {
        uint8_t *out = dst + (size_t)b * bb;
        switch (dtype) {
        case OR_Q8_0: synth_q8_0(out, (size_t)b, seed, stream, sd); break;
        case OR_Q6_K: synth_q6_k(out, (size_t)b, seed, stream, sd); break;
        case OR_Q5_K: synth_q5_k(out, (size_t)b, seed, stream, sd); break;
        default: synth_q2_k(out, (size_t)b, seed, stream, sd); break;
        }
    }
    return 0;
}

void or_synth_f32(float *dst, size_t n, uint64_t seed, uint64_t stream, float sd)
{
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) dst[i] = or_synth_gauss(seed, stream, (uint64_t)i, sd);
}
