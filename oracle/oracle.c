/*
 * oracle.c -- CPU restatement of emufpga's token-loop arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against,
 * never a product code path.  See oracle.h for what pins each function.
 * Reference citations are relative to the emufpga repository root.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* components/cli/crates/spm-gguf/src/tensor.rs:82-98 */
float or_f16_to_f32(uint16_t bits)
{
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    uint32_t exp = (bits >> 10) & 0x1fu;
    uint32_t fraction = bits & 0x03ffu;
    uint32_t out;
    if (exp == 0 && fraction == 0) {
        out = sign;
    } else if (exp == 0) {
        /* leading_zeros of a u32 minus 21: shift that brings bit 10 up */
        uint32_t shift = (uint32_t)__builtin_clz(fraction) - 21u;
        uint32_t normalized = fraction << shift;
        uint32_t exponent = 113u - shift;
        out = sign | (exponent << 23) | ((normalized & 0x03ffu) << 13);
    } else if (exp == 31) {
        out = sign | 0x7f800000u | (fraction << 13);
    } else {
        out = sign | ((exp + 112u) << 23) | (fraction << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

/* IEEE binary16 round-to-nearest-even, used for the fp16 KV cache.  No
 * reference counterpart (the reference cache is f32, spm-kv/src/cache.rs:11-31). */
uint16_t or_f32_to_f16(float x)
{
    uint32_t b;
    memcpy(&b, &x, 4);
    uint32_t sign = (b >> 16) & 0x8000u;
    uint32_t ax = b & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0));
    if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) { /* subnormal half (or zero) */
        /* value = ax as float; half subnormal unit = 2^-24 */
        float f;
        memcpy(&f, &ax, 4);
        float scaled = f * 16777216.0f; /* exact: power-of-two scaling of a float */
        /* nearbyintf rounds half to even in the default rounding mode */
        uint32_t m = (uint32_t)nearbyintf(scaled);
        return (uint16_t)(sign | m);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u)))
        h += 1u;
    return (uint16_t)(sign | h);
}

/* components/cli/crates/spm-gguf/src/parse.rs:10-29 (the subset on the path) */
int or_block_layout(int dtype, uint32_t *elems, uint32_t *bytes)
{
    switch (dtype) {
    case OR_F32: *elems = 1; *bytes = 4; return 0;
    case OR_F16: *elems = 1; *bytes = 2; return 0;
    case OR_Q8_0: *elems = 32; *bytes = 34; return 0;
    case OR_Q2_K: *elems = 256; *bytes = 84; return 0;
    case OR_Q5_K: *elems = 256; *bytes = 176; return 0;
    case OR_Q6_K: *elems = 256; *bytes = 210; return 0;
    default: return -1;
    }
}

static float f16_at(const uint8_t *p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* components/cli/crates/spm-gguf/src/tensor.rs:103-139 */
int or_decode_q6_k(const uint8_t *src, size_t len, float *out)
{
    if (len % 210 != 0)
        return -1;
    size_t blocks = len / 210;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *block = src + b * 210;
        float d = f16_at(block + 208);
        for (int half = 0; half < 2; ++half) {
            const uint8_t *ql = block + half * 64;
            const uint8_t *qh = block + 128 + half * 32;
            const int8_t *scales = (const int8_t *)(block + 192 + half * 8);
            float *base = out + b * 256 + half * 128;
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                uint8_t quants[4] = {
                    (uint8_t)((ql[l] & 0x0f) | ((qh[l] & 3) << 4)),
                    (uint8_t)((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)),
                    (uint8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)),
                    (uint8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)),
                };
                for (int lane = 0; lane < 4; ++lane) {
                    float q = (float)quants[lane] - 32.0f;
                    float scale = (float)scales[is + lane * 2];
                    base[l + lane * 32] = d * scale * q;
                }
            }
        }
    }
    return 0;
}

/* components/cli/crates/spm-gguf/src/tensor.rs:179-188 */
static void scale_min_q5(int index, const uint8_t *packed, uint8_t *scale, uint8_t *minimum)
{
    if (index < 4) {
        *scale = packed[index] & 63;
        *minimum = packed[index + 4] & 63;
    } else {
        *scale = (uint8_t)((packed[index + 4] & 0x0f) | ((packed[index - 4] >> 6) << 4));
        *minimum = (uint8_t)((packed[index + 4] >> 4) | ((packed[index] >> 6) << 4));
    }
}

/* components/cli/crates/spm-gguf/src/tensor.rs:144-177 */
int or_decode_q5_k(const uint8_t *src, size_t len, float *out)
{
    if (len % 176 != 0)
        return -1;
    size_t blocks = len / 176;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *block = src + b * 176;
        float d = f16_at(block);
        float dmin = f16_at(block + 2);
        const uint8_t *scales = block + 4;
        const uint8_t *qh = block + 16;
        const uint8_t *qs = block + 48;
        float *o = out + b * 256;
        for (int group = 0; group < 4; ++group) {
            for (int half = 0; half < 2; ++half) {
                int index = group * 2 + half;
                uint8_t scale, minimum;
                scale_min_q5(index, scales, &scale, &minimum);
                uint8_t bit = (uint8_t)(1u << index);
                for (int lane = 0; lane < 32; ++lane) {
                    uint8_t packed = qs[group * 32 + lane];
                    uint8_t low = half == 0 ? (packed & 0x0f) : (packed >> 4);
                    uint8_t quant = (uint8_t)(low + ((qh[lane] & bit) ? 16 : 0));
                    *o++ = d * (float)scale * (float)quant - dmin * (float)minimum;
                }
            }
        }
    }
    return 0;
}

/* components/cli/crates/spm-gguf/src/tensor.rs:193-210 */
int or_decode_q8_0(const uint8_t *src, size_t len, float *out)
{
    if (len % 34 != 0)
        return -1;
    size_t blocks = len / 34;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *block = src + b * 34;
        float d = f16_at(block);
        for (int i = 0; i < 32; ++i)
            out[b * 32 + i] = d * (float)(int8_t)block[2 + i];
    }
    return 0;
}

/* Q2_K has no decoder in the reference (docs/olmoe-placement-baseline.md:12;
 * only its size, parse.rs:20 -> (256, 84)).  Restated from the published GGML
 * block_q2_K format: scales[16] (low nibble scale, high nibble min), qs[64],
 * d (f16) at 80, dmin (f16) at 82.  Element 128N + 32j + 16s + l takes the
 * 2-bit code (qs[32N + 16s + l] >> 2j) & 3 and sub-block scale index
 * 8N + 2j + s; y = d*(sc&15)*code - dmin*(sc>>4). */
int or_decode_q2_k(const uint8_t *src, size_t len, float *out)
{
    if (len % 84 != 0)
        return -1;
    size_t blocks = len / 84;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *block = src + b * 84;
        const uint8_t *sc = block;
        const uint8_t *qs = block + 16;
        float d = f16_at(block + 80);
        float dmin = f16_at(block + 82);
        float *o = out + b * 256;
        for (int n = 0; n < 2; ++n) {
            for (int j = 0; j < 4; ++j) {
                for (int s = 0; s < 2; ++s) {
                    uint8_t packed = sc[8 * n + 2 * j + s];
                    float dl = d * (float)(packed & 15);
                    float ml = dmin * (float)(packed >> 4);
                    for (int l = 0; l < 16; ++l) {
                        int code = (qs[32 * n + 16 * s + l] >> (2 * j)) & 3;
                        *o++ = dl * (float)code - ml;
                    }
                }
            }
        }
    }
    return 0;
}

int or_decode(int dtype, const uint8_t *src, size_t len, float *out)
{
    switch (dtype) {
    case OR_Q6_K: return or_decode_q6_k(src, len, out);
    case OR_Q5_K: return or_decode_q5_k(src, len, out);
    case OR_Q8_0: return or_decode_q8_0(src, len, out);
    case OR_Q2_K: return or_decode_q2_k(src, len, out);
    case OR_F32:
        if (len % 4) return -1;
        memcpy(out, src, len);
        return 0;
    default: return -2;
    }
}

/* M1: components/cli/crates/spm-qwen3-slice/src/math.rs:12-20 and
 * components/cli/crates/spm-granite-moe/src/math.rs:13-21 (Rust Sum<f32>
 * folds from -0.0 with each product rounded before the add). */
void or_matvec_m1(const float *w, uint32_t rows, uint32_t cols, const float *x, float *y)
{
    for (uint32_t r = 0; r < rows; ++r) {
        const float *row = w + (size_t)r * cols;
        float acc = -0.0f;
        for (uint32_t c = 0; c < cols; ++c) {
            float p = row[c] * x[c];
            acc = acc + p;
        }
        y[r] = acc;
    }
}

/* M2: components/tensor/crates/spm-linear/src/stream.rs:31-55 with
 * apply_weight resident.rs:124-137: out zero-filled, then per weight
 * out = mul_add(w, x, out).  Every row sees its columns in ascending order in
 * both the column-major and the row-major stream, so the chain per row is the
 * same; w is row-major here. */
void or_matvec_m2(const float *w, uint32_t rows, uint32_t cols, const float *x,
                  uint32_t positions, float *out)
{
    for (uint32_t p = 0; p < positions; ++p) {
        for (uint32_t r = 0; r < rows; ++r) {
            const float *row = w + (size_t)r * cols;
            const float *xp = x + (size_t)p * cols;
            float acc = 0.0f;
            for (uint32_t c = 0; c < cols; ++c)
                acc = fmaf(row[c], xp[c], acc);
            out[(size_t)p * rows + r] = acc;
        }
    }
}

/* Threads for the row loops: 1 (the reference's single-threaded scalar
 * path, the default) up to the host's cores.  Results are identical for any
 * count. */
static int g_threads = 1;

void or_set_threads(int n) { g_threads = n > 0 ? n : 1; }

static int or_threads_in_use(uint32_t rows)
{
    /* small matrices are not worth a thread team */
    return rows >= 64 ? g_threads : 1;
}

/* Quantized projection: spm-qwen3-slice/src/weights.rs:27-63 (decode, M1 per
 * token) or spm-granite-moe/src/layout.rs:208-242 (decode, M2 chain). */
int or_qmatvec(int dtype, const uint8_t *w, uint32_t rows, uint32_t cols, const float *x,
               uint32_t n_tok, float *y, int mode)
{
    uint32_t be, bb;
    if (or_block_layout(dtype, &be, &bb) != 0)
        return -2;
    if (cols % be != 0)
        return -3;
    size_t row_bytes = (size_t)(cols / be) * bb;
    int failed = 0;
    /* Rows are independent and each keeps its own sequential fold, so the
     * result does not depend on how many threads share the rows. */
#pragma omp parallel num_threads(or_threads_in_use(rows))
    {
        float *row = (float *)malloc(sizeof(float) * cols);
        if (!row) {
#pragma omp atomic write
            failed = -4;
        }
#pragma omp for schedule(static)
        for (uint32_t r = 0; r < rows; ++r) {
            if (!row)
                continue;
            if (or_decode(dtype, w + (size_t)r * row_bytes, row_bytes, row) != 0) {
#pragma omp atomic write
                failed = -1;
                continue;
            }
            for (uint32_t t = 0; t < n_tok; ++t) {
                const float *xt = x + (size_t)t * cols;
                float acc;
                if (mode == 2) {
                    acc = 0.0f;
                    for (uint32_t c = 0; c < cols; ++c)
                        acc = fmaf(row[c], xt[c], acc);
                } else {
                    acc = -0.0f;
                    for (uint32_t c = 0; c < cols; ++c) {
                        float p = row[c] * xt[c];
                        acc = acc + p;
                    }
                }
                y[(size_t)t * rows + r] = acc;
            }
        }
        free(row);
    }
    return failed;
}

/* int8 activation blocks of 32 (no reference counterpart: the reference has
 * f32 activations only; this defines the int8 mode's quantizer). */
void or_quantize_act_q8(const float *x, uint32_t n, int8_t *q, float *scales)
{
    for (uint32_t b = 0; b < n / 32; ++b) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            float a = fabsf(x[b * 32 + i]);
            amax = a > amax ? a : amax;
        }
        float s = amax / 127.0f;
        float id = s != 0.0f ? 1.0f / s : 0.0f;
        scales[b] = s;
        for (int i = 0; i < 32; ++i) {
            float v = roundf(x[b * 32 + i] * id);
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            q[b * 32 + i] = (int8_t)v;
        }
    }
}

/* Integer code of element e of one block, and its sub-block index. */
static int block_code(int dtype, const uint8_t *block, int e)
{
    switch (dtype) {
    case OR_Q8_0:
        return (int8_t)block[2 + e];
    case OR_Q6_K: {
        int h = e / 128, r = e % 128, lane = r / 32, l = r % 32;
        const uint8_t *ql = block + h * 64, *qh = block + 128 + h * 32;
        int lo = (lane & 1) ? ql[l + 32] : ql[l];
        int nib = (lane >> 1) ? (lo >> 4) : (lo & 15);
        int hi = (qh[l] >> (2 * lane)) & 3;
        return (nib | (hi << 4)) - 32;
    }
    case OR_Q5_K: {
        int g = e / 64, half = (e / 32) & 1, lane = e % 32;
        uint8_t packed = block[48 + g * 32 + lane];
        int low = half ? (packed >> 4) : (packed & 15);
        return low + ((block[16 + lane] >> (2 * g + half)) & 1) * 16;
    }
    case OR_Q2_K: {
        int n = e / 128, j = (e / 32) & 3, s = (e / 16) & 1, l = e % 16;
        return (block[16 + 32 * n + 16 * s + l] >> (2 * j)) & 3;
    }
    }
    return 0;
}

int or_block_dots(int dtype, const uint8_t *w, uint32_t rows, uint32_t cols, const int8_t *xq,
                  uint32_t n_tok, int32_t *out)
{
    uint32_t be, bb;
    if (or_block_layout(dtype, &be, &bb) != 0 || dtype == OR_F32 || dtype == OR_F16)
        return -2;
    if (cols % be != 0)
        return -3;
    uint32_t sub = (dtype == OR_Q6_K || dtype == OR_Q2_K) ? 16 : 32;
    uint32_t nsub = cols / sub;
    size_t row_bytes = (size_t)(cols / be) * bb;
    for (uint32_t t = 0; t < n_tok; ++t)
        for (uint32_t r = 0; r < rows; ++r)
            for (uint32_t s = 0; s < nsub; ++s) {
                int32_t acc = 0;
                for (uint32_t i = 0; i < sub; ++i) {
                    uint32_t c = s * sub + i;
                    const uint8_t *block = w + (size_t)r * row_bytes + (size_t)(c / be) * bb;
                    acc += block_code(dtype, block, (int)(c % be)) * xq[(size_t)t * cols + c];
                }
                out[((size_t)t * rows + r) * nsub + s] = acc;
            }
    return 0;
}

/* spm-qwen3-slice/src/math.rs:1-10 == spm-granite-moe/src/math.rs:1-11 ==
 * spm-smol-ops/src/norm.rs:12-21: mean = (sum x*x)/n, scale = 1/sqrt(mean+eps),
 * y = x * scale * w evaluated left to right. */
void or_rms_norm(const float *x, const float *w, uint32_t n, float eps, float *y)
{
    float acc = -0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        float sq = x[i] * x[i];
        acc = acc + sq;
    }
    float mean = acc / (float)n;
    float scale = 1.0f / sqrtf(mean + eps);
    for (uint32_t i = 0; i < n; ++i) {
        float t = x[i] * scale;
        y[i] = t * w[i];
    }
}

/* spm-qwen3-slice/src/attention.rs:11-25 (NEOX halves, angle = pos/theta^(2i/d),
 * x' = x*cos - y*sin, y' = y*cos + x*sin) */
void or_rope_qwen3(float *head, uint32_t dim, uint32_t position, float theta)
{
    uint32_t half = dim / 2;
    for (uint32_t index = 0; index < half; ++index) {
        float index_f = (float)index;
        float width = (float)dim;
        float pos = (float)position;
        float exponent = 2.0f * index_f / width;
        float angle = pos / powf(theta, exponent);
        float s = sinf(angle), c = cosf(angle);
        float left = head[index], right = head[index + half];
        float a = left * c, b = right * s;
        head[index] = a - b;
        float e = right * c, f = left * s;
        head[index + half] = e + f;
    }
}

/* spm-ops/src/attention.rs:20-32 (used through spm-kv/src/attend.rs:13-19):
 * theta = base^(-2i/d) * pos; x' = fma(x, cos, -(y*sin)); y' = fma(x, sin, y*cos). */
void or_rope_fma(float *head, uint32_t dim, uint32_t position, float base)
{
    float width = (float)dim;
    float at = (float)position;
    for (uint32_t pair = 0; pair < dim / 2; ++pair) {
        float index = (float)pair;
        float theta = powf(base, -2.0f * index / width) * at;
        float s = sinf(theta), c = cosf(theta);
        float x = head[pair], y = head[pair + dim / 2];
        head[pair] = fmaf(x, c, -(y * s));
        head[pair + dim / 2] = fmaf(x, s, y * c);
    }
}

/* spm-granite-moe/src/attention.rs:12-26 (adjacent pairs, angle = pos/theta^(p/d)) */
void or_rope_interleaved(float *head, uint32_t dim, uint32_t position, float theta)
{
    for (uint32_t pair = 0; pair < dim; pair += 2) {
        float exponent = (float)pair / (float)dim;
        float pos = (float)position;
        float angle = pos / powf(theta, exponent);
        float s = sinf(angle), c = cosf(angle);
        float h0 = head[pair], h1 = head[pair + 1];
        float a = h0 * c, b = h1 * s;
        float e = h0 * s, f = h1 * c;
        head[pair] = a - b;
        head[pair + 1] = e + f;
    }
}

/* spm-qwen3-slice/src/attention.rs:36-46, spm-kv/src/attend.rs:22-34,
 * spm-granite-moe/src/math.rs:23-29: exp(v - max), sequential total, divide. */
void or_softmax_div(float *v, uint32_t n)
{
    if (n == 0)
        return;
    float max = -INFINITY;
    for (uint32_t i = 0; i < n; ++i)
        max = fmaxf(max, v[i]);
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        v[i] = expf(v[i] - max);
        sum = sum + v[i];
    }
    for (uint32_t i = 0; i < n; ++i)
        v[i] = v[i] / sum;
}

/* spm-ops/src/attention.rs:35-52: multiply by 1/total instead. */
void or_softmax_recip(float *v, uint32_t n)
{
    if (n == 0)
        return;
    float max = v[0];
    for (uint32_t i = 1; i < n; ++i)
        max = fmaxf(max, v[i]);
    float total = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        v[i] = expf(v[i] - max);
        total = total + v[i];
    }
    float scale = 1.0f / total;
    for (uint32_t i = 0; i < n; ++i)
        v[i] = v[i] * scale;
}

/* spm-ops/src/nonlinear.rs:5-7 and the inline forms in spm-qwen3-slice/src/
 * model.rs:113 and spm-granite-moe/src/moe.rs:52: x / (1 + exp(-x)). */
float or_silu(float x)
{
    float e = expf(-x);
    float den = 1.0f + e;
    return x / den;
}

/* spm-granite-moe/src/gemma_smoke.rs:88-90 */
float or_gelu_tanh(float v)
{
    float inner = 0.044715f * v;
    inner = inner * v;
    inner = 1.0f + inner;
    float arg = 0.7978846f * v;
    arg = arg * inner;
    float t = tanhf(arg);
    float half = 0.5f * v;
    return half * (1.0f + t);
}

/* Rust f32::total_cmp key. */
static int32_t total_key(float f)
{
    int32_t i;
    memcpy(&i, &f, 4);
    i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
    return i;
}

typedef struct {
    uint32_t index;
    float value;
} ranked_t;

static int ranked_cmp(const void *a, const void *b)
{
    const ranked_t *l = (const ranked_t *)a, *r = (const ranked_t *)b;
    int32_t kl = total_key(l->value), kr = total_key(r->value);
    if (kl != kr)
        return kl > kr ? -1 : 1; /* descending value */
    return l->index < r->index ? -1 : (l->index > r->index ? 1 : 0);
}

/* spm-qwen3-slice/src/math.rs:38-48, spm-granite-moe/src/math.rs:35-40 */
void or_top_k(const float *v, uint32_t n, uint32_t k, uint32_t *idx, float *val)
{
    ranked_t *r = (ranked_t *)malloc(sizeof(ranked_t) * (n ? n : 1));
    for (uint32_t i = 0; i < n; ++i) {
        r[i].index = i;
        r[i].value = v[i];
    }
    qsort(r, n, sizeof(ranked_t), ranked_cmp);
    for (uint32_t i = 0; i < k && i < n; ++i) {
        idx[i] = r[i].index;
        val[i] = r[i].value;
    }
    free(r);
}

/* spm-granite-moe/src/moe.rs:17-35 with math.rs:23-29 softmax (sum from -0.0). */
void or_route(const float *logits, uint32_t n_experts, uint32_t k, uint32_t *ids, float *weights)
{
    float *p = (float *)malloc(sizeof(float) * n_experts);
    float max = -INFINITY;
    for (uint32_t i = 0; i < n_experts; ++i)
        max = fmaxf(max, logits[i]);
    float sum = -0.0f;
    for (uint32_t i = 0; i < n_experts; ++i) {
        p[i] = expf(logits[i] - max);
        sum = sum + p[i];
    }
    for (uint32_t i = 0; i < n_experts; ++i)
        p[i] = p[i] / sum;
    float *sel = (float *)malloc(sizeof(float) * k);
    or_top_k(p, n_experts, k, ids, sel);
    float total = -0.0f;
    for (uint32_t i = 0; i < k; ++i)
        total = total + sel[i];
    for (uint32_t i = 0; i < k; ++i)
        weights[i] = sel[i] / total;
    free(sel);
    free(p);
}

/* Variant 0: spm-qwen3-slice/src/attention.rs:48-79.
 * Variant 1: spm-kv/src/attend.rs:37-94.
 * Variant 2: spm-granite-moe/src/attention.rs:28-61. */
void or_attend(const float *q, const float *keys, const float *values, uint32_t positions,
               uint32_t heads, uint32_t kv_heads, uint32_t hd, int variant, float c, float *out)
{
    uint32_t group = heads / kv_heads;
    uint32_t stride = kv_heads * hd;
    float *scores = (float *)malloc(sizeof(float) * (positions ? positions : 1));
    float inv = 1.0f / sqrtf((float)hd);
    for (uint32_t head = 0; head < heads; ++head) {
        uint32_t kvh = head / group;
        const float *qh = q + head * hd;
        for (uint32_t p = 0; p < positions; ++p) {
            const float *k = keys + (size_t)p * stride + kvh * hd;
            float dot = -0.0f;
            for (uint32_t i = 0; i < hd; ++i) {
                float t = qh[i] * k[i];
                dot = dot + t;
            }
            if (variant == 0)
                scores[p] = dot / c;
            else if (variant == 1)
                scores[p] = dot * inv;
            else
                scores[p] = dot * c;
        }
        or_softmax_div(scores, positions);
        float *o = out + head * hd;
        for (uint32_t lane = 0; lane < hd; ++lane) {
            if (variant == 1) {
                float acc = 0.0f;
                for (uint32_t p = 0; p < positions; ++p)
                    acc = fmaf(scores[p], values[(size_t)p * stride + kvh * hd + lane], acc);
                o[lane] = acc;
            } else {
                float acc = -0.0f;
                for (uint32_t p = 0; p < positions; ++p) {
                    float t = values[(size_t)p * stride + kvh * hd + lane] * scores[p];
                    acc = acc + t;
                }
                o[lane] = acc;
            }
        }
    }
    free(scores);
}

uint32_t or_argmax(const float *v, uint32_t n, int tie_last)
{
    uint32_t best = 0;
    for (uint32_t i = 1; i < n; ++i) {
        if (tie_last) {
            /* Iterator::max_by(partial_cmp): the last of equal maxima wins
             * (spm-batch/tests/batching.rs:111-123). */
            if (!(v[i] < v[best]))
                best = i;
        } else {
            /* top_k(.., 1): total order, the lowest index wins (math.rs:38-48). */
            if (total_key(v[i]) > total_key(v[best]))
                best = i;
        }
    }
    return best;
}

/* ---------------------------------------------------------------------- */
/* Dense decoder step.                                                     */
/* QWEN3 style composes spm-qwen3-slice/src/model.rs:35-171 (M1 projections,
 * QK-norm + NEOX RoPE, causal_gqa, SwiGLU) one position at a time the way
 * spm-batch/src/step.rs:19-39 drives a decode step.  SMOL style is
 * spm-batch/src/inner.rs:16-105 (M2 streamed projections, rotate_at,
 * attend_cached, tied M1 logits). */

static size_t row_bytes_of(int dtype, uint32_t cols)
{
    uint32_t be, bb;
    if (or_block_layout(dtype, &be, &bb) != 0)
        return 0;
    return (size_t)(cols / be) * bb;
}

size_t or_dense_layer_bytes(const or_dense_cfg *cfg)
{
    uint32_t H = cfg->hidden, QW = cfg->heads * cfg->head_dim, KW = cfg->kv_heads * cfg->head_dim;
    size_t rbH = row_bytes_of(cfg->dtype, H), rbQ = row_bytes_of(cfg->dtype, QW),
           rbF = row_bytes_of(cfg->dtype, cfg->ffn);
    return (size_t)QW * rbH + 2 * (size_t)KW * rbH + (size_t)H * rbQ + 2 * (size_t)cfg->ffn * rbH +
           (size_t)H * rbF;
}

/* Projection of every client's row at once: each weight row is decoded once
 * and applied to each client's vector with that client's own fold, so the
 * result equals one call per client. */
static int project(const or_dense_cfg *cfg, const uint8_t *w, uint32_t rows, uint32_t cols,
                   const float *x, uint32_t n, float *y)
{
    int mode = cfg->style == OR_STYLE_SMOL ? 2 : 1;
    return or_qmatvec(cfg->dtype, w, rows, cols, x, n, y, mode);
}

int or_dense_step(const or_dense_cfg *cfg, const or_dense_weights *w, float *kv_k, float *kv_v,
                  const uint32_t *positions, const uint32_t *tokens, uint32_t n_clients,
                  float *logits, uint32_t n_layers_limit)
{
    const uint32_t H = cfg->hidden, hd = cfg->head_dim, NH = cfg->heads, NKV = cfg->kv_heads;
    const uint32_t QW = NH * hd, KW = NKV * hd, F = cfg->ffn, L = cfg->layers;
    const uint32_t layers_run = n_layers_limit && n_layers_limit < L ? n_layers_limit : L;
    const size_t rbH = row_bytes_of(cfg->dtype, H), rbQ = row_bytes_of(cfg->dtype, QW);
    const size_t layer_bytes = or_dense_layer_bytes(cfg);
    const int smol = cfg->style == OR_STYLE_SMOL;
    const uint32_t n = n_clients;
    if (H % 32 || QW % 32 || F % 32 || NKV == 0 || NH % NKV)
        return -3;
    for (uint32_t ci = 0; ci < n; ++ci)
        if (positions[ci] >= cfg->context)
            return -5; /* context exhausted (spm-kv/src/cache.rs:50-54) */
    if (n == 0)
        return 0;

    /* per client: state, xn, q, k, v, att, proj, gate, up (client-major) */
    size_t per = (size_t)H * 3 + QW * 2 + KW * 2 + F * 2;
    float *buf = (float *)malloc(sizeof(float) * per * n);
    if (!buf)
        return -4;
    float *state = buf, *xn = state + (size_t)H * n, *q = xn + (size_t)H * n, *k = q + (size_t)QW * n,
          *v = k + (size_t)KW * n, *att = v + (size_t)KW * n, *proj = att + (size_t)QW * n,
          *gate = proj + (size_t)H * n, *up = gate + (size_t)F * n;

    /* embedding row: spm-qwen3-slice/src/model.rs:14-23, spm-batch/src/step.rs:27-30 */
    for (uint32_t ci = 0; ci < n; ++ci)
        if (or_decode(cfg->dtype, w->embed + (size_t)tokens[ci] * rbH, rbH, state + (size_t)ci * H) != 0) {
            free(buf);
            return -1;
        }
    for (uint32_t layer = 0; layer < layers_run; ++layer) {
        const uint8_t *base = w->layers + (size_t)layer * layer_bytes;
        const uint8_t *wq = base, *wk = wq + (size_t)QW * rbH, *wv = wk + (size_t)KW * rbH,
                      *wo = wv + (size_t)KW * rbH, *wg = wo + (size_t)H * rbQ,
                      *wu = wg + (size_t)F * rbH, *wd = wu + (size_t)F * rbH;
        for (uint32_t ci = 0; ci < n; ++ci)
            or_rms_norm(state + (size_t)ci * H, w->attn_norm + (size_t)layer * H, H, cfg->eps, xn + (size_t)ci * H);
        project(cfg, wq, QW, H, xn, n, q);
        project(cfg, wk, KW, H, xn, n, k);
        project(cfg, wv, KW, H, xn, n, v);
        for (uint32_t ci = 0; ci < n; ++ci) {
            const uint32_t pos = positions[ci];
            float *cq = q + (size_t)ci * QW, *ck_ = k + (size_t)ci * KW, *cv_ = v + (size_t)ci * KW;
            for (uint32_t h = 0; h < NH; ++h) {
                float *qh = cq + h * hd;
                if (cfg->qk_norm)
                    or_rms_norm(qh, w->q_norm + (size_t)layer * hd, hd, cfg->eps, qh);
                if (smol)
                    or_rope_fma(qh, hd, pos, cfg->rope_theta);
                else
                    or_rope_qwen3(qh, hd, pos, cfg->rope_theta);
            }
            for (uint32_t h = 0; h < NKV; ++h) {
                float *kh = ck_ + h * hd;
                if (cfg->qk_norm)
                    or_rms_norm(kh, w->k_norm + (size_t)layer * hd, hd, cfg->eps, kh);
                if (smol)
                    or_rope_fma(kh, hd, pos, cfg->rope_theta);
                else
                    or_rope_qwen3(kh, hd, pos, cfg->rope_theta);
            }
            /* KvCache::append (spm-kv/src/cache.rs:49-58) */
            float *ck = kv_k + (size_t)ci * L * cfg->context * KW;
            float *cv = kv_v + (size_t)ci * L * cfg->context * KW;
            float *kslot = ck + ((size_t)layer * cfg->context + pos) * KW;
            float *vslot = cv + ((size_t)layer * cfg->context + pos) * KW;
            for (uint32_t i = 0; i < KW; ++i) {
                kslot[i] = cfg->kv_f16 ? or_f16_to_f32(or_f32_to_f16(ck_[i])) : ck_[i];
                vslot[i] = cfg->kv_f16 ? or_f16_to_f32(or_f32_to_f16(cv_[i])) : cv_[i];
            }
            const float *pk = ck + (size_t)layer * cfg->context * KW;
            const float *pv = cv + (size_t)layer * cfg->context * KW;
            if (smol)
                or_attend(cq, pk, pv, pos + 1, NH, NKV, hd, 1, 0.0f, att + (size_t)ci * QW);
            else
                or_attend(cq, pk, pv, pos + 1, NH, NKV, hd, 0, sqrtf((float)hd), att + (size_t)ci * QW);
        }
        project(cfg, wo, H, QW, att, n, proj);
        for (size_t i = 0; i < (size_t)H * n; ++i)
            state[i] = state[i] + proj[i];
        for (uint32_t ci = 0; ci < n; ++ci)
            or_rms_norm(state + (size_t)ci * H, w->ffn_norm + (size_t)layer * H, H, cfg->eps, xn + (size_t)ci * H);
        project(cfg, wg, F, H, xn, n, gate);
        project(cfg, wu, F, H, xn, n, up);
        for (size_t i = 0; i < (size_t)F * n; ++i)
            gate[i] = or_silu(gate[i]) * up[i];
        project(cfg, wd, H, F, gate, n, proj);
        for (size_t i = 0; i < (size_t)H * n; ++i)
            state[i] = state[i] + proj[i];
    }
    for (uint32_t ci = 0; ci < n; ++ci) {
        float *cs = state + (size_t)ci * H, *cx = xn + (size_t)ci * H;
        or_rms_norm(cs, w->out_norm, H, cfg->eps, cx);
    }
    const uint8_t *out_w = cfg->tied ? w->embed : w->output;
    /* logits: M1 over vocabulary rows (spm-qwen3-slice/src/weights.rs:41-63,
     * spm-batch/src/inner.rs:97-104); none when the caller passes no buffer
     * (a prompt step that only fills the cache) */
    if (logits) or_qmatvec(cfg->dtype, out_w, cfg->vocab, H, xn, n, logits, 1);
    free(buf);
    return 0;
}

/* Selected-expert FFN: spm-granite-moe/src/moe.rs:37-159 (expert_tokens,
 * activate, accumulate, process_expert, run) and the Gemma expert form of
 * gemma_smoke.rs:92-139 (fused gate|up rows, gelu, per-expert down scale).
 * Experts run in ascending id (the BTreeSet of moe.rs:134); each projects the
 * tokens routed to it in token order with M1 (weights.rs:41-55 ->
 * math::matvec); output[t] starts at +0.0 and gets lane * weight[slot] added
 * per expert (moe.rs:58-75). */
int or_moe_ffn(const or_moe_desc *d, const float *x, uint32_t n_tok, const uint32_t *ids,
               const float *weights, float *out)
{
    uint32_t be_in, bb_in, be_ff, bb_ff;
    if (or_block_layout(d->enc_gate_up, &be_in, &bb_in) != 0 || or_block_layout(d->enc_down, &be_ff, &bb_ff) != 0)
        return -2;
    if (d->width % be_in != 0 || d->ff % be_ff != 0)
        return -3;
    const size_t rb_in = (size_t)(d->width / be_in) * bb_in, rb_ff = (size_t)(d->ff / be_ff) * bb_ff;
    const uint32_t W = d->width, FF = d->ff, K = d->k;
    float *xs = (float *)malloc(sizeof(float) * (size_t)n_tok * W);
    float *g = (float *)malloc(sizeof(float) * (size_t)n_tok * FF);
    float *u = (float *)malloc(sizeof(float) * (size_t)n_tok * FF);
    float *dn = (float *)malloc(sizeof(float) * (size_t)n_tok * W);
    uint32_t *tok = (uint32_t *)malloc(sizeof(uint32_t) * (n_tok ? n_tok : 1));
    int st = 0;
    for (size_t i = 0; i < (size_t)n_tok * W; ++i)
        out[i] = 0.0f;
    for (uint32_t e = 0; e < d->n_experts && st == 0; ++e) {
        uint32_t cnt = 0;
        for (uint32_t t = 0; t < n_tok; ++t)
            for (uint32_t s = 0; s < K; ++s)
                if (ids[(size_t)t * K + s] == e) {
                    tok[cnt++] = t;
                    break;
                }
        if (cnt == 0)
            continue;
        for (uint32_t i = 0; i < cnt; ++i)
            memcpy(xs + (size_t)i * W, x + (size_t)tok[i] * W, sizeof(float) * W);
        const uint8_t *gw, *uw;
        if (d->up) {
            gw = d->gate + (size_t)e * FF * rb_in;
            uw = d->up + (size_t)e * FF * rb_in;
        } else {
            gw = d->gate + (size_t)e * 2 * FF * rb_in;
            uw = gw + (size_t)FF * rb_in;
        }
        st |= or_qmatvec(d->enc_gate_up, gw, FF, W, xs, cnt, g, 1);
        st |= or_qmatvec(d->enc_gate_up, uw, FF, W, xs, cnt, u, 1);
        for (size_t i = 0; i < (size_t)cnt * FF; ++i) {
            float a = d->act == OR_ACT_GELU_TANH ? or_gelu_tanh(g[i]) : or_silu(g[i]);
            g[i] = a * u[i];
        }
        st |= or_qmatvec(d->enc_down, d->down + (size_t)e * W * rb_ff, W, FF, g, cnt, dn, 1);
        for (uint32_t i = 0; i < cnt; ++i) {
            const uint32_t t = tok[i];
            uint32_t slot = 0;
            while (ids[(size_t)t * K + slot] != e)
                ++slot;
            const float w = weights[(size_t)t * K + slot];
            const float sc = d->down_scale ? d->down_scale[e] : 1.0f;
            for (uint32_t c = 0; c < W; ++c) {
                float v = dn[(size_t)i * W + c];
                if (d->down_scale)
                    v = v * sc;
                float p = v * w;
                out[(size_t)t * W + c] = out[(size_t)t * W + c] + p;
            }
        }
    }
    free(xs);
    free(g);
    free(u);
    free(dn);
    free(tok);
    return st ? -1 : 0;
}

/* ---- mixture-of-experts decoder ------------------------------------------
 * spm-granite-moe/src/model.rs:330-411 (block, run), attention.rs:12-112
 * (interleaved rope, attend with score * 0.015625, add_scaled 0.22),
 * moe.rs:124-159 (router matvec, route, experts) and math.rs:1-40.  The
 * OLMoE form changes only constants and the RoPE / output choices; the
 * Gemma-4 form (oracle.h) follows gemma_smoke.rs for the experts. */
size_t or_moe_layer_bytes(const or_moe_model_cfg *c)
{
    const uint32_t QW = c->heads * c->head_dim, KW = c->kv_heads * c->head_dim, H = c->hidden;
    const size_t rbH = row_bytes_of(c->dtype, H), rbQ = row_bytes_of(c->dtype, QW);
    const size_t rbHe = row_bytes_of(c->expert_dtype, H);
    const size_t attn = (size_t)(QW + 2 * KW) * rbH + (size_t)H * rbQ;
    if (c->gemma) {
        const size_t rbFd = row_bytes_of(c->expert_down_dtype, c->expert_ff);
        const size_t shared = c->shared_ff ? 2 * (size_t)c->shared_ff * rbH +
                                                 (size_t)H * row_bytes_of(c->dtype, c->shared_ff)
                                           : 0;
        return attn + sizeof(float) * ((size_t)c->n_experts * H + H + c->n_experts) + shared +
               (size_t)c->n_experts * (2 * (size_t)c->expert_ff * rbHe + (size_t)H * rbFd);
    }
    const size_t rbFe = row_bytes_of(c->expert_dtype, c->expert_ff);
    return attn + sizeof(float) * c->n_experts * H +
           (size_t)c->n_experts * (2 * (size_t)c->expert_ff * rbHe + (size_t)H * rbFe);
}

static void add_scaled(float *a, const float *b, uint32_t n, float s)
{
    /* math.rs:31-33: a + b * scale, two roundings (built without contraction) */
    for (uint32_t i = 0; i < n; ++i)
        a[i] = s != 0.0f ? a[i] + b[i] * s : a[i] + b[i];
}

/* Gemma router input (gemma_smoke.rs:57-86): rms = (sum x^2 / W + 1e-6)
 * .sqrt().recip() / W.sqrt(); value * scale * rms. */
static void gemma_router_input(const float *x, const float *scale, uint32_t n, float *out)
{
    float acc = -0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        float sq = x[i] * x[i];
        acc = acc + sq;
    }
    const float w = (float)n;
    float mean = acc / w;
    float r = 1.0f / sqrtf(mean + 1e-6f);
    r = r / sqrtf(w);
    for (uint32_t i = 0; i < n; ++i) {
        float t = x[i] * scale[i];
        out[i] = t * r;
    }
}

int or_moe_model_step(const or_moe_model_cfg *c, const or_moe_model_weights *w, float *kv_k, float *kv_v,
                      const uint32_t *positions, const uint32_t *tokens, uint32_t n_clients, float *logits,
                      uint32_t n_layers_limit)
{
    const uint32_t H = c->hidden, hd = c->head_dim, NH = c->heads, NKV = c->kv_heads;
    const uint32_t QW = NH * hd, KW = NKV * hd, E = c->n_experts, K = c->experts_used, L = c->layers;
    const uint32_t FF = c->expert_ff, SF = c->gemma ? c->shared_ff : 0;
    const uint32_t layers_run = n_layers_limit && n_layers_limit < L ? n_layers_limit : L;
    if (NKV == 0 || NH % NKV || E == 0 || K == 0 || K > E || K > 64 || H % 256 || FF % 32)
        return -3;
    if (c->gemma && c->global_every == 0)
        return -3;
    const size_t rbH = row_bytes_of(c->dtype, H), rbQ = row_bytes_of(c->dtype, QW);
    const size_t rbHe = row_bytes_of(c->expert_dtype, H);
    const size_t layer_bytes = or_moe_layer_bytes(c);
    float *buf = (float *)malloc(sizeof(float) * ((size_t)H * 6 + QW * 2 + KW * 2 + E + K + 2 * SF + 16));
    uint32_t ids[64];
    if (!buf) {
        free(buf);
        return -4;
    }
    float *state = buf, *xn = state + H, *q = xn + H, *k = q + QW, *v = k + KW, *att = v + KW, *proj = att + QW,
          *moe = proj + H, *rin = moe + H, *xe = rin + H, *rl = xe + H, *rw = rl + E, *sg = rw + K, *su = sg + SF;
    for (uint32_t ci = 0; ci < n_clients; ++ci) {
        const uint32_t pos = positions[ci];
        if (pos >= c->context) {
            free(buf);
            return -5;
        }
        float *ck = kv_k + (size_t)ci * L * c->context * KW;
        float *cv = kv_v + (size_t)ci * L * c->context * KW;
        /* embeddings (model.rs:196-213): one row decoded, times 12.0 */
        if (or_decode(c->dtype, w->embed + (size_t)tokens[ci] * rbH, rbH, state) != 0) {
            free(buf);
            return -1;
        }
        if (c->embed_scale != 0.0f)
            for (uint32_t i = 0; i < H; ++i)
                state[i] = state[i] * c->embed_scale;
        for (uint32_t layer = 0; layer < layers_run; ++layer) {
            const uint8_t *base = w->layers + (size_t)layer * layer_bytes;
            const uint8_t *wq = base, *wk = wq + (size_t)QW * rbH, *wv = wk + (size_t)KW * rbH,
                          *wo = wv + (size_t)KW * rbH, *wr = wo + (size_t)H * rbQ;
            const int global = !c->gemma || c->window == 0 || (layer + 1) % c->global_every == 0;
            const float theta = c->gemma && global ? c->rope_theta_global : c->rope_theta;
            /* block (model.rs:330-363): attention half */
            or_rms_norm(state, w->attn_norm + (size_t)layer * H, H, c->eps, xn);
            or_qmatvec(c->dtype, wq, QW, H, xn, 1, q, 1);
            or_qmatvec(c->dtype, wk, KW, H, xn, 1, k, 1);
            or_qmatvec(c->dtype, wv, KW, H, xn, 1, v, 1);
            for (uint32_t h = 0; h < NH; ++h) {
                if (c->qk_norm)
                    or_rms_norm(q + h * hd, w->q_norm + (size_t)layer * hd, hd, c->eps, q + h * hd);
                if (c->rope_neox)
                    or_rope_qwen3(q + h * hd, hd, pos, theta);
                else
                    or_rope_interleaved(q + h * hd, hd, pos, theta);
            }
            for (uint32_t h = 0; h < NKV; ++h) {
                if (c->qk_norm)
                    or_rms_norm(k + h * hd, w->k_norm + (size_t)layer * hd, hd, c->eps, k + h * hd);
                if (c->rope_neox)
                    or_rope_qwen3(k + h * hd, hd, pos, theta);
                else
                    or_rope_interleaved(k + h * hd, hd, pos, theta);
            }
            float *kslot = ck + ((size_t)layer * c->context + pos) * KW;
            float *vslot = cv + ((size_t)layer * c->context + pos) * KW;
            for (uint32_t i = 0; i < KW; ++i) {
                kslot[i] = c->kv_f16 ? or_f16_to_f32(or_f32_to_f16(k[i])) : k[i];
                vslot[i] = c->kv_f16 ? or_f16_to_f32(or_f32_to_f16(v[i])) : v[i];
            }
            /* local layers see the last `window` positions, the new one included */
            const uint32_t lo = global || pos + 1 <= c->window ? 0 : pos + 1 - c->window;
            or_attend(q, ck + ((size_t)layer * c->context + lo) * KW, cv + ((size_t)layer * c->context + lo) * KW,
                      pos + 1 - lo, NH, NKV, hd, 2, c->score_mul, att);
            or_qmatvec(c->dtype, wo, H, QW, att, 1, proj, 1);
            add_scaled(state, proj, H, c->residual_scale);
            or_moe_desc d;
            if (c->gemma) {
                const float *router = (const float *)wr, *rscale = router + (size_t)E * H, *dscale = rscale + H;
                const uint8_t *sgw = (const uint8_t *)(dscale + E);
                const uint8_t *suw = sgw + (size_t)SF * rbH, *sdw = suw + (size_t)SF * rbH;
                const uint8_t *gue = sdw + (SF ? (size_t)H * row_bytes_of(c->dtype, SF) : 0);
                const uint8_t *dne = gue + (size_t)E * 2 * FF * rbHe;
                /* router and experts read the residual before the shared FFN */
                gemma_router_input(state, rscale, H, rin);
                or_rms_norm(state, w->ffn_norm2 + (size_t)layer * H, H, 1e-6f, xe);
                if (SF) {
                    or_rms_norm(state, w->ffn_norm + (size_t)layer * H, H, c->eps, xn);
                    or_qmatvec(c->dtype, sgw, SF, H, xn, 1, sg, 1);
                    or_qmatvec(c->dtype, suw, SF, H, xn, 1, su, 1);
                    for (uint32_t i = 0; i < SF; ++i)
                        sg[i] = or_gelu_tanh(sg[i]) * su[i];
                    or_qmatvec(c->dtype, sdw, H, SF, sg, 1, proj, 1);
                    add_scaled(state, proj, H, c->residual_scale);
                }
                or_matvec_m1(router, E, H, rin, rl);
                or_route(rl, E, K, ids, rw);
                d.enc_gate_up = c->expert_dtype;
                d.enc_down = c->expert_down_dtype;
                d.gate = gue;
                d.up = NULL;
                d.down = dne;
                d.down_scale = dscale;
                d.act = OR_ACT_GELU_TANH;
                d.n_experts = E;
                d.width = H;
                d.ff = FF;
                d.k = K;
                if (or_moe_ffn(&d, xe, 1, ids, rw, moe) != 0) {
                    free(buf);
                    return -6;
                }
            } else {
                const uint8_t *wg = wr + sizeof(float) * E * H, *wu = wg + (size_t)E * FF * rbHe,
                              *wd = wu + (size_t)E * FF * rbHe;
                /* MoE half: ffn_norm, router (f32 M1), route, experts, add_scaled */
                or_rms_norm(state, w->ffn_norm + (size_t)layer * H, H, c->eps, xn);
                or_matvec_m1((const float *)wr, E, H, xn, rl);
                or_route(rl, E, K, ids, rw);
                d.enc_gate_up = c->expert_dtype;
                d.enc_down = c->expert_dtype;
                d.gate = wg;
                d.up = wu;
                d.down = wd;
                d.down_scale = NULL;
                d.n_experts = E;
                d.width = H;
                d.ff = FF;
                d.k = K;
                d.act = OR_ACT_SILU;
                if (or_moe_ffn(&d, xn, 1, ids, rw, moe) != 0) {
                    free(buf);
                    return -6;
                }
            }
            add_scaled(state, moe, H, c->residual_scale);
        }
        /* run (model.rs:403-407): output norm, tied projection, / 6.0;
         * none without a logits buffer (a prompt step that only fills the
         * cache) */
        if (!logits) continue;
        or_rms_norm(state, w->out_norm, H, c->eps, xn);
        float *lg = logits + (size_t)ci * c->vocab;
        or_qmatvec(c->dtype, c->untied ? w->output : w->embed, c->vocab, H, xn, 1, lg, 1);
        if (c->logit_div != 0.0f)
            for (uint32_t i = 0; i < c->vocab; ++i)
                lg[i] = lg[i] / c->logit_div;
        if (c->softcap != 0.0f)
            for (uint32_t i = 0; i < c->vocab; ++i) {
                float t = lg[i] / c->softcap;
                lg[i] = c->softcap * tanhf(t);
            }
    }
    free(buf);
    return 0;
}
