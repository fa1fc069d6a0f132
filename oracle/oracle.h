/*
 * oracle.h -- CPU restatement of emufpga's token-loop arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: tests, the smoke
 * entry point and the CPU-baseline leg of the benchmark load it to produce the
 * values the HIP path must reproduce.  Nothing in the product links it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the emufpga repository).  Compiled with -O2 -ffp-contract=off -fno-fast-math
 * so each Rust expression keeps its own rounding: `a * b` then `+` stay two
 * roundings, `mul_add` is `fmaf`, Rust `Sum<f32>` is a left fold from -0.0.
 *
 * Pinning (what checks each function independently of this restatement):
 *   or_f16_to_f32        exhaustive over all 65536 codes against numpy's
 *                        IEEE half conversion (tests/test_oracle.py).
 *   or_decode_q6_k       reference KATs spm-gguf/tests/decode.rs:8-33, the
 *                        q6-pipeline fixture bytes (pipeline.rs:11-20) against
 *                        an independent numpy decoder, and the closed form
 *                        d*sc*(q-32).
 *   or_decode_q5_k       reference KAT decode.rs:35-46, numpy closed form.
 *   or_decode_q8_0       reference KAT decode.rs:48-58, numpy closed form.
 *   or_decode_q2_k       no reference decoder exists (docs/olmoe-placement-
 *                        baseline.md:12).  Pinned against the published GGML
 *                        block_q2_K layout via a numpy restatement written from
 *                        the closed form y = d*(sc&15)*q - dmin*(sc>>4) and
 *                        hand-built single-field blocks.
 *   or_matvec_m1/m2      reference KAT math.rs:62-71 ([[1,2],[3,4]].[5,6]),
 *                        dyadic inputs where every order is exact, and
 *                        sequential-fold brute force in numpy float32.
 *   or_rms_norm          reference KAT math.rs:54-60.
 *   or_rope_*            reference KATs attention.rs:85-99 (identity at 0,
 *                        cos(1)/sin(1) pair at position 1), rotation
 *                        invariance of the pair norm, and the float64
 *                        rotation by pos*theta^(-2i/d) at every index for
 *                        positions 1, 517 and 2047.
 *   or_softmax_*         reference KAT softmax([1000,1000]) == [0.5,0.5].
 *   or_top_k             reference KAT math.rs:67-70 tie order, moe.rs:183-191.
 *   or_attend_*          reference KATs attention.rs:101-131 (GQA head map,
 *                        causal exclusion), single-position identity, and a
 *                        float64 softmax(q.K*scale)V with non-zero queries
 *                        for each variant's score scale.
 *   or_block_dots_*      brute-force integer sums (order independent).
 *   or_dense_step        an independent float64 composition (tests/npref.py
 *                        dense_model_f64) in both styles, Q6_K/Q8_0, tied and
 *                        untied, f32 and fp16 KV, over 8 positions; the
 *                        batched == alone property (spm-batch/tests/
 *                        batching.rs:128-145); planted mistakes (RoPE
 *                        exponents, score scales, SwiGLU order, k QK-norm,
 *                        either residual, final gain, tied output) each fail
 *                        (tests/test_oracle_mutations.py).
 *   or_gelu_tanh         closed form in float64 (error bound), gelu(0) = 0,
 *                        odd-part identity gelu(v) - gelu(-v) = v.
 *   or_moe_ffn           composition of or_qmatvec / or_silu / or_gelu_tanh;
 *                        pinned by the reference's expert-order test
 *                        (moe.rs:166-185: ascending ids), a one-expert case
 *                        equal to a plain SwiGLU FFN, and weights summing the
 *                        same expert twice == that expert's output.
 */
#ifndef EMUFPGA_ORACLE_H
#define EMUFPGA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF dtype ids (spm-gguf/src/parse.rs:10-29). */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q2_K = 10, OR_Q5_K = 13, OR_Q6_K = 14 };

float or_f16_to_f32(uint16_t bits);
uint16_t or_f32_to_f16(float x); /* round-to-nearest-even (fp16 KV cache) */
int or_block_layout(int dtype, uint32_t *elems, uint32_t *bytes);

/* Decoders: return 0, or -1 when len is not a whole number of blocks. */
int or_decode_q6_k(const uint8_t *src, size_t len, float *out);
int or_decode_q5_k(const uint8_t *src, size_t len, float *out);
int or_decode_q8_0(const uint8_t *src, size_t len, float *out);
int or_decode_q2_k(const uint8_t *src, size_t len, float *out);
int or_decode(int dtype, const uint8_t *src, size_t len, float *out);

/* M1: y[r] = sum_c (W[r][c]*x[c]) sequential, separately rounded, from -0.0.
 * M2: out zero-filled then out = fma(w, x, out) in column order. */
void or_matvec_m1(const float *w, uint32_t rows, uint32_t cols, const float *x, float *y);
void or_matvec_m2(const float *w, uint32_t rows, uint32_t cols, const float *x,
                  uint32_t positions, float *out);
/* Threads used by or_qmatvec's row loop (default 1, the reference's
 * single-threaded path); any count gives bit-identical results. */
void or_set_threads(int n);
/* Quantized matvec: decode each row exactly, then M1 (mode 1) or M2 (mode 2)
 * for every token.  x is n_tok x cols, y is n_tok x rows. */
int or_qmatvec(int dtype, const uint8_t *w, uint32_t rows, uint32_t cols, const float *x,
               uint32_t n_tok, float *y, int mode);

/* Integer block dots (the int8-activation mode).  Activations are quantized per
 * 32 consecutive columns: s = amax/127, id = 1/s (0 when s == 0),
 * q = roundf(x*id) (half away from zero).  For each row and each scale
 * sub-block of the weight format (16 columns for Q6_K and Q2_K, 32 for Q8_0
 * and Q5_K) the int32 sum over the sub-block of code * q is written, where the
 * code is the integer the format multiplies by its sub-block scale: Q8_0 i8;
 * Q6_K q-32; Q5_K the 5-bit code; Q2_K the 2-bit code.
 * out is n_tok x rows x (cols/sub). */
void or_quantize_act_q8(const float *x, uint32_t n, int8_t *q, float *scales);
int or_block_dots(int dtype, const uint8_t *w, uint32_t rows, uint32_t cols, const int8_t *xq,
                  uint32_t n_tok, int32_t *out);

void or_rms_norm(const float *x, const float *w, uint32_t n, float eps, float *y);
void or_rope_qwen3(float *head, uint32_t dim, uint32_t position, float theta);
void or_rope_fma(float *head, uint32_t dim, uint32_t position, float base);
void or_rope_interleaved(float *head, uint32_t dim, uint32_t position, float theta);
void or_softmax_div(float *v, uint32_t n);
void or_softmax_recip(float *v, uint32_t n);
float or_silu(float x);

/* top-k by (value desc under total order, index asc).  Returns k items. */
void or_top_k(const float *v, uint32_t n, uint32_t k, uint32_t *idx, float *val);
/* MoE router (moe.rs:17-35): softmax, top_k, renormalize by the rank-order sum. */
void or_route(const float *logits, uint32_t n_experts, uint32_t k, uint32_t *ids, float *weights);

/* Decode attention for one token of one client.
 * q: heads x hd; keys/values: positions x (kv_heads*hd) rows.
 * variant 0: causal_gqa of spm-qwen3-slice (score = dot / c, softmax divide,
 *            out lane = sum v*score sequential from -0.0).
 * variant 1: attend_cached of spm-kv (score = dot * (1/sqrt(hd)), softmax
 *            divide, out = fma(w, v, out) from +0.0).
 * variant 2: granite attend (score = dot * c, softmax divide, sum v*score). */
void or_attend(const float *q, const float *keys, const float *values, uint32_t positions,
               uint32_t heads, uint32_t kv_heads, uint32_t hd, int variant, float c, float *out);

/* gelu with the tanh approximation, spm-granite-moe/src/gemma_smoke.rs:88-90,
 * evaluated left to right: (0.5*v) * (1 + tanh((0.7978846*v) * (1 + (0.044715*v)*v))). */
float or_gelu_tanh(float v);

/* ---- selected-expert FFN of one MoE layer ------------------------------- */
enum { OR_ACT_SILU = 0, OR_ACT_GELU_TANH = 1 };
typedef struct {
    int32_t enc_gate_up, enc_down;
    const uint8_t *gate;      /* n_experts x ff x width blocks (or fused, see up) */
    const uint8_t *up;        /* same layout; NULL: gate holds per expert 2*ff rows, gate then up */
    const uint8_t *down;      /* n_experts x width x ff blocks */
    const float *down_scale;  /* per-expert output scale (gemma_smoke.rs:129-137) or NULL */
    uint32_t n_experts, width, ff, k;
    int32_t act;              /* OR_ACT_* */
} or_moe_desc;
/* moe::run after routing: ids/weights are n_tok x k (or_route's output). */
int or_moe_ffn(const or_moe_desc *d, const float *x, uint32_t n_tok, const uint32_t *ids,
               const float *weights, float *out);

/* ---- dense decoder (one decode step for n clients) ---------------------- */
enum { OR_STYLE_QWEN3 = 0, OR_STYLE_SMOL = 1 };

typedef struct {
    uint32_t hidden, heads, kv_heads, head_dim, ffn, vocab, layers, context;
    float rope_theta, eps;
    int32_t style;   /* OR_STYLE_* */
    int32_t dtype;   /* encoding of every linear, the embedding and the output */
    int32_t kv_f16;  /* round cached K/V to fp16 on append */
    int32_t tied;    /* logits from the embedding matrix */
    int32_t qk_norm; /* per-head RMSNorm on q and k before RoPE */
} or_dense_cfg;

/* layers: per layer, q,k,v,o,gate,up,down bytes back to back (consume order).
 * norms: attn_norm[L][H], ffn_norm[L][H], q_norm[L][hd], k_norm[L][hd], out_norm[H].
 * kv_k/kv_v: per client [layers][context][kv_heads*hd] f32.
 * positions: per client, the position of the token being fed (== cache len). */
typedef struct {
    const uint8_t *layers;
    const uint8_t *embed;
    const uint8_t *output; /* ignored when tied */
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm, *out_norm;
} or_dense_weights;

size_t or_dense_layer_bytes(const or_dense_cfg *cfg);
int or_dense_step(const or_dense_cfg *cfg, const or_dense_weights *w, float *kv_k, float *kv_v,
                  const uint32_t *positions, const uint32_t *tokens, uint32_t n_clients,
                  float *logits, uint32_t n_layers_limit);
/* ---- mixture-of-experts decoder (Granite: spm-granite-moe) -------------- */
typedef struct {
    uint32_t hidden, heads, kv_heads, head_dim, vocab, layers, context;
    uint32_t n_experts, experts_used, expert_ff;
    float rope_theta, eps;
    float embed_scale;    /* embeddings x this (model.rs:196-213: 12.0) */
    float residual_scale; /* residual adds a + b*s (model.rs:356, attention.rs:103-107: 0.22) */
    float logit_div;      /* logits / this (model.rs:405-407: 6.0) */
    float score_mul;      /* attention score = dot * this (attention.rs:40-46: 0.015625) */
    int32_t dtype;        /* q, k, v, o, the embedding (also the tied output) */
    int32_t expert_dtype; /* gate/up/down experts */
    int32_t kv_f16;
    int32_t qk_norm;      /* per-head RMSNorm on q and k before RoPE */
    /* Forms beyond Granite's (all zero: the Granite decoder). */
    int32_t rope_neox;    /* half-split RoPE of spm-qwen3-slice/src/attention.rs:11-25
                             instead of Granite's adjacent pairs */
    int32_t untied;       /* logits from the separate output matrix */
    int32_t gemma;        /* Gemma-4 FFN half, below */
    int32_t expert_down_dtype; /* encoding of the down experts (gemma) */
    uint32_t shared_ff;   /* gemma: width of the shared dense GeGLU FFN (0: none) */
    uint32_t window;      /* gemma: sliding-window length of the local layers (0: all global) */
    uint32_t global_every;/* gemma: layer l is global when (l + 1) % global_every == 0 */
    float rope_theta_global; /* gemma: RoPE base of the global layers */
    float softcap;        /* gemma: logits -> softcap * tanh(logits / softcap) (0: none) */
} or_moe_model_cfg;

/* layers: per layer q, k, v, o, router (f32, n_experts x hidden), gate_exps,
 * up_exps (n_experts x expert_ff x hidden), down_exps (n_experts x hidden x
 * expert_ff), back to back; expert-major as in GGUF (weights.rs:57-73).
 * The gemma form instead holds q, k, v, o, router (f32 n_experts x hidden),
 * router scale (f32 hidden), down scale (f32 n_experts), the shared FFN's
 * gate, up (shared_ff x hidden) and down (hidden x shared_ff) in `dtype`,
 * then gate_up_exps (n_experts x 2*expert_ff x hidden: gate rows then up
 * rows) and down_exps (n_experts x hidden x expert_ff in expert_down_dtype).
 *
 * Gemma-4 FFN half (no reference decoder: the reference runs layer 0's
 * experts only, gemma_smoke.rs): with r the residual after attention,
 *   r += down_s(gelu(gate_s xn) * up_s xn),  xn = rms(r) * ffn_norm
 *   router input  r * rscale * (1/sqrt(mean(r^2) + 1e-6) / sqrt(hidden))
 *                 (gemma_smoke.rs:57-86); softmax, top_k, weights p/sum p
 *                 (gemma_smoke.rs:333-351)
 *   r += sum over routed e, ascending: w_e * dscale_e * down_e(gelu(g) * u),
 *        [g; u] = gate_up_e (rms(r0) * ffn_norm2) (gemma_smoke.rs:92-139,
 *        pre_ffw_norm_2 at :278), r0 the residual before the shared FFN
 * and attention with the half-split RoPE at theta (local layers, keys in the
 * last `window` positions) or rope_theta_global (global layers). */
typedef struct {
    const uint8_t *layers;
    const uint8_t *embed; /* vocab x hidden; the output projection too (tied) */
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm, *out_norm;
    const uint8_t *output; /* untied: vocab x hidden */
    const float *ffn_norm2; /* gemma: the experts' input gains [layer][hidden] */
} or_moe_model_weights;

size_t or_moe_layer_bytes(const or_moe_model_cfg *cfg);
/* One decode step (model.rs:330-411, one position per client). */
int or_moe_model_step(const or_moe_model_cfg *cfg, const or_moe_model_weights *w, float *kv_k, float *kv_v,
                      const uint32_t *positions, const uint32_t *tokens, uint32_t n_clients, float *logits,
                      uint32_t n_layers_limit);

/* greedy selection: tie 0 -> lowest index (top_k), 1 -> last index (max_by). */
uint32_t or_argmax(const float *v, uint32_t n, int tie_last);

/* ---- seeded synthetic weights (synth.c; no reference counterpart) -------
 * The bytes emu_model_synth writes: N(0, sd) draws keyed by (seed, stream,
 * element index), quantized per block.  or_synth_blocks fills nblocks blocks
 * of dtype (OR_Q8_0/Q6_K/Q5_K/Q2_K; -1 otherwise); or_synth_f32 n floats. */
float or_synth_gauss(uint64_t seed, uint64_t stream, uint64_t idx, float sd);
double or_synth_ln_int(uint32_t k);
double or_synth_cos_turn(uint32_t j);
double or_synth_sqrt(double y);
int or_synth_blocks(int dtype, uint8_t *dst, size_t nblocks, uint64_t seed, uint64_t stream, float sd);
void or_synth_f32(float *dst, size_t n, uint64_t seed, uint64_t stream, float sd);

#ifdef __cplusplus
}
#endif
#endif
