/*
 * emuhip.h -- C ABI of libemuhip.so, the MI355X (gfx950) implementation of
 * emufpga's token-loop hot path: GGUF block dequant-dot matvec, decode
 * attention with RoPE and RMSNorm, the MoE router and the selected-expert FFN,
 * and the per-token decode step that drives them.
 *
 * Conventions
 *  - Every entry point returns an emu_status; nothing aborts or throws across
 *    the boundary.  The reference's panics (config bugs, a full KV context)
 *    become EMU_E_CONFIG / EMU_E_CONTEXT_FULL.
 *  - Pointers named d_* are device pointers (from emu_malloc or any HIP
 *    allocation on the context's device).  Pointers named h_* are host memory.
 *  - Compute calls are asynchronous on the context's stream; emu_ctx_sync waits.
 *  - A context is not thread-safe (it mirrors the reference's `&mut` borrows);
 *    separate contexts may be used from separate threads.
 *  - Quantized tensors are GGUF blocks, row-major (each row is cols/block_elems
 *    whole blocks), uploaded byte-for-byte: no repacking.
 *  - Reference citations are relative to the emufpga repository root.
 */
#ifndef EMUHIP_H
#define EMUHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum emu_status {
    EMU_OK = 0,
    /* Partial block: "byte length is not divisible by 210/176/34"
     * (components/cli/crates/spm-gguf/src/tensor.rs:105-107,146-148,195-197);
     * DecodeError::Short (components/format/crates/spm-codec-any/src/decode.rs:8-19). */
    EMU_E_SHORT = 1,
    /* LinearError::WeightCount (components/tensor/crates/spm-linear/src/resident.rs:9-14);
     * "invalid matrix/vector shape" (spm-qwen3-slice/src/math.rs:13-15). */
    EMU_E_SHAPE = 2,
    /* LinearError::ActivationLen (spm-linear/src/resident.rs:15-21, stream.rs:63-71). */
    EMU_E_ACTIVATION_LEN = 3,
    /* LinearError::Truncated (spm-linear/src/resident.rs:27-33, stream.rs:44-49). */
    EMU_E_TRUNCATED = 4,
    /* DecodeError::Unsupported (spm-codec-any/src/decode.rs:43-45); unknown
     * GGUF dtype (spm-gguf/src/parse.rs:10-29). */
    EMU_E_UNSUPPORTED = 5,
    /* KvCache::append "context exhausted" panic (spm-serve spm-kv/src/cache.rs:50-54). */
    EMU_E_CONTEXT_FULL = 6,
    /* attend_cached "heads must group evenly" panic (spm-kv/src/attend.rs:82-85),
     * RoPE position past u16 (spm-qwen3-slice/src/attention.rs:14-16), bad model shape. */
    EMU_E_CONFIG = 7,
    EMU_E_HIP = 8,   /* a HIP runtime call failed */
    EMU_E_ARG = 9,   /* null pointer or out-of-range argument */
    EMU_E_NOMEM = 10, /* device or host allocation refused (tensor.rs:108-110) */
    /* A file refused by its reader: the GGUF parse errors of
     * spm-gguf/src/parse.rs:31-182 and wire.rs:12-90, the .spm HeaderError
     * (spm-header/src/model.rs:63-89) and LayoutError (spm-layout/src/model.rs:127-145),
     * FileError::Incomplete (spm-file/src/error.rs:34-40); the message is in
     * the reader's error string. */
    EMU_E_FORMAT = 11,
    EMU_E_IO = 12 /* the operating system refused a read (tensor.rs:59-66) */
} emu_status;

/* GGUF dtype ids (spm-gguf/src/parse.rs:10-29). */
typedef enum emu_encoding {
    EMU_ENC_F32 = 0,
    EMU_ENC_F16 = 1,
    EMU_ENC_Q8_0 = 8,
    EMU_ENC_Q2_K = 10,
    EMU_ENC_Q5_K = 13,
    EMU_ENC_Q6_K = 14
} emu_encoding;

typedef struct emu_ctx emu_ctx;
typedef struct emu_model emu_model;
typedef struct emu_session emu_session;

/* ---- context, memory ---------------------------------------------------- */
const char *emu_strerror(int status);
/* Text of the last HIP error seen by this context ("" if none). */
const char *emu_last_error(const emu_ctx *ctx);
int emu_ctx_create(int device, emu_ctx **out);
int emu_ctx_destroy(emu_ctx *ctx);
int emu_ctx_sync(emu_ctx *ctx);
/* The hipStream_t the context launches on (returned as void*). */
int emu_ctx_stream(emu_ctx *ctx, void **stream);
/* Device properties: compute units and the device's gfx arch name. */
int emu_device_info(emu_ctx *ctx, int *compute_units, char *arch, size_t arch_len);

int emu_malloc(emu_ctx *ctx, size_t bytes, void **d_out);
int emu_free(emu_ctx *ctx, void *d_ptr);
int emu_memcpy_htod(emu_ctx *ctx, void *d_dst, const void *h_src, size_t bytes);
int emu_memcpy_dtoh(emu_ctx *ctx, void *h_dst, const void *d_src, size_t bytes);
int emu_memcpy_dtod(emu_ctx *ctx, void *d_dst, const void *d_src, size_t bytes);
int emu_memset(emu_ctx *ctx, void *d_dst, int value, size_t bytes);

/* Event timing on the context's stream: record into slot (0..15), then read
 * the elapsed milliseconds between two recorded slots (waits for the later). */
int emu_event_record(emu_ctx *ctx, int slot);
int emu_event_elapsed(emu_ctx *ctx, int start_slot, int end_slot, float *ms);

/* (block elements, block bytes) of a GGUF dtype: layout() of
 * spm-gguf/src/parse.rs:10-29.  EMU_E_UNSUPPORTED for other ids. */
int emu_block_layout(int encoding, uint32_t *block_elems, uint32_t *block_bytes);

/* ---- decode (parity hook) ----------------------------------------------- */
/* Replaces decode_q6_k / decode_q5_k / decode_q8_0
 * (spm-gguf/src/tensor.rs:103,144,193) and adds Q2_K, which the reference
 * lacks.  d_out receives (src_len/block_bytes)*block_elems f32 in the same
 * element order.  EMU_E_SHORT when src_len is not whole blocks. */
int emu_dequant(emu_ctx *ctx, int encoding, const void *d_src, size_t src_len, float *d_out);

/* ---- quantized matvec --------------------------------------------------- */
/* y[t][r] = sum_c W[r][c] * x[t][c] for t < n_tok, r < rows: the projection of
 * spm_linear::streamed (components/tensor/crates/spm-linear/src/stream.rs:31-55),
 * spm-qwen3-slice weights::projection_batch (weights.rs:27-39) and
 * spm-granite-moe weights::project_expert (weights.rs:41-55).
 * W: rows x cols GGUF blocks (w_len bytes, must equal rows * row bytes:
 * EMU_E_SHAPE otherwise, EMU_E_SHORT if cols is not whole blocks).
 * x: n_tok x cols f32 (x_len elements; EMU_E_ACTIVATION_LEN if short).
 * y: n_tok x rows f32, overwritten (zero-fill semantics of stream.rs:41),
 * or accumulated into with EMU_MV_ACCUMULATE.  n_tok 1..8.
 * EMU_MV_LANE_MAJOR: W is in the Q6_K lane-major layout that
 * emu_weights_lane_major makes; taken by Q6_K at one token with 4096 or
 * 12288 columns, EMU_E_UNSUPPORTED otherwise.  Same results, bit for bit.
 * EMU_MV_MFMA_MAJOR: W is in the Q6_K matrix-core operand layout that
 * emu_weights_mfma_major makes (w_len = emu_weights_mfma_major_bytes(rows,
 * cols), EMU_E_SHAPE otherwise); taken by Q6_K at 2..8 tokens on the widths
 * the matrix-core matvec takes, EMU_E_UNSUPPORTED otherwise.  Same results
 * as GGUF order on that kernel, bit for bit.
 * Activations: by default a Q6_K matvec at one token over 4096 or 12288
 * columns, or at 2..8 tokens on the matrix-core widths, carries x as three
 * int8 limbs per column with a power-of-two scale per 16 columns (exact to
 * 2^-20 of each 16-column group's largest |x|) and sums codes x limbs in
 * int32.  EMU_MV_F32_ACT keeps x in f32 for every shape: each weight is
 * dequantized and multiplied in f32, the reference's arithmetic
 * (spm-qwen3-slice/src/math.rs:12-20) up to the order of the additions.
 * It cannot be combined with the two layout flags (EMU_E_UNSUPPORTED). */
enum { EMU_MV_ACCUMULATE = 1u, EMU_MV_LANE_MAJOR = 2u, EMU_MV_MFMA_MAJOR = 4u, EMU_MV_F32_ACT = 8u };
int emu_qmatvec(emu_ctx *ctx, int encoding, const void *d_w, size_t w_len, uint32_t rows,
                uint32_t cols, const float *d_x, size_t x_len, uint32_t n_tok, float *d_y,
                uint32_t flags);

/* Device layout of Q6_K weights for the batch-1 matvec.  No reference
 * counterpart: the reference streams GGUF block order (spm-gguf/src/
 * tensor.rs:103-139), which is kept as the resident order everywhere else.
 * The block stream is cut into chunks of 16 blocks (the last may hold n < 16)
 * and each chunk's bytes are rearranged so that a wavefront's loads read
 * contiguous kilobytes: unit L = 4*block + 2*half + slot finds three
 * 16-byte code words at 16L, 64n + 16L and 128n + 16L, made from its ql low
 * nibble bytes a, ql high nibble bytes b and qh bytes q (byte by byte) as
 *   W0 = (a & 15) | (q & 3) << 4 | (b >> 4 & 3) << 6
 *   W1 = (b & 15) | (q >> 2 & 3) << 4 | (b >> 6) << 6
 *   W2 = (a >> 4) | (q & 0xf0)
 * (the 6-bit codes of three of its four sub-blocks are the low six bits of
 * W0..W2, the fourth's the top two bits of each), its half-block's 8 scale
 * bytes at 192n + 8*(L/2) and its block's d at 208n + 2*(L/4).  Sizes and
 * chunk offsets are unchanged.
 * len must be whole 210-byte blocks (EMU_E_SHORT); src and dst must not
 * overlap (EMU_E_ARG); Q6_K only (EMU_E_UNSUPPORTED). */
int emu_weights_lane_major(emu_ctx *ctx, int encoding, const void *d_src, size_t len, void *d_dst);

/* Device layout of Q6_K weights for the 2..8-token matrix-core matvec.  No
 * reference counterpart (the reference streams GGUF block order,
 * spm-gguf/src/tensor.rs:103-139).  The rows x cols matrix (cols a multiple
 * of 256) is cut into 32-row tiles (the last one padded by repeating the last
 * row) and 256-column blocks; chunk (tile t, block k) is the 6720 bytes at
 * 6720 * (t * cols/256 + k): six 1024-byte code segments, then the tile's 32
 * rows' 16 scale bytes (512 B), then their f16 d (64 B).  Lane l = 32 kh + j
 * of a wavefront reads the 16 bytes at 16 l of each code segment: 24 words
 * holding row j's codes for columns 8 kh .. 8 kh + 7 of each 16-column
 * sub-block s, word 6 (s / 4) + 3 p + w (p: columns 8 kh + 4 p .. + 3;
 * w = 0..2) carrying in byte b the 6-bit code of sub-block 4 (s / 4) + w in
 * its low six bits and bits 2w, 2w + 1 of sub-block 4 (s / 4) + 3's code in
 * its top two.  emu_weights_mfma_major_bytes gives the size (0 if cols is
 * not a multiple of 256).  len must be rows * cols / 256 * 210 (EMU_E_SHAPE);
 * cols a multiple of 256 (EMU_E_SHORT); src and dst must not overlap
 * (EMU_E_ARG); Q6_K only (EMU_E_UNSUPPORTED). */
size_t emu_weights_mfma_major_bytes(uint32_t rows, uint32_t cols);
int emu_weights_mfma_major(emu_ctx *ctx, int encoding, const void *d_src, size_t len, uint32_t rows, uint32_t cols,
                           void *d_dst);

/* Fused forms used by the decode step (no separate reference entry point;
 * each equals a composition of reference calls):
 *  - gain != NULL: x is RMS-normalised with gain and eps first
 *    (spm-smol-ops/src/norm.rs:12-32 pre_norm, spm-qwen3-slice/src/math.rs:1-10);
 *    on the int8-limb kernels the limbs are of x * gain and the RMS factor
 *    multiplies each row's (each gate/up row's) sum, the same product with
 *    the factor's rounding moved: the limb bound above holds for x * gain;
 *  - d_w_up != NULL: SwiGLU pair, y = silu(W x) * (W_up x)
 *    (spm-batch/src/inner.rs:103-107, spm-qwen3-slice/src/model.rs:93-116). */
int emu_qmatvec_fused(emu_ctx *ctx, int encoding, const void *d_w, const void *d_w_up,
                      uint32_t rows, uint32_t cols, const float *d_x, uint32_t n_tok,
                      const float *d_gain, float eps, float *d_y, uint32_t flags);

/* ---- int8-activation mode (integer block dots) -------------------------- */
/* No reference counterpart: the reference multiplies f32 activations only.
 * Quantize x (n_tok x cols, cols % 32 == 0) per 32 columns: s = amax/127,
 * q = roundf(x * (1/s)), clamped to [-127,127]. */
int emu_quantize_act(emu_ctx *ctx, const float *d_x, uint32_t n_tok, uint32_t cols,
                     int8_t *d_q, float *d_scales);
/* Exact int32 sums of (weight code) * q over each scale sub-block (16 columns
 * for Q6_K/Q2_K, 32 for Q8_0/Q5_K); out is n_tok x rows x (cols/sub). */
int emu_block_dots(emu_ctx *ctx, int encoding, const void *d_w, size_t w_len, uint32_t rows,
                   uint32_t cols, const int8_t *d_q, uint32_t n_tok, int32_t *d_out);
/* y = W x with x given as int8 blocks + scales (the integer-dot matvec). */
int emu_qmatvec_i8(emu_ctx *ctx, int encoding, const void *d_w, size_t w_len, uint32_t rows,
                   uint32_t cols, const int8_t *d_q, const float *d_scales, uint32_t n_tok,
                   float *d_y);

/* What HBM delivers on this device: every 16-byte word of d_buf (bytes long,
 * larger than the 256 MB Infinity Cache for a DRAM figure) read once per
 * pass with the non-temporal hint the decode step's weight loads use, passes
 * back to back after one untimed pass, timed with HIP events; gbs = bytes *
 * passes / time.  The storage rate of the scan metrics' storage_time (the
 * reference's raw_bandwidth is bytes over measured storage time,
 * spm-stream-metrics/src/rates.rs:12-17).  The buffer's first word may be
 * overwritten.  d_buf may be any device-addressable memory: with the device
 * address of pinned host memory (emu_host_device_pointer) it measures the
 * host-memory stream over PCIe instead. */
int emu_hbm_read_rate(emu_ctx *ctx, const void *d_buf, size_t bytes, uint32_t passes, float *gbs);

/* ---- norms, RoPE, attention, router, selection -------------------------- */
/* out[r] = x[r] * (1/sqrt(mean(x[r]^2) + eps)) * gain, for n_rows rows of width
 * (spm-smol-ops/src/norm.rs:12-21; spm-qwen3-slice/src/math.rs:1-10). */
int emu_rms_norm(emu_ctx *ctx, const float *d_x, const float *d_gain, uint32_t n_rows,
                 uint32_t width, float eps, float *d_out);

/* RoPE styles. */
enum {
    EMU_ROPE_NEOX = 0,       /* halves: spm-qwen3-slice/src/attention.rs:11-25 and
                                spm-ops/src/attention.rs:20-32 */
    EMU_ROPE_INTERLEAVED = 1, /* adjacent pairs: spm-granite-moe/src/attention.rs:12-26 */
    EMU_ROPE_NEOX_FMA = 2     /* halves, spm_ops::rope (spm-ops/src/attention.rs:20-32, used by
                                 spm-kv/src/attend.rs:13-19): angle base^(-2i/d) * pos,
                                 x' = fma(x, cos, -(y*sin)), y' = fma(x, sin, y*cos) */
};
/* Host-built cos/sin table (glibc powf/sinf/cosf, the reference's libm):
 * d_table[pos][i] = (cos, sin) of pos / theta^(2i/head_dim), pos < positions.
 * Built on the host and uploaded; bytes = positions * head_dim/2 * 8. */
int emu_rope_table(emu_ctx *ctx, uint32_t positions, uint32_t head_dim, float theta,
                   float *d_table);
/* The table of one RoPE style: EMU_ROPE_NEOX and EMU_ROPE_INTERLEAVED take
 * pos / theta^(2i/head_dim) (as emu_rope_table); EMU_ROPE_NEOX_FMA takes
 * theta^(-2i/head_dim) * pos (spm-ops/src/attention.rs:24-27). */
int emu_rope_table_style(emu_ctx *ctx, int style, uint32_t positions, uint32_t head_dim, float theta,
                         float *d_table);
/* rotate_at (spm-kv/src/attend.rs:13-19): rotate n_tok tokens of `heads` heads
 * in place, token t at position d_positions[t]. */
int emu_rope(emu_ctx *ctx, float *d_x, uint32_t n_tok, uint32_t heads, uint32_t head_dim,
             const uint32_t *d_positions, const float *d_table, uint32_t table_positions,
             int style);

/* attend_cached (spm-kv/src/attend.rs:75-94) for one token over a cached
 * prefix of `positions` rows.  keys/values: f32 or f16 (kv_f16 != 0) rows of
 * kv_heads*head_dim; score = dot * scale; softmax; weighted sum of values. */
int emu_attend_cached(emu_ctx *ctx, const float *d_q, const void *d_keys, const void *d_values,
                      int kv_f16, uint32_t positions, uint32_t heads, uint32_t kv_heads,
                      uint32_t head_dim, float scale, float *d_out);
/* emu_attend_cached that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The scores
 * go to a fixed device scratch of 1,048,576 floats (4 MiB) per device, held
 * until the process ends: heads * positions beyond that is EMU_E_CONFIG.
 * Calls that overlap on one device share that scratch and race. */
int emu_attend_cached_noalloc(emu_ctx *ctx, const float *d_q, const void *d_keys, const void *d_values,
                              int kv_f16, uint32_t positions, uint32_t heads, uint32_t kv_heads,
                              uint32_t head_dim, float scale, float *d_out);

/* moe::route (spm-granite-moe/src/moe.rs:17-35): softmax over n_experts
 * logits per token, top-k by (prob desc, id asc), weights renormalised by the
 * selected sum.  ids/weights are n_tok x k. */
int emu_route(emu_ctx *ctx, const float *d_logits, uint32_t n_tok, uint32_t n_experts,
              uint32_t k, int32_t *d_ids, float *d_weights);

/* Selected-expert FFN of one MoE layer for n_tok (<= 8) tokens after routing:
 * moe::run (spm-granite-moe/src/moe.rs:37-159: expert_tokens, activate,
 * process_expert, accumulate) with weights::project_expert
 * (weights.rs:41-55), and the Gemma expert form (gemma_smoke.rs:92-139: one
 * fused gate|up matrix per expert, gelu, a per-expert down scale).
 * For token t: out[t] = +0.0, then for its slots in ascending expert id,
 * out[t] += down_e(act(gate_e x_t) * up_e x_t) (* down_scale[e]) * weight.
 * Expert tensors are expert-major GGUF blocks: gate/up n_experts x ff rows of
 * width columns (d_up NULL: d_gate holds 2*ff rows per expert, gate rows
 * then up rows); down n_experts x width rows of ff columns.  ids/weights are
 * n_tok x k as emu_route writes them (distinct ids per token).  The
 * workspace holds n_tok*k activation rows and contributions
 * (emu_moe_workspace_bytes). */
enum { EMU_ACT_SILU = 0, EMU_ACT_GELU_TANH = 1 };
/* flags: EMU_MOE_F32_ACT runs the experts on f32 activations (the vector
 * form: dequant + f32 FMA per weight) instead of the int8-limb matrix-core
 * form.  The matrix-core form takes layers of up to 256 experts; wider layers
 * take the vector form whatever the flags say. */
enum { EMU_MOE_F32_ACT = 1u };
typedef struct emu_moe_desc {
    int32_t enc_gate_up, enc_down;
    const void *d_gate, *d_up, *d_down;
    const float *d_down_scale; /* per-expert output scale or NULL */
    uint32_t n_experts, width, ff, k;
    int32_t act;               /* EMU_ACT_* */
    uint32_t flags;            /* EMU_MOE_* */
} emu_moe_desc;
size_t emu_moe_workspace_bytes(uint32_t n_tok, uint32_t k, uint32_t width, uint32_t ff);
int emu_moe_ffn(emu_ctx *ctx, const emu_moe_desc *desc, const float *d_x, uint32_t n_tok,
                const int32_t *d_ids, const float *d_weights, void *d_workspace, size_t workspace_bytes,
                float *d_out);

/* ---- expert cache: experts in host memory behind HBM slots -------------
 * The reference's ExpertCache (spm-granite-moe/src/expert_cache.rs:20-90) in
 * front of the GPU: n_slots HBM slots of expert_bytes hold resident experts;
 * an expert is admitted on its second miss (admit on second use), evicting
 * the least recently used resident expert, or with layer_aware the least
 * recently used one of the incoming expert's layer first
 * (tools/llama-logits/mmid-cache.hpp:134-173).  An expert not admitted is
 * streamed through one of n_transient slots for that call.  Experts of the
 * call in progress are never evicted by it.  An expert's host bytes are its
 * gate rows, up rows (ff x width each, in desc's enc_gate_up)
 * and down rows (width x ff) back to back, registered per (layer, expert);
 * they are uploaded with hipMemcpyAsync, so pinned memory (emu_host_alloc)
 * lets the copies run asynchronously. */
typedef struct emu_expert_cache emu_expert_cache;
typedef struct emu_cache_stats {
    uint64_t hits, misses, loads, evictions, streamed, bytes_uploaded;
    uint32_t resident;       /* slots holding an expert */
    uint64_t bytes_streamed; /* device policy: miss bytes the expert kernels read from host memory */
} emu_cache_stats;
int emu_host_alloc(emu_ctx *ctx, size_t bytes, void **h_out);
int emu_host_free(emu_ctx *ctx, void *h);
/* The device address of pinned host memory (from emu_host_alloc), which
 * kernels read over PCIe: the expert cache's misses, or emu_hbm_read_rate to
 * measure what that stream delivers. */
int emu_host_device_pointer(emu_ctx *ctx, void *h, void **d_out);
int emu_expert_cache_create(emu_ctx *ctx, uint32_t layers, uint32_t n_experts, size_t expert_bytes,
                            uint32_t n_slots, uint32_t n_transient, int layer_aware, emu_expert_cache **out);
int emu_expert_cache_destroy(emu_expert_cache *c);
int emu_expert_cache_set_source(emu_expert_cache *c, uint32_t layer, uint32_t expert, const void *h_bytes);
int emu_expert_cache_stats(const emu_expert_cache *c, emu_cache_stats *out);
/* The resident slot of (layer, expert), or -1. */
int emu_expert_cache_slot(const emu_expert_cache *c, uint32_t layer, uint32_t expert, int32_t *slot);
/* emu_moe_ffn with the layer's experts taken through the cache: h_ids is the
 * host copy of d_ids (n_tok x k), which decides what to upload; each
 * distinct expert is looked up once, in ascending id (the reference's
 * BTreeSet order).  d_gate/d_up/d_down of desc are not used.  EMU_E_CONFIG
 * when more experts must stream through than there are transient slots;
 * EMU_E_SHAPE when expert_bytes does not match desc. */
int emu_moe_ffn_cached(emu_ctx *ctx, const emu_moe_desc *desc, emu_expert_cache *c, uint32_t layer,
                       const float *d_x, uint32_t n_tok, const int32_t *h_ids, const int32_t *d_ids,
                       const float *d_weights, void *d_workspace, size_t workspace_bytes, float *d_out);
/* Every expert of a mixture-of-experts model as the cache's backing store:
 * expert e of layer l (gate rows, up rows, down rows) copied from the
 * model's HBM tensors to h_buf + (l * n_experts + e) * stride, stride =
 * expert_bytes rounded up to 256, and registered as its source.  h_buf must
 * hold layers * n_experts * stride bytes (EMU_E_ARG) and be pinned
 * (emu_host_alloc) for the device policy; the cache's shape must be the
 * model's (EMU_E_SHAPE).  No reference counterpart: the reference reads
 * experts from its GGUF file (spm-granite-moe/src/weights.rs:57-73). */
int emu_expert_cache_load_model(emu_expert_cache *c, emu_model *model, void *h_buf, size_t h_len);
/* The cache policy alone, on the CPU (no device): n lookups (calls[i] groups
 * them into calls; layers[i], experts[i]), each outcome 0 hit, 1 admitted,
 * 2 streamed through, and the slot (-1 when streamed). */
int emu_expert_cache_policy_trace(uint32_t n_slots, int layer_aware, const uint32_t *calls,
                                  const uint32_t *layers, const uint32_t *experts, uint32_t n,
                                  int32_t *outcome, int32_t *slot);

/* Greedy selection over n_rows rows of width: tie_last 0 = lowest index of the
 * maximum (top_k, spm-qwen3-slice/src/math.rs:38-48); 1 = last index
 * (max_by(partial_cmp), spm-batch/tests/batching.rs:111-123). */
int emu_argmax(emu_ctx *ctx, const float *d_x, uint32_t n_rows, uint32_t width, int tie_last,
               int32_t *d_out);

/* ---- dense decoder model and decode step (serve API) -------------------- */
enum { EMU_STYLE_QWEN3 = 0, EMU_STYLE_SMOL = 1, EMU_STYLE_GRANITE = 2 };

typedef struct emu_model_config {
    uint32_t hidden, heads, kv_heads, head_dim, ffn, vocab, layers;
    float rope_theta, eps;
    int32_t style;    /* EMU_STYLE_*: QK-norm + top_k greedy (Qwen3) or the
                         spm-batch SmolLM2 path (max_by greedy) */
    int32_t encoding; /* every linear, the embedding and the output matrix */
    int32_t tied;     /* logits from the embedding matrix (SmolLM2) */
    int32_t qk_norm;  /* per-head RMSNorm of q and k before RoPE (Qwen3) */
    /* EMU_STYLE_GRANITE (spm-granite-moe/src/model.rs:330-411): adjacent-pair
       RoPE (attention.rs:12-26), a tied output, and mixture-of-experts layers:
       an f32 router (n_experts x hidden, moe.rs:132-138) and experts_used of
       n_experts SwiGLU experts of width expert_ff in expert_encoding in place
       of the dense FFN (ffn unused).  Zero fields keep the plain forms. */
    uint32_t n_experts, experts_used, expert_ff;
    int32_t expert_encoding;
    float embed_scale;    /* embeddings x this (model.rs:196-213: 12.0) */
    float residual_scale; /* residual adds r + v * this (model.rs:356, attention.rs:103-107: 0.22) */
    float logit_div;      /* logits / this before selection (model.rs:405-407: 6.0) */
    float score_mul;      /* attention score = dot * this (attention.rs:40-46: 0.015625) */
    /* More mixture-of-experts forms (EMU_STYLE_GRANITE; zeros keep Granite's).
       rope_neox: the half-split RoPE of spm-qwen3-slice/src/attention.rs:11-25
       (the OLMoE-shaped decoder, which also takes tied = 0 for its separate
       output matrix and qk_norm for per-head QK-norm).
       gemma: the Gemma-4 FFN half.  No reference decoder exists for it (the
       reference runs layer 0's experts, gemma_smoke.rs), so it is defined
       here from those pieces: with r the residual after attention,
         r0 = r; r += down_s(gelu(gate_s x) * up_s x), x = rms(r0) * ffn_norm
             (a shared dense GeGLU FFN of shared_ff, in `encoding`; none if 0)
         router input r0 * rscale * (1/sqrt(mean(r0^2) + 1e-6) / sqrt(hidden))
             (gemma_smoke.rs:57-86), softmax, top_k, w = p / sum p (:333-351)
         r += sum over routed experts, ascending id, of
             w * dscale[e] * down_e(gelu(g) * u), [g; u] = gate_up_e(rms(r0) *
             ffn_norm2) (fused gate|up rows in expert_encoding, downs in
             expert_down_encoding; gemma_smoke.rs:92-139, pre_ffw_norm_2 :278);
       layers attend to the last `window` positions (window 0: all) except
       every global_every-th (l % global_every == global_every - 1), which
       attend to all and take rope_theta_global; logits are soft-capped as
       logit_softcap * tanh(l / logit_softcap) when logit_softcap != 0. */
    int32_t rope_neox, gemma, expert_down_encoding;
    uint32_t shared_ff, window, global_every;
    float rope_theta_global, logit_softcap;
} emu_model_config;

/* Tensor kinds addressable inside a model. */
enum {
    EMU_T_LAYER = 0,    /* layer's q,k,v,o,gate,up,down blocks back to back (consume order) */
    EMU_T_EMBED = 1,    /* vocab x hidden */
    EMU_T_OUTPUT = 2,   /* vocab x hidden (absent when tied) */
    EMU_T_ATTN_NORM = 3, EMU_T_FFN_NORM = 4, EMU_T_Q_NORM = 5, EMU_T_K_NORM = 6,
    EMU_T_OUT_NORM = 7, /* f32 gains */
    EMU_T_FFN_NORM2 = 8 /* gemma: the experts' input gains [layer][hidden] (pre_ffw_norm_2) */
};

/* EMU_E_CONFIG for shapes the kernels do not take; the mixture-of-experts
 * forms need n_experts <= 256, experts_used <= 8 and hidden a multiple of 8
 * up to 4096. */
int emu_model_create(emu_ctx *ctx, const emu_model_config *cfg, emu_model **out);
int emu_model_destroy(emu_model *model);
/* Device address and size of a tensor inside the model's HBM residency (for
 * uploading real weights or reading them back).  layer is ignored for
 * model-wide tensors. */
int emu_model_tensor(emu_model *model, int kind, uint32_t layer, void **d_ptr, size_t *bytes);
/* Seeded synthetic weights: every quantized tensor from N(0, 0.02) draws,
 * quantized on the device; gains 1.0. */
int emu_model_synth(emu_model *model, uint64_t seed);
/* Rebuild the model's lane-major copy of the Q6_K matrices that the batch-1
 * step reads (emu_weights_lane_major).  The decode entry points do this by
 * themselves after emu_model_synth, the GGUF loaders and any
 * emu_model_tensor call; call it after writing weights through a pointer
 * that emu_model_tensor returned earlier. */
int emu_model_sync(emu_model *model);
/* Device address of the lane-major copy: a layer (same offsets as its
 * EMU_T_LAYER tensor; only the matrices whose columns the batch-1 limb
 * matvec takes are filled) or EMU_T_OUTPUT (the output rows, or the tied
 * embedding's).  Brings the copy up to date first.  EMU_E_UNSUPPORTED when
 * the model keeps no such copy (not Q6_K, or no 4096/12288-column matrix). */
int emu_model_tensor_lane_major(emu_model *model, int kind, uint32_t layer, void **d_ptr, size_t *bytes);
/* Algorithmic weight bytes one decode step reads (all linears + output rows). */
int emu_model_weight_bytes(const emu_model *model, uint64_t *bytes);
/* HBM the model's parameters hold: its allocation in GGUF order (every
 * tensor, norms included) plus the lane-major and matrix-core operand copies
 * of its Q6_K matrices (about three times the weights for a dense Q6_K
 * model).  No reference counterpart. */
int emu_model_resident_bytes(const emu_model *model, uint64_t *bytes);

/* A set of clients (spm-batch/src/session.rs:13-38 Client, :46-79 Scratch):
 * per-client KV caches of `context` positions (f16 when kv_f16, else f32). */
int emu_session_create(emu_model *model, uint32_t n_clients, uint32_t context, int kv_f16,
                       emu_session **out);
int emu_session_destroy(emu_session *s);
int emu_session_reset(emu_session *s);
/* A fresh client in slot `client` while the others keep going (a new
 * Client::new, spm-batch/src/session.rs:24-31, swapped into the batch): its
 * position and step count return to 0 and the next decode step feeds it its
 * first token. */
int emu_session_reset_client(emu_session *s, uint32_t client);
/* decode_step (spm-batch/src/step.rs:19-39): feed h_tokens[c] to client c at
 * its current position, advance every position by one, and greedily select
 * each client's next token.  h_next may be NULL.  d_logits, when non-NULL,
 * receives n_clients x vocab logits. */
int emu_decode_step(emu_session *s, const uint32_t *h_tokens, uint32_t *h_next, float *d_logits);
/* Greedy generation: feed h_prompt (n_clients x prompt_len, one token per step
 * as examples/serve-demo.rs:62-91 does), then produce `steps` tokens per
 * client into h_out (n_clients x steps).  The loop is device-resident: token
 * selection feeds the next step without host round trips. */
int emu_generate(emu_session *s, const uint32_t *h_prompt, uint32_t prompt_len, uint32_t steps,
                 uint32_t *h_out);
/* Time `steps` greedy steps (after the caller's warmup) with events around the
 * region; ms receives the elapsed time. */
int emu_time_decode(emu_session *s, uint32_t steps, float *ms);
/* One decode step timed interval by interval (HIP events on the library's
 * stream, kernels launched one by one): h_us[0] the embedding, h_us[1 + l]
 * layer l, h_us[layers + 1] the output matvec and the selection, in
 * microseconds; n must be at least layers + 2 (EMU_E_ARG).  Consumes one
 * position like emu_time_decode (EMU_E_CONTEXT_FULL when none is left).  The
 * reference times its serial MoE layers the same way, read/decode/compute per
 * layer (spm-granite-moe/src/layout.rs:215-239); here reading and decoding
 * happen inside the same kernels as the arithmetic, so a layer is one
 * interval. */
int emu_session_time_layers(emu_session *s, float *h_us, uint32_t n);
/* Session options (0 by default), applied from the next step on:
 *  - EMU_SESSION_F32_ACT: every matvec and expert keeps its activations in
 *    f32 (dequant + f32 FMA per weight, the reference's arithmetic up to the
 *    order of the additions: spm-qwen3-slice/src/math.rs:12-20,
 *    spm-linear/src/stream.rs:31-125) instead of the int8-limb kernels
 *    (activations exact to 2^-20 of each 16- or 256-column group's largest
 *    |x|).  Slower; the mode in which greedy tokens are held identical to the
 *    reference's over long runs.
 *  - EMU_SESSION_DIRECT: the step's kernels are launched one by one instead
 *    of being captured once into a HIP graph and replayed (same kernels,
 *    same order, same results), for profilers and tracers.
 * No reference counterpart (the reference has one arithmetic and no graphs).
 * EMU_E_ARG for unknown bits. */
enum { EMU_SESSION_F32_ACT = 1u, EMU_SESSION_DIRECT = 2u };
int emu_session_set_options(emu_session *s, uint32_t flags);
/* The session's mixture-of-experts steps read their experts through the
 * expert cache instead of the model's tensors: per layer, after routing, the
 * cache's policy (the same admit-on-second-use LRU and layer-aware choice as
 * emu_moe_ffn_cached, expert_cache.rs:20-90, mmid-cache.hpp:134-173) runs on
 * the device over the routes the step just wrote, the layer's experts of the
 * step all in use until it ends.  A hit reads its HBM slot; an admission is
 * copied from its pinned host bytes into its slot by a copy kernel right
 * after the plan and read from there; any other miss is read by the expert
 * kernels straight from its host bytes (over PCIe, while the resident experts
 * compute in the same launch), so every missed byte crosses PCIe once.  The
 * step stays one captured graph.  Counters (emu_expert_cache_stats) come from
 * the device: bytes_uploaded the admissions' copies, bytes_streamed the other
 * misses read from host memory.  Sources: every (layer, expert) registered, pinned and 16-byte
 * aligned (emu_expert_cache_load_model), EMU_E_ARG otherwise; at most 2048
 * slots and 256 experts (EMU_E_CONFIG); the cache's shape must be the
 * model's (EMU_E_SHAPE).  Once attached, the cache's policy state is the
 * device's and emu_moe_ffn_cached refuses it (EMU_E_CONFIG).  NULL detaches. */
int emu_session_attach_expert_cache(emu_session *s, emu_expert_cache *c);
/* Routing for throughput runs of a mixture-of-experts model: with zipf_s > 0
 * every (client, position, layer) routes by the logits -s*ln(e+1) + G_e
 * (G_e Gumbel draws seeded by `seed`) in place of the router's, so its top k
 * is a sample without replacement with P(e) proportional to (e+1)^-s; the
 * router is still read.  zipf_s = 0 restores the model's own router.  No
 * reference counterpart (the reference routes by its router only). */
int emu_session_route_zipf(emu_session *s, float zipf_s, uint64_t seed);
/* Record every step's routes on the device: [capacity][layer][client][k]
 * expert ids and weights, a step going to slot (client's step count) %
 * capacity; the RouteEvent data of spm-viz-trace/src/lib.rs:27-39.
 * capacity 0 stops recording.  Mixture-of-experts models only. */
int emu_session_route_trace(emu_session *s, uint32_t capacity);
/* One slot of the route trace: layers x clients x k ids (-1 before any step
 * wrote the slot) and, when h_weights is not NULL, their weights. */
int emu_session_read_routes(emu_session *s, uint32_t slot, int32_t *h_ids, float *h_weights);
/* Current position (tokens consumed) of every client. */
int emu_session_positions(emu_session *s, uint32_t *h_positions);
/* Copy a client's cached K or V rows for one layer (positions x kv_width f32). */
int emu_session_read_kv(emu_session *s, uint32_t client, uint32_t layer, int which_v,
                        float *h_out, uint32_t positions);

/* ---- GGUF files (components/cli/crates/spm-gguf) ------------------------
 * A bounded, non-executing reader: the header, metadata and tensor directory
 * are parsed under the reference's limits (lib.rs:11-16) with its error texts;
 * tensor bodies are reached only through bounded range reads. */
typedef struct emu_gguf emu_gguf;
typedef struct emu_gguf_tensor_info { /* TensorInfo (spm-gguf/src/model.rs:3-10) */
    const char *name;                 /* valid while the reader is open */
    size_t name_len;                  /* bytes of name (names may hold NUL) */
    uint32_t n_dims;
    uint64_t dims[8];                 /* GGML order: dims[0] is the row length */
    uint32_t dtype;                   /* GGML dtype id */
    uint64_t offset;                  /* absolute file offset of the tensor's bytes */
    uint64_t len;                     /* bytes */
} emu_gguf_tensor_info;

/* spm_gguf::read (parse.rs:157-182).  On failure h_err (may be NULL) receives
 * the reference's message and no reader is returned. */
int emu_gguf_open(const char *path, emu_gguf **out, char *h_err, size_t err_len);
int emu_gguf_close(emu_gguf *g);
/* Message of the reader's last failed call. */
const char *emu_gguf_error(const emu_gguf *g);
/* Content's version, metadata_count, tensor_data_offset and tensor count. */
int emu_gguf_summary(const emu_gguf *g, uint32_t *version, uint64_t *metadata_count,
                     uint64_t *tensor_data_offset, uint64_t *tensor_count);
/* Metadata entry `index` in file order, the value rendered as the reference's
 * Content::metadata holds it ("<6>" for f32, "<9>" for arrays, "<12>" for f64).
 * The strings live as long as the reader; the lengths count every byte. */
int emu_gguf_metadata_at(const emu_gguf *g, uint64_t index, const char **key, size_t *key_len,
                         const char **value, size_t *value_len);
/* The numeric value of a scalar metadata entry, floats included (the
 * reference keeps no float values; model configuration needs them).
 * EMU_E_ARG when absent, EMU_E_UNSUPPORTED for strings and arrays. */
int emu_gguf_metadata_number(const emu_gguf *g, const char *key, double *value);
/* Tensor `index` in ascending file offset (Content::tensors order). */
int emu_gguf_tensor_at(const emu_gguf *g, uint64_t index, emu_gguf_tensor_info *info);
/* Index of a tensor by name; EMU_E_FORMAT "missing tensor NAME"
 * (spm-granite-moe/src/weights.rs:9-15). */
int emu_gguf_find(emu_gguf *g, const char *name, uint64_t *index);
/* read_tensor_range (tensor.rs:35-67): len bytes at rel_off inside the tensor,
 * refused past max_bytes or past the tensor's end. */
int emu_gguf_read_range(emu_gguf *g, uint64_t index, uint64_t rel_off, uint64_t len, uint64_t max_bytes,
                        void *h_dst);
/* The same range placed in device memory: the file is read through two
 * pinned 64 MiB host buffers so reading overlaps the copies.  Synchronous. */
int emu_gguf_upload(emu_ctx *ctx, emu_gguf *g, uint64_t index, uint64_t rel_off, uint64_t len, void *d_dst);

/* Every weight tensor of a model from a GGUF file of the model's architecture,
 * by the reference's tensor names (spm-qwen3-slice/src/model.rs:42-167,
 * spm-granite-moe/src/model.rs, weights.rs:57-94): token_embd, output (untied),
 * output_norm, blk.N.{attn_norm, attn_q, attn_k, attn_v, attn_output,
 * attn_q_norm, attn_k_norm (qk_norm), ffn_norm, ffn_gate, ffn_up, ffn_down}, or
 * for mixture-of-experts layers ffn_gate_inp (f32 router) and the expert-major
 * ffn_gate_exps / ffn_up_exps / ffn_down_exps.  Each tensor's dtype and shape
 * must be what the model was created with (EMU_E_FORMAT otherwise, message in
 * emu_last_error). */
int emu_model_load_gguf(emu_model *model, emu_gguf *g);

/* ---- .spm files (components/format/crates/spm-file; docs/spm-format.md) -- */
/* Encoding profiles (spm-layout/src/model.rs:14-58, codes :48-58). */
enum {
    EMU_SPM_TERNARY = 1, EMU_SPM_F32 = 2, EMU_SPM_BF16 = 3,
    EMU_SPM_Q6K = 4, EMU_SPM_Q5K = 5, EMU_SPM_Q8_0 = 6
};
typedef struct emu_spm emu_spm;
typedef struct emu_spm_writer emu_spm_writer;
typedef struct emu_spm_descriptor { /* OpDescriptor (spm-layout/src/model.rs:113-125) */
    uint32_t rows, cols, group_size;
    uint32_t encoding;   /* EMU_SPM_* */
    uint32_t lane_count; /* 16 bits on the wire */
} emu_spm_descriptor;
typedef struct emu_spm_group { /* Group (spm-file/src/read.rs:16-25) */
    uint32_t stream;
    float scale;
    uint32_t count;          /* weights in the group; short for a stream's last group */
    const uint8_t *packed;   /* points into the parsed bytes */
    size_t packed_len;
} emu_spm_group;

/* Encoding::bytes_for (spm-layout/src/model.rs:80-91). */
int emu_spm_bytes_for(uint32_t encoding, uint64_t count, uint64_t *bytes);
/* SpmReader::parse (read.rs:48-63): header and stream directory.  The reader
 * borrows h_bytes, which must outlive it.  On failure h_err receives the
 * reference's HeaderError / LayoutError text. */
int emu_spm_parse(const void *h_bytes, size_t len, emu_spm **out, char *h_err, size_t err_len);
int emu_spm_close(emu_spm *r);
const char *emu_spm_error(const emu_spm *r);
int emu_spm_header(const emu_spm *r, uint16_t *major, uint16_t *minor, uint32_t *stream_count);
int emu_spm_descriptor_at(const emu_spm *r, uint32_t index, emu_spm_descriptor *d);
/* The cursor: the stream and group next_group would return. */
int emu_spm_position(const emu_spm *r, uint32_t *stream, uint64_t *group);
/* SpmReader::next_group (read.rs:70-88): *has_group = 0 at the end of the
 * payload; EMU_E_TRUNCATED "payload truncated: group needs N bytes, M remain"
 * leaves the cursor where it was. */
int emu_spm_next_group(emu_spm *r, int *has_group, emu_spm_group *group);
/* The reader's current stream, from its first group, into device memory in
 * the layout the kernels read: Q6K / Q5K / Q8_0 blocks back to back in their
 * source row-major order (each group's inert scale dropped on the device), or
 * an F32 stream's column-major weights as a row-major rows x cols matrix.
 * Consumes the stream; *stream (may be NULL) receives its index.  Block
 * streams need group_size and rows*cols in whole blocks. */
int emu_spm_upload_stream(emu_ctx *ctx, emu_spm *r, void *d_dst, size_t dst_len, uint32_t *stream);
/* SpmWriter (spm-file/src/write.rs:15-107): new, write_raw_group, finish.
 * write_raw_group refuses a count or payload length the layout does not
 * expect (EMU_E_SHAPE, "group expects N weights, got M") and a group past the
 * last stream (EMU_E_FORMAT, "only W of D streams were written"); finish
 * refuses a file with groups still owed.  The finished bytes stay owned by the
 * writer until it is destroyed. */
int emu_spm_writer_create(const emu_spm_descriptor *descs, uint32_t n, emu_spm_writer **out);
int emu_spm_write_raw_group(emu_spm_writer *w, float scale, const void *h_payload, size_t payload_len,
                            uint64_t count);
int emu_spm_writer_finish(emu_spm_writer *w, const uint8_t **h_bytes, size_t *len);
const char *emu_spm_writer_error(const emu_spm_writer *w);
int emu_spm_writer_destroy(emu_spm_writer *w);

#ifdef __cplusplus
}
#endif
#endif /* EMUHIP_H */
