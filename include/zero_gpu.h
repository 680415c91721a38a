/*
 * zero_gpu.h -- C ABI of the MI355X (gfx950) quantized-matmul path.
 *
 * Drop-in for the decode-time matmul boundary of silicatetech/zero.  Every
 * entry point names the reference interface it replaces (paths relative to
 * the reference repository).  Plain pointers and sizes only; no C++ or torch
 * types cross this boundary.  Status codes, never exceptions or aborts.
 *
 * Threading: one caller thread per context (the reference calls its
 * dispatchers only from the BSP, kernel/src/smp.rs:1567-1712).  A context is
 * not re-entrant.  Host-pointer calls are synchronous; *_dev calls are
 * asynchronous on the stream given (NULL = the context's stream).
 */
#ifndef ZERO_GPU_H
#define ZERO_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The reference returns Result enums and panics on an
 * unsupported quant (crates/zero-llm-inference/src/ops.rs:486-523,
 * kernel/src/inference_avx512.rs:1122-1184); here both are codes. */
typedef int32_t zg_status;
#define ZG_OK 0
#define ZG_ERR_INVALID_ARG -1       /* null pointer, bad shape, bad interleave */
#define ZG_ERR_UNSUPPORTED_QUANT -2 /* LinearDispatchError::UnsupportedQuant  */
#define ZG_ERR_NOT_REGISTERED -3    /* weight pointer not uploaded            */
#define ZG_ERR_HIP -4               /* HIP runtime error; see zg_last_error    */
#define ZG_ERR_NONFINITE_LOGITS -5  /* LmHeadError::NonFiniteLogits (lm_head.rs:32-38) */
#define ZG_ERR_ARGMAX_IN_PADDING -6 /* LmHeadError::ArgmaxInPaddingRegion      */
#define ZG_ERR_REGISTRY_FULL -7     /* weight_layout::register returned false  */
#define ZG_ERR_OUT_OF_MEMORY -8
#define ZG_ERR_ATTENTION -9         /* AttentionError::NumericalInstability    */
#define ZG_ERR_CONTEXT_FULL -10     /* KvCache position out of range           */
#define ZG_ERR_MAGIC_MISMATCH -11   /* LoadError::MagicMismatch (model_loader.rs:149-159)    */
#define ZG_ERR_UNSUPPORTED_FORMAT -12 /* LoadError::UnsupportedFormat                        */
#define ZG_ERR_INVALID_CONTAINER -13  /* LoadError::InvalidContainer                         */

/* GgmlType ids (crates/zero-gguf-parser/src/lib.rs:95-126). */
#define ZG_Q4_0 2u
#define ZG_Q8_0 8u
#define ZG_Q4K 12u
#define ZG_Q6K 14u

typedef struct zg_ctx zg_ctx;

/* Create a context on HIP device `device` with its own stream.  Replaces
 * the SMP bring-up that the reference performs before its first dispatch
 * (kernel/src/main.rs:979-1113, smp::set_active_cores). */
zg_status zg_init(int device, zg_ctx **out);
/* Releases the context.  A context that still has models (zg_model_create)
 * is released by the last zg_model_destroy instead; the caller makes no
 * other call on it after zg_destroy. */
void zg_destroy(zg_ctx *ctx);
/* Human-readable message of the last failing call on this context. */
const char *zg_last_error(const zg_ctx *ctx);
/* The context's hipStream_t, as an opaque pointer. */
void *zg_stream(zg_ctx *ctx);

/* ------------------------------------------------------------------ */
/* Weight registry.                                                     */
/* ------------------------------------------------------------------ */

/* Upload `bytes` bytes at `host_ptr` and register them under that address
 * with layout `interleave` (1 = plain row-major, 4 = .smodel-v2 X4).
 * Replaces weight_layout::register (kernel/src/weight_layout.rs:94) plus
 * the SIDX dtype decode 100/101 -> (Q4_0|Q8_0, 4)
 * (kernel/src/model_loader.rs:82-90).  Lookups are by exact start address
 * or by an address inside a plain tensor (weight_layout.rs:133 semantics:
 * an interior pointer is never interleaved).  The bytes are copied once, at
 * registration: later changes to the host bytes are not seen, and the host
 * memory may be freed.  Byte ranges [host_ptr, host_ptr + bytes) of
 * registered tensors must not overlap (ZG_ERR_INVALID_ARG). */
zg_status zg_register_weight(zg_ctx *ctx, const void *host_ptr, size_t bytes, uint32_t ggml_type,
                             uint32_t interleave);
/* Same, but the bytes are already on the device at `dev_ptr` (borrowed,
 * not freed by the context). `key` is the host-side address to register. */
zg_status zg_register_weight_device(zg_ctx *ctx, const void *key, const void *dev_ptr,
                                    size_t bytes, uint32_t ggml_type, uint32_t interleave);
/* weight_layout::group_of (weight_layout.rs:133): 4 for a registered X4
 * tensor start, else 1. */
uint32_t zg_group_of(const zg_ctx *ctx, const void *host_ptr);
/* weight_layout::rebase (weight_layout.rs:76): shift every key by delta. */
void zg_rebase(zg_ctx *ctx, int64_t delta);
/* weight_layout::clear (weight_layout.rs:57): drops every registration.
 * Uploaded copies are freed, except those a live model reads: a model keeps
 * its weights until zg_model_destroy, so it stays valid after a clear (the
 * reference clears its registry before indexing the next model,
 * model_loader.rs:488). */
void zg_clear(zg_ctx *ctx);
/* Number of registered tensors (weight_layout::count). */
size_t zg_registered_count(const zg_ctx *ctx);

/* ------------------------------------------------------------------ */
/* Operator API: host pointers, synchronous.                            */
/* ------------------------------------------------------------------ */

/* out[0..out_dim) = W . x.  Replaces linear_dispatch (ops.rs:486-523) and
 * linear_dispatch_avx512 (inference_avx512.rs:1147-1184).  The layout
 * (plain or X4) comes from the registry, as the reference's comes from
 * weight_layout::group_of (inference_avx512.rs:638,690). */
zg_status zg_linear(zg_ctx *ctx, const float *x, const void *w, float *out, size_t in_dim,
                    size_t out_dim, uint32_t ggml_type);
/* Rows [start,end) only (the RowRange kernels, linear.rs:909,1096,...);
 * out is the full out_dim vector, rows outside the range are untouched. */
zg_status zg_linear_range(zg_ctx *ctx, const float *x, const void *w, float *out, size_t in_dim,
                          size_t out_dim, uint32_t ggml_type, size_t start, size_t end);

/* One projection of a fused same-input dispatch: FusedSegment
 * (inference_avx512.rs:743-764). */
typedef struct {
    const void *w;      /* registered weight (host key) or device ptr for _dev */
    float *out;         /* host output (or device output for _dev)           */
    size_t out_dim;
    uint32_t ggml_type;
    uint32_t interleave; /* used by the _dev variant only                     */
} zg_segment;
/* linear_fused_dispatch (inference_avx512.rs:890-945): up to 3 segments
 * sharing x, one launch over the concatenated row space. */
zg_status zg_linear_fused(zg_ctx *ctx, const float *x, const zg_segment *segs, size_t n_segs,
                          size_t in_dim);

/* lm_head_argmax_avx512 (inference_avx512.rs:1200-1270): rmsnorm(hidden,
 * norm_w) -> GEMV over vocab_padded rows -> first-max argmax with NaN
 * suppressed.  logits may be NULL.  Returns ZG_ERR_NONFINITE_LOGITS or
 * ZG_ERR_ARGMAX_IN_PADDING (index >= vocab_real) like LmHeadError. */
zg_status zg_lm_head_argmax(zg_ctx *ctx, const float *hidden, const float *norm_w, const void *w,
                            uint32_t ggml_type, float eps, size_t dim, size_t vocab_padded,
                            size_t vocab_real, float *logits, uint32_t *token, float *max_val);

/* ------------------------------------------------------------------ */
/* Device-pointer API: asynchronous on `stream` (NULL = ctx stream).    */
/* No registry; the caller states the layout: 1 plain row-major, 4     */
/* .smodel-v2 X4, or 5 for Q4_0 / Q8_0 only: split-scale X4 groups, the */
/* model's device layout (per group of four rows, its blocks' quants    */
/* [block][row][16 or 32 bytes], then their fp16 scales [block][row];   */
/* the same bytes as the X4 group, regrouped; GEMV, fused, LM-head,     */
/* Q8_0-activation GEMV and prefill-GEMM calls with in_dim a multiple   */
/* of 512 up to 8192, 16-byte aligned w and x; no reference             */
/* counterpart).                                                        */
/* ------------------------------------------------------------------ */

zg_status zg_linear_dev(zg_ctx *ctx, const float *d_x, const void *d_w, float *d_out,
                        size_t in_dim, size_t out_dim, uint32_t ggml_type, uint32_t interleave,
                        size_t start, size_t end, void *stream);
zg_status zg_linear_fused_dev(zg_ctx *ctx, const float *d_x, const zg_segment *segs,
                              size_t n_segs, size_t in_dim, void *stream);
/* GEMV + argmax; writes the packed candidate (see zg_argmax_unpack) to
 * d_best (uint64, reset by this call) and optionally logits. */
zg_status zg_lm_head_dev(zg_ctx *ctx, const float *d_x, const void *d_w, float *d_logits,
                         size_t in_dim, size_t out_dim, uint32_t ggml_type, uint32_t interleave,
                         uint64_t *d_best, void *stream);
/* Decode the packed argmax candidate. Returns 0 when no finite candidate. */
int zg_argmax_unpack(uint64_t packed, uint32_t *index, float *value);
/* The GEMV with a Q8_0-quantized activation (variant (ii) of the decode
 * GEMV: x encoded on the fly with zg_quantize_q8_0_dev, the packer's Q8_0
 * encoder): out = W . x over in_dim / 32 34-byte Q8_0 blocks at d_xq (2-byte
 * aligned), integer block dots (v_dot4_i32_i8) scaled by dW * dX, as
 * zg_gemm_q8act_dev computes one row.  No counterpart in the reference,
 * whose Q4_0/Q8_0 GEMVs take fp32 x (its only activation-quantized path is
 * the Q4_K x Q8_K one below).  Q4_0 or Q8_0 weights, X4 or plain;
 * in_dim a multiple of 512 up to 8192, out_dim % 4 == 0. */
zg_status zg_linear_q8act_dev(zg_ctx *ctx, const void *d_xq, const void *d_w, float *d_out, size_t in_dim,
                              size_t out_dim, uint32_t ggml_type, uint32_t interleave, void *stream);
/* Bit-exact dequantization of a device tensor into fp32 rows (test hook for
 * dequant parity with crates/zero-gguf-parser/src/dequant.rs). */
zg_status zg_dequant_dev(zg_ctx *ctx, const void *d_w, float *d_out, size_t rows, size_t in_dim,
                         uint32_t ggml_type, uint32_t interleave, void *stream);
/* fp16 bits -> f32 on the device (dequant.rs:28-61), n values. */
zg_status zg_fp16_to_f32_dev(zg_ctx *ctx, const uint16_t *d_in, float *d_out, size_t n,
                             void *stream);
/* Measurement hook, no reference counterpart: one launch that streams
 * `bytes` (a multiple of 16, 16-byte aligned source) with the GEMV's
 * nontemporal 128-bit loads and computes nothing, loads_per_thread
 * (1, 2, 4 or 8) loads per thread of 256-thread workgroups.  The floor a
 * GEMV of the same weight bytes is measured against.  d_sink: one uint32
 * that real data never writes. */
zg_status zg_read_floor_dev(zg_ctx *ctx, const void *d_src, size_t bytes, uint32_t loads_per_thread,
                            uint32_t *d_sink, void *stream);
/* Measurement hook, no reference counterpart: the Q4_0X4 strip GEMV's loads
 * without its decode, for `rows` x 2048 Q4_0X4 weights (rows % 4 == 0): the
 * GEMV's own per-lane load instructions, cache policy and launch form (one
 * batch of three groups per workgroup for decode-sized launches, else a
 * loop over four-group batches with two in flight), and with d_x non-null
 * (2048 floats) also each lane's two float4 quarters of x.  Together with
 * zg_read_floor_dev it separates a GEMV's time into the plain read, the
 * load pattern and the decode.  d_sink: one uint32 that real data never
 * writes. */
zg_status zg_strip_loads_dev(zg_ctx *ctx, const void *d_w, size_t rows, const float *d_x, uint32_t *d_sink,
                             void *stream);

/* On-the-fly Q8_0 activation quantization of rows x k values (k % 32 == 0):
 * the packer's quantize_q8_0_block (tools/silicatepack.py:893-907) bit for
 * bit: d = amax/127 and q = round-half-even(x/d) computed in double, d stored
 * as the round-to-nearest-even binary16 of the double d (:854-861).  A block
 * holding a non-finite value (a ValueError in the packer) is written with
 * q = 0 and d = NaN (0x7E00).
 * zg_quantize_q8_0_dev writes standard 34-byte blocks (fp16 d + 32 i8);
 * zg_quantize_q8_0_split_dev writes the same bytes as two arrays, int8
 * qs[rows][k] (16-byte aligned) and fp16 d[rows][k/32], the layout the
 * prefill GEMM reads. */
zg_status zg_quantize_q8_0_dev(zg_ctx *ctx, const float *d_x, void *d_q, size_t rows, size_t k,
                               void *stream);
zg_status zg_quantize_q8_0_split_dev(zg_ctx *ctx, const float *d_x, int8_t *d_qs, uint16_t *d_d,
                                     size_t rows, size_t k, void *stream);
/* Prefill GEMM, any M: Y[m][n] = sum_b dX[m][b]*dW[n][b]*(int8 dot of block b)
 * over Q4_0/Q8_0 weights (plain or X4) and split Q8_0 activations, on int8
 * MFMA; Y is fp32 row-major [m][n].  No reference counterpart: the
 * reference prefills token by token (kernel/src/inference.rs:1188-1330). */
zg_status zg_gemm_q8act_dev(zg_ctx *ctx, const int8_t *d_qs, const uint16_t *d_d, const void *d_w,
                            float *d_y, size_t m, size_t n, size_t k, uint32_t w_type,
                            uint32_t interleave, void *stream);
/* The K-quant prefill GEMM's activation operand: quantize_row_q8k
 * (kernel/src/arch/x86_64/math/vnni.rs:78-170, the arithmetic of
 * zg_quantize_q8k_dev) of rows x k values (k % 256 == 0), written as three
 * arrays: int8 qs[rows][k] (4-byte aligned; 16 for the GEMM), f32
 * d8[rows][k/256] and int16 bs32[rows][k/32], the sums of 32 quants
 * (bsum[2g] + bsum[2g+1] of the reference's block).  Bit-exact. */
zg_status zg_quantize_q8k_split_dev(zg_ctx *ctx, const float *d_x, int8_t *d_qs, float *d_d8,
                                    int16_t *d_bs32, size_t rows, size_t k, void *stream);
/* Prefill GEMM for K-quant weights on int8 MFMA: Y[m][n] (+)= X[m] . W[n]
 * for split Q8_K activations (zg_quantize_q8k_split_dev) and plain Q4_K or
 * Q6_K rows (w_type 12 / 14; n % 64 == 0, k % 256 == 0, qs 16-byte aligned,
 * d8 and bs32 4-byte aligned).  Each output is linear_q4k_vnni_range's arithmetic
 * (kernel/src/arch/x86_64/math/vnni.rs:258-476) bit for bit: per superblock
 * the exact integer sums, then dot += (d_w d8) int_sum, min += (dmin_w d8)
 * min_sum, y = dot - min; Q6_K the same construction with (q - 32) and its
 * 16 int8 scales, y += (d_w d8) int_sum.  accumulate != 0 adds the result
 * to Y.  No reference counterpart as a GEMM: the reference prefills token by
 * token (kernel/src/inference.rs:1188-1330). */
zg_status zg_gemm_q8k_dev(zg_ctx *ctx, const int8_t *d_qs, const float *d_d8, const int16_t *d_bs32,
                          const void *d_w, float *d_y, size_t m, size_t n, size_t k, uint32_t w_type,
                          int accumulate, void *stream);

/* ------------------------------------------------------------------ */
/* Forward pass.                                                        */
/* ------------------------------------------------------------------ */

/* LayerWeights (crates/zero-llm-inference/src/forward_pass.rs:227-239):
 * host keys of registered tensors (or device pointers when
 * zg_model_desc.device_pointers != 0). */
typedef struct {
    const void *attn_q, *attn_k, *attn_v, *attn_o;
    const void *ffn_gate, *ffn_up, *ffn_down;
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm; /* host fp32 arrays */
} zg_layer_weights;

/* ForwardPassDispatch's per-layer quant pathways
 * (crates/zero-llm-inference/src/forward_pass.rs:191-207): the ggml type
 * (Q4_0, Q8_0, Q4_K, Q6_K) and layout (1 plain rows, 4 X4; X4 only for
 * Q4_0/Q8_0) of each projection of one layer, indexed by ZG_PROJ_*. */
enum { ZG_PROJ_Q = 0, ZG_PROJ_K, ZG_PROJ_V, ZG_PROJ_O, ZG_PROJ_GATE, ZG_PROJ_UP, ZG_PROJ_DOWN, ZG_N_PROJ };
typedef struct {
    uint32_t type[ZG_N_PROJ];
    uint32_t interleave[ZG_N_PROJ];
} zg_layer_quants;

typedef struct {
    uint32_t n_layers, hidden, ffn, n_q_heads, n_kv_heads, head_dim;
    uint32_t vocab_padded, vocab_real, max_ctx;
    float rms_eps, rope_theta;
    uint32_t lin_type, lin_interleave;   /* every layer projection's quant and layout when
                                            layer_quants is NULL: Q4_0 or Q8_0 X4 (4), or any
                                            of Q4_0 / Q8_0 / Q4_K / Q6_K as plain rows (1) */
    uint32_t embd_type;                  /* token_embd quant (plain layout; token_embd_quant) */
    uint32_t head_type, head_interleave; /* output.weight quant + layout */
    const void *token_embd;
    const void *lm_head;
    const float *output_norm;
    const zg_layer_weights *layers;
    uint32_t device_pointers;            /* weights are device pointers, not keys */
    const zg_layer_quants *layer_quants; /* n_layers entries (the per-layer arrays of
                                            ForwardPassDispatch), or NULL */
} zg_model_desc;

typedef struct zg_model zg_model;

/* Builds device state (KV cache [L][K|V][t][kv_head][d] fp32 as
 * kv_cache.rs:17-31, scratch, norm weights) and captures the per-token
 * layer sequence of forward_single_token_avx512
 * (inference_avx512.rs:1826-1987) + lm_head_argmax_avx512 into a hipGraph.
 * Plain-row Q4_0 / Q8_0 projections and LM head whose rows come in fours
 * are copied once into model-owned device memory in the X4 layout (the
 * same results bit for bit, the X4 kernels' speed): the model then holds a
 * second copy of those weights until zg_model_destroy. */
zg_status zg_model_create(zg_ctx *ctx, const zg_model_desc *desc, zg_model **out);
void zg_model_destroy(zg_model *m);
/* One token through all layers at position pos, then the LM head.
 * hidden_out (dim floats) and logits (vocab_padded floats) may be NULL.
 * Returns the LmHeadError codes like zg_lm_head_argmax. */
zg_status zg_model_step(zg_model *m, uint32_t token, uint32_t pos, float *hidden_out,
                        float *logits, uint32_t *next_token, float *max_logit);
/* The caller loop of run_forward_pass (kernel/src/inference.rs:1188-1330,
 * 1644-1705, 1817-): prefill the prompt token by token, then n_gen greedy
 * tokens, with the token id fed back on the device (no host round trip).
 * out_tokens receives n_gen ids. *seconds (optional) = wall time of the
 * generation phase. */
zg_status zg_model_generate(zg_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                            uint32_t *out_tokens, double *prefill_seconds, double *gen_seconds);
/* Position reset (new sequence); also clears the non-finite latch. */
void zg_model_reset(zg_model *m);
/* The non-finite latch, first_nonfinite_detail (inference_avx512.rs:264-275):
 * when a model call fails with ZG_ERR_NONFINITE_LOGITS or ZG_ERR_ATTENTION,
 * the first stage holding a NaN/Inf is found (finite_diag's stages,
 * inference_avx512.rs:1896, 1946-1947, 1981-1982: attn_norm_in, attn_out,
 * post_attn_residual, mlp_out, post_mlp_residual) and latched as
 * "L{layer:02} {stage} n{0|1} i{0|1}" (the first non-finite element's
 * NaN / Inf flags), up to 32 bytes; the failing call's zg_last_error ends
 * with " @" and the same text.  The first failure after zg_model_create or
 * zg_model_reset latches; later ones keep it.  Found by running the step of
 * the first KV row holding a non-finite value (or of the failing step)
 * again with the scans, which rewrites that row with the same values; a row
 * written by the batched prefill is named as "k_cache[row]" /
 * "v_cache[row]" instead.  Copies up to cap bytes (no terminator) into buf
 * and returns the count; 0 when nothing is latched. */
size_t zg_model_first_nonfinite(const zg_model *m, char *buf, size_t cap);
/* Failure-path test hook; no counterpart in the reference, for tests of the
 * timeout report only.  The fused Q|K|V + attention launch of layer `layer`
 * (0-based) skips its tagged Q|K|V row stores, so every attention wave of
 * that layer gives up at its bounded wait (2^13 polls) and the call returns
 * ZG_ERR_HIP ("a completion wait timed out"): the GPU counterpart of the
 * reference's barrier-timeout recovery (kernel/src/smp.rs:1677-1711).
 * Every kernel still runs to its end.  layer < 0 restores the stores (the
 * default).  Affects only layers decoded by the fused launch. */
zg_status zg_model_test_drop_qkv_stores(zg_model *m, int32_t layer);

/* Batched prefill.  No counterpart in the reference, which runs the prompt
 * token by token through forward_single_token_avx512
 * (kernel/src/inference.rs:1188-1330); this is the M >= 64 prefill of the
 * int8-MFMA path: per layer the n prompt rows go through rmsnorm, Q8_0
 * activation quantization (the packer's encoder, silicatepack.py:893-907)
 * and zg_gemm_q8act_dev-style GEMMs (Q|K|V, O, gate|up, down), with the
 * decode step's QK-norm, RoPE, causal attention and SwiGLU per row.  Writes
 * KV rows pos0..pos0+n-1 (chunks of up to 512 rows attend to the rows
 * before them), then runs the LM head on the last row.  Leaves the model
 * ready to decode at position pos0 + n.  hidden_out (optional): the final
 * hidden state of the last row.  Activations are quantized to 8 bits, so
 * results differ from token-by-token prefill by that quantization.  The
 * GEMMs take Q4_0 / Q8_0 weights: a model with a Q4_K or Q6_K layer
 * projection returns ZG_ERR_UNSUPPORTED_QUANT here (it decodes, and
 * prefills token by token). */
zg_status zg_model_prefill(zg_model *m, const uint32_t *tokens, size_t n, uint32_t pos0,
                           float *hidden_out, uint32_t *next_token, float *max_logit);
#define ZG_GEN_BATCHED_PREFILL 1u
#define ZG_GEN_EAGER 2u
/* zg_model_generate with flags: ZG_GEN_BATCHED_PREFILL runs the prompt
 * through zg_model_prefill's batched path instead of token by token.
 * ZG_GEN_EAGER (not with ZG_GEN_BATCHED_PREFILL) issues each token's
 * kernels directly on the stream instead of replaying the captured step
 * graph: the same launches in the same order and the same tokens, slower;
 * for profilers that collect counters per dispatch.  Other flag bits are
 * ZG_ERR_INVALID_ARG. */
zg_status zg_model_generate_ex(zg_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                               uint32_t flags, uint32_t *out_tokens, double *prefill_seconds,
                               double *gen_seconds);

/* ------------------------------------------------------------------ */
/* Q4_K x Q8_K integer path (kernel/src/arch/x86_64/math/vnni.rs,       */
/* behind the reference's "vnni-acceleration" feature).  Q8_K blocks    */
/* are the reference's 292-byte form: f32 d, 256 int8, 16 int16 sums.   */
/* ------------------------------------------------------------------ */

/* quantize_row_q8k (vnni.rs:78-170) of n device floats (n % 256 == 0) into
 * n / 256 blocks at d_q8k (4-byte aligned); bit-exact. */
zg_status zg_quantize_q8k_dev(zg_ctx *ctx, const float *d_x, void *d_q8k, size_t n, void *stream);
/* linear_q4k_vnni_range (vnni.rs:258-476) over all out_dim rows: d_w is
 * plain Q4_K (144-byte superblocks), in_dim % 256 == 0, in_dim <= 32768. */
zg_status zg_linear_q4k_q8k_dev(zg_ctx *ctx, const void *d_q8k, const void *d_w, float *d_out,
                                size_t in_dim, size_t out_dim, void *stream);
/* linear_q4k_vnni_dispatch (kernel/src/inference_avx512.rs:519-547): host
 * x, registered Q4_K w, host out; quantizes x to Q8_K, then the integer
 * GEMV.  Synchronous. */
zg_status zg_linear_q4k_vnni(zg_ctx *ctx, const float *x, const void *w, float *out, size_t in_dim,
                             size_t out_dim);
/* No counterpart in the reference.  For callers that cannot allocate (code
 * under HIP graph capture, tight serving loops): zg_linear_q4k_vnni on device
 * pointers (d_x fp32, 16-byte aligned; d_w plain Q4_K, 16-byte aligned;
 * d_out fp32), asynchronous on `stream` (NULL = the context's stream), with
 * no hipMalloc or hipFree.  The Q8_K blocks of x go to a fixed device array
 * of the library: in_dim <= 32768 (37,376 bytes per GPU, held until the
 * process ends); a larger in_dim is ZG_ERR_INVALID_ARG.  Every call on one
 * GPU shares that array: calls that may overlap on the same GPU (streams
 * not ordered against each other) race. */
zg_status zg_linear_q4k_vnni_noalloc(zg_ctx *ctx, const float *d_x, const void *d_w, float *d_out,
                                     size_t in_dim, size_t out_dim, void *stream);

/* ------------------------------------------------------------------ */
/* .smodel native container (SilicatePack SILM + SIDX).                 */
/* ------------------------------------------------------------------ */

typedef struct zg_smodel zg_smodel;

/* Container header and SIDX model config (smodel_info,
 * kernel/src/model_loader.rs:599-659; smodel_native_tensor_index :380-454).
 * Optional u32 fields hold 0xFFFFFFFF when absent (SMODEL_NONE_U32). */
typedef struct {
    uint32_t version;      /* 1, or 2 (may carry row-interleaved dtypes) */
    uint32_t payload_kind; /* 2 = native (1 = GGUF compatibility: rejected) */
    uint32_t flags;        /* bit 0: payload 2 MiB aligned */
    uint64_t manifest_offset, manifest_len, payload_offset, payload_len;
    uint32_t architecture_id; /* 1 qwen3, 2 deepseek2, else unknown */
    uint32_t block_count, context_length, embedding_length, feed_forward_length;
    uint32_t head_count, head_count_kv, key_length, value_length;
    float rope_freq_base, layer_norm_rms_epsilon;
    uint32_t vocab_size, eos_token_id;
    uint64_t tensor_count;
} zg_smodel_info;

/* One SIDX tensor entry (104 bytes, model_loader.rs:480-520). */
typedef struct {
    const char *name;       /* not NUL-terminated: name_len bytes */
    size_t name_len;
    uint32_t dtype;         /* SIDX dtype id as stored (100 = Q4_0X4, 101 = Q8_0X4) */
    uint32_t ggml_type;     /* smodel_decode_dtype (model_loader.rs:82-90) */
    uint32_t interleave;    /* 1, or 4 for the X4 dtypes */
    uint32_t rank;
    uint64_t dims[8];       /* source (HF) order: dims[0] = output rows */
    uint64_t payload_offset;
    const void *data;       /* inside the caller's bytes */
    uint64_t byte_len;
} zg_smodel_tensor;

/* Validate a native .smodel held in memory (bytes..bytes+len, kept alive
 * by the caller) with the reference loader's checks: header (smodel_info),
 * SIDX magic/version/sizes, tensor count cap 10,000, names in range and
 * UTF-8, dtype known, every tensor inside the payload, X4 tensors rank 2
 * with rows % 4 == 0.  Errors are ZG_ERR_MAGIC_MISMATCH,
 * ZG_ERR_UNSUPPORTED_FORMAT, ZG_ERR_INVALID_CONTAINER as LoadError. */
zg_status zg_smodel_open(const void *bytes, size_t len, zg_smodel **out);
void zg_smodel_close(zg_smodel *sm);
zg_status zg_smodel_get_info(const zg_smodel *sm, zg_smodel_info *out);
zg_status zg_smodel_get_tensor(const zg_smodel *sm, uint64_t index, zg_smodel_tensor *out);
/* By exact name; ZG_ERR_INVALID_ARG when absent. */
zg_status zg_smodel_find(const zg_smodel *sm, const char *name, zg_smodel_tensor *out);
/* Register every quantized tensor (Q4_0/Q8_0 plain or X4, Q4_K, Q6_K) with
 * its layout, as smodel_native_tensor_index registers the X4 ones in
 * weight_layout (model_loader.rs:527-552); F32 tensors are skipped.  The
 * reference clears its registry before indexing a model; here the context
 * may hold other weights, so nothing is cleared: on an error the tensors
 * registered before the failing one stay registered (zg_clear drops all). */
zg_status zg_smodel_register_all(zg_ctx *ctx, const zg_smodel *sm);

#ifdef __cplusplus
}
#endif
#endif
