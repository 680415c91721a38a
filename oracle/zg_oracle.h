/*
 * zg_oracle.h -- CPU oracle for the quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the GPU
 * kernels are compared against, and the CPU baseline that bench.py times
 * beside them.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path (zero_amd/) never links,
 * loads or calls it.
 *
 * Every function restates an algorithm of the Rust reference
 * (silicatetech/zero), cited per function in zg_oracle.c.  Parity-pinning
 * status of each function is listed in the header comment of zg_oracle.c.
 */
#ifndef ZG_ORACLE_H
#define ZG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlType ids (crates/zero-gguf-parser/src/lib.rs:95-126). */
enum {
    ZO_F32 = 0,
    ZO_F16 = 1,
    ZO_Q4_0 = 2,
    ZO_Q8_0 = 8,
    ZO_Q4K = 12,
    ZO_Q6K = 14,
};

/* ---- fp16 / dequant (crates/zero-gguf-parser/src/dequant.rs) ---- */
float zo_fp16_to_f32(uint16_t bits);
void zo_fp16_to_f32_array(const uint16_t *bits, float *out, size_t n);
void zo_get_scale_min_k4(const uint8_t *scales, int j, uint8_t *sc, uint8_t *mn);
void zo_dequant_q4_0_row(const uint8_t *blocks, float *out, size_t nblocks);
void zo_dequant_q8_0_row(const uint8_t *blocks, float *out, size_t nblocks);
void zo_dequant_q4k_row(const uint8_t *blocks, float *out, size_t nblocks);
void zo_dequant_q6k_row(const uint8_t *blocks, float *out, size_t nblocks);
/* Dequantize a whole [rows x in_dim] tensor in the given layout
 * (interleave 1 = plain row-major, 4 = .smodel-v2 X4). Returns 0 on success. */
int zo_dequant_tensor(const uint8_t *w, float *out, size_t rows, size_t in_dim,
                      int ggml_type, int interleave);

/* ---- scalar crate operators (crates/zero-llm-inference/src/ops.rs) ---- */
int zo_linear_scalar(const float *x, const uint8_t *w, float *out,
                     size_t in_dim, size_t out_dim, int ggml_type);

/* ---- AVX-512 range kernels, same per-row FP operation order
 *      (kernel/src/arch/x86_64/math/linear.rs) ---- */
int zo_linear_range(const float *x, const uint8_t *w, float *out,
                    size_t in_dim, size_t out_dim, int ggml_type, int interleave,
                    size_t start, size_t end);

/* ---- the same range kernels in AVX-512 intrinsics (zg_avx512.c): the
 *      CPU baseline; bit-identical to zo_linear_range.  -2 without AVX-512F ---- */
int zo_avx512_available(void);
int zo_linear_range_avx512(const float *x, const uint8_t *w, float *out,
                           size_t in_dim, size_t out_dim, int ggml_type, int interleave,
                           size_t start, size_t end);
/* Which range kernels the pool dispatches (zo_linear_parallel, the fused and
 * LM-head dispatches, the model forward): 1 = the intrinsics, when the CPU
 * has AVX-512F; 0 = the scalar restatement.  Returns the setting in force. */
int zo_set_simd(int on);
/* attn_heads_kernel (inference_avx512.rs:1459-1512) over query heads
 * [h0, h1) in AVX-512 intrinsics: per-head score stripes of `stride`
 * floats.  1 on a softmax failure, -2 without AVX-512F. */
int zo_attn_heads_avx512(const float *q, const float *kc, const float *vc, size_t T, size_t kvd, size_t hd,
                         size_t gqa, float scale, float *scores, size_t stride, float *out, size_t h0,
                         size_t h1);

/* ---- f64 brute force (no reference counterpart; exact-ish checker) ---- */
int zo_linear_f64(const float *x, const uint8_t *w, double *out,
                  size_t in_dim, size_t out_dim, int ggml_type, int interleave);

/* ---- .smodel-v2 X4 interleave (tools/silicatepack.py:982-1029) ---- */
int zo_interleave_x4(const uint8_t *plain, uint8_t *x4, size_t rows, size_t in_dim, int ggml_type);
int zo_deinterleave_x4(const uint8_t *x4, uint8_t *plain, size_t rows, size_t in_dim, int ggml_type);

/* ---- packer quantizers (tools/silicatepack.py:854-940) ---- */
uint16_t zo_f64_to_fp16_bits(double v);
void zo_quantize_q8_0_row(const float *x, uint8_t *out, size_t n);
void zo_quantize_q4_0_row(const float *x, uint8_t *out, size_t n);

/* ---- argmax + merge (linear.rs:558-609, inference_avx512.rs:981-1044) ---- */
size_t zo_argmax(const float *v, size_t n, float *max_val);
/* candidate (va, ia) beats (vb, ib) iff va > vb or (va == vb and ia < ib) */
int zo_argmax_beats(float va, uint32_t ia, float vb, uint32_t ib);

/* ---- SMP partition (kernel/src/smp_partition.rs:143-220) ---- */
void zo_row_range_for(size_t total, uint32_t n_cores, size_t i, size_t align,
                      size_t *start, size_t *end);
void zo_row_range_for_discounted(size_t total, uint32_t n_cores, size_t i, size_t align,
                                 size_t discount_pct, size_t *start, size_t *end);

/* ---- pinned SMP worker pool (kernel/src/smp.rs:1107-1150,1567-1712) ---- */
int zo_pool_start(int n_threads);   /* returns threads in pool (incl. caller) */
void zo_pool_stop(void);
int zo_pool_size(void);
int zo_linear_parallel(const float *x, const uint8_t *w, float *out,
                       size_t in_dim, size_t out_dim, int ggml_type, int interleave);
/* segments of a fused same-x dispatch (inference_avx512.rs:743-945) */
typedef struct {
    const uint8_t *w;
    float *out;
    size_t out_dim;
    int ggml_type;
    int interleave;
} zo_segment;
int zo_linear_fused_parallel(const float *x, const zo_segment *segs, int n_segs, size_t in_dim);
/* LM head: linear over out_dim rows + argmax, per-range scan and merge
 * (inference_avx512.rs:1061-1118). Returns the index; *max_val set. */
size_t zo_lm_head_linear_argmax_parallel(const float *x, const uint8_t *w, float *logits,
                                         size_t in_dim, size_t out_dim, int ggml_type,
                                         int interleave, float *max_val);

/* ---- decode-step ops (ops.rs, attention.rs, forward_pass.rs) ---- */
void zo_rmsnorm(const float *in, const float *weight, float *out, size_t n, float eps);
void zo_rope_inv_freqs(float *inv, int half, float freq_base);
void zo_rope(float *qk, const float *inv, int half, size_t position);
int zo_softmax(float *s, size_t n);
void zo_silu_mul(const float *gate, const float *up, float *out, size_t n);

/* ---- Q8_0-activation quantized GEMM (no reference counterpart; the
 *      reference has no batched prefill).  Y[m][n] for Q4_0X4 or Q8_0X4
 *      weights times Q8_0 activations, block sums exact in int32,
 *      scaled in fp32 as  acc = fma(dw * dx, (float)isum, acc)  in ascending
 *      block order. ---- */
int zo_gemm_q8act(const uint8_t *xq, const uint8_t *w, float *y, size_t m, size_t n,
                  size_t k, int w_type, int interleave);

/* ---- Q4_K x Q8_K integer path (vnni.rs, feature "vnni-acceleration"):
 *      quantize_row_q8k :78-170 (292-byte blocks), unpack_mins_and_scales
 *      :176-205, linear_q4k_vnni_range :258-476 ---- */
#define ZO_Q8K_BYTES 292
void zo_quantize_row_q8k(const float *x, uint8_t *out, size_t n);
void zo_unpack_mins_and_scales(const uint8_t *s12, uint8_t *out16);
int zo_linear_q4k_q8k_range(const uint8_t *q8k, const uint8_t *w, float *out, size_t in_dim, size_t start,
                            size_t end);
/* the same integer construction on Q6_K rows (no reference counterpart:
 * the K-quant prefill GEMM's arithmetic) */
int zo_linear_q6k_q8k_range(const uint8_t *q8k, const uint8_t *w, float *out, size_t in_dim, size_t start,
                            size_t end);

/* ---- full single-token forward pass for a Qwen3-shaped model
 *      (inference_avx512.rs:1826-1987 order; scalar crate ops for norms,
 *      RoPE, softmax, SiLU) ---- */
typedef struct {
    const uint8_t *attn_q, *attn_k, *attn_v, *attn_o;
    const uint8_t *ffn_gate, *ffn_up, *ffn_down;
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
} zo_layer;

/* ForwardPassDispatch's per-layer quants (forward_pass.rs:191-207): type and
 * layout of the projections Q, K, V, O, gate, up, down, in that order. */
typedef struct {
    int type[7];
    int interleave[7];
} zo_layer_quants;

typedef struct {
    int n_layers, hidden, ffn, n_q_heads, n_kv_heads, head_dim;
    size_t vocab_padded, vocab_real, max_ctx;
    float rms_eps, rope_theta;
    int lin_type, lin_interleave;    /* layer linears, when layer_quants is NULL */
    int embd_type;                   /* token_embd (plain) */
    int head_type, head_interleave;  /* LM head */
    const uint8_t *token_embd;
    const uint8_t *lm_head;
    const float *output_norm;
    const zo_layer *layers;          /* n_layers entries */
    const zo_layer_quants *layer_quants; /* n_layers entries, or NULL */
} zo_model_desc;

typedef struct zo_model zo_model;
zo_model *zo_model_create(const zo_model_desc *desc);
void zo_model_destroy(zo_model *m);
/* Runs one token through all layers at position pos.  Returns 0 on success,
 * negative on error.  If hidden_out != NULL copies the final hidden state. */
int zo_model_forward(zo_model *m, uint32_t token, size_t pos, float *hidden_out);
/* Batched prefill with Q8_0-quantized activations (the GPU's int8-MFMA
 * prefill; no reference counterpart): n tokens at positions
 * pos0..pos0+n-1, KV rows stored; the last row's final hidden state is left
 * in the model for zo_model_lm_head and copied to hidden_out if non-NULL.
 * Returns -3 when a layer projection is not Q4_0 / Q8_0. */
int zo_model_prefill_q8(zo_model *m, const uint32_t *tokens, size_t n, size_t pos0, float *hidden_out);
/* record_first_nonfinite's text (inference_avx512.rs:237-262) for the first
 * non-finite element of buf[0..n): "L{layer:02} {stage} n{0|1} i{0|1}" with
 * that element's NaN / Inf flags, cut at 32 bytes, into out (no
 * terminator); returns its length, 0 when every element is finite. */
size_t zo_nonfinite_text(const float *buf, size_t n, int layer, const char *stage, char *out);
/* The non-finite latch of zo_model_forward (first_nonfinite_detail,
 * inference_avx512.rs:264-275): copies the latched text (at most 32 bytes,
 * no terminator) into buf and returns its length, 0 when nothing tripped. */
size_t zo_model_first_nonfinite(const zo_model *m, char *buf);
/* final rmsnorm + LM head + argmax; returns 0 / -1 non-finite / -2 padding */
int zo_model_lm_head(zo_model *m, float *logits_out, uint32_t *token, float *max_val);

#ifdef __cplusplus
}
#endif
#endif
