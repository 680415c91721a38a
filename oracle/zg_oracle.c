/*
 * zg_oracle.c -- CPU oracle (checker) and CPU baseline for the quantized
 * matmul hot path.  TEST INFRASTRUCTURE ONLY: loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
 * product path.
 *
 * Each function restates an algorithm of the Rust reference
 * (silicatetech/zero; paths below are relative to that repository).  The
 * reference cannot be compiled here (it is Rust and no Rust toolchain is
 * installed), so there is no oracle/_ref build; this restatement is pinned
 * instead by the checks listed here (all in tests/):
 *
 *   fp16_to_f32            exhaustive 65,536 patterns vs numpy's independent
 *                          binary16 decoder + dequant.rs KATs
 *   dequant_q4_0/q8_0      dequant.rs KATs + closed form (q-8)*d with numpy
 *   dequant_q4k            dequant.rs KATs + numpy restatement from the
 *                          ggml block spec
 *   dequant_q6k            dequant.rs KATs (-64, -66, 128, 31, zeros)
 *   linear_scalar          ops.rs KATs (528, 32, -256, -16, multi-block)
 *                          + f64 brute force
 *   linear_range (AVX order) equals linear_scalar within fp32 rounding,
 *                          X4 == plain bitwise, range split == full bitwise,
 *                          f64 brute force
 *   interleave_x4          test_silicatepack.py:341-378 permutation property
 *   quantize_q8_0/q4_0     test_silicatepack.py:270-306 KAT, numpy
 *                          float16 RNE, quantization-error bound, packer
 *                          golden vectors (tests/golden/)
 *   argmax / merge         lm_head.rs:168-201 semantics, brute force
 *   row_range_for          smp_partition.rs:226-401 properties
 *   rmsnorm / rope         ops.rs:530-772 KATs (incl. 16 gguf-py RoPE values)
 *   softmax / silu         closed form (sum=1, monotone) + numpy
 *   gemm_q8act             f64 brute force on the same quantized operands
 *   model_forward          composition of the above; parity vs GPU only
 *                          (real-model fixtures need an absent GGUF file)
 *
 * Build: oracle/Makefile (gcc only).  Compiled with -ffp-contract=off so
 * that the only fused multiply-adds are the explicit fmaf() calls that
 * restate the reference's _mm512_fmadd_ps/_mm512_fmsub_ps.
 */
#define _GNU_SOURCE
#include "zg_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#define ZO_PAUSE() _mm_pause()
#define ZO_CLONES __attribute__((target_clones("avx512f", "default")))
#else
#define ZO_PAUSE() ((void)0)
#define ZO_CLONES
#endif

/* ------------------------------------------------------------------ */
/* fp16 -> f32.  crates/zero-gguf-parser/src/dequant.rs:28-61           */
/* ------------------------------------------------------------------ */

static inline float f32_from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float zo_fp16_to_f32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u;
    uint32_t exp = (bits >> 10) & 0x1Fu;
    uint32_t mant = bits & 0x3FFu;
    if (exp == 0) {
        if (mant == 0) return f32_from_bits(sign << 31);
        /* denormal: mant * 2^-10 * 2^-14, exact in f32 */
        float val = ((float)mant) * (1.0f / 1024.0f) * (1.0f / 16384.0f);
        return sign ? -val : val;
    }
    if (exp == 31) {
        if (mant == 0) return f32_from_bits((sign << 31) | (0xFFu << 23));
        return f32_from_bits((sign << 31) | (0xFFu << 23) | (mant << 13));
    }
    return f32_from_bits((sign << 31) | ((exp + 112u) << 23) | (mant << 13));
}

void zo_fp16_to_f32_array(const uint16_t *bits, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = zo_fp16_to_f32(bits[i]);
}

static inline float rd_fp16(const uint8_t *p) {
    return zo_fp16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* ------------------------------------------------------------------ */
/* Dequant.  dequant.rs:75-85 (scale/min), 98-138 (Q4_K), 186-216      */
/* (Q4_0), 247-275 (Q8_0), 328-355 (Q6_K)                               */
/* ------------------------------------------------------------------ */

void zo_get_scale_min_k4(const uint8_t *s, int j, uint8_t *sc, uint8_t *mn) {
    if (j < 4) {
        *sc = s[j] & 0x3F;
        *mn = s[j + 4] & 0x3F;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

static void dq_q4_0_block(const uint8_t *blk, float *out) {
    float d = rd_fp16(blk);
    for (int j = 0; j < 16; j++) {
        uint8_t b = blk[2 + j];
        int x0 = (int)(b & 0x0F) - 8;
        int x1 = (int)((b >> 4) & 0x0F) - 8;
        out[j] = (float)x0 * d;
        out[j + 16] = (float)x1 * d;
    }
}

static void dq_q8_0_block(const uint8_t *blk, float *out) {
    float d = rd_fp16(blk);
    for (int k = 0; k < 32; k++) out[k] = (float)(int8_t)blk[2 + k] * d;
}

static void dq_q4k_block(const uint8_t *blk, float *out) {
    float d = rd_fp16(blk);
    float dmin = rd_fp16(blk + 2);
    const uint8_t *scales = blk + 4;
    const uint8_t *qs = blk + 16;
    int is = 0, qo = 0;
    for (int g = 0; g < 4; g++) {
        uint8_t sc0, mn0, sc1, mn1;
        zo_get_scale_min_k4(scales, is, &sc0, &mn0);
        zo_get_scale_min_k4(scales, is + 1, &sc1, &mn1);
        float d1 = d * (float)sc0, m1 = dmin * (float)mn0;
        float d2 = d * (float)sc1, m2 = dmin * (float)mn1;
        for (int l = 0; l < 32; l++) out[g * 64 + l] = d1 * (float)(qs[qo + l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) out[g * 64 + 32 + l] = d2 * (float)(qs[qo + l] >> 4) - m2;
        qo += 32;
        is += 2;
    }
}

static void dq_q6k_block(const uint8_t *blk, float *out) {
    float d = rd_fp16(blk + 208);
    const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
    for (int h = 0; h < 2; h++) {
        int qlo = 64 * h, qho = 32 * h, sco = 8 * h, yo = 128 * h;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = ((ql[qlo + l] & 0xF) | ((qh[qho + l] & 3) << 4)) - 32;
            int q2 = ((ql[qlo + l + 32] & 0xF) | (((qh[qho + l] >> 2) & 3) << 4)) - 32;
            int q3 = ((ql[qlo + l] >> 4) | (((qh[qho + l] >> 4) & 3) << 4)) - 32;
            int q4 = ((ql[qlo + l + 32] >> 4) | (((qh[qho + l] >> 6) & 3) << 4)) - 32;
            out[yo + l] = d * (float)(int8_t)sc[sco + is] * (float)q1;
            out[yo + l + 32] = d * (float)(int8_t)sc[sco + is + 2] * (float)q2;
            out[yo + l + 64] = d * (float)(int8_t)sc[sco + is + 4] * (float)q3;
            out[yo + l + 96] = d * (float)(int8_t)sc[sco + is + 6] * (float)q4;
        }
    }
}

void zo_dequant_q4_0_row(const uint8_t *b, float *o, size_t nb) {
    for (size_t i = 0; i < nb; i++) dq_q4_0_block(b + 18 * i, o + 32 * i);
}
void zo_dequant_q8_0_row(const uint8_t *b, float *o, size_t nb) {
    for (size_t i = 0; i < nb; i++) dq_q8_0_block(b + 34 * i, o + 32 * i);
}
void zo_dequant_q4k_row(const uint8_t *b, float *o, size_t nb) {
    for (size_t i = 0; i < nb; i++) dq_q4k_block(b + 144 * i, o + 256 * i);
}
void zo_dequant_q6k_row(const uint8_t *b, float *o, size_t nb) {
    for (size_t i = 0; i < nb; i++) dq_q6k_block(b + 210 * i, o + 256 * i);
}

static int type_geom(int t, size_t *blk_elems, size_t *blk_bytes) {
    switch (t) {
    case ZO_Q4_0: *blk_elems = 32; *blk_bytes = 18; return 0;
    case ZO_Q8_0: *blk_elems = 32; *blk_bytes = 34; return 0;
    case ZO_Q4K: *blk_elems = 256; *blk_bytes = 144; return 0;
    case ZO_Q6K: *blk_elems = 256; *blk_bytes = 210; return 0;
    default: return -1;
    }
}

/* Byte address of block b of row r for either layout. */
static inline const uint8_t *x4_qs(const uint8_t *w, size_t r, size_t b, size_t nb, int t) {
    size_t gb = (t == ZO_Q4_0) ? 72 : 136, qb = (t == ZO_Q4_0) ? 16 : 32;
    return w + (r / 4) * nb * gb + b * gb + 8 + (r % 4) * qb;
}
static inline const uint8_t *x4_d(const uint8_t *w, size_t r, size_t b, size_t nb, int t) {
    size_t gb = (t == ZO_Q4_0) ? 72 : 136;
    return w + (r / 4) * nb * gb + b * gb + 2 * (r % 4);
}

int zo_dequant_tensor(const uint8_t *w, float *out, size_t rows, size_t in_dim, int t, int il) {
    size_t be, bb;
    if (type_geom(t, &be, &bb) || in_dim % be) return -1;
    size_t nb = in_dim / be;
    if (il == 1) {
        for (size_t r = 0; r < rows; r++) {
            const uint8_t *row = w + r * nb * bb;
            float *o = out + r * in_dim;
            switch (t) {
            case ZO_Q4_0: zo_dequant_q4_0_row(row, o, nb); break;
            case ZO_Q8_0: zo_dequant_q8_0_row(row, o, nb); break;
            case ZO_Q4K: zo_dequant_q4k_row(row, o, nb); break;
            case ZO_Q6K: zo_dequant_q6k_row(row, o, nb); break;
            }
        }
        return 0;
    }
    if (il != 4 || (t != ZO_Q4_0 && t != ZO_Q8_0) || rows % 4) return -1;
    uint8_t tmp[34];
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < nb; b++) {
            memcpy(tmp, x4_d(w, r, b, nb, t), 2);
            memcpy(tmp + 2, x4_qs(w, r, b, nb, t), bb - 2);
            if (t == ZO_Q4_0) dq_q4_0_block(tmp, out + r * in_dim + b * 32);
            else dq_q8_0_block(tmp, out + r * in_dim + b * 32);
        }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Scalar crate operators.  crates/zero-llm-inference/src/ops.rs:179-457 */
/* One block dequantized into scratch, then acc += x*w sequentially     */
/* (Rust does not contract a*b+c, hence -ffp-contract=off).             */
/* ------------------------------------------------------------------ */

int zo_linear_scalar(const float *x, const uint8_t *w, float *out, size_t in_dim,
                     size_t out_dim, int t) {
    size_t be, bb;
    if (type_geom(t, &be, &bb) || in_dim % be) return -1;
    size_t nb = in_dim / be;
    float buf[256];
    for (size_t i = 0; i < out_dim; i++) {
        float acc = 0.0f;
        const uint8_t *row = w + i * nb * bb;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + b * bb;
            switch (t) {
            case ZO_Q4_0: dq_q4_0_block(blk, buf); break;
            case ZO_Q8_0: dq_q8_0_block(blk, buf); break;
            case ZO_Q4K: dq_q4k_block(blk, buf); break;
            case ZO_Q6K: dq_q6k_block(blk, buf); break;
            }
            for (size_t k = 0; k < be; k++) acc = acc + x[b * be + k] * buf[k];
        }
        out[i] = acc;
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* AVX-512 range kernels, restated lane by lane.                        */
/* kernel/src/arch/x86_64/math/linear.rs.  Each 16-wide __m512           */
/* accumulator is a float[16]; _mm512_fmadd_ps(a,b,c) is fmaf(a,b,c)    */
/* per lane; _mm512_reduce_add_ps is the halving tree                   */
/* (i, i+8) -> (i, i+4) -> (i, i+2) -> (0, 1).                          */
/* ------------------------------------------------------------------ */

static inline float reduce16(const float *v) {
    float s8[8], s4[4], s2[2];
    for (int i = 0; i < 8; i++) s8[i] = v[i] + v[i + 8];
    for (int i = 0; i < 4; i++) s4[i] = s8[i] + s8[i + 4];
    for (int i = 0; i < 2; i++) s2[i] = s4[i] + s4[i + 2];
    return s2[0] + s2[1];
}

/* One Q4_0 block (d, 16 nibble bytes) into the row's lo/hi lane
 * accumulators: linear.rs:830-851 (plain) == linear.rs:985-1040 (X4). */
static inline void q4_0_block_acc(float d, const uint8_t *qs, const float *xb, float *lo,
                                  float *hi) {
    for (int j = 0; j < 16; j++) {
        float lf = (float)(qs[j] & 0x0F);
        float hf = (float)((qs[j] >> 4) & 0x0F);
        lo[j] = fmaf(xb[j], d * (lf - 8.0f), lo[j]);
        hi[j] = fmaf(xb[16 + j], d * (hf - 8.0f), hi[j]);
    }
}

/* linear.rs:1164-1185 (X4) == linear.rs:1319-1343 (plain). */
static inline void q8_0_block_acc(float d, const uint8_t *qs, const float *xb, float *lo,
                                  float *hi) {
    for (int j = 0; j < 16; j++) {
        lo[j] = fmaf(xb[j], d * (float)(int8_t)qs[j], lo[j]);
        hi[j] = fmaf(xb[16 + j], d * (float)(int8_t)qs[16 + j], hi[j]);
    }
}

static inline float finish_lohi(const float *lo, const float *hi) {
    float s[16];
    for (int j = 0; j < 16; j++) s[j] = lo[j] + hi[j];
    return reduce16(s);
}

/* linear_q4_0x4_avx512_range / linear_q8_0x4_avx512_range
 * (linear.rs:909-1072, 1096-1213): whole groups are computed, only the
 * lanes inside [start,end) are stored. */
ZO_CLONES
static void range_x4(const float *x, const uint8_t *w, float *out, size_t in_dim, int t,
                     size_t start, size_t end) {
    size_t nb = in_dim / 32;
    size_t gbytes = (t == ZO_Q4_0) ? 72 : 136, qb = (t == ZO_Q4_0) ? 16 : 32;
    size_t i = start;
    while (i < end) {
        size_t g = i / 4, lane_lo = i - g * 4, rows_left = end - g * 4;
        size_t lane_hi = rows_left < 4 ? rows_left : 4;
        const uint8_t *gbase = w + g * nb * gbytes;
        float lo[4][16], hi[4][16];
        memset(lo, 0, sizeof lo);
        memset(hi, 0, sizeof hi);
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = gbase + b * gbytes;
            const float *xb = x + b * 32;
            for (int r = 0; r < 4; r++) {
                float d = rd_fp16(blk + 2 * r);
                if (t == ZO_Q4_0) q4_0_block_acc(d, blk + 8 + r * qb, xb, lo[r], hi[r]);
                else q8_0_block_acc(d, blk + 8 + r * qb, xb, lo[r], hi[r]);
            }
        }
        for (size_t r = lane_lo; r < lane_hi; r++) out[g * 4 + r] = finish_lohi(lo[r], hi[r]);
        i = g * 4 + lane_hi;
    }
}

/* linear_q4_0_avx512_range / linear_q8_0_avx512_range (plain layout;
 * row pairing does not change any row's operation order). */
ZO_CLONES
static void range_plain_q(const float *x, const uint8_t *w, float *out, size_t in_dim, int t,
                          size_t start, size_t end) {
    size_t nb = in_dim / 32, bb = (t == ZO_Q4_0) ? 18 : 34;
    for (size_t i = start; i < end; i++) {
        float lo[16] = {0}, hi[16] = {0};
        const uint8_t *row = w + i * nb * bb;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + b * bb;
            float d = rd_fp16(blk);
            if (t == ZO_Q4_0) q4_0_block_acc(d, blk + 2, x + b * 32, lo, hi);
            else q8_0_block_acc(d, blk + 2, x + b * 32, lo, hi);
        }
        out[i] = finish_lohi(lo, hi);
    }
}

/* linear_q4k_avx512_range (linear.rs:150-306). */
ZO_CLONES
static void range_q4k(const float *x, const uint8_t *w, float *out, size_t in_dim,
                      size_t start, size_t end) {
    size_t nb = in_dim / 256;
    for (size_t i = start; i < end; i++) {
        float a0[16] = {0}, a1[16] = {0}, a2[16] = {0}, a3[16] = {0};
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = w + (i * nb + b) * 144;
            float d = rd_fp16(blk), dmin = rd_fp16(blk + 2);
            const uint8_t *scales = blk + 4, *qs = blk + 16;
            const float *xb = x + b * 256;
            int is = 0, qo = 0;
            for (int g = 0; g < 4; g++) {
                uint8_t sc0, mn0, sc1, mn1;
                zo_get_scale_min_k4(scales, is, &sc0, &mn0);
                zo_get_scale_min_k4(scales, is + 1, &sc1, &mn1);
                float d1 = d * (float)sc0, m1 = dmin * (float)mn0;
                float d2 = d * (float)sc1, m2 = dmin * (float)mn1;
                const float *xg = xb + g * 64;
                for (int j = 0; j < 16; j++) {
                    a0[j] = fmaf(xg[j], fmaf(d1, (float)(qs[qo + j] & 0xF), -m1), a0[j]);
                    a1[j] = fmaf(xg[16 + j], fmaf(d1, (float)(qs[qo + 16 + j] & 0xF), -m1), a1[j]);
                    a2[j] = fmaf(xg[32 + j], fmaf(d2, (float)(qs[qo + j] >> 4), -m2), a2[j]);
                    a3[j] = fmaf(xg[48 + j], fmaf(d2, (float)(qs[qo + 16 + j] >> 4), -m2), a3[j]);
                }
                qo += 32;
                is += 2;
            }
        }
        float s[16];
        for (int j = 0; j < 16; j++) s[j] = (a0[j] + a1[j]) + (a2[j] + a3[j]);
        out[i] = reduce16(s);
    }
}

/* linear_q6k_avx512_range (linear.rs:352-504). */
ZO_CLONES
static void range_q6k(const float *x, const uint8_t *w, float *out, size_t in_dim,
                      size_t start, size_t end) {
    size_t nb = in_dim / 256;
    for (size_t i = start; i < end; i++) {
        float a0[16] = {0}, a1[16] = {0}, a2[16] = {0}, a3[16] = {0};
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = w + (i * nb + b) * 210;
            float d = rd_fp16(blk + 208);
            const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
            const float *xb = x + b * 256;
            for (int h = 0; h < 2; h++) {
                int qlo = 64 * h, qho = 32 * h, sco = 8 * h, yo = 128 * h;
                for (int is = 0; is < 2; is++) {
                    int l = is * 16;
                    float s1 = d * (float)(int8_t)sc[sco + is];
                    float s2 = d * (float)(int8_t)sc[sco + is + 2];
                    float s3 = d * (float)(int8_t)sc[sco + is + 4];
                    float s4 = d * (float)(int8_t)sc[sco + is + 6];
                    for (int j = 0; j < 16; j++) {
                        int lo_b = ql[qlo + l + j], hi_b = ql[qlo + l + 32 + j], hb = qh[qho + l + j];
                        int q1 = ((lo_b & 0xF) | ((hb & 3) << 4)) - 32;
                        int q2 = ((hi_b & 0xF) | (((hb >> 2) & 3) << 4)) - 32;
                        int q3 = ((lo_b >> 4) | (((hb >> 4) & 3) << 4)) - 32;
                        int q4 = ((hi_b >> 4) | (((hb >> 6) & 3) << 4)) - 32;
                        a0[j] = fmaf(xb[yo + l + j], s1 * (float)q1, a0[j]);
                        a1[j] = fmaf(xb[yo + l + 32 + j], s2 * (float)q2, a1[j]);
                        a2[j] = fmaf(xb[yo + l + 64 + j], s3 * (float)q3, a2[j]);
                        a3[j] = fmaf(xb[yo + l + 96 + j], s4 * (float)q4, a3[j]);
                    }
                }
            }
        }
        float s[16];
        for (int j = 0; j < 16; j++) s[j] = (a0[j] + a1[j]) + (a2[j] + a3[j]);
        out[i] = reduce16(s);
    }
}

int zo_linear_range(const float *x, const uint8_t *w, float *out, size_t in_dim,
                    size_t out_dim, int t, int il, size_t start, size_t end) {
    size_t be, bb;
    if (type_geom(t, &be, &bb) || in_dim % be || end > out_dim || start > end) return -1;
    if (il == 4) {
        if ((t != ZO_Q4_0 && t != ZO_Q8_0) || out_dim % 4) return -1;
        range_x4(x, w, out, in_dim, t, start, end);
        return 0;
    }
    if (il != 1) return -1;
    switch (t) {
    case ZO_Q4_0:
    case ZO_Q8_0: range_plain_q(x, w, out, in_dim, t, start, end); break;
    case ZO_Q4K: range_q4k(x, w, out, in_dim, start, end); break;
    case ZO_Q6K: range_q6k(x, w, out, in_dim, start, end); break;
    }
    return 0;
}

int zo_linear_f64(const float *x, const uint8_t *w, double *out, size_t in_dim,
                  size_t out_dim, int t, int il) {
    float *row = (float *)malloc(in_dim * sizeof(float));
    if (!row) return -1;
    size_t be, bb;
    if (type_geom(t, &be, &bb) || in_dim % be) { free(row); return -1; }
    size_t nb = in_dim / be;
    for (size_t r = 0; r < out_dim; r++) {
        if (il == 4) {
            if (out_dim % 4) { free(row); return -1; }
            uint8_t tmp[34];
            for (size_t b = 0; b < nb; b++) {
                memcpy(tmp, x4_d(w, r, b, nb, t), 2);
                memcpy(tmp + 2, x4_qs(w, r, b, nb, t), bb - 2);
                if (t == ZO_Q4_0) dq_q4_0_block(tmp, row + b * 32);
                else dq_q8_0_block(tmp, row + b * 32);
            }
        } else {
            zo_dequant_tensor(w + r * nb * bb, row, 1, in_dim, t, 1);
        }
        double acc = 0.0;
        for (size_t k = 0; k < in_dim; k++) acc += (double)x[k] * (double)row[k];
        out[r] = acc;
    }
    free(row);
    return 0;
}

/* ------------------------------------------------------------------ */
/* X4 interleave.  tools/silicatepack.py:982-1029: per group of 4 rows */
/* and K-block b: the four fp16 scales, then the four quant bodies.     */
/* ------------------------------------------------------------------ */

int zo_interleave_x4(const uint8_t *plain, uint8_t *x4, size_t rows, size_t in_dim, int t) {
    if ((t != ZO_Q4_0 && t != ZO_Q8_0) || rows % 4 || in_dim % 32) return -1;
    size_t nb = in_dim / 32, bb = (t == ZO_Q4_0) ? 18 : 34;
    uint8_t *o = x4;
    for (size_t g = 0; g < rows; g += 4)
        for (size_t b = 0; b < nb; b++) {
            for (int l = 0; l < 4; l++) {
                memcpy(o, plain + ((g + l) * nb + b) * bb, 2);
                o += 2;
            }
            for (int l = 0; l < 4; l++) {
                memcpy(o, plain + ((g + l) * nb + b) * bb + 2, bb - 2);
                o += bb - 2;
            }
        }
    return 0;
}

int zo_deinterleave_x4(const uint8_t *x4, uint8_t *plain, size_t rows, size_t in_dim, int t) {
    if ((t != ZO_Q4_0 && t != ZO_Q8_0) || rows % 4 || in_dim % 32) return -1;
    size_t nb = in_dim / 32, bb = (t == ZO_Q4_0) ? 18 : 34;
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < nb; b++) {
            uint8_t *dst = plain + (r * nb + b) * bb;
            memcpy(dst, x4_d(x4, r, b, nb, t), 2);
            memcpy(dst + 2, x4_qs(x4, r, b, nb, t), bb - 2);
        }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Packer quantizers.  tools/silicatepack.py:854-861 (fp16 bytes),     */
/* 893-907 (Q8_0), 910-940 (Q4_0).  Python float is IEEE double; Python  */
/* round() is round-half-even; struct.pack('<e') rounds to nearest even. */
/* ------------------------------------------------------------------ */

uint16_t zo_f64_to_fp16_bits(double v) {
    if (!isfinite(v)) v = 0.0;
    if (v > 65504.0) v = 65504.0;
    else if (v < -65504.0) v = -65504.0;
    uint64_t u;
    memcpy(&u, &v, 8);
    uint16_t sign = (uint16_t)((u >> 48) & 0x8000u);
    double a = fabs(v);
    if (a == 0.0) return sign;
    int e;
    frexp(a, &e); /* a = m * 2^e, m in [0.5,1): unbiased exponent of a is e-1 */
    int ue = e - 1;
    if (ue < -14) {
        /* subnormal half: units of 2^-24; round half even */
        double q = a * 16777216.0; /* exact scaling by 2^24 */
        double r = nearbyint(q);   /* default rounding mode: ties to even */
        return (uint16_t)(sign | (uint16_t)r); /* r==1024 becomes smallest normal */
    }
    /* normal: 11 significant bits */
    double scale = ldexp(1.0, 10 - ue);
    double m = nearbyint(a * scale); /* in [1024, 2048] */
    int eb = ue + 15;
    if (m >= 2048.0) {
        m = 1024.0;
        eb += 1;
    }
    /* clamp above guarantees eb <= 30 */
    return (uint16_t)(sign | (uint16_t)(eb << 10) | ((uint16_t)m & 0x3FF));
}

void zo_quantize_q8_0_row(const float *x, uint8_t *out, size_t n) {
    for (size_t b0 = 0; b0 < n; b0 += 32) {
        double v[32];
        for (int i = 0; i < 32; i++) v[i] = (b0 + i < n) ? (double)x[b0 + i] : 0.0;
        uint8_t *o = out + (b0 / 32) * 34;
        double max_abs = 0.0;
        for (int i = 0; i < 32; i++) if (fabs(v[i]) > max_abs) max_abs = fabs(v[i]);
        if (max_abs == 0.0) {
            memset(o, 0, 34);
            continue;
        }
        double d = max_abs / 127.0;
        double inv_d = 1.0 / d;
        uint16_t h = zo_f64_to_fp16_bits(d);
        o[0] = (uint8_t)(h & 0xFF);
        o[1] = (uint8_t)(h >> 8);
        for (int i = 0; i < 32; i++) {
            double q = nearbyint(v[i] * inv_d);
            if (q > 127.0) q = 127.0;
            if (q < -127.0) q = -127.0;
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

void zo_quantize_q4_0_row(const float *x, uint8_t *out, size_t n) {
    for (size_t b0 = 0; b0 < n; b0 += 32) {
        double v[32];
        for (int i = 0; i < 32; i++) v[i] = (b0 + i < n) ? (double)x[b0 + i] : 0.0;
        uint8_t *o = out + (b0 / 32) * 18;
        double max_abs = 0.0, max_signed = 0.0;
        for (int i = 0; i < 32; i++)
            if (fabs(v[i]) > max_abs) {
                max_abs = fabs(v[i]);
                max_signed = v[i];
            }
        if (max_abs == 0.0) {
            memset(o, 0, 18);
            continue;
        }
        double d = max_signed / -8.0;
        double inv_d = 1.0 / d;
        int nib[32];
        for (int i = 0; i < 32; i++) {
            double t = trunc(v[i] * inv_d + 8.5); /* Python int() truncates */
            int q = (int)t;
            nib[i] = q < 0 ? 0 : (q > 15 ? 15 : q);
        }
        uint16_t h = zo_f64_to_fp16_bits(d);
        o[0] = (uint8_t)(h & 0xFF);
        o[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 16; j++) o[2 + j] = (uint8_t)(nib[j] | (nib[j + 16] << 4));
    }
}

/* ------------------------------------------------------------------ */
/* Argmax.  argmax_f32_avx512 (linear.rs:558-609): pass 1 is the       */
/* NaN-suppressed max (ordered >), pass 2 the first index that compares */
/* equal.  Merge rule lm_argmax_propose (inference_avx512.rs:1027-1044). */
/* ------------------------------------------------------------------ */

size_t zo_argmax(const float *v, size_t n, float *max_val) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++) if (v[i] > m) m = v[i];
    if (max_val) *max_val = m;
    for (size_t i = 0; i < n; i++) if (v[i] == m) return i;
    return 0;
}

int zo_argmax_beats(float va, uint32_t ia, float vb, uint32_t ib) {
    return va > vb || (va == vb && ia < ib);
}

/* ------------------------------------------------------------------ */
/* Partition.  kernel/src/smp_partition.rs:143-220, MAX_CORES = 128,   */
/* MATMUL_BSP_DISCOUNT_PCT_CEILING = 90 (smp_partition.rs:28,33).        */
/* ------------------------------------------------------------------ */

#define ZO_MAX_CORES 128

void zo_row_range_for(size_t total, uint32_t n_cores, size_t i, size_t align, size_t *start,
                      size_t *end) {
    size_t n = n_cores < 1 ? 1 : (n_cores > ZO_MAX_CORES ? ZO_MAX_CORES : n_cores);
    if (total == 0 || i >= n) {
        *start = *end = 0;
        return;
    }
    size_t unit = align < 1 ? 1 : align;
    size_t units = unit == 1 ? total : (total + unit - 1) / unit;
    size_t base = units / n, extra = units % n;
    size_t su = i * base + (i < extra ? i : extra);
    size_t eu = su + base + (i < extra ? 1 : 0);
    size_t s = su * unit, e = eu * unit;
    *start = s < total ? s : total;
    *end = e < total ? e : total;
}

void zo_row_range_for_discounted(size_t total, uint32_t n_cores, size_t i, size_t align,
                                 size_t disc, size_t *start, size_t *end) {
    size_t n = n_cores < 1 ? 1 : (n_cores > ZO_MAX_CORES ? ZO_MAX_CORES : n_cores);
    if (disc == 0 || n <= 1) {
        zo_row_range_for(total, n_cores, i, align, start, end);
        return;
    }
    if (total == 0 || i >= n) {
        *start = *end = 0;
        return;
    }
    size_t d = disc > 90 ? 90 : disc;
    size_t unit = align < 1 ? 1 : align;
    size_t units = unit == 1 ? total : (total + unit - 1) / unit;
    size_t bsp = units * (100 - d) / (100 * n);
    size_t rem = units - bsp, m = n - 1, su, eu;
    if (i == 0) {
        su = 0;
        eu = bsp;
    } else {
        size_t j = i - 1, base = rem / m, extra = rem % m;
        su = bsp + j * base + (j < extra ? j : extra);
        eu = su + base + (j < extra ? 1 : 0);
    }
    size_t s = su * unit, e = eu * unit;
    *start = s < total ? s : total;
    *end = e < total ? e : total;
}

/* ------------------------------------------------------------------ */
/* Pinned worker pool.  Restates the reference's SMP dispatch           */
/* (smp.rs:1107-1150 AP loop spinning on an epoch; smp.rs:1567-1712      */
/* BSP publishes, runs slice 0 itself, then waits for every AP).         */
/* ------------------------------------------------------------------ */

typedef void (*zo_work_fn)(void *ctx, int idx, int n);

static struct {
    int n;                 /* participants incl. the calling thread */
    pthread_t th[ZO_MAX_CORES];
    _Atomic uint64_t epoch;
    _Atomic int done;
    _Atomic int stop;
    _Atomic int ready;
    zo_work_fn fn;
    void *ctx;
} g_pool;

static void *pool_worker(void *arg) {
    int idx = (int)(intptr_t)arg;
    /* The pool starts at epoch 0 and publishes nothing before every worker
     * is ready, so a late-starting worker cannot miss the first dispatch. */
    uint64_t last = 0;
    atomic_fetch_add_explicit(&g_pool.ready, 1, memory_order_acq_rel);
    for (;;) {
        uint64_t e;
        while ((e = atomic_load_explicit(&g_pool.epoch, memory_order_acquire)) == last) {
            if (atomic_load_explicit(&g_pool.stop, memory_order_relaxed)) return NULL;
            ZO_PAUSE();
        }
        last = e;
        g_pool.fn(g_pool.ctx, idx, g_pool.n);
        atomic_fetch_add_explicit(&g_pool.done, 1, memory_order_acq_rel);
    }
}

static void pin_to(pthread_t t, int k) {
    cpu_set_t allowed;
    if (sched_getaffinity(0, sizeof allowed, &allowed) != 0) return;
    int cnt = CPU_COUNT(&allowed), seen = 0;
    if (cnt <= 0) return;
    k %= cnt;
    for (int c = 0; c < CPU_SETSIZE; c++)
        if (CPU_ISSET(c, &allowed)) {
            if (seen == k) {
                cpu_set_t one;
                CPU_ZERO(&one);
                CPU_SET(c, &one);
                pthread_setaffinity_np(t, sizeof one, &one);
                return;
            }
            seen++;
        }
}

int zo_pool_start(int n_threads) {
    zo_pool_stop();
    if (n_threads < 1) n_threads = 1;
    if (n_threads > ZO_MAX_CORES) n_threads = ZO_MAX_CORES;
    atomic_store(&g_pool.stop, 0);
    atomic_store(&g_pool.epoch, 0);
    atomic_store(&g_pool.ready, 0);
    g_pool.n = n_threads;
    for (int i = 1; i < n_threads; i++) {
        if (pthread_create(&g_pool.th[i], NULL, pool_worker, (void *)(intptr_t)i) != 0) {
            g_pool.n = i;
            break;
        }
        pin_to(g_pool.th[i], i);
    }
    while (atomic_load_explicit(&g_pool.ready, memory_order_acquire) < g_pool.n - 1) ZO_PAUSE();
    return g_pool.n;
}

void zo_pool_stop(void) {
    if (g_pool.n > 1) {
        atomic_store(&g_pool.stop, 1);
        for (int i = 1; i < g_pool.n; i++) pthread_join(g_pool.th[i], NULL);
    }
    g_pool.n = 0;
}

int zo_pool_size(void) { return g_pool.n < 1 ? 1 : g_pool.n; }

static void pool_run(zo_work_fn fn, void *ctx) {
    int n = zo_pool_size();
    if (n <= 1) {
        fn(ctx, 0, 1);
        return;
    }
    g_pool.fn = fn;
    g_pool.ctx = ctx;
    atomic_store_explicit(&g_pool.done, 0, memory_order_relaxed);
    atomic_fetch_add_explicit(&g_pool.epoch, 1, memory_order_acq_rel);
    fn(ctx, 0, n);
    while (atomic_load_explicit(&g_pool.done, memory_order_acquire) < n - 1) ZO_PAUSE();
}

/* The range kernel the pool's slices run: the scalar restatement, or its
 * AVX-512 intrinsics form (zg_avx512.c) for the CPU baseline. */
static int g_use_avx512;

int zo_set_simd(int on) {
    g_use_avx512 = on && zo_avx512_available();
    return g_use_avx512;
}

static void run_range(const float *x, const uint8_t *w, float *out, size_t in_dim, size_t out_dim, int t,
                      int il, size_t s, size_t e) {
    if (g_use_avx512) zo_linear_range_avx512(x, w, out, in_dim, out_dim, t, il, s, e);
    else zo_linear_range(x, w, out, in_dim, out_dim, t, il, s, e);
}

/* for_active_cores_for_rows (smp.rs:1430-1457): at most rows/16 cores. */
static int cores_for_rows(size_t rows) {
    size_t n = (size_t)zo_pool_size(), cap = rows / 16;
    if (cap < 1) cap = 1;
    return (int)(n < cap ? n : cap);
}

typedef struct {
    const float *x;
    const uint8_t *w;
    float *out;
    size_t in_dim, out_dim;
    int t, il, n_eff;
} lin_job;

static void lin_work(void *p, int idx, int n) {
    (void)n;
    lin_job *j = (lin_job *)p;
    if (idx >= j->n_eff) return;
    size_t s, e;
    zo_row_range_for(j->out_dim, (uint32_t)j->n_eff, (size_t)idx, (size_t)j->il, &s, &e);
    if (s < e) run_range(j->x, j->w, j->out, j->in_dim, j->out_dim, j->t, j->il, s, e);
}

int zo_linear_parallel(const float *x, const uint8_t *w, float *out, size_t in_dim,
                       size_t out_dim, int t, int il) {
    size_t be, bb;
    if (type_geom(t, &be, &bb) || in_dim % be) return -1;
    lin_job j = {x, w, out, in_dim, out_dim, t, il, cores_for_rows(out_dim)};
    pool_run(lin_work, &j);
    return 0;
}

typedef struct {
    const float *x;
    const zo_segment *segs;
    int n_segs;
    size_t in_dim, total;
    size_t base[3];
    int align, n_eff;
} fused_job;

/* fused_linear_kernel (inference_avx512.rs:826-879): clip the global range
 * to each segment and run that segment's kernel on the local range. */
static void fused_work(void *p, int idx, int n) {
    (void)n;
    fused_job *j = (fused_job *)p;
    if (idx >= j->n_eff) return;
    size_t s, e;
    zo_row_range_for(j->total, (uint32_t)j->n_eff, (size_t)idx, (size_t)j->align, &s, &e);
    for (int k = 0; k < j->n_segs; k++) {
        size_t ss = j->base[k], se = ss + j->segs[k].out_dim;
        size_t lo = s > ss ? s : ss, hi = e < se ? e : se;
        if (lo < hi)
            run_range(j->x, j->segs[k].w, j->segs[k].out, j->in_dim, j->segs[k].out_dim,
                      j->segs[k].ggml_type, j->segs[k].interleave, lo - ss, hi - ss);
    }
}

int zo_linear_fused_parallel(const float *x, const zo_segment *segs, int n_segs, size_t in_dim) {
    if (n_segs < 1 || n_segs > 3) return -1;
    fused_job j;
    memset(&j, 0, sizeof j);
    j.x = x;
    j.segs = segs;
    j.n_segs = n_segs;
    j.in_dim = in_dim;
    j.align = 1;
    for (int k = 0; k < n_segs; k++) {
        j.base[k] = j.total;
        j.total += segs[k].out_dim;
        if (segs[k].interleave > j.align) j.align = segs[k].interleave;
    }
    j.n_eff = cores_for_rows(j.total);
    pool_run(fused_work, &j);
    return 0;
}

typedef struct {
    lin_job lin;
    pthread_mutex_t mu; /* per-range candidates merge under the beats() order */
    float best_v;
    uint32_t best_i;
} lm_job;

static void lm_work(void *p, int idx, int n) {
    (void)n;
    lm_job *j = (lm_job *)p;
    if (idx >= j->lin.n_eff) return;
    size_t s, e;
    zo_row_range_for(j->lin.out_dim, (uint32_t)j->lin.n_eff, (size_t)idx, (size_t)j->lin.il, &s, &e);
    if (s >= e) return;
    run_range(j->lin.x, j->lin.w, j->lin.out, j->lin.in_dim, j->lin.out_dim, j->lin.t, j->lin.il, s, e);
    float mv;
    size_t li = zo_argmax(j->lin.out + s, e - s, &mv);
    uint32_t gi = (uint32_t)(s + li);
    pthread_mutex_lock(&j->mu);
    if (zo_argmax_beats(mv, gi, j->best_v, j->best_i)) {
        j->best_v = mv;
        j->best_i = gi;
    }
    pthread_mutex_unlock(&j->mu);
}

size_t zo_lm_head_linear_argmax_parallel(const float *x, const uint8_t *w, float *logits,
                                         size_t in_dim, size_t out_dim, int t, int il,
                                         float *max_val) {
    lm_job j;
    memset(&j, 0, sizeof j);
    j.lin = (lin_job){x, w, logits, in_dim, out_dim, t, il, cores_for_rows(out_dim)};
    pthread_mutex_init(&j.mu, NULL);
    j.best_v = -INFINITY;
    j.best_i = UINT32_MAX;
    pool_run(lm_work, &j);
    pthread_mutex_destroy(&j.mu);
    if (max_val) *max_val = j.best_v;
    return j.best_i == UINT32_MAX ? 0 : j.best_i;
}

/* ------------------------------------------------------------------ */
/* Decode-step ops (scalar crate operators).                            */
/* rmsnorm ops.rs:29-52; RopeContext::new ops.rs:79-93; rope ops.rs:     */
/* 111-132 (NeoX half split); softmax attention.rs:48-84; SiLU*up in     */
/* operand order silu = g/(1+exp(-g)) then *up (activation.rs:115-148,   */
/* forward_pass.rs:421).                                                 */
/* ------------------------------------------------------------------ */

void zo_rmsnorm(const float *in, const float *weight, float *out, size_t n, float eps) {
    float ssq = 0.0f;
    for (size_t i = 0; i < n; i++) ssq = ssq + in[i] * in[i];
    float mean_sq = ssq / (float)n;
    float rms = sqrtf(mean_sq + eps);
    float rinv = 1.0f / rms;
    for (size_t i = 0; i < n; i++) out[i] = in[i] * rinv * weight[i];
}

void zo_rope_inv_freqs(float *inv, int half, float freq_base) {
    float hd = (float)(half * 2);
    for (int i = 0; i < half; i++) {
        float ex = -2.0f * (float)i / hd;
        inv[i] = powf(freq_base, ex);
    }
}

void zo_rope(float *qk, const float *inv, int half, size_t position) {
    float pos = (float)position;
    for (int i = 0; i < half; i++) {
        float th = pos * inv[i];
        float c = cosf(th), s = sinf(th);
        float x0 = qk[i], y0 = qk[i + half];
        qk[i] = x0 * c - y0 * s;
        qk[i + half] = x0 * s + y0 * c;
    }
}

int zo_softmax(float *s, size_t n) {
    if (n == 0) return 0;
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++) if (s[i] > m) m = s[i];
    if (!isfinite(m)) return -1;
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float e = expf(s[i] - m);
        s[i] = e;
        sum = sum + e;
    }
    if (sum <= 0.0f || !isfinite(sum)) return -1;
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) s[i] = s[i] * inv;
    return 0;
}

void zo_silu_mul(const float *g, const float *u, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float silu = g[i] / (1.0f + expf(-g[i]));
        out[i] = silu * u[i];
    }
}

/* dot_product_f32_avx512 (linear.rs:515-535): 16-lane fmadd + reduce. */
static float dot16(const float *a, const float *b, size_t len) {
    float acc[16] = {0};
    size_t ch = len / 16;
    for (size_t c = 0; c < ch; c++)
        for (int j = 0; j < 16; j++) acc[j] = fmaf(a[c * 16 + j], b[c * 16 + j], acc[j]);
    float r = reduce16(acc);
    for (size_t j = ch * 16; j < len; j++) r = r + a[j] * b[j];
    return r;
}

/* ------------------------------------------------------------------ */
/* Q8_0-activation GEMM (no reference counterpart).                      */
/* ------------------------------------------------------------------ */

int zo_gemm_q8act(const uint8_t *xq, const uint8_t *w, float *y, size_t m, size_t n, size_t k,
                  int wt, int il) {
    if (k % 32 || (wt != ZO_Q4_0 && wt != ZO_Q8_0) || (il != 1 && il != 4)) return -1;
    if (il == 4 && n % 4) return -1;
    size_t nb = k / 32, bb = (wt == ZO_Q4_0) ? 18 : 34;
    for (size_t i = 0; i < m; i++) {
        const uint8_t *xr = xq + i * nb * 34;
        for (size_t r = 0; r < n; r++) {
            float acc = 0.0f;
            for (size_t b = 0; b < nb; b++) {
                const uint8_t *xb = xr + b * 34;
                const uint8_t *dp, *qp;
                if (il == 4) {
                    dp = x4_d(w, r, b, nb, wt);
                    qp = x4_qs(w, r, b, nb, wt);
                } else {
                    dp = w + (r * nb + b) * bb;
                    qp = dp + 2;
                }
                int32_t isum = 0;
                if (wt == ZO_Q4_0) {
                    for (int j = 0; j < 16; j++) {
                        isum += ((int)(qp[j] & 15) - 8) * (int8_t)xb[2 + j];
                        isum += ((int)(qp[j] >> 4) - 8) * (int8_t)xb[2 + 16 + j];
                    }
                } else {
                    for (int j = 0; j < 32; j++) isum += (int8_t)qp[j] * (int8_t)xb[2 + j];
                }
                float s = rd_fp16(dp) * rd_fp16(xb);
                acc = fmaf(s, (float)isum, acc);
            }
            y[i * n + r] = acc;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Q4_K x Q8_K integer path (kernel/src/arch/x86_64/math/vnni.rs,       */
/* feature "vnni-acceleration"): the ggml Q8_K activation quantizer and  */
/* the integer Q4_K dot.                                                 */
/* ------------------------------------------------------------------ */

/* quantize_row_q8k (vnni.rs:78-170): per 256 values, the first value of
 * largest magnitude (max_val), iscale = -127 / max_val in f32, q =
 * rintf(v * iscale) clamped to [-128, 127], d = 1 / iscale, 16 int16 sums
 * of 16 q each.  Block: f32 d, 256 int8, 16 int16 (292 bytes). */
void zo_quantize_row_q8k(const float *x, uint8_t *out, size_t n) {
    for (size_t b = 0; b < n / 256; b++) {
        const float *v = x + b * 256;
        uint8_t *o = out + b * ZO_Q8K_BYTES;
        float amax = 0.0f, max_val = 0.0f;
        for (int j = 0; j < 256; j++) {
            float av = fabsf(v[j]);
            if (av > amax) {
                amax = av;
                max_val = v[j];
            }
        }
        if (amax == 0.0f) {
            memset(o, 0, ZO_Q8K_BYTES);
            continue;
        }
        float iscale = -127.0f / max_val;
        int32_t bsums[16] = {0};
        for (int j = 0; j < 256; j++) {
            float t = rintf(v[j] * iscale);
            /* Rust's `as i32`: NaN -> 0, saturating */
            int32_t q = isnan(t) ? 0 : (t >= 2147483647.0f ? INT32_MAX : (t <= -2147483648.0f ? INT32_MIN : (int32_t)t));
            if (q > 127) q = 127;
            if (q < -128) q = -128;
            o[4 + j] = (uint8_t)(int8_t)q;
            bsums[j / 16] += q;
        }
        float d = 1.0f / iscale;
        memcpy(o, &d, 4);
        for (int k = 0; k < 16; k++) {
            int32_t c = bsums[k] < -32768 ? -32768 : (bsums[k] > 32767 ? 32767 : bsums[k]);
            int16_t s16 = (int16_t)c;
            memcpy(o + 260 + 2 * k, &s16, 2);
        }
    }
}

/* unpack_mins_and_scales (vnni.rs:176-205): the 12 scale bytes of a Q4_K
 * superblock as 8 six-bit scales then 8 six-bit mins (ggml's utmp form). */
void zo_unpack_mins_and_scales(const uint8_t *s12, uint8_t *out16) {
    uint32_t u[4];
    memcpy(u, s12, 12);
    u[3] = ((u[2] >> 4) & 0x0f0f0f0fu) | (((u[1] >> 6) & 0x03030303u) << 4);
    uint32_t uaux = u[1] & 0x3f3f3f3fu;
    u[1] = (u[2] & 0x0f0f0f0fu) | (((u[0] >> 6) & 0x03030303u) << 4);
    u[2] = uaux;
    u[0] &= 0x3f3f3f3fu;
    memcpy(out16, u, 16);
}

/* linear_q4k_vnni_range (vnni.rs:258-476): per row, per superblock b in
 * order, int_sum = sum_g sc_g * sum_{i in g} nibble_i * q8_i (exact),
 * min_sum = sum_g m_g * (bsum[2g] + bsum[2g+1]);
 * sumf_dot += (d_w * d_q8) * (float)int_sum;
 * sumf_min += (dmin_w * d_q8) * (float)min_sum;  out = sumf_dot - sumf_min.
 * Sub-block g covers elements 32g..32g+31: low nibbles of qs[32(g/2)..+32]
 * for even g, high nibbles for odd g. */
int zo_linear_q4k_q8k_range(const uint8_t *q8k, const uint8_t *w, float *out, size_t in_dim, size_t start,
                            size_t end) {
    if (in_dim % 256) return -1;
    size_t nb = in_dim / 256;
    for (size_t r = start; r < end; r++) {
        float sumf_dot = 0.0f, sumf_min = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *wb = w + (r * nb + b) * 144;
            const uint8_t *xb = q8k + b * ZO_Q8K_BYTES;
            float dw = rd_fp16(wb), dminw = rd_fp16(wb + 2);
            uint8_t sm[16];
            zo_unpack_mins_and_scales(wb + 4, sm);
            const uint8_t *qs = wb + 16;
            const int8_t *q8 = (const int8_t *)(xb + 4);
            float dq8;
            memcpy(&dq8, xb, 4);
            int64_t int_sum = 0;
            for (int g = 0; g < 8; g++) {
                int32_t sub = 0;
                for (int i = 0; i < 32; i++) {
                    uint8_t byte = qs[(g / 2) * 32 + i];
                    int nib = (g & 1) ? (byte >> 4) : (byte & 15);
                    sub += nib * (int32_t)q8[g * 32 + i];
                }
                int_sum += (int64_t)sub * (int64_t)sm[g];
            }
            int32_t min_sum = 0;
            for (int g = 0; g < 8; g++) {
                int16_t lo, hi;
                memcpy(&lo, xb + 260 + 4 * g, 2);
                memcpy(&hi, xb + 262 + 4 * g, 2);
                min_sum += (int32_t)sm[8 + g] * ((int32_t)lo + (int32_t)hi);
            }
            float dc = dw * dq8, dmc = dminw * dq8;
            sumf_dot = sumf_dot + dc * (float)int_sum;
            sumf_min = sumf_min + dmc * (float)min_sum;
        }
        out[r] = sumf_dot - sumf_min;
    }
    return 0;
}

/* Q6_K x Q8_K: the integer construction of linear_q4k_vnni_range applied to
 * the Q6_K layout.  No reference counterpart (the reference's integer path,
 * vnni.rs:258-476, covers Q4_K only); it is the arithmetic of the K-quant
 * prefill GEMM.  Element e of a superblock (dequant.rs:328-355: half n =
 * e / 128, quarter Q = (e % 128) / 32, l = e % 32) has the 6-bit value
 * ((ql[64n + l + 32(Q & 1)] >> 4(Q >> 1)) & 15) | (((qh[32n + l] >> 2Q) & 3) << 4)
 * and the int8 scale sc[e / 16].  Per row, per superblock b in order:
 * int_sum = sum_g sc_g * sum_{e in 16g..16g+15} (q6_e - 32) * q8_e (exact),
 * sumf = sumf + (d_w * d_q8) * (float)int_sum. */
int zo_linear_q6k_q8k_range(const uint8_t *q8k, const uint8_t *w, float *out, size_t in_dim, size_t start,
                            size_t end) {
    if (in_dim % 256) return -1;
    size_t nb = in_dim / 256;
    for (size_t r = start; r < end; r++) {
        float sumf = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *wb = w + (r * nb + b) * 210;
            const uint8_t *xb = q8k + b * ZO_Q8K_BYTES;
            const uint8_t *ql = wb, *qh = wb + 128;
            const int8_t *sc = (const int8_t *)(wb + 192);
            const int8_t *q8 = (const int8_t *)(xb + 4);
            float dq8;
            memcpy(&dq8, xb, 4);
            int64_t int_sum = 0;
            for (int g = 0; g < 16; g++) {
                int32_t sub = 0;
                for (int i = 0; i < 16; i++) {
                    int e = 16 * g + i, n = e / 128, Q = (e % 128) / 32, l = e % 32;
                    int lo4 = (ql[64 * n + l + 32 * (Q & 1)] >> (4 * (Q >> 1))) & 15;
                    int hi2 = (qh[32 * n + l] >> (2 * Q)) & 3;
                    sub += ((lo4 | (hi2 << 4)) - 32) * (int32_t)q8[e];
                }
                int_sum += (int64_t)sub * (int64_t)sc[g];
            }
            float dc = rd_fp16(wb + 208) * dq8;
            sumf = sumf + dc * (float)int_sum;
        }
        out[r] = sumf;
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Full forward pass.  forward_single_token_avx512                      */
/* (kernel/src/inference_avx512.rs:1826-1987) with the attention block   */
/* gqa_attention_single_token_avx512 (:1527-1810) and the LM head        */
/* lm_head_argmax_avx512 (:1200-1270).  KV cache layout                  */
/* [layer][K|V][t][kv_head][head_dim] (kv_cache.rs:17-31).               */
/* ------------------------------------------------------------------ */

struct zo_model {
    zo_model_desc d;
    zo_layer *layers;
    zo_layer_quants *quants;  /* per layer, always filled */
    float *kv;
    float *hidden, *norm, *q, *k, *v, *attn, *proj, *gate, *up, *act, *scores, *logits;
    float *inv_freqs;
    /* the non-finite latch (FINITE_DIAG_TRIPPED / FIRST_NF_BUF,
     * inference_avx512.rs:95, 233-235), per model */
    int nf_tripped;
    size_t nf_len;
    char nf[32];
};

size_t zo_nonfinite_text(const float *buf, size_t n, int layer, const char *stage, char *out) {
    for (size_t i = 0; i < n; i++) {
        float v = buf[i];
        if (isfinite(v)) continue;
        /* finite_diag passes the first non-finite element's NaN / Inf flags
         * (inference_avx512.rs:108-113); the text is cut at FIRST_NF_CAP */
        char t[96];
        int k = snprintf(t, sizeof t, "L%02d %s n%d i%d", layer, stage, isnan(v) ? 1 : 0, isinf(v) ? 1 : 0);
        size_t len = k < 0 ? 0 : (k > 32 ? 32 : (size_t)k);
        memcpy(out, t, len);
        return len;
    }
    return 0;
}

/* finite_diag (inference_avx512.rs:101-131): the first call that finds a
 * NaN/Inf in buf latches its text; every later call returns at once. */
static void finite_diag(zo_model *m, const float *buf, size_t n, int layer, const char *stage) {
    if (m->nf_tripped) return;
    size_t len = zo_nonfinite_text(buf, n, layer, stage, m->nf);
    if (len) {
        m->nf_len = len;
        m->nf_tripped = 1;
    }
}

/* first_nonfinite_detail (inference_avx512.rs:264-275) */
size_t zo_model_first_nonfinite(const zo_model *m, char *buf) {
    memcpy(buf, m->nf, m->nf_len);
    return m->nf_len;
}

zo_model *zo_model_create(const zo_model_desc *desc) {
    zo_model *m = (zo_model *)calloc(1, sizeof *m);
    if (!m) return NULL;
    m->d = *desc;
    m->layers = (zo_layer *)malloc(sizeof(zo_layer) * (size_t)desc->n_layers);
    m->quants = (zo_layer_quants *)malloc(sizeof(zo_layer_quants) * (size_t)desc->n_layers);
    if (!m->layers || !m->quants) {
        free(m->layers);
        free(m->quants);
        free(m);
        return NULL;
    }
    memcpy(m->layers, desc->layers, sizeof(zo_layer) * (size_t)desc->n_layers);
    for (int l = 0; l < desc->n_layers; l++)
        for (int p = 0; p < 7; p++) {
            m->quants[l].type[p] = desc->layer_quants ? desc->layer_quants[l].type[p] : desc->lin_type;
            m->quants[l].interleave[p] = desc->layer_quants ? desc->layer_quants[l].interleave[p] : desc->lin_interleave;
        }
    m->d.layers = m->layers;
    m->d.layer_quants = m->quants;
    size_t H = (size_t)desc->hidden, F = (size_t)desc->ffn;
    size_t qd = (size_t)desc->n_q_heads * desc->head_dim, kvd = (size_t)desc->n_kv_heads * desc->head_dim;
    m->kv = (float *)calloc((size_t)desc->n_layers * 2 * desc->max_ctx * kvd, sizeof(float));
    m->hidden = (float *)calloc(H, 4);
    m->norm = (float *)calloc(H > qd ? H : qd, 4);
    m->q = (float *)calloc(qd, 4);
    m->k = (float *)calloc(kvd, 4);
    m->v = (float *)calloc(kvd, 4);
    m->attn = (float *)calloc(qd, 4);
    m->proj = (float *)calloc(H, 4);
    m->gate = (float *)calloc(F, 4);
    m->up = (float *)calloc(F, 4);
    m->act = (float *)calloc(F, 4);
    m->scores = (float *)calloc((size_t)desc->n_q_heads * desc->max_ctx, 4);  /* one stripe per head */
    m->logits = (float *)calloc(desc->vocab_padded, 4);
    m->inv_freqs = (float *)calloc((size_t)desc->head_dim / 2, 4);
    if (!m->kv || !m->logits) {
        zo_model_destroy(m);
        return NULL;
    }
    zo_rope_inv_freqs(m->inv_freqs, desc->head_dim / 2, desc->rope_theta);
    return m;
}

void zo_model_destroy(zo_model *m) {
    if (!m) return;
    free(m->layers);
    free(m->quants);
    free(m->kv);
    free(m->hidden); free(m->norm); free(m->q); free(m->k); free(m->v); free(m->attn);
    free(m->proj); free(m->gate); free(m->up); free(m->act); free(m->scores); free(m->logits);
    free(m->inv_freqs);
    free(m);
}

typedef struct {
    const float *q, *kc, *vc;
    size_t T, kvd, hd, gqa, nq, stride;
    float scale;
    float *scores, *out;
    int n_eff;
    _Atomic int err;
} attn_job;

/* One participant's heads: row_range_for over the query heads, align 1
 * (ParallelMatmulContext::for_work_units, smp.rs:1460-1480). */
static void attn_work(void *p, int idx, int n) {
    (void)n;
    attn_job *j = (attn_job *)p;
    if (idx >= j->n_eff) return;
    size_t s, e;
    zo_row_range_for(j->nq, (uint32_t)j->n_eff, (size_t)idx, 1, &s, &e);
    if (s < e && zo_attn_heads_avx512(j->q, j->kc, j->vc, j->T, j->kvd, j->hd, j->gqa, j->scale, j->scores,
                                      j->stride, j->out, s, e))
        atomic_store_explicit(&j->err, 1, memory_order_relaxed);
}

/* ATTN_PARALLEL_MIN_TOKENS default (inference_avx512.rs:1383). */
#define ZO_ATTN_PARALLEL_MIN_TOKENS 64

/* All query heads of one token over cache rows 0..T-1
 * (gqa_attention_single_token_avx512, inference_avx512.rs:1744-1800):
 * scores q.k * scale, softmax, weighted sum of V rows in row order.  With
 * the AVX-512 kernels in force (the CPU baseline) the heads run in
 * intrinsics, spread over the pool from 64 cached rows on, one head per
 * participant at most (inference_avx512.rs:1676-1730); every head's
 * arithmetic is the same either way.  `scores` holds one stripe of
 * d->max_ctx floats per query head. */
static int attend(const zo_model_desc *d, const float *kc, const float *vc, const float *q, size_t T,
                  float scale, float *scores, float *out) {
    size_t hd = (size_t)d->head_dim, nq = (size_t)d->n_q_heads, nkv = (size_t)d->n_kv_heads;
    size_t kvd = nkv * hd, gqa = nq / nkv;
    if (g_use_avx512) {
        int n = zo_pool_size();
        if (T >= ZO_ATTN_PARALLEL_MIN_TOKENS && nq >= 2 && n > 1) {
            attn_job j = {q, kc, vc, T, kvd, hd, gqa, nq, (size_t)d->max_ctx, scale, scores, out,
                          (int)(nq < (size_t)n ? nq : (size_t)n), 0};
            pool_run(attn_work, &j);
            return atomic_load(&j.err) ? -4 : 0;
        }
        return zo_attn_heads_avx512(q, kc, vc, T, kvd, hd, gqa, scale, scores, d->max_ctx, out, 0, nq) ? -4 : 0;
    }
    for (size_t h = 0; h < nq; h++) {
        size_t kh = h / gqa;
        const float *qv = q + h * hd;
        for (size_t t = 0; t < T; t++) scores[t] = dot16(qv, kc + t * kvd + kh * hd, hd) * scale;
        if (zo_softmax(scores, T)) return -4;
        float *o = out + h * hd;
        for (size_t i = 0; i < hd; i++) o[i] = 0.0f;
        for (size_t t = 0; t < T; t++) {
            const float *vv = vc + t * kvd + kh * hd;
            float wgt = scores[t];
            for (size_t i = 0; i < hd; i++) o[i] = fmaf(wgt, vv[i], o[i]);
        }
    }
    return 0;
}

int zo_model_forward(zo_model *m, uint32_t token, size_t pos, float *hidden_out) {
    const zo_model_desc *d = &m->d;
    size_t H = (size_t)d->hidden, F = (size_t)d->ffn, hd = (size_t)d->head_dim;
    size_t nq = (size_t)d->n_q_heads, nkv = (size_t)d->n_kv_heads;
    size_t qd = nq * hd, kvd = nkv * hd;
    if (pos >= d->max_ctx || token >= d->vocab_padded) return -3;
    /* embed_lookup_dispatch (forward_pass.rs:311-370) */
    size_t be, bb;
    if (type_geom(d->embd_type, &be, &bb) || H % be) return -3;
    zo_dequant_tensor(d->token_embd + (size_t)token * (H / be) * bb, m->hidden, 1, H, d->embd_type, 1);
    float scale = 1.0f / sqrtf((float)hd);
    size_t T = pos + 1;
    for (int l = 0; l < d->n_layers; l++) {
        const zo_layer *L = &m->layers[l];
        const int *qt = m->quants[l].type, *il = m->quants[l].interleave;
        zo_rmsnorm(m->hidden, L->attn_norm, m->norm, H, d->rms_eps);
        finite_diag(m, m->norm, H, l, "attn_norm_in");
        zo_segment qkv[3] = {
            {L->attn_q, m->q, qd, qt[0], il[0]},
            {L->attn_k, m->k, kvd, qt[1], il[1]},
            {L->attn_v, m->v, kvd, qt[2], il[2]},
        };
        zo_linear_fused_parallel(m->norm, qkv, 3, H);
        float tmp[512];
        for (size_t h = 0; h < nq; h++) {
            zo_rmsnorm(m->q + h * hd, L->q_norm, tmp, hd, d->rms_eps);
            memcpy(m->q + h * hd, tmp, hd * 4);
            zo_rope(m->q + h * hd, m->inv_freqs, (int)(hd / 2), pos);
        }
        for (size_t h = 0; h < nkv; h++) {
            zo_rmsnorm(m->k + h * hd, L->k_norm, tmp, hd, d->rms_eps);
            memcpy(m->k + h * hd, tmp, hd * 4);
            zo_rope(m->k + h * hd, m->inv_freqs, (int)(hd / 2), pos);
        }
        float *kc = m->kv + ((size_t)l * 2 + 0) * d->max_ctx * kvd;
        float *vc = m->kv + ((size_t)l * 2 + 1) * d->max_ctx * kvd;
        memcpy(kc + pos * kvd, m->k, kvd * 4);
        memcpy(vc + pos * kvd, m->v, kvd * 4);
        if (attend(d, kc, vc, m->q, T, scale, m->scores, m->attn)) return -4;
        zo_linear_parallel(m->attn, L->attn_o, m->proj, qd, H, qt[3], il[3]);
        for (size_t i = 0; i < H; i++) m->hidden[i] = m->hidden[i] + m->proj[i];
        finite_diag(m, m->proj, H, l, "attn_out");
        finite_diag(m, m->hidden, H, l, "post_attn_residual");
        zo_rmsnorm(m->hidden, L->ffn_norm, m->norm, H, d->rms_eps);
        zo_segment gu[2] = {
            {L->ffn_gate, m->gate, F, qt[4], il[4]},
            {L->ffn_up, m->up, F, qt[5], il[5]},
        };
        zo_linear_fused_parallel(m->norm, gu, 2, H);
        zo_silu_mul(m->gate, m->up, m->act, F);
        zo_linear_parallel(m->act, L->ffn_down, m->proj, F, H, qt[6], il[6]);
        for (size_t i = 0; i < H; i++) m->hidden[i] = m->hidden[i] + m->proj[i];
        finite_diag(m, m->proj, H, l, "mlp_out");
        finite_diag(m, m->hidden, H, l, "post_mlp_residual");
    }
    if (hidden_out) memcpy(hidden_out, m->hidden, H * 4);
    return 0;
}

typedef struct {
    const uint8_t *xk; /* n Q8_K rows of k values */
    const uint8_t *w;
    float *y;          /* [n][out_dim] */
    size_t n, out_dim, k;
    int qt, n_eff;
    _Atomic int rc;
} kq_gemm_job;

static void kq_gemm_work(void *p, int idx, int nt) {
    (void)nt;
    kq_gemm_job *j = (kq_gemm_job *)p;
    if (idx >= j->n_eff) return;
    size_t s, e, xb = j->k / 256 * ZO_Q8K_BYTES;
    zo_row_range_for(j->out_dim, (uint32_t)j->n_eff, (size_t)idx, 1, &s, &e);
    for (size_t i = 0; i < j->n && s < e; i++) {
        int rc = j->qt == 12 ? zo_linear_q4k_q8k_range(j->xk + i * xb, j->w, j->y + i * j->out_dim, j->k, s, e)
                             : zo_linear_q6k_q8k_range(j->xk + i * xb, j->w, j->y + i * j->out_dim, j->k, s, e);
        if (rc) atomic_store(&j->rc, rc);
    }
}

/* One GEMM of the batched prefill: n fp32 activation rows X ([n][k]) times
 * the out_dim rows of w into Y ([n][out_dim]).  Q4_0 / Q8_0 weights read the
 * rows' Q8_0 encoding xq (zo_quantize_q8_0_row of X, made by the caller)
 * through zo_gemm_q8act; plain Q4_K / Q6_K weights read each row's Q8_K
 * encoding (zo_quantize_row_q8k into xk, n * k / 256 blocks) through the
 * integer dot (zo_linear_q4k_q8k_range / zo_linear_q6k_q8k_range), the
 * output rows split over the pool (each output is one row's dot, so the
 * split changes no bits). */
static int prefill_gemm(const float *X, const uint8_t *xq, uint8_t *xk, const uint8_t *w, float *Y, size_t n,
                        size_t out_dim, size_t k, int qt, int il) {
    if (qt == 12 || qt == 14) {
        if (il != 1 || k % 256) return -3;
        for (size_t i = 0; i < n; i++) zo_quantize_row_q8k(X + i * k, xk + i * (k / 256) * ZO_Q8K_BYTES, k);
        kq_gemm_job j;
        memset(&j, 0, sizeof j);
        j.xk = xk;
        j.w = w;
        j.y = Y;
        j.n = n;
        j.out_dim = out_dim;
        j.k = k;
        j.qt = qt;
        j.n_eff = cores_for_rows(out_dim);
        atomic_store(&j.rc, 0);
        pool_run(kq_gemm_work, &j);
        return atomic_load(&j.rc) ? -3 : 0;
    }
    return zo_gemm_q8act(xq, w, Y, n, out_dim, k, qt, il) ? -3 : 0;
}

/* Batched prefill with quantized activations (no reference counterpart: the
 * reference runs the prompt token by token).  n rows at positions
 * pos0..pos0+n-1; per layer every row is rmsnormed, quantized (the packer's
 * Q8_0 encoder, zo_quantize_q8_0_row, for Q4_0 / Q8_0 weights; the
 * reference's quantize_row_q8k for plain Q4_K / Q6_K weights) and multiplied
 * by each projection's GEMM (prefill_gemm); QK-norm, RoPE, the cache store,
 * attention, SwiGLU and the residual adds are the single-token pass's per
 * row.  Leaves the last row's final hidden state in the model (for
 * zo_model_lm_head). */
int zo_model_prefill_q8(zo_model *m, const uint32_t *tokens, size_t n, size_t pos0, float *hidden_out) {
    const zo_model_desc *d = &m->d;
    size_t H = (size_t)d->hidden, F = (size_t)d->ffn, hd = (size_t)d->head_dim;
    size_t nq = (size_t)d->n_q_heads, nkv = (size_t)d->n_kv_heads;
    size_t qd = nq * hd, kvd = nkv * hd;
    if (n == 0 || pos0 + n > d->max_ctx) return -3;
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= d->vocab_padded) return -3;
    for (int l = 0; l < d->n_layers; l++)
        for (int p = 0; p < 7; p++)
            if (m->quants[l].type[p] != 2 && m->quants[l].type[p] != 8 && m->quants[l].type[p] != 12 &&
                m->quants[l].type[p] != 14)
                return -3;
    size_t be, bb;
    if (type_geom(d->embd_type, &be, &bb) || H % be) return -3;
    size_t km = H > qd ? H : qd;
    if (F > km) km = F;
    float *X = (float *)malloc(n * H * 4), *T = (float *)malloc(n * km * 4);
    float *Q = (float *)malloc(n * qd * 4), *K = (float *)malloc(n * kvd * 4), *V = (float *)malloc(n * kvd * 4);
    float *A = (float *)malloc(n * qd * 4), *P = (float *)malloc(n * H * 4);
    float *G = (float *)malloc(n * F * 4), *U = (float *)malloc(n * F * 4);
    uint8_t *xq = (uint8_t *)malloc(n * (km / 32) * 34);
    uint8_t *xk = (uint8_t *)malloc(n * (km / 256 + 1) * ZO_Q8K_BYTES);
    float *scores = (float *)malloc((pos0 + n) * 4);
    int rc = 0;
    if (!X || !T || !Q || !K || !V || !A || !P || !G || !U || !xq || !xk || !scores) rc = -5;
    for (size_t i = 0; i < n && !rc; i++)
        zo_dequant_tensor(d->token_embd + (size_t)tokens[i] * (H / be) * bb, X + i * H, 1, H, d->embd_type, 1);
    float scale = 1.0f / sqrtf((float)hd);
    float tmp[512];
    for (int l = 0; l < d->n_layers && !rc; l++) {
        const zo_layer *L = &m->layers[l];
        const int *qt = m->quants[l].type, *il = m->quants[l].interleave;
        float *kc = m->kv + ((size_t)l * 2 + 0) * d->max_ctx * kvd;
        float *vc = m->kv + ((size_t)l * 2 + 1) * d->max_ctx * kvd;
        for (size_t i = 0; i < n; i++) zo_rmsnorm(X + i * H, L->attn_norm, T + i * H, H, d->rms_eps);
        zo_quantize_q8_0_row(T, xq, n * H);
        if (prefill_gemm(T, xq, xk, L->attn_q, Q, n, qd, H, qt[0], il[0]) ||
            prefill_gemm(T, xq, xk, L->attn_k, K, n, kvd, H, qt[1], il[1]) ||
            prefill_gemm(T, xq, xk, L->attn_v, V, n, kvd, H, qt[2], il[2])) {
            rc = -3;
            break;
        }
        for (size_t i = 0; i < n; i++) {
            size_t pos = pos0 + i;
            for (size_t h = 0; h < nq; h++) {
                float *x = Q + i * qd + h * hd;
                zo_rmsnorm(x, L->q_norm, tmp, hd, d->rms_eps);
                memcpy(x, tmp, hd * 4);
                zo_rope(x, m->inv_freqs, (int)(hd / 2), pos);
            }
            for (size_t h = 0; h < nkv; h++) {
                float *x = K + i * kvd + h * hd;
                zo_rmsnorm(x, L->k_norm, tmp, hd, d->rms_eps);
                memcpy(x, tmp, hd * 4);
                zo_rope(x, m->inv_freqs, (int)(hd / 2), pos);
            }
            memcpy(kc + pos * kvd, K + i * kvd, kvd * 4);
            memcpy(vc + pos * kvd, V + i * kvd, kvd * 4);
        }
        for (size_t i = 0; i < n && !rc; i++)
            if (attend(d, kc, vc, Q + i * qd, pos0 + i + 1, scale, scores, A + i * qd)) rc = -4;
        if (rc) break;
        zo_quantize_q8_0_row(A, xq, n * qd);
        if (prefill_gemm(A, xq, xk, L->attn_o, P, n, H, qd, qt[3], il[3])) {
            rc = -3;
            break;
        }
        for (size_t i = 0; i < n * H; i++) X[i] = X[i] + P[i];
        for (size_t i = 0; i < n; i++) zo_rmsnorm(X + i * H, L->ffn_norm, T + i * H, H, d->rms_eps);
        zo_quantize_q8_0_row(T, xq, n * H);
        if (prefill_gemm(T, xq, xk, L->ffn_gate, G, n, F, H, qt[4], il[4]) ||
            prefill_gemm(T, xq, xk, L->ffn_up, U, n, F, H, qt[5], il[5])) {
            rc = -3;
            break;
        }
        zo_silu_mul(G, U, T, n * F);
        zo_quantize_q8_0_row(T, xq, n * F);
        if (prefill_gemm(T, xq, xk, L->ffn_down, P, n, H, F, qt[6], il[6])) {
            rc = -3;
            break;
        }
        for (size_t i = 0; i < n * H; i++) X[i] = X[i] + P[i];
    }
    if (!rc) {
        memcpy(m->hidden, X + (n - 1) * H, H * 4);
        if (hidden_out) memcpy(hidden_out, m->hidden, H * 4);
    }
    free(X); free(T); free(Q); free(K); free(V); free(A); free(P); free(G); free(U); free(xq); free(xk); free(scores);
    return rc;
}

int zo_model_lm_head(zo_model *m, float *logits_out, uint32_t *token, float *max_val) {
    const zo_model_desc *d = &m->d;
    size_t H = (size_t)d->hidden;
    zo_rmsnorm(m->hidden, d->output_norm, m->norm, H, d->rms_eps);
    float mv;
    size_t idx = zo_lm_head_linear_argmax_parallel(m->norm, d->lm_head, m->logits, H, d->vocab_padded,
                                                   d->head_type, d->head_interleave, &mv);
    if (logits_out) memcpy(logits_out, m->logits, d->vocab_padded * 4);
    if (token) *token = (uint32_t)idx;
    if (max_val) *max_val = mv;
    if (!isfinite(mv)) return -1;
    if (idx >= d->vocab_real) return -2;
    return 0;
}
