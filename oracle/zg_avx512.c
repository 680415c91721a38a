/*
 * zg_avx512.c -- AVX-512 intrinsics restatement of the reference's CPU
 * range kernels, the CPU baseline that bench.py times beside the GPU.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only tests/, __graft_entry__
 * smoke() and bench.py's cpu_baseline legs load it (through oracle/zo.py).
 *
 * Every function follows one kernel of
 * kernel/src/arch/x86_64/math/linear.rs instruction for instruction: the
 * same intrinsics (_mm512_cvtepu8_epi32 / _mm512_cvtepi8_epi32 widening,
 * _mm512_cvtepi32_ps, _mm512_mul_ps / _mm512_sub_ps dequant,
 * _mm512_fmadd_ps / _mm512_fmsub_ps accumulation), the same accumulator
 * assignment and the same final _mm512_reduce_add_ps.  The scalar
 * restatement in zg_oracle.c (zo_linear_range) models each __m512 lane as a
 * float and is pinned by the reference's KATs and f64 brute force; this
 * file must give the same bits (tests/test_oracle_avx512.py).
 *
 * The fp16 scale decode is the scalar fp16_to_f32 the reference calls per
 * block (linear.rs:66-92 replica of dequant.rs:28-61).
 */
#include <immintrin.h>
#include <stddef.h>
#include <stdint.h>

#include "zg_oracle.h"

int zo_avx512_available(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") ? 1 : 0;
#else
    return 0;
#endif
}

#if defined(__x86_64__)
#pragma GCC push_options
#pragma GCC target("avx512f")

static inline float half_at(const uint8_t *p) { return zo_fp16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

static inline __m512i widen_u8(const uint8_t *p) {
    return _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i *)p));
}
static inline __m512i widen_i8(const uint8_t *p) {
    return _mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)p));
}

/* One Q4_0 block body (16 nibble bytes at qs, scale dv) into a row's two
 * accumulators: low nibbles pair with x[0..16), high nibbles with
 * x[16..32), each as (q - 8) * d (linear.rs:985-1040 per row). */
static inline void q4_body(__m512 dv, const uint8_t *qs, __m512 xlo, __m512 xhi, __m512 *lo, __m512 *hi) {
    const __m512i mask = _mm512_set1_epi32(0x0F);
    const __m512 bias = _mm512_set1_ps(8.0f);
    const __m512i b = widen_u8(qs);
    const __m512 ql = _mm512_cvtepi32_ps(_mm512_and_epi32(b, mask));
    *lo = _mm512_fmadd_ps(xlo, _mm512_mul_ps(dv, _mm512_sub_ps(ql, bias)), *lo);
    const __m512 qh = _mm512_cvtepi32_ps(_mm512_and_epi32(_mm512_srli_epi32(b, 4), mask));
    *hi = _mm512_fmadd_ps(xhi, _mm512_mul_ps(dv, _mm512_sub_ps(qh, bias)), *hi);
}

/* One Q8_0 block body (32 signed bytes at qs): d * q, sign-extended
 * (linear.rs:1164-1195 per row). */
static inline void q8_body(__m512 dv, const uint8_t *qs, __m512 xlo, __m512 xhi, __m512 *lo, __m512 *hi) {
    *lo = _mm512_fmadd_ps(xlo, _mm512_mul_ps(dv, _mm512_cvtepi32_ps(widen_i8(qs))), *lo);
    *hi = _mm512_fmadd_ps(xhi, _mm512_mul_ps(dv, _mm512_cvtepi32_ps(widen_i8(qs + 16))), *hi);
}

/* linear_q4_0x4_avx512_range (linear.rs:909-1072) and
 * linear_q8_0x4_avx512_range (:1096-1213): a whole 4-row group is
 * computed, only the rows inside [start, end) are stored. */
static void x4_range(const float *x, const uint8_t *w, float *out, size_t in_dim, int t, size_t start,
                     size_t end) {
    const size_t nb = in_dim / 32;
    const size_t gbb = (t == ZO_Q4_0) ? 72 : 136, qb = (t == ZO_Q4_0) ? 16 : 32;
    const size_t gstride = nb * gbb;
    size_t i = start;
    while (i < end) {
        const size_t g = i / 4, lane_lo = i - 4 * g, left = end - 4 * g;
        const size_t lane_hi = left < 4 ? left : 4;
        const uint8_t *gb = w + g * gstride;
        __m512 lo[4], hi[4];
        for (int r = 0; r < 4; r++) lo[r] = hi[r] = _mm512_setzero_ps();
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = gb + b * gbb;
            const __m512 xlo = _mm512_loadu_ps(x + 32 * b), xhi = _mm512_loadu_ps(x + 32 * b + 16);
            for (int r = 0; r < 4; r++) {
                const __m512 dv = _mm512_set1_ps(half_at(blk + 2 * r));
                if (t == ZO_Q4_0) q4_body(dv, blk + 8 + qb * r, xlo, xhi, &lo[r], &hi[r]);
                else q8_body(dv, blk + 8 + qb * r, xlo, xhi, &lo[r], &hi[r]);
            }
        }
        for (size_t r = lane_lo; r < lane_hi; r++) out[4 * g + r] = _mm512_reduce_add_ps(_mm512_add_ps(lo[r], hi[r]));
        i = 4 * g + lane_hi;
    }
}

/* linear_q4_0_avx512_range (linear.rs:710-859) and
 * linear_q8_0_avx512_range (:1271-1402): row pairs share the x loads, an
 * odd last row takes the single-row body; both give each row the same
 * operation sequence. */
static void plain_range(const float *x, const uint8_t *w, float *out, size_t in_dim, int t, size_t start,
                        size_t end) {
    const size_t nb = in_dim / 32, bb = (t == ZO_Q4_0) ? 18 : 34, rb = nb * bb;
    size_t i = start;
    for (; i + 1 < end; i += 2) {
        const uint8_t *r0 = w + i * rb, *r1 = r0 + rb;
        __m512 lo0 = _mm512_setzero_ps(), hi0 = lo0, lo1 = lo0, hi1 = lo0;
        for (size_t b = 0; b < nb; b++) {
            const __m512 xlo = _mm512_loadu_ps(x + 32 * b), xhi = _mm512_loadu_ps(x + 32 * b + 16);
            const uint8_t *b0 = r0 + b * bb, *b1 = r1 + b * bb;
            const __m512 d0 = _mm512_set1_ps(half_at(b0)), d1 = _mm512_set1_ps(half_at(b1));
            if (t == ZO_Q4_0) {
                q4_body(d0, b0 + 2, xlo, xhi, &lo0, &hi0);
                q4_body(d1, b1 + 2, xlo, xhi, &lo1, &hi1);
            } else {
                q8_body(d0, b0 + 2, xlo, xhi, &lo0, &hi0);
                q8_body(d1, b1 + 2, xlo, xhi, &lo1, &hi1);
            }
        }
        out[i] = _mm512_reduce_add_ps(_mm512_add_ps(lo0, hi0));
        out[i + 1] = _mm512_reduce_add_ps(_mm512_add_ps(lo1, hi1));
    }
    for (; i < end; i++) {
        const uint8_t *r0 = w + i * rb;
        __m512 lo = _mm512_setzero_ps(), hi = lo;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *b0 = r0 + b * bb;
            const __m512 d0 = _mm512_set1_ps(half_at(b0));
            const __m512 xlo = _mm512_loadu_ps(x + 32 * b), xhi = _mm512_loadu_ps(x + 32 * b + 16);
            if (t == ZO_Q4_0) q4_body(d0, b0 + 2, xlo, xhi, &lo, &hi);
            else q8_body(d0, b0 + 2, xlo, xhi, &lo, &hi);
        }
        out[i] = _mm512_reduce_add_ps(_mm512_add_ps(lo, hi));
    }
}

/* linear_q4k_avx512_range (linear.rs:150-306): per 64-element group j, the
 * low nibbles of qs[32j..32j+32) take d*sc0 - dmin*mn0 (elements 64j..+32),
 * the high nibbles d*sc1 - dmin*mn1 (elements 64j+32..+64); the four
 * 16-element pieces accumulate round-robin into acc0..acc3, which reduce as
 * (acc0 + acc1) + (acc2 + acc3). */
static void q4k_range(const float *x, const uint8_t *w, float *out, size_t in_dim, size_t start, size_t end) {
    const size_t nb = in_dim / 256;
    const __m512i mask = _mm512_set1_epi32(0x0F);
    for (size_t i = start; i < end; i++) {
        __m512 acc[4];
        for (int a = 0; a < 4; a++) acc[a] = _mm512_setzero_ps();
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = w + (i * nb + b) * 144;
            const float d = half_at(blk), dmin = half_at(blk + 2);
            const uint8_t *qs = blk + 16;
            const float *xb = x + 256 * b;
            for (int j = 0; j < 4; j++) {
                uint8_t sc0, mn0, sc1, mn1;
                zo_get_scale_min_k4(blk + 4, 2 * j, &sc0, &mn0);
                zo_get_scale_min_k4(blk + 4, 2 * j + 1, &sc1, &mn1);
                const __m512 d1 = _mm512_set1_ps(d * (float)sc0), m1 = _mm512_set1_ps(dmin * (float)mn0);
                const __m512 d2 = _mm512_set1_ps(d * (float)sc1), m2 = _mm512_set1_ps(dmin * (float)mn1);
                const uint8_t *q = qs + 32 * j;
                const float *xg = xb + 64 * j;
                for (int half = 0; half < 2; half++) {  /* l = 0 and l = 16 */
                    const __m512i by = widen_u8(q + 16 * half);
                    const __m512 lo = _mm512_cvtepi32_ps(_mm512_and_epi32(by, mask));
                    acc[half] = _mm512_fmadd_ps(_mm512_loadu_ps(xg + 16 * half), _mm512_fmsub_ps(d1, lo, m1),
                                                acc[half]);
                }
                for (int half = 0; half < 2; half++) {
                    const __m512i by = widen_u8(q + 16 * half);
                    const __m512 hi = _mm512_cvtepi32_ps(_mm512_and_epi32(_mm512_srli_epi32(by, 4), mask));
                    acc[2 + half] = _mm512_fmadd_ps(_mm512_loadu_ps(xg + 32 + 16 * half),
                                                    _mm512_fmsub_ps(d2, hi, m2), acc[2 + half]);
                }
            }
        }
        out[i] = _mm512_reduce_add_ps(_mm512_add_ps(_mm512_add_ps(acc[0], acc[1]), _mm512_add_ps(acc[2], acc[3])));
    }
}

/* linear_q6k_avx512_range (linear.rs:352-504): per half h and 16-lane
 * piece l, four 6-bit values from ql[l], ql[l+32] (low / high nibble) and
 * qh[l] bits {0,2,4,6}, minus 32, scaled by d * sc (that product first),
 * into acc0..acc3 for elements y+l, +32, +64, +96. */
static void q6k_range(const float *x, const uint8_t *w, float *out, size_t in_dim, size_t start, size_t end) {
    const size_t nb = in_dim / 256;
    const __m512i m4 = _mm512_set1_epi32(0x0F), m2 = _mm512_set1_epi32(0x03), z = _mm512_set1_epi32(32);
    for (size_t i = start; i < end; i++) {
        __m512 acc[4];
        for (int a = 0; a < 4; a++) acc[a] = _mm512_setzero_ps();
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = w + (i * nb + b) * 210;
            const float d = half_at(blk + 208);
            const uint8_t *ql = blk, *qh = blk + 128;
            const int8_t *sc = (const int8_t *)(blk + 192);
            const float *xb = x + 256 * b;
            for (int h = 0; h < 2; h++) {
                for (int is = 0; is < 2; is++) {
                    const int l = 16 * is;
                    const __m512i lo = widen_u8(ql + 64 * h + l), hi = widen_u8(ql + 64 * h + l + 32);
                    const __m512i hb = widen_u8(qh + 32 * h + l);
                    __m512i q[4];
                    q[0] = _mm512_sub_epi32(
                        _mm512_or_epi32(_mm512_and_epi32(lo, m4), _mm512_slli_epi32(_mm512_and_epi32(hb, m2), 4)), z);
                    q[1] = _mm512_sub_epi32(
                        _mm512_or_epi32(_mm512_and_epi32(hi, m4),
                                        _mm512_slli_epi32(_mm512_and_epi32(_mm512_srli_epi32(hb, 2), m2), 4)),
                        z);
                    q[2] = _mm512_sub_epi32(
                        _mm512_or_epi32(_mm512_and_epi32(_mm512_srli_epi32(lo, 4), m4),
                                        _mm512_slli_epi32(_mm512_and_epi32(_mm512_srli_epi32(hb, 4), m2), 4)),
                        z);
                    q[3] = _mm512_sub_epi32(
                        _mm512_or_epi32(_mm512_and_epi32(_mm512_srli_epi32(hi, 4), m4),
                                        _mm512_slli_epi32(_mm512_and_epi32(_mm512_srli_epi32(hb, 6), m2), 4)),
                        z);
                    for (int s = 0; s < 4; s++) {
                        const __m512 scale = _mm512_set1_ps(d * (float)sc[8 * h + is + 2 * s]);
                        const __m512 xv = _mm512_loadu_ps(xb + 128 * h + l + 32 * s);
                        acc[s] = _mm512_fmadd_ps(xv, _mm512_mul_ps(scale, _mm512_cvtepi32_ps(q[s])), acc[s]);
                    }
                }
            }
        }
        out[i] = _mm512_reduce_add_ps(_mm512_add_ps(_mm512_add_ps(acc[0], acc[1]), _mm512_add_ps(acc[2], acc[3])));
    }
}

/* dot_product_f32_avx512 (linear.rs:515-535): 16-lane fmadd over the
 * head dim, one _mm512_reduce_add_ps, then the scalar tail. */
static inline float dot_avx512(const float *a, const float *b, size_t len) {
    __m512 acc = _mm512_setzero_ps();
    const size_t chunks = len / 16;
    for (size_t i = 0; i < chunks; i++)
        acc = _mm512_fmadd_ps(_mm512_loadu_ps(a + 16 * i), _mm512_loadu_ps(b + 16 * i), acc);
    float r = _mm512_reduce_add_ps(acc);
    for (size_t j = 16 * chunks; j < len; j++) r += a[j] * b[j];
    return r;
}

/* weighted_add_f32_avx512 (linear.rs:611-639): out += w * v. */
static inline void weighted_add_avx512(float w, const float *v, float *out, size_t len) {
    const __m512 wv = _mm512_set1_ps(w);
    const size_t chunks = len / 16;
    for (size_t i = 0; i < chunks; i++)
        _mm512_storeu_ps(out + 16 * i,
                         _mm512_fmadd_ps(wv, _mm512_loadu_ps(v + 16 * i), _mm512_loadu_ps(out + 16 * i)));
    for (size_t j = 16 * chunks; j < len; j++) out[j] += w * v[j];
}

static int attn_heads_avx512(const float *q, const float *kc, const float *vc, size_t T, size_t kvd, size_t hd,
                      size_t gqa, float scale, float *scores, size_t stride, float *out, size_t h0, size_t h1) {
    int err = 0;
    for (size_t h = h0; h < h1; h++) {
        const size_t kh = h / gqa;
        float *sb = scores + h * stride;
        for (size_t t = 0; t < T; t++) sb[t] = dot_avx512(q + h * hd, kc + t * kvd + kh * hd, hd) * scale;
        if (zo_softmax(sb, T)) {
            err = 1;
            continue;
        }
        float *o = out + h * hd;
        for (size_t i = 0; i < hd; i++) o[i] = 0.0f;
        for (size_t t = 0; t < T; t++) weighted_add_avx512(sb[t], vc + t * kvd + kh * hd, o, hd);
    }
    return err;
}

#pragma GCC pop_options
#endif

/* attn_heads_kernel (kernel/src/inference_avx512.rs:1459-1512) for query
 * heads [h0, h1): scores q.k * scale with dot_product_f32_avx512 in
 * ascending t into the head's score stripe, the scalar softmax, then
 * weighted_add_f32_avx512 of the V rows in ascending t.  1 if a head's
 * softmax failed (the reference's NumericalInstability), -2 without
 * AVX-512F. */
int zo_attn_heads_avx512(const float *q, const float *kc, const float *vc, size_t T, size_t kvd, size_t hd,
                         size_t gqa, float scale, float *scores, size_t stride, float *out, size_t h0,
                         size_t h1) {
    if (!zo_avx512_available()) return -2;
#if defined(__x86_64__)
    return attn_heads_avx512(q, kc, vc, T, kvd, hd, gqa, scale, scores, stride, out, h0, h1);
#else
    return -2;
#endif
}

/* Same contract as zo_linear_range; -2 when the CPU has no AVX-512F. */
int zo_linear_range_avx512(const float *x, const uint8_t *w, float *out, size_t in_dim, size_t out_dim, int t,
                           int il, size_t start, size_t end) {
    if (!zo_avx512_available()) return -2;
    const size_t be = (t == ZO_Q4K || t == ZO_Q6K) ? 256 : 32;
    if ((t != ZO_Q4_0 && t != ZO_Q8_0 && t != ZO_Q4K && t != ZO_Q6K) || in_dim % be || end > out_dim ||
        start > end)
        return -1;
#if defined(__x86_64__)
    if (il == 4) {
        if ((t != ZO_Q4_0 && t != ZO_Q8_0) || out_dim % 4) return -1;
        x4_range(x, w, out, in_dim, t, start, end);
        return 0;
    }
    if (il != 1) return -1;
    if (t == ZO_Q4_0 || t == ZO_Q8_0) plain_range(x, w, out, in_dim, t, start, end);
    else if (t == ZO_Q4K) q4k_range(x, w, out, in_dim, start, end);
    else q6k_range(x, w, out, in_dim, start, end);
    return 0;
#else
    return -2;
#endif
}
