// zg_device.h -- device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zg {

// GgmlType ids (crates/zero-gguf-parser/src/lib.rs:95-126).
enum QType : uint32_t { Q4_0 = 2, Q8_0 = 8, Q4K = 12, Q6K = 14 };

// IEEE binary16 bits -> f32, bit-exact with fp16_to_f32
// (crates/zero-gguf-parser/src/dequant.rs:28-61): normals and subnormals
// through v_cvt_f32_f16 (exact; fp16 denormals are not flushed in the HIP
// default float mode), inf/NaN rebuilt from the bits so that a signalling
// NaN keeps its payload exactly as the reference's bit construction does
// (the hardware conversion would quiet it).
__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
  h &= 0xFFFFu;
  const float f = (float)__builtin_bit_cast(_Float16, (unsigned short)h);
  const uint32_t special = ((h & 0x8000u) << 16) | 0x7F800000u | ((h & 0x3FFu) << 13);
  return ((h & 0x7C00u) == 0x7C00u) ? __uint_as_float(special) : f;
}

// A kernel's small output stores, written through the L2 (a relaxed
// agent-scope atomic store: global_store with sc1).  A launch that leaves
// dirty lines in the L2s of the eight XCDs pays for their write-back when it
// ends; stored through, they are on their way out when the last wave
// retires (the one-batch 6144x2048 GEMV: 3.34 against 3.47 us in a probe of
// its structure; nontemporal stores 3.67 us).  The value is stored as is.
#ifndef ZG_STORE_WT
#define ZG_STORE_WT 1
#endif
__device__ __forceinline__ void store_out(float* p, float v) {
  if (ZG_STORE_WT) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}
__device__ __forceinline__ void store_out(uint32_t* p, uint32_t v) {
  if (ZG_STORE_WT) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}
__device__ __forceinline__ void store_out(uint64_t* p, uint64_t v) {
  if (ZG_STORE_WT) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

// The value through an empty asm: the compiler can no longer see which
// bits are zero.  Used on masked quant words, so that a byte conversion
// stays one v_cvt_f32_ubyteN instead of being folded with the mask into a
// bit-field extract plus a conversion.
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

// Native 128-bit vector for global loads (nontemporal builtins need a
// clang vector type, not HIP's uint4 wrapper).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Wave64 butterfly sum over aligned lane segments of width W (power of 2,
// W <= 64).  Every lane of the segment ends with the segment total.
template <int W>
__device__ __forceinline__ float seg_sum(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// DPP move (row_mask/bank_mask all rows/banks, bound_ctrl off).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// A quad_perm read whose every source lane is valid: bound_ctrl on, so no
// old value is set up and the move can fold into its user.
template <int CTRL>
__device__ __forceinline__ float quad_pick(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Full wave64 sum, wave-uniform result: xor-1 and xor-2 within quads
// (quad_perm), half-row and row mirrors give every lane its 16-lane row
// sum, then the four row sums are read out with v_readlane.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Full wave64 max, wave-uniform result (same DPP pattern as wave_sum).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Sum over aligned groups of W lanes (W = 16 or 32).  Within a 16-lane DPP
// row: quad swaps, then rotations by 4 and 8 (every lane of the row gets the
// row total).  W = 32 then adds row 0's total into row 1 and row 2's into
// row 3 (row_bcast:15); the group total is valid in the upper row of each
// pair only (lanes 16..31 and 48..63).  Returns, for W = 16, the total in
// every lane.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x124>(v);  // row_ror:4
  v += dpp_f32<0x128>(v);  // row_ror:8
  if (W == 32)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
  return v;
}

// Orders this wave's LDS writes before its later LDS reads (lanes of one
// wave exchanging data through LDS; no workgroup barrier needed).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Split-context attention (flash-decoding).  Each split s of a query head's
// context leaves its unnormalised output o_s (sum_t e_t v_t with
// e_t = exp(score_t - m_s)), its running max m_s and its exp-sum l_s; a
// split past the context leaves (o, m, l) = (0, -inf, 0).  The merged output
// is sum_s w_s o_s / sum_s w_s l_s with w_s = exp(m_s - max_s m_s)
// (attention.rs:48-84 softmax, regrouped by split).  One thread merges 8
// consecutive dims of one head.
constexpr int kAttnSplits = 8;  // max splits per query head

struct AttnSplitIn {
  float4 o[kAttnSplits][2];
  float2 ml[kAttnSplits];
};

// part_o: [nsplit][k] split outputs; part_ml: [nsplit][k / hd] (m, l).
__device__ __forceinline__ void attn_split_load(AttnSplitIn& in, const float* part_o, const float* part_ml, int k,
                                                int hd, int nsplit, int e0) {
  const int nh = k / hd, h = e0 / hd;
#pragma unroll
  for (int s = 0; s < kAttnSplits; s++) {
    if (s < nsplit) {
      const float4* p = reinterpret_cast<const float4*>(part_o + (size_t)s * k + e0);
      in.o[s][0] = p[0];
      in.o[s][1] = p[1];
      in.ml[s] = reinterpret_cast<const float2*>(part_ml)[s * nh + h];
    }
  }
}

// The same for two 4-element pieces of one head: o[s][0] from element e_lo,
// o[s][1] from element e_hi (the quarters of a strip lane's x-block).
__device__ __forceinline__ void attn_split_load2(AttnSplitIn& in, const float* part_o, const float* part_ml, int k,
                                                 int hd, int nsplit, int e_lo, int e_hi) {
  const int nh = k / hd, h = e_lo / hd;
#pragma unroll
  for (int s = 0; s < kAttnSplits; s++) {
    if (s < nsplit) {
      in.o[s][0] = *reinterpret_cast<const float4*>(part_o + (size_t)s * k + e_lo);
      in.o[s][1] = *reinterpret_cast<const float4*>(part_o + (size_t)s * k + e_hi);
      in.ml[s] = reinterpret_cast<const float2*>(part_ml)[s * nh + h];
    }
  }
}

__device__ __forceinline__ float4 fma4(float w, float4 a, float4 acc) {
  return make_float4(fmaf(w, a.x, acc.x), fmaf(w, a.y, acc.y), fmaf(w, a.z, acc.z), fmaf(w, a.w, acc.w));
}

__device__ __forceinline__ void attn_split_merge(const AttnSplitIn& in, int nsplit, float4& x0, float4& x1) {
  float m = in.ml[0].x;
#pragma unroll
  for (int s = 1; s < kAttnSplits; s++)
    if (s < nsplit) m = fmaxf(m, in.ml[s].x);
  float l = 0.0f;
  float4 a0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), a1 = a0;
#pragma unroll
  for (int s = 0; s < kAttnSplits; s++) {
    if (s < nsplit) {
      const float w = expf(in.ml[s].x - m);
      l = fmaf(w, in.ml[s].y, l);
      a0 = fma4(w, in.o[s][0], a0);
      a1 = fma4(w, in.o[s][1], a1);
    }
  }
  const float inv = 1.0f / l;
  x0 = make_float4(a0.x * inv, a0.y * inv, a0.z * inv, a0.w * inv);
  x1 = make_float4(a1.x * inv, a1.y * inv, a1.z * inv, a1.w * inv);
}

// Order-preserving encoding of an argmax candidate into one u64 so that a
// single atomicMax implements lm_argmax_propose
// (kernel/src/inference_avx512.rs:1027-1044): larger value wins, equal
// values go to the smaller index.  NaN is never encoded (callers skip it).
// 0 means "no candidate".
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  uint32_t b = __float_as_uint(v);
  // monotone float -> uint map: negative values flip all bits, positive set sign
  uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  // -0.0 and +0.0 compare equal in IEEE; map both to the same key
  if ((b & 0x7FFFFFFFu) == 0) k = 0x80000000u;
  return ((uint64_t)k << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

// binary64 -> binary16, round to nearest even, for finite |v| <= 65504
// (the packer clamps to that range first, silicatepack.py:854-861).
__device__ __forceinline__ uint32_t f64_to_f16_rne(double v) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t sign = (uint32_t)(u >> 48) & 0x8000u;
  const uint64_t a = u & 0x7FFFFFFFFFFFFFFFull;
  if (a == 0) return sign;
  const int e = (int)(a >> 52) - 1023;
  const uint64_t mant = (a & ((1ull << 52) - 1)) | (1ull << 52);
  if (e < -14) {
    // subnormal half: count units of 2^-24
    const int s = 28 - e;
    if (s >= 64) return sign;
    const uint64_t q = mant >> s;
    const uint64_t rem = mant & ((1ull << s) - 1);
    const uint64_t half = 1ull << (s - 1);
    const uint64_t r = q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0);
    return sign | (uint32_t)r;  // r == 1024 encodes the smallest normal
  }
  uint64_t q = mant >> 42;
  const uint64_t rem = mant & ((1ull << 42) - 1);
  const uint64_t half = 1ull << 41;
  if (rem > half || (rem == half && (q & 1))) q++;
  int eb = e + 15;
  if (q == 2048) {
    q = 1024;
    eb++;
  }
  return sign | ((uint32_t)eb << 10) | ((uint32_t)q & 0x3FFu);
}

// The packer's Q8_0 block encoder (tools/silicatepack.py:893-907) on 32
// values: amax, d = amax/127, 1/d and v/d in double as Python computes them,
// round-half-even, clamp to +-127, d stored as the RNE binary16 of the
// double d.  A block holding a non-finite value (the packer raises
// ValueError there, :877-887) gets q = 0 and d = NaN (0x7E00) so that it
// cannot pass unnoticed.  Returns the fp16 bits of d.
__device__ __forceinline__ uint32_t q8_0_encode(const float v[32], int8_t q[32]) {
  bool finite = true;
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    finite = finite && isfinite(v[i]);
    amax = fmaxf(amax, fabsf(v[i]));
  }
  if (!finite || amax == 0.0f) {
#pragma unroll
    for (int i = 0; i < 32; i++) q[i] = 0;
    return finite ? 0u : 0x7E00u;
  }
  const double dd = (double)amax / 127.0;
  const double inv = 1.0 / dd;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    double r = rint((double)v[i] * inv);
    r = fmin(127.0, fmax(-127.0, r));
    q[i] = (int8_t)(int)r;
  }
  return f64_to_f16_rne(fmin(dd, 65504.0));
}

// The same encoder with one value per lane: each aligned 32-lane segment of
// the wave is one block (every lane of the segment must be active).  Returns
// this lane's q; *dbits gets the block's fp16 d bits.
__device__ __forceinline__ int8_t q8_0_encode_lane(float v, uint32_t* dbits) {
  float amax = fabsf(v);
  float bad = isfinite(v) ? 0.0f : 1.0f;
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    bad += __shfl_xor(bad, o, 64);
  }
  if (bad != 0.0f || amax == 0.0f) {
    *dbits = bad != 0.0f ? 0x7E00u : 0u;
    return 0;
  }
  const double dd = (double)amax / 127.0;
  const double inv = 1.0 / dd;
  double r = rint((double)v * inv);
  r = fmin(127.0, fmax(-127.0, r));
  *dbits = f64_to_f16_rne(fmin(dd, 65504.0));
  return (int8_t)(int)r;
}

// Element dequantization of one block (plain-layout block bytes, or for X4
// the (d, qs) pointers), shared by the generic GEMV, the dequant kernel and
// the embedding lookups.
__device__ __forceinline__ float rd_half(const uint8_t* p) {
  return half_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}

// Dequantize element e (0..blk_elems-1) of the block at blk (plain-layout
// block bytes, or for X4 the (d, qs) pointers).  Operation order follows
// dequant.rs: Q4_0 (q-8)*d; Q8_0 q*d; Q4_K d1*q - m1; Q6_K (d*sc)*q.
__device__ __forceinline__ float deq_q4_0(float d, const uint8_t* qs, int e) {
  const int q = (e < 16) ? (qs[e] & 0xF) : (qs[e - 16] >> 4);
  return (float)(q - 8) * d;
}
__device__ __forceinline__ float deq_q8_0(float d, const uint8_t* qs, int e) {
  return (float)(int8_t)qs[e] * d;
}
__device__ __forceinline__ void q4k_scale_min(const uint8_t* s, int j, int& sc, int& mn) {
  if (j < 4) {
    sc = s[j] & 0x3F;
    mn = s[j + 4] & 0x3F;
  } else {
    sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
    mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}
__device__ __forceinline__ float deq_q4k(const uint8_t* blk, int e) {
  const float d = rd_half(blk), dmin = rd_half(blk + 2);
  const int g = e >> 6, w = e & 63;
  int sc, mn;
  q4k_scale_min(blk + 4, 2 * g + (w >= 32 ? 1 : 0), sc, mn);
  const uint8_t byte = blk[16 + 32 * g + (w & 31)];
  const int q = (w < 32) ? (byte & 0xF) : (byte >> 4);
  const float dd = d * (float)sc, m = dmin * (float)mn;
  return dd * (float)q - m;
}
__device__ __forceinline__ float deq_q6k(const uint8_t* blk, int e) {
  const float d = rd_half(blk + 208);
  const int h = e >> 7, w = e & 127, quarter = w >> 5, l = w & 31;
  const uint8_t* ql = blk + 64 * h;
  const uint8_t* qh = blk + 128 + 32 * h;
  const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * h);
  const int is = l >> 4;
  int q;
  switch (quarter) {
    case 0: q = (ql[l] & 0xF) | ((qh[l] & 3) << 4); break;
    case 1: q = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4); break;
    case 2: q = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4); break;
    default: q = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4); break;
  }
  return d * (float)sc[is + 2 * quarter] * (float)(q - 32);
}

struct BlockRef {
  const uint8_t* d;   // scale location (Q4_0/Q8_0) or block start (k-quants)
  const uint8_t* qs;  // quant bytes (Q4_0/Q8_0)
};

__device__ __forceinline__ BlockRef block_ref(const uint8_t* w, uint32_t qt, int il, size_t row,
                                              size_t b, size_t nb) {
  BlockRef br;
  if (qt == Q4_0 || qt == Q8_0) {
    const size_t bb = (qt == Q4_0) ? 18 : 34;
    if (il == 4) {
      const size_t gb = 4 * bb;
      const uint8_t* g = w + (row >> 2) * nb * gb + b * gb;
      br.d = g + 2 * (row & 3);
      br.qs = g + 8 + (row & 3) * (bb - 2);
    } else {
      br.d = w + (row * nb + b) * bb;
      br.qs = br.d + 2;
    }
  } else {
    const size_t bb = (qt == Q4K) ? 144 : 210;
    br.d = w + (row * nb + b) * bb;
    br.qs = br.d;
  }
  return br;
}

__device__ __forceinline__ float deq_elem(const BlockRef& br, uint32_t qt, float d, int e) {
  switch (qt) {
    case Q4_0: return deq_q4_0(d, br.qs, e);
    case Q8_0: return deq_q8_0(d, br.qs, e);
    case Q4K: return deq_q4k(br.d, e);
    default: return deq_q6k(br.d, e);
  }
}

// Q4_K helpers shared by the Q4_K kernels and the strip GEMV.
// sum_i q_i x_i over 4 dwords of unsigned bytes (q in 0..255) against
// 16 consecutive x values.
__device__ __forceinline__ float u8_dot16(const uint32_t* q, const float4* x) {
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const uint32_t v = q[c];
    const float4 xv = x[c];
    float& s = (c & 1) ? s1 : s0;
    s = fmaf(xv.x, (float)(v & 0xFFu), s);
    s = fmaf(xv.y, (float)((v >> 8) & 0xFFu), s);
    s = fmaf(xv.z, (float)((v >> 16) & 0xFFu), s);
    s = fmaf(xv.w, (float)(v >> 24), s);
  }
  return s0 + s1;
}

// get_scale_min_k4 (dequant.rs:75-85) for the lane's sub-blocks 2j and 2j+1,
// branch-free over the wave (j differs between lanes): for j < 2 the low six
// bits of bytes 2j, 2j+1 of w0 (scales) and w1 (mins); for j >= 2 the low /
// high nibbles of bytes 2j-4, 2j-3 of w2, with the top two bits of the same
// bytes of w0 / w1 above them.
__device__ __forceinline__ void q4k_lane_scales(uint32_t w0, uint32_t w1, uint32_t w2, int j, uint32_t& sA,
                                                uint32_t& sB, uint32_t& nA, uint32_t& nB) {
  const uint32_t sh = 16u * (uint32_t)(j & 1);
  const bool lowj = j < 2;
  const uint32_t a = w0 >> sh, b = w1 >> sh, c = w2 >> sh;
  const uint32_t wid = lowj ? 6u : 4u;
  const uint32_t hmask = lowj ? 0u : ~0u;
  const uint32_t ls = lowj ? a : c, lm = lowj ? b : (c >> 4);
  const uint32_t hs = a & hmask, hm = b & hmask;
  sA = __builtin_amdgcn_ubfe(ls, 0, wid) | (__builtin_amdgcn_ubfe(hs, 6, 2) << 4);
  sB = __builtin_amdgcn_ubfe(ls, 8, wid) | (__builtin_amdgcn_ubfe(hs, 14, 2) << 4);
  nA = __builtin_amdgcn_ubfe(lm, 0, wid) | (__builtin_amdgcn_ubfe(hm, 6, 2) << 4);
  nB = __builtin_amdgcn_ubfe(lm, 8, wid) | (__builtin_amdgcn_ubfe(hm, 14, 2) << 4);
}

// The superblock's d and dmin through the hardware fp16 conversion: exact
// for every finite value; a NaN scale gives a NaN row either way.
// get_scale_min_k4 (dequant.rs:75-85) for one sub-block sbi (0..7) of the
// 12 scale bytes w0..w2; the shifts and widths depend on sbi only, so they
// are constant per lane where sbi is: sbi < 4 takes the low six bits of
// byte sbi of w0 (scale) and w1 (min); sbi >= 4 the low / high nibble of
// byte sbi - 4 of w2, with the top two bits of byte sbi - 4 of w0 / w1
// above them (a zero-width field is 0).
__device__ __forceinline__ void q4k_sub_scale(uint32_t w0, uint32_t w1, uint32_t w2, int sbi, uint32_t& sc,
                                              uint32_t& mn) {
  const bool low = sbi < 4;
  const uint32_t o = 8u * (uint32_t)(sbi & 3);
  const uint32_t wid = low ? 6u : 4u, hw = low ? 0u : 2u;
  sc = __builtin_amdgcn_ubfe(low ? w0 : w2, o, wid) | (__builtin_amdgcn_ubfe(w0, o + 6u, hw) << 4);
  mn = __builtin_amdgcn_ubfe(low ? w1 : w2, low ? o : o + 4u, wid) | (__builtin_amdgcn_ubfe(w1, o + 6u, hw) << 4);
}

__device__ __forceinline__ float kq_half(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}

// ---------------------------------------------------------------------------
// Activations as exact integers for v_dot4_i32_i8.
//
// A 32-value block with largest magnitude M is scaled by 127 * 2^14 / M and
// rounded to the nearest integer V (|V| <= 127 * 2^14: 22 significant bits,
// an error of at most 2^-22 M per value, the order of one fp32 rounding of
// the block's largest product).  V is split into three signed bytes,
// V = 2^14 a + 2^7 b + c with b, c in [-64, 63] and a in [-127, 127], so
// that sum_j q_j V_j over int8 quants q comes out of three v_dot4_i32_i8
// chains exactly, and the row's block term is that integer times
// d * M / (127 * 2^14).
//
// Lane layout: the four lanes of a quad share one block; quad lane r holds
// the block's values 4r..4r+3 ("lo") and 16+4r..16+4r+3 ("hi").  After the
// quad exchange every lane holds, per digit k, dwords dg[k][c] = values
// 4c..4c+3 for c < 4 and 16+4(c-4).. for c >= 4: the order of the quant
// dwords of a Q4_0 block (low nibbles of dword c are values 4c..4c+3, high
// nibbles 16+4c..) and of a Q8_0 block (dword c = values 4c..4c+3).
// ---------------------------------------------------------------------------
struct XDig {
  uint32_t dg[3][8];  // digits a, b, c of the block's 32 values, packed 4 per dword
  int sum[3];         // per digit, the sum of the block's 32 digits
  float sinv;         // M / (127 * 2^14): one unit of V
};

// Three signed base-128 digits of V, each in the low byte of an int.
__device__ __forceinline__ void split_digits(int v, int& a, int& b, int& c) {
  c = __builtin_amdgcn_sbfe(v, 0, 7);   // sign-extended low 7 bits: [-64, 63]
  const int w = (v - c) >> 7;           // exact
  b = __builtin_amdgcn_sbfe(w, 0, 7);
  a = (w - b) >> 7;
}

// Low bytes of four ints into one dword (byte j from p[j]).
__device__ __forceinline__ uint32_t pack_low_bytes(int p0, int p1, int p2, int p3) {
  const uint32_t p01 = __builtin_amdgcn_perm((uint32_t)p1, (uint32_t)p0, 0x0C0C0400u);
  const uint32_t p23 = __builtin_amdgcn_perm((uint32_t)p3, (uint32_t)p2, 0x0C0C0400u);
  return __builtin_amdgcn_perm(p23, p01, 0x05040100u);
}

// Digits of four values at scale s, packed: out[k] holds digit k.
__device__ __forceinline__ void digits4(float4 x, float s, uint32_t (&out)[3]) {
  int a[4], b[4], c[4];
  const float v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int j = 0; j < 4; j++) split_digits(__float2int_rn(v[j] * s), a[j], b[j], c[j]);
  out[0] = pack_low_bytes(a[0], a[1], a[2], a[3]);
  out[1] = pack_low_bytes(b[0], b[1], b[2], b[3]);
  out[2] = pack_low_bytes(c[0], c[1], c[2], c[3]);
}

template <int S>
__device__ __forceinline__ uint32_t quad_bcast_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, S | (S << 2) | (S << 4) | (S << 6), 0xF, 0xF, false);
}

__device__ __forceinline__ int quad_sum_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  return v;
}

// The quad's block from this lane's quarter (lo = values 4r..4r+3, hi =
// 16+4r..16+4r+3).  Returns true when the integer form does not apply to
// the block: a NaN or infinity among its values, or a largest magnitude
// below 1e-30 other than zero (the scale would overflow).  The block's
// largest magnitude is an integer max over the sign-cleared bit patterns,
// which orders every finite value below +inf below every NaN.
__device__ __forceinline__ bool xdig_quad(float4 lo, float4 hi, XDig& X) {
  const uint32_t m7 = 0x7FFFFFFFu;
  uint32_t mb = max(max(__float_as_uint(lo.x) & m7, __float_as_uint(lo.y) & m7), max(__float_as_uint(lo.z) & m7, __float_as_uint(lo.w) & m7));
  mb = max(mb, max(max(__float_as_uint(hi.x) & m7, __float_as_uint(hi.y) & m7), max(__float_as_uint(hi.z) & m7, __float_as_uint(hi.w) & m7)));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0xB1, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x4E, 0xF, 0xF, false));
  const bool bad = mb >= 0x7F800000u || (mb != 0u && mb < 0x0DA24260u);  // 1e-30f
  const float m = __uint_as_float(mb);
  const float s = (mb != 0u && !bad) ? (127.0f * 16384.0f) / m : 0.0f;
  X.sinv = m * (1.0f / (127.0f * 16384.0f));
  uint32_t dl[3], dh[3];
  digits4(lo, s, dl);
  digits4(hi, s, dh);
#pragma unroll
  for (int k = 0; k < 3; k++) {
    X.dg[k][0] = quad_bcast_u32<0>(dl[k]);
    X.dg[k][1] = quad_bcast_u32<1>(dl[k]);
    X.dg[k][2] = quad_bcast_u32<2>(dl[k]);
    X.dg[k][3] = quad_bcast_u32<3>(dl[k]);
    X.dg[k][4] = quad_bcast_u32<0>(dh[k]);
    X.dg[k][5] = quad_bcast_u32<1>(dh[k]);
    X.dg[k][6] = quad_bcast_u32<2>(dh[k]);
    X.dg[k][7] = quad_bcast_u32<3>(dh[k]);
    X.sum[k] = quad_sum_i32(__builtin_amdgcn_sdot4((int)dl[k], 0x01010101, __builtin_amdgcn_sdot4((int)dh[k], 0x01010101, 0, false), false));
  }
  return bad;
}

// The three digit chains of sum_j q_j V_j for a block of 32 signed int8
// quants q, given as 8 dwords in the dg order; t0, t1, t2 enter with the
// chains' start values.  V = 2^14 a + 2^7 b + c, so the block's integer sum
// is 2^14 t0 + 2^7 t1 + t2.
// A dependent v_dot4_i32_i8 issues ~16 cycles after its predecessor, so
// each digit's chain is split into two (even and odd dwords; six chains in
// flight) and the halves are added at the end: integer sums, so the result
// is the same in any order.
__device__ __forceinline__ void xdig_chains(const uint32_t (&q)[8], const XDig& X, int& t0, int& t1, int& t2) {
  int u0 = 0, u1 = 0, u2 = 0;
#pragma unroll
  for (int c = 0; c < 8; c += 2) {
    t0 = __builtin_amdgcn_sdot4((int)q[c], (int)X.dg[0][c], t0, false);
    t1 = __builtin_amdgcn_sdot4((int)q[c], (int)X.dg[1][c], t1, false);
    t2 = __builtin_amdgcn_sdot4((int)q[c], (int)X.dg[2][c], t2, false);
    u0 = __builtin_amdgcn_sdot4((int)q[c + 1], (int)X.dg[0][c + 1], u0, false);
    u1 = __builtin_amdgcn_sdot4((int)q[c + 1], (int)X.dg[1][c + 1], u1, false);
    u2 = __builtin_amdgcn_sdot4((int)q[c + 1], (int)X.dg[2][c + 1], u2, false);
  }
  t0 += u0;
  t1 += u1;
  t2 += u2;
}

// quantize_row_q8k (kernel/src/arch/x86_64/math/vnni.rs:78-170) for one
// 256-value block held by one wave, four values per lane (e = values
// 4 lane .. 4 lane + 3 of the block):
//   max_val  the first value of largest magnitude (strict > scan: ties keep
//            the lower index; NaN never wins): the (|v| bits, ~index) key is
//            order-preserving for non-negative floats, and the winning
//            lane's own first largest value is max_val (read by shuffle)
//   q        rintf(e * iscale), iscale = -127 / max_val, clamped to
//            [-128, 127] (NaN -> 0, as Rust's `as i32` saturates)
//   d        1 / iscale
// An all-zero block gives q = 0 and d = 0.  Returns the lane's four quants
// as little-endian bytes; q holds their values.
__device__ __forceinline__ uint32_t q8k_block_lane(int lane, const float (&e)[4], int (&q)[4], float& d) {
  float best = 0.0f, bval = 0.0f;
  int bi = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float av = fabsf(e[i]);
    if (av > best) {
      best = av;
      bval = e[i];
      bi = 4 * lane + i;
    }
  }
  uint64_t key = ((uint64_t)__float_as_uint(best) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)bi);
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    const uint64_t other = __shfl_xor(key, s, 64);
    key = other > key ? other : key;
  }
  const float max_val = __shfl(bval, (int)((0xFFFFFFFFu - (uint32_t)key) >> 2), 64);
  if (__uint_as_float((uint32_t)(key >> 32)) == 0.0f) {
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = 0;
    d = 0.0f;
    return 0u;
  }
  const float iscale = -127.0f / max_val;
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float t = rintf(e[i] * iscale);
    q[i] = (t != t) ? 0 : (int)fminf(fmaxf(t, -128.0f), 127.0f);
    packed |= (uint32_t)(uint8_t)(int8_t)q[i] << (8 * i);
  }
  d = 1.0f / iscale;
  return packed;
}

// One 256-value block (four values per lane, as q8k_block_lane) into the
// K-quant GEMM's split activation arrays: the 256 int8 quants at qs, the
// block's d at *d8, the eight sums of 32 quants at bs32[0..8).
__device__ __forceinline__ void q8k_split_store(int lane, const float (&e)[4], int8_t* qs, float* d8, int16_t* bs32) {
  int q[4];
  float d;
  reinterpret_cast<uint32_t*>(qs)[lane] = q8k_block_lane(lane, e, q, d);
  int s = (q[0] + q[1]) + (q[2] + q[3]);
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 4, 64);
  if ((lane & 7) == 0) bs32[lane >> 3] = (int16_t)s;
  if (lane == 0) *d8 = d;
}

}  // namespace zg
