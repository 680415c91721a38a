// zg_strip.h -- the strip GEMV (device code shared by the GEMV launchers
// and the model's fused Q|K|V + attention kernel).
//
// Replaces the AVX-512 X4 / plain row-range kernels of the reference
// (kernel/src/arch/x86_64/math/linear.rs:710-859, 909-1072, 1096-1213,
// 1271-1402) for in_dim a multiple of 512 up to 8192.
#pragma once

#include <type_traits>

#include "zg_device.h"
#include "zg_kernels.h"

namespace zg {

// Segment of a group index.  The fields are picked with constant indices so
// that they stay in scalar registers: a dynamically indexed a.seg[s] is
// re-read from the kernel-argument segment with a vector load, a full
// memory round trip in front of every weight load that depends on it.
__device__ __forceinline__ GemvSeg seg_of(const GemvArgs& a, uint32_t item) {
  GemvSeg s = a.seg[0];
  if (a.nseg > 1 && item >= a.seg[1].g_begin) s = a.seg[1];
  if (a.nseg > 2 && item >= a.seg[2].g_begin) s = a.seg[2];
  return s;
}

// Nibble bytes (every byte 0..15) read as OCP fp8 e4m3 are exactly n * 2^-9
// (a subnormal for n < 8, exponent field 1 for 8..15), so one
// v_cvt_pk_f32_fp8 gives two elements' exact values; kNibUnit undoes the
// scale (products and sums scale by a power of two without rounding).
constexpr float kNibUnit = 512.0f;
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Sum over one Q4_0 block of one row: sum_j q_j * x_j with q the raw nibble
// (0..15); the caller applies d * (s - 8 * sum(x)).  Low nibbles of byte j
// are element j, high nibbles element j+16 (dequant.rs:186-216).  The
// nibbles are converted as fp8 bytes (two per instruction, against one
// v_cvt_f32_ubyte per element: decode 1,585-1,588 -> 1,597-1,599 tok/s,
// 151936x2048 32.5 -> 32.25 us) and the sum is rescaled by 2^9, so the
// result is bit for bit the sum of the converted nibbles.
__device__ __forceinline__ float q4_block_dot(const uint32_t* qs, const float4* xb) {
  float s_lo = 0.0f, s_hi = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const uint32_t v = qs[c];
    const uint32_t lo = opaque_u32(v & 0x0F0F0F0Fu);
    const uint32_t hi = opaque_u32((v >> 4) & 0x0F0F0F0Fu);
    const f32x2 l0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false), l1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
    const f32x2 h0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false), h1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
    const float4 xl = xb[c];
    const float4 xh = xb[4 + c];
    s_lo = fmaf(xl.x, l0.x, s_lo);
    s_lo = fmaf(xl.y, l0.y, s_lo);
    s_lo = fmaf(xl.z, l1.x, s_lo);
    s_lo = fmaf(xl.w, l1.y, s_lo);
    s_hi = fmaf(xh.x, h0.x, s_hi);
    s_hi = fmaf(xh.y, h0.y, s_hi);
    s_hi = fmaf(xh.z, h1.x, s_hi);
    s_hi = fmaf(xh.w, h1.y, s_hi);
  }
  return (s_lo + s_hi) * kNibUnit;
}

// Q8_0 block sum with the int8 quants read as unsigned bytes (q ^ 0x80 =
// q + 128); the caller subtracts 128 * sum(x).  (Converting them as
// sign-extended bytes, v_cvt_f32_i32 with an SDWA byte select, and dropping
// the offset term measured slower: fused Q|K|V Q8_0X4 4.01 against 3.87 us.)
__device__ __forceinline__ float q8u_block_dot(const uint32_t* qs, const float4* xb) {
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; c++) {
    const uint32_t v = qs[c] ^ 0x80808080u;
    const float4 xv = xb[c];
    float& s = (c & 1) ? s1 : s0;
    s = fmaf(xv.x, (float)(v & 0xFFu), s);
    s = fmaf(xv.y, (float)((v >> 8) & 0xFFu), s);
    s = fmaf(xv.z, (float)((v >> 16) & 0xFFu), s);
    s = fmaf(xv.w, (float)(v >> 24), s);
  }
  return s0 + s1;
}

// ---------------------------------------------------------------------------
// X4 strip kernel (in_dim a multiple of 512, at most 8192).
//
// The K axis is cut into strips of 16 blocks (512 values).  A wave owns one
// strip and keeps that strip's activations in registers: lane (b, r) holds
// x-block b of the strip (32 floats) and decodes row r of that block for
// every group the wave visits, loading its own 16 (Q4_0) or 32 (Q8_0) quant
// bytes and its fp16 d straight from HBM (lanes 4b..4b+3 cover one
// group-block's quant bytes contiguously, so a wave instruction spans
// ~1.1-2.2 KB of consecutive bytes).  A workgroup has one wave per strip
// (times 1, 2 or 4 when there are fewer than 4 strips) and walks batches of
// groups; per group a lane's partial is reduced over the 4 lanes of a DPP
// row with the same r (row_ror 4, 8), the 16-lane row sums go to LDS, and
// after one barrier per batch each row's total is summed over strips and
// rows in a fixed order, then the epilogue runs.  Every lane loads all of
// its batch's weight bytes before the first of them is used.
// ---------------------------------------------------------------------------
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <uint32_t QT>
struct StripGeom {
  static constexpr int GB = (QT == Q4_0) ? 72 : 136;  // group-block bytes
  static constexpr int QW = (QT == Q4_0) ? 4 : 8;     // quant dwords per row-block
};

template <uint32_t QT>
struct LaneW {
  uint32_t q[StripGeom<QT>::QW];
  uint32_t d;
};

// Q4_K (row-major 144-byte superblocks: fp16 d, fp16 dmin, 12 bytes of
// 6-bit scales and mins, 128 quant bytes; dequant.rs:75-124).  A lane unit
// is 32 elements of one row: the 16 quant bytes [32 j + 16 h, +16) of a
// superblock, whose low nibbles are run A (elements 64 j + 16 h + i, in
// sub-block 2 j) and high nibbles run B (32 elements later, sub-block
// 2 j + 1), with the superblock's 16-byte header.  Unit kb of a row is
// (superblock kb / 8, j = (kb / 2) % 4, h = kb % 2), so the 16 units of a
// 512-element strip cover it once, and run B sits where the second half of
// a 32-element block does for the other types.
template <>
struct LaneW<Q4K> {
  uint32_t q[4];
  uint32_t h[4];
};

// Element offset of lane unit kb's first half, and of its second half
// from there.
template <uint32_t QT>
__device__ __forceinline__ int unit_x0(int kb) {
  if (QT == Q4K) return 256 * (kb >> 3) + 64 * ((kb >> 1) & 3) + 16 * (kb & 1);
  return 32 * kb;
}
template <uint32_t QT>
constexpr int unit_hoff() {
  return QT == Q4K ? 32 : 16;
}


// Quant loads of the strip kernels: 16-byte loads (8-byte aligned) or
// 8-byte loads, nontemporal or not.  The scale load always uses the same
// cache policy as the quant loads: the two share cache lines.
#ifndef ZG_STRIP_LD16_Q8
#define ZG_STRIP_LD16_Q8 1
#endif
#ifndef ZG_STRIP_LD16_Q4
#define ZG_STRIP_LD16_Q4 0
#endif
#ifndef ZG_STRIP_NT_Q8
#define ZG_STRIP_NT_Q8 0
#endif
#ifndef ZG_STRIP_NT_Q4
#define ZG_STRIP_NT_Q4 1
#endif
typedef uint32_t u32x4a8 __attribute__((ext_vector_type(4), aligned(8)));

// load through pointer p with the nontemporal hint when NT (a macro: the
// pointee's alignment attribute must reach the load)
#define ZG_LD_POL(NT, p) ((NT) ? __builtin_nontemporal_load(p) : *(p))

// Plain (GGUF / .smodel-v1) row-major blocks: the lane's block starts at
// blk (fp16 d, then the quants): 2-byte aligned, so the quant loads use a
// 2-byte-aligned vector type (still single dwordx4 loads, unaligned access).
typedef uint32_t u32x4s2 __attribute__((ext_vector_type(4), aligned(2)));

// STREAM: nontemporal loads whatever the type's default (a decode-step LM
// head, whose cache-allocating read would evict the KV cache).
template <uint32_t QT, bool STREAM = false>
__device__ __forceinline__ void strip_load_plain(LaneW<QT>& L, const uint8_t* blk) {
  constexpr int QW = StripGeom<QT>::QW;
  constexpr bool NT = STREAM || (QT == Q8_0 ? ZG_STRIP_NT_Q8 : ZG_STRIP_NT_Q4);
  const u32x4s2* p = reinterpret_cast<const u32x4s2*>(blk + 2);
#pragma unroll
  for (int i = 0; i < QW / 4; i++) {
    const u32x4s2 v = ZG_LD_POL(NT, p + i);
    L.q[4 * i] = v.x;
    L.q[4 * i + 1] = v.y;
    L.q[4 * i + 2] = v.z;
    L.q[4 * i + 3] = v.w;
  }
  L.d = ZG_LD_POL(NT, reinterpret_cast<const uint16_t*>(blk));
}

// Tall Q4_0 launches (a batch loop, four groups per batch) read with
// cache-allocating loads: Q4_0X4 151936x2048 37.6 vs 40.2 us, 49152x2048
// 15.2 vs 15.9 us; one-batch (decode-sized) launches keep nontemporal loads
#ifndef ZG_STRIP_NT_Q4_TALL
#define ZG_STRIP_NT_Q4_TALL 0
#endif
#ifndef ZG_STRIP_LD16_Q4_TALL
#define ZG_STRIP_LD16_Q4_TALL 0
#endif
// TALL: a launch with a batch loop (four groups per batch); STREAM:
// nontemporal loads whatever the type's default (a decode-step LM head)
template <uint32_t QT, bool TALL = false, bool STREAM = false>
__device__ __forceinline__ void strip_load(LaneW<QT>& L, const uint8_t* blk, int r) {
  constexpr int QW = StripGeom<QT>::QW;
  constexpr bool LD16 = QT == Q8_0 ? ZG_STRIP_LD16_Q8 : (TALL ? ZG_STRIP_LD16_Q4_TALL : ZG_STRIP_LD16_Q4);
  constexpr bool NT = STREAM || (QT == Q8_0 ? ZG_STRIP_NT_Q8 : (TALL ? ZG_STRIP_NT_Q4_TALL : ZG_STRIP_NT_Q4));
  if (LD16) {
    // row quants start at 8 + 16r (Q4_0) or 8 + 32r (Q8_0): 8-byte aligned
    const u32x4a8* p = reinterpret_cast<const u32x4a8*>(blk + 8 + 4 * QW * r);
#pragma unroll
    for (int i = 0; i < QW / 4; i++) {
      const u32x4a8 v = ZG_LD_POL(NT, p + i);
      L.q[4 * i] = v.x;
      L.q[4 * i + 1] = v.y;
      L.q[4 * i + 2] = v.z;
      L.q[4 * i + 3] = v.w;
    }
  } else {
    const u32x2* p = reinterpret_cast<const u32x2*>(blk + 8 + 4 * QW * r);
#pragma unroll
    for (int i = 0; i < QW / 2; i++) {
      const u32x2 v = ZG_LD_POL(NT, p + i);
      L.q[2 * i] = v.x;
      L.q[2 * i + 1] = v.y;
    }
  }
  L.d = ZG_LD_POL(NT, reinterpret_cast<const uint16_t*>(blk + 2 * r));
}

// Split-scale X4 groups (the model's device layout, IL 5): a group of 4
// rows holds its nb blocks' quants first, [kb][row][QB bytes] (QB = 16 for
// Q4_0, 32 for Q8_0), then their fp16 scales, [kb][row], so a wave's 16
// blocks are 16 QB contiguous quant bytes and 128 contiguous scale bytes
// (the X4 group-block interleaves 8 scale bytes with every 4 QB quant bytes,
// so its scale loads touch ~9 cache lines per wave instruction).  q: the
// lane's quants (16-byte aligned), d: its scale.  Same cache policy as
// strip_load.
#ifndef ZG_SPLIT_LD16
#define ZG_SPLIT_LD16 1
#endif
// Tall launches over split-scale groups stream with nontemporal loads: each
// wave reads its quants and its scales as contiguous runs, every line once
// (Q4_0 151936x2048: 31.1 against 33.5 us cache-allocating); X4 group-blocks
// keep cache-allocating loads, whose three loads per lane touch each line
// again (34.8 against 32.8 us nontemporal)
#ifndef ZG_SPLIT_NT_TALL
#define ZG_SPLIT_NT_TALL 1
#endif
template <uint32_t QT, bool TALL = false>
__device__ __forceinline__ void strip_load_split(LaneW<QT>& L, const uint8_t* q, const uint8_t* d) {
  constexpr int QW = StripGeom<QT>::QW;
  constexpr bool NT = QT == Q8_0 ? ZG_STRIP_NT_Q8 : (TALL ? ZG_SPLIT_NT_TALL : ZG_STRIP_NT_Q4);
  if (ZG_SPLIT_LD16) {
    const u32x4* p = reinterpret_cast<const u32x4*>(q);
#pragma unroll
    for (int i = 0; i < QW / 4; i++) {
      const u32x4 v = ZG_LD_POL(NT, p + i);
      L.q[4 * i] = v.x;
      L.q[4 * i + 1] = v.y;
      L.q[4 * i + 2] = v.z;
      L.q[4 * i + 3] = v.w;
    }
  } else {
    const u32x2* p = reinterpret_cast<const u32x2*>(q);
#pragma unroll
    for (int i = 0; i < QW / 2; i++) {
      const u32x2 v = ZG_LD_POL(NT, p + i);
      L.q[2 * i] = v.x;
      L.q[2 * i + 1] = v.y;
    }
  }
  L.d = ZG_LD_POL(NT, reinterpret_cast<const uint16_t*>(d));
}

// Q4_K unit loads: the header and the unit's quant bytes, 16 bytes each
// (16-byte aligned).  Cache-allocating unless NT.
template <bool NT>
__device__ __forceinline__ void strip_load_q4k(LaneW<Q4K>& L, const uint8_t* sb, int jh) {
  const u32x4 h = ZG_LD_POL(NT, reinterpret_cast<const u32x4*>(sb));
  const u32x4 q = ZG_LD_POL(NT, reinterpret_cast<const u32x4*>(sb + 16 + 32 * (jh >> 1) + 16 * (jh & 1)));
  L.h[0] = h.x, L.h[1] = h.y, L.h[2] = h.z, L.h[3] = h.w;
  L.q[0] = q.x, L.q[1] = q.y, L.q[2] = q.z, L.q[3] = q.w;
}

// The block scale through the hardware fp16 conversion: exact for every
// finite value, subnormals and infinities; a NaN scale gives a NaN row
// either way (only a signalling NaN's payload would differ from
// half_bits_to_f32, and the scale only ever feeds a multiply).
__device__ __forceinline__ float scale_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}

template <uint32_t QT>
__device__ __forceinline__ float strip_dot(const LaneW<QT>& L, const float4* xb, float mterm) {
  const float d = scale_f32(L.d);
  if (QT == Q4_0) return d * (q4_block_dot(L.q, xb) + mterm);
  return d * (q8u_block_dot(L.q, xb) + mterm);
}

// The same block against the activations as exact integers (XDig): the
// three digit chains of sum_j q_j V_j with v_dot4_i32_i8, then one scale
// d * M / (127 * 2^14).  Q4_0: the nibbles n enter as they are and the
// chains start at -8 * sum_j V_j, so the block's integer sum is
// sum_j (n_j - 8) V_j, |.| <= 32 * 8 * 127 * 2^14 + ... < 2^31, recombined
// in int32.  Q8_0: quants up to 128 in magnitude, so the top digit's chain
// joins the other two in float (one rounding).
template <uint32_t QT>
__device__ __forceinline__ float strip_dot_dig(const LaneW<QT>& L, const XDig& X) {
  const float ds = scale_f32(L.d) * X.sinv;
  if constexpr (QT == Q4_0) {
    uint32_t q[8];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      q[c] = L.q[c] & 0x0F0F0F0Fu;
      q[4 + c] = (L.q[c] >> 4) & 0x0F0F0F0Fu;
    }
    int t0 = -8 * X.sum[0], t1 = -8 * X.sum[1], t2 = -8 * X.sum[2];
    xdig_chains(q, X, t0, t1, t2);
    return (float)((t0 << 14) + (t1 << 7) + t2) * ds;
  } else {
    int t0 = 0, t1 = 0, t2 = 0;
    xdig_chains(L.q, X, t0, t1, t2);
    return fmaf((float)t0, 16384.0f, (float)((t1 << 7) + t2)) * ds;
  }
}

// The same block with a Q8_0 activation block (int8 x8, fp16 scale dx,
// sx = sum of x8): the integer dot (v_dot4_i32_i8; Q4_0 nibbles enter
// unsigned and the -8 offset is -8 sx), then (dW dX) * isum, the per-block
// term of zo_gemm_q8act.
template <uint32_t QT>
__device__ __forceinline__ float strip_dot_q8x(const LaneW<QT>& L, const uint32_t* x8, float dx, int sx) {
  // four independent chains (a dependent v_dot4_i32_i8 issues ~16 cycles
  // after its predecessor); integer sums, so the order is free
  int s4[4] = {0, 0, 0, 0};
  if (QT == Q4_0) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      s4[(c & 1) * 2] = __builtin_amdgcn_sdot4((int)(L.q[c] & 0x0F0F0F0Fu), (int)x8[c], s4[(c & 1) * 2], false);
      s4[(c & 1) * 2 + 1] =
          __builtin_amdgcn_sdot4((int)((L.q[c] >> 4) & 0x0F0F0F0Fu), (int)x8[4 + c], s4[(c & 1) * 2 + 1], false);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 8; c++) s4[c & 3] = __builtin_amdgcn_sdot4((int)L.q[c], (int)x8[c], s4[c & 3], false);
  }
  int isum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  if (QT == Q4_0) isum -= 8 * sx;
  return (half_bits_to_f32(L.d) * dx) * (float)isum;
}

// Q4_K unit with fp32 activations, kq_dot's arithmetic: run A = xb[0..3],
// run B = xb[4..7], sa and sb their sums; j the unit's sub-block pair.
__device__ __forceinline__ float strip_dot_q4k(const LaneW<Q4K>& L, const float4* xb, float sa, float sb, int j) {
  const float d = kq_half(L.h[0]), dmin = kq_half(L.h[0] >> 16);
  uint32_t iA, iB, nA, nB;
  q4k_lane_scales(L.h[1], L.h[2], L.h[3], j, iA, iB, nA, nB);
  // high nibbles stay in place (16 x the value): the 1/16 goes into the
  // sub-block scale (exact).  (Converting the nibbles as fp8 bytes, as the
  // Q4_0 blocks do, needs a shift for the high nibbles here and measured
  // slower: 14336x4096 11.15-11.20 against 11.04-11.14 us.)
  uint32_t lo[4], hi[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    lo[c] = opaque_u32(L.q[c] & 0x0F0F0F0Fu);
    hi[c] = opaque_u32(L.q[c] & 0xF0F0F0F0u);
  }
  const float sA = u8_dot16(lo, xb);
  const float sB = u8_dot16(hi, xb + 4);
  float acc = (d * (float)iA) * sA;
  acc = fmaf(-(dmin * (float)nA), sa, acc);
  acc = fmaf((d * 0.0625f) * (float)iB, sB, acc);
  return fmaf(-(dmin * (float)nB), sb, acc);
}

// The same unit against integer-digit activations (XDig of the unit's 32
// values, run A first): per run the three digit chains of sum_i q_i V_i
// (|.| <= 16 * 15 * 127 * 2^14 < 2^31, recombined in int32), then
// d * M / (127 * 2^14) times the scaled run sums, minus the min terms on
// the fp32 run sums.
__device__ __forceinline__ float strip_dot_dig_q4k(const LaneW<Q4K>& L, const XDig& X, float sa, float sb, int j) {
  const float d = kq_half(L.h[0]), dmin = kq_half(L.h[0] >> 16);
  uint32_t iA, iB, nA, nB;
  q4k_lane_scales(L.h[1], L.h[2], L.h[3], j, iA, iB, nA, nB);
  int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const int lo = (int)(L.q[c] & 0x0F0F0F0Fu), hi = (int)((L.q[c] >> 4) & 0x0F0F0F0Fu);
    a0 = __builtin_amdgcn_sdot4(lo, (int)X.dg[0][c], a0, false);
    a1 = __builtin_amdgcn_sdot4(lo, (int)X.dg[1][c], a1, false);
    a2 = __builtin_amdgcn_sdot4(lo, (int)X.dg[2][c], a2, false);
    b0 = __builtin_amdgcn_sdot4(hi, (int)X.dg[0][4 + c], b0, false);
    b1 = __builtin_amdgcn_sdot4(hi, (int)X.dg[1][4 + c], b1, false);
    b2 = __builtin_amdgcn_sdot4(hi, (int)X.dg[2][4 + c], b2, false);
  }
  const float IA = (float)((a0 << 14) + (a1 << 7) + a2), IB = (float)((b0 << 14) + (b1 << 7) + b2);
  const float acc = fmaf((float)iA, IA, (float)iB * IB) * (d * X.sinv);
  return fmaf(-dmin, fmaf((float)nA, sa, (float)nB * sb), acc);
}

// partial sums over the 4 lanes of each DPP row that share lane & 3
// (lane l of a row holds block l >> 2; row_ror:n reads lane l - n mod 16):
// lane l < 4 ends with (P0 + P3) + (P2 + P1) over that row's blocks P0..P3.
// The compiler contracts the first add with the block product into an fma,
// so the lane's own term enters unrounded: fma(P0) + P3, fma(P2) + P1.
__device__ __forceinline__ float row_sum4(float v) {
  v += dpp_f32<0x124>(v);  // row_ror:4
  v += dpp_f32<0x128>(v);  // row_ror:8
  return v;
}

// Broadcast of lane S of every quad (DPP quad_perm [S,S,S,S]).
template <int S>
__device__ __forceinline__ float quad_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), S | (S << 2) | (S << 4) | (S << 6), 0xF, 0xF, false));
}
template <int S>
__device__ __forceinline__ float4 quad_bcast4(float4 v) {
  return make_float4(quad_bcast<S>(v.x), quad_bcast<S>(v.y), quad_bcast<S>(v.z), quad_bcast<S>(v.w));
}

// The four lanes of a quad (the four rows of one K-block) each hold a
// quarter of the block's 32 activations: lo = x[4r .. 4r+4), hi =
// x[16+4r .. 16+4r+4) for quad lane r.  Every lane gets the whole block,
// xb[c] = lane c's lo and xb[4+c] = lane c's hi, with 32 DPP moves instead
// of four redundant 128-byte loads per block.
__device__ __forceinline__ void quad_gather_block(float4 lo, float4 hi, float4 (&xb)[8]) {
  xb[0] = quad_bcast4<0>(lo);
  xb[1] = quad_bcast4<1>(lo);
  xb[2] = quad_bcast4<2>(lo);
  xb[3] = quad_bcast4<3>(lo);
  xb[4] = quad_bcast4<0>(hi);
  xb[5] = quad_bcast4<1>(hi);
  xb[6] = quad_bcast4<2>(hi);
  xb[7] = quad_bcast4<3>(hi);
}

// Sum over a quad: every lane gets ((a + b) + (c + d)), bitwise the same
// in all four lanes.
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp_f32<0xB1>(v);  // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);  // quad_perm [2,3,0,1]
  return v;
}

// The 32 activations of K-block kb as the prologue forms them: from x, times
// the rmsnorm gain (the 1/rms factor is applied to the row totals).
// (Q4_K: the unit's runs A and B, as xf[0..3] and xf[4..7].)
template <int PRO, uint32_t QT = Q4_0>
__device__ __forceinline__ void strip_x_block(float4 (&xf)[8], const GemvArgs& a, int kb) {
  constexpr int H4 = unit_hoff<QT>() / 4;
  const int x0 = unit_x0<QT>(kb);
  const float4* x4 = reinterpret_cast<const float4*>(a.x + x0);
#pragma unroll
  for (int c = 0; c < 8; c++) xf[c] = x4[c < 4 ? c : c - 4 + H4];
  if (PRO == PRO_RMSNORM) {
    const float4* g4 = reinterpret_cast<const float4*>(a.norm_w + x0);
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const float4 g = g4[c < 4 ? c : c - 4 + H4];
      xf[c] = make_float4(xf[c].x * g.x, xf[c].y * g.y, xf[c].z * g.z, xf[c].w * g.w);
    }
  }
}

__device__ __forceinline__ float f4_sum(float4 v) { return (v.x + v.y) + (v.z + v.w); }

// IL 4: X4 group-blocks (IL 3: the same with nontemporal loads); IL 5:
// split-scale X4 groups (strip_load_split); IL 1: plain row-major blocks
// (IL 2: the same with nontemporal loads), a "group" being 4
// consecutive rows (lane (b, r) reads block b of row 4 g + r, b = lane >> 2,
// r = lane & 3 in either layout, so both give the same bits).  A plain
// mapping with 16 lanes per row (b = lane & 15, r = lane >> 4: one row's 16
// blocks contiguous per 16 lanes) measured slower: 5.80 vs 5.22 us at
// 6144x2048.
// ONEB: the grid is the batch count (every workgroup runs exactly one
// batch), so there is no second register set and no batch loop.
// SC: the strip count as a compile-time constant (0: the argument S_rt),
// for the common one-batch shapes (in_dim 2048 and 6144).
// DIG: fp32 activations as exact integers (XDig) and int8 dot chains; a
// wave with a block that the integer form does not take (NaN, infinity, a
// largest magnitude below 1e-30) runs the fp32 decode instead.
template <uint32_t QT, int PRO, int EPI, int GBATCH, int MAXT = 1024, bool SEG1 = false, int IL = 4,
          bool ONEB = false, int SC = 0, bool DIG = false, bool SIG = false>
__device__ __forceinline__ void gemv_strip_body(const GemvArgs& a, int S_rt, int bid, int nblk) {
  static_assert(!DIG || PRO != PRO_Q8X, "Q8_0 activations have their own integer form");
  static_assert(QT != Q4K || ((IL == 1 || IL == 2) && PRO != PRO_Q8X), "Q4_K: row-major superblocks, fp32 x");
  static_assert(!SIG || EPI == EPI_STORE, "tagged stores replace plain stores");
  const int S = SC ? SC : S_rt;
  constexpr int GBY = StripGeom<QT>::GB;
  constexpr int BB = QT == Q4_0 ? 18 : 34;  // plain block bytes
  constexpr int PARTS = (EPI == EPI_SWIGLU) ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) float part[];  // [2][NW][GBATCH][PARTS][16]
  __shared__ float red[16];
  // S >= 3 strips: one wave per strip; S in {1, 2}: four waves, 4 / S per
  // strip (the launch's block size; no integer division on the way to the
  // first load)
  const int WPS = S >= 3 ? 1 : (S == 2 ? 2 : 4);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = S >= 3 ? wave : (S == 2 ? (wave & 1) : 0);
  const int sub = S >= 3 ? 0 : (S == 2 ? (wave >> 1) : wave);
  const int NW = S >= 3 ? S : 4;
  const int b = lane >> 2, r = lane & 3;
  const int nb = a.k >> 5;
  const int kb = strip * 16 + b;  // this lane's K-block
  const int items = (int)(EPI == EPI_SWIGLU ? a.total_groups / 2 : a.total_groups);
  const int per_batch = WPS * GBATCH;
  const int nbatch = (items + per_batch - 1) / per_batch;

  // SEG1: a single projection (g_begin 0), no per-item segment search
  auto locate = [&](int item, int p, uint32_t& lg) -> GemvSeg {
    if (EPI == EPI_SWIGLU) {
      lg = (uint32_t)item;
      return p ? a.seg[1] : a.seg[0];
    }
    if (SEG1) {
      lg = (uint32_t)item;
      return a.seg[0];
    }
    const GemvSeg sg = seg_of(a, (uint32_t)item);
    lg = (uint32_t)item - sg.g_begin;
    return sg;
  };

  // unconditional loads (items past the end are clamped to the last one
  // and their results dropped), so the compiler's wait counts stay exact
  // and a batch's loads stay in flight while the previous batch is used
  auto load_batch = [&](LaneW<QT> (&L)[GBATCH][PARTS], int batch) {
    const int base = batch * per_batch + sub * GBATCH;
#pragma unroll
    for (int j = 0; j < GBATCH; j++) {
#pragma unroll
      for (int p = 0; p < PARTS; p++) {
        uint32_t lg;
        const GemvSeg sg = locate(min(base + j, items - 1), p, lg);
        // the group's start is wave-uniform (scalar registers), the lane's
        // byte offset inside it a 32-bit vector offset
        if constexpr (QT == Q4K)
          // row 4 lg + r, superblock kb / 8 (rows of nb / 8 superblocks)
          strip_load_q4k<IL == 2>(L[j][p], sg.w + (size_t)(4 * lg + (uint32_t)r) * (size_t)(nb * 18) +
                                               (uint32_t)((kb >> 3) * 144),
                                  kb & 7);
        else if constexpr (IL == 4 || IL == 3)
          strip_load<QT, GBATCH == 4, IL == 3>(L[j][p], sg.w + (size_t)lg * (size_t)(nb * GBY) + (uint32_t)(kb * GBY),
                                               r);
        else if constexpr (IL == 5) {
          constexpr int QB = 4 * StripGeom<QT>::QW;  // quant bytes per row and block
          const uint8_t* gp = sg.w + (size_t)lg * (size_t)(nb * GBY);
          strip_load_split<QT, GBATCH == 4>(L[j][p], gp + (uint32_t)((4 * kb + r) * QB),
                                            gp + (uint32_t)(nb * 4 * QB + 2 * (4 * kb + r)));
        }
        else
          strip_load_plain<QT, IL == 2>(L[j][p], sg.w + (size_t)lg * (size_t)(4 * nb * BB) +
                                                     (uint32_t)((r * nb + kb) * BB));
      }
    }
  };

  // activation block of this lane, then the first batch's weights: all
  // loads are issued before any of them is waited for, x first because it
  // is consumed first
  float4 xb[8], gw[8];
  uint32_t x8[8];  // PRO_Q8X: the lane's Q8_0 activation block
  float dxq = 0.0f;
  AttnSplitIn am;
  if (PRO == PRO_ATTN) {
    // the attention splits' values at this lane's two quarters of its
    // x-block (one head: the head dim is a multiple of the unit's span)
    const int x0 = unit_x0<QT>(kb) + 4 * r;
    attn_split_load2(am, a.x, a.attn_ml, a.k, a.attn_hd, a.attn_nsplit, x0, x0 + unit_hoff<QT>());
  } else if (PRO == PRO_Q8X) {
    const uint8_t* xbk = a.xq + (size_t)kb * 34;
    const u32x4s2* p = reinterpret_cast<const u32x4s2*>(xbk + 2);
    const u32x4s2 v0 = p[0], v1 = p[1];
    x8[0] = v0.x, x8[1] = v0.y, x8[2] = v0.z, x8[3] = v0.w;
    x8[4] = v1.x, x8[5] = v1.y, x8[6] = v1.z, x8[7] = v1.w;
    dxq = half_bits_to_f32(*reinterpret_cast<const uint16_t*>(xbk));
  } else {
    // this lane's quarter of the x-block (and of the rmsnorm gain, loaded
    // with x ahead of the barrier that waits for the sum of squares); the
    // quad shares its quarters through DPP below
    constexpr int H4 = unit_hoff<QT>() / 4;
    const float4* x4 = reinterpret_cast<const float4*>(a.x + unit_x0<QT>(kb));
    xb[0] = x4[r];
    xb[1] = x4[H4 + r];
    if (PRO == PRO_RMSNORM) {
      const float4* g4 = reinterpret_cast<const float4*>(a.norm_w + unit_x0<QT>(kb));
      gw[0] = g4[r];
      gw[1] = g4[H4 + r];
    }
  }
  // two batches in flight: this workgroup's first and second
  // The grid never exceeds the batch count, so the first batch exists and
  // its loads are unconditional: the prologue's wait for x can then leave
  // them in flight.  The second batch is issued after the prologue (a
  // conditional load ahead of the prologue would make the compiler wait for
  // every outstanding load before it uses x).
  LaneW<QT> LA[GBATCH][PARTS], LB[GBATCH][PARTS];
  const int b0 = bid, bstep = nblk;
  const uint32_t sig_tag = SIG ? *a.sync_epoch * a.sync_mul + a.sync_add : 0u;  // this step and layer's tag
  const bool sig_drop = SIG && a.sync_drop && *a.sync_drop == a.sync_add + 1;
  load_batch(LA, b0);

  // prologue and block sum
  if (PRO == PRO_ATTN) {
    // each lane merges the splits at its own quarters while the weight
    // loads are in flight (no LDS staging, no workgroup barrier: the O
    // projection 2048x2048 in a probe, 3.24 us with the workgroup merging the
    // whole vector into LDS, 2.58 us on a plain x)
    attn_split_merge(am, a.attn_nsplit, xb[0], xb[1]);
  }
  if (PRO == PRO_RMSNORM) {
    // ops.rs:29-52: x * (1/sqrt(mean(x^2)+eps)) * w.  The scalar
    // 1/sqrt(...) factors out of every row's dot product, so the decode runs
    // on x * w and the row totals are scaled in the epilogue: the sum of
    // squares (the first wave of each strip: its 64 lanes hold the strip's
    // 512 values once) goes to LDS here and is read after the batch's
    // barrier, off the path between the loads and the decode
    float ssq = 0.0f;
    if (sub == 0) {
#pragma unroll
      for (int c = 0; c < 2; c++) ssq += xb[c].x * xb[c].x + xb[c].y * xb[c].y + xb[c].z * xb[c].z + xb[c].w * xb[c].w;
    }
    ssq = wave_sum(ssq);
    if (lane == 0) red[wave] = ssq;
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const float4 g = gw[c];
      xb[c].x = xb[c].x * g.x;
      xb[c].y = xb[c].y * g.y;
      xb[c].z = xb[c].z * g.z;
      xb[c].w = xb[c].w * g.w;
    }
  }
  float mterm = 0.0f;
  float xsa = 0.0f, xsb = 0.0f;  // Q4_K: the unit's run sums
  int sx = 0;
  XDig xd;
  bool fp32 = !DIG;  // wave-uniform: this wave decodes with fp32 activations
  if (QT == Q4K) {
    // the quad's quarter sums: run A from the lo quarters, run B from the hi ones
    xsa = quad_sum(f4_sum(xb[0]));
    xsb = quad_sum(f4_sum(xb[1]));
  }
  if (DIG) {
    const bool bad = xdig_quad(xb[0], xb[1], xd);
    fp32 = __builtin_amdgcn_ballot_w64(bad) != 0;
    asm volatile("" : "+v"(xd.sum[0]), "+v"(xd.sum[1]), "+v"(xd.sum[2]), "+v"(xd.sinv));
  }
  if (PRO == PRO_Q8X) {
#pragma unroll
    for (int c = 0; c < 8; c++) sx = __builtin_amdgcn_sdot4((int)x8[c], 0x01010101, sx, false);
    asm volatile("" : "+v"(sx));  // computed here, not sunk below the next load
  } else if (!DIG) {
    // the quad's four quarters: block sum, then the whole block in every lane
    const float t =
        quad_sum(((xb[0].x + xb[0].y) + (xb[0].z + xb[0].w)) + ((xb[1].x + xb[1].y) + (xb[1].z + xb[1].w)));
    const float4 lo = xb[0], hi = xb[1];
    quad_gather_block(lo, hi, xb);
    mterm = (QT == Q4_0 ? -8.0f : -128.0f) * t;
    asm volatile("" : "+v"(mterm));  // computed here, not sunk below the next load
  }
  if (!ONEB && b0 + bstep < nbatch) load_batch(LB, b0 + bstep);

  uint64_t key = 0;
  // one batch: partials -> LDS, barrier, per-row totals over strips and
  // DPP rows in a fixed order, epilogue
  auto process = [&](const LaneW<QT> (&L)[GBATCH][PARTS], int batch, int buf) {
    const int base = batch * per_batch + sub * GBATCH;
    float* pb = part + (size_t)buf * NW * GBATCH * PARTS * 16;
    // a single projection's stored row range, in scalar registers before
    // the decode rather than loaded after the barrier, on the way to the
    // stores
    if constexpr (SEG1 && EPI != EPI_SWIGLU) asm volatile("" ::"s"(a.seg[0].row_lo), "s"(a.seg[0].row_hi));
    // in batch-loop launches (and single-projection ones) every group of the
    // batch is decoded, also the clamped repeats past the last item (their
    // totals are dropped in the epilogue): a skipped decode leaves its loads
    // unconsumed, and the compiler then waits for the other batch's loads
    // before it reuses their registers (C1 6144x2048: 3.53 vs 3.63 us; the
    // fused Q|K|V one-batch launch keeps the skip: 3.99 vs 4.20 us)
#pragma unroll
    for (int j = 0; j < GBATCH; j++) {
      if (SEG1 || !ONEB || base + j < items) {
#pragma unroll
        for (int p = 0; p < PARTS; p++) {
          float dot;
          if constexpr (QT == Q4K) {
            const int pj = (kb >> 1) & 3;
            if (!DIG) {
              dot = strip_dot_q4k(L[j][p], xb, xsa, xsb, pj);
            } else if (!fp32) {
              dot = strip_dot_dig_q4k(L[j][p], xd, xsa, xsb, pj);
            } else {
              float4 xf[8];
              if constexpr (PRO == PRO_ATTN) quad_gather_block(xb[0], xb[1], xf);  // the merged quarters
              else strip_x_block<PRO, QT>(xf, a, kb);
              const float fa = (f4_sum(xf[0]) + f4_sum(xf[1])) + (f4_sum(xf[2]) + f4_sum(xf[3]));
              const float fb = (f4_sum(xf[4]) + f4_sum(xf[5])) + (f4_sum(xf[6]) + f4_sum(xf[7]));
              dot = strip_dot_q4k(L[j][p], xf, fa, fb, pj);
            }
          } else if (PRO == PRO_Q8X) {
            dot = strip_dot_q8x<QT>(L[j][p], x8, dxq, sx);
          } else if (!DIG) {
            dot = strip_dot<QT>(L[j][p], xb, mterm);
          } else if (!fp32) {
            dot = strip_dot_dig<QT>(L[j][p], xd);
          } else {
            // the fp32 decode on the lane's whole block, reloaded per group
            // (a wave that met a block the integer form does not take)
            float4 xf[8];
            if constexpr (PRO == PRO_ATTN) quad_gather_block(xb[0], xb[1], xf);  // the merged quarters
            else strip_x_block<PRO>(xf, a, kb);
            float t = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; c++) t += (xf[c].x + xf[c].y) + (xf[c].z + xf[c].w);
            dot = strip_dot<QT>(L[j][p], xf, (QT == Q4_0 ? -8.0f : -128.0f) * t);
          }
          const float v = row_sum4(dot);
          // [wave][group][part][r][DPP row]: a row's four DPP-row sums
          // are one 16-byte LDS read below
          if ((lane & 15) < 4) pb[((wave * GBATCH + j) * PARTS + p) * 16 + r * 4 + (lane >> 4)] = v;
        }
      }
    }
    __syncthreads();
    const int tt = threadIdx.x;
    if (tt < per_batch * 4) {
      const int su = tt / (GBATCH * 4), j = (tt >> 2) % GBATCH, rr = tt & 3;
      const int item = batch * per_batch + su * GBATCH + j;
      if (item < items) {
        float rinv = 1.0f;
        if (PRO == PRO_RMSNORM) {
          float ss = 0.0f;
          for (int i = 0; i < S; i++) ss += red[i];
          rinv = 1.0f / sqrtf(ss / (float)a.k + a.eps);
        }
        float tot[PARTS];
#pragma unroll
        for (int p = 0; p < PARTS; p++) {
          float acc = 0.0f;
          for (int st = 0; st < S; st++) {
            const float4 q = *reinterpret_cast<const float4*>(pb + (((su * S + st) * GBATCH + j) * PARTS + p) * 16 + 4 * rr);
            acc += (q.x + q.y) + (q.z + q.w);
          }
          tot[p] = PRO == PRO_RMSNORM ? acc * rinv : acc;
        }
        uint32_t lg;
        const GemvSeg sg = locate(item, 0, lg);
        const uint32_t row = 4 * lg + (uint32_t)rr;
        if (row >= sg.row_lo && row < sg.row_hi) {
          const float v = tot[PARTS - 1];
          if (EPI == EPI_SWIGLU) {
            const float g = tot[0];
            // activation.rs:115-148 operand order: silu = g/(1+exp(-g)), then *up
            store_out(a.seg[0].y + row, (g / (1.0f + expf(-g))) * v);
          } else if (EPI == EPI_RESID) {
            store_out(sg.y + row, sg.resid[row] + v);
          } else if (SIG) {
            // read by other workgroups of this launch: the value with this
            // step and layer's tag, as one agent-scope 64-bit store (the
            // reader takes a row once it carries that tag)
            const uint64_t tw = ((uint64_t)sig_tag << 32) | (uint64_t)__float_as_uint(v);
            if (!sig_drop)
              __hip_atomic_store(reinterpret_cast<uint64_t*>(sg.y) + row, tw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          } else {
            if (sg.y) store_out(sg.y + row, v);
            if (EPI == EPI_ARGMAX && !(v != v)) {
              const uint64_t kk = argmax_key(v, row);
              key = kk > key ? kk : key;
            }
          }
        }
      }
    }
  };
  if (ONEB) {
    process(LA, b0, 0);
  } else {
    // batches b0, b0 + bstep, ... alternate between the two register sets;
    // a set is refilled with the batch two steps ahead as soon as it is used
    for (int batch = b0; batch < nbatch; batch += 2 * bstep) {
      process(LA, batch, 0);
      if (batch + 2 * bstep < nbatch) load_batch(LA, batch + 2 * bstep);
      if (batch + bstep < nbatch) {
        process(LB, batch + bstep, 1);
        if (batch + 3 * bstep < nbatch) load_batch(LB, batch + 3 * bstep);
      }
    }
  }
  if (EPI == EPI_ARGMAX) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t other = __shfl_xor(key, o, 64);
      key = other > key ? other : key;
    }
    if (lane == 0 && key) atomicMax(reinterpret_cast<unsigned long long*>(a.best), (unsigned long long)key);
  }
  if (PRO == PRO_RMSNORM && a.xn_out && bid == 0 && sub == 0) {
    // the normalized x for other consumers: (x * gain) * (1 / rms), the
    // sums of squares having crossed the batch barrier; the quarters of the
    // first strip set's lanes cover every element once
    float ss = 0.0f;
    for (int i = 0; i < S; i++) ss += red[i];
    const float rinv = 1.0f / sqrtf(ss / (float)a.k + a.eps);
    constexpr int H4 = unit_hoff<QT>() / 4;
    const int x0 = unit_x0<QT>(kb);
    const float4* x4 = reinterpret_cast<const float4*>(a.x + x0);
    const float4* g4 = reinterpret_cast<const float4*>(a.norm_w + x0);
    float4* o4 = reinterpret_cast<float4*>(a.xn_out + x0);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int i = h ? H4 + r : r;
      const float4 v = x4[i], g = g4[i];
      o4[i] = make_float4((v.x * g.x) * rinv, (v.y * g.y) * rinv, (v.z * g.z) * rinv, (v.w * g.w) * rinv);
    }
  }
}

template <uint32_t QT, int PRO, int EPI, int GBATCH, int MAXT = 1024, bool SEG1 = false, int IL = 4,
          bool ONEB = false, int SC = 0, bool DIG = false>
__global__ __launch_bounds__(MAXT) void gemv_strip_kernel(GemvArgs a, int S_rt) {
  gemv_strip_body<QT, PRO, EPI, GBATCH, MAXT, SEG1, IL, ONEB, SC, DIG>(a, S_rt, blockIdx.x, gridDim.x);
}

}  // namespace zg
