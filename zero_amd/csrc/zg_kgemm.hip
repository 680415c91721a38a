// zg_kgemm.hip -- batched-prefill GEMM for K-quant weights (Q4_K, Q6_K) on
// Q8_K activations, int8 MFMA, for gfx950.
//
// No reference counterpart as a GEMM: the reference prefills token by token
// (kernel/src/inference.rs:1188-1330).  Per output row it computes the
// reference's integer Q4_K x Q8_K dot (linear_q4k_vnni_range,
// kernel/src/arch/x86_64/math/vnni.rs:258-476): per superblock b,
//   int_sum = sum_g sc_g * sum_{i in sub-block g} nibble_i * q8_i   (exact)
//   min_sum = sum_g m_g * (bsum[2g] + bsum[2g+1])                  (exact)
//   dot = dot + (d_w * d8) * (float)int_sum
//   min = min + (dmin_w * d8) * (float)min_sum,   y = dot - min,
// the f32 operations in that order, so every output equals the per-row
// restatement bit for bit.  Q6_K takes the same construction on its layout
// (dequant.rs:328-355; the reference's integer path has no Q6_K form):
//   int_sum = sum_g sc_g * sum_{i in g} (q6_i - 32) * q8_i over the 16
//   sub-blocks of 16, y = y + (d_w * d8) * (float)int_sum.
//
// MFMA form.  A weight element times its sub-block scale fits 13 bits
// (Q4_K: nibble * sc <= 945; Q6_K: (q6 - 32) * sc in [-4096, 4064]), so it is
// split into two int8 digits, w*sc = 128 hi + lo with lo in [0, 127].  Two
// v_mfma_i32_16x16x64_i8 chains (one per digit) then accumulate a
// superblock's whole integer sum, all its sub-blocks, in int32 (|sum| <
// 256 * 4096 * 128 = 2^27), and int_sum = 128 hi_acc + lo_acc exactly.  The
// Q4_K min term is one more pair of MFMAs per superblock: the activation's
// 32-value sums (|s| <= 4096) split the same way against the 8 mins.  The
// float work is then once per output and superblock, not per sub-block.
//
// Tiles: 64 x 64 outputs per 256-thread workgroup (2 x 2 waves of 32 x 32),
// K staged 128 values (half a superblock) at a time, double-buffered in LDS;
// the next stage's global loads are issued before the current stage is
// multiplied.  The weight digits are formed once per workgroup when a stage
// is written to LDS (packed 16-bit multiplies, two elements per operation).
#include <hip/hip_runtime.h>

#include "../../include/zero_gpu.h"
#include "zg_device.h"
#include "zg_internal.h"
#include "zg_kernels.h"

using namespace zg;

namespace zg {

constexpr int kKgBM = 64, kKgBN = 64;  // workgroup tile
constexpr int kKgKS = 128;             // K per stage
constexpr int kKgRP = kKgKS + 16;      // LDS row pitch (bytes)
constexpr int kKgSegs = 3;             // weight segments per launch (Q|K|V)
#ifndef ZG_KG_PD
#define ZG_KG_PD 2
#endif
constexpr int kKgPD = ZG_KG_PD;        // stages in flight
#ifndef ZG_KG_WPE
#define ZG_KG_WPE 1
#endif
#ifndef ZG_KG_GROUPS
#define ZG_KG_GROUPS 2
#endif

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4a2 __attribute__((ext_vector_type(4), aligned(2)));

// ---------------------------------------------------------------------------
// Q8_K activations as split arrays (qs[row][k] int8, d8[row][k/256] f32,
// bs32[row][k/32] int16: the sums of 32 quants, bsum[2g] + bsum[2g+1] of the
// reference's block).  One wave per 256-value block, q8k_block_lane's
// arithmetic, so the values are the reference quantizer's.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void quantize_q8k_split_kernel(const float* __restrict__ x, int8_t* __restrict__ qs,
                                                                float* __restrict__ d8, int16_t* __restrict__ bs32,
                                                                int k) {
  const int nsb = k / 256;
  const size_t row = blockIdx.x / nsb;
  const int sb = blockIdx.x % nsb, lane = threadIdx.x;
  const float* v = x + row * k + (size_t)sb * 256;
  const float4 f = reinterpret_cast<const float4*>(v)[lane];
  const float e[4] = {f.x, f.y, f.z, f.w};
  q8k_split_store(lane, e, qs + row * k + (size_t)sb * 256, d8 + row * nsb + sb, bs32 + row * (k / 32) + (size_t)sb * 8);
}

// ---------------------------------------------------------------------------
// Weight digits.
// ---------------------------------------------------------------------------

// get_scale_min_k4 (dequant.rs:75-85) for sub-block g from the Q4_K header's
// scale words (w1 = scale bytes 0..3, w2 = 4..7, w3 = 8..11).
__device__ __forceinline__ void kg_scale_min(uint32_t w1, uint32_t w2, uint32_t w3, int g, int& sc, int& m) {
  const int sh = 8 * (g & 3);
  const int b1 = (int)((w1 >> sh) & 0xFFu), b2 = (int)((w2 >> sh) & 0xFFu), b3 = (int)((w3 >> sh) & 0xFFu);
  if (g < 4) {
    sc = b1 & 63;
    m = b2 & 63;
  } else {
    sc = (b3 & 0xF) | ((b1 >> 6) << 4);
    m = (b3 >> 4) | ((b2 >> 6) << 4);
  }
}

// Four unsigned weight values (one per byte of v, each < 16) times sc
// (0..63): the digits lo = p & 127, hi = p >> 7 as packed bytes.
__device__ __forceinline__ void digits_u4(uint32_t v, uint32_t sc2, uint32_t& lo, uint32_t& hi) {
  const u16x2 p0 = __builtin_bit_cast(u16x2, v & 0x000F000Fu) * __builtin_bit_cast(u16x2, sc2);
  const u16x2 p1 = __builtin_bit_cast(u16x2, (v >> 8) & 0x000F000Fu) * __builtin_bit_cast(u16x2, sc2);
  const uint32_t q0 = __builtin_bit_cast(uint32_t, p0), q1 = __builtin_bit_cast(uint32_t, p1);
  lo = (q0 & 0x007F007Fu) | ((q1 & 0x007F007Fu) << 8);
  hi = __builtin_bit_cast(uint32_t, p0 >> (unsigned short)7) | (__builtin_bit_cast(uint32_t, p1 >> (unsigned short)7) << 8);
}

// Four Q6_K values (one per byte of v, each < 64) minus 32, times the signed
// scale sc: lo = p & 127, hi = p >> 7 (arithmetic, in [-32, 31]) as bytes.
__device__ __forceinline__ void digits_q6(uint32_t v, uint32_t sc2, uint32_t& lo, uint32_t& hi) {
  const s16x2 off = {32, 32};
  const s16x2 e0 = __builtin_bit_cast(s16x2, v & 0x00FF00FFu) - off;
  const s16x2 e1 = __builtin_bit_cast(s16x2, (v >> 8) & 0x00FF00FFu) - off;
  const s16x2 p0 = e0 * __builtin_bit_cast(s16x2, sc2), p1 = e1 * __builtin_bit_cast(s16x2, sc2);
  const uint32_t q0 = __builtin_bit_cast(uint32_t, p0), q1 = __builtin_bit_cast(uint32_t, p1);
  lo = (q0 & 0x007F007Fu) | ((q1 & 0x007F007Fu) << 8);
  const uint32_t h0 = __builtin_bit_cast(uint32_t, p0 >> (short)7), h1 = __builtin_bit_cast(uint32_t, p1 >> (short)7);
  hi = (h0 & 0x00FF00FFu) | ((h1 & 0x00FF00FFu) << 8);
}

struct KgemmArgs {
  const int8_t* qs;     // [m][k]
  const float* d8;      // [m][k/256]
  const int16_t* bs32;  // [m][k/32]
  const uint8_t* w[kKgSegs];
  float* y[kKgSegs];
  int seg_end[kKgSegs];  // cumulative columns (multiples of 64)
  int nseg;
  int accumulate;  // y += product (residual adds)
  int m, n, k;
};

// Per-thread staging registers of one stage.
template <uint32_t WT>
struct KgStage;
template <>
struct KgStage<Q4K> {
  u32x4 a[2];   // 32 bytes of the A tile
  u32x4 q, h;   // 16 quant bytes and the 16-byte superblock header
  uint32_t bs;  // two 32-value sums of one row (int16 pair) of the stage's superblock
  float d8;     // d8 of row tid % 64 for the stage's superblock
};
template <>
struct KgStage<Q6K> {
  u32x4 a[2];
  u32x4 l0, l1, h0, h1;  // 32 ql bytes, 32 qh bytes
  uint32_t sc;           // the two scale bytes of the lane's quarter (low 16 bits)
  uint32_t d;            // fp16 d
  float d8;
};

// PD: stages whose global loads are in flight while a stage is multiplied
// (a ring of PD register stages; the stage count is a multiple of PD, so
// every load is unconditional and the wait counts stay exact).
// G: groups of four waves per workgroup that share the tile's superblocks,
// group g taking superblocks g, g + G, ... (launches with few tiles: one
// workgroup per CU walks its K range G times as fast).  The integer sums are
// exact in any split; the float terms still enter each output in superblock
// order: group g > 0 hands its superblock's two products to group 0 through
// LDS, and group 0 adds its own, then group 1's, ...
template <uint32_t WT, int PD, int G>
__global__ __launch_bounds__(256 * G) __attribute__((amdgpu_waves_per_eu(ZG_KG_WPE))) void gemm_q8k_kernel(KgemmArgs a) {
  // the reference rounds every product and sum of the superblock terms on
  // its own: no fused multiply-add in this function (a pragma here does not
  // reach the operators inside HIP's __fadd_rn / __fmul_rn, which hipcc
  // contracts after inlining)
#pragma clang fp contract(off)
  constexpr int BM = kKgBM, BN = kKgBN, KS = kKgKS, RP = kKgRP;
  constexpr int MI = BM / 32, NJ = BN / 32;  // 16 x 16 tiles per wave
  constexpr int SBB = WT == Q4K ? 144 : 210;
  static_assert(PD % 2 == 0, "stages come in superblock pairs");
  // per group: the stage buffers, and per superblock (by parity) the
  // 32-value sums split hi / lo [row][8], the mins [col][8], d8 per row, d
  // / dmin per column
  __shared__ __attribute__((aligned(16))) int8_t AsG[G][2][BM * RP];
  __shared__ __attribute__((aligned(16))) int8_t BlG[G][2][BN * RP];
  __shared__ __attribute__((aligned(16))) int8_t BhG[G][2][BN * RP];
  __shared__ __attribute__((aligned(16))) int8_t AmlG[G][2][BM * 8], AmhG[G][2][BM * 8], BmnG[G][2][BN * 8];
  __shared__ __attribute__((aligned(16))) float Ad8G[G][2][BM];
  __shared__ float BdG[G][2][BN], BdmG[G][2][BN];
  // the float terms of groups 1.. for group 0: [group - 1][dot, min][output][thread]
  constexpr int NX = WT == Q4K ? 2 : 1;
  __shared__ float xch[G > 1 ? G - 1 : 1][NX][MI * NJ * 4][G > 1 ? 256 : 1];
  const int grp = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8);
  const int tid = threadIdx.x & 255, lane = tid & 63, wave = tid >> 6;
  auto& As = AsG[grp];
  auto& Bl = BlG[grp];
  auto& Bh = BhG[grp];
  auto& Aml = AmlG[grp];
  auto& Amh = AmhG[grp];
  auto& Bmn = BmnG[grp];
  auto& Ad8 = Ad8G[grp];
  auto& Bd = BdG[grp];
  auto& Bdm = BdmG[grp];
  const int m0 = blockIdx.y * BM;
  const int nt0 = blockIdx.x * BN;
  const int sg = (a.nseg > 1 && nt0 >= a.seg_end[0]) ? ((a.nseg > 2 && nt0 >= a.seg_end[1]) ? 2 : 1) : 0;
  const int base = sg == 0 ? 0 : a.seg_end[sg - 1];
  const int ns = a.seg_end[sg] - base, n0 = nt0 - base;
  const uint8_t* w = a.w[sg];
  float* y = a.y[sg];
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
  const int r16 = lane & 15, rq = (lane >> 4) * 4, kq16 = (lane >> 4) * 16;
  const int nsb = a.k / 256, nst = 2 * nsb / G;  // stages of this group
  const size_t wrow = (size_t)nsb * SBB;
  const int wc = tid >> 2, wp = tid & 3;  // weight staging: column, part (Q4_K 16-byte chunk; Q6_K quarter)
  const int mlast = a.m - 1;
  // rows past m clamp to the last row (their outputs are dropped)
  const int8_t* arow[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int c = tid + 256 * i, row = c >> 3, ch = c & 7;
    arow[i] = a.qs + (size_t)min(m0 + row, mlast) * a.k + ch * 16;
  }
  const float* d8row = a.d8 + (size_t)min(m0 + lane, mlast) * nsb;
  const int16_t* bsrow = a.bs32 + (size_t)min(m0 + (tid >> 2), mlast) * (a.k / 32) + 2 * (tid & 3);
  const uint8_t* wcol = w + (size_t)(n0 + wc) * wrow;

  KgStage<WT> S[PD];
  auto stage_load = [&](KgStage<WT>& R, int st) {
    const int sb = (st >> 1) * G + grp, h = st & 1;
#pragma unroll
    for (int i = 0; i < 2; i++) R.a[i] = *reinterpret_cast<const u32x4*>(arow[i] + sb * 256 + h * KS);
    const uint8_t* blk = wcol + (size_t)sb * SBB;
    R.d8 = d8row[sb];
    if constexpr (WT == Q4K) {
      R.h = *reinterpret_cast<const u32x4*>(blk);
      R.q = *reinterpret_cast<const u32x4*>(blk + 16 + 64 * h + 16 * wp);
      R.bs = *reinterpret_cast<const uint32_t*>(bsrow + sb * 8);
    } else {
      // quarter wp of half h: ql[64h + 32(wp & 1) .. +32], qh[32h .. +32]
      const u32x4a2* lp = reinterpret_cast<const u32x4a2*>(blk + 64 * h + 32 * (wp & 1));
      const u32x4a2* hp = reinterpret_cast<const u32x4a2*>(blk + 128 + 32 * h);
      const u32x4a2 l0 = lp[0], l1 = lp[1], h0 = hp[0], h1 = hp[1];
      R.l0 = u32x4{l0.x, l0.y, l0.z, l0.w};
      R.l1 = u32x4{l1.x, l1.y, l1.z, l1.w};
      R.h0 = u32x4{h0.x, h0.y, h0.z, h0.w};
      R.h1 = u32x4{h1.x, h1.y, h1.z, h1.w};
      R.sc = *reinterpret_cast<const uint16_t*>(blk + 192 + 8 * h + 2 * wp);
      R.d = *reinterpret_cast<const uint16_t*>(blk + 208);
    }
  };
  // h: the stage's half of its superblock (0: also the superblock's terms)
  auto stage_store = [&](const KgStage<WT>& R, int sp, int h, int buf) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int c = tid + 256 * i, row = c >> 3, ch = c & 7;
      *reinterpret_cast<u32x4*>(&As[buf][row * RP + ch * 16]) = R.a[i];
    }
    int8_t* bl = &Bl[buf][wc * RP];
    int8_t* bh = &Bh[buf][wc * RP];
    if constexpr (WT == Q4K) {
      // chunk wp: pair j = 2h + wp / 2, elements 16 (wp & 1) .. +16 of
      // sub-blocks 2j (low nibbles) and 2j + 1 (high nibbles)
      const int j = 2 * h + (wp >> 1);
      int scA, mA, scB, mB;
      kg_scale_min(R.h.y, R.h.z, R.h.w, 2 * j, scA, mA);
      kg_scale_min(R.h.y, R.h.z, R.h.w, 2 * j + 1, scB, mB);
      const uint32_t sA2 = (uint32_t)scA * 0x00010001u, sB2 = (uint32_t)scB * 0x00010001u;
      const int kA = (wp >> 1) * 64 + (wp & 1) * 16, kB = kA + 32;
      const uint32_t qv[4] = {R.q.x, R.q.y, R.q.z, R.q.w};
      uint32_t loA[4], hiA[4], loB[4], hiB[4];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        digits_u4(qv[c] & 0x0F0F0F0Fu, sA2, loA[c], hiA[c]);
        digits_u4((qv[c] >> 4) & 0x0F0F0F0Fu, sB2, loB[c], hiB[c]);
      }
      *reinterpret_cast<u32x4*>(bl + kA) = u32x4{loA[0], loA[1], loA[2], loA[3]};
      *reinterpret_cast<u32x4*>(bh + kA) = u32x4{hiA[0], hiA[1], hiA[2], hiA[3]};
      *reinterpret_cast<u32x4*>(bl + kB) = u32x4{loB[0], loB[1], loB[2], loB[3]};
      *reinterpret_cast<u32x4*>(bh + kB) = u32x4{hiB[0], hiB[1], hiB[2], hiB[3]};
      if (h == 0) {
        if (wp == 0) {
          Bd[sp][wc] = (float)__builtin_bit_cast(_Float16, (unsigned short)(R.h.x & 0xFFFFu));
          Bdm[sp][wc] = (float)__builtin_bit_cast(_Float16, (unsigned short)(R.h.x >> 16));
          uint32_t mw[2] = {0u, 0u};
#pragma unroll
          for (int g = 0; g < 8; g++) {
            int s_, m_;
            kg_scale_min(R.h.y, R.h.z, R.h.w, g, s_, m_);
            mw[g >> 2] |= (uint32_t)m_ << (8 * (g & 3));
          }
          *reinterpret_cast<uint2*>(&Bmn[sp][wc * 8]) = make_uint2(mw[0], mw[1]);
        }
        // row tid / 4, sums 2 (tid % 4) and + 1: digits lo = v & 127, hi = v >> 7
        const int v0 = (int)(int16_t)(R.bs & 0xFFFFu), v1 = (int)(int16_t)(R.bs >> 16);
        const int o = (tid >> 2) * 8 + 2 * (tid & 3);
        *reinterpret_cast<uint16_t*>(&Aml[sp][o]) = (uint16_t)((v0 & 127) | ((v1 & 127) << 8));
        *reinterpret_cast<uint16_t*>(&Amh[sp][o]) = (uint16_t)(((v0 >> 7) & 0xFF) | (((v1 >> 7) & 0xFF) << 8));
      }
    } else {
      // quarter Q = wp of half h: element 128 h + 32 Q + l (l < 32) is
      // ((ql[64 h + l + 32 (Q & 1)] >> 4 (Q >> 1)) & 15) | (((qh[32 h + l] >>
      // 2 Q) & 3) << 4), scale sc[8 h + 2 Q + l / 16]
      const int nsh = 4 * (wp >> 1), hsh = 2 * wp;
      const int sc0 = (int)(int8_t)(R.sc & 0xFFu), sc1 = (int)(int8_t)(R.sc >> 8);
      const uint32_t s02 = ((uint32_t)sc0 & 0xFFFFu) * 0x00010001u, s12 = ((uint32_t)sc1 & 0xFFFFu) * 0x00010001u;
      const uint32_t lv[8] = {R.l0.x, R.l0.y, R.l0.z, R.l0.w, R.l1.x, R.l1.y, R.l1.z, R.l1.w};
      const uint32_t hv[8] = {R.h0.x, R.h0.y, R.h0.z, R.h0.w, R.h1.x, R.h1.y, R.h1.z, R.h1.w};
      uint32_t lo[8], hi[8];
#pragma unroll
      for (int c = 0; c < 8; c++) {
        const uint32_t q6 = ((lv[c] >> nsh) & 0x0F0F0F0Fu) | (((hv[c] >> hsh) & 0x03030303u) << 4);
        digits_q6(q6, c < 4 ? s02 : s12, lo[c], hi[c]);
      }
      const int k0 = 32 * wp;
      *reinterpret_cast<u32x4*>(bl + k0) = u32x4{lo[0], lo[1], lo[2], lo[3]};
      *reinterpret_cast<u32x4*>(bl + k0 + 16) = u32x4{lo[4], lo[5], lo[6], lo[7]};
      *reinterpret_cast<u32x4*>(bh + k0) = u32x4{hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<u32x4*>(bh + k0 + 16) = u32x4{hi[4], hi[5], hi[6], hi[7]};
      if (h == 0 && wp == 0) Bd[sp][wc] = (float)__builtin_bit_cast(_Float16, (unsigned short)(R.d & 0xFFFFu));
    }
    if (h == 0 && tid < BM) Ad8[sp][tid] = R.d8;
  };

  float fdot[MI][NJ][4], fmin[MI][NJ][4];
  v4i ahi[MI][NJ], alo[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      ahi[i][j] = v4i{0, 0, 0, 0};
      alo[i][j] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < 4; r++) fdot[i][j][r] = fmin[i][j][r] = 0.0f;
    }
  // stage st lives in ring slot st % PD and LDS buffer st % 2
#pragma unroll
  for (int u = 0; u < PD; u++) stage_load(S[u], min(u, nst - 1));
  stage_store(S[0], 0, 0, 0);
  __syncthreads();
  for (int s0 = 0; s0 < nst; s0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; u++) {
      const int st = s0 + u, buf = u & 1;
      // slot u is in LDS already: refill it PD stages ahead (clamped: the
      // last stages reload the final stage and never store it)
      stage_load(S[u], min(st + PD, nst - 1));
#pragma unroll
      for (int kk = 0; kk < KS / 64; kk++) {
        v4i av[MI], bl[NJ], bh[NJ];
#pragma unroll
        for (int i = 0; i < MI; i++)
          av[i] = *reinterpret_cast<const v4i*>(&As[buf][(wm + 16 * i + r16) * RP + kk * 64 + kq16]);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          bl[j] = *reinterpret_cast<const v4i*>(&Bl[buf][(wn + 16 * j + r16) * RP + kk * 64 + kq16]);
          bh[j] = *reinterpret_cast<const v4i*>(&Bh[buf][(wn + 16 * j + r16) * RP + kk * 64 + kq16]);
        }
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
          for (int j = 0; j < NJ; j++) {
            alo[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i], bl[j], alo[i][j], 0, 0, 0);
            ahi[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i], bh[j], ahi[i][j], 0, 0, 0);
          }
      }
      float tdot[MI][NJ][4], tmin[MI][NJ][4];  // G > 1: this group's terms of the superblock
      if (u & 1) {
        // superblock done: the float terms in the reference's order
        const int sp = (st >> 1) & 1;
        long aml[MI], amh[MI], bm[NJ];
        if constexpr (WT == Q4K) {
          // min_sum through one MFMA per digit: k = sub-block 0..7 in lanes
          // 0..15, zeros elsewhere
#pragma unroll
          for (int i = 0; i < MI; i++) {
            aml[i] = lane < 16 ? *reinterpret_cast<const long*>(&Aml[sp][(wm + 16 * i + r16) * 8]) : 0;
            amh[i] = lane < 16 ? *reinterpret_cast<const long*>(&Amh[sp][(wm + 16 * i + r16) * 8]) : 0;
          }
#pragma unroll
          for (int j = 0; j < NJ; j++)
            bm[j] = lane < 16 ? *reinterpret_cast<const long*>(&Bmn[sp][(wn + 16 * j + r16) * 8]) : 0;
        }
#pragma unroll
        for (int i = 0; i < MI; i++) {
          const float4 d8v = *reinterpret_cast<const float4*>(&Ad8[sp][wm + 16 * i + rq]);
          const float d8r[4] = {d8v.x, d8v.y, d8v.z, d8v.w};
#pragma unroll
          for (int j = 0; j < NJ; j++) {
            const float dw = Bd[sp][wn + 16 * j + r16];
            if constexpr (WT == Q4K) {
              const v4i ml = __builtin_amdgcn_mfma_i32_16x16x32_i8(aml[i], bm[j], v4i{0, 0, 0, 0}, 0, 0, 0);
              const v4i mh = __builtin_amdgcn_mfma_i32_16x16x32_i8(amh[i], bm[j], v4i{0, 0, 0, 0}, 0, 0, 0);
              const float dmw = Bdm[sp][wn + 16 * j + r16];
#pragma unroll
              for (int r = 0; r < 4; r++) {
                const int isum = (ahi[i][j][r] << 7) + alo[i][j][r];
                const int msum = (mh[r] << 7) + ml[r];
                const float dc = dw * d8r[r], dmc = dmw * d8r[r];
                if (G == 1) {
                  fdot[i][j][r] = fdot[i][j][r] + dc * (float)isum;
                  fmin[i][j][r] = fmin[i][j][r] + dmc * (float)msum;
                } else {
                  tdot[i][j][r] = dc * (float)isum;
                  tmin[i][j][r] = dmc * (float)msum;
                }
              }
            } else {
#pragma unroll
              for (int r = 0; r < 4; r++) {
                const int isum = (ahi[i][j][r] << 7) + alo[i][j][r];
                if (G == 1)
                  fdot[i][j][r] = fdot[i][j][r] + (dw * d8r[r]) * (float)isum;
                else
                  tdot[i][j][r] = (dw * d8r[r]) * (float)isum;
              }
            }
            ahi[i][j] = v4i{0, 0, 0, 0};
            alo[i][j] = v4i{0, 0, 0, 0};
          }
        }
        if (G > 1 && grp > 0) {
#pragma unroll
          for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
              for (int r = 0; r < 4; r++) {
                const int o = (i * NJ + j) * 4 + r;
                xch[grp - 1][0][o][tid] = tdot[i][j][r];
                if (WT == Q4K) xch[grp - 1][NX - 1][o][tid] = tmin[i][j][r];
              }
        }
      }
      // the next stage into the other buffer (past the end: a clamped
      // repeat that nothing reads)
      stage_store(S[(u + 1) % PD], ((st + 1) >> 1) & 1, (u + 1) & 1, buf ^ 1);
      __syncthreads();
      if (G > 1 && (u & 1) && grp == 0) {
        // superblocks G j, G j + 1, ...: own terms, then each group's (the
        // next exchange is written two barriers later)
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
          for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const int o = (i * NJ + j) * 4 + r;
              fdot[i][j][r] = fdot[i][j][r] + tdot[i][j][r];
              if (WT == Q4K) fmin[i][j][r] = fmin[i][j][r] + tmin[i][j][r];
#pragma unroll
              for (int g = 1; g < G; g++) {
                fdot[i][j][r] = fdot[i][j][r] + xch[g - 1][0][o][tid];
                if (WT == Q4K) fmin[i][j][r] = fmin[i][j][r] + xch[g - 1][NX - 1][o][tid];
              }
            }
      }
    }
  }
  if (grp != 0) return;
  // D layout of v_mfma_*_16x16*: lane l holds rows 4 (l / 16) + r, column l % 16
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int gm = m0 + wm + 16 * i + rq + r;
        const int gn = n0 + wn + 16 * j + r16;
        if (gm < a.m) {
          const float v = WT == Q4K ? fdot[i][j][r] - fmin[i][j][r] : fdot[i][j][r];
          float* o = y + (size_t)gm * ns + gn;
          store_out(o, a.accumulate ? *o + v : v);  // through the L2, as the Q8_0 GEMM
        }
      }
}

}  // namespace zg

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// compute units of the device (queried once; a thread-safe static)
static int kg_cu_count() {
  static const int n = [] {
    int dev = 0, v = 0;
    return hipGetDevice(&dev) == hipSuccess &&
                   hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
               ? v
               : 256;
  }();
  return n;
}

zg_status zg::run_quantize_q8k_split(zg_ctx* ctx, const float* x, int8_t* qs, float* d8, int16_t* bs32, size_t rows,
                                     size_t k, hipStream_t st) {
  if (!x || !qs || !d8 || !bs32) return set_error(ctx, ZG_ERR_INVALID_ARG, "quantize_q8k_split: null pointer");
  if (k == 0 || k % 256) return set_error(ctx, ZG_ERR_INVALID_ARG, "quantize_q8k_split: k %% 256 != 0");
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(qs) & 3) ||
      (reinterpret_cast<uintptr_t>(d8) & 3) || (reinterpret_cast<uintptr_t>(bs32) & 1))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "quantize_q8k_split: misaligned buffer");
  if (rows == 0) return ZG_OK;
  const size_t blocks = rows * (k / 256);
  if (blocks > (size_t)INT32_MAX || k > (size_t)INT32_MAX) return set_error(ctx, ZG_ERR_INVALID_ARG, "quantize_q8k_split: too large");
  hipLaunchKernelGGL(quantize_q8k_split_kernel, dim3((unsigned)blocks), dim3(64), 0, st, x, qs, d8, bs32, (int)k);
  return hip_check(ctx, hipGetLastError(), "quantize_q8k_split launch");
}

zg_status zg::run_gemm_q8k(zg_ctx* ctx, const int8_t* qs, const float* d8, const int16_t* bs32, const GemmSegDev* segs,
                           int nseg, size_t m, size_t k, uint32_t w_type, bool accumulate, hipStream_t st) {
  if (!qs || !d8 || !bs32 || !segs || nseg < 1 || nseg > kKgSegs)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm_q8k: bad arguments");
  if (w_type != ZG_Q4K && w_type != ZG_Q6K) return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "gemm_q8k: weights must be Q4_K/Q6_K");
  if (k == 0 || k % 256) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm_q8k: k %% 256 != 0");
  if ((reinterpret_cast<uintptr_t>(qs) & 15) || (k % 16) || (reinterpret_cast<uintptr_t>(d8) & 3) ||
      (reinterpret_cast<uintptr_t>(bs32) & 3))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm_q8k: activations misaligned");
  KgemmArgs a{};
  a.qs = qs;
  a.d8 = d8;
  a.bs32 = bs32;
  size_t n = 0;
  for (int i = 0; i < nseg; i++) {
    if (!segs[i].w || !segs[i].y) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm_q8k: null pointer");
    if (segs[i].n == 0 || segs[i].n % kKgBN) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm_q8k: width %% %d", kKgBN);
    if (w_type == ZG_Q4K && (reinterpret_cast<uintptr_t>(segs[i].w) & 15))
      return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm_q8k: Q4_K weights misaligned");
    if (w_type == ZG_Q6K && (reinterpret_cast<uintptr_t>(segs[i].w) & 1))
      return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm_q8k: Q6_K weights misaligned");
    n += segs[i].n;
    a.w[i] = segs[i].w;
    a.y[i] = segs[i].y;
    a.seg_end[i] = (int)n;
  }
  if (m == 0) return ZG_OK;
  if (m > (size_t)INT32_MAX || n > (size_t)INT32_MAX || k > (size_t)INT32_MAX)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm_q8k: shape too large");
  for (int i = nseg; i < kKgSegs; i++) {
    a.w[i] = a.w[0];
    a.y[i] = a.y[0];
    a.seg_end[i] = (int)n;
  }
  a.nseg = nseg;
  a.accumulate = accumulate ? 1 : 0;
  a.m = (int)m;
  a.n = (int)n;
  a.k = (int)k;
  const dim3 grid((unsigned)(n / kKgBN), (unsigned)((m + kKgBM - 1) / kKgBM));
  // kKgPD stages in flight when the stage count is a multiple of it, else two
  // two groups per workgroup when the tiles give at most one workgroup per
  // CU (a prefill's few rows, the narrow down projection) and the
  // superblocks split evenly; else one
  const bool split = ZG_KG_GROUPS > 1 && (size_t)grid.x * grid.y <= (size_t)kg_cu_count() && (k / 256) % 2 == 0;
  const bool deep = (k / 256) % (kKgPD / 2) == 0;
  if (w_type == ZG_Q4K) {
    if (split) hipLaunchKernelGGL((gemm_q8k_kernel<Q4K, 2, 2>), grid, dim3(512), 0, st, a);
    else if (deep) hipLaunchKernelGGL((gemm_q8k_kernel<Q4K, kKgPD, 1>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((gemm_q8k_kernel<Q4K, 2, 1>), grid, dim3(256), 0, st, a);
  } else {
    if (split) hipLaunchKernelGGL((gemm_q8k_kernel<Q6K, 2, 2>), grid, dim3(512), 0, st, a);
    else if (deep) hipLaunchKernelGGL((gemm_q8k_kernel<Q6K, kKgPD, 1>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((gemm_q8k_kernel<Q6K, 2, 1>), grid, dim3(256), 0, st, a);
  }
  return hip_check(ctx, hipGetLastError(), "gemm_q8k launch");
}

static hipStream_t kg_stream(zg_ctx* ctx, void* s) { return s ? reinterpret_cast<hipStream_t>(s) : ctx->stream; }

extern "C" zg_status zg_quantize_q8k_split_dev(zg_ctx* ctx, const float* d_x, int8_t* d_qs, float* d_d8,
                                               int16_t* d_bs32, size_t rows, size_t k, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  return run_quantize_q8k_split(ctx, d_x, d_qs, d_d8, d_bs32, rows, k, kg_stream(ctx, stream));
}

extern "C" zg_status zg_gemm_q8k_dev(zg_ctx* ctx, const int8_t* d_qs, const float* d_d8, const int16_t* d_bs32,
                                     const void* d_w, float* d_y, size_t m, size_t n, size_t k, uint32_t w_type,
                                     int accumulate, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_w || !d_y) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm_q8k: null pointer");
  const GemmSegDev seg{static_cast<const uint8_t*>(d_w), d_y, n};
  return run_gemm_q8k(ctx, d_qs, d_d8, d_bs32, &seg, 1, m, k, w_type, accumulate != 0, kg_stream(ctx, stream));
}
