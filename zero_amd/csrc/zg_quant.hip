// zg_quant.hip -- on-the-fly Q8_0 activation quantization and the M >= 64
// prefill GEMM (int8 MFMA) for gfx950.
//
// The reference has no batched prefill (kernel/src/inference.rs:1188-1330
// runs the prompt token by token) and never quantizes activations on its
// Q4_0/Q8_0 path.  The quantizer restates the packer's Q8_0 block encoder
// (tools/silicatepack.py:893-907, fp16 bytes :854-861) bit for bit: the
// amax, d = amax/127, 1/d and x/d are computed in double as Python does,
// round() is round-half-even (rint), and d is stored as the
// round-to-nearest-even binary16 of the double d.
#include <hip/hip_runtime.h>
#include <type_traits>

#include "../../include/zero_gpu.h"
#include "zg_device.h"
#include "zg_internal.h"

using namespace zg;

namespace zg {

struct QuantArgs {
  const float* x;   // [rows][k]
  uint8_t* blocks;  // optional: [rows][k/32] x 34-byte Q8_0 blocks
  int8_t* qs;       // optional: [rows][k] int8
  uint16_t* d;      // optional: [rows][k/32] fp16 bits
  size_t rows, k;
};

// One thread per 32-element block.  A block holding a non-finite value (the
// packer raises ValueError there, silicatepack.py:877-887) is written with
// q = 0 and d = NaN (0x7E00) so that it cannot pass unnoticed.
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(QuantArgs a) {
  const size_t nb = a.k / 32;
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= a.rows * nb) return;
  const size_t row = t / nb, b = t % nb;
  const float4* src = reinterpret_cast<const float4*>(a.x + row * a.k + b * 32);
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float4 f = src[i];
    v[4 * i] = f.x;
    v[4 * i + 1] = f.y;
    v[4 * i + 2] = f.z;
    v[4 * i + 3] = f.w;
  }
  int8_t q[32];
  const uint32_t dbits = q8_0_encode(v, q);
  if (a.qs) {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
      w[i] = (uint32_t)(uint8_t)q[4 * i] | ((uint32_t)(uint8_t)q[4 * i + 1] << 8) |
             ((uint32_t)(uint8_t)q[4 * i + 2] << 16) | ((uint32_t)(uint8_t)q[4 * i + 3] << 24);
    u32x4* dst = reinterpret_cast<u32x4*>(a.qs + row * a.k + b * 32);
    dst[0] = u32x4{w[0], w[1], w[2], w[3]};
    dst[1] = u32x4{w[4], w[5], w[6], w[7]};
  }
  if (a.d) a.d[row * nb + b] = (uint16_t)dbits;
  if (a.blocks) {
    uint8_t* o = a.blocks + (row * nb + b) * 34;
    // 34-byte blocks are only 2-byte aligned: 17 halfword stores
    uint16_t* o16 = reinterpret_cast<uint16_t*>(o);
    o16[0] = (uint16_t)dbits;
#pragma unroll
    for (int i = 0; i < 16; i++) o16[1 + i] = (uint16_t)((uint8_t)q[2 * i] | ((uint16_t)(uint8_t)q[2 * i + 1] << 8));
  }
}

// ---------------------------------------------------------------------------
// Prefill GEMM: Y[m][n] = sum_b dX[m][b] * dW[n][b] * sum_{k in b} qX*qW.
// v_mfma_i32_16x16x32_i8: one MFMA is exactly one 32-element block of a
// 16x16 output tile, so each block's int32 dot is scaled once by its two
// fp16 scales and accumulated in fp32 as acc = fma(dX*dW, isum, acc) in
// ascending block order (the operation order of the oracle's
// zo_gemm_q8act, so results match it bit for bit).  Workgroup tile 64 (m) x 64 (n), 4 waves of
// 32 x 32 (2 x 2 MFMA tiles), 4 blocks (128 K) staged in LDS per step.
// ---------------------------------------------------------------------------
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// The 64-row tile's waves each own a 32 x 32 output block and multiply one
// 32-element block with a single v_mfma_i32_32x32x32_i8 (32 cycles for the
// 32 x 32 outputs, where four v_mfma_i32_16x16x32_i8 take 64).
#ifndef ZG_GEMM_MFMA32
#define ZG_GEMM_MFMA32 1
#endif

// Up to three weight matrices that share the activations (Q|K|V, gate|up)
// in one launch: the output columns are the concatenation of the segments,
// seg_end[s] is the end column of segment s, and every 64-column tile lies
// in one segment (segment widths are multiples of 64 when there are
// several).  Segment s writes y[s] as [m][width of s].
constexpr int kGemmSegs = 3;

struct GemmArgs {
  const int8_t* xq;    // [m][k]
  const uint16_t* xd;  // [m][k/32]
  const uint8_t* w[kGemmSegs];  // weights, Q4_0/Q8_0, plain or X4
  float* y[kGemmSegs];          // [m][n_s]
  int seg_end[kGemmSegs];
  int nseg;
  int accumulate;  // 1: y += result (residual add), 0: y = result
  int m, n, k;     // n: total columns
  // XCD rectangles: 0, or the tile grid cut into 8 rectangles of rx x ry
  // tiles, one per XCD (see gemm_tile)
  int rx, ry;
};

// The tile of this workgroup.  Workgroups go to the eight XCDs round-robin
// in dispatch order, so with the plain order XCD j holds the column tiles
// j, j + 8, ... of every row tile and each XCD's L2 fetches every
// activation row.  With rectangles, the k-th workgroup of XCD j takes tile
// k of rectangle j (row-major inside it): each XCD reads the activation
// rows and weight columns of one rectangle only.  Both orders cover every
// tile once.
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, int& tx, int& ty) {
  if (a.rx == 0) {
    tx = blockIdx.x;
    ty = blockIdx.y;
    return;
  }
  const int lin = blockIdx.x + gridDim.x * blockIdx.y;
  const int j = lin & 7, k = lin >> 3;
  const int rects_x = gridDim.x / a.rx;
  tx = (j % rects_x) * a.rx + k % a.rx;
  ty = (j / rects_x) * a.ry + k / a.rx;
}

constexpr int kBN = 64;  // tile columns (tile rows BM: 64 or 32)
// LDS row stride in bytes for BK blocks of 32 per stage (padded, 16-B aligned)
// (36 dwords for 4-block stages: the 16 rows of an MFMA operand read start
// on 16 distinct 4-bank groups of the 64 banks, so the per-block 8-byte
// operand reads are conflict-free)
template <int BK>
constexpr int lds_row() { return BK * 32 + 16; }

// One stage's global operands held in registers between the load and the
// LDS store (so that the next stage's loads fly while the current stage is
// multiplied).  Per thread of NT: NA 16-byte activation chunks, ND
// activation scales, NW weight block rows (raw quants + scale).
template <uint32_t WT, int BM, int BK, int NT>
struct GemmStage {
  static_assert(BM * BK * 2 % NT == 0 && kBN * BK % NT == 0, "every thread stages whole chunks and blocks");
  static constexpr int NA = BM * BK * 2 / NT;
  static constexpr int ND = (BM * BK + NT - 1) / NT;
  static constexpr int NW = kBN * BK / NT;
  static constexpr int QW = WT == Q4_0 ? 4 : 8;
  u32x4 a[NA];
  uint32_t ad[ND];
  uint32_t q[NW][QW];
  uint32_t wd[NW];
};

// FULL: the whole tile lies inside the matrix and k is a whole number of
// stages, so every load is in bounds and none is guarded
template <uint32_t WT, int IL, int BM, int BK, bool FULL, int NT>
__device__ __forceinline__ void gemm_stage_load(GemmStage<WT, BM, BK, NT>& S, const GemmArgs& a, const uint8_t* w,
                                                int ns, int m0, int n0, int b0, int tid) {
  using St = GemmStage<WT, BM, BK, NT>;
  const int nb = a.k / 32;
#pragma unroll
  for (int i = 0; i < St::NA; i++) {
    const int c = tid + NT * i, row = c / (BK * 2), ch = c % (BK * 2);
    const int gm = m0 + row, kb = b0 + ch / 2;
    S.a[i] = u32x4{0, 0, 0, 0};
    if (FULL || (gm < a.m && kb < nb))
      S.a[i] = *reinterpret_cast<const u32x4*>(a.xq + (size_t)gm * a.k + (size_t)kb * 32 + (ch & 1) * 16);
  }
  // scales and weight blocks: consecutive threads take consecutive rows
  // (columns) of one block, so that their LDS stores are conflict-free (the
  // 64-row tile had 0.59 M conflict cycles with the block index fastest)
#pragma unroll
  for (int i = 0; i < St::ND; i++) {
    const int c = tid + NT * i, row = c % BM, kk = c / BM;
    const int gm = m0 + row, kb = b0 + kk;
    S.ad[i] = (kk < BK && (FULL || (gm < a.m && kb < nb))) ? (uint32_t)a.xd[(size_t)gm * nb + kb] : 0u;
  }
#pragma unroll
  for (int i = 0; i < St::NW; i++) {
    const int c = tid + NT * i, row = c % kBN, kk = c / kBN;
    const int gn = n0 + row, kb = b0 + kk;
#pragma unroll
    for (int j = 0; j < St::QW; j++) S.q[i][j] = 0;
    S.wd[i] = 0;
    if (FULL || (gn < ns && kb < nb)) {
      const uint8_t* dp;
      const uint8_t* qp;
      if (IL == 4) {
        const size_t gb = (WT == Q4_0) ? 72 : 136;
        const uint8_t* g = w + (size_t)(gn >> 2) * nb * gb + (size_t)kb * gb;
        dp = g + 2 * (gn & 3);
        qp = g + 8 + (gn & 3) * ((WT == Q4_0) ? 16 : 32);
#pragma unroll
        for (int j = 0; j < St::QW / 2; j++) {
          const uint2 v = *reinterpret_cast<const uint2*>(qp + 8 * j);
          S.q[i][2 * j] = v.x;
          S.q[i][2 * j + 1] = v.y;
        }
      } else if (IL == 5) {
        // split-scale X4 group: [kb][row] quants, then [kb][row] fp16 scales
        const size_t gb = (WT == Q4_0) ? 72 : 136;
        constexpr int QB = (WT == Q4_0) ? 16 : 32;
        const uint8_t* g = w + (size_t)(gn >> 2) * nb * gb;
        const size_t u = (size_t)kb * 4 + (gn & 3);
        dp = g + (size_t)nb * 4 * QB + 2 * u;
        qp = g + u * QB;
#pragma unroll
        for (int j = 0; j < St::QW / 2; j++) {
          const uint2 v = *reinterpret_cast<const uint2*>(qp + 8 * j);
          S.q[i][2 * j] = v.x;
          S.q[i][2 * j + 1] = v.y;
        }
      } else {
        const size_t bb = (WT == Q4_0) ? 18 : 34;
        dp = w + ((size_t)gn * nb + kb) * bb;
        qp = dp + 2;
#pragma unroll
        for (int j = 0; j < St::QW; j++)
          S.q[i][j] = (uint32_t)qp[4 * j] | ((uint32_t)qp[4 * j + 1] << 8) | ((uint32_t)qp[4 * j + 2] << 16) |
                      ((uint32_t)qp[4 * j + 3] << 24);
      }
      S.wd[i] = (uint32_t)dp[0] | ((uint32_t)dp[1] << 8);
    }
  }
}

// A full tile's loads (FULL below, with activations and every weight
// segment under 2 GB): each thread's byte offsets from the per-stage bases
// are fixed for the whole kernel, so a stage's loads take a wave-uniform
// base (scalar registers, advanced once per stage) plus a fixed 32-bit
// per-lane offset, and cost no vector address arithmetic.
template <uint32_t WT, int IL, int BM, int BK, int NT>
struct GemmOffs {
  using St = GemmStage<WT, BM, BK, NT>;
  uint32_t a[St::NA], ad[St::ND], q[St::NW], d[St::NW];
};

template <uint32_t WT, int IL, int BM, int BK, int NT>
__device__ __forceinline__ void gemm_offsets(GemmOffs<WT, IL, BM, BK, NT>& O, const GemmArgs& a, int m0, int n0,
                                             int tid) {
  using St = GemmStage<WT, BM, BK, NT>;
  const uint32_t nb = (uint32_t)a.k / 32;
  constexpr uint32_t gb = WT == Q4_0 ? 72 : 136, QB = WT == Q4_0 ? 16 : 32, bb = WT == Q4_0 ? 18 : 34;
#pragma unroll
  for (int i = 0; i < St::NA; i++) {
    const int c = tid + NT * i, row = c / (BK * 2), ch = c % (BK * 2);
    O.a[i] = (uint32_t)(m0 + row) * (uint32_t)a.k + (uint32_t)(ch / 2) * 32 + (uint32_t)(ch & 1) * 16;
  }
#pragma unroll
  for (int i = 0; i < St::ND; i++) {
    const int c = tid + NT * i, row = c % BM, kk = c / BM;
    O.ad[i] = ((uint32_t)(m0 + row) * nb + (uint32_t)kk) * 2;
  }
#pragma unroll
  for (int i = 0; i < St::NW; i++) {
    const int c = tid + NT * i, row = c % kBN, kk = c / kBN;
    const uint32_t gn = (uint32_t)(n0 + row);
    if (IL == 4) {
      const uint32_t g = (gn >> 2) * nb * gb + (uint32_t)kk * gb;
      O.d[i] = g + 2 * (gn & 3);
      O.q[i] = g + 8 + (gn & 3) * QB;
    } else if (IL == 5) {
      const uint32_t g = (gn >> 2) * nb * gb, u = (uint32_t)kk * 4 + (gn & 3);
      O.q[i] = g + u * QB;
      O.d[i] = g + nb * 4 * QB + 2 * u;
    } else {
      O.d[i] = (gn * nb + (uint32_t)kk) * bb;
      O.q[i] = O.d[i] + 2;
    }
  }
}

// The offset as a 32-bit value defined where it is used, so that the load
// is selected as a scalar base plus a 32-bit vector offset (hoisted out of
// the stage loop it would be widened to a 64-bit vector add per load).
// Raw buffer loads with the stage advance as the scalar offset measured
// slower (M=512 x 2048x6144: 32.4 against 30.9 us).
__device__ __forceinline__ uint32_t pin_off(uint32_t o) {
  asm volatile("" : "+v"(o));
  return o;
}

template <uint32_t WT, int IL, int BM, int BK, int NT>
__device__ __forceinline__ void gemm_stage_load_full(GemmStage<WT, BM, BK, NT>& S, const GemmOffs<WT, IL, BM, BK, NT>& O,
                                                     const GemmArgs& a, const uint8_t* w, int b0, int tid) {
  using St = GemmStage<WT, BM, BK, NT>;
  constexpr uint32_t gb = WT == Q4_0 ? 72 : 136, QB = WT == Q4_0 ? 16 : 32, bb = WT == Q4_0 ? 18 : 34;
  const int8_t* xa = a.xq + (size_t)b0 * 32;
  const uint8_t* xd = reinterpret_cast<const uint8_t*>(a.xd) + (size_t)b0 * 2;
  const uint8_t* wq = w + (size_t)b0 * (IL == 4 ? gb : IL == 5 ? 4 * QB : bb);
  const uint8_t* wd = IL == 5 ? w + (size_t)b0 * 8 : wq;
#pragma unroll
  for (int i = 0; i < St::NA; i++) S.a[i] = *reinterpret_cast<const u32x4*>(xa + pin_off(O.a[i]));
#pragma unroll
  for (int i = 0; i < St::ND; i++) {
    const int kk = (tid + NT * i) / BM;
    S.ad[i] = kk < BK ? (uint32_t)*reinterpret_cast<const uint16_t*>(xd + pin_off(O.ad[i])) : 0u;
  }
#pragma unroll
  for (int i = 0; i < St::NW; i++) {
    const uint8_t* qp = wq + pin_off(O.q[i]);
    const uint8_t* dp = wd + pin_off(O.d[i]);
    if (IL == 4 || IL == 5) {
#pragma unroll
      for (int j = 0; j < St::QW / 2; j++) {
        const uint2 v = *reinterpret_cast<const uint2*>(qp + 8 * j);
        S.q[i][2 * j] = v.x;
        S.q[i][2 * j + 1] = v.y;
      }
      S.wd[i] = *reinterpret_cast<const uint16_t*>(dp);
    } else {
#pragma unroll
      for (int j = 0; j < St::QW; j++)
        S.q[i][j] = (uint32_t)qp[4 * j] | ((uint32_t)qp[4 * j + 1] << 8) | ((uint32_t)qp[4 * j + 2] << 16) |
                    ((uint32_t)qp[4 * j + 3] << 24);
      S.wd[i] = (uint32_t)dp[0] | ((uint32_t)dp[1] << 8);
    }
  }
}

// block-loop unroll of the 64-row tile's 16 x 16 form (ZG_GEMM_MFMA32 0;
// unrolled by 4: M=512 x 6144x2048 41.2 vs 35.0 us rolled; by 2: 36.5 us)
#ifndef ZG_GEMM_UNR64
#define ZG_GEMM_UNR64 1
#endif
// full tiles load through gemm_offsets / gemm_stage_load_full
#ifndef ZG_GEMM_OFFS
#define ZG_GEMM_OFFS 1
#endif
// block-loop unroll of the 32 x 32 form (M=512 x 6144x2048: 25.5-25.7 us by
// 2, 26.1-26.4 us rolled; by 4 the registers of a stage pair grow to 356
// and one wave fits a SIMD)
#ifndef ZG_GEMM_UNR32
#define ZG_GEMM_UNR32 2
#endif

// Block scales: the hardware fp16 conversion when ZG_GEMM_HWCVT (exact
// for every finite value; a NaN scale gives a NaN output either way), else
// the bit construction of half_bits_to_f32 (M=512: 34.2 / 42.9 us against
// 35.0 / 43.9 us for the up / down shapes)
#ifndef ZG_GEMM_HWCVT
#define ZG_GEMM_HWCVT 1
#endif
__device__ __forceinline__ float gemm_scale(uint32_t h) {
  if (ZG_GEMM_HWCVT) return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
  return half_bits_to_f32(h);
}

template <uint32_t WT, int BM, int BK, int NT>
__device__ __forceinline__ void gemm_stage_store(const GemmStage<WT, BM, BK, NT>& S, int8_t* As, int8_t* Bs, float* Ad,
                                                 float* Bd, int tid) {
  using St = GemmStage<WT, BM, BK, NT>;
  constexpr int R = lds_row<BK>();
#pragma unroll
  for (int i = 0; i < St::NA; i++) {
    const int c = tid + NT * i, row = c / (BK * 2), ch = c % (BK * 2);
    *reinterpret_cast<u32x4*>(As + row * R + ch * 16) = S.a[i];
  }
#pragma unroll
  for (int i = 0; i < St::ND; i++) {
    const int c = tid + NT * i, row = c % BM, kk = c / BM;
    if (kk < BK) Ad[kk * BM + row] = gemm_scale(S.ad[i]);
  }
#pragma unroll
  for (int i = 0; i < St::NW; i++) {
    const int c = tid + NT * i, row = c % kBN, kk = c / kBN;
    uint32_t q[8];
    if (WT == Q4_0) {
      // nibble n as the signed byte (n ^ 8) << 4 = 16 (n - 8): the block's
      // integer dot is 16 times the oracle's, and the weight scale is stored
      // divided by 16 (both exact: |16 isum| < 2^24, and dX dW is exact in
      // fp32), so every fma sees the same real product dX dW isum.
      // v_bitop3_b32 table 0x6A is (a & b) ^ c.
#pragma unroll
      for (int j = 0; j < 4; j++) {
        q[j] = __builtin_amdgcn_bitop3_b32(S.q[i][j] << 4, 0xF0F0F0F0u, 0x80808080u, 0x6A);  // elements 4j..4j+3
        q[4 + j] = __builtin_amdgcn_bitop3_b32(S.q[i][j], 0xF0F0F0F0u, 0x80808080u, 0x6A);   // elements 16+4j..
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) q[j] = S.q[i][St::QW == 8 ? j : 0];
    }
    u32x4* dst = reinterpret_cast<u32x4*>(Bs + row * R + kk * 32);
    dst[0] = u32x4{q[0], q[1], q[2], q[3]};
    dst[1] = u32x4{q[4], q[5], q[6], q[7]};
    Bd[kk * kBN + row] = WT == Q4_0 ? gemm_scale(S.wd[i]) * 0.0625f : gemm_scale(S.wd[i]);
  }
}

// Workgroup tile BM (m) x 64 (n) of NT threads, BK blocks (BK * 32 of K) per
// stage, double-buffered in LDS; the next stage's global loads are issued
// before the current stage is multiplied.  Per 32-K block an MFMA gives the
// block's integer dots, and every output adds dX*dW*isum with one fma,
// blocks in ascending order.  (Reading one activation scale per lane and
// taking a row's value by DPP row broadcast inside v_mul_f32_dpp, instead
// of a float4 of scales per lane, measured slower: 26.8 / 31.6 against
// 25.7 / 31.0 us.)  Shapes (M=512 times the Qwen3-1.7B FFN
// matrices, graph replays):
//   BM 64, BK 4, 256   large M: four waves of 32 x 32, one
//                      v_mfma_i32_32x32x32_i8 per block; three workgroups
//                      per CU (6144x2048: 25.5 us, against 27.1 us with
//                      four v_mfma_i32_16x16x32_i8 per block)
//   BM 32, BK 8, 512   fewer 64-row tiles: eight waves of 16 x 16, four
//                      waves per SIMD at two workgroups per CU (2048x6144:
//                      30.9 us, against 35.4 us with four waves of 16 x 32
//                      and 4-block stages); also at most one tile per CU
//                      (the batched prefill's 128 rows: 2.84 against 3.03
//                      ms with four waves)
template <uint32_t WT, int IL, int BM, int BK, bool FULL, int NT>
__global__ __launch_bounds__(NT) void gemm_q8act_kernel(GemmArgs a) {
  // waves: two along m, NT / 128 along n; each wave owns WR x WC outputs
  constexpr int WGN = NT / 128, WR = BM / 2, WC = kBN / WGN;
  constexpr int MI = WR / 16, NJ = WC / 16;  // 16 x 16 MFMA tiles per wave (16 x 16 form)
  constexpr bool W32 = BM == 64 && NT == 256 && ZG_GEMM_MFMA32;
  constexpr int R = lds_row<BK>();
  __shared__ __attribute__((aligned(16))) int8_t As[2][BM * R];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][kBN * R];
  __shared__ __attribute__((aligned(16))) float Ad[2][BK * BM];   // [kk][row]
  __shared__ __attribute__((aligned(16))) float Bd[2][BK * kBN];  // [kk][col]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int tx, ty;
  gemm_tile(a, tx, ty);
  const int m0 = ty * BM;
  // this tile's segment (uniform): its weights, output and local columns
  const int nt0 = tx * kBN;
  const int sg = (a.nseg > 1 && nt0 >= a.seg_end[0]) ? ((a.nseg > 2 && nt0 >= a.seg_end[1]) ? 2 : 1) : 0;
  const int base = sg == 0 ? 0 : a.seg_end[sg - 1];
  const int ns = a.seg_end[sg] - base, n0 = nt0 - base;
  const uint8_t* w = a.w[sg];
  float* y = a.y[sg];
  const int nb = a.k / 32;
  const int nst = (nb + BK - 1) / BK;
  const int wm = (wave / WGN) * WR, wn = (wave % WGN) * WC;
  const int r16 = lane & 15, kq = (lane >> 4) * 8, rq = (lane >> 4) * 4;
  const int r32 = lane & 31, h32 = lane >> 5;
  // 16 x 16 form: acc[(i * NJ + j) * 4 + r] is row wm + 16 i + rq + r,
  // column wn + 16 j + r16; 32 x 32 form: acc[4 g + r] is row wm + 8 g +
  // 4 h32 + r, column wn + r32
  constexpr int NACC = MI * NJ * 4;
  float acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; i++) acc[i] = 0.0f;

  GemmStage<WT, BM, BK, NT> S;
  GemmOffs<WT, IL, BM, BK, NT> O;
  if constexpr (FULL && ZG_GEMM_OFFS) gemm_offsets<WT, IL, BM, BK, NT>(O, a, m0, n0, tid);
  auto load = [&](int b0) {
    if constexpr (FULL && ZG_GEMM_OFFS) gemm_stage_load_full<WT, IL, BM, BK, NT>(S, O, a, w, b0, tid);
    else gemm_stage_load<WT, IL, BM, BK, FULL>(S, a, w, ns, m0, n0, b0, tid);
  };
  load(0);
  gemm_stage_store<WT, BM, BK>(S, As[0], Bs[0], Ad[0], Bd[0], tid);
  __syncthreads();
  // One stage: the next stage's global loads are issued, this stage's blocks
  // are multiplied out of LDS buffer buf, the next stage is stored to the
  // other buffer.  Stages run in pairs so that buf is a constant and every
  // LDS address is a fixed register plus an immediate offset.
  auto stage = [&](auto bufc, int st) {
    constexpr int buf = decltype(bufc)::value;
    if (st + 1 < nst) load((st + 1) * BK);
    const int8_t* A = As[buf];
    const int8_t* B = Bs[buf];
    // blocks past k in the last stage hold zero quants and scales: they add
    // fma(0, 0, acc) = acc
    // the 32-row tile's block loop is unrolled (the rolled loop: 13 % more
    // VALU work, 55 vs 48 us); left to itself the compiler then pairs the
    // operand reads of blocks kk and kk + 1 into conflicting ds_read2_b64
    // (4.7 M conflict cycles for M=512 x 2048x6144), which the clobber below
    // prevents (down 42.0-42.3 vs 42.6 us)
    constexpr int UNR = W32 ? ZG_GEMM_UNR32 : BM == 64 ? ZG_GEMM_UNR64 : 4;
#pragma unroll UNR
    for (int kk = 0; kk < BK; kk++) {
      if constexpr (W32) {
        // lane: operand row r32, bytes 16 h32..16 h32 + 15 of the block (the
        // same K order in both operands, so the dot is the block's)
        const v4i av = *reinterpret_cast<const v4i*>(A + (wm + r32) * R + kk * 32 + h32 * 16);
        const v4i bv = *reinterpret_cast<const v4i*>(B + (wn + r32) * R + kk * 32 + h32 * 16);
        float4 da[4];
#pragma unroll
        for (int g = 0; g < 4; g++) da[g] = *reinterpret_cast<const float4*>(&Ad[buf][kk * BM + wm + 8 * g + 4 * h32]);
        const float db = Bd[buf][kk * kBN + wn + r32];
        const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0},
                                                             0, 0, 0);
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float dag[4] = {da[g].x, da[g].y, da[g].z, da[g].w};
#pragma unroll
          for (int r = 0; r < 4; r++) acc[4 * g + r] = fmaf(__fmul_rn(dag[r], db), (float)c[4 * g + r], acc[4 * g + r]);
        }
        continue;
      }
      // the 32-row tile: no pairing of LDS reads across blocks
      if constexpr (BM == 32) asm volatile("" ::: "memory");
      long av[MI], bv[NJ];
      float4 da[MI];
      float db[NJ];
#pragma unroll
      for (int i = 0; i < MI; i++) {
        av[i] = *reinterpret_cast<const long*>(A + (wm + 16 * i + r16) * R + kk * 32 + kq);
        da[i] = *reinterpret_cast<const float4*>(&Ad[buf][kk * BM + wm + 16 * i + rq]);
      }
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        bv[j] = *reinterpret_cast<const long*>(B + (wn + 16 * j + r16) * R + kk * 32 + kq);
        db[j] = Bd[buf][kk * kBN + wn + 16 * j + r16];
      }
      v4i c[MI][NJ];
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) c[i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[i], bv[j], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const float dai[4] = {da[i].x, da[i].y, da[i].z, da[i].w};
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            acc[(i * NJ + j) * 4 + r] = fmaf(__fmul_rn(dai[r], db[j]), (float)c[i][j][r], acc[(i * NJ + j) * 4 + r]);
      }
    }
    if (st + 1 < nst) gemm_stage_store<WT, BM, BK>(S, As[buf ^ 1], Bs[buf ^ 1], Ad[buf ^ 1], Bd[buf ^ 1], tid);
    __syncthreads();
  };
  int st = 0;
  for (; st + 2 <= nst; st += 2) {
    stage(std::integral_constant<int, 0>{}, st);
    stage(std::integral_constant<int, 1>{}, st + 1);
  }
  if (st < nst) stage(std::integral_constant<int, 0>{}, st);
  // D layout of v_mfma_*_16x16*: lane l holds rows 4*(l/16)+r, column l%16;
  // of v_mfma_*_32x32*: element 4g+r of lane l is row 8g+4*(l/32)+r, column
  // l%32.  Stored through the L2 (M=512 x 6144x2048: 28.3 against 29.4 us).
#pragma unroll
  for (int e = 0; e < NACC; e++) {
    const int gm = m0 + wm + (W32 ? 8 * (e >> 2) + 4 * h32 + (e & 3) : 16 * (e / (NJ * 4)) + rq + (e & 3));
    const int gn = n0 + wn + (W32 ? r32 : 16 * ((e >> 2) % NJ) + r16);
    if (gm < a.m && gn < ns) {
      float* o = y + (size_t)gm * ns + gn;
      store_out(o, a.accumulate ? *o + acc[e] : acc[e]);
    }
  }
}

}  // namespace zg

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

static hipStream_t qstream(zg_ctx* ctx, void* s) { return s ? reinterpret_cast<hipStream_t>(s) : ctx->stream; }

static zg_status launch_quant(zg_ctx* ctx, const float* x, uint8_t* blocks, int8_t* qs, uint16_t* d, size_t rows,
                              size_t k, void* stream) {
  if (!x || (!blocks && !qs && !d)) return set_error(ctx, ZG_ERR_INVALID_ARG, "quantize: null pointer");
  if (k == 0 || k % 32) return set_error(ctx, ZG_ERR_INVALID_ARG, "quantize: k %% 32 != 0");
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (qs && (reinterpret_cast<uintptr_t>(qs) & 15)) ||
      (blocks && (reinterpret_cast<uintptr_t>(blocks) & 1)) || (d && (reinterpret_cast<uintptr_t>(d) & 1)))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "quantize: misaligned buffer");
  if (rows == 0) return ZG_OK;
  QuantArgs a{x, blocks, qs, d, rows, k};
  const size_t n = rows * (k / 32);
  hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, qstream(ctx, stream), a);
  return hip_check(ctx, hipGetLastError(), "quantize launch");
}

extern "C" zg_status zg_quantize_q8_0_dev(zg_ctx* ctx, const float* d_x, void* d_q, size_t rows, size_t k,
                                         void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  return launch_quant(ctx, d_x, static_cast<uint8_t*>(d_q), nullptr, nullptr, rows, k, stream);
}

extern "C" zg_status zg_quantize_q8_0_split_dev(zg_ctx* ctx, const float* d_x, int8_t* d_qs, uint16_t* d_d,
                                               size_t rows, size_t k, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_qs || !d_d) return set_error(ctx, ZG_ERR_INVALID_ARG, "quantize: null output");
  return launch_quant(ctx, d_x, nullptr, d_qs, d_d, rows, k, stream);
}

static int gemm_cu_count() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

// blocks per stage of the 64-row tile (M=512 x 6144x2048: 33.0 us at 4,
// 40.2 us at 8; the 32-row tile's 8 against 4 or 16: 42.9 / 42.7 / 42.9 us)
#ifndef ZG_GEMM_BK64
#define ZG_GEMM_BK64 4
#endif
#ifndef ZG_GEMM_SMALL_BK
#define ZG_GEMM_SMALL_BK 8
#endif
constexpr int kSmallBK = ZG_GEMM_SMALL_BK;  // blocks per stage of the 32-row tile
#ifndef ZG_GEMM_XCD_RECT
#define ZG_GEMM_XCD_RECT 1
#endif
// the 32-row tile with eight waves of 16 x 16 outputs and 8-block stages
// (twice the waves per SIMD of the four-wave tile)
#ifndef ZG_GEMM_W8
#define ZG_GEMM_W8 1
#endif
#ifndef ZG_GEMM_W8S
#define ZG_GEMM_W8S 1
#endif

// Every tile full (m a multiple of the tile rows, each segment's width a
// multiple of 64, k a whole number of stages): the kernel form with
// unguarded loads.
// XCD rectangles for a grid of gx x gy tiles (gx a multiple of 8): of the
// rx x ry (rx dividing gx, eight rectangles covering the grid) the one whose
// activation rows and weight columns are the fewest bytes, when that is
// fewer than the plain order's share (column tiles j, j + 8, ... of every
// row tile); else 0 x 0, the plain order.  wb: weight bytes per element.
static void gemm_rects(GemmArgs& a, int gx, int gy, int bm, double wb) {
  a.rx = a.ry = 0;
  if (!ZG_GEMM_XCD_RECT || (long)gx * gy % 8 || gx % 8) return;
  const double xrow = 1.0625 * a.k * bm, wcol = wb * a.k * kBN;  // bytes of a row tile / column tile
  double best = (double)gy * xrow + (double)(gx / 8) * wcol;    // plain order
  for (int rx = 1; rx <= gx; rx++) {
    if (gx % rx) continue;
    const int nx = gx / rx;
    if (8 % nx || gy % (8 / nx)) continue;
    const int ry = gy / (8 / nx);
    const double bytes = (double)ry * xrow + (double)rx * wcol;
    if (bytes < best) {
      best = bytes;
      a.rx = rx;
      a.ry = ry;
    }
  }
}

template <uint32_t WT, int IL, int BM, int BK, int NT>
static void launch_gemm(GemmArgs a, hipStream_t st) {
  const dim3 grid((unsigned)((a.n + kBN - 1) / kBN), (unsigned)((a.m + BM - 1) / BM));
  gemm_rects(a, (int)grid.x, (int)grid.y, BM, WT == Q4_0 ? 0.5625 : 1.0625);
  // every tile whole, and every byte offset from a stage base under 2^31
  bool full = a.m % BM == 0 && (a.k / 32) % BK == 0 && (size_t)a.m * (size_t)a.k < ((size_t)1 << 31);
  for (int i = 0, lo = 0; i < a.nseg; lo = a.seg_end[i], i++)
    full = full && (a.seg_end[i] - lo) % kBN == 0 && (size_t)(a.seg_end[i] - lo) * (size_t)(a.k / 32) * 34 < ((size_t)1 << 31);
  if (full) hipLaunchKernelGGL((gemm_q8act_kernel<WT, IL, BM, BK, true, NT>), grid, dim3(NT), 0, st, a);
  else hipLaunchKernelGGL((gemm_q8act_kernel<WT, IL, BM, BK, false, NT>), grid, dim3(NT), 0, st, a);
}

// the weight type and layout (1 plain rows, 4 X4, 5 split-scale X4)
template <int BM, int BK, int NT = 256>
static void launch_gemm_il(GemmArgs& a, uint32_t w_type, uint32_t il, hipStream_t st) {
  if (w_type == ZG_Q4_0) {
    if (il == 4) launch_gemm<Q4_0, 4, BM, BK, NT>(a, st);
    else if (il == 5) launch_gemm<Q4_0, 5, BM, BK, NT>(a, st);
    else launch_gemm<Q4_0, 1, BM, BK, NT>(a, st);
  } else {
    if (il == 4) launch_gemm<Q8_0, 4, BM, BK, NT>(a, st);
    else if (il == 5) launch_gemm<Q8_0, 5, BM, BK, NT>(a, st);
    else launch_gemm<Q8_0, 1, BM, BK, NT>(a, st);
  }
}

// Checks and launches one Q8_0-activation GEMM over 1..3 weight segments.
zg_status zg::run_gemm(zg_ctx* ctx, const int8_t* qs, const uint16_t* xd, const GemmSegDev* segs, int nseg, size_t m,
                       size_t k, uint32_t w_type, uint32_t interleave, bool accumulate, hipStream_t st) {
  if (!qs || !xd || !segs || nseg < 1 || nseg > kGemmSegs) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm: bad arguments");
  if (w_type != ZG_Q4_0 && w_type != ZG_Q8_0) return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "gemm: weights must be Q4_0/Q8_0");
  if (reinterpret_cast<uintptr_t>(qs) & 15) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm: activations misaligned");
  GemmArgs a{};
  a.xq = qs;
  a.xd = xd;
  size_t n = 0;
  for (int i = 0; i < nseg; i++) {
    if (!segs[i].w || !segs[i].y) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm: null pointer");
    zg_status s = check_shape(ctx, w_type, interleave, k, segs[i].n);
    if (s) return s;
    if (nseg > 1 && segs[i].n % kBN) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm: segment width %% %d", kBN);
    if (interleave != 1 && (reinterpret_cast<uintptr_t>(segs[i].w) & 7))
      return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm: weights misaligned");
    n += segs[i].n;
    a.w[i] = segs[i].w;
    a.y[i] = segs[i].y;
    a.seg_end[i] = (int)n;
  }
  if (m == 0) return ZG_OK;
  if (m > (size_t)INT32_MAX || n > (size_t)INT32_MAX) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm: shape too large");
  for (int i = nseg; i < kGemmSegs; i++) {
    a.w[i] = a.w[0];
    a.y[i] = a.y[0];
    a.seg_end[i] = (int)n;
  }
  a.nseg = nseg;
  a.accumulate = accumulate ? 1 : 0;
  a.m = (int)m;
  a.n = (int)n;
  a.k = (int)k;
  // 64-row tiles unless they would not give every CU three workgroups
  const size_t tiles64 = ((n + kBN - 1) / kBN) * ((m + 63) / 64);
  if (tiles64 >= (size_t)3 * gemm_cu_count()) {
    launch_gemm_il<64, ZG_GEMM_BK64>(a, w_type, interleave, st);
  } else if (((n + kBN - 1) / kBN) * ((m + 31) / 32) <= (size_t)gemm_cu_count()) {
    // at most one 32-row tile per CU: each stage's round trip is exposed,
    // so fewer, larger stages
    if (ZG_GEMM_W8S) launch_gemm_il<32, 8, 512>(a, w_type, interleave, st);
    else launch_gemm_il<32, kSmallBK>(a, w_type, interleave, st);
  } else {
    if (ZG_GEMM_W8) launch_gemm_il<32, 8, 512>(a, w_type, interleave, st);
    else launch_gemm_il<32, 4>(a, w_type, interleave, st);
  }
  return hip_check(ctx, hipGetLastError(), "gemm launch");
}

extern "C" zg_status zg_gemm_q8act_dev(zg_ctx* ctx, const int8_t* d_qs, const uint16_t* d_d, const void* d_w,
                                      float* d_y, size_t m, size_t n, size_t k, uint32_t w_type, uint32_t interleave,
                                      void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_qs || !d_d || !d_w || !d_y) return set_error(ctx, ZG_ERR_INVALID_ARG, "gemm: null pointer");
  const GemmSegDev seg{static_cast<const uint8_t*>(d_w), d_y, n};
  return run_gemm(ctx, d_qs, d_d, &seg, 1, m, k, w_type, interleave, false, qstream(ctx, stream));
}
