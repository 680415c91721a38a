// zg_gemv.hip -- decode-time GEMV kernels for gfx950.
//
// Replaces the AVX-512 row-range kernels of the reference
// (kernel/src/arch/x86_64/math/linear.rs:150,352,710,909,1096,1271) and the
// SMP row partitioning that fans them out (kernel/src/smp.rs:1567-1712):
// output rows map to the launch grid instead of to cores.
//
// Fast path (X4 pair kernel): .smodel-v2 Q4_0X4 / Q8_0X4 tensors whose
// blocks-per-row is even.  Two consecutive 4-row group-blocks (2 x 72 B or
// 2 x 136 B) form a 16-byte aligned "pair" that a lane fetches with
// 9 (Q4_0) or 17 (Q8_0) 128-bit loads.  The activation vector is staged in
// LDS once per workgroup (after the lane's first weight loads are already in
// flight) and broadcast from there; nibbles/bytes are unpacked in registers
// (v_cvt_f32_ubyte*), each block sum is scaled by its fp16 d once, and the
// LPG lanes that share a group finish with a butterfly reduction.  No MFMA:
// the GEMV is HBM-bound.
//
// Generic path: any layout / block type, one wave per output row, byte
// loads.  Used for plain Q4_0/Q8_0, odd blocks-per-row and as the first
// Q4_K/Q6_K implementation.
#include "zg_device.h"
#include "zg_kernels.h"

namespace zg {

// ---------------------------------------------------------------------------
// Prologue: how the kernel forms the activation vector in LDS.
// ---------------------------------------------------------------------------

// Stage x (K floats) into LDS, applying the prologue.  rmsnorm follows
// ops.rs:29-52: x * (1/sqrt(mean(x^2)+eps)) * w.
template <int PRO, int NT>
__device__ __forceinline__ void stage_x(float* xs, float* red, const GemvArgs& a) {
  const int tid = threadIdx.x;
  const int K = a.k;
  const float4* x4 = reinterpret_cast<const float4*>(a.x);
  float ssq = 0.0f;
  for (int i = tid; i < K / 4; i += NT) {
    const float4 v = x4[i];
    reinterpret_cast<float4*>(xs)[i] = v;
    if (PRO == PRO_RMSNORM) ssq += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  if (PRO == PRO_RMSNORM) {
    ssq = seg_sum<64>(ssq);
    if ((tid & 63) == 0) red[tid >> 6] = ssq;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < NT / 64; i++) tot += red[i];
    const float rinv = 1.0f / sqrtf(tot / (float)K + a.eps);
    for (int i = tid; i < K; i += NT) xs[i] = xs[i] * rinv * a.norm_w[i];
  }
}

// ---------------------------------------------------------------------------
// X4 pair kernel.
//   QT = Q4_0 or Q8_0;  LPG = lanes per 4-row group (power of 2, <= 64);
//   NW = waves per workgroup.
// Group g of segment s covers rows 4g..4g+3 of that segment; a lane owns
// pairs p = lane_in_group, +LPG, ... (blocks 2p, 2p+1) of its group.
// ---------------------------------------------------------------------------
template <uint32_t QT>
struct X4 {
  static constexpr int GB = (QT == Q4_0) ? 72 : 136;  // group-block bytes
  static constexpr int PU4 = (2 * GB) / 16;            // uint4 per pair: 9 or 17
  static constexpr int BDW = GB / 4;                   // dwords per group-block
  static constexpr int QDW = (QT == Q4_0) ? 4 : 8;     // qs dwords per row
};

// Sum over one Q4_0 block of row r: returns sum_j q_j * x_j with q the raw
// nibble (0..15); the caller applies d * (s - 8 * sum(x)).  Low nibbles of
// byte j are element j, high nibbles element j+16 (dequant.rs:186-216).
// High nibbles are masked in place (value 16*q) and rescaled by 1/16, an
// exact power-of-two scaling.
__device__ __forceinline__ float q4_block_dot(const uint32_t* qs, const float4* xb) {
  float s_lo = 0.0f, s_hi = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const uint32_t v = qs[c];
    const uint32_t lo = v & 0x0F0F0F0Fu;
    const uint32_t hi = v & 0xF0F0F0F0u;
    const float4 xl = xb[c];
    const float4 xh = xb[4 + c];
    s_lo = fmaf(xl.x, (float)(lo & 0xFFu), s_lo);
    s_lo = fmaf(xl.y, (float)((lo >> 8) & 0xFFu), s_lo);
    s_lo = fmaf(xl.z, (float)((lo >> 16) & 0xFFu), s_lo);
    s_lo = fmaf(xl.w, (float)(lo >> 24), s_lo);
    s_hi = fmaf(xh.x, (float)(hi & 0xFFu), s_hi);
    s_hi = fmaf(xh.y, (float)((hi >> 8) & 0xFFu), s_hi);
    s_hi = fmaf(xh.z, (float)((hi >> 16) & 0xFFu), s_hi);
    s_hi = fmaf(xh.w, (float)(hi >> 24), s_hi);
  }
  return fmaf(s_hi, 0.0625f, s_lo);
}

// Sum over one Q8_0 block of row r: sum_j q_j * x_j, q signed bytes
// (dequant.rs:247-275).
__device__ __forceinline__ float q8_block_dot(const uint32_t* qs, const float4* xb) {
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; c++) {
    const uint32_t v = qs[c];
    const float4 xv = xb[c];
    float& s = (c & 1) ? s1 : s0;
    s = fmaf(xv.x, (float)(int32_t)((int8_t)(v & 0xFFu)), s);
    s = fmaf(xv.y, (float)(int32_t)((int8_t)((v >> 8) & 0xFFu)), s);
    s = fmaf(xv.z, (float)(int32_t)((int8_t)((v >> 16) & 0xFFu)), s);
    s = fmaf(xv.w, (float)(int32_t)((int8_t)(v >> 24)), s);
  }
  return s0 + s1;
}

template <uint32_t QT, int LPG, int NW, int PRO, int EPI>
__global__ __launch_bounds__(NW * 64) void gemv_x4_pair_kernel(GemvArgs a) {
  constexpr int NT = NW * 64;
  constexpr int GPW = 64 / LPG;
  constexpr int PU4 = X4<QT>::PU4;
  constexpr int BDW = X4<QT>::BDW;
  constexpr int QDW = X4<QT>::QDW;
  extern __shared__ float smem[];
  float* xs = smem;             // K floats
  float* sx = smem + a.k;       // K/32 block sums (Q4_0 only)
  __shared__ float red[NW];
  __shared__ uint64_t wbest[NW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lig = lane % LPG;
  const uint32_t group = (blockIdx.x * NW + wave) * GPW + lane / LPG;
  const bool active = group < a.total_groups;

  // Locate the segment owning this group (<= 3 segments, fused Q|K|V).
  // SwiGLU mode interleaves two equal segments group by group (gate g, up
  // g, gate g+1, ...) so one wave holds matching gate and up rows.
  int s = 0;
  uint32_t lg;
  if (EPI == EPI_SWIGLU) {
    s = (int)(group & 1u);
    lg = group >> 1;
  } else {
    if (a.nseg > 1 && group >= a.seg[1].g_begin) s = 1;
    if (a.nseg > 2 && group >= a.seg[2].g_begin) s = 2;
    lg = group - a.seg[s].g_begin;
  }
  const GemvSeg& sg = a.seg[s];
  const int nb = a.k / 32;
  const int npairs = nb / 2;
  const u32x4* gp = reinterpret_cast<const u32x4*>(sg.w + (size_t)lg * (size_t)nb * X4<QT>::GB);

  // Issue the first pair's loads before staging x so that HBM latency
  // overlaps the LDS staging.
  u32x4 cur[PU4];
  if (active && lig < npairs) {
#pragma unroll
    for (int i = 0; i < PU4; i++) cur[i] = __builtin_nontemporal_load(gp + (size_t)lig * PU4 + i);
  }

  stage_x<PRO, NT>(xs, red, a);
  __syncthreads();
  if (QT == Q4_0) {
    for (int b = tid; b < nb; b += NT) {
      const float4* xb = reinterpret_cast<const float4*>(xs + 32 * b);
      float t = 0.0f;
#pragma unroll
      for (int c = 0; c < 8; c++) {
        const float4 v = xb[c];
        t += (v.x + v.y) + (v.z + v.w);
      }
      sx[b] = t;
    }
    __syncthreads();
  }

  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (active) {
    for (int p = lig; p < npairs; p += LPG) {
      u32x4 nxt[PU4];
      const bool more = (p + LPG) < npairs;
      if (more) {
#pragma unroll
        for (int i = 0; i < PU4; i++)
          nxt[i] = __builtin_nontemporal_load(gp + (size_t)(p + LPG) * PU4 + i);
      }
      const uint32_t* dw = reinterpret_cast<const uint32_t*>(cur);
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int kb = 2 * p + h;
        const float4* xb = reinterpret_cast<const float4*>(xs + 32 * kb);
        const uint32_t* blk = dw + h * BDW;
        float d[4];
        d[0] = half_bits_to_f32(blk[0]);
        d[1] = half_bits_to_f32(blk[0] >> 16);
        d[2] = half_bits_to_f32(blk[1]);
        d[3] = half_bits_to_f32(blk[1] >> 16);
        if (QT == Q4_0) {
          const float m8 = -8.0f * sx[kb];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float t = q4_block_dot(blk + 2 + QDW * r, xb);
            acc[r] = fmaf(d[r], t + m8, acc[r]);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float t = q8_block_dot(blk + 2 + QDW * r, xb);
            acc[r] = fmaf(d[r], t, acc[r]);
          }
        }
      }
      if (more) {
#pragma unroll
        for (int i = 0; i < PU4; i++) cur[i] = nxt[i];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; r++) acc[r] = seg_sum<LPG>(acc[r]);

  // Every lane of the group holds all four row sums; row r is stored by
  // lane r % LPG of the group (one row per lane when LPG >= 4).
  uint64_t key = 0;
  float up[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (EPI == EPI_SWIGLU) {
    // up rows of the same local group sit LPG lanes higher (next group)
#pragma unroll
    for (int r = 0; r < 4; r++) up[r] = __shfl(acc[r], (lane + LPG) & 63, 64);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t row = 4 * lg + (uint32_t)r;
    const bool owner = active && lig == (r & (LPG - 1)) && row >= sg.row_lo && row < sg.row_hi;
    if (!owner) continue;
    const float v = acc[r];
    if (EPI == EPI_SWIGLU) {
      // activation.rs:115-148 operand order: silu = g/(1+exp(-g)), then *up
      if (s == 0) sg.y[row] = (v / (1.0f + expf(-v))) * up[r];
    } else if (EPI == EPI_RESID) {
      sg.y[row] = sg.resid[row] + v;
    } else {
      if (sg.y) sg.y[row] = v;
      if (EPI == EPI_ARGMAX && !(v != v)) {
        const uint64_t kk = argmax_key(v, row);
        key = kk > key ? kk : key;
      }
    }
  }
  if (EPI == EPI_ARGMAX) {
    // wave max, then workgroup max, then one global atomic per workgroup
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t other = __shfl_xor(key, o, 64);
      key = other > key ? other : key;
    }
    if (lane == 0) wbest[wave] = key;
    __syncthreads();
    if (tid == 0) {
      uint64_t b = 0;
#pragma unroll
      for (int i = 0; i < NW; i++) b = wbest[i] > b ? wbest[i] : b;
      if (b) atomicMax(reinterpret_cast<unsigned long long*>(a.best), (unsigned long long)b);
    }
  }
}

// ---------------------------------------------------------------------------
// Generic kernel: one wave per output row, any (type, layout).  Dequantizes
// each element with the reference's operation order (bit-exact weights) and
// accumulates x*w with fmaf.
// ---------------------------------------------------------------------------
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

__global__ __launch_bounds__(256) void gemv_generic_kernel(GenericArgs a) {
  const int lane = threadIdx.x & 63;
  const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6) + a.row_lo;
  const bool active = row < a.row_hi;
  const int be = (a.qt == Q4_0 || a.qt == Q8_0) ? 32 : 256;
  const size_t nb = a.k / be;
  float acc = 0.0f;
  if (active) {
    for (size_t b = lane; b < nb; b += 64) {
      const BlockRef br = block_ref(a.w, a.qt, a.il, row, b, nb);
      const float d = (a.qt == Q4_0 || a.qt == Q8_0) ? rd_half(br.d) : 0.0f;
      const float* xb = a.x + b * be;
      for (int e = 0; e < be; e++) acc = fmaf(xb[e], deq_elem(br, a.qt, d, e), acc);
    }
  }
  acc = seg_sum<64>(acc);
  uint64_t key = 0;
  if (active && lane == 0) {
    if (a.epi == EPI_RESID) a.y[row] = a.resid[row] + acc;
    else if (a.y) a.y[row] = acc;
    if (a.epi == EPI_ARGMAX && !(acc != acc)) key = argmax_key(acc, (uint32_t)row);
  }
  if (a.epi == EPI_ARGMAX && lane == 0 && key)
    atomicMax(reinterpret_cast<unsigned long long*>(a.best), (unsigned long long)key);
}

// Dequantize a whole tensor: one thread per (row, block).  Uses the same
// element mapping and operation order as the generic kernel.
__global__ void dequant_kernel(DequantArgs a) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int be = (a.qt == Q4_0 || a.qt == Q8_0) ? 32 : 256;
  const size_t nb = a.k / be;
  if (t >= a.rows * nb) return;
  const size_t row = t / nb, b = t % nb;
  const BlockRef br = block_ref(a.w, a.qt, a.il, row, b, nb);
  const float d = (a.qt == Q4_0 || a.qt == Q8_0) ? rd_half(br.d) : 0.0f;
  float* o = a.out + row * a.k + b * be;
  for (int e = 0; e < be; e++) o[e] = deq_elem(br, a.qt, d, e);
}

// Dequantize X4 tensors through the pair kernel's own register mapping
// (one lane per pair), so the fast path's byte->element map is checked
// bit for bit.
template <uint32_t QT>
__global__ void dequant_x4_pair_kernel(DequantArgs a) {
  constexpr int PU4 = X4<QT>::PU4, BDW = X4<QT>::BDW, QDW = X4<QT>::QDW;
  const size_t nb = a.k / 32, npairs = nb / 2;
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (a.rows / 4) * npairs) return;
  const size_t g = t / npairs, p = t % npairs;
  const u32x4* gp = reinterpret_cast<const u32x4*>(a.w + g * nb * X4<QT>::GB);
  u32x4 cur[PU4];
#pragma unroll
  for (int i = 0; i < PU4; i++) cur[i] = gp[p * PU4 + i];
  const uint32_t* dw = reinterpret_cast<const uint32_t*>(cur);
  for (int h = 0; h < 2; h++) {
    const uint32_t* blk = dw + h * BDW;
    for (int r = 0; r < 4; r++) {
      const float d = half_bits_to_f32(blk[r >> 1] >> (16 * (r & 1)));
      float* o = a.out + (4 * g + r) * a.k + (2 * p + h) * 32;
      const uint32_t* qs = blk + 2 + QDW * r;
      for (int e = 0; e < 32; e++) {
        float v;
        if (QT == Q4_0) {
          const uint32_t word = qs[(e & 15) >> 2];
          const uint32_t nib = (e < 16) ? ((word >> (8 * (e & 3))) & 0xF) : ((word >> (8 * (e & 3) + 4)) & 0xF);
          v = (float)((int)nib - 8) * d;
        } else {
          const uint32_t word = qs[e >> 2];
          v = (float)(int8_t)((word >> (8 * (e & 3))) & 0xFF) * d;
        }
        o[e] = v;
      }
    }
  }
}

__global__ void fp16_kernel(const uint16_t* in, float* out, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = half_bits_to_f32(in[i]);
}

__global__ void fill_u64_kernel(uint64_t* p, uint64_t v) { *p = v; }

// ---------------------------------------------------------------------------
// Host-side launchers.
// ---------------------------------------------------------------------------

template <uint32_t QT, int LPG, int NW, int PRO, int EPI>
static hipError_t launch_pair(const GemvArgs& a, hipStream_t st) {
  constexpr int GPB = NW * (64 / LPG);
  const uint32_t grid = (a.total_groups + GPB - 1) / GPB;
  const size_t shm = (size_t)a.k * sizeof(float) + (QT == Q4_0 ? (size_t)(a.k / 32) * sizeof(float) : 0);
  hipLaunchKernelGGL((gemv_x4_pair_kernel<QT, LPG, NW, PRO, EPI>), dim3(grid), dim3(NW * 64), shm, st, a);
  return hipGetLastError();
}

template <uint32_t QT, int PRO, int EPI>
static hipError_t pick_lpg(const GemvArgs& a, hipStream_t st) {
  // Lanes per group: enough lanes that every lane owns at least one pair,
  // up to 32 (two groups per wave keep the reduction short).
  const int npairs = a.k / 64;
  // SwiGLU pairs two groups per wave, so LPG <= 32 always holds here.
  if (npairs >= 32) return launch_pair<QT, 32, 4, PRO, EPI>(a, st);
  if (npairs >= 16) return launch_pair<QT, 16, 4, PRO, EPI>(a, st);
  if (npairs >= 8) return launch_pair<QT, 8, 4, PRO, EPI>(a, st);
  if (npairs >= 4) return launch_pair<QT, 4, 4, PRO, EPI>(a, st);
  if (npairs >= 2) return launch_pair<QT, 2, 4, PRO, EPI>(a, st);
  return launch_pair<QT, 1, 4, PRO, EPI>(a, st);
}

template <uint32_t QT>
static hipError_t dispatch_pair_qt(const GemvArgs& a, int pro, int epi, hipStream_t st) {
  if (pro == PRO_PLAIN && epi == EPI_STORE) return pick_lpg<QT, PRO_PLAIN, EPI_STORE>(a, st);
  if (pro == PRO_PLAIN && epi == EPI_RESID) return pick_lpg<QT, PRO_PLAIN, EPI_RESID>(a, st);
  if (pro == PRO_PLAIN && epi == EPI_ARGMAX) return pick_lpg<QT, PRO_PLAIN, EPI_ARGMAX>(a, st);
  if (pro == PRO_RMSNORM && epi == EPI_STORE) return pick_lpg<QT, PRO_RMSNORM, EPI_STORE>(a, st);
  if (pro == PRO_RMSNORM && epi == EPI_ARGMAX) return pick_lpg<QT, PRO_RMSNORM, EPI_ARGMAX>(a, st);
  if (pro == PRO_RMSNORM && epi == EPI_SWIGLU) return pick_lpg<QT, PRO_RMSNORM, EPI_SWIGLU>(a, st);
  if (pro == PRO_PLAIN && epi == EPI_SWIGLU) return pick_lpg<QT, PRO_PLAIN, EPI_SWIGLU>(a, st);
  return hipErrorInvalidValue;
}

hipError_t launch_gemv_x4_pair(const GemvArgs& a, uint32_t qt, int pro, int epi, hipStream_t st) {
  if (qt == Q4_0) return dispatch_pair_qt<Q4_0>(a, pro, epi, st);
  if (qt == Q8_0) return dispatch_pair_qt<Q8_0>(a, pro, epi, st);
  return hipErrorInvalidValue;
}

hipError_t launch_gemv_generic(const GenericArgs& a, hipStream_t st) {
  const size_t rows = a.row_hi - a.row_lo;
  if (rows == 0) return hipSuccess;
  const uint32_t grid = (uint32_t)((rows + 3) / 4);
  hipLaunchKernelGGL(gemv_generic_kernel, dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_dequant(const DequantArgs& a, bool pair_path, hipStream_t st) {
  if (pair_path && (a.qt == Q4_0 || a.qt == Q8_0)) {
    const size_t n = (a.rows / 4) * (a.k / 64);
    const uint32_t grid = (uint32_t)((n + 255) / 256);
    if (a.qt == Q4_0) hipLaunchKernelGGL(dequant_x4_pair_kernel<Q4_0>, dim3(grid), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(dequant_x4_pair_kernel<Q8_0>, dim3(grid), dim3(256), 0, st, a);
    return hipGetLastError();
  }
  const int be = (a.qt == Q4_0 || a.qt == Q8_0) ? 32 : 256;
  const size_t n = a.rows * (a.k / be);
  const uint32_t grid = (uint32_t)((n + 255) / 256);
  hipLaunchKernelGGL(dequant_kernel, dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_fp16(const uint16_t* in, float* out, size_t n, hipStream_t st) {
  const uint32_t grid = (uint32_t)((n + 255) / 256);
  hipLaunchKernelGGL(fp16_kernel, dim3(grid), dim3(256), 0, st, in, out, n);
  return hipGetLastError();
}

hipError_t launch_fill_u64(uint64_t* p, uint64_t v, hipStream_t st) {
  hipLaunchKernelGGL(fill_u64_kernel, dim3(1), dim3(1), 0, st, p, v);
  return hipGetLastError();
}

}  // namespace zg
