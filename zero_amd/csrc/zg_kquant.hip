// zg_kquant.hip -- Q4_K and Q6_K GEMV for gfx950.
//
// Replaces linear_q4k_avx512_range and linear_q6k_avx512_range
// (kernel/src/arch/x86_64/math/linear.rs:150-306, 352-504) and their SMP
// row split.  Both are HBM-bound dequant-dot GEMVs over 256-element
// superblocks (Q4_K: 144 bytes, Q6_K: 210 bytes, row-major).
//
// Layout of the work: a wave reduces whole rows.  One wave step covers 8
// consecutive superblocks of a row with 8 lanes per superblock; each lane
// loads its own bytes with 128-bit loads (the 8 lanes of a superblock read
// adjacent 16-byte pieces, so one wave instruction touches ~1.1-1.7 KB of
// consecutive bytes) and decodes 32 elements in registers.  The workgroup
// stages the activation vector in LDS once, together with its 16-element
// partial sums, which carry the per-sub-block min / offset terms:
//   Q4_K  sum_i x_i (d sc q_i - dmin m) = d sc sum_i q_i x_i - dmin m sum_i x_i
//   Q6_K  sum_i x_i (d sc)(q_i - 32)    = (d sc) (sum_i q_i x_i - 32 sum_i x_i)
// The dequantized weights are the reference's (dequant.rs:98-138,328-355);
// the dot products are regrouped per sub-block, which changes only the
// rounding of the sums (bounded by the rel 1e-3 parity bar).
// Waves loop persistently over rows; the row result is a wave-wide DPP sum.
#include "zg_device.h"
#include "zg_kernels.h"

namespace zg {

constexpr int kKqWaves = 8;  // waves per workgroup

__device__ __forceinline__ uint32_t byte_of(const uint32_t* w, int i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xFFu; }


// Stage x (k floats) and its 16-element sums into LDS.
__device__ __forceinline__ void stage_x_kq(float* xs, float* x16, const float* x, int k) {
  const float4* x4 = reinterpret_cast<const float4*>(x);
  for (int t = threadIdx.x; t < k / 16; t += kKqWaves * 64) {
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float4 v = x4[4 * t + c];
      reinterpret_cast<float4*>(xs)[4 * t + c] = v;
      s += (v.x + v.y) + (v.z + v.w);
    }
    x16[t] = s;
  }
}

template <uint32_t QT>
struct KqGeom;
template <>
struct KqGeom<Q4K> {
  static constexpr int BB = 144;
};
template <>
struct KqGeom<Q6K> {
  static constexpr int BB = 210;
};

// One lane's share of one superblock (32 elements): its bytes are loaded
// first (kq_load) and decoded later (kq_dot), so that a wave keeps the next
// unit's loads in flight while it computes the current one.
//
// Q4_K lane (j = sub-block pair 0..3, h = half 0..1): qs bytes
// [32j + 16h, +16): low nibbles are elements 64j + 16h + i (sub-block 2j),
// high nibbles elements 64j + 32 + 16h + i (sub-block 2j+1).
//
// Q6_K lane (n = half 0..1, is = 0..1, qp = quarter pair 0..1): l in
// [16 is, 16 is + 16) of half n, quarters Q = 2 qp and 2 qp + 1
// (dequant.rs:328-355 element map: quarter Q of l is element 128n + l + 32Q,
// low 4 bits from ql[l] (Q even) or ql[l+32] (Q odd), nibble selected by
// Q >= 2, high 2 bits qh[l] >> 2Q, scale sc[8n + is + 2Q]).
template <uint32_t QT>
struct KqLane;
template <>
struct KqLane<Q4K> {
  u32x4 hdr, q;
};
template <>
struct KqLane<Q6K> {
  u32x4 la, lb, hb;
  uint32_t sc0, sc1;  // scales sc[8n .. 8n+7] of the lane's half
  uint32_t d;
};

// Weight loads allocate in the caches (nontemporal loads measured slower
// here: 14.8 vs 13.6 us for Q4_K 14336x4096).  Q6_K fields sit at any even
// offset: the 2-byte-aligned vector types still give single dwordx4 /
// dwordx2 loads (unaligned access mode).
typedef uint32_t u32x4a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32x2a2 __attribute__((ext_vector_type(2), aligned(2)));

__device__ __forceinline__ void kq_load(KqLane<Q4K>& L, const uint8_t* blk, int lane) {
  const int j = (lane >> 1) & 3, h = lane & 1;
  L.hdr = *reinterpret_cast<const u32x4*>(blk);
  L.q = *reinterpret_cast<const u32x4*>(blk + 16 + 32 * j + 16 * h);
}

__device__ __forceinline__ void kq_load(KqLane<Q6K>& L, const uint8_t* blk, int lane) {
  const int n = (lane >> 2) & 1, is = (lane >> 1) & 1;
  L.la = *reinterpret_cast<const u32x4a2*>(blk + 64 * n + 16 * is);
  L.lb = *reinterpret_cast<const u32x4a2*>(blk + 64 * n + 32 + 16 * is);
  L.hb = *reinterpret_cast<const u32x4a2*>(blk + 128 + 32 * n + 16 * is);
  const u32x2a2 scw = *reinterpret_cast<const u32x2a2*>(blk + 192 + 8 * n);
  L.sc0 = scw.x;
  L.sc1 = scw.y;
  L.d = (uint32_t)*reinterpret_cast<const uint16_t*>(blk + 208);
}

// Element offset (within the superblock) of the lane's first 16-element run;
// its second run starts 32 elements later.
template <uint32_t QT>
__device__ __forceinline__ int kq_lane_elem(int lane) {
  if (QT == Q4K) return 64 * ((lane >> 1) & 3) + 16 * (lane & 1);
  return 128 * ((lane >> 2) & 1) + 16 * ((lane >> 1) & 1) + 64 * (lane & 1);
}

// The lane's activations: runs A and B (16 values each) and their sums.
struct KqX {
  float4 a[4], b[4];
  float sa, sb;
};



__device__ __forceinline__ float kq_dot(const KqLane<Q4K>& L, const KqX& x, int lane) {
  const int j = (lane >> 1) & 3, h = lane & 1;
  const float d = kq_half(L.hdr.x), dmin = kq_half(L.hdr.x >> 16);
  // The two lanes of a sub-block pair (h = 0, 1; quad lanes 0,1 and 2,3)
  // each decode one of its sub-blocks, 2j + h, into the factors d*sc and
  // dmin*m, and take the pair's factors by DPP: sub-block 2j's from the
  // even lane (quad_perm [0,0,2,2]), 2j + 1's from the odd lane ([1,1,3,3]).
  // High nibbles stay in place (16 x the value): the 1/16 goes into
  // sub-block 2j + 1's scale (exact).  The same products as decoding both
  // sub-blocks in every lane, in the same order (8.6 % fewer VALU in the
  // 14336x4096 loop; 10.90-11.03 against 11.03-11.15 us).
  uint32_t sc, mn;
  q4k_sub_scale(L.hdr.y, L.hdr.z, L.hdr.w, 2 * j + h, sc, mn);
  const float ds = (d * (h ? 0.0625f : 1.0f)) * (float)sc, dm = dmin * (float)mn;
  const float dA = quad_pick<0xA0>(ds), mA = quad_pick<0xA0>(dm);
  const float dB = quad_pick<0xF5>(ds), mB = quad_pick<0xF5>(dm);
  const uint32_t q[4] = {L.q.x, L.q.y, L.q.z, L.q.w};
  uint32_t lo[4], hi[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    lo[c] = opaque_u32(q[c] & 0x0F0F0F0Fu);
    hi[c] = opaque_u32(q[c] & 0xF0F0F0F0u);
  }
  const float sA = u8_dot16(lo, x.a);
  const float sB = u8_dot16(hi, x.b);
  float acc = dA * sA;
  acc = fmaf(-mA, x.sa, acc);
  acc = fmaf(dB, sB, acc);
  return fmaf(-mB, x.sb, acc);
}

__device__ __forceinline__ float kq_dot(const KqLane<Q6K>& L, const KqX& x, int lane) {
  const int is = (lane >> 1) & 1, qp = lane & 1;
  const uint32_t scw[2] = {L.sc0, L.sc1};
  const int ia = is + 4 * qp, ib = ia + 2;  // sc[8n + is + 2Q] within the half's 8 scales
  const float scA = (float)(int8_t)byte_of(scw, ia), scB = (float)(int8_t)byte_of(scw, ib);
  const float d = half_bits_to_f32(L.d);
  const uint32_t a[4] = {L.la.x, L.la.y, L.la.z, L.la.w}, b[4] = {L.lb.x, L.lb.y, L.lb.z, L.lb.w},
                 hh[4] = {L.hb.x, L.hb.y, L.hb.z, L.hb.w};
  const int nsh = 4 * qp;                  // nibble select
  const int hA = 4 * qp, hB = 4 * qp + 2;  // qh shift of quarters 2qp, 2qp+1
  uint32_t qA[4], qB[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    qA[c] = opaque_u32(((a[c] >> nsh) & 0x0F0F0F0Fu) | (((hh[c] >> hA) & 0x03030303u) << 4));
    qB[c] = opaque_u32(((b[c] >> nsh) & 0x0F0F0F0Fu) | (((hh[c] >> hB) & 0x03030303u) << 4));
  }
  const float sA = u8_dot16(qA, x.a);
  const float sB = u8_dot16(qB, x.b);
  float acc = (d * scA) * fmaf(-32.0f, x.sa, sA);
  return fmaf(d * scB, fmaf(-32.0f, x.sb, sB), acc);
}

// Activations of the lane's runs in superblock sb (from LDS or global).
template <uint32_t QT>
__device__ __forceinline__ KqX kq_x(const float* x, int sb, int lane) {
  KqX r;
  const float4* p = reinterpret_cast<const float4*>(x + sb * 256 + kq_lane_elem<QT>(lane));
  float sa = 0.0f, sbs = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    r.a[c] = p[c];
    r.b[c] = p[8 + c];
  }
#pragma unroll
  for (int c = 0; c < 4; c++) {
    sa += (r.a[c].x + r.a[c].y) + (r.a[c].z + r.a[c].w);
    sbs += (r.b[c].x + r.b[c].y) + (r.b[c].z + r.b[c].w);
  }
  r.sa = sa;
  r.sb = sbs;
  return r;
}

// A wave walks units (row, step of 8 superblocks) of its rows; unit u + 1's
// loads are issued before unit u is decoded.  Loads are unconditional, with
// row and superblock indices clamped into the tensor (a clamped lane's
// result is discarded), so the compiler's wait counts stay exact.
template <uint32_t QT, int EPI>
__global__ __launch_bounds__(kKqWaves * 64) void kq_gemv_kernel(GenericArgs a) {
  constexpr int BB = KqGeom<QT>::BB;
  extern __shared__ __attribute__((aligned(16))) float kq_smem[];
  const int k = (int)a.k;
  const int lane = threadIdx.x & 63;
  const int sl = lane >> 3;  // superblock of the step
  const int nsb = k / 256;
  const int steps = (nsb + 7) / 8;
  const size_t rowbytes = (size_t)nsb * BB;
  const size_t nrows = a.row_hi - a.row_lo;
  const size_t wave_id = (size_t)blockIdx.x * kKqWaves + (threadIdx.x >> 6);
  const size_t nwaves = (size_t)gridDim.x * kKqWaves;
  const size_t my_rows = wave_id < nrows ? (nrows - wave_id + nwaves - 1) / nwaves : 0;
  const size_t nunits = my_rows * steps;
  auto unit_blk = [&](size_t u) -> const uint8_t* {
    const size_t ri = u / steps;
    const int st = (int)(u % steps);
    const size_t row = a.row_lo + wave_id + ri * nwaves;
    const int sb = min(st * 8 + sl, nsb - 1);
    return a.w + row * rowbytes + (size_t)sb * BB;
  };
  KqLane<QT> cur, nxt;
  if (nunits) kq_load(nxt, unit_blk(0), lane);
  float* xs = kq_smem;
  float* x16 = kq_smem + k;
  stage_x_kq(xs, x16, a.x, k);
  __syncthreads();
  uint64_t key = 0;
  float acc = 0.0f;
  for (size_t u = 0; u < nunits; u++) {
    cur = nxt;
    if (u + 1 < nunits) kq_load(nxt, unit_blk(u + 1), lane);
    const int st = (int)(u % steps);
    const int sb = st * 8 + sl;
    if (sb < nsb) acc += kq_dot(cur, kq_x<QT>(xs, sb, lane), lane);
    if (st == steps - 1) {
      const float v = wave_sum(acc);
      acc = 0.0f;
      const size_t row = a.row_lo + wave_id + (u / steps) * nwaves;
      if (lane == 0) {
        if (EPI == EPI_RESID)
          store_out(a.y + row, a.resid[row] + v);
        else if (a.y)
          store_out(a.y + row, v);
        if (EPI == EPI_ARGMAX && !(v != v)) {
          const uint64_t kk = argmax_key(v, (uint32_t)row);
          key = kk > key ? kk : key;
        }
      }
    }
  }
  if (EPI == EPI_ARGMAX && lane == 0 && key)
    atomicMax(reinterpret_cast<unsigned long long*>(a.best), (unsigned long long)key);
}

// Strip form for Q4_K (in_dim a multiple of 2048): the K axis is cut into
// strips of 8 superblocks; a wave owns one strip and keeps its lanes' activations in
// registers while it walks rows, so no activation is re-read per row.  A
// workgroup has one wave per strip (times WPS when there are fewer than 4
// strips) and walks batches of rows; two batches of loads are in flight
// (clamped unconditional loads), a row's partials are summed over the wave
// (DPP) and then over strips through LDS in a fixed order.
// Row r of a segmented launch: its weights and output slot.
__device__ __forceinline__ int kq_seg(const GenericArgs& a, int r) {
  return r < (int)a.seg_end[0] ? 0 : (r < (int)a.seg_end[1] ? 1 : 2);
}

// PRO 1: rmsnorm prologue (ops.rs:29-52): the sum of squares over the whole
// vector (the strip waves of sub 0, each lane's 32 values), then each lane
// scales its activations by rinv * gain before the run sums.  PRO 2: x is
// the decode attention's split outputs; the workgroup merges them into LDS
// (8 dims per thread, attn_split_merge) and the lanes read their runs there.  EPI_SWIGLU: a
// wave's two rows are gate row r and up row r (RB 2), and the epilogue
// writes silu(gate) * up (activation.rs:115-148 operand order).
template <uint32_t QT, int EPI, int RB, int PRO = 0>
__global__ __launch_bounds__(1024) void kq_strip_kernel(GenericArgs a, int S) {
  constexpr int BB = KqGeom<QT>::BB;
  constexpr int RPU = EPI == EPI_SWIGLU ? 1 : RB;  // output rows per wave per batch
  static_assert(EPI != EPI_SWIGLU || RB == 2, "SwiGLU pairs a gate and an up row");
  __shared__ float part[2][32][RB];  // [buffer][wave][row of the batch]
  __shared__ float red[32];
  extern __shared__ __attribute__((aligned(16))) float xs[];  // PRO 2: merged x [k]
  const int NW = blockDim.x >> 6;
  const int WPS = NW / S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = wave % S, sub = wave / S;
  const int nsb = (int)(a.k / 256);
  const int sb = strip * 8 + (lane >> 3);  // this lane's superblock
  const size_t rowbytes = (size_t)nsb * BB;
  const int nrows = (int)(a.row_hi - a.row_lo);
  const int per_batch = WPS * RPU;
  const int nbatch = (nrows + per_batch - 1) / per_batch;
  auto load_batch = [&](KqLane<QT> (&L)[RB], int batch) {
    const int base = batch * per_batch + sub * RPU;
#pragma unroll
    for (int j = 0; j < RB; j++) {
      if (EPI == EPI_SWIGLU) {
        const size_t row = a.row_lo + (size_t)min(base, nrows - 1);
        kq_load(L[j], (j == 0 ? a.w : a.w_up) + row * rowbytes + (size_t)sb * BB, lane);
      } else if (a.nseg > 1) {
        const int r = min(base + j, nrows - 1), sg = kq_seg(a, r);
        const size_t local = (size_t)(r - (sg == 0 ? 0 : (int)a.seg_end[sg - 1]));
        kq_load(L[j], a.seg_w[sg] + local * rowbytes + (size_t)sb * BB, lane);
      } else {
        const size_t row = a.row_lo + (size_t)min(base + j, nrows - 1);
        kq_load(L[j], a.w + row * rowbytes + (size_t)sb * BB, lane);
      }
    }
  };
  // x first, then the first batch (unconditional: the grid never exceeds
  // the batch count); the second batch is issued after the activation sums,
  // so that their wait leaves the first batch's loads in flight
  KqLane<QT> LA[RB], LB[RB];
  const int b0 = blockIdx.x, bstep = gridDim.x;
  KqX x, g;
  AttnSplitIn am;
  const int k = (int)a.k;
  if (PRO == 2) {
    // the first 8 merged dims' inputs ahead of the weights (the wait for
    // them then leaves the weight loads in flight)
    if (8 * (int)threadIdx.x < k) attn_split_load(am, a.x, a.attn_ml, k, a.attn_hd, a.attn_nsplit, 8 * threadIdx.x);
  } else {
    x = kq_x<QT>(a.x, sb, lane);
  }
  if (PRO == 1) g = kq_x<QT>(a.norm_w, sb, lane);
  load_batch(LA, b0);
  if (PRO == 2) {
    for (int e0 = 8 * threadIdx.x; e0 < k; e0 += 8 * blockDim.x) {
      if (e0 != 8 * (int)threadIdx.x) attn_split_load(am, a.x, a.attn_ml, k, a.attn_hd, a.attn_nsplit, e0);
      float4 m0, m1;
      attn_split_merge(am, a.attn_nsplit, m0, m1);
      reinterpret_cast<float4*>(xs + e0)[0] = m0;
      reinterpret_cast<float4*>(xs + e0)[1] = m1;
    }
    __syncthreads();
    x = kq_x<QT>(xs, sb, lane);
  }
  if (PRO == 1) {
    float ssq = 0.0f;
    if (sub == 0) {
#pragma unroll
      for (int c = 0; c < 4; c++)
        ssq += (x.a[c].x * x.a[c].x + x.a[c].y * x.a[c].y + x.a[c].z * x.a[c].z + x.a[c].w * x.a[c].w) +
               (x.b[c].x * x.b[c].x + x.b[c].y * x.b[c].y + x.b[c].z * x.b[c].z + x.b[c].w * x.b[c].w);
    }
    // the scalar 1/sqrt(mean + eps) factors out of every row's dot
    // product: the decode runs on x * w, and the row totals (and the
    // normalised copy of x) are scaled once the sum of squares has crossed
    // the batch's barrier
    ssq = wave_sum(ssq);
    if (lane == 0) red[wave] = ssq;
    float sa = 0.0f, sbs = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      x.a[c] = make_float4(x.a[c].x * g.a[c].x, x.a[c].y * g.a[c].y, x.a[c].z * g.a[c].z, x.a[c].w * g.a[c].w);
      x.b[c] = make_float4(x.b[c].x * g.b[c].x, x.b[c].y * g.b[c].y, x.b[c].z * g.b[c].z, x.b[c].w * g.b[c].w);
      sa += (x.a[c].x + x.a[c].y) + (x.a[c].z + x.a[c].w);
      sbs += (x.b[c].x + x.b[c].y) + (x.b[c].z + x.b[c].w);
    }
    x.sa = sa;
    x.sb = sbs;
  }
  // 1/rms from the strips' sums of squares (valid after a batch barrier)
  auto rms_inv = [&]() {
    float tot = 0.0f;
    for (int i = 0; i < S; i++) tot += red[i];
    return 1.0f / sqrtf(tot / (float)a.k + a.eps);
  };
  asm volatile("" : "+v"(x.sa), "+v"(x.sb));
  if (b0 + bstep < nbatch) load_batch(LB, b0 + bstep);
  uint64_t key = 0;
  auto process = [&](const KqLane<QT> (&L)[RB], int batch, int buf) {
    const int base = batch * per_batch + sub * RPU;
#pragma unroll
    for (int j = 0; j < RB; j++) {
      const float v = wave_sum(kq_dot(L[j], x, lane));
      if (lane == 0) part[buf][wave][j] = v;
    }
    __syncthreads();
    const int tt = threadIdx.x;
    const float rinv = PRO == 1 ? rms_inv() : 1.0f;
    if (EPI == EPI_SWIGLU) {
      if (tt < per_batch) {
        const int ri = batch * per_batch + tt;
        if (ri < nrows) {
          float gv = 0.0f, uv = 0.0f;
          for (int st = 0; st < S; st++) {
            gv += part[buf][tt * S + st][0];
            uv += part[buf][tt * S + st][1];
          }
          if (PRO == 1) {
            gv *= rinv;
            uv *= rinv;
          }
          store_out(a.y + a.row_lo + ri, (gv / (1.0f + expf(-gv))) * uv);
        }
      }
    } else if (tt < per_batch) {
      const int su = tt / RB, j = tt % RB;
      const int ri = batch * per_batch + su * RB + j;
      if (ri < nrows) {
        float v = 0.0f;
        for (int st = 0; st < S; st++) v += part[buf][su * S + st][j];
        if (PRO == 1) v *= rinv;
        const size_t row = a.row_lo + ri;
        if (EPI == EPI_STORE && a.nseg > 1) {
          const int sg = kq_seg(a, ri);
          store_out(a.seg_y[sg] + (ri - (sg == 0 ? 0 : (int)a.seg_end[sg - 1])), v);
        } else if (EPI == EPI_RESID)
          store_out(a.y + row, a.resid[row] + v);
        else if (a.y)
          store_out(a.y + row, v);
        if (EPI == EPI_ARGMAX && !(v != v)) {
          const uint64_t kk = argmax_key(v, (uint32_t)row);
          key = kk > key ? kk : key;
        }
      }
    }
    (void)base;
  };
  for (int batch = b0; batch < nbatch; batch += 2 * bstep) {
    process(LA, batch, 0);
    if (batch + 2 * bstep < nbatch) load_batch(LA, batch + 2 * bstep);
    if (batch + bstep < nbatch) {
      process(LB, batch + bstep, 1);
      if (batch + 3 * bstep < nbatch) load_batch(LB, batch + 3 * bstep);
    }
  }
  if (PRO == 1 && a.xn_out && blockIdx.x == 0 && sub == 0) {
    // the normalised x for other consumers (every workgroup processed at
    // least one batch, so the sums of squares are visible); the sub-0
    // waves' lanes hold every element once
    const float rinv = rms_inv();
    float4* o = reinterpret_cast<float4*>(a.xn_out + sb * 256 + kq_lane_elem<QT>(lane));
#pragma unroll
    for (int c = 0; c < 4; c++) {
      o[c] = make_float4(x.a[c].x * rinv, x.a[c].y * rinv, x.a[c].z * rinv, x.a[c].w * rinv);
      o[8 + c] = make_float4(x.b[c].x * rinv, x.b[c].y * rinv, x.b[c].z * rinv, x.b[c].w * rinv);
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
}

// Strip form for Q6_K (in_dim a multiple of 2048).  The K axis is cut into
// strips of 8 superblocks; a wave owns one strip and keeps its lanes'
// activations in registers while it walks rows.  Four lanes per superblock
// decode 64 elements each, so a half-wave covers one row's strip and a wave
// decodes two rows at a time.  Lane (n, is): half n, l in [16 is, 16 is +
// 16), all four quarters Q: element 128 n + l + 32 Q, low 4 bits from ql[l]
// (Q even) or ql[l + 32] (Q odd), nibble selected by Q >= 2, high 2 bits
// qh[l] >> 2Q, scale sc[8 n + is + 2 Q] (dequant.rs:328-355).
// A workgroup has one wave per strip (times WPS when there are fewer than 4
// strips) and walks batches of row pairs with two batches of loads in
// flight (clamped unconditional loads).  A row's partial is summed over its
// half-wave with DPP, then over strips through LDS in a fixed order.
template <uint32_t QT>
struct Kq2Lane;
template <>
struct Kq2Lane<Q6K> {
  u32x4 la, lb, hb;
  uint32_t sc0, sc1, d;
};

__device__ __forceinline__ void kq2_load(Kq2Lane<Q6K>& L, const uint8_t* blk, int lane) {
  const int n = (lane >> 1) & 1, is = lane & 1;
  L.la = *reinterpret_cast<const u32x4a2*>(blk + 64 * n + 16 * is);
  L.lb = *reinterpret_cast<const u32x4a2*>(blk + 64 * n + 32 + 16 * is);
  L.hb = *reinterpret_cast<const u32x4a2*>(blk + 128 + 32 * n + 16 * is);
  const u32x2a2 scw = *reinterpret_cast<const u32x2a2*>(blk + 192 + 8 * n);
  L.sc0 = scw.x;
  L.sc1 = scw.y;
  L.d = (uint32_t)*reinterpret_cast<const uint16_t*>(blk + 208);
}

// The lane's 64 activations as four runs of 16 (quarter Q: elements
// 128 n + 16 is + 32 Q ..) and their sums.
struct Kq2X {
  float4 r[4][4];
  float s[4];
};

__device__ __forceinline__ Kq2X kq2_x(const float* x, int sb, int lane) {
  Kq2X r;
  const int e0 = 128 * ((lane >> 1) & 1) + 16 * (lane & 1);
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const float4* p = reinterpret_cast<const float4*>(x + sb * 256 + e0 + 32 * q);
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      r.r[q][c] = p[c];
      s += (r.r[q][c].x + r.r[q][c].y) + (r.r[q][c].z + r.r[q][c].w);
    }
    r.s[q] = s;
  }
  return r;
}

__device__ __forceinline__ float kq2_dot(const Kq2Lane<Q6K>& L, const Kq2X& x, int lane) {
  const int is = lane & 1;
  const uint32_t scw[2] = {L.sc0, L.sc1};
  const float d = half_bits_to_f32(L.d);
  const uint32_t a[4] = {L.la.x, L.la.y, L.la.z, L.la.w}, b[4] = {L.lb.x, L.lb.y, L.lb.z, L.lb.w},
                 hh[4] = {L.hb.x, L.hb.y, L.hb.z, L.hb.w};
  float acc = 0.0f;
#pragma unroll
  for (int Q = 0; Q < 4; Q++) {
    uint32_t q[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const uint32_t lowsrc = (Q & 1) ? b[c] : a[c];
      const uint32_t lo4 = (Q >= 2) ? ((lowsrc >> 4) & 0x0F0F0F0Fu) : (lowsrc & 0x0F0F0F0Fu);
      q[c] = opaque_u32(lo4 | (((hh[c] >> (2 * Q)) & 0x03030303u) << 4));
    }
    const float sc = (float)(int8_t)byte_of(scw, is + 2 * Q);
    const float sQ = u8_dot16(q, x.r[Q]);
    acc = fmaf(d * sc, fmaf(-32.0f, x.s[Q], sQ), acc);
  }
  return acc;
}

template <uint32_t QT, int EPI, int RB>
__global__ __launch_bounds__(1024) void kq2_strip_kernel(GenericArgs a, int S) {
  constexpr int BB = KqGeom<QT>::BB;
  constexpr int RPB = 2 * RB;                // rows per wave per batch
  __shared__ float part[2][32][RPB];  // [buffer][wave][row of the batch]
  const int NW = blockDim.x >> 6;
  const int WPS = NW / S;
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = wave % S, sub = wave / S;
  const int nsb = (int)(a.k / 256);
  const int sb = strip * 8 + ((lane >> 2) & 7);  // this lane's superblock
  const size_t rowbytes = (size_t)nsb * BB;
  const int nrows = (int)(a.row_hi - a.row_lo);
  const int per_batch = WPS * RPB;
  const int nbatch = (nrows + per_batch - 1) / per_batch;
  // row j of this wave's share of a batch: j = 2 * pair + half
  auto load_batch = [&](Kq2Lane<QT> (&L)[RB], int batch) {
    const int base = batch * per_batch + sub * RPB;
#pragma unroll
    for (int p = 0; p < RB; p++) {
      const size_t row = a.row_lo + (size_t)min(base + 2 * p + half, nrows - 1);
      kq2_load(L[p], a.w + row * rowbytes + (size_t)sb * BB, lane);
    }
  };
  // x first, then the first batch (unconditional: the grid never exceeds
  // the batch count); the second batch is issued after the activation sums
  Kq2Lane<QT> LA[RB], LB[RB];
  const int b0 = blockIdx.x, bstep = gridDim.x;
  Kq2X x = kq2_x(a.x, sb, lane);
  load_batch(LA, b0);
  asm volatile("" : "+v"(x.s[0]), "+v"(x.s[1]), "+v"(x.s[2]), "+v"(x.s[3]));
  if (b0 + bstep < nbatch) load_batch(LB, b0 + bstep);
  uint64_t key = 0;
  auto process = [&](const Kq2Lane<QT> (&L)[RB], int batch, int buf) {
#pragma unroll
    for (int p = 0; p < RB; p++) {
      // sum over the half-wave: the row total lands in lanes 16..31 / 48..63
      const float v = group_sum<32>(kq2_dot(L[p], x, lane));
      if ((lane & 31) == 31) part[buf][wave][2 * p + half] = v;
    }
    __syncthreads();
    const int tt = threadIdx.x;
    if (tt < per_batch) {
      const int su = tt / RPB, j = tt % RPB;
      const int ri = batch * per_batch + su * RPB + j;
      if (ri < nrows) {
        float v = 0.0f;
        for (int st = 0; st < S; st++) v += part[buf][su * S + st][j];
        const size_t row = a.row_lo + ri;
        if (EPI == EPI_RESID)
          store_out(a.y + row, a.resid[row] + v);
        else if (a.y)
          store_out(a.y + row, v);
        if (EPI == EPI_ARGMAX && !(v != v)) {
          const uint64_t kk = argmax_key(v, (uint32_t)row);
          key = kk > key ? kk : key;
        }
      }
    }
  };
  for (int batch = b0; batch < nbatch; batch += 2 * bstep) {
    process(LA, batch, 0);
    if (batch + 2 * bstep < nbatch) load_batch(LA, batch + 2 * bstep);
    if (batch + bstep < nbatch) {
      process(LB, batch + bstep, 1);
      if (batch + 3 * bstep < nbatch) load_batch(LB, batch + 3 * bstep);
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
}

size_t kq_lds_bytes(int k) { return (size_t)k * sizeof(float) + (size_t)(k / 16) * sizeof(float); }

static int kq_cu_count() {
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

// Q6_K strip GEMV with the activations in LDS.  The lane layout is
// kq2_strip_kernel's (four lanes per superblock, 64 elements per lane, a
// half-wave per row, so a wave decodes a row pair), but the activations are
// staged once per workgroup into LDS in lane order (strip, quarter, float4
// column, lane % 32) and read per quarter while the rows are decoded: a lane
// holds 16 activations at a time instead of 64, which leaves the registers
// to more waves per CU, and the workgroup reads x from L2 once instead of
// once per wave.  Workgroups of S strips x WPS waves walk batches of RB row
// pairs per wave with two batches in flight and no barrier in the loop: the
// half-wave partials of every batch go to LDS and the strips are summed once
// at the end.
constexpr int kKq6Waves = 16;  // waves per workgroup (at most)

__device__ __forceinline__ int kq6_lds_index(int strip, int Q, int c, int slot) {
  return ((strip * 4 + Q) * 4 + c) * 32 + slot;  // float4 units
}

template <int EPI, int RB>
__global__ __launch_bounds__(1024) void kq6l_kernel(GenericArgs a, int S, int WPS, int nbl) {
  constexpr int BB = KqGeom<Q6K>::BB;
  constexpr int RPB = 2 * RB;  // rows per wave per batch
  extern __shared__ __attribute__((aligned(16))) float kq6_smem[];
  float4* xl = reinterpret_cast<float4*>(kq6_smem);  // [S][4][4][32] float4
  const int NW = S * WPS;
  float* part = kq6_smem + S * 2048;                  // [nbl][NW][RPB]
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5, slot = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = wave % S, sub = wave / S;
  const int nsb = (int)(a.k / 256);
  const int sb = strip * 8 + ((lane >> 2) & 7);  // this lane's superblock
  const size_t rowbytes = (size_t)nsb * BB;
  const int nrows = (int)(a.row_hi - a.row_lo);
  const int per_batch = WPS * RPB;
  const int nbatch = (nrows + per_batch - 1) / per_batch;
  auto load_batch = [&](Kq2Lane<Q6K> (&L)[RB], int batch) {
    const int base = batch * per_batch + sub * RPB;
#pragma unroll
    for (int p = 0; p < RB; p++) {
      const size_t row = a.row_lo + (size_t)min(base + 2 * p + half, nrows - 1);
      kq2_load(L[p], a.w + row * rowbytes + (size_t)sb * BB, lane);
    }
  };
  // first batch's weights (unconditional: the grid never exceeds the batch
  // count), then x into LDS in lane order while they fly
  Kq2Lane<Q6K> LA[RB], LB[RB];
  const int b0 = blockIdx.x, bstep = gridDim.x;
  load_batch(LA, b0);
  {
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    for (int f = threadIdx.x; f < (int)(a.k / 4); f += blockDim.x) {
      const int e = 4 * f;
      const int st = e >> 11, r = e & 255, sbl = (e >> 8) & 7;
      const int n = r >> 7, t = r & 127, Q = t >> 5, u = t & 31;
      const int sl = (sbl << 2) | (n << 1) | (u >> 4);
      xl[kq6_lds_index(st, Q, (u & 15) >> 2, sl)] = x4[f];
    }
  }
  __syncthreads();
  // the lane's quarter sums
  float xs4[4];
#pragma unroll
  for (int Q = 0; Q < 4; Q++) {
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float4 v = xl[kq6_lds_index(strip, Q, c, slot)];
      sum += (v.x + v.y) + (v.z + v.w);
    }
    xs4[Q] = sum;
  }
  asm volatile("" : "+v"(xs4[0]), "+v"(xs4[1]), "+v"(xs4[2]), "+v"(xs4[3]));
  if (b0 + bstep < nbatch) load_batch(LB, b0 + bstep);
  uint64_t key = 0;
  auto process = [&](const Kq2Lane<Q6K> (&L)[RB], int bi) {
    const int is = lane & 1;
    float acc[RB];
#pragma unroll
    for (int p = 0; p < RB; p++) acc[p] = 0.0f;
#pragma unroll
    for (int Q = 0; Q < 4; Q++) {
      float4 xq[4];
#pragma unroll
      for (int c = 0; c < 4; c++) xq[c] = xl[kq6_lds_index(strip, Q, c, slot)];
#pragma unroll
      for (int p = 0; p < RB; p++) {
        const uint32_t a4[4] = {L[p].la.x, L[p].la.y, L[p].la.z, L[p].la.w};
        const uint32_t b4[4] = {L[p].lb.x, L[p].lb.y, L[p].lb.z, L[p].lb.w};
        const uint32_t h4[4] = {L[p].hb.x, L[p].hb.y, L[p].hb.z, L[p].hb.w};
        uint32_t q[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const uint32_t lowsrc = (Q & 1) ? b4[c] : a4[c];
          const uint32_t lo4 = (Q >= 2) ? ((lowsrc >> 4) & 0x0F0F0F0Fu) : (lowsrc & 0x0F0F0F0Fu);
          q[c] = opaque_u32(lo4 | (((h4[c] >> (2 * Q)) & 0x03030303u) << 4));
        }
        const uint32_t scw[2] = {L[p].sc0, L[p].sc1};
        const float dsc = kq_half(L[p].d) * (float)(int8_t)byte_of(scw, is + 2 * Q);
        acc[p] = fmaf(dsc, fmaf(-32.0f, xs4[Q], u8_dot16(q, xq)), acc[p]);
      }
    }
#pragma unroll
    for (int p = 0; p < RB; p++) {
      // sum over the half-wave: the row total lands in lanes 16..31 / 48..63
      const float v = group_sum<32>(acc[p]);
      if ((lane & 31) == 31) part[(bi * NW + wave) * RPB + 2 * p + half] = v;
    }
  };
  int bi = 0;
  for (int batch = b0; batch < nbatch; batch += 2 * bstep, bi += 2) {
    process(LA, bi);
    if (batch + 2 * bstep < nbatch) load_batch(LA, batch + 2 * bstep);
    if (batch + bstep < nbatch) {
      process(LB, bi + 1);
      if (batch + 3 * bstep < nbatch) load_batch(LB, batch + 3 * bstep);
    }
  }
  __syncthreads();
  const int nb_mine = (nbatch - b0 + bstep - 1) / bstep;
  for (int idx = threadIdx.x; idx < nb_mine * per_batch; idx += blockDim.x) {
    const int lb = idx / per_batch, tt = idx - lb * per_batch;
    const float* pb = part + lb * NW * RPB;
    const int su = tt / RPB, j = tt - su * RPB;
    const int ri = (b0 + lb * bstep) * per_batch + tt;
    if (ri < nrows) {
      float v = 0.0f;
      for (int st = 0; st < S; st++) v += pb[(su * S + st) * RPB + j];
      const size_t row = a.row_lo + ri;
      if (EPI == EPI_RESID)
        store_out(a.y + row, a.resid[row] + v);
      else if (a.y)
        store_out(a.y + row, v);
      if (EPI == EPI_ARGMAX && !(v != v)) {
        const uint64_t kk = argmax_key(v, (uint32_t)row);
        key = kk > key ? kk : key;
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
  (void)nbl;
}

#ifndef ZG_KQ_STRIP_WAVES_PER_CU
#define ZG_KQ_STRIP_WAVES_PER_CU 16
#endif


template <uint32_t QT, int EPI, int PRO = 0>
static hipError_t launch_kq_strip(const GenericArgs& a, hipStream_t st) {
  // Q4_K: 32-element lanes, two rows per wave per batch.  Q6_K: 64-element
  // lanes (half a wave per row), one row pair per wave per batch.  Measured
  // on the Llama-3-8B shapes: Q4_K 12.6 us with 32-element lanes vs 14.6
  // with 64 (the longer per-lane chains stall); Q6_K 18.1 vs 21.2 us.
  constexpr int RPW = 2;  // rows per wave per batch
  const int S = (int)(a.k / 2048);
  const int nw = S >= 4 ? S : (S == 3 ? 6 : 4);
  const int wps = nw / S;
  const size_t rows = a.row_hi - a.row_lo;
  const size_t rpw = EPI == EPI_SWIGLU ? 1 : RPW;  // output rows per wave per batch
  const size_t nbatch = (rows + (size_t)wps * rpw - 1) / ((size_t)wps * rpw);
  const size_t per_cu = nw >= ZG_KQ_STRIP_WAVES_PER_CU ? 1 : (size_t)(ZG_KQ_STRIP_WAVES_PER_CU / nw);
  const size_t cap = (size_t)kq_cu_count() * per_cu;
  const size_t grid = nbatch < cap ? nbatch : cap;
  if (grid == 0) return hipSuccess;
  if constexpr (QT == Q4K)
    hipLaunchKernelGGL((kq_strip_kernel<QT, EPI, 2, PRO>), dim3((unsigned)grid), dim3(nw * 64), 0, st, a, S);
  else
    hipLaunchKernelGGL((kq2_strip_kernel<QT, EPI, 1>), dim3((unsigned)grid), dim3(nw * 64), 0, st, a, S);
  return hipGetLastError();
}

// one row pair per wave per batch and one workgroup per CU (two workgroups
// per CU read x twice and measured 19.9 vs 15.5 us at 4096x14336; two row
// pairs per batch spill)
constexpr int kKq6lRB = 1;
constexpr int kKq6lWgPerCu = 1;
// Q6_K with the activations in LDS (kq6l_kernel): in_dim a multiple of 2048
// from 8192 up to 14336 (the staged x then fits 56 KB of LDS), and enough
// rows that one workgroup per CU gets at least two batches.  Other launches
// keep kq2_strip_kernel's wider grid: 4096x14336 15.5 vs 16.9 us, but
// 2048x6144 6.8 vs 6.6 us, and the Q4_K_M pattern's Q6_K LM head
// (151936x2048) made its decode 1,004 vs 1,019 tok/s.
static bool kq6l_ok(const GenericArgs& a) {
  if (a.k % 2048 != 0 || a.k / 2048 < 4 || a.k / 2048 > 7) return false;
  const size_t S = a.k / 2048, rpb = (size_t)(kKq6Waves / S) * 2 * kKq6lRB;
  return (a.row_hi - a.row_lo + rpb - 1) / rpb >= (size_t)2 * kq_cu_count() * kKq6lWgPerCu;
}
template <int EPI>
static hipError_t launch_kq6l(const GenericArgs& a, hipStream_t st) {
  constexpr int RB = kKq6lRB, RPB = 2 * RB;
  const int S = (int)(a.k / 2048);
  const int WPS = kKq6Waves / S;
  const int nw = S * WPS;
  const size_t rows = a.row_hi - a.row_lo;
  const size_t nbatch = (rows + (size_t)WPS * RPB - 1) / ((size_t)WPS * RPB);
  size_t grid = (size_t)kq_cu_count() * kKq6lWgPerCu;
  if (grid > nbatch) grid = nbatch;
  if (grid == 0) return hipSuccess;
  const size_t xbytes = (size_t)S * 2048 * sizeof(float);
  const size_t max_part = 8 * 1024;
  size_t nbl = (nbatch + grid - 1) / grid;
  if (nbl * nw * RPB * sizeof(float) > max_part) {
    nbl = max_part / ((size_t)nw * RPB * sizeof(float));
    grid = (nbatch + nbl - 1) / nbl;
    nbl = (nbatch + grid - 1) / grid;
  }
  const size_t shm = xbytes + nbl * nw * RPB * sizeof(float);
  hipLaunchKernelGGL((kq6l_kernel<EPI, RB>), dim3((unsigned)grid), dim3(nw * 64), shm, st, a, S, WPS, (int)nbl);
  return hipGetLastError();
}

template <uint32_t QT, int EPI>
static hipError_t launch_kq(const GenericArgs& a, hipStream_t st) {
  if (QT == Q6K && kq6l_ok(a)) return launch_kq6l<EPI>(a, st);
  if (a.k % 2048 == 0 && a.k / 2048 <= 16) return launch_kq_strip<QT, EPI>(a, st);
  const size_t rows = a.row_hi - a.row_lo;
  const size_t shm = kq_lds_bytes((int)a.k);
  // LDS decides how many workgroups fit a CU (160 KB per CU)
  size_t per_cu = (160 * 1024) / (shm + 1024);
  if (per_cu > 4) per_cu = 4;
  if (per_cu < 1) per_cu = 1;
  const size_t want = (rows + kKqWaves - 1) / kKqWaves;
  const size_t cap = (size_t)kq_cu_count() * per_cu;
  const size_t grid = want < cap ? want : cap;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((kq_gemv_kernel<QT, EPI>), dim3((unsigned)grid), dim3(kKqWaves * 64), shm, st, a);
  return hipGetLastError();
}

// Q4_K through the strip kernel with the rmsnorm prologue (EPI_STORE,
// EPI_RESID, EPI_ARGMAX), gate|up with the SwiGLU epilogue (EPI_SWIGLU, with
// or without the prologue), or up to 3 segments of one x (EPI_STORE, with or
// without the prologue): in_dim a multiple of 2048 up to 32768.
bool kq_fused_ok(uint32_t qt, uint32_t il, size_t k, const void* w, const void* x) {
  return qt == Q4K && il == 1 && k % 2048 == 0 && k / 2048 <= 16 && kq_path_ok(qt, il, k, w, x);
}

hipError_t launch_kq_fused(const GenericArgs& a, bool rmsnorm, hipStream_t st) {
  if (a.qt != Q4K || a.k % 2048 || a.k / 2048 > 16) return hipErrorInvalidValue;
  if (a.nseg > 1 && (a.epi != EPI_STORE || a.nseg > 3 || a.row_lo != 0 || a.row_hi != a.seg_end[a.nseg - 1]))
    return hipErrorInvalidValue;
  if (!rmsnorm && a.epi == EPI_STORE) return launch_kq_strip<Q4K, EPI_STORE, 0>(a, st);
  if (rmsnorm) {
    if (a.epi == EPI_STORE) return launch_kq_strip<Q4K, EPI_STORE, 1>(a, st);
    if (a.epi == EPI_RESID) return launch_kq_strip<Q4K, EPI_RESID, 1>(a, st);
    if (a.epi == EPI_ARGMAX) return launch_kq_strip<Q4K, EPI_ARGMAX, 1>(a, st);
    if (a.epi == EPI_SWIGLU) return launch_kq_strip<Q4K, EPI_SWIGLU, 1>(a, st);
  } else if (a.epi == EPI_SWIGLU) {
    return launch_kq_strip<Q4K, EPI_SWIGLU, 0>(a, st);
  }
  return hipErrorInvalidValue;
}

// Q4_K O projection with the attention-merge prologue and the residual
// epilogue; the merged x (k floats) sits in LDS.
bool kq_attn_o_ok(uint32_t qt, uint32_t il, size_t k, int nsplit, int hd, const void* w, const void* x) {
  return kq_fused_ok(qt, il, k, w, x) && k <= 8192 && nsplit >= 1 && nsplit <= kAttnSplits && hd % 8 == 0 &&
         k % hd == 0;
}

hipError_t launch_kq_attn_o(const GenericArgs& a, hipStream_t st) {
  if (!kq_attn_o_ok(a.qt, a.il, a.k, a.attn_nsplit, a.attn_hd, a.w, a.x) || a.epi != EPI_RESID || a.nseg > 1)
    return hipErrorInvalidValue;
  constexpr int RPW = 2;
  const int S = (int)(a.k / 2048);
  const int nw = S >= 4 ? S : (S == 3 ? 6 : 4);
  const int wps = nw / S;
  const size_t rows = a.row_hi - a.row_lo;
  const size_t nbatch = (rows + (size_t)wps * RPW - 1) / ((size_t)wps * RPW);
  const size_t per_cu = nw >= ZG_KQ_STRIP_WAVES_PER_CU ? 1 : (size_t)(ZG_KQ_STRIP_WAVES_PER_CU / nw);
  const size_t cap = (size_t)kq_cu_count() * per_cu;
  const size_t grid = nbatch < cap ? nbatch : cap;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((kq_strip_kernel<Q4K, EPI_RESID, 2, 2>), dim3((unsigned)grid), dim3(nw * 64), a.k * sizeof(float),
                     st, a, S);
  return hipGetLastError();
}

bool kq_path_ok(uint32_t qt, uint32_t il, size_t k, const void* w, const void* x) {
  if ((qt != Q4K && qt != Q6K) || il != 1) return false;
  if (k % 256 != 0 || k > kMaxKqK) return false;
  // Q4_K lanes use aligned 128-bit loads; Q6_K loads are unaligned by design
  if (qt == Q4K && (reinterpret_cast<uintptr_t>(w) & 15u)) return false;
  return (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

hipError_t launch_gemv_kq(const GenericArgs& a, hipStream_t st) {
  if (a.qt == Q4K) {
    if (a.epi == EPI_STORE) return launch_kq<Q4K, EPI_STORE>(a, st);
    if (a.epi == EPI_RESID) return launch_kq<Q4K, EPI_RESID>(a, st);
    if (a.epi == EPI_ARGMAX) return launch_kq<Q4K, EPI_ARGMAX>(a, st);
  } else if (a.qt == Q6K) {
    if (a.epi == EPI_STORE) return launch_kq<Q6K, EPI_STORE>(a, st);
    if (a.epi == EPI_RESID) return launch_kq<Q6K, EPI_RESID>(a, st);
    if (a.epi == EPI_ARGMAX) return launch_kq<Q6K, EPI_ARGMAX>(a, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace zg
