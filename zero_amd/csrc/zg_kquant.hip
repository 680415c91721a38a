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

// 16 bytes from a possibly unaligned address (Q6_K superblocks are 210
// bytes, so their fields sit at any even offset); gfx950 runs in unaligned
// access mode and this is a single global_load_dwordx4.
__device__ __forceinline__ u32x4 ld16u(const uint8_t* p) {
  u32x4 v;
  __builtin_memcpy(&v, p, 16);
  return v;
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t* w, int i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xFFu; }

// get_scale_min_k4 (dequant.rs:75-85) over the 12 packed scale bytes.
__device__ __forceinline__ void scale_min_k4(const uint32_t* s, int j, float& sc, float& mn) {
  uint32_t a, b;
  if (j < 4) {
    a = byte_of(s, j) & 63u;
    b = byte_of(s, j + 4) & 63u;
  } else {
    a = (byte_of(s, j + 4) & 0xFu) | ((byte_of(s, j - 4) >> 6) << 4);
    b = (byte_of(s, j + 4) >> 4) | ((byte_of(s, j) >> 6) << 4);
  }
  sc = (float)a;
  mn = (float)b;
}

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

// One lane's share of one superblock: 32 elements -> partial dot.
// Q4_K lane (j = sub-block pair 0..3, h = half 0..1): qs bytes
// [32j + 16h, +16): low nibbles are elements 64j + 16h + i (sub-block 2j),
// high nibbles elements 64j + 32 + 16h + i (sub-block 2j+1).
__device__ __forceinline__ float q4k_lane(const uint8_t* blk, const float* xsb, const float* x16sb, int j, int h) {
  const u32x4 hdr = *reinterpret_cast<const u32x4*>(blk);
  const u32x4 qv = *reinterpret_cast<const u32x4*>(blk + 16 + 32 * j + 16 * h);
  const float d = half_bits_to_f32(hdr.x), dmin = half_bits_to_f32(hdr.x >> 16);
  const uint32_t sb[3] = {hdr.y, hdr.z, hdr.w};
  float scA, mA, scB, mB;
  scale_min_k4(sb, 2 * j, scA, mA);
  scale_min_k4(sb, 2 * j + 1, scB, mB);
  const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
  uint32_t lo[4], hi[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    lo[c] = q[c] & 0x0F0F0F0Fu;
    hi[c] = (q[c] >> 4) & 0x0F0F0F0Fu;
  }
  const int eA = 64 * j + 16 * h;
  const float sA = u8_dot16(lo, reinterpret_cast<const float4*>(xsb + eA));
  const float sB = u8_dot16(hi, reinterpret_cast<const float4*>(xsb + eA + 32));
  const float xA = x16sb[eA >> 4], xB = x16sb[(eA >> 4) + 2];
  float acc = (d * scA) * sA;
  acc = fmaf(-(dmin * mA), xA, acc);
  acc = fmaf(d * scB, sB, acc);
  return fmaf(-(dmin * mB), xB, acc);
}

// Q6_K lane (n = half 0..1, is = 0..1, qp = quarter pair 0..1): l in
// [16 is, 16 is + 16) of half n, quarters Q = 2 qp and 2 qp + 1
// (dequant.rs:328-355 element map: quarter Q of l is element 128n + l + 32Q,
// low 4 bits from ql[l] (Q even) or ql[l+32] (Q odd), nibble selected by
// Q >= 2, high 2 bits qh[l] >> 2Q, scale sc[8n + is + 2Q]).
__device__ __forceinline__ float q6k_lane(const uint8_t* blk, const float* xsb, const float* x16sb, int n, int is,
                                          int qp) {
  const u32x4 la = ld16u(blk + 64 * n + 16 * is);
  const u32x4 lb = ld16u(blk + 64 * n + 32 + 16 * is);
  const u32x4 hb = ld16u(blk + 128 + 32 * n + 16 * is);
  const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * n + is);
  const float scA = (float)sc[4 * qp], scB = (float)sc[4 * qp + 2];
  const float d = half_bits_to_f32((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
  const uint32_t a[4] = {la.x, la.y, la.z, la.w}, b[4] = {lb.x, lb.y, lb.z, lb.w}, hh[4] = {hb.x, hb.y, hb.z, hb.w};
  const int nsh = 4 * qp;  // nibble select
  const int hA = 4 * qp, hB = 4 * qp + 2;  // qh shift of quarters 2qp, 2qp+1
  uint32_t qA[4], qB[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    qA[c] = ((a[c] >> nsh) & 0x0F0F0F0Fu) | (((hh[c] >> hA) & 0x03030303u) << 4);
    qB[c] = ((b[c] >> nsh) & 0x0F0F0F0Fu) | (((hh[c] >> hB) & 0x03030303u) << 4);
  }
  const int eA = 128 * n + 16 * is + 64 * qp;  // quarter 2qp
  const float sA = u8_dot16(qA, reinterpret_cast<const float4*>(xsb + eA));
  const float sB = u8_dot16(qB, reinterpret_cast<const float4*>(xsb + eA + 32));
  const float xA = x16sb[eA >> 4], xB = x16sb[(eA >> 4) + 2];
  float acc = (d * scA) * fmaf(-32.0f, xA, sA);
  return fmaf(d * scB, fmaf(-32.0f, xB, sB), acc);
}

template <uint32_t QT, int EPI>
__global__ __launch_bounds__(kKqWaves * 64) void kq_gemv_kernel(GenericArgs a) {
  constexpr int BB = KqGeom<QT>::BB;
  extern __shared__ __attribute__((aligned(16))) float kq_smem[];
  const int k = (int)a.k;
  float* xs = kq_smem;
  float* x16 = kq_smem + k;
  stage_x_kq(xs, x16, a.x, k);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int sl = lane >> 3;  // superblock of the step
  const int nsb = k / 256;
  const size_t rowbytes = (size_t)nsb * BB;
  const size_t nrows = a.row_hi - a.row_lo;
  const size_t wave_id = (size_t)blockIdx.x * kKqWaves + (threadIdx.x >> 6);
  const size_t nwaves = (size_t)gridDim.x * kKqWaves;
  uint64_t key = 0;
  for (size_t r = wave_id; r < nrows; r += nwaves) {
    const size_t row = a.row_lo + r;
    const uint8_t* wrow = a.w + row * rowbytes;
    float acc = 0.0f;
    for (int s = sl; s < nsb; s += 8) {
      const uint8_t* blk = wrow + (size_t)s * BB;
      const float* xsb = xs + s * 256;
      const float* x16sb = x16 + s * 16;
      if (QT == Q4K)
        acc += q4k_lane(blk, xsb, x16sb, (lane >> 1) & 3, lane & 1);
      else
        acc += q6k_lane(blk, xsb, x16sb, (lane >> 2) & 1, (lane >> 1) & 1, lane & 1);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      if (EPI == EPI_RESID)
        a.y[row] = a.resid[row] + acc;
      else if (a.y)
        a.y[row] = acc;
      if (EPI == EPI_ARGMAX && !(acc != acc)) {
        const uint64_t kk = argmax_key(acc, (uint32_t)row);
        key = kk > key ? kk : key;
      }
    }
  }
  if (EPI == EPI_ARGMAX && lane == 0 && key)
    atomicMax(reinterpret_cast<unsigned long long*>(a.best), (unsigned long long)key);
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

template <uint32_t QT, int EPI>
static hipError_t launch_kq(const GenericArgs& a, hipStream_t st) {
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
