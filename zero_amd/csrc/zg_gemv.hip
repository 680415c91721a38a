// zg_gemv.hip -- decode-time GEMV kernels for gfx950.
//
// Replaces the AVX-512 row-range kernels of the reference
// (kernel/src/arch/x86_64/math/linear.rs:150,352,710,909,1096,1271) and the
// SMP row partitioning that fans them out (kernel/src/smp.rs:1567-1712):
// output rows map to the launch grid instead of to cores.
//
// Fast path (X4 streaming kernel): .smodel-v2 Q4_0X4 / Q8_0X4 tensors
// whose blocks-per-row is even.  Waves stream the weight bytes with fully
// coalesced 128-bit loads into LDS and decode them there (see gemv_x4_kernel
// below); the activation vector is staged in LDS once per workgroup and
// broadcast from there; nibbles/bytes are unpacked in registers
// (v_cvt_f32_ubyte*), each block sum is scaled by its fp16 d once, and the
// 64 lanes that share a group finish with a butterfly reduction.  No MFMA:
// the GEMV is HBM-bound.
//
// Generic path: any layout / block type, one wave per output row, byte
// loads.  Used for plain Q4_0/Q8_0, odd blocks-per-row and as the first
// Q4_K/Q6_K implementation.
#include <mutex>
#include <type_traits>
#include <vector>

#include "zg_device.h"
#include "zg_kernels.h"
#include "zg_strip.h"  // the strip GEMV (gemv_strip_body, gemv_strip_kernel)

namespace zg {

// ---------------------------------------------------------------------------
// Prologue: how the kernel forms the activation vector in LDS.
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// X4 streaming kernel.
//
// A group is 4 output rows; its .smodel-v2 stream is K/32 group-blocks of
// GB bytes (72 for Q4_0X4, 136 for Q8_0X4), contiguous, and consecutive
// groups are contiguous too.  Work unit = one "segment" of up to 64
// group-blocks of one group.  A wave
//   1. streams the segment with lane-contiguous 128-bit loads (a wave
//      instruction covers 1 KiB of consecutive bytes: fully coalesced),
//   2. parks it in its own LDS slot,
//   3. issues the loads of its next segment (they fly while it computes),
//   4. lane l decodes group-block l from LDS (ds_read_b64 at a 72/136-byte
//      stride, conflict-free) against x-block l broadcast from LDS.
// At the end of a group the 64 lane partials are reduced with a butterfly
// and lanes 0..3 write rows 0..3.  Waves loop persistently over groups; the
// workgroup stages the activation vector in LDS once.
// ---------------------------------------------------------------------------

template <uint32_t QT>
struct X4 {
  static constexpr int GB = (QT == Q4_0) ? 72 : 136;  // group-block bytes
  static constexpr int QDW = (QT == Q4_0) ? 4 : 8;     // qs dwords per row
  static constexpr int SEG = 64;                       // group-blocks per segment
  static constexpr int SEG_BYTES = SEG * GB;           // 4608 or 8704
  static constexpr int NL = (SEG_BYTES / 16 + 63) / 64;  // 128-bit loads per lane: 5 or 9
};

constexpr int kNW = 4;     // waves per workgroup
constexpr int kXBlk = 36;  // LDS floats per 32-float x-block (padded: lane stride 144 B)

__device__ __forceinline__ int x_off(int e) { return (e >> 5) * kXBlk + (e & 31); }

// Stage x (K floats) into LDS, applying the prologue.  rmsnorm follows
// ops.rs:29-52: x * (1/sqrt(mean(x^2)+eps)) * w; the scalar 1/sqrt(...)
// factors out of every row's dot product, so x * w is staged and the
// per-wave sums of squares go to red[]: the caller scales the row totals by
// stage_rinv() after the barrier that follows.
template <int PRO>
__device__ __forceinline__ void stage_x(float* xs, float* red, const GemvArgs& a) {
  constexpr int NT = kNW * 64;
  const int tid = threadIdx.x;
  const int K = a.k;
  const float4* x4 = reinterpret_cast<const float4*>(a.x);
  const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
  float ssq = 0.0f;
  for (int i = tid; i < K / 4; i += NT) {
    float4 v = x4[i];
    if (PRO == PRO_RMSNORM) {
      const float4 g = w4[i];
      ssq += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      v = make_float4(v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w);
    }
    *reinterpret_cast<float4*>(xs + x_off(4 * i)) = v;
  }
  if (PRO == PRO_RMSNORM) {
    ssq = seg_sum<64>(ssq);
    if ((tid & 63) == 0) red[tid >> 6] = ssq;
  }
}

__device__ __forceinline__ float stage_rinv(const float* red, const GemvArgs& a) {
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kNW; i++) tot += red[i];
  return 1.0f / sqrtf(tot / (float)a.k + a.eps);
}


// One group-block (GB bytes, 8-byte aligned in LDS) -> its 4 scales and
// 4 x QDW quant dwords.
template <uint32_t QT>
__device__ __forceinline__ void lds_group_block(const uint8_t* src, uint32_t* dw) {
  const uint2* p = reinterpret_cast<const uint2*>(src);
#pragma unroll
  for (int i = 0; i < X4<QT>::GB / 8; i++) {
    const uint2 v = p[i];
    dw[2 * i] = v.x;
    dw[2 * i + 1] = v.y;
  }
}

// Issue the 128-bit loads of one segment (nbytes, a multiple of 16) into
// registers: load i of lane l is bytes [16*(64*i + l), +16).
template <uint32_t QT>
__device__ __forceinline__ void seg_load(const uint8_t* src, int nbytes, int lane, u32x4* r) {
  const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
#pragma unroll
  for (int i = 0; i < X4<QT>::NL; i++) {
    const int c = 64 * i + lane;
    if (16 * c < nbytes) r[i] = __builtin_nontemporal_load(s4 + c);
  }
}

template <uint32_t QT>
__device__ __forceinline__ void seg_park(uint8_t* dst, int nbytes, int lane, const u32x4* r) {
  u32x4* d4 = reinterpret_cast<u32x4*>(dst);
#pragma unroll
  for (int i = 0; i < X4<QT>::NL; i++) {
    const int c = 64 * i + lane;
    if (16 * c < nbytes) d4[c] = r[i];
  }
}

// Work decomposition shared by the GEMV and its dequant test hook.
//   item  = logical group (SwiGLU: a gate group and its up group)
//   part  = which of the item's groups (0 unless SwiGLU)
//   seg   = segment of that group's K stream
struct UnitIter {
  int item, part, seg;
};

template <uint32_t QT, int PRO, int EPI>
__global__ __launch_bounds__(kNW * 64) void gemv_x4_kernel(GemvArgs a) {
  constexpr int GB = X4<QT>::GB, QDW = X4<QT>::QDW, SEG = X4<QT>::SEG, SEGB = X4<QT>::SEG_BYTES;
  constexpr int NL = X4<QT>::NL;
  constexpr int PARTS = (EPI == EPI_SWIGLU) ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  __shared__ float red[kNW];
  const int nb = a.k / 32;
  const int nseg = (nb + SEG - 1) / SEG;
  float* xs = smem;  // nb padded x-blocks
  uint8_t* wslot = reinterpret_cast<uint8_t*>(xs + nb * kXBlk) + (threadIdx.x >> 6) * SEGB;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int items = (int)(EPI == EPI_SWIGLU ? a.total_groups / 2 : a.total_groups);
  const int wave_id = blockIdx.x * kNW + wave;
  const int wave_stride = gridDim.x * kNW;

  // group stream of (item, part): segment table lookup (<= 3 segments)
  auto locate = [&](int item, int part, uint32_t& lg) -> GemvSeg {
    if (EPI == EPI_SWIGLU) {
      lg = (uint32_t)item;
      return part ? a.seg[1] : a.seg[0];
    }
    const GemvSeg sg = seg_of(a, (uint32_t)item);
    lg = (uint32_t)item - sg.g_begin;
    return sg;
  };
  auto seg_src = [&](const UnitIter& u, int& nbytes) -> const uint8_t* {
    uint32_t lg;
    const GemvSeg sg = locate(u.item, u.part, lg);
    const int blocks = min(SEG, nb - u.seg * SEG);
    nbytes = blocks * GB;
    return sg.w + ((size_t)lg * nb + (size_t)u.seg * SEG) * GB;
  };
  auto advance = [&](UnitIter& u) {
    if (++u.seg == nseg) {
      u.seg = 0;
      if (++u.part == PARTS) {
        u.part = 0;
        u.item += wave_stride;
      }
    }
  };

  UnitIter u{wave_id, 0, 0};
  u32x4 r[NL];
  int nbytes = 0;
  const uint8_t* src = nullptr;
  if (u.item < items) {
    src = seg_src(u, nbytes);
    seg_load<QT>(src, nbytes, lane, r);  // first loads fly during x staging
  }
  stage_x<PRO>(xs, red, a);
  __syncthreads();
  const float rinv = PRO == PRO_RMSNORM ? stage_rinv(red, a) : 1.0f;

  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float gate[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  uint64_t key = 0;
  while (u.item < items) {
    const int cur_bytes = nbytes;
    const UnitIter cu = u;
    seg_park<QT>(wslot, cur_bytes, lane, r);
    wave_lds_sync();
    advance(u);
    if (u.item < items) {
      src = seg_src(u, nbytes);
      seg_load<QT>(src, nbytes, lane, r);
    }
    // lane l: group-block l of the segment
    const int b = cu.seg * SEG + lane;
    if (lane * GB < cur_bytes) {
      uint32_t dw[GB / 4];
      lds_group_block<QT>(wslot + lane * GB, dw);
      float4 xb[8];
#pragma unroll
      for (int c = 0; c < 8; c++) xb[c] = reinterpret_cast<const float4*>(xs + b * kXBlk)[c];
      float d[4];
      d[0] = half_bits_to_f32(dw[0]);
      d[1] = half_bits_to_f32(dw[0] >> 16);
      d[2] = half_bits_to_f32(dw[1]);
      d[3] = half_bits_to_f32(dw[1] >> 16);
      // sum of this x-block: the -8 (Q4_0) or -128 (Q8_0 read as unsigned
      // bytes) offset of every row
      float t = 0.0f;
#pragma unroll
      for (int c = 0; c < 8; c++) t += (xb[c].x + xb[c].y) + (xb[c].z + xb[c].w);
      if (QT == Q4_0) {
        const float m8 = -8.0f * t;
#pragma unroll
        for (int rr = 0; rr < 4; rr++) acc[rr] = fmaf(d[rr], q4_block_dot(dw + 2 + QDW * rr, xb) + m8, acc[rr]);
      } else {
        const float m128 = -128.0f * t;
#pragma unroll
        for (int rr = 0; rr < 4; rr++) acc[rr] = fmaf(d[rr], q8u_block_dot(dw + 2 + QDW * rr, xb) + m128, acc[rr]);
      }
    }
    wave_lds_sync();  // the slot is rewritten next iteration
    if (cu.seg != nseg - 1) continue;
    // group finished: reduce and write
#pragma unroll
    for (int rr = 0; rr < 4; rr++) acc[rr] = PRO == PRO_RMSNORM ? wave_sum(acc[rr]) * rinv : wave_sum(acc[rr]);
    uint32_t lg;
    const GemvSeg sg = locate(cu.item, cu.part, lg);
    if (EPI == EPI_SWIGLU && cu.part == 0) {
#pragma unroll
      for (int rr = 0; rr < 4; rr++) gate[rr] = acc[rr];
    } else if (lane < 4) {
      const float v = (lane == 0) ? acc[0] : (lane == 1) ? acc[1] : (lane == 2) ? acc[2] : acc[3];
      const uint32_t row = 4 * lg + (uint32_t)lane;
      if (row >= sg.row_lo && row < sg.row_hi) {
        if (EPI == EPI_SWIGLU) {
          const float g = (lane == 0) ? gate[0] : (lane == 1) ? gate[1] : (lane == 2) ? gate[2] : gate[3];
          // activation.rs:115-148 operand order: silu = g/(1+exp(-g)), then *up
          store_out(a.seg[0].y + row, (g / (1.0f + expf(-g))) * v);
        } else if (EPI == EPI_RESID) {
          store_out(sg.y + row, sg.resid[row] + v);
        } else {
          if (sg.y) store_out(sg.y + row, v);
          if (EPI == EPI_ARGMAX && !(v != v)) {
            const uint64_t kk = argmax_key(v, row);
            key = kk > key ? kk : key;
          }
        }
      }
    }
#pragma unroll
    for (int rr = 0; rr < 4; rr++) acc[rr] = 0.0f;
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



// ---------------------------------------------------------------------------
// Generic kernel: one wave per output row, any (type, layout).  Dequantizes
// each element with the reference's operation order (bit-exact weights) and
// accumulates x*w with fmaf.
// ---------------------------------------------------------------------------
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
    if (a.epi == EPI_RESID) store_out(a.y + row, a.resid[row] + acc);
    else if (a.y) store_out(a.y + row, acc);
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

// Dequantize X4 tensors through the streaming kernel's own path (segment
// loads, LDS slot, per-lane group-block decode), so the fast path's
// byte -> element map is checked bit for bit.  One wave per segment.
template <uint32_t QT>
__global__ __launch_bounds__(kNW * 64) void dequant_x4_stream_kernel(DequantArgs a) {
  constexpr int GB = X4<QT>::GB, QDW = X4<QT>::QDW, SEG = X4<QT>::SEG, SEGB = X4<QT>::SEG_BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t slots[kNW * SEGB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb = (int)(a.k / 32), nseg = (nb + SEG - 1) / SEG;
  const size_t unit = (size_t)blockIdx.x * kNW + wave;
  if (unit >= (a.rows / 4) * (size_t)nseg) return;  // wave-uniform
  const size_t g = unit / nseg;
  const int seg = (int)(unit % nseg);
  const int nbytes = min(SEG, nb - seg * SEG) * GB;
  u32x4 r[X4<QT>::NL];
  seg_load<QT>(a.w + (g * nb + (size_t)seg * SEG) * GB, nbytes, lane, r);
  uint8_t* slot = slots + wave * SEGB;
  seg_park<QT>(slot, nbytes, lane, r);
  wave_lds_sync();
  if (lane * GB >= nbytes) return;
  uint32_t dw[GB / 4];
  lds_group_block<QT>(slot + lane * GB, dw);
  const int b = seg * SEG + lane;
  for (int rr = 0; rr < 4; rr++) {
    const float d = half_bits_to_f32(dw[rr >> 1] >> (16 * (rr & 1)));
    float* o = a.out + (4 * g + rr) * a.k + (size_t)b * 32;
    const uint32_t* qs = dw + 2 + QDW * rr;
    for (int e = 0; e < 32; e++) {
      float v;
      if (QT == Q4_0) {
        const uint32_t word = qs[(e & 15) >> 2];
        const uint32_t nib = (word >> (8 * (e & 3) + (e < 16 ? 0 : 4))) & 0xF;
        v = (float)((int)nib - 8) * d;
      } else {
        v = (float)(int8_t)((qs[e >> 2] >> (8 * (e & 3))) & 0xFF) * d;
      }
      o[e] = v;
    }
  }
}

__global__ void fp16_kernel(const uint16_t* in, float* out, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = half_bits_to_f32(in[i]);
}

__global__ void fill_u64_kernel(uint64_t* p, uint64_t v) { *p = v; }

// The floor of one launch that streams n16 16-byte words and computes
// nothing: thread t of workgroup g reads words (256 U) g + t + 256 u,
// u < U, with the GEMV's nontemporal 128-bit loads.  The XOR of the words
// feeds a store that real data never triggers, so the loads stay live.
template <int U>
__global__ __launch_bounds__(256) void read_floor_kernel(const u32x4* __restrict__ src, size_t n16, uint32_t* sink) {
  const size_t base = (size_t)blockIdx.x * 256 * U + threadIdx.x;
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const size_t i = base + (size_t)u * 256;
    if (i < n16) {
      const u32x4 v = __builtin_nontemporal_load(src + i);
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  if (acc == 0x9E3779B9u) *sink = acc;
}

// The strip GEMV's loads without its decode, Q4_0X4 at in_dim 2048 (four
// strips, one wave each): lane (b, r) of wave s loads, per group, the quant
// bytes and fp16 d of row r of block 16 s + b through strip_load (the
// GEMV's own load instructions and cache policy) and, with X, its two
// float4 quarters of x.  ONEB: one batch of GB groups per workgroup (the
// decode-sized form); else a batch loop over GB-group batches, the next
// batch's loads issued before the current one is consumed (the tall form,
// cache-allocating loads as there).  Indices past the last group clamp.
// The words feed a store that real data never triggers.
template <int GB, bool ONEB, bool X>
__global__ __launch_bounds__(256) void strip_load_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                         int groups, uint32_t* sink) {
  constexpr size_t kGroupBytes = 64 * 72;  // 64 group-blocks of 72 bytes
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = lane >> 2, r = lane & 3, kb = wave * 16 + b;
  uint32_t acc = 0;
  if (X) {
    const float4* x4 = reinterpret_cast<const float4*>(x + kb * 32);
    const float4 xl = x4[r], xh = x4[4 + r];
    acc = (__float_as_uint(xl.x) ^ __float_as_uint(xl.y) ^ __float_as_uint(xl.z) ^ __float_as_uint(xl.w)) ^
          (__float_as_uint(xh.x) ^ __float_as_uint(xh.y) ^ __float_as_uint(xh.z) ^ __float_as_uint(xh.w));
  }
  auto load = [&](LaneW<Q4_0> (&L)[GB], int batch) {
#pragma unroll
    for (int j = 0; j < GB; j++) {
      const int g = min(batch * GB + j, groups - 1);
      strip_load<Q4_0, !ONEB>(L[j], w + (size_t)g * kGroupBytes + kb * 72, r);
    }
  };
  auto consume = [&](const LaneW<Q4_0> (&L)[GB]) {
#pragma unroll
    for (int j = 0; j < GB; j++) acc ^= L[j].q[0] ^ L[j].q[1] ^ L[j].q[2] ^ L[j].q[3] ^ L[j].d;
  };
  if (ONEB) {
    LaneW<Q4_0> L[GB];
    load(L, blockIdx.x);
    consume(L);
  } else {
    const int nbatch = (groups + GB - 1) / GB, step = gridDim.x;
    LaneW<Q4_0> A[GB], B[GB];
    load(A, blockIdx.x);
    for (int bt = blockIdx.x; bt < nbatch; bt += 2 * step) {
      load(B, min(bt + step, nbatch - 1));
      consume(A);
      load(A, min(bt + 2 * step, nbatch - 1));
      consume(B);
    }
  }
  if (acc == 0x9E3779B9u) *sink = acc;
}

// ---------------------------------------------------------------------------
// Host-side launchers.
// ---------------------------------------------------------------------------

// Resident workgroups per CU of kernel f at (threads, shm), queried once per
// distinct (kernel, threads, shm) and cached under a lock: one template
// instance can be launched with different block and LDS sizes, and several
// host threads may launch at once.  big_lds: raise the kernel's dynamic LDS
// limit to shm first (needed above 64 KiB).
static int resident_per_cu(const void* f, int threads, size_t shm, bool big_lds = false) {
  struct Entry {
    const void* f;
    int threads;
    size_t shm;
    int n;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  std::lock_guard<std::mutex> lock(mu);
  for (const Entry& e : cache)
    if (e.f == f && e.threads == threads && e.shm == shm) return e.n;
  int n = 0;
  if ((big_lds && hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) != hipSuccess) ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, threads, shm) != hipSuccess || n <= 0)
    n = 1;
  try {
    cache.push_back({f, threads, shm, n});
  } catch (const std::bad_alloc&) {  // the value is still right; only the cache entry is lost
  }
  return n;
}

static int cu_count() {
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

size_t gemv_x4_lds_bytes(uint32_t qt, int k) {
  const int nb = k / 32;
  const size_t segb = (qt == Q4_0) ? X4<Q4_0>::SEG_BYTES : X4<Q8_0>::SEG_BYTES;
  return (size_t)nb * kXBlk * sizeof(float) + kNW * segb;
}

template <uint32_t QT, int PRO, int EPI>
static hipError_t launch_x4(const GemvArgs& a, hipStream_t st) {
  constexpr int SEG = X4<QT>::SEG;
  const int nb = a.k / 32, nseg = (nb + SEG - 1) / SEG;
  const size_t units = (size_t)a.total_groups * nseg;
  const size_t shm = gemv_x4_lds_bytes(QT, a.k);
  // enough workgroups that every wave has work, capped at a few resident
  // workgroups per CU (the waves loop over the remaining groups)
  const size_t want = (units + kNW - 1) / kNW;
  const size_t per_cu = shm <= 32768 ? 4 : (shm <= 53248 ? 3 : 2);
  const size_t grid = want < (size_t)cu_count() * per_cu ? want : (size_t)cu_count() * per_cu;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((gemv_x4_kernel<QT, PRO, EPI>), dim3((unsigned)grid), dim3(kNW * 64), shm, st, a);
  return hipGetLastError();
}

// Tuning constants of the strip launch (overridable at build time).
#ifndef ZG_STRIP_WAVES_PER_CU
#define ZG_STRIP_WAVES_PER_CU 16
#endif
#ifndef ZG_STRIP_SMALL_ITEMS_PER_CU
#define ZG_STRIP_SMALL_ITEMS_PER_CU 8
#endif
#ifndef ZG_STRIP_ENABLE
#define ZG_STRIP_ENABLE 1
#endif


bool strip_path_ok(int k) { return ZG_STRIP_ENABLE && k % 512 == 0 && k <= 8192; }

// decode-sized Q4_K projections take the strip kernel
#ifndef ZG_Q4K_STRIP
#define ZG_Q4K_STRIP 1
#endif

#ifndef ZG_ONEB_PER_CU
#define ZG_ONEB_PER_CU 4
#endif
#ifndef ZG_SWIGLU_GB
#define ZG_SWIGLU_GB 2
#endif
// groups per batch of the attention-merging O projection (Qwen3-1.7B
// decode: 1,500 tok/s at 2, 1,466 at 1, 1,489 at 3, 1,482 at 4: each
// workgroup merges the whole split output, so fewer rows per workgroup
// re-read it more often, and more leave CUs idle; with six attention
// splits: 1,486 at 2, 1,470 at 3, 1,472 at 4)
#ifndef ZG_ATTN_O_GB
#define ZG_ATTN_O_GB 2
#endif
#ifndef ZG_SWIGLU_DIG
#define ZG_SWIGLU_DIG 0
#endif
#ifndef ZG_STRIP_TALL_GB
#define ZG_STRIP_TALL_GB 4
#endif
#ifndef ZG_Q4K_TALL_GB
#define ZG_Q4K_TALL_GB 4
#endif

// Which strip launches take the integer activation form: 0 none, 1 the
// batch-loop launches, 2 every launch with fp32 activations.
#ifndef ZG_STRIP_DIG
#define ZG_STRIP_DIG 1
#endif

template <uint32_t QT, int PRO, int EPI, int GBATCH, int MAXT = 1024, bool SEG1 = false, int IL = 4>
static hipError_t launch_strip_gb1(const GemvArgs& a, int S, int nw, size_t items, hipStream_t st) {
  constexpr int PARTS = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr bool DIG1 = PRO != PRO_Q8X && (ZG_STRIP_DIG >= 2 || (EPI == EPI_SWIGLU && ZG_SWIGLU_DIG));  // one-batch
  // batch-loop launches (four groups per batch spill under the 1024-thread bound)
  constexpr bool DIGL = PRO != PRO_Q8X && ZG_STRIP_DIG >= 1 && (MAXT < 1024 || GBATCH < 4);
  // a workgroup never exceeds the kernel's thread bound (the compiler sized
  // its registers and index arithmetic for it)
  if (nw * 64 > MAXT) return hipErrorInvalidConfiguration;
  const int wps = nw / S;
  const size_t nbatch = (items + (size_t)wps * GBATCH - 1) / ((size_t)wps * GBATCH);
  const size_t shm = (size_t)2 * nw * GBATCH * PARTS * 16 * sizeof(float);
  if (MAXT == 1024 && nbatch <= (size_t)cu_count() * ZG_ONEB_PER_CU) {
    // one batch per workgroup (every decode-sized launch): no batch loop
    if (S == 4)
      hipLaunchKernelGGL((gemv_strip_kernel<QT, PRO, EPI, GBATCH, MAXT, SEG1, IL, true, 4, DIG1>),
                         dim3((unsigned)nbatch), dim3(nw * 64), shm, st, a, S);
    else if (S == 12)
      hipLaunchKernelGGL((gemv_strip_kernel<QT, PRO, EPI, GBATCH, MAXT, SEG1, IL, true, 12, DIG1>),
                         dim3((unsigned)nbatch), dim3(nw * 64), shm, st, a, S);
    else
      hipLaunchKernelGGL((gemv_strip_kernel<QT, PRO, EPI, GBATCH, MAXT, SEG1, IL, true, 0, DIG1>),
                         dim3((unsigned)nbatch), dim3(nw * 64), shm, st, a, S);
    return hipGetLastError();
  }
  // about 16 resident waves per CU; the remaining batches are looped over.
  // A 256-thread bound lets the compiler use more registers: the grid is
  // then what the occupancy query says fits.
  size_t per_cu = nw >= ZG_STRIP_WAVES_PER_CU ? 1 : (size_t)(ZG_STRIP_WAVES_PER_CU / nw);
  if (MAXT < 1024) {
    const int resident = resident_per_cu(
        reinterpret_cast<const void*>(gemv_strip_kernel<QT, PRO, EPI, GBATCH, MAXT, SEG1, IL, false, 0, DIGL>), nw * 64,
        shm);
    if ((size_t)resident < per_cu) per_cu = (size_t)resident;
  }
  const size_t cap = (size_t)cu_count() * per_cu;
  const size_t grid = nbatch < cap ? nbatch : cap;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((gemv_strip_kernel<QT, PRO, EPI, GBATCH, MAXT, SEG1, IL, false, 0, DIGL>), dim3((unsigned)grid),
                     dim3(nw * 64), shm, st, a, S);
  return hipGetLastError();
}

template <uint32_t QT, int PRO, int EPI, int GBATCH, int MAXT = 1024, int IL = 4>
static hipError_t launch_strip_gb(const GemvArgs& a, int S, int nw, size_t items, hipStream_t st) {
  if constexpr (EPI != EPI_SWIGLU) {
    if (a.nseg == 1) return launch_strip_gb1<QT, PRO, EPI, GBATCH, MAXT, true, IL>(a, S, nw, items, st);
  }
  return launch_strip_gb1<QT, PRO, EPI, GBATCH, MAXT, false, IL>(a, S, nw, items, st);
}

template <uint32_t QT, int PRO, int EPI, int IL = 4>
static hipError_t launch_strip(const GemvArgs& a, hipStream_t st) {
  const int S = a.k / 512;
  const int nw = S >= 3 ? S : 4;  // S in {1, 2} -> 4 waves: 4 / S waves per strip
  const size_t items = EPI == EPI_SWIGLU ? a.total_groups / 2 : a.total_groups;
  // small launches use short batches so that more workgroups share the
  // work; with argmax epilogues two batches in flight only fit the
  // 1024-thread register budget at two groups per batch
  const size_t wps = nw / S;
  if constexpr ((QT == Q4_0 || QT == Q4K) && (EPI == EPI_STORE || EPI == EPI_RESID) && PRO != PRO_ATTN) {
    // tall launches: the integer activation form needs more than the 128
    // registers of a 1024-thread bound, so its workgroups (one wave per
    // strip) take the tightest bound that holds them; past eight strips
    // the fp32 form
    if (items > (size_t)cu_count() * ZG_STRIP_SMALL_ITEMS_PER_CU * wps) {
      constexpr int TGB = QT == Q4K ? ZG_Q4K_TALL_GB : ZG_STRIP_TALL_GB;
      if (nw <= 4) return launch_strip_gb<QT, PRO, EPI, TGB, (ZG_STRIP_DIG >= 1 ? 256 : 1024), IL>(a, S, nw, items, st);
      if (nw <= 8) return launch_strip_gb<QT, PRO, EPI, TGB, (ZG_STRIP_DIG >= 1 ? 512 : 1024), IL>(a, S, nw, items, st);
      return launch_strip_gb<QT, PRO, EPI, TGB, 1024, IL>(a, S, nw, items, st);
    }
    // one-batch launches: groups per wave ~ items / (2 CUs), 1 to 3, so
    // that every CU gets about two workgroups (C1 6144x2048: three groups
    // per wave, 512 workgroups of four waves, 3.47 vs 3.56 us at two in a
    // probe)
    const size_t per = items / ((size_t)cu_count() * 2 * wps);
    if (per >= 3) return launch_strip_gb<QT, PRO, EPI, 3, 1024, IL>(a, S, nw, items, st);
    // one group per wave for the smallest launches, but two from 8 strips
    // on once every CU gets a workgroup: a wave's x quarters (2 KB) then
    // outweigh one group's weights (1.15 KB) (the 2048x6144 down projection:
    // 3.71 against 3.91 us in a probe)
    if (per < 2 && !(S >= 8 && per >= 1)) return launch_strip_gb<QT, PRO, EPI, 1, 1024, IL>(a, S, nw, items, st);
  }
  if constexpr (QT == Q8_0 && EPI != EPI_SWIGLU && PRO != PRO_ATTN) {
    // tall Q8_0X4 (the LM head): four groups per batch with 16-byte loads
    // need more than 128 registers, so these launches are 256-thread
    // workgroups (in_dim at most 2048)
    if (nw == 4 && items > (size_t)cu_count() * ZG_STRIP_SMALL_ITEMS_PER_CU * wps)
      return launch_strip_gb<QT, PRO, EPI, 4, 256, IL>(a, S, nw, items, st);
  }
  // gate|up (SwiGLU): two items (a gate and an up group each) per batch,
  // 768 one-batch workgroups at Qwen3-1.7B's FFN (decode 1,326 vs 1,297
  // tok/s with one item per batch and a batch loop)
  if constexpr (EPI == EPI_SWIGLU) return launch_strip_gb<QT, PRO, EPI, ZG_SWIGLU_GB, 1024, IL>(a, S, nw, items, st);
  if constexpr (PRO == PRO_ATTN) return launch_strip_gb<QT, PRO, EPI, ZG_ATTN_O_GB, 1024, IL>(a, S, nw, items, st);
  return launch_strip_gb<QT, PRO, EPI, 2, 1024, IL>(a, S, nw, items, st);
}

// Tall single-projection Q8_0X4 launches (the LM head: 37,984 groups) take
// the strip kernel with four groups per batch and cache-allocating loads
// (66 vs 85 us for 151936x2048 as a standalone call); smaller Q8_0X4
// launches, and tall ones that stream their weights (kGemvStream: inside
// the decode step the cache-allocating read would evict the KV cache, a net
// loss there), keep the segment-streaming kernel and its nontemporal loads.
#ifndef ZG_TALL_MIN_GROUPS
#define ZG_TALL_MIN_GROUPS 8192
#endif
static bool tall_path_ok(const GemvArgs& a) {
  return a.nseg == 1 && !(a.flags & kGemvStream) && a.k % 512 == 0 && a.k <= 2048 &&
         a.total_groups >= ZG_TALL_MIN_GROUPS;
}
#ifndef ZG_STREAM_STRIP
#define ZG_STREAM_STRIP 1
#endif
#ifndef ZG_STREAM_IL
#define ZG_STREAM_IL 3
#endif
static bool tall_stream_ok(const GemvArgs& a) {
  return a.nseg == 1 && (a.flags & kGemvStream) && a.k % 512 == 0 && a.k <= 2048 &&
         a.total_groups >= ZG_TALL_MIN_GROUPS;
}

// ---------------------------------------------------------------------------
// LDS-staged strip GEMV for tall single-projection X4 launches, in_dim 2048.
//
// The strip kernel's per-lane loads span ~1.1 KB at a 72/136-byte stride;
// here the workgroup streams each batch of G consecutive groups (G x 64
// group-blocks, contiguous) into LDS with gfx950's direct global-to-LDS
// 16-byte loads (global_load_lds_dwordx4: consecutive lanes, consecutive 16
// bytes, no VGPR staging), double-buffered, and the lanes decode their
// (block, row) pieces from LDS with the strip kernel's lane map (wave w =
// strip w, lane (b, r)).  Every wave issues exactly ROUNDS loads per batch
// (chunk indices clamped into the tensor, each buffer padded to whole
// rounds), so one s_waitcnt count covers a batch.
// ---------------------------------------------------------------------------
template <uint32_t QT>
__device__ __forceinline__ void lds_lane(LaneW<QT>& L, const uint8_t* gb, int r) {
  constexpr int QW = StripGeom<QT>::QW;
  const u32x2* p = reinterpret_cast<const u32x2*>(gb + 8 + 4 * QW * r);
#pragma unroll
  for (int i = 0; i < QW / 2; i++) {
    const u32x2 v = p[i];
    L.q[2 * i] = v.x;
    L.q[2 * i + 1] = v.y;
  }
  L.d = *reinterpret_cast<const uint16_t*>(gb + 2 * r);
}

// Workgroup barrier after this wave's LDS reads and writes have completed
// (its global loads may still be in flight).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <uint32_t QT, int G>
struct LdsGeom {
  static constexpr int GS = 64 * StripGeom<QT>::GB;         // group stream bytes at in_dim 2048
  static constexpr int ROUNDS = (G * GS / 16 + 255) / 256;  // 16-byte loads per thread per batch
  static constexpr int BUF = ROUNDS * 4096;                 // buffer bytes (whole rounds)
  static constexpr size_t SHM = 2 * (size_t)BUF + 2 * 4 * G * 16 * sizeof(float);
};

template <uint32_t QT, int PRO, int EPI, int G, bool STREAM>
__global__ __launch_bounds__(256) void gemv_lds_kernel(GemvArgs a) {
  using Geo = LdsGeom<QT, G>;
  constexpr int GBY = StripGeom<QT>::GB, GS = Geo::GS, ROUNDS = Geo::ROUNDS, BUF = Geo::BUF;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_stage[];  // [2][BUF] bytes, then [2][4][G][16] partials
  float* part = reinterpret_cast<float*>(lds_stage + 2 * BUF);
  __shared__ float red[4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = lane >> 2, r = lane & 3;
  const int kb = wave * 16 + b;
  const int items = (int)a.total_groups;
  const int nbatch = (items + G - 1) / G;
  const size_t nchunk = (size_t)items * GS / 16;  // 16-byte chunks of the tensor
  const uint8_t* w = a.seg[0].w;
  // batch `batch` into buffer `buf`: chunk c of the batch (thread c % 256,
  // round c / 256) from global chunk batch*G*GS/16 + c, clamped into the
  // tensor (a clamped chunk lands in a group whose result is dropped); the
  // padding after the batch re-reads the batch's own first chunks (lines
  // this workgroup is fetching anyway, not the next batch's)
  auto issue = [&](int batch, int buf) {
    constexpr int BC = G * GS / 16;  // chunks per batch
    const size_t c0 = (size_t)batch * BC;
#pragma unroll
    for (int q = 0; q < ROUNDS; q++) {
      int cl = q * 256 + (int)threadIdx.x;
      if (q * 256 + 255 >= BC) cl = cl >= BC ? cl - BC : cl;
      const size_t c = min(c0 + (size_t)cl, nchunk - 1);
      __builtin_amdgcn_global_load_lds(
          w + 16 * c,
          (__attribute__((address_space(3))) void*)(lds_stage + buf * BUF + 16 * (q * 256 + wave * 64)), 16, 0,
          STREAM ? 2 : 0);
    }
  };
  float4 xb[2], gw[2];
  const float4* x4 = reinterpret_cast<const float4*>(a.x + 32 * kb);
  xb[0] = x4[r];
  xb[1] = x4[4 + r];
  if (PRO == PRO_RMSNORM) {
    const float4* g4 = reinterpret_cast<const float4*>(a.norm_w + 32 * kb);
    gw[0] = g4[r];
    gw[1] = g4[4 + r];
  }
  const int b0 = blockIdx.x, bstep = gridDim.x;
  issue(b0, 0);
  if (PRO == PRO_RMSNORM) {
    float ssq = 0.0f;
#pragma unroll
    for (int c = 0; c < 2; c++) ssq += xb[c].x * xb[c].x + xb[c].y * xb[c].y + xb[c].z * xb[c].z + xb[c].w * xb[c].w;
    ssq = wave_sum(ssq);
    if (lane == 0) red[wave] = ssq;
#pragma unroll
    for (int c = 0; c < 2; c++)
      xb[c] = make_float4(xb[c].x * gw[c].x, xb[c].y * gw[c].y, xb[c].z * gw[c].z, xb[c].w * gw[c].w);
  }
  XDig xd;
  const bool fp32 = __builtin_amdgcn_ballot_w64(xdig_quad(xb[0], xb[1], xd)) != 0;
  uint64_t key = 0;
  int i = 0;
  for (int batch = b0; batch < nbatch; batch += bstep, i++) {
    const int cur = i & 1;
    const bool more = batch + bstep < nbatch;
    if (more) {
      issue(batch + bstep, cur ^ 1);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(ROUNDS) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    // the batch's bytes are in LDS for every wave (a plain s_barrier: the
    // compiler's workgroup fence would also wait for the next batch's
    // loads, which are LDS writes to it)
    lds_barrier();
    float* pb = part + cur * 4 * G * 16;
#pragma unroll
    for (int j = 0; j < G; j++) {
      LaneW<QT> L;
      lds_lane<QT>(L, lds_stage + cur * BUF + j * GS + kb * GBY, r);
      float dot;
      if (!fp32) {
        dot = strip_dot_dig<QT>(L, xd);
      } else {
        float4 xf[8];
        strip_x_block<PRO>(xf, a, kb);
        float t = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) t += (xf[c].x + xf[c].y) + (xf[c].z + xf[c].w);
        dot = strip_dot<QT>(L, xf, (QT == Q4_0 ? -8.0f : -128.0f) * t);
      }
      const float v = row_sum4(dot);
      if ((lane & 15) < 4) pb[(wave * G + j) * 16 + (lane >> 4) * 4 + r] = v;
    }
    lds_barrier();  // partials visible; every wave is done with this buffer
    const int tt = threadIdx.x;
    if (tt < G * 4) {
      const int j = tt >> 2, rr = tt & 3;
      const int item = batch * G + j;
      if (item < items) {
        float acc = 0.0f;
#pragma unroll
        for (int st = 0; st < 4; st++) {
          const float* q = pb + (st * G + j) * 16 + rr;
          acc += (q[0] + q[4]) + (q[8] + q[12]);
        }
        if (PRO == PRO_RMSNORM) acc *= 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)a.k + a.eps);
        const GemvSeg& sg = a.seg[0];
        const uint32_t row = 4 * (uint32_t)item + (uint32_t)rr;
        if (row >= sg.row_lo && row < sg.row_hi) {
          if (EPI == EPI_RESID) {
            store_out(sg.y + row, sg.resid[row] + acc);
          } else {
            if (sg.y) store_out(sg.y + row, acc);
            if (EPI == EPI_ARGMAX && !(acc != acc)) {
              const uint64_t kk = argmax_key(acc, row);
              key = kk > key ? kk : key;
            }
          }
        }
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
}

#ifndef ZG_LDS_TALL_Q4
#define ZG_LDS_TALL_Q4 1
#endif
#ifndef ZG_LDS_TALL
#define ZG_LDS_TALL 1
#endif
// Groups per batch.  Q4_0 4 (18,432 bytes in five rounds, three workgroups
// per CU): 151936x2048 31.0-31.6 us against 31.8 with eight (36,864 bytes,
// two workgroups per CU), 31.1-31.4 with three, 32.9 with two.  Q8_0 4
// (34,816 bytes in nine rounds, two workgroups per CU; eight groups leave
// one workgroup per CU: 65.2 vs 58.8 us for the LM head).
#ifndef ZG_LDS_G_Q4
#define ZG_LDS_G_Q4 4
#endif
#ifndef ZG_LDS_G_Q8
#define ZG_LDS_G_Q8 4
#endif
template <uint32_t QT>
constexpr int lds_groups() {
  return QT == Q4_0 ? ZG_LDS_G_Q4 : ZG_LDS_G_Q8;
}
// Q4_0X4 launches of at least this many groups take the LDS-staged kernel
// (151936x2048: 31.1-31.6 against 32.2 us for the register strip kernel in
// the same runs); shorter ones keep the strip kernel (49152x2048: 12.4
// against 12.9-13.1 us staged).
#ifndef ZG_LDS_Q4_MIN_GROUPS
#define ZG_LDS_Q4_MIN_GROUPS 24576
#endif
// The LDS-staged kernel streams with nontemporal loads also outside the
// decode step (cache-allocating: the LM head 60.9 against 54.8 us,
// 151936x2048 Q4_0X4 32.6 against 30.9 us).
// The LDS-staged kernel takes tall Q8_0X4 single projections at in_dim 2048
// (the LM head: 58.8 us against 64.2 us for the register strip kernel's
// cache-allocating loads and 77 us for its nontemporal ones), the tallest
// Q4_0X4 ones, and streamed tall launches of either type (inside the
// decode step its nontemporal read leaves the KV cache in the caches).
// One-batch launches gain nothing from staging (C1 6144x2048: 4.8 vs
// 3.5 us).
template <uint32_t QT>
static bool lds_tall_ok(const GemvArgs& a) {
  return ZG_LDS_TALL && a.nseg == 1 && a.k == 2048 && a.total_groups >= ZG_TALL_MIN_GROUPS &&
         (QT == Q8_0 || (ZG_LDS_TALL_Q4 && a.total_groups >= ZG_LDS_Q4_MIN_GROUPS) || (a.flags & kGemvStream));
}

template <uint32_t QT, int PRO, int EPI, bool STREAM>
static hipError_t launch_lds(const GemvArgs& a, hipStream_t st) {
  constexpr int G = lds_groups<QT>();
  const size_t shm = LdsGeom<QT, G>::SHM;
  const int resident =
      resident_per_cu(reinterpret_cast<const void*>(gemv_lds_kernel<QT, PRO, EPI, G, STREAM>), 256, shm, true);
  const size_t nbatch = (a.total_groups + G - 1) / G;
  const size_t cap = (size_t)cu_count() * resident;
  const size_t grid = nbatch < cap ? nbatch : cap;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((gemv_lds_kernel<QT, PRO, EPI, G, STREAM>), dim3((unsigned)grid), dim3(256), shm, st, a);
  return hipGetLastError();
}

// Q4_0X4 takes the strip kernel (measured faster at every decode shape).
template <uint32_t QT, int PRO, int EPI>
static hipError_t launch_x4_any(const GemvArgs& a, hipStream_t st) {
  if (a.flags & kGemvSplit) {
    // split-scale groups: the strip kernel's forms only
    if (!strip_path_ok(a.k)) return hipErrorInvalidValue;
    if constexpr (PRO == PRO_ATTN) {
      if (QT != Q4_0 || a.attn_nsplit < 1 || a.attn_nsplit > kAttnSplits || !attn_merge_hd_ok(QT, a.attn_hd) ||
          a.k % a.attn_hd != 0)
        return hipErrorInvalidValue;
    }
    return launch_strip<QT, PRO, EPI, 5>(a, st);
  }
  if constexpr (PRO == PRO_Q8X) {
    // Q8_0 activations: strip kernel only
    if (strip_path_ok(a.k)) return launch_strip<QT, PRO, EPI>(a, st);
    return hipErrorInvalidValue;
  } else if constexpr (PRO == PRO_ATTN) {
    // only the Q4_0 strip kernel merges attention splits
    if constexpr (QT == Q4_0) {
      if (strip_path_ok(a.k) && a.attn_nsplit >= 1 && a.attn_nsplit <= kAttnSplits && attn_merge_hd_ok(QT, a.attn_hd) &&
          a.k % a.attn_hd == 0)
        return launch_strip<QT, PRO, EPI>(a, st);
    }
    return hipErrorInvalidValue;
  } else {
    if constexpr ((PRO == PRO_PLAIN || PRO == PRO_RMSNORM) && (EPI == EPI_STORE || EPI == EPI_ARGMAX)) {
      if (lds_tall_ok<QT>(a)) return launch_lds<QT, PRO, EPI, true>(a, st);
    }
    if constexpr (QT == Q8_0 && (EPI == EPI_STORE || EPI == EPI_ARGMAX)) {
      if (tall_path_ok(a)) return launch_strip<QT, PRO, EPI>(a, st);
      if (ZG_STREAM_STRIP && tall_stream_ok(a)) return launch_strip<QT, PRO, EPI, ZG_STREAM_IL>(a, st);
    }
    if constexpr (QT == Q4_0) {
      if (strip_path_ok(a.k)) return launch_strip<QT, PRO, EPI>(a, st);
    }
    if constexpr (QT == Q8_0) {
      // decode-sized Q8_0X4 launches (fused Q|K|V): the one-batch strip
      // form; streamed ones (the decode step's LM head) keep the segment
      // kernel's nontemporal loads
      if (strip_path_ok(a.k) && !(a.flags & kGemvStream) && a.total_groups <= (uint32_t)cu_count() * 8)
        return launch_strip<QT, PRO, EPI>(a, st);
    }
    return launch_x4<QT, PRO, EPI>(a, st);
  }
}

// Q4_0X4 or plain Q4_0 weights
bool attn_merge_gemv_ok(uint32_t qt, uint32_t il, size_t k) {
  return qt == Q4_0 && (il == 4 || il == 5) && k <= 8192 && strip_path_ok((int)k);
}

template <uint32_t QT>
static hipError_t dispatch_x4_qt(const GemvArgs& a, int pro, int epi, hipStream_t st) {
  if (pro == PRO_PLAIN && epi == EPI_STORE) return launch_x4_any<QT, PRO_PLAIN, EPI_STORE>(a, st);
  if (pro == PRO_PLAIN && epi == EPI_RESID) return launch_x4_any<QT, PRO_PLAIN, EPI_RESID>(a, st);
  if (pro == PRO_PLAIN && epi == EPI_ARGMAX) return launch_x4_any<QT, PRO_PLAIN, EPI_ARGMAX>(a, st);
  if (pro == PRO_RMSNORM && epi == EPI_STORE) return launch_x4_any<QT, PRO_RMSNORM, EPI_STORE>(a, st);
  if (pro == PRO_RMSNORM && epi == EPI_ARGMAX) return launch_x4_any<QT, PRO_RMSNORM, EPI_ARGMAX>(a, st);
  if (pro == PRO_RMSNORM && epi == EPI_SWIGLU) return launch_x4_any<QT, PRO_RMSNORM, EPI_SWIGLU>(a, st);
  if (pro == PRO_PLAIN && epi == EPI_SWIGLU) return launch_x4_any<QT, PRO_PLAIN, EPI_SWIGLU>(a, st);
  if (pro == PRO_ATTN && epi == EPI_RESID) return launch_x4_any<QT, PRO_ATTN, EPI_RESID>(a, st);
  if (pro == PRO_Q8X && epi == EPI_STORE) return launch_x4_any<QT, PRO_Q8X, EPI_STORE>(a, st);
  return hipErrorInvalidValue;
}

// Plain row-major Q4_0 / Q8_0 (GGUF and .smodel-v1 layouts) through the
// strip kernel: rows in fours, in_dim a multiple of 512 up to 8192.
bool plain_strip_ok(uint32_t qt, uint32_t il, size_t k, size_t n, const void* w, const void* x) {
  return il == 1 && (qt == Q4_0 || qt == Q8_0) && strip_path_ok((int)k) && n % 4 == 0 &&
         (reinterpret_cast<uintptr_t>(w) & 1u) == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

// Plain rows take no rmsnorm-store, SwiGLU or attention-merge forms: the
// model interleaves its plain-row Q4_0 / Q8_0 tensors to X4 at creation, and
// the operator API reaches plain rows only without a prologue or as an LM
// head (rmsnorm + argmax).
template <uint32_t QT>
static hipError_t dispatch_plain_qt(const GemvArgs& a, int pro, int epi, hipStream_t st) {
  if (pro == PRO_PLAIN && epi == EPI_STORE) return launch_strip<QT, PRO_PLAIN, EPI_STORE, 1>(a, st);
  if (pro == PRO_PLAIN && epi == EPI_RESID) return launch_strip<QT, PRO_PLAIN, EPI_RESID, 1>(a, st);
  if (pro == PRO_PLAIN && epi == EPI_ARGMAX) return launch_strip<QT, PRO_PLAIN, EPI_ARGMAX, 1>(a, st);
  if (pro == PRO_RMSNORM && epi == EPI_ARGMAX) {
    // a streamed LM head (the decode step's): 1,032 vs 1,005 tok/s for the
    // plain-layout Qwen3-1.7B-shape decode
    if (a.flags & kGemvStream) return launch_strip<QT, PRO_RMSNORM, EPI_ARGMAX, 2>(a, st);
    return launch_strip<QT, PRO_RMSNORM, EPI_ARGMAX, 1>(a, st);
  }
  if (pro == PRO_Q8X && epi == EPI_STORE) return launch_strip<QT, PRO_Q8X, EPI_STORE, 1>(a, st);
  return hipErrorInvalidValue;
}

// Q4_K rows through the strip kernel (lane units of 32 elements, four rows
// per group): in_dim a multiple of 512 up to 8192, rows in fours, weights
// and x 16-byte aligned.
bool kq_strip_ok(uint32_t qt, uint32_t il, size_t k, size_t n, const void* w, const void* x) {
  if (!ZG_Q4K_STRIP || qt != Q4K || il != 1 || !strip_path_ok((int)k) || n % 4 != 0 ||
      (reinterpret_cast<uintptr_t>(w) & 15u) != 0 || (reinterpret_cast<uintptr_t>(x) & 15u) != 0)
    return false;
  // one-batch launches only (the tall batch-loop form measured slower than
  // the Q4_K strip kernel of zg_kquant.hip: 13.4 vs 11.8 us at 14336x4096
  // with four groups per batch, 13.3 at two; one group per batch 12.0, and
  // fp32 activations at two groups 11.85 vs 11.9: no form beats it).
  // A Q6_K unit of the same shape (three 16-byte quant loads at 2-byte
  // alignment, 15 registers per row) was slower than zg_kquant.hip's Q6_K
  // kernels at the decode shapes: down 7.72 vs 7.25 us, attn_v 3.99 vs 3.75.
  // The one-batch launches decode with fp32 activations: the integer-digit
  // form there took the Q4_K_M decode from 1,160 to 1,007 tok/s (SwiGLU
  // launch only) and 964 tok/s (every Q4_K launch)
  const int S = (int)k / 512, nw = S >= 3 ? S : 4;  // S >= 1 here
  return ZG_Q4K_STRIP >= 2 || n / 4 <= (size_t)cu_count() * ZG_STRIP_SMALL_ITEMS_PER_CU * (size_t)(nw / S);
}

// The strip kernel's merge prologue takes these attention splits.
bool attn_merge_strip_ok(int nsplit, int hd, size_t k) {
  return nsplit >= 1 && nsplit <= kAttnSplits && attn_merge_hd_ok(Q4K, hd) && k % (size_t)hd == 0;
}

static hipError_t dispatch_q4k_strip(const GemvArgs& a, int pro, int epi, hipStream_t st) {
  if (pro == PRO_PLAIN && epi == EPI_STORE) return launch_strip<Q4K, PRO_PLAIN, EPI_STORE, 1>(a, st);
  if (pro == PRO_PLAIN && epi == EPI_RESID) return launch_strip<Q4K, PRO_PLAIN, EPI_RESID, 1>(a, st);
  if (pro == PRO_RMSNORM && epi == EPI_STORE) return launch_strip<Q4K, PRO_RMSNORM, EPI_STORE, 1>(a, st);
  if (pro == PRO_RMSNORM && epi == EPI_SWIGLU) return launch_strip<Q4K, PRO_RMSNORM, EPI_SWIGLU, 1>(a, st);
  if (pro == PRO_ATTN && epi == EPI_RESID && attn_merge_strip_ok(a.attn_nsplit, a.attn_hd, (size_t)a.k))
    return launch_strip<Q4K, PRO_ATTN, EPI_RESID, 1>(a, st);
  return hipErrorInvalidValue;
}

hipError_t launch_gemv_plain(const GemvArgs& a, uint32_t qt, int pro, int epi, hipStream_t st) {
  if (qt == Q4_0) return dispatch_plain_qt<Q4_0>(a, pro, epi, st);
  if (qt == Q8_0) return dispatch_plain_qt<Q8_0>(a, pro, epi, st);
  if (qt == Q4K) return dispatch_q4k_strip(a, pro, epi, st);
  return hipErrorInvalidValue;
}

hipError_t launch_gemv_x4(const GemvArgs& a, uint32_t qt, int pro, int epi, hipStream_t st) {
  if (qt == Q4_0) return dispatch_x4_qt<Q4_0>(a, pro, epi, st);
  if (qt == Q8_0) return dispatch_x4_qt<Q8_0>(a, pro, epi, st);
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
    const size_t nseg = (a.k / 32 + 63) / 64;
    const size_t units = (a.rows / 4) * nseg;
    const uint32_t grid = (uint32_t)((units + kNW - 1) / kNW);
    if (a.qt == Q4_0) hipLaunchKernelGGL(dequant_x4_stream_kernel<Q4_0>, dim3(grid), dim3(kNW * 64), 0, st, a);
    else hipLaunchKernelGGL(dequant_x4_stream_kernel<Q8_0>, dim3(grid), dim3(kNW * 64), 0, st, a);
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

hipError_t launch_read_floor(const void* src, size_t bytes, int loads_per_thread, uint32_t* sink, hipStream_t st) {
  const size_t n16 = bytes / 16;
  const size_t per_wg = (size_t)256 * loads_per_thread;
  const uint32_t grid = (uint32_t)((n16 + per_wg - 1) / per_wg);
  if (grid == 0) return hipSuccess;
  const u32x4* s4 = static_cast<const u32x4*>(src);
  switch (loads_per_thread) {
    case 1: hipLaunchKernelGGL(read_floor_kernel<1>, dim3(grid), dim3(256), 0, st, s4, n16, sink); break;
    case 2: hipLaunchKernelGGL(read_floor_kernel<2>, dim3(grid), dim3(256), 0, st, s4, n16, sink); break;
    case 4: hipLaunchKernelGGL(read_floor_kernel<4>, dim3(grid), dim3(256), 0, st, s4, n16, sink); break;
    case 8: hipLaunchKernelGGL(read_floor_kernel<8>, dim3(grid), dim3(256), 0, st, s4, n16, sink); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_strip_loads(const uint8_t* w, const float* x, size_t rows, uint32_t* sink, hipStream_t st) {
  const int groups = (int)(rows / 4);
  if (groups == 0) return hipSuccess;
  // the strip GEMV's forms: one batch of three groups per workgroup when
  // that gives at most ZG_ONEB_PER_CU workgroups per CU (C1's 512), else
  // four-group batches over four resident workgroups per CU
  const int nb3 = (groups + 2) / 3;
  if (nb3 <= cu_count() * ZG_ONEB_PER_CU) {
    if (x) hipLaunchKernelGGL((strip_load_kernel<3, true, true>), dim3(nb3), dim3(256), 0, st, w, x, groups, sink);
    else hipLaunchKernelGGL((strip_load_kernel<3, true, false>), dim3(nb3), dim3(256), 0, st, w, x, groups, sink);
  } else {
    const int nb4 = (groups + 3) / 4, grid = std::min(nb4, cu_count() * 4);
    if (x) hipLaunchKernelGGL((strip_load_kernel<4, false, true>), dim3(grid), dim3(256), 0, st, w, x, groups, sink);
    else hipLaunchKernelGGL((strip_load_kernel<4, false, false>), dim3(grid), dim3(256), 0, st, w, x, groups, sink);
  }
  return hipGetLastError();
}

hipError_t launch_fill_u64(uint64_t* p, uint64_t v, hipStream_t st) {
  hipLaunchKernelGGL(fill_u64_kernel, dim3(1), dim3(1), 0, st, p, v);
  return hipGetLastError();
}

}  // namespace zg
