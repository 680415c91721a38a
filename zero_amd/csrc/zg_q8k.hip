// zg_q8k.hip -- the Q4_K x Q8_K integer path for gfx950.
//
// Restates the reference's VNNI path (kernel/src/arch/x86_64/math/vnni.rs,
// feature "vnni-acceleration"): the activation vector is quantized to Q8_K
// (quantize_row_q8k, :78-170) and each Q4_K row is dotted with it in
// integers (linear_q4k_vnni_range, :258-476); VPDPBUSD becomes v_dot4_i32_i8.
//
// Q8_K block, 292 bytes (the reference's packed form, kept as is): f32 d,
// 256 int8 q, 16 int16 sums of 16 q each.
//
// Per Q4_K superblock b of a row the reference forms, exactly in integers,
//   int_sum = sum_g sc_g * sum_{i in sub-block g} nibble_i * q_i
//   min_sum = sum_g m_g * (bsum[2g] + bsum[2g+1])
// and accumulates in f32: dot += (d_w d8) * (float)int_sum,
// min += (dmin_w d8) * (float)min_sum; the row is dot - min.  Here the
// integer sums of a superblock are formed by its 8 lanes (exact, any order)
// and the per-superblock f32 products are the reference's; only the order
// in which the superblock terms are added differs (wave and strip sums).
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/zero_gpu.h"
#include "zg_device.h"
#include "zg_internal.h"
#include "zg_kernels.h"

using namespace zg;

namespace zg {

constexpr int kQ8kBytes = 292;

// dword-aligned 128-bit loads (Q8_K blocks start at multiples of 4 bytes)
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

// quantize_row_q8k: one wave per 256-value block, 4 values per lane
// (q8k_block_lane); bsums are exact int sums of 16 (int16).
__global__ __launch_bounds__(64) void quantize_q8k_kernel(const float* __restrict__ x, uint8_t* __restrict__ out) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const float* v = x + (size_t)b * 256;
  uint8_t* o = out + (size_t)b * kQ8kBytes;
  const float4 f = reinterpret_cast<const float4*>(v)[lane];
  const float e[4] = {f.x, f.y, f.z, f.w};
  int q[4];
  float d;
  reinterpret_cast<uint32_t*>(o + 4)[lane] = q8k_block_lane(lane, e, q, d);
  // sums of 16: four lanes per group
  int s16 = (q[0] + q[1]) + (q[2] + q[3]);
  s16 += __shfl_xor(s16, 1, 64);
  s16 += __shfl_xor(s16, 2, 64);
  if ((lane & 3) == 0) {
    const int c = s16 < -32768 ? -32768 : (s16 > 32767 ? 32767 : s16);
    reinterpret_cast<int16_t*>(o + 260)[lane >> 2] = (int16_t)c;
  }
  if (lane == 0) reinterpret_cast<float*>(o)[0] = d;
}

// Scale and min j (0..7) of a Q4_K superblock from its 12 scale bytes
// (words s[0..2]), the get_scale_min_k4 rule (dequant.rs:75-85), as ints.
__device__ __forceinline__ void scale_min_i(const uint32_t* s, int j, int& sc, int& mn) {
  auto byte = [&](int i) -> int { return (int)((s[i >> 2] >> (8 * (i & 3))) & 0xFFu); };
  if (j < 4) {
    sc = byte(j) & 63;
    mn = byte(j + 4) & 63;
  } else {
    sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
    mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
  }
}

// The lane's fixed share of the activations: lane (superblock sl = lane / 8,
// j = sub-block pair 0..3, h = half 0..1) covers elements 64 j + 16 h ..+16
// (sub-block 2j) and 64 j + 32 + 16 h ..+16 (sub-block 2j+1), i.e. the Q4_K
// qs bytes [32 j + 16 h, +16) (low nibbles, then high nibbles).
struct Q8kX {
  u32x4 qa, qb;   // 16 int8 each
  int bsa, bsb;   // bsum[4j + h], bsum[4j + 2 + h]
  float d8;
};

__device__ __forceinline__ Q8kX q8k_lane(const uint8_t* q8k, int sb, int lane) {
  const int j = (lane >> 1) & 3, h = lane & 1;
  const uint8_t* blk = q8k + (size_t)sb * kQ8kBytes;
  Q8kX r;
  const u32x4a4 a = *reinterpret_cast<const u32x4a4*>(blk + 4 + 64 * j + 16 * h);
  const u32x4a4 bb = *reinterpret_cast<const u32x4a4*>(blk + 4 + 64 * j + 32 + 16 * h);
  r.qa = u32x4{a.x, a.y, a.z, a.w};
  r.qb = u32x4{bb.x, bb.y, bb.z, bb.w};
  const int16_t* bs = reinterpret_cast<const int16_t*>(blk + 260);
  r.bsa = bs[4 * j + h];
  r.bsb = bs[4 * j + 2 + h];
  r.d8 = *reinterpret_cast<const float*>(blk);
  return r;
}

struct Q4kW {
  u32x4 hdr, q;  // d, dmin, 12 scale bytes; the lane's 16 qs bytes
};

__device__ __forceinline__ void q4k_load(Q4kW& L, const uint8_t* blk, int lane) {
  const int j = (lane >> 1) & 3, h = lane & 1;
  L.hdr = *reinterpret_cast<const u32x4*>(blk);
  L.q = *reinterpret_cast<const u32x4*>(blk + 16 + 32 * j + 16 * h);
}

// This lane's integer terms of the superblock: sc * (nibbles . q) and
// m * bsum for its two half sub-blocks.
__device__ __forceinline__ void q4k_q8k_lane(const Q4kW& L, const Q8kX& x, int lane, int& isum, int& msum) {
  const int j = (lane >> 1) & 3;
  const uint32_t s[3] = {L.hdr.y, L.hdr.z, L.hdr.w};
  int scA, mA, scB, mB;
  scale_min_i(s, 2 * j, scA, mA);
  scale_min_i(s, 2 * j + 1, scB, mB);
  const uint32_t q[4] = {L.q.x, L.q.y, L.q.z, L.q.w};
  const uint32_t xa[4] = {x.qa.x, x.qa.y, x.qa.z, x.qa.w}, xb[4] = {x.qb.x, x.qb.y, x.qb.z, x.qb.w};
  // four chains (a dependent v_dot4_i32_i8 issues ~16 cycles after its
  // predecessor); integer sums, so the split leaves the result unchanged
  int sa = 0, sbv = 0, sa1 = 0, sb1 = 0;
#pragma unroll
  for (int c = 0; c < 4; c += 2) {
    sa = __builtin_amdgcn_sdot4((int)(q[c] & 0x0F0F0F0Fu), (int)xa[c], sa, false);
    sbv = __builtin_amdgcn_sdot4((int)((q[c] >> 4) & 0x0F0F0F0Fu), (int)xb[c], sbv, false);
    sa1 = __builtin_amdgcn_sdot4((int)(q[c + 1] & 0x0F0F0F0Fu), (int)xa[c + 1], sa1, false);
    sb1 = __builtin_amdgcn_sdot4((int)((q[c + 1] >> 4) & 0x0F0F0F0Fu), (int)xb[c + 1], sb1, false);
  }
  sa += sa1;
  sbv += sb1;
  isum = scA * sa + scB * sbv;
  msum = mA * x.bsa + mB * x.bsb;
}

// Strip GEMV: the K axis is cut into strips of 8 superblocks; a wave owns
// one strip (its lanes' Q8_K activations stay in registers) and walks
// batches of rows, two batches of loads in flight (clamped unconditional
// loads).  Per row: the 8 lanes of each superblock sum their integer terms
// (exact), the superblock's first lane forms the reference's two f32
// products, the wave sums them (DPP), strips are added through LDS in a
// fixed order, and the row is dot - min.
template <int RB>
__global__ __launch_bounds__(1024) void q4k_q8k_strip_kernel(const uint8_t* __restrict__ w,
                                                             const uint8_t* __restrict__ q8k, float* __restrict__ y,
                                                             int nsb, int nrows, int S) {
  __shared__ float part[2][32][RB][2];  // [buffer][wave][row of the batch][dot, min]
  const int NW = blockDim.x >> 6;
  const int WPS = NW / S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = wave % S, sub = wave / S;
  const int sb_raw = strip * 8 + (lane >> 3);
  const bool live = sb_raw < nsb;
  const int sb = live ? sb_raw : nsb - 1;  // clamped: a dead lane's terms are discarded
  const size_t rowbytes = (size_t)nsb * 144;
  const int per_batch = WPS * RB;
  const int nbatch = (nrows + per_batch - 1) / per_batch;
  auto load_batch = [&](Q4kW (&L)[RB], int batch) {
    const int base = batch * per_batch + sub * RB;
#pragma unroll
    for (int j = 0; j < RB; j++) {
      const size_t row = (size_t)min(base + j, nrows - 1);
      q4k_load(L[j], w + row * rowbytes + (size_t)sb * 144, lane);
    }
  };
  Q4kW LA[RB], LB[RB];
  const int b0 = blockIdx.x, bstep = gridDim.x;
  const Q8kX x = q8k_lane(q8k, sb, lane);
  load_batch(LA, b0);
  if (b0 + bstep < nbatch) load_batch(LB, b0 + bstep);
  auto process = [&](const Q4kW (&L)[RB], int batch, int buf) {
#pragma unroll
    for (int j = 0; j < RB; j++) {
      int isum, msum;
      q4k_q8k_lane(L[j], x, lane, isum, msum);
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) {
        isum += __shfl_xor(isum, o, 64);
        msum += __shfl_xor(msum, o, 64);
      }
      float pd = 0.0f, pm = 0.0f;
      if ((lane & 7) == 0 && live) {
        const float dw = half_bits_to_f32(L[j].hdr.x), dmw = half_bits_to_f32(L[j].hdr.x >> 16);
        pd = (dw * x.d8) * (float)isum;
        pm = (dmw * x.d8) * (float)msum;
      }
      pd = wave_sum(pd);
      pm = wave_sum(pm);
      if (lane == 0) {
        part[buf][wave][j][0] = pd;
        part[buf][wave][j][1] = pm;
      }
    }
    __syncthreads();
    const int tt = threadIdx.x;
    if (tt < per_batch) {
      const int su = tt / RB, j = tt % RB;
      const int ri = batch * per_batch + su * RB + j;
      if (ri < nrows) {
        float dsum = 0.0f, msum = 0.0f;
        for (int st = 0; st < S; st++) {
          dsum += part[buf][su * S + st][j][0];
          msum += part[buf][su * S + st][j][1];
        }
        y[ri] = dsum - msum;
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
}

static int q8k_cu_count() {
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

constexpr int kQ8kMaxStrips = 16;  // in_dim up to 32768

static zg_status q8k_check(zg_ctx* ctx, size_t in_dim, size_t out_dim) {
  if (in_dim == 0 || in_dim % 256) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: in_dim %zu %% 256 != 0", in_dim);
  if ((in_dim / 256 + 7) / 8 > (size_t)kQ8kMaxStrips)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: in_dim %zu above %d", in_dim, kQ8kMaxStrips * 2048);
  if (out_dim > (size_t)INT32_MAX) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: out_dim too large");
  return ZG_OK;
}

static zg_status run_q8k_quant(zg_ctx* ctx, const float* x, uint8_t* q8k, size_t n, hipStream_t st) {
  if (reinterpret_cast<uintptr_t>(x) & 15) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: activations misaligned");
  if (reinterpret_cast<uintptr_t>(q8k) & 3) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: output misaligned");
  hipLaunchKernelGGL(quantize_q8k_kernel, dim3((unsigned)(n / 256)), dim3(64), 0, st, x, q8k);
  return hip_check(ctx, hipGetLastError(), "q8k quantize launch");
}

static zg_status run_q4k_q8k(zg_ctx* ctx, const uint8_t* q8k, const uint8_t* w, float* y, size_t in_dim,
                             size_t out_dim, hipStream_t st) {
  if (reinterpret_cast<uintptr_t>(w) & 15) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: weights misaligned");
  if (reinterpret_cast<uintptr_t>(q8k) & 3) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: activations misaligned");
  if (out_dim == 0) return ZG_OK;
  constexpr int RB = 2;
  const int nsb = (int)(in_dim / 256);
  const int S = (nsb + 7) / 8;
  const int nw = S >= 4 ? S : (S == 3 ? 6 : 4);
  const int wps = nw / S;
  const size_t nbatch = (out_dim + (size_t)wps * RB - 1) / ((size_t)wps * RB);
  const size_t per_cu = nw >= 16 ? 1 : (size_t)(16 / nw);
  const size_t cap = (size_t)q8k_cu_count() * per_cu;
  const size_t grid = nbatch < cap ? nbatch : cap;
  hipLaunchKernelGGL((q4k_q8k_strip_kernel<RB>), dim3((unsigned)grid), dim3(nw * 64), 0, st, w, q8k, y, nsb,
                     (int)out_dim, S);
  return hip_check(ctx, hipGetLastError(), "q4k x q8k launch");
}

// ---------------------------------------------------------------------------
// No-allocation variant of zg_linear_q4k_vnni.  Its Q8_K activation blocks
// go to a fixed device array of this library instead of a context buffer
// grown with hipMalloc: in_dim <= 32768 gives at most 128 blocks, 37,376
// bytes, held by every GPU the library runs on until the process ends.
// On the host, `scratch` names a host-side stand-in, not device memory:
// zg_init looks up each device's address of the array once
// (noalloc_scratch_setup) and host code only ever passes that address.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocMaxK = (size_t)kQ8kMaxStrips * 2048;
constexpr size_t kNoAllocScratchBytes = kNoAllocMaxK / 256 * kQ8kBytes;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_addr[kMaxDevices];  // per device, filled once
}  // namespace

// Called by zg_init with ctx->device current.
zg_status noalloc_scratch_setup(zg_ctx* ctx) {
  if (ctx->device < 0 || ctx->device >= kMaxDevices)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "noalloc scratch: device %d above %d", ctx->device, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[ctx->device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_check(ctx, e != hipSuccess ? e : hipErrorInvalidSymbol, "noalloc scratch lookup");
    g_scratch_addr[ctx->device] = static_cast<uint8_t*>(p);
  }
  ctx->noalloc_scratch = g_scratch_addr[ctx->device];
  return ZG_OK;
}

}  // namespace zg

extern "C" zg_status zg_quantize_q8k_dev(zg_ctx* ctx, const float* d_x, void* d_q8k, size_t n, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_x || !d_q8k) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: null pointer");
  if (n % 256) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: n %zu %% 256 != 0", n);
  if (n == 0) return ZG_OK;
  hipSetDevice(ctx->device);
  return run_q8k_quant(ctx, d_x, static_cast<uint8_t*>(d_q8k), n,
                       stream ? reinterpret_cast<hipStream_t>(stream) : ctx->stream);
}

extern "C" zg_status zg_linear_q4k_q8k_dev(zg_ctx* ctx, const void* d_q8k, const void* d_w, float* d_out,
                                          size_t in_dim, size_t out_dim, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_q8k || !d_w || !d_out) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: null pointer");
  zg_status s = q8k_check(ctx, in_dim, out_dim);
  if (s) return s;
  hipSetDevice(ctx->device);
  return run_q4k_q8k(ctx, static_cast<const uint8_t*>(d_q8k), static_cast<const uint8_t*>(d_w), d_out, in_dim,
                     out_dim, stream ? reinterpret_cast<hipStream_t>(stream) : ctx->stream);
}

extern "C" zg_status zg_linear_q4k_vnni(zg_ctx* ctx, const float* x, const void* w, float* out, size_t in_dim,
                                       size_t out_dim) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!x || !w || !out) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: null pointer");
  zg_status s = q8k_check(ctx, in_dim, out_dim);
  if (s) return s;
  hipSetDevice(ctx->device);
  const uint8_t* dw;
  uint32_t il;
  if ((s = resolve(ctx, w, tensor_bytes(ZG_Q4K, out_dim, in_dim), ZG_Q4K, &dw, &il))) return s;
  if (il != 1) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k: Q4_K weights are never interleaved");
  if ((s = stage_in(ctx, x, in_dim * sizeof(float), ctx->d_x))) return s;
  if ((s = ensure_buf(ctx, ctx->d_aux, in_dim / 256 * kQ8kBytes))) return s;
  if ((s = ensure_buf(ctx, ctx->d_out, out_dim * sizeof(float)))) return s;
  uint8_t* q8k = static_cast<uint8_t*>(ctx->d_aux.ptr);
  float* dout = static_cast<float*>(ctx->d_out.ptr);
  if ((s = run_q8k_quant(ctx, static_cast<const float*>(ctx->d_x.ptr), q8k, in_dim, ctx->stream))) return s;
  if ((s = run_q4k_q8k(ctx, q8k, dw, dout, in_dim, out_dim, ctx->stream))) return s;
  if (out_dim && (s = hip_check(ctx, hipMemcpyAsync(out, dout, out_dim * sizeof(float), hipMemcpyDeviceToHost,
                                                    ctx->stream), "download")))
    return s;
  return hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync");
}

// Device pointers, asynchronous on `stream`; no hipMalloc / hipFree.  The
// quantizer writes every byte of the blocks the GEMV then reads, so the
// array needs no clearing between calls.  Calls on one GPU share its array:
// calls that may overlap on that GPU (unordered streams) race.
extern "C" zg_status zg_linear_q4k_vnni_noalloc(zg_ctx* ctx, const float* d_x, const void* d_w, float* d_out,
                                               size_t in_dim, size_t out_dim, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_x || !d_w || !d_out) return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k noalloc: null pointer");
  if (in_dim > kNoAllocMaxK)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "q8k noalloc: in_dim %zu above the %zu values the fixed scratch holds",
                     in_dim, kNoAllocMaxK);
  zg_status s = q8k_check(ctx, in_dim, out_dim);
  if (s) return s;
  if (!ctx->noalloc_scratch) return set_error(ctx, ZG_ERR_HIP, "q8k noalloc: scratch address not resolved");
  hipSetDevice(ctx->device);
  const hipStream_t st = stream ? reinterpret_cast<hipStream_t>(stream) : ctx->stream;
  if ((s = run_q8k_quant(ctx, d_x, ctx->noalloc_scratch, in_dim, st))) return s;
  return run_q4k_q8k(ctx, ctx->noalloc_scratch, static_cast<const uint8_t*>(d_w), d_out, in_dim, out_dim, st);
}
