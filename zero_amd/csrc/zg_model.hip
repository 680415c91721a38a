// zg_model.hip -- single-token forward pass on the GPU, captured as HIP
// graphs.
//
// Restates forward_single_token_avx512 (kernel/src/inference_avx512.rs:
// 1826-1987) and lm_head_argmax_avx512 (:1200-1270) as a fixed sequence of
// launches that reads the token id and position from device memory, so the
// whole per-token sequence is one graph replay and greedy decoding feeds the
// argmax back to the next step without a host round trip (the reference's
// caller loop is kernel/src/inference.rs:1188-1330, 1644-1705, 1817-).
//
// Per layer:
//   1. fused Q|K|V GEMV with rmsnorm(attn_norm) in the prologue
//   2. attention: QK-norm + RoPE + KV-cache store + scores/softmax, up to
//      four workgroups per query head, each over its split of the context
//   3. O GEMV with the split merge in the prologue and the residual add in
//      the epilogue
//   4. fused gate|up GEMV with rmsnorm(ffn_norm) and SiLU(gate)*up epilogue
//   5. down GEMV with the residual add in the epilogue
// LM head: GEMV with rmsnorm(output_norm) prologue and argmax epilogue, then
// a one-thread finalize kernel that feeds the argmax to the next step.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/zero_gpu.h"
#include "zg_device.h"
#include "zg_internal.h"
#include "zg_kernels.h"
#include "zg_strip.h"

using namespace zg;

namespace zg {

constexpr int kMaxG = 8;          // max query heads per KV head

constexpr uint32_t kNoStep = 0xFFFFFFFFu;

// Device-resident decode state.
struct DevState {
  uint32_t token;    // token fed to the next forward pass
  uint32_t pos;      // its position
  uint32_t gen;      // tokens produced by finalize so far
  uint32_t err;      // bit 0 non-finite logits, 1 argmax in padding, 2 attention, 3 fused-attention wait timeout
  uint32_t n_prompt;
  uint32_t gen_cap;
  uint32_t err_step;  // gen index of the first finalize that saw an error bit (kNoStep: none)
  uint32_t err_first; // the error bits at that finalize: the first failure
  uint64_t best;     // last packed argmax (copy of the LM head slot)
};

// embed_lookup_dispatch (forward_pass.rs:311-370): row tok of a plain
// token_embd (Q4_0, Q8_0, Q4_K or Q6_K), each element dequantized in the
// reference's operation order.  Each thread decodes eight elements per pass with all their loads issued
// before the first store (indexes past the row clamp to its last element),
// so the row's cache lines arrive together rather than one memory round
// trip per element.
template <uint32_t QT>
__device__ __forceinline__ void embed_row_q(const uint8_t* __restrict__ embd, int hidden, uint32_t tok,
                                            float* __restrict__ out) {
  constexpr int be = (QT == Q4_0 || QT == Q8_0) ? 32 : 256;
  constexpr int kPer = 8;
  const size_t nb = (size_t)(hidden / be);
  const int nt = (int)blockDim.x;
  for (int e0 = 0; e0 < hidden; e0 += kPer * nt) {
    float v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = min(e0 + (int)threadIdx.x + i * nt, hidden - 1);
      const BlockRef br = block_ref(embd, QT, 1, tok, (size_t)(e / be), nb);
      const float d = (QT == Q4_0 || QT == Q8_0) ? rd_half(br.d) : 0.0f;
      v[i] = deq_elem(br, QT, d, e % be);
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = e0 + (int)threadIdx.x + i * nt;
      if (e < hidden) store_out(out + e, v[i]);
    }
  }
}

__device__ __forceinline__ void embed_row(const uint8_t* __restrict__ embd, uint32_t qt, int hidden, uint32_t tok,
                                          float* __restrict__ out) {
  switch (qt) {
    case Q4_0: embed_row_q<Q4_0>(embd, hidden, tok, out); break;
    case Q8_0: embed_row_q<Q8_0>(embd, hidden, tok, out); break;
    case Q4K: embed_row_q<Q4K>(embd, hidden, tok, out); break;
    default: embed_row_q<Q6K>(embd, hidden, tok, out); break;
  }
}

// The decode step's embedding lookup; also clears the LM-head argmax slot
// for this step, and fills this position's RoPE table once for all layers,
// as the reference builds its sin/cos table once per token
// (trig.rs:148-216): cs[i] = cos(pos * inv_freq[i]), cs[half + i] =
// sin(pos * inv_freq[i]).
struct EmbedArgs {
  const uint8_t* embd;
  uint32_t qt;
  int hidden;
  float* out;  // the residual stream
  const float* inv_freq;
  int half;
  float* rope_cs;
  uint32_t* epoch;  // step counter of the fused Q|K|V + attention launches
  uint64_t* best;   // LM-head argmax slot
};

// The start of a step at (tok, pos): step counter, argmax slot, RoPE table,
// embedding row.  Thread 0 writes the shared words; the caller has read
// everything it needs from them.
__device__ __forceinline__ void step_start(const EmbedArgs& e, uint32_t tok, uint32_t pos) {
  if (threadIdx.x == 0) {
    store_out(e.epoch, *e.epoch + 1);
    store_out(e.best, (uint64_t)0);
  }
  if ((int)threadIdx.x < e.half) {
    const float th = (float)pos * e.inv_freq[threadIdx.x];
    store_out(e.rope_cs + threadIdx.x, cosf(th));
    store_out(e.rope_cs + e.half + threadIdx.x, sinf(th));
  }
  embed_row(e.embd, e.qt, e.hidden, tok, e.out);
}

__global__ void embed_kernel(EmbedArgs e, const DevState* __restrict__ st) {
  step_start(e, st->token, st->pos);
}

// Poll bound of the fused attention's wait: 2^13 polls of ~1 us, a few ms,
// against a wait of a few us (the GEMV it waits for has no wait).
constexpr uint32_t kSyncSpinLimit = 1u << 13;

struct AttnArgs {
  const float* q;      // raw Q projection [nq*HD]
  const float* k;      // raw K projection [nkv*HD]
  const float* v;      // raw V projection [nkv*HD]
  const float* q_norm; // [HD]
  const float* k_norm; // [HD]
  const float* rope_cs;   // [HD]: cos then sin of pos * inv_freq
  float* kcache;       // this layer's K rows [max_ctx][nkv*HD]
  float* vcache;       // this layer's V rows
  float* out;          // one split: attention output [nq*HD]; else split outputs [nsplit][nq*HD]
  float* part_ml;      // split (max, exp-sum) pairs [nsplit][nq] (nsplit > 1)
  DevState* st;
  int nkv, g, nsplit;
  int split_len;       // prefill form (one split): max_ctx; decode splits follow attn_split_rows
  float eps, scale;
  // batched prefill: query row z of the chunk sits at position pos0 + z,
  // its (already normalised and rotated) query at q + z * row_stride; its
  // output goes to out + z * row_stride as fp32 when out is set, else
  // Q8_0-encoded into qs + z * row_stride (int8) and qsd + z * row_stride /
  // 32 (fp16 d bits)
  int pos0;
  int row_stride;
  int8_t* qs;
  uint16_t* qsd;
  // fused decode form: the GEMV's tagged Q|K|V rows ([nq*HD | nkv*HD |
  // nkv*HD] 64-bit words: tag << 32 | fp32 bits) and the step counter; this
  // layer's rows carry tag = *epoch * tag_mul + tag_add
  const uint64_t* tagged;
  const uint32_t* epoch;
  uint32_t tag_mul, tag_add;
};

#ifndef ZG_ATTN_WAVES
#define ZG_ATTN_WAVES 4
#endif
#ifndef ZG_ATTN_PASSES
#define ZG_ATTN_PASSES 4
#endif
constexpr int kAttnWaves = ZG_ATTN_WAVES;
#ifndef ZG_ATTN_SPLITS
#define ZG_ATTN_SPLITS 6
#endif
constexpr int kAttnDecodeSplits = ZG_ATTN_SPLITS;
static_assert(kAttnDecodeSplits >= 1 && kAttnDecodeSplits <= kAttnSplits, "decode splits within the merge's capacity");

// Decode attention, flash-decoding over splits: grid (query heads, splits),
// one 4-wave workgroup per (head, split).  The live context (rows 0..pos)
// is cut evenly over the splits, in multiples of 8 rows
// (attn_split_rows), so every position spreads its rows over all the
// splits' CUs.  Rows are visited in rounds of 128 (4 passes of 32 rows, 8
// rows per wave per pass) whose K/V loads are all issued before any is
// used, so a split of up to 128 rows costs one memory round trip.
//   prologue  every wave normalises and rotates the query head and the new
//             key itself (QK-norm, ops.rs:29-52; NeoX RoPE, ops.rs:111-132)
//             and parks them in its own LDS rows: no workgroup barrier
//   score     lane (row r, slice s) holds float4 columns s, s+8, ... of its
//             K row; the partial dot is summed over the row's 8 lanes by DPP;
//             softmax as attention.rs:48-84, per wave, rescaled per round.
//             The softmax fails there (NumericalInstability) when the max
//             score is not finite or the exp-sum is not finite: any NaN
//             score, or a +inf one.  Here a wave that saw a NaN score gives
//             a NaN exp-sum (fmaxf alone would skip NaN), and the merge sets
//             error bit 2 when the head's max or exp-sum is not finite.
//   P.V       lane l holds dims VPL*l.. of the pass's 8 rows of V; the row
//             weights are read out with v_readlane
//   end       the 4 waves are merged through LDS.  A single split writes
//             o / sum (attention.rs:76-81 multiplies by 1/sum); otherwise
//             each split writes (o, max, sum) and the consumer merges them
//             (attn_split_merge).  Splits past the context write the neutral
//             (0, -inf, 0).
// The current row (written by this step) comes from the wave's registers
// and LDS, never from the cache: the first query head of each KV head
// stores it, concurrently with the other workgroups' reads of older rows.
//
// Prefill form (PF): grid (query heads, 1, chunk rows), one split; query row
// z attends to cache rows 0..pos0+z, all of which are in the cache already
// (qk_rope_store_kernel ran first), and its query is already normalised and
// rotated.  The output row goes out Q8_0-encoded for the O GEMM (each 32-lane
// segment of the output waves is one block), or as fp32 (a.out) for a
// K-quant O projection, whose Q8_K blocks span two heads.  Everything else is
// the decode kernel's arithmetic.
// Rows per split for position pos: ceil((pos + 1) / nsplit) rounded up to a
// multiple of 8; splits starting past pos hold no row.
__device__ __forceinline__ int attn_split_rows(int pos, int nsplit) {
  return (pos + 8 * nsplit) / (8 * nsplit) * 8;
}

// FUSED: the workgroup runs in the Q|K|V GEMV's launch (qkv_attn_kernel):
// it issues its first round of K/V cache loads, then each wave reads the
// Q, K and V values it needs from the GEMV's tagged words (a.tagged) until
// every word carries this step and layer's tag.  NP: passes per round.
template <int HD, bool PF, int NP = ZG_ATTN_PASSES, bool FUSED = false>
__device__ __forceinline__ void attn_split_body(AttnArgs a, int qh, int sp, int nq, int bz) {
  constexpr int F4 = HD / 4;            // float4 per head row
  constexpr int LPR = 8;                // lanes per row in the score layout
  constexpr int CPL = F4 / LPR;         // K float4 columns per lane
  constexpr int RPW = 64 / LPR;         // rows per wave per pass
  constexpr int NWV = kAttnWaves;
  constexpr int PASS = RPW * NWV;       // rows per pass
  constexpr int ROUND = NP * PASS;      // rows per round
  constexpr int VPL = HD / 64;          // V dims per lane
  constexpr int HALF = HD / 2;
  typedef float vlane_t __attribute__((ext_vector_type(VPL)));
  static_assert(!(FUSED && PF), "the fused form is the decode step's");
  const int kvh = qh / a.g;
  const int pos = PF ? a.pos0 + bz : (int)a.st->pos;
  if (PF) {
    a.q += (size_t)bz * a.row_stride;
    a.qs += (size_t)bz * a.row_stride;
    a.qsd += (size_t)bz * a.row_stride / 32;
  }
  const int slen = PF ? a.split_len : attn_split_rows(pos, a.nsplit);
  const int c0 = sp * slen;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (c0 > pos) {
    // split past the context: neutral partial (uniform per workgroup)
    if (tid < HD) store_out(a.out + ((size_t)sp * nq + qh) * HD + tid, 0.0f);
    if (tid == 0) {
      store_out(a.part_ml + 2 * ((size_t)sp * nq + qh), -INFINITY);
      store_out(a.part_ml + 2 * ((size_t)sp * nq + qh) + 1, 0.0f);
    }
    return;
  }
  const int n_t = min(slen, pos + 1 - c0);
  const bool has_pos = !PF && pos - c0 < slen;  // this split holds the current row (decode)
  const size_t rowf4 = (size_t)a.nkv * F4;
  const size_t rowv = (size_t)a.nkv * (HD / VPL);
  const int r = lane / LPR, sl = lane % LPR;
  __shared__ __attribute__((aligned(16))) float qk[NWV][2][HD];  // per wave: rotated q, new k
  __shared__ __attribute__((aligned(16))) float wo[NWV][HD];
  __shared__ float wm[NWV], wl[NWV];
  const float4* K4 = reinterpret_cast<const float4*>(a.kcache);
  const vlane_t* VL = reinterpret_cast<const vlane_t*>(a.vcache);

  float4 kr[NP][CPL];
  vlane_t vr[NP][RPW];
  // all passes of a round (rows past the split clamped to its last row)
  auto load_round = [&](int rb) {
#pragma unroll
    for (int p = 0; p < NP; p++) {
      if (rb + p * PASS < n_t) {
        const int tk = min(rb + p * PASS + wave * RPW + r, n_t - 1);
        const size_t ko = (size_t)(c0 + tk) * rowf4 + kvh * F4;
#pragma unroll
        for (int i = 0; i < CPL; i++) kr[p][i] = K4[ko + sl + LPR * i];
#pragma unroll
        for (int j = 0; j < RPW; j++) {
          const int tv = min(rb + p * PASS + wave * RPW + j, n_t - 1);
          vr[p][j] = VL[(size_t)(c0 + tv) * rowv + kvh * (HD / VPL) + lane];
        }
      }
    }
  };
  // prologue operands, then the first step's K/V loads (fused: the K/V
  // loads first, then the wait for this head's Q|K|V rows, then those rows)
  const int hl = lane % HALF;
  float qx0 = 0.0f, qx1 = 0.0f;
  float kx0 = 0.0f, kx1 = 0.0f, qw0 = 0.0f, qw1 = 0.0f, kw0 = 0.0f, kw1 = 0.0f, cs0 = 0.0f, cs1 = 0.0f;
  vlane_t vnew = (vlane_t)(0.0f);
  if (FUSED) {
    load_round(0);
    // every wave polls the tagged words it needs itself (lane l: Q and K
    // dims l, l + HALF, V dims VPL*l..) until each carries this step and
    // layer's tag: no barrier and no LDS round trip on the way
    const uint32_t ep = *a.epoch * a.tag_mul + a.tag_add;
    const uint64_t* tq = a.tagged + qh * HD;
    const uint64_t* tk = a.tagged + nq * HD + kvh * HD;
    const uint64_t* tv = a.tagged + (nq + a.nkv) * HD + kvh * HD;
    constexpr int NWD = 4 + VPL;
    const uint64_t* src[NWD] = {tq + hl, tq + hl + HALF, tk + hl, tk + hl + HALF};
#pragma unroll
    for (int i = 0; i < VPL; i++) src[4 + i] = tv + VPL * lane + i;
    uint64_t w[NWD];
    uint32_t spins = 0;
    for (;;) {
      bool ok = true;
#pragma unroll
      for (int j = 0; j < NWD; j++) {
        w[j] = __hip_atomic_load(src[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // wrap-safe: the tags of earlier layers and steps are behind
        ok = ok && (int)((uint32_t)(w[j] >> 32) - ep) >= 0;
      }
      if (__all(ok)) break;
      if (++spins > kSyncSpinLimit) {
        if (lane == 0) atomicOr(&a.st->err, 8u);
        break;
      }
    }
    qx0 = __uint_as_float((uint32_t)w[0]);
    qx1 = __uint_as_float((uint32_t)w[1]);
    kx0 = __uint_as_float((uint32_t)w[2]);
    kx1 = __uint_as_float((uint32_t)w[3]);
#pragma unroll
    for (int i = 0; i < VPL; i++) vnew[i] = __uint_as_float((uint32_t)w[4 + i]);
  } else {
    qx0 = a.q[qh * HD + hl];
    qx1 = a.q[qh * HD + hl + HALF];
    if (!PF) {
      kx0 = a.k[kvh * HD + hl];
      kx1 = a.k[kvh * HD + hl + HALF];
      vnew = reinterpret_cast<const vlane_t*>(a.v)[kvh * (HD / VPL) + lane];
    }
  }
  if (!PF) {
    qw0 = a.q_norm[hl];
    qw1 = a.q_norm[hl + HALF];
    kw0 = a.k_norm[hl];
    kw1 = a.k_norm[hl + HALF];
    cs0 = a.rope_cs[hl];
    cs1 = a.rope_cs[hl + HALF];
  }
  if (!FUSED) load_round(0);

  // QK-norm + RoPE of one head vector held as (x0, x1) = dims (l, l + HALF)
  // by lanes l < HALF; result into this wave's LDS row
  float* qrow = qk[wave][0];
  float* krow = qk[wave][1];
  auto norm_rope = [&](float x0, float x1, float w0, float w1, float* dst, float& y0, float& y1) {
    const float ssq = wave_sum(lane < HALF ? x0 * x0 + x1 * x1 : 0.0f);
    const float rinv = 1.0f / sqrtf(ssq / (float)HD + a.eps);
    const float xa = x0 * rinv * w0;
    const float xb = x1 * rinv * w1;
    y0 = xa * cs0 - xb * cs1;
    y1 = xa * cs1 + xb * cs0;
    if (lane < HALF) {
      dst[lane] = y0;
      dst[lane + HALF] = y1;
    }
  };
  float q0, q1, k0, k1;
  if (PF) {
    if (lane < HALF) {
      qrow[lane] = qx0;
      qrow[lane + HALF] = qx1;
    }
  } else {
    norm_rope(qx0, qx1, qw0, qw1, qrow, q0, q1);
    norm_rope(kx0, kx1, kw0, kw1, krow, k0, k1);
  }
  if (has_pos && qh % a.g == 0 && wave == 0) {
    // KvCache::store_kv (kv_cache.rs:139-183): row `pos` of this KV head
    float* kc = a.kcache + (size_t)pos * rowf4 * 4 + kvh * HD;
    if (lane < HALF) {
      store_out(kc + lane, k0);
      store_out(kc + lane + HALF, k1);
    }
    float* vc = a.vcache + ((size_t)pos * rowv + kvh * (HD / VPL) + lane) * VPL;
#pragma unroll
    for (int i = 0; i < VPL; i++) store_out(vc + i, vnew[i]);
  }
  wave_lds_sync();
  float4 q[CPL];
#pragma unroll
  for (int i = 0; i < CPL; i++) q[i] = reinterpret_cast<const float4*>(qrow)[sl + LPR * i];

  vlane_t acc = (vlane_t)(0.0f);
  float m_w = -INFINITY, l_w = 0.0f;
  bool nan_score = false;
  for (int rb = 0; rb < n_t; rb += ROUND) {
    if (rb > 0) load_round(rb);
    float sc[NP];
    float cmax = -INFINITY;
#pragma unroll
    for (int p = 0; p < NP; p++) {
      sc[p] = -INFINITY;
      if (rb + p * PASS < n_t) {
        const int t = rb + p * PASS + wave * RPW + r;
        float4 kk[CPL];
#pragma unroll
        for (int i = 0; i < CPL; i++) kk[i] = kr[p][i];
        if (!PF && c0 + t == pos) {
#pragma unroll
          for (int i = 0; i < CPL; i++) kk[i] = reinterpret_cast<const float4*>(krow)[sl + LPR * i];
        }
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < CPL; i++) {
          d = fmaf(q[i].x, kk[i].x, d);
          d = fmaf(q[i].y, kk[i].y, d);
          d = fmaf(q[i].z, kk[i].z, d);
          d = fmaf(q[i].w, kk[i].w, d);
        }
        d += dpp_f32<0xB1>(d);   // quad_perm [1,0,3,2]
        d += dpp_f32<0x4E>(d);   // quad_perm [2,3,0,1]
        d += dpp_f32<0x141>(d);  // row_half_mirror: the 8 lanes of the row
        sc[p] = t < n_t ? d * a.scale : -INFINITY;
        nan_score = nan_score || __builtin_isnan(sc[p]);
        cmax = fmaxf(cmax, sc[p]);
      }
    }
    const float cm = wave_max(cmax);
    if (cm == -INFINITY) continue;  // no row of this wave in the round (uniform)
    const float m_new = fmaxf(m_w, cm);
    const float alpha = m_w == -INFINITY ? 0.0f : expf(m_w - m_new);
    acc *= alpha;
    float esum = 0.0f;
#pragma unroll
    for (int p = 0; p < NP; p++) {
      if (rb + p * PASS < n_t) {
        const float e = sc[p] == -INFINITY ? 0.0f : expf(sc[p] - m_new);
        esum += sl == 0 ? e : 0.0f;
        const int t0 = rb + p * PASS + wave * RPW;
#pragma unroll
        for (int j = 0; j < RPW; j++) {
          const float ej = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j * LPR));
          const vlane_t v = (!PF && c0 + t0 + j == pos) ? vnew : vr[p][j];
          acc += ej * v;
        }
      }
    }
    l_w = fmaf(l_w, alpha, wave_sum(esum));
    m_w = m_new;
  }
  reinterpret_cast<vlane_t*>(wo[wave])[lane] = acc;
  const bool wave_nan = __any(nan_score);
  if (lane == 0) {
    wm[wave] = m_w;
    wl[wave] = wave_nan ? __builtin_nanf("") : l_w;
  }
  __syncthreads();
  if (tid < HD) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWV; w++) M = fmaxf(M, wm[w]);
    float L = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < NWV; w++) {
      const float f = wm[w] == -INFINITY ? 0.0f : expf(wm[w] - M);
      L = fmaf(f, wl[w], L);
      o = fmaf(f, wo[w][tid], o);
    }
    if (tid == 0 && !(isfinite(M) && isfinite(L))) atomicOr(&a.st->err, 4u);
    if (PF && a.out) {
      a.out[(size_t)bz * a.row_stride + qh * HD + tid] = o * (1.0f / L);
    } else if (PF) {
      uint32_t dbits;
      const int8_t qv = q8_0_encode_lane(o * (1.0f / L), &dbits);
      a.qs[qh * HD + tid] = qv;
      if ((tid & 31) == 0) a.qsd[(qh * HD + tid) / 32] = (uint16_t)dbits;
    } else if (a.nsplit == 1) {
      store_out(a.out + qh * HD + tid, o * (1.0f / L));
    } else {
      store_out(a.out + ((size_t)sp * nq + qh) * HD + tid, o);
      if (tid == 0) {
        store_out(a.part_ml + 2 * ((size_t)sp * nq + qh), M);
        store_out(a.part_ml + 2 * ((size_t)sp * nq + qh) + 1, L);
      }
    }
  }
}

template <int HD, bool PF>
__global__ __launch_bounds__(kAttnWaves * 64) void attn_split_kernel(AttnArgs a) {
  attn_split_body<HD, PF>(a, blockIdx.x, blockIdx.y, gridDim.x, blockIdx.z);
}

// Q|K|V GEMV and decode attention in one launch.  Workgroups 0..n_attn-1 are
// the attention splits (query head b % nq, split b / nq), the rest the
// one-batch strip GEMV (rmsnorm prologue, four strips: in_dim 2048, two
// groups per batch).  The attention workgroups come first, so they are
// dispatched first: they issue their K/V cache loads while the GEMV runs,
// then poll the GEMV's rows, each stored once with this step and layer's
// tag (the GEMV never waits, so every poll ends; it is also bounded).
// One launch instead of two, and the attention's cache reads overlap the
// GEMV.  A counter that every batch incremented serialised the 512 atomics
// of a step on one line (19 vs 8.8 us for the two kernels).
#ifndef ZG_FUSED_ATTN_PASSES
#define ZG_FUSED_ATTN_PASSES 2
#endif
constexpr int kFusedAttnPasses = ZG_FUSED_ATTN_PASSES;

template <uint32_t QT, int IL, int HD>
__global__ __launch_bounds__(256) void qkv_attn_kernel(GemvArgs ga, AttnArgs aa, int n_attn) {
  const int b = blockIdx.x;
  if (b < n_attn) {
    const int nq = n_attn / aa.nsplit;
    attn_split_body<HD, false, kFusedAttnPasses, true>(aa, b % nq, b / nq, nq, 0);
  } else {
    gemv_strip_body<QT, PRO_RMSNORM, EPI_STORE, 2, 1024, false, IL, true, 4, false, true>(ga, 4, b - n_attn,
                                                                                           (int)gridDim.x - n_attn);
  }
}

// Plain row-major Q4_0 / Q8_0 blocks (bb bytes: fp16 d, then the quants) to
// the X4 layout the packer writes for .smodel-v2 (per group of four rows
// and block: the four rows' d, then their quant bytes in row order), one
// thread per (group, block); every field sits at an even offset.
__global__ __launch_bounds__(256) void interleave_x4_kernel(const uint8_t* __restrict__ plain, uint8_t* __restrict__ x4,
                                                            size_t units, int nb, int bb) {
  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= units) return;
  const size_t g = t / (size_t)nb;
  const int b = (int)(t - g * (size_t)nb);
  uint16_t* o = reinterpret_cast<uint16_t*>(x4 + t * (size_t)(4 * bb));
  const int qh = (bb - 2) / 2;  // quant halfwords per block
  for (int l = 0; l < 4; l++) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(plain + ((4 * g + l) * (size_t)nb + b) * (size_t)bb);
    o[l] = src[0];
    for (int i = 0; i < qh; i++) o[4 + l * qh + i] = src[1 + i];
  }
}

// X4 group-blocks (gb bytes: 4 fp16 scales, then 4 rows of qb quant bytes)
// to the split-scale X4 groups the strip kernel reads with one 16-byte-
// aligned quant load and one contiguous scale load per wave (IL 5): per
// group of nb blocks, [block][row][qb] quants, then [block][row] scales.
// Thread t moves group-block t (group t / nb, block t % nb).
__global__ __launch_bounds__(256) void split_x4_kernel(const uint8_t* __restrict__ x4, uint8_t* __restrict__ out,
                                                       size_t units, int nb, int qb) {
  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= units) return;
  const size_t g = t / (size_t)nb;
  const int b = (int)(t - g * (size_t)nb);
  const size_t gb = 8 + 4 * (size_t)qb;
  const uint8_t* src = x4 + t * gb;
  uint8_t* grp = out + g * (size_t)nb * gb;
  const uint2* sq = reinterpret_cast<const uint2*>(src + 8);
  uint2* dq = reinterpret_cast<uint2*>(grp + (size_t)b * 4 * qb);
  for (int i = 0; i < qb / 2; i++) dq[i] = sq[i];  // the 4 rows' quants, in order
  *reinterpret_cast<uint2*>(grp + (size_t)nb * 4 * qb + 8 * (size_t)b) = *reinterpret_cast<const uint2*>(src);
}

// Split merge for O projections that cannot take the merging GEMV: thread t
// merges dims 8t..8t+7 of the attention output.
__global__ void attn_merge_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml, int k, int hd,
                                  int nsplit, float* __restrict__ out) {
  const int e0 = 8 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (e0 >= k) return;
  AttnSplitIn in;
  attn_split_load(in, part_o, part_ml, k, hd, nsplit, e0);
  float4 x0, x1;
  attn_split_merge(in, nsplit, x0, x1);
  reinterpret_cast<float4*>(out + e0)[0] = x0;
  reinterpret_cast<float4*>(out + e0)[1] = x1;
}

// One row of n per workgroup (row blockIdx.x).
__global__ void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ out,
                               int n, float eps) {
  __shared__ float red[4];
  x += (size_t)blockIdx.x * n;
  out += (size_t)blockIdx.x * n;
  float ssq = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) ssq += x[i] * x[i];
  ssq = seg_sum<64>(ssq);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ssq;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float rinv = 1.0f / sqrtf(tot / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += 256) out[i] = x[i] * rinv * w[i];
}

// The same for one row of up to 16,384 floats (16-byte aligned, n % 4 == 0):
// 1024 threads, every x and w load issued before the first is used (the
// loop above pays one memory round trip per step: 7.8 us for 2048 floats).
constexpr int kRmsV = 4;  // float4 per thread
__global__ __launch_bounds__(1024) void rmsnorm_row_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                          float* __restrict__ out, int n, float eps) {
  __shared__ float red[16];
  const int n4 = n >> 2;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  const float4* w4 = reinterpret_cast<const float4*>(w);
  float4 xv[kRmsV], wv[kRmsV];
#pragma unroll
  for (int j = 0; j < kRmsV; j++) {
    const int i = threadIdx.x + 1024 * j;
    xv[j] = i < n4 ? x4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    wv[j] = i < n4 ? w4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float ssq = 0.0f;
#pragma unroll
  for (int j = 0; j < kRmsV; j++) ssq += xv[j].x * xv[j].x + xv[j].y * xv[j].y + xv[j].z * xv[j].z + xv[j].w * xv[j].w;
  ssq = seg_sum<64>(ssq);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ssq;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; i++) tot += red[i];
  const float rinv = 1.0f / sqrtf(tot / (float)n + eps);
  float4* o4 = reinterpret_cast<float4*>(out);
#pragma unroll
  for (int j = 0; j < kRmsV; j++) {
    const int i = threadIdx.x + 1024 * j;
    if (i < n4)
      o4[i] = make_float4(xv[j].x * rinv * wv[j].x, xv[j].y * rinv * wv[j].y, xv[j].z * rinv * wv[j].z,
                          xv[j].w * rinv * wv[j].w);
  }
}

// After the LM head: argmax -> next token, error bits, output record, then
// move to the next position.
// Every input is loaded before the first store (one memory round trip).
// The LM head's packed argmax key -> token, error bits 0 (non-finite or no
// candidate) and 1 (padding row).  The token is always a row of the head
// (0 when there is no candidate), so it indexes the embedding safely.
__device__ __forceinline__ uint32_t argmax_token(uint64_t key, uint32_t vocab_real, uint32_t& err) {
  err = 0;
  if (key == 0) {
    err = 1;
    return 0;
  }
  const uint32_t k = (uint32_t)(key >> 32);
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  const uint32_t idx = 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu);
  if (!isfinite(__uint_as_float(b))) err = 1;
  else if (idx >= vocab_real) err = 2;
  return idx;
}

// The step's record: error bits, output token, next position (thread 0).
__device__ __forceinline__ void finalize_state(DevState* __restrict__ st, uint64_t key, uint32_t idx, uint32_t err,
                                               uint32_t err0, uint32_t err_step, uint32_t gen, uint32_t gen_cap,
                                               uint32_t pos, uint32_t* __restrict__ out_tokens) {
  if ((err | err0) && err_step == kNoStep) {
    store_out(&st->err_step, gen);
    store_out(&st->err_first, err | err0);
  }
  store_out(&st->err, err0 | err);
  store_out(&st->best, key);
  store_out(&st->token, idx);
  if (out_tokens && gen < gen_cap) store_out(out_tokens + gen, idx);
  store_out(&st->gen, gen + 1);
  store_out(&st->pos, pos + 1);
}

__global__ void finalize_kernel(DevState* __restrict__ st, const uint64_t* __restrict__ best, uint32_t vocab_real,
                                uint32_t* __restrict__ out_tokens) {
  const uint64_t key = *best;
  const uint32_t err0 = st->err, err_step = st->err_step, gen = st->gen, gen_cap = st->gen_cap, pos = st->pos;
  uint32_t err;
  const uint32_t idx = argmax_token(key, vocab_real, err);
  finalize_state(st, key, idx, err, err0, err_step, gen, gen_cap, pos, out_tokens);
}

// finalize_kernel and the start of the next step in one launch (the step
// graph of the greedy loop): the token just chosen is embedded at the next
// position.  Every thread decodes the key itself; the barrier keeps the
// argmax slot and the state unchanged until every wave has read them.
__global__ void finalize_embed_kernel(DevState* __restrict__ st, uint32_t vocab_real, uint32_t* __restrict__ out_tokens,
                                      EmbedArgs e) {
  const uint64_t key = *e.best;
  const uint32_t err0 = st->err, err_step = st->err_step, gen = st->gen, gen_cap = st->gen_cap, pos = st->pos;
  uint32_t err;
  const uint32_t idx = argmax_token(key, vocab_real, err);
  __syncthreads();
  if (threadIdx.x == 0) finalize_state(st, key, idx, err, err0, err_step, gen, gen_cap, pos, out_tokens);
  step_start(e, idx, pos + 1);
}

// Move to the next position; during the prompt, feed the next prompt token;
// then start that step (embedding, RoPE table, step counter).
__global__ void advance_embed_kernel(DevState* __restrict__ st, const uint32_t* __restrict__ prompt, EmbedArgs e) {
  const uint32_t p = st->pos + 1, n_prompt = st->n_prompt, tok0 = st->token;
  const uint32_t tok = p < n_prompt ? prompt[p] : tok0;
  __syncthreads();
  if (threadIdx.x == 0) {
    store_out(&st->pos, p);
    store_out(&st->token, tok);
  }
  step_start(e, tok, p);
}

// ---------------------------------------------------------------------------
// Non-finite localisation.  The reference scans the activations of every
// layer for NaN/Inf during the forward pass and latches the first stage that
// holds one (finite_diag, inference_avx512.rs:88-131, call sites :1896,
// :1946-1947, :1981-1982; the latch text record_first_nonfinite, :233-262).
// Here the decode step carries no such scans: after a call fails with a
// non-finite error, the host finds the first KV row holding a non-finite
// value (kv_scan_kernel) and runs that row's decode step again, eagerly,
// with nf_scan_kernel after each of the reference's stages.  The O and down
// projections then also run once into a zeroed buffer (their residual
// epilogue adds 0), which gives the sublayer output alone; the step's own
// launches are unchanged, so the replay writes the bits the step wrote.
// ---------------------------------------------------------------------------

// Stages, in the reference's forward order within a layer.
enum NfStage : uint32_t {
  NF_ATTN_NORM_IN = 1,  // rmsnorm(hidden, attn_norm)
  NF_ATTN_OUT,          // O projection output
  NF_POST_ATTN,         // hidden after the attention residual add
  NF_MLP_OUT,           // down projection output
  NF_POST_MLP,          // hidden after the MLP residual add
  NF_K_CACHE,           // a K cache row (rows the decode step cannot replay)
  NF_V_CACHE,
};

// FIRST_NF_CAP (inference_avx512.rs:233): the latch text's byte capacity
constexpr size_t kNfCap = 32;

struct NfScan {
  uint32_t tag;     // (layer << 8) | stage of the first hit; 0 none
  uint32_t idx;     // its first non-finite element
  uint32_t bits;    // that element's bits
  uint32_t kv_key;  // (row << 8) | (2 * layer + 0 K / 1 V): first non-finite KV row; ~0 none
};

// One workgroup: the first non-finite element of v[0..n) latches tag,
// unless an earlier stage has latched or attention has failed (the
// reference's forward returns at the softmax failure, before the stages
// after it are scanned).
__global__ __launch_bounds__(1024) void nf_scan_kernel(const float* __restrict__ v, int n,
                                                       const uint32_t* __restrict__ err, NfScan* res, uint32_t tag) {
  __shared__ int first;
  if (res->tag != 0 || (err && (*err & 4u))) return;  // uniform
  if (threadIdx.x == 0) first = n;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x)
    if (!isfinite(v[i])) {
      atomicMin(&first, i);
      break;
    }
  __syncthreads();
  if (threadIdx.x == 0 && first < n) {
    res->idx = (uint32_t)first;
    res->bits = __float_as_uint(v[first]);
    res->tag = tag;
  }
}

// grid (rows, 2 * layers): whether cache row blockIdx.x of K (even y) or V
// (odd y) of layer y / 2 holds a non-finite value; the smallest
// (row, layer, K before V) wins.
__global__ __launch_bounds__(256) void kv_scan_kernel(const float* __restrict__ kv, size_t max_ctx, int kvd,
                                                      NfScan* res) {
  const float* row = kv + ((size_t)blockIdx.y * max_ctx + blockIdx.x) * kvd;
  int bad = 0;
  for (int i = threadIdx.x; i < kvd; i += blockDim.x) bad |= !isfinite(row[i]);
  if (__syncthreads_or(bad) && threadIdx.x == 0) atomicMin(&res->kv_key, (blockIdx.x << 8) | blockIdx.y);
}

__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// Batched prefill support (no reference counterpart: the reference runs the
// prompt token by token, kernel/src/inference.rs:1188-1330).  Each kernel
// does per row what the decode step does for its one token.
// ---------------------------------------------------------------------------

// Rows of token_embd for tokens[0..rows) (embed_kernel per row); block 0 also
// clears the LM-head argmax slot.
__global__ void embed_rows_kernel(const uint8_t* __restrict__ embd, uint32_t qt, int hidden,
                                  const uint32_t* __restrict__ tokens, float* __restrict__ out,
                                  uint64_t* __restrict__ best) {
  embed_row(embd, qt, hidden, tokens[blockIdx.x], out + (size_t)blockIdx.x * hidden);
  if (blockIdx.x == 0 && threadIdx.x == 0) *best = 0;
}

struct QkStoreArgs {
  float* q;              // [rows][nq*HD], normalised and rotated in place
  const float* k;        // [rows][nkv*HD]
  const float* v;        // [rows][nkv*HD]
  const float* q_norm;   // [HD]
  const float* k_norm;   // [HD]
  const float* inv_freq; // [HD/2]
  float* kcache;         // this layer's K rows [max_ctx][nkv*HD]
  float* vcache;
  int nq, nkv, pos0;
  float eps;
};

// grid (rows, nq + nkv), one wave: QK-norm + RoPE of one head of one row at
// position pos0 + row, with the decode step's arithmetic (the cos/sin of
// embed_kernel, the norm_rope of attn_split_kernel).  Query heads are
// written back in place; KV heads go to the cache row with their V.
template <int HD>
__global__ __launch_bounds__(64) void qk_rope_store_kernel(QkStoreArgs a) {
  constexpr int HALF = HD / 2;
  const int row = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int pos = a.pos0 + row;
  const bool isq = h < a.nq;
  const int kvh = h - a.nq;
  const size_t qd = (size_t)a.nq * HD, kvd = (size_t)a.nkv * HD;
  const float* x = isq ? a.q + row * qd + (size_t)h * HD : a.k + row * kvd + (size_t)kvh * HD;
  const float* w = isq ? a.q_norm : a.k_norm;
  const int hl = lane % HALF;
  const float x0 = x[hl], x1 = x[hl + HALF];
  const float th = (float)pos * a.inv_freq[hl];
  const float c = cosf(th), sn = sinf(th);
  const float ssq = wave_sum(lane < HALF ? x0 * x0 + x1 * x1 : 0.0f);
  const float rinv = 1.0f / sqrtf(ssq / (float)HD + a.eps);
  const float xa = x0 * rinv * w[hl];
  const float xb = x1 * rinv * w[hl + HALF];
  const float y0 = xa * c - xb * sn;
  const float y1 = xa * sn + xb * c;
  float* dst = isq ? a.q + row * qd + (size_t)h * HD : a.kcache + (size_t)pos * kvd + (size_t)kvh * HD;
  if (lane < HALF) {
    dst[lane] = y0;
    dst[lane + HALF] = y1;
  }
  if (!isq) {
    const float* vs = a.v + row * kvd + (size_t)kvh * HD;
    float* vd = a.vcache + (size_t)pos * kvd + (size_t)kvh * HD;
    for (int e = lane; e < HD; e += 64) vd[e] = vs[e];
  }
}

// 1 / rms of one row of n, by a 256-thread workgroup (rmsnorm_kernel's
// arithmetic); red: 4 floats of LDS.
__device__ __forceinline__ float row_rms_inv(const float* __restrict__ x, int n, float eps, float* red) {
  float ssq = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) ssq += x[i] * x[i];
  ssq = seg_sum<64>(ssq);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ssq;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  return 1.0f / sqrtf(tot / (float)n + eps);
}

// One row of n per workgroup: rmsnorm (rmsnorm_kernel's arithmetic) and the
// Q8_0 encoding of the normalised row, 32 values per thread at a time.
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                            int8_t* __restrict__ qs, uint16_t* __restrict__ qd, int n,
                                                            float eps) {
  __shared__ float red[4];
  const size_t row = blockIdx.x;
  x += row * n;
  const float rinv = row_rms_inv(x, n, eps, red);
  for (int b = threadIdx.x; b < n / 32; b += 256) {
    const float4* x4 = reinterpret_cast<const float4*>(x + b * 32);
    const float4* w4 = reinterpret_cast<const float4*>(w + b * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 xv = x4[i], wv = w4[i];
      v[4 * i] = xv.x * rinv * wv.x;
      v[4 * i + 1] = xv.y * rinv * wv.y;
      v[4 * i + 2] = xv.z * rinv * wv.z;
      v[4 * i + 3] = xv.w * rinv * wv.w;
    }
    int8_t q[32];
    const uint32_t dbits = q8_0_encode(v, q);
    u32x4* dst = reinterpret_cast<u32x4*>(qs + row * n + b * 32);
    uint32_t wq[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
      wq[i] = (uint32_t)(uint8_t)q[4 * i] | ((uint32_t)(uint8_t)q[4 * i + 1] << 8) |
              ((uint32_t)(uint8_t)q[4 * i + 2] << 16) | ((uint32_t)(uint8_t)q[4 * i + 3] << 24);
    dst[0] = u32x4{wq[0], wq[1], wq[2], wq[3]};
    dst[1] = u32x4{wq[4], wq[5], wq[6], wq[7]};
    qd[row * (n / 32) + b] = (uint16_t)dbits;
  }
}

// One row of n per workgroup: silu(g) * u with the decode epilogue's operand
// order (activation.rs:115-148: g / (1 + exp(-g)), then * up), Q8_0-encoded.
// act = silu(act) * up in place (activation.rs:115-148 operand order), for
// decode steps whose gate and up projections are separate launches
__global__ __launch_bounds__(256) void silu_mul_kernel(float* __restrict__ g, const float* __restrict__ u, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const float gv = g[i];
    g[i] = (gv / (1.0f + expf(-gv))) * u[i];
  }
}

__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                           int8_t* __restrict__ qs, uint16_t* __restrict__ qd, int n) {
  const size_t row = blockIdx.x;
  for (int b = threadIdx.x; b < n / 32; b += 256) {
    const float4* g4 = reinterpret_cast<const float4*>(g + row * n + b * 32);
    const float4* u4 = reinterpret_cast<const float4*>(u + row * n + b * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 gv = g4[i], uv = u4[i];
      v[4 * i] = (gv.x / (1.0f + expf(-gv.x))) * uv.x;
      v[4 * i + 1] = (gv.y / (1.0f + expf(-gv.y))) * uv.y;
      v[4 * i + 2] = (gv.z / (1.0f + expf(-gv.z))) * uv.z;
      v[4 * i + 3] = (gv.w / (1.0f + expf(-gv.w))) * uv.w;
    }
    int8_t q[32];
    const uint32_t dbits = q8_0_encode(v, q);
    u32x4* dst = reinterpret_cast<u32x4*>(qs + row * n + b * 32);
    uint32_t wq[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
      wq[i] = (uint32_t)(uint8_t)q[4 * i] | ((uint32_t)(uint8_t)q[4 * i + 1] << 8) |
              ((uint32_t)(uint8_t)q[4 * i + 2] << 16) | ((uint32_t)(uint8_t)q[4 * i + 3] << 24);
    dst[0] = u32x4{wq[0], wq[1], wq[2], wq[3]};
    dst[1] = u32x4{wq[4], wq[5], wq[6], wq[7]};
    qd[row * (n / 32) + b] = (uint16_t)dbits;
  }
}

// Q8_K split rows for the K-quant GEMM (qs [rows][n] int8, d8 [rows][n/256]
// f32, bs32 [rows][n/32] int16).
struct Q8kRows {
  int8_t* qs;
  float* d8;
  int16_t* bs32;
};

// One row of n (a multiple of 256) per workgroup: rmsnorm_quant_kernel's
// normalised values, Q8_K-encoded (quantize_row_q8k,
// kernel/src/arch/x86_64/math/vnni.rs:78-170), one wave per 256-value block.
__global__ __launch_bounds__(256) void rmsnorm_q8k_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                          Q8kRows o, int n, float eps) {
  __shared__ float red[4];
  const size_t row = blockIdx.x;
  x += row * n;
  const float rinv = row_rms_inv(x, n, eps, red);
  const int lane = threadIdx.x & 63;
  for (int sb = threadIdx.x >> 6; sb < n / 256; sb += 4) {
    const float4 xv = reinterpret_cast<const float4*>(x + sb * 256)[lane];
    const float4 wv = reinterpret_cast<const float4*>(w + sb * 256)[lane];
    const float e[4] = {xv.x * rinv * wv.x, xv.y * rinv * wv.y, xv.z * rinv * wv.z, xv.w * rinv * wv.w};
    q8k_split_store(lane, e, o.qs + row * n + sb * 256, o.d8 + row * (n / 256) + sb, o.bs32 + row * (n / 32) + sb * 8);
  }
}

// One row of n (a multiple of 256) per workgroup: swiglu_quant_kernel's
// values, Q8_K-encoded, one wave per 256-value block.
__global__ __launch_bounds__(256) void swiglu_q8k_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                         Q8kRows o, int n) {
  const size_t row = blockIdx.x;
  const int lane = threadIdx.x & 63;
  for (int sb = threadIdx.x >> 6; sb < n / 256; sb += 4) {
    const float4 gv = reinterpret_cast<const float4*>(g + row * n + sb * 256)[lane];
    const float4 uv = reinterpret_cast<const float4*>(u + row * n + sb * 256)[lane];
    const float e[4] = {(gv.x / (1.0f + expf(-gv.x))) * uv.x, (gv.y / (1.0f + expf(-gv.y))) * uv.y,
                        (gv.z / (1.0f + expf(-gv.z))) * uv.z, (gv.w / (1.0f + expf(-gv.w))) * uv.w};
    q8k_split_store(lane, e, o.qs + row * n + sb * 256, o.d8 + row * (n / 256) + sb, o.bs32 + row * (n / 32) + sb * 8);
  }
}

}  // namespace zg

hipError_t zg::launch_rmsnorm(const float* x, const float* w, float* out, int n, float eps, hipStream_t st) {
  const bool row = n % 4 == 0 && n <= 4096 * kRmsV && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                                                       reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
  if (row) hipLaunchKernelGGL(rmsnorm_row_kernel, dim3(1), dim3(1024), 0, st, x, w, out, n, eps);
  else hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(256), 0, st, x, w, out, n, eps);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Model object
// ---------------------------------------------------------------------------

struct ZLayer {
  const uint8_t *q, *k, *v, *o, *gate, *up, *down;
  float *attn_norm, *ffn_norm, *q_norm, *k_norm;
  uint32_t qt[ZG_N_PROJ], il[ZG_N_PROJ];  // ggml type and layout per projection (ZG_PROJ_*)
  bool qkv_one = false, gu_one = false;    // Q|K|V, gate|up (SwiGLU) as one rmsnorm GEMV launch
  bool qkv_norm_each = false;              // else Q, K, V each with the rmsnorm prologue
  bool qk_norm_v = false;                  // else Q4_K Q|K with the prologue, which leaves x' for V
  bool gu_kq = false;                      // else Q4_K gate|up with rmsnorm and SwiGLU in one launch
  bool o_merge = false;                    // the O GEMV merges the attention splits itself
  bool qkv_attn = false;                   // Q|K|V GEMV and attention in one launch (qkv_attn_kernel)
};

struct zg_model {
  zg_ctx* ctx = nullptr;
  zg_model_desc d{};
  std::vector<ZLayer> layers;
  const uint8_t* embd = nullptr;
  const uint8_t* head = nullptr;
  float* out_norm = nullptr;
  float* inv_freq = nullptr;
  float* rope_cs = nullptr;  // this position's RoPE cos/sin table [head_dim]
  float* kv = nullptr;
  float *hidden = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *act = nullptr;
  float* xn = nullptr;  // rmsnorm output where a GEMV has no rmsnorm prologue [hidden]
  float* up = nullptr;  // up projection where gate|up is not one launch [ffn]
  float* logits = nullptr;
  float* part_o = nullptr;   // attention split outputs [nsplit][nq*HD]
  float* part_ml = nullptr;  // attention split (max, exp-sum) [nsplit][nq]
  uint64_t* best = nullptr;
  zg::DevState* st = nullptr;
  // qkv_attn_kernel: the step counter (every step start adds one: the
  // embedding launch or the previous step's last launch; never reset while
  // the model lives) and the Q|K|V rows as tagged 64-bit words (the counter
  // of the step that stored the row << 32 | fp32 bits)
  uint32_t* sync = nullptr;  // [0] step counter of the fused launches; [1] test hook: layer + 1 whose
                             // fused launch skips its tagged stores (0: none)
  uint64_t* qkv_tag = nullptr;
  int cus = 0;  // compute units of the device
  uint32_t* prompt = nullptr;  // device prompt buffer
  size_t prompt_cap = 0;
  uint32_t* out_tokens = nullptr;
  size_t out_cap = 0;
  int nsplit = 1;
  bool head_norm = false;  // the LM-head GEMV takes the output rmsnorm itself
  bool pf_ok = false;      // every layer projection has a batched-prefill GEMM (Q4_0 / Q8_0; Q4_K / Q6_K rows)
  bool pf_kq = false;      // some projection is Q4_K / Q6_K (Q8_K activation rows)
  std::vector<void*> owned;  // device allocations to free
  // references to the registry's uploaded weight copies this model reads,
  // each with the device address it resolved to: they outlive a zg_clear of
  // the context until the model is destroyed (a tensor interleaved into
  // model memory at creation drops its reference)
  std::vector<std::pair<const void*, std::shared_ptr<void>>> weight_refs;
  // Step graphs; each starts at the first layer, its embedding and RoPE
  // table already in place (start_step before a call's first graph, then
  // the previous graph's last launch):
  // g_prefill: layers + advance and the next prompt token's start;
  // g_step: layers + LM head + finalize and the chosen token's start (the
  // greedy loop); g_step_host: layers + LM head + finalize (zg_model_step,
  // which returns the step's final hidden state)
  hipGraphExec_t g_prefill = nullptr, g_step = nullptr, g_step_host = nullptr;
  // batched prefill: row buffers for chunks of up to pf_cap tokens,
  // allocated on first use
  size_t pf_cap = 0;
  float *pf_x = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr;
  float *pf_g = nullptr, *pf_u = nullptr;
  int8_t* pf_qs = nullptr;
  uint16_t* pf_qd = nullptr;
  // Q8_K activation rows of the K-quant GEMMs, and the attention's fp32
  // output rows they are quantized from when the O projection is K-quant
  int8_t* pf_ks = nullptr;
  float* pf_k8 = nullptr;
  int16_t* pf_kb = nullptr;
  float* pf_a = nullptr;
  // non-finite localisation: device result, [2][hidden] scan buffers
  // (rmsnorm output, sublayer output), and per KV row the token whose step
  // wrote it and how (kRowDecode rows can be replayed)
  NfScan* nf = nullptr;
  float* nf_buf = nullptr;
  std::vector<uint32_t> row_token;
  std::vector<uint8_t> row_kind;
  // the latch (record_first_nonfinite, inference_avx512.rs:233-262): first
  // localisation since the model was created or reset
  char nf_detail[kNfCap] = {};
  size_t nf_len = 0;
};

enum RowKind : uint8_t { kRowUnknown = 0, kRowDecode = 1, kRowBatched = 2 };

// Rows per batched-prefill chunk: longer prompts run in chunks, each
// attending to the cache rows of the chunks before it.
constexpr size_t kPrefillChunk = 512;

static zg_status model_alloc(zg_model* m, void** p, size_t bytes) {
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) return alloc_failed(m->ctx, e, "model", bytes);
  try {
    m->owned.push_back(*p);
  } catch (const std::bad_alloc&) {  // no exception crosses the C ABI
    hipFree(*p);
    *p = nullptr;
    return set_error(m->ctx, ZG_ERR_OUT_OF_MEMORY, "model: host allocation");
  }
  e = hipMemset(*p, 0, bytes);
  return hip_check(m->ctx, e, "model: memset");
}

static zg_status upload_f32(zg_model* m, float** dst, const float* src, size_t n) {
  zg_status s = model_alloc(m, reinterpret_cast<void**>(dst), n * sizeof(float));
  if (s) return s;
  return hip_check(m->ctx, hipMemcpy(*dst, src, n * sizeof(float), hipMemcpyHostToDevice), "model: upload");
}

static zg_status weight_dev(zg_model* m, const void* key, uint32_t qt, uint32_t il, size_t rows, size_t k,
                            const uint8_t** out) {
  if (!key) return set_error(m->ctx, ZG_ERR_INVALID_ARG, "model: null weight");
  if (m->d.device_pointers) {
    *out = static_cast<const uint8_t*>(key);
    return ZG_OK;
  }
  uint32_t got_il;
  std::shared_ptr<void> hold;
  zg_status s = resolve(m->ctx, key, tensor_bytes(qt, rows, k), qt, out, &got_il, &hold);
  if (s) return s;
  if (got_il != il) return set_error(m->ctx, ZG_ERR_INVALID_ARG, "model: weight %p layout %u, expected %u", key, got_il, il);
  if (hold) {
    try {
      m->weight_refs.emplace_back(*out, std::move(hold));
    } catch (const std::bad_alloc&) {  // no exception crosses the C ABI
      return set_error(m->ctx, ZG_ERR_OUT_OF_MEMORY, "model: host allocation");
    }
  }
  return ZG_OK;
}

// A plain-row Q4_0 / Q8_0 tensor of rows in fours, copied to X4 into model
// memory (*w and *il then name the copy); other tensors are left as they are.
static zg_status repack_x4(zg_model* m, const uint8_t** w, uint32_t qt, uint32_t* il, size_t rows, size_t k) {
  if (*il != 1 || (qt != ZG_Q4_0 && qt != ZG_Q8_0) || rows % 4 || k % 32 || (reinterpret_cast<uintptr_t>(*w) & 1u))
    return ZG_OK;
  const size_t bytes = tensor_bytes(qt, rows, k);
  void* dst = nullptr;
  zg_status s = model_alloc(m, &dst, bytes);
  if (s) return s;
  const int nb = (int)(k / 32), bb = qt == ZG_Q4_0 ? 18 : 34;
  const size_t units = rows / 4 * (size_t)nb;
  hipLaunchKernelGGL(interleave_x4_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, m->ctx->stream, *w,
                     static_cast<uint8_t*>(dst), units, nb, bb);
  s = hip_check(m->ctx, hipGetLastError(), "model: interleave launch");
  if (s) return s;
  *w = static_cast<const uint8_t*>(dst);
  *il = 4;
  return ZG_OK;
}

// An X4 Q4_0 / Q8_0 layer projection of a strip-sized in_dim, copied to
// split-scale X4 groups into model memory (*w and *il then name the copy;
// a model-owned source is queued on *drop for release once the copy has
// landed); other tensors are left as they are.  The strip kernel decodes the
// same lanes from either layout, so results keep their bits.
#ifndef ZG_MODEL_SPLIT
#define ZG_MODEL_SPLIT 1
#endif
static zg_status split_x4(zg_model* m, const uint8_t** w, uint32_t qt, uint32_t* il, size_t rows, size_t k,
                          std::vector<void*>* drop) {
  if (!ZG_MODEL_SPLIT || *il != 4 || (qt != ZG_Q4_0 && qt != ZG_Q8_0) || rows % 4 || !strip_path_ok((int)k) ||
      (reinterpret_cast<uintptr_t>(*w) & 15u))
    return ZG_OK;
  const size_t bytes = tensor_bytes(qt, rows, k);
  void* dst = nullptr;
  zg_status s = model_alloc(m, &dst, bytes);
  if (s) return s;
  const int nb = (int)(k / 32), qb = qt == ZG_Q4_0 ? 16 : 32;
  const size_t units = rows / 4 * (size_t)nb;
  hipLaunchKernelGGL(split_x4_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, m->ctx->stream, *w,
                     static_cast<uint8_t*>(dst), units, nb, qb);
  s = hip_check(m->ctx, hipGetLastError(), "model: split launch");
  if (s) return s;
  if (std::find(m->owned.begin(), m->owned.end(), static_cast<const void*>(*w)) != m->owned.end()) {
    try {
      drop->push_back(const_cast<uint8_t*>(*w));
    } catch (const std::bad_alloc&) {  // the copy stays owned until the model is destroyed
    }
  }
  *w = static_cast<const uint8_t*>(dst);
  *il = 5;
  return ZG_OK;
}

// rmsnorm of x into m->xn, for GEMVs without a rmsnorm prologue (the
// model's own buffer: a captured graph must not hold context scratch, which
// a later call may reallocate)
static zg_status model_rmsnorm(zg_model* m, const float* x, const float* gain, hipStream_t st) {
  return hip_check(m->ctx, launch_rmsnorm(x, gain, m->xn, (int)m->d.hidden, m->d.rms_eps, st), "rmsnorm launch");
}

// Output rmsnorm + LM head + argmax of the hidden state x.
static zg_status head_argmax(zg_model* m, const float* x, hipStream_t st) {
  const zg_model_desc& d = m->d;
  const float* xin = x;
  if (!m->head_norm) {
    zg_status s = model_rmsnorm(m, x, m->out_norm, st);
    if (s) return s;
    xin = m->xn;
  }
  return run_linear(m->ctx, xin, m->head, m->logits, d.hidden, d.vocab_padded, d.head_type, d.head_interleave, 0,
                    d.vocab_padded, EPI_ARGMAX, nullptr, m->best, m->head_norm ? PRO_RMSNORM : PRO_PLAIN, m->out_norm,
                    d.rms_eps, st, kGemvStream);
}

// Layer l's Q|K|V GEMV (rmsnorm prologue) and decode attention as one
// qkv_attn_kernel launch; aa holds the attention arguments.
static zg_status run_qkv_attn(zg_model* m, uint32_t l, const ZLayer& L, AttnArgs aa, hipStream_t st) {
  const zg_model_desc& d = m->d;
  const int HD = (int)d.head_dim, nkv = (int)d.n_kv_heads, g = (int)(d.n_q_heads / d.n_kv_heads);
  const size_t qd = (size_t)d.n_q_heads * HD, kvd = (size_t)nkv * HD;
  GemvArgs ga{};
  ga.nseg = 3;
  ga.k = (int)d.hidden;
  ga.x = m->hidden;
  ga.norm_w = L.attn_norm;
  ga.eps = d.rms_eps;
  const uint8_t* w[3] = {L.q, L.k, L.v};
  float* y[3] = {m->q, m->k, m->v};
  const size_t n[3] = {qd, kvd, kvd};
  uint32_t gb = 0;
  for (int i = 0; i < 3; i++) {
    ga.seg[i].w = w[i];
    ga.seg[i].y = y[i];
    ga.seg[i].resid = nullptr;
    ga.seg[i].g_begin = gb;
    ga.seg[i].row_lo = 0;
    ga.seg[i].row_hi = (uint32_t)n[i];
    gb += (uint32_t)(n[i] / 4);
  }
  ga.total_groups = gb;
  // the GEMV's rows go to the tagged buffer only: [Q | K | V] 64-bit words
  ga.seg[0].y = reinterpret_cast<float*>(m->qkv_tag);
  ga.seg[1].y = reinterpret_cast<float*>(m->qkv_tag + qd);
  ga.seg[2].y = reinterpret_cast<float*>(m->qkv_tag + qd + kvd);
  // one tag per step and layer: the buffer is shared by the layers
  ga.sync_epoch = m->sync;
  ga.sync_drop = m->sync + 1;
  ga.sync_mul = d.n_layers;
  ga.sync_add = l;
  aa.tagged = m->qkv_tag;
  aa.epoch = m->sync;
  aa.tag_mul = d.n_layers;
  aa.tag_add = l;
  const int n_attn = (int)d.n_q_heads * m->nsplit;
  const dim3 grid((unsigned)(n_attn + gb / 2)), block(256);
  const size_t shm = 2 * 4 * 2 * 16 * sizeof(float);  // the strip body's [2][4 waves][2 groups][16] partials
  const uint32_t qt = L.qt[ZG_PROJ_Q], il = L.il[ZG_PROJ_Q];
#define ZG_QKV_ATTN(QT, IL, HDV) hipLaunchKernelGGL((qkv_attn_kernel<QT, IL, HDV>), grid, block, shm, st, ga, aa, n_attn)
  // Q4_K rows, or X4 / split-scale X4 Q4_0 / Q8_0 (plain-row Q4_0 / Q8_0
  // projections are interleaved at model creation)
  if (qt != ZG_Q4K && il != 4 && il != 5)
    return set_error(m->ctx, ZG_ERR_UNSUPPORTED_QUANT, "qkv+attention: plain-row Q4_0/Q8_0");
  if (HD == 128) {
    if (qt == ZG_Q4K) ZG_QKV_ATTN(Q4K, 1, 128);
    else if (qt == ZG_Q4_0 && il == 5) ZG_QKV_ATTN(Q4_0, 5, 128);
    else if (qt == ZG_Q4_0) ZG_QKV_ATTN(Q4_0, 4, 128);
    else if (il == 5) ZG_QKV_ATTN(Q8_0, 5, 128);
    else ZG_QKV_ATTN(Q8_0, 4, 128);
  } else {
    if (qt == ZG_Q4K) ZG_QKV_ATTN(Q4K, 1, 64);
    else if (qt == ZG_Q4_0 && il == 5) ZG_QKV_ATTN(Q4_0, 5, 64);
    else if (qt == ZG_Q4_0) ZG_QKV_ATTN(Q4_0, 4, 64);
    else if (il == 5) ZG_QKV_ATTN(Q8_0, 5, 64);
    else ZG_QKV_ATTN(Q8_0, 4, 64);
  }
#undef ZG_QKV_ATTN
  return hip_check(m->ctx, hipGetLastError(), "qkv+attention launch");
}

// Record the per-token sequence on the context stream.  diag adds the
// non-finite scans of a localisation replay (never captured).
static zg_status record_layers(zg_model* m, hipStream_t st, bool diag = false) {
  const zg_model_desc& d = m->d;
  const int H = (int)d.hidden, F = (int)d.ffn, HD = (int)d.head_dim;
  const int qd = (int)(d.n_q_heads * d.head_dim), kvd = (int)(d.n_kv_heads * d.head_dim);
  zg_ctx* ctx = m->ctx;
  zg_status s = ZG_OK;
  const float scale = 1.0f / sqrtf((float)HD);
  for (uint32_t l = 0; l < d.n_layers; l++) {
    const ZLayer& L = m->layers[l];
    const uint32_t *qt = L.qt, *il = L.il;
    float* sub = m->nf_buf + H;  // diag: sublayer output alone
    auto scan = [&](const float* v, uint32_t stage) {
      hipLaunchKernelGGL(nf_scan_kernel, dim3(1), dim3(1024), 0, st, v, H, &m->st->err, m->nf, (l << 8) | stage);
      return hip_check(ctx, hipGetLastError(), "scan launch");
    };
    auto zero_sub = [&]() {
      hipLaunchKernelGGL(zero_kernel, dim3((H + 255) / 256), dim3(256), 0, st, sub, H);
      return hip_check(ctx, hipGetLastError(), "zero launch");
    };
    if (diag) {
      if ((s = hip_check(ctx, launch_rmsnorm(m->hidden, L.attn_norm, m->nf_buf, H, d.rms_eps, st), "rmsnorm launch")) ||
          (s = scan(m->nf_buf, NF_ATTN_NORM_IN)))
        return s;
    }
    AttnArgs aa{};
    aa.q = m->q;
    aa.k = m->k;
    aa.v = m->v;
    aa.q_norm = L.q_norm;
    aa.k_norm = L.k_norm;
    aa.rope_cs = m->rope_cs;
    aa.kcache = m->kv + (size_t)(2 * l) * d.max_ctx * kvd;
    aa.vcache = m->kv + (size_t)(2 * l + 1) * d.max_ctx * kvd;
    aa.out = m->nsplit == 1 ? m->attn : m->part_o;
    aa.part_ml = m->part_ml;
    aa.st = m->st;
    aa.nkv = (int)d.n_kv_heads;
    aa.g = (int)(d.n_q_heads / d.n_kv_heads);
    aa.nsplit = m->nsplit;
    aa.eps = d.rms_eps;
    aa.scale = scale;
    if (L.qkv_attn) {
      if ((s = run_qkv_attn(m, l, L, aa, st))) return s;
    } else {
      FusedDev qkv[3] = {{L.q, m->q, (size_t)qd, qt[ZG_PROJ_Q], il[ZG_PROJ_Q]},
                         {L.k, m->k, (size_t)kvd, qt[ZG_PROJ_K], il[ZG_PROJ_K]},
                         {L.v, m->v, (size_t)kvd, qt[ZG_PROJ_V], il[ZG_PROJ_V]}};
      if (L.qkv_one) {
        if ((s = run_fused(ctx, m->hidden, qkv, 3, H, PRO_RMSNORM, L.attn_norm, d.rms_eps, EPI_STORE, st))) return s;
      } else if (L.qkv_norm_each) {
        for (const FusedDev& f : qkv)
          if ((s = run_linear(ctx, m->hidden, f.w, f.y, H, f.n, f.qt, f.il, 0, f.n, EPI_STORE, nullptr, nullptr,
                              PRO_RMSNORM, L.attn_norm, d.rms_eps, st)))
            return s;
      } else if (L.qk_norm_v) {
        if ((s = run_kq_segs(ctx, m->hidden, qkv, 2, H, PRO_RMSNORM, L.attn_norm, d.rms_eps, st, m->xn))) return s;
        if ((s = run_linear(ctx, m->xn, qkv[2].w, qkv[2].y, H, qkv[2].n, qkv[2].qt, qkv[2].il, 0, qkv[2].n, EPI_STORE,
                            nullptr, nullptr, PRO_PLAIN, nullptr, 0.0f, st)))
          return s;
      } else {
        if ((s = model_rmsnorm(m, m->hidden, L.attn_norm, st))) return s;
        if ((s = run_fused(ctx, m->xn, qkv, 3, H, PRO_PLAIN, nullptr, 0.0f, EPI_STORE, st))) return s;
      }
      const dim3 ag(d.n_q_heads, m->nsplit), ab(kAttnWaves * 64);
      if (HD == 128) hipLaunchKernelGGL((attn_split_kernel<128, false>), ag, ab, 0, st, aa);
      else hipLaunchKernelGGL((attn_split_kernel<64, false>), ag, ab, 0, st, aa);
      if ((s = hip_check(ctx, hipGetLastError(), "attention launch"))) return s;
    }
    // y += O * attention (y the hidden state, or the zeroed scan buffer)
    auto o_proj = [&](float* y) -> zg_status {
      if (L.o_merge)
        return run_attn_o(ctx, m->part_o, m->part_ml, m->nsplit, HD, L.o, y, qd, H, qt[ZG_PROJ_O], il[ZG_PROJ_O], st);
      if (m->nsplit > 1) {
        const int thr = 256, nthr = qd / 8;
        hipLaunchKernelGGL(attn_merge_kernel, dim3((nthr + thr - 1) / thr), dim3(thr), 0, st, m->part_o, m->part_ml,
                           qd, HD, m->nsplit, m->attn);
        zg_status e = hip_check(ctx, hipGetLastError(), "attention merge launch");
        if (e) return e;
      }
      return run_linear(ctx, m->attn, L.o, y, qd, H, qt[ZG_PROJ_O], il[ZG_PROJ_O], 0, H, EPI_RESID, y, nullptr,
                        PRO_PLAIN, nullptr, 0.0f, st);
    };
    if (diag && ((s = zero_sub()) || (s = o_proj(sub)) || (s = scan(sub, NF_ATTN_OUT)))) return s;
    if ((s = o_proj(m->hidden))) return s;
    if (diag && (s = scan(m->hidden, NF_POST_ATTN))) return s;
    if (L.gu_one) {
      FusedDev gu[2] = {{L.gate, m->act, (size_t)F, qt[ZG_PROJ_GATE], il[ZG_PROJ_GATE]},
                        {L.up, nullptr, (size_t)F, qt[ZG_PROJ_UP], il[ZG_PROJ_UP]}};
      if ((s = run_fused(ctx, m->hidden, gu, 2, H, PRO_RMSNORM, L.ffn_norm, d.rms_eps, EPI_SWIGLU, st))) return s;
    } else if (L.gu_kq) {
      if ((s = run_kq_swiglu(ctx, m->hidden, L.gate, L.up, m->act, H, F, L.ffn_norm, d.rms_eps, st))) return s;
    } else {
      FusedDev gu[2] = {{L.gate, m->act, (size_t)F, qt[ZG_PROJ_GATE], il[ZG_PROJ_GATE]},
                        {L.up, m->up, (size_t)F, qt[ZG_PROJ_UP], il[ZG_PROJ_UP]}};
      if ((s = model_rmsnorm(m, m->hidden, L.ffn_norm, st))) return s;
      if ((s = run_fused(ctx, m->xn, gu, 2, H, PRO_PLAIN, nullptr, 0.0f, EPI_STORE, st))) return s;
      hipLaunchKernelGGL(silu_mul_kernel, dim3((F + 255) / 256), dim3(256), 0, st, m->act, m->up, F);
      if ((s = hip_check(ctx, hipGetLastError(), "swiglu launch"))) return s;
    }
    auto down_proj = [&](float* y) {
      return run_linear(ctx, m->act, L.down, y, F, H, qt[ZG_PROJ_DOWN], il[ZG_PROJ_DOWN], 0, H, EPI_RESID, y, nullptr,
                        PRO_PLAIN, nullptr, 0.0f, st);
    };
    if (diag && ((s = zero_sub()) || (s = down_proj(sub)) || (s = scan(sub, NF_MLP_OUT)))) return s;
    if ((s = down_proj(m->hidden))) return s;
    if (diag && (s = scan(m->hidden, NF_POST_MLP))) return s;
  }
  return ZG_OK;
}

static EmbedArgs embed_args(const zg_model* m) {
  EmbedArgs e;
  e.embd = m->embd;
  e.qt = m->d.embd_type;
  e.hidden = (int)m->d.hidden;
  e.out = m->hidden;
  e.inv_freq = m->inv_freq;
  e.half = (int)m->d.head_dim / 2;
  e.rope_cs = m->rope_cs;
  e.epoch = m->sync;
  e.best = m->best;
  return e;
}

// Start the step the state names (token, pos): issued by the host before
// the first layer launch of a call; after that every step graph starts the
// next step in its last launch.
static zg_status start_step(zg_model* m, hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(256), 0, st, embed_args(m), m->st);
  return hip_check(m->ctx, hipGetLastError(), "embed launch");
}

// A prompt token through the layers, then the next prompt token's start.
static zg_status record_prefill(zg_model* m, hipStream_t st) {
  zg_status s = record_layers(m, st);
  if (s) return s;
  hipLaunchKernelGGL(advance_embed_kernel, dim3(1), dim3(256), 0, st, m->st, m->prompt, embed_args(m));
  return hip_check(m->ctx, hipGetLastError(), "advance launch");
}

// A token through the layers and the LM head, then the start of the step of
// the token it chose (the greedy loop: no launch of its own for the embedding).
static zg_status record_step(zg_model* m, hipStream_t st) {
  const zg_model_desc& d = m->d;
  zg_status s = record_layers(m, st);
  if (s) return s;
  s = head_argmax(m, m->hidden, st);
  if (s) return s;
  hipLaunchKernelGGL(finalize_embed_kernel, dim3(1), dim3(256), 0, st, m->st, d.vocab_real, m->out_tokens,
                     embed_args(m));
  return hip_check(m->ctx, hipGetLastError(), "finalize launch");
}

// The same without the next step's start: zg_model_step returns this step's
// final hidden state, which the next embedding would overwrite.
static zg_status record_step_host(zg_model* m, hipStream_t st) {
  const zg_model_desc& d = m->d;
  zg_status s = record_layers(m, st);
  if (s) return s;
  s = head_argmax(m, m->hidden, st);
  if (s) return s;
  hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(1), 0, st, m->st, m->best, d.vocab_real, m->out_tokens);
  return hip_check(m->ctx, hipGetLastError(), "finalize launch");
}

static zg_status capture(zg_model* m, zg_status (*rec)(zg_model*, hipStream_t), hipGraphExec_t* out) {
  zg_ctx* ctx = m->ctx;
  hipGraph_t g = nullptr;
  zg_status s = hip_check(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "begin capture");
  if (s) return s;
  zg_status rs = rec(m, ctx->stream);
  hipError_t e = hipStreamEndCapture(ctx->stream, &g);
  if (rs) {
    if (g) hipGraphDestroy(g);
    return rs;
  }
  if ((s = hip_check(ctx, e, "end capture"))) return s;
  e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  return hip_check(ctx, e, "graph instantiate");
}

static zg_status prefill_alloc(zg_model* m) {
  if (m->pf_cap) return ZG_OK;
  const zg_model_desc& d = m->d;
  const size_t C = d.max_ctx < kPrefillChunk ? d.max_ctx : kPrefillChunk;
  const size_t H = d.hidden, F = d.ffn, qd = (size_t)d.n_q_heads * d.head_dim, kvd = (size_t)d.n_kv_heads * d.head_dim;
  const size_t kmax = std::max(H, std::max(qd, F));
  zg_status s = ZG_OK;
  auto al = [&](auto** p, size_t bytes) {
    if (!s) s = model_alloc(m, reinterpret_cast<void**>(p), bytes);
  };
  al(&m->pf_x, C * H * 4);
  al(&m->pf_q, C * qd * 4);
  al(&m->pf_k, C * kvd * 4);
  al(&m->pf_v, C * kvd * 4);
  al(&m->pf_g, C * F * 4);
  al(&m->pf_u, C * F * 4);
  al(&m->pf_qs, C * kmax);
  al(&m->pf_qd, C * (kmax / 32) * 2);
  if (m->pf_kq) {
    al(&m->pf_ks, C * kmax);
    al(&m->pf_k8, C * (kmax / 256) * 4);
    al(&m->pf_kb, C * (kmax / 32) * 2);
    al(&m->pf_a, C * qd * 4);
  }
  if (!s) m->pf_cap = C;
  return s;
}

static bool kq_type(uint32_t t) { return t == ZG_Q4K || t == ZG_Q6K; }

// Which activation encodings layer projections p0..p0+nseg-1 read: Q8_0
// rows (Q4_0 / Q8_0 weights), Q8_K rows (Q4_K / Q6_K weights).
static void act_needs(const ZLayer& L, int p0, int nseg, bool& q80, bool& q8k) {
  q80 = q8k = false;
  for (int i = 0; i < nseg; i++) (kq_type(L.qt[p0 + i]) ? q8k : q80) = true;
}

// rmsnorm of the chunk's rows into the encodings projections p0..p0+nseg-1
// read.
static zg_status norm_rows(zg_model* m, const ZLayer& L, int p0, int nseg, const float* w, size_t n, hipStream_t st) {
  const int H = (int)m->d.hidden;
  bool q80, q8k;
  act_needs(L, p0, nseg, q80, q8k);
  if (q80)
    hipLaunchKernelGGL(rmsnorm_quant_kernel, dim3((unsigned)n), dim3(256), 0, st, m->pf_x, w, m->pf_qs, m->pf_qd, H,
                       m->d.rms_eps);
  if (q8k)
    hipLaunchKernelGGL(rmsnorm_q8k_kernel, dim3((unsigned)n), dim3(256), 0, st, m->pf_x, w,
                       Q8kRows{m->pf_ks, m->pf_k8, m->pf_kb}, H, m->d.rms_eps);
  return hip_check(m->ctx, hipGetLastError(), "prefill rmsnorm launch");
}

// One chunk of n <= pf_cap prompt rows (device tokens) at positions
// pos0..pos0+n-1 through every layer, leaving the final hidden states in
// pf_x.  Per layer: rmsnorm + activation rows -> Q|K|V GEMM -> QK-norm +
// RoPE + cache store -> causal attention (+ activation rows) -> O GEMM (+=
// residual) -> rmsnorm + activation rows -> gate|up GEMM -> SwiGLU +
// activation rows -> down GEMM (+= residual).  Activation rows are Q8_0 for
// Q4_0 / Q8_0 weights and Q8_K for Q4_K / Q6_K weights; each fused encode
// gives the bits the separate quantizer would give for the same fp32 row.
// GEMMs of layer projections p0..p0+nseg-1 on the chunk's activation rows:
// one segmented launch per run of projections that share a type and layout.
static zg_status layer_gemm(zg_model* m, const ZLayer& L, int p0, const GemmSegDev* segs, int nseg, size_t n,
                            size_t k, bool accumulate, hipStream_t st) {
  for (int i = 0; i < nseg;) {
    int j = i + 1;
    while (j < nseg && L.qt[p0 + j] == L.qt[p0 + i] && L.il[p0 + j] == L.il[p0 + i]) j++;
    const uint32_t t = L.qt[p0 + i];
    zg_status s = kq_type(t) ? run_gemm_q8k(m->ctx, m->pf_ks, m->pf_k8, m->pf_kb, segs + i, j - i, n, k, t, accumulate, st)
                             : run_gemm(m->ctx, m->pf_qs, m->pf_qd, segs + i, j - i, n, k, t, L.il[p0 + i], accumulate, st);
    if (s) return s;
    i = j;
  }
  return ZG_OK;
}

static zg_status prefill_chunk(zg_model* m, const uint32_t* d_tokens, size_t n, uint32_t pos0, hipStream_t st) {
  const zg_model_desc& d = m->d;
  zg_ctx* ctx = m->ctx;
  const int H = (int)d.hidden, F = (int)d.ffn, HD = (int)d.head_dim;
  const int nq = (int)d.n_q_heads, nkv = (int)d.n_kv_heads;
  const size_t qd = (size_t)nq * HD, kvd = (size_t)nkv * HD;
  hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)n), dim3(256), 0, st, m->embd, d.embd_type, H, d_tokens,
                     m->pf_x, m->best);
  zg_status s = hip_check(ctx, hipGetLastError(), "prefill embed launch");
  const float scale = 1.0f / sqrtf((float)HD);
  for (uint32_t l = 0; l < d.n_layers && !s; l++) {
    const ZLayer& L = m->layers[l];
    float* kc = m->kv + (size_t)(2 * l) * d.max_ctx * kvd;
    float* vc = m->kv + (size_t)(2 * l + 1) * d.max_ctx * kvd;
    if ((s = norm_rows(m, L, ZG_PROJ_Q, 3, L.attn_norm, n, st))) break;
    const GemmSegDev qkv[3] = {{L.q, m->pf_q, qd}, {L.k, m->pf_k, kvd}, {L.v, m->pf_v, kvd}};
    if ((s = layer_gemm(m, L, ZG_PROJ_Q, qkv, 3, n, H, false, st))) break;
    QkStoreArgs qa{m->pf_q, m->pf_k, m->pf_v, L.q_norm, L.k_norm, m->inv_freq, kc, vc, nq, nkv, (int)pos0, d.rms_eps};
    const dim3 qg((unsigned)n, (unsigned)(nq + nkv));
    if (HD == 128) hipLaunchKernelGGL(qk_rope_store_kernel<128>, qg, dim3(64), 0, st, qa);
    else hipLaunchKernelGGL(qk_rope_store_kernel<64>, qg, dim3(64), 0, st, qa);
    if ((s = hip_check(ctx, hipGetLastError(), "prefill qk-rope launch"))) break;
    AttnArgs aa{};
    aa.q = m->pf_q;
    aa.kcache = kc;
    aa.vcache = vc;
    const bool o_kq = kq_type(L.qt[ZG_PROJ_O]);
    aa.out = o_kq ? m->pf_a : nullptr;
    aa.qs = m->pf_qs;
    aa.qsd = m->pf_qd;
    aa.part_ml = m->part_ml;
    aa.st = m->st;
    aa.nkv = nkv;
    aa.g = nq / nkv;
    aa.nsplit = 1;
    aa.split_len = (int)d.max_ctx;
    aa.eps = d.rms_eps;
    aa.scale = scale;
    aa.pos0 = (int)pos0;
    aa.row_stride = (int)qd;
    const dim3 ag((unsigned)nq, 1, (unsigned)n), ab(kAttnWaves * 64);
    if (HD == 128) hipLaunchKernelGGL((attn_split_kernel<128, true>), ag, ab, 0, st, aa);
    else hipLaunchKernelGGL((attn_split_kernel<64, true>), ag, ab, 0, st, aa);
    if ((s = hip_check(ctx, hipGetLastError(), "prefill attention launch"))) break;
    if (o_kq && (s = run_quantize_q8k_split(ctx, m->pf_a, m->pf_ks, m->pf_k8, m->pf_kb, n, qd, st))) break;
    const GemmSegDev o{L.o, m->pf_x, (size_t)H};
    if ((s = layer_gemm(m, L, ZG_PROJ_O, &o, 1, n, qd, true, st))) break;
    if ((s = norm_rows(m, L, ZG_PROJ_GATE, 2, L.ffn_norm, n, st))) break;
    const GemmSegDev gu[2] = {{L.gate, m->pf_g, (size_t)F}, {L.up, m->pf_u, (size_t)F}};
    if ((s = layer_gemm(m, L, ZG_PROJ_GATE, gu, 2, n, H, false, st))) break;
    if (kq_type(L.qt[ZG_PROJ_DOWN]))
      hipLaunchKernelGGL(swiglu_q8k_kernel, dim3((unsigned)n), dim3(256), 0, st, m->pf_g, m->pf_u,
                         Q8kRows{m->pf_ks, m->pf_k8, m->pf_kb}, F);
    else
      hipLaunchKernelGGL(swiglu_quant_kernel, dim3((unsigned)n), dim3(256), 0, st, m->pf_g, m->pf_u, m->pf_qs,
                         m->pf_qd, F);
    if ((s = hip_check(ctx, hipGetLastError(), "prefill swiglu launch"))) break;
    const GemmSegDev dn{L.down, m->pf_x, (size_t)H};
    if ((s = layer_gemm(m, L, ZG_PROJ_DOWN, &dn, 1, n, F, true, st))) break;
  }
  return s;
}

// The whole prompt (already in m->prompt[off..off+n)) in chunks, then the LM
// head on the last row and finalize: the state must hold pos = pos0 + n - 1
// (finalize advances it past the prompt).  Returns the last chunk's row count.
static zg_status prefill_run(zg_model* m, size_t off, size_t n, uint32_t pos0, size_t* last_rows) {
  const zg_model_desc& d = m->d;
  hipStream_t st = m->ctx->stream;
  zg_status s = prefill_alloc(m);
  size_t rows = 0;
  for (size_t c = 0; c < n && !s; c += rows) {
    rows = std::min(m->pf_cap, n - c);
    s = prefill_chunk(m, m->prompt + off + c, rows, pos0 + (uint32_t)c, st);
  }
  if (s) return s;
  s = head_argmax(m, m->pf_x + (rows - 1) * d.hidden, st);
  if (s) return s;
  hipLaunchKernelGGL(finalize_embed_kernel, dim3(1), dim3(256), 0, st, m->st, d.vocab_real, m->out_tokens,
                     embed_args(m));
  *last_rows = rows;
  return hip_check(m->ctx, hipGetLastError(), "finalize launch");
}

extern "C" zg_status zg_model_create(zg_ctx* ctx, const zg_model_desc* desc, zg_model** out) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!desc || !out || !desc->layers) return set_error(ctx, ZG_ERR_INVALID_ARG, "model: null descriptor");
  *out = nullptr;
  const zg_model_desc& d = *desc;
  if (d.n_layers == 0 || d.hidden == 0 || d.ffn == 0 || d.n_kv_heads == 0 || d.n_q_heads % d.n_kv_heads ||
      d.n_q_heads / d.n_kv_heads > (uint32_t)kMaxG || (d.head_dim != 128 && d.head_dim != 64) || d.max_ctx == 0 ||
      d.vocab_real > d.vocab_padded || d.vocab_padded == 0)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "model: unsupported dimensions");
  const size_t qd = (size_t)d.n_q_heads * d.head_dim, kvd = (size_t)d.n_kv_heads * d.head_dim;
  // ForwardPassDispatch quants: each projection Q4_0 / Q8_0 (plain or X4) or
  // Q4_K / Q6_K (plain, in_dim a multiple of 256); token_embd any of the four
  const size_t proj_k[ZG_N_PROJ] = {d.hidden, d.hidden, d.hidden, qd, d.hidden, d.hidden, d.ffn};
  for (uint32_t l = 0; l < d.n_layers; l++)
    for (int p = 0; p < ZG_N_PROJ; p++) {
      const uint32_t qt = d.layer_quants ? d.layer_quants[l].type[p] : d.lin_type;
      const uint32_t il = d.layer_quants ? d.layer_quants[l].interleave[p] : d.lin_interleave;
      const bool q40 = qt == ZG_Q4_0 || qt == ZG_Q8_0, kq = qt == ZG_Q4K || qt == ZG_Q6K;
      if (!(q40 && (il == 1 || il == 4)) && !(kq && il == 1))
        return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "model: layer %u projection %d: type %u layout %u", l, p, qt, il);
      if (kq && proj_k[p] % 256)
        return set_error(ctx, ZG_ERR_INVALID_ARG, "model: layer %u projection %d: K-quant in_dim %zu %% 256", l, p,
                         proj_k[p]);
    }
  if (d.embd_type != ZG_Q4_0 && d.embd_type != ZG_Q8_0 && d.embd_type != ZG_Q4K && d.embd_type != ZG_Q6K)
    return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "model: token_embd type %u", d.embd_type);
  if ((d.embd_type == ZG_Q4K || d.embd_type == ZG_Q6K) && d.hidden % 256)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "model: K-quant token_embd needs hidden %% 256 == 0");
  for (size_t kk : {(size_t)d.hidden, qd, (size_t)d.ffn})
    if (kk % 64 || kk > kMaxPairK) return set_error(ctx, ZG_ERR_INVALID_ARG, "model: in_dim %zu not supported", kk);
  if (qd % 4 || kvd % 4 || d.ffn % 4 || d.hidden % 4) return set_error(ctx, ZG_ERR_INVALID_ARG, "model: rows % 4");
  hipSetDevice(ctx->device);
  zg_model* m = new (std::nothrow) zg_model();
  if (!m) return set_error(ctx, ZG_ERR_OUT_OF_MEMORY, "model: host allocation");
  m->ctx = ctx;
  m->d = d;
  m->d.layers = nullptr;
  m->d.layer_quants = nullptr;
  zg_status s = ZG_OK;
  const size_t H = d.hidden, F = d.ffn;
  try {
    m->layers.resize(d.n_layers);
    m->owned.reserve(40 + 4 * (size_t)d.n_layers);  // room for every buffer the model allocates
  } catch (const std::bad_alloc&) {  // no exception crosses the C ABI
    delete m;  // not yet counted: the context stays destroyable
    return set_error(ctx, ZG_ERR_OUT_OF_MEMORY, "model: host allocation");
  }
  ctx->live_models++;  // released by zg_model_destroy (also on the error path below)
  for (uint32_t l = 0; l < d.n_layers && !s; l++) {
    const zg_layer_weights& W = d.layers[l];
    ZLayer& L = m->layers[l];
    if (!W.attn_norm || !W.ffn_norm || !W.q_norm || !W.k_norm) {
      s = set_error(ctx, ZG_ERR_INVALID_ARG, "model: null norm weight");
      break;
    }
    for (int p = 0; p < ZG_N_PROJ; p++) {
      L.qt[p] = d.layer_quants ? d.layer_quants[l].type[p] : d.lin_type;
      L.il[p] = d.layer_quants ? d.layer_quants[l].interleave[p] : d.lin_interleave;
    }
    const uint32_t *qt = L.qt, *il = L.il;
    if ((s = weight_dev(m, W.attn_q, qt[ZG_PROJ_Q], il[ZG_PROJ_Q], qd, H, &L.q))) break;
    if ((s = weight_dev(m, W.attn_k, qt[ZG_PROJ_K], il[ZG_PROJ_K], kvd, H, &L.k))) break;
    if ((s = weight_dev(m, W.attn_v, qt[ZG_PROJ_V], il[ZG_PROJ_V], kvd, H, &L.v))) break;
    if ((s = weight_dev(m, W.attn_o, qt[ZG_PROJ_O], il[ZG_PROJ_O], H, qd, &L.o))) break;
    if ((s = weight_dev(m, W.ffn_gate, qt[ZG_PROJ_GATE], il[ZG_PROJ_GATE], F, H, &L.gate))) break;
    if ((s = weight_dev(m, W.ffn_up, qt[ZG_PROJ_UP], il[ZG_PROJ_UP], F, H, &L.up))) break;
    if ((s = weight_dev(m, W.ffn_down, qt[ZG_PROJ_DOWN], il[ZG_PROJ_DOWN], H, F, &L.down))) break;
    if ((s = upload_f32(m, &L.attn_norm, W.attn_norm, H))) break;
    if ((s = upload_f32(m, &L.ffn_norm, W.ffn_norm, H))) break;
    if ((s = upload_f32(m, &L.q_norm, W.q_norm, d.head_dim))) break;
    if ((s = upload_f32(m, &L.k_norm, W.k_norm, d.head_dim))) break;
  }
  if (!s) s = weight_dev(m, d.token_embd, d.embd_type, 1, d.vocab_padded, H, &m->embd);
  if (!s) s = weight_dev(m, d.lm_head, d.head_type, d.head_interleave, d.vocab_padded, H, &m->head);
  // plain-row Q4_0 / Q8_0 projections and LM head (the .smodel-v1 and GGUF
  // layouts) are interleaved to X4 into memory the model owns: the X4
  // kernels give the same bits as the plain-row ones on the same weights
  // (lane (b, r) decodes block b of row 4 g + r in either layout) and read
  // 16 contiguous quant bytes per lane instead of 2-byte-aligned blocks
  for (uint32_t l = 0; l < d.n_layers && !s; l++) {
    ZLayer& L = m->layers[l];
    const uint8_t** w[ZG_N_PROJ] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
    const size_t rows[ZG_N_PROJ] = {qd, kvd, kvd, H, F, F, H}, ks[ZG_N_PROJ] = {H, H, H, qd, H, H, F};
    for (int p = 0; p < ZG_N_PROJ && !s; p++) s = repack_x4(m, w[p], L.qt[p], &L.il[p], rows[p], ks[p]);
  }
  if (!s) s = repack_x4(m, &m->head, d.head_type, &m->d.head_interleave, d.vocab_padded, H);
  // then the layer projections to split-scale X4 groups (the LM head keeps
  // X4: its tall launches stream contiguous group-blocks into LDS)
  std::vector<void*> drop;
  for (uint32_t l = 0; l < d.n_layers && !s; l++) {
    ZLayer& L = m->layers[l];
    const uint8_t** w[ZG_N_PROJ] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
    const size_t rows[ZG_N_PROJ] = {qd, kvd, kvd, H, F, F, H}, ks[ZG_N_PROJ] = {H, H, H, qd, H, H, F};
    for (int p = 0; p < ZG_N_PROJ && !s; p++) s = split_x4(m, w[p], L.qt[p], &L.il[p], rows[p], ks[p], &drop);
  }
  if (!s) s = hip_check(ctx, hipStreamSynchronize(ctx->stream), "model: interleave");
  if (!s) {
    // the X4 copies made from plain rows and since split are not read again
    for (void* p : drop) {
      auto it = std::find(m->owned.begin(), m->owned.end(), p);
      if (it != m->owned.end()) {
        hipFree(p);
        m->owned.erase(it);
      }
    }
  }
  if (!s) {
    // the interleave copies have landed: registry uploads that no tensor of
    // the model reads any more (every repacked plain-row tensor's) are
    // released, so a zg_clear frees them instead of the model keeping two
    // copies of those weights alive
    std::vector<const void*> used = {m->embd, m->head};
    for (const ZLayer& L : m->layers)
      for (const uint8_t* w : {L.q, L.k, L.v, L.o, L.gate, L.up, L.down}) used.push_back(w);
    auto unused = [&](const std::pair<const void*, std::shared_ptr<void>>& e) {
      return std::find(used.begin(), used.end(), e.first) == used.end();
    };
    m->weight_refs.erase(std::remove_if(m->weight_refs.begin(), m->weight_refs.end(), unused), m->weight_refs.end());
  }
  if (!s && !d.output_norm) s = set_error(ctx, ZG_ERR_INVALID_ARG, "model: null output_norm");
  if (!s) s = upload_f32(m, &m->out_norm, d.output_norm, H);
  if (!s) {
    // RopeContext::new (ops.rs:79-93): inv_freq[i] = theta^(-2i/head_dim) in f32
    float inv[64];  // head_dim <= 128
    for (uint32_t i = 0; i < d.head_dim / 2; i++) {
      const float ex = -2.0f * (float)i / (float)d.head_dim;
      inv[i] = powf(d.rope_theta, ex);
    }
    s = upload_f32(m, &m->inv_freq, inv, d.head_dim / 2);
  }
  // kAttnDecodeSplits workgroups per query head share its live context (one
  // CU loads ~150 GB/s, so a head's K/V rows are spread over several CUs);
  // fewer when max_ctx has fewer than 8 rows per split.  More splits make
  // attention faster but the merge in the O projection's prologue slower:
  // every O workgroup reads nsplit x 8 KB of split outputs (Qwen3-1.7B,
  // eager trace: 8 splits 4.42 + 4.78 us, 4 splits 5.26 + 4.04 us with the
  // splits cut by max_ctx).  With the fused Q|K|V + attention launch, at
  // max_ctx 384 (every split one 64-row round of K/V loads at 6): decode
  // 1,491 / 1,495 tok/s at 6 splits against 1,478 / 1,476 at 4 on one box,
  // and 1,491 / 1,491 at 6 against 1,471 / 1,470 at 5, 1,471 / 1,469 at 7
  // and 1,468 / 1,470 at 8 on another; token-by-token prompt steps, short
  // contexts, lose 1.7 % at 6
  {
    const uint32_t ns = (d.max_ctx + 7) / 8;
    m->nsplit = (int)(ns < (uint32_t)kAttnDecodeSplits ? ns : (uint32_t)kAttnDecodeSplits);
  }
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->kv), (size_t)d.n_layers * 2 * d.max_ctx * kvd * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->rope_cs), d.head_dim * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->hidden), H * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->q), qd * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->k), kvd * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->v), kvd * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->attn), qd * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->act), F * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->logits), (size_t)d.vocab_padded * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->part_o), (size_t)m->nsplit * qd * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->part_ml), (size_t)m->nsplit * d.n_q_heads * 2 * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->best), sizeof(uint64_t));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->st), sizeof(DevState));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->sync), 2 * sizeof(uint32_t));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->qkv_tag), (qd + 2 * kvd) * sizeof(uint64_t));
  if (!s) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device) != hipSuccess || cus <= 0) cus = 256;
    m->cus = cus;
  }
  m->prompt_cap = d.max_ctx;
  m->out_cap = d.max_ctx;
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->prompt), m->prompt_cap * sizeof(uint32_t));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->out_tokens), m->out_cap * sizeof(uint32_t));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->xn), H * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->up), F * sizeof(float));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->nf), sizeof(NfScan));
  if (!s) s = model_alloc(m, reinterpret_cast<void**>(&m->nf_buf), 2 * H * sizeof(float));
  if (!s) {
    try {
      m->row_token.assign(d.max_ctx, 0);
      m->row_kind.assign(d.max_ctx, kRowUnknown);
    } catch (const std::bad_alloc&) {  // no exception crosses the C ABI
      s = set_error(ctx, ZG_ERR_OUT_OF_MEMORY, "model: host allocation");
    }
  }
  if (!s) {
    // per layer, which GEMVs are one launch with the rmsnorm (or
    // attention-merge) prologue: X4 weights, or plain Q4_0 / Q8_0 at a
    // strip-sized in_dim, of one type across the fused projections
    m->pf_ok = true;
    for (ZLayer& L : m->layers) {
      const uint32_t *qt = L.qt, *il = L.il;
      const FusedDev q3[3] = {{L.q, m->q, qd, qt[ZG_PROJ_Q], il[ZG_PROJ_Q]},
                              {L.k, m->k, kvd, qt[ZG_PROJ_K], il[ZG_PROJ_K]},
                              {L.v, m->v, kvd, qt[ZG_PROJ_V], il[ZG_PROJ_V]}};
      const FusedDev g2[2] = {{L.gate, m->act, F, qt[ZG_PROJ_GATE], il[ZG_PROJ_GATE]},
                              {L.up, nullptr, F, qt[ZG_PROJ_UP], il[ZG_PROJ_UP]}};
      L.qkv_one = fused_x4_ok(m->hidden, q3, 3, H) || fused_plain_ok(m->hidden, q3, 3, H, PRO_RMSNORM) ||
                  fused_kq_ok(m->hidden, q3, 3, H, PRO_RMSNORM, L.attn_norm);
      L.gu_one = fused_x4_ok(m->hidden, g2, 2, H) || fused_plain_ok(m->hidden, g2, 2, H, PRO_RMSNORM);
      L.qkv_norm_each = !L.qkv_one;
      for (const FusedDev& f : q3)
        L.qkv_norm_each = L.qkv_norm_each && rmsnorm_fused_ok(f.qt, f.il, H, f.n, f.w, m->hidden, EPI_STORE);
      L.qk_norm_v = !L.qkv_one && !L.qkv_norm_each && fused_kq_ok(m->hidden, q3, 2, H, PRO_RMSNORM, L.attn_norm);
      L.gu_kq = !L.gu_one && kq_swiglu_ok(qt[ZG_PROJ_GATE], qt[ZG_PROJ_UP], il[ZG_PROJ_GATE], il[ZG_PROJ_UP], H,
                                          L.gate, L.up, m->hidden, L.ffn_norm);
      const uint32_t ot = qt[ZG_PROJ_O], oil = il[ZG_PROJ_O];
      L.o_merge = m->nsplit > 1 && ((attn_merge_gemv_ok(ot, oil, qd) && attn_merge_hd_ok(ot, (int)d.head_dim) &&
                                     pair_path_ok(ot, oil, qd, H, L.o, m->part_o)) ||
                                    kq_attn_o_ok(ot, oil, qd, m->nsplit, (int)d.head_dim, L.o, m->part_o));
      // batched prefill: Q4_0 / Q8_0 any shape; Q4_K / Q6_K plain rows of a
      // width in 64-column tiles and an in_dim in whole superblocks
      const size_t width[ZG_N_PROJ] = {qd, kvd, kvd, H, F, F, H}, in_dim[ZG_N_PROJ] = {H, H, H, qd, H, H, F};
      for (int p = 0; p < ZG_N_PROJ; p++) {
        const bool kq = kq_type(qt[p]) && il[p] == 1 && width[p] % 64 == 0 && in_dim[p] % 256 == 0;
        m->pf_ok = m->pf_ok && (qt[p] == ZG_Q4_0 || qt[p] == ZG_Q8_0 || kq);
        m->pf_kq = m->pf_kq || kq_type(qt[p]);
      }
      // Q|K|V and attention in one launch: Q4_0 / Q8_0 / Q4_K of one type and
      // layout on the one-launch strip path, in_dim 2048 (four strips, the
      // attention's 256-thread workgroups), two-group batches that never
      // straddle a KV head, and one batch per workgroup
      const size_t groups = (qd + 2 * kvd) / 4;
      L.qkv_attn = (fused_x4_ok(m->hidden, q3, 3, H) || fused_plain_ok(m->hidden, q3, 3, H, PRO_RMSNORM)) &&
                   (qt[ZG_PROJ_Q] == ZG_Q4_0 || qt[ZG_PROJ_Q] == ZG_Q8_0 || qt[ZG_PROJ_Q] == ZG_Q4K) &&
                   il[ZG_PROJ_Q] == il[ZG_PROJ_K] &&
                   il[ZG_PROJ_Q] == il[ZG_PROJ_V] && H == 2048 && (d.head_dim == 128 || d.head_dim == 64) &&
                   groups / 2 <= (size_t)m->cus * 4;
    }
    m->head_norm =
        rmsnorm_fused_ok(d.head_type, m->d.head_interleave, H, d.vocab_padded, m->head, m->hidden, EPI_ARGMAX);
  }
  if (!s) s = capture(m, record_prefill, &m->g_prefill);
  if (!s) s = capture(m, record_step, &m->g_step);
  if (!s) s = capture(m, record_step_host, &m->g_step_host);
  if (s) {
    zg_model_destroy(m);
    return s;
  }
  *out = m;
  return ZG_OK;
}

extern "C" void zg_model_destroy(zg_model* m) {
  if (!m) return;
  zg_ctx* ctx = m->ctx;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  for (hipGraphExec_t g : {m->g_prefill, m->g_step, m->g_step_host})
    if (g) hipGraphExecDestroy(g);
  for (void* p : m->owned) hipFree(p);
  delete m;  // drops the weight references: copies cleared from the registry are freed here
  if (--ctx->live_models == 0 && ctx->destroy_pending) destroy_context(ctx);
}

static zg_status set_state(zg_model* m, uint32_t token, uint32_t pos, uint32_t n_prompt, uint32_t gen_cap) {
  DevState h{};
  h.token = token;
  h.pos = pos;
  h.n_prompt = n_prompt;
  h.gen_cap = gen_cap;
  h.err_step = kNoStep;
  return hip_check(m->ctx, hipMemcpyAsync(m->st, &h, sizeof h, hipMemcpyHostToDevice, m->ctx->stream), "state upload");
}

static const char* nf_stage_name(uint32_t stage) {
  switch (stage) {
    case NF_ATTN_NORM_IN: return "attn_norm_in";
    case NF_ATTN_OUT: return "attn_out";
    case NF_POST_ATTN: return "post_attn_residual";
    case NF_MLP_OUT: return "mlp_out";
    case NF_POST_MLP: return "post_mlp_residual";
    case NF_K_CACHE: return "k_cache";
    case NF_V_CACHE: return "v_cache";
    default: return "?";
  }
}

// Fills the latch after a call failed with a non-finite error whose first
// failing step ran at position p_fail.  The first KV row (in position
// order, then layer) holding a non-finite value is where a non-finite value
// first reached a later step; with none, the failing step itself made it
// (after the last layer's K/V, or in the LM head).  That row's step runs
// again with the scans when it was a decode step (same token, same rows
// before it, same launches: the same bits); a row written by the batched
// prefill names the cache row instead.  A value that reached neither the
// cache nor the logits is not seen.  Best effort: a HIP failure here leaves
// the latch empty.
static void localise_nonfinite(zg_model* m, uint32_t p_fail) {
  zg_ctx* ctx = m->ctx;
  const zg_model_desc& d = m->d;
  hipStream_t st = ctx->stream;
  if (m->nf_len || p_fail >= d.max_ctx || p_fail >= (1u << 24) || 2 * d.n_layers > 255) return;
  const size_t kvd = (size_t)d.n_kv_heads * d.head_dim;
  NfScan h{0, 0, 0, 0xFFFFFFFFu};
  if (hipMemcpyAsync(m->nf, &h, sizeof h, hipMemcpyHostToDevice, st) != hipSuccess) return;
  hipLaunchKernelGGL(kv_scan_kernel, dim3(p_fail + 1, 2 * d.n_layers), dim3(256), 0, st, m->kv, (size_t)d.max_ctx,
                     (int)kvd, m->nf);
  if (hipGetLastError() != hipSuccess || hipMemcpyAsync(&h, m->nf, sizeof h, hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return;
  const bool kv_hit = h.kv_key != 0xFFFFFFFFu;
  const uint32_t q = kv_hit ? h.kv_key >> 8 : p_fail;
  uint32_t row = 0;
  if (m->row_kind[q] == kRowDecode) {
    if (set_state(m, m->row_token[q], q, 0, 0) || start_step(m, st) || record_layers(m, st, true)) return;
  } else if (kv_hit) {
    // a cache row the decode step cannot reproduce: name it
    const uint32_t slot = h.kv_key & 0xFFu;
    row = q;
    hipLaunchKernelGGL(nf_scan_kernel, dim3(1), dim3(1024), 0, st, m->kv + ((size_t)slot * d.max_ctx + q) * kvd,
                       (int)kvd, nullptr, m->nf, ((slot / 2) << 8) | (slot & 1 ? NF_V_CACHE : NF_K_CACHE));
    if (hipGetLastError() != hipSuccess) return;
  } else {
    return;
  }
  if (hipMemcpyAsync(&h, m->nf, sizeof h, hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess || h.tag == 0)
    return;
  const uint32_t stage = h.tag & 0xFFu, layer = h.tag >> 8;
  const float v = __builtin_bit_cast(float, h.bits);
  char name[32];
  if (stage == NF_K_CACHE || stage == NF_V_CACHE) snprintf(name, sizeof name, "%s[%u]", nf_stage_name(stage), row);
  else snprintf(name, sizeof name, "%s", nf_stage_name(stage));
  // "L{:02} {} n{} i{}" (inference_avx512.rs:259), here for the first
  // non-finite element (finite_diag's flags, :108-113)
  char text[64];
  const int n = snprintf(text, sizeof text, "L%02u %s n%d i%d", layer, name, std::isnan(v) ? 1 : 0, std::isinf(v) ? 1 : 0);
  m->nf_len = n < 0 ? 0 : std::min((size_t)n, kNfCap);
  memcpy(m->nf_detail, text, m->nf_len);
}

// Status of a finished call: its first failure, as the reference's loop
// stops at the first error (within one step an attention failure comes
// before the LM head's).  p_fail: the position of the step at err_step.
static zg_status state_status(zg_model* m, const DevState& h, uint32_t p_fail) {
  const uint32_t e = h.err_step != kNoStep ? h.err_first : h.err;
  if ((h.err | e) & 8u)
    return set_error(m->ctx, ZG_ERR_HIP, "qkv+attention: a completion wait timed out (step %u)", h.err_step);
  if (e & 5u) localise_nonfinite(m, p_fail);
  char at[kNfCap + 3] = "";
  if (m->nf_len) snprintf(at, sizeof at, " @%.*s", (int)m->nf_len, m->nf_detail);
  if (e & 4u) return set_error(m->ctx, ZG_ERR_ATTENTION, "attention: non-finite scores (step %u)%s", h.err_step, at);
  if (e & 1u) return set_error(m->ctx, ZG_ERR_NONFINITE_LOGITS, "LM head: non-finite logits (step %u)%s", h.err_step, at);
  if (e & 2u) return set_error(m->ctx, ZG_ERR_ARGMAX_IN_PADDING, "LM head: argmax in padding (step %u)", h.err_step);
  return ZG_OK;
}

static void note_rows(zg_model* m, size_t pos0, const uint32_t* tokens, size_t n, RowKind kind) {
  for (size_t i = 0; i < n && pos0 + i < m->row_kind.size(); i++) {
    m->row_token[pos0 + i] = tokens[i];
    m->row_kind[pos0 + i] = kind;
  }
}

// Every step writes KV row `pos` before any read of rows <= pos, and every
// step or generate call uploads its own position, so a new sequence needs
// no device work: reset waits for in-flight work and clears the non-finite
// latch.
extern "C" void zg_model_reset(zg_model* m) {
  if (!m) return;
  hipSetDevice(m->ctx->device);
  hipStreamSynchronize(m->ctx->stream);
  m->nf_len = 0;
}

extern "C" zg_status zg_model_test_drop_qkv_stores(zg_model* m, int32_t layer) {
  if (!m) return ZG_ERR_INVALID_ARG;
  hipSetDevice(m->ctx->device);
  const uint32_t v = layer < 0 ? 0u : (uint32_t)layer + 1u;
  zg_status s = hip_check(m->ctx, hipMemcpyAsync(m->sync + 1, &v, sizeof v, hipMemcpyHostToDevice, m->ctx->stream),
                          "drop hook upload");
  if (!s) s = hip_check(m->ctx, hipStreamSynchronize(m->ctx->stream), "drop hook upload");
  return s;
}

extern "C" size_t zg_model_first_nonfinite(const zg_model* m, char* buf, size_t cap) {
  if (!m || !buf) return 0;
  const size_t n = std::min(m->nf_len, cap);
  memcpy(buf, m->nf_detail, n);
  return n;
}

extern "C" zg_status zg_model_step(zg_model* m, uint32_t token, uint32_t pos, float* hidden_out, float* logits,
                                   uint32_t* next_token, float* max_logit) {
  if (!m) return ZG_ERR_INVALID_ARG;
  zg_ctx* ctx = m->ctx;
  if (pos >= m->d.max_ctx) return set_error(ctx, ZG_ERR_CONTEXT_FULL, "position %u >= max_ctx %u", pos, m->d.max_ctx);
  if (token >= m->d.vocab_padded) return set_error(ctx, ZG_ERR_INVALID_ARG, "token %u out of range", token);
  hipSetDevice(ctx->device);
  note_rows(m, pos, &token, 1, kRowDecode);
  zg_status s = set_state(m, token, pos, 0, 0);
  if (!s) s = start_step(m, ctx->stream);
  if (s) return s;
  if ((s = hip_check(ctx, hipGraphLaunch(m->g_step_host, ctx->stream), "graph launch"))) return s;
  zg::DevState h{};
  if ((s = hip_check(ctx, hipMemcpyAsync(&h, m->st, sizeof h, hipMemcpyDeviceToHost, ctx->stream), "state download")))
    return s;
  if (hidden_out &&
      (s = hip_check(ctx, hipMemcpyAsync(hidden_out, m->hidden, m->d.hidden * 4, hipMemcpyDeviceToHost, ctx->stream),
                     "download")))
    return s;
  if (logits && (s = hip_check(ctx, hipMemcpyAsync(logits, m->logits, (size_t)m->d.vocab_padded * 4,
                                                   hipMemcpyDeviceToHost, ctx->stream), "download")))
    return s;
  if ((s = hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync"))) return s;
  if ((s = state_status(m, h, pos))) return s;
  return lm_head_status(ctx, h.best, m->d.vocab_real, next_token, max_logit);
}

extern "C" zg_status zg_model_prefill(zg_model* m, const uint32_t* tokens, size_t n, uint32_t pos0, float* hidden_out,
                                      uint32_t* next_token, float* max_logit) {
  if (!m) return ZG_ERR_INVALID_ARG;
  zg_ctx* ctx = m->ctx;
  if (!tokens || n == 0) return set_error(ctx, ZG_ERR_INVALID_ARG, "prefill: no tokens");
  if (!m->pf_ok) return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "prefill: the GEMMs take Q4_0 / Q8_0 projections and plain Q4_K / Q6_K ones of widths in 64s and in_dims in 256s");
  if ((size_t)pos0 + n > m->d.max_ctx)
    return set_error(ctx, ZG_ERR_CONTEXT_FULL, "prefill: positions %u..%zu exceed max_ctx %u", pos0, pos0 + n - 1,
                     m->d.max_ctx);
  for (size_t i = 0; i < n; i++)
    if (tokens[i] >= m->d.vocab_padded) return set_error(ctx, ZG_ERR_INVALID_ARG, "prefill: token %u out of range", tokens[i]);
  hipSetDevice(ctx->device);
  note_rows(m, pos0, tokens, n, kRowBatched);
  zg_status s = hip_check(ctx, hipMemcpyAsync(m->prompt, tokens, n * 4, hipMemcpyHostToDevice, ctx->stream),
                          "prompt upload");
  if (!s) s = set_state(m, 0, pos0 + (uint32_t)n - 1, 0, 0);
  size_t rows = 0;
  if (!s) s = prefill_run(m, 0, n, pos0, &rows);
  if (s) return s;
  zg::DevState h{};
  if ((s = hip_check(ctx, hipMemcpyAsync(&h, m->st, sizeof h, hipMemcpyDeviceToHost, ctx->stream), "state download")))
    return s;
  if (hidden_out && (s = hip_check(ctx, hipMemcpyAsync(hidden_out, m->pf_x + (rows - 1) * m->d.hidden, m->d.hidden * 4,
                                                      hipMemcpyDeviceToHost, ctx->stream), "download")))
    return s;
  if ((s = hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync"))) return s;
  if ((s = state_status(m, h, pos0 + (uint32_t)n - 1))) return s;
  return lm_head_status(ctx, h.best, m->d.vocab_real, next_token, max_logit);
}

extern "C" zg_status zg_model_generate(zg_model* m, const uint32_t* prompt, size_t n_prompt, size_t n_gen,
                                       uint32_t* out_tokens, double* prefill_seconds, double* gen_seconds) {
  return zg_model_generate_ex(m, prompt, n_prompt, n_gen, 0, out_tokens, prefill_seconds, gen_seconds);
}

extern "C" zg_status zg_model_generate_ex(zg_model* m, const uint32_t* prompt, size_t n_prompt, size_t n_gen,
                                          uint32_t flags, uint32_t* out_tokens, double* prefill_seconds,
                                          double* gen_seconds) {
  if (!m) return ZG_ERR_INVALID_ARG;
  zg_ctx* ctx = m->ctx;
  if (!prompt || n_prompt == 0 || n_gen == 0 || !out_tokens) return set_error(ctx, ZG_ERR_INVALID_ARG, "generate: bad args");
  if (n_prompt + n_gen - 1 > m->d.max_ctx || n_prompt > m->prompt_cap || n_gen > m->out_cap)
    return set_error(ctx, ZG_ERR_CONTEXT_FULL, "generate: %zu + %zu tokens exceed max_ctx %u", n_prompt, n_gen,
                     m->d.max_ctx);
  for (size_t i = 0; i < n_prompt; i++)
    if (prompt[i] >= m->d.vocab_padded) return set_error(ctx, ZG_ERR_INVALID_ARG, "generate: prompt token out of range");
  hipSetDevice(ctx->device);
  zg_status s = hip_check(ctx, hipMemcpyAsync(m->prompt, prompt, n_prompt * 4, hipMemcpyHostToDevice, ctx->stream),
                          "prompt upload");
  if (s) return s;
  const bool batched = (flags & ZG_GEN_BATCHED_PREFILL) != 0;
  const bool eager = (flags & ZG_GEN_EAGER) != 0;
  if (flags & ~(ZG_GEN_BATCHED_PREFILL | ZG_GEN_EAGER))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "generate: unknown flags 0x%x", flags);
  if (batched && eager) return set_error(ctx, ZG_ERR_INVALID_ARG, "generate: ZG_GEN_EAGER is for token-by-token steps");
  // one token through the layers (and the LM head): the captured graph, or
  // the same launches issued directly
  auto run_one = [&](bool head) -> zg_status {
    if (eager) return head ? record_step(m, ctx->stream) : record_prefill(m, ctx->stream);
    return hip_check(ctx, hipGraphLaunch(head ? m->g_step : m->g_prefill, ctx->stream), "graph launch");
  };
  if (batched && !m->pf_ok)
    return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "generate: the batched prefill's GEMMs take Q4_0 / Q8_0 and plain Q4_K / Q6_K projections");
  if (batched && (s = prefill_alloc(m))) return s;
  note_rows(m, 0, prompt, n_prompt, batched ? kRowBatched : kRowDecode);
  if ((s = set_state(m, prompt[0], batched ? (uint32_t)n_prompt - 1 : 0, (uint32_t)n_prompt, (uint32_t)n_gen)))
    return s;
  if ((s = hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync"))) return s;
  auto t0 = std::chrono::steady_clock::now();
  if (batched) {
    // the whole prompt as Q8_0-activation GEMMs, then the LM head on its
    // last row, producing generated token 0
    size_t rows = 0;
    if ((s = prefill_run(m, 0, n_prompt, 0, &rows))) return s;
  } else {
    // prompt tokens 0..n-2 through the layers one by one; the last one also
    // through the LM head, producing generated token 0
    if ((s = start_step(m, ctx->stream))) return s;
    for (size_t i = 0; i + 1 < n_prompt; i++)
      if ((s = run_one(false))) return s;
    if ((s = run_one(true))) return s;
  }
  if ((s = hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync"))) return s;
  auto t1 = std::chrono::steady_clock::now();
  // greedy decode: each generated token goes back through the layers
  for (size_t j = 1; j < n_gen; j++)
    if ((s = run_one(true))) return s;
  if ((s = hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync"))) return s;
  auto t2 = std::chrono::steady_clock::now();
  if (prefill_seconds) *prefill_seconds = std::chrono::duration<double>(t1 - t0).count();
  if (gen_seconds) *gen_seconds = std::chrono::duration<double>(t2 - t1).count();
  zg::DevState h{};
  if ((s = hip_check(ctx, hipMemcpy(&h, m->st, sizeof h, hipMemcpyDeviceToHost), "state download"))) return s;
  if ((s = hip_check(ctx, hipMemcpy(out_tokens, m->out_tokens, n_gen * 4, hipMemcpyDeviceToHost), "tokens download")))
    return s;
  // generated token j - 1 was the input of the step at position n_prompt - 1 + j
  note_rows(m, n_prompt, out_tokens, n_gen - 1, kRowDecode);
  const size_t last = n_prompt + n_gen - 2;
  return state_status(m, h, (uint32_t)(h.err_step == kNoStep ? last : n_prompt - 1 + h.err_step));
}
