// zg_kernels.h -- kernel argument blocks and host launchers (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace zg {

// PRO_ATTN: x holds split-context attention outputs and the kernel merges
// them into the activation vector (strip path only).
// PRO_Q8X: the activation is a row of Q8_0 blocks (GemvArgs::xq) and the
// block dots are integer (strip kernel only).
enum Prologue : int { PRO_PLAIN = 0, PRO_RMSNORM = 1, PRO_ATTN = 2, PRO_Q8X = 3 };
enum Epilogue : int { EPI_STORE = 0, EPI_RESID = 1, EPI_ARGMAX = 2, EPI_SWIGLU = 3 };

// One projection of a (possibly fused) X4 GEMV launch.  Groups
// [g_begin, g_begin + rows/4) of the launch's group space belong to it;
// only local rows in [row_lo, row_hi) are stored.
struct GemvSeg {
  const uint8_t* w;
  float* y;
  const float* resid;  // EPI_RESID: y[row] = resid[row] + dot
  uint32_t g_begin;
  uint32_t row_lo, row_hi;
};

struct GemvArgs {
  GemvSeg seg[3];
  int nseg;
  int k;                  // in_dim (multiple of 64 on the pair path)
  uint32_t total_groups;  // groups over all segments
  const float* x;         // activation (16-byte aligned)
  const float* norm_w;    // PRO_RMSNORM gain
  float eps;
  uint64_t* best;         // EPI_ARGMAX packed candidate slot
  // PRO_ATTN: x is [attn_nsplit][k] split outputs, attn_ml [attn_nsplit][k /
  // attn_hd] their (max, exp-sum) pairs
  const float* attn_ml;
  int attn_nsplit, attn_hd;
  uint32_t flags;  // kGemvStream
  const uint8_t* xq;  // PRO_Q8X: k / 32 Q8_0 blocks (34 bytes, 2-byte aligned)
  // tagged stores (the fused Q|K|V + attention launch): each segment's y is
  // a uint64_t array, row r holding (tag << 32) | the row's fp32 bits,
  // stored as one agent-scope 64-bit store; tag = *sync_epoch * sync_mul +
  // sync_add (the step counter times the layer count plus the layer)
  const uint32_t* sync_epoch;
  uint32_t sync_mul, sync_add;
  // tagged stores: when sync_drop is non-null and *sync_drop == sync_add + 1,
  // the launch skips its tagged row stores (a test of the readers' bounded
  // wait: they give up and report the timeout; 0 drops nothing)
  const uint32_t* sync_drop;
  // PRO_RMSNORM: workgroup 0 also stores the normalized x here (k floats)
  // when non-null, for a following GEMV without the prologue
  float* xn_out;
};

// The weights are streamed without allocating in the last-level cache:
// set by the device-resident decode step, whose KV cache and activations
// should stay cached across the 330 MB LM-head read.
constexpr uint32_t kGemvStream = 1;
// The weights are split-scale X4 groups (interleave 5, strip_load_split):
// strip-kernel launches only.
constexpr uint32_t kGemvSplit = 2;

struct GenericArgs {
  const uint8_t* w;
  const float* x;
  float* y;
  const float* resid;
  uint64_t* best;
  size_t k;
  size_t row_lo, row_hi;
  uint32_t qt;
  int il;
  int epi;
  // Q4_K strip kernel only: rmsnorm prologue (norm_w non-null) and, with
  // EPI_SWIGLU, the up projection paired row for row with w (gate):
  // y[r] = silu(gate . x) * (up . x)
  const float* norm_w;
  float eps;
  const uint8_t* w_up;
  // Q4_K strip kernel, EPI_STORE: nseg > 1 concatenates up to 3 projections
  // of the same x (rows [seg_end[i-1], seg_end[i]) are segment i's rows 0..,
  // weights seg_w[i], outputs seg_y[i]); w / y / row range are then unused
  int nseg;
  const uint8_t* seg_w[3];
  float* seg_y[3];
  uint32_t seg_end[3];
  // Q4_K strip kernel, attention-merge prologue: x holds the attention
  // splits [attn_nsplit][k], attn_ml their (max, exp-sum) per head of attn_hd
  const float* attn_ml;
  int attn_nsplit, attn_hd;
  // rmsnorm prologue: workgroup 0 also stores the normalized x here (k
  // floats) when non-null, for a following GEMV without the prologue
  float* xn_out;
};

struct DequantArgs {
  const uint8_t* w;
  float* out;
  size_t rows, k;
  uint32_t qt;
  int il;
};

hipError_t launch_gemv_x4(const GemvArgs& a, uint32_t qt, int pro, int epi, hipStream_t st);
// Plain row-major Q4_0 / Q8_0 through the strip kernel (groups = 4 rows);
// prologue none or rmsnorm, epilogue store, residual or argmax.
bool plain_strip_ok(uint32_t qt, uint32_t il, size_t k, size_t n, const void* w, const void* x);
// in_dim accepted by the strip kernel: a multiple of 512 up to 8192
bool strip_path_ok(int k);
// Q4_K rows the strip kernel takes (launch_gemv_plain with qt Q4_K)
bool kq_strip_ok(uint32_t qt, uint32_t il, size_t k, size_t n, const void* w, const void* x);
// attention splits the strip kernel's merge prologue takes
bool attn_merge_strip_ok(int nsplit, int hd, size_t k);
hipError_t launch_gemv_plain(const GemvArgs& a, uint32_t qt, int pro, int epi, hipStream_t st);
// LDS bytes the X4 streaming kernel needs for in_dim k.
size_t gemv_x4_lds_bytes(uint32_t qt, int k);
hipError_t launch_gemv_generic(const GenericArgs& a, hipStream_t st);
hipError_t launch_dequant(const DequantArgs& a, bool pair_path, hipStream_t st);
// Q4_K / Q6_K fast path (row-major superblocks, in_dim a multiple of 256
// and at most kMaxKqK so that x and its 16-element sums fit 64 KiB of LDS).
constexpr size_t kMaxKqK = 15360;
bool kq_path_ok(uint32_t qt, uint32_t il, size_t k, const void* w, const void* x);
size_t kq_lds_bytes(int k);
hipError_t launch_gemv_kq(const GenericArgs& a, hipStream_t st);
bool kq_fused_ok(uint32_t qt, uint32_t il, size_t k, const void* w, const void* x);
hipError_t launch_kq_fused(const GenericArgs& a, bool rmsnorm, hipStream_t st);
bool kq_attn_o_ok(uint32_t qt, uint32_t il, size_t k, int nsplit, int hd, const void* w, const void* x);
hipError_t launch_kq_attn_o(const GenericArgs& a, hipStream_t st);
// The strip GEMV can merge attention splits in its prologue (PRO_ATTN).
bool attn_merge_gemv_ok(uint32_t qt, uint32_t il, size_t k);
// Its lanes merge the splits at their own x-block quarters, so a head must
// hold whole lane units: 32 elements (Q4_0 / Q8_0 blocks), 64 (Q4_K, id 12:
// a sub-block pair).
inline bool attn_merge_hd_ok(uint32_t qt, int hd) { return hd > 0 && hd % (qt == 12u ? 64 : 32) == 0; }
hipError_t launch_fp16(const uint16_t* in, float* out, size_t n, hipStream_t st);
hipError_t launch_fill_u64(uint64_t* p, uint64_t v, hipStream_t st);
hipError_t launch_read_floor(const void* src, size_t bytes, int loads_per_thread, uint32_t* sink, hipStream_t st);
hipError_t launch_strip_loads(const uint8_t* w, const float* x, size_t rows, uint32_t* sink, hipStream_t st);

}  // namespace zg
