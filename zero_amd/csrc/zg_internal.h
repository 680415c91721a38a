// zg_internal.h -- host-side internals shared by the C ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <memory>
#include <string>
#include <vector>

#include "../../include/zero_gpu.h"

namespace zg {

// weight_layout.rs:45 caps the registry at 512 interleaved tensors; this
// registry also holds plain tensors, so it is larger.
constexpr size_t kMaxEntries = 4096;
// Largest in_dim the LDS-staged pair kernel accepts: the padded x copy
// (36 floats per 32) plus the block sums must fit a 64 KiB workgroup LDS
// allocation.
constexpr size_t kMaxPairK = 14080;

struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
};

struct RegEntry {
  uintptr_t key = 0;  // host start address (weight_layout.rs ADDRS)
  size_t bytes = 0;
  uint32_t qt = 0;
  uint32_t il = 1;    // weight_layout.rs GROUPS
  void* dev = nullptr;
  // Owner of an uploaded copy (null for borrowed device bytes).  A model
  // that resolved this tensor holds a second reference, so zg_clear drops
  // the registry entry while the bytes live until the last model using
  // them is destroyed.
  std::shared_ptr<void> hold;
};

// One weight segment of a prefill GEMM: n output columns into y [m][n].
struct GemmSegDev {
  const uint8_t* w;
  float* y;
  size_t n;
};

struct FusedDev {
  const uint8_t* w;
  float* y;
  size_t n;
  uint32_t qt;
  uint32_t il;
};

}  // namespace zg

struct zg_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::vector<zg::RegEntry> reg;  // sorted by key
  zg::DevBuf d_x, d_out, d_aux;
  void* h_pinned = nullptr;
  uint64_t* d_best = nullptr;
  std::string last_error;
  // models created on this context and not yet destroyed; zg_destroy of a
  // context with live models is deferred to the last zg_model_destroy
  int live_models = 0;
  bool destroy_pending = false;
  // this device's copy of the fixed Q8_K scratch array of
  // zg_linear_q4k_vnni_noalloc (resolved by zg_init)
  uint8_t* noalloc_scratch = nullptr;
};

namespace zg {

zg_status set_error(zg_ctx* ctx, zg_status code, const char* fmt, ...);
zg_status hip_check(zg_ctx* ctx, hipError_t e, const char* what);
// ZG_ERR_OUT_OF_MEMORY for a failed hipMalloc, with the runtime's error slot cleared
zg_status alloc_failed(zg_ctx* ctx, hipError_t e, const char* what, size_t bytes);
size_t tensor_bytes(uint32_t qt, size_t rows, size_t k);
zg_status ensure_buf(zg_ctx* ctx, DevBuf& b, size_t bytes);
zg_status resolve(zg_ctx* ctx, const void* w, size_t need, uint32_t qt, const uint8_t** dev, uint32_t* il,
                  std::shared_ptr<void>* hold = nullptr);
// releases the context's own device resources and the context itself
void destroy_context(zg_ctx* ctx);
// looks up this device's address of the fixed no-allocation scratch array
zg_status noalloc_scratch_setup(zg_ctx* ctx);
bool pair_path_ok(uint32_t qt, uint32_t il, size_t k, size_t n, const void* w, const void* x);
zg_status check_shape(zg_ctx* ctx, uint32_t qt, uint32_t il, size_t k, size_t n);
zg_status run_linear(zg_ctx* ctx, const float* x, const uint8_t* w, float* y, size_t k, size_t n, uint32_t qt,
                     uint32_t il, size_t start, size_t end, int epi, const float* resid, uint64_t* best, int pro,
                     const float* norm_w, float eps, hipStream_t st, uint32_t gemv_flags = 0);
bool rmsnorm_fused_ok(uint32_t qt, uint32_t il, size_t k, size_t n, const void* w, const void* x, int epi);
bool kq_swiglu_ok(uint32_t qt_gate, uint32_t qt_up, uint32_t il_gate, uint32_t il_up, size_t k, const void* gate,
                  const void* up, const void* x, const float* norm_w);
zg_status run_kq_swiglu(zg_ctx* ctx, const float* x, const uint8_t* gate, const uint8_t* up, float* y, size_t k,
                        size_t n, const float* norm_w, float eps, hipStream_t st);
bool fused_x4_ok(const float* x, const FusedDev* segs, size_t nseg, size_t k);
bool fused_plain_ok(const float* x, const FusedDev* segs, size_t nseg, size_t k, int pro);
bool fused_kq_ok(const float* x, const FusedDev* segs, size_t nseg, size_t k, int pro, const float* norm_w);
zg_status run_kq_segs(zg_ctx* ctx, const float* x, const FusedDev* segs, size_t nseg, size_t k, int pro,
                      const float* norm_w, float eps, hipStream_t st, float* xn_out = nullptr);
zg_status run_fused(zg_ctx* ctx, const float* x, const FusedDev* segs, size_t nseg, size_t k, int pro,
                    const float* norm_w, float eps, int epi, hipStream_t st);
zg_status run_attn_o(zg_ctx* ctx, const float* part_o, const float* part_ml, int nsplit, int hd, const uint8_t* w,
                     float* y, size_t k, size_t n, uint32_t qt, uint32_t il, hipStream_t st);
zg_status stage_in(zg_ctx* ctx, const void* src, size_t bytes, DevBuf& dst);
zg_status lm_head_status(zg_ctx* ctx, uint64_t packed, size_t vocab_real, uint32_t* token, float* max_val);

zg_status run_gemm(zg_ctx* ctx, const int8_t* qs, const uint16_t* xd, const GemmSegDev* segs, int nseg, size_t m,
                   size_t k, uint32_t w_type, uint32_t interleave, bool accumulate, hipStream_t st);
// Q8_K split activations (qs [rows][k], d8 [rows][k/256], bs32 [rows][k/32])
// and the K-quant (Q4_K / Q6_K, one type per call) prefill GEMM over 1..3
// segments of widths that are multiples of 64 (zg_kgemm.hip)
zg_status run_quantize_q8k_split(zg_ctx* ctx, const float* x, int8_t* qs, float* d8, int16_t* bs32, size_t rows,
                                 size_t k, hipStream_t st);
zg_status run_gemm_q8k(zg_ctx* ctx, const int8_t* qs, const float* d8, const int16_t* bs32, const GemmSegDev* segs,
                       int nseg, size_t m, size_t k, uint32_t w_type, bool accumulate, hipStream_t st);

hipError_t launch_rmsnorm(const float* x, const float* w, float* out, int n, float eps, hipStream_t st);

}  // namespace zg
