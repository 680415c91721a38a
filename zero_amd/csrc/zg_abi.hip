// zg_abi.hip -- C ABI of include/zero_gpu.h: context, weight registry and
// operator dispatch for the gfx950 kernels.
//
// The registry restates kernel/src/weight_layout.rs (sorted table keyed by
// the tensor's host start address, exact-match group lookup, uniform
// rebase) and adds what a GPU needs on top: every registered key maps to a
// device copy of the tensor bytes (byte-identical to the host bytes).
#include <hip/hip_runtime.h>

#include <new>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <iterator>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/zero_gpu.h"
#include "zg_internal.h"
#include "zg_kernels.h"

using namespace zg;

// ---------------------------------------------------------------------------
// Context helpers
// ---------------------------------------------------------------------------

zg_status zg::set_error(zg_ctx* ctx, zg_status code, const char* fmt, ...) {
  if (ctx) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    ctx->last_error = buf;
  }
  return code;
}

// A failing HIP call also leaves its code in the runtime's per-thread
// last-error slot, which the next hipGetLastError() after an unrelated
// launch would report: every error path reads that slot once to clear it.
zg_status zg::hip_check(zg_ctx* ctx, hipError_t e, const char* what) {
  if (e == hipSuccess) return ZG_OK;
  (void)hipGetLastError();
  return set_error(ctx, ZG_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

zg_status zg::alloc_failed(zg_ctx* ctx, hipError_t e, const char* what, size_t bytes) {
  (void)hipGetLastError();
  return set_error(ctx, ZG_ERR_OUT_OF_MEMORY, "%s: hipMalloc(%zu): %s", what, bytes, hipGetErrorString(e));
}

static bool type_geom(uint32_t qt, size_t* be, size_t* bb) {
  switch (qt) {
    case ZG_Q4_0: *be = 32; *bb = 18; return true;
    case ZG_Q8_0: *be = 32; *bb = 34; return true;
    case ZG_Q4K: *be = 256; *bb = 144; return true;
    case ZG_Q6K: *be = 256; *bb = 210; return true;
    default: return false;
  }
}

size_t zg::tensor_bytes(uint32_t qt, size_t rows, size_t k) {
  size_t be, bb;
  if (!type_geom(qt, &be, &bb)) return 0;
  return rows * (k / be) * bb;
}

zg_status zg::ensure_buf(zg_ctx* ctx, DevBuf& b, size_t bytes) {
  if (b.bytes >= bytes) return ZG_OK;
  if (b.ptr) hipFree(b.ptr);
  b.ptr = nullptr;
  b.bytes = 0;
  hipError_t e = hipMalloc(&b.ptr, bytes);
  if (e != hipSuccess) return alloc_failed(ctx, e, "scratch", bytes);
  b.bytes = bytes;
  return ZG_OK;
}

static hipStream_t pick_stream(zg_ctx* ctx, void* stream) {
  return stream ? reinterpret_cast<hipStream_t>(stream) : ctx->stream;
}

// ---------------------------------------------------------------------------
// Lifecycle
// ---------------------------------------------------------------------------

extern "C" zg_status zg_init(int device, zg_ctx** out) {
  if (!out) return ZG_ERR_INVALID_ARG;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return ZG_ERR_HIP;
  if (hipSetDevice(device) != hipSuccess) return ZG_ERR_HIP;
  zg_ctx* ctx = new (std::nothrow) zg_ctx();
  if (!ctx) return ZG_ERR_OUT_OF_MEMORY;
  ctx->device = device;
  // A blocking stream: work on it is ordered against the legacy null stream,
  // so callers that stage data with null-stream copies need no extra sync.
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamDefault) != hipSuccess) {
    delete ctx;
    return ZG_ERR_HIP;
  }
  if (hipMalloc(&ctx->d_best, sizeof(uint64_t) * 4) != hipSuccess) {
    (void)hipGetLastError();
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return ZG_ERR_OUT_OF_MEMORY;
  }
  // the no-allocation entry point's scratch address on this device
  if (noalloc_scratch_setup(ctx) != ZG_OK) {
    hipFree(ctx->d_best);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return ZG_ERR_HIP;
  }
  *out = ctx;
  return ZG_OK;
}

void zg::destroy_context(zg_ctx* ctx) {
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  zg_clear(ctx);
  for (DevBuf* b : {&ctx->d_x, &ctx->d_out, &ctx->d_aux}) {
    if (b->ptr) hipFree(b->ptr);
  }
  if (ctx->h_pinned) hipHostFree(ctx->h_pinned);
  if (ctx->d_best) hipFree(ctx->d_best);
  hipStreamDestroy(ctx->stream);
  delete ctx;
}

// A model keeps using its context's stream and error slot, so a context
// with live models is released by the last zg_model_destroy instead.
extern "C" void zg_destroy(zg_ctx* ctx) {
  if (!ctx) return;
  if (ctx->live_models > 0) {
    ctx->destroy_pending = true;
    return;
  }
  destroy_context(ctx);
}

extern "C" const char* zg_last_error(const zg_ctx* ctx) { return ctx ? ctx->last_error.c_str() : "null context"; }

extern "C" void* zg_stream(zg_ctx* ctx) { return ctx ? reinterpret_cast<void*>(ctx->stream) : nullptr; }

// ---------------------------------------------------------------------------
// Registry (kernel/src/weight_layout.rs)
// ---------------------------------------------------------------------------

static zg_status do_register(zg_ctx* ctx, uintptr_t key, const void* host, const void* dev, size_t bytes,
                             uint32_t qt, uint32_t il) {
  if (!ctx || !key || bytes == 0) return set_error(ctx, ZG_ERR_INVALID_ARG, "register: null key or zero bytes");
  size_t be, bb;
  if (!type_geom(qt, &be, &bb)) return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "register: unsupported quant %u", qt);
  if (il != 1 && il != 4) return set_error(ctx, ZG_ERR_INVALID_ARG, "register: interleave %u not in {1,4}", il);
  // The packer only interleaves Q4_0/Q8_0 (silicatepack.py:836-851).
  if (il == 4 && qt != ZG_Q4_0 && qt != ZG_Q8_0)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "register: interleave 4 needs Q4_0 or Q8_0");
  if (ctx->reg.size() >= kMaxEntries) return set_error(ctx, ZG_ERR_REGISTRY_FULL, "register: registry full");
  if (key > UINTPTR_MAX - bytes) return set_error(ctx, ZG_ERR_INVALID_ARG, "register: key range wraps");
  // Registered byte ranges are disjoint: an interior address resolves to
  // exactly one tensor.  The table is sorted, so only the neighbours of the
  // insertion point can overlap [key, key + bytes).
  auto it = std::upper_bound(ctx->reg.begin(), ctx->reg.end(), key,
                             [](uintptr_t k, const RegEntry& r) { return k < r.key; });
  if (it != ctx->reg.begin() && std::prev(it)->key + std::prev(it)->bytes > key)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "register: [%#zx, +%zu) overlaps a registered tensor", (size_t)key, bytes);
  if (it != ctx->reg.end() && key + bytes > it->key)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "register: [%#zx, +%zu) overlaps a registered tensor", (size_t)key, bytes);
  hipSetDevice(ctx->device);
  RegEntry e;
  e.key = key;
  e.bytes = bytes;
  e.qt = qt;
  e.il = il;
  if (dev) {
    e.dev = const_cast<void*>(dev);
  } else {
    hipError_t he = hipMalloc(&e.dev, bytes);
    if (he != hipSuccess) return alloc_failed(ctx, he, "register", bytes);
    he = hipMemcpy(e.dev, host, bytes, hipMemcpyHostToDevice);
    if (he != hipSuccess) {
      hipFree(e.dev);
      return hip_check(ctx, he, "register: upload");
    }
    const int device = ctx->device;
    try {
      e.hold = std::shared_ptr<void>(e.dev, [device](void* p) {
        hipSetDevice(device);
        hipFree(p);
      });
    } catch (const std::bad_alloc&) {  // the deleter has already run
      return set_error(ctx, ZG_ERR_OUT_OF_MEMORY, "register: host allocation");
    }
  }
  try {
    ctx->reg.insert(it, e);
  } catch (const std::bad_alloc&) {  // no exception crosses the C ABI; e.hold frees the copy
    return set_error(ctx, ZG_ERR_OUT_OF_MEMORY, "register: registry growth failed");
  }
  return ZG_OK;
}

extern "C" zg_status zg_register_weight(zg_ctx* ctx, const void* host_ptr, size_t bytes, uint32_t ggml_type,
                                        uint32_t interleave) {
  if (!host_ptr) return set_error(ctx, ZG_ERR_INVALID_ARG, "register: null host pointer");
  return do_register(ctx, reinterpret_cast<uintptr_t>(host_ptr), host_ptr, nullptr, bytes, ggml_type, interleave);
}

extern "C" zg_status zg_register_weight_device(zg_ctx* ctx, const void* key, const void* dev_ptr, size_t bytes,
                                               uint32_t ggml_type, uint32_t interleave) {
  if (!dev_ptr) return set_error(ctx, ZG_ERR_INVALID_ARG, "register: null device pointer");
  return do_register(ctx, reinterpret_cast<uintptr_t>(key), nullptr, dev_ptr, bytes, ggml_type, interleave);
}

extern "C" uint32_t zg_group_of(const zg_ctx* ctx, const void* host_ptr) {
  if (!ctx) return 1;
  const uintptr_t k = reinterpret_cast<uintptr_t>(host_ptr);
  auto it = std::lower_bound(ctx->reg.begin(), ctx->reg.end(), k,
                             [](const RegEntry& r, uintptr_t key) { return r.key < key; });
  if (it != ctx->reg.end() && it->key == k) return it->il;
  return 1;
}

extern "C" void zg_rebase(zg_ctx* ctx, int64_t delta) {
  if (!ctx || delta == 0) return;
  for (RegEntry& e : ctx->reg) e.key = (uintptr_t)((int64_t)e.key + delta);
}

// Drops every registration.  Uploaded copies that a live model resolved
// stay allocated (the model holds a reference) until that model is
// destroyed; the others are freed here.
extern "C" void zg_clear(zg_ctx* ctx) {
  if (!ctx) return;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  ctx->reg.clear();
}

extern "C" size_t zg_registered_count(const zg_ctx* ctx) { return ctx ? ctx->reg.size() : 0; }

// Resolve a host weight pointer to its device bytes.  Exact start match
// gives the tensor and its layout; an interior pointer resolves only inside
// a plain (interleave 1) tensor, as weight_layout::group_of treats interior
// pointers as plain (weight_layout.rs:13-19).
zg_status zg::resolve(zg_ctx* ctx, const void* w, size_t need, uint32_t qt, const uint8_t** dev, uint32_t* il,
                      std::shared_ptr<void>* hold) {
  const uintptr_t k = reinterpret_cast<uintptr_t>(w);
  auto it = std::upper_bound(ctx->reg.begin(), ctx->reg.end(), k,
                             [](uintptr_t key, const RegEntry& r) { return key < r.key; });
  if (it == ctx->reg.begin()) return set_error(ctx, ZG_ERR_NOT_REGISTERED, "weight %p is not registered", w);
  --it;
  const size_t off = k - it->key;
  if (off >= it->bytes) return set_error(ctx, ZG_ERR_NOT_REGISTERED, "weight %p is not registered", w);
  if (it->qt != qt)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "weight %p registered as quant %u, called with %u", w, it->qt, qt);
  if (off != 0 && it->il != 1)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "interior pointer into an interleaved tensor");
  if (off + need > it->bytes)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "weight %p: %zu bytes needed, %zu registered", w, need, it->bytes - off);
  *dev = static_cast<const uint8_t*>(it->dev) + off;
  *il = off ? 1u : it->il;
  if (hold) *hold = it->hold;
  return ZG_OK;
}

// ---------------------------------------------------------------------------
// Dispatch core (device pointers)
// ---------------------------------------------------------------------------

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// X4 (interleave 4) or split-scale X4 (interleave 5: strip-sized in_dim
// only) Q4_0 / Q8_0 groups through the X4 dispatch
bool zg::pair_path_ok(uint32_t qt, uint32_t il, size_t k, size_t n, const void* w, const void* x) {
  if ((qt != ZG_Q4_0 && qt != ZG_Q8_0) || n % 4 || !aligned16(w) || !aligned16(x)) return false;
  if (il == 5) return strip_path_ok((int)k);  // strip-kernel launches only
  return il == 4 && k % 64 == 0 && k <= kMaxPairK && gemv_x4_lds_bytes(qt, (int)k) <= 65536;
}

zg_status zg::check_shape(zg_ctx* ctx, uint32_t qt, uint32_t il, size_t k, size_t n) {
  size_t be, bb;
  if (!type_geom(qt, &be, &bb)) return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "unsupported quant type %u", qt);
  if (k == 0 || k % be) return set_error(ctx, ZG_ERR_INVALID_ARG, "in_dim %zu not a multiple of %zu", k, be);
  if (il != 1 && il != 4 && il != 5) return set_error(ctx, ZG_ERR_INVALID_ARG, "interleave %u", il);
  if ((il == 4 || il == 5) && ((qt != ZG_Q4_0 && qt != ZG_Q8_0) || n % 4))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "interleave %u needs Q4_0/Q8_0 and out_dim %% 4 == 0", il);
  if (il == 5 && !strip_path_ok((int)k))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "interleave 5 needs in_dim a multiple of 512 up to 8192");
  if (k > (size_t)INT32_MAX || n > (size_t)UINT32_MAX / 2) return set_error(ctx, ZG_ERR_INVALID_ARG, "shape too large");
  return ZG_OK;
}

// One GEMV (optionally a row range, residual or argmax epilogue).
zg_status zg::run_linear(zg_ctx* ctx, const float* x, const uint8_t* w, float* y, size_t k, size_t n, uint32_t qt,
                         uint32_t il, size_t start, size_t end, int epi, const float* resid, uint64_t* best,
                         int pro, const float* norm_w, float eps, hipStream_t st, uint32_t gemv_flags) {
  if (start >= end) return ZG_OK;
  if (pair_path_ok(qt, il, k, n, w, x)) {
    const size_t gbytes = (k / 32) * (qt == ZG_Q4_0 ? 72 : 136);
    const size_t g0 = start / 4, g1 = (end + 3) / 4;
    GemvArgs a{};
    a.nseg = 1;
    a.k = (int)k;
    a.total_groups = (uint32_t)(g1 - g0);
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.best = best;
    a.flags = gemv_flags | (il == 5 ? kGemvSplit : 0u);
    a.seg[0].w = w + g0 * gbytes;
    a.seg[0].y = y ? y + 4 * g0 : nullptr;
    a.seg[0].resid = resid ? resid + 4 * g0 : nullptr;
    a.seg[0].g_begin = 0;
    a.seg[0].row_lo = (uint32_t)(start - 4 * g0);
    a.seg[0].row_hi = (uint32_t)(end - 4 * g0);
    return hip_check(ctx, launch_gemv_x4(a, qt, pro, epi, st), "gemv_x4 launch");
  }
  if (il == 5) return set_error(ctx, ZG_ERR_INVALID_ARG, "split-scale X4 weights need 16-byte aligned w and x");
  if (plain_strip_ok(qt, il, k, n, w, x) && (pro == PRO_PLAIN || pro == PRO_RMSNORM) &&
      (epi == EPI_STORE || epi == EPI_RESID || epi == EPI_ARGMAX) && !(pro == PRO_RMSNORM && epi == EPI_RESID)) {
    // plain rows in fours: group g is rows 4g..4g+3
    const size_t rbytes = (k / 32) * (qt == ZG_Q4_0 ? 18 : 34);
    const size_t g0 = start / 4, g1 = (end + 3) / 4;
    GemvArgs a{};
    a.nseg = 1;
    a.k = (int)k;
    a.total_groups = (uint32_t)(g1 - g0);
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.best = best;
    a.flags = gemv_flags;
    a.seg[0].w = w + 4 * g0 * rbytes;
    a.seg[0].y = y ? y + 4 * g0 : nullptr;
    a.seg[0].resid = resid ? resid + 4 * g0 : nullptr;
    a.seg[0].g_begin = 0;
    a.seg[0].row_lo = (uint32_t)(start - 4 * g0);
    a.seg[0].row_hi = (uint32_t)(end - 4 * g0);
    return hip_check(ctx, launch_gemv_plain(a, qt, pro, epi, st), "gemv plain launch");
  }
  if (pro == PRO_PLAIN && (epi == EPI_STORE || epi == EPI_RESID) && kq_strip_ok(qt, il, k, n, w, x)) {
    // Q4_K rows in fours through the strip kernel
    const size_t rbytes = (k / 256) * 144;
    const size_t g0 = start / 4, g1 = (end + 3) / 4;
    GemvArgs a{};
    a.nseg = 1;
    a.k = (int)k;
    a.total_groups = (uint32_t)(g1 - g0);
    a.x = x;
    a.flags = gemv_flags;
    a.seg[0].w = w + 4 * g0 * rbytes;
    a.seg[0].y = y ? y + 4 * g0 : nullptr;
    a.seg[0].resid = resid ? resid + 4 * g0 : nullptr;
    a.seg[0].g_begin = 0;
    a.seg[0].row_lo = (uint32_t)(start - 4 * g0);
    a.seg[0].row_hi = (uint32_t)(end - 4 * g0);
    return hip_check(ctx, launch_gemv_plain(a, qt, pro, epi, st), "gemv Q4_K strip launch");
  }
  if (pro == PRO_RMSNORM && (epi == EPI_STORE || epi == EPI_RESID || epi == EPI_ARGMAX) && aligned16(norm_w) &&
      kq_fused_ok(qt, il, k, w, x)) {
    // Q4_K strip kernel with the rmsnorm prologue
    GenericArgs g{};
    g.w = w;
    g.x = x;
    g.y = y;
    g.resid = resid;
    g.best = best;
    g.k = k;
    g.row_lo = start;
    g.row_hi = end;
    g.qt = qt;
    g.il = (int)il;
    g.epi = epi;
    g.norm_w = norm_w;
    g.eps = eps;
    return hip_check(ctx, launch_kq_fused(g, true, st), "gemv_kq rmsnorm launch");
  }
  const float* xin = x;
  if (pro == PRO_RMSNORM) {
    // generic path: normalize into the context's aux buffer first
    zg_status s = ensure_buf(ctx, ctx->d_aux, k * sizeof(float));
    if (s) return s;
    hipError_t e = launch_rmsnorm(x, norm_w, static_cast<float*>(ctx->d_aux.ptr), (int)k, eps, st);
    if (e != hipSuccess) return hip_check(ctx, e, "rmsnorm launch");
    xin = static_cast<float*>(ctx->d_aux.ptr);
  }
  GenericArgs g{};
  g.w = w;
  g.x = xin;
  g.y = y;
  g.resid = resid;
  g.best = best;
  g.k = k;
  g.row_lo = start;
  g.row_hi = end;
  g.qt = qt;
  g.il = (int)il;
  g.epi = epi;
  if (kq_path_ok(qt, il, k, w, xin)) return hip_check(ctx, launch_gemv_kq(g, st), "gemv_kq launch");
  return hip_check(ctx, launch_gemv_generic(g, st), "gemv_generic launch");
}

// run_fused's one-launch forms: X4 segments through the X4 kernels, plain
// row-major Q4_0 / Q8_0 segments through the strip kernel (no prologue),
// Q4_K rows through the strip kernel (rmsnorm or no prologue)
bool zg::fused_x4_ok(const float* x, const FusedDev* segs, size_t nseg, size_t k) {
  bool ok = nseg >= 1 && nseg <= 3;
  for (size_t i = 0; i < nseg && ok; i++)
    ok = pair_path_ok(segs[i].qt, segs[i].il, k, segs[i].n, segs[i].w, x) && segs[i].qt == segs[0].qt &&
         segs[i].il == segs[0].il;
  return ok;
}

bool zg::fused_plain_ok(const float* x, const FusedDev* segs, size_t nseg, size_t k, int pro) {
  bool ok = nseg >= 1 && nseg <= 3 && (pro == PRO_PLAIN || pro == PRO_RMSNORM);
  for (size_t i = 0; i < nseg && ok; i++)
    ok = ((pro == PRO_PLAIN && plain_strip_ok(segs[i].qt, segs[i].il, k, segs[i].n, segs[i].w, x)) ||
          kq_strip_ok(segs[i].qt, segs[i].il, k, segs[i].n, segs[i].w, x)) &&
         segs[i].qt == segs[0].qt;
  return ok;
}

// Whether run_linear takes a rmsnorm prologue inside the GEMV kernel (else
// it normalizes into the context's aux buffer first).
bool zg::rmsnorm_fused_ok(uint32_t qt, uint32_t il, size_t k, size_t n, const void* w, const void* x, int epi) {
  if (pair_path_ok(qt, il, k, n, w, x)) return true;
  if (kq_fused_ok(qt, il, k, w, x)) return epi == EPI_STORE || epi == EPI_RESID || epi == EPI_ARGMAX;
  return plain_strip_ok(qt, il, k, n, w, x) && epi == EPI_ARGMAX;
}

// Q4_K gate|up in one launch: y[r] = silu(gate_r . x') * (up_r . x'), x' the
// rmsnorm of x (norm_w non-null) or x itself.
bool zg::kq_swiglu_ok(uint32_t qt_gate, uint32_t qt_up, uint32_t il_gate, uint32_t il_up, size_t k, const void* gate,
                      const void* up, const void* x, const float* norm_w) {
  return qt_gate == ZG_Q4K && qt_up == ZG_Q4K && kq_fused_ok(qt_gate, il_gate, k, gate, x) &&
         kq_fused_ok(qt_up, il_up, k, up, x) && (!norm_w || aligned16(norm_w));
}

zg_status zg::run_kq_swiglu(zg_ctx* ctx, const float* x, const uint8_t* gate, const uint8_t* up, float* y, size_t k,
                            size_t n, const float* norm_w, float eps, hipStream_t st) {
  GenericArgs g{};
  g.w = gate;
  g.w_up = up;
  g.x = x;
  g.y = y;
  g.k = k;
  g.row_lo = 0;
  g.row_hi = n;
  g.qt = ZG_Q4K;
  g.il = 1;
  g.epi = EPI_SWIGLU;
  g.norm_w = norm_w;
  g.eps = eps;
  return hip_check(ctx, launch_kq_fused(g, norm_w != nullptr, st), "gemv_kq swiglu launch");
}

// Q4_K segments through the segmented K-quant strip form (EPI_STORE).
bool zg::fused_kq_ok(const float* x, const FusedDev* segs, size_t nseg, size_t k, int pro, const float* norm_w) {
  bool ok = nseg >= 1 && nseg <= 3 && (pro == PRO_PLAIN || (pro == PRO_RMSNORM && aligned16(norm_w)));
  for (size_t i = 0; i < nseg && ok; i++) ok = segs[i].qt == ZG_Q4K && kq_fused_ok(segs[i].qt, segs[i].il, k, segs[i].w, x);
  return ok;
}

// xn_out (rmsnorm prologue only): also store the normalized x there.
zg_status zg::run_kq_segs(zg_ctx* ctx, const float* x, const FusedDev* segs, size_t nseg, size_t k, int pro,
                          const float* norm_w, float eps, hipStream_t st, float* xn_out) {
  bool strip = (pro == PRO_PLAIN || (pro == PRO_RMSNORM && aligned16(norm_w) && (!xn_out || aligned16(xn_out))));
  for (size_t i = 0; i < nseg && strip; i++) strip = kq_strip_ok(segs[i].qt, segs[i].il, k, segs[i].n, segs[i].w, x);
  if (strip) {
    // Q4_K segments through the strip kernel (rows in fours per segment)
    GemvArgs a{};
    a.nseg = (int)nseg;
    a.k = (int)k;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.xn_out = pro == PRO_RMSNORM ? xn_out : nullptr;
    uint32_t gb = 0;
    for (size_t i = 0; i < nseg; i++) {
      a.seg[i].w = segs[i].w;
      a.seg[i].y = segs[i].y;
      a.seg[i].resid = nullptr;
      a.seg[i].g_begin = gb;
      a.seg[i].row_lo = 0;
      a.seg[i].row_hi = (uint32_t)segs[i].n;
      gb += (uint32_t)(segs[i].n / 4);
    }
    a.total_groups = gb;
    return hip_check(ctx, launch_gemv_plain(a, ZG_Q4K, pro, EPI_STORE, st), "gemv Q4_K strip segmented launch");
  }
  GenericArgs g{};
  g.xn_out = pro == PRO_RMSNORM ? xn_out : nullptr;
  g.x = x;
  g.k = k;
  g.qt = ZG_Q4K;
  g.il = 1;
  g.epi = EPI_STORE;
  g.norm_w = pro == PRO_RMSNORM ? norm_w : nullptr;
  g.eps = eps;
  g.nseg = (int)nseg;
  uint32_t end = 0;
  for (size_t i = 0; i < 3; i++) {
    const size_t j = i < nseg ? i : nseg - 1;
    if (i < nseg) end += (uint32_t)segs[i].n;
    g.seg_w[i] = segs[j].w;
    g.seg_y[i] = segs[j].y;
    g.seg_end[i] = end;
  }
  g.w = segs[0].w;
  g.y = segs[0].y;
  g.row_lo = 0;
  g.row_hi = end;
  return hip_check(ctx, launch_kq_fused(g, pro == PRO_RMSNORM, st), "gemv_kq segmented launch");
}

// Fused same-x dispatch: one launch over the concatenated group space when
// every segment qualifies, else one launch per segment (a leading run of
// two or more Q4_K segments still shares one launch).
zg_status zg::run_fused(zg_ctx* ctx, const float* x, const FusedDev* segs, size_t nseg, size_t k, int pro,
                        const float* norm_w, float eps, int epi, hipStream_t st) {
  const bool pair = fused_x4_ok(x, segs, nseg, k);
  const bool plain = !pair && fused_plain_ok(x, segs, nseg, k, pro);
  if (epi == EPI_SWIGLU && !((pair || plain) && nseg == 2 && segs[0].n == segs[1].n))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "swiglu fusion needs two equal Q4_0/Q8_0 segments on a one-launch path");
  if (pair || plain) {
    GemvArgs a{};
    a.nseg = (int)nseg;
    a.k = (int)k;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    uint32_t g = 0;
    for (size_t i = 0; i < nseg; i++) {
      a.seg[i].w = segs[i].w;
      a.seg[i].y = segs[i].y;
      a.seg[i].resid = nullptr;
      a.seg[i].g_begin = g;
      a.seg[i].row_lo = 0;
      a.seg[i].row_hi = (uint32_t)segs[i].n;
      g += (uint32_t)(segs[i].n / 4);
    }
    a.total_groups = g;
    if (pair && segs[0].il == 5) a.flags |= kGemvSplit;
    return hip_check(ctx, pair ? launch_gemv_x4(a, segs[0].qt, pro, epi, st) : launch_gemv_plain(a, segs[0].qt, pro, epi, st),
                     "fused gemv launch");
  }
  size_t first = 0;
  if (epi == EPI_STORE) {
    size_t run = 0;
    while (run < nseg && fused_kq_ok(x, segs, run + 1, k, pro, norm_w)) run++;
    if (run == nseg || run >= 2) {
      zg_status s = run_kq_segs(ctx, x, segs, run, k, pro, norm_w, eps, st);
      if (s) return s;
      first = run;
    }
  }
  for (size_t i = first; i < nseg; i++) {
    // (split-scale segments that do not share a launch go one by one)
    zg_status s = run_linear(ctx, x, segs[i].w, segs[i].y, k, segs[i].n, segs[i].qt, segs[i].il, 0, segs[i].n,
                             EPI_STORE, nullptr, nullptr, pro, norm_w, eps, st);
    if (s) return s;
  }
  return ZG_OK;
}

// O projection of the decode step: y += W * merge(attention splits), the
// split merge in the strip kernel's prologue.
zg_status zg::run_attn_o(zg_ctx* ctx, const float* part_o, const float* part_ml, int nsplit, int hd,
                         const uint8_t* w, float* y, size_t k, size_t n, uint32_t qt, uint32_t il, hipStream_t st) {
  if (kq_strip_ok(qt, il, k, n, w, part_o) && attn_merge_strip_ok(nsplit, hd, k)) {
    // Q4_K rows in fours through the strip kernel, the merge in its prologue
    GemvArgs a{};
    a.nseg = 1;
    a.k = (int)k;
    a.total_groups = (uint32_t)(n / 4);
    a.x = part_o;
    a.attn_ml = part_ml;
    a.attn_nsplit = nsplit;
    a.attn_hd = hd;
    a.seg[0].w = w;
    a.seg[0].y = y;
    a.seg[0].resid = y;
    a.seg[0].g_begin = 0;
    a.seg[0].row_lo = 0;
    a.seg[0].row_hi = (uint32_t)n;
    return hip_check(ctx, launch_gemv_plain(a, qt, PRO_ATTN, EPI_RESID, st), "attention-merge gemv Q4_K strip launch");
  }
  if (qt == ZG_Q4K) {
    if (!kq_attn_o_ok(qt, il, k, nsplit, hd, w, part_o))
      return set_error(ctx, ZG_ERR_INVALID_ARG, "attention-merge Q4_K GEMV: in_dim %zu not supported", k);
    GenericArgs g{};
    g.w = w;
    g.x = part_o;
    g.y = y;
    g.resid = y;
    g.k = k;
    g.row_lo = 0;
    g.row_hi = n;
    g.qt = qt;
    g.il = (int)il;
    g.epi = EPI_RESID;
    g.attn_ml = part_ml;
    g.attn_nsplit = nsplit;
    g.attn_hd = hd;
    return hip_check(ctx, launch_kq_attn_o(g, st), "attention-merge gemv_kq launch");
  }
  if (!attn_merge_gemv_ok(qt, il, k) || !pair_path_ok(qt, il, k, n, w, part_o))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "attention-merge GEMV needs Q4_0X4 weights and a strip-sized in_dim");
  if (!attn_merge_hd_ok(qt, hd) || k % (size_t)hd != 0)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "attention-merge GEMV needs a head dim in whole 32-element blocks");
  GemvArgs a{};
  a.nseg = 1;
  a.k = (int)k;
  a.total_groups = (uint32_t)(n / 4);
  a.x = part_o;
  a.attn_ml = part_ml;
  a.attn_nsplit = nsplit;
  a.attn_hd = hd;
  a.flags = il == 5 ? kGemvSplit : 0u;
  a.seg[0].w = w;
  a.seg[0].y = y;
  a.seg[0].resid = y;
  a.seg[0].g_begin = 0;
  a.seg[0].row_lo = 0;
  a.seg[0].row_hi = (uint32_t)n;
  return hip_check(ctx, launch_gemv_x4(a, qt, PRO_ATTN, EPI_RESID, st), "attention-merge gemv launch");
}

// ---------------------------------------------------------------------------
// Host-pointer operator API
// ---------------------------------------------------------------------------

zg_status zg::stage_in(zg_ctx* ctx, const void* src, size_t bytes, DevBuf& dst) {
  zg_status s = ensure_buf(ctx, dst, bytes);
  if (s) return s;
  return hip_check(ctx, hipMemcpyAsync(dst.ptr, src, bytes, hipMemcpyHostToDevice, ctx->stream), "upload");
}

extern "C" zg_status zg_linear_range(zg_ctx* ctx, const float* x, const void* w, float* out, size_t in_dim,
                                     size_t out_dim, uint32_t ggml_type, size_t start, size_t end) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!x || !w || !out) return set_error(ctx, ZG_ERR_INVALID_ARG, "linear: null pointer");
  if (start > end || end > out_dim) return set_error(ctx, ZG_ERR_INVALID_ARG, "linear: bad range [%zu,%zu)", start, end);
  hipSetDevice(ctx->device);
  size_t be, bb;
  if (!type_geom(ggml_type, &be, &bb))
    return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "linear_dispatch: unsupported quant type %u", ggml_type);
  const uint8_t* dw;
  uint32_t il;
  zg_status s = resolve(ctx, w, tensor_bytes(ggml_type, out_dim, in_dim), ggml_type, &dw, &il);
  if (s) return s;
  if ((s = check_shape(ctx, ggml_type, il, in_dim, out_dim))) return s;
  if ((s = stage_in(ctx, x, in_dim * sizeof(float), ctx->d_x))) return s;
  if ((s = ensure_buf(ctx, ctx->d_out, out_dim * sizeof(float)))) return s;
  float* dout = static_cast<float*>(ctx->d_out.ptr);
  s = run_linear(ctx, static_cast<const float*>(ctx->d_x.ptr), dw, dout, in_dim, out_dim, ggml_type, il, start, end,
                 EPI_STORE, nullptr, nullptr, PRO_PLAIN, nullptr, 0.0f, ctx->stream);
  if (s) return s;
  if (end > start) {
    s = hip_check(ctx, hipMemcpyAsync(out + start, dout + start, (end - start) * sizeof(float), hipMemcpyDeviceToHost,
                                      ctx->stream), "download");
    if (s) return s;
  }
  return hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync");
}

extern "C" zg_status zg_linear(zg_ctx* ctx, const float* x, const void* w, float* out, size_t in_dim, size_t out_dim,
                               uint32_t ggml_type) {
  return zg_linear_range(ctx, x, w, out, in_dim, out_dim, ggml_type, 0, out_dim);
}

extern "C" zg_status zg_linear_fused(zg_ctx* ctx, const float* x, const zg_segment* segs, size_t n_segs,
                                     size_t in_dim) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!x || !segs || n_segs == 0 || n_segs > 3) return set_error(ctx, ZG_ERR_INVALID_ARG, "fused: bad segments");
  hipSetDevice(ctx->device);
  FusedDev fd[3];
  size_t total = 0;
  for (size_t i = 0; i < n_segs; i++) {
    if (!segs[i].w || !segs[i].out) return set_error(ctx, ZG_ERR_INVALID_ARG, "fused: null segment pointer");
    size_t be, bb;
    if (!type_geom(segs[i].ggml_type, &be, &bb))
      return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "fused: unsupported quant type %u", segs[i].ggml_type);
    zg_status s = resolve(ctx, segs[i].w, tensor_bytes(segs[i].ggml_type, segs[i].out_dim, in_dim), segs[i].ggml_type,
                          &fd[i].w, &fd[i].il);
    if (s) return s;
    if ((s = check_shape(ctx, segs[i].ggml_type, fd[i].il, in_dim, segs[i].out_dim))) return s;
    fd[i].qt = segs[i].ggml_type;
    fd[i].n = segs[i].out_dim;
    total += segs[i].out_dim;
  }
  zg_status s = stage_in(ctx, x, in_dim * sizeof(float), ctx->d_x);
  if (s) return s;
  if ((s = ensure_buf(ctx, ctx->d_out, total * sizeof(float)))) return s;
  float* dout = static_cast<float*>(ctx->d_out.ptr);
  size_t off = 0;
  for (size_t i = 0; i < n_segs; i++) {
    fd[i].y = dout + off;
    off += fd[i].n;
  }
  s = run_fused(ctx, static_cast<const float*>(ctx->d_x.ptr), fd, n_segs, in_dim, PRO_PLAIN, nullptr, 0.0f, EPI_STORE,
                ctx->stream);
  if (s) return s;
  off = 0;
  for (size_t i = 0; i < n_segs; i++) {
    s = hip_check(ctx, hipMemcpyAsync(segs[i].out, dout + off, fd[i].n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
                  "download");
    if (s) return s;
    off += fd[i].n;
  }
  return hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync");
}

extern "C" int zg_argmax_unpack(uint64_t packed, uint32_t* index, float* value) {
  if (packed == 0) {
    if (index) *index = 0;
    if (value) *value = -INFINITY;
    return 0;
  }
  const uint32_t k = (uint32_t)(packed >> 32);
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  float v;
  memcpy(&v, &b, 4);
  if (index) *index = 0xFFFFFFFFu - (uint32_t)(packed & 0xFFFFFFFFu);
  if (value) *value = v;
  return 1;
}

zg_status zg::lm_head_status(zg_ctx* ctx, uint64_t packed, size_t vocab_real, uint32_t* token, float* max_val) {
  uint32_t idx;
  float v;
  const int have = zg_argmax_unpack(packed, &idx, &v);
  if (token) *token = idx;
  if (max_val) *max_val = v;
  if (!have || !std::isfinite(v)) return set_error(ctx, ZG_ERR_NONFINITE_LOGITS, "LM head: non-finite logits");
  if (idx >= vocab_real) return set_error(ctx, ZG_ERR_ARGMAX_IN_PADDING, "LM head: argmax %u in padding region", idx);
  return ZG_OK;
}

extern "C" zg_status zg_lm_head_argmax(zg_ctx* ctx, const float* hidden, const float* norm_w, const void* w,
                                       uint32_t ggml_type, float eps, size_t dim, size_t vocab_padded,
                                       size_t vocab_real, float* logits, uint32_t* token, float* max_val) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!hidden || !norm_w || !w) return set_error(ctx, ZG_ERR_INVALID_ARG, "lm_head: null pointer");
  if (vocab_real > vocab_padded) return set_error(ctx, ZG_ERR_INVALID_ARG, "lm_head: vocab_real > vocab_padded");
  hipSetDevice(ctx->device);
  size_t be, bb;
  if (!type_geom(ggml_type, &be, &bb))
    return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "lm_head: unsupported quant type %u", ggml_type);
  const uint8_t* dw;
  uint32_t il;
  zg_status s = resolve(ctx, w, tensor_bytes(ggml_type, vocab_padded, dim), ggml_type, &dw, &il);
  if (s) return s;
  if ((s = check_shape(ctx, ggml_type, il, dim, vocab_padded))) return s;
  // d_x holds [hidden | norm_w]
  if ((s = ensure_buf(ctx, ctx->d_x, 2 * dim * sizeof(float) + 64))) return s;
  float* dx = static_cast<float*>(ctx->d_x.ptr);
  float* dn = dx + ((dim + 15) & ~size_t(15));
  if ((s = hip_check(ctx, hipMemcpyAsync(dx, hidden, dim * 4, hipMemcpyHostToDevice, ctx->stream), "upload"))) return s;
  if ((s = hip_check(ctx, hipMemcpyAsync(dn, norm_w, dim * 4, hipMemcpyHostToDevice, ctx->stream), "upload"))) return s;
  if ((s = ensure_buf(ctx, ctx->d_out, vocab_padded * sizeof(float)))) return s;
  float* dl = static_cast<float*>(ctx->d_out.ptr);
  if ((s = hip_check(ctx, launch_fill_u64(ctx->d_best, 0, ctx->stream), "reset"))) return s;
  s = run_linear(ctx, dx, dw, dl, dim, vocab_padded, ggml_type, il, 0, vocab_padded, EPI_ARGMAX, nullptr, ctx->d_best,
                 PRO_RMSNORM, dn, eps, ctx->stream);
  if (s) return s;
  uint64_t packed = 0;
  if ((s = hip_check(ctx, hipMemcpyAsync(&packed, ctx->d_best, 8, hipMemcpyDeviceToHost, ctx->stream), "download")))
    return s;
  if (logits &&
      (s = hip_check(ctx, hipMemcpyAsync(logits, dl, vocab_padded * 4, hipMemcpyDeviceToHost, ctx->stream), "download")))
    return s;
  if ((s = hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync"))) return s;
  return lm_head_status(ctx, packed, vocab_real, token, max_val);
}

// ---------------------------------------------------------------------------
// Device-pointer API
// ---------------------------------------------------------------------------

extern "C" zg_status zg_linear_dev(zg_ctx* ctx, const float* d_x, const void* d_w, float* d_out, size_t in_dim,
                                   size_t out_dim, uint32_t ggml_type, uint32_t interleave, size_t start, size_t end,
                                   void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_x || !d_w || !d_out) return set_error(ctx, ZG_ERR_INVALID_ARG, "linear_dev: null pointer");
  if (start > end || end > out_dim) return set_error(ctx, ZG_ERR_INVALID_ARG, "linear_dev: bad range");
  zg_status s = check_shape(ctx, ggml_type, interleave, in_dim, out_dim);
  if (s) return s;
  return run_linear(ctx, d_x, static_cast<const uint8_t*>(d_w), d_out, in_dim, out_dim, ggml_type, interleave, start,
                    end, EPI_STORE, nullptr, nullptr, PRO_PLAIN, nullptr, 0.0f, pick_stream(ctx, stream));
}

extern "C" zg_status zg_linear_q8act_dev(zg_ctx* ctx, const void* d_xq, const void* d_w, float* d_out, size_t in_dim,
                                         size_t out_dim, uint32_t ggml_type, uint32_t interleave, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_xq || !d_w || !d_out) return set_error(ctx, ZG_ERR_INVALID_ARG, "linear_q8act: null pointer");
  if (ggml_type != ZG_Q4_0 && ggml_type != ZG_Q8_0)
    return set_error(ctx, ZG_ERR_UNSUPPORTED_QUANT, "linear_q8act: weights must be Q4_0/Q8_0");
  zg_status s = check_shape(ctx, ggml_type, interleave, in_dim, out_dim);
  if (s) return s;
  if (!strip_path_ok((int)in_dim) || out_dim % 4)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "linear_q8act: in_dim %zu (multiple of 512 up to 8192) / out_dim %zu (%% 4)",
                     in_dim, out_dim);
  const uintptr_t wa = reinterpret_cast<uintptr_t>(d_w);
  if ((reinterpret_cast<uintptr_t>(d_xq) & 1) || (interleave == 4 ? (wa & 7) : interleave == 5 ? (wa & 15) : (wa & 1)))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "linear_q8act: misaligned buffer");
  if (out_dim == 0) return ZG_OK;
  GemvArgs a{};
  a.nseg = 1;
  a.k = (int)in_dim;
  a.total_groups = (uint32_t)(out_dim / 4);
  a.xq = static_cast<const uint8_t*>(d_xq);
  a.seg[0].w = static_cast<const uint8_t*>(d_w);
  a.seg[0].y = d_out;
  a.seg[0].g_begin = 0;
  a.seg[0].row_lo = 0;
  a.seg[0].row_hi = (uint32_t)out_dim;
  a.flags = interleave == 5 ? kGemvSplit : 0u;
  hipStream_t st = pick_stream(ctx, stream);
  const hipError_t e = interleave != 1 ? launch_gemv_x4(a, ggml_type, PRO_Q8X, EPI_STORE, st)
                                       : launch_gemv_plain(a, ggml_type, PRO_Q8X, EPI_STORE, st);
  return hip_check(ctx, e, "linear_q8act launch");
}

extern "C" zg_status zg_linear_fused_dev(zg_ctx* ctx, const float* d_x, const zg_segment* segs, size_t n_segs,
                                         size_t in_dim, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_x || !segs || n_segs == 0 || n_segs > 3) return set_error(ctx, ZG_ERR_INVALID_ARG, "fused_dev: bad segments");
  FusedDev fd[3];
  for (size_t i = 0; i < n_segs; i++) {
    if (!segs[i].w || !segs[i].out) return set_error(ctx, ZG_ERR_INVALID_ARG, "fused_dev: null pointer");
    zg_status s = check_shape(ctx, segs[i].ggml_type, segs[i].interleave, in_dim, segs[i].out_dim);
    if (s) return s;
    fd[i].w = static_cast<const uint8_t*>(segs[i].w);
    fd[i].y = segs[i].out;
    fd[i].n = segs[i].out_dim;
    fd[i].qt = segs[i].ggml_type;
    fd[i].il = segs[i].interleave;
  }
  return run_fused(ctx, d_x, fd, n_segs, in_dim, PRO_PLAIN, nullptr, 0.0f, EPI_STORE, pick_stream(ctx, stream));
}

extern "C" zg_status zg_lm_head_dev(zg_ctx* ctx, const float* d_x, const void* d_w, float* d_logits, size_t in_dim,
                                    size_t out_dim, uint32_t ggml_type, uint32_t interleave, uint64_t* d_best,
                                    void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_x || !d_w || !d_best) return set_error(ctx, ZG_ERR_INVALID_ARG, "lm_head_dev: null pointer");
  zg_status s = check_shape(ctx, ggml_type, interleave, in_dim, out_dim);
  if (s) return s;
  hipStream_t st = pick_stream(ctx, stream);
  if ((s = hip_check(ctx, launch_fill_u64(d_best, 0, st), "reset"))) return s;
  return run_linear(ctx, d_x, static_cast<const uint8_t*>(d_w), d_logits, in_dim, out_dim, ggml_type, interleave, 0,
                    out_dim, EPI_ARGMAX, nullptr, d_best, PRO_PLAIN, nullptr, 0.0f, st);
}

extern "C" zg_status zg_dequant_dev(zg_ctx* ctx, const void* d_w, float* d_out, size_t rows, size_t in_dim,
                                    uint32_t ggml_type, uint32_t interleave, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_w || !d_out) return set_error(ctx, ZG_ERR_INVALID_ARG, "dequant_dev: null pointer");
  zg_status s = check_shape(ctx, ggml_type, interleave, in_dim, rows);
  if (!s && interleave == 5) s = set_error(ctx, ZG_ERR_INVALID_ARG, "dequant: interleave 5 is a GEMV layout only");
  if (s) return s;
  DequantArgs a{static_cast<const uint8_t*>(d_w), d_out, rows, in_dim, ggml_type, (int)interleave};
  const bool pair = pair_path_ok(ggml_type, interleave, in_dim, rows, d_w, d_out);
  return hip_check(ctx, launch_dequant(a, pair, pick_stream(ctx, stream)), "dequant launch");
}

extern "C" zg_status zg_fp16_to_f32_dev(zg_ctx* ctx, const uint16_t* d_in, float* d_out, size_t n, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_in || !d_out) return set_error(ctx, ZG_ERR_INVALID_ARG, "fp16_dev: null pointer");
  return hip_check(ctx, launch_fp16(d_in, d_out, n, pick_stream(ctx, stream)), "fp16 launch");
}

extern "C" zg_status zg_read_floor_dev(zg_ctx* ctx, const void* d_src, size_t bytes, uint32_t loads_per_thread,
                                       uint32_t* d_sink, void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_src || !d_sink) return set_error(ctx, ZG_ERR_INVALID_ARG, "read_floor: null pointer");
  if (bytes % 16 || (reinterpret_cast<uintptr_t>(d_src) & 15))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "read_floor: bytes and source must be 16-byte multiples");
  if (loads_per_thread != 1 && loads_per_thread != 2 && loads_per_thread != 4 && loads_per_thread != 8)
    return set_error(ctx, ZG_ERR_INVALID_ARG, "read_floor: loads_per_thread %u not in {1,2,4,8}", loads_per_thread);
  return hip_check(ctx, launch_read_floor(d_src, bytes, (int)loads_per_thread, d_sink, pick_stream(ctx, stream)),
                   "read_floor launch");
}

extern "C" zg_status zg_strip_loads_dev(zg_ctx* ctx, const void* d_w, size_t rows, const float* d_x, uint32_t* d_sink,
                                        void* stream) {
  if (!ctx) return ZG_ERR_INVALID_ARG;
  if (!d_w || !d_sink) return set_error(ctx, ZG_ERR_INVALID_ARG, "strip_loads: null pointer");
  if (rows % 4 || rows / 4 > (size_t)INT32_MAX || (reinterpret_cast<uintptr_t>(d_w) & 15) ||
      (d_x && (reinterpret_cast<uintptr_t>(d_x) & 15)))
    return set_error(ctx, ZG_ERR_INVALID_ARG, "strip_loads: rows %% 4 != 0 or misaligned buffer");
  return hip_check(ctx, launch_strip_loads(static_cast<const uint8_t*>(d_w), d_x, rows, d_sink, pick_stream(ctx, stream)),
                   "strip_loads launch");
}
