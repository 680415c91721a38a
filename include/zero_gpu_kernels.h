/*
 * zero_gpu_kernels.h -- the code-object route to the decode GEMV.
 *
 * For a host that loads kernels itself (hipModuleLoad, hipModuleGetFunction,
 * hipModuleLaunchKernel, and stream capture of those launches into a
 * hipGraph for the per-token sequence) instead of calling the C ABI of
 * zero_gpu.h.  zero_amd/zg_kernels.hsaco is an unbundled gfx950 code object
 * (built by zero_amd/build.py from zero_amd/csrc/module/zg_module.hip); its
 * entry points are the library's strip GEMV for X4 weights, y = W x, and
 * replace the reference's row-range kernels
 *   Q4_0X4  linear_q4_0x4_avx512_range (kernel/src/arch/x86_64/math/linear.rs:909-1072)
 *   Q8_0X4  linear_q8_0x4_avx512_range (kernel/src/arch/x86_64/math/linear.rs:1096-1213)
 * as linear_dispatch reaches them (crates/zero-llm-inference/src/ops.rs:486-523),
 * over all rows at once instead of the SMP row split.
 *
 * Every entry takes the same arguments (zg_mk_gemv_args, in kernel-argument
 * order): W as X4 group-blocks (rows a multiple of 4, 8-byte aligned), x
 * (k floats, 16-byte aligned), y (rows floats); k a multiple of 512 up to
 * 8192.  The launch geometry comes from zg_mk_plan below, the rule the
 * library applies to the same shape, so an entry launched as planned gives
 * the library's bits.  The module carries the strip kernel's forms only:
 * where the library takes another kernel for a shape (its LDS-staged tall
 * launch at in_dim 2048: Q8_0X4, and Q4_0X4 of at least 24,576 groups; its
 * segment kernel for mid-sized Q8_0X4 at in_dim above 2048) the planned
 * strip form gives results within the same tolerance, not the same bits.
 *
 * Pure host code: nothing here calls HIP.
 */
#ifndef ZERO_GPU_KERNELS_H
#define ZERO_GPU_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZG_MK_CODE_OBJECT "zg_kernels.hsaco"

/* Kernel arguments of every zg_mk_* entry, in order (32 bytes as a packed
 * kernel-argument buffer, or one kernelParams pointer per field). */
typedef struct zg_mk_gemv_args {
  const void* w;  /* X4 group-blocks, rows/4 groups of k/32 blocks        */
  const float* x; /* k activations                                         */
  float* y;       /* rows outputs                                          */
  uint32_t rows;
  uint32_t k;
} zg_mk_gemv_args;

/* One launch: grid.x = min(nbatch, cu_count * per_cu), where per_cu is
 * per_cu_cap, further capped by the entry's resident workgroups per CU at
 * (block, shm_bytes) when occupancy_bound (hipModuleOccupancyMaxActive-
 * BlocksPerMultiprocessor); one_batch plans launch exactly nbatch. */
typedef struct zg_mk_launch {
  char entry[40];     /* kernel name in the code object                  */
  uint32_t block;     /* block.x (64 per wave)                            */
  uint32_t shm_bytes; /* dynamic LDS                                      */
  uint32_t nbatch;    /* batches of groups                               */
  uint32_t per_cu_cap;
  int one_batch;      /* grid.x = nbatch                                  */
  int occupancy_bound;
} zg_mk_launch;

#define ZG_MK_Q4_0 2u
#define ZG_MK_Q8_0 8u

/* The library's choice for a single-projection X4 GEMV (zg_gemv.hip,
 * launch_strip): strips S = k / 512 of 16 blocks, one wave per strip (4
 * waves when S < 3), groups of 4 rows in batches of GB per wave.  Returns 0,
 * or -1 for a shape outside the module (type, k, rows). */
static inline int zg_mk_plan(uint32_t qtype, uint32_t rows, uint32_t k, uint32_t cu_count, zg_mk_launch* out) {
  const char* t;
  uint32_t S, nw, wps, items, gb, maxt, nbatch, per;
  int tall = 0;
  if ((qtype != ZG_MK_Q4_0 && qtype != ZG_MK_Q8_0) || k == 0 || k % 512 || k > 8192 || rows == 0 || rows % 4 ||
      cu_count == 0 || !out)
    return -1;
  t = qtype == ZG_MK_Q4_0 ? "q4_0x4" : "q8_0x4";
  S = k / 512;
  nw = S >= 3 ? S : 4;
  wps = nw / S;
  items = rows / 4;
  maxt = 1024;
  if (items > cu_count * 8u * wps && (qtype == ZG_MK_Q4_0 || nw == 4)) {
    /* tall: four groups per batch; Q4_0 takes the tightest thread bound
     * that holds the integer-activation form up to 8 strips */
    tall = 1;
    gb = 4;
    if (qtype == ZG_MK_Q8_0 || nw <= 4) maxt = 256;
    else if (nw <= 8) maxt = 512;
  } else if (qtype == ZG_MK_Q4_0) {
    per = items / (cu_count * 2u * wps);
    gb = per >= 3 ? 3 : ((per < 2 && !(S >= 8 && per >= 1)) ? 1 : 2);
  } else {
    gb = 2;
  }
  nbatch = (items + wps * gb - 1) / (wps * gb);
  out->block = nw * 64;
  out->shm_bytes = 2u * nw * gb * 16u * (uint32_t)sizeof(float);
  out->nbatch = nbatch;
  out->per_cu_cap = nw >= 16 ? 1 : 16 / nw;
  out->one_batch = maxt == 1024 && nbatch <= cu_count * 4u;
  out->occupancy_bound = maxt < 1024;
  {
    char* e = out->entry;
    const char* parts[4];
    char g[8] = "_g0";
    int i, n = 0;
    parts[n++] = "zg_mk_";
    parts[n++] = t;
    if (out->one_batch) {
      g[2] = (char)('0' + gb);
      parts[n++] = "_oneb";
      parts[n++] = g;
    } else if (tall) {
      parts[n++] = maxt == 256 ? "_tall_t256" : (maxt == 512 ? "_tall_t512" : "_tall_t1024");
    } else {
      g[2] = (char)('0' + gb);
      parts[n++] = "_loop";
      parts[n++] = g;
    }
    for (i = 0; i < n; i++) {
      const char* p = parts[i];
      while (*p) *e++ = *p++;
    }
    if (out->one_batch && (S == 4 || S == 12)) {
      const char* p = S == 4 ? "_k2048" : "_k6144";
      while (*p) *e++ = *p++;
    }
    *e = 0;
  }
  return 0;
}

/* Entry points of zg_kernels.hsaco (extern "C" kernels; arguments as
 * zg_mk_gemv_args):
 *   zg_mk_q4_0x4_oneb_g{1,2,3,4}[_k2048|_k6144]  one batch per workgroup
 *   zg_mk_q4_0x4_tall_t{256,512,1024}             four-group batch loop
 *   zg_mk_q8_0x4_oneb_g2[_k2048|_k6144]
 *   zg_mk_q8_0x4_loop_g2                          batch loop, 1024 threads
 *   zg_mk_q8_0x4_tall_t256
 * (the _g4 one-batch forms only as _k6144 and without suffix: tall Q4_0X4
 * launches of more than 8 strips.  A Q4_0X4 launch below the tall size
 * always fits one batch per workgroup, so it has no batch-loop form.) */

#ifdef __cplusplus
}
#endif

#endif /* ZERO_GPU_KERNELS_H */
