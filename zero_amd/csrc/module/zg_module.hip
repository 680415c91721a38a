// zg_module.hip -- the strip GEMV as a standalone gfx950 code object with
// C-named entry points, for a host that loads kernels itself
// (hipModuleLoad, hipModuleGetFunction, hipModuleLaunchKernel, and stream
// capture of those launches into a hipGraph) instead of calling the
// library's C ABI.
//
// Replaces, like the library's strip launches, the AVX-512 X4 range kernels
// (kernel/src/arch/x86_64/math/linear.rs:909-1072 for Q4_0X4, 743-906 for
// Q8_0X4) behind linear_dispatch (crates/zero-llm-inference/src/ops.rs:486-523).
//
// Built by zero_amd/build.py into zero_amd/zg_kernels.hsaco (hipcc
// --genco), not into libzero_amd.so.  Every entry is the library's strip
// kernel body (zg_strip.h) instantiated with the template arguments the
// library's launcher picks for the same shape, so the same launch geometry
// gives the same bits.  The entries, their arguments and the launch
// geometry a host must use are listed in include/zero_gpu_kernels.h.
#include "../zg_strip.h"

namespace zg {

// The GemvArgs of a single-projection X4 GEMV y = W x (W: rows x k, X4
// group-blocks; rows a multiple of 4).  Every field is a kernel argument or
// a constant, so it stays in scalar registers.
__device__ __forceinline__ GemvArgs module_args(const uint8_t* w, const float* x, float* y, uint32_t rows,
                                                uint32_t k) {
  GemvArgs a{};
  a.seg[0] = GemvSeg{w, y, nullptr, 0u, 0u, rows};
  a.seg[1] = a.seg[0];
  a.seg[2] = a.seg[0];
  a.nseg = 1;
  a.k = (int)k;
  a.total_groups = rows / 4;
  a.x = x;
  return a;
}

}  // namespace zg

// NAME: entry point; QT weight type; GB groups per batch (per wave); MAXT
// the thread bound; ONEB one batch per workgroup; SC the strip count as a
// constant (0: k / 512 at run time); DIG integer-digit activations.
#define ZG_MODULE_GEMV(NAME, QT, GB, MAXT, ONEB, SC, DIG)                                                   \
  extern "C" __global__ __launch_bounds__(MAXT) void NAME(const uint8_t* w, const float* x, float* y,      \
                                                          uint32_t rows, uint32_t k) {                     \
    zg::gemv_strip_body<QT, zg::PRO_PLAIN, zg::EPI_STORE, GB, MAXT, true, 4, ONEB, SC, DIG>(               \
        zg::module_args(w, x, y, rows, k), (int)(k / 512), (int)blockIdx.x, (int)gridDim.x);               \
  }

// Q4_0X4: one batch per workgroup (decode-sized launches), 1-3 groups per wave
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g1_k2048, zg::Q4_0, 1, 1024, true, 4, false)
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g1_k6144, zg::Q4_0, 1, 1024, true, 12, false)
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g1, zg::Q4_0, 1, 1024, true, 0, false)
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g2_k2048, zg::Q4_0, 2, 1024, true, 4, false)
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g2_k6144, zg::Q4_0, 2, 1024, true, 12, false)
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g2, zg::Q4_0, 2, 1024, true, 0, false)
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g3_k2048, zg::Q4_0, 3, 1024, true, 4, false)
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g3_k6144, zg::Q4_0, 3, 1024, true, 12, false)
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g3, zg::Q4_0, 3, 1024, true, 0, false)
// Q4_0X4 tall launches of more than 8 strips whose batches fit one per
// workgroup: four groups per wave, fp32 activations
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g4_k6144, zg::Q4_0, 4, 1024, true, 12, false)
ZG_MODULE_GEMV(zg_mk_q4_0x4_oneb_g4, zg::Q4_0, 4, 1024, true, 0, false)
// Q4_0X4 tall launches: four groups per batch; integer activations up to 8
// strips (256- and 512-thread bounds), fp32 beyond
ZG_MODULE_GEMV(zg_mk_q4_0x4_tall_t256, zg::Q4_0, 4, 256, false, 0, true)
ZG_MODULE_GEMV(zg_mk_q4_0x4_tall_t512, zg::Q4_0, 4, 512, false, 0, true)
ZG_MODULE_GEMV(zg_mk_q4_0x4_tall_t1024, zg::Q4_0, 4, 1024, false, 0, false)
// Q8_0X4: two groups per batch, one batch per workgroup or a batch loop
ZG_MODULE_GEMV(zg_mk_q8_0x4_oneb_g2_k2048, zg::Q8_0, 2, 1024, true, 4, false)
ZG_MODULE_GEMV(zg_mk_q8_0x4_oneb_g2_k6144, zg::Q8_0, 2, 1024, true, 12, false)
ZG_MODULE_GEMV(zg_mk_q8_0x4_oneb_g2, zg::Q8_0, 2, 1024, true, 0, false)
ZG_MODULE_GEMV(zg_mk_q8_0x4_loop_g2, zg::Q8_0, 2, 1024, false, 0, true)
// Q8_0X4 tall launches at in_dim 2048: four groups per batch, 256 threads
ZG_MODULE_GEMV(zg_mk_q8_0x4_tall_t256, zg::Q8_0, 4, 256, false, 0, true)
