"""The code-object route to the decode GEMV (include/zero_gpu_kernels.h).

zero_amd/zg_kernels.hsaco holds the library's strip GEMV for X4 weights as
C-named gfx950 kernels.  This module is the thin FFI layer a host that
launches kernels itself would hold: it binds hipModuleLoad,
hipModuleGetFunction, hipModuleOccupancyMaxActiveBlocksPerMultiprocessor
and hipModuleLaunchKernel of the HIP runtime (the one torch has loaded: the
same SONAME, so one runtime per process) through ctypes, plans each launch
with the library's rule (`plan`, the Python form of zg_mk_plan) and launches
it on a caller stream.  Launches on a stream being captured go into the
graph like any other kernel launch.

Replaces, for the X4 weights, the reference's row-range kernels
(kernel/src/arch/x86_64/math/linear.rs:909-1072 Q4_0X4, 1096-1213 Q8_0X4)
behind linear_dispatch (crates/zero-llm-inference/src/ops.rs:486-523).
A missing code object raises ImportError: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from pathlib import Path

from . import _lib

CODE_OBJECT = Path(__file__).resolve().parent / "zg_kernels.hsaco"

Q4_0 = 2
Q8_0 = 8

# every entry point of the code object (include/zero_gpu_kernels.h)
ENTRIES = (
    [f"zg_mk_q4_0x4_oneb_g{g}{s}" for g in (1, 2, 3) for s in ("_k2048", "_k6144", "")]
    + ["zg_mk_q4_0x4_oneb_g4_k6144", "zg_mk_q4_0x4_oneb_g4"]
    + [f"zg_mk_q4_0x4_tall_t{t}" for t in (256, 512, 1024)]
    + [f"zg_mk_q8_0x4_oneb_g2{s}" for s in ("_k2048", "_k6144", "")]
    + ["zg_mk_q8_0x4_loop_g2", "zg_mk_q8_0x4_tall_t256"]
)


class ModuleError(RuntimeError):
    """A HIP module call failed, or a shape is outside the module."""


@dataclass(frozen=True)
class Launch:
    entry: str
    block: int
    shm_bytes: int
    nbatch: int
    per_cu_cap: int
    one_batch: bool
    occupancy_bound: bool


def plan(qtype: int, rows: int, k: int, cu_count: int) -> Launch:
    """The launch the library makes for a single-projection X4 GEMV of this
    shape (zg_gemv.hip, launch_strip; zg_mk_plan in
    include/zero_gpu_kernels.h states the same rule in C)."""
    if qtype not in (Q4_0, Q8_0) or k <= 0 or k % 512 or k > 8192 or rows <= 0 or rows % 4 or cu_count <= 0:
        raise ModuleError(f"shape outside the module: qtype {qtype}, rows {rows}, k {k}")
    t = "q4_0x4" if qtype == Q4_0 else "q8_0x4"
    S = k // 512
    nw = S if S >= 3 else 4
    wps = nw // S
    items = rows // 4
    maxt = 1024
    tall = False
    if items > cu_count * 8 * wps and (qtype == Q4_0 or nw == 4):
        tall = True
        gb = 4
        if qtype == Q8_0 or nw <= 4:
            maxt = 256
        elif nw <= 8:
            maxt = 512
    elif qtype == Q4_0:
        per = items // (cu_count * 2 * wps)
        gb = 3 if per >= 3 else (1 if (per < 2 and not (S >= 8 and per >= 1)) else 2)
    else:
        gb = 2
    nbatch = -(-items // (wps * gb))
    one = maxt == 1024 and nbatch <= cu_count * 4
    if one:
        entry = f"zg_mk_{t}_oneb_g{gb}" + {4: "_k2048", 12: "_k6144"}.get(S, "")
    elif tall:
        entry = f"zg_mk_{t}_tall_t{maxt}"
    else:
        entry = f"zg_mk_{t}_loop_g{gb}"
    return Launch(entry, nw * 64, 2 * nw * gb * 16 * 4, nbatch, 1 if nw >= 16 else 16 // nw, one, maxt < 1024)


def _runtime() -> C.CDLL:
    _lib.load()  # binds libamdhip64.so.7, torch's runtime when torch is loaded
    hip = C.CDLL("libamdhip64.so.7")
    P, I, U = C.c_void_p, C.c_int, C.c_uint
    hip.hipModuleLoad.argtypes = [C.POINTER(P), C.c_char_p]
    hip.hipModuleLoad.restype = I
    hip.hipModuleUnload.argtypes = [P]
    hip.hipModuleUnload.restype = I
    hip.hipModuleGetFunction.argtypes = [C.POINTER(P), P, C.c_char_p]
    hip.hipModuleGetFunction.restype = I
    hip.hipModuleOccupancyMaxActiveBlocksPerMultiprocessor.argtypes = [C.POINTER(I), P, I, C.c_size_t]
    hip.hipModuleOccupancyMaxActiveBlocksPerMultiprocessor.restype = I
    hip.hipModuleLaunchKernel.argtypes = [P, U, U, U, U, U, U, U, P, C.POINTER(P), C.POINTER(P)]
    hip.hipModuleLaunchKernel.restype = I
    hip.hipGetErrorString.argtypes = [I]
    hip.hipGetErrorString.restype = C.c_char_p
    hip.hipGetLastError.argtypes = []
    hip.hipGetLastError.restype = I
    return hip


class KernelModule:
    """zg_kernels.hsaco loaded on the current device."""

    def __init__(self, path: os.PathLike | str = CODE_OBJECT, cu_count: int | None = None):
        path = Path(path)
        if not path.exists():
            raise ImportError(f"{path} is missing: build it first (zero_amd/build.py); there is no CPU fallback")
        self._hip = _runtime()
        self._mod = C.c_void_p()
        self._check(self._hip.hipModuleLoad(C.byref(self._mod), os.fspath(path).encode()), "hipModuleLoad")
        self._fn: dict[str, C.c_void_p] = {}
        self._occ: dict[tuple, int] = {}
        if cu_count is None:
            import torch

            cu_count = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
        self.cu_count = int(cu_count)

    def _check(self, err: int, what: str) -> None:
        if err != 0:
            # a failed call also becomes the thread's last HIP error; it is
            # reported here, so clear it rather than let the next launch
            # check elsewhere in the process (the library's) report it again
            self._hip.hipGetLastError()
            raise ModuleError(f"{what}: {self._hip.hipGetErrorString(err).decode()} ({err})")

    def function(self, name: str) -> C.c_void_p:
        f = self._fn.get(name)
        if f is None:
            f = C.c_void_p()
            self._check(self._hip.hipModuleGetFunction(C.byref(f), self._mod, name.encode()), f"hipModuleGetFunction {name}")
            self._fn[name] = f
        return f

    def resident(self, name: str, block: int, shm: int) -> int:
        key = (name, block, shm)
        n = self._occ.get(key)
        if n is None:
            v = C.c_int()
            self._check(self._hip.hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(
                C.byref(v), self.function(name), block, shm), "occupancy query")
            n = self._occ[key] = max(1, v.value)
        return n

    def grid(self, lp: Launch) -> int:
        if lp.one_batch:
            return lp.nbatch
        per_cu = lp.per_cu_cap
        if lp.occupancy_bound:
            per_cu = min(per_cu, self.resident(lp.entry, lp.block, lp.shm_bytes))
        return min(lp.nbatch, self.cu_count * per_cu)

    def gemv_x4(self, w: int, x: int, y: int, rows: int, k: int, qtype: int, stream: int = 0) -> Launch:
        """y = W x for X4 weights W (rows x k) at device addresses w, x, y,
        launched asynchronously on `stream` (a HIP stream handle, 0 = the
        null stream).  Returns the launch made."""
        if not w or not x or not y:
            raise ModuleError("null pointer")
        if w % 8 or x % 16 or y % 4:
            raise ModuleError("misaligned buffer")
        lp = plan(qtype, rows, k, self.cu_count)
        args = (C.c_void_p(w), C.c_void_p(x), C.c_void_p(y), C.c_uint32(rows), C.c_uint32(k))
        params = (C.c_void_p * len(args))(*[C.cast(C.pointer(a), C.c_void_p) for a in args])
        self._check(self._hip.hipModuleLaunchKernel(self.function(lp.entry), self.grid(lp), 1, 1, lp.block, 1, 1,
                                                    lp.shm_bytes, C.c_void_p(stream), params, None),
                    f"hipModuleLaunchKernel {lp.entry}")
        return lp

    def close(self) -> None:
        if self._mod:
            self._check(self._hip.hipModuleUnload(self._mod), "hipModuleUnload")
            self._mod = C.c_void_p()
            self._fn.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
