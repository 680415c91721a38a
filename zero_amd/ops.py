"""Host-side mirror of the reference's quantized-matmul operator API.

Same names, argument meaning and error behaviour as the Rust operators this
path replaces, re-expressed in Python over the C ABI:

* ``linear_dispatch``      crates/zero-llm-inference/src/ops.rs:486-523
* ``linear_dispatch_avx512``  kernel/src/inference_avx512.rs:1147-1184
* ``linear_fused_dispatch``   kernel/src/inference_avx512.rs:890-945
* ``lm_head_argmax``          kernel/src/inference_avx512.rs:1200-1270
* ``register`` / ``group_of`` / ``rebase`` / ``clear``
                              kernel/src/weight_layout.rs:57-149
* ``linear_q4k_vnni``         kernel/src/inference_avx512.rs:519-547
                              (feature "vnni-acceleration")

Weights are numpy uint8 arrays (the ``&[u8]`` block bytes); activations and
outputs are float32 arrays.  Every call runs on the GPU; there is no CPU
fallback.
"""
from __future__ import annotations

import ctypes as C
from enum import IntEnum

import numpy as np

from . import _lib


class GgmlType(IntEnum):
    """GgmlType ids (crates/zero-gguf-parser/src/lib.rs:95-126)."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    Q4K = 12
    Q6K = 14


SUPPORTED = (GgmlType.Q4_0, GgmlType.Q8_0, GgmlType.Q4K, GgmlType.Q6K)
BLOCK = {GgmlType.Q4_0: (32, 18), GgmlType.Q8_0: (32, 34), GgmlType.Q4K: (256, 144), GgmlType.Q6K: (256, 210)}

# lm_head.rs:12-15
VOCAB_SIZE_REAL = 151_643
VOCAB_SIZE_PADDED = 151_936


class ZgError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class LinearDispatchError(ZgError):
    """LinearDispatchError::UnsupportedQuant (ops.rs:467-474)."""

    def __init__(self, quant: int, msg: str = ""):
        super().__init__(_lib.ZG_ERR_UNSUPPORTED_QUANT, msg or f"linear_dispatch: unsupported quant type {int(quant)}")
        self.quant = quant


class LmHeadError(ZgError):
    """LmHeadError (crates/zero-llm-inference/src/lm_head.rs:32-38)."""


class NonFiniteLogits(LmHeadError):
    pass


class ArgmaxInPaddingRegion(LmHeadError):
    def __init__(self, code: int, msg: str, index: int):
        super().__init__(code, msg)
        self.index = index


def tensor_bytes(quant: int, rows: int, in_dim: int) -> int:
    be, bb = BLOCK[GgmlType(quant)]
    return rows * (in_dim // be) * bb


def _ptr(a) -> int:
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return int(a)


class Context:
    """One GPU context: stream, weight registry and staging buffers.

    Mirrors the reference's single-caller (BSP-only) contract: a Context is
    not thread-safe (kernel/src/smp.rs:1567-1712)."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        h = C.c_void_p()
        rc = self.lib.zg_init(device, C.byref(h))
        if rc != _lib.ZG_OK:
            raise ZgError(rc, f"zg_init(device={device}) failed")
        self.h = h
        self._keep = {}  # registered host arrays stay alive (their address is the key)

    def close(self):
        if getattr(self, "h", None):
            self.lib.zg_destroy(self.h)
            self.h = None
            self._keep.clear()

    def __del__(self):  # pragma: no cover - interpreter teardown order
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def stream(self) -> int:
        return self.lib.zg_stream(self.h) or 0

    def last_error(self) -> str:
        return (self.lib.zg_last_error(self.h) or b"").decode()

    def check(self, rc: int):
        if rc == _lib.ZG_OK:
            return
        msg = self.last_error()
        if rc == _lib.ZG_ERR_UNSUPPORTED_QUANT:
            raise LinearDispatchError(-1, msg)
        if rc == _lib.ZG_ERR_NONFINITE_LOGITS:
            raise NonFiniteLogits(rc, msg)
        raise ZgError(rc, msg)

    # ---- registry (weight_layout.rs) ----
    def register(self, w: np.ndarray, quant: int, interleave: int = 1):
        """Upload ``w`` and register it under its host address
        (weight_layout::register + the model loader's upload)."""
        if not (isinstance(w, np.ndarray) and w.dtype == np.uint8 and w.flags.c_contiguous):
            raise TypeError("weights must be a C-contiguous uint8 numpy array")
        self.check(self.lib.zg_register_weight(self.h, w.ctypes.data, w.nbytes, int(quant), int(interleave)))
        self._keep[w.ctypes.data] = w
        return w

    def register_device(self, key: int, dev_ptr: int, nbytes: int, quant: int, interleave: int = 1):
        self.check(self.lib.zg_register_weight_device(self.h, key, dev_ptr, nbytes, int(quant), int(interleave)))

    def group_of(self, w) -> int:
        return int(self.lib.zg_group_of(self.h, _ptr(w)))

    def rebase(self, delta: int):
        self.lib.zg_rebase(self.h, int(delta))

    def clear(self):
        self.lib.zg_clear(self.h)
        self._keep.clear()

    def registered_count(self) -> int:
        return int(self.lib.zg_registered_count(self.h))

    # ---- operators ----
    def linear_dispatch(self, x: np.ndarray, w_blocks: np.ndarray, out: np.ndarray, in_dim: int, out_dim: int,
                        quant: int) -> None:
        """ops.rs:486-523 / inference_avx512.rs:1147-1184: out = W . x.
        Raises LinearDispatchError for a quant without a kernel (the
        reference panics with the same message)."""
        if int(quant) not in [int(q) for q in SUPPORTED]:
            raise LinearDispatchError(int(quant))
        x = np.ascontiguousarray(x, dtype=np.float32)
        if out.dtype != np.float32 or not out.flags.c_contiguous or out.size < out_dim or x.size < in_dim:
            raise ValueError("x/out must be float32 and sized in_dim/out_dim")
        self.check(self.lib.zg_linear(self.h, x.ctypes.data, _ptr(w_blocks), out.ctypes.data, in_dim, out_dim,
                                      int(quant)))

    linear_dispatch_avx512 = linear_dispatch

    def linear_range(self, x, w_blocks, out, in_dim, out_dim, quant, start, end) -> None:
        x = np.ascontiguousarray(x, dtype=np.float32)
        self.check(self.lib.zg_linear_range(self.h, x.ctypes.data, _ptr(w_blocks), out.ctypes.data, in_dim, out_dim,
                                            int(quant), start, end))

    def linear_fused_dispatch(self, x: np.ndarray, segments, in_dim: int) -> None:
        """inference_avx512.rs:890-945; segments = [(w, out, quant), ...]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        arr = (_lib.zg_segment * len(segments))()
        for i, (w, out, quant) in enumerate(segments):
            arr[i] = _lib.zg_segment(_ptr(w), out.ctypes.data, out.size, int(quant), 0)
        self.check(self.lib.zg_linear_fused(self.h, x.ctypes.data, arr, len(segments), in_dim))

    def lm_head_argmax(self, final_hidden, output_norm_weight, output_weight, output_quant, rms_eps,
                       embedding_dim, logits_buf=None, vocab_padded=VOCAB_SIZE_PADDED,
                       vocab_real=VOCAB_SIZE_REAL) -> int:
        """inference_avx512.rs:1200-1270; returns the token id or raises
        NonFiniteLogits / ArgmaxInPaddingRegion."""
        h = np.ascontiguousarray(final_hidden, dtype=np.float32)
        nw = np.ascontiguousarray(output_norm_weight, dtype=np.float32)
        tok = C.c_uint32()
        mv = C.c_float()
        lp = logits_buf.ctypes.data if logits_buf is not None else None
        rc = self.lib.zg_lm_head_argmax(self.h, h.ctypes.data, nw.ctypes.data, _ptr(output_weight), int(output_quant),
                                        float(rms_eps), embedding_dim, vocab_padded, vocab_real, lp, C.byref(tok),
                                        C.byref(mv))
        if rc == _lib.ZG_ERR_ARGMAX_IN_PADDING:
            raise ArgmaxInPaddingRegion(rc, self.last_error(), int(tok.value))
        self.check(rc)
        return int(tok.value)

    # ---- device-pointer API (torch tensors or raw addresses) ----
    def linear_dev(self, x, w, out, in_dim, out_dim, quant, interleave, start=0, end=None, stream=None):
        end = out_dim if end is None else end
        self.check(self.lib.zg_linear_dev(self.h, _ptr(x), _ptr(w), _ptr(out), in_dim, out_dim, int(quant),
                                          int(interleave), start, end, stream))

    def linear_fused_dev(self, x, segments, in_dim, stream=None):
        """segments = [(w, out, out_dim, quant, interleave), ...] device pointers."""
        arr = (_lib.zg_segment * len(segments))()
        for i, (w, out, n, q, il) in enumerate(segments):
            arr[i] = _lib.zg_segment(_ptr(w), _ptr(out), n, int(q), int(il))
        self.check(self.lib.zg_linear_fused_dev(self.h, _ptr(x), arr, len(segments), in_dim, stream))

    def lm_head_dev(self, x, w, logits, in_dim, out_dim, quant, interleave, best, stream=None):
        self.check(self.lib.zg_lm_head_dev(self.h, _ptr(x), _ptr(w), _ptr(logits) if logits is not None else None,
                                           in_dim, out_dim, int(quant), int(interleave), _ptr(best), stream))

    def dequant_dev(self, w, out, rows, in_dim, quant, interleave, stream=None):
        self.check(self.lib.zg_dequant_dev(self.h, _ptr(w), _ptr(out), rows, in_dim, int(quant), int(interleave),
                                           stream))

    def fp16_to_f32_dev(self, src, out, n, stream=None):
        self.check(self.lib.zg_fp16_to_f32_dev(self.h, _ptr(src), _ptr(out), n, stream))

    def read_floor_dev(self, src, nbytes, loads_per_thread, sink, stream=None):
        """One streaming read of nbytes (zg_read_floor_dev): the per-launch
        floor that a GEMV of the same weight bytes is measured against."""
        self.check(self.lib.zg_read_floor_dev(self.h, _ptr(src), nbytes, loads_per_thread, _ptr(sink), stream))

    def strip_loads_dev(self, w, rows, x, sink, stream=None):
        """The Q4_0X4 strip GEMV's loads alone, rows x 2048 (zg_strip_loads_dev);
        x None: the weight loads only."""
        self.check(self.lib.zg_strip_loads_dev(self.h, _ptr(w), rows, None if x is None else _ptr(x), _ptr(sink),
                                               stream))

    def quantize_q8_0_dev(self, x, q_blocks, rows, k, stream=None):
        self.check(self.lib.zg_quantize_q8_0_dev(self.h, _ptr(x), _ptr(q_blocks), rows, k, stream))

    def quantize_q8_0_split_dev(self, x, qs, d, rows, k, stream=None):
        self.check(self.lib.zg_quantize_q8_0_split_dev(self.h, _ptr(x), _ptr(qs), _ptr(d), rows, k, stream))

    def linear_q8act_dev(self, xq, w, out, in_dim, out_dim, quant, interleave, stream=None):
        """GEMV with a Q8_0-encoded activation row (34-byte blocks)."""
        self.check(self.lib.zg_linear_q8act_dev(self.h, _ptr(xq), _ptr(w), _ptr(out), in_dim, out_dim, int(quant),
                                                int(interleave), stream))

    def gemm_q8act_dev(self, qs, d, w, y, m, n, k, w_type, interleave, stream=None):
        self.check(self.lib.zg_gemm_q8act_dev(self.h, _ptr(qs), _ptr(d), _ptr(w), _ptr(y), m, n, k, int(w_type),
                                              int(interleave), stream))

    def quantize_q8k_split_dev(self, x, qs, d8, bs32, rows, k, stream=None):
        """quantize_row_q8k per 256 values of rows x k floats, as the K-quant
        GEMM's split arrays: int8 qs [rows][k], f32 d8 [rows][k/256], int16
        bs32 [rows][k/32] (sums of 32 quants)."""
        self.check(self.lib.zg_quantize_q8k_split_dev(self.h, _ptr(x), _ptr(qs), _ptr(d8), _ptr(bs32), rows, k,
                                                      stream))

    def gemm_q8k_dev(self, qs, d8, bs32, w, y, m, n, k, w_type, accumulate=False, stream=None):
        """K-quant prefill GEMM: Y (+)= Xq8k . W for plain Q4_K / Q6_K rows."""
        self.check(self.lib.zg_gemm_q8k_dev(self.h, _ptr(qs), _ptr(d8), _ptr(bs32), _ptr(w), _ptr(y), m, n, k,
                                            int(w_type), 1 if accumulate else 0, stream))

    # ---- Q4_K x Q8_K integer path (kernel/src/arch/x86_64/math/vnni.rs) ----
    def linear_q4k_vnni(self, x: np.ndarray, w_blocks: np.ndarray, out: np.ndarray, in_dim: int,
                        out_dim: int) -> None:
        """linear_q4k_vnni_dispatch (inference_avx512.rs:519-547): x is
        quantized to Q8_K and dotted with the registered Q4_K rows in
        integers; out = W . x up to the activation quantization."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if out.dtype != np.float32 or not out.flags.c_contiguous or out.size < out_dim or x.size < in_dim:
            raise ValueError("x/out must be float32 and sized in_dim/out_dim")
        self.check(self.lib.zg_linear_q4k_vnni(self.h, x.ctypes.data, _ptr(w_blocks), out.ctypes.data, in_dim,
                                               out_dim))

    def linear_q4k_vnni_noalloc(self, x, w, out, in_dim, out_dim, stream=None):
        """linear_q4k_vnni_dispatch on device pointers with no allocation:
        the Q8_K blocks of x live in the library's fixed device array
        (in_dim <= 32768)."""
        self.check(self.lib.zg_linear_q4k_vnni_noalloc(self.h, _ptr(x), _ptr(w), _ptr(out), in_dim, out_dim,
                                                       stream))

    def quantize_q8k_dev(self, x, q8k, n, stream=None):
        """quantize_row_q8k (vnni.rs:78-170) into 292-byte blocks."""
        self.check(self.lib.zg_quantize_q8k_dev(self.h, _ptr(x), _ptr(q8k), n, stream))

    def linear_q4k_q8k_dev(self, q8k, w, out, in_dim, out_dim, stream=None):
        """linear_q4k_vnni_range (vnni.rs:258-476) over all rows."""
        self.check(self.lib.zg_linear_q4k_q8k_dev(self.h, _ptr(q8k), _ptr(w), _ptr(out), in_dim, out_dim, stream))

    @staticmethod
    def argmax_unpack(packed: int):
        idx = C.c_uint32()
        v = C.c_float()
        ok = _lib.load().zg_argmax_unpack(C.c_uint64(packed), C.byref(idx), C.byref(v))
        return bool(ok), int(idx.value), float(v.value)
