"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg; the product package never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

_P, _S, _I, _U32, _F = C.c_void_p, C.c_size_t, C.c_int, C.c_uint32, C.c_float


class zo_segment(C.Structure):
    _fields_ = [("w", _P), ("out", _P), ("out_dim", _S), ("ggml_type", _I), ("interleave", _I)]


class zo_layer(C.Structure):
    _fields_ = [(n, _P) for n in ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_gate", "ffn_up", "ffn_down",
                                  "attn_norm", "ffn_norm", "q_norm", "k_norm")]


class zo_layer_quants(C.Structure):
    _fields_ = [("type", _I * 7), ("interleave", _I * 7)]


class zo_model_desc(C.Structure):
    _fields_ = [
        ("n_layers", _I), ("hidden", _I), ("ffn", _I), ("n_q_heads", _I), ("n_kv_heads", _I), ("head_dim", _I),
        ("vocab_padded", _S), ("vocab_real", _S), ("max_ctx", _S),
        ("rms_eps", _F), ("rope_theta", _F),
        ("lin_type", _I), ("lin_interleave", _I), ("embd_type", _I), ("head_type", _I), ("head_interleave", _I),
        ("token_embd", _P), ("lm_head", _P), ("output_norm", _P), ("layers", C.POINTER(zo_layer)),
        ("layer_quants", C.POINTER(zo_layer_quants)),
    ]


_SIG = {
    "zo_fp16_to_f32": (_F, [C.c_uint16]),
    "zo_fp16_to_f32_array": (None, [_P, _P, _S]),
    "zo_get_scale_min_k4": (None, [_P, _I, _P, _P]),
    "zo_dequant_q4_0_row": (None, [_P, _P, _S]),
    "zo_dequant_q8_0_row": (None, [_P, _P, _S]),
    "zo_dequant_q4k_row": (None, [_P, _P, _S]),
    "zo_dequant_q6k_row": (None, [_P, _P, _S]),
    "zo_dequant_tensor": (_I, [_P, _P, _S, _S, _I, _I]),
    "zo_linear_scalar": (_I, [_P, _P, _P, _S, _S, _I]),
    "zo_linear_range": (_I, [_P, _P, _P, _S, _S, _I, _I, _S, _S]),
    "zo_avx512_available": (_I, []),
    "zo_linear_range_avx512": (_I, [_P, _P, _P, _S, _S, _I, _I, _S, _S]),
    "zo_set_simd": (_I, [_I]),
    "zo_linear_f64": (_I, [_P, _P, _P, _S, _S, _I, _I]),
    "zo_interleave_x4": (_I, [_P, _P, _S, _S, _I]),
    "zo_deinterleave_x4": (_I, [_P, _P, _S, _S, _I]),
    "zo_f64_to_fp16_bits": (C.c_uint16, [C.c_double]),
    "zo_quantize_q8_0_row": (None, [_P, _P, _S]),
    "zo_quantize_q4_0_row": (None, [_P, _P, _S]),
    "zo_argmax": (_S, [_P, _S, C.POINTER(_F)]),
    "zo_argmax_beats": (_I, [_F, _U32, _F, _U32]),
    "zo_row_range_for": (None, [_S, _U32, _S, _S, C.POINTER(_S), C.POINTER(_S)]),
    "zo_row_range_for_discounted": (None, [_S, _U32, _S, _S, _S, C.POINTER(_S), C.POINTER(_S)]),
    "zo_pool_start": (_I, [_I]),
    "zo_pool_stop": (None, []),
    "zo_pool_size": (_I, []),
    "zo_linear_parallel": (_I, [_P, _P, _P, _S, _S, _I, _I]),
    "zo_linear_fused_parallel": (_I, [_P, C.POINTER(zo_segment), _I, _S]),
    "zo_lm_head_linear_argmax_parallel": (_S, [_P, _P, _P, _S, _S, _I, _I, C.POINTER(_F)]),
    "zo_rmsnorm": (None, [_P, _P, _P, _S, _F]),
    "zo_rope_inv_freqs": (None, [_P, _I, _F]),
    "zo_rope": (None, [_P, _P, _I, _S]),
    "zo_softmax": (_I, [_P, _S]),
    "zo_silu_mul": (None, [_P, _P, _P, _S]),
    "zo_gemm_q8act": (_I, [_P, _P, _P, _S, _S, _S, _I, _I]),
    "zo_model_create": (_P, [C.POINTER(zo_model_desc)]),
    "zo_model_destroy": (None, [_P]),
    "zo_model_forward": (_I, [_P, _U32, _S, _P]),
    "zo_model_lm_head": (_I, [_P, _P, C.POINTER(_U32), C.POINTER(_F)]),
    "zo_model_first_nonfinite": (_S, [_P, C.c_char_p]),
    "zo_nonfinite_text": (_S, [_P, _S, _I, C.c_char_p, C.c_char_p]),
    "zo_model_prefill_q8": (_I, [_P, _P, _S, _S, _P]),
    "zo_quantize_row_q8k": (None, [_P, _P, _S]),
    "zo_unpack_mins_and_scales": (None, [_P, _P]),
    "zo_linear_q4k_q8k_range": (_I, [_P, _P, _P, _S, _S, _S]),
    "zo_linear_q6k_q8k_range": (_I, [_P, _P, _P, _S, _S, _S]),
}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", os.fspath(HERE)], check=True)
    return LIB


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = C.CDLL(os.fspath(LIB))
        for name, (res, args) in _SIG.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _lib = lib
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def fp16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.size, np.float32)
    load().zo_fp16_to_f32_array(_p(bits), _p(out), bits.size)
    return out


def dequant(w: np.ndarray, rows: int, in_dim: int, quant: int, interleave: int = 1) -> np.ndarray:
    out = np.empty((rows, in_dim), np.float32)
    rc = load().zo_dequant_tensor(_p(w), _p(out), rows, in_dim, quant, interleave)
    assert rc == 0, rc
    return out


def linear_scalar(x, w, in_dim, out_dim, quant) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(out_dim, np.float32)
    assert load().zo_linear_scalar(_p(x), _p(w), _p(out), in_dim, out_dim, quant) == 0
    return out


def linear_range(x, w, in_dim, out_dim, quant, interleave=1, start=0, end=None, out=None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    end = out_dim if end is None else end
    if out is None:
        out = np.zeros(out_dim, np.float32)
    assert load().zo_linear_range(_p(x), _p(w), _p(out), in_dim, out_dim, quant, interleave, start, end) == 0
    return out


def avx512_available() -> bool:
    return bool(load().zo_avx512_available())


def linear_range_avx512(x, w, in_dim, out_dim, quant, interleave=1, start=0, end=None, out=None) -> np.ndarray:
    """The AVX-512 intrinsics form of linear_range (zg_avx512.c)."""
    x = np.ascontiguousarray(x, np.float32)
    end = out_dim if end is None else end
    if out is None:
        out = np.zeros(out_dim, np.float32)
    rc = load().zo_linear_range_avx512(_p(x), _p(w), _p(out), in_dim, out_dim, quant, interleave, start, end)
    assert rc == 0, rc
    return out


def set_simd(on: bool) -> bool:
    """Route the pool's range kernels through the AVX-512 intrinsics (when
    the CPU has AVX-512F); returns whether they are in force."""
    return bool(load().zo_set_simd(1 if on else 0))


def linear_f64(x, w, in_dim, out_dim, quant, interleave=1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(out_dim, np.float64)
    assert load().zo_linear_f64(_p(x), _p(w), _p(out), in_dim, out_dim, quant, interleave) == 0
    return out


def linear_parallel(x, w, in_dim, out_dim, quant, interleave=1, out=None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    if out is None:
        out = np.empty(out_dim, np.float32)
    assert load().zo_linear_parallel(_p(x), _p(w), _p(out), in_dim, out_dim, quant, interleave) == 0
    return out


def linear_fused_parallel(x, segs, in_dim, outs=None):
    """linear_fused_dispatch over the pool: segs = [(w, out_dim, quant,
    interleave)], one row split over the concatenated rows."""
    x = np.ascontiguousarray(x, np.float32)
    if outs is None:
        outs = [np.empty(n, np.float32) for _, n, _, _ in segs]
    arr = (zo_segment * len(segs))()
    for i, ((w, n, q, il), o) in enumerate(zip(segs, outs)):
        arr[i] = zo_segment(_p(w), _p(o), n, q, il)
    assert load().zo_linear_fused_parallel(_p(x), arr, len(segs), in_dim) == 0
    return outs


def lm_head_parallel(x, w, in_dim, out_dim, quant, interleave, logits=None) -> tuple[int, float, np.ndarray]:
    """lm_head_linear_argmax_dispatch over the pool: logits and the merged
    first-max argmax."""
    x = np.ascontiguousarray(x, np.float32)
    if logits is None:
        logits = np.empty(out_dim, np.float32)
    mv = C.c_float()
    idx = load().zo_lm_head_linear_argmax_parallel(_p(x), _p(w), _p(logits), in_dim, out_dim, quant, interleave,
                                                   C.byref(mv))
    return int(idx), float(mv.value), logits


def interleave_x4(plain, rows, in_dim, quant) -> np.ndarray:
    out = np.empty_like(plain)
    assert load().zo_interleave_x4(_p(plain), _p(out), rows, in_dim, quant) == 0
    return out


def quantize_q8_0(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // 32 * 34, np.uint8)
    load().zo_quantize_q8_0_row(_p(x), _p(out), x.size)
    return out


def quantize_q4_0(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // 32 * 18, np.uint8)
    load().zo_quantize_q4_0_row(_p(x), _p(out), x.size)
    return out


Q8K_BYTES = 292


def quantize_q8k(x) -> np.ndarray:
    """quantize_row_q8k: 292-byte blocks (f32 d, 256 int8, 16 int16 sums)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // 256 * Q8K_BYTES, np.uint8)
    load().zo_quantize_row_q8k(_p(x), _p(out), x.size)
    return out


def unpack_mins_and_scales(s12) -> np.ndarray:
    s = np.ascontiguousarray(s12, np.uint8)
    out = np.empty(16, np.uint8)
    load().zo_unpack_mins_and_scales(_p(s), _p(out))
    return out


def linear_q4k_q8k(q8k, w, in_dim, out_dim, start=0, end=None) -> np.ndarray:
    """linear_q4k_vnni_range over rows [start, end)."""
    end = out_dim if end is None else end
    out = np.zeros(out_dim, np.float32)
    assert load().zo_linear_q4k_q8k_range(_p(q8k), _p(w), _p(out), in_dim, start, end) == 0
    return out


def linear_q6k_q8k(q8k, w, in_dim, out_dim, start=0, end=None) -> np.ndarray:
    """The Q6_K x Q8_K integer construction over rows [start, end)."""
    end = out_dim if end is None else end
    out = np.zeros(out_dim, np.float32)
    assert load().zo_linear_q6k_q8k_range(_p(q8k), _p(w), _p(out), in_dim, start, end) == 0
    return out


def gemm_q8k(x, w, m, n, k, w_type) -> np.ndarray:
    """The K-quant prefill GEMM's arithmetic, row by row: each of the m rows
    of x (fp32, [m][k]) quantized to Q8_K, then the integer dot with the n
    Q4_K (w_type 12) or Q6_K (14) rows of w."""
    x = np.ascontiguousarray(x, np.float32).reshape(m, k)
    f = linear_q4k_q8k if w_type == 12 else linear_q6k_q8k
    y = np.empty((m, n), np.float32)
    for i in range(m):
        y[i] = f(quantize_q8k(x[i]), w, k, n)
    return y


def nonfinite_text(buf, layer: int, stage: str) -> str:
    """The latch text finite_diag would record for buf ("" when finite)."""
    b = np.ascontiguousarray(buf, np.float32)
    out = C.create_string_buffer(32)
    n = load().zo_nonfinite_text(_p(b), b.size, layer, stage.encode(), out)
    return out.raw[:n].decode()


def argmax(v) -> tuple[int, float]:
    v = np.ascontiguousarray(v, np.float32)
    mv = _F()
    i = load().zo_argmax(_p(v), v.size, C.byref(mv))
    return int(i), float(mv.value)


def row_range_for(total, n, i, align, discount=0) -> tuple[int, int]:
    s, e = _S(), _S()
    if discount:
        load().zo_row_range_for_discounted(total, n, i, align, discount, C.byref(s), C.byref(e))
    else:
        load().zo_row_range_for(total, n, i, align, C.byref(s), C.byref(e))
    return int(s.value), int(e.value)


def gemm_q8act(xq_blocks, w, m, n, k, w_type, interleave) -> np.ndarray:
    y = np.empty((m, n), np.float32)
    assert load().zo_gemm_q8act(_p(xq_blocks), _p(w), _p(y), m, n, k, w_type, interleave) == 0
    return y


class Pool:
    """Pinned worker pool of the SMP restatement (start/stop around use)."""

    def __init__(self, n_threads: int):
        self.n = load().zo_pool_start(n_threads)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        load().zo_pool_stop()


class OracleModel:
    """C restatement of the single-token forward pass over a RandomModel."""

    def __init__(self, model):
        cfg = model.cfg
        self.cfg = cfg
        self.model = model
        self._layers = (zo_layer * cfg.n_layers)()
        for i, L in enumerate(model.layers):
            self._layers[i] = zo_layer(*[getattr(L, f).ctypes.data for f, _ in zo_layer._fields_])
        d = zo_model_desc()
        d.n_layers, d.hidden, d.ffn = cfg.n_layers, cfg.hidden, cfg.ffn
        d.n_q_heads, d.n_kv_heads, d.head_dim = cfg.n_q_heads, cfg.n_kv_heads, cfg.head_dim
        d.vocab_padded, d.vocab_real, d.max_ctx = cfg.vocab_padded, cfg.vocab_real, cfg.max_ctx
        d.rms_eps, d.rope_theta = cfg.rms_eps, cfg.rope_theta
        d.lin_type, d.lin_interleave, d.embd_type = cfg.lin_type, cfg.lin_interleave, cfg.embd_type
        d.head_type, d.head_interleave = cfg.head_type, cfg.head_interleave
        d.token_embd, d.lm_head, d.output_norm = (model.token_embd.ctypes.data, model.lm_head.ctypes.data,
                                                  model.output_norm.ctypes.data)
        d.layers = self._layers
        if cfg.layer_quants is not None:
            self._quants = (zo_layer_quants * cfg.n_layers)()
            for i, lq in enumerate(cfg.layer_quants):
                for p, (t, il) in enumerate(lq):
                    self._quants[i].type[p], self._quants[i].interleave[p] = t, il
            d.layer_quants = self._quants
        self._desc = d
        self.h = load().zo_model_create(C.byref(d))
        assert self.h

    def close(self):
        if self.h:
            load().zo_model_destroy(self.h)
            self.h = None

    def forward(self, token, pos):
        hid = np.empty(self.cfg.hidden, np.float32)
        rc = load().zo_model_forward(self.h, token, pos, _p(hid))
        assert rc == 0, rc
        return hid

    def forward_status(self, token, pos) -> int:
        """zo_model_forward's status (-4: the attention softmax failed)."""
        return load().zo_model_forward(self.h, token, pos, None)

    def first_nonfinite(self) -> str:
        """The latch of finite_diag: e.g. "L03 attn_out n1 i0", or ""."""
        buf = C.create_string_buffer(32)
        n = load().zo_model_first_nonfinite(self.h, buf)
        return buf.raw[:n].decode()

    def prefill_q8(self, tokens, pos0=0):
        """Batched prefill with Q8_0 activations; returns the last row's
        final hidden state (the model is then ready for lm_head())."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        hid = np.empty(self.cfg.hidden, np.float32)
        rc = load().zo_model_prefill_q8(self.h, _p(t), t.size, pos0, _p(hid))
        assert rc == 0, rc
        return hid

    def generate_batched(self, prompt, n_gen):
        """prefill_q8 of the prompt, then the single-token greedy loop."""
        self.prefill_q8(prompt, 0)
        rc, tok, _, _ = self.lm_head()
        assert rc == 0, rc
        toks = [tok]
        pos = len(prompt)
        while len(toks) < n_gen:
            self.forward(toks[-1], pos)
            pos += 1
            rc, tok, _, _ = self.lm_head()
            assert rc == 0, rc
            toks.append(tok)
        return np.array(toks, np.uint32)

    def lm_head(self):
        lg = np.empty(self.cfg.vocab_padded, np.float32)
        tok = _U32()
        mv = _F()
        rc = load().zo_model_lm_head(self.h, _p(lg), C.byref(tok), C.byref(mv))
        return rc, int(tok.value), float(mv.value), lg

    def generate(self, prompt, n_gen):
        """Same caller loop as zg_model_generate; returns the tokens."""
        toks = []
        for i, t in enumerate(prompt):
            self.forward(int(t), i)
        rc, tok, _, _ = self.lm_head()
        assert rc == 0, rc
        toks.append(tok)
        pos = len(prompt)
        while len(toks) < n_gen:
            self.forward(toks[-1], pos)
            pos += 1
            rc, tok, _, _ = self.lm_head()
            assert rc == 0, rc
            toks.append(tok)
        return np.array(toks, np.uint32)
