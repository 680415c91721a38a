"""Forward pass over the C ABI: the GPU counterpart of
forward_single_token_avx512 + lm_head_argmax_avx512
(kernel/src/inference_avx512.rs:1200-1270, 1826-1987) and of the caller's
prefill/greedy loop (kernel/src/inference.rs:1188-1330, 1817-).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .ops import ArgmaxInPaddingRegion, Context, NonFiniteLogits, ZgError
from .synth import RandomModel


class GpuModel:
    """Uploads a model's tensors through the weight registry and builds the
    per-token HIP graphs (zg_model_create)."""

    def __init__(self, ctx: Context, model: RandomModel, register: bool = True):
        """``register=False`` when the weights are already in the context's
        registry (``from_smodel``)."""
        self.ctx = ctx
        self.cfg = cfg = model.cfg
        self.model = model
        if register:
            for li, L in enumerate(model.layers):
                for p, w in enumerate((L.attn_q, L.attn_k, L.attn_v, L.attn_o, L.ffn_gate, L.ffn_up, L.ffn_down)):
                    ctx.register(w, *cfg.proj_quant(li, p))
            ctx.register(model.token_embd, cfg.embd_type, 1)
            ctx.register(model.lm_head, cfg.head_type, cfg.head_interleave)
        self._layers = (_lib.zg_layer_weights * cfg.n_layers)()
        for i, L in enumerate(model.layers):
            self._layers[i] = _lib.zg_layer_weights(
                L.attn_q.ctypes.data, L.attn_k.ctypes.data, L.attn_v.ctypes.data, L.attn_o.ctypes.data,
                L.ffn_gate.ctypes.data, L.ffn_up.ctypes.data, L.ffn_down.ctypes.data,
                L.attn_norm.ctypes.data, L.ffn_norm.ctypes.data, L.q_norm.ctypes.data, L.k_norm.ctypes.data)
        d = _lib.zg_model_desc()
        d.n_layers, d.hidden, d.ffn = cfg.n_layers, cfg.hidden, cfg.ffn
        d.n_q_heads, d.n_kv_heads, d.head_dim = cfg.n_q_heads, cfg.n_kv_heads, cfg.head_dim
        d.vocab_padded, d.vocab_real, d.max_ctx = cfg.vocab_padded, cfg.vocab_real, cfg.max_ctx
        d.rms_eps, d.rope_theta = cfg.rms_eps, cfg.rope_theta
        d.lin_type, d.lin_interleave = cfg.lin_type, cfg.lin_interleave
        d.embd_type = cfg.embd_type
        d.head_type, d.head_interleave = cfg.head_type, cfg.head_interleave
        d.token_embd = model.token_embd.ctypes.data
        d.lm_head = model.lm_head.ctypes.data
        d.output_norm = model.output_norm.ctypes.data
        d.layers = self._layers
        d.device_pointers = 0
        if cfg.layer_quants is not None:
            self._quants = (_lib.zg_layer_quants * cfg.n_layers)()
            for i, lq in enumerate(cfg.layer_quants):
                for p, (t, il) in enumerate(lq):
                    self._quants[i].type[p], self._quants[i].interleave[p] = t, il
            d.layer_quants = self._quants
        self._desc = d
        h = C.c_void_p()
        ctx.check(ctx.lib.zg_model_create(ctx.h, C.byref(d), C.byref(h)))
        self.h = h

    @classmethod
    def from_smodel(cls, ctx: Context, sm, max_ctx: int | None = None) -> "GpuModel":
        """A packed ``.smodel`` (zero_amd.smodel.SModel): every quantized
        tensor enters the registry with its SIDX layout
        (zg_smodel_register_all), then the dense Qwen3 graph is built over
        those registered views."""
        model = sm.to_model(max_ctx)
        sm.register_all(ctx)
        return cls(ctx, model, register=False)

    def close(self):
        if getattr(self, "h", None):
            self.ctx.lib.zg_model_destroy(self.h)
            self.h = None

    def reset(self):
        """New sequence (zg_model_reset); also clears the non-finite latch."""
        self.ctx.lib.zg_model_reset(self.h)

    def first_nonfinite(self) -> str:
        """The non-finite latch (zg_model_first_nonfinite): the first stage
        that held a NaN/Inf in a failed call, e.g. "L03 attn_out n1 i0"; ""
        when nothing is latched."""
        buf = C.create_string_buffer(32)
        n = self.ctx.lib.zg_model_first_nonfinite(self.h, buf, 32)
        return buf.raw[:n].decode()

    def _raise(self, rc, tok):
        if rc == _lib.ZG_ERR_ARGMAX_IN_PADDING:
            raise ArgmaxInPaddingRegion(rc, self.ctx.last_error(), tok)
        if rc == _lib.ZG_ERR_NONFINITE_LOGITS:
            raise NonFiniteLogits(rc, self.ctx.last_error())
        if rc != _lib.ZG_OK:
            raise ZgError(rc, self.ctx.last_error())

    def step(self, token: int, pos: int, want_hidden=False, want_logits=False):
        """One token through all layers and the LM head.  Returns
        (next_token, max_logit, hidden or None, logits or None)."""
        cfg = self.cfg
        hid = np.empty(cfg.hidden, np.float32) if want_hidden else None
        lg = np.empty(cfg.vocab_padded, np.float32) if want_logits else None
        tok = C.c_uint32()
        mv = C.c_float()
        rc = self.ctx.lib.zg_model_step(self.h, token, pos, hid.ctypes.data if hid is not None else None,
                                        lg.ctypes.data if lg is not None else None, C.byref(tok), C.byref(mv))
        self._raise(rc, int(tok.value))
        return int(tok.value), float(mv.value), hid, lg

    def prefill(self, tokens: np.ndarray, pos0: int = 0, want_hidden: bool = False):
        """Batched prefill (zg_model_prefill): tokens at positions
        pos0..pos0+n-1 through Q8_0-activation GEMMs, then the LM head on the
        last row.  Returns (next_token, max_logit, last hidden or None)."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        hid = np.empty(self.cfg.hidden, np.float32) if want_hidden else None
        tok = C.c_uint32()
        mv = C.c_float()
        rc = self.ctx.lib.zg_model_prefill(self.h, t.ctypes.data, t.size, pos0,
                                           hid.ctypes.data if hid is not None else None, C.byref(tok), C.byref(mv))
        self._raise(rc, int(tok.value))
        return int(tok.value), float(mv.value), hid

    def generate(self, prompt: np.ndarray, n_gen: int, batched_prefill: bool = False, eager: bool = False):
        """Prefill `prompt` (token by token, or batched with Q8_0-activation
        GEMMs), then n_gen greedy tokens.  eager: launch each token's kernels
        directly instead of replaying the step graph (per-dispatch profiling).
        Returns (tokens, prefill_seconds, generation_seconds)."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(n_gen, np.uint32)
        t_pre = C.c_double()
        t_gen = C.c_double()
        flags = (_lib.ZG_GEN_BATCHED_PREFILL if batched_prefill else 0) | (_lib.ZG_GEN_EAGER if eager else 0)
        rc = self.ctx.lib.zg_model_generate_ex(self.h, p.ctypes.data, p.size, n_gen, flags, out.ctypes.data,
                                               C.byref(t_pre), C.byref(t_gen))
        self._raise(rc, -1)
        return out, float(t_pre.value), float(t_gen.value)
