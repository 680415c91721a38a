"""Native ``.smodel`` containers (SilicatePack SILM + SIDX) over the C ABI.

``SModel`` validates a packed artifact with zg_smodel_open, which restates
the reference loader's checks (kernel/src/model_loader.rs: smodel_info
:599-659, smodel_native_tensor_index :380-575), and exposes the header, the
SIDX model config and every tensor as a zero-copy numpy view of the file.
``SModel.to_model()`` resolves the dense Qwen3 tensors by the runtime names
the packer writes (tools/silicatepack.py:634-661) into the same model
object ``GpuModel`` takes for random-init weights, with the reference's
shape checks (kernel/src/inference.rs:985-1050, main.rs:2745-2760).
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os
from dataclasses import dataclass

import numpy as np

from . import _lib
from .ops import ZgError
from .synth import BLOCK_BYTES, BLOCK_ELEMS, Layer, ModelConfig, RandomModel

# the seven layer projections in ZG_PROJ_* order: runtime tensor names and
# the model object's fields
PROJ_NAMES = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
LAYER_FIELDS = ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_gate", "ffn_up", "ffn_down")

NONE_U32 = 0xFFFF_FFFF  # SMODEL_NONE_U32 (model_loader.rs:76)
ARCH_QWEN3 = 1
F32 = 0


class LoadError(ZgError):
    """LoadError (kernel/src/model_loader.rs:152-160)."""


class MagicMismatch(LoadError):
    pass


class UnsupportedFormat(LoadError):
    pass


class InvalidContainer(LoadError):
    pass


_ERRORS = {
    _lib.ZG_ERR_MAGIC_MISMATCH: MagicMismatch,
    _lib.ZG_ERR_UNSUPPORTED_FORMAT: UnsupportedFormat,
    _lib.ZG_ERR_INVALID_CONTAINER: InvalidContainer,
}


@dataclass(frozen=True)
class Tensor:
    """One SIDX entry; ``data`` is a uint8 view into the container."""

    name: str
    dtype: int        # SIDX dtype id as stored (100 Q4_0X4, 101 Q8_0X4, else GgmlType)
    ggml_type: int
    interleave: int
    shape: tuple      # source order: shape[0] = output rows
    payload_offset: int
    data: np.ndarray

    @property
    def byte_len(self) -> int:
        return self.data.nbytes


def _raise(rc: int, what: str):
    if rc == _lib.ZG_OK:
        return
    raise _ERRORS.get(rc, ZgError)(rc, what)


class SModel:
    """A validated ``.smodel`` image (a path, bytes or a uint8 array).

    A path is memory-mapped read-only; the image must stay alive while any
    tensor view or registered weight uses it, which this object ensures by
    holding it."""

    def __init__(self, source):
        if isinstance(source, (str, os.PathLike)):
            img = np.memmap(source, dtype=np.uint8, mode="r")
        elif isinstance(source, np.ndarray):
            img = np.ascontiguousarray(source.reshape(-1).view(np.uint8))
        else:
            img = np.frombuffer(bytes(source), dtype=np.uint8)
        self.image = img
        self._lib = _lib.load()
        h = C.c_void_p()
        # an empty image still needs a valid address for the length check
        base = img.ctypes.data if img.size else C.addressof(C.c_uint8())
        _raise(self._lib.zg_smodel_open(base, img.size, C.byref(h)), "zg_smodel_open")
        self.h = h
        info = _lib.zg_smodel_info()
        _raise(self._lib.zg_smodel_get_info(h, C.byref(info)), "zg_smodel_get_info")
        self.info = info
        self.tensors = [self._tensor(i) for i in range(info.tensor_count)]
        self._by_name = {t.name: t for t in self.tensors}

    def _tensor(self, i: int) -> Tensor:
        t = _lib.zg_smodel_tensor()
        _raise(self._lib.zg_smodel_get_tensor(self.h, i, C.byref(t)), "zg_smodel_get_tensor")
        name = C.string_at(t.name, t.name_len).decode("utf-8") if t.name_len else ""
        off = int(self.info.payload_offset) + int(t.payload_offset)
        return Tensor(name, int(t.dtype), int(t.ggml_type), int(t.interleave), tuple(int(d) for d in t.dims[:t.rank]),
                      int(t.payload_offset), self.image[off:off + int(t.byte_len)])

    def close(self):
        if getattr(self, "h", None):
            self._lib.zg_smodel_close(self.h)
            self.h = None

    def __del__(self):  # pragma: no cover - interpreter teardown order
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __contains__(self, name: str) -> bool:
        return name in self._by_name

    def __getitem__(self, name: str) -> Tensor:
        return self._by_name[name]

    def find(self, name: str) -> Tensor:
        """zg_smodel_find: the entry the C reader resolves for ``name``."""
        t = _lib.zg_smodel_tensor()
        _raise(self._lib.zg_smodel_find(self.h, name.encode(), C.byref(t)), f"tensor {name!r} not in container")
        return self._by_name[C.string_at(t.name, t.name_len).decode("utf-8")]

    def register_all(self, ctx) -> None:
        """zg_smodel_register_all: upload and register every quantized
        tensor with its row layout (weight_layout registration of the
        loader, model_loader.rs:527-552)."""
        ctx.check(self._lib.zg_smodel_register_all(ctx.h, self.h))
        ctx._keep[self.image.ctypes.data] = self.image

    # ---- model view ---------------------------------------------------
    def config(self, max_ctx: int | None = None) -> ModelConfig:
        """ModelConfig from the SIDX model config and the tensor types."""
        i = self.info
        if i.architecture_id != ARCH_QWEN3:
            raise UnsupportedFormat(_lib.ZG_ERR_UNSUPPORTED_FORMAT,
                                    f"architecture id {i.architecture_id}: only dense Qwen3 (1) runs here")
        need = ("block_count", "embedding_length", "feed_forward_length", "head_count", "head_count_kv",
                "key_length")
        for f in need:
            if getattr(i, f) in (0, NONE_U32):
                raise InvalidContainer(_lib.ZG_ERR_INVALID_CONTAINER, f"model config field {f} missing")
        if i.value_length not in (NONE_U32, i.key_length):
            raise UnsupportedFormat(_lib.ZG_ERR_UNSUPPORTED_FORMAT, "value_length != key_length")
        for name in ("token_embd.weight", "output.weight", "output_norm.weight", "blk.0.attn_q.weight"):
            if name not in self:
                raise InvalidContainer(_lib.ZG_ERR_INVALID_CONTAINER, f"{name} missing")
        head = self["output.weight"]
        vocab_padded = head.shape[0]
        vocab_real = vocab_padded if i.vocab_size == NONE_U32 else int(i.vocab_size)
        ctx_len = int(i.context_length) if i.context_length != NONE_U32 else 4096
        return ModelConfig(
            n_layers=int(i.block_count), hidden=int(i.embedding_length), ffn=int(i.feed_forward_length),
            n_q_heads=int(i.head_count), n_kv_heads=int(i.head_count_kv), head_dim=int(i.key_length),
            vocab_padded=vocab_padded, vocab_real=vocab_real,
            max_ctx=min(ctx_len, max_ctx) if max_ctx else ctx_len,
            rms_eps=float(i.layer_norm_rms_epsilon), rope_theta=float(i.rope_freq_base),
            lin_type=self["blk.0.attn_q.weight"].ggml_type, embd_type=self["token_embd.weight"].ggml_type,
            head_type=head.ggml_type, lin_interleave=self["blk.0.attn_q.weight"].interleave,
            head_interleave=head.interleave)

    def _quant(self, name: str, rows: int, cols: int, qtype: int, interleave: int) -> np.ndarray:
        if name not in self:
            raise InvalidContainer(_lib.ZG_ERR_INVALID_CONTAINER, f"{name} missing")
        t = self[name]
        if t.ggml_type != qtype or t.interleave != interleave:
            raise UnsupportedFormat(_lib.ZG_ERR_UNSUPPORTED_FORMAT,
                                    f"{name}: type {t.ggml_type}/x{t.interleave}, expected {qtype}/x{interleave}")
        if t.shape != (rows, cols) or cols % BLOCK_ELEMS[qtype] or \
                t.byte_len != rows * (cols // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]:
            raise InvalidContainer(_lib.ZG_ERR_INVALID_CONTAINER,
                                   f"{name}: shape {t.shape} / {t.byte_len} B, expected ({rows}, {cols})")
        return t.data

    def _f32(self, name: str, n: int) -> np.ndarray:
        if name not in self:
            raise InvalidContainer(_lib.ZG_ERR_INVALID_CONTAINER, f"{name} missing")
        t = self[name]
        if t.ggml_type != F32 or t.shape != (n,) or t.byte_len != 4 * n:
            raise InvalidContainer(_lib.ZG_ERR_INVALID_CONTAINER, f"{name}: expected F32 [{n}]")
        return t.data.view(np.float32)

    def to_model(self, max_ctx: int | None = None) -> RandomModel:
        """The dense Qwen3 tensors as the model object GpuModel and the
        oracle take: each layer projection in its own quant type and layout
        (X4 in a v2 artifact, plain rows in v1), plain token embedding, the
        LM head in its own layout, F32 norms.  Arrays are views of the
        file."""
        cfg = self.config(max_ctx)
        H, hd = cfg.hidden, cfg.head_dim
        # ForwardPassDispatch's per-layer quants: each projection's own type
        # and layout from the file (a per-layer table only when they differ)
        quants = []
        for b in range(cfg.n_layers):
            row = []
            for name in PROJ_NAMES:
                key = f"blk.{b}.{name}.weight"
                if key not in self:
                    raise InvalidContainer(_lib.ZG_ERR_INVALID_CONTAINER, f"{key} missing")
                row.append((self[key].ggml_type, self[key].interleave))
            quants.append(tuple(row))
        if any(q != (cfg.lin_type, cfg.lin_interleave) for row in quants for q in row):
            cfg = dataclasses.replace(cfg, layer_quants=tuple(quants))
        m = RandomModel(cfg)
        for b in range(cfg.n_layers):
            p = f"blk.{b}."
            w = {field: self._quant(p + name + ".weight", rows, k, *cfg.proj_quant(b, i))
                 for i, (field, name, (rows, k)) in enumerate(zip(LAYER_FIELDS, PROJ_NAMES, cfg.proj_shapes()))}
            m.layers.append(Layer(
                **w, attn_norm=self._f32(p + "attn_norm.weight", H), ffn_norm=self._f32(p + "ffn_norm.weight", H),
                q_norm=self._f32(p + "attn_q_norm.weight", hd), k_norm=self._f32(p + "attn_k_norm.weight", hd)))
        # one row per token id the LM head can emit
        m.token_embd = self._quant("token_embd.weight", cfg.vocab_padded, H, cfg.embd_type, 1)
        m.lm_head = self._quant("output.weight", cfg.vocab_padded, H, cfg.head_type, cfg.head_interleave)
        m.output_norm = self._f32("output_norm.weight", H)
        return m
