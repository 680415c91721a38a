"""Seeded synthetic tensors in the reference's block formats.

Weights are generated directly as block bytes with the distributions of the
benchmark workloads: fp16 scale d = RNE(|N(0, 0.02)| / 8) per 32-element
block, Q4_0 nibbles uniform 0..15 (value q - 8), Q8_0 int8 uniform
-127..127.  .smodel-v2 X4 tensors are the plain tensors permuted exactly as
the packer writes them (tools/silicatepack.py:982-1029).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

Q4_0, Q8_0, Q4K, Q6K = 2, 8, 12, 14
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4K: 144, Q6K: 210}
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4K: 256, Q6K: 256}


def _scales(rng: np.random.Generator, n: int, sigma: float = 0.02) -> np.ndarray:
    """fp16 bit patterns of |N(0, sigma)| / 8 (round to nearest even)."""
    return (np.abs(rng.standard_normal(n, dtype=np.float64) * sigma) / 8.0).astype(np.float16).view(np.uint16)


def plain_q4_0(rng, rows: int, k: int, sigma: float = 0.02) -> np.ndarray:
    nb = k // 32
    blk = np.empty((rows * nb, 18), np.uint8)
    blk[:, :2] = _scales(rng, rows * nb, sigma).view(np.uint8).reshape(-1, 2)
    blk[:, 2:] = rng.integers(0, 256, size=(rows * nb, 16), dtype=np.uint8)
    return blk.reshape(-1)


def plain_q8_0(rng, rows: int, k: int, sigma: float = 0.02) -> np.ndarray:
    nb = k // 32
    blk = np.empty((rows * nb, 34), np.uint8)
    blk[:, :2] = _scales(rng, rows * nb, sigma).view(np.uint8).reshape(-1, 2)
    blk[:, 2:] = rng.integers(-127, 128, size=(rows * nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    return blk.reshape(-1)


def interleave_x4(plain: np.ndarray, rows: int, k: int, quant: int) -> np.ndarray:
    """Plain row-major blocks -> X4 group-blocks (d0 d1 d2 d3, qs0..qs3)."""
    bb = BLOCK_BYTES[quant]
    nb = k // 32
    p = plain.reshape(rows // 4, 4, nb, bb)
    d = p[..., :2].transpose(0, 2, 1, 3).reshape(rows // 4, nb, 8)
    q = p[..., 2:].transpose(0, 2, 1, 3).reshape(rows // 4, nb, 4 * (bb - 2))
    return np.ascontiguousarray(np.concatenate([d, q], axis=2)).reshape(-1)


def deinterleave_x4(x4: np.ndarray, rows: int, k: int, quant: int) -> np.ndarray:
    bb = BLOCK_BYTES[quant]
    nb = k // 32
    g = x4.reshape(rows // 4, nb, 4 * bb)
    d = g[..., :8].reshape(rows // 4, nb, 4, 2).transpose(0, 2, 1, 3)
    q = g[..., 8:].reshape(rows // 4, nb, 4, bb - 2).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(np.concatenate([d, q], axis=3)).reshape(-1)


def q4k(rng, rows: int, k: int) -> np.ndarray:
    """Random Q4_K superblocks: fp16 d, dmin ~ |N(0,0.02)|/8, random 6-bit
    scale/min bytes, random nibbles."""
    nb = k // 256
    blk = rng.integers(0, 256, size=(rows * nb, 144), dtype=np.uint8)
    blk[:, 0:2] = _scales(rng, rows * nb).view(np.uint8).reshape(-1, 2)
    blk[:, 2:4] = _scales(rng, rows * nb).view(np.uint8).reshape(-1, 2)
    return blk.reshape(-1)


def q6k(rng, rows: int, k: int) -> np.ndarray:
    """Random Q6_K superblocks: random ql/qh, int8 scales in [-64, 63],
    fp16 d ~ |N(0,0.02)|/8."""
    nb = k // 256
    blk = rng.integers(0, 256, size=(rows * nb, 210), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-64, 64, size=(rows * nb, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
    blk[:, 208:210] = _scales(rng, rows * nb).view(np.uint8).reshape(-1, 2)
    return blk.reshape(-1)


def weight(rng, quant: int, rows: int, k: int, interleave: int = 1) -> np.ndarray:
    if quant == Q4_0:
        w = plain_q4_0(rng, rows, k)
    elif quant == Q8_0:
        w = plain_q8_0(rng, rows, k)
    elif quant == Q4K:
        return q4k(rng, rows, k)
    elif quant == Q6K:
        return q6k(rng, rows, k)
    else:
        raise ValueError(quant)
    return interleave_x4(w, rows, k, quant) if interleave == 4 else w


def x4_split(w_x4, rows: int, k: int, quant: int) -> np.ndarray:
    """X4 group-blocks to split-scale X4 groups (interleave 5, the model's
    device layout): per group of 4 rows, the nb blocks' quants
    [block][row][qb bytes], then their fp16 scales [block][row]."""
    qb = 16 if quant == Q4_0 else 32
    gb, nb = 8 + 4 * qb, k // 32
    a = np.asarray(w_x4, np.uint8).reshape(rows // 4, nb, gb)
    q = a[:, :, 8:].reshape(rows // 4, nb * 4 * qb)
    d = a[:, :, :8].reshape(rows // 4, nb * 8)
    return np.ascontiguousarray(np.concatenate([q, d], axis=1).reshape(-1))


def activations(rng, *shape) -> np.ndarray:
    return rng.standard_normal(shape, dtype=np.float32)


# ---------------------------------------------------------------------------
# Qwen3-shaped random-init model
# ---------------------------------------------------------------------------

@dataclass
class ModelConfig:
    n_layers: int = 28
    hidden: int = 2048
    ffn: int = 6144
    n_q_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    vocab_padded: int = 151_936
    vocab_real: int = 151_643
    max_ctx: int = 384
    rms_eps: float = 1e-6
    rope_theta: float = 1e6
    lin_type: int = Q4_0
    embd_type: int = Q8_0
    head_type: int = Q8_0
    lin_interleave: int = 4   # 4: Q4_0X4/Q8_0X4 layer linears (.smodel-v2); 1: plain rows (v1, GGUF)
    head_interleave: int = 4
    # per layer, (type, interleave) of Q, K, V, O, gate, up, down (the
    # per-layer arrays of ForwardPassDispatch); None: lin_type / lin_interleave
    layer_quants: tuple = None

    def proj_quant(self, layer: int, p: int) -> tuple:
        if self.layer_quants is None:
            return self.lin_type, self.lin_interleave
        return tuple(self.layer_quants[layer][p])

    def proj_shapes(self) -> tuple:
        """(rows, in_dim) of Q, K, V, O, gate, up, down."""
        H, F = self.hidden, self.ffn
        return ((self.q_dim, H), (self.kv_dim, H), (self.kv_dim, H), (H, self.q_dim), (F, H), (F, H), (H, F))

    @property
    def q_dim(self):
        return self.n_q_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    def weight_bytes_per_token(self) -> int:
        """Weight bytes one decode step streams (layers + LM head + one
        embedding row)."""
        lin = 0.0
        for layer in range(self.n_layers):
            for p, (rows, k) in enumerate(self.proj_shapes()):
                t = self.proj_quant(layer, p)[0]
                lin += rows * k * BLOCK_BYTES[t] / BLOCK_ELEMS[t]
        head = self.vocab_padded * self.hidden * BLOCK_BYTES[self.head_type] / BLOCK_ELEMS[self.head_type]
        embd_row = self.hidden * BLOCK_BYTES[self.embd_type] / BLOCK_ELEMS[self.embd_type]
        return int(lin + head + embd_row)


QWEN3_1_7B = ModelConfig()


@dataclass
class Layer:
    attn_q: np.ndarray
    attn_k: np.ndarray
    attn_v: np.ndarray
    attn_o: np.ndarray
    ffn_gate: np.ndarray
    ffn_up: np.ndarray
    ffn_down: np.ndarray
    attn_norm: np.ndarray
    ffn_norm: np.ndarray
    q_norm: np.ndarray
    k_norm: np.ndarray


@dataclass
class RandomModel:
    cfg: ModelConfig
    layers: list = field(default_factory=list)
    token_embd: np.ndarray = None
    lm_head: np.ndarray = None
    output_norm: np.ndarray = None


def random_model(cfg: ModelConfig, seed: int = 0) -> RandomModel:
    """Random-init weights of the given shape: layer linears and LM head in
    the configured layouts (X4 by default), plain token_embd, the LM head's
    padding rows (vocab_real..vocab_padded) zeroed so that an argmax can
    never land there, fp32 norm gains 1 + 0.05 N(0,1)."""
    rng = np.random.default_rng(seed)
    H = cfg.hidden

    def gain(n):
        return (1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32)

    m = RandomModel(cfg)
    names = ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_gate", "ffn_up", "ffn_down")
    for layer in range(cfg.n_layers):
        ws = {}
        for p, (name, (rows, k)) in enumerate(zip(names, cfg.proj_shapes())):
            qt, il = cfg.proj_quant(layer, p)
            ws[name] = weight(rng, qt, rows, k, il)
        m.layers.append(Layer(**ws, attn_norm=gain(H), ffn_norm=gain(H), q_norm=gain(cfg.head_dim),
                              k_norm=gain(cfg.head_dim)))
    m.token_embd = weight(rng, cfg.embd_type, cfg.vocab_padded, H, 1)
    head_plain = weight(rng, cfg.head_type, cfg.vocab_padded, H, 1)
    bb, nb = BLOCK_BYTES[cfg.head_type], H // BLOCK_ELEMS[cfg.head_type]
    head_plain.reshape(cfg.vocab_padded, nb * bb)[cfg.vocab_real:] = 0
    m.lm_head = interleave_x4(head_plain, cfg.vocab_padded, H, cfg.head_type) if cfg.head_interleave == 4 else head_plain
    m.output_norm = gain(H)
    return m


def q4_k_m_layers(n_layers: int) -> tuple:
    """Per-layer projection quants in the pattern of a GGUF Q4_K_M
    checkpoint (the reference's default dispatch, forward_pass.rs:209-224,
    is Q4_K everywhere; such files carry Q6_K attn_v and ffn_down on the
    first and last eighth of the layers and every third layer between)."""
    out = []
    for i in range(n_layers):
        more = i < n_layers // 8 or i >= 7 * n_layers // 8 or (i - n_layers // 8) % 3 == 2
        t = [Q4K] * 7
        if more:
            t[2] = t[6] = Q6K
        out.append(tuple((q, 1) for q in t))
    return tuple(out)


def prompt(seed: int, n: int, vocab_real: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, vocab_real, size=n, dtype=np.int64).astype(np.uint32)
