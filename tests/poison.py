"""Writes a non-finite scale into one weight block, for the non-finite latch
tests.  The block's fp16 d sits at byte 0 of a Q4_0, Q8_0 or Q4_K block
(block_q4_K: d, dmin, scales, qs) and at byte 208 of a Q6_K block
(block_q6_K: ql, qh, scales, d), in the plain layout; X4 tensors are
de-interleaved, patched and interleaved back."""
import numpy as np

from zero_amd import synth

NAN16 = 0x7E00


def poison_block(w: np.ndarray, qt: int, il: int, rows: int, k: int, row: int, block: int, d_bits: int) -> None:
    assert il == 1 or qt in (synth.Q4_0, synth.Q8_0)
    plain = synth.deinterleave_x4(w, rows, k, qt) if il == 4 else w
    bb, nb = synth.BLOCK_BYTES[qt], k // synth.BLOCK_ELEMS[qt]
    off = block * bb + (208 if qt == synth.Q6K else 0)
    v = plain.reshape(rows, nb * bb)
    v[row, off:off + 2] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
    if il == 4:
        w[...] = synth.interleave_x4(plain, rows, k, qt).reshape(w.shape)


def poison_proj(model, layer: int, name: str, row: int, block: int, d_bits: int) -> None:
    """Block `block` of row `row` of layer projection `name` (attn_q ...
    ffn_down) gets the fp16 scale d_bits."""
    cfg = model.cfg
    names = ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_gate", "ffn_up", "ffn_down")
    p = names.index(name)
    rows, k = cfg.proj_shapes()[p]
    qt, il = cfg.proj_quant(layer, p)
    poison_block(getattr(model.layers[layer], name), qt, il, rows, k, row, block, d_bits)


def poison_embedding(model, token: int, block: int, d_bits: int) -> None:
    cfg = model.cfg
    poison_block(model.token_embd, cfg.embd_type, 1, cfg.vocab_padded, cfg.hidden, token, block, d_bits)
