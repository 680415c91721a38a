"""Pins the oracle's non-finite latch (finite_diag + record_first_nonfinite,
kernel/src/inference_avx512.rs:88-131, 233-275; scans at :1896, 1946-1947,
1981-1982).

The latch text: for hand-made vectors, "L{layer:02} {stage} n{nan} i{inf}"
carries the FIRST non-finite element's flags (a latch that reported "any
NaN" or "any Inf" fails the mixed cases), -Inf counts as Inf, and the text
is cut at 32 bytes.

The stages: NaN fp16 scales planted in single weight blocks of a tiny
model, where the first stage to hold a NaN follows from the structure:

* a token_embd row: rmsnorm of a row holding NaN is NaN everywhere, so
  attn_norm_in of layer 0 trips, then the softmax fails (the forward
  returns the attention error, -4);
* one row of attn_o or ffn_down: that element of the projection output is
  NaN, so attn_out / mlp_out trips at that layer, before the residuals;
* the latch is one-shot: a later failure keeps the first text;
* attn_k: the scores go NaN and the softmax fails before any scanned stage
  holds a non-finite value, so nothing is latched.

(An infinite scale is no use here: the reference multiplies each weight by
its block scale before the dot, so inf * 0 makes NaN.)
"""
import numpy as np
import pytest

from poison import NAN16, poison_embedding, poison_proj
from zero_amd import synth

CFG = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                        vocab_padded=512, vocab_real=500, max_ctx=16, lin_interleave=1, head_interleave=1)


def fresh(seed=11):
    return synth.random_model(CFG, seed=seed)


def test_clean_model_latches_nothing(zo):
    om = zo.OracleModel(fresh())
    for pos, tok in enumerate((3, 9, 27)):
        assert om.forward_status(tok, pos) == 0
    assert om.first_nonfinite() == ""
    om.close()


def test_embedding_nan_trips_attn_norm_in(zo):
    m = fresh()
    poison_embedding(m, 9, 2, NAN16)
    om = zo.OracleModel(m)
    assert om.forward_status(3, 0) == 0
    assert om.first_nonfinite() == ""
    assert om.forward_status(9, 1) == -4  # the softmax sees the NaN key
    assert om.first_nonfinite() == "L00 attn_norm_in n1 i0"
    om.close()


@pytest.mark.parametrize("buf,want", [
    ([1.0, 2.0, np.inf, np.nan], "L03 attn_out n0 i1"),
    ([1.0, np.nan, np.inf], "L03 attn_out n1 i0"),
    ([-np.inf, np.nan], "L03 attn_out n0 i1"),
    ([0.0, -0.0, 3.4e38], ""),
])
def test_latch_text(zo, buf, want):
    assert zo.nonfinite_text(np.array(buf, np.float32), 3, "attn_out") == want


def test_latch_text_cap(zo):
    t = zo.nonfinite_text(np.array([np.nan], np.float32), 12, "post_attn_residual_and_more")
    assert t == "L12 post_attn_residual_and_more "[:32] and len(t) == 32


@pytest.mark.parametrize("layer,name,want", [
    (1, "attn_o", "L01 attn_out n1 i0"),
    (0, "attn_o", "L00 attn_out n1 i0"),
    (1, "ffn_down", "L01 mlp_out n1 i0"),
    (0, "ffn_down", "L00 mlp_out n1 i0"),
])
def test_projection_row_trips_its_stage(zo, layer, name, want):
    m = fresh()
    poison_proj(m, layer, name, 5, 3, NAN16)
    om = zo.OracleModel(m)
    om.forward_status(7, 0)
    assert om.first_nonfinite() == want
    om.close()


def test_latch_is_one_shot(zo):
    m = fresh()
    poison_proj(m, 1, "ffn_down", 5, 3, NAN16)
    poison_embedding(m, 9, 0, NAN16)
    om = zo.OracleModel(m)
    om.forward_status(7, 0)
    assert om.first_nonfinite() == "L01 mlp_out n1 i0"
    om.forward_status(9, 1)  # would trip L00 attn_norm_in on a fresh latch
    assert om.first_nonfinite() == "L01 mlp_out n1 i0"
    om.close()


def test_attention_failure_before_any_stage(zo):
    m = fresh()
    poison_proj(m, 0, "attn_k", 0, 0, NAN16)
    om = zo.OracleModel(m)
    assert om.forward_status(7, 0) == -4
    assert om.first_nonfinite() == ""
    om.close()
