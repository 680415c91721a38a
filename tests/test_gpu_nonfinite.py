"""The decode path's non-finite latch against the oracle's restatement of
the reference's (finite_diag + record_first_nonfinite,
kernel/src/inference_avx512.rs:88-131, 233-275): NaN fp16 scales planted in
single weight blocks, the same failure through the greedy loop on both, and
the same latched text ("L{layer:02} {stage} n{0|1} i{0|1}") and failure kind
(the attention softmax failure, ZG_ERR_ATTENTION, or non-finite logits).

The models run the production kernels: Q4_0 X4 projections at hidden 2048
(fused strip GEMVs, the O GEMV that merges the attention splits) and a
Q4_K / Q6_K mix (the K-quant GEMVs).
"""
import numpy as np
import pytest

from poison import NAN16, poison_embedding, poison_proj
from zero_amd import _lib, synth
from zero_amd.model import GpuModel
from zero_amd.ops import ZgError

pytestmark = pytest.mark.gpu

X4 = synth.ModelConfig(n_layers=3, vocab_padded=4096, vocab_real=4000, max_ctx=64)
KQ = synth.ModelConfig(n_layers=3, vocab_padded=4096, vocab_real=4000, max_ctx=64, embd_type=synth.Q4K,
                       head_type=synth.Q6K, head_interleave=1, layer_quants=synth.q4_k_m_layers(3))
PROMPT = np.array([11, 22, 33, 44, 55, 66], np.uint32)


def oracle_run(om, prompt, n_gen):
    """The reference's caller loop, stopping at the first error: returns
    ("attention" | "logits" | None, latched text)."""
    for pos, t in enumerate(prompt):
        if om.forward_status(int(t), pos) == -4:
            return "attention", om.first_nonfinite()
    pos = len(prompt)
    for j in range(n_gen):
        rc, tok, _, _ = om.lm_head()
        if rc == -1:
            return "logits", om.first_nonfinite()
        assert rc == 0
        if j + 1 == n_gen:
            break
        if om.forward_status(tok, pos) == -4:
            return "attention", om.first_nonfinite()
        pos += 1
    return None, om.first_nonfinite()


def gpu_run(gm, prompt, n_gen, batched=False):
    try:
        gm.generate(prompt, n_gen, batched_prefill=batched)
    except ZgError as e:
        kind = {_lib.ZG_ERR_ATTENTION: "attention", _lib.ZG_ERR_NONFINITE_LOGITS: "logits"}[e.code]
        return kind, gm.first_nonfinite(), str(e)
    return None, gm.first_nonfinite(), ""


CASES = [
    # (config, what, layer, projection or token, row, block, expected text)
    ("x4", "embd", None, 33, None, 1, "L00 attn_norm_in n1 i0"),
    ("x4", "proj", 1, "attn_o", 5, 3, "L01 attn_out n1 i0"),
    ("x4", "proj", 2, "attn_o", 2000, 60, "L02 attn_out n1 i0"),
    ("x4", "proj", 0, "ffn_down", 7, 100, "L00 mlp_out n1 i0"),
    ("x4", "proj", 2, "ffn_down", 1, 0, "L02 mlp_out n1 i0"),
    ("x4", "proj", 0, "attn_k", 0, 0, ""),
    ("kq", "proj", 1, "attn_o", 9, 2, "L01 attn_out n1 i0"),
    ("kq", "proj", 2, "ffn_down", 3, 5, "L02 mlp_out n1 i0"),
    ("kq", "proj", 0, "ffn_down", 30, 1, "L00 mlp_out n1 i0"),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[1]}-{c[3]}-L{c[2]}" for c in CASES])
def test_latch_matches_oracle(ctx, zo, case):
    cfg_name, what, layer, target, row, block, want = case
    model = synth.random_model(X4 if cfg_name == "x4" else KQ, seed=4)
    if what == "embd":
        poison_embedding(model, target, block, NAN16)
    else:
        poison_proj(model, layer, target, row, block, NAN16)
    om = zo.OracleModel(model)
    with zo.Pool(8):
        ref_kind, ref_text = oracle_run(om, PROMPT, 4)
    om.close()
    assert ref_kind is not None and ref_text == want
    gm = GpuModel(ctx, model)
    kind, text, msg = gpu_run(gm, PROMPT, 4)
    print(f"{case}: {msg}")
    assert (kind, text) == (ref_kind, ref_text)
    if text:
        assert msg.endswith(" @" + text)
    gm.close()
    ctx.clear()


def test_latch_step_history_and_reset(ctx):
    """zg_model_step: the latch holds the first failure across calls, reset
    clears it, and a later step that fails on a row an earlier step wrote
    replays that row's step (its token kept from the earlier call)."""
    model = synth.random_model(X4, seed=4)
    poison_embedding(model, 99, 0, NAN16)
    gm = GpuModel(ctx, model)
    for pos, t in enumerate((11, 22, 33, 44)):
        gm.step(t, pos)
    assert gm.first_nonfinite() == ""
    with pytest.raises(ZgError) as ei:
        gm.step(99, 4)
    assert ei.value.code == _lib.ZG_ERR_ATTENTION
    assert gm.first_nonfinite() == "L00 attn_norm_in n1 i0"
    gm.reset()
    assert gm.first_nonfinite() == ""
    with pytest.raises(ZgError) as ei:
        gm.step(55, 5)  # attends to row 4
    assert ei.value.code == _lib.ZG_ERR_ATTENTION
    assert gm.first_nonfinite() == "L00 attn_norm_in n1 i0"
    # a clean sequence after a reset latches nothing
    gm.reset()
    for pos, t in enumerate((11, 22, 33)):
        gm.step(t, pos)
    assert gm.first_nonfinite() == ""
    gm.close()
    ctx.clear()


def test_latch_names_batched_prefill_row(ctx):
    """Rows written by the batched prefill are named, not replayed: a NaN
    scale in layer 1's attn_k row 0 makes K head 0 NaN after the QK-norm in
    every prompt row, and the prefill attention fails at layer 1."""
    model = synth.random_model(X4, seed=4)
    poison_proj(model, 1, "attn_k", 0, 0, NAN16)
    gm = GpuModel(ctx, model)
    kind, text, msg = gpu_run(gm, PROMPT, 3, batched=True)
    print(msg)
    assert (kind, text) == ("attention", "L01 k_cache[0] n1 i0")
    gm.close()
    ctx.clear()


def test_clean_generate_latches_nothing(ctx):
    model = synth.random_model(X4, seed=4)
    gm = GpuModel(ctx, model)
    gm.generate(PROMPT, 4)
    gm.generate(PROMPT, 4, batched_prefill=True)
    assert gm.first_nonfinite() == ""
    gm.close()
    ctx.clear()
