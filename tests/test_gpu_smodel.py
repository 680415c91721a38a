"""A packed .smodel through the GPU path: the tiny Qwen3 artifacts that the
reference packer wrote (tests/golden/tiny_qwen3_v2*.smodel: Q4_0X4 and
Q8_0X4 layer linears; tiny_qwen3_v1.smodel: the packer's default v1
layout, plain Q4_0 rows) are read by
zg_smodel_open, registered by zg_smodel_register_all with its SIDX
layouts, and decoded by the HIP model; the oracle decodes the same tensor
views on the CPU.

Bar: hidden state and logits within rel 1e-3 at every step, identical greedy
tokens; a registered X4 tensor through zg_linear within rel 1e-4 of the
oracle's f64 row dot."""
from pathlib import Path

import numpy as np
import pytest

from zero_amd import synth
from zero_amd.model import GpuModel
from zero_amd.smodel import SModel

pytestmark = pytest.mark.gpu
FIX = Path(__file__).parent / "golden" / "tiny_qwen3_v2.smodel"
REL_TOL = 1e-3


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def test_register_all_layouts(ctx, zo):
    sm = SModel(FIX)
    sm.register_all(ctx)
    try:
        quant = [t for t in sm.tensors if t.ggml_type != 0]
        assert ctx.registered_count() == len(quant) == 16
        for t in quant:
            assert ctx.group_of(t.data) == t.interleave, t.name
        rng = np.random.default_rng(11)
        for name in ("blk.0.attn_q.weight", "blk.1.ffn_down.weight", "output.weight"):
            t = sm[name]
            rows, k = t.shape
            x = rng.standard_normal(k).astype(np.float32)
            y = np.zeros(rows, np.float32)
            ctx.linear_dispatch(x, t.data, y, k, rows, t.ggml_type)
            ref = zo.linear_f64(x, t.data, k, rows, t.ggml_type, t.interleave)
            print(f"{name}: rel err {rel_err(y, ref):.2e}")
            assert rel_err(y, ref) <= 1e-4, name
    finally:
        ctx.clear()


@pytest.mark.parametrize("stem", ["tiny_qwen3_v2", "tiny_qwen3_v2_q8", "tiny_qwen3_v1"])
def test_smodel_decode_matches_oracle(ctx, zo, stem):
    sm = SModel(FIX.parent / f"{stem}.smodel")
    gm = GpuModel.from_smodel(ctx, sm, max_ctx=64)
    om = zo.OracleModel(gm.model)
    try:
        tok = 7
        worst_h = worst_l = 0.0
        for pos in range(40):
            nxt, _, hid, lg = gm.step(tok, pos, want_hidden=True, want_logits=True)
            h_ref = om.forward(tok, pos)
            rc, t_ref, _, lg_ref = om.lm_head()
            assert rc == 0
            worst_h, worst_l = max(worst_h, rel_err(hid, h_ref)), max(worst_l, rel_err(lg, lg_ref))
            assert nxt == t_ref, pos
            tok = nxt
        print(f"packed tiny Qwen3: worst hidden rel err {worst_h:.2e}, worst logits rel err {worst_l:.2e}")
        assert worst_h <= REL_TOL and worst_l <= REL_TOL
        prompt = synth.prompt(9, 12, gm.cfg.vocab_real)
        toks, _, _ = gm.generate(prompt, 48)
        assert np.array_equal(toks, om.generate(prompt, 48))
        # the batched prefill on the packed weights (Q4_0X4 or Q8_0X4 GEMMs)
        toks_b, _, _ = gm.generate(prompt, 40, batched_prefill=True)
        assert np.array_equal(toks_b, om.generate_batched(prompt, 40))
    finally:
        om.close()
        gm.close()
        ctx.clear()
