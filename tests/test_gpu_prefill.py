"""GPU parity of the batched prefill (zg_model_prefill, zg_model_generate_ex
with ZG_GEN_BATCHED_PREFILL) against the oracle's zo_model_prefill_q8: the
prompt rows go through rmsnorm, Q8_0 activation quantization and the int8
MFMA GEMMs, with the decode step's QK-norm, RoPE, causal attention and
SwiGLU per row.

Bar: the last row's hidden state and the next token's logits within rel
1e-3 of the oracle, identical greedy tokens after the prefill; chunked calls
(pos0 > 0) bit-identical to one call; at the Qwen3-1.7B shape, within the
activation-quantization distance of the token-by-token pass."""
import numpy as np
import pytest

from zero_amd import _lib, synth
from zero_amd.model import GpuModel
from zero_amd.ops import ZgError

pytestmark = pytest.mark.gpu
REL_TOL = 1e-3


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


TINY = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                         vocab_padded=1024, vocab_real=1000, max_ctx=160)


@pytest.fixture(scope="module")
def tiny():
    return synth.random_model(TINY, seed=8)


@pytest.mark.parametrize("n", [1, 5, 64, 150])
def test_prefill_matches_oracle(ctx, zo, tiny, n):
    gm = GpuModel(ctx, tiny)
    om = zo.OracleModel(tiny)
    try:
        prompt = synth.prompt(20 + n, n, TINY.vocab_real)
        tok, mv, hid = gm.prefill(prompt, want_hidden=True)
        h_ref = om.prefill_q8(prompt)
        rc, t_ref, m_ref, lg_ref = om.lm_head()
        assert rc == 0
        print(f"n={n}: hidden rel err {rel_err(hid, h_ref):.2e}")
        assert rel_err(hid, h_ref) <= REL_TOL
        assert tok == t_ref and abs(mv - m_ref) <= REL_TOL * abs(m_ref)
        # decoding continues from the prefilled cache
        pos = n
        for _ in range(min(8, TINY.max_ctx - n)):
            nxt, _, h2, lg = gm.step(tok, pos, want_hidden=True, want_logits=True)
            h2_ref = om.forward(tok, pos)
            rc, t2_ref, _, lg2_ref = om.lm_head()
            assert rel_err(h2, h2_ref) <= REL_TOL and rel_err(lg, lg2_ref) <= REL_TOL
            assert nxt == t2_ref, pos
            tok, pos = nxt, pos + 1
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_q8_0_linears_and_q4_0_embedding(ctx, zo):
    """The other layer and embedding types the model takes: Q8_0X4 linears
    (Q8_0 weight GEMMs) and a plain Q4_0 token embedding."""
    cfg = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=1, head_dim=64,
                            vocab_padded=512, vocab_real=500, max_ctx=96, lin_type=synth.Q8_0,
                            embd_type=synth.Q4_0)
    model = synth.random_model(cfg, seed=12)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(13, 40, cfg.vocab_real)
        tok, _, hid = gm.prefill(prompt, want_hidden=True)
        assert rel_err(hid, om.prefill_q8(prompt)) <= REL_TOL
        assert tok == om.lm_head()[1]
        toks, _, _ = gm.generate(prompt, 30, batched_prefill=True)
        assert np.array_equal(toks, om.generate_batched(prompt, 30))
        toks, _, _ = gm.generate(prompt, 30)
        assert np.array_equal(toks, om.generate(prompt, 30))
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_generate_batched_matches_oracle(ctx, zo, tiny):
    gm = GpuModel(ctx, tiny)
    om = zo.OracleModel(tiny)
    try:
        prompt = synth.prompt(31, 48, TINY.vocab_real)
        toks, t_pre, t_gen = gm.generate(prompt, 40, batched_prefill=True)
        assert np.array_equal(toks, om.generate_batched(prompt, 40))
        # the token-by-token path on the same model is unchanged
        toks2, _, _ = gm.generate(prompt, 12)
        assert np.array_equal(toks2, om.generate(prompt, 12))
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_prefill_chunks_bit_identical(ctx, tiny):
    gm = GpuModel(ctx, tiny)
    try:
        prompt = synth.prompt(40, 90, TINY.vocab_real)
        t1, m1, h1 = gm.prefill(prompt, want_hidden=True)
        gm.prefill(prompt[:33])
        gm.prefill(prompt[33:70], pos0=33)
        t2, m2, h2 = gm.prefill(prompt[70:], pos0=70, want_hidden=True)
        assert np.array_equal(h1, h2) and t1 == t2 and m1 == m2
    finally:
        gm.close()
        ctx.clear()


def test_prefill_longer_than_a_chunk(ctx, zo):
    """620 rows: one 512-row chunk, then 108 rows attending to it."""
    cfg = synth.ModelConfig(n_layers=1, hidden=128, ffn=256, n_q_heads=2, n_kv_heads=1, head_dim=64,
                            vocab_padded=512, vocab_real=500, max_ctx=640)
    model = synth.random_model(cfg, seed=9)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(41, 620, cfg.vocab_real)
        tok, _, hid = gm.prefill(prompt, want_hidden=True)
        h_ref = om.prefill_q8(prompt)
        rc, t_ref, _, _ = om.lm_head()
        assert rel_err(hid, h_ref) <= REL_TOL and tok == t_ref
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_prefill_bounds(ctx, tiny):
    gm = GpuModel(ctx, tiny)
    try:
        with pytest.raises(ZgError) as e:
            gm.prefill(np.arange(10, dtype=np.uint32), pos0=TINY.max_ctx - 5)
        assert e.value.code == _lib.ZG_ERR_CONTEXT_FULL
        with pytest.raises(ZgError) as e:
            gm.prefill(np.array([1, TINY.vocab_padded], np.uint32))
        assert e.value.code == _lib.ZG_ERR_INVALID_ARG
        with pytest.raises(ZgError):
            gm.prefill(np.array([], np.uint32))
    finally:
        gm.close()
        ctx.clear()


def test_qwen3_1_7b_shape_batched_prefill(ctx):
    """128-token prefill at the Qwen3-1.7B shape: the last hidden state is
    within the Q8_0 activation-quantization distance of the token-by-token
    pass (the oracle's prefill at this size takes minutes on the CPU; the
    parity cases above cover the arithmetic)."""
    cfg = synth.ModelConfig(max_ctx=256)
    model = synth.random_model(cfg, seed=1)
    gm = GpuModel(ctx, model)
    try:
        prompt = synth.prompt(7, 128, cfg.vocab_real)
        tok_b, _, h_b = gm.prefill(prompt, want_hidden=True)
        for i, t in enumerate(prompt[:-1]):
            gm.step(int(t), i)
        tok_s, _, h_s, _ = gm.step(int(prompt[-1]), len(prompt) - 1, want_hidden=True)
        err = rel_err(h_b, h_s)
        print(f"batched vs token-by-token hidden rel err {err:.2e}; tokens {tok_b} / {tok_s}")
        assert 1e-5 < err < 5e-2
        toks, t_pre, t_gen = gm.generate(prompt, 16, batched_prefill=True)
        print(f"batched prefill of 128 tokens: {t_pre * 1e3:.2f} ms")
        assert toks[0] == tok_b
    finally:
        gm.close()
        ctx.clear()
