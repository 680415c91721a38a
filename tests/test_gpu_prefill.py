"""GPU parity of the batched prefill (zg_model_prefill, zg_model_generate_ex
with ZG_GEN_BATCHED_PREFILL) against the oracle's zo_model_prefill_q8: the
prompt rows go through rmsnorm, activation quantization (Q8_0 for Q4_0 /
Q8_0 weights, Q8_K for Q4_K / Q6_K weights) and the int8 MFMA GEMMs, with
the decode step's QK-norm, RoPE, causal attention and SwiGLU per row.

Bar: the last row's hidden state and the next token's logits within rel
1e-3 of the oracle, identical greedy tokens after the prefill; chunked calls
(pos0 > 0) bit-identical to one call; at the Qwen3-1.7B shape, within the
activation-quantization distance of the token-by-token pass."""
import dataclasses

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


@pytest.mark.parametrize("lin_type", [synth.Q4_0, synth.Q8_0])
def test_plain_row_layouts(ctx, zo, lin_type):
    """Plain row-major layer linears and LM head (.smodel-v1 / GGUF layouts)
    at strip-sized dims: the model interleaves them to X4 on the device when
    it is created; its batched prefill and decode match the oracle, which
    reads the plain rows."""
    cfg = synth.ModelConfig(n_layers=2, hidden=512, ffn=1024, n_q_heads=8, n_kv_heads=2, head_dim=64,
                            vocab_padded=1024, vocab_real=1000, max_ctx=160, lin_type=lin_type,
                            lin_interleave=1, head_interleave=1)
    model = synth.random_model(cfg, seed=14)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(17, 70, cfg.vocab_real)
        tok, _, hid = gm.prefill(prompt, want_hidden=True)
        err = rel_err(hid, om.prefill_q8(prompt))
        print(f"plain layout type {lin_type}: prefill hidden rel err {err:.2e}")
        assert err <= REL_TOL and tok == om.lm_head()[1]
        pos = len(prompt)
        for _ in range(6):
            nxt, _, h2, lg = gm.step(tok, pos, want_hidden=True, want_logits=True)
            h2_ref = om.forward(tok, pos)
            rc, t2_ref, _, lg2_ref = om.lm_head()
            assert rel_err(h2, h2_ref) <= REL_TOL and rel_err(lg, lg2_ref) <= REL_TOL
            assert nxt == t2_ref, pos
            tok, pos = nxt, pos + 1
        toks, _, _ = gm.generate(prompt, 24, batched_prefill=True)
        assert np.array_equal(toks, om.generate_batched(prompt, 24))
        toks, _, _ = gm.generate(prompt[:20], 24)
        assert np.array_equal(toks, om.generate(prompt[:20], 24))
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_mixed_q4_0_q8_0_projections(ctx, zo):
    """Per-projection Q4_0 / Q8_0 types and layouts: the prefill runs one
    GEMM per projection where a fused group's types differ.

    The synthetic Q8_0 weights are ~16x the Q4_0 ones, and in this mix one
    Q8_0 rounding flip of an activation moves the hidden state by 1e-3..5e-3
    (on the CPU a 1e-6 relative perturbation of the quantizer inputs already
    does; the oracle's f32 prefill and an f64 numpy restatement differ by
    1.7e-3).  The device expf and the host's can differ in the last bit on a
    SwiGLU input, so the prefill is held to 2e-2 here (a wrong GEMM type or
    layout gives errors of order 1); the token-by-token decode, which has no
    quantization step, to the usual 1e-3 and identical tokens."""
    lq = ((synth.Q4_0, 4), (synth.Q4_0, 4), (synth.Q8_0, 4), (synth.Q4_0, 1), (synth.Q8_0, 1), (synth.Q8_0, 1),
          (synth.Q4_0, 4))
    cfg = synth.ModelConfig(n_layers=2, hidden=512, ffn=1024, n_q_heads=8, n_kv_heads=2, head_dim=64,
                            vocab_padded=1024, vocab_real=1000, max_ctx=128, layer_quants=(lq, lq[::-1]))
    model = synth.random_model(cfg, seed=19)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(29, 50, cfg.vocab_real)
        tok, _, hid = gm.prefill(prompt, want_hidden=True)
        err = rel_err(hid, om.prefill_q8(prompt))
        print(f"mixed Q4_0/Q8_0 projections: prefill hidden rel err vs oracle {err:.2e}")
        assert err <= 2e-2
        toks, _, _ = gm.generate(prompt, 8, batched_prefill=True)
        assert toks[0] == tok
        for pos in range(12):
            t = int(prompt[pos])
            _, _, h2, lg = gm.step(t, pos, want_hidden=True, want_logits=True)
            h2_ref = om.forward(t, pos)
            lg_ref = om.lm_head()[3]
            assert rel_err(h2, h2_ref) <= REL_TOL and rel_err(lg, lg_ref) <= REL_TOL, pos
        toks, _, _ = gm.generate(prompt[:10], 30)
        assert np.array_equal(toks, om.generate(prompt[:10], 30))
    finally:
        om.close()
        gm.close()
        ctx.clear()


def _x4_layers(model):
    """The same weights with X4 layer linears (copies throughout: a host
    array is one registry key)."""
    c = model.cfg
    x4 = synth.RandomModel(dataclasses.replace(c, lin_interleave=4), token_embd=model.token_embd.copy(),
                           lm_head=model.lm_head.copy(), output_norm=model.output_norm)
    shapes = {"attn_q": (c.q_dim, c.hidden), "attn_k": (c.kv_dim, c.hidden), "attn_v": (c.kv_dim, c.hidden),
              "attn_o": (c.hidden, c.q_dim), "ffn_gate": (c.ffn, c.hidden), "ffn_up": (c.ffn, c.hidden),
              "ffn_down": (c.hidden, c.ffn)}
    for L in model.layers:
        x4.layers.append(dataclasses.replace(
            L, **{k: synth.interleave_x4(getattr(L, k), r, kk, c.lin_type) for k, (r, kk) in shapes.items()}))
    return x4


def test_qwen3_1_7b_shape_plain_layout_bit_identical(ctx):
    """At the Qwen3-1.7B shape the plain-row Q4_0 model gives the X4 model's
    bits: the device interleave at model creation reproduces the packer's
    X4 bytes (the X4 model here is interleaved on the host).  Checked on a
    64-token batched prefill, then 16 decode steps."""
    cfg = synth.ModelConfig(max_ctx=128, lin_interleave=1)
    plain = synth.random_model(cfg, seed=3)
    models = [GpuModel(ctx, plain), GpuModel(ctx, _x4_layers(plain))]
    try:
        prompt = synth.prompt(23, 64, cfg.vocab_real)
        outs = [m.prefill(prompt, want_hidden=True) for m in models]
        assert outs[0][0] == outs[1][0] and np.array_equal(outs[0][2], outs[1][2])
        toks = [outs[0][0]] * 2
        for pos in range(64, 80):
            r = [m.step(t, pos, want_hidden=True, want_logits=True) for m, t in zip(models, toks)]
            assert np.array_equal(r[0][2], r[1][2]) and np.array_equal(r[0][3], r[1][3]), pos
            assert r[0][0] == r[1][0]
            toks = [r[0][0], r[1][0]]
    finally:
        for m in models:
            m.close()
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


def test_qwen3_1_7b_shape_batched_prefill_matches_oracle(ctx, zo):
    """12-row batched prefill through all 28 layers of the Qwen3-1.7B shape
    against the oracle's zo_model_prefill_q8 on the same prompt: last hidden
    state and logits within rel 1e-3, the same next token, then 8 decode
    steps from the prefilled cache token for token."""
    cfg = synth.ModelConfig(max_ctx=64)
    model = synth.random_model(cfg, seed=21)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(31, 12, cfg.vocab_real)
        tok, mv, hid = gm.prefill(prompt, want_hidden=True)
        h_ref = om.prefill_q8(prompt)
        rc, t_ref, m_ref, _ = om.lm_head()
        assert rc == 0
        err = rel_err(hid, h_ref)
        print(f"Qwen3-1.7B shape, 12-row prefill: hidden rel err {err:.2e}")
        assert err <= REL_TOL
        assert tok == t_ref and abs(mv - m_ref) <= REL_TOL * abs(m_ref)
        pos = len(prompt)
        with zo.Pool(16):
            for _ in range(8):
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


KQ_TINY = dataclasses.replace(TINY, embd_type=synth.Q4K, head_type=synth.Q6K, head_interleave=1,
                              layer_quants=synth.q4_k_m_layers(2))


@pytest.mark.parametrize("n", [1, 7, 130])
def test_k_quant_prefill_matches_oracle(ctx, zo, n):
    """Q4_K_M-pattern layers (Q4_K, Q6_K attn_v / ffn_down on the last
    layer): Q8_K rows into the K-quant GEMMs, then decode from the cache."""
    model = synth.random_model(KQ_TINY, seed=30)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(50 + n, n, KQ_TINY.vocab_real)
        tok, mv, hid = gm.prefill(prompt, want_hidden=True)
        h_ref = om.prefill_q8(prompt)
        rc, t_ref, m_ref, _ = om.lm_head()
        assert rc == 0
        print(f"K-quant n={n}: hidden rel err {rel_err(hid, h_ref):.2e}")
        assert rel_err(hid, h_ref) <= REL_TOL
        assert tok == t_ref and abs(mv - m_ref) <= REL_TOL * abs(m_ref)
        pos = n
        for _ in range(6):
            nxt, _, h2, _ = gm.step(tok, pos, want_hidden=True)
            h2_ref = om.forward(tok, pos)
            rc, t2_ref, _, _ = om.lm_head()
            assert rel_err(h2, h2_ref) <= REL_TOL and nxt == t2_ref, pos
            tok, pos = nxt, pos + 1
        # chunked calls give the same bits as one call
        if n > 2:
            gm.prefill(prompt[:n // 2])
            t2, m2, h2 = gm.prefill(prompt[n // 2:], pos0=n // 2, want_hidden=True)
            assert np.array_equal(h2, hid) and t2 == t_ref
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_k_quant_generate_batched_matches_oracle(ctx, zo):
    model = synth.random_model(KQ_TINY, seed=31)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(32, 40, KQ_TINY.vocab_real)
        toks, _, _ = gm.generate(prompt, 32, batched_prefill=True)
        assert np.array_equal(toks, om.generate_batched(prompt, 32))
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_qwen3_1_7b_shape_q4_k_m_batched_prefill_matches_oracle(ctx, zo):
    """12-row batched prefill through all 28 Q4_K_M-pattern layers of the
    Qwen3-1.7B shape (Q4_K projections, Q6_K attn_v / ffn_down on 14 layers,
    Q4_K token embedding, Q6_K LM head) against zo_model_prefill_q8: last
    hidden state within rel 1e-3 and the same next token, then 8 decode
    steps token for token; the 128-token prefill within the Q8_K
    activation-quantization distance of the token-by-token pass."""
    cfg = synth.ModelConfig(max_ctx=160, embd_type=synth.Q4K, head_type=synth.Q6K, head_interleave=1,
                            layer_quants=synth.q4_k_m_layers(28))
    model = synth.random_model(cfg, seed=22)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(33, 12, cfg.vocab_real)
        with zo.Pool(16):
            tok, mv, hid = gm.prefill(prompt, want_hidden=True)
            h_ref = om.prefill_q8(prompt)
            rc, t_ref, m_ref, _ = om.lm_head()
            assert rc == 0
            err = rel_err(hid, h_ref)
            print(f"Q4_K_M Qwen3-1.7B shape, 12-row prefill: hidden rel err {err:.2e}")
            assert err <= REL_TOL
            assert tok == t_ref and abs(mv - m_ref) <= REL_TOL * abs(m_ref)
            pos = len(prompt)
            for _ in range(8):
                nxt, _, h2, lg = gm.step(tok, pos, want_hidden=True, want_logits=True)
                h2_ref = om.forward(tok, pos)
                rc, t2_ref, _, lg2_ref = om.lm_head()
                assert rel_err(h2, h2_ref) <= REL_TOL and rel_err(lg, lg2_ref) <= REL_TOL
                assert nxt == t2_ref, pos
                tok, pos = nxt, pos + 1
        long = synth.prompt(8, 128, cfg.vocab_real)
        tok_b, _, h_b = gm.prefill(long, want_hidden=True)
        for i, t in enumerate(long[:-1]):
            gm.step(int(t), i)
        tok_s, _, h_s, _ = gm.step(int(long[-1]), len(long) - 1, want_hidden=True)
        err = rel_err(h_b, h_s)
        print(f"Q4_K_M batched vs token-by-token hidden rel err {err:.2e}; tokens {tok_b} / {tok_s}")
        assert 1e-5 < err < 5e-2
        toks, t_pre, _ = gm.generate(long, 8, batched_prefill=True)
        print(f"Q4_K_M batched prefill of 128 tokens: {t_pre * 1e3:.2f} ms")
        assert toks[0] == tok_b
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_k_quant_prefill_longer_than_a_chunk(ctx, zo):
    """620 rows of a Q4_K / Q6_K model (hidden 256: whole superblocks): one
    512-row chunk of Q8_K GEMMs, then 108 rows attending to its cache rows."""
    cfg = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                            vocab_padded=512, vocab_real=500, max_ctx=640, embd_type=synth.Q4K,
                            head_type=synth.Q6K, head_interleave=1, layer_quants=synth.q4_k_m_layers(2))
    model = synth.random_model(cfg, seed=19)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(43, 620, cfg.vocab_real)
        tok, _, hid = gm.prefill(prompt, want_hidden=True)
        h_ref = om.prefill_q8(prompt)
        rc, t_ref, _, _ = om.lm_head()
        assert rc == 0
        assert rel_err(hid, h_ref) <= REL_TOL and tok == t_ref
    finally:
        om.close()
        gm.close()
        ctx.clear()
