"""GPU parity of the single-token forward pass (forward_single_token_avx512,
kernel/src/inference_avx512.rs:1826-1987) and the greedy loop, against the
oracle's C restatement on the same random-init weights.

Bar: final hidden state and logits within rel 1e-3 at every compared step,
identical greedy tokens (64 decode steps after a 128-token prompt at the
Qwen3-1.7B shape).
"""
import numpy as np
import pytest

from zero_amd import synth
from zero_amd.model import GpuModel

pytestmark = pytest.mark.gpu
REL_TOL = 1e-3


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


TINY = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                         vocab_padded=1024, vocab_real=1000, max_ctx=96)


@pytest.fixture(scope="module")
def tiny():
    return synth.random_model(TINY, seed=3)


def test_tiny_model_stepwise(ctx, zo, tiny):
    gm = GpuModel(ctx, tiny)
    om = zo.OracleModel(tiny)
    tok = 7
    worst_h = worst_l = 0.0
    for pos in range(70):  # crosses the 32-row attention splits twice
        nxt, mx, hid, lg = gm.step(tok, pos, want_hidden=True, want_logits=True)
        h_ref = om.forward(tok, pos)
        rc, t_ref, m_ref, lg_ref = om.lm_head()
        assert rc == 0
        worst_h, worst_l = max(worst_h, rel_err(hid, h_ref)), max(worst_l, rel_err(lg, lg_ref))
        assert nxt == t_ref, pos
        tok = nxt
    print(f"tiny model: worst hidden rel err {worst_h:.2e}, worst logits rel err {worst_l:.2e}")
    assert worst_h <= REL_TOL and worst_l <= REL_TOL
    om.close()
    gm.close()
    ctx.clear()


@pytest.mark.parametrize("n_q,n_kv,hd", [(8, 1, 64), (4, 4, 64), (8, 2, 128)])
def test_attention_head_groupings(ctx, zo, n_q, n_kv, hd):
    """Query heads per KV head G = 8, 1 and 4 (the Qwen shape has G = 2).
    Three 32-row splits; the 512- and 1024-wide attention outputs are merged
    by the O GEMV's prologue, the 256-wide one by the separate merge kernel."""
    cfg = synth.ModelConfig(n_layers=1, hidden=256, ffn=512, n_q_heads=n_q, n_kv_heads=n_kv, head_dim=hd,
                            vocab_padded=512, vocab_real=500, max_ctx=72)
    model = synth.random_model(cfg, seed=n_q + 3 * n_kv + hd)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    tok, worst = 3, 0.0
    for pos in range(40):
        nxt, _, hid, _ = gm.step(tok, pos, want_hidden=True, want_logits=False)
        h_ref = om.forward(tok, pos)
        rc, t_ref, _, _ = om.lm_head()
        worst = max(worst, rel_err(hid, h_ref))
        assert nxt == t_ref, pos
        tok = nxt
    print(f"G={n_q // n_kv} hd={hd}: worst hidden rel err {worst:.2e}")
    assert worst <= REL_TOL
    om.close()
    gm.close()
    ctx.clear()


def test_attention_split_context(ctx, zo):
    """Long context: four 544-row splits per query head, each visited in
    five 128-row rounds (online softmax across rounds)."""
    cfg = synth.ModelConfig(n_layers=1, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                            vocab_padded=512, vocab_real=500, max_ctx=2100)
    model = synth.random_model(cfg, seed=11)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    prompt = synth.prompt(12, 8, cfg.vocab_real)
    toks, _, _ = gm.generate(prompt, 2090)
    assert np.array_equal(toks, om.generate(prompt, 2090))
    om.close()
    gm.close()
    ctx.clear()


@pytest.mark.parametrize("n_q,n_kv,hd,max_ctx,n_gen", [(8, 2, 128, 30, 26), (8, 2, 128, 520, 500), (8, 4, 64, 200, 190)])
def test_attention_split_geometries(ctx, zo, n_q, n_kv, hd, max_ctx, n_gen):
    """One split (max_ctx <= 32, the output written directly); four 160-row
    splits of two rounds each, merged in the O GEMV; four 64-row splits at
    head_dim 64, merged in the O GEMV."""
    cfg = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=n_q, n_kv_heads=n_kv, head_dim=hd,
                            vocab_padded=512, vocab_real=500, max_ctx=max_ctx)
    model = synth.random_model(cfg, seed=max_ctx + hd)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    prompt = synth.prompt(max_ctx, 4, cfg.vocab_real)
    toks, _, _ = gm.generate(prompt, n_gen)
    assert np.array_equal(toks, om.generate(prompt, n_gen))
    om.close()
    gm.close()
    ctx.clear()


@pytest.mark.parametrize("head_type", [synth.Q6K, synth.Q4K])
def test_kquant_lm_head(ctx, zo, head_type):
    """A K-quant output.weight (GGUF Q4_K_M checkpoints carry a Q6_K one):
    the model normalizes into its own buffer, then the K-quant GEMV with the
    argmax epilogue.  Midway an op-level LM head 4096 wide goes through the
    context's rmsnorm buffer and reallocates it; the captured decode graph
    does not use that buffer."""
    cfg = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                            vocab_padded=1024, vocab_real=1000, max_ctx=64, head_type=head_type, head_interleave=1)
    model = synth.random_model(cfg, seed=21 + head_type)
    rng = np.random.default_rng(head_type)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        tok = 3
        for pos in range(24):
            if pos == 12:
                k, rows = 4096, 64
                w = synth.weight(rng, head_type, rows, k, 1)
                ctx.register(w, head_type, 1)
                h = synth.activations(rng, k)
                g = (1.0 + 0.05 * rng.standard_normal(k)).astype(np.float32)
                lg_op = np.empty(rows, np.float32)
                t_op = ctx.lm_head_argmax(h, g, w, head_type, 1e-6, k, lg_op, vocab_padded=rows, vocab_real=rows)
                assert t_op == int(np.argmax(lg_op))
            nxt, _, hid, lg = gm.step(tok, pos, want_hidden=True, want_logits=True)
            h_ref = om.forward(tok, pos)
            rc, t_ref, _, lg_ref = om.lm_head()
            assert rc == 0
            assert rel_err(hid, h_ref) <= REL_TOL and rel_err(lg, lg_ref) <= REL_TOL, pos
            assert nxt == t_ref, pos
            tok = nxt
        prompt = synth.prompt(head_type, 20, cfg.vocab_real)
        toks, _, _ = gm.generate(prompt, 30, batched_prefill=True)
        assert np.array_equal(toks, om.generate_batched(prompt, 30))
    finally:
        om.close()
        gm.close()
        ctx.clear()


MIXED = ((synth.Q4K, 1), (synth.Q6K, 1), (synth.Q4_0, 4), (synth.Q8_0, 1), (synth.Q4K, 1), (synth.Q4K, 1),
         (synth.Q6K, 1))


def test_mixed_projection_quants(ctx, zo):
    """ForwardPassDispatch's per-layer, per-projection quants: a layer of
    mixed Q4_K / Q6_K / Q4_0X4 / plain Q8_0 projections and a layer of the
    Q4_K_M pattern, Q4_K token embedding, Q6_K LM head.  The batched
    prefill runs each projection's GEMM on its own activation format (Q8_K
    rows for Q4_K / Q6_K, Q8_0 rows for Q4_0 / Q8_0)."""
    cfg = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                            vocab_padded=1024, vocab_real=1000, max_ctx=80, embd_type=synth.Q4K,
                            head_type=synth.Q6K, head_interleave=1, layer_quants=(MIXED, synth.q4_k_m_layers(8)[0]))
    model = synth.random_model(cfg, seed=17)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        tok = 11
        for pos in range(40):
            nxt, _, hid, lg = gm.step(tok, pos, want_hidden=True, want_logits=True)
            h_ref = om.forward(tok, pos)
            rc, t_ref, _, lg_ref = om.lm_head()
            assert rc == 0
            assert rel_err(hid, h_ref) <= REL_TOL and rel_err(lg, lg_ref) <= REL_TOL, pos
            assert nxt == t_ref, pos
            tok = nxt
        prompt = synth.prompt(4, 12, cfg.vocab_real)
        toks, _, _ = gm.generate(prompt, 30)
        assert np.array_equal(toks, om.generate(prompt, 30))
        toks, _, _ = gm.generate(prompt, 20, batched_prefill=True)
        assert np.array_equal(toks, om.generate_batched(prompt, 20))
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_qwen3_1_7b_shape_q8_0_projections(ctx, zo):
    """Q8_0X4 layer projections at the Qwen3-1.7B shape (the model splits
    them into scale-split groups, which run every layer launch on the strip
    kernel: gate|up with SwiGLU at 3,072 groups, down at 12 strips): a
    6-token prompt token by token, its logits at the last two positions
    within rel 1e-3 of the oracle, then 8 greedy tokens equal to the
    oracle's, token-by-token and batched prefill."""
    cfg = synth.ModelConfig(n_layers=4, max_ctx=32, lin_type=synth.Q8_0)
    model = synth.random_model(cfg, seed=13)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(13, 6, cfg.vocab_real)
        with zo.Pool(16):
            for i, t in enumerate(prompt):
                nxt, _, _, lg = gm.step(int(t), i, want_logits=i >= 4)
                om.forward(int(t), i)
                if i >= 4:
                    rc, t_ref, _, lg_ref = om.lm_head()
                    assert rc == 0 and rel_err(lg, lg_ref) <= REL_TOL and nxt == t_ref
            toks, _, _ = gm.generate(prompt, 8)
            assert np.array_equal(toks, om.generate(prompt, 8))
            toks_b, _, _ = gm.generate(prompt, 8, batched_prefill=True)
            assert np.array_equal(toks_b, om.generate_batched(prompt, 8))
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_qwen3_1_7b_shape_q4_k_m(ctx, zo):
    """The reference's default dispatch at the Qwen3-1.7B shape: Q4_K layer
    projections with the Q4_K_M pattern's Q6_K attn_v / ffn_down, Q4_K token
    embedding, Q6_K LM head.  8-token prompt, then 24 greedy tokens against
    the oracle; logits compared at the last 4 prompt positions."""
    cfg = synth.ModelConfig(max_ctx=64, embd_type=synth.Q4K, head_type=synth.Q6K, head_interleave=1,
                            layer_quants=synth.q4_k_m_layers(28))
    model = synth.random_model(cfg, seed=6)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    try:
        prompt = synth.prompt(8, 8, cfg.vocab_real)
        for i, t in enumerate(prompt):
            nxt, _, _, lg = gm.step(int(t), i, want_logits=i >= 4)
            om.forward(int(t), i)
            if i >= 4:
                rc, t_ref, _, lg_ref = om.lm_head()
                err = rel_err(lg, lg_ref)
                print(f"Q4_K_M-pattern Qwen3-1.7B shape, pos {i}: logits rel err {err:.2e}")
                assert err <= REL_TOL and nxt == t_ref
        toks, _, _ = gm.generate(prompt, 24)
        assert np.array_equal(toks, om.generate(prompt, 24))
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_tiny_model_generate_matches_oracle(ctx, zo, tiny):
    gm = GpuModel(ctx, tiny)
    om = zo.OracleModel(tiny)
    prompt = synth.prompt(5, 16, TINY.vocab_real)
    toks, _, _ = gm.generate(prompt, 40)
    ref = om.generate(prompt, 40)
    assert np.array_equal(toks, ref)
    # a second, shorter sequence on the same model restarts at position 0
    toks2, _, _ = gm.generate(prompt[:5], 10)
    assert np.array_equal(toks2, om.generate(prompt[:5], 10))
    om.close()
    gm.close()
    ctx.clear()


def test_eager_generate_matches_graph(ctx, tiny):
    """ZG_GEN_EAGER issues the step's launches directly: same tokens as the
    graph replay; combined with the batched prefill, or an unknown flag bit,
    it is an argument error."""
    gm = GpuModel(ctx, tiny)
    try:
        prompt = synth.prompt(9, 12, TINY.vocab_real)
        toks_g, _, _ = gm.generate(prompt, 20)
        toks_e, _, _ = gm.generate(prompt, 20, eager=True)
        assert np.array_equal(toks_g, toks_e)
        import zero_amd
        from zero_amd import _lib
        with pytest.raises(zero_amd.ZgError) as e:
            gm.generate(prompt, 4, batched_prefill=True, eager=True)
        assert e.value.code == _lib.ZG_ERR_INVALID_ARG
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(4, np.uint32)
        assert ctx.lib.zg_model_generate_ex(gm.h, p.ctypes.data, p.size, 4, 8, out.ctypes.data, None,
                                            None) == _lib.ZG_ERR_INVALID_ARG
    finally:
        gm.close()
        ctx.clear()


def test_generate_bounds(ctx, tiny):
    gm = GpuModel(ctx, tiny)
    import zero_amd
    with pytest.raises(zero_amd.ZgError):
        gm.generate(synth.prompt(1, 90, TINY.vocab_real), 10)  # 90 + 10 - 1 > max_ctx
    with pytest.raises(zero_amd.ZgError):
        gm.step(5, TINY.max_ctx, False, False)
    gm.close()
    ctx.clear()


def test_qwen3_1_7b_shape_greedy_64(ctx, zo):
    """Config 3: random-init Qwen3-1.7B shape, 128-token seeded prompt, then
    64 greedy decode steps compared token by token and logit by logit.

    Then the path the bench times: zg_model_generate (the captured step
    graph, the next token fed back on the device) must give the oracle's
    tokens too.  Finally the steps are replayed after zg_model_reset and
    every logit must repeat bit for bit (the reference's bitwise-invariance
    contract, kernel/src/smp.rs:33-40)."""
    cfg = synth.ModelConfig(max_ctx=256)
    model = synth.random_model(cfg, seed=11)
    gm = GpuModel(ctx, model)
    om = zo.OracleModel(model)
    prompt = synth.prompt(12, 128, cfg.vocab_real)
    worst = 0.0
    margins = []
    ref_tokens, logits = [], []
    try:
        with zo.Pool(16):
            for pos, t in enumerate(prompt[:-1]):
                gm.step(int(t), pos)
                om.forward(int(t), pos)
            tok, pos = int(prompt[-1]), len(prompt) - 1
            for step in range(65):
                nxt, _, hid, lg = gm.step(tok, pos, want_hidden=True, want_logits=True)
                h_ref = om.forward(tok, pos)
                rc, t_ref, _, lg_ref = om.lm_head()
                assert rc == 0
                worst = max(worst, rel_err(lg, lg_ref), rel_err(hid, h_ref))
                top = np.sort(lg_ref)[-2:]
                margins.append(float(top[1] - top[0]))
                assert nxt == t_ref, (step, nxt, t_ref)
                ref_tokens.append(t_ref)
                logits.append(np.array(lg, np.float32))
                tok, pos = nxt, pos + 1
        print(f"Qwen3-1.7B shape: 65 greedy tokens identical, worst rel err {worst:.2e}, "
              f"min top-2 logit margin {min(margins):.4f}")
        assert worst <= REL_TOL

        # the device-fed greedy loop (what bench.py times) against the oracle
        toks, _, _ = gm.generate(prompt, 64)
        assert np.array_equal(np.asarray(toks), np.asarray(ref_tokens[:64], np.uint32))
        toks2, _, _ = gm.generate(prompt, 64)
        assert np.array_equal(toks2, toks)

        # the same steps again after a reset: identical logit bits
        gm.reset()
        for pos, t in enumerate(prompt[:-1]):
            gm.step(int(t), pos)
        tok, pos = int(prompt[-1]), len(prompt) - 1
        for step in range(65):
            nxt, _, _, lg = gm.step(tok, pos, want_logits=True)
            assert np.array_equal(np.asarray(lg, np.float32).view(np.uint32), logits[step].view(np.uint32)), step
            tok, pos = nxt, pos + 1
    finally:
        om.close()
        gm.close()
        ctx.clear()


def test_fused_attention_wait_timeout(ctx):
    """The bounded wait of the fused Q|K|V + attention launch, forced from
    the host: with layer 1's tagged Q|K|V stores dropped
    (zg_model_test_drop_qkv_stores), that layer's attention waves give up
    after their poll bound and the step reports ZG_ERR_HIP with the timeout
    message, the GPU counterpart of the reference's barrier-timeout recovery
    (kernel/src/smp.rs:1677-1711).  Every kernel still runs to its end.
    With the stores restored and a reset, the model decodes the same tokens
    as before the failure."""
    import zero_amd
    from zero_amd import _lib
    cfg = synth.ModelConfig(n_layers=3, hidden=2048, ffn=2048, vocab_padded=4096, vocab_real=4000, max_ctx=32)
    model = synth.random_model(cfg, seed=21)
    gm = GpuModel(ctx, model)
    try:
        prompt = synth.prompt(21, 6, cfg.vocab_real)
        ref, _, _ = gm.generate(prompt, 8)
        gm.reset()
        assert ctx.lib.zg_model_test_drop_qkv_stores(gm.h, 1) == _lib.ZG_OK
        with pytest.raises(zero_amd.ZgError) as e:
            gm.step(int(prompt[0]), 0)
        assert e.value.code == _lib.ZG_ERR_HIP
        assert "wait timed out" in str(e.value)
        assert ctx.lib.zg_model_test_drop_qkv_stores(gm.h, -1) == _lib.ZG_OK
        gm.reset()
        toks, _, _ = gm.generate(prompt, 8)
        assert np.array_equal(toks, ref)
        # a layer outside the model drops nothing
        assert ctx.lib.zg_model_test_drop_qkv_stores(gm.h, 7) == _lib.ZG_OK
        gm.reset()
        toks, _, _ = gm.generate(prompt, 8)
        assert np.array_equal(toks, ref)
        assert ctx.lib.zg_model_test_drop_qkv_stores(None, 0) == _lib.ZG_ERR_INVALID_ARG
    finally:
        ctx.lib.zg_model_test_drop_qkv_stores(gm.h, -1)
        gm.close()
        ctx.clear()
