"""Pins the oracle pieces with no reference counterpart.

* zo_gemm_q8act (the prefill GEMM semantics) against an f64 brute force over
  the same dequantized Q8_0 activations and dequantized weights, and a
  closed-form KAT;
* zo_model_forward (the composition of the pinned operators in the order of
  forward_single_token_avx512, kernel/src/inference_avx512.rs:1826-1987)
  against an independent numpy restatement written from the Qwen3 block
  definition, on a tiny random model;
* zo_model_prefill_q8 (batched prefill with quantized activations) against
  the same numpy restatement with each matmul input quantized to Q8_0 for
  Q4_0 / Q8_0 weights (numpy's own round-half-even and binary16 rounding) or
  to Q8_K for Q4_K / Q6_K weights (quantize_row_q8k restated in float64),
  and for chunk invariance.
"""
import dataclasses

import numpy as np
import pytest

from zero_amd import synth


@pytest.mark.parametrize("m,n,k,wt,il", [(3, 8, 64, 2, 4), (5, 12, 96, 8, 1), (2, 4, 256, 2, 1), (4, 16, 128, 8, 4)])
def test_gemm_q8act_vs_f64(zo, m, n, k, wt, il):
    rng = np.random.default_rng(m * n + k)
    w = synth.weight(rng, wt, n, k, il)
    x = synth.activations(rng, m, k)
    xq = zo.quantize_q8_0(x.reshape(-1))
    y = zo.gemm_q8act(xq, w, m, n, k, wt, il)
    xd = zo.dequant(xq, m, k, 8, 1).astype(np.float64)
    wd = zo.dequant(w, n, k, wt, il).astype(np.float64)
    ref = xd @ wd.T
    err = np.max(np.abs(y - ref)) / np.max(np.abs(ref))
    assert err < 1e-5, err


def test_gemm_q8act_kat(zo):
    # all-ones activations (d = 1/127, q = 127) against the Q4_0 unit row
    # (ops.rs:955-965, every weight +1): y = 32 * 127 * (1/127 rounded to fp16)
    x = np.ones((1, 32), np.float32)
    xq = zo.quantize_q8_0(x.reshape(-1))
    from golden import kats
    w = np.frombuffer(kats.Q4_0_UNIT, np.uint8).copy()
    y = zo.gemm_q8act(xq, w, 1, 1, 32, 2, 1)
    d = float(np.float16(1.0 / 127.0))
    assert y[0, 0] == np.float32(d) * np.float32(32 * 127)


def _np_q8(v):
    """Q8_0 round trip of a vector: per 32 values d = amax/127, q =
    round-half-even(v/d) clamped to +-127, value q * fp16(d)."""
    b = v.reshape(-1, 32)
    amax = np.abs(b).max(axis=1, keepdims=True)
    d = amax / 127.0
    q = np.clip(np.rint(np.divide(b, d, out=np.zeros_like(b), where=d > 0)), -127, 127)
    return (q * d.astype(np.float16).astype(np.float64)).reshape(-1)


def _np_q8k(v):
    """Q8_K round trip of a vector (quantize_row_q8k,
    kernel/src/arch/x86_64/math/vnni.rs:78-170): per 256 values the first
    value of largest magnitude m, iscale = -127 / m, q = round-half-even(v *
    iscale) clamped to [-128, 127], value q / iscale; an all-zero block stays
    zero."""
    b = v.reshape(-1, 256)
    out = np.zeros_like(b)
    for i, row in enumerate(b):
        mx = row[int(np.argmax(np.abs(row)))]
        if mx != 0:
            iscale = -127.0 / mx
            out[i] = np.clip(np.rint(row * iscale), -128, 127) / iscale
    return out.reshape(-1)


def test_np_q8k_matches_the_oracle_quantizer(zo):
    x = synth.activations(np.random.default_rng(9), 2048)
    x[300] = -9.0
    x[301] = 9.0  # the first of equal magnitudes sets the sign
    blocks = zo.quantize_q8k(x).reshape(-1, 292)
    q = blocks[:, 4:260].view(np.int8).astype(np.float64)
    d = blocks[:, :4].copy().view(np.float32).astype(np.float64)
    want = (q * d).reshape(-1)
    assert np.max(np.abs(_np_q8k(x.astype(np.float64)) - want)) <= 1e-6 * np.max(np.abs(want))


def _np_forward(model, tokens, q8_rows=0):
    """Qwen3 decoder restated in numpy float64: pre-norm GQA with QK-norm,
    NeoX RoPE, causal softmax attention, SwiGLU MLP, residuals, final norm,
    LM head.  Positions below q8_rows quantize every matmul input first (the
    batched prefill's arithmetic): to Q8_0 for Q4_0 / Q8_0 weights, to Q8_K
    for Q4_K / Q6_K weights."""
    cfg = model.cfg
    H, hd, nq, nkv = cfg.hidden, cfg.head_dim, cfg.n_q_heads, cfg.n_kv_heads

    def deq(w, rows, k, q, il):
        from oracle import zo
        return zo.dequant(w, rows, k, q, il).astype(np.float64)

    def rms(v, g):
        return v / np.sqrt(np.mean(v * v) + cfg.rms_eps) * g

    inv = cfg.rope_theta ** (-2.0 * np.arange(hd // 2) / hd)
    emb = deq(model.token_embd, cfg.vocab_padded, H, cfg.embd_type, 1)
    head = deq(model.lm_head, cfg.vocab_padded, H, cfg.head_type, cfg.head_interleave)
    names = ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_gate", "ffn_up", "ffn_down")
    Ws = [{k: deq(getattr(L, k), *shape, *cfg.proj_quant(li, p))
           for p, (k, shape) in enumerate(zip(names, cfg.proj_shapes()))} for li, L in enumerate(model.layers)]
    Ts = [{k: cfg.proj_quant(li, p)[0] for p, k in enumerate(names)} for li in range(len(model.layers))]
    kc = [[] for _ in model.layers]
    vc = [[] for _ in model.layers]
    logits = []
    for pos, tok in enumerate(tokens):
        h = emb[tok].copy()
        c, s = np.cos(pos * inv), np.sin(pos * inv)

        def a8(v, t):
            if pos >= q8_rows:
                return v
            return _np_q8k(v) if t in (synth.Q4K, synth.Q6K) else _np_q8(v)

        def rope(v):
            a, b = v[:hd // 2], v[hd // 2:]
            return np.concatenate([a * c - b * s, a * s + b * c])

        for li, (L, W, T) in enumerate(zip(model.layers, Ws, Ts)):
            xn = rms(h, L.attn_norm)
            q = (W["attn_q"] @ a8(xn, T["attn_q"])).reshape(nq, hd)
            k = (W["attn_k"] @ a8(xn, T["attn_k"])).reshape(nkv, hd)
            v = (W["attn_v"] @ a8(xn, T["attn_v"])).reshape(nkv, hd)
            q = np.stack([rope(rms(qh, L.q_norm)) for qh in q])
            k = np.stack([rope(rms(kh, L.k_norm)) for kh in k])
            kc[li].append(k)
            vc[li].append(v)
            K, V = np.stack(kc[li]), np.stack(vc[li])
            out = np.empty((nq, hd))
            for hh in range(nq):
                g = hh // (nq // nkv)
                sc = K[:, g] @ q[hh] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                p /= p.sum()
                out[hh] = p @ V[:, g]
            h = h + W["attn_o"] @ a8(out.reshape(-1), T["attn_o"])
            xn = rms(h, L.ffn_norm)
            gt, up = W["ffn_gate"] @ a8(xn, T["ffn_gate"]), W["ffn_up"] @ a8(xn, T["ffn_up"])
            h = h + W["ffn_down"] @ a8(gt / (1 + np.exp(-gt)) * up, T["ffn_down"])
        logits.append(head @ rms(h, model.output_norm))
    return np.array(logits)


@pytest.mark.parametrize("il,head", [(4, synth.Q8_0), (1, synth.Q8_0), (4, synth.Q6K)])
def test_model_forward_vs_numpy(zo, il, head):
    """X4 (.smodel-v2) and plain-row (v1) layer linears and LM head, and a
    Q6_K LM head."""
    hil = il if head == synth.Q8_0 else 1
    cfg = synth.ModelConfig(n_layers=2, hidden=256, ffn=256, n_q_heads=4, n_kv_heads=2, head_dim=32,
                            vocab_padded=256, vocab_real=250, max_ctx=16, lin_interleave=il, head_type=head,
                            head_interleave=hil)
    model = synth.random_model(cfg, seed=2)
    toks = [3, 17, 101, 5, 5, 42]
    ref = _np_forward(model, toks)
    om = zo.OracleModel(model)
    for pos, t in enumerate(toks):
        om.forward(t, pos)
        rc, tok, mv, lg = om.lm_head()
        assert rc == 0
        err = np.max(np.abs(lg - ref[pos])) / np.max(np.abs(ref[pos]))
        assert err < 1e-4, (pos, err)
        assert tok == int(np.argmax(ref[pos][:cfg.vocab_real]))
    om.close()


MIXED = ((synth.Q4K, 1), (synth.Q6K, 1), (synth.Q4_0, 4), (synth.Q8_0, 1), (synth.Q4K, 1), (synth.Q4K, 1),
         (synth.Q6K, 1))


def test_model_forward_mixed_quants_vs_numpy(zo):
    """Per-layer, per-projection quants (ForwardPassDispatch): one layer of
    mixed K-quant / Q4_0X4 / plain Q8_0 projections and one of the Q4_K_M
    pattern, with a Q4_K token embedding and a Q6_K LM head."""
    cfg = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                            vocab_padded=256, vocab_real=250, max_ctx=16, embd_type=synth.Q4K, head_type=synth.Q6K,
                            head_interleave=1, layer_quants=(MIXED, synth.q4_k_m_layers(8)[0]))
    model = synth.random_model(cfg, seed=5)
    assert model.layers[0].attn_k.nbytes == cfg.kv_dim * 210 and model.layers[1].attn_v.nbytes == cfg.kv_dim * 210
    toks = [3, 17, 101, 5, 42]
    ref = _np_forward(model, toks)
    om = zo.OracleModel(model)
    for pos, t in enumerate(toks):
        om.forward(t, pos)
        rc, tok, mv, lg = om.lm_head()
        assert rc == 0
        err = np.max(np.abs(lg - ref[pos])) / np.max(np.abs(ref[pos]))
        assert err < 1e-4, (pos, err)
    om.close()
    # batched prefill over the same mixed layers: each projection's input is
    # quantized to its weight type's activation format
    ref = _np_forward(model, toks, q8_rows=len(toks))
    om = zo.OracleModel(model)
    om.prefill_q8(np.array(toks, np.uint32))
    rc, tok, mv, lg = om.lm_head()
    assert rc == 0
    err = np.max(np.abs(lg - ref[-1])) / np.max(np.abs(ref[-1]))
    assert err < 1e-3, err
    om.close()


def test_prefill_q4_k_m_vs_numpy(zo):
    """Batched prefill of a Q4_K_M-pattern model (Q4_K projections, Q6_K
    attn_v / ffn_down on the last layer): Q8_K activation rows throughout,
    then two decode steps from the prefilled cache."""
    cfg = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                            vocab_padded=256, vocab_real=250, max_ctx=16, embd_type=synth.Q4K, head_type=synth.Q6K,
                            head_interleave=1, layer_quants=synth.q4_k_m_layers(2))
    model = synth.random_model(cfg, seed=12)
    toks = [3, 17, 101, 5, 5, 42, 9, 200, 7]
    n = 7
    ref = _np_forward(model, toks, q8_rows=n)
    om = zo.OracleModel(model)
    om.prefill_q8(np.array(toks[:n], np.uint32))
    for pos in range(n - 1, len(toks)):
        if pos >= n:
            om.forward(toks[pos], pos)
        rc, tok, mv, lg = om.lm_head()
        assert rc == 0
        err = np.max(np.abs(lg - ref[pos])) / np.max(np.abs(ref[pos]))
        assert err < 1e-3, (pos, err)
        assert tok == int(np.argmax(ref[pos][:cfg.vocab_real]))
    # the fp32 token-by-token pass differs by the activation quantization only
    fp = _np_forward(model, toks)
    q_err = np.max(np.abs(ref[n - 1] - fp[n - 1])) / np.max(np.abs(fp[n - 1]))
    assert 1e-4 < q_err < 5e-2, q_err
    om.close()


PREFILL_CFG = synth.ModelConfig(n_layers=2, hidden=128, ffn=256, n_q_heads=4, n_kv_heads=2, head_dim=32,
                                vocab_padded=256, vocab_real=250, max_ctx=24)


def test_np_q8_matches_the_oracle_quantizer(zo):
    x = synth.activations(np.random.default_rng(5), 4096)
    want = zo.dequant(zo.quantize_q8_0(x), 1, 4096, 8, 1)[0]
    assert np.array_equal(_np_q8(x.astype(np.float64)).astype(np.float32), want)


@pytest.mark.parametrize("il", [4, 1])
def test_prefill_q8_vs_numpy(zo, il):
    model = synth.random_model(dataclasses.replace(PREFILL_CFG, lin_interleave=il, head_interleave=il), seed=4)
    toks = [3, 17, 101, 5, 5, 42, 9, 200, 7]
    n = 7  # prefill 7 tokens, then decode the last two one by one
    ref = _np_forward(model, toks, q8_rows=n)
    om = zo.OracleModel(model)
    om.prefill_q8(toks[:n])
    for pos in range(n - 1, len(toks)):
        if pos >= n:
            om.forward(toks[pos], pos)
        rc, tok, mv, lg = om.lm_head()
        assert rc == 0
        err = np.max(np.abs(lg - ref[pos])) / np.max(np.abs(ref[pos]))
        assert err < 1e-3, (pos, err)
        assert tok == int(np.argmax(ref[pos][:PREFILL_CFG.vocab_real]))
    # the fp32 token-by-token pass differs by the activation quantization only
    fp = _np_forward(model, toks)
    q_err = np.max(np.abs(ref[n - 1] - fp[n - 1])) / np.max(np.abs(fp[n - 1]))
    assert 1e-4 < q_err < 5e-2, q_err
    om.close()


def test_prefill_q8_chunks_are_invariant(zo):
    """Rows are independent through the GEMMs and attend only to earlier
    positions, so prefilling in chunks (pos0 > 0) gives the same bits."""
    model = synth.random_model(PREFILL_CFG, seed=6)
    toks = np.array([11, 2, 99, 140, 3, 3, 77, 18, 60, 201, 5], np.uint32)
    a = zo.OracleModel(model)
    ha = a.prefill_q8(toks)
    la = a.lm_head()[3]
    b = zo.OracleModel(model)
    b.prefill_q8(toks[:4])
    b.prefill_q8(toks[4:9], pos0=4)
    hb = b.prefill_q8(toks[9:], pos0=9)
    lb = b.lm_head()[3]
    assert np.array_equal(ha, hb) and np.array_equal(la, lb)
    a.close()
    b.close()
