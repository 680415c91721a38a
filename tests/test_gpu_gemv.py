"""GPU parity of the GEMV path, called through the C ABI.

Bar: dequantized weights bit-exact with the oracle's restatement of
dequant.rs; GEMV outputs within rel 1e-3 (max |gpu - oracle| <= 1e-3 *
max |oracle| per vector) of the oracle's AVX-512-order kernels, and no
further from an f64 brute force than the oracle itself is (x 4).
"""
import numpy as np
import pytest
import torch

import zero_amd
from golden import kats
from zero_amd import synth

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4K, Q6K = 2, 8, 12, 14
REL_TOL = 1e-3  # parity bar for dot products / logits (rel 1e-3)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def same_bits(got, want):
    """Bitwise equality; NaN results only need to be NaN on both sides
    (the NaN-scale decode itself is checked bitwise by the fp16 test)."""
    g, w = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan = np.isnan(w)
    return np.array_equal(np.isnan(g), nan) and np.array_equal(g[~nan].view(np.uint32), w[~nan].view(np.uint32))


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def test_fp16_exhaustive_on_gpu(ctx, zo):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    src = dev(bits.view(np.int16))
    out = torch.empty(65536, dtype=torch.float32, device="cuda")
    ctx.fp16_to_f32_dev(src, out, 65536, stream=torch.cuda.current_stream().cuda_stream)
    got = out.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, zo.fp16_to_f32(bits).view(np.uint32))


DEQ_CASES = [(Q4_0, 4, 64, 2048), (Q8_0, 4, 64, 2048), (Q4_0, 4, 8, 96), (Q8_0, 4, 8, 32),
             (Q4_0, 1, 9, 256), (Q8_0, 1, 7, 64), (Q4K, 1, 6, 1024), (Q6K, 1, 5, 768)]


@pytest.mark.parametrize("quant,il,rows,k", DEQ_CASES)
def test_dequant_bit_exact(ctx, zo, quant, il, rows, k):
    rng = np.random.default_rng(rows * 7 + k + quant)
    w = synth.weight(rng, quant, rows, k, il)
    # all 65,536 fp16 scale patterns appear across the scale slots
    if quant in (Q4_0, Q8_0):
        bb = 18 if quant == Q4_0 else 34
        nblk = w.size // bb
        sc = rng.integers(0, 65536, nblk, dtype=np.uint32).astype(np.uint16)
        if il == 4:
            g = w.reshape(rows // 4, k // 32, 4 * bb)
            g[..., :8] = sc.view(np.uint8).reshape(rows // 4, k // 32, 4, 2).reshape(rows // 4, k // 32, 8)
        else:
            w.reshape(nblk, bb)[:, :2] = sc.view(np.uint8).reshape(nblk, 2)
    out = torch.empty((rows, k), dtype=torch.float32, device="cuda")
    ctx.dequant_dev(dev(w), out, rows, k, quant, il, stream=torch.cuda.current_stream().cuda_stream)
    got = out.cpu().numpy()
    want = zo.dequant(w, rows, k, quant, il)
    assert same_bits(got, want)


@pytest.mark.parametrize("case", kats.DEQUANT, ids=lambda c: c[4])
def test_dequant_kats_on_gpu(ctx, case):
    quant, blk, checks, tol, src = case
    w = np.frombuffer(blk, np.uint8).copy()
    be, bb = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}[quant]
    k = (w.size // bb) * be
    out = torch.empty((1, k), dtype=torch.float32, device="cuda")
    ctx.dequant_dev(dev(w), out, 1, k, quant, 1, stream=torch.cuda.current_stream().cuda_stream)
    kats.check_dequant(out.cpu().numpy()[0], checks, tol)


@pytest.mark.parametrize("case", kats.LINEAR, ids=lambda c: c[7])
def test_linear_kats_through_abi(ctx, case):
    quant, k, n, x, wb, want, tol, src = case
    w = np.frombuffer(wb, np.uint8).copy()
    ctx.register(w, quant, 1)
    out = np.empty(n, np.float32)
    ctx.linear_dispatch(x, w, out, k, n, quant)
    np.testing.assert_allclose(out, want, atol=tol, rtol=0, err_msg=src)
    ctx.clear()


GEMV_CASES = [
    # (quant, interleave, rows, k)
    (Q4_0, 4, 6144, 2048),   # Qwen3-1.7B FFN up-proj (pair path)
    (Q4_0, 4, 2048, 6144),   # down-proj
    (Q8_0, 4, 4096, 2048),   # fused-QKV-sized Q8_0X4
    (Q4_0, 4, 4, 64),
    (Q4_0, 4, 12, 96),       # odd blocks per row: generic path
    (Q8_0, 4, 8, 32),
    (Q4_0, 1, 7, 256),       # plain layouts
    (Q8_0, 1, 100, 512),
    (Q4K, 1, 64, 4096),      # Q4_K strip path: 16 groups of four rows
    (Q4K, 1, 36, 6144),      # twelve strips per row (the down shape's in_dim)
    (Q4K, 1, 2052, 2048),    # 513 groups: two or three groups per workgroup, a partial last one
    (Q6K, 1, 48, 1024),      # Q6_K strip path (in_dim a multiple of 512)
    (Q6K, 1, 2048, 6144),    # the down shape: twelve strips
    (Q6K, 1, 1028, 2048),    # 257 groups, a partial last workgroup
    (Q4K, 1, 33, 2304),      # 9 superblocks per row: a partial 8-superblock step
    (Q6K, 1, 17, 2304),      # odd superblocks per row: unaligned Q6_K row starts
    (Q6K, 1, 8, 16384),      # in_dim above the LDS-staged limit: generic path
    (Q8_0, 4, 32768, 512),   # tall Q8_0X4 (LM-head strip path): one strip, four waves per strip
    (Q8_0, 4, 33000, 1024),  # tall strip path, last batch of two groups
    (Q8_0, 4, 32772, 4096),  # tall but in_dim above 2048: segment kernel, last group alone
    (Q4_0, 4, 151936, 2048), # tall Q4_0X4: the LDS-staged kernel, four groups per batch
    (Q4_0, 4, 49152, 2048),  # tall Q4_0X4 below the staging threshold: strip kernel batch loop
    (Q4_0, 4, 8320, 4096),   # tall at eight strips: 512-thread workgroups under a 512-thread bound
    (Q4_0, 4, 8208, 6144),   # tall at twelve strips: the fp32 form under the 1024-thread bound
    (Q8_0, 4, 32776, 2048),  # tall Q8_0X4 at in_dim 2048: LDS-staged kernel, last batch of two groups
    # DeepSeek2 / Kimi K2 projections through linear_dispatch_avx512
    # (kernel/src/inference_avx512.rs:2101-2825): MLA kv_a_mqa, q_a, q_b,
    # the kv_b decompressions, o_proj and the MoE expert FFN, Q4_0 as GGUF
    # rows (plain) and as .smodel X4 (Kimi K2 dims: hidden 7168, q_lora
    # 1536, kv_lora 512 + rope 64, 64 heads x (128 + 64), expert FFN 2048)
    (Q4_0, 4, 576, 7168),
    (Q4_0, 1, 576, 7168),
    (Q4_0, 4, 1536, 7168),
    (Q4_0, 4, 12288, 1536),
    (Q4_0, 1, 12288, 1536),
    (Q4_0, 4, 8192, 512),
    (Q4_0, 4, 7168, 8192),
    (Q4_0, 1, 7168, 8192),
    (Q4_0, 4, 2048, 7168),
    (Q4_0, 4, 7168, 2048),
    (Q4_0, 1, 2048, 7168),
    # DeepSeek-V2-Lite: expert FFN 1408 (44 blocks: an in_dim not a multiple of 64 blocks)
    (Q4_0, 4, 1408, 2048),
    (Q4_0, 4, 2048, 1408),
    (Q4_0, 1, 2048, 1408),
]


@pytest.mark.parametrize("quant,il,rows,k", GEMV_CASES)
def test_gemv_parity_host_api(ctx, zo, quant, il, rows, k):
    rng = np.random.default_rng(rows + 3 * k + quant)
    w = synth.weight(rng, quant, rows, k, il)
    x = synth.activations(rng, k)
    ctx.register(w, quant, il)
    assert ctx.group_of(w) == il
    out = np.empty(rows, np.float32)
    ctx.linear_dispatch(x, w, out, k, rows, quant)
    ref = zo.linear_range(x, w, k, rows, quant, il)
    f64 = zo.linear_f64(x, w, k, rows, quant, il)
    e_gpu, e_ref = rel_err(out, ref), rel_err(ref, f64)
    print(f"quant={quant} il={il} {rows}x{k}: rel err vs oracle {e_gpu:.2e}, oracle vs f64 {e_ref:.2e}, "
          f"gpu vs f64 {rel_err(out, f64):.2e}")
    assert e_gpu <= REL_TOL
    assert rel_err(out, f64) <= 4 * e_ref + 1e-6
    ctx.clear()


Q8X_CASES = [(Q4_0, 4, 6144, 2048), (Q8_0, 4, 4096, 2048), (Q4_0, 1, 2048, 6144), (Q4_0, 4, 12288, 1536),
             (Q8_0, 1, 64, 512), (Q8_0, 4, 151936, 2048)]


@pytest.mark.parametrize("quant,il,rows,k", Q8X_CASES)
def test_gemv_q8_0_activation(ctx, zo, quant, il, rows, k):
    """The GEMV on a Q8_0-encoded x (zg_linear_q8act_dev) against the oracle's
    Q8_0-activation GEMM at one row: the same per-block integer dots and
    dW * dX scales, summed in another order."""
    rng = np.random.default_rng(rows + k + il)
    w = synth.weight(rng, quant, rows, k, il)
    x = synth.activations(rng, k)
    xq = zo.quantize_q8_0(x)
    # the GPU encoder gives the same blocks
    qd = torch.empty(xq.size, dtype=torch.uint8, device="cuda")
    ctx.quantize_q8_0_dev(dev(x), qd, 1, k, stream=torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(qd.cpu().numpy(), xq)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.linear_q8act_dev(qd, dev(w), y, k, rows, quant, il, stream=torch.cuda.current_stream().cuda_stream)
    ref = zo.gemm_q8act(xq, w, 1, rows, k, quant, il)[0]
    got = y.cpu().numpy()
    print(f"Q8_0-activation GEMV quant={quant} il={il} {rows}x{k}: rel err {rel_err(got, ref):.2e}")
    assert rel_err(got, ref) <= 1e-5


def test_gemv_device_api_matches_host_api(ctx, zo):
    rng = np.random.default_rng(1)
    rows, k = 6144, 2048
    w = synth.weight(rng, Q4_0, rows, k, 4)
    x = synth.activations(rng, k)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.linear_dev(dev(x), dev(w), y, k, rows, Q4_0, 4, stream=torch.cuda.current_stream().cuda_stream)
    ctx.register(w, Q4_0, 4)
    out = np.empty(rows, np.float32)
    ctx.linear_dispatch(x, w, out, k, rows, Q4_0)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), out.view(np.uint32))
    ctx.clear()


@pytest.mark.parametrize("quant,il", [(Q4_0, 4), (Q8_0, 4), (Q4_0, 1), (Q8_0, 1), (Q4K, 1), (Q6K, 1)])
def test_row_ranges(ctx, zo, quant, il):
    rng = np.random.default_rng(2)
    rows, k = 40, 1024
    w = synth.weight(rng, quant, rows, k, il)
    x = synth.activations(rng, k)
    ctx.register(w, quant, il)
    ref = zo.linear_range(x, w, k, rows, quant, il)
    for s, e in ((0, 40), (1, 7), (13, 14), (20, 40), (5, 5)):
        out = np.full(rows, -7.0, np.float32)
        ctx.linear_range(x, w, out, k, rows, quant, s, e)
        assert np.all(out[:s] == -7.0) and np.all(out[e:] == -7.0)
        assert rel_err(out[s:e], ref[s:e]) <= REL_TOL if e > s else True
    ctx.clear()


def test_tall_q8_0_ranges(ctx, zo):
    """Row ranges of tall Q8_0X4 matrices (the LM head's register strip and
    LDS-staged paths): rows outside the range stay untouched, partial first
    and last groups."""
    rng = np.random.default_rng(9)
    for rows, k in ((32800, 1024), (32804, 2048)):  # register strip kernel; LDS-staged kernel
        w = synth.weight(rng, Q8_0, rows, k, 4)
        x = synth.activations(rng, k)
        ctx.register(w, Q8_0, 4)
        ref = zo.linear_range(x, w, k, rows, Q8_0, 4)
        for s, e in ((0, rows), (1, rows - 1), (6, rows - 23)):
            out = np.full(rows, -7.0, np.float32)
            ctx.linear_range(x, w, out, k, rows, Q8_0, s, e)
            assert np.all(out[:s] == -7.0) and np.all(out[e:] == -7.0)
            assert rel_err(out[s:e], ref[s:e]) <= REL_TOL
        ctx.clear()


def _edge_activations(rng, k, kind):
    """Activation vectors whose blocks stress the integer form of the tall
    launches (x scaled per 32-block to 22-bit integers): a zero block, a
    block of magnitudes below 1e-30 (no integer form: its wave decodes in
    fp32), a block spanning eight decades, and non-finite values."""
    x = synth.activations(rng, k)
    x[0:32] = 0.0
    x[64:96] = np.float32(1e-31) * rng.standard_normal(32).astype(np.float32)
    x[128:160] *= np.float32(1e-4)
    x[131] = 1e4
    if kind == "inf":
        x[700] = np.inf
    elif kind == "nan":
        x[1500] = np.nan
    return x


@pytest.mark.parametrize("kind", ["finite", "inf", "nan"])
@pytest.mark.parametrize("quant,rows,k", [(Q4_0, 12288, 2048), (Q4_0, 98304, 2048), (Q8_0, 32768, 2048)])
def test_tall_integer_activation_edges(ctx, zo, quant, rows, k, kind):
    """Tall X4 launches take the activations as exact integers (three int8
    digits per value, int32 dot chains): the register strip kernel's batch
    loop (12288 rows) and the LDS-staged kernel (98304 Q4_0 rows, 32768
    Q8_0 rows).  Finite edge
    blocks stay within the parity bar and as close to f64 as the oracle
    (x 4); non-finite inputs give non-finite rows exactly where the
    oracle's do."""
    rng = np.random.default_rng(rows + k + len(kind))
    w = synth.weight(rng, quant, rows, k, 4)
    x = _edge_activations(rng, k, kind)
    ctx.register(w, quant, 4)
    out = np.empty(rows, np.float32)
    ctx.linear_dispatch(x, w, out, k, rows, quant)
    ref = zo.linear_range(x, w, k, rows, quant, 4)
    ctx.clear()
    if kind == "finite":
        f64 = zo.linear_f64(x, w, k, rows, quant, 4)
        e_gpu, e_ref = rel_err(out, ref), rel_err(ref, f64)
        print(f"{kind} quant={quant}: rel err vs oracle {e_gpu:.2e}, oracle vs f64 {e_ref:.2e}, "
              f"gpu vs f64 {rel_err(out, f64):.2e}")
        assert e_gpu <= REL_TOL
        assert rel_err(out, f64) <= 4 * e_ref + 1e-6
    else:
        assert np.array_equal(np.isfinite(out), np.isfinite(ref))
        assert not np.isfinite(ref).any()


@pytest.mark.parametrize("il", [4, 1])
def test_fused_qkv_q8_0(ctx, zo, il):
    """Config 2: fused Q|K|V Q8_0, Qwen3-1.7B attention (2048 + 1024 + 1024) x 2048,
    in the X4 layout and in the plain (GGUF) layout."""
    rng = np.random.default_rng(3)
    k = 2048
    ws = [synth.weight(rng, Q8_0, n, k, il) for n in (2048, 1024, 1024)]
    x = synth.activations(rng, k)
    outs = [np.empty(w.size // (k // 32 * 34), np.float32) for w in ws]
    for w in ws:
        ctx.register(w, Q8_0, il)
    ctx.linear_fused_dispatch(x, [(w, o, Q8_0) for w, o in zip(ws, outs)], k)
    for w, o in zip(ws, outs):
        ref = zo.linear_range(x, w, k, o.size, Q8_0, il)
        assert rel_err(o, ref) <= REL_TOL
    ctx.clear()


@pytest.mark.parametrize("types", [(Q4K, Q4K, Q4K), (Q4K, Q4K, Q6K), (Q6K, Q4K, Q4K)])
def test_fused_qkv_kquants(ctx, zo, types):
    """Q|K|V in K-quants (the Q4_K_M pattern): Q4_K segments share one
    segmented strip launch (a leading run of two when V is Q6_K); the rest
    go one by one."""
    rng = np.random.default_rng(sum(types))
    k = 2048
    ws = [synth.weight(rng, t, n, k, 1) for t, n in zip(types, (2048, 1024, 1024))]
    x = synth.activations(rng, k)
    outs = [np.empty(n, np.float32) for n in (2048, 1024, 1024)]
    for w, t in zip(ws, types):
        ctx.register(w, t, 1)
    ctx.linear_fused_dispatch(x, [(w, o, t) for w, o, t in zip(ws, outs, types)], k)
    for w, o, t in zip(ws, outs, types):
        ref = zo.linear_range(x, w, k, o.size, t, 1)
        assert rel_err(o, ref) <= REL_TOL
    ctx.clear()


@pytest.fixture(scope="module")
def lm_head():
    rng = np.random.default_rng(4)
    V, H = kats.VOCAB_SIZE_PADDED, 2048
    plain = synth.weight(rng, Q8_0, V, H, 1)
    plain.reshape(V, -1)[kats.VOCAB_SIZE_REAL:] = 0  # padding rows
    w = synth.interleave_x4(plain, V, H, Q8_0)
    hidden = synth.activations(rng, H)
    norm = (1 + 0.05 * rng.standard_normal(H)).astype(np.float32)
    return w, hidden, norm


def test_lm_head_argmax(ctx, zo, lm_head):
    """Config 2: LM head Q8_0X4 151936 x 2048 with fused rmsnorm + argmax."""
    w, hidden, norm = lm_head
    V, H = kats.VOCAB_SIZE_PADDED, 2048
    ctx.register(w, Q8_0, 4)
    logits = np.empty(V, np.float32)
    tok = ctx.lm_head_argmax(hidden, norm, w, Q8_0, 1e-6, H, logits_buf=logits)
    xn = np.empty(H, np.float32)
    zo.load().zo_rmsnorm(hidden.ctypes.data, norm.ctypes.data, xn.ctypes.data, H, 1e-6)
    with zo.Pool(8):
        ref = zo.linear_parallel(xn, w, H, V, Q8_0, 4)
    assert rel_err(logits, ref) <= REL_TOL
    idx, val = zo.argmax(ref)
    top2 = np.sort(ref)[-2:]
    print(f"LM head: argmax {tok} (oracle {idx}), margin {top2[1] - top2[0]:.4f}, rel err {rel_err(logits, ref):.2e}")
    assert tok == idx and tok == int(np.argmax(logits))
    ctx.clear()


def test_lm_head_argmax_plain_q8_0(ctx, zo, lm_head):
    """The same LM head in the plain (GGUF) Q8_0 layout."""
    w4, hidden, norm = lm_head
    V, H = kats.VOCAB_SIZE_PADDED, 2048
    w = synth.deinterleave_x4(w4, V, H, Q8_0)
    ctx.register(w, Q8_0, 1)
    logits = np.empty(V, np.float32)
    tok = ctx.lm_head_argmax(hidden, norm, w, Q8_0, 1e-6, H, logits_buf=logits)
    xn = np.empty(H, np.float32)
    zo.load().zo_rmsnorm(hidden.ctypes.data, norm.ctypes.data, xn.ctypes.data, H, 1e-6)
    with zo.Pool(8):
        ref = zo.linear_parallel(xn, w, H, V, Q8_0, 1)
    assert rel_err(logits, ref) <= REL_TOL
    assert tok == zo.argmax(ref)[0]
    ctx.clear()


@pytest.mark.parametrize("qt,H", [(Q6K, 4096), (Q4K, 4096), (Q6K, 8192)])
def test_lm_head_argmax_kquant(ctx, zo, qt, H):
    """LM head in Q6_K (the output.weight type of Q4_K_M GGUF artifacts) and
    Q4_K (OutputQuant::Q4K, kernel/src/inference.rs:3119-3125); Q6_K at
    in_dim 8192 takes the LDS-activation kernel with the argmax epilogue."""
    rng = np.random.default_rng(5 + qt + H)
    V = 32000
    w = synth.weight(rng, qt, V, H, 1)
    hidden = synth.activations(rng, H)
    norm = (1 + 0.05 * rng.standard_normal(H)).astype(np.float32)
    ctx.register(w, qt, 1)
    logits = np.empty(V, np.float32)
    tok = ctx.lm_head_argmax(hidden, norm, w, qt, 1e-6, H, vocab_padded=V, vocab_real=V, logits_buf=logits)
    xn = np.empty(H, np.float32)
    zo.load().zo_rmsnorm(hidden.ctypes.data, norm.ctypes.data, xn.ctypes.data, H, 1e-6)
    with zo.Pool(8):
        ref = zo.linear_parallel(xn, w, H, V, qt, 1)
    assert rel_err(logits, ref) <= REL_TOL
    idx, _ = zo.argmax(ref)
    assert tok == idx
    ctx.clear()


def test_lm_head_errors(ctx, lm_head):
    w, hidden, norm = lm_head
    V, H = kats.VOCAB_SIZE_PADDED, 2048
    ctx.register(w, Q8_0, 4)
    bad = hidden.copy()
    bad[3] = np.nan
    with pytest.raises(zero_amd.NonFiniteLogits):
        ctx.lm_head_argmax(bad, norm, w, Q8_0, 1e-6, H)
    # a vocab_real below the argmax puts it in the padding region
    tok = ctx.lm_head_argmax(hidden, norm, w, Q8_0, 1e-6, H)
    with pytest.raises(zero_amd.ArgmaxInPaddingRegion) as ei:
        ctx.lm_head_argmax(hidden, norm, w, Q8_0, 1e-6, H, vocab_real=tok)
    assert ei.value.index == tok
    ctx.clear()


def test_registry_semantics(ctx):
    """weight_layout.rs:155-170: sorted registry, exact-start lookups,
    interior pointers are plain, clear() empties it; rebase shifts keys."""
    fake = torch.empty(64, dtype=torch.uint8, device="cuda")
    for key in (0x5000, 0x1000, 0x3000):
        ctx.register_device(key, fake.data_ptr(), 36, Q4_0, 4)
    assert ctx.registered_count() == 3
    for key in (0x1000, 0x3000, 0x5000):
        assert ctx.group_of(key) == 4
    assert ctx.group_of(0x3010) == 1 and ctx.group_of(0) == 1
    ctx.rebase(0x100)
    assert ctx.group_of(0x1100) == 4 and ctx.group_of(0x1000) == 1
    ctx.clear()
    assert ctx.group_of(0x1100) == 1 and ctx.registered_count() == 0


def test_dispatch_errors(ctx):
    w = synth.weight(np.random.default_rng(0), Q4_0, 4, 64, 1)
    x = np.zeros(64, np.float32)
    out = np.empty(4, np.float32)
    with pytest.raises(zero_amd.LinearDispatchError):  # ops.rs:513-521 panics on F16
        ctx.linear_dispatch(x, w, out, 64, 4, zero_amd.GgmlType.F16)
    with pytest.raises(zero_amd.ZgError) as ei:  # not uploaded
        ctx.linear_dispatch(x, w, out, 64, 4, Q4_0)
    assert ei.value.code == -3
    ctx.register(w, Q4_0, 1)
    with pytest.raises(zero_amd.ZgError):  # registered as Q4_0, called as Q8_0
        ctx.linear_dispatch(x, w, out, 64, 4, Q8_0)
    # interior pointer of a plain tensor resolves to that row (weight_layout.rs:13-19)
    row = w[36:]
    x = synth.activations(np.random.default_rng(1), 64)
    full = np.empty(4, np.float32)
    ctx.linear_dispatch(x, w, full, 64, 4, Q4_0)
    tail = np.empty(3, np.float32)
    ctx.linear_dispatch(x, row, tail, 64, 3, Q4_0)
    assert np.array_equal(tail, full[1:])
    ctx.clear()


@pytest.mark.parametrize("quant,rows,k", [(Q4K, 14336, 4096), (Q6K, 4096, 14336)])
def test_kquant_llama3_shapes(ctx, zo, quant, rows, k):
    """Config 4: Q4_K gate/up 14336x4096 and Q6_K down 4096x14336."""
    rng = np.random.default_rng(rows)
    w = synth.weight(rng, quant, rows, k, 1)
    x = synth.activations(rng, k)
    ctx.register(w, quant, 1)
    out = np.empty(rows, np.float32)
    ctx.linear_dispatch(x, w, out, k, rows, quant)
    with zo.Pool(8):
        ref = zo.linear_parallel(x, w, k, rows, quant, 1)
    print(f"quant={quant} {rows}x{k}: rel err {rel_err(out, ref):.2e}")
    assert rel_err(out, ref) <= REL_TOL
    ctx.clear()
