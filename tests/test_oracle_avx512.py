"""The AVX-512 intrinsics restatement of the reference's range kernels
(oracle/zg_avx512.c, the CPU baseline) against the oracle's lane-order
restatement (zo_linear_range, pinned by the reference's KATs and f64 brute
force in test_oracle_linear.py).

Both follow kernel/src/arch/x86_64/math/linear.rs (Q4_0X4 :909-1072,
Q8_0X4 :1096-1213, plain Q4_0 :710-859, plain Q8_0 :1271-1402, Q4_K
:150-306, Q6_K :352-504): the same per-lane fma chains and the same
_mm512_reduce_add_ps tree, so every row must agree bit for bit, on full,
ragged and odd-length row ranges (the plain kernels pair rows; an odd last
row takes the single-row body).
"""
import numpy as np
import pytest

from oracle import zo
from zero_amd import synth

pytestmark = pytest.mark.skipif(not zo.avx512_available(), reason="host CPU has no AVX-512F")

CASES = [
    (synth.Q4_0, 4, 64, 2048), (synth.Q8_0, 4, 64, 2048), (synth.Q4_0, 1, 37, 1024), (synth.Q8_0, 1, 37, 1024),
    (synth.Q4K, 1, 23, 4096), (synth.Q6K, 1, 21, 2304), (synth.Q4_0, 4, 4, 32), (synth.Q8_0, 1, 1, 32),
]


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("quant,il,rows,k", CASES)
def test_avx512_bit_identical_to_lane_order(quant, il, rows, k):
    rng = np.random.default_rng(rows * 7 + k + quant)
    w = synth.weight(rng, quant, rows, k, il)
    x = synth.activations(rng, k)
    ref = zo.linear_range(x, w, k, rows, quant, il)
    got = zo.linear_range_avx512(x, w, k, rows, quant, il)
    assert np.array_equal(_bits(got), _bits(ref)), np.flatnonzero(_bits(got) != _bits(ref))[:8]
    # ragged ranges: rows outside [s, e) stay untouched
    for s, e in ((1, rows - 1), (min(2, rows - 1), rows), (0, 1), (rows // 2, rows // 2 + 3)):
        e = min(e, rows)
        if s >= e:
            continue
        o = np.full(rows, -7.0, np.float32)
        zo.linear_range_avx512(x, w, k, rows, quant, il, s, e, out=o)
        assert np.array_equal(_bits(o[s:e]), _bits(ref[s:e]))
        assert np.all(o[:s] == -7.0) and np.all(o[e:] == -7.0)


def test_special_values():
    """Subnormal and zero fp16 scales, -0 activations, all-zero blocks."""
    rng = np.random.default_rng(5)
    k, rows = 512, 8
    for quant, il in ((synth.Q4_0, 4), (synth.Q8_0, 1), (synth.Q4K, 1), (synth.Q6K, 1)):
        w = synth.weight(rng, quant, rows, k, il)
        x = synth.activations(rng, k)
        x[::7] = -0.0
        x[5] = 1e-38
        if quant in (synth.Q4_0, synth.Q8_0) and il == 1:
            bb = 18 if quant == synth.Q4_0 else 34
            w[0:2] = (1, 0)  # smallest subnormal d in row 0 block 0
            w[bb:bb + 2] = 0  # d = 0
        ref = zo.linear_range(x, w, k, rows, quant, il)
        got = zo.linear_range_avx512(x, w, k, rows, quant, il)
        assert np.array_equal(_bits(got), _bits(ref))


def test_pool_dispatch_uses_intrinsics_bitwise():
    """zo_set_simd(1) routes the pinned pool's slices (row_range_for, align
    = interleave) through the intrinsics; the rows equal the scalar pool's."""
    rng = np.random.default_rng(9)
    w = synth.weight(rng, synth.Q4_0, 512, 2048, 4)
    x = synth.activations(rng, 2048)
    with zo.Pool(4):
        zo.set_simd(False)
        ref = zo.linear_parallel(x, w, 2048, 512, synth.Q4_0, 4)
        assert zo.set_simd(True)
        got = zo.linear_parallel(x, w, 2048, 512, synth.Q4_0, 4)
        zo.set_simd(False)
    assert np.array_equal(_bits(got), _bits(ref))


def test_model_forward_with_intrinsics_bitwise():
    """The forward pass with the intrinsics in force (the CPU decode
    baseline: AVX-512 GEMVs, and from 64 cached rows on the attention heads
    spread over the pool, inference_avx512.rs:1676-1730) gives the scalar
    restatement's hidden states bit for bit."""
    cfg = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                            vocab_padded=1024, vocab_real=1000, max_ctx=80)
    model = synth.random_model(cfg, seed=4)
    outs = {}
    with zo.Pool(3):
        for simd in (False, True):
            assert zo.set_simd(simd) == simd
            om = zo.OracleModel(model)
            tok, hs = 3, []
            for pos in range(72):  # crosses the 64-row parallel-attention threshold
                hs.append(om.forward(tok, pos))
                rc, tok, _, _ = om.lm_head()
                assert rc == 0
            om.close()
            outs[simd] = np.stack(hs)
        zo.set_simd(False)
    assert np.array_equal(_bits(outs[True]), _bits(outs[False]))
