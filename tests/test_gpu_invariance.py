"""Bitwise invariance of GEMV rows under launch geometry, the GPU analogue of
the reference's contract that a parallel split equals the single-core
result bit for bit (kernel/src/smp.rs:33-40, self-test at
kernel/src/inference_avx512.rs:2007).

Each output row is reduced by one fixed lane order and one fixed strip order
whatever the grid, groups per batch or segment table, so a row's bits may
only depend on the kernel form (the fp32 decode of one-batch launches, the
integer-activation decode of tall batch-loop launches, the K-quant unit).
These tests pick row ranges and fused tables that stay in one form and
require identical bits.
"""
import numpy as np
import pytest

from zero_amd import synth

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4K, Q6K = 2, 8, 12, 14


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# (quant, interleave, rows, k, ranges): ranges small enough to stay one-batch
# launches when the full matrix is one (fp32 decode), or large enough to stay
# batch-loop launches when it is tall (integer-activation decode)
CASES = [
    (Q4_0, 4, 6144, 2048, [(0, 6144), (4, 3000), (1, 6143), (2048, 2052), (5000, 5001)]),
    (Q4_0, 4, 2048, 6144, [(0, 2048), (7, 1100), (1024, 2048)]),
    (Q8_0, 4, 4096, 2048, [(0, 4096), (3, 2049), (2048, 4096)]),
    (Q4_0, 1, 6144, 2048, [(0, 6144), (4, 3000), (6140, 6144)]),
    (Q4K, 1, 6144, 2048, [(0, 6144), (4, 3000), (6000, 6144)]),
    (Q6K, 1, 2048, 6144, [(0, 2048), (4, 1000), (1999, 2048)]),
    (Q4_0, 4, 151936, 2048, [(0, 151936), (1000, 120000), (3, 151933)]),
    (Q8_0, 4, 151936, 2048, [(0, 151936), (996, 140000)]),
]


@pytest.mark.parametrize("quant,il,rows,k,ranges", CASES,
                         ids=[f"q{c[0]}-il{c[1]}-{c[2]}x{c[3]}" for c in CASES])
def test_range_rows_equal_full_launch_bits(ctx, quant, il, rows, k, ranges):
    """zg_linear_range rows equal the same rows of zg_linear, bit for bit."""
    rng = np.random.default_rng(rows + k + quant)
    w = synth.weight(rng, quant, rows, k, il)
    x = synth.activations(rng, k)
    ctx.register(w, quant, il)
    try:
        full = np.empty(rows, np.float32)
        ctx.linear_dispatch(x, w, full, k, rows, quant)
        for s, e in ranges:
            out = np.full(rows, -7.0, np.float32)
            ctx.linear_range(x, w, out, k, rows, quant, s, e)
            assert np.array_equal(bits(out[s:e]), bits(full[s:e])), (s, e)
            assert np.all(out[:s] == -7.0) and np.all(out[e:] == -7.0)
        # the same call again: identical bits (no run-to-run variation)
        again = np.empty(rows, np.float32)
        ctx.linear_dispatch(x, w, again, k, rows, quant)
        assert np.array_equal(bits(again), bits(full))
    finally:
        ctx.clear()


@pytest.mark.parametrize("quant,il,dims", [
    (Q4_0, 4, (2048, 1024, 1024)),   # Qwen3-1.7B Q|K|V
    (Q8_0, 4, (2048, 1024, 1024)),
    (Q4_0, 4, (3072, 3072)),         # a gate|up pair without the SwiGLU epilogue (one-batch)
    (Q4K, 1, (2048, 1024, 1024)),
])
def test_fused_segments_equal_single_projection_bits(ctx, quant, il, dims):
    """A projection's rows in a fused launch (linear_fused_dispatch,
    inference_avx512.rs:890-945) equal the rows of its own launch, bit for bit,
    when both are one-batch launches (a fused table past 2,048 groups of
    in_dim 2048 runs the tall integer-activation form instead)."""
    rng = np.random.default_rng(sum(dims) + quant)
    k = 2048
    ws = [synth.weight(rng, quant, n, k, il) for n in dims]
    x = synth.activations(rng, k)
    for w in ws:
        ctx.register(w, quant, il)
    try:
        fused = [np.empty(n, np.float32) for n in dims]
        ctx.linear_fused_dispatch(x, [(w, o, quant) for w, o in zip(ws, fused)], k)
        for w, n, f in zip(ws, dims, fused):
            single = np.empty(n, np.float32)
            ctx.linear_dispatch(x, w, single, k, n, quant)
            assert np.array_equal(bits(f), bits(single))
    finally:
        ctx.clear()
