"""Pins the oracle's GEMV restatements.

* scalar crate operators (ops.rs:179-457) and the AVX-512 range kernels
  (linear.rs:150-1213) against the reference's linear KATs (ops.rs:953-1160);
* both against an f64 brute-force dot (a dropped term, a wrong sign or a
  transposed block would exceed the fp32 rounding bound by orders of
  magnitude);
* invariants the reference states: the X4 kernel equals the plain kernel
  bit for bit (linear.rs:887-895), any row split equals the full range bit
  for bit (smp.rs:33-40, inference_avx512.rs:1989-2062), fused dispatch
  equals separate dispatches (inference_avx512.rs:726-731).
"""
import numpy as np
import pytest

from golden import kats
from zero_amd import synth


@pytest.mark.parametrize("case", kats.LINEAR, ids=lambda c: c[7])
def test_linear_kats_scalar_and_range(zo, case):
    quant, k, n, x, wb, want, tol, src = case
    w = np.frombuffer(wb, np.uint8).copy()
    for got in (zo.linear_scalar(x, w, k, n, quant), zo.linear_range(x, w, k, n, quant, 1)):
        np.testing.assert_allclose(got, want, atol=tol, rtol=0, err_msg=src)
    if n % 4 == 0:
        x4 = zo.interleave_x4(w, n, k, quant)
        np.testing.assert_allclose(zo.linear_range(x, x4, k, n, quant, 4), want, atol=tol, rtol=0)


SHAPES = [(2, 64, 256), (8, 32, 96), (8, 2048, 64), (12, 12, 512), (14, 8, 1024)]


def _err_vs_f64(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("quant,n,k", [(q, n, k) for q, n, k in
                                      [(2, 64, 256), (8, 32, 96), (2, 8, 2048), (8, 12, 512), (12, 8, 1024),
                                       (14, 8, 1024), (12, 4, 4096), (14, 4, 2048)]])
def test_kernels_vs_f64(zo, quant, n, k):
    rng = np.random.default_rng(n * 131 + k + quant)
    w = synth.weight(rng, quant, n, k, 1)
    x = synth.activations(rng, k)
    ref = zo.linear_f64(x, w, k, n, quant)
    # fp32 accumulation over k terms: error bound ~ k * eps relative to sum |x w|
    bound = 2e-6 * np.sqrt(k)
    assert _err_vs_f64(zo.linear_scalar(x, w, k, n, quant), ref) < bound
    assert _err_vs_f64(zo.linear_range(x, w, k, n, quant), ref) < bound


@pytest.mark.parametrize("quant", [2, 8])
def test_x4_equals_plain_bitwise(zo, quant):
    rng = np.random.default_rng(7)
    n, k = 64, 512
    plain = synth.weight(rng, quant, n, k, 1)
    x4 = synth.interleave_x4(plain, n, k, quant)
    x = synth.activations(rng, k)
    a = zo.linear_range(x, plain, k, n, quant, 1)
    b = zo.linear_range(x, x4, k, n, quant, 4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("quant,il", [(2, 4), (8, 4), (2, 1), (12, 1), (14, 1)])
def test_row_split_equals_full(zo, quant, il):
    rng = np.random.default_rng(11)
    n, k = 40, 512
    w = synth.weight(rng, quant, n, k, il)
    x = synth.activations(rng, k)
    full = zo.linear_range(x, w, k, n, quant, il)
    for cuts in ([0, 1, 7, 20, 33, 40], [0, 4, 8, 40], [0, 13, 14, 40]):
        out = np.full(n, np.nan, np.float32)
        for s, e in zip(cuts[:-1], cuts[1:]):
            zo.linear_range(x, w, k, n, quant, il, s, e, out=out)
        assert np.array_equal(out.view(np.uint32), full.view(np.uint32)), cuts


def test_parallel_and_fused_equal_single(zo):
    rng = np.random.default_rng(3)
    k = 1024
    ws = [synth.weight(rng, 2, n, k, 4) for n in (256, 128, 128)]
    x = synth.activations(rng, k)
    single = [zo.linear_range(x, w, k, w.size // (k // 32 * 18), 2, 4) for w in ws]
    with zo.Pool(4):
        par = [zo.linear_parallel(x, w, k, s.size, 2, 4) for w, s in zip(ws, single)]
        outs = [np.empty_like(s) for s in single]
        import ctypes as C
        segs = (zo.zo_segment * 3)(*[zo.zo_segment(w.ctypes.data, o.ctypes.data, o.size, 2, 4)
                                     for w, o in zip(ws, outs)])
        assert zo.load().zo_linear_fused_parallel(x.ctypes.data, segs, 3, k) == 0
    for a, b, c in zip(single, par, outs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))


def test_lm_head_parallel_argmax_matches_sequential_scan(zo):
    rng = np.random.default_rng(5)
    n, k = 2048, 256
    w = synth.weight(rng, 8, n, k, 4)
    x = synth.activations(rng, k)
    import ctypes as C
    logits = np.empty(n, np.float32)
    mv = C.c_float()
    with zo.Pool(8):
        idx = zo.load().zo_lm_head_linear_argmax_parallel(x.ctypes.data, w.ctypes.data, logits.ctypes.data, k, n,
                                                          8, 4, C.byref(mv))
    assert idx == int(np.argmax(logits)) and mv.value == logits.max()
