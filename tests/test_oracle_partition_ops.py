"""Pins the partition math (smp_partition.rs:226-401 properties), the
decode-step scalar ops (ops.rs:530-772 KATs incl. the 16 gguf-py RoPE
values), softmax/SiLU closed forms and the argmax semantics
(lm_head.rs:174-201, linear.rs:538-609, inference_avx512.rs:1027-1044)."""
import ctypes as C

import numpy as np
import pytest

from golden import kats


def test_split_properties(zo):
    r = [zo.row_range_for(100, 8, i, 1) for i in range(8)]
    lens = [e - s for s, e in r]
    assert sum(lens) == 100 and max(lens) - min(lens) <= 1
    r = [zo.row_range_for(3, 8, i, 1) for i in range(8)]
    assert [e - s for s, e in r] == [1, 1, 1, 0, 0, 0, 0, 0]
    assert all(s == e for s, e in (zo.row_range_for(0, 8, i, 4) for i in range(8)))


def test_aligned_boundaries(zo):
    prev = 0
    for i in range(64):
        s, e = zo.row_range_for(151_936, 64, i, 4)
        assert s % 4 == 0 and e % 4 == 0 and s == prev
        prev = e
    assert prev == 151_936
    cur = 0
    for i in range(8):
        s, e = zo.row_range_for(103, 8, i, 4)
        assert s == cur and (e == 103 or e % 4 == 0)
        cur = max(cur, e)
    assert cur == 103


@pytest.mark.parametrize("total,n,align", kats.PARTITION_CLOSED_FORM)
def test_closed_form_matches_split(zo, total, n, align):
    # split_rows_aligned: even split of ceil(total/align) units, clamp
    units = -(-total // align) if align > 1 else total
    base, extra = divmod(units, n) if n else (0, 0)
    cur = 0
    for i in range(n):
        take = base + (1 if i < extra else 0)
        s, e = min(cur * align, total), min((cur + take) * align, total)
        assert zo.row_range_for(total, n, i, align) == (s, e)
        assert zo.row_range_for(total, n, i, align, discount=0) == (s, e)
        cur += take


@pytest.mark.parametrize("total,n,align", kats.PARTITION_DISCOUNT)
def test_discounted_contiguous_complete(zo, total, n, align):
    for d in kats.PARTITION_DISCOUNTS:
        cur = 0
        for i in range(n):
            s, e = zo.row_range_for(total, n, i, align, discount=d)
            assert s == cur or s == e == total
            assert s <= e
            cur = max(cur, e)
        assert cur == total


def test_discount_shrinks_bsp(zo):
    even = zo.row_range_for(151_936, 64, 0, 4)
    disc = zo.row_range_for(151_936, 64, 0, 4, discount=25)
    assert disc[1] - disc[0] < even[1] - even[0]
    ap_e = zo.row_range_for(151_936, 64, 1, 4)
    ap_d = zo.row_range_for(151_936, 64, 1, 4, discount=25)
    assert ap_d[1] - ap_d[0] >= ap_e[1] - ap_e[0]


@pytest.mark.parametrize("x,w,want,tol,src", kats.RMSNORM)
def test_rmsnorm_kats(zo, x, w, want, tol, src):
    x = np.array(x, np.float32)
    out = np.full(x.size, 99.0, np.float32)
    zo.load().zo_rmsnorm(x.ctypes.data, np.array(w, np.float32).ctypes.data, out.ctypes.data, x.size, 1e-6)
    np.testing.assert_allclose(out, want, atol=tol, rtol=0, err_msg=src)
    assert np.all(np.isfinite(out))


def test_rmsnorm_unit_rms(zo):
    x = np.array(kats.RMSNORM_UNIT_RMS[0], np.float32)
    out = np.empty_like(x)
    zo.load().zo_rmsnorm(x.ctypes.data, np.ones_like(x).ctypes.data, out.ctypes.data, x.size, 1e-6)
    assert abs(np.sqrt(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 1e-3


def _rope(zo, half, base, pos, x):
    inv = np.empty(half, np.float32)
    zo.load().zo_rope_inv_freqs(inv.ctypes.data, half, base)
    q = np.array(x, np.float32)
    zo.load().zo_rope(q.ctypes.data, inv.ctypes.data, half, pos)
    return q, inv


@pytest.mark.parametrize("half,base,pos,x,want,tol,src", kats.ROPE)
def test_rope_kats(zo, half, base, pos, x, want, tol, src):
    q, _ = _rope(zo, half, base, pos, x)
    np.testing.assert_allclose(q[:len(want)], want, atol=tol, rtol=0, err_msg=src)


def test_rope_identity_and_inv_freq(zo):
    half, base, x, _ = kats.ROPE_IDENTITY
    q, _ = _rope(zo, half, base, 0, x)
    np.testing.assert_allclose(q, x, atol=1e-6)
    _, inv = _rope(zo, 64, 1e6, 0, [0.0] * 128)
    for i, v, tol in kats.ROPE_INV_FREQ:
        assert abs(inv[i] - v) < tol
    assert 0 < inv[63] < 1e-3
    _, inv1 = _rope(zo, 64, 1.0, 0, [0.0] * 128)
    assert np.allclose(inv1, 1.0)


def test_softmax_and_silu_closed_form(zo):
    rng = np.random.default_rng(4)
    s = rng.standard_normal(300).astype(np.float32) * 5
    p = s.copy()
    assert zo.load().zo_softmax(p.ctypes.data, p.size) == 0
    e = np.exp(s.astype(np.float64) - s.max())
    np.testing.assert_allclose(p, e / e.sum(), rtol=1e-5, atol=1e-9)
    bad = np.array([np.inf, 1.0], np.float32)
    assert zo.load().zo_softmax(bad.ctypes.data, 2) != 0
    g, u = rng.standard_normal(64).astype(np.float32), rng.standard_normal(64).astype(np.float32)
    out = np.empty(64, np.float32)
    zo.load().zo_silu_mul(g.ctypes.data, u.ctypes.data, out.ctypes.data, 64)
    gd = g.astype(np.float64)
    np.testing.assert_allclose(out, gd / (1 + np.exp(-gd)) * u, rtol=1e-5, atol=1e-7)


def test_argmax_semantics(zo):
    a = kats.ARGMAX_BASIC
    v = np.full(kats.VOCAB_SIZE_PADDED, a["fill"], np.float32)
    for i, x in a["set"].items():
        v[i] = x
    assert zo.argmax(v) == (a["index"], a["value"])
    v = np.array([1.0, np.nan, 3.0, 3.0, -np.inf], np.float32)
    assert zo.argmax(v) == (2, 3.0)  # first max wins, NaN suppressed
    assert zo.argmax(np.array([np.nan, np.nan], np.float32))[1] == -np.inf
    beats = zo.load().zo_argmax_beats
    assert beats(2.0, 5, 1.0, 1) and not beats(1.0, 1, 2.0, 5)
    assert beats(2.0, 3, 2.0, 4) and not beats(2.0, 4, 2.0, 3)
    assert beats(0.0, 1, -0.0, 2)  # +-0 compare equal; smaller index wins
