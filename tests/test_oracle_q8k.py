"""Pins the oracle's restatement of the Q4_K x Q8_K integer path
(kernel/src/arch/x86_64/math/vnni.rs, feature "vnni-acceleration"; the
reference has no host-side tests for it, vnni.rs:480-487):

* unpack_mins_and_scales (ggml's utmp form) against the textbook
  get_scale_min_k4 rule on random and all-ones scale bytes;
* quantize_row_q8k against its defining properties (the first value of
  largest magnitude maps to -127, |x - d q| <= |d|/2, int16 sums of 16,
  zero blocks) and a numpy float32 restatement;
* linear_q4k_vnni_range against an f64 brute force over the dequantized
  Q4_K weights and the dequantized Q8_K activations (the integer
  regrouping is exact, so only the final f32 roundings differ), and
  against the fp32 Q4_K path within the activation-quantization error.
"""
import numpy as np
import pytest

from zero_amd import synth


def _scale_min_k4(s, j):
    """get_scale_min_k4 (dequant.rs:75-85, the ggml rule)."""
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)


def test_unpack_mins_and_scales_matches_get_scale_min_k4(zo):
    rng = np.random.default_rng(0)
    cases = [rng.integers(0, 256, 12, dtype=np.uint8) for _ in range(500)]
    cases += [np.full(12, 0xFF, np.uint8), np.zeros(12, np.uint8), np.arange(12, dtype=np.uint8) * 21]
    for s in cases:
        got = zo.unpack_mins_and_scales(s)
        want = [_scale_min_k4([int(v) for v in s], j) for j in range(8)]
        assert list(got[:8]) == [w[0] for w in want] and list(got[8:]) == [w[1] for w in want]


def _np_q8k(x):
    """quantize_row_q8k in numpy float32: (d, q int8[256], bsums int16[16]) per block."""
    out = []
    for blk in x.reshape(-1, 256):
        a = np.abs(blk)
        amax = a.max()
        if amax == 0:
            out.append((np.float32(0), np.zeros(256, np.int8), np.zeros(16, np.int16)))
            continue
        max_val = blk[int(np.argmax(a))]  # argmax: the first occurrence
        iscale = np.float32(-127.0) / max_val
        q = np.clip(np.rint(blk * iscale), -128, 127).astype(np.int32)
        out.append((np.float32(1.0) / iscale, q.astype(np.int8), q.reshape(16, 16).sum(1).astype(np.int16)))
    return out


def _unpack_q8k(buf):
    blocks = buf.reshape(-1, 292)
    return [(b[:4].view(np.float32)[0], b[4:260].view(np.int8), b[260:].view(np.int16)) for b in blocks]


@pytest.mark.parametrize("seed,scale", [(1, 1.0), (2, 1e-3), (3, 300.0), (4, 1e-30)])
def test_quantize_q8k_properties(zo, seed, scale):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(4096) * scale).astype(np.float32)
    x[256:512] = 0.0                      # an all-zero block
    x[512 + 7], x[512 + 90] = -50.0 * scale, 50.0 * scale  # equal magnitude: the first (negative) wins
    got = _unpack_q8k(zo.quantize_q8k(x))
    want = _np_q8k(x)
    for b, ((d, q, bs), (wd, wq, wbs)) in enumerate(zip(got, want)):
        blk = x[256 * b:256 * (b + 1)].astype(np.float64)
        assert d.view(np.uint32) == np.float32(wd).view(np.uint32)
        assert np.array_equal(q, wq) and np.array_equal(bs, wbs)
        if b == 1:
            assert d == 0 and not q.any() and not bs.any()
            continue
        i = int(np.argmax(np.abs(blk)))
        assert q[i] == -127
        assert np.all(np.abs(blk - float(d) * q.astype(np.float64)) <= abs(float(d)) * (0.5 + 1e-5))
        assert np.array_equal(bs, q.astype(np.int32).reshape(16, 16).sum(1))
    assert got[2][0] > 0 and got[2][1][7] == -127  # max_val = -50: d > 0, q keeps the sign


def _q8k_dequant(buf, k):
    return np.concatenate([float(d) * q.astype(np.float64) for d, q, _ in _unpack_q8k(buf)])[:k]


@pytest.mark.parametrize("rows,k", [(16, 256), (40, 2048), (7, 4096)])
def test_linear_q4k_q8k_vs_f64(zo, rows, k):
    rng = np.random.default_rng(rows + k)
    w = synth.q4k(rng, rows, k)
    x = synth.activations(rng, k)
    q8 = zo.quantize_q8k(x)
    got = zo.linear_q4k_q8k(q8, w, k, rows)
    wd = zo.dequant(w, rows, k, 12).astype(np.float64)
    ref = wd @ _q8k_dequant(q8, k)
    err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    assert err < 1e-5, err
    # a row range touches only its rows
    part = zo.linear_q4k_q8k(q8, w, k, rows, start=3, end=5)
    assert np.array_equal(part[3:5], got[3:5]) and not part[:3].any() and not part[5:].any()
    # the fp32 Q4_K path differs by the activation quantization only
    fp = zo.linear_range(x, w, k, rows, 12)
    q_err = np.max(np.abs(got - fp)) / np.max(np.abs(fp))
    assert 1e-5 < q_err < 3e-2, q_err


def test_linear_q4k_q8k_kat(zo):
    """One superblock, all scale/min bytes 0x01 (sc = m = 1 for every
    sub-block), d = 1, dmin = 0, every nibble 1; activations all 1.0:
    max_val 1 -> iscale -127, q = -127, d8 = -1/127 -> out = 256 * 127 / 127."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)  # d = 1.0
    blk[4:16] = 0x01
    blk[16:] = 0x11
    x = np.ones(256, np.float32)
    q8 = zo.quantize_q8k(x)
    d8 = np.float32(1.0) / (np.float32(-127.0) / np.float32(1.0))
    assert q8[:4].view(np.float32)[0] == d8 and (q8[4:260].view(np.int8) == -127).all()
    got = zo.linear_q4k_q8k(q8, blk, 256, 1)[0]
    # sc_g = 1 for g < 4 and (1 | (0 << 4)) = 1 for g >= 4: int_sum = 256 * 1 * -127
    assert got == np.float32(d8) * np.float32(256 * -127)


@pytest.mark.parametrize("rows,k", [(16, 256), (40, 2048), (5, 6144)])
def test_linear_q6k_q8k_vs_f64(zo, rows, k):
    """The Q6_K x Q8_K integer construction (the K-quant prefill GEMM's
    arithmetic) against an f64 brute force over the dequantized Q6_K weights
    (dequant.rs:328-355, pinned by the reference's KATs) and the dequantized
    Q8_K activations: a wrong element, scale or -32 mapping would not come
    within 1e-5."""
    rng = np.random.default_rng(3 * rows + k)
    w = synth.weight(rng, 14, rows, k, 1)
    x = synth.activations(rng, k)
    q8 = zo.quantize_q8k(x)
    got = zo.linear_q6k_q8k(q8, w, k, rows)
    wd = zo.dequant(w, rows, k, 14).astype(np.float64)
    ref = wd @ _q8k_dequant(q8, k)
    err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    assert err < 1e-5, err
    part = zo.linear_q6k_q8k(q8, w, k, rows, start=1, end=4)
    assert np.array_equal(part[1:4], got[1:4]) and not part[:1].any() and not part[4:].any()
    fp = zo.linear_range(x, w, k, rows, 14)
    q_err = np.max(np.abs(got - fp)) / np.max(np.abs(fp))
    assert 1e-5 < q_err < 3e-2, q_err


def test_linear_q6k_q8k_kat(zo):
    """One superblock, d = 1, every scale 2, every 6-bit value 33 (low
    nibbles 1, high bits 2: q - 32 = 1); activations all 1.0 (q8 = -127,
    d8 = -1/127): int_sum = 256 * 2 * -127, out = d8 * int_sum."""
    blk = np.zeros(210, np.uint8)
    blk[0:128] = 0x11
    blk[128:192] = 0xAA
    blk[192:208] = 2
    blk[208:210] = np.array([0x3C00], np.uint16).view(np.uint8)
    assert np.all(zo.dequant(blk, 1, 256, 14) == 2.0)
    x = np.ones(256, np.float32)
    q8 = zo.quantize_q8k(x)
    d8 = q8[:4].view(np.float32)[0]
    got = zo.linear_q6k_q8k(q8, blk, 256, 1)[0]
    assert got == np.float32(np.float32(1.0) * d8) * np.float32(256 * 2 * -127)


def test_gemm_q8k_rows_are_per_row_dots(zo):
    """gemm_q8k is the per-row Q8_K quantization and integer dot."""
    rng = np.random.default_rng(5)
    m, n, k = 3, 8, 512
    x = synth.activations(rng, m * k).reshape(m, k)
    for wt in (12, 14):
        w = synth.weight(rng, wt, n, k, 1)
        y = zo.gemm_q8k(x, w, m, n, k, wt)
        f = zo.linear_q4k_q8k if wt == 12 else zo.linear_q6k_q8k
        for i in range(m):
            assert np.array_equal(y[i], f(zo.quantize_q8k(x[i]), w, k, n))
