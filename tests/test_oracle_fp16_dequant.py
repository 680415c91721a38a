"""Pins the oracle's fp16 decode and block dequantizers.

fp16_to_f32 (dequant.rs:28-61) against numpy's independent binary16 decoder
over all 65,536 bit patterns (NaN payloads included) and the reference KATs;
dequant_* against the reference KATs (dequant.rs:553-1292), closed forms and
bit-flip sensitivity of the Q6_K element map (linear.rs:396-401).
"""
import numpy as np
import pytest

from golden import kats


def test_fp16_exhaustive_matches_numpy(zo):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = zo.fp16_to_f32(bits).view(np.uint32)
    want = bits.view(np.float16).astype(np.float32).view(np.uint32)
    # numpy keeps NaN payloads (mant << 13) exactly as the reference does
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits,val,tol,src", kats.FP16)
def test_fp16_kats(zo, bits, val, tol, src):
    got = float(zo.fp16_to_f32(np.array([bits], np.uint16))[0])
    if val != val:
        assert got != got, src
    elif tol is None:
        assert got == val and np.signbit(got) == np.signbit(val), src
    else:
        assert abs(got - val) < tol, src


@pytest.mark.parametrize("scales,j,want,src", kats.SCALE_MIN_K4)
def test_scale_min_k4_kats(zo, scales, j, want, src):
    import ctypes as C
    s = np.frombuffer(scales, np.uint8).copy()
    sc, mn = C.c_uint8(), C.c_uint8()
    zo.load().zo_get_scale_min_k4(s.ctypes.data, j, C.addressof(sc), C.addressof(mn))
    assert (sc.value, mn.value) == want, src


@pytest.mark.parametrize("case", kats.DEQUANT, ids=lambda c: c[4])
def test_dequant_kats(zo, case):
    quant, blk, checks, tol, src = case
    w = np.frombuffer(blk, np.uint8).copy()
    be, bb = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}[quant]
    nb = w.size // bb
    out = zo.dequant(w, 1, nb * be, quant)[0]
    kats.check_dequant(out, checks, tol)


def test_q4_0_q8_0_closed_form(zo):
    rng = np.random.default_rng(1)
    from zero_amd import synth
    for quant, gen in ((2, synth.plain_q4_0), (8, synth.plain_q8_0)):
        w = gen(rng, 8, 256)
        got = zo.dequant(w, 8, 256, quant)
        bb = 18 if quant == 2 else 34
        blk = w.reshape(-1, bb)
        d = blk[:, :2].copy().view(np.float16).astype(np.float32)
        if quant == 2:
            lo = (blk[:, 2:] & 15).astype(np.int32) - 8
            hi = (blk[:, 2:] >> 4).astype(np.int32) - 8
            q = np.concatenate([lo, hi], axis=1)
        else:
            q = blk[:, 2:].view(np.int8).astype(np.int32)
        want = (q.astype(np.float32) * d).reshape(8, 256)  # exact products
        assert np.array_equal(got, want)


def _q4k_numpy(blk):
    """Q4_K decode from the ggml block description (d, dmin, 8 six-bit
    scale/min pairs, 4 x 32 bytes of nibble pairs)."""
    d = blk[0:2].copy().view(np.float16).astype(np.float32)[0]
    dmin = blk[2:4].copy().view(np.float16).astype(np.float32)[0]
    s = blk[4:16].astype(np.int32)
    sc = np.empty(8, np.int32)
    mn = np.empty(8, np.int32)
    sc[:4], mn[:4] = s[0:4] & 63, s[4:8] & 63
    sc[4:] = (s[8:12] & 15) | ((s[0:4] >> 6) << 4)
    mn[4:] = (s[8:12] >> 4) | ((s[4:8] >> 6) << 4)
    qs = blk[16:].reshape(4, 32).astype(np.int32)
    out = np.empty(256, np.float32)
    for g in range(4):
        out[g * 64:g * 64 + 32] = np.float32(d * sc[2 * g]) * (qs[g] & 15).astype(np.float32) - np.float32(dmin * mn[2 * g])
        out[g * 64 + 32:g * 64 + 64] = (np.float32(d * sc[2 * g + 1]) * (qs[g] >> 4).astype(np.float32)
                                        - np.float32(dmin * mn[2 * g + 1]))
    return out


def test_q4k_matches_numpy(zo):
    from zero_amd import synth
    w = synth.q4k(np.random.default_rng(2), 4, 512)
    got = zo.dequant(w, 4, 512, 12).reshape(-1, 256)
    for i, blk in enumerate(w.reshape(-1, 144)):
        assert np.array_equal(got[i], _q4k_numpy(blk))


def test_q6k_element_map_bitflips(zo):
    """Flip one bit of ql/qh and check that exactly the element named by the
    canonical ggml map changes: element 128h + l + 32*quarter for
    ql[64h + l (+32)], qh[32h + l] (linear.rs:396-401, dequant.rs:328-355)."""
    base = np.zeros(210, np.uint8)
    base[192:208] = 1  # all scales 1
    base[208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    ref = zo.dequant(base, 1, 256, 14)[0]
    for h in range(2):
        for l in (0, 5, 17, 31):
            for which, quarter in (("ql_lo", 0), ("ql_hi32_lo", 1), ("ql_hi", 2), ("ql_hi32_hi", 3)):
                b = base.copy()
                if which == "ql_lo":
                    b[64 * h + l] ^= 0x01
                elif which == "ql_hi32_lo":
                    b[64 * h + l + 32] ^= 0x01
                elif which == "ql_hi":
                    b[64 * h + l] ^= 0x10
                else:
                    b[64 * h + l + 32] ^= 0x10
                diff = np.nonzero(zo.dequant(b, 1, 256, 14)[0] != ref)[0]
                assert list(diff) == [128 * h + l + 32 * quarter], (h, l, which, diff)
            for quarter in range(4):
                b = base.copy()
                b[128 + 32 * h + l] ^= 1 << (2 * quarter)
                diff = np.nonzero(zo.dequant(b, 1, 256, 14)[0] != ref)[0]
                assert list(diff) == [128 * h + l + 32 * quarter]
    # scale index is = l // 16 selects sc[8h + is + 2*quarter]
    for h in range(2):
        for si in range(8):
            b = base.copy()
            b[192 + 8 * h + si] = 3
            diff = set(np.nonzero(zo.dequant(b, 1, 256, 14)[0] != ref)[0].tolist())
            is_, quarter = si % 2, si // 2
            want = {128 * h + 16 * is_ + l + 32 * quarter for l in range(16)}
            assert diff == want, (h, si)
