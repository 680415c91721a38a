"""Pins the oracle's packer restatements (tools/silicatepack.py):
fp16 bytes (:854-861), quantize_q8_0_block (:893-907), quantize_q4_0_block
(:910-940) and the X4 writer (:982-1029), against golden vectors written by
the reference packer itself (tests/golden/make_packer_vectors.py), the
packer's own KATs (test_silicatepack.py:270-387) and numpy's independent
binary16 rounding.
"""
import json
import struct
from pathlib import Path

import numpy as np
import pytest

from golden import kats
from zero_amd import synth

VEC = json.loads((Path(__file__).parent / "golden" / "packer_vectors.json").read_text())


def test_fp16_bytes_golden(zo):
    for dhex, want in VEC["fp16"]:
        d = float.fromhex(dhex)
        assert zo.load().zo_f64_to_fp16_bits(d).to_bytes(2, "little").hex() == want, dhex


def test_fp16_rounding_matches_numpy(zo):
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.uniform(-65504, 65504, 2000), 10 ** rng.uniform(-10, 4.8, 4000)])
    for v in vals:
        assert zo.load().zo_f64_to_fp16_bits(float(v)) == int(np.float64(v).astype(np.float16).view(np.uint16))


def _blocks():
    return [np.array(b, np.uint32).view(np.float32) for b in VEC["blocks"]]


def test_quantize_q8_0_golden(zo):
    for b, want in zip(_blocks(), VEC["q8_0"]):
        assert zo.quantize_q8_0(b).tobytes().hex() == want


def test_quantize_q4_0_golden(zo):
    for b, want in zip(_blocks(), VEC["q4_0"]):
        assert zo.quantize_q4_0(b).tobytes().hex() == want


def test_q4_0_encoding_kat(zo):
    # test_silicatepack.py:270-306
    v = np.zeros(32, np.float32)
    v[0], v[1], v[2] = -8.0, 4.0, 1.0
    blk = zo.quantize_q4_0(v)
    dec = zo.dequant(blk, 1, 32, 2)[0]
    assert dec[0] == -8.0 and dec[1] == 4.0 and dec[2] == 1.0 and (blk[2] & 0x0F) == 0
    v = np.zeros(32, np.float32)
    v[0], v[1] = 8.0, -4.0
    dec = zo.dequant(zo.quantize_q4_0(v), 1, 32, 2)[0]
    assert dec[0] == 8.0 and dec[1] == -4.0
    assert zo.quantize_q4_0(np.zeros(32, np.float32)).tobytes() == b"\0" * 18


def test_q8_0_error_bound_and_extremes(zo):
    rng = np.random.default_rng(9)
    x = rng.standard_normal(32 * 500).astype(np.float32)
    q = zo.quantize_q8_0(x).reshape(-1, 34)
    d = q[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    qs = q[:, 2:].view(np.int8).astype(np.float64)
    xb = x.reshape(-1, 32).astype(np.float64)
    dd = np.abs(xb).max(1) / 127.0  # unrounded d the packer divides by
    assert np.all(np.abs(xb / dd[:, None] - qs) <= 0.5 + 1e-12)
    assert np.all(np.abs(qs).max(1) == 127)  # amax maps to +-127
    assert np.all(np.abs(d - dd) <= dd * 2 ** -11)  # fp16 RNE of d


def test_x4_tensor_golden(zo):
    t = VEC["tensor"]
    rows, cols = t["rows"], t["cols"]
    vals = kats.packer_source_values(rows, cols)
    for quant, plain_t, x4_t in ((2, "q4_0", "q4_0x4"), (8, "q8_0", "q8_0x4")):
        fn = zo.quantize_q4_0 if quant == 2 else zo.quantize_q8_0
        plain = np.concatenate([fn(vals[r]) for r in range(rows)])
        assert plain.tobytes().hex() == t[plain_t]
        assert zo.interleave_x4(plain, rows, cols, quant).tobytes().hex() == t[x4_t]
        assert synth.interleave_x4(plain, rows, cols, quant).tobytes().hex() == t[x4_t]


@pytest.mark.parametrize("quant,bb", [(2, 18), (8, 34)])
def test_x4_is_exact_block_permutation(zo, quant, bb):
    # test_silicatepack.py:341-378 property, on random blocks
    rows, cols = 8, 64
    nb = cols // 32
    plain = synth.weight(np.random.default_rng(1), quant, rows, cols, 1)
    x4 = zo.interleave_x4(plain, rows, cols, quant)
    expected = bytearray()
    for g in range(0, rows, 4):
        for b in range(nb):
            for lane in range(4):
                off = ((g + lane) * nb + b) * bb
                expected += plain[off:off + 2].tobytes()
            for lane in range(4):
                off = ((g + lane) * nb + b) * bb
                expected += plain[off + 2:off + bb].tobytes()
    assert bytes(expected) == x4.tobytes()
    assert np.array_equal(synth.deinterleave_x4(x4, rows, cols, quant), plain)


def test_x4_rejects_partial_groups(zo):
    # test_silicatepack.py:380-387
    plain = synth.weight(np.random.default_rng(1), 2, 6, 64, 1)
    out = np.empty_like(plain)
    assert zo.load().zo_interleave_x4(plain.ctypes.data, out.ctypes.data, 6, 64, 2) != 0
