"""Known-answer fixtures transcribed from the reference's own unit tests.

Each entry is data: the block bytes (built exactly as the reference test
builds them) and the outputs the reference test asserts, with its tolerance
and the file:line of the test.  Used to pin the CPU oracle (tests/test_oracle_*)
and the GPU kernels (tests/test_gpu_*).
"""
from __future__ import annotations

import struct

import numpy as np

# ---------------------------------------------------------------------------
# fp16_to_f32 (crates/zero-gguf-parser/src/dequant.rs:553-630)
# (bits, expected, abs tolerance or None for exact/bitwise, source)
# ---------------------------------------------------------------------------
FP16 = [
    (0x0000, 0.0, None, "dequant.rs:555 +0"),
    (0x8000, -0.0, None, "dequant.rs:561 -0"),
    (0x3C00, 1.0, None, "dequant.rs:568"),
    (0xBC00, -1.0, None, "dequant.rs:573"),
    (0x7BFF, 65504.0, None, "dequant.rs:578"),
    (0x0400, 6.103_515_6e-5, 1e-10, "dequant.rs:582-591"),
    (0x0001, 5.960_464_5e-8, 1e-14, "dequant.rs:594-604"),
    (0x7C00, float("inf"), None, "dequant.rs:607"),
    (0xFC00, float("-inf"), None, "dequant.rs:612"),
    (0x7E00, float("nan"), None, "dequant.rs:617"),
    (0x4000, 2.0, None, "dequant.rs:623"),
    (0x3800, 0.5, None, "dequant.rs:629"),
]

# get_scale_min_k4 (dequant.rs:634-661): (scales bytes, j, (sc, mn))
SCALE_MIN_K4 = []
_s = [0] * 12
_s[0], _s[4] = 0xFF, 0xAA
SCALE_MIN_K4.append((bytes(_s), 0, (63, 42), "dequant.rs:635-644"))
_s = [0] * 12
_s[0], _s[4], _s[8] = 0xC0, 0x80, 0x53
SCALE_MIN_K4.append((bytes(_s), 4, (51, 37), "dequant.rs:647-660"))


def q4k_block(d: int, dmin: int, scales, qs) -> bytes:
    """build_q4k_block (dequant.rs:665-672)."""
    return struct.pack("<HH", d, dmin) + bytes(scales) + bytes(qs)


def q4_0_block(d: int, qs) -> bytes:
    """build_q4_0_block (dequant.rs:800-806)."""
    return struct.pack("<H", d) + bytes(qs)


def q8_0_block(d: int, qs) -> bytes:
    """build_q8_0_block (dequant.rs:937-946); qs are signed."""
    return struct.pack("<H", d) + np.array(qs, dtype=np.int8).tobytes()


def q6k_block(ql, qh, scales, d: int) -> bytes:
    """build_q6k_block (dequant.rs:1097-1109)."""
    return bytes(ql) + bytes(qh) + np.array(scales, dtype=np.int8).tobytes() + struct.pack("<H", d)


def _arr(n, **at):
    a = [0] * n
    for k, v in at.items():
        a[int(k[1:])] = v
    return a


# Dequant KATs: (quant, block bytes, n_blocks, {index: expected} or
# ("all", value) / ("range", lo, hi, value) checks, tolerance, source)
DEQUANT = []
Q4_0, Q8_0, Q4K, Q6K = 2, 8, 12, 14

DEQUANT.append((Q4K, q4k_block(0, 0, [0] * 12, [0] * 128), [("all", 0.0)], 0.0, "dequant.rs:675-683"))
_sc = [1, 1, 1, 1, 1, 1, 1, 1, 0x11, 0x11, 0x11, 0x11]
DEQUANT.append((Q4K, q4k_block(0x3C00, 0x3800, _sc, [0] * 128), [("all", -0.5)], 1e-6, "dequant.rs:686-711"))
_sc = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
DEQUANT.append((Q4K, q4k_block(0x3C00, 0, _sc, [0xFF] * 128), [("all", 15.0)], 1e-6, "dequant.rs:714-732"))
_sc = _arr(12, i0=3, i1=5, i4=2, i5=4)
DEQUANT.append((Q4K, q4k_block(0x4000, 0x3C00, _sc, _arr(128, i0=0x73)), [("at", 0, 16.0), ("at", 32, 66.0)], 1e-4,
                "dequant.rs:735-763"))
_sc = [0, 0, 0, 0, 10, 10, 10, 10, 0xA0, 0xA0, 0xA0, 0xA0]
DEQUANT.append((Q4K, q4k_block(0, 0x4000, _sc, [0] * 128), [("all", -20.0)], 1e-4, "dequant.rs:766-782"))
DEQUANT.append((Q4K, q4k_block(0x3C00, 0, [0] * 12, [0xFF] * 128), [("all", 0.0)], 0.0, "dequant.rs:785-794"))
DEQUANT.append((Q4K, q4k_block(0x3C00, 0, _arr(12, i0=2), _arr(128, i0=5))
                + q4k_block(0x3800, 0, _arr(12, i0=4), _arr(128, i0=3)),
                [("at", 0, 10.0), ("at", 256, 6.0)], 1e-4, "dequant.rs:815-847"))

DEQUANT.append((Q4_0, q4_0_block(0, [0xFF] * 16), [("all", 0.0)], 0.0, "dequant.rs:815-824"))
DEQUANT.append((Q4_0, q4_0_block(0x3C00, [0xFF] * 16), [("all", 7.0)], 1e-6, "dequant.rs:827-835"))
DEQUANT.append((Q4_0, q4_0_block(0x3C00, [0x00] * 16), [("all", -8.0)], 1e-6, "dequant.rs:838-846"))
DEQUANT.append((Q4_0, q4_0_block(0x3C00, _arr(16, i0=0x80)),
                [("at", 0, -8.0), ("at", 16, 0.0), ("range", 1, 16, -8.0), ("range", 17, 32, -8.0)], 1e-6,
                "dequant.rs:849-883"))
DEQUANT.append((Q4_0, q4_0_block(0x4000, _arr(16, i0=0x12)), [("at", 0, -12.0), ("at", 16, -14.0)], 1e-6,
                "dequant.rs:886-899"))
DEQUANT.append((Q4_0, q4_0_block(0x3C00, [0xFF] * 16) + q4_0_block(0x3800, [0] * 16),
                [("range", 0, 32, 7.0), ("range", 32, 64, -4.0)], 1e-6, "dequant.rs:902-919"))

DEQUANT.append((Q8_0, q8_0_block(0, [127] * 32), [("all", 0.0)], 0.0, "dequant.rs:955-964"))
DEQUANT.append((Q8_0, q8_0_block(0x3C00, [127] * 32), [("all", 127.0)], 1e-6, "dequant.rs:967-975"))
DEQUANT.append((Q8_0, q8_0_block(0x3C00, [-128] * 32), [("all", -128.0)], 1e-6, "dequant.rs:978-989"))
DEQUANT.append((Q8_0, q8_0_block(0x3C00, [-1, 1, -100, 100, 0] + [0] * 27),
                [("at", 0, -1.0), ("at", 1, 1.0), ("at", 2, -100.0), ("at", 3, 100.0), ("at", 4, 0.0)], 1e-6,
                "dequant.rs:992-1014"))
DEQUANT.append((Q8_0, q8_0_block(0x4000, [3, -7] + [0] * 30), [("at", 0, 6.0), ("at", 1, -14.0)], 1e-6,
                "dequant.rs:1017-1029"))
DEQUANT.append((Q8_0, q8_0_block(0x3C00, [10] * 32) + q8_0_block(0x3800, [-20] * 32),
                [("range", 0, 32, 10.0), ("range", 32, 64, -10.0)], 1e-6, "dequant.rs:1032-1050"))

DEQUANT.append((Q6K, q6k_block([0] * 128, [0] * 64, [0] * 16, 0), [("all", 0.0)], 0.0, "dequant.rs:1112-1119"))
DEQUANT.append((Q6K, q6k_block([0] * 128, [0] * 64, _arr(16, i0=2), 0x3C00),
                [("range", 0, 16, -64.0), ("range", 16, 32, 0.0)], 1e-4, "dequant.rs:1122-1141"))
DEQUANT.append((Q6K, q6k_block([0xFF] * 128, [0xFF] * 64, [1] * 16, 0x3C00), [("all", 31.0)], 1e-4,
                "dequant.rs:1144-1159 (all-0xFF block: every layout decodes 31)"))
DEQUANT.append((Q6K, q6k_block(_arr(128, i0=0x05), _arr(64, i0=0x01), _arr(16, i0=3), 0x4000), [("at", 0, -66.0)],
                1e-4, "dequant.rs:1174-1196"))
DEQUANT.append((Q6K, q6k_block([0] * 128, [0] * 64, _arr(16, i0=-4), 0x3C00), [("at", 0, 128.0)], 1e-4,
                "dequant.rs:1269-1279"))
DEQUANT.append((Q6K, q6k_block([0] * 128, [0] * 64, [0] * 16, 0) * 2, [("all", 0.0)], 0.0, "dequant.rs:1282-1292"))


def check_dequant(out: np.ndarray, checks, tol: float) -> None:
    for c in checks:
        if c[0] == "all":
            np.testing.assert_allclose(out, c[1], atol=tol, rtol=0)
        elif c[0] == "at":
            assert abs(float(out[c[1]]) - c[2]) <= tol, (c, float(out[c[1]]))
        elif c[0] == "range":
            np.testing.assert_allclose(out[c[1]:c[2]], c[3], atol=tol, rtol=0)


# ---------------------------------------------------------------------------
# Scalar linear KATs (crates/zero-llm-inference/src/ops.rs:953-1160)
# (quant, in_dim, out_dim, x, w bytes, expected outputs, tol, source)
# ---------------------------------------------------------------------------
Q4_0_UNIT = q4_0_block(0x3C00, [0x99] * 16)     # ops.rs:955-965: all +1.0
Q8_0_UNIT = q8_0_block(0x3C00, [1] * 32)         # ops.rs:1093-1104
_ramp = np.arange(1, 33, dtype=np.float32)
LINEAR = [
    (Q4_0, 32, 1, _ramp, Q4_0_UNIT, [528.0], 1e-3, "ops.rs:967-986"),
    (Q4_0, 32, 2, np.ones(32, np.float32), Q4_0_UNIT + q4_0_block(0x3C00, [0] * 16), [32.0, -256.0], 1e-4,
     "ops.rs:988-1008"),
    (Q4_0, 64, 1, np.full(64, 0.5, np.float32), Q4_0_UNIT * 2, [32.0], 1e-3, "ops.rs:1010-1023"),
    (Q8_0, 32, 1, _ramp, Q8_0_UNIT, [528.0], 1e-3, "ops.rs:1106-1124"),
    (Q8_0, 32, 1, np.full(32, 0.5, np.float32), q8_0_block(0x3C00, [-1] * 32), [-16.0], 1e-3, "ops.rs:1126-1143"),
    (Q8_0, 64, 1, np.full(64, 0.5, np.float32), Q8_0_UNIT * 2, [32.0], 1e-3, "ops.rs:1145-1157"),
]

# ---------------------------------------------------------------------------
# rmsnorm / RoPE KATs (ops.rs:530-772)
# ---------------------------------------------------------------------------
RMSNORM = [
    ([1.0] * 4, [1.0] * 4, [1.0] * 4, 1e-3, "ops.rs:531-542"),
    ([0.0] * 4, [1.0] * 4, [0.0] * 4, 0.0, "ops.rs:545-556"),
    ([3.0, 4.0], [1.0, 1.0], [0.8485281, 1.1313708], 1e-4, "ops.rs:559-582"),
    ([1.0, 1.0], [2.0, 3.0], [2.0, 3.0], 1e-3, "ops.rs:585-594"),
]
RMSNORM_UNIT_RMS = ([0.1, -0.2, 0.3, -0.1, 0.4, -0.3, 0.2, -0.05], "ops.rs:609-629")

# RoPE: (half, freq_base, position, input, expected (first n), tol, source)
ROPE = [
    (2, 1.0, 1, [1.0, 2.0, 3.0, 4.0], [-1.9842, -2.2854, 2.4624, 3.8442], 1e-3, "ops.rs:650-665"),
    (64, 1_000_000.0, 1, [0.01 * (i + 1) for i in range(128)],
     [-0.5415531171, -0.4622832390, -0.3812512551, -0.3051765074, -0.2368033646, -0.1767538593, -0.1246151535,
      -0.0795384381, -0.0405505749, -0.0067053730, 0.0228510916, 0.0488593503, 0.0719468978, 0.0926380198,
      0.1113669505, 0.1284913603], 1e-4, "ops.rs:682-721 (gguf-py reference values)"),
]
ROPE_IDENTITY = (4, 1_000_000.0, [1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0], "ops.rs:634-647")
ROPE_INV_FREQ = [(0, 1.0, 1e-6), (1, 0.8058, 1e-3)]  # ops.rs:726-748; [63] in (0, 0.001)

# ---------------------------------------------------------------------------
# LM-head argmax (lm_head.rs:174-201, lm_head.rs:12-15)
# ---------------------------------------------------------------------------
VOCAB_SIZE_REAL = 151_643
VOCAB_SIZE_PADDED = 151_936
ARGMAX_BASIC = {"fill": -10.0, "set": {25: 12.0, 100: 10.0}, "index": 25, "value": 12.0, "source": "lm_head.rs:174-192"}

# ---------------------------------------------------------------------------
# SMP partition cases (kernel/src/smp_partition.rs:226-401)
# ---------------------------------------------------------------------------
PARTITION_CLOSED_FORM = [(151_936, 64, 1), (151_936, 64, 4), (2048, 64, 4), (1024, 17, 4), (6144, 64, 4),
                         (100, 8, 1), (103, 8, 4), (3, 8, 1), (3, 8, 4), (0, 8, 4)]
PARTITION_DISCOUNT = [(151_936, 64, 1), (151_936, 64, 4), (2048, 64, 4), (6144, 64, 4), (1024, 17, 4),
                      (103, 8, 4), (16, 64, 4), (3, 8, 1), (0, 8, 4)]
PARTITION_DISCOUNTS = [5, 10, 25, 50, 90, 100]

# ---------------------------------------------------------------------------
# Packer (tools/test_silicatepack.py)
# ---------------------------------------------------------------------------


def packer_source_values(rows: int, cols: int) -> np.ndarray:
    """_write_f32_source (test_silicatepack.py:321-339): deterministic,
    non-degenerate values, stored as f32."""
    v = [((r * 31 + c * 7) % 17 - 8) * 0.25 + 0.0625 * ((r + c) % 5) for r in range(rows) for c in range(cols)]
    return np.array(v, dtype=np.float32).reshape(rows, cols)
