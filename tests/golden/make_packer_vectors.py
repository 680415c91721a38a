"""Write tests/golden/packer_vectors.json from the reference packer.

Runs the reference's stdlib-only packer (tools/silicatepack.py of
silicatetech/zero, read from /root/reference in the build container) on
small seeded inputs and records inputs and outputs as data:

* float_to_fp16_bytes (silicatepack.py:854-861) on doubles that include
  exact round-to-nearest-even ties, subnormal halves and clamped values;
* quantize_q8_0_block (:893-907) and quantize_q4_0_block (:910-940) on
  float32 blocks (N(0,1) activations, exact .5 ties, tiny and huge scales);
* write_transformed_tensor (:943-1059) X4 emission for the 8x64 source of
  test_silicatepack.py:321-339, transforms q4_0x4 and q8_0x4.

The fixtures are what travels; the reference itself does not.
Usage: python tests/golden/make_packer_vectors.py [/path/to/reference]
"""
from __future__ import annotations

import hashlib
import io
import json
import random
import struct
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent


def f32(v: float) -> float:
    return struct.unpack("<f", struct.pack("<f", v))[0]


def f32_bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


def main(ref_root: str) -> None:
    sys.path.insert(0, str(Path(ref_root) / "tools"))
    import silicatepack as sp  # noqa: E402  (reference packer, stdlib only)

    rnd = random.Random(20261201)
    out: dict = {"source": "tools/silicatepack.py of silicatetech/zero"}

    # --- fp16 bytes of doubles -------------------------------------------
    doubles = [0.0, -0.0, 1.0, 65504.0, 65519.0, 65520.0, 70000.0, -70000.0, 1e-9, 2.0 ** -24, 2.0 ** -25,
               3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 * (1 - 2.0 ** -11)]
    for _ in range(200):  # exact midpoints between adjacent halves: ties
        h = rnd.randrange(0x0001, 0x7BFF)
        lo = struct.unpack("<e", struct.pack("<H", h))[0]
        hi = struct.unpack("<e", struct.pack("<H", h + 1))[0]
        doubles.append((lo + hi) / 2)
    for _ in range(300):
        doubles.append(10 ** rnd.uniform(-9, 5) * rnd.choice([1, -1]))
    out["fp16"] = [[d.hex(), sp.float_to_fp16_bytes(d).hex()] for d in doubles]

    # --- block quantizers ---------------------------------------------------
    blocks = []
    for _ in range(64):
        blocks.append([f32(rnd.gauss(0, 1)) for _ in range(32)])
    ties = [127.0, 63.5, -63.5, 0.5, -0.5, 1.5, 2.5, -2.5, 3.5, 125.5, -126.5] + [0.0] * 21
    blocks.append([f32(v) for v in ties])
    blocks.append([f32(v * 1e-6) for v in blocks[0]])  # d underflows to fp16 subnormal / zero
    blocks.append([f32(v * 1e7) for v in blocks[1]])   # d clamps to 65504
    blocks.append([0.0] * 32)
    blocks.append([0.0] * 31 + [f32(-3.0)])
    q4_ties = [-8.0, 4.0, 1.0] + [0.0] * 29           # test_silicatepack.py:285-297
    blocks.append(q4_ties)
    blocks.append([8.0, -4.0] + [0.0] * 30)
    out["blocks"] = [[f32_bits(v) for v in b] for b in blocks]
    out["q8_0"] = [sp.quantize_q8_0_block(tuple(b)).hex() for b in blocks]
    out["q4_0"] = [sp.quantize_q4_0_block(tuple(b)).hex() for b in blocks]

    # --- X4 emission --------------------------------------------------------
    rows, cols = 8, 64
    vals = [((r * 31 + c * 7) % 17 - 8) * 0.25 + 0.0625 * ((r + c) % 5) for r in range(rows) for c in range(cols)]
    data = struct.pack(f"<{rows * cols}f", *vals)
    x4 = {}
    with tempfile.TemporaryDirectory() as tmp:
        src_path = Path(tmp) / "weights.bin"
        src_path.write_bytes(data)
        src = sp.TensorSource(name="blk.0.attn_q.weight", dtype="F32", shape=(rows, cols), file=src_path,
                              data_begin=0, data_end=len(data), file_data_offset=0)
        for t in ("q4_0", "q4_0x4", "q8_0", "q8_0x4"):
            buf = io.BytesIO()
            sp.write_transformed_tensor(src=src, dst=buf, payload_hash=hashlib.sha256(), transform=t)
            x4[t] = buf.getvalue().hex()
    out["tensor"] = {"rows": rows, "cols": cols, "source": "test_silicatepack.py:321-339", **x4}

    dst = HERE / "packer_vectors.json"
    dst.write_text(json.dumps(out, indent=0))
    print(f"wrote {dst}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
