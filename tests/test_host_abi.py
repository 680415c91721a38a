"""The C ABI as a boundary, without a GPU: libzero_amd.so loads, exports
every function include/zero_gpu.h declares, the ctypes bindings cover them,
and the ctypes mirrors of the header's structs and status codes agree with
what a C compiler makes of the header (gcc, offsetof/sizeof).  No call here
touches a device."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from zero_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "zero_gpu.h"
STRUCTS = [_lib.zg_segment, _lib.zg_layer_weights, _lib.zg_layer_quants, _lib.zg_model_desc, _lib.zg_smodel_info, _lib.zg_smodel_tensor]


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^\s*(?!typedef|#)[A-Za-z_][\w \t\*]*?\b(zg_\w+)\s*\(", text, flags=re.M)
    assert len(names) == len(set(names))
    return names


def _status_codes() -> dict[str, int]:
    return {k: int(v) for k, v in re.findall(r"#define\s+(ZG_(?:OK|ERR_\w+))\s+(-?\d+)", HEADER.read_text())}


def test_header_declares_the_abi():
    names = _declared_functions()
    for must in ("zg_init", "zg_linear", "zg_linear_fused", "zg_lm_head_argmax", "zg_gemm_q8act_dev",
                 "zg_model_generate", "zg_smodel_open", "zg_smodel_register_all"):
        assert must in names
    assert len(names) >= 30


def test_library_exports_every_declared_function():
    lib = _lib.load()
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, f"libzero_amd.so lacks {missing}"


def test_bindings_cover_the_header():
    declared = set(_declared_functions())
    assert declared == set(_lib.SIGNATURES), (declared ^ set(_lib.SIGNATURES))


def test_status_codes_match_header():
    codes = _status_codes()
    assert codes["ZG_OK"] == 0 and len(codes) >= 14
    for k, v in codes.items():
        assert getattr(_lib, k) == v, k
    flags = {k: int(v) for k, v in re.findall(r"#define\s+(ZG_GEN_\w+)\s+(\d+)u", HEADER.read_text())}
    assert set(flags) == {"ZG_GEN_BATCHED_PREFILL", "ZG_GEN_EAGER"}
    for k, v in flags.items():
        assert getattr(_lib, k) == v, k


def test_struct_layouts_match_gcc(tmp_path):
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "zero_gpu.h"', "int main(void) {"]
    for s in STRUCTS:
        lines.append(f'printf("{s.__name__} sizeof %zu\\n", sizeof({s.__name__}));')
        for f, _ in s._fields_:
            lines.append(f'printf("{s.__name__} {f} %zu\\n", offsetof({s.__name__}, {f}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", str(HEADER.parent), str(src), "-o", str(exe)],
                   check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        s, f, v = line.split()
        got[(s, f)] = int(v)
    for s in STRUCTS:
        assert got[(s.__name__, "sizeof")] == C.sizeof(s), s.__name__
        for f, _ in s._fields_:
            assert got[(s.__name__, f)] == getattr(s, f).offset, (s.__name__, f)


def test_null_handles_are_rejected_without_a_device():
    """Entry points that check their arguments before any HIP call."""
    lib = _lib.load()
    out = C.c_void_p()
    assert lib.zg_smodel_open(None, 0, C.byref(out)) == _lib.ZG_ERR_INVALID_ARG
    info = _lib.zg_smodel_info()
    assert lib.zg_smodel_get_info(None, C.byref(info)) == _lib.ZG_ERR_INVALID_ARG
    assert lib.zg_smodel_register_all(None, None) == _lib.ZG_ERR_INVALID_ARG
    assert lib.zg_model_create(None, None, C.byref(out)) == _lib.ZG_ERR_INVALID_ARG


def _pack(value: float, index: int) -> int:
    """The device argmax word: an order-preserving key of the fp32 bits in
    the high half (sign flipped for positives, all bits for negatives), and
    0xFFFFFFFF - index in the low half so that a 64-bit max keeps the first
    index among equal values (the reference's strict `>` scan,
    kernel/src/inference_avx512.rs:1027-1044).  +0 and -0 compare equal
    there, so both take the key of +0."""
    b = int(C.c_uint32.from_buffer_copy(C.c_float(value)).value)
    key = (b | 0x8000_0000) if not b & 0x8000_0000 else (~b & 0xFFFF_FFFF)
    if b & 0x7FFF_FFFF == 0:
        key = 0x8000_0000
    return (key << 32) | (0xFFFF_FFFF - index)


@pytest.mark.parametrize("value,index", [(1.0, 7), (-2.0, 3), (0.0, 0), (-0.0, 151_935), (3.4e38, 12), (-1e-40, 5)])
def test_argmax_unpack_round_trip(value, index):
    lib = _lib.load()
    idx, val = C.c_uint32(), C.c_float()
    assert lib.zg_argmax_unpack(_pack(value, index), C.byref(idx), C.byref(val)) == 1
    assert idx.value == index
    want = C.c_uint32.from_buffer_copy(C.c_float(value)).value
    assert C.c_uint32.from_buffer_copy(val).value == (0 if value == 0 else want)


def test_argmax_packing_orders_like_a_first_max_scan():
    assert _pack(1.0, 7) > _pack(-2.0, 3) > _pack(-3.0, 0)
    assert _pack(1.0, 3) > _pack(1.0, 7)       # ties: the smaller index wins
    assert _pack(-0.0, 1) > _pack(0.0, 9)      # +0 == -0: the first index wins
    lib = _lib.load()
    idx, val = C.c_uint32(), C.c_float()
    assert lib.zg_argmax_unpack(0, C.byref(idx), C.byref(val)) == 0  # untouched slot: no candidate
    assert val.value == float("-inf")


if __name__ == "__main__":  # pragma: no cover
    pytest.main([__file__, "-q"])
