"""The code-object route without a GPU: zero_amd/zg_kernels.hsaco is a gfx950
ELF that defines every entry point (and its kernel descriptor) that
include/zero_gpu_kernels.h and zero_amd/module.py name, and the launch rule
of the header (zg_mk_plan, compiled here with gcc) and its Python form
(module.plan) agree with each other and with the library's launch shapes.
No call here touches a device."""
import re
import struct
import subprocess
from pathlib import Path

import pytest

from zero_amd import module

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "zero_gpu_kernels.h"
SOURCE = ROOT / "zero_amd" / "csrc" / "module" / "zg_module.hip"

EM_AMDGPU = 224
EF_AMDGPU_MACH_GFX950 = 0x04F


def _elf_symbols(path: Path) -> tuple[dict, set[str]]:
    """ELF64 header fields and the names of all symbol-table entries."""
    b = path.read_bytes()
    assert b[:4] == b"\x7fELF" and b[4] == 2 and b[5] == 1, "not a little-endian ELF64"
    e_machine = struct.unpack_from("<H", b, 0x12)[0]
    e_flags = struct.unpack_from("<I", b, 0x30)[0]
    shoff = struct.unpack_from("<Q", b, 0x28)[0]
    shentsize, shnum = struct.unpack_from("<HH", b, 0x3A)
    secs = [struct.unpack_from("<IIQQQQIIQQ", b, shoff + i * shentsize) for i in range(shnum)]
    names = set()
    for s in secs:
        if s[1] not in (2, 11):  # SHT_SYMTAB, SHT_DYNSYM
            continue
        off, size, link = s[4], s[5], s[6]
        stroff = secs[link][4]
        for j in range(size // 24):
            st_name = struct.unpack_from("<I", b, off + 24 * j)[0]
            end = b.index(b"\0", stroff + st_name)
            names.add(b[stroff + st_name:end].decode())
    return {"machine": e_machine, "flags": e_flags}, names


def _source_entries() -> list[str]:
    return re.findall(r"^ZG_MODULE_GEMV\((zg_mk_\w+),", SOURCE.read_text(), flags=re.M)


def test_entry_lists_agree():
    src = _source_entries()
    assert len(src) == len(set(src))
    assert set(src) == set(module.ENTRIES)


def test_code_object_is_gfx950_and_defines_every_entry():
    assert module.CODE_OBJECT.exists(), "build zero_amd/zg_kernels.hsaco first (zero_amd/build.py)"
    hdr, names = _elf_symbols(module.CODE_OBJECT)
    assert hdr["machine"] == EM_AMDGPU
    assert hdr["flags"] & 0xFF == EF_AMDGPU_MACH_GFX950
    missing = [e for e in module.ENTRIES if e not in names or e + ".kd" not in names]
    assert not missing, f"code object lacks {missing}"


_HARNESS = r"""
#include <stdio.h>
#include "zero_gpu_kernels.h"
int main(void) {
  unsigned q, r, k, cu;
  while (scanf("%u %u %u %u", &q, &r, &k, &cu) == 4) {
    zg_mk_launch L;
    if (zg_mk_plan(q, r, k, cu, &L)) { printf("-\n"); continue; }
    printf("%s %u %u %u %u %d %d\n", L.entry, L.block, L.shm_bytes, L.nbatch, L.per_cu_cap, L.one_batch,
           L.occupancy_bound);
  }
  return 0;
}
"""

SHAPES = [(q, r, k, cu)
          for q in (module.Q4_0, module.Q8_0)
          for r in (4, 1024, 2048, 4096, 6144, 8192, 12288, 16384, 32768, 49152, 151936)
          for k in (512, 1024, 1536, 2048, 3072, 4096, 5120, 6144, 8192)
          for cu in (256, 80)]


@pytest.fixture(scope="module")
def c_plans(tmp_path_factory):
    d = tmp_path_factory.mktemp("mk")
    (d / "h.c").write_text(_HARNESS)
    exe = d / "h"
    subprocess.run(["gcc", "-std=c99", "-O1", "-Wall", "-Werror", "-I", str(HEADER.parent), str(d / "h.c"), "-o",
                    str(exe)], check=True)
    inp = "".join(f"{q} {r} {k} {cu}\n" for q, r, k, cu in SHAPES) + "2 6 2048 256\n3 64 2048 256\n2 64 2000 256\n"
    out = subprocess.run([str(exe)], input=inp, capture_output=True, text=True, check=True).stdout.split("\n")
    return out


def test_c_and_python_plans_agree(c_plans):
    for shape, line in zip(SHAPES, c_plans):
        lp = module.plan(*shape)
        assert line == (f"{lp.entry} {lp.block} {lp.shm_bytes} {lp.nbatch} {lp.per_cu_cap} {int(lp.one_batch)} "
                        f"{int(lp.occupancy_bound)}"), shape
        assert lp.entry in module.ENTRIES, (shape, lp.entry)
    # rows not a multiple of 4, an unknown type, k not a multiple of 512
    assert c_plans[len(SHAPES):len(SHAPES) + 3] == ["-", "-", "-"]


def test_every_entry_is_planned_somewhere():
    planned = {module.plan(*s).entry for s in SHAPES}
    assert planned == set(module.ENTRIES), set(module.ENTRIES) - planned


def test_plans_are_the_library_launches():
    # the headline 6144x2048 Q4_0X4 GEMV: 512 one-batch workgroups of four
    # waves, three groups per wave (the trace's gemv_strip_kernel<2u, 0, 0,
    # 3, 1024, true, 4, true, 4, false>, 256 threads)
    lp = module.plan(module.Q4_0, 6144, 2048, 256)
    assert (lp.entry, lp.block, lp.nbatch, lp.one_batch, lp.shm_bytes) == ("zg_mk_q4_0x4_oneb_g3_k2048", 256, 512,
                                                                           True, 2 * 4 * 3 * 16 * 4)
    # down 2048x6144: twelve strips, two groups per wave
    lp = module.plan(module.Q4_0, 2048, 6144, 256)
    assert (lp.entry, lp.block, lp.nbatch) == ("zg_mk_q4_0x4_oneb_g2_k6144", 768, 256)
    # the LM-head height: a batch loop over four-group batches, 256 threads
    lp = module.plan(module.Q4_0, 151936, 2048, 256)
    assert (lp.entry, lp.block, lp.one_batch, lp.occupancy_bound) == ("zg_mk_q4_0x4_tall_t256", 256, False, True)
    assert lp.nbatch == 151936 // 16
    # fused-QKV-sized Q8_0X4: two groups per wave, one batch
    lp = module.plan(module.Q8_0, 4096, 2048, 256)
    assert (lp.entry, lp.nbatch, lp.one_batch) == ("zg_mk_q8_0x4_oneb_g2_k2048", 512, True)


@pytest.mark.parametrize("shape", [(module.Q4_0, 6, 2048), (3, 64, 2048), (module.Q4_0, 64, 2000),
                                   (module.Q4_0, 64, 8704), (module.Q8_0, 0, 2048)])
def test_plan_rejects_shapes_outside_the_module(shape):
    with pytest.raises(module.ModuleError):
        module.plan(*shape, 256)


def test_missing_code_object_raises_import_error(tmp_path):
    with pytest.raises(ImportError):
        module.KernelModule(tmp_path / "absent.hsaco", cu_count=256)
