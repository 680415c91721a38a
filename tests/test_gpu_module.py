"""GPU parity of the code-object route (include/zero_gpu_kernels.h): the strip
GEMV loaded from zero_amd/zg_kernels.hsaco with hipModuleLoad and launched
with hipModuleLaunchKernel.

Bar: where the plan is the library's launch (every Q4_0X4 shape the strip
kernel takes, decode-sized Q8_0X4), the module's output is bitwise the
library's (zg_linear_dev on the same buffers); every output is within rel
1e-3 of the oracle and no further from an f64 brute force than the oracle
itself is (x 4); launches captured into a graph replay to the eager bits.
"""
import numpy as np
import pytest
import torch

from zero_amd import module, synth

pytestmark = pytest.mark.gpu

Q4_0, Q8_0 = module.Q4_0, module.Q8_0


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.fixture(scope="module")
def km():
    m = module.KernelModule()
    yield m
    m.close()


# (quant, rows, k, same launch as the library): one shape per planned entry
CASES = [
    (Q4_0, 6144, 2048, True),     # oneb_g3_k2048 (the headline GEMV)
    (Q4_0, 4096, 2048, True),     # oneb_g2_k2048
    (Q4_0, 2048, 2048, True),     # oneb_g1_k2048
    (Q4_0, 1024, 6144, True),     # oneb_g1_k6144
    (Q4_0, 2048, 6144, True),     # oneb_g2_k6144 (the decode's down projection)
    (Q4_0, 4096, 6144, True),     # oneb_g2_k6144
    (Q4_0, 6144, 6144, True),     # oneb_g3_k6144
    (Q4_0, 12288, 6144, True),    # oneb_g4_k6144 (tall, twelve strips, one batch)
    (Q4_0, 12288, 5120, True),    # oneb_g4 (ten strips)
    (Q4_0, 1024, 1024, True),     # oneb_g1 (two strips, two waves each)
    (Q4_0, 4096, 3072, True),     # oneb_g2 (six strips)
    (Q4_0, 6144, 3072, True),     # oneb_g3
    (Q4_0, 49152, 2048, True),    # tall_t256
    (Q4_0, 151936, 2048, False),  # tall_t256 (the library takes its LDS-staged kernel)
    (Q4_0, 16384, 4096, True),    # tall_t512
    (Q4_0, 32768, 6144, True),    # tall_t1024
    (Q8_0, 4096, 2048, True),     # q8 oneb_g2_k2048 (fused-QKV size)
    (Q8_0, 2048, 6144, True),     # q8 oneb_g2_k6144
    (Q8_0, 1024, 1536, True),     # q8 oneb_g2 (three strips)
    (Q8_0, 16384, 4096, False),   # q8 loop_g2 (the library takes its segment kernel)
    (Q8_0, 40960, 2048, False),   # q8 tall_t256 (the library takes its LDS-staged kernel)
]


@pytest.mark.parametrize("quant,rows,k,same", CASES, ids=[f"q{c[0]}-{c[1]}x{c[2]}" for c in CASES])
def test_module_gemv_matches_library_and_oracle(ctx, zo, km, quant, rows, k, same):
    rng = np.random.default_rng(rows * 7 + k + quant)
    w = synth.weight(rng, quant, rows, k, 4)
    x = synth.activations(rng, k)
    wd, xd = dev(w), dev(x)
    y_mod = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    y_lib = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    lp = km.gemv_x4(wd.data_ptr(), xd.data_ptr(), y_mod.data_ptr(), rows, k, quant)
    print(f"quant={quant} {rows}x{k}: {lp.entry} grid {km.grid(lp)} block {lp.block}", flush=True)
    ctx.linear_dev(xd, wd, y_lib, k, rows, quant, 4)
    torch.cuda.synchronize()
    got, lib = y_mod.cpu().numpy(), y_lib.cpu().numpy()
    if same:
        assert np.array_equal(got.view(np.uint32), lib.view(np.uint32)), f"{lp.entry}: not the library's bits"
    ref = zo.linear_range(x, w, k, rows, quant, 4)
    f64 = zo.linear_f64(x, w, k, rows, quant, 4)
    e_gpu, e_ref = rel_err(got, ref), rel_err(ref, f64)
    assert e_gpu <= 1e-3, e_gpu
    assert rel_err(got, f64) <= 4 * e_ref + 1e-6


def test_module_launches_replay_in_a_graph(km):
    """Module launches captured on a side stream replay to the eager bits,
    with other eager work and synchronizations between replays."""
    rng = np.random.default_rng(5)
    shapes = [(Q4_0, 6144, 2048), (Q4_0, 2048, 6144), (Q8_0, 4096, 2048)]
    bufs = []
    for q, rows, k in shapes:
        w, x = synth.weight(rng, q, rows, k, 4), synth.activations(rng, k)
        bufs.append((q, rows, k, dev(w), dev(x), torch.zeros(rows, dtype=torch.float32, device="cuda")))
    eager = []
    for q, rows, k, wd, xd, y in bufs:
        km.gemv_x4(wd.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, k, q)
    torch.cuda.synchronize()
    eager = [b[5].clone() for b in bufs]
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for q, rows, k, wd, xd, y in bufs:
            km.gemv_x4(wd.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, k, q, stream=stream.cuda_stream)
    for rep in range(3):
        for b in bufs:
            b[5].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for b, e in zip(bufs, eager):
            assert torch.equal(b[5].view(torch.int32), e.view(torch.int32)), (rep, b[:3])
    del g


def test_module_rejects_bad_arguments(km):
    x = torch.zeros(2048, dtype=torch.float32, device="cuda")
    y = torch.zeros(64, dtype=torch.float32, device="cuda")
    w = torch.zeros(64 * 2048 // 32 * 18, dtype=torch.uint8, device="cuda")
    with pytest.raises(module.ModuleError):
        km.gemv_x4(w.data_ptr(), x.data_ptr(), y.data_ptr(), 64, 2000, Q4_0)
    with pytest.raises(module.ModuleError):
        km.gemv_x4(w.data_ptr(), x.data_ptr() + 4, y.data_ptr(), 64, 2048, Q4_0)
    with pytest.raises(module.ModuleError):
        km.gemv_x4(0, x.data_ptr(), y.data_ptr(), 64, 2048, Q4_0)
    with pytest.raises(module.ModuleError):
        km.function("zg_mk_no_such_entry")


def test_failed_module_call_leaves_no_error_behind(ctx, km):
    """A failed module call is reported once: the library's next launch
    check does not see it."""
    with pytest.raises(module.ModuleError):
        km.function("zg_mk_no_such_entry")
    rng = np.random.default_rng(3)
    w, x = synth.weight(rng, Q4_0, 256, 2048, 4), synth.activations(rng, 2048)
    y = torch.empty(256, dtype=torch.float32, device="cuda")
    ctx.linear_dev(dev(x), dev(w), y, 2048, 256, Q4_0, 4)
    torch.cuda.synchronize()
