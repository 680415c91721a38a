"""zg_linear_q4k_vnni_noalloc against zg_linear_q4k_vnni, the allocating
entry point it varies (linear_q4k_vnni_dispatch,
kernel/src/inference_avx512.rs:519-547).

The no-allocation call quantizes x to Q8_K into the library's fixed device
array and runs the same integer GEMV, so its rows are bit-identical to the
allocating call's.  Two calls in a row, the second smaller, show that the
fixed array's stale bytes from the first call never leak into the second.
"""
import numpy as np
import pytest
import torch

from zero_amd import _lib, synth
from zero_amd.ops import ZgError

pytestmark = pytest.mark.gpu
Q4K = 12


def _case(ctx, rows, k, seed):
    rng = np.random.default_rng(seed)
    w = synth.q4k(rng, rows, k)
    x = synth.activations(rng, k)
    ctx.register(w, Q4K, 1)
    want = np.empty(rows, np.float32)
    ctx.linear_q4k_vnni(x, w, want, k, rows)
    dx = torch.from_numpy(x).cuda()
    dw = torch.from_numpy(w).cuda()
    out = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    ctx.linear_q4k_vnni_noalloc(dx, dw, out, k, rows, stream=s.cuda_stream)
    s.synchronize()
    got = out.cpu().numpy()
    return got, want


def test_noalloc_matches_allocating_call(ctx):
    try:
        for rows, k, seed in ((2048, 32768, 1), (512, 2048, 2)):  # the second call is smaller
            got, want = _case(ctx, rows, k, seed)
            print(f"noalloc Q4_K x Q8_K {rows}x{k}: bit-identical {np.array_equal(got, want)}")
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        ctx.clear()


def test_noalloc_rejects_in_dim_above_scratch(ctx):
    x = torch.zeros(32768 + 256, dtype=torch.float32, device="cuda")
    w = torch.zeros(144 * 129 * 4, dtype=torch.uint8, device="cuda")
    out = torch.zeros(4, dtype=torch.float32, device="cuda")
    with pytest.raises(ZgError) as ei:
        ctx.linear_q4k_vnni_noalloc(x, w, out, 32768 + 256, 4)
    assert ei.value.code == _lib.ZG_ERR_INVALID_ARG
    assert "fixed scratch" in ctx.last_error()
