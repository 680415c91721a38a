"""GPU parity of the Q4_K x Q8_K integer path (zg_quantize_q8k_dev,
zg_linear_q4k_q8k_dev, zg_linear_q4k_vnni) against the oracle's restatement
of quantize_row_q8k and linear_q4k_vnni_range
(kernel/src/arch/x86_64/math/vnni.rs:78-170, 258-476).

Bar: the Q8_K blocks byte-identical; GEMV rows within rel 1e-4 of the oracle
(the per-superblock integer sums and f32 products are the reference's; only
the order in which superblock terms are added differs)."""
import numpy as np
import pytest
import torch

from zero_amd import _lib, synth
from zero_amd.ops import ZgError

pytestmark = pytest.mark.gpu
Q4K = 12


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def stream():
    return torch.cuda.current_stream().cuda_stream


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _activations(seed, n, scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    if n >= 1024:
        x[256:512] = 0.0                                  # zero block
        x[512 + 3], x[512 + 200] = -40.0 * scale, 40.0 * scale  # tie: the first (negative) wins
        x[768:1024] = np.float32(1.5) * scale              # all equal: index 0 wins
    return x


@pytest.mark.parametrize("n,scale", [(4096, 1.0), (14336, 1e-3), (256, 250.0), (2048, 1e-20)])
def test_quantize_q8k_bit_exact(ctx, zo, n, scale):
    x = _activations(n, n, scale)
    q = torch.empty(n // 256 * 292, dtype=torch.uint8, device="cuda")
    ctx.quantize_q8k_dev(dev(x), q, n, stream=stream())
    got = q.cpu().numpy()
    want = zo.quantize_q8k(x)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]


GEMV_CASES = [(14336, 4096), (4096, 14336), (64, 256), (33, 2304), (100, 768), (16, 32768), (7, 2048)]


@pytest.mark.parametrize("rows,k", GEMV_CASES)
def test_q4k_q8k_gemv_matches_oracle(ctx, zo, rows, k):
    rng = np.random.default_rng(rows * 3 + k)
    w = synth.q4k(rng, rows, k)
    x = _activations(k + 1, k)
    q8 = zo.quantize_q8k(x)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.linear_q4k_q8k_dev(dev(q8), dev(w), y, k, rows, stream=stream())
    got = y.cpu().numpy()
    ref = zo.linear_q4k_q8k(q8, w, k, rows)
    print(f"Q4_K x Q8_K {rows}x{k}: rel err vs oracle {rel_err(got, ref):.2e}")
    assert rel_err(got, ref) <= 1e-4


def test_q4k_vnni_host_api(ctx, zo):
    rows, k = 1536, 4096
    rng = np.random.default_rng(5)
    w = synth.q4k(rng, rows, k)
    x = synth.activations(rng, k)
    ctx.register(w, Q4K, 1)
    try:
        out = np.empty(rows, np.float32)
        ctx.linear_q4k_vnni(x, w, out, k, rows)
        ref = zo.linear_q4k_q8k(zo.quantize_q8k(x), w, k, rows)
        assert rel_err(out, ref) <= 1e-4
        # the fp32 Q4_K path on the same weights differs by the Q8_K rounding only
        fp = np.empty(rows, np.float32)
        ctx.linear_dispatch(x, w, fp, k, rows, Q4K)
        assert rel_err(out, fp) < 3e-2
        with pytest.raises(ZgError) as e:
            ctx.linear_q4k_vnni(x[:200], w, out, 200, rows)
        assert e.value.code == _lib.ZG_ERR_INVALID_ARG
    finally:
        ctx.clear()
    with pytest.raises(ZgError) as e:
        ctx.linear_q4k_vnni(x, w, out, k, rows)  # no longer registered
    assert e.value.code == _lib.ZG_ERR_NOT_REGISTERED


def test_q4k_q8k_bounds(ctx):
    y = torch.empty(8, dtype=torch.float32, device="cuda")
    w = torch.zeros(8 * 129 * 144, dtype=torch.uint8, device="cuda")
    q = torch.zeros(129 * 292, dtype=torch.uint8, device="cuda")
    with pytest.raises(ZgError):
        ctx.linear_q4k_q8k_dev(q, w, y, 129 * 256, 8, stream=stream())  # 33024 > 32768
    with pytest.raises(ZgError):
        ctx.quantize_q8k_dev(y, q, 100, stream=stream())
