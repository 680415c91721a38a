"""GPU parity of the K-quant prefill GEMM (Q8_K activations x Q4_K / Q6_K
weights, int8 MFMA; zero_amd/csrc/zg_kgemm.hip) and its split Q8_K
quantizer, through the C ABI.

Bar: bit-exact.  The split quantizer's bytes equal quantize_row_q8k's
(vnni.rs:78-170, the oracle's zo_quantize_row_q8k); every GEMM output equals
the oracle's per-row integer dot (zo_linear_q4k_q8k_range, the reference's
linear_q4k_vnni_range at vnni.rs:258-476, and zo_linear_q6k_q8k_range) on
the same quantized rows, bit for bit.
"""
import numpy as np
import pytest
import torch

import zero_amd
from zero_amd import _lib, synth

pytestmark = pytest.mark.gpu
Q4K, Q6K = 12, 14


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _split(ctx, x, m, k):
    qs = torch.empty((m, k), dtype=torch.int8, device="cuda")
    d8 = torch.empty((m, k // 256), dtype=torch.float32, device="cuda")
    bs = torch.empty((m, k // 32), dtype=torch.int16, device="cuda")
    ctx.quantize_q8k_split_dev(dev(x), qs, d8, bs, m, k)
    return qs, d8, bs


@pytest.mark.parametrize("m,k,scale", [(3, 256, 1.0), (17, 2048, 1e-3), (4, 6144, 300.0)])
def test_quantize_q8k_split_matches_reference_blocks(ctx, zo, m, k, scale):
    rng = np.random.default_rng(m + k)
    x = (synth.activations(rng, m * k) * np.float32(scale)).reshape(m, k)
    x[0, :256] = 0.0                     # an all-zero block
    x[1, k - 20], x[1, k - 19] = -7.0 * scale, 7.0 * scale  # magnitude tie: the first wins
    qs, d8, bs = _split(ctx, x, m, k)
    qs, d8, bs = qs.cpu().numpy(), d8.cpu().numpy(), bs.cpu().numpy()
    for i in range(m):
        blocks = zo.quantize_q8k(x[i]).reshape(-1, 292)
        assert np.array_equal(qs[i].reshape(-1, 256), blocks[:, 4:260].view(np.int8))
        assert np.array_equal(d8[i].view(np.uint32), blocks[:, :4].copy().view(np.uint32).ravel())
        b16 = blocks[:, 260:].copy().view(np.int16).astype(np.int32).reshape(-1, 8, 2).sum(2).ravel()
        assert np.array_equal(bs[i].astype(np.int32), b16)


def _oracle_rows(zo, x, w, rows, n, k, wt):
    f = zo.linear_q4k_q8k if wt == Q4K else zo.linear_q6k_q8k
    return np.stack([f(zo.quantize_q8k(x[i]), w, k, n) for i in rows])


@pytest.mark.parametrize("wt", [Q4K, Q6K])
@pytest.mark.parametrize("m,n,k", [(1, 64, 256), (5, 128, 512), (70, 192, 2048), (130, 64, 6144)])
def test_gemm_q8k_bit_exact(ctx, zo, wt, m, n, k):
    """Partial 64-row tiles, one and several superblocks per row."""
    rng = np.random.default_rng(m * 7 + n + k + wt)
    w = synth.weight(rng, wt, n, k, 1)
    x = synth.activations(rng, m * k).reshape(m, k)
    qs, d8, bs = _split(ctx, x, m, k)
    y = torch.full((m, n), -3.0, dtype=torch.float32, device="cuda")
    ctx.gemm_q8k_dev(qs, d8, bs, dev(w), y, m, n, k, wt)
    got = y.cpu().numpy()
    ref = _oracle_rows(zo, x, w, range(m), n, k, wt)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # accumulate: y + product, one more rounding
    y0 = synth.activations(rng, m * n).reshape(m, n)
    y = dev(y0)
    ctx.gemm_q8k_dev(qs, d8, bs, dev(w), y, m, n, k, wt, accumulate=True)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), (y0 + ref).view(np.uint32))


@pytest.mark.parametrize("wt,n,k", [(Q4K, 6144, 2048), (Q6K, 2048, 6144), (Q4K, 2048, 6144)])
def test_gemm_q8k_prefill_shapes(ctx, zo, wt, n, k):
    """M = 512 at the Qwen3-1.7B FFN shapes (Q4_K gate / up, Q6_K and Q4_K
    down): every output of a sample of 96 rows, the first and last tiles
    included, bit-exact."""
    m = 512
    rng = np.random.default_rng(n + k + wt)
    w = synth.weight(rng, wt, n, k, 1)
    x = synth.activations(rng, m * k).reshape(m, k)
    qs, d8, bs = _split(ctx, x, m, k)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ctx.gemm_q8k_dev(qs, d8, bs, dev(w), y, m, n, k, wt)
    got = y.cpu().numpy()
    rows = list(range(0, 40)) + list(range(250, 266)) + list(range(472, 512))
    ref = _oracle_rows(zo, x, w, rows, n, k, wt)
    assert np.array_equal(got[rows].view(np.uint32), ref.view(np.uint32))


def test_gemm_q8k_errors(ctx):
    m, n, k = 4, 64, 256
    qs = torch.zeros((m, k), dtype=torch.int8, device="cuda")
    d8 = torch.zeros((m, 1), dtype=torch.float32, device="cuda")
    bs = torch.zeros((m, 8), dtype=torch.int16, device="cuda")
    w = torch.zeros(n * 144, dtype=torch.uint8, device="cuda")
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    for args, code in (((m, 48, k, Q4K), _lib.ZG_ERR_INVALID_ARG), ((m, n, 200, Q4K), _lib.ZG_ERR_INVALID_ARG),
                       ((m, n, k, 2), _lib.ZG_ERR_UNSUPPORTED_QUANT)):
        with pytest.raises(zero_amd.ZgError) as e:
            ctx.gemm_q8k_dev(qs, d8, bs, w, y, *args)
        assert e.value.code == code
    # m = 0 is a no-op
    ctx.gemm_q8k_dev(qs, d8, bs, w, y, 0, n, k, Q4K)
