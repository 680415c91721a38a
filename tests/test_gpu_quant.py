"""GPU parity of on-the-fly Q8_0 activation quantization and the int8-MFMA
prefill GEMM, through the C ABI.

Bar: the quantizer is byte-exact with the oracle's restatement of the
packer's quantize_q8_0_block (itself pinned by the packer's own output,
tests/golden/packer_vectors.json); the GEMM is bit-exact with the oracle's
zo_gemm_q8act (same block order, same fma).  The error of the Q8_0 path
against the fp32-activation GEMV is reported, not gated: the reference
notes 0.5-2 % per matmul for 8-bit activations (vnni.rs:14-16).
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from zero_amd import synth

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 8
VEC = json.loads((Path(__file__).parent / "golden" / "packer_vectors.json").read_text())


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def quantize_gpu(ctx, x2d):
    rows, k = x2d.shape
    xb = dev(x2d)
    blocks = torch.empty(rows * (k // 32) * 34, dtype=torch.uint8, device="cuda")
    qs = torch.empty((rows, k), dtype=torch.int8, device="cuda")
    d = torch.empty((rows, k // 32), dtype=torch.int16, device="cuda")
    ctx.quantize_q8_0_dev(xb, blocks, rows, k)
    ctx.quantize_q8_0_split_dev(xb, qs, d, rows, k)
    return blocks.cpu().numpy(), qs.cpu().numpy(), d.cpu().numpy().view(np.uint16)


def test_quantizer_packer_vectors(ctx, zo):
    blocks = np.array(VEC["blocks"], np.uint32).view(np.float32)
    got, _, _ = quantize_gpu(ctx, blocks.reshape(1, -1))
    assert got.tobytes().hex() == "".join(VEC["q8_0"])


@pytest.mark.parametrize("rows,k", [(512, 2048), (3, 6144), (1, 32)])
def test_quantizer_matches_oracle(ctx, zo, rows, k):
    x = synth.activations(np.random.default_rng(rows + k), rows, k)
    x[0, :32] = 0.0                        # all-zero block
    x[-1, -32:] *= 1e-7                    # d in the fp16 subnormal range
    got, qs, d = quantize_gpu(ctx, x)
    want = zo.quantize_q8_0(x.reshape(-1))
    assert np.array_equal(got, want)
    wb = want.reshape(-1, 34)
    assert np.array_equal(qs.reshape(-1, 32), wb[:, 2:].view(np.int8))
    assert np.array_equal(d.reshape(-1), wb[:, :2].copy().view(np.uint16).reshape(-1))


def test_quantizer_nonfinite_block(ctx):
    x = np.ones((1, 64), np.float32)
    x[0, 40] = np.inf
    got, _, _ = quantize_gpu(ctx, x)
    b = got.reshape(2, 34)
    assert b[1, :2].copy().view(np.uint16)[0] == 0x7E00 and not b[1, 2:].any()
    assert b[0, 2:].view(np.int8).tolist() == [127] * 32


def _gemm(ctx, x, w, n, k, wt, il):
    m = x.shape[0]
    xb = dev(x)
    qs = torch.empty((m, k), dtype=torch.int8, device="cuda")
    d = torch.empty((m, k // 32), dtype=torch.int16, device="cuda")
    ctx.quantize_q8_0_split_dev(xb, qs, d, m, k)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ctx.gemm_q8act_dev(qs, d, dev(w), y, m, n, k, wt, il)
    return y.cpu().numpy()


GEMM_CASES = [
    (512, 6144, 2048, Q4_0, 4),  # prefill M=512, FFN up-proj shape
    (512, 2048, 6144, Q4_0, 4),  # down-proj shape
    (512, 6144, 2048, Q8_0, 1),  # the 64-row tile, plain Q8_0 rows
    (700, 6100, 1024, Q8_0, 4),  # the 64-row tile with ragged M and N (guarded loads and stores)
    (512, 2048, 1024, Q4_0, 1),  # the eight-wave 32-row tile, plain rows, XCD rectangles of 8x8 tiles
    (65, 100, 256, Q8_0, 1),     # ragged M and N, plain Q8_0
    (1, 64, 96, Q4_0, 4),        # M=1, odd blocks per row
    (70, 132, 64, Q8_0, 4),
]


@pytest.mark.parametrize("m,n,k,wt,il", GEMM_CASES)
def test_gemm_bit_exact_with_oracle(ctx, zo, m, n, k, wt, il):
    rng = np.random.default_rng(m + n + k)
    w = synth.weight(rng, wt, n, k, il)
    x = synth.activations(rng, m, k)
    y = _gemm(ctx, x, w, n, k, wt, il)
    xq = zo.quantize_q8_0(x.reshape(-1))
    # every row (the oracle takes ~6 s per 512-row prefill shape)
    ref = zo.gemm_q8act(xq, w, m, n, k, wt, il)
    bad = np.flatnonzero(np.any(y.view(np.uint32) != ref.view(np.uint32), axis=1))
    assert bad.size == 0, f"{bad.size} of {m} rows differ, first {bad[:8]}"
    # report the Q8_0-activation error against the fp32-activation GEMV
    f = zo.linear_range(x[0], w, k, n, wt, il)
    err = float(np.max(np.abs(y[0] - f)) / np.max(np.abs(f)))
    print(f"M={m} N={n} K={k}: Q8_0 activations vs fp32 GEMV rel err {err:.2e}")
    assert err < 5e-2
