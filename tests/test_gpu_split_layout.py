"""The split-scale X4 device layout (interleave 5: per group of four rows,
the blocks' quants first, then their fp16 scales), the layout a model
repacks its Q4_0 / Q8_0 X4 layer projections into.  The strip kernel
decodes the same lanes from it as from the reference's X4 group-blocks
(weight_layout.rs:57-149), so every kernel form gives the same bits from
either layout: GEMV, fused segments with each prologue and epilogue the
operator API reaches, the Q8_0-activation GEMV and the prefill GEMM."""
import numpy as np
import pytest
import torch

import zero_amd
from zero_amd import _lib, synth

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 8


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bits(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("quant,rows,k", [(Q4_0, 6144, 2048), (Q4_0, 2048, 6144), (Q4_0, 49152, 2048),
                                          (Q4_0, 1024, 512), (Q8_0, 4096, 2048), (Q8_0, 8192, 1024)])
def test_gemv_bits_equal_x4(ctx, quant, rows, k):
    rng = np.random.default_rng(rows + k + quant)
    w = synth.weight(rng, quant, rows, k, 4)
    x = dev(synth.activations(rng, k))
    wx, ws = dev(w), dev(synth.x4_split(w, rows, k, quant))
    y4 = torch.empty(rows, device="cuda")
    y5 = torch.full((rows,), -1.0, device="cuda")
    ctx.linear_dev(x, wx, y4, k, rows, quant, 4)
    ctx.linear_dev(x, ws, y5, k, rows, quant, 5)
    assert np.array_equal(bits(y4), bits(y5))
    # a row range
    y5r = torch.full((rows,), -1.0, device="cuda")
    ctx.linear_dev(x, ws, y5r, k, rows, quant, 5, start=8, end=rows - 4)
    assert np.array_equal(bits(y5r)[8:rows - 4], bits(y4)[8:rows - 4])
    assert torch.all(y5r[:8] == -1.0) and torch.all(y5r[rows - 4:] == -1.0)


@pytest.mark.parametrize("quant,rows,k", [(Q8_0, 2048, 6144), (Q8_0, 2048, 8192), (Q8_0, 12288, 2048),
                                          (Q8_0, 151936, 2048)])
def test_q8_0_strip_forms_vs_oracle(ctx, zo, quant, rows, k):
    """Split Q8_0 groups take the strip kernel at shapes where X4 groups
    take the segment or LDS-staged kernels (12 and 16 strips, more than
    eight groups per CU, the LM-head height): within rel 1e-3 of the
    oracle's f32 GEMV on the same weights, and the argmax epilogue's
    token equal to the oracle's."""
    rng = np.random.default_rng(rows * 3 + k)
    w = synth.weight(rng, quant, rows, k, 4)
    x_h = synth.activations(rng, k)
    y = torch.empty(rows, device="cuda")
    ws = dev(synth.x4_split(w, rows, k, quant))
    ctx.linear_dev(dev(x_h), ws, y, k, rows, quant, 5)
    got = y.cpu().numpy()
    for s0, s1 in ((0, 256), (rows - 256, rows)):
        ref = zo.linear_range(x_h, w, k, rows, quant, 4, s0, s1)[s0:s1]
        assert np.max(np.abs(got[s0:s1] - ref)) <= 1e-3 * np.max(np.abs(ref)), (s0, s1)
    if rows == 151936:
        best = torch.zeros(1, dtype=torch.int64, device="cuda")
        logits = torch.empty(rows, device="cuda")
        ctx.lm_head_dev(dev(x_h), ws, logits, k, rows, quant, 5, best)
        assert int(np.argmax(logits.cpu().numpy())) == int(np.argmax(got))


@pytest.mark.parametrize("quant", [Q4_0, Q8_0])
def test_fused_bits_equal_x4(ctx, quant):
    """Q|K|V-shaped segments in one launch."""
    rng = np.random.default_rng(40 + quant)
    k, dims = 2048, (2048, 1024, 1024)
    ws = [synth.weight(rng, quant, n, k, 4) for n in dims]
    x = dev(synth.activations(rng, k))
    outs = {}
    for il in (4, 5):
        ys = [torch.empty(n, device="cuda") for n in dims]
        segs = [(dev(w if il == 4 else synth.x4_split(w, n, k, quant)), y, n, quant, il)
                for w, y, n in zip(ws, ys, dims)]
        ctx.linear_fused_dev(x, segs, k)
        outs[il] = [bits(y) for y in ys]
    for a, b in zip(outs[4], outs[5]):
        assert np.array_equal(a, b)


def test_q8act_gemv_and_gemm_bits_equal_x4(ctx, zo):
    rng = np.random.default_rng(77)
    for quant, rows, k in ((Q4_0, 6144, 2048), (Q8_0, 1024, 512)):
        w = synth.weight(rng, quant, rows, k, 4)
        wx, ws = dev(w), dev(synth.x4_split(w, rows, k, quant))
        xq = dev(zo.quantize_q8_0(synth.activations(rng, k)))
        y4, y5 = torch.empty(rows, device="cuda"), torch.empty(rows, device="cuda")
        ctx.linear_q8act_dev(xq, wx, y4, k, rows, quant, 4)
        ctx.linear_q8act_dev(xq, ws, y5, k, rows, quant, 5)
        assert np.array_equal(bits(y4), bits(y5))
        # the prefill GEMM, a ragged M
        m = 70
        xm = dev(synth.activations(rng, m, k))
        qs = torch.empty((m, k), dtype=torch.int8, device="cuda")
        dd = torch.empty((m, k // 32), dtype=torch.int16, device="cuda")
        ctx.quantize_q8_0_split_dev(xm, qs, dd, m, k)
        g4, g5 = torch.empty((m, rows), device="cuda"), torch.empty((m, rows), device="cuda")
        ctx.gemm_q8act_dev(qs, dd, wx, g4, m, rows, k, quant, 4)
        ctx.gemm_q8act_dev(qs, dd, ws, g5, m, rows, k, quant, 5)
        assert np.array_equal(bits(g4), bits(g5))


def test_split_layout_errors(ctx):
    rng = np.random.default_rng(3)
    w = dev(synth.x4_split(synth.weight(rng, Q4_0, 64, 256, 4), 64, 256, Q4_0))
    x = dev(synth.activations(rng, 256))
    y = torch.empty(64, device="cuda")
    for call in (lambda: ctx.linear_dev(x, w, y, 256, 64, Q4_0, 5),           # in_dim not a multiple of 512
                 lambda: ctx.dequant_dev(w, torch.empty(64 * 256, device="cuda"), 64, 256, Q4_0, 5),
                 lambda: ctx.linear_dev(x, w, y, 256, 64, 12, 5)):             # K-quants have no such layout
        with pytest.raises(zero_amd.ZgError) as e:
            call()
        assert e.value.code == _lib.ZG_ERR_INVALID_ARG
