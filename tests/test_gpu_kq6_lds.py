"""The Q6_K GEMV with LDS-staged activations (kq6l_kernel, in_dim
8192..14336) at three shapes: within rel 1e-3 of the oracle's f32 GEMV
(linear.rs:352-504) and no further from an f64 dot than 4x the oracle's
own distance, with an all-zero and a tiny activation chunk; a NaN, an
infinity or a chunk of magnitude 1e-35 in x gives non-finite rows where the
oracle's are (every row), NaN for NaN, and finite results within the bar."""
import numpy as np
import pytest
import torch

from zero_amd import synth

pytestmark = pytest.mark.gpu
Q6K = 14


def run(ctx, w, x, rows, k):
    y = torch.empty(rows, device="cuda")
    ctx.linear_dev(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), y, k, rows, Q6K, 1)
    return y.cpu().numpy()


@pytest.mark.parametrize("rows,k", [(4096, 14336), (8192, 8192), (6144, 12288)])
def test_q6k_lds_kernel_vs_oracle(ctx, zo, rows, k):
    rng = np.random.default_rng(rows + k)
    w = synth.weight(rng, Q6K, rows, k, 1)
    x = synth.activations(rng, k)
    x[:16] = 0.0          # an all-zero chunk
    x[16:32] *= 1e-20     # a small but representable chunk
    got = run(ctx, w, x, rows, k)
    sample = np.r_[0:96, rows - 96:rows]
    ref = np.concatenate([zo.linear_range(x, w, k, rows, Q6K, 1, 0, 96)[:96],
                          zo.linear_range(x, w, k, rows, Q6K, 1, rows - 96, rows)[rows - 96:]])
    f64 = zo.dequant(w, rows, k, Q6K, 1)[sample].astype(np.float64) @ x.astype(np.float64)
    scale = np.max(np.abs(ref))
    assert np.max(np.abs(got[sample] - ref)) <= 1e-3 * scale
    assert np.max(np.abs(got[sample] - f64)) <= 4 * max(np.max(np.abs(ref - f64)), 1e-7 * scale)


@pytest.mark.parametrize("case", ["nan", "inf", "tiny"])
def test_q6k_lds_kernel_nonfinite_and_tiny_inputs(ctx, zo, case):
    rows, k = 4096, 14336
    rng = np.random.default_rng(9)
    w = synth.weight(rng, Q6K, rows, k, 1)
    x = synth.activations(rng, k)
    if case == "nan":
        x[5000] = np.nan
    elif case == "inf":
        x[777] = np.inf
    else:
        x[1024:1040] = 1e-35
    got = run(ctx, w, x, rows, k)
    ref = zo.linear_range(x, w, k, rows, Q6K, 1, 0, 256)[:256]
    if case == "tiny":
        assert np.max(np.abs(got[:256] - ref)) <= 1e-3 * np.max(np.abs(ref))
    else:
        # every row sees the non-finite value: the fp32 form's rows are
        # non-finite where the oracle's are (NaN against NaN; an infinity
        # may meet a zero product as NaN in either order of operations)
        assert not np.any(np.isfinite(got[:256])) and not np.any(np.isfinite(ref))
        if case == "nan":
            assert np.all(np.isnan(got[:256]))
