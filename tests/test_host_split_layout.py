"""synth.x4_split, the numpy restatement of the split-scale X4 layout the
GPU tests compare against: per group of four rows, the blocks' quants
[block][row][qb], then their fp16 scales [block][row]."""
import numpy as np

from zero_amd import synth

Q4_0, Q8_0 = 2, 8


def test_split_matches_x4_numpy():
    rng = np.random.default_rng(1)
    for quant in (Q4_0, Q8_0):
        w = synth.weight(rng, quant, 8, 64, 4)
        s = synth.x4_split(w, 8, 64, quant)
        qb = 16 if quant == Q4_0 else 32
        assert s.size == w.size
        # group 1, block 1, row 2: quants and scale
        gb = 8 + 4 * qb
        src = w[(1 * 2 + 1) * gb:(1 * 2 + 2) * gb]
        g = s[2 * gb:4 * gb]
        assert np.array_equal(g[(4 * 1 + 2) * qb:(4 * 1 + 3) * qb], src[8 + 2 * qb:8 + 3 * qb])
        assert np.array_equal(g[2 * 4 * qb + 2 * (4 * 1 + 2):2 * 4 * qb + 2 * (4 * 1 + 2) + 2], src[4:6])
