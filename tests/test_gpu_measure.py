"""The measurement hooks bench.py times against (zg_read_floor_dev,
zg_strip_loads_dev): they run to completion on weight-sized buffers without
touching the sink, and refuse bad arguments with ZG_ERR_INVALID_ARG."""
import pytest
import torch

import zero_amd
from zero_amd import _lib

pytestmark = pytest.mark.gpu


def test_read_floor_and_strip_loads(ctx):
    # constant bytes: every XOR the hooks form is one of a few fixed words,
    # never the sink's trigger value
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    for rows in (6144, 151_936):
        w = torch.full((rows * 2048 // 32 * 18,), 0x11, dtype=torch.uint8, device="cuda")
        x = torch.zeros(2048, dtype=torch.float32, device="cuda")
        for u in (1, 2, 4, 8):
            ctx.read_floor_dev(w, w.numel(), u, sink)
        ctx.strip_loads_dev(w, rows, None, sink)
        ctx.strip_loads_dev(w, rows, x, sink)
        torch.cuda.synchronize()
        assert int(sink.item()) == 0
    for call in (lambda: ctx.read_floor_dev(w, 100, 1, sink), lambda: ctx.read_floor_dev(w, 4096, 3, sink),
                 lambda: ctx.strip_loads_dev(w, 6, None, sink)):
        with pytest.raises(zero_amd.ZgError) as e:
            call()
        assert e.value.code == _lib.ZG_ERR_INVALID_ARG
