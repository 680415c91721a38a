"""Lifetimes and failure codes at the C ABI.

* zg_clear while a model is alive: the reference clears its layout registry
  before it indexes the next model (kernel/src/model_loader.rs:488,
  weight_layout.rs:57); a live model keeps the uploaded copies it reads, so
  its decode is unchanged after the clear.
* zg_destroy before zg_model_destroy: the context is released by the last
  model instead, and the model keeps decoding until then.
* overlapping registrations are refused.
* HIP failures come back as status codes (the GPU side of the reference's
  failure handling, kernel/src/smp.rs:1677-1711): an allocation no GPU can
  satisfy is ZG_ERR_OUT_OF_MEMORY with the HIP message, a device that does
  not exist is ZG_ERR_HIP.  Neither runs a kernel.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import zero_amd
from zero_amd import _lib, synth
from zero_amd.model import GpuModel
from zero_amd.ops import ZgError

pytestmark = pytest.mark.gpu
Q4_0 = 2

TINY = synth.ModelConfig(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64,
                         vocab_padded=1024, vocab_real=1000, max_ctx=64)


def _decode(gm, n=12, tok=5):
    toks, hids = [], []
    for pos in range(n):
        tok, _, hid, _ = gm.step(tok, pos, want_hidden=True)
        toks.append(tok)
        hids.append(hid)
    return toks, np.stack(hids)


@pytest.fixture(scope="module")
def tiny():
    return synth.random_model(TINY, seed=11)


def test_clear_keeps_live_model_weights(tiny):
    with zero_amd.Context(0) as c:
        gm = GpuModel(c, tiny)
        toks0, hid0 = _decode(gm)
        c.clear()
        assert c.registered_count() == 0
        # the freed registry slots take new tensors of the same sizes; the
        # model must still read its own copies
        junk = [np.full(w.nbytes, 0x77, np.uint8) for w in (tiny.layers[0].attn_q, tiny.layers[0].ffn_down)]
        for j in junk:
            c.register(j, Q4_0, 4)
        toks1, hid1 = _decode(gm)
        assert toks1 == toks0
        assert np.array_equal(hid1, hid0)
        gm.close()
        c.clear()


def test_destroy_context_before_model(tiny):
    c = zero_amd.Context(0)
    gm = GpuModel(c, tiny)
    toks0, hid0 = _decode(gm)
    lib = c.lib
    lib.zg_destroy(c.h)  # deferred: the model still holds the context
    toks1, hid1 = _decode(gm)
    assert toks1 == toks0 and np.array_equal(hid1, hid0)
    lib.zg_model_destroy(gm.h)  # releases the model, then the context
    gm.h = None
    c.h = None


def test_overlapping_registration_refused():
    with zero_amd.Context(0) as c:
        fake = torch.empty(256, dtype=torch.uint8, device="cuda")
        c.register_device(0x10000, fake.data_ptr(), 144, Q4_0, 4)
        for key in (0x10000 - 72, 0x10000 + 72, 0x10000 + 143):
            with pytest.raises(ZgError) as ei:
                c.register_device(key, fake.data_ptr(), 144, Q4_0, 4)
            assert ei.value.code == _lib.ZG_ERR_INVALID_ARG
            assert "overlaps" in c.last_error()
        # adjacent ranges are fine
        c.register_device(0x10000 + 144, fake.data_ptr(), 72, Q4_0, 4)
        c.register_device(0x10000 - 72, fake.data_ptr(), 72, Q4_0, 4)
        assert c.registered_count() == 3
        c.clear()


def test_impossible_allocation_is_a_status(tiny):
    """A KV cache of 2 layers x 2 x 2^30 positions x 128 floats (2 TiB)
    cannot be allocated: zg_model_create returns ZG_ERR_OUT_OF_MEMORY with
    the HIP message, frees what it had allocated, and the context stays
    usable."""
    with zero_amd.Context(0) as c:
        gm = GpuModel(c, tiny)  # registers the weights and builds a normal model
        toks0, hid0 = _decode(gm, n=4)
        d = _lib.zg_model_desc()
        C.memmove(C.byref(d), C.byref(gm._desc), C.sizeof(d))
        d.max_ctx = 1 << 30
        h = C.c_void_p()
        rc = c.lib.zg_model_create(c.h, C.byref(d), C.byref(h))
        assert rc == _lib.ZG_ERR_OUT_OF_MEMORY, (rc, c.last_error())
        assert "hipMalloc" in c.last_error()
        assert not h.value
        toks1, hid1 = _decode(gm, n=4)
        assert toks1 == toks0 and np.array_equal(hid1, hid0)
        gm.close()
        # the failed hipMalloc must not surface later as the error of an
        # unrelated launch: building a model checks every launch it records
        gm2 = GpuModel(c, tiny, register=False)
        toks2, hid2 = _decode(gm2, n=4)
        assert toks2 == toks0 and np.array_equal(hid2, hid0)
        gm2.close()
        c.clear()


def test_bad_device_is_hip_error():
    h = C.c_void_p()
    rc = _lib.load().zg_init(1 << 20, C.byref(h))
    assert rc == _lib.ZG_ERR_HIP and not h.value
