"""The .smodel reader (zg_smodel_*, zero_amd.smodel) on the CPU.

Pinned three ways:
* against the packer's own record of each fixture (tiny_qwen3_v2*.inspect.json,
  written by tools/silicatepack.py's `inspect` from its manifest, not from
  the SIDX bytes this reader parses): header fields, every tensor's name,
  dtype, shape, payload offset, byte length and sha256;
* byte for byte against the oracle's quantizers (themselves pinned to the
  packer's golden vectors) applied to the seeded fp32 checkpoint the
  fixture was packed from: Q4_0X4 (or, in the q8 fixture, Q8_0X4) linears,
  Q8_0 embedding, Q8_0X4 LM head, F32 norms; in the v1 fixture (the
  packer's default layout) plain Q4_0 linears and a plain Q8_0 LM head;
* the reference loader's rejection rules
  (kernel/src/model_loader.rs:380-575, 599-659), one patched field at a
  time, each mapped to its LoadError kind.
"""
import json
import struct
from pathlib import Path

import numpy as np
import pytest

from golden import make_smodel_fixture as fx
from zero_amd import _lib
from zero_amd.smodel import InvalidContainer, MagicMismatch, SModel, UnsupportedFormat
from zero_amd.synth import Q4_0, Q8_0

GOLDEN = Path(__file__).parent / "golden"
FIX = (GOLDEN / "tiny_qwen3_v2.smodel").read_bytes()
REC = json.loads((GOLDEN / "tiny_qwen3_v2.inspect.json").read_text())
MAN = REC["manifest"]
# (fixture stem, make_smodel_fixture variant): the 2-layer --quant auto
# artifact, the 1-layer --quant q8_0 artifact (Q8_0X4 layer linears) and the
# 1-layer v1 artifact (no --interleave: plain rows)
FIXTURES = [("tiny_qwen3_v2", "auto"), ("tiny_qwen3_v2_q8", "q8_0"), ("tiny_qwen3_v1", "v1")]

DTYPE_ID = {"F32": 0, "Q8_0": 8, "Q4_0": 2, "Q4_0X4": 100, "Q8_0X4": 101}
P0 = REC["header"]["payload_offset"]  # SIDX header position in the file
ENTRY0 = P0 + 128


def _load(stem):
    return (GOLDEN / f"{stem}.smodel").read_bytes(), json.loads((GOLDEN / f"{stem}.inspect.json").read_text())


def _index(name: str) -> int:
    return [t.name for t in SModel(FIX).tensors].index(name)


@pytest.mark.parametrize("stem,variant", FIXTURES)
def test_header_matches_packer_record(stem, variant):
    fix, rec = _load(stem)
    s = SModel(fix)
    h = rec["header"]
    for f in ("version", "payload_kind", "flags", "manifest_offset", "manifest_len", "payload_offset", "payload_len"):
        assert getattr(s.info, f) == h[f], f
    assert s.info.tensor_count == rec["manifest"]["tensor_count"] == 3 + 11 * fx.VARIANTS[variant][2]


@pytest.mark.parametrize("stem,variant", FIXTURES)
def test_model_config_matches_packer_record(stem, variant):
    fix, rec = _load(stem)
    i, c = SModel(fix).info, rec["manifest"]["model_config"]
    assert i.architecture_id == 1  # qwen3
    assert (i.block_count, i.embedding_length, i.feed_forward_length) == (
        c["num_hidden_layers"], c["hidden_size"], c["intermediate_size"])
    assert (i.head_count, i.head_count_kv, i.key_length, i.value_length) == (
        c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"], c["head_dim"])
    assert (i.context_length, i.vocab_size, i.eos_token_id) == (
        c["max_position_embeddings"], c["vocab_size"], c["eos_token_id"])
    assert i.rope_freq_base == np.float32(c["rope_theta"])
    assert i.layer_norm_rms_epsilon == np.float32(c["rms_norm_eps"])


@pytest.mark.parametrize("stem,variant", FIXTURES)
def test_tensors_match_packer_record(stem, variant):
    import hashlib

    fix, rec = _load(stem)
    s = SModel(fix)
    want = {t["name"]: t for t in rec["manifest"]["tensors"]}
    assert sorted(t.name for t in s.tensors) == sorted(want)
    for t in s.tensors:
        w = want[t.name]
        assert t.dtype == DTYPE_ID[w["dtype"]], t.name
        assert list(t.shape) == w["shape"], t.name
        assert (t.payload_offset, t.byte_len) == (w["payload_offset"], w["byte_len"]), t.name
        assert t.interleave == w.get("row_interleave", 1), t.name
        assert hashlib.sha256(t.data.tobytes()).hexdigest() == w["sha256"], t.name
    # v2: the 7 linears per layer and the LM head interleaved, embedding and
    # norms plain; v1: every tensor plain
    _, _, layers, il = fx.VARIANTS[variant]
    assert s.info.version == (2 if il else 1)
    assert sum(t.interleave == 4 for t in s.tensors) == (7 * layers + 1 if il else 0)
    assert s["token_embd.weight"].interleave == 1 and s["output.weight"].ggml_type == Q8_0
    assert s["blk.0.attn_q.weight"].ggml_type == (Q8_0 if variant == "q8_0" else Q4_0)


def test_find_uses_exact_names():
    s = SModel(FIX)
    assert s.find("blk.1.ffn_down.weight") is s["blk.1.ffn_down.weight"]
    with pytest.raises(Exception):
        s.find("blk.1.ffn_down")


@pytest.mark.parametrize("stem,variant", FIXTURES)
def test_tensor_bytes_rebuild_from_the_checkpoint(zo, stem, variant):
    """Every packed tensor equals the oracle's quantization of the seeded
    fp32 source named in the manifest."""
    src = fx.checkpoint(variant=variant)
    fix, rec = _load(stem)
    s = SModel(fix)
    for w in rec["manifest"]["tensors"]:
        x = src[w["source"]["name"]]
        rows = x.shape[0]
        cols = x.shape[1] if x.ndim == 2 else 1
        dt = w["dtype"]
        if dt == "F32":
            want = x.astype("<f4").tobytes()
        elif dt.startswith("Q8_0"):
            want = zo.quantize_q8_0(x.reshape(-1))
            if dt.endswith("X4"):
                want = zo.interleave_x4(want, rows, cols, Q8_0)
            want = want.tobytes()
        else:
            assert dt.startswith("Q4_0")
            want = zo.quantize_q4_0(x.reshape(-1))
            if dt.endswith("X4"):
                want = zo.interleave_x4(want, rows, cols, Q4_0)
            want = want.tobytes()
        assert s[w["name"]].data.tobytes() == want, w["name"]


def test_to_model_shapes_and_views():
    s = SModel(FIX)
    m = s.to_model(max_ctx=48)
    c = m.cfg
    assert (c.n_layers, c.hidden, c.ffn, c.n_q_heads, c.n_kv_heads, c.head_dim) == (2, 128, 256, 2, 1, 64)
    assert (c.vocab_padded, c.vocab_real, c.max_ctx) == (256, 256, 48)
    assert (c.lin_type, c.embd_type, c.head_type) == (Q4_0, Q8_0, Q8_0)
    L = m.layers[1]
    assert L.attn_q.nbytes == 128 * 4 * 18 and L.ffn_down.nbytes == 128 * 8 * 18
    assert L.q_norm.dtype == np.float32 and L.q_norm.size == 64
    # zero-copy: the arrays alias the container image
    assert np.shares_memory(m.lm_head, s.image) and np.shares_memory(L.attn_norm, s.image)


def test_to_model_plain_layout():
    """A v1 artifact: the model view keeps the plain row layouts."""
    m = SModel(GOLDEN / "tiny_qwen3_v1.smodel").to_model()
    c = m.cfg
    assert (c.n_layers, c.lin_type, c.lin_interleave, c.head_type, c.head_interleave) == (1, Q4_0, 1, Q8_0, 1)
    assert m.layers[0].attn_o.nbytes == 128 * 4 * 18 and m.lm_head.nbytes == 256 * 4 * 34
    v2 = SModel(FIX).to_model().cfg
    assert (v2.lin_interleave, v2.head_interleave) == (4, 4)


def test_path_and_memmap_source(tmp_path):
    p = tmp_path / "m.smodel"
    p.write_bytes(FIX)
    s = SModel(p)
    assert isinstance(s.image, np.memmap) and s.info.tensor_count == 25


# ---------------------------------------------------------------------------
# rejection rules, one field at a time
# ---------------------------------------------------------------------------

def _patched(*edits, cut=None) -> bytes:
    b = bytearray(FIX)
    for fmt, off, val in edits:
        struct.pack_into(fmt, b, off, val)
    return bytes(b[:cut] if cut is not None else b)


def _entry(i: int, field: int) -> int:
    return ENTRY0 + 104 * i + field


HEADER_CASES = [
    ("magic", _patched(("<I", 0, 0x46554747)), MagicMismatch),
    ("version 0", _patched(("<I", 4, 0)), UnsupportedFormat),
    ("version 3", _patched(("<I", 4, 3)), UnsupportedFormat),
    ("header_len 64", _patched(("<I", 8, 64)), UnsupportedFormat),
    ("payload kind 0", _patched(("<I", 44, 0)), UnsupportedFormat),
    ("payload kind 3", _patched(("<I", 44, 3)), UnsupportedFormat),
    ("payload kind 1 (GGUF wrapper)", _patched(("<I", 44, 1)), UnsupportedFormat),
    ("manifest_len 0", _patched(("<Q", 20, 0)), InvalidContainer),
    ("manifest inside header", _patched(("<Q", 12, 64)), InvalidContainer),
    ("manifest past payload", _patched(("<Q", 20, P0)), InvalidContainer),
    ("manifest offset overflow", _patched(("<Q", 12, 2**64 - 8)), InvalidContainer),
    ("payload past end", _patched(("<Q", 36, len(FIX))), InvalidContainer),
    ("payload under SIDX header", _patched(("<Q", 36, 100)), InvalidContainer),
    ("payload under 4 bytes", _patched(("<Q", 36, 3)), InvalidContainer),
    ("2 MiB flag, offset 20480", _patched(("<I", 48, 1)), InvalidContainer),
    ("truncated file", _patched(cut=len(FIX) - 1), InvalidContainer),
    ("shorter than a header", FIX[:127], InvalidContainer),
    ("empty", b"", InvalidContainer),
]

INDEX_CASES = [
    ("SIDX magic", _patched(("<I", P0, 0x58444958)), UnsupportedFormat),
    ("SIDX version 2", _patched(("<I", P0 + 4, 2)), UnsupportedFormat),
    ("SIDX header 64", _patched(("<I", P0 + 8, 64)), UnsupportedFormat),
    ("tensor count 10001", _patched(("<I", P0 + 12, 10001)), InvalidContainer),
    ("entry size 96", _patched(("<I", P0 + 16, 96)), UnsupportedFormat),
    ("names inside entries", _patched(("<I", P0 + 20, 128)), InvalidContainer),
    ("names past payload", _patched(("<I", P0 + 24, 1 << 30)), InvalidContainer),
    ("entries past payload", _patched(("<I", P0 + 12, 9999)), InvalidContainer),
    ("rank 9", _patched(("<I", _entry(0, 12), 9)), InvalidContainer),
    ("name past names", _patched(("<I", _entry(0, 4), 1 << 20)), InvalidContainer),
    ("name not UTF-8", None, InvalidContainer),
    ("unknown dtype 4", _patched(("<I", _entry(0, 8), 4)), UnsupportedFormat),
    ("unknown dtype 99", _patched(("<I", _entry(0, 8), 99)), UnsupportedFormat),
    ("unknown dtype 31", _patched(("<I", _entry(0, 8), 31)), UnsupportedFormat),
    ("tensor past payload", _patched(("<Q", _entry(0, 88), 1 << 40)), InvalidContainer),
    ("tensor offset overflow", _patched(("<Q", _entry(0, 80), 2**64 - 16)), InvalidContainer),
]


def _utf8_case() -> bytes:
    b = bytearray(FIX)
    name_off, = struct.unpack_from("<I", b, _entry(0, 0))
    names_offset, = struct.unpack_from("<I", b, P0 + 20)
    b[P0 + names_offset + name_off] = 0xFF
    return bytes(b)


@pytest.mark.parametrize("label,data,err", HEADER_CASES + INDEX_CASES, ids=[c[0] for c in HEADER_CASES + INDEX_CASES])
def test_rejections(label, data, err):
    if data is None:
        data = _utf8_case()
    with pytest.raises(err) as e:
        SModel(data)
    assert e.value.code == {MagicMismatch: _lib.ZG_ERR_MAGIC_MISMATCH, UnsupportedFormat: _lib.ZG_ERR_UNSUPPORTED_FORMAT,
                            InvalidContainer: _lib.ZG_ERR_INVALID_CONTAINER}[err]


def test_interleaved_geometry_rules():
    q = _index("blk.0.attn_q.weight")
    embd = _index("token_embd.weight")
    with pytest.raises(InvalidContainer):  # rows % 4 != 0
        SModel(_patched(("<Q", _entry(q, 16), 126)))
    with pytest.raises(InvalidContainer):  # rank 1
        SModel(_patched(("<I", _entry(q, 12), 1)))
    with pytest.raises(InvalidContainer):  # rank 3
        SModel(_patched(("<I", _entry(q, 12), 3)))
    # a plain tensor may have any row count; an X4 dtype on it needs rows % 4
    SModel(_patched(("<Q", _entry(embd, 16), 255)))
    with pytest.raises(InvalidContainer):
        SModel(_patched(("<Q", _entry(embd, 16), 255), ("<I", _entry(embd, 8), 101)))
    s = SModel(_patched(("<I", _entry(embd, 8), 101)))
    assert s["token_embd.weight"].interleave == 4


def test_accepted_variants():
    # version 1 and an unused 2 MiB flag on an aligned offset are fine
    assert SModel(_patched(("<I", 4, 1))).info.version == 1
    # trailing bytes after the payload are allowed (payload_end <= len)
    assert SModel(FIX + b"\0" * 100).info.tensor_count == 25
    # zero tensors: a valid, empty index
    assert SModel(_patched(("<I", P0 + 12, 0))).tensors == []


def test_payload_moved_to_a_2mib_boundary():
    """The packer's --payload-alignment 2M layout with header flag bit 0:
    tensor offsets are payload-relative, so moving the payload keeps every
    tensor's bytes."""
    mib2 = 2 << 20
    hdr = bytearray(FIX[:128])
    struct.pack_into("<Q", hdr, 28, mib2)
    struct.pack_into("<I", hdr, 48, 1)
    img = bytes(hdr) + FIX[128:P0] + b"\0" * (mib2 - P0) + FIX[P0:]
    s, ref = SModel(img), SModel(FIX)
    assert s.info.flags == 1 and s.info.payload_offset == mib2
    for a, b in zip(s.tensors, ref.tensors):
        assert a.name == b.name and a.data.tobytes() == b.data.tobytes()
    # the same image without 2 MiB alignment is rejected under the flag
    hdr2 = bytearray(hdr)
    struct.pack_into("<Q", hdr2, 28, mib2 - 4096)
    with pytest.raises(InvalidContainer):
        SModel(bytes(hdr2) + img[128:])


def test_model_view_rejections():
    s = SModel(_patched(("<I", P0 + 36, 2)))  # deepseek2 architecture id
    with pytest.raises(UnsupportedFormat):
        s.to_model()
    q = _index("blk.1.attn_q.weight")
    # per-projection types are taken from the file (ForwardPassDispatch's
    # per-layer table), so relabelling one Q4_0X4 tensor Q8_0X4 is caught by
    # its byte length, not its type
    s = SModel(_patched(("<I", _entry(q, 8), 101)))
    with pytest.raises(InvalidContainer):
        s.to_model()
    s = SModel(_patched(("<I", _entry(q, 8), 12)))  # Q4_K in place of Q4_0X4: same check
    with pytest.raises(InvalidContainer):
        s.to_model()
    n = _index("blk.0.attn_q_norm.weight")
    s = SModel(_patched(("<Q", _entry(n, 16), 32)))  # q_norm of the wrong length
    with pytest.raises(InvalidContainer):
        s.to_model()
