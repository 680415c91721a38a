"""ctypes binding of libzero_amd.so (the C ABI of include/zero_gpu.h).

The library is loaded from the package directory only.  When torch is
importable it is imported first: torch ships its own libamdhip64 and our
library's DT_NEEDED "libamdhip64.so.7" then binds to that already-loaded
runtime (same SONAME), so torch tensors and our kernels share one HIP
runtime in the process.  A missing library raises ImportError: there is no
CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

try:  # one HIP runtime per process: torch's copy, when torch is present
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - torch is part of the supported stack
    torch = None

LIB_PATH = Path(__file__).resolve().parent / "libzero_amd.so"

# status codes (include/zero_gpu.h)
ZG_OK = 0
ZG_ERR_INVALID_ARG = -1
ZG_ERR_UNSUPPORTED_QUANT = -2
ZG_ERR_NOT_REGISTERED = -3
ZG_ERR_HIP = -4
ZG_ERR_NONFINITE_LOGITS = -5
ZG_ERR_ARGMAX_IN_PADDING = -6
ZG_ERR_REGISTRY_FULL = -7
ZG_ERR_OUT_OF_MEMORY = -8
ZG_ERR_ATTENTION = -9
ZG_ERR_CONTEXT_FULL = -10
ZG_ERR_MAGIC_MISMATCH = -11
ZG_ERR_UNSUPPORTED_FORMAT = -12
ZG_ERR_INVALID_CONTAINER = -13

ZG_GEN_BATCHED_PREFILL = 1
ZG_GEN_EAGER = 2


class zg_segment(C.Structure):
    _fields_ = [
        ("w", C.c_void_p),
        ("out", C.c_void_p),
        ("out_dim", C.c_size_t),
        ("ggml_type", C.c_uint32),
        ("interleave", C.c_uint32),
    ]


class zg_layer_weights(C.Structure):
    _fields_ = [
        ("attn_q", C.c_void_p), ("attn_k", C.c_void_p), ("attn_v", C.c_void_p), ("attn_o", C.c_void_p),
        ("ffn_gate", C.c_void_p), ("ffn_up", C.c_void_p), ("ffn_down", C.c_void_p),
        ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p), ("q_norm", C.c_void_p), ("k_norm", C.c_void_p),
    ]


N_PROJ = 7  # ZG_PROJ_Q .. ZG_PROJ_DOWN: Q, K, V, O, gate, up, down


class zg_layer_quants(C.Structure):
    _fields_ = [("type", C.c_uint32 * N_PROJ), ("interleave", C.c_uint32 * N_PROJ)]


class zg_model_desc(C.Structure):
    _fields_ = [
        ("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("ffn", C.c_uint32),
        ("n_q_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
        ("vocab_padded", C.c_uint32), ("vocab_real", C.c_uint32), ("max_ctx", C.c_uint32),
        ("rms_eps", C.c_float), ("rope_theta", C.c_float),
        ("lin_type", C.c_uint32), ("lin_interleave", C.c_uint32),
        ("embd_type", C.c_uint32),
        ("head_type", C.c_uint32), ("head_interleave", C.c_uint32),
        ("token_embd", C.c_void_p), ("lm_head", C.c_void_p), ("output_norm", C.c_void_p),
        ("layers", C.POINTER(zg_layer_weights)),
        ("device_pointers", C.c_uint32),
        ("layer_quants", C.POINTER(zg_layer_quants)),
    ]


class zg_smodel_info(C.Structure):
    _fields_ = [
        ("version", C.c_uint32), ("payload_kind", C.c_uint32), ("flags", C.c_uint32),
        ("manifest_offset", C.c_uint64), ("manifest_len", C.c_uint64),
        ("payload_offset", C.c_uint64), ("payload_len", C.c_uint64),
        ("architecture_id", C.c_uint32), ("block_count", C.c_uint32), ("context_length", C.c_uint32),
        ("embedding_length", C.c_uint32), ("feed_forward_length", C.c_uint32),
        ("head_count", C.c_uint32), ("head_count_kv", C.c_uint32),
        ("key_length", C.c_uint32), ("value_length", C.c_uint32),
        ("rope_freq_base", C.c_float), ("layer_norm_rms_epsilon", C.c_float),
        ("vocab_size", C.c_uint32), ("eos_token_id", C.c_uint32),
        ("tensor_count", C.c_uint64),
    ]


class zg_smodel_tensor(C.Structure):
    _fields_ = [
        ("name", C.c_void_p), ("name_len", C.c_size_t),
        ("dtype", C.c_uint32), ("ggml_type", C.c_uint32), ("interleave", C.c_uint32), ("rank", C.c_uint32),
        ("dims", C.c_uint64 * 8),
        ("payload_offset", C.c_uint64),
        ("data", C.c_void_p),
        ("byte_len", C.c_uint64),
    ]


_P = C.c_void_p
_S = C.c_size_t
_U32 = C.c_uint32
_ST = C.c_int32

# name -> (restype, argtypes); every symbol include/zero_gpu.h declares
SIGNATURES = {
    "zg_init": (_ST, [C.c_int, C.POINTER(_P)]),
    "zg_destroy": (None, [_P]),
    "zg_last_error": (C.c_char_p, [_P]),
    "zg_stream": (_P, [_P]),
    "zg_register_weight": (_ST, [_P, _P, _S, _U32, _U32]),
    "zg_register_weight_device": (_ST, [_P, _P, _P, _S, _U32, _U32]),
    "zg_group_of": (_U32, [_P, _P]),
    "zg_rebase": (None, [_P, C.c_int64]),
    "zg_clear": (None, [_P]),
    "zg_registered_count": (_S, [_P]),
    "zg_linear": (_ST, [_P, _P, _P, _P, _S, _S, _U32]),
    "zg_linear_range": (_ST, [_P, _P, _P, _P, _S, _S, _U32, _S, _S]),
    "zg_linear_fused": (_ST, [_P, _P, C.POINTER(zg_segment), _S, _S]),
    "zg_lm_head_argmax": (_ST, [_P, _P, _P, _P, _U32, C.c_float, _S, _S, _S, _P,
                                C.POINTER(_U32), C.POINTER(C.c_float)]),
    "zg_linear_dev": (_ST, [_P, _P, _P, _P, _S, _S, _U32, _U32, _S, _S, _P]),
    "zg_linear_fused_dev": (_ST, [_P, _P, C.POINTER(zg_segment), _S, _S, _P]),
    "zg_lm_head_dev": (_ST, [_P, _P, _P, _P, _S, _S, _U32, _U32, _P, _P]),
    "zg_argmax_unpack": (C.c_int, [C.c_uint64, C.POINTER(_U32), C.POINTER(C.c_float)]),
    "zg_dequant_dev": (_ST, [_P, _P, _P, _S, _S, _U32, _U32, _P]),
    "zg_fp16_to_f32_dev": (_ST, [_P, _P, _P, _S, _P]),
    "zg_read_floor_dev": (_ST, [_P, _P, _S, _U32, _P, _P]),
    "zg_strip_loads_dev": (_ST, [_P, _P, _S, _P, _P, _P]),
    "zg_quantize_q8_0_dev": (_ST, [_P, _P, _P, _S, _S, _P]),
    "zg_quantize_q8_0_split_dev": (_ST, [_P, _P, _P, _P, _S, _S, _P]),
    "zg_gemm_q8act_dev": (_ST, [_P, _P, _P, _P, _P, _S, _S, _S, _U32, _U32, _P]),
    "zg_quantize_q8k_split_dev": (_ST, [_P, _P, _P, _P, _P, _S, _S, _P]),
    "zg_gemm_q8k_dev": (_ST, [_P, _P, _P, _P, _P, _P, _S, _S, _S, _U32, C.c_int, _P]),
    "zg_model_create": (_ST, [_P, C.POINTER(zg_model_desc), C.POINTER(_P)]),
    "zg_model_destroy": (None, [_P]),
    "zg_model_step": (_ST, [_P, _U32, _U32, _P, _P, C.POINTER(_U32), C.POINTER(C.c_float)]),
    "zg_model_generate": (_ST, [_P, _P, _S, _S, _P, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "zg_model_reset": (None, [_P]),
    "zg_model_first_nonfinite": (_S, [_P, C.c_char_p, _S]),
    "zg_model_test_drop_qkv_stores": (_ST, [_P, C.c_int32]),
    "zg_model_prefill": (_ST, [_P, _P, _S, _U32, _P, C.POINTER(_U32), C.POINTER(C.c_float)]),
    "zg_model_generate_ex": (_ST, [_P, _P, _S, _S, _U32, _P, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "zg_linear_q8act_dev": (_ST, [_P, _P, _P, _P, _S, _S, _U32, _U32, _P]),
    "zg_quantize_q8k_dev": (_ST, [_P, _P, _P, _S, _P]),
    "zg_linear_q4k_q8k_dev": (_ST, [_P, _P, _P, _P, _S, _S, _P]),
    "zg_linear_q4k_vnni": (_ST, [_P, _P, _P, _P, _S, _S]),
    "zg_linear_q4k_vnni_noalloc": (_ST, [_P, _P, _P, _P, _S, _S, _P]),
    "zg_smodel_open": (_ST, [_P, _S, C.POINTER(_P)]),
    "zg_smodel_close": (None, [_P]),
    "zg_smodel_get_info": (_ST, [_P, C.POINTER(zg_smodel_info)]),
    "zg_smodel_get_tensor": (_ST, [_P, C.c_uint64, C.POINTER(zg_smodel_tensor)]),
    "zg_smodel_find": (_ST, [_P, C.c_char_p, C.POINTER(zg_smodel_tensor)]),
    "zg_smodel_register_all": (_ST, [_P, _P]),
}

_lib = None


def load() -> C.CDLL:
    """Load libzero_amd.so (built in-tree by zero_amd/build.py)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build the gfx950 library first "
            "(python -c 'import __graft_entry__ as g; g.build()'); there is no CPU fallback")
    lib = C.CDLL(os.fspath(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
