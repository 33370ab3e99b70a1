"""ctypes binding of ``libedgebert_hip.so`` (the C ABI in ``include/``).

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
# EDGEBERT_HIP_LIB selects another build of the same sources (the host
# sanitizer build of `make -C edgebert_amd/csrc sanitize`).
LIB_PATH = os.environ.get("EDGEBERT_HIP_LIB") or os.path.join(_HERE, "libedgebert_hip.so")
HEADERS = [os.path.join(os.path.dirname(_HERE), "include", h)
           for h in ("edgebert_hip.h", "edgebert_hip_ops.h")]

EBH_OK = 0
EBH_ERR_INVALID_ARG = -1
EBH_ERR_NOT_FOUND = -2
EBH_ERR_SHAPE = -3
EBH_ERR_STATE = -4
EBH_ERR_HIP = -5
EBH_ERR_RANGE = -6
EBH_DTYPE_F32 = 0
EBH_DTYPE_BF16 = 1
EBH_DTYPE_F32_BF16X6 = 2
NOALLOC_SCRATCH_BYTES = 128 << 20   # EBH_NOALLOC_SCRATCH_BYTES
EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RESID, EPI_NONE = 0, 1, 2, 3
PROF = {"none": 0, "gemm_qkv": 1, "attention": 2, "gemm_out": 3, "gemm_ffn_up": 4,
        "gemm_ffn_down": 5, "layernorm": 6, "embed": 7, "pool": 8}

_ERR_NAMES = {EBH_ERR_INVALID_ARG: "EBH_ERR_INVALID_ARG", EBH_ERR_NOT_FOUND: "EBH_ERR_NOT_FOUND",
              EBH_ERR_SHAPE: "EBH_ERR_SHAPE", EBH_ERR_STATE: "EBH_ERR_STATE",
              EBH_ERR_HIP: "EBH_ERR_HIP", EBH_ERR_RANGE: "EBH_ERR_RANGE"}


class EbhError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_ERR_NAMES.get(code, code)}: {msg}")
        self.code = code


class EbhConfig(ctypes.Structure):
    _fields_ = [("hidden_size", ctypes.c_int32), ("num_attention_heads", ctypes.c_int32),
                ("num_hidden_layers", ctypes.c_int32), ("intermediate_size", ctypes.c_int32),
                ("vocab_size", ctypes.c_int32), ("max_position_embeddings", ctypes.c_int32),
                ("type_vocab_size", ctypes.c_int32), ("layer_norm_eps", ctypes.c_float)]


_vp = ctypes.c_void_p
_i32, _i64, _f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
_SIGS = {
    "ebh_last_error": (ctypes.c_char_p, []),
    "ebh_create": (_i32, [ctypes.POINTER(EbhConfig), ctypes.POINTER(_vp)]),
    "ebh_set_tensor": (_i32, [_vp, ctypes.c_char_p, _vp, ctypes.POINTER(_i64), _i32]),
    "ebh_load_safetensors": (_i32, [_vp, ctypes.c_char_p]),
    "ebh_finalize": (_i32, [_vp, _i32]),
    "ebh_destroy": (None, [_vp]),
    "ebh_forward": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp]),
    "ebh_encode": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "ebh_encode_device": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp]),
    "ebh_encode_device_noalloc": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp]),
    "ebh_score": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp]),
    "ebh_score_device": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "ebh_synchronize": (_i32, [_vp]),
    "ebh_set_graph_replay": (_i32, [_vp, _i32]),
    "ebh_tokenizer_load": (_i32, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "ebh_tokenizer_from_json": (_i32, [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "ebh_tokenizer_destroy": (None, [_vp]),
    "ebh_tokenize": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp, _vp, ctypes.POINTER(_i32), _i32]),
    "ebh_encode_texts": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _vp, _i32]),
    "ebh_score_texts": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32]),
    "ebh_last_tokens": (_i32, [_vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "ebh_model_info": (_i32, [_vp, ctypes.POINTER(EbhConfig), ctypes.POINTER(_i32)]),
    "ebh_profile_enable": (_i32, [_vp, _i32]),
    "ebh_profile_read": (_i32, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_double)]),
    "ebh_op_gemm": (_i32, [_vp, _i64, _vp, _i64, _i32, _vp, _vp, _i64, _vp, _i64, _i32, _i32,
                           _i32, _i32, _vp]),
    "ebh_op_gemm_bf16": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32,
                                _vp]),
    "ebh_op_attention": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "ebh_op_attention_bf16": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "ebh_op_layer_norm": (_i32, [_vp, _vp, _vp, _i32, _i32, _f32, _vp, _vp]),
    "ebh_op_add_layer_norm": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "ebh_op_gemm_add_layer_norm": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _i32,
                                          _f32, _vp]),
    "ebh_op_add_layer_norm_y16": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "ebh_op_add_layer_norm_b16": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "ebh_op_pool": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "ebh_op_pool_b16": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "ebh_op_pack": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ebh_op_embed_ln": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32,
                               _vp, _vp, _vp]),
    "ebh_op_f32_to_bf16": (_i32, [_vp, _vp, _i64, _vp]),
    "ebh_op_widen16": (_i32, [_vp, _vp, _i64, _i32, _vp]),
    "ebh_op_gelu": (_i32, [_vp, _vp, _i64, _vp]),
}

_LIB = None


def header_symbols() -> list:
    """Every function the public headers declare."""
    names = []
    for h in HEADERS:
        with open(h) as f:
            names += re.findall(r"^EBH_API\s+[\w\s\*]+?\b(ebh_\w+)\s*\(", f.read(), flags=re.M)
    return names


def lib():
    """The loaded library (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with "
                               "`python -c 'import __graft_entry__ as g; g.build()'` "
                               "(or `make -C edgebert_amd/csrc`)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def last_error() -> str:
    # messages quote names taken from the caller's files, which may hold any bytes
    return lib().ebh_last_error().decode("utf-8", errors="replace")


def check(rc: int):
    if rc != EBH_OK:
        raise EbhError(rc, last_error())
