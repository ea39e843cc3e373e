"""ctypes binding of liblongctx100m_attn.so (include/longctx100m_attn.h and
include/longctx100m_layer.h).

Loading never falls back to anything: if the library is missing the import
of the product path fails with a message naming the build command.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "liblongctx100m_attn.so"

LC_DTYPE_F32 = 0
LC_DTYPE_BF16 = 1
LC_FLAG_PRECISE = 1
LC_FLAG_ACCUMULATE = 2

LC_OK = 0
LC_ERR_INVALID = 1
LC_ERR_HIP = 2
LC_ERR_UNSUPPORTED = 3
LC_ERR_WORKSPACE = 4

LC_DECODE_STATIC_SCRATCH_BYTES = 16 << 20


class Shape(ctypes.Structure):
    _fields_ = [
        ("batch", c_int32),
        ("q_tokens", c_int32),
        ("kv_tokens", c_int32),
        ("heads_q", c_int32),
        ("heads_kv", c_int32),
        ("head_dim", c_int32),
        ("dtype", c_int32),
        ("flags", c_uint32),
    ]


class Mask(ctypes.Structure):
    _fields_ = [
        ("q_pos0", c_int64),
        ("k_pos0", c_int64),
        ("valid_length", c_int64),
        ("causal", c_int32),
        ("reserved", c_int32),
    ]


class RingDesc(ctypes.Structure):
    _fields_ = [
        ("world", c_int32),
        ("rank", c_int32),
        ("batch", c_int32),
        ("local_tokens", c_int32),
        ("heads_q", c_int32),
        ("heads_kv", c_int32),
        ("head_dim", c_int32),
        ("dtype", c_int32),
        ("flags", c_uint32),
        ("causal", c_int32),
        ("block_q", c_int32),
        ("block_k", c_int32),
        ("valid_length", c_int64),
        ("q_position_start", c_int64),
    ]


class Rope(ctypes.Structure):
    _fields_ = [
        ("head_dim", c_int32),
        ("type", c_int32),
        ("theta", ctypes.c_double),
        ("factor", ctypes.c_double),
        ("low_freq_factor", ctypes.c_double),
        ("high_freq_factor", ctypes.c_double),
        ("original_max_position_embeddings", ctypes.c_double),
        ("attention_factor", ctypes.c_double),
    ]


LC_GEMV_IN_BF16, LC_GEMV_IN_F32, LC_GEMV_IN_RMSNORM = 0, 1, 2
LC_GEMV_OUT_PLAIN, LC_GEMV_OUT_SWIGLU, LC_GEMV_OUT_ROPE_QKV = 0, 1, 2


class GemvFused(ctypes.Structure):
    _fields_ = [
        ("in_form", c_int32),
        ("out_form", c_int32),
        ("residual", c_void_p),
        ("residual_out", c_void_p),
        ("norm_weight", c_void_p),
        ("eps", ctypes.c_float),
        ("q_heads", c_int32),
        ("kv_heads", c_int32),
        ("head_dim", c_int32),
        ("rope_row", c_void_p),
        ("k_out", c_void_p),
        ("v_out", c_void_p),
    ]


_vpp = POINTER(c_void_p)
_S, _M, _R = POINTER(Shape), POINTER(Mask), POINTER(RingDesc)

# name -> (restype, argtypes); exactly the entry points the header declares.
SIGNATURES = {
    "lc_attn_fwd_shard": (c_int, [_S, _M, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_void_p]),
    "lc_attn_decode_workspace_bytes": (c_size_t, [_S]),
    "lc_attn_decode": (c_int, [_S, _M, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                               c_void_p, c_void_p, c_size_t, c_void_p]),
    "lc_attn_decode_static": (c_int, [_S, _M, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p]),
    "lc_attn_merge": (c_int, [_S, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                              c_void_p, c_void_p]),
    "lc_attn_init_state": (c_int, [_S, c_void_p, c_void_p, c_void_p, c_void_p]),
    "lc_attn_cast": (c_int, [c_void_p, c_void_p, c_int64, c_int32, c_void_p]),
    "lc_attn_bwd_preprocess": (c_int, [_S, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p]),
    "lc_attn_bwd_shard": (c_int, [_S, _M, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "lc_attn_bwd_shard_workspace_bytes": (c_size_t, [_S]),
    "lc_attn_bwd_shard_ws": (c_int, [_S, _M, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                     c_void_p]),
    "lc_ring_fwd_workspace_bytes": (c_size_t, [_R]),
    "lc_ring_bwd_workspace_bytes": (c_size_t, [_R]),
    "lc_ring_bwd_ds_workspace_bytes": (c_size_t, [_R]),
    "lc_ring_fwd_with_stats": (c_int, [_R, _vpp, _vpp, _vpp, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_size_t, c_void_p]),
    "lc_ring_bwd": (c_int, [_R, _vpp, _vpp, _vpp, _vpp, _vpp, _vpp, _vpp, c_void_p, c_void_p,
                            c_void_p, c_void_p, c_size_t, c_void_p]),
    "lc_ring_fwd_with_stats_host": (c_int, [_R, _vpp, _vpp, _vpp, c_void_p, c_void_p,
                                            c_void_p]),
    "lc_ring_bwd_host": (c_int, [_R, _vpp, _vpp, _vpp, _vpp, _vpp, _vpp, _vpp, c_void_p,
                                 c_void_p, c_void_p]),
    "lc_reference_causal_attention_host": (c_int, [c_int32, c_int32, c_int32, c_int32, c_int32,
                                                   c_int32, c_void_p, c_void_p, c_void_p,
                                                   c_int32, c_int64, c_void_p]),
    "lc_rmsnorm": (c_int, [c_int32, c_int64, c_int32, ctypes.c_float, c_void_p, c_int64, c_void_p,
                           c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p]),
    "lc_rope_inv_freq": (c_int, [POINTER(Rope), c_void_p, c_void_p]),
    "lc_rope_table": (c_int, [POINTER(Rope), c_int64, c_int64, c_void_p, c_void_p]),
    "lc_rope_apply": (c_int, [c_int32, c_int64, c_int32, c_int32, c_void_p, c_void_p, c_int64,
                              c_void_p, c_void_p]),
    "lc_swiglu": (c_int, [c_int32, c_int64, c_int32, c_void_p, c_int64, c_void_p, c_int64,
                          c_void_p, c_void_p]),
    "lc_gemv": (c_int, [c_int32, c_int64, c_int32, c_void_p, c_int64, c_void_p, c_void_p,
                        c_void_p]),
    "lc_gemv_fused": (c_int, [POINTER(GemvFused), c_int64, c_int32, c_void_p, c_int64, c_void_p,
                              c_void_p, c_void_p]),
    "lc_last_error": (ctypes.c_char_p, []),
    "lc_abi_version": (c_int32, []),
}

_lib = None


class LcError(RuntimeError):
    """A nonzero status from the library; ``code`` is the LC_ERR_* value."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class LcValueError(LcError, ValueError):
    """LC_ERR_INVALID: the reference raises ValueError / bails for these."""


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m longctx100m_amd.build` (hipcc, gfx950)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != LC_OK:
        msg = load().lc_last_error().decode()
        if rc == LC_ERR_INVALID:
            raise LcValueError(rc, msg)
        raise LcError(rc, msg)


def ptr_array(ptrs):
    arr = (c_void_p * len(ptrs))(*ptrs)
    return ctypes.cast(arr, _vpp), arr
