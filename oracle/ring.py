"""ctypes bindings to the C restatement of the reference ring attention.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Mirrors the reference's
public functions (rust/longctx100m-model/src/lib.rs:16-19):

* ring_fwd_with_stats  <- ring_causal_attention_forward_with_stats (rs:139-233)
* ring_bwd             <- ring_causal_attention_backward           (rs:281-475)
* dense                <- reference_causal_attention               (rs:237-270)

Inputs are numpy arrays in the reference layout [B, n, H, D]; they are
converted to fp32 first, which is the Python twin's bf16 rule (upcast before
every matmul, ring_attention.py:17,28).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "lib" / "libring_ref.so"
_lib = None


class OracleError(RuntimeError):
    pass


def build() -> Path:
    """Compile ring_ref.c (make in oracle/)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        fp = ctypes.POINTER(ctypes.c_void_p)
        i, ll = ctypes.c_int, ctypes.c_longlong
        vp = ctypes.c_void_p
        lib.ref_ring_fwd_with_stats.argtypes = [i, i, i, i, i, i, fp, fp, fp, i, i, i, ll, ll, vp,
                                                vp, vp]
        lib.ref_ring_fwd_with_stats.restype = i
        lib.ref_ring_bwd.argtypes = [i, i, i, i, i, i, fp, fp, fp, fp, fp, fp, fp, i, i, i, ll,
                                     ll, vp, vp, vp]
        lib.ref_ring_bwd.restype = i
        lib.ref_dense_attention.argtypes = [i, i, i, i, vp, vp, vp, i, ll, vp]
        lib.ref_dense_attention.restype = i
        lib.ref_last_error.restype = ctypes.c_char_p
        lib.ref_num_threads.restype = i
        _lib = lib
    return _lib


def _f32(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _ptrs(arrs):
    arr = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    return ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p))


def _opt(x):
    return -1 if x is None else int(x)


def _check(rc):
    if rc != 0:
        raise OracleError(_load().ref_last_error().decode())


def num_threads() -> int:
    return int(_load().ref_num_threads())


def ring_fwd_with_stats(qs, ks, vs, rank, *, causal=True, block_q=64, block_k=128,
                        valid_length=None, q_position_start=None):
    """Returns (out [B,n,H,D], m [B,H,n], l [B,H,n]) as fp32 numpy arrays."""
    lib = _load()
    qs, ks, vs = [_f32(x) for x in qs], [_f32(x) for x in ks], [_f32(x) for x in vs]
    world = len(qs)
    b, n, h, d = qs[0].shape if qs[0].ndim == 4 else (0, 0, 0, 0)
    out = np.zeros((b, n, h, d), np.float32)
    m = np.zeros((b, h, n), np.float32)
    l = np.zeros((b, h, n), np.float32)
    _check(lib.ref_ring_fwd_with_stats(world, rank, b, n, h, d, _ptrs(qs), _ptrs(ks), _ptrs(vs),
                                       int(causal), block_q, block_k, _opt(valid_length),
                                       _opt(q_position_start), out.ctypes.data, m.ctypes.data,
                                       l.ctypes.data))
    return out, m, l


def ring_bwd(qs, ks, vs, outs, ms, ls, grad_outs, rank, *, causal=True, block_q=64, block_k=128,
             valid_length=None, q_position_start=None):
    """Returns (dq, dk, dv) of rank ``rank``'s shard as fp32 numpy arrays."""
    lib = _load()
    conv = lambda xs: [_f32(x) for x in xs]  # noqa: E731
    qs, ks, vs, outs, ms, ls, grad_outs = map(conv, (qs, ks, vs, outs, ms, ls, grad_outs))
    world = len(qs)
    b, n, h, d = qs[0].shape
    dq = np.zeros((b, n, h, d), np.float32)
    dk = np.zeros_like(dq)
    dv = np.zeros_like(dq)
    _check(lib.ref_ring_bwd(world, rank, b, n, h, d, _ptrs(qs), _ptrs(ks), _ptrs(vs), _ptrs(outs),
                            _ptrs(ms), _ptrs(ls), _ptrs(grad_outs), int(causal), block_q, block_k,
                            _opt(valid_length), _opt(q_position_start), dq.ctypes.data,
                            dk.ctypes.data, dv.ctypes.data))
    return dq, dk, dv


def dense(q, k, v, *, causal=True, valid_length=None):
    """reference_causal_attention in fp32 ([B,T,H,D])."""
    lib = _load()
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, t, h, d = q.shape
    out = np.zeros_like(q)
    _check(lib.ref_dense_attention(b, t, h, d, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                   int(causal), _opt(valid_length), out.ctypes.data))
    return out

