"""Ring-attention parity driver in the reference's harness format.

    python -m longctx100m_amd.ringcheck <spec.json> [--backward]

Reads the JSON spec of rust/longctx100m-model/src/bin/ringcheck.rs:17-33
(written by scripts/verify_model_parity.py:172-255) and prints the same JSON
line on stdout, computed on the GPU through the C ABI's host-pointer entry
points (lc_ring_fwd_with_stats_host, lc_ring_bwd_host):

* forward:    {"rank": r, "output": [...]}            (ringcheck.rs:80-90)
* --backward: {"rank": r, "dq": [...], "dk": [...], "dv": [...]}  (:36-77)

Spec fields: ``world_size``, ``rank``, ``block_q`` (default 2), ``block_k``
(default 3), ``valid_length`` and ``q_position_start`` (null = None), and
``q``/``k``/``v`` lists of ``{"data": [...], "shape": [B, n, H, D]}`` in rank
order; ``grad_out`` for --backward.  Values are fp32 (ringcheck.rs:94-108);
attention is causal, as the binary hard-wires.  Behaviour kept from the
binary:

* --backward runs the forward with stats for every rank, each with the spec's
  ``q_position_start`` (ringcheck.rs:38-51), and gives the single
  ``grad_out`` to every rank (:56).  The reference backward reads token rows
  [0, local_tokens) of it (candle ``narrow``, ring_attention.rs:380,430), so
  a ``grad_out`` of the full sequence, as the parity script passes
  (verify_model_parity.py:370-372), is accepted and its first shard of rows
  used.
* Floats print as Rust's ``{:?}`` of ``Vec<f32>`` does: shortest round-trip
  digits, decimal for 1e-4 <= |x| < 1e16 (``1.0``, ``-0.25``), otherwise
  exponential (``1e-7``, ``2.5e16``).
* Errors print ``Error: <message>`` on stderr with exit status 1, as a Rust
  ``main`` returning ``Err`` does; validation messages are the reference's
  (ring_attention.rs:148-171).
"""

from __future__ import annotations

import json
import sys
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np

USAGE = "usage: longctx100m-ringcheck <spec.json> [--backward]"


class RingcheckError(Exception):
    """A failure reported as ``Error: <message>``."""


@dataclass
class Spec:
    world: int
    rank: int
    block_q: int
    block_k: int
    valid_length: Optional[int]
    q_position_start: Optional[int]
    q: List[np.ndarray]
    k: List[np.ndarray]
    v: List[np.ndarray]
    grad_out: Optional[np.ndarray]


def tensor_from_json(obj) -> np.ndarray:
    """{"data": flat numbers, "shape": dims} -> fp32 array (ringcheck.rs:94-108)."""
    if not isinstance(obj, dict) or "data" not in obj or "shape" not in obj:
        raise RingcheckError("tensor must be an object with \"data\" and \"shape\"")
    dims = [int(x) for x in obj["shape"]]
    flat = np.asarray(obj["data"], dtype=np.float64).astype(np.float32)
    if flat.size != int(np.prod(dims, dtype=np.int64)):
        raise RingcheckError(f"shape mismatch in reshape, lhs: [{flat.size}], rhs: {dims}")
    return flat.reshape(dims)


def _uint(spec: dict, key: str, default: Optional[int] = None, required: bool = False):
    val = spec.get(key)
    if val is None:
        if required:
            raise RingcheckError(f"spec field \"{key}\" must be a non-negative integer")
        return default
    if isinstance(val, bool) or not isinstance(val, int) or val < 0:
        if required:
            raise RingcheckError(f"spec field \"{key}\" must be a non-negative integer")
        return default  # serde's as_u64() is None for anything else
    return val


def parse_spec(spec: dict, backward: bool) -> Spec:
    world = _uint(spec, "world_size", required=True)
    rank = _uint(spec, "rank", required=True)
    tensors = {}
    for name in ("q", "k", "v"):
        lst = spec.get(name)
        if not isinstance(lst, list) or len(lst) < world:
            raise RingcheckError(f"spec field \"{name}\" must hold one tensor per rank")
        tensors[name] = [tensor_from_json(lst[i]) for i in range(world)]
    grad_out = None
    if backward:
        if "grad_out" not in spec:
            raise RingcheckError("spec field \"grad_out\" is required with --backward")
        grad_out = tensor_from_json(spec["grad_out"])
    return Spec(world, rank, _uint(spec, "block_q", 2), _uint(spec, "block_k", 3),
                _uint(spec, "valid_length"), _uint(spec, "q_position_start"),
                tensors["q"], tensors["k"], tensors["v"], grad_out)


def _desc(spec: Spec, rank: int, q_position_start: Optional[int]):
    from . import _lib

    if not 0 <= rank < spec.world:
        raise RingcheckError(f"rank {rank} out of range for world_size {spec.world}")
    q0 = spec.q[rank]
    if any(x.ndim != 4 for x in (*spec.q, *spec.k, *spec.v)):
        raise RingcheckError("q, k, v must have shape [batch, tokens, heads, head_dim]")
    if any(x.shape != q0.shape for x in (*spec.q, *spec.k, *spec.v)):
        raise RingcheckError("q, k, v shard shapes must match")
    b, n, h, d = q0.shape
    opt = lambda x: -1 if x is None else int(x)  # noqa: E731
    return _lib.RingDesc(spec.world, rank, b, n, h, h, d, _lib.LC_DTYPE_F32, 0, 1,
                         spec.block_q, spec.block_k, opt(spec.valid_length),
                         opt(q_position_start))


def _ptrs(arrays: Sequence[np.ndarray]):
    from . import _lib

    return _lib.ptr_array([a.ctypes.data for a in arrays])


def _check(rc: int) -> None:
    from . import _lib

    if rc != _lib.LC_OK:
        raise RingcheckError(_lib.load().lc_last_error().decode())


def forward_with_stats(spec: Spec, rank: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(out [B,n,H,D], m [B,H,n,1], l [B,H,n,1]) of ``rank`` (fp32)."""
    from . import _lib

    desc = _desc(spec, rank, spec.q_position_start)
    b, n, h, d = spec.q[rank].shape
    out = np.empty((b, n, h, d), np.float32)
    m = np.empty((b, h, n, 1), np.float32)
    l = np.empty((b, h, n, 1), np.float32)
    qs, _a = _ptrs(spec.q)
    ks, _b = _ptrs(spec.k)
    vs, _c = _ptrs(spec.v)
    _check(_lib.load().lc_ring_fwd_with_stats_host(desc, qs, ks, vs, out.ctypes.data,
                                                   m.ctypes.data, l.ctypes.data))
    return out, m, l


def backward(spec: Spec) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(dq, dk, dv) of spec.rank, as ringcheck.rs:36-77 computes them."""
    from . import _lib

    desc = _desc(spec, spec.rank, spec.q_position_start)
    stats = [forward_with_stats(spec, r) for r in range(spec.world)]
    b, n, h, d = spec.q[spec.rank].shape
    g = spec.grad_out
    if g.ndim != 4 or g.shape[0] != b or g.shape[2] != h or g.shape[3] != d or g.shape[1] < n:
        raise RingcheckError(f"grad_out of shape {list(g.shape)} does not cover a "
                             f"[{b}, {n}, {h}, {d}] shard")
    g = np.ascontiguousarray(g[:, :n])  # rows [0, local_tokens), rs:380,430
    outs = [np.ascontiguousarray(s[0]) for s in stats]
    ms = [np.ascontiguousarray(s[1]) for s in stats]
    ls = [np.ascontiguousarray(s[2]) for s in stats]
    dq = np.empty((b, n, h, d), np.float32)
    dk = np.empty_like(dq)
    dv = np.empty_like(dq)
    arrs = [_ptrs(x) for x in (spec.q, spec.k, spec.v, outs, ms, ls, [g] * spec.world)]
    _check(_lib.load().lc_ring_bwd_host(desc, *[a[0] for a in arrs], dq.ctypes.data,
                                        dk.ctypes.data, dv.ctypes.data))
    return dq, dk, dv


def rust_f32_debug(x: float) -> str:
    """One fp32 value as Rust's ``{:?}`` prints it."""
    f = np.float32(x)
    if np.isnan(f):
        return "NaN"
    if np.isinf(f):
        return "inf" if f > 0 else "-inf"
    a = np.abs(f)  # compared in fp32, as Rust's f32 formatter does
    if a == 0 or np.float32(1e-4) <= a < np.float32(1e16):
        return np.format_float_positional(f, unique=True, trim="0")
    return np.format_float_scientific(f, unique=True, trim="-", exp_digits=1).replace("e+", "e")


def _vec(a: np.ndarray) -> str:
    return "[" + ", ".join(rust_f32_debug(x) for x in np.asarray(a, np.float32).ravel()) + "]"


def format_output(rank: int, out: np.ndarray) -> str:
    return f"{{\"rank\": {rank}, \"output\": {_vec(out)}}}"


def format_backward(rank: int, dq: np.ndarray, dk: np.ndarray, dv: np.ndarray) -> str:
    return f"{{\"rank\": {rank}, \"dq\": {_vec(dq)}, \"dk\": {_vec(dk)}, \"dv\": {_vec(dv)}}}"


def run(argv: Sequence[str]) -> str:
    """The line ringcheck prints for ``argv`` (without the program name)."""
    if not argv:
        raise RingcheckError(USAGE)
    path = argv[0]
    mode = argv[1] if len(argv) > 1 else ""
    try:
        with open(path) as f:
            raw = json.load(f)
    except OSError as e:
        raise RingcheckError(f"{e.strerror or e} (os error {e.errno})") from None
    except json.JSONDecodeError as e:
        raise RingcheckError(str(e)) from None
    if not isinstance(raw, dict):
        raise RingcheckError("spec must be a JSON object")
    spec = parse_spec(raw, mode == "--backward")
    if mode == "--backward":
        return format_backward(spec.rank, *backward(spec))
    out, _, _ = forward_with_stats(spec, spec.rank)
    return format_output(spec.rank, out)


def main(argv: Optional[Sequence[str]] = None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    try:
        line = run(argv)
    except RingcheckError as e:
        print(f"Error: {e}", file=sys.stderr, flush=True)
        return 1
    print(line, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
