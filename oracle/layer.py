"""numpy restatements of the decoder-layer row ops around attention.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

* ``rmsnorm`` -- RmsNorm::forward, rust/longctx100m-model/src/model.rs:53-62
  (src/longctx100m/model.py:114-118), with the decoder's residual add
  (model.rs:387-393) optionally in front.
* ``rope_inv_freq`` / ``rope_table`` / ``rope_apply`` -- apply_rope,
  rust/longctx100m-model/src/rope.rs:10-127, step for step in float32 (candle's
  affine(mul, add) on an fp32 tensor is x * float32(mul) + float32(add)).
* ``swiglu`` -- SwiGlu::forward's gate, model.rs:323-327.

Every float32 operation is a separate numpy float32 op (one rounding each, no
fused multiply-add), which is how the reference's tensor ops round; exp, cos
and sin are evaluated in float64 and rounded once to float32 (the correctly
rounded value the reference's libm returns within its 0.5-ulp-class error).
bf16 results use round-to-nearest-even (``bf16``).
"""

from __future__ import annotations

import math

import numpy as np

F32 = np.float32


def bf16(x):
    """Round float32 values to bfloat16 (nearest even), returned as float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=F32))
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(F32).reshape(a.shape)
    return np.where(np.isnan(a), a, out)


def _f32(fn, x):
    """fn evaluated in float64 on float32 arguments, rounded once to float32."""
    with np.errstate(over="ignore"):
        return fn(np.asarray(x, dtype=F32).astype(np.float64)).astype(F32)


def _rnd(x, dtype):
    return bf16(x) if dtype == "bf16" else np.asarray(x, dtype=F32)


def rmsnorm(x, weight, eps, *, residual=None, dtype="bf16"):
    """(out, h): h = x (+ residual, rounded), out = dtype(dtype(h * inv) * weight)
    with inv = 1 / sqrt(mean(h^2) + eps) (mean taken in float64 here; the
    reference sums in fp32, a rounding-order difference only)."""
    h = np.asarray(x, dtype=F32)
    if residual is not None:
        h = _rnd(h + np.asarray(residual, dtype=F32), dtype)
    ms = (h.astype(np.float64) ** 2).mean(-1, keepdims=True).astype(F32)
    inv = F32(1) / np.sqrt(ms + F32(eps))
    normed = _rnd(h * inv, dtype)
    return _rnd(normed * np.asarray(weight, dtype=F32), dtype), h


ROPE_TYPES = {"default": 0, "linear": 1, "llama3": 2}


def rope_inv_freq(head_dim, theta, *, rope_type="default", factor=1.0, low_freq_factor=None,
                  high_freq_factor=None, original_max_position_embeddings=None,
                  attention_factor=1.0):
    """(inv [head_dim/2] float32, cos_factor, position scale) of rope.rs:15-99."""
    half = head_dim // 2
    mul = F32(-2.0 * math.log(theta) / head_dim)
    inv = _f32(np.exp, np.arange(half, dtype=F32) * mul + F32(0))
    cos_factor, pos_scale = F32(1), None
    if rope_type == "linear":
        if factor <= 0:
            raise ValueError("rope scaling factor must be positive")
        pos_scale = F32(1.0 / factor)
    elif rope_type == "llama3":
        low, high, orig = low_freq_factor, high_freq_factor, original_max_position_embeddings
        if low is None or high is None or orig is None:
            raise ValueError("llama3 RoPE needs low/high frequency factors and original context length")
        if low <= 0 or high <= low or orig <= 0:
            raise ValueError("invalid llama3 RoPE scaling values")
        if attention_factor <= 0:
            raise ValueError("llama3 attention_factor must be positive")
        # rope.rs:70 computes inv.affine(2*pi, 0).div(&inv) (not 2*pi / inv)
        wavelength = (inv * F32(2.0 * math.pi) + F32(0)) / inv
        low_wl, high_wl = F32(orig / low), F32(orig / high)
        scaled = inv * F32(1.0 / factor) + F32(0)
        smooth = (F32(1) / wavelength) * F32(orig / (high - low)) + F32(-(low / (high - low)))
        mid = (smooth * F32(-1) + F32(1)) * scaled + smooth * inv
        inv = np.where(wavelength > low_wl, scaled, inv)
        inv = np.where((wavelength >= high_wl) & (wavelength <= low_wl), mid, inv)
        cos_factor = F32(attention_factor)
    elif rope_type != "default":
        raise ValueError(f"unsupported RoPE type {rope_type!r}")
    return inv.astype(F32), cos_factor, pos_scale


def rope_table(inv, cos_factor, pos_scale, tokens, pos0):
    """[tokens, 2, half] float32: cos(f) * cos_factor, sin(f); f = position * inv
    with the position converted to float32 (and scaled for the linear profile)."""
    pos = (np.arange(tokens, dtype=np.int64) + pos0).astype(F32)
    if pos_scale is not None:
        pos = pos * F32(pos_scale)
    f = pos[:, None] * inv[None, :]
    return np.stack([_f32(np.cos, f) * F32(cos_factor), _f32(np.sin, f)], axis=1).astype(F32)


def rope_apply(x, table, *, dtype="bf16"):
    """x [T, H, D] -> rotate-half RoPE with the table's rows (rope.rs:116-127)."""
    x = np.asarray(x, dtype=F32)
    half = x.shape[-1] // 2
    c = table[:, 0, None, :]
    s = table[:, 1, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    o1 = x1 * c - x2 * s
    o2 = x2 * c + x1 * s
    return _rnd(np.concatenate([o1, o2], axis=-1), dtype)


def swiglu(gate, up, *, dtype="bf16"):
    """dtype(dtype(silu(gate)) * up), silu(g) = g / (1 + exp(-g)) in float32."""
    g = np.asarray(gate, dtype=F32)
    with np.errstate(over="ignore"):
        sl = _rnd(g / (F32(1) + _f32(np.exp, -g)), dtype)
    return _rnd(sl * np.asarray(up, dtype=F32), dtype)
