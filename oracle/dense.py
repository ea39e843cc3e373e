"""fp64 brute-force dense attention with closed-form gradients (numpy).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

This is the textbook definition the reference's own tests compare against:
``softmax(q k^T * d^-1/2 + mask) v`` (reference_causal_attention,
rust/longctx100m-model/src/ring_attention.rs:237-270 and
src/longctx100m/ring_attention.py:156-173), generalised to

* explicit global positions for queries and keys (the ring's
  ``q_start``/``k_start``, ring_attention.rs:57-106),
* ``valid_length`` (mask = causal ∪ key >= valid_length, rs:79-91),
* GQA: query head h reads KV head h // (Hq // Hkv), the map the callers build
  with repeat_interleave (model.rs:85-94, model.py:250-253); dK/dV of a KV
  head is the sum over its query-head group.

The statistics follow the reference's definitions: m = row max of the masked
scaled scores (natural-log units), l = sum exp(s - m).  A row without any
valid key gives out = 0, m = -inf, l = 0 (the ring's finalize rule
out = acc / max(l, FLT_MIN), rs:227).  Gradients use the closed form
dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dO * O)), dQ = dS K * scale,
dK = dS^T Q * scale.
"""

from __future__ import annotations

import numpy as np


def invalid_mask(tq, tk, *, q_pos0=0, k_pos0=0, causal=True, valid_length=None):
    """Boolean [tq, tk]: True where the (query, key) pair is masked out."""
    qp = q_pos0 + np.arange(tq)[:, None]
    kp = k_pos0 + np.arange(tk)[None, :]
    bad = np.zeros((tq, tk), dtype=bool)
    if causal:
        bad |= kp > qp
    if valid_length is not None:
        bad |= kp >= valid_length
    return bad


def _expand(x, hq):
    hkv = x.shape[2]
    assert hq % hkv == 0
    return np.repeat(x, hq // hkv, axis=2)


def attention_fwd(q, k, v, *, causal=True, valid_length=None, q_pos0=0, k_pos0=0, scale=None):
    """q [B,Tq,Hq,D], k/v [B,Tk,Hkv,D] -> (out [B,Tq,Hq,D], m [B,Hq,Tq], l [B,Hq,Tq]) in fp64."""
    q = np.asarray(q, dtype=np.float64)
    hq = q.shape[2]
    k = _expand(np.asarray(k, dtype=np.float64), hq)
    v = _expand(np.asarray(v, dtype=np.float64), hq)
    d = q.shape[-1]
    scale = d**-0.5 if scale is None else scale
    s = np.einsum("bqhd,bkhd->bhqk", q, k) * scale
    bad = invalid_mask(q.shape[1], k.shape[1], q_pos0=q_pos0, k_pos0=k_pos0, causal=causal,
                       valid_length=valid_length)
    s = np.where(bad[None, None], -np.inf, s)
    m = s.max(axis=-1)
    finite = np.isfinite(m)
    msafe = np.where(finite, m, 0.0)
    p = np.exp(s - msafe[..., None])
    p = np.where(bad[None, None], 0.0, p)
    l = p.sum(axis=-1)
    lsafe = np.where(l > 0, l, 1.0)
    out = np.einsum("bhqk,bkhd->bqhd", p / lsafe[..., None], v)
    return out, m, l


def attention_bwd(q, k, v, dout, *, causal=True, valid_length=None, q_pos0=0, k_pos0=0,
                  out=None, scale=None):
    """Closed-form gradients (dq [B,Tq,Hq,D], dk/dv [B,Tk,Hkv,D]) in fp64.

    ``out`` is the forward output used in delta = rowsum(dO * O); pass the
    output rounded to the input dtype to reproduce the reference's bf16 rule
    (ring_attention.py:314 computes delta from the cast output).
    """
    q = np.asarray(q, dtype=np.float64)
    hq = q.shape[2]
    hkv = np.asarray(k).shape[2]
    ke = _expand(np.asarray(k, dtype=np.float64), hq)
    ve = _expand(np.asarray(v, dtype=np.float64), hq)
    do = np.asarray(dout, dtype=np.float64)
    d = q.shape[-1]
    scale = d**-0.5 if scale is None else scale
    s = np.einsum("bqhd,bkhd->bhqk", q, ke) * scale
    bad = invalid_mask(q.shape[1], ke.shape[1], q_pos0=q_pos0, k_pos0=k_pos0, causal=causal,
                       valid_length=valid_length)
    s = np.where(bad[None, None], -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    msafe = np.where(np.isfinite(m), m, 0.0)
    p = np.where(bad[None, None], 0.0, np.exp(s - msafe))
    l = p.sum(axis=-1, keepdims=True)
    p = p / np.where(l > 0, l, 1.0)
    if out is None:
        out = np.einsum("bhqk,bkhd->bqhd", p, ve)
    o = np.asarray(out, dtype=np.float64)
    delta = np.einsum("bqhd,bqhd->bhq", do, o)[..., None]
    dp = np.einsum("bqhd,bkhd->bhqk", do, ve)
    ds = p * (dp - delta)
    dq = np.einsum("bhqk,bkhd->bqhd", ds, ke) * scale
    dke = np.einsum("bhqk,bqhd->bkhd", ds, q) * scale
    dve = np.einsum("bhqk,bqhd->bkhd", p, do)
    g = hq // hkv
    b, tk = dke.shape[0], dke.shape[1]
    dk = dke.reshape(b, tk, hkv, g, d).sum(axis=3)
    dv = dve.reshape(b, tk, hkv, g, d).sum(axis=3)
    return dq, dk, dv


def ring_rows(qs, ks, vs, rank, *, causal=True, valid_length=None, q_position_start=None):
    """Rank ``rank``'s ring forward expressed densely: its query shard against
    the concatenation of every rank's KV shard (K positions owner*n + j, Q
    positions q_position_start or rank*n)."""
    n = qs[rank].shape[1]
    k = np.concatenate(ks, axis=1)
    v = np.concatenate(vs, axis=1)
    q0 = rank * n if q_position_start is None else q_position_start
    return attention_fwd(qs[rank], k, v, causal=causal, valid_length=valid_length, q_pos0=q0,
                         k_pos0=0)


def lcg_shards(tokens, heads, dim, world):
    """The reference Rust unit tests' deterministic generator
    (ring_attention.rs:490-517), including its quirk: the seed restarts at 42
    on every call, so q, k and v built by separate calls are identical and
    every value lies in [-0.5, 0)."""
    out = []
    seed = 42
    mask = (1 << 64) - 1
    for _ in range(world):
        vals = np.empty(tokens * heads * dim, dtype=np.float32)
        for i in range(vals.size):
            seed = (seed * 6364136223846793005 + 1442695040888963407) & mask
            vals[i] = np.float32(np.float32(seed >> 33) / np.float32(4294967295.0)) - np.float32(0.5)
        out.append(vals.reshape(1, tokens, heads, dim))
    return out
