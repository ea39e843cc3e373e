"""Torch-facing mirror of the reference's ring-attention API, on MI355X.

Function names, argument meaning and error behaviour follow the reference's
Rust module (rust/longctx100m-model/src/ring_attention.rs, re-exported at
lib.rs:16-19):

* ring_causal_attention_forward            rs:116-135
* ring_causal_attention_forward_with_stats rs:139-233
* ring_causal_attention_backward           rs:281-475
* reference_causal_attention               rs:237-270

and the Python module's process-group entry (src/longctx100m/ring_attention.py):

* ring_causal_attention(q, k, v, *, group, ...)  py:176-191, with the autograd
  of _RingCausalAttention (py:194-255): what model.py:254-265 calls

``shards`` is every rank's (q, k, v) triple in rank order, each a contiguous
``[B, local_tokens, H, D]`` tensor on the GPU; the ring is emulated on one GPU
as an ordered loop over the KV shards held in HBM.  Unlike the reference,
K/V may carry fewer heads than Q (GQA, query head h reads KV head
h // (Hq // Hkv)); the reference's callers expand with repeat_interleave
instead (model.rs:85-94).

The per-hop building blocks (``fwd_shard``, ``merge``, ``bwd_preprocess``,
``bwd_shard``) expose the C ABI one kernel step at a time, the shape a real
xGMI ring drives them in.  Everything runs through liblongctx100m_attn.so;
there is no CPU or PyTorch fallback.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.LC_DTYPE_F32, torch.bfloat16: _lib.LC_DTYPE_BF16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16") from None


def _check_dev(*ts: torch.Tensor) -> None:
    for t in ts:
        if not isinstance(t, torch.Tensor):
            raise TypeError("expected torch tensors")
        if not t.is_cuda:
            raise ValueError("tensors must live on the GPU (device pointers are passed to HIP)")
        if not t.is_contiguous():
            raise ValueError("tensors must be contiguous")


def _check_buf(t: Optional[torch.Tensor], shape, name: str, dtype=torch.float32) -> None:
    """A caller-supplied output or state buffer must have exactly the shape and
    dtype the kernels index (they take raw device pointers)."""
    if t is None:
        return
    _check_dev(t)
    if tuple(t.shape) != tuple(shape) or t.dtype != dtype:
        raise ValueError(f"{name} must be a {dtype} tensor of shape {tuple(shape)}, "
                         f"got {t.dtype} {tuple(t.shape)}")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _opt(x: Optional[int]) -> int:
    return -1 if x is None else int(x)


def _shape(q: torch.Tensor, k: torch.Tensor, precise: bool) -> _lib.Shape:
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError("q, k, v must have shape [batch, tokens, heads, head_dim]")
    b, nq, hq, d = q.shape
    bk, nk, hkv, dk = k.shape
    if b != bk or d != dk:
        raise ValueError("q, k, v shard shapes must match")
    flags = _lib.LC_FLAG_PRECISE if precise else 0
    return _lib.Shape(b, nq, nk, hq, hkv, d, _dtype_code(q), flags)


# ---------------------------------------------------------------- per hop ----

def fwd_shard(q, k, v, *, q_pos0: int, k_pos0: int, causal: bool = True,
              valid_length: Optional[int] = None, precise: bool = False,
              o: Optional[torch.Tensor] = None, m: Optional[torch.Tensor] = None,
              l: Optional[torch.Tensor] = None, accumulate: bool = False):
    """One hop: attention of the query shard over one KV shard.

    Returns (o [B,Nq,Hq,D] fp32 normalised, m [B,Hq,Nq], l [B,Hq,Nq]).  With
    ``accumulate`` the given o, m, l hold a running state and the hop's result
    is LSE-merged into them in the kernel's epilogue (as :func:`merge` would
    merge a separate partial), the reference's state carried over the hop loop
    (rs:195-225)."""
    _check_dev(q, k, v)
    if k.shape != v.shape or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v shard shapes must match")
    if accumulate and (o is None or m is None or l is None):
        raise ValueError("accumulate needs the running o, m and l")
    s = _shape(q, k, precise)
    if accumulate:
        s.flags |= _lib.LC_FLAG_ACCUMULATE
    b, nq, hq, d = q.shape
    _check_buf(o, (b, nq, hq, d), "o")
    _check_buf(m, (b, hq, nq), "m")
    _check_buf(l, (b, hq, nq), "l")
    o = torch.empty((b, nq, hq, d), dtype=torch.float32, device=q.device) if o is None else o
    m = torch.empty((b, hq, nq), dtype=torch.float32, device=q.device) if m is None else m
    l = torch.empty((b, hq, nq), dtype=torch.float32, device=q.device) if l is None else l
    mk = _lib.Mask(q_pos0, k_pos0, _opt(valid_length), int(causal), 0)
    _lib.check(_lib.load().lc_attn_fwd_shard(s, mk, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                             o.data_ptr(), m.data_ptr(), l.data_ptr(), _stream()))
    return o, m, l


def decode(q, k, v, *, q_pos0: int, k_pos0: int = 0, causal: bool = True,
           valid_length: Optional[int] = None, o: Optional[torch.Tensor] = None,
           m: Optional[torch.Tensor] = None, l: Optional[torch.Tensor] = None,
           workspace: Optional[torch.Tensor] = None):
    """Split-KV decode of a few query tokens against a long KV shard (a KV
    cache): same outputs as fwd_shard, (o [B,Nq,Hq,D] fp32, m, l [B,Hq,Nq])."""
    _check_dev(q, k, v)
    s = _shape(q, k, False)
    mk = _lib.Mask(q_pos0, k_pos0, _opt(valid_length), int(causal), 0)
    b, nq, hq, d = q.shape
    _check_buf(o, (b, nq, hq, d), "o")
    _check_buf(m, (b, hq, nq), "m")
    _check_buf(l, (b, hq, nq), "l")
    o = torch.empty((b, nq, hq, d), dtype=torch.float32, device=q.device) if o is None else o
    m = torch.empty((b, hq, nq), dtype=torch.float32, device=q.device) if m is None else m
    l = torch.empty_like(m) if l is None else l
    lib = _lib.load()
    need = lib.lc_attn_decode_workspace_bytes(ctypes.byref(s))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    _lib.check(lib.lc_attn_decode(ctypes.byref(s), ctypes.byref(mk), q.data_ptr(), k.data_ptr(),
                                  v.data_ptr(), o.data_ptr(), m.data_ptr(), l.data_ptr(),
                                  workspace.data_ptr(), workspace.numel(), _stream()))
    return o, m, l


def merge(o_run, m_run, l_run, o_part, m_part, l_part, out: Optional[torch.Tensor] = None):
    """In-place LSE merge of a hop's partial into the running state; optionally
    also writes the merged output cast to ``out``'s dtype."""
    _check_dev(o_run, m_run, l_run, o_part, m_part, l_part)
    b, nq, hq, d = o_run.shape
    _check_buf(o_run, (b, nq, hq, d), "o_run")
    _check_buf(o_part, (b, nq, hq, d), "o_part")
    for name, t in (("m_run", m_run), ("l_run", l_run), ("m_part", m_part), ("l_part", l_part)):
        _check_buf(t, (b, hq, nq), name)
    if out is not None:
        _check_buf(out, (b, nq, hq, d), "out", out.dtype)
    dt = _lib.LC_DTYPE_F32 if out is None else _dtype_code(out)
    s = _lib.Shape(b, nq, nq, hq, hq, d, dt, 0)
    _lib.check(_lib.load().lc_attn_merge(s, o_run.data_ptr(), m_run.data_ptr(), l_run.data_ptr(),
                                         o_part.data_ptr(), m_part.data_ptr(), l_part.data_ptr(),
                                         None if out is None else out.data_ptr(), _stream()))


def cast(src: torch.Tensor, dst: torch.Tensor) -> torch.Tensor:
    _check_dev(src, dst)
    if src.dtype != torch.float32 or src.numel() != dst.numel():
        raise ValueError("cast takes an fp32 source of the destination's size")
    _lib.check(_lib.load().lc_attn_cast(src.data_ptr(), dst.data_ptr(), src.numel(),
                                        _dtype_code(dst), _stream()))
    return dst


def bwd_preprocess(out, dout, m, l, delta=None, lse2=None):
    """delta = rowsum(dout * out), lse2 = m*log2(e) + log2(max(l, FLT_MIN))."""
    _check_dev(out, dout, m, l)
    b, nq, hq, d = out.shape
    _check_buf(dout, (b, nq, hq, d), "dout", out.dtype)
    for name, t in (("m", m), ("l", l), ("delta", delta), ("lse2", lse2)):
        _check_buf(t, (b, hq, nq), name)
    delta = torch.empty((b, hq, nq), dtype=torch.float32, device=out.device) if delta is None else delta
    lse2 = torch.empty_like(delta) if lse2 is None else lse2
    s = _lib.Shape(b, nq, nq, hq, hq, d, _dtype_code(out), 0)
    _lib.check(_lib.load().lc_attn_bwd_preprocess(s, out.data_ptr(), dout.data_ptr(),
                                                  m.data_ptr(), l.data_ptr(), delta.data_ptr(),
                                                  lse2.data_ptr(), _stream()))
    return delta, lse2


def bwd_shard(q, k, v, dout, lse2, delta, *, q_pos0: int, k_pos0: int, causal: bool = True,
              valid_length: Optional[int] = None, dq_acc=None, dk_acc=None, dv_acc=None,
              precise: bool = False, workspace=None):
    """One hop of the backward; adds into the fp32 accumulators given.

    With ``workspace`` (a CUDA tensor, see :func:`bwd_shard_workspace_bytes`)
    and all three accumulators, the dK/dV kernel stores dS there and dQ is
    computed from it instead of recomputing the scores."""
    _check_dev(q, k, v, dout, lse2, delta)
    s = _shape(q, k, precise)
    b, nq, hq, d = q.shape
    nk, hkv = k.shape[1], k.shape[2]
    _check_buf(dout, (b, nq, hq, d), "dout", q.dtype)
    _check_buf(lse2, (b, hq, nq), "lse2")
    _check_buf(delta, (b, hq, nq), "delta")
    _check_buf(dq_acc, (b, nq, hq, d), "dq_acc")
    _check_buf(dk_acc, (b, nk, hkv, d), "dk_acc")
    _check_buf(dv_acc, (b, nk, hkv, d), "dv_acc")
    mk = _lib.Mask(q_pos0, k_pos0, _opt(valid_length), int(causal), 0)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    args = (s, mk, q.data_ptr(), k.data_ptr(), v.data_ptr(), dout.data_ptr(), lse2.data_ptr(),
            delta.data_ptr(), ptr(dq_acc), ptr(dk_acc), ptr(dv_acc))
    if workspace is None:
        _lib.check(_lib.load().lc_attn_bwd_shard(*args, _stream()))
    else:
        _check_dev(workspace)
        nbytes = workspace.numel() * workspace.element_size()
        _lib.check(_lib.load().lc_attn_bwd_shard_ws(*args, workspace.data_ptr(), nbytes,
                                                    _stream()))


def bwd_shard_workspace_bytes(q, k, precise: bool = False) -> int:
    """Workspace bytes for :func:`bwd_shard` to share dS between its kernels
    (0 when the shape does not take that path)."""
    return int(_lib.load().lc_attn_bwd_shard_workspace_bytes(_shape(q, k, precise)))


# ------------------------------------------------------- reference signatures --

def _ring_desc(shards, rank, causal, block_q, block_k, valid_length, q_position_start, precise):
    world = len(shards)
    if world == 0:
        raise ValueError(f"rank {rank} out of range for world_size {world}")
    q, k, v = shards[0]
    for (qq, kk, vv) in shards:
        _check_dev(qq, kk, vv)
        if qq.ndim != 4 or kk.ndim != 4 or vv.ndim != 4:
            raise ValueError("q, k, v must have shape [batch, tokens, heads, head_dim]")
        if (qq.shape != q.shape or kk.shape != k.shape or vv.shape != k.shape
                or qq.dtype != q.dtype or kk.dtype != q.dtype or vv.dtype != q.dtype):
            raise ValueError("q, k, v shard shapes must match")
    b, n, hq, d = q.shape
    if k.shape[0] != b or k.shape[1] != n or k.shape[3] != d:
        raise ValueError("q, k, v shard shapes must match")
    flags = _lib.LC_FLAG_PRECISE if precise else 0
    return _lib.RingDesc(world, rank, b, n, hq, k.shape[2], d, _dtype_code(q), flags,
                         int(causal), block_q, block_k, _opt(valid_length),
                         _opt(q_position_start))


def ring_causal_attention_forward_with_stats(
        shards: Sequence[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]], rank: int,
        causal: bool = True, block_q: int = 64, block_k: int = 128,
        valid_length: Optional[int] = None, q_position_start: Optional[int] = None,
        *, precise: bool = False):
    """(out [B,n,Hq,D] in the input dtype, m [B,Hq,n,1] fp32, l [B,Hq,n,1] fp32)."""
    desc = _ring_desc(shards, rank, causal, block_q, block_k, valid_length, q_position_start,
                      precise)
    if not 0 <= rank < len(shards):
        raise ValueError(f"rank {rank} out of range for world_size {len(shards)}")
    lib = _lib.load()
    q = shards[rank][0]
    b, n, hq, d = q.shape
    out = torch.empty_like(q)
    m = torch.empty((b, hq, n, 1), dtype=torch.float32, device=q.device)
    l = torch.empty_like(m)
    ws_bytes = lib.lc_ring_fwd_workspace_bytes(desc)
    if ws_bytes == 0:
        _lib.check(lib.lc_ring_fwd_with_stats(desc, None, None, None, None, None, None, None, 0,
                                              None))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    qs, _a = _lib.ptr_array([s[0].data_ptr() for s in shards])
    ks, _b = _lib.ptr_array([s[1].data_ptr() for s in shards])
    vs, _c = _lib.ptr_array([s[2].data_ptr() for s in shards])
    _lib.check(lib.lc_ring_fwd_with_stats(desc, qs, ks, vs, out.data_ptr(), m.data_ptr(),
                                          l.data_ptr(), ws.data_ptr(), ws_bytes, _stream()))
    return out, m, l


def ring_causal_attention_forward(shards, rank, causal=True, block_q=64, block_k=128,
                                  valid_length=None, q_position_start=None, *, precise=False):
    out, _, _ = ring_causal_attention_forward_with_stats(
        shards, rank, causal, block_q, block_k, valid_length, q_position_start, precise=precise)
    return out


def ring_causal_attention_backward(shards, rank, outs, ms, ls, grad_outs, causal=True,
                                   block_q=64, block_k=128, valid_length=None,
                                   q_position_start=None, *, precise=False, share_ds=True):
    """(dq [B,n,Hq,D], dk [B,n,Hkv,D], dv [B,n,Hkv,D]) of rank ``rank``'s shard.

    ``share_ds``: give lc_ring_bwd the workspace of lc_ring_bwd_ds_workspace_bytes,
    so that the diagonal pair (hop 0 of both passes; the whole backward at
    world 1) runs its dK/dV and dQ kernels on one shared dS instead of
    recomputing the scores twice."""
    desc = _ring_desc(shards, rank, causal, block_q, block_k, valid_length, q_position_start,
                      precise)
    world = len(shards)
    if not 0 <= rank < world:
        raise ValueError(f"rank {rank} out of range for world_size {world}")
    if not (len(outs) == len(ms) == len(ls) == len(grad_outs) == world):
        raise ValueError("outs, ms, ls and grad_outs must hold one tensor per rank")
    q, k, _ = shards[rank]
    for t in (*outs, *grad_outs):
        _check_dev(t)
        if t.shape != q.shape or t.dtype != q.dtype:
            raise ValueError("outs and grad_outs must match the query shard")
    ms = [x.float().contiguous() for x in ms]
    ls = [x.float().contiguous() for x in ls]
    lib = _lib.load()
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(k)
    ws_bytes = (lib.lc_ring_bwd_ds_workspace_bytes(desc) if share_ds
                else lib.lc_ring_bwd_workspace_bytes(desc))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    arrs = [_lib.ptr_array([t.data_ptr() for t in ts]) for ts in
            ([s[0] for s in shards], [s[1] for s in shards], [s[2] for s in shards], outs, ms,
             ls, grad_outs)]
    _lib.check(lib.lc_ring_bwd(desc, *[a[0] for a in arrs], dq.data_ptr(), dk.data_ptr(),
                               dv.data_ptr(), ws.data_ptr(), ws_bytes, _stream()))
    return dq, dk, dv


def reference_causal_attention(q, k, v, causal: bool = True,
                               valid_length: Optional[int] = None, *, precise: bool = False):
    """Dense attention of one [B,T,H,D] sequence (a one-rank ring)."""
    return ring_causal_attention_forward([(q, k, v)], 0, causal, 64, 128, valid_length, None,
                                         precise=precise)


def local_decode_backward(q, k, v, out, m, l, grad_out, *, causal: bool = True,
                          q_position_start: int = 0, valid_length: Optional[int] = None,
                          precise: bool = False):
    """Single-rank backward with query positions from ``q_position_start`` and
    key positions from 0 (_local_decode_backward,
    src/longctx100m/ring_attention.py:258-287, taken by the autograd backward
    when q_position_start is set and the group has one rank, :226-239).

    The reference recomputes the probabilities with a dense softmax; here P
    comes from the forward's (m, l), which hold the same row statistics for
    the same positions.  delta uses ``out`` as given (the cast output, :314).
    Returns (dq, dk, dv) in the dtypes of q, k, v."""
    if q_position_start is None or q_position_start < 0:
        raise ValueError("q_position_start must be a non-negative position")
    _check_dev(q, k, v, out, grad_out)
    b, n, hq, _ = q.shape
    mm = m.reshape(b, hq, n).float().contiguous()
    ll = l.reshape(b, hq, n).float().contiguous()
    delta, lse2 = bwd_preprocess(out.contiguous(), grad_out.contiguous(), mm, ll)
    dq = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
    dk = torch.zeros(k.shape, dtype=torch.float32, device=q.device)
    dv = torch.zeros(k.shape, dtype=torch.float32, device=q.device)
    bwd_shard(q, k, v, grad_out.contiguous(), lse2, delta, q_pos0=int(q_position_start),
              k_pos0=0, causal=causal, valid_length=valid_length, dq_acc=dq, dk_acc=dk,
              dv_acc=dv, precise=precise)
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


class RingCausalAttention(torch.autograd.Function):
    """Autograd wrapper of one rank's share, mirroring _RingCausalAttention
    (src/longctx100m/ring_attention.py:194-255) with the in-process ring: the
    forward saves (out, m, l) and the backward recomputes P from them.

    Gradients flow to this rank's q, k and v; the other ranks' shards are
    treated as constants (their owners differentiate their own shares).
    ``q_position_start`` applies to this rank's queries; with one rank the
    backward takes the reference's decode path (local_decode_backward)."""

    @staticmethod
    def forward(ctx, q, k, v, shards, rank, causal, valid_length, q_position_start=None):
        shards = list(shards)
        shards[rank] = (q.detach(), k.detach(), v.detach())
        outs, ms, ls = [], [], []
        for r in range(len(shards)):
            qps = q_position_start if r == rank else None
            o, m, l = ring_causal_attention_forward_with_stats(shards, r, causal, 64, 128,
                                                               valid_length, qps)
            outs.append(o)
            ms.append(m)
            ls.append(l)
        ctx.shards, ctx.rank, ctx.causal, ctx.valid_length = shards, rank, causal, valid_length
        ctx.q_position_start = q_position_start
        ctx.outs, ctx.ms, ctx.ls = outs, ms, ls
        return outs[rank]

    @staticmethod
    def backward(ctx, grad_out):
        if ctx.q_position_start is not None and len(ctx.shards) == 1:
            q, k, v = ctx.shards[0]
            dq, dk, dv = local_decode_backward(
                q, k, v, ctx.outs[0], ctx.ms[0], ctx.ls[0], grad_out.contiguous(),
                causal=ctx.causal, q_position_start=ctx.q_position_start,
                valid_length=ctx.valid_length)
            return dq, dk, dv, None, None, None, None, None
        grad_outs = [torch.zeros_like(o) for o in ctx.outs]
        grad_outs[ctx.rank] = grad_out.contiguous()
        dq, dk, dv = ring_causal_attention_backward(ctx.shards, ctx.rank, ctx.outs, ctx.ms,
                                                    ctx.ls, grad_outs, ctx.causal, 64, 128,
                                                    ctx.valid_length, ctx.q_position_start)
        return dq, dk, dv, None, None, None, None, None


# ------------------------------------------------- the Python module's entry --

def ring_causal_attention(q, k, v, *, group=None, causal=True, block_q=64, block_k=128,
                          valid_length=None, q_position_start=None):
    """Exact ring attention over a torch.distributed process group with the
    activation-recomputing backward: the signature of
    ring_causal_attention (src/longctx100m/ring_attention.py:176-191), which
    model.py:254-265 calls with this rank's [B, local_tokens, H, D] shards.

    Each rank gathers the group's K and V shards once (one all_gather each;
    the reference rotates them hop by hop) and runs the ring over them in HBM.
    The backward gathers Q, dO, O, m and l the same way for the reference's
    pass 1 (each rank differentiates its own K/V against every query owner)
    and returns this rank's (dq, dk, dv).  With one rank and
    ``q_position_start`` set, the backward takes the reference's decode path
    (py:226-239).  Tensors must be on the GPU (the kernels have no CPU form),
    with an NCCL (RCCL) group as the reference requires for CUDA tensors."""
    return _GroupRingAttention.apply(q, k, v, group, causal, block_q, block_k, valid_length,
                                     q_position_start)


def _group_checks(q, k, v, group, block_q, block_k, valid_length):
    """The reference's argument checks (py:78-101), in its order and texts."""
    import torch.distributed as dist

    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, v must have shape [batch, tokens, heads, head_dim]")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, v shard shapes must match")
    if block_q <= 0 or block_k <= 0:
        raise ValueError("block_q and block_k must be positive")
    if q.device.type != "cuda":
        raise ValueError("ring attention on this backend requires CUDA (HIP) tensors")
    if not dist.is_available() or not dist.is_initialized():
        raise RuntimeError("torch.distributed must be initialized")
    if not str(dist.get_backend(group)).lower().endswith("nccl"):
        raise RuntimeError("CUDA ring attention requires an NCCL process group")
    world, rank = dist.get_world_size(group), dist.get_rank(group)
    if world < 1:
        raise RuntimeError("invalid distributed group")
    if q.shape[1] == 0:
        raise ValueError("local_tokens must be positive")
    if valid_length is not None and not 0 < valid_length <= world * q.shape[1]:
        raise ValueError("valid_length must be within the padded distributed sequence")
    return world, rank


def _gather(x, world, group):
    """Every rank's copy of x, in rank order (one all_gather)."""
    import torch.distributed as dist

    x = x.contiguous()
    if world == 1:
        return [x]
    out = [torch.empty_like(x) for _ in range(world)]
    dist.all_gather(out, x, group=group)
    return out


class _GroupRingAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, group, causal, block_q, block_k, valid_length, q_position_start):
        world, rank = _group_checks(q, k, v, group, block_q, block_k, valid_length)
        with torch.no_grad():
            ks, vs = _gather(k, world, group), _gather(v, world, group)
            shards = [(q.contiguous(), kk, vv) for kk, vv in zip(ks, vs)]
            out, m, l = ring_causal_attention_forward_with_stats(
                shards, rank, causal, block_q, block_k, valid_length, q_position_start)
        ctx.group, ctx.world, ctx.rank = group, world, rank
        ctx.causal, ctx.block_q, ctx.block_k = causal, block_q, block_k
        ctx.valid_length, ctx.q_position_start = valid_length, q_position_start
        ctx.save_for_backward(q, k, v, out, m, l)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, m, l = ctx.saved_tensors
        none6 = (None,) * 6
        if ctx.q_position_start is not None and ctx.world == 1:
            return (*local_decode_backward(q, k, v, out, m, l, grad_out.contiguous(),
                                           causal=ctx.causal,
                                           q_position_start=ctx.q_position_start,
                                           valid_length=ctx.valid_length), *none6)
        w, g = ctx.world, ctx.group
        qs, ks, vs = _gather(q, w, g), _gather(k, w, g), _gather(v, w, g)
        outs, gos = _gather(out, w, g), _gather(grad_out, w, g)
        ms, ls = _gather(m, w, g), _gather(l, w, g)
        dq, dk, dv = ring_causal_attention_backward(
            list(zip(qs, ks, vs)), ctx.rank, outs, ms, ls, gos, ctx.causal, ctx.block_q,
            ctx.block_k, ctx.valid_length, ctx.q_position_start)
        return (dq, dk, dv, *none6)
