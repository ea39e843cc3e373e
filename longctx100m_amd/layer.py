"""Decoder-layer prefill share on MI355X: RMSNorm, RoPE and SwiGLU kernels
(include/longctx100m_layer.h) around the ring attention of this package, with
the projections as library GEMMs (torch.matmul -> hipBLASLt), except one decode token,
which goes through lc_gemv.

Mirrors the reference's decoder (rust/longctx100m-model/src/model.rs:387-393):
    h = RMSNorm(x); q, k, v = proj(h); q, k = RoPE(q, k); a = attention(q, k, v)
    x = x + o_proj(a); h = RMSNorm(x); x = x + down(silu(gate(h)) * up(h))
with the attention of one rank's shard taken over the ring
(SelfAttention::forward_ring, model.rs:155-222).  The q/k/v projections run
as one GEMM against the stacked [q; k; v] weight, and gate/up as one GEMM
against [gate; up].  RoPE writes the q and k columns of the fused output
straight into contiguous attention inputs, and each residual add is fused
into the RMSNorm that follows it.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib
from . import ring_attention as ra
from .ring_attention import _dtype_code, _stream


def _chk_cuda(*ts):
    for t in ts:
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError("tensors must live on the GPU (device pointers are passed to HIP)")


def _chk_out(t: Optional[torch.Tensor], rows: int, cols: int, dtype, name: str) -> None:
    """A caller-supplied output of ``rows`` rows of ``cols`` contiguous elements
    (row stride free): the kernels take raw pointers and write every row."""
    if t is None:
        return
    _chk_cuda(t)
    if t.dtype != dtype or t.numel() == 0 or t.shape[-1] != cols or t.stride(-1) != 1 or \
            t.reshape(-1, cols).shape[0] != rows:
        raise ValueError(f"{name} must be a {dtype} tensor of {rows} rows of {cols} "
                         f"contiguous elements, got {t.dtype} {tuple(t.shape)}")


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: Optional[torch.Tensor] = None, residual_out: Optional[torch.Tensor] = None,
            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm over the last dim (model.rs:53-62); with ``residual`` the input
    is x + residual (rounded to the dtype), written to ``residual_out`` if given."""
    _chk_cuda(x, weight)
    cols = x.shape[-1]
    x2 = x.reshape(-1, cols)
    if x2.stride(-1) != 1:
        raise ValueError("rows must be contiguous")
    if weight.numel() != cols or weight.dtype != x.dtype:
        raise ValueError(f"weight must hold {cols} elements of {x.dtype}")
    _chk_out(residual, x2.shape[0], cols, x.dtype, "residual")
    _chk_out(residual_out, x2.shape[0], cols, x.dtype, "residual_out")
    _chk_out(out, x2.shape[0], cols, x.dtype, "out")
    out = torch.empty(x2.shape, dtype=x.dtype, device=x.device) if out is None else out
    r2 = residual.reshape(-1, cols) if residual is not None else None
    ro = residual_out.reshape(-1, cols) if residual_out is not None else None
    if ro is not None and ro.stride(-1) != 1:
        raise ValueError("rows must be contiguous")
    _lib.check(_lib.load().lc_rmsnorm(
        _dtype_code(x), x2.shape[0], cols, float(eps), x2.data_ptr(), x2.stride(0),
        r2.data_ptr() if r2 is not None else None, r2.stride(0) if r2 is not None else 0,
        ro.data_ptr() if ro is not None else None, ro.stride(0) if ro is not None else 0,
        weight.data_ptr(), out.data_ptr(), out.reshape(-1, cols).stride(0), _stream()))
    return out.reshape(x.shape)


def rope_params(head_dim: int, theta: float, rope_scaling: Optional[dict] = None) -> _lib.Rope:
    """The lc_rope_t of a config's rope_theta / rope_scaling (rope.rs:24-99)."""
    r = _lib.Rope(head_dim, 0, float(theta), 1.0, 0.0, 0.0, 0.0, 1.0)
    if rope_scaling:
        kind = rope_scaling.get("rope_type", rope_scaling.get("type", "default"))
        r.type = {"default": 0, "linear": 1, "llama3": 2}.get(kind, -1)
        if r.type < 0:
            raise ValueError(f"unsupported RoPE type {kind!r}")
        r.factor = float(rope_scaling.get("factor", 1.0))
        if r.type == 2:
            need = ("low_freq_factor", "high_freq_factor", "original_max_position_embeddings")
            if any(k not in rope_scaling for k in need):
                raise ValueError("llama3 RoPE needs low/high frequency factors and original "
                                 "context length")
            r.low_freq_factor = float(rope_scaling["low_freq_factor"])
            r.high_freq_factor = float(rope_scaling["high_freq_factor"])
            r.original_max_position_embeddings = float(
                rope_scaling["original_max_position_embeddings"])
            r.attention_factor = float(rope_scaling.get("attention_factor", 1.0))
    return r


def rope_inv_freq(rope: _lib.Rope) -> Tuple[List[float], float]:
    """Host inverse frequencies and cosine factor (no GPU needed)."""
    inv = (ctypes.c_float * (rope.head_dim // 2))()
    cf = ctypes.c_float()
    _lib.check(_lib.load().lc_rope_inv_freq(ctypes.byref(rope), ctypes.addressof(inv),
                                            ctypes.addressof(cf)))
    return list(inv), cf.value


def rope_table(rope: _lib.Rope, tokens: int, pos0: int, device="cuda") -> torch.Tensor:
    """[tokens, 2, head_dim/2] fp32 cos/sin table for positions pos0 .. pos0+tokens-1."""
    table = torch.empty((tokens, 2, rope.head_dim // 2), dtype=torch.float32, device=device)
    _lib.check(_lib.load().lc_rope_table(ctypes.byref(rope), tokens, pos0, table.data_ptr(),
                                         _stream()))
    return table


def rope_apply(src: torch.Tensor, table: torch.Tensor, heads: int, head_dim: int,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rotate-half RoPE of the [tokens, heads*head_dim] columns ``src`` (row stride
    free, e.g. a column slice of the fused QKV output) into contiguous
    [tokens, heads, head_dim] (rope.rs:116-127)."""
    _chk_cuda(src, table)
    tokens = src.shape[0]
    if src.dim() != 2 or src.shape[1] != heads * head_dim or src.stride(1) != 1:
        raise ValueError("src must be [tokens, heads*head_dim] with contiguous rows")
    if table.dtype != torch.float32 or table.dim() != 3 or table.shape[0] < tokens or \
            table.shape[1:] != (2, head_dim // 2) or not table.is_contiguous():
        raise ValueError("table must be a contiguous [tokens, 2, head_dim/2] fp32 rope_table")
    if out is not None and (not out.is_contiguous() or out.numel() != tokens * heads * head_dim):
        raise ValueError("out must be a contiguous [tokens, heads, head_dim] tensor")
    _chk_out(out, tokens * heads, head_dim, src.dtype, "out")
    out = torch.empty((tokens, heads, head_dim), dtype=src.dtype, device=src.device) \
        if out is None else out
    _lib.check(_lib.load().lc_rope_apply(_dtype_code(src), tokens, heads, head_dim,
                                         table.data_ptr(), src.data_ptr(), src.stride(0),
                                         out.data_ptr(), _stream()))
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor, out: Optional[torch.Tensor] = None):
    """silu(gate) * up over [rows, cols] views (row strides free)."""
    _chk_cuda(gate, up)
    rows, cols = gate.shape
    if up.shape != gate.shape or gate.stride(1) != 1 or up.stride(1) != 1:
        raise ValueError("gate and up must be [rows, cols] with contiguous rows")
    if out is not None and (not out.is_contiguous() or out.numel() != rows * cols):
        raise ValueError("out must be a contiguous [rows, cols] tensor")
    _chk_out(out, rows, cols, gate.dtype, "out")
    out = torch.empty((rows, cols), dtype=gate.dtype, device=gate.device) if out is None else out
    _lib.check(_lib.load().lc_swiglu(_dtype_code(gate), rows, cols, gate.data_ptr(),
                                     gate.stride(0), up.data_ptr(), up.stride(0),
                                     out.data_ptr(), _stream()))
    return out


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x @ w.T for a bias-free linear layer (candle Linear,
    rust/longctx100m-model/src/model.rs:64-76).  One bf16 token goes through
    the bandwidth-bound lc_gemv (the decode step); anything else is a library
    GEMM."""
    if (x.dim() == 2 and x.shape[0] == 1 and x.dtype == torch.bfloat16
            and w.dtype == torch.bfloat16 and x.is_contiguous() and w.stride(1) == 1
            and w.shape[1] % 8 == 0 and w.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0):
        _chk_cuda(x, w)
        rows, cols = w.shape
        if x.shape[1] != cols:
            raise ValueError("x and w do not match")
        y = torch.empty((1, rows), dtype=x.dtype, device=x.device)
        _lib.check(_lib.load().lc_gemv(_dtype_code(x), rows, cols, w.data_ptr(), w.stride(0),
                                       x.data_ptr(), y.data_ptr(), _stream()))
        return y
    return torch.matmul(x, w.t())


def gemv_fused(x: torch.Tensor, w: torch.Tensor, *, norm_weight: Optional[torch.Tensor] = None,
               eps: float = 0.0, residual: Optional[torch.Tensor] = None,
               residual_out: Optional[torch.Tensor] = None, swiglu: bool = False,
               rope_row: Optional[torch.Tensor] = None, heads: Optional[Tuple[int, int]] = None,
               k_out: Optional[torch.Tensor] = None,
               v_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One token through lc_gemv_fused: the projection x @ w.T of the decode
    step with its neighbouring row operation folded in, bit-identical to the
    unfused calls.
    * x: bf16 [1, cols], or fp32 [1, cols] (rounded to bf16 first: the
      attention output cast);
    * norm_weight (+ eps, residual, residual_out): the multiplied vector is
      rmsnorm(x (+ residual)) as :func:`rmsnorm` computes it (bf16 x);
    * swiglu: w holds gate rows then up rows; returns swiglu(gate, up) [1, rows/2];
    * rope_row (+ heads = (q_heads, kv_heads), k_out, v_out): w is a fused
      q/k/v weight; returns RoPE(q) [1, q_heads * head_dim] and writes RoPE(k)
      to k_out and v to v_out (e.g. a KV cache's row of the token)."""
    _chk_cuda(x, w)
    rows, cols = w.shape
    if x.dim() != 2 or x.shape != (1, cols) or not x.is_contiguous():
        raise ValueError(f"x must be a contiguous [1, {cols}] tensor")
    if w.dtype != torch.bfloat16 or w.stride(1) != 1:
        raise ValueError("w must be bf16 with contiguous rows")
    f = _lib.GemvFused()
    if x.dtype == torch.float32:
        f.in_form = _lib.LC_GEMV_IN_F32
    elif x.dtype == torch.bfloat16:
        f.in_form = _lib.LC_GEMV_IN_BF16
    else:
        raise ValueError("x must be bf16 or fp32")
    if norm_weight is not None:
        if x.dtype != torch.bfloat16:
            raise ValueError("the folded rmsnorm takes a bf16 x")
        _chk_out(norm_weight.view(1, -1), 1, cols, x.dtype, "norm_weight")
        _chk_out(residual, 1, cols, x.dtype, "residual")
        _chk_out(residual_out, 1, cols, x.dtype, "residual_out")
        f.in_form = _lib.LC_GEMV_IN_RMSNORM
        f.norm_weight = norm_weight.data_ptr()
        f.eps = float(eps)
        f.residual = residual.data_ptr() if residual is not None else None
        f.residual_out = residual_out.data_ptr() if residual_out is not None else None
    elif residual is not None or residual_out is not None:
        raise ValueError("residual and residual_out belong to the folded rmsnorm (norm_weight)")
    if swiglu and rope_row is not None:
        raise ValueError("one output form: swiglu or rope")
    if swiglu:
        f.out_form = _lib.LC_GEMV_OUT_SWIGLU
        y = torch.empty((1, rows // 2), dtype=torch.bfloat16, device=x.device)
    elif rope_row is not None:
        if heads is None or k_out is None or v_out is None:
            raise ValueError("the rope form needs heads, k_out and v_out")
        hq, hkv = heads
        d = rows // (hq + 2 * hkv)
        if rope_row.dtype != torch.float32 or not rope_row.is_contiguous() or \
                rope_row.numel() != d or rope_row.device != x.device:
            raise ValueError(f"rope_row must be one contiguous [2, {d // 2}] fp32 table row")
        _chk_out(k_out.reshape(1, -1), 1, hkv * d, torch.bfloat16, "k_out")
        _chk_out(v_out.reshape(1, -1), 1, hkv * d, torch.bfloat16, "v_out")
        f.out_form = _lib.LC_GEMV_OUT_ROPE_QKV
        f.q_heads, f.kv_heads, f.head_dim = hq, hkv, d
        f.rope_row, f.k_out, f.v_out = rope_row.data_ptr(), k_out.data_ptr(), v_out.data_ptr()
        y = torch.empty((1, hq * d), dtype=torch.bfloat16, device=x.device)
    else:
        f.out_form = _lib.LC_GEMV_OUT_PLAIN
        y = torch.empty((1, rows), dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.load().lc_gemv_fused(ctypes.byref(f), rows, cols, w.data_ptr(), w.stride(0),
                                         x.data_ptr(), y.data_ptr(), _stream()))
    return y


# ------------------------------------------------------------- the model --

@dataclass
class ModelConfig:
    """The fields of rust/longctx100m-model/src/config.rs this path uses."""
    hidden_size: int = 4096
    num_heads: int = 32
    num_key_value_heads: int = 8
    intermediate_size: int = 14336
    num_layers: int = 24
    vocab_size: int = 128256
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_scaling: Optional[dict] = None

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads


C4 = ModelConfig()


def init_layer_weights(cfg: ModelConfig, gen: torch.Generator, device, dtype=torch.bfloat16,
                       std: float = 0.02) -> Dict[str, torch.Tensor]:
    """Random-init weights of one decoder layer: N(0, std) projections, unit
    RMSNorm weights (RmsNorm::new's Init::Const(1.0), model.rs:43-46)."""
    d, hq, hkv = cfg.head_dim, cfg.num_heads, cfg.num_key_value_heads
    c, inter = cfg.hidden_size, cfg.intermediate_size

    def randn(*shape):
        return (torch.randn(*shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)

    return {
        "wqkv": randn((hq + 2 * hkv) * d, c),  # rows: q_proj, k_proj, v_proj
        "wo": randn(c, hq * d),
        "wgu": randn(2 * inter, c),            # rows: gate_proj, up_proj
        "wd": randn(c, inter),
        "norm1": torch.ones(c, device=device, dtype=dtype),
        "norm2": torch.ones(c, device=device, dtype=dtype),
    }


def layer_prefill(x: torch.Tensor, w: Dict[str, torch.Tensor], cfg: ModelConfig,
                  table: torch.Tensor, rank: int,
                  preceding_kv: Sequence[Tuple[torch.Tensor, torch.Tensor]],
                  residual: Optional[torch.Tensor] = None,
                  timers: Optional[Dict[str, list]] = None,
                  cache: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
    """One decoder layer over this rank's shard x [T, hidden].

    ``preceding_kv`` holds the (k, v) [1, T, Hkv, d] shards of ranks 0..rank-1
    (the ring's incoming KV).  ``cache``, when given, is this layer's KV cache
    ([1, capacity, Hkv, d] K and V) and receives the shard's rotated K and V.  ``residual``, when given, is the previous
    layer's MLP output still to be added to x (the add is fused into this
    layer's first RMSNorm).  Returns (x_after_attention, mlp_out): the layer
    output is their sum, which the next layer's (or the final) RMSNorm forms."""
    T, c = x.shape
    d, hq, hkv = cfg.head_dim, cfg.num_heads, cfg.num_key_value_heads
    if len(preceding_kv) != rank:
        raise ValueError("preceding_kv must hold one (k, v) per earlier rank")

    def tick(name):
        if timers is not None:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            timers.setdefault("_events", []).append((name, e))

    tick("start")
    if residual is not None:
        xin = torch.empty_like(x)
        h = rmsnorm(x, w["norm1"], cfg.rms_norm_eps, residual=residual, residual_out=xin)
    else:
        xin = x
        h = rmsnorm(x, w["norm1"], cfg.rms_norm_eps)
    tick("norm")
    qkv = torch.matmul(h, w["wqkv"].t())
    tick("gemm")
    q = rope_apply(qkv[:, :hq * d], table, hq, d)
    k = rope_apply(qkv[:, hq * d:(hq + hkv) * d], table, hkv, d)
    v = qkv[:, (hq + hkv) * d:].contiguous().view(T, hkv, d)
    tick("rope")
    qb, kb, vb = q.view(1, T, hq, d), k.view(1, T, hkv, d), v.view(1, T, hkv, d)
    if cache is not None:  # keep this shard's rotated K and V for incremental decode
        cache[0][:, :T].copy_(kb)
        cache[1][:, :T].copy_(vb)
    shards = [(qb, pk, pv) for pk, pv in preceding_kv] + [(qb, kb, vb)]
    attn, _, _ = ra.ring_causal_attention_forward_with_stats(shards, rank)
    tick("attention")
    o = torch.matmul(attn.view(T, hq * d), w["wo"].t())
    tick("gemm")
    x2 = torch.empty_like(x)
    h2 = rmsnorm(xin, w["norm2"], cfg.rms_norm_eps, residual=o, residual_out=x2)
    tick("norm")
    gu = torch.matmul(h2, w["wgu"].t())
    tick("gemm")
    inter = cfg.intermediate_size
    a = swiglu(gu[:, :inter], gu[:, inter:])
    tick("swiglu")
    mlp = torch.matmul(a, w["wd"].t())
    tick("gemm")
    return x2, mlp


def layer_flops(cfg: ModelConfig, tokens: int, rank: int) -> Dict[str, float]:
    """Algorithmic FLOPs of one layer's prefill share: GEMMs and attention
    (4*Nq*Nk*Hq*d per full shard pair, the diagonal counting half)."""
    d, hq, hkv = cfg.head_dim, cfg.num_heads, cfg.num_key_value_heads
    c, inter = cfg.hidden_size, cfg.intermediate_size
    gemm = 2.0 * tokens * c * ((hq + 2 * hkv) * d + hq * d + 2 * inter) + 2.0 * tokens * inter * c
    attn = (rank + 0.5) * 4.0 * tokens * tokens * hq * d
    return {"gemm": gemm, "attention": attn}


# ------------------------------------------------------- incremental decode --

def layer_decode(x: torch.Tensor, w: Dict[str, torch.Tensor], cfg: ModelConfig,
                 table: torch.Tensor, pos: int, cache: Tuple[torch.Tensor, torch.Tensor],
                 residual: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None, fused: bool = True):
    """One decoder layer for the token at position ``pos`` (x [1, hidden]),
    attending to the cache rows 0..pos after appending its own K and V.  The
    reference recomputes the whole prefill for each new token
    (src/longctx100m/distributed_infer.py:185-219,
    rust/longctx100m-model/src/bin/infer.rs:96-106); this computes the same
    last-position result from the cache.  ``table`` row ``pos`` holds the
    token's RoPE angles.  Returns (x_after_attention, mlp_out) as layer_prefill.

    ``fused`` runs each projection as one lc_gemv_fused launch with its row
    operation folded in (norm + QKV + RoPE + cache append, the fp32 attention
    output's cast + o, norm + gate/up + SwiGLU, down): five launches with the
    attention instead of thirteen, with bit-identical results."""
    d, hq, hkv = cfg.head_dim, cfg.num_heads, cfg.num_key_value_heads
    if fused:
        kc, vc = cache
        xin = torch.empty_like(x) if residual is not None else x
        q = gemv_fused(x, w["wqkv"], norm_weight=w["norm1"], eps=cfg.rms_norm_eps,
                       residual=residual, residual_out=xin if residual is not None else None,
                       rope_row=table[pos], heads=(hq, hkv), k_out=kc[0, pos], v_out=vc[0, pos])
        o, _, _ = ra.decode(q.view(1, 1, hq, d), kc[:, :pos + 1], vc[:, :pos + 1], q_pos0=pos,
                            k_pos0=0, workspace=workspace)
        ao = gemv_fused(o.view(1, hq * d), w["wo"])
        x2 = torch.empty_like(x)
        a = gemv_fused(xin, w["wgu"], norm_weight=w["norm2"], eps=cfg.rms_norm_eps, residual=ao,
                       residual_out=x2, swiglu=True)
        return x2, gemv_fused(a, w["wd"])
    if residual is not None:
        xin = torch.empty_like(x)
        h = rmsnorm(x, w["norm1"], cfg.rms_norm_eps, residual=residual, residual_out=xin)
    else:
        xin = x
        h = rmsnorm(x, w["norm1"], cfg.rms_norm_eps)
    qkv = linear(h, w["wqkv"])
    trow = table[pos:pos + 1]
    q = rope_apply(qkv[:, :hq * d], trow, hq, d)
    kc, vc = cache
    rope_apply(qkv[:, hq * d:(hq + hkv) * d], trow, hkv, d, out=kc[0, pos:pos + 1])
    vc[0, pos:pos + 1].copy_(qkv[:, (hq + hkv) * d:].view(1, hkv, d))
    o, _, _ = ra.decode(q.view(1, 1, hq, d), kc[:, :pos + 1], vc[:, :pos + 1], q_pos0=pos,
                        k_pos0=0, workspace=workspace)
    attn = o.to(x.dtype).view(1, hq * d)  # the forward output in the model dtype
    ao = linear(attn, w["wo"])
    x2 = torch.empty_like(x)
    h2 = rmsnorm(xin, w["norm2"], cfg.rms_norm_eps, residual=ao, residual_out=x2)
    gu = linear(h2, w["wgu"])
    inter = cfg.intermediate_size
    a = swiglu(gu[:, :inter], gu[:, inter:])
    return x2, linear(a, w["wd"])


def new_cache(cfg: ModelConfig, capacity: int, device, dtype=torch.bfloat16):
    """Per-layer (K, V) caches [1, capacity, Hkv, d]."""
    shape = (1, capacity, cfg.num_key_value_heads, cfg.head_dim)
    return [(torch.zeros(shape, device=device, dtype=dtype),
             torch.zeros(shape, device=device, dtype=dtype)) for _ in range(cfg.num_layers)]


def model_prefill(ids: torch.Tensor, weights: Dict, cfg: ModelConfig, table: torch.Tensor,
                  caches=None) -> torch.Tensor:
    """Logits [T, vocab] of a one-rank prefill (embedding, layers, final norm,
    LM head), filling ``caches`` with each layer's rotated K and V if given."""
    x = torch.nn.functional.embedding(ids, weights["embed"])
    res = None
    for li, lw in enumerate(weights["layers"]):
        x, res = layer_prefill(x, lw, cfg, table, 0, [], residual=res,
                               cache=caches[li] if caches is not None else None)
    h = rmsnorm(x, weights["final_norm"], cfg.rms_norm_eps, residual=res)
    return torch.matmul(h, weights["lm_head"].t())


def model_decode_step(token: int, pos: int, weights: Dict, cfg: ModelConfig,
                      table: torch.Tensor, caches, workspace=None,
                      fused: bool = True) -> torch.Tensor:
    """Logits [1, vocab] of the token at ``pos`` given caches holding 0..pos-1
    (``fused`` as layer_decode)."""
    dev = weights["embed"].device
    x = torch.nn.functional.embedding(torch.tensor([token], device=dev), weights["embed"])
    res = None
    for li, lw in enumerate(weights["layers"]):
        x, res = layer_decode(x, lw, cfg, table, pos, caches[li], residual=res,
                              workspace=workspace, fused=fused)
    # The final norm stays a launch of its own: folded into the LM head
    # (32,064 row blocks) its per-workgroup cost outweighs the launch it saves
    # (155-161 us against 151 us).
    h = rmsnorm(x, weights["final_norm"], cfg.rms_norm_eps, residual=res)
    return linear(h, weights["lm_head"])


def init_model_weights(cfg: ModelConfig, gen: torch.Generator, device, dtype=torch.bfloat16,
                       std: float = 0.02) -> Dict:
    """Random-init weights of the whole model (untied LM head)."""
    def randn(*shape):
        return (torch.randn(*shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)

    return {
        "embed": randn(cfg.vocab_size, cfg.hidden_size),
        "lm_head": randn(cfg.vocab_size, cfg.hidden_size),
        "final_norm": torch.ones(cfg.hidden_size, device=device, dtype=dtype),
        "layers": [init_layer_weights(cfg, gen, device, dtype, std) for _ in range(cfg.num_layers)],
    }
