"""The C-ABI library loads, exports exactly what include/longctx100m_attn.h
and include/longctx100m_layer.h declare, and rejects bad arguments with the reference's messages
(rust/longctx100m-model/src/ring_attention.rs:148-171) before touching the
GPU.  Runs without a GPU: no compute entry point is reached."""

import ctypes
import re
from pathlib import Path

import pytest

from longctx100m_amd import _lib

HEADERS = [Path(__file__).resolve().parents[1] / "include" / name
           for name in ("longctx100m_attn.h", "longctx100m_layer.h")]


def header_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(lc_\w+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_library_exports_every_declared_symbol(lib):
    declared = header_functions()
    assert len(declared) >= 15
    assert sorted(_lib.SIGNATURES) == declared
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.lc_abi_version() == 2


def test_struct_layouts_match_header():
    assert ctypes.sizeof(_lib.Shape) == 32
    assert ctypes.sizeof(_lib.Mask) == 32
    assert ctypes.sizeof(_lib.RingDesc) == 64
    assert ctypes.sizeof(_lib.Rope) == 56
    assert _lib.RingDesc.valid_length.offset == 48
    assert ctypes.sizeof(_lib.GemvFused) == 72
    assert _lib.GemvFused.eps.offset == 32 and _lib.GemvFused.rope_row.offset == 48


def _desc(**kw):
    d = dict(world=2, rank=0, batch=1, local_tokens=8, heads_q=4, heads_kv=2, head_dim=64,
             dtype=_lib.LC_DTYPE_BF16, flags=0, causal=1, block_q=64, block_k=128,
             valid_length=-1, q_position_start=-1)
    d.update(kw)
    return _lib.RingDesc(**d)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(rank=2), _lib.LC_ERR_INVALID, "rank 2 out of range for world_size 2"),
    (dict(block_q=0), _lib.LC_ERR_INVALID, "block_q and block_k must be positive"),
    (dict(block_k=-3), _lib.LC_ERR_INVALID, "block_q and block_k must be positive"),
    (dict(local_tokens=0), _lib.LC_ERR_INVALID, "local_tokens must be positive"),
    (dict(valid_length=17), _lib.LC_ERR_INVALID,
     "valid_length must be within the padded distributed sequence"),
    (dict(valid_length=0), _lib.LC_ERR_INVALID,
     "valid_length must be within the padded distributed sequence"),
    (dict(heads_kv=3), _lib.LC_ERR_INVALID, "q, k, v shard shapes must match"),
    (dict(head_dim=0), _lib.LC_ERR_INVALID,
     "q, k, v must have shape [batch, tokens, heads, head_dim]"),
    (dict(dtype=7), _lib.LC_ERR_UNSUPPORTED, "unsupported dtype 7"),
    (dict(flags=4), _lib.LC_ERR_INVALID, "unknown flag bits 0x4"),
    (dict(flags=0x80000001), _lib.LC_ERR_INVALID, "unknown flag bits 0x80000000"),
])
def test_ring_validation_messages(lib, kw, code, msg):
    d = _desc(**kw)
    assert lib.lc_ring_fwd_workspace_bytes(d) == 0
    rc = lib.lc_ring_fwd_with_stats(d, None, None, None, None, None, None, None, 0, None)
    assert rc == code
    assert lib.lc_last_error().decode() == msg
    rc = lib.lc_ring_bwd(d, None, None, None, None, None, None, None, None, None, None, None, 0,
                         None)
    assert rc == code
    assert lib.lc_last_error().decode() == msg
    with pytest.raises(ValueError if code == _lib.LC_ERR_INVALID else _lib.LcError, match=re.escape(msg)):
        _lib.check(rc)


def test_workspace_sizes(lib):
    d = _desc(local_tokens=32768, heads_q=16, heads_kv=16, head_dim=128, world=8, rank=7)
    n_o = 32768 * 16 * 128
    n_s = 16 * 32768
    assert lib.lc_ring_fwd_workspace_bytes(d) == 4 * n_o  # the running output; m, l are outputs
    assert lib.lc_ring_bwd_workspace_bytes(d) == 3 * 4 * n_o + 2 * 4 * n_s
    # with room for the diagonal pair's dS: 32,768^2 keys x 16 heads x 2 bytes = the 32 GiB cap
    base = lib.lc_ring_bwd_workspace_bytes(d)
    assert lib.lc_ring_bwd_ds_workspace_bytes(d) == base + (32 << 30)
    # no sharing: q_position_start away from rank * n, fp32, the fp32-math flag, d != 128
    for kw in (dict(q_position_start=5), dict(dtype=_lib.LC_DTYPE_F32),
               dict(flags=_lib.LC_FLAG_PRECISE), dict(head_dim=64)):
        dd = _desc(**dict(dict(local_tokens=32768, heads_q=16, heads_kv=16, head_dim=128,
                               world=8, rank=7), **kw))
        assert lib.lc_ring_bwd_ds_workspace_bytes(dd) == lib.lc_ring_bwd_workspace_bytes(dd)
    dd = _desc(local_tokens=32768, heads_q=16, heads_kv=16, head_dim=128, world=8, rank=7,
               q_position_start=7 * 32768)  # the default position given explicitly
    assert lib.lc_ring_bwd_ds_workspace_bytes(dd) == base + (32 << 30)
    one = _desc(world=1, rank=0, local_tokens=100, heads_q=4, heads_kv=2, head_dim=128)
    assert lib.lc_ring_bwd_ds_workspace_bytes(one) == \
        lib.lc_ring_bwd_workspace_bytes(one) + 4 * 4 * 4 * 2048
    assert lib.lc_ring_bwd_ds_workspace_bytes(_desc(rank=5)) == 0  # invalid descriptor


def test_null_and_workspace_errors(lib):
    d = _desc()
    ptrs = (ctypes.c_void_p * 2)(1, 2)
    pp = ctypes.cast(ptrs, ctypes.POINTER(ctypes.c_void_p))
    rc = lib.lc_ring_fwd_with_stats(d, pp, pp, pp, 16, 16, 16, 16, 1, None)
    assert rc == _lib.LC_ERR_WORKSPACE
    assert "workspace" in lib.lc_last_error().decode()
    rc = lib.lc_ring_fwd_with_stats(d, None, pp, pp, 16, 16, 16, 16, 1 << 30, None)
    assert rc == _lib.LC_ERR_INVALID
    assert lib.lc_last_error().decode() == "null q pointer array"
    shape = _lib.Shape(1, 4, 4, 2, 2, 64, _lib.LC_DTYPE_BF16, 0)
    rc = lib.lc_attn_fwd_shard(shape, None, None, None, None, None, None, None, None)
    assert rc == _lib.LC_ERR_INVALID
    bad = _lib.Shape(1, 4, 4, 3, 2, 64, _lib.LC_DTYPE_BF16, 0)
    rc = lib.lc_attn_fwd_shard(bad, None, 16, 16, 16, 16, 16, 16, None)
    assert rc == _lib.LC_ERR_INVALID
    assert "multiple of heads_kv" in lib.lc_last_error().decode()
    big = _lib.Shape(1, 4, 4, 2, 2, 512, _lib.LC_DTYPE_F32, 0)
    rc = lib.lc_attn_fwd_shard(big, None, 16, 16, 16, 16, 16, 16, None)
    assert rc == _lib.LC_ERR_UNSUPPORTED
    rc = lib.lc_attn_cast(None, None, 10, 5, None)
    assert rc == _lib.LC_ERR_UNSUPPORTED


def test_accumulate_flag_is_for_fwd_shard_only(lib):
    """LC_FLAG_ACCUMULATE merges a hop into a running state in lc_attn_fwd_shard;
    the decode entry points and the ring descriptor reject it before any GPU work."""
    acc = _lib.LC_FLAG_ACCUMULATE
    msg = "LC_FLAG_ACCUMULATE applies to lc_attn_fwd_shard only"
    shape = _lib.Shape(1, 1, 4096, 8, 2, 128, _lib.LC_DTYPE_BF16, acc)
    mask = _lib.Mask(4095, 0, -1, 1, 0)
    rc = lib.lc_attn_decode(shape, mask, 16, 16, 16, 16, 16, 16, 16, 1 << 20, None)
    assert rc == _lib.LC_ERR_INVALID and lib.lc_last_error().decode() == msg
    rc = lib.lc_attn_decode_static(shape, mask, 16, 16, 16, 16, 16, 16, None)
    assert rc == _lib.LC_ERR_INVALID and lib.lc_last_error().decode() == msg
    d = _desc(flags=acc)
    assert lib.lc_ring_fwd_workspace_bytes(d) == 0
    rc = lib.lc_ring_fwd_with_stats(d, None, None, None, None, None, None, None, 0, None)
    assert rc == _lib.LC_ERR_INVALID and lib.lc_last_error().decode() == msg


def test_unknown_flag_bits_rejected(lib):
    """A flags word with a bit this library does not define (a stray or
    uninitialised value) is rejected before any device work by every entry
    point that takes a shape, instead of selecting a mode by accident."""
    shape = _lib.Shape(1, 4, 4, 2, 2, 64, _lib.LC_DTYPE_BF16, 4)
    mask = _lib.Mask(0, 0, -1, 1, 0)
    msg = "unknown flag bits 0x4"
    assert lib.lc_attn_fwd_shard(shape, mask, 16, 16, 16, 16, 16, 16, None) == _lib.LC_ERR_INVALID
    assert lib.lc_last_error().decode() == msg
    assert lib.lc_attn_bwd_shard(shape, mask, 16, 16, 16, 16, 16, 16, 16, 16, 16,
                                 None) == _lib.LC_ERR_INVALID
    assert lib.lc_last_error().decode() == msg
    assert lib.lc_attn_bwd_shard_workspace_bytes(shape) == 0
    assert lib.lc_attn_decode_static(shape, mask, 16, 16, 16, 16, 16, 16,
                                     None) == _lib.LC_ERR_INVALID
    assert lib.lc_last_error().decode() == msg
    shape.flags = _lib.LC_FLAG_PRECISE | _lib.LC_FLAG_ACCUMULATE | 8
    assert lib.lc_attn_merge(shape, 16, 16, 16, 16, 16, 16, None, None) == _lib.LC_ERR_INVALID
    assert lib.lc_last_error().decode() == "unknown flag bits 0x8"


def test_last_error_is_per_thread(lib):
    import threading

    lib.lc_ring_fwd_with_stats(_desc(rank=5), None, None, None, None, None, None, None, 0, None)
    seen = {}

    def other():
        lib.lc_ring_fwd_with_stats(_desc(block_q=0), None, None, None, None, None, None, None, 0,
                                   None)
        seen["msg"] = lib.lc_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == "block_q and block_k must be positive"
    assert lib.lc_last_error().decode() == "rank 5 out of range for world_size 2"


def test_shared_ds_workspace_size_and_errors(lib):
    """lc_attn_bwd_shard_workspace_bytes: 2 bytes per (query, key, query head) of up to
    65,536 query rows, in 32 x 32 blocks; 0 off the d=128 bf16 path.  The workspace entry
    rejects bad arguments before touching the GPU."""
    bf, f32 = _lib.LC_DTYPE_BF16, _lib.LC_DTYPE_F32
    size = lambda *s: lib.lc_attn_bwd_shard_workspace_bytes(_lib.Shape(*s))  # noqa: E731
    assert size(1, 32768, 32768, 16, 16, 128, bf, 0) == 16 * 1024 * 1024 * 2048
    assert size(2, 100, 70, 4, 2, 128, bf, 0) == 2 * 4 * 4 * 3 * 2048
    assert size(1, 200000, 64, 1, 1, 128, bf, 0) == 2048 * 2 * 2048  # 65,536-row chunks
    # capped at 32 GiB: a 1M-key shard gets the largest multiple of 256 rows that fits
    cap = 32 << 30
    per32 = 16 * (1_000_000 // 32) * 2048  # one 32-row query tile, 16 heads
    assert size(1, 1_000_000, 1_000_000, 16, 16, 128, bf, 0) == (cap // per32 * 32 // 256 * 256 // 32) * per32
    assert size(1, 1_000_000, 1_000_000, 16, 16, 128, bf, 0) <= cap
    assert size(1, 65536, 65536, 16, 16, 128, bf, 0) == cap  # 128 GiB for 65,536 rows: 16,384
    assert size(1, 4096, 8_000_000, 16, 16, 128, bf, 0) == 0  # not even 256 rows fit
    assert size(1, 256, 256, 2, 2, 64, bf, 0) == 0
    assert size(1, 256, 256, 2, 2, 128, f32, 0) == 0
    assert size(1, 256, 256, 2, 2, 128, bf, _lib.LC_FLAG_PRECISE) == 0
    assert size(1, 256, 256, 3, 2, 128, bf, 0) == 0  # invalid shape
    shape = _lib.Shape(1, 64, 64, 2, 2, 128, bf, 0)
    mask = _lib.Mask(0, 0, -1, 1, 0)
    rc = lib.lc_attn_bwd_shard_ws(shape, mask, None, 16, 16, 16, 16, 16, 16, 16, 16, None, 0,
                                  None)
    assert rc == _lib.LC_ERR_INVALID and lib.lc_last_error().decode() == "null pointer argument"
    rc = lib.lc_attn_bwd_shard_ws(shape, mask, 16, 16, 16, 16, 16, 16, 16, 16, None, None, 0,
                                  None)
    assert rc == _lib.LC_ERR_INVALID and "both be set" in lib.lc_last_error().decode()
    rc = lib.lc_attn_bwd_shard_ws(shape, mask, 16, 16, 16, 16, 16, 16, 16, 16, 16, None, 4096,
                                  None)
    assert rc == _lib.LC_ERR_INVALID and "workspace is NULL" in lib.lc_last_error().decode()


def test_gemv_argument_errors(lib):
    bf, f32 = _lib.LC_DTYPE_BF16, _lib.LC_DTYPE_F32
    assert lib.lc_gemv(f32, 4, 8, 16, 8, 16, 16, None) == _lib.LC_ERR_UNSUPPORTED
    assert lib.lc_gemv(bf, 4, 12, 16, 16, 16, 16, None) == _lib.LC_ERR_INVALID
    assert lib.lc_gemv(bf, 4, 8, 16, 12, 16, 16, None) == _lib.LC_ERR_INVALID
    assert lib.lc_gemv(bf, 4, 8, None, 8, 16, 16, None) == _lib.LC_ERR_INVALID
    assert lib.lc_last_error().decode() == "null pointer argument"
    assert lib.lc_gemv(bf, 4, 8, 24, 8, 16, 16, None) == _lib.LC_ERR_INVALID
    assert "aligned" in lib.lc_last_error().decode()
    assert lib.lc_gemv(bf, 0, 8, 16, 8, 16, 16, None) == _lib.LC_OK


def test_gemv_fused_argument_errors(lib):
    """lc_gemv_fused checks its forms before any launch.  Every call here fails
    a check or has rows = 0 (which returns after the checks), so none reaches
    a launch with these placeholder pointers.  Outputs (y, and k_out / v_out of
    the rope form) that share a byte with x, residual or residual_out are
    rejected: other workgroups still read those while one writes its rows."""
    G = _lib.GemvFused

    def call(f, rows=0, cols=64):
        rc = lib.lc_gemv_fused(ctypes.byref(f) if f is not None else None, rows, cols, 16, cols,
                               16, 16, None)
        return rc, lib.lc_last_error().decode()

    assert call(None)[0] == _lib.LC_ERR_INVALID
    assert call(G(in_form=3)) == (_lib.LC_ERR_INVALID, "unknown gemv input form 3")
    assert call(G(out_form=5)) == (_lib.LC_ERR_INVALID, "unknown gemv output form 5")
    assert call(G(in_form=_lib.LC_GEMV_IN_RMSNORM, norm_weight=16), cols=4104)[1] == \
        "the folded rmsnorm needs cols <= 4096"
    assert call(G(in_form=_lib.LC_GEMV_IN_RMSNORM))[1] == "rmsnorm needs norm_weight"
    assert call(G(in_form=_lib.LC_GEMV_IN_RMSNORM, norm_weight=16, residual_out=16))[1] == \
        "residual_out needs a residual input"
    assert call(G(in_form=_lib.LC_GEMV_IN_RMSNORM, norm_weight=24))[1] == \
        "rmsnorm pointers must be 16-byte aligned"
    assert call(G(in_form=_lib.LC_GEMV_IN_RMSNORM, norm_weight=16, eps=-1.0))[1] == \
        "eps must be non-negative"
    assert call(G(in_form=_lib.LC_GEMV_IN_RMSNORM, norm_weight=16, residual=4096,
                  residual_out=16 + 64))[1] == "residual_out must not overlap x or residual"
    assert call(G(in_form=_lib.LC_GEMV_IN_RMSNORM, norm_weight=16, residual=4096,
                  residual_out=4096 + 112))[1] == "residual_out must not overlap x or residual"
    assert call(G(in_form=_lib.LC_GEMV_IN_RMSNORM, norm_weight=16, residual=4096,
                  residual_out=16 + 128))[0] == _lib.LC_OK  # adjacent, rows = 0: no launch
    assert call(G(out_form=_lib.LC_GEMV_OUT_SWIGLU), rows=6)[0] == _lib.LC_ERR_INVALID
    rope = dict(out_form=_lib.LC_GEMV_OUT_ROPE_QKV, q_heads=2, kv_heads=1, head_dim=16,
                rope_row=16, k_out=16, v_out=16)
    assert "rows = (q_heads + 2 kv_heads) head_dim" in call(G(**rope), rows=48)[1]
    assert "head_dim % 16 == 0" in call(G(**dict(rope, head_dim=8)), rows=32)[1]
    assert call(G(**dict(rope, k_out=None)), rows=64)[1] == \
        "rope form needs rope_row, k_out and v_out"
    assert call(G(**dict(rope, rope_row=18)), rows=64)[1] == \
        "rope_row must be 4-byte and k_out, v_out 2-byte aligned"
    assert call(G(**dict(rope, v_out=17)), rows=64)[1] == \
        "rope_row must be 4-byte and k_out, v_out 2-byte aligned"

    def call_xy(f, rows, cols, x, y):
        rc = lib.lc_gemv_fused(ctypes.byref(f), rows, cols, 16, cols, x, y, None)
        return rc, lib.lc_last_error().decode()

    ovl = "gemv outputs must not overlap x, residual or residual_out"
    # y (rows bf16) against x (cols bf16 / fp32): in place, or sharing a byte
    assert call_xy(G(), 64, 64, 4096, 4096) == (_lib.LC_ERR_INVALID, ovl)
    assert call_xy(G(), 64, 64, 4096, 4096 + 126) == (_lib.LC_ERR_INVALID, ovl)
    assert call_xy(G(), 64, 64, 4096 + 16, 4096 + 16 - 126) == (_lib.LC_ERR_INVALID, ovl)
    assert call_xy(G(in_form=_lib.LC_GEMV_IN_F32), 64, 64, 4096, 4096 + 254) == \
        (_lib.LC_ERR_INVALID, ovl)
    # the folded norm: y against residual and residual_out
    nrm = dict(in_form=_lib.LC_GEMV_IN_RMSNORM, norm_weight=16, residual=8192,
               residual_out=12288)
    assert call_xy(G(**nrm), 64, 64, 4096, 8192 + 64) == (_lib.LC_ERR_INVALID, ovl)
    assert call_xy(G(**nrm), 64, 64, 4096, 12288 - 64) == (_lib.LC_ERR_INVALID, ovl)
    # swiglu writes rows / 2 elements; rope writes q_heads * head_dim, k_out, v_out
    assert call_xy(G(out_form=_lib.LC_GEMV_OUT_SWIGLU), 128, 64, 4096, 4096 - 126) == \
        (_lib.LC_ERR_INVALID, ovl)
    rq = dict(rope, rope_row=16, k_out=20480, v_out=24576)
    assert call_xy(G(**dict(rq, k_out=4096 + 64)), 64, 64, 4096, 16384) == \
        (_lib.LC_ERR_INVALID, ovl)
    assert call_xy(G(**dict(rq, v_out=4096 - 30)), 64, 64, 4096, 16384) == \
        (_lib.LC_ERR_INVALID, ovl)
    assert call_xy(G(**rq), 64, 64, 4096, 4096 - 62) == (_lib.LC_ERR_INVALID, ovl)


def test_decode_workspace_checks(lib):
    """lc_attn_decode rejects a short or misaligned workspace before any device
    work (the split kernel stores 16-byte vectors of partials)."""
    s = _lib.Shape(1, 1, 4096, 32, 8, 128, _lib.LC_DTYPE_BF16, 0)
    mk = _lib.Mask(4095, 0, -1, 1, 0)
    need = lib.lc_attn_decode_workspace_bytes(ctypes.byref(s))
    assert need > 0 and need % 256 == 0
    fake = 1 << 20  # never dereferenced
    rc = lib.lc_attn_decode(ctypes.byref(s), ctypes.byref(mk), fake, fake, fake, fake, fake, fake,
                            fake, need - 256, None)
    assert rc == _lib.LC_ERR_WORKSPACE and "smaller than" in lib.lc_last_error().decode()
    rc = lib.lc_attn_decode(ctypes.byref(s), ctypes.byref(mk), fake, fake, fake, fake, fake, fake,
                            fake + 8, need, None)
    assert rc == _lib.LC_ERR_INVALID
    assert lib.lc_last_error().decode() == "decode workspace must be 16-byte aligned"


def test_rmsnorm_residual_out_stride_checked(lib):
    """residual_out has its own row stride (ABI version 2), validated like the others."""
    fake = 1 << 20
    rc = lib.lc_rmsnorm(_lib.LC_DTYPE_BF16, 4, 64, 1e-5, fake, 64, fake, 64, fake, 60, fake,
                        fake, 64, None)
    assert rc == _lib.LC_ERR_INVALID
    assert lib.lc_last_error().decode() == "row strides must be >= cols and multiples of 8 elements"


def test_python_signature_argument_checks():
    """ring_causal_attention(q, k, v, *, group, ...) checks its arguments as the
    reference does (src/longctx100m/ring_attention.py:78-101), before any device
    work; this backend has no CPU kernels, so CPU tensors are refused."""
    import torch

    from longctx100m_amd import ring_attention as ra

    x = torch.zeros(1, 8, 2, 4)
    with pytest.raises(ValueError, match=re.escape("q, k, v must have shape [batch, tokens, heads, head_dim]")):
        ra.ring_causal_attention(x[0], x, x)
    with pytest.raises(ValueError, match="q, k, v shard shapes must match"):
        ra.ring_causal_attention(x, x[:, :4], x)
    with pytest.raises(ValueError, match="block_q and block_k must be positive"):
        ra.ring_causal_attention(x, x, x, block_q=0)
    with pytest.raises(ValueError, match="requires CUDA"):
        ra.ring_causal_attention(x, x, x)
