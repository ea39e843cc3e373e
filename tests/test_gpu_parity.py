"""GPU parity: the HIP kernels, called through the C ABI, against the oracle.

Bars (BASELINE config notes): fp32 path within 1e-5 and bf16 path within
2e-2, both norm-relative (max|a-b| / max|b|).  bf16 references are computed
in fp32/fp64 on the bf16-rounded inputs, with the forward output rounded to
bf16 before it enters delta, the reference's bf16 rule
(src/longctx100m/ring_attention.py:17,28,151,314).
"""

import zlib

import numpy as np
import pytest

from oracle import dense, ring
from tests.conftest import norm_rel

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
FP32_TOL = 1e-5


@pytest.fixture(scope="module")
def ra(gpu):
    from longctx100m_amd import ring_attention

    return ring_attention


def _t(gpu, arr, dtype):
    return gpu.tensor(np.ascontiguousarray(arr), dtype=gpu.float32).to(dtype).cuda()


def _np(t):
    return t.detach().float().cpu().numpy()


def _rand_shards(gpu, rng, world, n, hq, hkv, d, dtype, b=1):
    qs, ks, vs = [], [], []
    for _ in range(world):
        qs.append(_t(gpu, rng.standard_normal((b, n, hq, d)), dtype))
        ks.append(_t(gpu, rng.standard_normal((b, n, hkv, d)), dtype))
        vs.append(_t(gpu, rng.standard_normal((b, n, hkv, d)), dtype))
    return qs, ks, vs


# ------------------------------------------------------------- per-hop kernels --

FWD_CASES = [
    # nq, nk, hq, hkv, d, q_pos0, k_pos0, causal, valid
    (256, 256, 2, 2, 128, 0, 0, True, None),      # diagonal block
    (300, 200, 4, 2, 128, 500, 100, True, None),  # tails, GQA, offsets
    (200, 333, 2, 1, 64, 100, 0, True, 250),      # d=64, valid_length
    (128, 192, 2, 2, 128, 0, 0, False, None),     # non-causal
    (96, 64, 3, 1, 128, 0, 64, True, None),       # partly fully-masked rows
    (64, 64, 1, 1, 128, 0, 64, True, None),       # keys after every query
    # full hops (every key before every query) run the 256-query workgroups
    (520, 300, 2, 2, 128, 1000, 0, True, 250),    # valid_length inside the shard, 3 tiles
    (257, 129, 8, 2, 128, 0, 0, False, 100),      # GQA 4, non-causal, one-row tail tile
]


@pytest.mark.parametrize("precise", [False, True])
@pytest.mark.parametrize("case", FWD_CASES)
def test_fwd_shard_bf16(ra, gpu, case, precise):
    nq, nk, hq, hkv, d, qp, kp, causal, valid = case
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    q = _t(gpu, rng.standard_normal((1, nq, hq, d)), gpu.bfloat16)
    k = _t(gpu, rng.standard_normal((1, nk, hkv, d)), gpu.bfloat16)
    v = _t(gpu, rng.standard_normal((1, nk, hkv, d)), gpu.bfloat16)
    o, m, l = ra.fwd_shard(q, k, v, q_pos0=qp, k_pos0=kp, causal=causal, valid_length=valid,
                           precise=precise)
    gpu.cuda.synchronize()
    eo, em, el = dense.attention_fwd(_np(q), _np(k), _np(v), causal=causal, valid_length=valid,
                                     q_pos0=qp, k_pos0=kp)
    tol = FP32_TOL if precise else BF16_TOL
    assert norm_rel(_np(o), eo) <= tol
    m, l = _np(m), _np(l)
    fin = np.isfinite(em)
    assert np.array_equal(np.isfinite(m), fin)
    if fin.any():
        assert np.abs(m[fin] - em[fin]).max() <= 1e-4 * max(1.0, np.abs(em[fin]).max())
        assert norm_rel(l, el) <= 1e-4
    assert np.all(l[~fin] == 0) and np.all(_np(o)[:, ~fin[0].T] == 0)


LONG_KEY_CASES = [
    # b, nq, nk, hq, hkv, q_pos0, causal, valid
    (2, 64, 66000, 2, 1, 65950, True, None),      # two sub-shards, batch stride, GQA
    (1, 64, 140000, 1, 1, 139950, True, 70000),   # valid_length in sub-shard 2, sub-shard 3 skipped
    (1, 64, 70000, 2, 2, 0, False, None),         # non-causal
    (1, 64, 70000, 1, 1, 30, True, None),         # sub-shard 2 masked for every query
    (1, 256, 66000, 2, 2, 65800, True, None),     # diagonal inside the second sub-shard
]


@pytest.mark.parametrize("case", LONG_KEY_CASES)
def test_fwd_shard_long_keys(ra, gpu, case):
    """A shard of more than 65,536 keys runs as key sub-shards whose results the
    kernel epilogue LSE-merges into the running state; same bars as above."""
    b, nq, nk, hq, hkv, qp, causal, valid = case
    d = 128
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    q = _t(gpu, rng.standard_normal((b, nq, hq, d)), gpu.bfloat16)
    k = _t(gpu, rng.standard_normal((b, nk, hkv, d)), gpu.bfloat16)
    v = _t(gpu, rng.standard_normal((b, nk, hkv, d)), gpu.bfloat16)
    o, m, l = ra.fwd_shard(q, k, v, q_pos0=qp, k_pos0=0, causal=causal, valid_length=valid)
    gpu.cuda.synchronize()
    eo, em, el = dense.attention_fwd(_np(q), _np(k), _np(v), causal=causal, valid_length=valid,
                                     q_pos0=qp, k_pos0=0)
    assert norm_rel(_np(o), eo) <= BF16_TOL
    m, l = _np(m), _np(l)
    fin = np.isfinite(em)
    assert np.array_equal(np.isfinite(m), fin)
    assert np.abs(m[fin] - em[fin]).max() <= 1e-4 * max(1.0, np.abs(em[fin]).max())
    assert norm_rel(l[fin], el[fin]) <= 1e-4


@pytest.mark.parametrize("case", FWD_CASES[:4])
def test_fwd_shard_fp32(ra, gpu, case):
    nq, nk, hq, hkv, d, qp, kp, causal, valid = case
    rng = np.random.default_rng(7 + nq)
    q = _t(gpu, rng.standard_normal((1, nq, hq, d)), gpu.float32)
    k = _t(gpu, rng.standard_normal((1, nk, hkv, d)), gpu.float32)
    v = _t(gpu, rng.standard_normal((1, nk, hkv, d)), gpu.float32)
    o, m, l = ra.fwd_shard(q, k, v, q_pos0=qp, k_pos0=kp, causal=causal, valid_length=valid)
    gpu.cuda.synchronize()
    eo, em, el = dense.attention_fwd(_np(q), _np(k), _np(v), causal=causal, valid_length=valid,
                                     q_pos0=qp, k_pos0=kp)
    assert norm_rel(_np(o), eo) <= FP32_TOL
    assert np.abs(_np(m) - em).max() <= 1e-5 * max(1.0, np.abs(em).max())
    assert norm_rel(_np(l), el) <= FP32_TOL


BWD_CASES = [
    (256, 256, 2, 2, 128, 0, 0, True, None),
    (300, 200, 4, 2, 128, 500, 100, True, None),
    (200, 333, 2, 1, 64, 100, 0, True, 250),
    (160, 130, 4, 1, 128, 0, 0, False, None),
]


@pytest.mark.parametrize("dtype_name,precise", [("bfloat16", False), ("bfloat16", True),
                                                ("float32", False)])
@pytest.mark.parametrize("case", BWD_CASES)
def test_bwd_shard(ra, gpu, case, dtype_name, precise):
    nq, nk, hq, hkv, d, qp, kp, causal, valid = case
    dtype = getattr(gpu, dtype_name)
    rng = np.random.default_rng(31 + nq + nk)
    q = _t(gpu, rng.standard_normal((1, nq, hq, d)), dtype)
    k = _t(gpu, rng.standard_normal((1, nk, hkv, d)), dtype)
    v = _t(gpu, rng.standard_normal((1, nk, hkv, d)), dtype)
    do = _t(gpu, rng.standard_normal((1, nq, hq, d)), dtype)
    kw = dict(q_pos0=qp, k_pos0=kp, causal=causal, valid_length=valid)
    o32, m, l = ra.fwd_shard(q, k, v, precise=precise, **kw)
    out = o32.to(dtype)
    delta, lse2 = ra.bwd_preprocess(out, do, m, l)
    dq = gpu.zeros((1, nq, hq, d), dtype=gpu.float32, device="cuda")
    dk = gpu.zeros((1, nk, hkv, d), dtype=gpu.float32, device="cuda")
    dv = gpu.zeros_like(dk)
    ra.bwd_shard(q, k, v, do, lse2, delta, dq_acc=dq, dk_acc=dk, dv_acc=dv, precise=precise, **kw)
    gpu.cuda.synchronize()
    edq, edk, edv = dense.attention_bwd(_np(q), _np(k), _np(v), _np(do), out=_np(out), **kw)
    tol = FP32_TOL if (dtype_name == "float32" or precise) else BF16_TOL
    assert norm_rel(_np(dq), edq) <= tol
    assert norm_rel(_np(dk), edk) <= tol
    assert norm_rel(_np(dv), edv) <= tol


FP32_LONG_CASES = [
    # nq, nk, hq, hkv, d, q_pos0, k_pos0, causal: longer fp32 reductions (dQ over up to
    # 8192 keys, dK/dV over up to 4096 queries x a GQA group of 2)
    (128, 8192, 2, 2, 64, 8100, 0, True),
    (4096, 256, 2, 1, 128, 0, 0, False),
    (1024, 1536, 2, 1, 96, 600, 0, True),
]


@pytest.mark.parametrize("case", FP32_LONG_CASES)
def test_bwd_shard_fp32_long(ra, gpu, case):
    """The fp32 path keeps the 1e-5 bar as the reductions grow (the generic
    kernels' fp32 sums stay near 1e-6 of the fp64 dense closed form)."""
    nq, nk, hq, hkv, d, qp, kp, causal = case
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    f32 = gpu.float32
    q = _t(gpu, rng.standard_normal((1, nq, hq, d)), f32)
    k = _t(gpu, rng.standard_normal((1, nk, hkv, d)), f32)
    v = _t(gpu, rng.standard_normal((1, nk, hkv, d)), f32)
    do = _t(gpu, rng.standard_normal((1, nq, hq, d)), f32)
    kw = dict(q_pos0=qp, k_pos0=kp, causal=causal)
    out, m, l = ra.fwd_shard(q, k, v, **kw)
    delta, lse2 = ra.bwd_preprocess(out, do, m, l)
    dq = gpu.zeros((1, nq, hq, d), dtype=f32, device="cuda")
    dk = gpu.zeros((1, nk, hkv, d), dtype=f32, device="cuda")
    dv = gpu.zeros_like(dk)
    ra.bwd_shard(q, k, v, do, lse2, delta, dq_acc=dq, dk_acc=dk, dv_acc=dv, **kw)
    gpu.cuda.synchronize()
    eo = dense.attention_fwd(_np(q), _np(k), _np(v), **kw)[0]
    edq, edk, edv = dense.attention_bwd(_np(q), _np(k), _np(v), _np(do), out=_np(out), **kw)
    errs = [norm_rel(_np(out), eo), norm_rel(_np(dq), edq), norm_rel(_np(dk), edk),
            norm_rel(_np(dv), edv)]
    assert max(errs) <= FP32_TOL, errs


@pytest.mark.parametrize("dtype_name,b,n,h,d", [("bfloat16", 2, 300, 3, 128), ("float32", 1, 77, 2, 64),
                                                ("bfloat16", 1, 50, 4, 36), ("float32", 1, 33, 1, 30)])
def test_bwd_preprocess(ra, gpu, dtype_name, b, n, h, d):
    """delta = rowsum(dO * O) in fp32 from the given dtype and lse2 = m log2(e) +
    log2(max(l, FLT_MIN)), +inf for rows without a key (ring_attention.py:314,
    rs:382; the 16-byte-load path for d*size % 16 == 0, the scalar path else)."""
    dtype = getattr(gpu, dtype_name)
    rng = np.random.default_rng(zlib.crc32(repr((dtype_name, b, n, h, d)).encode()))
    out = _t(gpu, rng.standard_normal((b, n, h, d)), dtype)
    do = _t(gpu, rng.standard_normal((b, n, h, d)), dtype)
    m = rng.standard_normal((b, h, n)).astype(np.float32)
    l = (1 + 50 * rng.random((b, h, n))).astype(np.float32)
    m[0, 0, :3] = -np.inf
    l[0, 0, :3] = 0.0
    l[0, -1, 5] = 0.0  # clamped to FLT_MIN
    delta, lse2 = ra.bwd_preprocess(out, do, _t(gpu, m, gpu.float32), _t(gpu, l, gpu.float32))
    gpu.cuda.synchronize()
    want = np.einsum("bnhd,bnhd->bhn", _np(out).astype(np.float64), _np(do).astype(np.float64))
    assert norm_rel(_np(delta), want) <= 1e-6
    fin = np.isfinite(m)
    wl = m.astype(np.float64) * np.log2(np.e) + np.log2(np.maximum(l, 1.17549435e-38))
    got = _np(lse2)
    assert np.all(np.isposinf(got[~fin]))
    assert np.abs(got[fin] - wl[fin]).max() <= 2e-6 * max(1.0, np.abs(wl[fin]).max())


LONG_BWD_CASES = [
    # b, nq, nk, hq, hkv, q_pos0, k_pos0, causal
    (2, 32, 70000, 1, 1, 69980, 0, True),       # dQ over key sub-shards, batch stride
    (1, 70000, 64, 2, 2, 0, 0, True),           # dK/dV over query sub-shards
    (1, 70000, 64, 1, 1, 0, 65600, True),       # first query sub-shard sees no key (skipped)
    (2, 66000, 32, 2, 1, 0, 0, False),          # dK/dV sub-shards, GQA group walk, batch stride
]


@pytest.mark.parametrize("case", LONG_BWD_CASES)
def test_bwd_shard_long_stream(ra, gpu, case):
    """More than 65,536 streamed rows (keys for dQ, queries for dK/dV) run as
    sub-shards accumulating into the same gradients; bf16 bar as above."""
    b, nq, nk, hq, hkv, qp, kp, causal = case
    d = 128
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    q = _t(gpu, rng.standard_normal((b, nq, hq, d)), gpu.bfloat16)
    k = _t(gpu, rng.standard_normal((b, nk, hkv, d)), gpu.bfloat16)
    v = _t(gpu, rng.standard_normal((b, nk, hkv, d)), gpu.bfloat16)
    do = _t(gpu, rng.standard_normal((b, nq, hq, d)), gpu.bfloat16)
    kw = dict(q_pos0=qp, k_pos0=kp, causal=causal)
    o32, m, l = ra.fwd_shard(q, k, v, **kw)
    out = o32.to(gpu.bfloat16)
    delta, lse2 = ra.bwd_preprocess(out, do, m, l)
    dq = gpu.zeros((b, nq, hq, d), dtype=gpu.float32, device="cuda")
    dk = gpu.zeros((b, nk, hkv, d), dtype=gpu.float32, device="cuda")
    dv = gpu.zeros_like(dk)
    ra.bwd_shard(q, k, v, do, lse2, delta, dq_acc=dq, dk_acc=dk, dv_acc=dv, **kw)
    gpu.cuda.synchronize()
    edq, edk, edv = dense.attention_bwd(_np(q), _np(k), _np(v), _np(do), out=_np(out), **kw)
    assert norm_rel(_np(dq), edq) <= BF16_TOL
    assert norm_rel(_np(dk), edk) <= BF16_TOL
    assert norm_rel(_np(dv), edv) <= BF16_TOL


DS_CASES = [
    # b, nq, nk, hq, hkv, q_pos0, k_pos0, causal, valid, workspace fraction
    (1, 256, 256, 2, 2, 0, 0, True, None, 1.0),       # diagonal block
    (1, 300, 200, 4, 2, 500, 100, True, None, 1.0),   # tails, GQA, offsets
    (2, 200, 333, 2, 1, 100, 0, True, 250, 1.0),      # batch, valid_length, odd key blocks
    (1, 160, 130, 4, 1, 0, 0, False, None, 1.0),      # non-causal, partial last key block
    (1, 96, 64, 3, 1, 0, 64, True, None, 1.0),        # rows that see no key
    (1, 700, 500, 2, 2, 0, 0, True, None, 0.4),       # query chunks of 256 rows
    (1, 256, 256, 1, 1, 0, 0, True, None, 0.01),      # no usable workspace: recompute path
    (2, 32, 70000, 1, 1, 69980, 0, True, None, 1.0),  # dQ over key sub-shards of the blocks
    (1, 70000, 64, 2, 2, 0, 0, True, None, 1.0),      # query chunks of 65,536 rows
    (2, 600, 450, 8, 2, 1000, 900, True, 1300, 0.5),  # batch, GQA 4, offsets, valid_length, chunks
    (1, 300, 70000, 2, 1, 69800, 0, True, None, 1.0),  # GQA with dQ over key sub-shards
]


@pytest.mark.parametrize("case", DS_CASES)
def test_bwd_shard_shared_ds(ra, gpu, case):
    """dS sharing (dK/dV stores dS, dQ reads it back): against the oracle at
    the bf16 bar, dK/dV bit-identical to the recomputing path (same kernel,
    plus stores) unless the workspace splits the queries into more chunks, dQ
    equal to it up to the rounding of dS."""
    b, nq, nk, hq, hkv, qp, kp, causal, valid, frac = case
    d = 128
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    q = _t(gpu, rng.standard_normal((b, nq, hq, d)), gpu.bfloat16)
    k = _t(gpu, rng.standard_normal((b, nk, hkv, d)), gpu.bfloat16)
    v = _t(gpu, rng.standard_normal((b, nk, hkv, d)), gpu.bfloat16)
    do = _t(gpu, rng.standard_normal((b, nq, hq, d)), gpu.bfloat16)
    kw = dict(q_pos0=qp, k_pos0=kp, causal=causal, valid_length=valid)
    o32, m, l = ra.fwd_shard(q, k, v, **kw)
    out = o32.to(gpu.bfloat16)
    delta, lse2 = ra.bwd_preprocess(out, do, m, l)
    full = ra.bwd_shard_workspace_bytes(q, k)
    assert full == b * hq * -(-min(nq, 65536) // 32) * -(-nk // 32) * 2048
    # stale non-finite bytes: every block the dQ kernel uses must be written first
    ws = gpu.full((max(256, int(full * frac)) // 2,), float("nan"), dtype=gpu.bfloat16,
                  device="cuda")
    grads = []
    for w in (ws, None):
        dq = gpu.zeros((b, nq, hq, d), dtype=gpu.float32, device="cuda")
        dk = gpu.zeros((b, nk, hkv, d), dtype=gpu.float32, device="cuda")
        dv = gpu.zeros_like(dk)
        ra.bwd_shard(q, k, v, do, lse2, delta, dq_acc=dq, dk_acc=dk, dv_acc=dv, workspace=w, **kw)
        grads.append((_np(dq), _np(dk), _np(dv)))
    gpu.cuda.synchronize()
    # the dS path ran (it overwrote part of the NaN workspace) exactly when the workspace
    # holds 256 query rows or the whole shard; the 1% case falls back to recomputing
    per_tile = b * hq * -(-nk // 32) * 2048
    rows = ws.numel() * 2 // per_tile * 32
    assert bool(gpu.isnan(ws).all()) == (rows < 256 and rows < nq)
    (dq, dk, dv), (rdq, rdk, rdv) = grads
    tiles = full // (b * hq * -(-nk // 32) * 2048)  # 32-row query tiles of the full workspace
    chunked = 8 <= int(full * frac) // (full // tiles) < -(-nq // 32)
    if chunked:  # dK/dV summed chunk by chunk: same terms, another fp32 order
        assert norm_rel(dk, rdk) <= 1e-5 and norm_rel(dv, rdv) <= 1e-5
    else:
        assert np.array_equal(dk, rdk) and np.array_equal(dv, rdv)
    assert norm_rel(dq, rdq) <= 4e-3
    edq, edk, edv = dense.attention_bwd(_np(q), _np(k), _np(v), _np(do), out=_np(out), **kw)
    assert norm_rel(dq, edq) <= BF16_TOL
    assert norm_rel(dk, edk) <= BF16_TOL
    assert norm_rel(dv, edv) <= BF16_TOL


@pytest.mark.parametrize("n,offset", [(8 * 40000, 0), (8 * 40000 + 3, 0), (8 * 1000, 1)])
def test_cast_rounds_to_nearest_even(ra, gpu, n, offset):
    """lc_attn_cast to bf16 (the 8-wide kernel for aligned multiples of 8, the
    scalar one otherwise) rounds to nearest even, bit for bit as torch's CPU
    conversion, including ties, subnormals, infinities and NaN."""
    rng = np.random.default_rng(n + offset)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    bits[: n // 4] = (bits[: n // 4] & 0xFFFF0000) | 0x8000  # exact ties
    special = np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001, 0x807FFFFF,
                        0x3F808000, 0x3F818000, 0x7F7FFFFF], dtype=np.uint32)
    bits[-len(special):] = special
    src_cpu = gpu.from_numpy(bits.view(np.float32).copy())
    src = src_cpu.cuda()
    dst_full = gpu.empty(n + offset, dtype=gpu.bfloat16, device="cuda")
    dst = dst_full[offset:]
    ra.cast(src, dst)
    gpu.cuda.synchronize()
    got = dst.cpu().view(gpu.int16).numpy()
    exp_t = src_cpu.to(gpu.bfloat16)
    exp = exp_t.view(gpu.int16).numpy()
    nan = np.isnan(src_cpu.numpy())
    assert np.array_equal(got[~nan], exp[~nan])
    assert np.isnan(dst.cpu().float().numpy()[nan]).all()


def test_merge_is_order_invariant(ra, gpu):
    rng = np.random.default_rng(5)
    nq, hq, d = 192, 2, 128
    q = _t(gpu, rng.standard_normal((1, nq, hq, d)), gpu.bfloat16)
    kv = [(_t(gpu, rng.standard_normal((1, 100, hq, d)), gpu.bfloat16),
           _t(gpu, rng.standard_normal((1, 100, hq, d)), gpu.bfloat16)) for _ in range(3)]
    parts = [ra.fwd_shard(q, k, v, q_pos0=300, k_pos0=100 * i) for i, (k, v) in enumerate(kv)]
    results = []
    for order in ([0, 1, 2], [2, 0, 1], [1, 2, 0]):
        o, m, l = (x.clone() for x in parts[order[0]])
        for j in order[1:]:
            ra.merge(o, m, l, *parts[j])
        results.append((_np(o), _np(m), _np(l)))
    k_all = np.concatenate([_np(k) for k, _ in kv], axis=1)
    v_all = np.concatenate([_np(v) for _, v in kv], axis=1)
    eo, em, el = dense.attention_fwd(_np(q), k_all, v_all, q_pos0=300, k_pos0=0)
    for o, m, l in results:
        assert norm_rel(o, eo) <= BF16_TOL
        assert np.abs(m - em).max() <= 1e-4 * np.abs(em).max()
        assert norm_rel(l, el) <= 1e-4
    for o, m, l in results[1:]:
        assert norm_rel(o, results[0][0]) <= 1e-5


ACC_CASES = [
    # b, nq, nk_a, nk_b, hq, hkv, d, dtype, precise, q_pos0, shift, valid: hop A holds
    # the keys from q_pos0 + shift on, hop B the nk_b keys just before them
    (1, 300, 300, 300, 4, 2, 128, "bfloat16", False, 600, 0, None),   # diagonal, then full hop
    (1, 520, 300, 260, 2, 2, 128, "bfloat16", False, 1000, 0, 1100),  # 8-wave hop, valid_length
    (2, 200, 160, 130, 8, 2, 128, "bfloat16", False, 500, 100, None),  # rows with no key in A
    (1, 96, 64, 64, 2, 1, 128, "bfloat16", False, 0, 64, None),       # no A key for rows < 64
    (1, 200, 200, 150, 2, 1, 64, "bfloat16", False, 300, 0, 320),     # d=64 kernel
    (1, 150, 100, 90, 3, 1, 128, "float32", False, 200, 0, None),     # fp32 kernel
    (1, 130, 70, 80, 2, 2, 40, "float32", False, 100, 0, None),       # fp32, d=40
    (1, 120, 100, 100, 2, 1, 128, "bfloat16", True, 150, 0, 180),     # bf16 inputs, fp32 math
    (1, 48, 64, 70000, 1, 1, 128, "bfloat16", False, 70000, 0, None),  # B over key sub-shards
]


@pytest.mark.parametrize("case", ACC_CASES)
def test_fwd_accumulate_matches_separate_merge(ra, gpu, case):
    """LC_FLAG_ACCUMULATE: hop B merged into hop A's state in the forward's
    epilogue equals hop B into its own buffers followed by lc_attn_merge (m and
    l bit for bit, o to fp32 rounding; a hop of key sub-shards merges them one
    by one into A's state instead of into each other first, so l then agrees
    to fp32 rounding), and both equal the fp64 dense oracle over the union of
    the two hops' keys."""
    b, nq, nka, nkb, hq, hkv, d, dt, precise, qp, shift, valid = case
    dtype = getattr(gpu, dt)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    q = _t(gpu, rng.standard_normal((b, nq, hq, d)), dtype)
    ka, va, kb, vb = (_t(gpu, rng.standard_normal((b, n, hkv, d)), dtype)
                      for n in (nka, nka, nkb, nkb))
    kpa = qp + shift  # hop A's first key position
    kpb = kpa - nkb
    kw = dict(valid_length=valid, precise=precise)
    o_a, m_a, l_a = ra.fwd_shard(q, ka, va, q_pos0=qp, k_pos0=kpa, **kw)
    o_b, m_b, l_b = ra.fwd_shard(q, kb, vb, q_pos0=qp, k_pos0=kpb, **kw)
    sep = [x.clone() for x in (o_a, m_a, l_a)]
    ra.merge(*sep, o_b, m_b, l_b)
    acc = [x.clone() for x in (o_a, m_a, l_a)]
    ra.fwd_shard(q, kb, vb, q_pos0=qp, k_pos0=kpb, o=acc[0], m=acc[1], l=acc[2],
                 accumulate=True, **kw)
    gpu.cuda.synchronize()
    (so, sm, sl), (ao, am, al) = ([_np(x) for x in t] for t in (sep, acc))
    assert np.array_equal(am, sm)
    if nkb <= 65536:
        assert np.array_equal(al, sl)
    else:
        assert np.abs(al - sl).max() <= 1e-6 * np.abs(sl).max()
    assert np.abs(ao - so).max() <= 1e-6 * max(np.abs(so).max(), 1e-30)
    kcat = np.concatenate([_np(kb), _np(ka)], axis=1)
    vcat = np.concatenate([_np(vb), _np(va)], axis=1)
    eo, em, el = dense.attention_fwd(_np(q), kcat, vcat, q_pos0=qp, k_pos0=kpb,
                                     valid_length=valid)
    tol = FP32_TOL if (dt == "float32" or precise) else BF16_TOL
    assert norm_rel(ao, eo) <= tol
    fin = np.isfinite(em)
    assert np.array_equal(np.isfinite(am), fin)
    assert np.abs(am[fin] - em[fin]).max() <= 1e-4 * max(np.abs(em[fin]).max(), 1.0)
    assert norm_rel(al, el) <= 1e-4


def test_rank_step_merge_forms_agree(ra, gpu):
    """The benched step's forward with the epilogue merge and with a separate
    lc_attn_merge per hop (bench.py --separate-merge): the same m and l bit for
    bit, the bf16 output to its rounding, and both at the bf16 bar of the dense
    oracle over the whole visible sequence."""
    from longctx100m_amd.rank_step import RankStep

    rng = np.random.default_rng(23)
    world, rank, n, h, d = 4, 3, 300, 2, 128
    q = _t(gpu, rng.standard_normal((1, n, h, d)), gpu.bfloat16)
    do = _t(gpu, rng.standard_normal((1, n, h, d)), gpu.bfloat16)
    ks = [_t(gpu, rng.standard_normal((1, n, h, d)), gpu.bfloat16) for _ in range(world)]
    vs = [_t(gpu, rng.standard_normal((1, n, h, d)), gpu.bfloat16) for _ in range(world)]
    res = []
    for sep in (False, True):
        rs = RankStep(q, do, ks, vs, rank, share_ds=False, separate_merge=sep)
        rs.forward()
        gpu.cuda.synchronize()
        res.append((_np(rs.out), _np(rs.m), _np(rs.l)))
    (fo, fm, fl), (so, sm, sl) = res
    assert np.array_equal(fm, sm) and np.array_equal(fl, sl)
    assert norm_rel(fo, so) <= 8e-3
    kcat = np.concatenate([_np(x) for x in ks], axis=1)
    vcat = np.concatenate([_np(x) for x in vs], axis=1)
    eo, em, el = dense.attention_fwd(_np(q), kcat, vcat, q_pos0=rank * n, k_pos0=0)
    for o in (fo, so):
        assert norm_rel(o, eo) <= BF16_TOL
    assert norm_rel(fl, el) <= 1e-4


def test_wrappers_reject_mis_sized_buffers(ra, gpu):
    """The kernels take raw pointers, so the Python mirror checks every
    caller-supplied output or state buffer before a launch could write past it."""
    bf, f32 = gpu.bfloat16, gpu.float32
    q = gpu.zeros((1, 64, 4, 128), dtype=bf, device="cuda")
    k = gpu.zeros((1, 80, 2, 128), dtype=bf, device="cuda")
    good_o = gpu.zeros((1, 64, 4, 128), dtype=f32, device="cuda")
    stats = gpu.zeros((1, 4, 64), dtype=f32, device="cuda")
    with pytest.raises(ValueError, match="o must be"):
        ra.fwd_shard(q, k, k, q_pos0=0, k_pos0=0, o=good_o[:, :32], m=stats, l=stats)
    with pytest.raises(ValueError, match="m must be"):
        ra.fwd_shard(q, k, k, q_pos0=0, k_pos0=0, o=good_o, m=stats[:, :2], l=stats,
                     accumulate=True)
    with pytest.raises(ValueError, match="accumulate needs"):
        ra.fwd_shard(q, k, k, q_pos0=0, k_pos0=0, accumulate=True)
    with pytest.raises(ValueError, match="dk_acc must be"):
        ra.bwd_shard(q, k, k, q, stats, stats, q_pos0=0, k_pos0=0, dq_acc=good_o,
                     dk_acc=gpu.zeros((1, 64, 2, 128), dtype=f32, device="cuda"),
                     dv_acc=gpu.zeros((1, 80, 2, 128), dtype=f32, device="cuda"))
    with pytest.raises(ValueError, match="o_part must be"):
        ra.merge(good_o, stats, stats, good_o.to(bf), stats, stats)
    gpu.cuda.synchronize()


def test_fwd_accumulate_masked_pair_keeps_state(ra, gpu):
    """A hop with no unmasked pair leaves an accumulated state as it is (the
    reference's alpha = 1, p = 0), where a write would reset it."""
    rng = np.random.default_rng(11)
    q = _t(gpu, rng.standard_normal((1, 64, 2, 128)), gpu.bfloat16)
    k, v = (_t(gpu, rng.standard_normal((1, 64, 2, 128)), gpu.bfloat16) for _ in range(2))
    o, m, l = ra.fwd_shard(q, k, v, q_pos0=100, k_pos0=0)
    before = [_np(x) for x in (o, m, l)]
    ra.fwd_shard(q, k, v, q_pos0=100, k_pos0=500, o=o, m=m, l=l, accumulate=True)  # keys after
    gpu.cuda.synchronize()
    for x, y in zip(before, (o, m, l)):
        assert np.array_equal(x, _np(y))


# ------------------------------------------------------------------ whole ring --

def _oracle_ring(qs, ks, vs, world, hq, hkv, rank=None, gos=None, **kw):
    """C-restatement results on the (rounded) inputs, KV heads expanded by
    repeat_interleave as the reference's callers do; returns per-rank
    (out, m, l) and, if gos is given, rank's (dq, dk, dv) with dk/dv summed
    over each GQA group."""
    g = hq // hkv
    qn = [_np(x) for x in qs]
    kn = [np.repeat(_np(x), g, axis=2) for x in ks]
    vn = [np.repeat(_np(x), g, axis=2) for x in vs]
    fw = [ring.ring_fwd_with_stats(qn, kn, vn, r, **kw) for r in range(world)]
    if gos is None:
        return fw, None
    dtype_round = qs[0].dtype
    import torch

    outs = [torch.tensor(o).to(dtype_round).float().numpy() for o, _, _ in fw]
    dq, dk, dv = ring.ring_bwd(qn, kn, vn, outs, [x[1] for x in fw], [x[2] for x in fw],
                               [_np(x) for x in gos], rank, **kw)
    b, n, _, d = dk.shape
    return fw, (dq, dk.reshape(b, n, hkv, g, d).sum(3), dv.reshape(b, n, hkv, g, d).sum(3))


@pytest.mark.parametrize("dtype_name", ["float32", "bfloat16"])
def test_ring_config1(ra, gpu, dtype_name):
    """world 2 x 512 tokens, Hq=9, Hkv=3 (GQA), d=64."""
    dtype = getattr(gpu, dtype_name)
    tol = FP32_TOL if dtype_name == "float32" else BF16_TOL
    rng = np.random.default_rng(1)
    world, n, hq, hkv, d = 2, 512, 9, 3, 64
    qs, ks, vs = _rand_shards(gpu, rng, world, n, hq, hkv, d, dtype)
    gos = [_t(gpu, rng.standard_normal((1, n, hq, d)), dtype) for _ in range(world)]
    shards = list(zip(qs, ks, vs))
    outs, ms, ls = [], [], []
    for r in range(world):
        o, m, l = ra.ring_causal_attention_forward_with_stats(shards, r)
        outs.append(o)
        ms.append(m)
        ls.append(l)
    gpu.cuda.synchronize()
    for r in range(world):
        fw, grads = _oracle_ring(qs, ks, vs, world, hq, hkv, rank=r, gos=gos)
        eo, em, el = fw[r]
        assert norm_rel(_np(outs[r]), eo) <= tol
        assert np.abs(_np(ms[r])[..., 0] - em).max() <= 1e-4 * np.abs(em).max()
        assert norm_rel(_np(ls[r])[..., 0], el) <= 1e-4
        dq, dk, dv = ra.ring_causal_attention_backward(shards, r, outs, ms, ls, gos)
        gpu.cuda.synchronize()
        for a, b in zip((dq, dk, dv), grads):
            assert norm_rel(_np(a), b) <= tol


def _random_rings(seed, n):
    """Random ring geometries (drawn once): world, rank, shard length, heads, d,
    dtype, causal, valid_length, q_position_start."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        world = int(rng.integers(1, 5))
        tokens = int(rng.integers(1, 261))
        dt = str(rng.choice(["float32", "bfloat16"]))
        hkv = int(rng.integers(1, 3))
        valid = None if rng.integers(0, 2) else int(rng.integers(1, world * tokens + 1))
        qps = None if rng.integers(0, 3) else int(rng.integers(0, world * tokens))
        out.append(dict(world=world, rank=int(rng.integers(0, world)), n=tokens, hkv=hkv,
                        hq=hkv * int(rng.integers(1, 4)), dtype=dt,
                        d=int(rng.choice([64, 128] if dt == "bfloat16" else [40, 64, 128])),
                        causal=bool(rng.integers(0, 4)), valid_length=valid,
                        q_position_start=qps))
    return out


@pytest.mark.parametrize("case", _random_rings(2027, 32),
                         ids=lambda c: "w{world}r{rank}n{n}h{hq}/{hkv}d{d}-{dtype}".format(**c))
def test_random_rings_against_the_c_restatement(ra, gpu, case):
    """Whole-ring forward and backward of one rank through the C ABI (the
    reference's signatures) against the C restatement of rs:139-475 on the same
    inputs, at the fp32 / bf16 bars: random world sizes, ranks, shard lengths
    that are not multiples of any tile, GQA, head dims, causal or not,
    valid_length and q_position_start."""
    c = dict(case)
    dtype = getattr(gpu, c["dtype"])
    tol = FP32_TOL if c["dtype"] == "float32" else BF16_TOL
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    world, rank, n, hq, hkv, d = c["world"], c["rank"], c["n"], c["hq"], c["hkv"], c["d"]
    kw = dict(causal=c["causal"], valid_length=c["valid_length"],
              q_position_start=c["q_position_start"])
    qs, ks, vs = _rand_shards(gpu, rng, world, n, hq, hkv, d, dtype)
    gos = [_t(gpu, rng.standard_normal((1, n, hq, d)), dtype) for _ in range(world)]
    shards = list(zip(qs, ks, vs))
    fw = [ra.ring_causal_attention_forward_with_stats(shards, r, c["causal"], 64, 128,
                                                      c["valid_length"], c["q_position_start"])
          for r in range(world)]
    outs, ms, ls = (list(x) for x in zip(*fw))
    dq, dk, dv = ra.ring_causal_attention_backward(shards, rank, outs, ms, ls, gos, c["causal"],
                                                   64, 128, c["valid_length"],
                                                   c["q_position_start"])
    gpu.cuda.synchronize()
    efw, egrads = _oracle_ring(qs, ks, vs, world, hq, hkv, rank=rank, gos=gos, **kw)
    eo, em, el = efw[rank]
    assert norm_rel(_np(outs[rank]), eo) <= tol
    m, l = _np(ms[rank])[..., 0], _np(ls[rank])[..., 0]
    fin = np.isfinite(em)
    assert np.array_equal(np.isfinite(m), fin)
    if fin.any():
        assert np.abs(m[fin] - em[fin]).max() <= 1e-4 * max(np.abs(em[fin]).max(), 1.0)
        assert norm_rel(l, el) <= 1e-4
    for a, e in zip((dq, dk, dv), egrads):
        assert norm_rel(_np(a), e) <= tol


def test_reference_unit_cases_on_gpu(ra, gpu):
    """The reference's Rust unit tests (ring_attention.rs:519-668) through
    the HIP path, fp32, same shapes, blocks and tolerances."""
    f32 = gpu.float32
    rng = np.random.default_rng(0)
    q, k, v = (_t(gpu, rng.standard_normal((1, 8, 2, 4)), f32) for _ in range(3))
    out = ra.ring_causal_attention_forward([(q, k, v)], 0, True, 2, 3, None, None)
    exp = dense.attention_fwd(_np(q), _np(k), _np(v))[0]
    assert np.abs(_np(out) - exp).max() < 1e-5
    ref = ra.reference_causal_attention(q, k, v)
    assert np.abs(_np(ref) - exp).max() < 1e-5
    for valid in (None, 6):
        qs = [_t(gpu, x, f32) for x in dense.lcg_shards(4, 2, 4, 2)]
        shards = [(x, x, x) for x in qs]
        full = np.concatenate([_np(x) for x in qs], axis=1)
        e = dense.attention_fwd(full, full, full, valid_length=valid)[0]
        for r in range(2):
            o = ra.ring_causal_attention_forward(shards, r, True, 2, 3, valid, None)
            assert np.abs(_np(o) - e[:, 4 * r:4 * r + 4]).max() < 1e-5
    # single-rank backward vs dense autograd, grad_out = ones, abs 1e-4
    out, m, l = ra.ring_causal_attention_forward_with_stats([(q, k, v)], 0, True, 2, 3)
    go = gpu.ones_like(q)
    dq, dk, dv = ra.ring_causal_attention_backward([(q, k, v)], 0, [out], [m], [l], [go], True,
                                                   2, 3)
    edq, edk, edv = dense.attention_bwd(_np(q), _np(k), _np(v), np.ones((1, 8, 2, 4)))
    for a, b in ((dq, edq), (dk, edk), (dv, edv)):
        assert np.abs(_np(a) - b).max() < 1e-4


def test_two_rank_python_case_on_gpu(ra, gpu):
    """tests/test_ring_attention.py:277-321 of the reference: seed 123, T=8
    over 2 ranks, H=2, D=4, blocks 2/2, loss = sum(out): fwd 2e-5, grads 3e-4."""
    import torch

    torch.manual_seed(123)
    q = torch.randn(1, 8, 2, 4)
    k = torch.randn(1, 8, 2, 4)
    v = torch.randn(1, 8, 2, 4)
    shards = [tuple(x[:, 4 * r:4 * r + 4].contiguous().cuda() for x in (q, k, v))
              for r in range(2)]
    stats = [ra.ring_causal_attention_forward_with_stats(shards, r, True, 2, 2) for r in range(2)]
    outs, ms, ls = (list(x) for x in zip(*stats))
    exp = dense.attention_fwd(q.numpy(), k.numpy(), v.numpy())[0]
    edq, edk, edv = dense.attention_bwd(q.numpy(), k.numpy(), v.numpy(), np.ones((1, 8, 2, 4)))
    gos = [gpu.ones_like(o) for o in outs]
    for r in range(2):
        sl = slice(4 * r, 4 * r + 4)
        assert np.abs(_np(outs[r]) - exp[:, sl]).max() < 2e-5
        dq, dk, dv = ra.ring_causal_attention_backward(shards, r, outs, ms, ls, gos, True, 2, 2)
        assert np.abs(_np(dq) - edq[:, sl]).max() < 3e-4
        assert np.abs(_np(dk) - edk[:, sl]).max() < 3e-4
        assert np.abs(_np(dv) - edv[:, sl]).max() < 3e-4


def test_ring_c2_shape_reduced(ra, gpu):
    """Config 2/3 geometry (rank 7 of 8, Hq=Hkv=16, d=128, bf16) at 512
    tokens per shard against the C restatement."""
    rng = np.random.default_rng(2)
    world, n, h, d = 8, 512, 16, 128
    qs, ks, vs = _rand_shards(gpu, rng, world, n, h, h, d, gpu.bfloat16)
    gos = [_t(gpu, rng.standard_normal((1, n, h, d)), gpu.bfloat16) for _ in range(world)]
    shards = list(zip(qs, ks, vs))
    stats = [ra.ring_causal_attention_forward_with_stats(shards, r) for r in range(world)]
    outs, ms, ls = (list(x) for x in zip(*stats))
    fw, grads = _oracle_ring(qs, ks, vs, world, h, h, rank=7, gos=gos)
    assert norm_rel(_np(outs[7]), fw[7][0]) <= BF16_TOL
    dq, dk, dv = ra.ring_causal_attention_backward(shards, 7, outs, ms, ls, gos)
    gpu.cuda.synchronize()
    for a, b in zip((dq, dk, dv), grads):
        assert norm_rel(_np(a), b) <= BF16_TOL


def test_ring_c4_shape_reduced(ra, gpu):
    """The C4 model's attention share (GQA Hq=32 / Hkv=8, d=128, bf16, the
    local shard plus 3 preceding KV shards: rank 3 of a 4-rank ring) at 384
    tokens per shard against the C restatement."""
    rng = np.random.default_rng(4)
    world, n, hq, hkv, d = 4, 384, 32, 8, 128
    qs, ks, vs = _rand_shards(gpu, rng, world, n, hq, hkv, d, gpu.bfloat16)
    gos = [_t(gpu, rng.standard_normal((1, n, hq, d)), gpu.bfloat16) for _ in range(world)]
    shards = list(zip(qs, ks, vs))
    stats = [ra.ring_causal_attention_forward_with_stats(shards, r) for r in range(world)]
    outs, ms, ls = (list(x) for x in zip(*stats))
    fw, grads = _oracle_ring(qs, ks, vs, world, hq, hkv, rank=3, gos=gos)
    assert norm_rel(_np(outs[3]), fw[3][0]) <= BF16_TOL
    dq, dk, dv = ra.ring_causal_attention_backward(shards, 3, outs, ms, ls, gos)
    gpu.cuda.synchronize()
    for a, b in zip((dq, dk, dv), grads):
        assert norm_rel(_np(a), b) <= BF16_TOL


@pytest.mark.parametrize("world,rank,n,hq,hkv,valid,chunked", [
    (1, 0, 700, 4, 2, None, False),     # the dense replacement: one diagonal pair, GQA, tails
    (1, 0, 700, 4, 2, None, True),      # the same with a workspace for 256-row chunks only
    (3, 2, 300, 4, 4, 830, False),      # diagonal shared, two recomputed dQ hops, valid_length
    (2, 1, 513, 2, 1, None, True),      # chunks of 256 rows plus a 1-row tail chunk
])
def test_ring_bwd_shares_ds_on_the_diagonal(ra, gpu, world, rank, n, hq, hkv, valid, chunked):
    """lc_ring_bwd with the workspace of lc_ring_bwd_ds_workspace_bytes runs the
    diagonal pair (hop 0 of both reference passes, rs:367-460) as one dS-sharing
    run; with the base workspace it recomputes the scores in each pass.  Both
    against the C restatement at the bf16 bar, through the C ABI."""
    from longctx100m_amd import _lib

    rng = np.random.default_rng(world * 1000 + n + int(chunked))
    d = 128
    qs, ks, vs = _rand_shards(gpu, rng, world, n, hq, hkv, d, gpu.bfloat16)
    gos = [_t(gpu, rng.standard_normal((1, n, hq, d)), gpu.bfloat16) for _ in range(world)]
    shards = list(zip(qs, ks, vs))
    fw = [ra.ring_causal_attention_forward_with_stats(shards, r, True, 64, 128, valid)
          for r in range(world)]
    outs, ms, ls = (list(x) for x in zip(*fw))
    _, grads = _oracle_ring(qs, ks, vs, world, hq, hkv, rank=rank, gos=gos, valid_length=valid)
    lib = _lib.load()
    desc = _lib.RingDesc(world, rank, 1, n, hq, hkv, d, _lib.LC_DTYPE_BF16, 0, 1, 64, 128,
                         -1 if valid is None else valid, -1)
    base = lib.lc_ring_bwd_workspace_bytes(desc)
    full = lib.lc_ring_bwd_ds_workspace_bytes(desc)
    per32 = hq * ((n + 31) // 32) * 2048  # dS bytes of one 32-row query tile
    assert full == base + per32 * ((n + 31) // 32)
    sizes = [base, base + 8 * per32] if chunked else [base, full]
    arrs = [_lib.ptr_array([t.data_ptr() for t in ts]) for ts in
            (qs, ks, vs, outs, [x.contiguous() for x in ms], [x.contiguous() for x in ls], gos)]
    results = []
    for ws_bytes in sizes:
        dq, dk, dv = (gpu.empty_like(x) for x in (qs[rank], ks[rank], ks[rank]))
        ws = gpu.full((ws_bytes,), 0xFF, dtype=gpu.uint8, device="cuda")  # bf16 NaN pattern
        _lib.check(lib.lc_ring_bwd(desc, *[a[0] for a in arrs], dq.data_ptr(), dk.data_ptr(),
                                   dv.data_ptr(), ws.data_ptr(), ws_bytes, None))
        gpu.cuda.synchronize()
        for a, e in zip((dq, dk, dv), grads):
            assert norm_rel(_np(a), e) <= BF16_TOL
        if ws_bytes > base:
            # the shared run stored the diagonal's dS past the base workspace (about half
            # of its blocks: the causal triangle), so the dS path did run
            written = float((ws[base:] != 0xFF).float().mean())
            assert written > 0.25, written
        results.append((dq, dk, dv))
    # the two paths agree far inside the bar (bf16 outputs; different kernels)
    for a, b in zip(*results):
        assert norm_rel(_np(a), _np(b)) <= 8e-3


def test_host_pointer_entry_points(gpu):
    """lc_ring_fwd_with_stats_host / lc_ring_bwd_host (the CPU-tensor form a
    candle backend binds) agree with the oracle."""
    from longctx100m_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(4)
    world, n, h, d = 2, 96, 2, 64
    mk = lambda: [rng.standard_normal((1, n, h, d)).astype(np.float32) for _ in range(world)]  # noqa: E731
    qs, ks, vs, gos = mk(), mk(), mk(), mk()
    desc = _lib.RingDesc(world, 1, 1, n, h, h, d, _lib.LC_DTYPE_F32, 0, 1, 64, 128, -1, -1)
    out = np.zeros((1, n, h, d), np.float32)
    m = np.zeros((1, h, n), np.float32)
    l = np.zeros_like(m)
    pq, _a = _lib.ptr_array([x.ctypes.data for x in qs])
    pk, _b = _lib.ptr_array([x.ctypes.data for x in ks])
    pv, _c = _lib.ptr_array([x.ctypes.data for x in vs])
    _lib.check(lib.lc_ring_fwd_with_stats_host(desc, pq, pk, pv, out.ctypes.data, m.ctypes.data,
                                               l.ctypes.data))
    eo, em, el = ring.ring_fwd_with_stats(qs, ks, vs, 1)
    assert norm_rel(out, eo) <= FP32_TOL and norm_rel(l, el) <= FP32_TOL
    fw = [ring.ring_fwd_with_stats(qs, ks, vs, r) for r in range(world)]
    outs = [x[0] for x in fw]
    ms = [x[1] for x in fw]
    ls = [x[2] for x in fw]
    dq = np.zeros_like(out)
    dk = np.zeros_like(out)
    dv = np.zeros_like(out)
    arrs = [_lib.ptr_array([x.ctypes.data for x in xs]) for xs in (qs, ks, vs, outs, ms, ls, gos)]
    _lib.check(lib.lc_ring_bwd_host(desc, *[a[0] for a in arrs], dq.ctypes.data, dk.ctypes.data,
                                    dv.ctypes.data))
    edq, edk, edv = ring.ring_bwd(qs, ks, vs, outs, ms, ls, gos, 1)
    for a, b in ((dq, edq), (dk, edk), (dv, edv)):
        assert norm_rel(a, b) <= FP32_TOL
    ref = np.zeros((1, n, h, d), np.float32)
    _lib.check(lib.lc_reference_causal_attention_host(1, n, h, h, d, _lib.LC_DTYPE_F32,
                                                      qs[0].ctypes.data, ks[0].ctypes.data,
                                                      vs[0].ctypes.data, 1, -1, ref.ctypes.data))
    assert norm_rel(ref, ring.dense(qs[0], ks[0], vs[0])) <= FP32_TOL


def test_autograd_wrapper(ra, gpu):
    import torch

    rng = np.random.default_rng(8)
    world, n, hq, hkv, d = 2, 128, 4, 2, 128
    qs, ks, vs = _rand_shards(gpu, rng, world, n, hq, hkv, d, gpu.bfloat16)
    shards = list(zip(qs, ks, vs))
    q = qs[1].clone().requires_grad_()
    k = ks[1].clone().requires_grad_()
    v = vs[1].clone().requires_grad_()
    out = ra.RingCausalAttention.apply(q, k, v, shards, 1, True, None)
    go = _t(gpu, rng.standard_normal((1, n, hq, d)), gpu.bfloat16)
    out.backward(go)
    # reference: this rank's rows of dense attention, differentiated w.r.t.
    # this rank's q, k, v only
    kall = np.concatenate([_np(x) for x in ks], 1)
    vall = np.concatenate([_np(x) for x in vs], 1)
    eo = dense.attention_fwd(_np(qs[1]), kall, vall, q_pos0=n, k_pos0=0)[0]
    assert norm_rel(_np(out), eo) <= BF16_TOL
    rounded = torch.tensor(eo, dtype=torch.float32).to(torch.bfloat16).float().numpy()
    edq, edk, edv = dense.attention_bwd(_np(qs[1]), kall, vall, _np(go), q_pos0=n, k_pos0=0,
                                        out=rounded)
    assert norm_rel(_np(q.grad), edq) <= BF16_TOL
    assert norm_rel(_np(k.grad), edk[:, n:]) <= BF16_TOL
    assert norm_rel(_np(v.grad), edv[:, n:]) <= BF16_TOL


@pytest.mark.parametrize("dtype_name,d,valid_length,qps", [
    ("bfloat16", 128, None, 57),
    ("bfloat16", 64, 150, 300),
    ("float32", 128, 170, 0),
    ("float32", 96, None, 13),
])
def test_decode_path_q_position_start(ra, gpu, dtype_name, d, valid_length, qps):
    """One rank with q_position_start: the forward places queries at
    qps + i and keys at j (ring_attention.py:117-130 with world 1) and the
    autograd backward takes _local_decode_backward (py:226-239, :258-287).
    Checked against the fp64 dense closed form at the same positions."""
    import torch

    dtype = getattr(gpu, dtype_name)
    rng = np.random.default_rng(zlib.crc32(repr((dtype_name, d, valid_length, qps)).encode()))
    n, hq, hkv = 200, 4, 2
    qs, ks, vs = _rand_shards(gpu, rng, 1, n, hq, hkv, d, dtype)
    q = qs[0].clone().requires_grad_()
    k = ks[0].clone().requires_grad_()
    v = vs[0].clone().requires_grad_()
    out = ra.RingCausalAttention.apply(q, k, v, [(q, k, v)], 0, True, valid_length, qps)
    go = _t(gpu, rng.standard_normal((1, n, hq, d)), dtype)
    out.backward(go)
    tol = BF16_TOL if dtype_name == "bfloat16" else FP32_TOL
    eo = dense.attention_fwd(_np(qs[0]), _np(ks[0]), _np(vs[0]), q_pos0=qps, k_pos0=0,
                             valid_length=valid_length)[0]
    assert norm_rel(_np(out), eo) <= tol
    oref = _np(out) if dtype_name == "bfloat16" else eo  # delta uses the cast output
    edq, edk, edv = dense.attention_bwd(_np(qs[0]), _np(ks[0]), _np(vs[0]), _np(go), q_pos0=qps,
                                        k_pos0=0, valid_length=valid_length, out=oref)
    assert norm_rel(_np(q.grad), edq) <= tol
    assert norm_rel(_np(k.grad), edk) <= tol
    assert norm_rel(_np(v.grad), edv) <= tol


def test_full_size_c2_c3_spot_check(ra, gpu):
    """BASELINE configs 2/3 at full size (rank 7 of 8, 32768-token bf16 shards,
    Hq=Hkv=16, d=128) through the ring entry points.  Sampled output rows,
    statistics, dQ rows and dK/dV keys are recomputed independently in fp32
    over all 8 x 32768 keys (torch on the GPU) and must agree within the bf16
    bar."""
    torch = gpu
    world, rank, n, h, d = 8, 7, 32768, 16, 128
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    rnd = lambda *s: torch.randn(*s, generator=gen, device="cuda").to(torch.bfloat16)  # noqa: E731
    q = rnd(1, n, h, d)
    ks = [rnd(1, n, h, d) for _ in range(world)]
    vs = [rnd(1, n, h, d) for _ in range(world)]
    dout = rnd(1, n, h, d)
    shards = [(q, ks[r], vs[r]) for r in range(world)]  # only rank 7's Q is read
    out, m, l = ra.ring_causal_attention_forward_with_stats(shards, rank)
    dq, dk, dv = ra.ring_causal_attention_backward(shards, rank, [out] * world, [m] * world,
                                                   [l] * world, [dout] * world)
    torch.cuda.synchronize()
    scale = d ** -0.5
    kall = torch.cat(ks, 1)[0].float()  # [world*n, h, d]
    vall = torch.cat(vs, 1)[0].float()
    q0, o0, do0 = q[0].float(), out[0].float(), dout[0].float()
    rows = [0, 1, 4097, 16384, 32766, 32767] + torch.randint(0, n, (6,), generator=gen, device="cuda").tolist()
    heads = [0, 11]
    errs = {"out": [], "dq": [], "m": [], "l": []}
    refs = {"out": [], "dq": []}
    for hh in heads:
        for r in rows:
            kv = kall[: rank * n + r + 1, hh]  # causal: keys up to the query's position
            vv = vall[: rank * n + r + 1, hh]
            s = (kv @ q0[r, hh]) * scale
            mx = s.max()
            p = torch.exp(s - mx)
            lsum = p.sum()
            ref_o = (p / lsum) @ vv
            errs["m"].append(abs(float(m[0, hh, r, 0]) - float(mx)) / max(1.0, abs(float(mx))))
            errs["l"].append(abs(float(l[0, hh, r, 0]) - float(lsum)) / float(lsum))
            errs["out"].append(float((o0[r, hh] - ref_o).abs().max()))
            refs["out"].append(float(ref_o.abs().max()))
            delta = float((do0[r, hh] * o0[r, hh]).sum())
            pn = p / lsum
            ds = pn * (vv @ do0[r, hh] - delta)
            ref_dq = (ds @ kv) * scale
            errs["dq"].append(float((dq[0, r, hh].float() - ref_dq).abs().max()))
            refs["dq"].append(float(ref_dq.abs().max()))
    assert max(errs["out"]) / max(refs["out"]) <= 2e-2
    assert max(errs["dq"]) / max(refs["dq"]) <= 2e-2
    assert max(errs["m"]) <= 1e-4 and max(errs["l"]) <= 1e-3
    # dK / dV of sampled keys of this rank's own shard (pass 1 of the reference backward):
    # contributions of every query i of the shard with i >= key.
    lse = (m[0, :, :, 0] + torch.log(l[0, :, :, 0])).float()  # [h, n]
    delta_all = (do0 * o0).sum(-1)  # [n, h]
    kerr, kref, verr, vref = [], [], [], []
    for hh in heads:
        for j in [0, 5, 4096, 20000, 32767]:
            kj = ks[rank][0, j, hh].float()
            vj = vs[rank][0, j, hh].float()
            qi = q0[j:, hh]
            s = (qi @ kj) * scale
            p = torch.exp(s - lse[hh, j:])
            dsj = p * (do0[j:, hh] @ vj - delta_all[j:, hh])
            ref_dk = (dsj @ qi) * scale
            ref_dv = p @ do0[j:, hh]
            kerr.append(float((dk[0, j, hh].float() - ref_dk).abs().max()))
            kref.append(float(ref_dk.abs().max()))
            verr.append(float((dv[0, j, hh].float() - ref_dv).abs().max()))
            vref.append(float(ref_dv.abs().max()))
    assert max(kerr) / max(kref) <= 2e-2
    assert max(verr) / max(vref) <= 2e-2
    assert torch.isfinite(out.float()).all() and torch.isfinite(dq.float()).all()


def _random_cases(seed, n):
    """Random d=128 bf16 shapes, GQA groups, positions and masks (drawn once)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        hkv = int(rng.choice([1, 2]))
        out.append(dict(b=int(rng.integers(1, 3)), nq=int(rng.integers(1, 700)),
                        nk=int(rng.integers(1, 700)), hkv=hkv, hq=hkv * int(rng.choice([1, 2, 4])),
                        causal=bool(rng.integers(0, 2)), q_pos0=int(rng.integers(0, 1500)),
                        k_pos0=int(rng.integers(0, 1500)),
                        valid_length=None if rng.integers(0, 3) else int(rng.integers(1, 2500))))
    return out


@pytest.mark.parametrize("case", _random_cases(2026, 24), ids=lambda c: "q{nq}k{nk}h{hq}/{hkv}".format(**c))
def test_random_shapes_fwd_and_shared_ds_bwd(ra, gpu, case):
    """Random shapes through the benched kernels (forward, preprocess, dS-sharing backward) against
    the fp64 dense oracle at the bf16 bar: query and key counts that are not multiples of any tile,
    offsets that make hops full, diagonal, partial or empty, valid_length cuts, GQA 1/2/4."""
    c = dict(case)
    b, nq, nk, hq, hkv = c.pop("b"), c.pop("nq"), c.pop("nk"), c.pop("hq"), c.pop("hkv")
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    q = _t(gpu, rng.standard_normal((b, nq, hq, 128)), gpu.bfloat16)
    k = _t(gpu, rng.standard_normal((b, nk, hkv, 128)), gpu.bfloat16)
    v = _t(gpu, rng.standard_normal((b, nk, hkv, 128)), gpu.bfloat16)
    do = _t(gpu, rng.standard_normal((b, nq, hq, 128)), gpu.bfloat16)
    o32, m, l = ra.fwd_shard(q, k, v, **c)
    out = o32.to(gpu.bfloat16)
    delta, lse2 = ra.bwd_preprocess(out, do, m, l)
    ws = gpu.empty(max(256, ra.bwd_shard_workspace_bytes(q, k)), dtype=gpu.uint8, device="cuda")
    dq = gpu.zeros((b, nq, hq, 128), dtype=gpu.float32, device="cuda")
    dk = gpu.zeros((b, nk, hkv, 128), dtype=gpu.float32, device="cuda")
    dv = gpu.zeros_like(dk)
    ra.bwd_shard(q, k, v, do, lse2, delta, dq_acc=dq, dk_acc=dk, dv_acc=dv, workspace=ws, **c)
    gpu.cuda.synchronize()
    eo, em, el = dense.attention_fwd(_np(q), _np(k), _np(v), **c)
    edq, edk, edv = dense.attention_bwd(_np(q), _np(k), _np(v), _np(do), out=_np(out), **c)
    assert norm_rel(_np(o32), eo) <= BF16_TOL
    assert norm_rel(_np(dq), edq) <= BF16_TOL
    assert norm_rel(_np(dk), edk) <= BF16_TOL
    assert norm_rel(_np(dv), edv) <= BF16_TOL


@pytest.mark.parametrize("case", _random_cases(2031, 10), ids=lambda c: "q{nq}k{nk}h{hq}/{hkv}".format(**c))
def test_random_shapes_shared_ds_partial_workspace(ra, gpu, case):
    """The dS-sharing backward with a workspace smaller than the whole shard
    pair's dS: the pair runs in query chunks of multiples of 256 rows, or, below
    one chunk, the recomputing dQ kernel.  Random shapes and a random fraction
    (0 to 0.8) of the full workspace, against the fp64 dense oracle."""
    c = dict(case)
    b, nq, nk, hq, hkv = c.pop("b"), c.pop("nq"), c.pop("nk"), c.pop("hq"), c.pop("hkv")
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()) + 1)
    q = _t(gpu, rng.standard_normal((b, nq, hq, 128)), gpu.bfloat16)
    k = _t(gpu, rng.standard_normal((b, nk, hkv, 128)), gpu.bfloat16)
    v = _t(gpu, rng.standard_normal((b, nk, hkv, 128)), gpu.bfloat16)
    do = _t(gpu, rng.standard_normal((b, nq, hq, 128)), gpu.bfloat16)
    o32, m, l = ra.fwd_shard(q, k, v, **c)
    out = o32.to(gpu.bfloat16)
    delta, lse2 = ra.bwd_preprocess(out, do, m, l)
    full = ra.bwd_shard_workspace_bytes(q, k)
    nbytes = max(256, int(full * float(rng.choice([0.0, 0.2, 0.4, 0.6, 0.8]))) // 256 * 256)
    ws = gpu.empty(nbytes, dtype=gpu.uint8, device="cuda")
    dq = gpu.zeros((b, nq, hq, 128), dtype=gpu.float32, device="cuda")
    dk = gpu.zeros((b, nk, hkv, 128), dtype=gpu.float32, device="cuda")
    dv = gpu.zeros_like(dk)
    ra.bwd_shard(q, k, v, do, lse2, delta, dq_acc=dq, dk_acc=dk, dv_acc=dv, workspace=ws, **c)
    gpu.cuda.synchronize()
    edq, edk, edv = dense.attention_bwd(_np(q), _np(k), _np(v), _np(do), out=_np(out), **c)
    assert norm_rel(_np(dq), edq) <= BF16_TOL
    assert norm_rel(_np(dk), edk) <= BF16_TOL
    assert norm_rel(_np(dv), edv) <= BF16_TOL


@pytest.fixture
def one_rank_nccl_group(gpu):
    """A one-process NCCL (RCCL) group on this GPU, as the reference's Python entry
    requires for CUDA tensors (py:88-92); nothing is communicated."""
    import socket

    import torch.distributed as dist

    assert not dist.is_initialized()
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    dist.init_process_group("nccl", init_method=f"tcp://127.0.0.1:{port}", rank=0, world_size=1)
    try:
        yield dist.group.WORLD
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("dtype_name,qps,valid_length", [("bfloat16", None, None),
                                                         ("float32", None, 250),
                                                         ("bfloat16", 500, None)])
def test_python_signature_in_a_group(ra, gpu, one_rank_nccl_group, dtype_name, qps,
                                     valid_length):
    """ring_causal_attention(q, k, v, *, group, ...) with the Python reference's
    signature (src/longctx100m/ring_attention.py:176-191), called as model.py:254-265
    calls it: autograd forward and backward on a one-rank NCCL group, against the fp64
    dense closed form (with q_position_start, the reference's decode backward)."""
    d, n, h = 128, 300, 4
    dtype = getattr(gpu, dtype_name)
    rng = np.random.default_rng(zlib.crc32(repr((dtype_name, qps, valid_length)).encode()))
    qs, ks, vs = _rand_shards(gpu, rng, 1, n, h, h, d, dtype)
    q = qs[0].clone().requires_grad_()
    k = ks[0].clone().requires_grad_()
    v = vs[0].clone().requires_grad_()
    out = ra.ring_causal_attention(q, k, v, group=one_rank_nccl_group, valid_length=valid_length,
                                   q_position_start=qps)
    go = _t(gpu, rng.standard_normal((1, n, h, d)), dtype)
    out.backward(go)
    gpu.cuda.synchronize()
    tol = BF16_TOL if dtype_name == "bfloat16" else FP32_TOL
    qp = 0 if qps is None else qps
    eo = dense.attention_fwd(_np(qs[0]), _np(ks[0]), _np(vs[0]), q_pos0=qp, k_pos0=0,
                             valid_length=valid_length)[0]
    assert norm_rel(_np(out), eo) <= tol
    oref = _np(out) if dtype_name == "bfloat16" else eo  # delta uses the cast output
    edq, edk, edv = dense.attention_bwd(_np(qs[0]), _np(ks[0]), _np(vs[0]), _np(go), q_pos0=qp,
                                        k_pos0=0, valid_length=valid_length, out=oref)
    for a, e in ((q.grad, edq), (k.grad, edk), (v.grad, edv)):
        assert norm_rel(_np(a), e) <= tol
