"""GPU parity of the split-KV decode (lc_attn_decode) against the fp64 dense
oracle: a few query tokens at the end of a long KV shard, GQA rows packed per
KV head, causal / valid_length masks, ragged cache lengths, many splits, the
fallback shapes, and a decode over two KV shards merged by LSE.  Same bars as
lc_attn_fwd_shard (bf16 2e-2 norm-relative; m within 1e-4, l within 1e-4)."""

import zlib

import numpy as np
import pytest

from oracle import dense
from tests.conftest import norm_rel

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


@pytest.fixture(scope="module")
def ra(gpu):
    from longctx100m_amd import ring_attention

    return ring_attention


def _t(gpu, arr, dtype):
    return gpu.tensor(np.ascontiguousarray(arr), dtype=gpu.float32).to(dtype).cuda()


def _np(t):
    return t.detach().float().cpu().numpy()


def _check(o, m, l, eo, em, el, tol=BF16_TOL):
    assert norm_rel(_np(o), eo) <= tol
    m, l = _np(m), _np(l)
    fin = np.isfinite(em)
    assert np.array_equal(np.isfinite(m), fin)
    if fin.any():
        assert np.abs(m[fin] - em[fin]).max() <= 1e-4 * max(1.0, np.abs(em[fin]).max())
        assert norm_rel(l, el) <= 1e-4
    assert np.all(l[~fin] == 0)


# (B, Nq, Hq, Hkv, Nk, q_pos0 offset from the cache end, k_pos0, causal, valid_length)
DECODE_CASES = [
    (1, 1, 32, 8, 5000, 0, 0, True, None),        # C4-style GQA, one new token
    (2, 4, 8, 2, 3333, 0, 0, True, None),         # 16 rows per KV head, causal within the block
    (1, 1, 16, 16, 70000, 0, 0, True, None),      # one row per KV head, many splits
    (1, 2, 4, 4, 1000, 0, 131072, True, 131072 + 777),  # offset cache, valid_length cut
    (1, 3, 8, 8, 4096, -40, 0, True, None),       # queries inside the cache (causal masks keys)
    (1, 1, 8, 8, 64, 0, 0, False, None),          # tiny cache, non-causal
    (1, 8, 8, 2, 2000, 0, 0, True, None),         # 32 rows: the blockwise fallback
]


@pytest.mark.parametrize("case", DECODE_CASES)
def test_decode_matches_dense(ra, gpu, case):
    b, nq, hq, hkv, nk, qoff, kp, causal, valid = case
    d = 128
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    q = _t(gpu, rng.standard_normal((b, nq, hq, d)), gpu.bfloat16)
    k = _t(gpu, rng.standard_normal((b, nk, hkv, d)), gpu.bfloat16)
    v = _t(gpu, rng.standard_normal((b, nk, hkv, d)), gpu.bfloat16)
    qp = kp + nk - nq + qoff
    o, m, l = ra.decode(q, k, v, q_pos0=qp, k_pos0=kp, causal=causal, valid_length=valid)
    gpu.cuda.synchronize()
    eo, em, el = dense.attention_fwd(_np(q), _np(k), _np(v), causal=causal, valid_length=valid,
                                     q_pos0=qp, k_pos0=kp)
    _check(o, m, l, eo, em, el)


def _random_decode_cases(seed, n):
    """Random decode geometries (drawn once), in DECODE_CASES' tuple form: batch,
    1-4 new tokens, GQA groups up to 8 (16 or fewer rows per KV head take the
    split kernel, more the blockwise fallback), caches of 1 to 20,000 keys at
    an offset, queries anywhere from before the first key to the cache end,
    causal or not, valid_length inside or past the cache."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        hkv = int(rng.choice([1, 2, 4]))
        nq = int(rng.integers(1, 5))
        nk = int(rng.integers(1, 20001))
        kp = int(rng.choice([0, int(rng.integers(0, 300000))]))
        qoff = -int(rng.integers(0, min(nk, 50) + 1)) if rng.integers(0, 3) else 0
        valid = None if rng.integers(0, 3) else int(rng.integers(1, kp + nk + 100))
        out.append((int(rng.integers(1, 3)), nq, hkv * int(rng.choice([1, 2, 4, 8])), hkv, nk,
                    qoff, kp, bool(rng.integers(0, 4)), valid))
    return out


@pytest.mark.parametrize("case", _random_decode_cases(77, 24))
def test_decode_random_against_dense(ra, gpu, case):
    """Seeded random decode geometries through lc_attn_decode against the fp64
    dense oracle, at the bars of DECODE_CASES."""
    test_decode_matches_dense(ra, gpu, case)


def test_decode_equals_fwd_shard(ra, gpu):
    """Both entry points give the same statistics for the same decode step."""
    rng = np.random.default_rng(77)
    q = _t(gpu, rng.standard_normal((1, 1, 32, 128)), gpu.bfloat16)
    k = _t(gpu, rng.standard_normal((1, 9001, 8, 128)), gpu.bfloat16)
    v = _t(gpu, rng.standard_normal((1, 9001, 8, 128)), gpu.bfloat16)
    o1, m1, l1 = ra.decode(q, k, v, q_pos0=9000, k_pos0=0)
    o2, m2, l2 = ra.fwd_shard(q, k, v, q_pos0=9000, k_pos0=0)
    gpu.cuda.synchronize()
    assert norm_rel(_np(o1), _np(o2)) <= 1e-2
    assert np.abs(_np(m1) - _np(m2)).max() <= 1e-5
    assert norm_rel(_np(l1), _np(l2)) <= 1e-3


def test_decode_over_two_shards_merged(ra, gpu):
    """A decode step over a cache held as two KV shards (two ring owners):
    decode each, LSE-merge, compare with dense attention over both."""
    rng = np.random.default_rng(78)
    n0, n1, hq, hkv, d = 6000, 2500, 32, 8, 128
    q = _t(gpu, rng.standard_normal((1, 1, hq, d)), gpu.bfloat16)
    ks = [_t(gpu, rng.standard_normal((1, n, hkv, d)), gpu.bfloat16) for n in (n0, n1)]
    vs = [_t(gpu, rng.standard_normal((1, n, hkv, d)), gpu.bfloat16) for n in (n0, n1)]
    qp = n0 + n1 - 1
    o0, m0, l0 = ra.decode(q, ks[0], vs[0], q_pos0=qp, k_pos0=0)
    o1, m1, l1 = ra.decode(q, ks[1], vs[1], q_pos0=qp, k_pos0=n0)
    out = gpu.empty((1, 1, hq, d), dtype=gpu.bfloat16, device="cuda")
    ra.merge(o0, m0, l0, o1, m1, l1, out=out)
    gpu.cuda.synchronize()
    kall = np.concatenate([_np(x) for x in ks], 1)
    vall = np.concatenate([_np(x) for x in vs], 1)
    eo, em, el = dense.attention_fwd(_np(q), kall, vall, q_pos0=qp, k_pos0=0)
    _check(o0, m0, l0, eo, em, el)
    assert norm_rel(_np(out), eo) <= BF16_TOL
