"""Pins the CPU oracle (oracle/) before anything is compared against it.

The reference stores no attention vectors (its tests recompute a dense
oracle), so the C restatement of its blocked algorithm is pinned by
  * the reference's own test cases, inputs and tolerances
    (rust/longctx100m-model/src/ring_attention.rs:519-668,
    tests/test_ring_attention.py:36-95,277-321,403-445), against
  * an fp64 brute-force dense attention with closed-form gradients, which is
    itself pinned to torch's SDPA and autograd (library routines; the
    reference's own test at tests/test_ring_attention.py:36-49 does the same),
  * and invariants: block-size invariance, world=1 == dense, valid_length ==
    truncation, GQA == repeat_interleave + group sum, fully masked rows.
Planted-mistake checks show a plausible bug (mask off by one, wrong scale,
swapped operands, dropped delta term) fails these comparisons.
"""

import numpy as np
import pytest
import torch

from oracle import dense, ring
from tests.conftest import norm_rel


def _randn(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


# ----------------------------------------------------------- dense vs torch --

def test_dense_matches_torch_sdpa():
    # tests/test_ring_attention.py:36-49: [1, 9, 2, 8], seed 7, SDPA is_causal.
    torch.manual_seed(7)
    q = torch.randn(1, 9, 2, 8, dtype=torch.float64)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    exp = torch.nn.functional.scaled_dot_product_attention(
        q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3),
        is_causal=True).permute(0, 2, 1, 3)
    out, _, _ = dense.attention_fwd(q.numpy(), k.numpy(), v.numpy())
    assert np.abs(out - exp.numpy()).max() < 1e-12


@pytest.mark.parametrize("case", [
    dict(tq=7, tk=7, hq=2, hkv=2, causal=True, valid=None, qp=0, kp=0),
    dict(tq=5, tk=9, hq=4, hkv=2, causal=True, valid=11, qp=3, kp=0),
    dict(tq=6, tk=6, hq=3, hkv=1, causal=False, valid=4, qp=0, kp=0),
    dict(tq=4, tk=8, hq=2, hkv=1, causal=True, valid=None, qp=10, kp=4),
])
def test_dense_fwd_bwd_match_torch_autograd(case):
    rng = np.random.default_rng(11)
    d = 8
    q = rng.standard_normal((1, case["tq"], case["hq"], d))
    k = rng.standard_normal((1, case["tk"], case["hkv"], d))
    v = rng.standard_normal((1, case["tk"], case["hkv"], d))
    do = rng.standard_normal((1, case["tq"], case["hq"], d))
    kw = dict(causal=case["causal"], valid_length=case["valid"], q_pos0=case["qp"],
              k_pos0=case["kp"])
    out, m, l = dense.attention_fwd(q, k, v, **kw)
    dq, dk, dv = dense.attention_bwd(q, k, v, do, **kw)

    tq = torch.tensor(q, requires_grad=True)
    tk = torch.tensor(k, requires_grad=True)
    tv = torch.tensor(v, requires_grad=True)
    g = case["hq"] // case["hkv"]
    ke = tk.repeat_interleave(g, dim=2)
    ve = tv.repeat_interleave(g, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", tq, ke) * d**-0.5
    bad = torch.tensor(dense.invalid_mask(case["tq"], case["tk"], **kw))
    s = s.masked_fill(bad, float("-inf"))
    p = torch.softmax(s, -1).nan_to_num(0.0)
    ref = torch.einsum("bhqk,bkhd->bqhd", p, ve)
    (ref * torch.tensor(do)).sum().backward()
    assert np.abs(out - ref.detach().numpy()).max() < 1e-12
    assert np.abs(dq - tq.grad.numpy()).max() < 1e-12
    assert np.abs(dk - tk.grad.numpy()).max() < 1e-12
    assert np.abs(dv - tv.grad.numpy()).max() < 1e-12
    # statistics: LSE = m + ln l equals torch.logsumexp of the masked scores
    lse = torch.logsumexp(s.detach(), -1).numpy()
    fin = np.isfinite(lse)
    assert np.abs((m + np.log(np.where(l > 0, l, 1)))[fin] - lse[fin]).max() < 1e-12
    assert np.all(np.isneginf(m[~fin])) and np.all(l[~fin] == 0)


# ---------------------------------------- reference unit tests on the oracle --

def test_ring_single_rank_matches_reference_dense():
    # ring_attention.rs:519-534: B=1, T=8, H=2, D=4, block_q=2, block_k=3, abs 1e-5.
    rng = np.random.default_rng(0)
    q, k, v = (_randn(rng, 1, 8, 2, 4) for _ in range(3))
    out, _, _ = ring.ring_fwd_with_stats([q], [k], [v], 0, block_q=2, block_k=3)
    exp = ring.dense(q, k, v)
    assert np.abs(out - exp).max() < 1e-5
    exp64, _, _ = dense.attention_fwd(q, k, v)
    assert np.abs(out - exp64).max() < 1e-5


@pytest.mark.parametrize("valid", [None, 6])
def test_ring_two_rank_lcg_matches_dense(valid):
    # ring_attention.rs:536-594: LCG shards (q = k = v quirk), t=4/rank, h=2,
    # d=4, world 2, blocks 2/3, valid_length None or 6; abs 1e-5.
    qs = dense.lcg_shards(4, 2, 4, 2)
    ks = dense.lcg_shards(4, 2, 4, 2)
    vs = dense.lcg_shards(4, 2, 4, 2)
    assert all(np.array_equal(a, b) for a, b in zip(qs, ks))  # the generator's quirk
    assert all(((x >= -0.5) & (x < 0)).all() for x in qs)
    full = [np.concatenate(x, axis=1) for x in (qs, ks, vs)]
    exp = dense.attention_fwd(*full, valid_length=valid)[0]
    exp32 = ring.dense(*full, valid_length=valid)
    for r in range(2):
        out, _, _ = ring.ring_fwd_with_stats(qs, ks, vs, r, block_q=2, block_k=3,
                                             valid_length=valid)
        assert np.abs(out - exp[:, 4 * r:4 * r + 4]).max() < 1e-5
        assert np.abs(out - exp32[:, 4 * r:4 * r + 4]).max() < 1e-5


def test_ring_backward_single_rank_matches_autograd():
    # ring_attention.rs:596-668: loss = sum(out), so grad_out = ones; abs 1e-4.
    rng = np.random.default_rng(3)
    q, k, v = (_randn(rng, 1, 8, 2, 4) for _ in range(3))
    out, m, l = ring.ring_fwd_with_stats([q], [k], [v], 0, block_q=2, block_k=3)
    go = np.ones_like(q)
    dq, dk, dv = ring.ring_bwd([q], [k], [v], [out], [m], [l], [go], 0, block_q=2, block_k=3)
    edq, edk, edv = dense.attention_bwd(q, k, v, go)
    for a, b in ((dq, edq), (dk, edk), (dv, edv)):
        assert np.abs(a - b).max() < 1e-4


def test_two_rank_ring_forward_backward_python_case():
    # tests/test_ring_attention.py:277-321: T=8 split over 2 ranks, H=2, D=4,
    # block 2/2, loss = sum(out); fwd <= 2e-5, grads <= 3e-4.
    torch.manual_seed(123)
    q = torch.randn(1, 8, 2, 4).numpy()
    k = torch.randn(1, 8, 2, 4).numpy()
    v = torch.randn(1, 8, 2, 4).numpy()
    qs, ks, vs = ([x[:, 4 * r:4 * r + 4] for r in range(2)] for x in (q, k, v))
    exp = dense.attention_fwd(q, k, v)[0]
    stats = [ring.ring_fwd_with_stats(qs, ks, vs, r, block_q=2, block_k=2) for r in range(2)]
    outs, ms, ls = zip(*stats)
    for r in range(2):
        assert np.abs(outs[r] - exp[:, 4 * r:4 * r + 4]).max() < 2e-5
    gos = [np.ones_like(x) for x in qs]
    edq, edk, edv = dense.attention_bwd(q, k, v, np.ones_like(q))
    for r in range(2):
        dq, dk, dv = ring.ring_bwd(qs, ks, vs, outs, ms, ls, gos, r, block_q=2, block_k=2)
        sl = slice(4 * r, 4 * r + 4)
        assert np.abs(dq - edq[:, sl]).max() < 3e-4
        assert np.abs(dk - edk[:, sl]).max() < 3e-4
        assert np.abs(dv - edv[:, sl]).max() < 3e-4


def test_config1_fp32_two_rank_gqa_forward_backward():
    # fp32, B=1, Hq=9, Hkv=3 (expanded by repeat_interleave,
    # the reference callers' rule), d=64, world 2 x 512 tokens; 1e-5 norm-rel.
    rng = np.random.default_rng(2024)
    n, hq, hkv, d = 512, 9, 3, 64
    q = _randn(rng, 1, 2 * n, hq, d)
    k = _randn(rng, 1, 2 * n, hkv, d)
    v = _randn(rng, 1, 2 * n, hkv, d)
    do = _randn(rng, 1, 2 * n, hq, d)
    ke, ve = (np.repeat(x, hq // hkv, axis=2) for x in (k, v))
    sh = lambda x: [x[:, r * n:(r + 1) * n] for r in range(2)]  # noqa: E731
    qs, ks, vs, gos = sh(q), sh(ke), sh(ve), sh(do)
    out64, m64, l64 = dense.attention_fwd(q, k, v)
    dq64, dk64, dv64 = dense.attention_bwd(q, k, v, do)
    stats = [ring.ring_fwd_with_stats(qs, ks, vs, r) for r in range(2)]
    outs, ms, ls = zip(*stats)
    for r in range(2):
        sl = slice(r * n, (r + 1) * n)
        assert norm_rel(outs[r], out64[:, sl]) < 1e-5
        assert np.abs(ms[r] - m64[:, :, sl]).max() < 1e-5
        assert norm_rel(ls[r], l64[:, :, sl]) < 1e-5
        dq, dk, dv = ring.ring_bwd(qs, ks, vs, outs, ms, ls, gos, r)
        dkg = dk.reshape(1, n, hkv, hq // hkv, d).sum(3)  # GQA group sum
        dvg = dv.reshape(1, n, hkv, hq // hkv, d).sum(3)
        assert norm_rel(dq, dq64[:, sl]) < 1e-5
        assert norm_rel(dkg, dk64[:, sl]) < 1e-5
        assert norm_rel(dvg, dv64[:, sl]) < 1e-5


# ------------------------------------------------------------------ invariants --

@pytest.mark.parametrize("bq,bk", [(1, 1), (3, 5), (64, 128), (100, 7)])
def test_block_size_invariance(bq, bk):
    rng = np.random.default_rng(5)
    qs = [_randn(rng, 1, 24, 2, 8) for _ in range(3)]
    ks = [_randn(rng, 1, 24, 2, 8) for _ in range(3)]
    vs = [_randn(rng, 1, 24, 2, 8) for _ in range(3)]
    base = ring.ring_fwd_with_stats(qs, ks, vs, 2, block_q=2, block_k=3, valid_length=70)
    got = ring.ring_fwd_with_stats(qs, ks, vs, 2, block_q=bq, block_k=bk, valid_length=70)
    for a, b in zip(got, base):
        assert np.abs(a - b).max() < 1e-5


def test_world1_equals_dense_and_valid_length_is_truncation():
    # tests/test_ring_attention.py:85-95
    rng = np.random.default_rng(9)
    q, k, v = (_randn(rng, 1, 6, 1, 4) for _ in range(3))
    out, _, _ = ring.ring_fwd_with_stats([q], [k], [v], 0, valid_length=4)
    trunc, _, _ = ring.ring_fwd_with_stats([q[:, :4]], [k[:, :4]], [v[:, :4]], 0)
    assert np.isfinite(out).all()
    assert np.abs(out[:, :4] - trunc).max() < 1e-6
    assert np.abs(out - dense.attention_fwd(q, k, v, valid_length=4)[0]).max() < 1e-5


def test_fully_masked_hops_and_rows():
    rng = np.random.default_rng(1)
    q, k, v = (_randn(rng, 1, 6, 2, 4) for _ in range(3))
    qs, ks, vs = [q, q], [k, k], [v, v]
    # q_position_start = 3: queries at 3..8 see part of owner 1 (keys 6..11)
    # and all of owner 0 (keys 0..5)
    out, m, l = ring.ring_fwd_with_stats(qs, ks, vs, 1, q_position_start=3)
    exp, em, el = dense.ring_rows(qs, ks, vs, 1, q_position_start=3)
    assert np.abs(out - exp).max() < 1e-5
    assert np.abs(m - em).max() < 1e-5 and np.abs(l - el).max() < 1e-5
    # q_position_start = 0: the owner-1 hop is fully masked and leaves the
    # state exactly as a one-rank ring over owner 0 alone
    got = ring.ring_fwd_with_stats(qs, ks, vs, 1, q_position_start=0)
    only0 = ring.ring_fwd_with_stats([q], [k], [v], 0)
    for a, b in zip(got, only0):
        assert np.array_equal(a, b)
    # rows that see no key at all (keys after every query): out 0, m -inf, l 0,
    # and zero gradients
    o2, m2, l2 = dense.attention_fwd(q, k, v, q_pos0=0, k_pos0=2)
    assert np.all(o2[:, :2] == 0) and np.all(np.isneginf(m2[:, :, :2])) and np.all(l2[:, :, :2] == 0)
    dq2, dk2, dv2 = dense.attention_bwd(q, k, v, np.ones_like(q), q_pos0=0, k_pos0=2)
    assert np.all(dq2[:, :2] == 0) and np.isfinite(dk2).all() and np.isfinite(dv2).all()


def test_error_messages_match_reference():
    q = np.zeros((1, 4, 1, 4), np.float32)
    with pytest.raises(ring.OracleError, match="rank 2 out of range for world_size 2"):
        ring.ring_fwd_with_stats([q, q], [q, q], [q, q], 2)
    with pytest.raises(ring.OracleError, match="block_q and block_k must be positive"):
        ring.ring_fwd_with_stats([q], [q], [q], 0, block_q=0)
    with pytest.raises(ring.OracleError, match="valid_length must be within"):
        ring.ring_fwd_with_stats([q], [q], [q], 0, valid_length=5)


# ---------------------------------------------------------- planted mistakes --

def test_planted_mistakes_fail_the_checks():
    """Each plausible oracle bug, planted in the fp64 oracle, must break the
    comparison the suite relies on."""
    rng = np.random.default_rng(21)
    n = 16
    qs = [_randn(rng, 1, n, 2, 8) for _ in range(2)]
    ks = [_randn(rng, 1, n, 2, 8) for _ in range(2)]
    vs = [_randn(rng, 1, n, 2, 8) for _ in range(2)]
    gos = [_randn(rng, 1, n, 2, 8) for _ in range(2)]
    out, m, l = ring.ring_fwd_with_stats(qs, ks, vs, 1)
    full = [np.concatenate(x, axis=1) for x in (qs, ks, vs, gos)]
    good = dense.attention_fwd(*full[:3])[0][:, n:]
    assert norm_rel(out, good) < 1e-5
    # mask off by one (key >= query masked)
    bad = dense.attention_fwd(*full[:3], q_pos0=-1)[0][:, n:]
    assert norm_rel(out, bad) > 1e-3
    # wrong scale (1/d instead of d^-1/2)
    bad = dense.attention_fwd(*full[:3], scale=1 / 8)[0][:, n:]
    assert norm_rel(out, bad) > 1e-3
    # q and k transposed
    bad = dense.attention_fwd(full[1], full[0], full[2])[0][:, n:]
    assert norm_rel(out, bad) > 1e-3
    # dropped delta term in dS
    outs, ms, ls = zip(*[ring.ring_fwd_with_stats(qs, ks, vs, r) for r in range(2)])
    dq, dk, dv = ring.ring_bwd(qs, ks, vs, outs, ms, ls, gos, 1)
    edq = dense.attention_bwd(*full)[0][:, n:]
    assert norm_rel(dq, edq) < 1e-5
    zero_out = np.zeros_like(full[0])
    bad_dq = dense.attention_bwd(*full, out=zero_out)[0][:, n:]
    assert norm_rel(dq, bad_dq) > 1e-3
