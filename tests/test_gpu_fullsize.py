"""Full-size parity of the benchmarked workloads, through the same launches
bench.py times (longctx100m_amd.rank_step).

* BASELINE configs 2+3: rank 7 of 8, 32,768-token bf16 shards, Hq = Hkv = 16,
  d = 128; the forward over the diagonal + 7 full KV shards with LSE merges,
  then the backward with dS sharing (lc_attn_bwd_shard_ws: the dK/dV kernel
  stores dS in the full 32 GiB workspace, the dQ kernel reads it back), dQ
  accumulated across owners and dK/dV kept per owner.  Two heads are
  recomputed in full in fp32 (every query row against all 262,144 keys, every
  key of every owner), following ring_attention.rs:139-233 (forward) and
  :367-460 (backward: P = exp(s - m) / l, dS = P (dO V^T - delta), delta from
  the bf16-cast output, ring_attention.py:314).
* The config-4 model's attention share: 65,536-token shards, GQA Hq = 32 /
  Hkv = 8, rank 3 of 4, forward and backward through the same step with a
  16 GiB dS workspace (query chunks; the full one would be 275 GB), one KV
  head and its 4 query heads checked in full (dK/dV summed over the group).
* The reference's signatures at configs 2/3 size (lc_ring_fwd_with_stats and
  lc_ring_bwd, the diagonal pair sharing dS), checked in full for two heads.
* a 1,000,000-token bf16 shard at rank 1 of 2 (diagonal +
  one full 1M-token KV shard), forward with LSE merge; sampled rows of two
  heads against an fp32 recompute over all visible keys, including the rows
  around the 65,536-key sub-shard boundaries and the 64-row tail tile.

Bars: bf16 outputs and gradients within 2e-2 norm-relative
(max|a - b| / max|b|); m within 1e-4 (relative to max(1, |m|)) and l within
1e-3 relative (sums of up to 2M terms).
"""

import pytest

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _nrel(a, b) -> float:
    den = float(b.abs().max())
    return float((a - b).abs().max()) / (den if den > 0 else 1.0)


def _head_reference(torch, q, kall, vall, dout, q_pos0, scale, chunk=1024):
    """fp32 forward + backward of one head: q, dout [n, d]; kall, vall [N, d]
    with key j at position j; query i at q_pos0 + i (causal).  Returns
    out, m, l, dq [n...] and dk, dv [N, d]."""
    n, d = q.shape
    N = kall.shape[0]
    out = torch.empty(n, d, device=q.device)
    dq = torch.empty(n, d, device=q.device)
    m = torch.empty(n, device=q.device)
    l = torch.empty(n, device=q.device)
    dk = torch.zeros(N, d, device=q.device)
    dv = torch.zeros(N, d, device=q.device)
    kpos = torch.arange(N, device=q.device)
    for r0 in range(0, n, chunk):
        r1 = min(n, r0 + chunk)
        qc, doc = q[r0:r1], dout[r0:r1]
        qpos = q_pos0 + torch.arange(r0, r1, device=q.device)
        s = (qc @ kall.t()) * scale
        s.masked_fill_(kpos[None, :] > qpos[:, None], float("-inf"))
        mc = s.max(dim=1).values
        p = torch.exp(s - mc[:, None])
        del s
        lc = p.sum(dim=1)
        p /= lc[:, None]
        oc = p @ vall
        delta = (doc * oc.to(torch.bfloat16).float()).sum(dim=1)  # delta from the cast output
        ds = p * ((doc @ vall.t()) - delta[:, None])
        dq[r0:r1] = (ds @ kall) * scale
        dk += (ds.t() @ qc) * scale
        dv += p.t() @ doc
        out[r0:r1], m[r0:r1], l[r0:r1] = oc, mc, lc
        del p, ds
    return out, m, l, dq, dk, dv


def test_c2_c3_benched_step_full_size(gpu):
    """The exact step bench.py times, at its full size, checked in full for
    heads 0 and 11: output, statistics, dQ of every row, and dK/dV of every
    key of every owner (the diagonal owner 7 and the full-hop owners 0-6,
    including their first and last 32-key blocks)."""
    torch = gpu
    from longctx100m_amd.rank_step import RankStep

    world, rank, n, h, d = 8, 7, 32768, 16, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    rnd = lambda *s: torch.randn(*s, generator=gen, device=dev).to(torch.bfloat16)  # noqa: E731
    q = rnd(1, n, h, d)
    dout = rnd(1, n, h, d)
    ks = [rnd(1, n, h, d) for _ in range(world)]
    vs = [rnd(1, n, h, d) for _ in range(world)]
    rs = RankStep(q, dout, ks, vs, rank, share_ds=True)
    assert rs.owners == [7, 6, 5, 4, 3, 2, 1, 0]
    assert rs.workspace is not None and rs.workspace.numel() >= 32 * 2**30  # full dS workspace
    print(f"fullsize C2/C3: world={world} rank={rank} n={n} H={h} d={d} bf16, "
          f"dS workspace {rs.workspace.numel() / 2**30:.1f} GiB", flush=True)
    rs.step()
    torch.cuda.synchronize()

    scale = d ** -0.5
    for hh in (0, 11):
        kall = torch.cat([x[0, :, hh] for x in ks], 0).float()  # owner order = position order
        vall = torch.cat([x[0, :, hh] for x in vs], 0).float()
        eo, em, el, edq, edk, edv = _head_reference(torch, q[0, :, hh].float(), kall, vall,
                                                    dout[0, :, hh].float(), rank * n, scale)
        errs = {
            "out": _nrel(rs.out[0, :, hh].float(), eo),
            "dq": _nrel(rs.dq_acc[0, :, hh], edq),
            "m": float(((rs.m[0, hh] - em).abs() / em.abs().clamp(min=1.0)).max()),
            "l": float(((rs.l[0, hh] - el).abs() / el).max()),
        }
        for b in rs.owners:
            ek, ev = edk[b * n:(b + 1) * n], edv[b * n:(b + 1) * n]
            gk, gv = rs.dk_acc[b][0, :, hh], rs.dv_acc[b][0, :, hh]
            errs[f"dk{b}"] = _nrel(gk, ek)
            errs[f"dv{b}"] = _nrel(gv, ev)
            for name, sl in (("first", slice(0, 32)), ("last", slice(n - 32, n))):
                errs[f"dk{b}_{name}32"] = _nrel(gk[sl], ek[sl])
                errs[f"dv{b}_{name}32"] = _nrel(gv[sl], ev[sl])
        print(f"fullsize C2/C3 head {hh}: " +
              ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
        bad = {k: v for k, v in errs.items()
               if not v <= {"m": 1e-4, "l": 1e-3}.get(k, BF16_TOL)}
        assert not bad, f"head {hh}: {bad}"
        del kall, vall, eo, edq, edk, edv
    assert torch.isfinite(rs.dq_acc).all()
    for b in rs.owners:
        assert torch.isfinite(rs.dk_acc[b]).all() and torch.isfinite(rs.dv_acc[b]).all()
    del rs
    torch.cuda.empty_cache()


def test_c2_reference_signatures_full_size(gpu):
    """The reference's own signatures at configs 2/3 size, rank 7 of 8:
    ring_causal_attention_forward_with_stats, then ring_causal_attention_backward
    (rs:139-233, rs:281-475) through lc_ring_fwd_with_stats and lc_ring_bwd. The
    backward gets the workspace of lc_ring_bwd_ds_workspace_bytes (32 GiB more),
    so the diagonal pair (hop 0 of both passes) shares dS; the other 7 hops of
    pass 2 recompute dQ.  Heads 0 and 11 in full: the output, dQ of every row,
    and dK/dV of the rank's own shard (from its own queries only: no later rank
    exists)."""
    torch = gpu
    from longctx100m_amd import _lib
    from longctx100m_amd import ring_attention as ra

    world, rank, n, h, d = 8, 7, 32768, 16, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(777)
    rnd = lambda *s: torch.randn(*s, generator=gen, device=dev).to(torch.bfloat16)  # noqa: E731
    qs = [rnd(1, n, h, d) for _ in range(world)]
    ks = [rnd(1, n, h, d) for _ in range(world)]
    vs = [rnd(1, n, h, d) for _ in range(world)]
    go = rnd(1, n, h, d)
    shards = list(zip(qs, ks, vs))
    desc = ra._ring_desc(shards, rank, True, 64, 128, None, None, False)
    lib = _lib.load()
    extra = lib.lc_ring_bwd_ds_workspace_bytes(desc) - lib.lc_ring_bwd_workspace_bytes(desc)
    assert extra == 32 << 30
    print(f"fullsize reference signatures: world={world} rank={rank} n={n} H={h} d={d} bf16, "
          f"dS workspace {extra / 2**30:.1f} GiB", flush=True)
    out, m, l = ra.ring_causal_attention_forward_with_stats(shards, rank)
    # only this rank's forward results and upstream gradient enter its backward (every
    # pass-1 pair of an earlier query owner is masked for the last rank's keys)
    dq, dk, dv = ra.ring_causal_attention_backward(shards, rank, [out] * world, [m] * world,
                                                   [l] * world, [go] * world)
    torch.cuda.synchronize()
    scale = d ** -0.5
    for hh in (0, 11):
        kall = torch.cat([x[0, :, hh] for x in ks], 0).float()
        vall = torch.cat([x[0, :, hh] for x in vs], 0).float()
        eo, em, el, edq, edk, edv = _head_reference(torch, qs[rank][0, :, hh].float(), kall,
                                                    vall, go[0, :, hh].float(), rank * n, scale)
        own = slice(rank * n, (rank + 1) * n)
        errs = {"out": _nrel(out[0, :, hh].float(), eo),
                "m": float(((m[0, hh, :, 0] - em).abs() / em.abs().clamp(min=1.0)).max()),
                "l": float(((l[0, hh, :, 0] - el).abs() / el).max()),
                "dq": _nrel(dq[0, :, hh].float(), edq),
                "dk": _nrel(dk[0, :, hh].float(), edk[own]),
                "dv": _nrel(dv[0, :, hh].float(), edv[own])}
        print(f"fullsize reference signatures head {hh}: " +
              ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
        bad = {k: v for k, v in errs.items()
               if not v <= {"m": 1e-4, "l": 1e-3}.get(k, BF16_TOL)}
        assert not bad, f"head {hh}: {bad}"
        del kall, vall, eo, edq, edk, edv
    del out, m, l, dq, dk, dv
    torch.cuda.empty_cache()


def test_c5_long_shard_full_size(gpu):
    """BASELINE config 5 at its own shape (capacity.rs:162-178): the
    1,000,000-token shard through bench.py --long-shard's launches, sampled
    rows of heads 0 and 13 against an fp32 recompute over every visible key."""
    torch = gpu
    from longctx100m_amd.rank_step import LongShardForward

    n, h, d = 1_000_000, 16, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(4321)
    rnd = lambda *s: torch.randn(*s, generator=gen, device=dev).to(torch.bfloat16)  # noqa: E731
    q = rnd(1, n, h, d)
    ks = [rnd(1, n, h, d) for _ in range(2)]
    vs = [rnd(1, n, h, d) for _ in range(2)]
    print(f"fullsize C5: n={n} H={h} d={d} bf16, diagonal + 1 full shard", flush=True)
    lsf = LongShardForward(q, ks, vs)
    lsf.forward()
    torch.cuda.synchronize()

    rows = [0, 1, 63, 64, 127, 128, 4095, 65535, 65536, 65537, 131071, 131072, 500000,
            983039, 983040, 999935, 999936, 999998, 999999]
    rows += torch.randint(0, n, (13,), generator=gen, device=dev).tolist()
    ridx = torch.tensor(rows, device=dev)
    scale = d ** -0.5
    for hh in (0, 13):
        kall = torch.cat([x[0, :, hh] for x in ks], 0).float()  # [2n, d], key j at position j
        vall = torch.cat([x[0, :, hh] for x in vs], 0).float()
        qr = q[0, ridx, hh].float()
        s = (qr @ kall.t()) * scale
        kpos = torch.arange(2 * n, device=dev)
        s.masked_fill_(kpos[None, :] > (n + ridx)[:, None], float("-inf"))
        em = s.max(dim=1).values
        p = torch.exp(s - em[:, None])
        del s
        el = p.sum(dim=1)
        eo = (p @ vall) / el[:, None]
        del p
        errs = {
            "out": _nrel(lsf.out[0, ridx, hh].float(), eo),
            "m": float(((lsf.m[0, hh, ridx] - em).abs() / em.abs().clamp(min=1.0)).max()),
            "l": float(((lsf.l[0, hh, ridx] - el).abs() / el).max()),
        }
        print(f"fullsize C5 head {hh}: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()),
              flush=True)
        assert errs["out"] <= BF16_TOL and errs["m"] <= 1e-4 and errs["l"] <= 1e-3, errs
        del kall, vall
    assert torch.isfinite(lsf.out.float()).all()
    del lsf
    torch.cuda.empty_cache()


def _gqa_head_reference(torch, q, kall, vall, dout, q_pos0, scale, chunk=1024):
    """_head_reference over the query heads of one GQA group: q, dout [n, g, d];
    kall, vall [N, d] (the group's KV head).  Returns out, m, l, dq [n, g, ...]
    and dk, dv [N, d] summed over the group (model.rs:85-94 expands K/V with
    repeat_interleave, so the gradient of a KV head is its group's sum)."""
    outs, ms, ls, dqs = [], [], [], []
    dk = dv = None
    for j in range(q.shape[1]):
        o, m, l, dq, k_, v_ = _head_reference(torch, q[:, j], kall, vall, dout[:, j], q_pos0,
                                              scale, chunk)
        outs.append(o), ms.append(m), ls.append(l), dqs.append(dq)
        dk = k_ if dk is None else dk + k_
        dv = v_ if dv is None else dv + v_
    st = lambda xs: torch.stack(xs, 1)  # noqa: E731
    return st(outs), st(ms), st(ls), st(dqs), dk, dv


def test_c4_attention_share_full_size_gqa_chunked(gpu):
    """The config-4 model's attention share at its real shape (65,536-token
    shards, GQA Hq=32 / Hkv=8, d=128, rank 3 of 4: diagonal + 3 full hops)
    through the bench's step with a 16 GiB dS workspace, so every hop's pair
    runs in query chunks (the full workspace would be 275 GB).  KV head 5 and
    its 4 query heads are checked in full: output and statistics of every row,
    dQ of every row, dK/dV of every key of every owner (summed over the group)."""
    torch = gpu
    from longctx100m_amd.rank_step import RankStep

    world, rank, n, hq, hkv, d = 4, 3, 65536, 32, 8, 128
    g = hq // hkv
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(2468)
    rnd = lambda *s: torch.randn(*s, generator=gen, device=dev).to(torch.bfloat16)  # noqa: E731
    q = rnd(1, n, hq, d)
    dout = rnd(1, n, hq, d)
    ks = [rnd(1, n, hkv, d) for _ in range(world)]
    vs = [rnd(1, n, hkv, d) for _ in range(world)]
    rs = RankStep(q, dout, ks, vs, rank, share_ds=True, workspace_bytes=16 << 30)
    assert rs.owners == [3, 2, 1, 0]
    assert rs.workspace is not None and rs.workspace.numel() == 16 << 30
    print(f"fullsize C4 share: n={n} Hq={hq} Hkv={hkv} rank {rank} of {world}, "
          f"dS workspace 16 GiB (query chunks)", flush=True)
    rs.step()
    torch.cuda.synchronize()

    kvh = 5
    heads = list(range(kvh * g, (kvh + 1) * g))
    kall = torch.cat([x[0, :, kvh] for x in ks], 0).float()
    vall = torch.cat([x[0, :, kvh] for x in vs], 0).float()
    eo, em, el, edq, edk, edv = _gqa_head_reference(
        torch, q[0, :, heads].float(), kall, vall, dout[0, :, heads].float(), rank * n, d ** -0.5)
    errs = {
        "out": _nrel(rs.out[0, :, heads].float(), eo),
        "dq": _nrel(rs.dq_acc[0, :, heads], edq),
        "m": float(((rs.m[0, heads].t() - em).abs() / em.abs().clamp(min=1.0)).max()),
        "l": float(((rs.l[0, heads].t() - el).abs() / el).max()),
    }
    for b in rs.owners:
        errs[f"dk{b}"] = _nrel(rs.dk_acc[b][0, :, kvh], edk[b * n:(b + 1) * n])
        errs[f"dv{b}"] = _nrel(rs.dv_acc[b][0, :, kvh], edv[b * n:(b + 1) * n])
    print("fullsize C4 share KV head 5: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()),
          flush=True)
    bad = {k: v for k, v in errs.items() if not v <= {"m": 1e-4, "l": 1e-3}.get(k, BF16_TOL)}
    assert not bad, bad
    del rs
    torch.cuda.empty_cache()
