"""One rank's share of the ring, forward then backward, with every input
resident in HBM: the step ``bench.py`` times and the full-size parity tests
check, so both run exactly the same launches.

Forward (ring_attention.rs:139-233): the query shard attends the KV shard of
owner (rank - h) mod world at hop h, fully masked hops skipped; hop 0 writes
the running state, every later hop LSE-merges its result into it in the
forward kernel's epilogue (the carried state of rs:195-225), and a cast
writes the bf16 output (rs:227-231); with ``separate_merge`` each later hop
writes its own partial and lc_attn_merge merges it, the last merge also
writing the bf16 output.

Backward (rs:281-475, one rank's share): the preprocess forms delta from the
cast output and the log2-domain LSE; then, per visited owner, the hop
backward adds dS K into dQ (accumulated across owners) and dS^T Q, P^T dO into
that owner's own dK/dV accumulators (the per-shard gradients a ring sends back
to their owner).  With ``share_ds`` the dK/dV kernel stores dS in a workspace
and dQ is computed from it (lc_attn_bwd_shard_ws); otherwise the dQ kernel
recomputes the scores.
"""

from __future__ import annotations

from typing import Callable, Dict, List, Optional, Sequence

import torch

from . import ring_attention as ra

Timer = Callable[[str, Callable[[], None]], None]


def _run(timed: Optional[Timer], name: str, fn: Callable[[], None]) -> None:
    if timed is None:
        fn()
    else:
        timed(name, fn)


def visited_owners(rank: int, world: int, local_tokens: int,
                   q_pos0: Optional[int] = None) -> List[int]:
    """Owners in hop order whose KV shard has a key visible to the query
    shard (causal), the hops the reference's loop changes the state in."""
    n = local_tokens
    qp = rank * n if q_pos0 is None else q_pos0
    owners = [(rank - hop) % world for hop in range(world)]
    return [b for b in owners if b * n <= qp + n - 1]


class RankStep:
    """Buffers and launches of one rank's forward + backward share.

    ``q`` and ``dout`` are this rank's [B, n, Hq, D] bf16 query shard and
    upstream gradient; ``ks``/``vs`` every rank's [B, n, Hkv, D] KV shards in
    rank order.  ``workspace_bytes`` caps the dS workspace (default: the full
    size, ``lc_attn_bwd_shard_workspace_bytes``).  After :meth:`forward`,
    ``out``/``m``/``l`` hold the rank's output and statistics; after
    :meth:`backward`, ``dq_acc`` holds dQ and ``dk_acc[b]``/``dv_acc[b]`` owner
    b's dK/dV contribution (fp32)."""

    def __init__(self, q: torch.Tensor, dout: torch.Tensor, ks: Sequence[torch.Tensor],
                 vs: Sequence[torch.Tensor], rank: int, *, share_ds: bool = True,
                 workspace_bytes: Optional[int] = None, separate_merge: bool = False):
        self.q, self.dout, self.ks, self.vs, self.rank = q, dout, list(ks), list(vs), rank
        b, n, h, d = q.shape
        self.n = n
        self.q_pos0 = rank * n
        self.owners = visited_owners(rank, len(self.ks), n)
        dev = q.device
        f32 = dict(device=dev, dtype=torch.float32)
        self.o_run = torch.empty(b, n, h, d, **f32)
        self.m = torch.empty(b, h, n, **f32)
        self.l = torch.empty(b, h, n, **f32)
        self.out = torch.empty(b, n, h, d, device=dev, dtype=q.dtype)
        self.separate_merge = separate_merge
        if separate_merge:  # each later hop's partial, merged by lc_attn_merge
            self.o_part = torch.empty_like(self.o_run)
            self.m_part = torch.empty_like(self.m)
            self.l_part = torch.empty_like(self.l)
        self.delta = torch.empty_like(self.m)
        self.lse2 = torch.empty_like(self.m)
        hkv = self.ks[0].shape[2]
        self.dq_acc = torch.empty(b, n, h, d, **f32)
        self.dk_acc: Dict[int, torch.Tensor] = {o: torch.empty(b, n, hkv, d, **f32)
                                                for o in self.owners}
        self.dv_acc: Dict[int, torch.Tensor] = {o: torch.empty(b, n, hkv, d, **f32)
                                                for o in self.owners}
        self.workspace: Optional[torch.Tensor] = None
        if share_ds:
            # the full size holds the dS of up to 65,536 query rows; a smaller workspace runs
            # each hop's pair in query chunks of multiples of 256 rows
            nbytes = ra.bwd_shard_workspace_bytes(q, self.ks[0])
            if nbytes and workspace_bytes is not None:
                nbytes = min(nbytes, workspace_bytes)
            if nbytes:
                self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)

    def tag(self, owner: int) -> str:
        return "diag" if owner == self.rank else "full"

    def forward(self, timed: Optional[Timer] = None) -> None:
        n, qp = self.n, self.q_pos0
        if self.separate_merge:
            for i, b in enumerate(self.owners):
                dst = (self.o_run, self.m, self.l) if i == 0 else (self.o_part, self.m_part,
                                                                   self.l_part)
                _run(timed, f"fwd_{self.tag(b)}", lambda b=b, dst=dst: ra.fwd_shard(
                    self.q, self.ks[b], self.vs[b], q_pos0=qp, k_pos0=b * n,
                    o=dst[0], m=dst[1], l=dst[2]))
                if i > 0:
                    last = i + 1 == len(self.owners)
                    _run(timed, "merge", lambda last=last: ra.merge(
                        self.o_run, self.m, self.l, self.o_part, self.m_part, self.l_part,
                        out=self.out if last else None))
            if len(self.owners) == 1:
                ra.cast(self.o_run, self.out)
            return
        for i, b in enumerate(self.owners):
            _run(timed, f"fwd_{self.tag(b)}", lambda b=b, i=i: ra.fwd_shard(
                self.q, self.ks[b], self.vs[b], q_pos0=qp, k_pos0=b * n,
                o=self.o_run, m=self.m, l=self.l, accumulate=i > 0))
        _run(timed, "cast", lambda: ra.cast(self.o_run, self.out))

    def backward(self, timed: Optional[Timer] = None) -> None:
        n, qp = self.n, self.q_pos0
        _run(timed, "bwd_preprocess", lambda: ra.bwd_preprocess(
            self.out, self.dout, self.m, self.l, self.delta, self.lse2))
        self.dq_acc.zero_()
        for b in self.owners:
            self.dk_acc[b].zero_()
            self.dv_acc[b].zero_()
        for b in self.owners:
            args = (self.q, self.ks[b], self.vs[b], self.dout, self.lse2, self.delta)
            if self.workspace is not None:  # dK/dV stores dS, dQ reads it back
                _run(timed, f"bwd_{self.tag(b)}", lambda b=b, args=args: ra.bwd_shard(
                    *args, q_pos0=qp, k_pos0=b * n, dq_acc=self.dq_acc,
                    dk_acc=self.dk_acc[b], dv_acc=self.dv_acc[b], workspace=self.workspace))
                continue
            _run(timed, f"dq_{self.tag(b)}", lambda b=b, args=args: ra.bwd_shard(
                *args, q_pos0=qp, k_pos0=b * n, dq_acc=self.dq_acc))
            _run(timed, f"dkdv_{self.tag(b)}", lambda b=b, args=args: ra.bwd_shard(
                *args, q_pos0=qp, k_pos0=b * n, dk_acc=self.dk_acc[b], dv_acc=self.dv_acc[b]))

    def step(self, timed: Optional[Timer] = None) -> None:
        self.forward(timed)
        self.backward(timed)


class LongShardForward:
    """BASELINE config 5's forward: the query shard at rank 1 of a 2-shard
    layout attends its diagonal KV shard and one full incoming shard, whose
    result the forward LSE-merges into the diagonal's (``out`` bf16, ``m``/``l``
    fp32 statistics)."""

    def __init__(self, q: torch.Tensor, ks: Sequence[torch.Tensor], vs: Sequence[torch.Tensor]):
        self.q, self.ks, self.vs = q, list(ks), list(vs)
        b, n, h, d = q.shape
        self.n = n
        f32 = dict(device=q.device, dtype=torch.float32)
        self.o_run = torch.empty(b, n, h, d, **f32)
        self.m, self.l = (torch.empty(b, h, n, **f32) for _ in range(2))
        self.out = torch.empty(b, n, h, d, device=q.device, dtype=q.dtype)

    def resident(self) -> List[torch.Tensor]:
        return [self.q, *self.ks, *self.vs, self.o_run, self.m, self.l, self.out]

    def forward(self) -> None:
        n = self.n
        ra.fwd_shard(self.q, self.ks[1], self.vs[1], q_pos0=n, k_pos0=n,
                     o=self.o_run, m=self.m, l=self.l)                      # diagonal
        ra.fwd_shard(self.q, self.ks[0], self.vs[0], q_pos0=n, k_pos0=0,
                     o=self.o_run, m=self.m, l=self.l, accumulate=True)     # full shard
        ra.cast(self.o_run, self.out)
