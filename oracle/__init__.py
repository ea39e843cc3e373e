"""Parity oracle for longctx100m's exact causal ring attention.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing
measured or shipped.  The product package (longctx100m_amd) does not import it.

Two independent oracles live here:

* ``ring`` -- ctypes bindings to ``ring_ref.c``, a C restatement of the
  reference's blocked fp32 algorithm (rust/longctx100m-model/src/
  ring_attention.rs:15-475).  Also the timed CPU baseline.
* ``dense`` -- an fp64 brute-force dense attention with closed-form gradients
  (numpy).  It pins the restatement through the reference's own invariant:
  a rank's ring output equals its rows of dense causal attention over the
  concatenated sequence (tests/test_ring_attention.py:300 and
  ring_attention.rs:548-561 in the reference).
* ``layer`` -- numpy float32 restatements of the decoder-layer row ops around
  attention (RMSNorm, RoPE, SwiGLU; model.rs and rope.rs).
"""

from . import dense, layer, ring  # noqa: F401
