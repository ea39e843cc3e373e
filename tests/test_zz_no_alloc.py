"""lc_attn_decode_static, the decode entry point that allocates nothing (its
split partials live in a file-scope device array), against lc_attn_decode
with a caller workspace: same kernels, so the outputs must be identical, on
two calls in a row with the second smaller; and the fp64 dense oracle within
the bf16 bar.  The size check runs without a GPU (it rejects before any
device work)."""

import ctypes
import zlib

import numpy as np
import pytest

from longctx100m_amd import _lib
from oracle import dense
from tests.conftest import norm_rel


def _shape(b, nq, nk, hq, hkv, d=128):
    return _lib.Shape(b, nq, nk, hq, hkv, d, _lib.LC_DTYPE_BF16, 0)


def test_static_decode_rejects_oversized_scratch():
    lib = _lib.load()
    # 65,536 query heads over 4,096 KV heads, one query: one split of 65,536
    # rows needs ~34 MB of partials, above the 16 MiB array.
    s = _shape(1, 1, 64, 65536, 4096)
    need = lib.lc_attn_decode_workspace_bytes(ctypes.byref(s))
    assert need > _lib.LC_DECODE_STATIC_SCRATCH_BYTES
    mk = _lib.Mask(63, 0, -1, 1, 0)
    fake = 1 << 20  # never dereferenced: the call returns before any device work
    rc = lib.lc_attn_decode_static(ctypes.byref(s), ctypes.byref(mk), fake, fake, fake, fake,
                                   fake, fake, None)
    assert rc == _lib.LC_ERR_WORKSPACE
    msg = lib.lc_last_error().decode()
    assert "more than the static maximum of 16777216" in msg and "lc_attn_decode" in msg


CASES = [
    # b, nq, nk, hq, hkv, q_pos0, valid: C4-style GQA over a 70k-key cache,
    # then a smaller call (batch 2, two queries, valid_length) reusing the array
    (1, 1, 70000, 32, 8, 69999, None),
    (2, 2, 5000, 8, 2, 4998, 4900),
]


@pytest.mark.gpu
def test_static_decode_matches_workspace_entry(gpu):
    torch = gpu
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for case in CASES:
        b, nq, nk, hq, hkv, qp, valid = case
        print(f"no-alloc decode case {case}", flush=True)
        rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
        mk = lambda *sh: torch.tensor(rng.standard_normal(sh), dtype=torch.float32).to(  # noqa: E731
            torch.bfloat16).cuda()
        q, k, v = mk(b, nq, hq, 128), mk(b, nk, hkv, 128), mk(b, nk, hkv, 128)
        s = _shape(b, nq, nk, hq, hkv)
        mask = _lib.Mask(qp, 0, -1 if valid is None else valid, 1, 0)
        need = lib.lc_attn_decode_workspace_bytes(ctypes.byref(s))
        assert 0 < need <= _lib.LC_DECODE_STATIC_SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        outs = {}
        for name in ("workspace", "static"):
            o = torch.full((b, nq, hq, 128), float("nan"), device="cuda")
            m = torch.full((b, hq, nq), float("nan"), device="cuda")
            l = torch.full((b, hq, nq), float("nan"), device="cuda")
            ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), m.data_ptr(),
                    l.data_ptr())
            if name == "workspace":
                rc = lib.lc_attn_decode(ctypes.byref(s), ctypes.byref(mask), *ptrs,
                                        ws.data_ptr(), need, stream)
            else:
                rc = lib.lc_attn_decode_static(ctypes.byref(s), ctypes.byref(mask), *ptrs,
                                               stream)
            assert rc == 0, lib.lc_last_error().decode()
            outs[name] = (o, m, l)
        torch.cuda.synchronize()
        for a, bb in zip(outs["workspace"], outs["static"]):
            assert torch.equal(a, bb)
        eo, em, el = dense.attention_fwd(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                         v.float().cpu().numpy(), q_pos0=qp, k_pos0=0,
                                         valid_length=valid)
        o, m, l = (x.cpu().numpy() for x in outs["static"])
        assert norm_rel(o, eo) <= 2e-2
        assert np.abs(m - em).max() <= 1e-4 * max(1.0, np.abs(em).max())
        assert norm_rel(l, el) <= 1e-4
