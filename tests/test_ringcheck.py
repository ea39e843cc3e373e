"""The ringcheck-format parity driver (longctx100m_amd.ringcheck), mirroring
rust/longctx100m-model/src/bin/ringcheck.rs and the ring checks of
scripts/verify_model_parity.py:337-380.

CPU tests cover spec parsing, the Rust float format and the error texts that
are raised before any GPU work; the GPU tests run the parity script's own
case (world 2, t = 4 per rank, h = 2, d = 4, torch seed 7) and compare with
the fp64 dense oracle at the script's bar (max abs 1e-4) and the fp32 bar
(1e-5 norm-relative)."""

import json

import numpy as np
import pytest

from longctx100m_amd import ringcheck as rc
from oracle import dense
from tests.conftest import norm_rel


def _tensor(a):
    a = np.asarray(a, dtype=np.float32)
    return {"data": a.ravel().tolist(), "shape": list(a.shape)}


def _spec(shards, rank, grad_out=None, **extra):
    spec = {
        "world_size": len(shards),
        "rank": rank,
        "q": [_tensor(q) for q, _, _ in shards],
        "k": [_tensor(k) for _, k, _ in shards],
        "v": [_tensor(v) for _, _, v in shards],
    }
    if grad_out is not None:
        spec["grad_out"] = _tensor(grad_out)
    spec.update(extra)
    return spec


def _shards(seed=0, world=2, t=4, h=2, d=4):
    rng = np.random.default_rng(seed)
    return [tuple(rng.standard_normal((1, t, h, d)).astype(np.float32) for _ in range(3))
            for _ in range(world)]


def test_rust_float_format():
    cases = {1.0: "1.0", -0.25: "-0.25", 0.1: "0.1", 0.0: "0.0", 100.0: "100.0",
             1e-4: "0.0001", 1e-7: "1e-7", 1.5e-5: "1.5e-5", 2.5e16: "2.5e16",
             123456.5: "123456.5", float("nan"): "NaN", float("inf"): "inf",
             float("-inf"): "-inf"}
    for x, want in cases.items():
        assert rc.rust_f32_debug(x) == want, (x, rc.rust_f32_debug(x))
    # shortest digits that round-trip in fp32
    for x in np.random.default_rng(1).standard_normal(200).astype(np.float32):
        assert np.float32(float(rc.rust_f32_debug(x))) == x


def test_output_lines_are_json():
    out = np.arange(6, dtype=np.float32).reshape(1, 3, 1, 2) / 8
    line = rc.format_output(1, out)
    assert line == '{"rank": 1, "output": [0.0, 0.125, 0.25, 0.375, 0.5, 0.625]}'
    assert json.loads(line)["output"] == out.ravel().tolist()
    bl = json.loads(rc.format_backward(0, out, 2 * out, -out))
    assert set(bl) == {"rank", "dq", "dk", "dv"} and bl["dv"][1] == -0.125


def test_spec_defaults_and_tensors():
    shards = _shards()
    spec = rc.parse_spec(_spec(shards, 1), backward=False)
    assert (spec.world, spec.rank, spec.block_q, spec.block_k) == (2, 1, 2, 3)
    assert spec.valid_length is None and spec.q_position_start is None
    np.testing.assert_array_equal(spec.k[1], shards[1][1])
    spec = rc.parse_spec(_spec(shards, 0, grad_out=np.ones((1, 8, 2, 4)), block_q=5,
                               valid_length=7, q_position_start=None), backward=True)
    assert spec.block_q == 5 and spec.valid_length == 7 and spec.grad_out.shape == (1, 8, 2, 4)


def test_errors_before_gpu_work(tmp_path, capsys):
    assert rc.main([]) == 1
    assert capsys.readouterr().err.strip() == f"Error: {rc.USAGE}"

    def run(spec, *flags):
        p = tmp_path / "spec.json"
        p.write_text(json.dumps(spec))
        code = rc.main([str(p), *flags])
        return code, capsys.readouterr().err.strip()

    shards = _shards()
    assert run(_spec(shards, 2)) == (1, "Error: rank 2 out of range for world_size 2")
    bad = [shards[0], (shards[1][0], shards[1][1][:, :3], shards[1][2])]
    assert run(_spec(bad, 0)) == (1, "Error: q, k, v shard shapes must match")
    assert run(_spec(shards, 0), "--backward")[1] == \
        'Error: spec field "grad_out" is required with --backward'
    # rejected by the library's validation (rs:148-171) before any HIP call
    assert run(_spec(shards, 0, block_q=0)) == (1, "Error: block_q and block_k must be positive")
    assert run(_spec(shards, 0, valid_length=9)) == \
        (1, "Error: valid_length must be within the padded distributed sequence")
    code, err = run({"world_size": 1, "rank": 0, "q": [{"data": [1, 2], "shape": [1, 1, 1, 3]}],
                     "k": [], "v": []})
    assert code == 1 and err.startswith("Error: ")


# ---------------------------------------------------------------------- GPU --

def _script_case():
    """verify_model_parity.py:349-361: torch.manual_seed(7), world 2, t = 4,
    h = 2, d = 4, randn q, k, v per rank in rank order."""
    torch = pytest.importorskip("torch")
    torch.manual_seed(7)
    shards = [tuple(torch.randn(1, 4, 2, 4).numpy() for _ in range(3)) for _ in range(2)]
    return shards


@pytest.mark.gpu
def test_script_ring_forward_case(gpu, tmp_path, capsys):
    shards = _script_case()
    q = np.concatenate([s[0] for s in shards], 1)
    k = np.concatenate([s[1] for s in shards], 1)
    v = np.concatenate([s[2] for s in shards], 1)
    ref = dense.attention_fwd(q, k, v)[0]
    for rank in range(2):
        p = tmp_path / f"spec{rank}.json"
        p.write_text(json.dumps(_spec(shards, rank)))
        assert rc.main([str(p)]) == 0
        line = json.loads(capsys.readouterr().out.strip())
        assert line["rank"] == rank
        got = np.asarray(line["output"], np.float64)
        want = ref[0, rank * 4:(rank + 1) * 4].ravel()
        assert np.abs(got - want).max() < 1e-4  # the script's bar
        assert norm_rel(got, want) <= 1e-5


@pytest.mark.gpu
def test_script_ring_backward_case(gpu, tmp_path, capsys):
    """grad_out = ones of the full sequence (verify_model_parity.py:370-372),
    handed to every rank; dq/dk/dv against the dense gradients of loss = sum."""
    shards = _script_case()
    q = np.concatenate([s[0] for s in shards], 1)
    k = np.concatenate([s[1] for s in shards], 1)
    v = np.concatenate([s[2] for s in shards], 1)
    go = np.ones((1, 8, 2, 4), np.float32)
    edq, edk, edv = dense.attention_bwd(q, k, v, go)
    for rank in range(2):
        p = tmp_path / f"bspec{rank}.json"
        p.write_text(json.dumps(_spec(shards, rank, grad_out=go)))
        assert rc.main([str(p), "--backward"]) == 0
        line = json.loads(capsys.readouterr().out.strip())
        assert line["rank"] == rank
        sl = slice(rank * 4, (rank + 1) * 4)
        for name, want in (("dq", edq), ("dk", edk), ("dv", edv)):
            got = np.asarray(line[name], np.float64)
            w = want[0, sl].ravel()
            assert np.abs(got - w).max() < 1e-4, name
            assert norm_rel(got, w) <= 1e-5, name


@pytest.mark.gpu
def test_valid_length_and_blocks_case(gpu, tmp_path, capsys):
    """A padded tail (valid_length) and non-default blocks through the driver."""
    shards = _shards(seed=3, world=3, t=5, h=2, d=8)
    q = np.concatenate([s[0] for s in shards], 1)
    k = np.concatenate([s[1] for s in shards], 1)
    v = np.concatenate([s[2] for s in shards], 1)
    ref = dense.attention_fwd(q, k, v, valid_length=12)[0]
    p = tmp_path / "spec.json"
    p.write_text(json.dumps(_spec(shards, 2, block_q=4, block_k=2, valid_length=12)))
    assert rc.main([str(p)]) == 0
    got = np.asarray(json.loads(capsys.readouterr().out.strip())["output"], np.float64)
    assert norm_rel(got, ref[0, 10:15].ravel()) <= 1e-5
