"""Pins the decoder-layer oracle (oracle/layer.py) against independent library
routines and the mathematics, and the host-side RoPE frequencies of the C ABI
against the oracle.  CPU only."""

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import layer as L

F32 = np.float32


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(10000) * 10.0 ** rng.integers(-6, 6, 10000)).astype(F32)
    x[:4] = [0.0, -0.0, 1e-40, 3.3895314e38]
    want = torch.tensor(x).bfloat16().float().numpy()
    np.testing.assert_array_equal(L.bf16(x), want)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_rmsnorm_matches_torch(dtype):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((33, 512)).astype(F32) * 3
    r = rng.standard_normal((33, 512)).astype(F32)
    w = (1 + 0.1 * rng.standard_normal(512)).astype(F32)
    if dtype == "bf16":
        x, r, w = L.bf16(x), L.bf16(r), L.bf16(w)
    out, h = L.rmsnorm(x, w, 1e-5, residual=r, dtype=dtype)
    th = torch.tensor(x) + torch.tensor(r)
    if dtype == "bf16":
        th = th.bfloat16().float()
    np.testing.assert_array_equal(h, th.numpy())
    normed = torch.nn.functional.rms_norm(th.double(), (512,), eps=1e-5).float()
    if dtype == "bf16":
        want = (normed.bfloat16() * torch.tensor(w).bfloat16()).float().numpy()
        assert np.max(np.abs(out - want) / np.maximum(np.abs(want), 1e-3)) <= 2 ** -7
    else:
        want = (normed * torch.tensor(w)).numpy()
        np.testing.assert_allclose(out, want, rtol=2e-6, atol=1e-7)


def test_rope_inv_freq_closed_form_and_profiles():
    d, theta = 128, 500000.0
    inv, cf, ps = L.rope_inv_freq(d, theta)
    exact = theta ** (-np.arange(0, d, 2, dtype=np.float64) / d)
    np.testing.assert_allclose(inv, exact, rtol=3e-6)
    assert cf == 1 and ps is None
    inv_l, _, ps_l = L.rope_inv_freq(d, theta, rope_type="linear", factor=4.0)
    np.testing.assert_array_equal(inv_l, inv)
    assert ps_l == F32(0.25)
    with pytest.raises(ValueError, match="rope scaling factor must be positive"):
        L.rope_inv_freq(d, theta, rope_type="linear", factor=0.0)
    with pytest.raises(ValueError, match="invalid llama3 RoPE scaling values"):
        L.rope_inv_freq(d, theta, rope_type="llama3", factor=8, low_freq_factor=4,
                        high_freq_factor=1, original_max_position_embeddings=8192)


def test_rope_llama3_follows_the_rust_wavelength():
    """rope.rs:70 forms the wavelength as inv * 2*pi / inv (= 2*pi), so with the
    usual factors no frequency is rescaled and only the cosine factor applies;
    the Python reference (model.py:159, 2*pi / inv) rescales the low
    frequencies.  Both are computed here to show where they part."""
    d, theta = 128, 500000.0
    kw = dict(rope_type="llama3", factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
              original_max_position_embeddings=8192, attention_factor=1.25)
    inv, cf, _ = L.rope_inv_freq(d, theta, **kw)
    base, _, _ = L.rope_inv_freq(d, theta)
    np.testing.assert_array_equal(inv, base)
    assert cf == F32(1.25)
    # the Python formula, in float64, does rescale
    wl = 2 * math.pi / base.astype(np.float64)
    assert np.any(wl > 8192 / 1.0)


def test_rope_table_matches_torch_float32():
    inv, cf, ps = L.rope_inv_freq(128, 500000.0)
    pos0, n = 3 * 65536 - 100, 300
    tab = L.rope_table(inv, cf, ps, n, pos0)
    f = torch.outer(torch.arange(pos0, pos0 + n).float(), torch.tensor(inv))
    np.testing.assert_allclose(tab[:, 0], f.cos().numpy(), rtol=0, atol=3e-7)
    np.testing.assert_allclose(tab[:, 1], f.sin().numpy(), rtol=0, atol=3e-7)


def test_rope_apply_is_a_rotation():
    rng = np.random.default_rng(2)
    T, H, D = 64, 3, 128
    x = rng.standard_normal((T, H, D)).astype(F32)
    inv, cf, ps = L.rope_inv_freq(D, 10000.0)
    tab = L.rope_table(inv, cf, ps, T, 0)
    y = L.rope_apply(x, tab, dtype="f32")
    # position 0 is the identity
    np.testing.assert_array_equal(y[0], x[0])
    # complex form: (x1 + i x2) * (cos + i sin)
    z = (x[..., :D // 2] + 1j * x[..., D // 2:].astype(np.float64)) * \
        (tab[:, 0, None, :] + 1j * tab[:, 1, None, :].astype(np.float64))
    np.testing.assert_allclose(y[..., :D // 2], z.real, rtol=0, atol=2e-6)
    np.testing.assert_allclose(y[..., D // 2:], z.imag, rtol=0, atol=2e-6)
    # pair norms are preserved
    np.testing.assert_allclose(np.abs(z), np.hypot(x[..., :D // 2], x[..., D // 2:]), rtol=1e-6)
    # scores depend on the position difference only
    q = rng.standard_normal((1, 1, D)).astype(F32)
    k = rng.standard_normal((1, 1, D)).astype(F32)
    tq = L.rope_table(inv, cf, ps, 1, 40)
    tk = L.rope_table(inv, cf, ps, 1, 33)
    tq2 = L.rope_table(inv, cf, ps, 1, 17)
    tk2 = L.rope_table(inv, cf, ps, 1, 10)
    s1 = float((L.rope_apply(q, tq, dtype="f32") * L.rope_apply(k, tk, dtype="f32")).sum())
    s2 = float((L.rope_apply(q, tq2, dtype="f32") * L.rope_apply(k, tk2, dtype="f32")).sum())
    assert abs(s1 - s2) <= 1e-4 * max(1.0, abs(s1))


def test_swiglu_matches_torch():
    rng = np.random.default_rng(3)
    g = (rng.standard_normal((17, 64)) * 6).astype(F32)
    u = rng.standard_normal((17, 64)).astype(F32)
    g[0, :3] = [-200.0, 200.0, 0.0]
    out = L.swiglu(g, u, dtype="f32")
    want = (torch.nn.functional.silu(torch.tensor(g).double()) * torch.tensor(u).double()).numpy()
    np.testing.assert_allclose(out, want, rtol=3e-6, atol=1e-30)
    gb, ub = L.bf16(g), L.bf16(u)
    outb = L.swiglu(gb, ub, dtype="bf16")
    wantb = (torch.nn.functional.silu(torch.tensor(gb)).bfloat16() *
             torch.tensor(ub).bfloat16()).float().numpy()
    assert np.max(np.abs(outb - wantb) / np.maximum(np.abs(wantb), 1e-3)) <= 2 ** -7


# -- the C ABI's host-side RoPE frequencies (no GPU needed) --------------------

def _c_inv(**kw):
    from longctx100m_amd import _lib

    lib = _lib.load()
    r = _lib.Rope(kw.get("head_dim", 128), kw.get("type", 0), kw.get("theta", 500000.0),
                  kw.get("factor", 1.0), kw.get("low", 0.0), kw.get("high", 0.0),
                  kw.get("orig", 0.0), kw.get("af", 1.0))
    half = r.head_dim // 2
    inv = (ctypes.c_float * half)()
    cf = ctypes.c_float()
    rc = lib.lc_rope_inv_freq(ctypes.byref(r), ctypes.addressof(inv), ctypes.addressof(cf))
    return rc, np.array(list(inv), dtype=F32), F32(cf.value), lib.lc_last_error().decode()


@pytest.mark.parametrize("theta,d", [(500000.0, 128), (10000.0, 64), (1e6, 256)])
def test_c_rope_inv_freq_matches_oracle(theta, d):
    rc, inv, cf, _ = _c_inv(theta=theta, head_dim=d)
    assert rc == 0
    want, wcf, _ = L.rope_inv_freq(d, theta)
    # expf of the same fp32 argument: libm and numpy agree to 1 ulp
    assert np.max(np.abs(inv - want) / want) <= 2 ** -23
    assert cf == wcf
    rc, inv3, cf3, _ = _c_inv(theta=theta, head_dim=d, type=2, factor=8.0, low=1.0, high=4.0,
                              orig=8192.0, af=1.25)
    want3, wcf3, _ = L.rope_inv_freq(d, theta, rope_type="llama3", factor=8.0,
                                     low_freq_factor=1.0, high_freq_factor=4.0,
                                     original_max_position_embeddings=8192,
                                     attention_factor=1.25)
    assert rc == 0 and cf3 == wcf3
    assert np.max(np.abs(inv3 - want3) / want3) <= 2 ** -23


@pytest.mark.parametrize("kw,msg", [
    (dict(type=1, factor=0.0), "rope scaling factor must be positive"),
    (dict(type=2, low=4.0, high=1.0, orig=8192.0), "invalid llama3 RoPE scaling values"),
    (dict(type=2, low=1.0, high=4.0, orig=8192.0, af=0.0), "llama3 attention_factor must be positive"),
    (dict(type=7), "unsupported RoPE type 7"),
    (dict(head_dim=127), "head dimension must be even for rotary embeddings"),
])
def test_c_rope_validation_messages(kw, msg):
    rc, _, _, err = _c_inv(**kw)
    assert rc == 1 and err == msg
