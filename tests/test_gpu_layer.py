"""GPU parity of the decoder-layer row kernels (include/longctx100m_layer.h)
and of one composed layer against the numpy oracle (oracle/layer.py, with
oracle/dense.py for the attention).

Bars: bf16 results within one bf16 ulp of the oracle (2^-7 relative, the two
roundings the reference makes can each land on the other side; for RMSNorm a
few elements in 10^5 within two, from the fp32 sum of squares), fp32 within
2e-6 relative; RoPE given the same table and the fused residual add are
bit-exact; the composed bf16 layer within 2e-2 norm-relative.
"""

import numpy as np
import pytest

from oracle import dense
from oracle import layer as L
from tests.conftest import norm_rel

pytestmark = pytest.mark.gpu

BF16_ULP = 2.0 ** -7


@pytest.fixture(scope="module")
def ly(gpu):
    from longctx100m_amd import layer

    return layer


def _t(gpu, arr, dtype):
    return gpu.tensor(np.ascontiguousarray(arr), dtype=gpu.float32).to(dtype).cuda()


def _np(t):
    return t.detach().float().cpu().numpy()


def _close(got, want, dtype, rare=0.0):
    """bf16: within one ulp; with rare > 0 up to rare * size + 2 elements may be
    within two (the kernel sums squares in fp32, the oracle in float64: the
    ~1e-7 difference moves h * inv across a bf16 rounding boundary for ~1e-5
    of the elements, and the rounding after the weight can add one ulp more;
    a 300-case random sweep measured up to 1.1e-5)."""
    if dtype == "bf16":
        rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-30)
        far = np.abs(got - want) > 1e-30
        bad = (rel > BF16_ULP) & far
        assert not ((rel > 2 * BF16_ULP) & far).any(), (got[bad][:5], want[bad][:5])
        limit = rare * bad.size + (2 if rare > 0 else 0)
        assert bad.sum() <= limit, (bad.sum(), got[bad][:5], want[bad][:5])
    else:
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-30)


def _dt(gpu, name):
    return gpu.bfloat16 if name == "bf16" else gpu.float32


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rows,cols,with_res", [(37, 4096, False), (64, 1000, True), (5, 16384, True),
                                                 (2000, 4096, True), (3, 6000, True),
                                                 (9, 16384, False)])
def test_rmsnorm(ly, gpu, dtype, rows, cols, with_res):
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 2
    r = rng.standard_normal((rows, cols)).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(cols)).astype(np.float32)
    if dtype == "bf16":
        x, r, w = L.bf16(x), L.bf16(r), L.bf16(w)
    tdt = _dt(gpu, dtype)
    # x as a strided view (row stride cols + 16)
    xbig = _t(gpu, np.pad(x, ((0, 0), (0, 16))), tdt)
    xv = xbig[:, :cols]
    tw = _t(gpu, w, tdt)
    if with_res:
        tr = _t(gpu, r, tdt)
        # residual_out contiguous while x is strided: each operand uses its own row stride
        hout = gpu.full((rows + 1, cols), 7.0, dtype=tdt, device="cuda")
        out = ly.rmsnorm(xv, tw, 1e-5, residual=tr, residual_out=hout[:rows])
        want, h = L.rmsnorm(x, w, 1e-5, residual=r, dtype=dtype)
        np.testing.assert_array_equal(_np(hout[:rows]), h)
        assert (_np(hout[rows]) == 7.0).all()  # nothing written past the last row
    else:
        out = ly.rmsnorm(xv, tw, 1e-5)
        want, _ = L.rmsnorm(x, w, 1e-5, dtype=dtype)
    gpu.cuda.synchronize()
    _close(_np(out), want, dtype, rare=5e-5)


@pytest.mark.parametrize("scaling", [None, {"rope_type": "linear", "factor": 4.0},
                                     {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                      "high_freq_factor": 4.0,
                                      "original_max_position_embeddings": 8192,
                                      "attention_factor": 1.25}])
def test_rope_table(ly, gpu, scaling):
    d, theta, n, pos0 = 128, 500000.0, 700, 3 * 65536 - 300
    rope = ly.rope_params(d, theta, scaling)
    tab = _np(ly.rope_table(rope, n, pos0))
    kw = {}
    if scaling:
        kw = {k: v for k, v in scaling.items() if k != "rope_type"}
        kw["rope_type"] = scaling["rope_type"]
    inv, cf, ps = L.rope_inv_freq(d, theta, **kw)
    want = L.rope_table(inv, cf, ps, n, pos0)
    # the same fp32 angle; device and host cos/sin agree to a couple of ulp
    np.testing.assert_allclose(tab, want, rtol=0, atol=4e-7)


@pytest.mark.parametrize("T", [96, 1100])  # 1100 tokens: the non-temporal (prefill) kernel
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_rope_apply_strided_and_in_place(ly, gpu, dtype, T):
    rng = np.random.default_rng(5)
    hq, hkv, d = 6, 2, 128
    tdt = _dt(gpu, dtype)
    qkv = rng.standard_normal((T, (hq + 2 * hkv) * d)).astype(np.float32)
    if dtype == "bf16":
        qkv = L.bf16(qkv)
    tq = _t(gpu, qkv, tdt)
    rope = ly.rope_params(d, 500000.0)
    table = ly.rope_table(rope, T, 12345)
    q = ly.rope_apply(tq[:, :hq * d], table, hq, d)
    k = ly.rope_apply(tq[:, hq * d:(hq + hkv) * d], table, hkv, d)
    gtab = _np(table)
    np.testing.assert_array_equal(_np(q), L.rope_apply(qkv[:, :hq * d].reshape(T, hq, d), gtab, dtype=dtype))
    np.testing.assert_array_equal(_np(k), L.rope_apply(qkv[:, hq * d:(hq + hkv) * d].reshape(T, hkv, d), gtab, dtype=dtype))
    # in place on a contiguous tensor
    kc = _t(gpu, qkv[:, hq * d:(hq + hkv) * d], tdt)
    ly.rope_apply(kc, table, hkv, d, out=kc.view(T, hkv, d))
    np.testing.assert_array_equal(_np(kc).reshape(T, hkv, d), _np(k))


@pytest.mark.parametrize("rows", [33, 1100])  # 1100 rows: the non-temporal (prefill) kernel
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_swiglu(ly, gpu, dtype, rows):
    rng = np.random.default_rng(6)
    inter = 2048
    gu = (rng.standard_normal((rows, 2 * inter)) * 4).astype(np.float32)
    gu[0, :4] = [-120.0, 120.0, 0.0, -0.0]
    if dtype == "bf16":
        gu = L.bf16(gu)
    t = _t(gpu, gu, _dt(gpu, dtype))
    out = ly.swiglu(t[:, :inter], t[:, inter:])
    gpu.cuda.synchronize()
    _close(_np(out), L.swiglu(gu[:, :inter], gu[:, inter:], dtype=dtype), dtype)


def test_layer_prefill_reduced(ly, gpu):
    """One decoder layer (hidden 1024, GQA 8/2, d 128, intermediate 2048, bf16)
    on rank 1 of a 2-rank ring, 256 tokens per shard, against the oracle
    composition (GEMMs in fp32 on the bf16 operands, rounded to bf16)."""
    import torch

    cfg = ly.ModelConfig(hidden_size=1024, num_heads=8, num_key_value_heads=2,
                         intermediate_size=2048, num_layers=1, rope_theta=500000.0)
    T, rank, d = 256, 1, cfg.head_dim
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    w = ly.init_layer_weights(cfg, gen, "cuda", std=0.05)
    w["norm1"] = (1 + 0.1 * torch.randn(1024, generator=gen, device="cuda")).to(torch.bfloat16)
    w["norm2"] = (1 + 0.1 * torch.randn(1024, generator=gen, device="cuda")).to(torch.bfloat16)
    x = torch.randn(T, 1024, generator=gen, device="cuda").to(torch.bfloat16)
    res = (0.5 * torch.randn(T, 1024, generator=gen, device="cuda")).to(torch.bfloat16)
    pk = torch.randn(1, T, 2, d, generator=gen, device="cuda").to(torch.bfloat16)
    pv = torch.randn(1, T, 2, d, generator=gen, device="cuda").to(torch.bfloat16)
    table = ly.rope_table(ly.rope_params(d, cfg.rope_theta), T, rank * T)
    x2, mlp = ly.layer_prefill(x, w, cfg, table, rank, [(pk, pv)], residual=res)
    gpu.cuda.synchronize()

    W = {k: _np(v) for k, v in w.items()}
    xn, rn = _np(x), _np(res)
    gtab = _np(table)

    def gemm(a, b):  # a @ b.T, fp32 accumulate, bf16 result
        return L.bf16(a.astype(np.float64) @ b.astype(np.float64).T)

    h, xin = L.rmsnorm(xn, W["norm1"], cfg.rms_norm_eps, residual=rn)
    qkv = gemm(h, W["wqkv"])
    q = L.rope_apply(qkv[:, :8 * d].reshape(T, 8, d), gtab)
    k = L.rope_apply(qkv[:, 8 * d:10 * d].reshape(T, 2, d), gtab)
    v = qkv[:, 10 * d:].reshape(T, 2, d)
    kall = np.concatenate([_np(pk)[0], k], 0)[None]
    vall = np.concatenate([_np(pv)[0], v], 0)[None]
    att = L.bf16(dense.attention_fwd(q[None], kall, vall, q_pos0=rank * T, k_pos0=0)[0][0])
    o = gemm(att.reshape(T, 8 * d), W["wo"])
    h2, x2w = L.rmsnorm(xin, W["norm2"], cfg.rms_norm_eps, residual=o)
    gu = gemm(h2, W["wgu"])
    a = L.swiglu(gu[:, :2048], gu[:, 2048:])
    mlpw = gemm(a, W["wd"])
    assert norm_rel(_np(x2), x2w) <= 2e-2
    assert norm_rel(_np(mlp), mlpw) <= 2e-2


def test_layer_prefill_c4_shape(ly, gpu):
    """Config 4's decoder layer at its own shape (model.rs:387-393): hidden 4096,
    GQA 32/8, d 128, SwiGLU 14336, RoPE theta 5e5, bf16 weights N(0, 0.02), rank 3
    of a 4-rank ring with 65,536 tokens per shard, so every query attends the 3
    preceding KV shards and its own shard's keys up to it (196,609-262,144 keys).
    The GPU computes the whole layer; 14 rows (shard ends, tile and wave
    boundaries, random) are recomputed by the oracle composition in float64:
    RMSNorm with the residual add, the projections on the bf16 operands rounded to
    bf16, RoPE, attention of the row over every visible key, the output projection,
    the second RMSNorm, SwiGLU and the down projection.  The oracle's K and V rows
    of this shard (every one a sampled query sees) come from the oracle RMSNorm and
    RoPE with the K/V projection as a float32 GEMM (torch) rounded to bf16; those
    rows are checked against the float64 projection at the sampled rows."""
    import torch

    cfg = ly.C4
    T, rank, d, hq, hkv = 65536, 3, cfg.head_dim, cfg.num_heads, cfg.num_key_value_heads
    c, inter = cfg.hidden_size, cfg.intermediate_size
    gen = torch.Generator(device="cuda")
    gen.manual_seed(404)
    w = ly.init_layer_weights(cfg, gen, "cuda")
    w["norm1"] = (1 + 0.1 * torch.randn(c, generator=gen, device="cuda")).to(torch.bfloat16)
    w["norm2"] = (1 + 0.1 * torch.randn(c, generator=gen, device="cuda")).to(torch.bfloat16)
    x = torch.randn(T, c, generator=gen, device="cuda").to(torch.bfloat16)
    res = (0.5 * torch.randn(T, c, generator=gen, device="cuda")).to(torch.bfloat16)
    pre = [tuple((1.3 * torch.randn(1, T, hkv, d, generator=gen, device="cuda")).to(torch.bfloat16)
                 for _ in range(2)) for _ in range(rank)]
    table = ly.rope_table(ly.rope_params(d, cfg.rope_theta), T, rank * T)
    x2, mlp = ly.layer_prefill(x, w, cfg, table, rank, pre, residual=res)
    gpu.cuda.synchronize()
    rows = np.array([0, 1, 31, 32, 255, 256, 4095, 4096, 32767, 32768, 50001, 65279, 65534,
                     65535])
    got_x2, got_mlp = _np(x2[rows]), _np(mlp[rows])
    del x2, mlp

    # oracle: first RMSNorm of every row (its K/V rows are visible to later queries)
    W = {k: _np(v) for k, v in w.items()}
    h_all, xin_all = L.rmsnorm(_np(x), W["norm1"], cfg.rms_norm_eps, residual=_np(res))
    hb = torch.tensor(h_all, device="cuda")
    wkv = w["wqkv"][hq * d:].float()
    kvp = L.bf16(_np(hb @ wkv.t()))  # [T, 2 * hkv * d], float32 GEMM of the bf16 operands
    del hb, wkv
    gtab = _np(table)
    k_loc = L.rope_apply(kvp[:, :hkv * d].reshape(T, hkv, d), gtab)
    v_loc = kvp[:, hkv * d:].reshape(T, hkv, d)
    del kvp

    def gemm(a, b):  # a @ b.T on the bf16 operands in float64, rounded to bf16
        return L.bf16(a.astype(np.float64) @ b.astype(np.float64).T)

    h_r = h_all[rows]
    qkv = gemm(h_r, W["wqkv"])
    q = L.rope_apply(qkv[:, :hq * d].reshape(len(rows), hq, d), gtab[rows])
    k_chk = L.rope_apply(qkv[:, hq * d:(hq + hkv) * d].reshape(len(rows), hkv, d), gtab[rows])
    # the float32-GEMM K/V rows equal the float64 ones up to a bf16 rounding step
    assert np.abs(k_chk - k_loc[rows]).max() <= 2 * BF16_ULP * np.abs(k_chk).max()
    assert np.abs(qkv[:, (hq + hkv) * d:].reshape(len(rows), hkv, d) - v_loc[rows]).max() <= \
        2 * BF16_ULP * np.abs(v_loc[rows]).max()
    n_pre = rank * T
    g = hq // hkv
    scale = 1.0 / np.sqrt(d)
    att = np.zeros((len(rows), hq, d))
    for kh in range(hkv):
        K = np.concatenate([_np(p[0][0, :, kh]) for p in pre] + [k_loc[:, kh]]).astype(np.float64)
        V = np.concatenate([_np(p[1][0, :, kh]) for p in pre] + [v_loc[:, kh]]).astype(np.float64)
        Q = q[:, kh * g:(kh + 1) * g].astype(np.float64).reshape(-1, d)  # [rows * g, d]
        s = (Q @ K.T) * scale
        vis = np.arange(K.shape[0])[None, :] <= (n_pre + np.repeat(rows, g))[:, None]
        s = np.where(vis, s, -np.inf)
        s -= s.max(1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(1, keepdims=True)
        att[:, kh * g:(kh + 1) * g] = (p @ V).reshape(len(rows), g, d)
    o = gemm(L.bf16(att).reshape(len(rows), hq * d), W["wo"])
    h2, x2w = L.rmsnorm(xin_all[rows], W["norm2"], cfg.rms_norm_eps, residual=o)
    gu = gemm(h2, W["wgu"])
    mlpw = gemm(L.swiglu(gu[:, :inter], gu[:, inter:]), W["wd"])
    assert norm_rel(got_x2, x2w) <= 2e-2
    assert norm_rel(got_mlp, mlpw) <= 2e-2


def test_decode_steps_match_prefill(ly, gpu):
    """Incremental decode against the reference's generation semantics, which
    recompute the whole prefill per new token and read the last position
    (bin/infer.rs:96-106): a 2-layer model (hidden 512, GQA 4/2, d 128) is
    prefilled on 300 tokens, then 4 tokens are decoded from the KV cache; each
    step's logits equal the full prefill's logits at that position."""
    import torch

    cfg = ly.ModelConfig(hidden_size=512, num_heads=4, num_key_value_heads=2,
                         intermediate_size=1024, num_layers=2, vocab_size=1000,
                         rope_theta=500000.0)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    weights = ly.init_model_weights(cfg, gen, "cuda", std=0.05)
    T, extra = 300, 4
    ids = torch.randint(0, cfg.vocab_size, (T + extra,), generator=gen, device="cuda")
    table = ly.rope_table(ly.rope_params(cfg.head_dim, cfg.rope_theta), T + extra, 0)
    full = ly.model_prefill(ids, weights, cfg, table)
    caches = ly.new_cache(cfg, T + extra, "cuda")
    ly.model_prefill(ids[:T], weights, cfg, table[:T], caches)
    for step in range(extra):
        pos = T + step
        logits = ly.model_decode_step(int(ids[pos]), pos, weights, cfg, table, caches)
        gpu.cuda.synchronize()
        assert norm_rel(_np(logits[0]), _np(full[pos])) <= 2e-2, step


@pytest.mark.parametrize("rows,cols,stride", [(1000, 512, 512), (33, 4096, 4104), (5, 8, 8),
                                              (70, 14336, 14336), (129, 1000, 1008)])
def test_gemv_single_token(ly, gpu, rows, cols, stride):
    """lc_gemv (one token through a linear layer, bf16, fp32 accumulation)
    against the fp64 product of the same bf16 values: within one bf16 rounding
    of the exact value plus the fp32 summation error bound."""
    rng = np.random.default_rng(rows + cols)
    w = L.bf16(rng.standard_normal((rows, stride)).astype(np.float32) * 0.05)
    x = L.bf16(rng.standard_normal((1, cols)).astype(np.float32))
    tw = _t(gpu, w, gpu.bfloat16)[:, :cols]
    tx = _t(gpu, x, gpu.bfloat16)
    got = _np(ly.linear(tx, tw))
    gpu.cuda.synchronize()
    prod = w[:, :cols].astype(np.float64) * x[0].astype(np.float64)
    want = prod.sum(axis=1)[None, :]
    bound = 2.0 ** -8 * np.abs(want) + 2.0 ** -22 * cols * np.abs(prod).sum(axis=1)[None, :]
    assert got.shape == (1, rows)
    assert np.all(np.abs(got - want) <= bound + 1e-30)


def _rand_bf16(torch, g, shape, scale=1.0, shift=0.0):
    return (shift + scale * torch.randn(*shape, generator=g, device="cuda")).to(torch.bfloat16)


@pytest.mark.parametrize("rows,cols", [(1000, 512), (33, 4096), (1001, 200), (70, 2056),
                                       (40000, 1024)])
@pytest.mark.parametrize("form", ["bf16", "f32", "norm", "norm_res"])
def test_gemv_fused_input_forms_bit_identical(ly, gpu, rows, cols, form):
    """lc_gemv_fused's input forms against the unfused calls they fold (lc_gemv
    after a bf16 cast, after lc_rmsnorm with or without the residual add): the
    same bits.  200 and 1024 columns take the two-chunk sum-of-squares order,
    2056 and 4096 the eight-chunk one; 40,000 rows (10,000 row blocks) loop
    each workgroup of the capped normalising grid over several blocks."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(rows * 7 + cols)
    w = _rand_bf16(torch, g, (rows, cols), 0.05)
    x32 = torch.randn(1, cols, generator=g, device="cuda")
    x = x32.to(torch.bfloat16)
    if form == "bf16":
        got, want = ly.gemv_fused(x, w), ly.linear(x, w)
    elif form == "f32":
        got, want = ly.gemv_fused(x32, w), ly.linear(x32.to(torch.bfloat16), w)
    else:
        nw = _rand_bf16(torch, g, (cols,), 0.1, 1.0)
        res = _rand_bf16(torch, g, (1, cols)) if form == "norm_res" else None
        ro_got = torch.empty_like(x) if res is not None else None
        ro_want = torch.empty_like(x) if res is not None else None
        got = ly.gemv_fused(x, w, norm_weight=nw, eps=1e-5, residual=res, residual_out=ro_got)
        want = ly.linear(ly.rmsnorm(x, nw, 1e-5, residual=res, residual_out=ro_want), w)
        if res is not None:
            torch.cuda.synchronize()
            assert torch.equal(ro_got, ro_want)
    torch.cuda.synchronize()
    assert got.shape == want.shape == (1, rows)
    assert torch.equal(got, want)


@pytest.mark.parametrize("rows,cols", [(64, 4104), (37, 4168), (129, 4144)])
@pytest.mark.parametrize("form", ["bf16", "f32"])
def test_gemv_fused_uneven_wave_split(ly, gpu, rows, cols, form):
    """Widths whose 16-byte chunks split unevenly over the four waves of a
    workgroup, so that the last wave holds fewer chunks than the others (at
    4104-4168 columns: three waves past one round of chunks, the last within
    it).  Every wave must take the same loop, whose barriers the row sum
    crosses; the result is lc_gemv's, bit for bit."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(rows * 13 + cols)
    w = _rand_bf16(torch, g, (rows, cols), 0.05)
    x32 = torch.randn(1, cols, generator=g, device="cuda")
    x = x32.to(torch.bfloat16)
    got = ly.gemv_fused(x if form == "bf16" else x32, w)
    want = ly.linear(x, w)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("rows,cols", [(70, 14336), (4096, 8200), (9, 16384)])
def test_gemv_fused_long_rows_bit_identical(ly, gpu, rows, cols):
    """Rows longer than 8192 columns: lc_gemv takes several rounds of four
    chunks per lane, the fp32-input form several rounds of two; both sum each
    lane's chunks in the same order, so the results are the same bits."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(rows + cols)
    w = _rand_bf16(torch, g, (rows, cols), 0.05)
    x32 = torch.randn(1, cols, generator=g, device="cuda")
    got, want = ly.gemv_fused(x32, w), ly.linear(x32.to(torch.bfloat16), w)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("inter,cols,norm", [(14336, 4096, True), (1000, 512, False),
                                             (8, 64, True), (3000, 200, False)])
def test_gemv_fused_swiglu_bit_identical(ly, gpu, inter, cols, norm):
    """The SwiGLU output form (gate rows then up rows of one weight) against
    lc_gemv + lc_swiglu of the two halves, with the folded norm of the model's
    MLP input where ``norm`` is set (the decode step's gate/up projection)."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(inter + cols)
    w = _rand_bf16(torch, g, (2 * inter, cols), 0.05)
    x = _rand_bf16(torch, g, (1, cols))
    if norm:
        nw, res = _rand_bf16(torch, g, (cols,), 0.1, 1.0), _rand_bf16(torch, g, (1, cols))
        got = ly.gemv_fused(x, w, norm_weight=nw, eps=1e-5, residual=res, swiglu=True)
        h = ly.rmsnorm(x, nw, 1e-5, residual=res)
    else:
        got, h = ly.gemv_fused(x, w, swiglu=True), x
    gu = ly.linear(h, w)
    want = ly.swiglu(gu[:, :inter], gu[:, inter:])
    torch.cuda.synchronize()
    assert got.shape == want.shape == (1, inter)
    assert torch.equal(got, want)


@pytest.mark.parametrize("hq,hkv,d,cols", [(32, 8, 128, 4096), (4, 2, 64, 256), (3, 1, 16, 64)])
def test_gemv_fused_rope_qkv_bit_identical(ly, gpu, hq, hkv, d, cols):
    """The RoPE/QKV output form with the folded norm (the decode step's first
    projection) against lc_rmsnorm, lc_gemv, lc_rope_apply of the q and k
    columns and the copy of v into the cache: q, the cache's k and v rows of
    the token bit for bit, every other cache row untouched."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(hq * 100 + d)
    rows = (hq + 2 * hkv) * d
    w = _rand_bf16(torch, g, (rows, cols), 0.05)
    x, res = _rand_bf16(torch, g, (1, cols)), _rand_bf16(torch, g, (1, cols))
    nw = _rand_bf16(torch, g, (cols,), 0.1, 1.0)
    cap, pos = 50, 37
    table = ly.rope_table(ly.rope_params(d, 500000.0), cap, 0)
    kc = torch.zeros(1, cap, hkv, d, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    xin = torch.empty_like(x)
    q = ly.gemv_fused(x, w, norm_weight=nw, eps=1e-5, residual=res, residual_out=xin,
                      rope_row=table[pos], heads=(hq, hkv), k_out=kc[0, pos], v_out=vc[0, pos])
    xin_w = torch.empty_like(x)
    qkv = ly.linear(ly.rmsnorm(x, nw, 1e-5, residual=res, residual_out=xin_w), w)
    qw = ly.rope_apply(qkv[:, :hq * d], table[pos:pos + 1], hq, d)
    kw = ly.rope_apply(qkv[:, hq * d:(hq + hkv) * d], table[pos:pos + 1], hkv, d)
    torch.cuda.synchronize()
    assert torch.equal(xin, xin_w)
    assert torch.equal(q.view(-1), qw.view(-1))
    assert torch.equal(kc[0, pos].reshape(-1), kw.view(-1))
    assert torch.equal(vc[0, pos].reshape(-1), qkv[0, (hq + hkv) * d:])
    others = torch.ones(cap, dtype=torch.bool)
    others[pos] = False
    assert not kc[0, others].any() and not vc[0, others].any()


def test_decode_step_fused_equals_unfused(ly, gpu):
    """The whole decode step with every projection's row operation folded
    (five launches per layer with the attention) against the unfused
    sequence: identical logits and caches over several tokens of a 2-layer
    GQA model."""
    import torch

    cfg = ly.ModelConfig(hidden_size=512, num_heads=4, num_key_value_heads=2,
                         intermediate_size=1024, num_layers=2, vocab_size=1000,
                         rope_theta=500000.0)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    weights = ly.init_model_weights(cfg, gen, "cuda", std=0.05)
    T, extra = 200, 3
    ids = torch.randint(0, cfg.vocab_size, (T + extra,), generator=gen, device="cuda")
    table = ly.rope_table(ly.rope_params(cfg.head_dim, cfg.rope_theta), T + extra, 0)
    caches = [ly.new_cache(cfg, T + extra, "cuda") for _ in range(2)]
    for c in caches:
        ly.model_prefill(ids[:T], weights, cfg, table[:T], c)
    for step in range(extra):
        pos = T + step
        a = ly.model_decode_step(int(ids[pos]), pos, weights, cfg, table, caches[0], fused=True)
        b = ly.model_decode_step(int(ids[pos]), pos, weights, cfg, table, caches[1], fused=False)
        torch.cuda.synchronize()
        assert torch.equal(a, b), step
        for (k0, v0), (k1, v1) in zip(*caches):
            assert torch.equal(k0, k1) and torch.equal(v0, v1), step


@pytest.mark.parametrize("seed", [*range(24), 106])
def test_gemv_fused_random_shapes(ly, gpu, seed):
    """Seeded random shapes through every input x output form combination
    lc_gemv_fused accepts, each against the unfused calls it folds, bit for
    bit: cols any multiple of 8 up to 4096 (up to 9000 without the norm),
    rows with ragged row blocks, GQA head counts and head dims of 16 to 256.
    Seed 106 (norm + RoPE, head_dim 208) caught one RoPE output an ulp apart
    while the RoPE products could still be contracted into an FMA."""
    import torch

    rng = np.random.default_rng(1000 + seed)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    in_form = ["bf16", "f32", "norm", "norm_res"][seed % 4]
    out_form = ["plain", "swiglu", "rope"][(seed // 4) % 3]
    cols = 8 * int(rng.integers(1, (4096 if in_form.startswith("norm") else 9000) // 8 + 1))
    if out_form == "rope":
        d = 16 * int(rng.integers(1, 17))
        hkv = int(rng.integers(1, 5))
        hq = hkv * int(rng.integers(1, 5))
        rows = (hq + 2 * hkv) * d
    elif out_form == "swiglu":
        rows = 2 * 8 * int(rng.integers(1, 700))
    else:
        rows = int(rng.integers(1, 9000))
    w = _rand_bf16(torch, g, (rows, cols), 0.05)
    x32 = torch.randn(1, cols, generator=g, device="cuda")
    x = x32.to(torch.bfloat16)
    kw, ro_got, ro_want, res, nw = {}, None, None, None, None
    if in_form.startswith("norm"):
        nw = _rand_bf16(torch, g, (cols,), 0.1, 1.0)
        if in_form == "norm_res":
            res = _rand_bf16(torch, g, (1, cols))
            ro_got, ro_want = torch.empty_like(x), torch.empty_like(x)
        kw = dict(norm_weight=nw, eps=1e-6, residual=res, residual_out=ro_got)
        h = ly.rmsnorm(x, nw, 1e-6, residual=res, residual_out=ro_want)
        xin = x
    elif in_form == "f32":
        xin, h = x32, x
    else:
        xin, h = x, x
    if out_form == "plain":
        got = ly.gemv_fused(xin, w, **kw)
        want = ly.linear(h, w)
        checks = [(got, want)]
    elif out_form == "swiglu":
        got = ly.gemv_fused(xin, w, swiglu=True, **kw)
        gu = ly.linear(h, w)
        want = ly.swiglu(gu[:, :rows // 2], gu[:, rows // 2:])
        checks = [(got, want)]
    else:
        table = ly.rope_table(ly.rope_params(d, 10000.0), 5, 100)
        kc = torch.zeros(hkv * d, dtype=torch.bfloat16, device="cuda")
        vc = torch.zeros_like(kc)
        got = ly.gemv_fused(xin, w, rope_row=table[2], heads=(hq, hkv), k_out=kc, v_out=vc, **kw)
        qkv = ly.linear(h, w)
        qw = ly.rope_apply(qkv[:, :hq * d], table[2:3], hq, d)
        kw_ = ly.rope_apply(qkv[:, hq * d:(hq + hkv) * d], table[2:3], hkv, d)
        checks = [(got.view(-1), qw.view(-1)), (kc, kw_.view(-1)), (vc, qkv[0, (hq + hkv) * d:])]
    torch.cuda.synchronize()
    for a, b in checks:
        assert a.shape == b.shape and torch.equal(a, b), (in_form, out_form, rows, cols)
    if ro_got is not None:
        assert torch.equal(ro_got, ro_want)


def test_gemv_fused_rejects_bad_forms(ly, gpu):
    """lc_gemv_fused validates the forms and their arguments before a launch."""
    import torch

    bf = torch.bfloat16
    w = torch.zeros(48, 64, dtype=bf, device="cuda")
    x = torch.zeros(1, 64, dtype=bf, device="cuda")
    with pytest.raises(ValueError, match="rows .2 x intermediate. % 4"):
        ly.gemv_fused(x, torch.zeros(6, 64, dtype=bf, device="cuda"), swiglu=True)
    table = ly.rope_table(ly.rope_params(16, 10000.0), 4, 0)
    kv = torch.zeros(1, 16, dtype=bf, device="cuda")
    with pytest.raises(ValueError, match="rows = .q_heads . 2 kv_heads. head_dim"):
        ly.gemv_fused(x, torch.zeros(50, 64, dtype=bf, device="cuda"), rope_row=table[0],
                      heads=(1, 1), k_out=kv, v_out=kv)
    with pytest.raises(ValueError, match="k_out must be"):
        ly.gemv_fused(x, w, rope_row=table[0], heads=(1, 1),
                      k_out=torch.zeros(1, 8, dtype=bf, device="cuda"), v_out=kv)
    with pytest.raises(ValueError, match="cols <= 4096"):
        big = torch.zeros(1, 4104, dtype=bf, device="cuda")
        ly.gemv_fused(big, torch.zeros(4, 4104, dtype=bf, device="cuda"),
                      norm_weight=torch.ones(4104, dtype=bf, device="cuda"))
    with pytest.raises(ValueError, match="folded rmsnorm takes a bf16 x"):
        ly.gemv_fused(x.float(), w, norm_weight=torch.ones(64, dtype=bf, device="cuda"))
    with pytest.raises(ValueError, match="belong to the folded rmsnorm"):
        ly.gemv_fused(x, w, residual=x)


def test_wrappers_reject_mis_sized_buffers(ly, gpu):
    """The layer kernels take raw pointers: the wrappers check caller-supplied
    outputs, residuals, weights and tables before a launch could overrun them."""
    bf = gpu.bfloat16
    x = gpu.zeros((8, 256), dtype=bf, device="cuda")
    w = gpu.ones(256, dtype=bf, device="cuda")
    with pytest.raises(ValueError, match="residual_out must be"):
        ly.rmsnorm(x, w, 1e-5, residual=x, residual_out=gpu.zeros((4, 256), dtype=bf, device="cuda"))
    with pytest.raises(ValueError, match="weight must hold"):
        ly.rmsnorm(x, w[:128], 1e-5)
    with pytest.raises(ValueError, match="out must be"):
        ly.rmsnorm(x, w, 1e-5, out=gpu.zeros((8, 256), dtype=gpu.float32, device="cuda"))
    table = ly.rope_table(ly.rope_params(64, 5e5), 8, 0)
    src = gpu.zeros((8, 2 * 64), dtype=bf, device="cuda")
    with pytest.raises(ValueError, match="out must be"):
        ly.rope_apply(src, table, 2, 64, out=gpu.zeros((4, 2, 64), dtype=bf, device="cuda"))
    with pytest.raises(ValueError, match="table must be"):
        ly.rope_apply(src, table[:4], 2, 64)
    gate = gpu.zeros((4, 32), dtype=bf, device="cuda")
    with pytest.raises(ValueError, match="out must be"):
        ly.swiglu(gate, gate, out=gpu.zeros((4, 16), dtype=bf, device="cuda"))
    gpu.cuda.synchronize()
