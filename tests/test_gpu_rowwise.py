"""GPU parity of online softmax, RMS norm, layer norm and Llama RoPE against the oracle.

Sweeps follow the reference tests (test/softmax_tests.jl:12-16, test/rmsnorm_tests.jl:11-17,
test/layernorm_tests.jl:13-18, test/rope_tests.jl:21-28); inputs are seeded, rounded to the
dtype, and the oracle runs in float64 on the same values.  Tolerance: norm-wise relative
error <= 1e-5 (float32), <= 2e-2 (float16, bfloat16).
"""
import numpy as np
import pytest
import torch

import nnop
import oracle
from helpers import DTYPES, TOL, host, make, rel_err

pytestmark = pytest.mark.gpu


def check(errs, tol):
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"tolerance {tol}: {bad} (all: {errs})"


# ------------------------------------------------------------------ softmax

@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("n", [32, 33, 63, 255, 256, 511, 512, 513, 1024, 4095, 8192])
def test_softmax(dev, dt, n):
    dtype = DTYPES[dt]
    rng = np.random.default_rng(n)
    x, xn = make(rng, (4, n), dtype, dev, kind="uniform")
    g, gn = make(rng, (4, n), dtype, dev)
    y = nnop._online_softmax(x)
    dx = nnop.grad_online_softmax(g, y)
    torch.cuda.synchronize()
    y_r = oracle.softmax_fwd(xn)
    dx_r = oracle.softmax_bwd(gn, host(y))  # the backward's own input is the forward output
    dx_full = oracle.softmax_bwd(gn, y_r)
    check({"y": rel_err(host(y), y_r), "dx": rel_err(host(dx), dx_r), "dx_full": rel_err(host(dx), dx_full)},
          TOL[dtype] if dtype != torch.float32 else 1e-5)
    assert np.allclose(host(y).sum(-1), 1.0, atol=1e-5 if dtype == torch.float32 else 1e-2)


def test_softmax_autograd(dev):
    rng = np.random.default_rng(0)
    x, xn = make(rng, (5, 300), torch.float32, dev)
    x.requires_grad_(True)
    y = nnop.online_softmax(x)
    (y * torch.arange(300, device=dev)).sum().backward()
    g = np.broadcast_to(np.arange(300.0), (5, 300))
    check({"dx": rel_err(host(x.grad), oracle.softmax_bwd(g, oracle.softmax_fwd(xn)))}, 1e-5)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("n", [33, 256, 513, 4095, 8192])
def test_softmax_bwd_bwd(dev, dt, n):
    """Pullback of the softmax backward (second order) against the oracle's float64 form."""
    dtype = DTYPES[dt]
    rng = np.random.default_rng(100 + n)
    x, _ = make(rng, (3, n), dtype, dev, kind="uniform")
    y = nnop._online_softmax(x)
    dy, dyn = make(rng, (3, n), dtype, dev)
    g, gn = make(rng, (3, n), dtype, dev)
    d_dy, d_y = nnop.grad_online_softmax_pullback(g, dy, y)
    torch.cuda.synchronize()
    r_dy, r_y = oracle.softmax_bwd_bwd(gn, dyn, host(y))
    check({"d_dy": rel_err(host(d_dy), r_dy), "d_y": rel_err(host(d_y), r_y)},
          TOL[dtype] if dtype != torch.float32 else 1e-5)


def test_softmax_second_order_autograd(dev):
    """d/dx <G, d<dy, softmax(x)>/dx> through two GPU backward launches (create_graph)."""
    rng = np.random.default_rng(7)
    x, xn = make(rng, (4, 200), torch.float32, dev)
    dy, dyn = make(rng, (4, 200), torch.float32, dev)
    G, Gn = make(rng, (4, 200), torch.float32, dev)
    x.requires_grad_(True)
    dy.requires_grad_(True)
    y = nnop.online_softmax(x)
    (gx,) = torch.autograd.grad(y, x, dy, create_graph=True)
    gdy, gx2 = torch.autograd.grad(gx, (dy, x), G)
    torch.cuda.synchronize()
    y_r = oracle.softmax_fwd(xn)
    r_dy, r_y = oracle.softmax_bwd_bwd(Gn, dyn, y_r)
    check({"gx": rel_err(host(gx), oracle.softmax_bwd(dyn, y_r)), "d_dy": rel_err(host(gdy), r_dy),
           "d_x": rel_err(host(gx2), oracle.softmax_bwd(r_y, y_r))}, 1e-5)


# ------------------------------------------------------------------ RMS norm

RMS_CASES = [(emb, n, off) for emb in (15, 255, 256, 257, 511, 512, 513, 1024)
             for n in (1, 4, 17, 25) for off in (0.0, 1.0)]


@pytest.mark.parametrize("case", RMS_CASES, ids=lambda c: "-".join(map(str, c)))
def test_rms_norm_f32(dev, case):
    emb, n, off = case
    rng = np.random.default_rng(emb * 100 + n)
    x, xn = make(rng, (n, emb), torch.float32, dev, kind="uniform")
    w, wn = make(rng, (emb,), torch.float32, dev, kind="uniform")
    g, gn = make(rng, (n, emb), torch.float32, dev)
    y, rstd = nnop._rms_norm(x, w, offset=off)
    dx, dw = nnop.grad_rms_norm(g, rstd, x, w, offset=off)
    torch.cuda.synchronize()
    y_r, r_r = oracle.rms_norm_fwd(xn, wn, 1e-6, off)
    dx_r, dw_r = oracle.rms_norm_bwd(gn, r_r, xn, wn, off)
    check({"y": rel_err(host(y), y_r), "rstd": rel_err(host(rstd), r_r), "dx": rel_err(host(dx), dx_r),
           "dw": rel_err(host(dw), dw_r)}, 1e-5)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("emb,n", [(4096, 64), (1024, 3000), (520, 7)])
def test_rms_norm_16bit(dev, dt, emb, n):
    dtype = DTYPES[dt]
    rng = np.random.default_rng(emb + n)
    x, xn = make(rng, (n, emb), dtype, dev)
    w, wn = make(rng, (emb,), dtype, dev, scale=0.02, offset=1.0)
    g, gn = make(rng, (n, emb), dtype, dev)
    y, rstd = nnop._rms_norm(x, w)
    dx, dw = nnop.grad_rms_norm(g, rstd, x, w)
    torch.cuda.synchronize()
    y_r, r_r = oracle.rms_norm_fwd(xn, wn)
    dx_r, dw_r = oracle.rms_norm_bwd(gn, r_r, xn, wn)
    check({"y": rel_err(host(y), y_r), "rstd": rel_err(host(rstd), r_r), "dx": rel_err(host(dx), dx_r),
           "dw": rel_err(host(dw), dw_r)}, TOL[dtype])


# ------------------------------------------------------------------ layer norm

LN_CASES = [(emb, n) for emb in (15, 255, 256, 257, 511, 512, 513, 1024) for n in (1, 2, 16, 23)]


@pytest.mark.parametrize("case", LN_CASES, ids=lambda c: "-".join(map(str, c)))
def test_layer_norm_f32(dev, case):
    emb, n = case
    rng = np.random.default_rng(emb * 7 + n)
    x, xn = make(rng, (n, emb), torch.float32, dev, kind="uniform")
    w, wn = make(rng, (emb,), torch.float32, dev, kind="uniform")
    b, bn = make(rng, (emb,), torch.float32, dev, kind="uniform")
    g, gn = make(rng, (n, emb), torch.float32, dev)
    y, mu, rstd = nnop._layer_norm(x, w, b)
    dx, dw, db = nnop.grad_layer_norm(g, mu, rstd, x, w)
    torch.cuda.synchronize()
    y_r, mu_r, r_r = oracle.layer_norm_fwd(xn, wn, bn)
    dx_r, dw_r, db_r = oracle.layer_norm_bwd(gn, mu_r, r_r, xn, wn)
    check({"y": rel_err(host(y), y_r), "mu": rel_err(host(mu), mu_r), "rstd": rel_err(host(rstd), r_r),
           "dx": rel_err(host(dx), dx_r), "dw": rel_err(host(dw), dw_r), "db": rel_err(host(db), db_r)}, 1e-5)


@pytest.mark.parametrize("emb", [513, 4096])
def test_layer_norm_large_mean(dev, emb):
    """x = 1000 + U[0,1): the variance is 1e-7 of E[x^2], so E[x^2] - mean^2 in float32 would
    lose it entirely; the two-pass statistics keep rstd to float32 rounding of the mean."""
    rng = np.random.default_rng(emb)
    x, xn = make(rng, (16, emb), torch.float32, dev, kind="uniform", offset=1000.0)
    w, wn = make(rng, (emb,), torch.float32, dev, kind="uniform")
    b, bn = make(rng, (emb,), torch.float32, dev, kind="uniform")
    y, mu, rstd = nnop._layer_norm(x, w, b)
    torch.cuda.synchronize()
    y_r, mu_r, r_r = oracle.layer_norm_fwd(xn, wn, bn)
    check({"mu": rel_err(host(mu), mu_r), "rstd": rel_err(host(rstd), r_r)}, 1e-4)
    check({"y": rel_err(host(y), y_r)}, 1e-3)  # x - mu carries the float32 rounding of mu (ulp 6e-5)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("emb,n", [(4096, 64), (1024, 3000)])
def test_layer_norm_16bit(dev, dt, emb, n):
    dtype = DTYPES[dt]
    rng = np.random.default_rng(emb + 3 * n)
    x, xn = make(rng, (n, emb), dtype, dev)
    w, wn = make(rng, (emb,), dtype, dev, scale=0.02, offset=1.0)
    b, bn = make(rng, (emb,), dtype, dev, scale=0.02)
    g, gn = make(rng, (n, emb), dtype, dev)
    y, mu, rstd = nnop._layer_norm(x, w, b)
    dx, dw, db = nnop.grad_layer_norm(g, mu, rstd, x, w)
    torch.cuda.synchronize()
    y_r, mu_r, r_r = oracle.layer_norm_fwd(xn, wn, bn)
    dx_r, dw_r, db_r = oracle.layer_norm_bwd(gn, mu_r, r_r, xn, wn)
    check({"y": rel_err(host(y), y_r), "mu": rel_err(host(mu), mu_r), "rstd": rel_err(host(rstd), r_r),
           "dx": rel_err(host(dx), dx_r), "dw": rel_err(host(dw), dw_r), "db": rel_err(host(db), db_r)},
          TOL[dtype])


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("emb,n", [(4096, 64), (1024, 300), (16384, 8), (520, 7)])
def test_norm_weight_layouts(dev, dt, emb, n):
    """16-bit weights of the rows' own dtype at a 16-byte aligned address are held packed in
    registers; the same values at an unaligned address, or as float32, take the float
    path.  The float32 arithmetic is the same, so the statistics agree bit for bit and the
    16-bit outputs to one unit in the last place: the compiler may round an output once
    from an exact fused multiply-add (v_fma_mixlo_f16) in one kernel variant and via
    float32 in another."""
    dtype = DTYPES[dt]
    rng = np.random.default_rng(emb + 5 * n)
    x, _ = make(rng, (n, emb), dtype, dev)
    g, _ = make(rng, (n, emb), dtype, dev)
    w, _ = make(rng, (emb,), dtype, dev, scale=0.02, offset=1.0)
    b, _ = make(rng, (emb,), dtype, dev, scale=0.02)

    def shifted(t):  # the same values 2 bytes past a 16-byte boundary
        buf = torch.zeros(emb + 8, dtype=dtype, device=dev)
        v = buf[1:emb + 1]
        v.copy_(t)
        assert v.data_ptr() % 16 == 2
        return v

    def ulps(a, c):  # largest distance in units in the last place (16-bit) or exact (float32)
        if a.dtype == torch.float32:
            return 0 if torch.equal(a, c) else float("inf")
        ia, ic = a.view(torch.int16).int(), c.view(torch.int16).int()
        ia = torch.where(ia < 0, -(ia & 0x7FFF), ia)  # sign-magnitude to a monotone integer
        ic = torch.where(ic < 0, -(ic & 0x7FFF), ic)
        return int((ia - ic).abs().max())

    out = {}
    for name, (wl, bl) in {"packed": (w, b), "unaligned": (shifted(w), shifted(b)),
                           "float32": (w.float(), b.float())}.items():
        y, mu, rstd = nnop._layer_norm(x, wl, bl)
        dx, dw, db = nnop.grad_layer_norm(g, mu, rstd, x, wl)
        ry, rr = nnop._rms_norm(x, wl, offset=0.5)
        rdx, rdw = nnop.grad_rms_norm(g, rr, x, wl, offset=0.5)
        out[name] = [y, mu, rstd, dx, dw.to(dtype), db.to(dtype), ry, rr, rdx, rdw.to(dtype)]
    torch.cuda.synchronize()
    names = ["y", "mu", "rstd", "dx", "dw", "db", "rms y", "rms rstd", "rms dx", "rms dw"]
    for other in ("unaligned", "float32"):
        d = {nm: ulps(a, c) for nm, a, c in zip(names, out["packed"], out[other])}
        assert max(d.values()) <= 1, f"packed vs {other} weights: {d}"


def test_norm_autograd(dev):
    rng = np.random.default_rng(2)
    x, xn = make(rng, (9, 300), torch.float32, dev)
    w, wn = make(rng, (300,), torch.float32, dev)
    b, bn = make(rng, (300,), torch.float32, dev)
    for t in (x, w, b):
        t.requires_grad_(True)
    nnop.layer_norm(x, w, b).sum().backward()
    y_r, mu_r, r_r = oracle.layer_norm_fwd(xn, wn, bn)
    dx_r, dw_r, db_r = oracle.layer_norm_bwd(np.ones((9, 300)), mu_r, r_r, xn, wn)
    check({"dx": rel_err(host(x.grad), dx_r), "dw": rel_err(host(w.grad), dw_r),
           "db": rel_err(host(b.grad), db_r)}, 1e-5)
    x.grad = w.grad = None
    nnop.rms_norm(x, w, offset=1.0).sum().backward()
    _, r_r = oracle.rms_norm_fwd(xn, wn, 1e-6, 1.0)
    dx_r, dw_r = oracle.rms_norm_bwd(np.ones((9, 300)), r_r, xn, wn, 1.0)
    check({"dx": rel_err(host(x.grad), dx_r), "dw": rel_err(host(w.grad), dw_r)}, 1e-5)


# ------------------------------------------------------------------ RoPE

ROPE_CASES = [(L, QH, KH) for L in (13, 255, 256, 257, 1024, 1025) for QH, KH in ((1, 1), (3, 4), (4, 3), (5, 1))]


@pytest.mark.parametrize("case", ROPE_CASES, ids=lambda c: "-".join(map(str, c)))
def test_rope_f32_dim16(dev, case):
    """The reference's RoPE sweep (dim 16, batch 1), with random rather than all-ones inputs."""
    L, QH, KH = case
    rng = np.random.default_rng(L * 10 + QH)
    emb = nnop.LlamaRotaryEmbedding(16)
    pos = torch.arange(L, dtype=torch.float32)[None]
    cos, sin = emb(pos)
    q, qn = make(rng, (1, QH, L, 16), torch.float32, dev)
    k, kn = make(rng, (1, KH, L, 16), torch.float32, dev)
    qo, ko = nnop._llama_rope(q, k, cos.to(dev), sin.to(dev), bwd=False)
    qb, kb = nnop._llama_rope(qo, ko, cos.to(dev), sin.to(dev), bwd=True)
    torch.cuda.synchronize()
    cn, sn = cos.double().numpy(), sin.double().numpy()
    qo_r, ko_r = oracle.llama_rope(qn, kn, cn, sn, 1.0)
    check({"q": rel_err(host(qo), qo_r), "k": rel_err(host(ko), ko_r), "q_roundtrip": rel_err(host(qb), qn),
           "k_roundtrip": rel_err(host(kb), kn)}, 1e-5)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_rope_llama_128(dev, dt):
    dtype = DTYPES[dt]
    rng = np.random.default_rng(4)
    B, QH, KH, L, E = 2, 8, 2, 300, 128
    pos = torch.from_numpy(rng.integers(0, 8192, size=(B, L)).astype(np.float32))
    cos, sin = nnop.LlamaRotaryEmbedding(E)(pos)
    q, qn = make(rng, (B, QH, L, E), dtype, dev)
    k, kn = make(rng, (B, KH, L, E), dtype, dev)
    qo, ko = nnop._llama_rope(q, k, cos.to(dev), sin.to(dev), bwd=False)
    gq, gk = nnop.grad_llama_rope(q, k, cos=cos.to(dev), sin=sin.to(dev))
    torch.cuda.synchronize()
    cn, sn = cos.double().numpy(), sin.double().numpy()
    qo_r, ko_r = oracle.llama_rope(qn, kn, cn, sn, 1.0)
    gq_r, gk_r = oracle.llama_rope(qn, kn, cn, sn, -1.0)
    check({"q": rel_err(host(qo), qo_r), "k": rel_err(host(ko), ko_r), "gq": rel_err(host(gq), gq_r),
           "gk": rel_err(host(gk), gk_r)}, TOL[dtype])


def test_rope_autograd(dev):
    rng = np.random.default_rng(9)
    cos, sin = nnop.LlamaRotaryEmbedding(64)(torch.arange(40, dtype=torch.float32)[None])
    cos, sin = cos.to(dev), sin.to(dev)
    q, qn = make(rng, (1, 3, 40, 64), torch.float32, dev)
    k, kn = make(rng, (1, 1, 40, 64), torch.float32, dev)
    q.requires_grad_(True)
    k.requires_grad_(True)
    qo, ko = nnop.llama_rope(q, k, cos=cos, sin=sin)
    (qo.sum() + ko.sum()).backward()
    gq_r, gk_r = oracle.llama_rope(np.ones(qn.shape), np.ones(kn.shape), host(cos), host(sin), -1.0)
    check({"gq": rel_err(host(q.grad), gq_r), "gk": rel_err(host(k.grad), gk_r)}, 1e-5)
