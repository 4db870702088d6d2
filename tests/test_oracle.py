"""Pins of the CPU oracle (no GPU).

The reference ships no golden vectors and cannot run here (Julia, GPU-only kernels), so
every oracle function is pinned by checks that a plausible mistake would fail:
  * library routines: torch float64 (softmax, layer_norm, rms_norm, scaled_dot_product_attention,
    autograd for every gradient), numpy float16 / torch bfloat16 rounding;
  * the reference's own test-side naive formulas (oracle.naive);
  * finite differences on tiny shapes for every gradient, including dpair;
  * invariants and special cases (sums to one, L = 1, GQA = repeated heads, zero bias,
    all-true padding, RoPE norm preservation and inverse, causal first row);
  * FAITHFUL (the reference's float32 algorithm) against EXACT, and the reference's NaN
    on fully masked rows.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import EXACT, FAITHFUL, naive
from helpers import rel_err

RNG = np.random.default_rng


# ------------------------------------------------------------------ rounding

def test_round_f16_matches_numpy():
    rng = RNG(0)
    x = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
                        [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 3e-8, 6.1e-5, 2.0 ** -24, 1 + 2.0 ** -11,
                         1 + 3 * 2.0 ** -11]])
    x = x.astype(np.float32).astype(np.float64)
    got = oracle.round_to("f16", x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float64)
    assert np.array_equal(got, want)


def test_round_bf16_matches_torch():
    rng = RNG(1)
    x = (rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000)).astype(np.float32).astype(np.float64)
    x = np.concatenate([x, [1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, 0.0]])
    got = oracle.round_to("bf16", x)
    want = torch.from_numpy(x).to(torch.float32).to(torch.bfloat16).double().numpy()
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ softmax

def test_softmax_fwd():
    rng = RNG(2)
    x = rng.standard_normal((7, 513)) * 3
    y = oracle.softmax_fwd(x)
    assert rel_err(y, torch.softmax(torch.from_numpy(x), -1).numpy()) < 1e-14
    assert rel_err(y, naive.softmax(x)) < 1e-14
    assert np.allclose(y.sum(-1), 1.0, atol=1e-14)
    assert np.allclose(oracle.softmax_fwd(np.full((1, 10), 3.7)), 0.1)
    assert rel_err(oracle.softmax_fwd(x, FAITHFUL), y) < 1e-6


def test_softmax_bwd():
    rng = RNG(3)
    x = rng.standard_normal((5, 64))
    g = rng.standard_normal((5, 64))
    xt = torch.from_numpy(x).requires_grad_(True)
    torch.softmax(xt, -1).backward(torch.from_numpy(g))
    dx = oracle.softmax_bwd(g, oracle.softmax_fwd(x))
    assert rel_err(dx, xt.grad.numpy()) < 1e-13
    assert rel_err(oracle.softmax_bwd(g, oracle.softmax_fwd(x), FAITHFUL), dx) < 1e-6
    # finite differences of <g, softmax(x)>
    h = 1e-6
    fd = np.zeros_like(x)
    for j in range(5):
        for i in range(0, 64, 7):
            xp, xm = x.copy(), x.copy()
            xp[j, i] += h
            xm[j, i] -= h
            fd[j, i] = (np.sum(g * oracle.softmax_fwd(xp)) - np.sum(g * oracle.softmax_fwd(xm))) / (2 * h)
    sel = np.zeros_like(x, dtype=bool)
    sel[:, ::7] = True
    assert np.allclose(dx[sel], fd[sel], atol=1e-8)


def test_softmax_bwd_bwd():
    """Pullback of the softmax backward (second order): finite differences of
    <G, softmax_bwd(dy, y)> in dy and in y, and torch float64 double backward."""
    rng = RNG(31)
    x = rng.standard_normal((4, 48))
    dy = rng.standard_normal((4, 48))
    G = rng.standard_normal((4, 48))
    y = oracle.softmax_fwd(x)
    d_dy, d_y = oracle.softmax_bwd_bwd(G, dy, y)
    h = 1e-6
    for j in range(4):
        for i in range(0, 48, 5):
            for arg, got in ((0, d_dy), (1, d_y)):
                a = [dy.copy(), y.copy()]
                b = [dy.copy(), y.copy()]
                a[arg][j, i] += h
                b[arg][j, i] -= h
                fd = (np.sum(G * oracle.softmax_bwd(*a)) - np.sum(G * oracle.softmax_bwd(*b))) / (2 * h)
                assert abs(got[j, i] - fd) < 1e-7, (arg, j, i, got[j, i], fd)
    # library routine: torch autograd of its own float64 softmax backward
    xt = torch.from_numpy(x).requires_grad_(True)
    dyt = torch.from_numpy(dy).requires_grad_(True)
    yt = torch.softmax(xt, -1)
    (gx,) = torch.autograd.grad(yt, xt, dyt, create_graph=True)
    gdy, gx2 = torch.autograd.grad(gx, (dyt, xt), torch.from_numpy(G))
    assert rel_err(d_dy, gdy.numpy()) < 1e-13
    # through y = softmax(x): dL/dx = softmax_bwd(d_y, y)
    assert rel_err(oracle.softmax_bwd(d_y, y), gx2.numpy()) < 1e-12


# ------------------------------------------------------------------ RMS norm

@pytest.mark.parametrize("offset", [0.0, 1.0])
def test_rms_norm(offset):
    rng = RNG(4)
    x = rng.random((9, 257))
    w = rng.random(257)
    g = rng.standard_normal((9, 257))
    y, r = oracle.rms_norm_fwd(x, w, 1e-6, offset)
    assert rel_err(y, naive.rms_norm(x, w, offset)) < 1e-14
    xt = torch.from_numpy(x).requires_grad_(True)
    wt = torch.from_numpy(w).requires_grad_(True)
    yt = F.rms_norm(xt, (257,), wt + offset, eps=1e-6)
    assert rel_err(y, yt.detach().numpy()) < 1e-14
    yt.backward(torch.from_numpy(g))
    dx, dw = oracle.rms_norm_bwd(g, r, x, w, offset)
    assert rel_err(dx, xt.grad.numpy()) < 1e-13
    assert rel_err(dw, wt.grad.numpy()) < 1e-13
    yf, rf = oracle.rms_norm_fwd(x, w, 1e-6, offset, FAITHFUL)
    dxf, dwf = oracle.rms_norm_bwd(g, rf, x, w, offset, FAITHFUL)
    assert max(rel_err(yf, y), rel_err(rf, r), rel_err(dxf, dx), rel_err(dwf, dw)) < 2e-6


def test_rms_norm_special_case():
    """offset = 1 with w = 0 is a plain RMS normalisation."""
    rng = RNG(5)
    x = rng.standard_normal((3, 100))
    y, r = oracle.rms_norm_fwd(x, np.zeros(100), 0.0, 1.0)
    assert np.allclose(y, x / np.sqrt(np.mean(x * x, -1, keepdims=True)), rtol=1e-14)
    assert np.allclose(np.mean(y * y, -1), 1.0)


# ------------------------------------------------------------------ layer norm

def test_layer_norm():
    rng = RNG(6)
    x = rng.random((11, 513)) * 4 - 1
    w = rng.random(513)
    b = rng.random(513)
    g = rng.standard_normal((11, 513))
    y, mu, r = oracle.layer_norm_fwd(x, w, b)
    assert rel_err(y, naive.layer_norm(x, w, b)) < 1e-14
    xt = torch.from_numpy(x).requires_grad_(True)
    wt = torch.from_numpy(w).requires_grad_(True)
    bt = torch.from_numpy(b).requires_grad_(True)
    yt = F.layer_norm(xt, (513,), wt, bt, eps=1e-6)
    assert rel_err(y, yt.detach().numpy()) < 1e-14
    yt.backward(torch.from_numpy(g))
    dx, dw, db = oracle.layer_norm_bwd(g, mu, r, x, w)
    assert rel_err(dx, xt.grad.numpy()) < 1e-12
    assert rel_err(dw, wt.grad.numpy()) < 1e-13
    assert rel_err(db, bt.grad.numpy()) < 1e-13
    yn, _, _ = oracle.layer_norm_fwd(x, np.ones(513), np.zeros(513), 0.0)
    assert np.allclose(yn.mean(-1), 0.0, atol=1e-13) and np.allclose(yn.var(-1), 1.0, atol=1e-12)
    yf, muf, rf = oracle.layer_norm_fwd(x, w, b, 1e-6, FAITHFUL)
    dxf, dwf, dbf = oracle.layer_norm_bwd(g, muf, rf, x, w, FAITHFUL)
    assert max(rel_err(yf, y), rel_err(rf, r), rel_err(dxf, dx), rel_err(dwf, dw), rel_err(dbf, db)) < 2e-6


# ------------------------------------------------------------------ RoPE

def test_rotary_embedding():
    pos = np.arange(0, 100, dtype=np.float64)[None]
    c, s = oracle.rotary_embedding(16, pos, mode=EXACT)
    i = np.arange(8)
    f = pos[0][:, None] / 10000.0 ** (2 * i / 16)
    assert np.allclose(c[0, :, :8], np.cos(f), atol=1e-14) and np.allclose(c[0, :, 8:], np.cos(f), atol=1e-14)
    assert np.allclose(s[0, :, :8], np.sin(f), atol=1e-14) and np.allclose(s[0, :, 8:], np.sin(f), atol=1e-14)
    cf, sf = oracle.rotary_embedding(16, pos, mode=FAITHFUL)
    assert np.abs(cf - c).max() < 2e-5 and np.abs(sf - s).max() < 2e-5


def test_rope():
    rng = RNG(7)
    B, QH, KH, L, E = 2, 3, 2, 37, 16
    q = rng.standard_normal((B, QH, L, E))
    k = rng.standard_normal((B, KH, L, E))
    c, s = oracle.rotary_embedding(E, rng.integers(0, 1000, (B, L)).astype(float), mode=EXACT)
    qo, ko = oracle.llama_rope(q, k, c, s, 1.0)
    qn, kn = naive.llama_rope(q, k, c, s)
    assert rel_err(qo, qn) < 1e-15 and rel_err(ko, kn) < 1e-15
    # each (i, i + E/2) pair keeps its norm; the backward (sin -> -sin) inverts the forward
    h = E // 2
    assert np.allclose(qo[..., :h] ** 2 + qo[..., h:] ** 2, q[..., :h] ** 2 + q[..., h:] ** 2)
    qb, kb = oracle.llama_rope(qo, ko, c, s, -1.0)
    assert rel_err(qb, q) < 1e-14 and rel_err(kb, k) < 1e-14
    # the backward is the adjoint (rotation by -theta is the transpose)
    g = rng.standard_normal(qo.shape)
    gq, _ = oracle.llama_rope(g, k, c, s, -1.0)
    assert np.isclose(np.sum(g * qo), np.sum(gq * q))
    qf, kf = oracle.llama_rope(q, k, c, s, 1.0, FAITHFUL)
    assert rel_err(qf, qo) < 1e-6


# ------------------------------------------------------------------ attention

def _inputs(seed, B, QH, KH, QL, KL, E, pair=False):
    rng = RNG(seed)
    q = rng.standard_normal((B, QH, QL, E))
    k = rng.standard_normal((B, KH, KL, E))
    v = rng.standard_normal((B, KH, KL, E))
    p = rng.standard_normal((B, KL, QL, QH)) if pair else None
    return q, k, v, p


def _torch_attention(q, k, v, pair, kpad, causal, scale):
    """torch float64 scaled_dot_product_attention with the same additive mask / bias."""
    QH, KH = q.shape[1], k.shape[1]
    qt, kt, vt = (torch.from_numpy(a) for a in (q, k, v))
    if QH != KH:
        kt = kt.repeat_interleave(QH // KH, dim=1)
        vt = vt.repeat_interleave(QH // KH, dim=1)
    QL, KL = q.shape[2], k.shape[2]
    bias = torch.zeros((q.shape[0], QH, QL, KL), dtype=torch.float64)
    if pair is not None:
        bias = bias + torch.from_numpy(pair).permute(0, 3, 2, 1)
    if causal:
        bias = bias.masked_fill(torch.ones(QL, KL, dtype=torch.bool).triu(1), float("-inf"))
    if kpad is not None:
        bias = bias.masked_fill(~torch.from_numpy(kpad)[:, None, None, :], float("-inf"))
    return F.scaled_dot_product_attention(qt, kt, vt, attn_mask=bias, scale=scale)


ATT = [
    # B, QH, KH, QL, KL, E, causal, pair, kpad
    (2, 2, 2, 37, 45, 16, False, False, False),
    (2, 4, 2, 33, 33, 16, True, True, False),
    (3, 2, 2, 29, 40, 32, False, True, True),
    (2, 6, 2, 20, 20, 16, True, False, True),
]


@pytest.mark.parametrize("case", ATT)
def test_attention_fwd_against_torch_and_naive(case):
    B, QH, KH, QL, KL, E, causal, use_pair, use_kpad = case
    q, k, v, p = _inputs(1, B, QH, KH, QL, KL, E, use_pair)
    kpad = None
    if use_kpad:  # interior keys, so that no tile of the reference algorithm is fully masked
        kpad = np.ones((B, KL), dtype=bool)
        kpad[-1, 2:7] = False
    scale = 1 / np.sqrt(E)
    o, ms, ls = oracle.attn_fwd(q, k, v, p, kpad, causal, scale)
    assert rel_err(o, naive.attention(q, k, v, p, kpad, causal)) < 1e-13
    assert rel_err(o, _torch_attention(q, k, v, p, kpad, causal, scale).numpy()) < 1e-13
    of, msf, lsf = oracle.attn_fwd(q, k, v, p, kpad, causal, scale, mode=FAITHFUL, gsz=16)
    assert max(rel_err(of, o), rel_err(msf, ms), rel_err(lsf, ls)) < 2e-6


@pytest.mark.parametrize("case", ATT)
def test_attention_bwd_against_torch_autograd(case):
    B, QH, KH, QL, KL, E, causal, use_pair, use_kpad = case
    q, k, v, p = _inputs(2, B, QH, KH, QL, KL, E, use_pair)
    kpad = None
    if use_kpad:
        kpad = np.ones((B, KL), dtype=bool)
        kpad[0, 3:6] = False  # interior keys: no row or tile is fully masked
    scale = 1 / np.sqrt(E)
    do = RNG(9).standard_normal(q.shape)
    ts = [torch.from_numpy(a).requires_grad_(True) for a in (q, k, v)]
    pt = torch.from_numpy(p).requires_grad_(True) if p is not None else None
    QHr = QH // KH
    kk = ts[1].repeat_interleave(QHr, dim=1)
    vv = ts[2].repeat_interleave(QHr, dim=1)
    a = torch.einsum("bhie,bhje->bhij", ts[0], kk) * scale
    if pt is not None:
        a = a + pt.permute(0, 3, 2, 1)
    if causal:
        a = a.masked_fill(torch.ones(QL, KL, dtype=torch.bool).triu(1), float("-inf"))
    if kpad is not None:
        a = a.masked_fill(~torch.from_numpy(kpad)[:, None, None, :], float("-inf"))
    o = torch.einsum("bhij,bhje->bhie", torch.softmax(a, -1), vv)
    o.backward(torch.from_numpy(do))
    dq, dk, dv, dp = oracle.attn_bwd(do, q, k, v, p, kpad, causal, scale)
    assert rel_err(dq, ts[0].grad.numpy()) < 1e-12
    assert rel_err(dk, ts[1].grad.numpy()) < 1e-12
    assert rel_err(dv, ts[2].grad.numpy()) < 1e-12
    if p is not None:
        assert rel_err(dp, pt.grad.numpy()) < 1e-12
    # the reference's float32 algorithm (without its Float16 Q/K) against the mathematics
    of, ms, ls = oracle.attn_fwd(q, k, v, p, kpad, causal, scale, mode=FAITHFUL, gsz=16)
    g = oracle.attn_bwd(do, q, k, v, p, kpad, causal, scale, mode=FAITHFUL, o=of, ms=ms, ls=ls, gsz=16)
    for got, want in zip(g, (dq, dk, dv, dp)):
        if want is not None:
            assert rel_err(got, want) < 1e-5


def test_attention_bwd_finite_differences():
    """Central differences of <dO, o> in every input, dpair included (E = 16, L <= 17)."""
    B, QH, KH, QL, KL, E = 1, 2, 1, 9, 17, 16
    q, k, v, p = _inputs(3, B, QH, KH, QL, KL, E, pair=True)
    kpad = np.ones((B, KL), dtype=bool)
    kpad[0, 5] = False
    do = RNG(4).standard_normal(q.shape)
    scale = 0.25
    for causal in (False, True):
        grads = oracle.attn_bwd(do, q, k, v, p, kpad, causal, scale)

        def loss(qq, kk, vv, pp):
            return float(np.sum(do * oracle.attn_fwd(qq, kk, vv, pp, kpad, causal, scale)[0]))

        h = 1e-6
        rng = RNG(5)
        for which, arr in enumerate((q, k, v, p)):
            for _ in range(12):
                idx = tuple(rng.integers(0, s) for s in arr.shape)
                args = [q, k, v, p]
                ap, am = arr.copy(), arr.copy()
                ap[idx] += h
                am[idx] -= h
                args[which] = ap
                fp = loss(*args)
                args[which] = am
                fm = loss(*args)
                assert abs((fp - fm) / (2 * h) - grads[which][idx]) < 1e-7, (which, idx, causal)


def test_attention_invariants():
    rng = RNG(6)
    B, H, L, E = 2, 2, 31, 16
    q, k, v, _ = _inputs(7, B, H, H, L, L, E)
    # causal first row attends only key 0; L = 1 gives o = v
    o, _, _ = oracle.attn_fwd(q, k, v, causal=True)
    assert np.allclose(o[:, :, 0], v[:, :, 0], atol=1e-15)
    o1, _, ls1 = oracle.attn_fwd(q[:, :, :1], k[:, :, :1], v[:, :, :1])
    assert np.allclose(o1, v[:, :, :1]) and np.all(ls1 == 1.0)
    # zero bias == no bias; all-true padding == no padding
    o0, _, _ = oracle.attn_fwd(q, k, v)
    assert np.array_equal(oracle.attn_fwd(q, k, v, np.zeros((B, L, L, H)))[0], o0)
    assert np.array_equal(oracle.attn_fwd(q, k, v, kpad=np.ones((B, L), bool))[0], o0)
    # GQA == MHA with each kv head repeated over its group (test/attention_testsetup.jl:23-30)
    qg = rng.standard_normal((B, 4, L, E))
    og, _, _ = oracle.attn_fwd(qg, k, v, causal=True)
    orep, _, _ = oracle.attn_fwd(qg, np.repeat(k, 2, 1), np.repeat(v, 2, 1), causal=True)
    assert np.array_equal(og, orep)
    dgq = oracle.attn_bwd(np.ones_like(qg), qg, k, v, causal=True)
    drep = oracle.attn_bwd(np.ones_like(qg), qg, np.repeat(k, 2, 1), np.repeat(v, 2, 1), causal=True)
    assert rel_err(dgq[1], drep[1].reshape(B, 2, 2, L, E).sum(2)) < 1e-14
    # d sum(o) / dv[j] = sum_i P[i, j]  (each row of P sums to one, so sum_j dv = L per e)
    dv = oracle.attn_bwd(np.ones_like(q), q, k, v)[2]
    assert np.allclose(dv.sum(2), L)


def test_fully_masked_rows_exact_zero_faithful_nan():
    """EXACT gives o = 0 on a row with every key masked; the reference algorithm gives NaN
    (a fully masked tile makes exp(-Inf - -Inf)), src/attention.jl:92-104."""
    q, k, v, _ = _inputs(8, 2, 2, 2, 10, 20, 16)
    kpad = np.ones((2, 20), dtype=bool)
    kpad[1] = False
    o, ms, ls = oracle.attn_fwd(q, k, v, kpad=kpad)
    assert np.all(o[1] == 0) and np.all(ms[1] == -np.inf) and np.all(ls[1] == 0)
    of, _, _ = oracle.attn_fwd(q, k, v, kpad=kpad, mode=FAITHFUL, gsz=16)
    assert np.all(np.isnan(of[1])) and rel_err(of[0], o[0]) < 1e-6
    g = oracle.attn_bwd(np.ones_like(q), q, k, v, kpad=kpad)
    assert all(np.all(np.isfinite(x)) for x in g[:3]) and np.all(g[0][1] == 0)


def test_qk_fp16_mode():
    """With qk_fp16 the EXACT backward is the float64 mathematics of the reference backward
    (Float16 Q/K in the recomputed scores and in dK/dQ); it matches the FAITHFUL replay."""
    q, k, v, p = _inputs(10, 1, 2, 2, 70, 70, 32, pair=True)
    do = RNG(11).standard_normal(q.shape)
    for causal in (False, True):
        o, ms, ls = oracle.attn_fwd(q, k, v, p, None, causal, 0.125, mode=FAITHFUL, gsz=16)
        f = oracle.attn_bwd(do, q, k, v, p, None, causal, 0.125, mode=FAITHFUL, o=o, ms=ms, ls=ls, gsz=16,
                            qk_fp16=True)
        e = oracle.attn_bwd(do, q, k, v, p, None, causal, 0.125, qk_fp16=True)
        e0 = oracle.attn_bwd(do, q, k, v, p, None, causal, 0.125, qk_fp16=False)
        for a, b, c in zip(f, e, e0):
            assert rel_err(a, b) < 1e-5
            assert rel_err(b, c) > 1e-5  # the rounding is visible


def test_bf16_inputs_rounding_path():
    """Inputs rounded to bf16 then fed to EXACT equal torch float64 on the same values."""
    q, k, v, _ = _inputs(12, 1, 2, 2, 16, 16, 16)
    qr, kr, vr = (oracle.round_to("bf16", a) for a in (q, k, v))
    o, _, _ = oracle.attn_fwd(qr, kr, vr, causal=True)
    assert rel_err(o, _torch_attention(qr, kr, vr, None, None, True, 0.25).numpy()) < 1e-13
