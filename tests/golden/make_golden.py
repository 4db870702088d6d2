#!/usr/bin/env python3
"""Writes the golden fixtures in this directory (inputs + expected outputs, .npz).

The reference holds no golden vectors, so each fixture's expected values come from the
EXACT (float64) oracle and are accepted only if torch float64 (autograd, SDPA,
layer_norm, softmax) agrees to 1e-12; a fixture therefore pins the oracle to a library
routine and lets GPU tests check committed data.  Inputs are rounded to the fixture's
dtype first (the values the GPU sees).  Run from the repo root:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402


def rel(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def attention_case(name, dtype, B, QH, KH, QL, KL, E, causal, use_pair, use_kpad, seed):
    rng = np.random.default_rng(seed)
    rd = lambda a: oracle.round_to(dtype, a)  # noqa: E731
    q, k, v = rd(rng.standard_normal((B, QH, QL, E))), rd(rng.standard_normal((B, KH, KL, E))), rd(
        rng.standard_normal((B, KH, KL, E)))
    do = rd(rng.standard_normal((B, QH, QL, E)))
    pair = rd(rng.standard_normal((B, KL, QL, QH))) if use_pair else None
    kpad = None
    if use_kpad:
        kpad = np.ones((B, KL), dtype=bool)
        kpad[-1, -11:] = False
    scale = float(oracle.round_to(dtype, np.array([1.0 / np.sqrt(E)]))[0])
    o, ms, ls = oracle.attn_fwd(q, k, v, pair, kpad, causal, scale)
    dq, dk, dv, dp = oracle.attn_bwd(do, q, k, v, pair, kpad, causal, scale)
    # accept only if torch float64 autograd agrees
    ts = [torch.from_numpy(a).requires_grad_(True) for a in (q, k, v)]
    pt = torch.from_numpy(pair).requires_grad_(True) if use_pair else None
    rep = QH // KH
    a = torch.einsum("bhie,bhje->bhij", ts[0], ts[1].repeat_interleave(rep, 1)) * scale
    if pt is not None:
        a = a + pt.permute(0, 3, 2, 1)
    if causal:
        a = a.masked_fill(torch.ones(QL, KL, dtype=torch.bool).triu(1), float("-inf"))
    if kpad is not None:
        a = a.masked_fill(~torch.from_numpy(kpad)[:, None, None, :], float("-inf"))
    ot = torch.einsum("bhij,bhje->bhie", torch.softmax(a, -1), ts[2].repeat_interleave(rep, 1))
    ot.backward(torch.from_numpy(do))
    checks = [rel(o, ot.detach().numpy()), rel(dq, ts[0].grad.numpy()), rel(dk, ts[1].grad.numpy()),
              rel(dv, ts[2].grad.numpy())]
    if pt is not None:
        checks.append(rel(dp, pt.grad.numpy()))
    assert max(checks) < 1e-12, (name, checks)
    f32 = lambda a: a.astype(np.float32)  # noqa: E731  (inputs are exact in float32)
    arrs = dict(q=f32(q), k=f32(k), v=f32(v), do=f32(do), o=f32(o), ms=f32(ms), ls=f32(ls), dq=f32(dq),
                dk=f32(dk), dv=f32(dv), meta=np.array([B, QH, KH, QL, KL, E, int(causal)]),
                scale=np.array([scale]), dtype=np.array([dtype]))
    if use_pair:
        arrs.update(pair=f32(pair), dpair=f32(dp))
    if use_kpad:
        arrs.update(kpad=kpad)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrs)


def rowwise_cases():
    rng = np.random.default_rng(100)
    rd = lambda a: oracle.round_to("bf16", a)  # noqa: E731
    x = rd(rng.standard_normal((6, 264)))
    g = rd(rng.standard_normal((6, 264)))
    w = rd(1 + 0.02 * rng.standard_normal(264))
    b = rd(0.02 * rng.standard_normal(264))
    y = oracle.softmax_fwd(x)
    dx = oracle.softmax_bwd(g, y)
    assert rel(y, torch.softmax(torch.from_numpy(x), -1).numpy()) < 1e-13
    np.savez_compressed(os.path.join(HERE, "softmax_bf16.npz"), **{n: a.astype(np.float32) for n, a in dict(x=x, dy=g, y=y, dx=dx).items()})
    yr, r = oracle.rms_norm_fwd(x, w)
    dxr, dwr = oracle.rms_norm_bwd(g, r, x, w)
    xt = torch.from_numpy(x).requires_grad_(True)
    wt = torch.from_numpy(w).requires_grad_(True)
    yt = F.rms_norm(xt, (264,), wt, eps=1e-6)
    yt.backward(torch.from_numpy(g))
    assert max(rel(yr, yt.detach().numpy()), rel(dxr, xt.grad.numpy()), rel(dwr, wt.grad.numpy())) < 1e-12
    np.savez_compressed(os.path.join(HERE, "rms_norm_bf16.npz"), **{n: a.astype(np.float32) for n, a in dict(x=x, w=w, dy=g, y=yr, rstd=r, dx=dxr, dw=dwr).items()})
    yl, mu, rl = oracle.layer_norm_fwd(x, w, b)
    dxl, dwl, dbl = oracle.layer_norm_bwd(g, mu, rl, x, w)
    xt = torch.from_numpy(x).requires_grad_(True)
    wt = torch.from_numpy(w).requires_grad_(True)
    bt = torch.from_numpy(b).requires_grad_(True)
    yt = F.layer_norm(xt, (264,), wt, bt, eps=1e-6)
    yt.backward(torch.from_numpy(g))
    assert max(rel(yl, yt.detach().numpy()), rel(dxl, xt.grad.numpy()), rel(dwl, wt.grad.numpy()),
               rel(dbl, bt.grad.numpy())) < 1e-12
    np.savez_compressed(os.path.join(HERE, "layer_norm_bf16.npz"), **{n: a.astype(np.float32) for n, a in dict(
        x=x, w=w, b=b, dy=g, y=yl, mu=mu, rstd=rl, dx=dxl, dw=dwl, db=dbl).items()})
    q = rd(rng.standard_normal((2, 3, 40, 64)))
    k = rd(rng.standard_normal((2, 1, 40, 64)))
    pos = rng.integers(0, 4096, (2, 40)).astype(np.float64)
    c, s = oracle.rotary_embedding(64, pos, mode=oracle.FAITHFUL)
    c, s = oracle.round_to("f32", c), oracle.round_to("f32", s)
    qo, ko = oracle.llama_rope(q, k, c, s, 1.0)
    np.savez_compressed(os.path.join(HERE, "llama_rope_bf16.npz"), **{n: a.astype(np.float32) for n, a in dict(
        q=q, k=k, pos=pos, cos=c, sin=s, qo=qo, ko=ko).items()})


def main():
    attention_case("attn_f32_e16_gqa_causal_pair", "f32", 2, 4, 2, 37, 37, 16, True, True, False, 1)
    attention_case("attn_f32_e32_kpad_ragged", "f32", 3, 2, 2, 29, 70, 32, False, False, True, 2)
    attention_case("attn_bf16_e64_causal", "bf16", 1, 2, 2, 100, 100, 64, True, False, False, 3)
    attention_case("attn_f16_e128_pair_kpad", "f16", 1, 2, 1, 33, 50, 128, False, True, True, 4)
    rowwise_cases()
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
