"""GPU parity at the full sizes of the five benchmark configurations.

Each test runs the HIP path at the full shape of one configuration and checks it two ways:
  * against the oracle (float64) on the same seeded inputs, over the whole problem where
    the oracle finishes in seconds, else over independent slices of it (heads, or the
    valid prefix of one sequence, which is an exact sub-problem);
  * through invariants that hold at any size: softmax rows sum to 1; every valid causal
    attention row's P sums to 1, so sum_k dV[k] = sum_q dO[q] per head; keys hidden by
    the padding mask get exactly zero dK and dV; the first causal row's output is v[0].
Configurations (Julia shapes; numpy/torch shapes are reversed):
  1. flash_attention f32 (E,L,H,B) = (64,1024,4,2), non-causal, q,k,v ~ U[0,1), loss = sum(o)
  2. online_softmax f32 (8192,1024); rms_norm / layer_norm fwd+bwd bf16 x (4096,16384)
  3. flash_attention bf16 (64,4096,4,4) causal, q,k,v ~ N(0,1)/sqrt(E), loss = sum(o)
  4. flash_attention bf16 (32,768,8,2) with pair bias (8,768,768,2), grads incl. dpair
  5. llama_rope bf16 q (128,8192,32,4), k (128,8192,8,4), then causal GQA attention with
     per-sequence lengths U[1024,8192] as a key-padding mask; padded query rows are left
     out of the loss (dO = 0 there), as the reference's own semantics require.
Tolerances: norm-wise relative error <= 1e-5 (float32), <= 2e-2 (bfloat16).
"""
import numpy as np
import pytest
import torch

import nnop
import oracle
from helpers import TOL, host, make, rel_err

pytestmark = pytest.mark.gpu


def check(errs, tol):
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"tolerance {tol}: {bad} (all: {errs})"


def test_config1_f32_attention(dev):
    B, H, L, E = 2, 4, 1024, 64
    rng = np.random.default_rng(0)
    q, qn = make(rng, (B, H, L, E), torch.float32, dev, kind="uniform")
    k, kn = make(rng, (B, H, L, E), torch.float32, dev, kind="uniform")
    v, vn = make(rng, (B, H, L, E), torch.float32, dev, kind="uniform")
    do = torch.ones_like(q)
    print("config 1: f32 (64,1024,4,2) non-causal", flush=True)
    o, ms, ls = nnop._flash_attention(q, k, v, causal=False)
    scale = nnop.attention_scale(E, torch.float32)
    o_r, _, _ = oracle.attn_fwd(qn, kn, vn, causal=False, scale=scale)
    of, msf, lsf = oracle.attn_fwd(qn, kn, vn, causal=False, scale=scale, mode=oracle.FAITHFUL)
    errs = {"o": rel_err(host(o), o_r)}
    # With q, k, v ~ U[0,1) and dO = 1, dQ = scale sum_k dS K cancels on K's mean of 0.5.
    # The exact float32 backward centres K (every row of dS sums to zero) and is held to
    # 1e-5 against float64 like every other output.  In the reference's Float16 Q/K mode the
    # rows of P do not sum to one (S from rounded Q/K, lse from the float32 forward), so dQ
    # carries the reference algorithm's own error (~1e-4 against float64): there dQ is held
    # to "no worse than that algorithm" (the oracle's FAITHFUL replay of it) and its
    # distance to that replay is printed.
    extra = {}
    for qk16 in (False, True):
        sfx = "_16" if qk16 else ""
        dq, dk, dv, _ = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, causal=False, qk_fp16=qk16)
        dq_r, dk_r, dv_r, _ = oracle.attn_bwd(np.ones_like(qn), qn, kn, vn, causal=False, scale=scale,
                                              qk_fp16=qk16)
        errs.update({"dk" + sfx: rel_err(host(dk), dk_r), "dv" + sfx: rel_err(host(dv), dv_r)})
        if not qk16:
            errs["dq"] = rel_err(host(dq), dq_r)
            continue
        dq_f, dk_f, dv_f, _ = oracle.attn_bwd(np.ones_like(qn), qn, kn, vn, causal=False, scale=scale,
                                              mode=oracle.FAITHFUL, o=of, ms=msf, ls=lsf, qk_fp16=True)
        bound = max(1e-5, rel_err(dq_f, dq_r))
        dq_err = rel_err(host(dq), dq_r)
        extra = {"dq_16 vs float64": dq_err, "FAITHFUL dq_16 vs float64": bound,
                 "dq_16 vs FAITHFUL": rel_err(host(dq), dq_f), "dk_16 vs FAITHFUL": rel_err(host(dk), dk_f),
                 "dv_16 vs FAITHFUL": rel_err(host(dv), dv_f)}
        assert dq_err <= bound, (dq_err, bound)
    print("config 1 errors", errs, "Float16 Q/K mode", extra, flush=True)
    check(errs, 1e-5)


def test_config2_softmax(dev):
    rng = np.random.default_rng(1)
    x, xn = make(rng, (1024, 8192), torch.float32, dev)
    g, gn = make(rng, (1024, 8192), torch.float32, dev)
    print("config 2: online_softmax f32 (8192,1024)", flush=True)
    y = nnop._online_softmax(x)
    dx = nnop.grad_online_softmax(g, y)
    y_r = oracle.softmax_fwd(xn)
    check({"y": rel_err(host(y), y_r), "dx": rel_err(host(dx), oracle.softmax_bwd(gn, y_r))}, 1e-5)
    assert np.allclose(host(y).sum(-1), 1.0, atol=1e-5)


@pytest.mark.parametrize("norm", ["rms", "layer"])
def test_config2_norms(dev, norm):
    n, emb = 16384, 4096
    rng = np.random.default_rng(1)
    x, xn = make(rng, (n, emb), torch.bfloat16, dev)
    w, wn = make(rng, (emb,), torch.bfloat16, dev, scale=0.02, offset=1.0)
    b, bn = make(rng, (emb,), torch.bfloat16, dev, scale=0.02)
    dy, dyn = make(rng, (n, emb), torch.bfloat16, dev)
    print(f"config 2: {norm}_norm bf16 (4096,16384) fwd+bwd", flush=True)
    if norm == "rms":
        y, rstd = nnop._rms_norm(x, w, eps=1e-6)
        dx, dw = nnop.grad_rms_norm(dy, rstd, x, w)
        y_r, rstd_r = oracle.rms_norm_fwd(xn, wn, eps=1e-6)
        dx_r, dw_r = oracle.rms_norm_bwd(dyn, rstd_r, xn, wn)
        errs = {"y": rel_err(host(y), y_r), "rstd": rel_err(host(rstd), rstd_r), "dx": rel_err(host(dx), dx_r),
                "dw": rel_err(host(dw), dw_r)}
    else:
        y, mu, rstd = nnop._layer_norm(x, w, b, eps=1e-6)
        dx, dw, db = nnop.grad_layer_norm(dy, mu, rstd, x, w, b)
        y_r, mu_r, rstd_r = oracle.layer_norm_fwd(xn, wn, bn, eps=1e-6)
        dx_r, dw_r, db_r = oracle.layer_norm_bwd(dyn, mu_r, rstd_r, xn, wn)
        errs = {"y": rel_err(host(y), y_r), "mu": rel_err(host(mu), mu_r), "rstd": rel_err(host(rstd), rstd_r),
                "dx": rel_err(host(dx), dx_r), "dw": rel_err(host(dw), dw_r), "db": rel_err(host(db), db_r)}
    check(errs, TOL[torch.bfloat16])


def test_config3_headline_attention(dev):
    B, H, L, E = 4, 4, 4096, 64
    rng = np.random.default_rng(2)
    s = 1.0 / np.sqrt(E)
    q, qn = make(rng, (B, H, L, E), torch.bfloat16, dev, scale=s)
    k, kn = make(rng, (B, H, L, E), torch.bfloat16, dev, scale=s)
    v, vn = make(rng, (B, H, L, E), torch.bfloat16, dev, scale=s)
    do = torch.ones_like(q)
    print("config 3: bf16 (64,4096,4,4) causal, full size; oracle on heads (0,0) and (3,3)", flush=True)
    o, ms, ls = nnop._flash_attention(q, k, v, causal=True)
    dq, dk, dv, _ = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, causal=True)
    torch.cuda.synchronize()
    scale = nnop.attention_scale(E, torch.bfloat16)
    errs = {}
    for b, h in ((0, 0), (3, 3)):  # heads are independent: each slice is an exact sub-problem
        sl = (slice(b, b + 1), slice(h, h + 1))
        o_r, _, _ = oracle.attn_fwd(qn[sl], kn[sl], vn[sl], causal=True, scale=scale)
        dq_r, dk_r, dv_r, _ = oracle.attn_bwd(np.ones_like(qn[sl]), qn[sl], kn[sl], vn[sl], causal=True,
                                              scale=scale)
        errs.update({f"o{b}{h}": rel_err(host(o[sl]), o_r), f"dq{b}{h}": rel_err(host(dq[sl]), dq_r),
                     f"dk{b}{h}": rel_err(host(dk[sl]), dk_r), f"dv{b}{h}": rel_err(host(dv[sl]), dv_r)})
    check(errs, TOL[torch.bfloat16])
    # every head: sum_k dV[k] = sum_q dO[q] = L (each causal row of P sums to 1), and the
    # first query only sees key 0
    dvsum = host(dv).sum(axis=2)
    assert np.allclose(dvsum, L, rtol=2e-2), float(np.abs(dvsum / L - 1).max())
    assert torch.allclose(o[:, :, 0, :].float(), v[:, :, 0, :].float(), rtol=1e-2, atol=1e-2)
    assert torch.isfinite(dq).all() and torch.isfinite(dk).all()


def test_config4_pair_bias(dev):
    B, H, L, E = 2, 8, 768, 32
    rng = np.random.default_rng(3)
    q, qn = make(rng, (B, H, L, E), torch.bfloat16, dev)
    k, kn = make(rng, (B, H, L, E), torch.bfloat16, dev)
    v, vn = make(rng, (B, H, L, E), torch.bfloat16, dev)
    pair, pn = make(rng, (B, L, L, H), torch.bfloat16, dev)  # Julia (H, Lq, Lk, B)
    do, don = make(rng, (B, H, L, E), torch.bfloat16, dev)
    print("config 4: bf16 (32,768,8,2) pair bias, grads incl. dpair", flush=True)
    o, ms, ls = nnop._flash_attention(q, k, v, pair, causal=False)
    dq, dk, dv, dpair = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, pair, causal=False)
    scale = nnop.attention_scale(E, torch.bfloat16)
    o_r, _, _ = oracle.attn_fwd(qn, kn, vn, pn, causal=False, scale=scale)
    dq_r, dk_r, dv_r, dp_r = oracle.attn_bwd(don, qn, kn, vn, pn, causal=False, scale=scale)
    check({"o": rel_err(host(o), o_r), "dq": rel_err(host(dq), dq_r), "dk": rel_err(host(dk), dk_r),
           "dv": rel_err(host(dv), dv_r), "dpair": rel_err(host(dpair), dp_r)}, TOL[torch.bfloat16])


def test_config5_rope_gqa_varlen(dev):
    B, QH, KH, L, E = 4, 32, 8, 8192, 128
    rng = np.random.default_rng(4)
    lens = rng.integers(1024, 8193, size=B)
    print(f"config 5: bf16 rope + causal GQA 32:8, E=128, L=8192, lengths {lens.tolist()}", flush=True)
    q, qn = make(rng, (B, QH, L, E), torch.bfloat16, dev)
    k, kn = make(rng, (B, KH, L, E), torch.bfloat16, dev)
    v, vn = make(rng, (B, KH, L, E), torch.bfloat16, dev)
    pos = torch.arange(L, dtype=torch.float32)[None].expand(B, L)
    cos, sin = nnop.LlamaRotaryEmbedding(E)(pos)
    cos, sin = cos.to(dev), sin.to(dev)
    qr, kr = nnop._llama_rope(q, k, cos, sin, bwd=False)
    torch.cuda.synchronize()
    # RoPE: batch 0 against the oracle on the same cos/sin values
    c0, s0 = host(cos[:1]), host(sin[:1])
    qr_r, kr_r = oracle.llama_rope(qn[:1], kn[:1], c0, s0)
    check({"rope_q": rel_err(host(qr[:1]), qr_r), "rope_k": rel_err(host(kr[:1]), kr_r)}, TOL[torch.bfloat16])

    kpad = np.arange(L)[None, :] < lens[:, None]          # (B, L): key j of batch b is real
    kp = torch.from_numpy(kpad).to(dev)
    do_np = rng.standard_normal((B, QH, L, E)) * kpad[:, None, :, None]  # padded rows out of the loss
    do = torch.from_numpy(do_np).to(torch.bfloat16).to(dev)
    don = do.double().cpu().numpy()
    o, ms, ls = nnop._flash_attention(qr, kr, v, causal=True, kpad_mask=kp)
    dq, dk, dv, _ = nnop.grad_flash_attention(do, o, ms, ls, qr, kr, v, causal=True, kpad_mask=kp)
    torch.cuda.synchronize()

    # Oracle on the shortest sequence's valid prefix for kv head 0 and its 4 q heads: with
    # dO = 0 past the length, that prefix is an exact sub-problem (causal rows never see a
    # later key, padded keys are masked, padded queries contribute no gradient).
    b = int(np.argmin(lens))
    n = int(lens[b])
    qs = host(qr[b:b + 1, 0:4, :n])
    ks = host(kr[b:b + 1, 0:1, :n])
    vs = vn[b:b + 1, 0:1, :n]
    scale = nnop.attention_scale(E, torch.bfloat16)
    o_r, _, _ = oracle.attn_fwd(qs, ks, vs, causal=True, scale=scale)
    dq_r, dk_r, dv_r, _ = oracle.attn_bwd(don[b:b + 1, 0:4, :n], qs, ks, vs, causal=True, scale=scale)
    check({"o": rel_err(host(o[b:b + 1, 0:4, :n]), o_r), "dq": rel_err(host(dq[b:b + 1, 0:4, :n]), dq_r),
           "dk": rel_err(host(dk[b:b + 1, 0:1, :n]), dk_r), "dv": rel_err(host(dv[b:b + 1, 0:1, :n]), dv_r)},
          TOL[torch.bfloat16])

    # Full size: padded keys get exactly zero gradient; sum_k dV over a kv head equals the
    # sum of dO over its 4 q heads and the valid rows; everything finite.
    dk_h, dv_h = host(dk), host(dv)
    for bb in range(B):
        assert not dk_h[bb, :, lens[bb]:].any() and not dv_h[bb, :, lens[bb]:].any()
    lhs = dv_h.sum(axis=2)                                         # (B, KH, E)
    rhs = don.reshape(B, KH, QH // KH, L, E).sum(axis=(2, 3))     # (B, KH, E)
    assert rel_err(lhs, rhs) <= 2e-2, rel_err(lhs, rhs)
    assert torch.isfinite(o).all() and torch.isfinite(dq).all()


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_long_sequence_causal(dev, dt):
    """A 65536-token causal sequence (E = 64, 2 heads): large row and tile indices in every
    kernel.  Under the causal mask the first 256 queries see only the first 256 keys, so
    o and dq of those rows are an exact sub-problem for the oracle; for every head,
    sum_k dV = sum_q dO (each causal row of P sums to one) checks the whole dV, and every
    gradient is finite."""
    dtype = {"bf16": torch.bfloat16, "f32": torch.float32}[dt]
    B, H, L, E = 1, 2, 65536, 64
    rng = np.random.default_rng(17)
    s = 1.0 / np.sqrt(E)
    q, qn = make(rng, (B, H, L, E), dtype, dev, scale=s)
    k, kn = make(rng, (B, H, L, E), dtype, dev, scale=s)
    v, vn = make(rng, (B, H, L, E), dtype, dev)
    do, don = make(rng, (B, H, L, E), dtype, dev)
    print(f"long sequence: {dt} (64, 65536, 2, 1) causal", flush=True)
    o, ms, ls = nnop._flash_attention(q, k, v, causal=True)
    dq, dk, dv, _ = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, causal=True, qk_fp16=False)
    torch.cuda.synchronize()
    scale = nnop.attention_scale(E, dtype)
    P = 256
    o_r, _, _ = oracle.attn_fwd(qn[:, :, :P], kn[:, :, :P], vn[:, :, :P], causal=True, scale=scale)
    dq_r, _, _, _ = oracle.attn_bwd(don[:, :, :P], qn[:, :, :P], kn[:, :, :P], vn[:, :, :P], causal=True, scale=scale)
    errs = {"o[:256]": rel_err(host(o[:, :, :P]), o_r), "dq[:256]": rel_err(host(dq[:, :, :P]), dq_r)}
    check(errs, TOL[dtype])
    dvsum = host(dv).astype(np.float64).sum(axis=2)
    dosum = host(do).astype(np.float64).sum(axis=2)
    assert rel_err(dvsum, dosum) <= (2e-2 if dtype != torch.float32 else 1e-4), rel_err(dvsum, dosum)
    assert torch.isfinite(dq).all() and torch.isfinite(dk).all() and torch.isfinite(dv).all()
