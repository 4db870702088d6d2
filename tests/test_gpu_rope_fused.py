"""RoPE on the device: LlamaRotaryEmbedding's tables from the library's kernel, and the
backward of flash_attention(llama_rope(q, k)..., v) with ∇llama_rope fused into the attention
backward's dQ / dK epilogues (onionop_flash_attn_bwd_rope, onionop_flash_attn_varlen_bwd_rope).

The fused gradients are checked against the unfused composition (attention backward, then the
library's ∇llama_rope, src/rope/llama_rope.jl:92) and against the oracle: float64 attention
backward on the same rotated q, k, then the oracle's rotate-half pullback.  dv and dpair do not
involve the rotation and must equal the unfused ones bit for bit.
"""
import zlib

import numpy as np
import pytest
import torch

import nnop
import oracle
from helpers import DTYPES, TOL, host, make, rel_err

pytestmark = pytest.mark.gpu


def test_rotary_tables_on_device(dev):
    """LlamaRotaryEmbedding (src/rope/llama_rope.jl:1-22) computed on the device: dim 128,
    positions 0..8191 of 4 sequences, and arbitrary float positions at dim 64."""
    for dim, pos in ((128, torch.arange(8192, dtype=torch.float32)[None].expand(4, 8192).contiguous()),
                     (64, torch.from_numpy(np.random.default_rng(3).integers(0, 20000, (3, 257)).astype(np.float32)))):
        print(f"case tables dim={dim} pos={tuple(pos.shape)}", flush=True)
        c, s = nnop.LlamaRotaryEmbedding(dim)(pos.to(dev))
        torch.cuda.synchronize()
        assert c.is_cuda and tuple(c.shape) == (pos.shape[0], pos.shape[1], dim)
        c, s = host(c), host(s)
        assert np.array_equal(c[..., : dim // 2], c[..., dim // 2:])
        cf, sf = oracle.rotary_embedding(dim, pos.double().numpy(), mode=oracle.FAITHFUL)
        assert np.abs(c - cf).max() <= 2e-7 and np.abs(s - sf).max() <= 2e-7
        # the host generator (torch float32 on the CPU) gives the same table
        ch, sh = nnop.LlamaRotaryEmbedding(dim)(pos)
        assert np.abs(c - ch.double().numpy()).max() <= 2e-7 and np.abs(s - sh.double().numpy()).max() <= 2e-7


def _oracle_rope_grads(qr, kr, v, do, pair, kpad, causal, scale, qk16, cos, sin):
    """Float64 attention backward on the rotated q, k, then the rotate-half pullback."""
    dqr, dkr, dv, dp = oracle.attn_bwd(do, qr, kr, v, pair, kpad, causal, scale, qk_fp16=qk16)
    dq, dk = oracle.llama_rope(dqr, dkr, cos, sin, sin_sign=-1.0)
    return dq, dk, dv, dp


@pytest.mark.parametrize("case", [
    ("bf16", 64, 300, 4, 2, 2, True, False, False),
    ("f16", 128, 257, 4, 4, 1, True, True, False),
    ("f32", 32, 200, 2, 2, 2, False, False, True),
    ("bf16", 256, 130, 2, 1, 1, True, False, False),
    ("f32", 64, 129, 4, 2, 1, True, False, False),
    ("bf16", 16, 100, 2, 2, 1, False, True, True),
], ids=lambda c: "-".join(map(str, c)))
def test_fused_rope_backward(dev, case):
    dt, E, L, QH, KH, B, causal, use_kpad, use_pair = case
    dtype = DTYPES[dt]
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    q, _ = make(rng, (B, QH, L, E), dtype, dev)
    k, _ = make(rng, (B, KH, L, E), dtype, dev)
    v, vn = make(rng, (B, KH, L, E), dtype, dev)
    do, don = make(rng, (B, QH, L, E), dtype, dev)
    pair = pairn = None
    if use_pair:
        pair, pairn = make(rng, (B, L, L, QH), dtype, dev)
    kpad = kp = None
    if use_kpad:
        kpad = np.ones((B, L), dtype=bool)
        kpad[-1, -11:] = False
        kp = torch.from_numpy(kpad).to(dev)
    pos = torch.from_numpy(rng.integers(0, 4 * L, (B, L)).astype(np.float32)).to(dev)
    cos, sin = nnop.LlamaRotaryEmbedding(E)(pos)
    print(f"case {case}", flush=True)
    qr, kr = nnop._llama_rope(q, k, cos, sin, bwd=False)
    o, ms, ls = nnop._flash_attention(qr, kr, v, pair, causal=causal, kpad_mask=kp)
    qk16 = dtype == torch.float32
    dq, dk, dv, dpair = nnop.grad_flash_attention_rope(do, o, ms, ls, qr, kr, v, cos, sin, pair, causal=causal,
                                                       kpad_mask=kp, qk_fp16=qk16)
    # unfused: attention backward, then the library's ∇llama_rope
    dqr2, dkr2, dv2, dpair2 = nnop.grad_flash_attention(do, o, ms, ls, qr, kr, v, pair, causal=causal, kpad_mask=kp,
                                                        qk_fp16=qk16)
    dq2, dk2 = nnop.grad_llama_rope(dqr2, dkr2, cos=cos, sin=sin)
    torch.cuda.synchronize()
    assert torch.equal(dv, dv2)
    if use_pair:
        assert torch.equal(dpair, dpair2)
    # the fused path rotates the float32 accumulators; the unfused one rounds dq', dk' to the
    # element type first
    close = 1e-6 if dtype == torch.float32 else 1e-2
    assert rel_err(host(dq), host(dq2)) <= close and rel_err(host(dk), host(dk2)) <= close
    dq_r, dk_r, dv_r, _ = _oracle_rope_grads(host(qr), host(kr), vn, don, pairn, kpad, causal,
                                             nnop.attention_scale(E, dtype), qk16, host(cos), host(sin))
    errs = {"dq": rel_err(host(dq), dq_r), "dk": rel_err(host(dk), dk_r), "dv": rel_err(host(dv), dv_r)}
    tol = TOL[dtype]
    assert all(e <= tol for e in errs.values()), f"tolerance {tol}: {errs}"


@pytest.mark.parametrize("dt,E,causal", [("bf16", 128, True), ("f32", 64, False)])
def test_fused_rope_backward_varlen(dev, dt, E, causal):
    """Packed sequences whose positions restart per sequence, the way the packed GQA workload
    runs: one cos / sin row per packed position."""
    dtype = DTYPES[dt]
    rng = np.random.default_rng(9)
    lens = [100, 37, 64, 1]
    QH, KH = 4, 2
    T = sum(lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32), device=dev)
    q, _ = make(rng, (QH, T, E), dtype, dev)
    k, _ = make(rng, (KH, T, E), dtype, dev)
    v, _ = make(rng, (KH, T, E), dtype, dev)
    do, _ = make(rng, (QH, T, E), dtype, dev)
    pos = torch.from_numpy(np.concatenate([np.arange(n) for n in lens]).astype(np.float32))[None].to(dev)
    cos, sin = nnop.LlamaRotaryEmbedding(E)(pos)  # (1, T, E)
    print(f"case varlen {dt} E={E} causal={causal}", flush=True)
    qr, kr = nnop._llama_rope(q[None], k[None], cos, sin, bwd=False)
    qr, kr = qr[0], kr[0]
    mx = max(lens)
    o, ms, ls = nnop._flash_attention_varlen(qr, kr, v, cu, cu, mx, mx, causal=causal)
    qk16 = dtype == torch.float32
    dq, dk, dv = nnop.grad_flash_attention_varlen_rope(do, o, ms, ls, qr, kr, v, cos[0], sin[0], cu, mx,
                                                       causal=causal, qk_fp16=qk16)
    dqr2, dkr2, dv2 = nnop.grad_flash_attention_varlen(do, o, ms, ls, qr, kr, v, cu, cu, mx, mx, causal=causal,
                                                       qk_fp16=qk16)
    dq2, dk2 = nnop.grad_llama_rope(dqr2[None].contiguous(), dkr2[None].contiguous(), cos=cos, sin=sin)
    torch.cuda.synchronize()
    assert torch.equal(dv, dv2)
    close = 1e-6 if dtype == torch.float32 else 1e-2
    assert rel_err(host(dq), host(dq2[0])) <= close and rel_err(host(dk), host(dk2[0])) <= close


def test_flash_attention_rope_autograd(dev):
    """nnop.flash_attention_rope under autograd equals llama_rope then flash_attention."""
    rng = np.random.default_rng(12)
    B, QH, KH, L, E = 2, 4, 2, 150, 64
    q0, _ = make(rng, (B, QH, L, E), torch.bfloat16, dev)
    k0, _ = make(rng, (B, KH, L, E), torch.bfloat16, dev)
    v0, _ = make(rng, (B, KH, L, E), torch.bfloat16, dev)
    do, _ = make(rng, (B, QH, L, E), torch.bfloat16, dev)
    cos, sin = nnop.LlamaRotaryEmbedding(E)(torch.arange(L, dtype=torch.float32, device=dev)[None].expand(B, L))
    q, k, v = (t.clone().requires_grad_(True) for t in (q0, k0, v0))
    nnop.flash_attention_rope(q, k, v, cos, sin, causal=True).backward(do)
    q2, k2, v2 = (t.clone().requires_grad_(True) for t in (q0, k0, v0))
    qr, kr = nnop.llama_rope(q2, k2, cos=cos, sin=sin)
    nnop.flash_attention(qr, kr, v2, causal=True).backward(do)
    torch.cuda.synchronize()
    assert torch.equal(v.grad, v2.grad)
    assert rel_err(host(q.grad), host(q2.grad)) <= 1e-2 and rel_err(host(k.grad), host(k2.grad)) <= 1e-2
