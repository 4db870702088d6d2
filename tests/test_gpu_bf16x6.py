"""float32 flash attention with every product on the bf16 matrix cores
(nnop.set_float32_attention_precision("bf16x6"), element type code ONIONOP_F32_BF16X6).

Each float32 operand is split exactly into three bf16 parts and each product is the sum of
the six part products above 2^-23 relative size, accumulated in float32.  The bar is the
float32 one: norm-wise relative error <= 1e-5 against the float64 oracle on o, ms, ls, dq,
dk, dv (and dpair), over the float32 cases of the dense, GQA, Float16 Q/K, head-dim-256 and
packed-sequence sweeps, and config 1 at full size.  The results must also agree with the
float32 MFMA path to well inside that bar.
"""
import zlib

import numpy as np
import pytest
import torch

import nnop
import oracle
from helpers import host, make, rel_err
from test_gpu_attention import CASES, GQA, run_case
from test_gpu_varlen import CASES as VARLEN_CASES
from test_gpu_varlen import run_varlen

pytestmark = pytest.mark.gpu

F32_CASES = [c for c in CASES if c[0] == "f32"]


@pytest.mark.parametrize("case", F32_CASES, ids=lambda c: "-".join(map(str, c)))
def test_bf16x6_parity(dev, case):
    dt, E, QL, KL, QH, KH, B, causal, pair, kpad = case
    with nnop.float32_attention_precision("bf16x6"):
        run_case(dev, dt, E, QL, KL, QH, KH, B, causal, pair, kpad, seed=zlib.crc32(repr(case).encode()) % 1000)


@pytest.mark.parametrize("case", GQA, ids=lambda c: "-".join(map(str, c)))
def test_bf16x6_gqa(dev, case):
    QH, KH, causal, E, L = case
    with nnop.float32_attention_precision("bf16x6"):
        run_case(dev, "f32", E, L, L, QH, KH, 2, causal, False, False, seed=7)


@pytest.mark.parametrize("use_pair", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16x6_qk_fp16_mode(dev, causal, use_pair):
    """The reference backward's Float16 Q/K (src/attention_bwd.jl:20-21) under bf16x6: the
    float16 values are split exactly, so the products are the reference's."""
    with nnop.float32_attention_precision("bf16x6"):
        run_case(dev, "f32", 64, 300, 300, 2, 2, 2, causal, use_pair, False, seed=3, qk16=True)


@pytest.mark.parametrize("case", [("f32", 256, 130, 2, 1, 1, True, False, False),
                                  ("f32", 16, 100, 2, 2, 1, False, True, True),
                                  ("f32", 32, 640, 4, 4, 2, True, False, True)],
                         ids=lambda c: "-".join(map(str, c)))
def test_bf16x6_head_dims(dev, case):
    dt, E, L, QH, KH, B, causal, pair, kpad = case
    with nnop.float32_attention_precision("bf16x6"):
        run_case(dev, dt, E, L, L, QH, KH, B, causal, pair, kpad, seed=11)


@pytest.mark.parametrize("case", [c for c in VARLEN_CASES if c[0] == "f32"],
                         ids=lambda c: f"{c[0]}-E{c[1]}-{c[2]}x{c[3]}-{len(c[4])}seq-c{int(c[6])}")
def test_bf16x6_varlen(dev, case):
    dt, E, QH, KH, qlens, klens, causal = case
    with nnop.float32_attention_precision("bf16x6"):
        run_varlen(dev, dt, E, QH, KH, qlens, klens, causal, seed=sum(qlens) % 997)


def test_bf16x6_config1(dev):
    """Config 1 (float32 (64,1024,4,2), non-causal, q, k, v ~ U[0,1), dO = 1) at full size:
    every output within 1e-5 of float64 (exact Q/K), and no further from float64 than twice
    the float32 MFMA path's distance (or 1e-6)."""
    B, H, L, E = 2, 4, 1024, 64
    rng = np.random.default_rng(0)
    q, qn = make(rng, (B, H, L, E), torch.float32, dev, kind="uniform")
    k, kn = make(rng, (B, H, L, E), torch.float32, dev, kind="uniform")
    v, vn = make(rng, (B, H, L, E), torch.float32, dev, kind="uniform")
    do = torch.ones_like(q)
    print("config 1 under bf16x6", flush=True)
    with nnop.float32_attention_precision("bf16x6"):
        o, ms, ls = nnop._flash_attention(q, k, v, causal=False)
        dq, dk, dv, _ = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, causal=False, qk_fp16=False)
    o2, ms2, ls2 = nnop._flash_attention(q, k, v, causal=False)
    dq2, dk2, dv2, _ = nnop.grad_flash_attention(do, o2, ms2, ls2, q, k, v, causal=False, qk_fp16=False)
    torch.cuda.synchronize()
    scale = nnop.attention_scale(E, torch.float32)
    o_r, ms_r, ls_r = oracle.attn_fwd(qn, kn, vn, causal=False, scale=scale)
    dq_r, dk_r, dv_r, _ = oracle.attn_bwd(np.ones_like(qn), qn, kn, vn, causal=False, scale=scale)
    errs = {"o": rel_err(host(o), o_r), "ms": rel_err(host(ms), ms_r), "ls": rel_err(host(ls), ls_r),
            "dq": rel_err(host(dq), dq_r), "dk": rel_err(host(dk), dk_r), "dv": rel_err(host(dv), dv_r)}
    f32 = {"o": rel_err(host(o2), o_r), "dq": rel_err(host(dq2), dq_r), "dk": rel_err(host(dk2), dk_r),
           "dv": rel_err(host(dv2), dv_r)}
    print("bf16x6 vs float64", errs, "float32 MFMA vs float64", f32, flush=True)
    assert all(e <= 1e-5 for e in errs.values()), errs
    assert all(errs[n] <= max(2 * f32[n], 1e-6) for n in f32), (errs, f32)


def test_bf16x6_autograd_and_mode(dev):
    """flash_attention under autograd takes the mode of the call; the mode is restored
    after the context, and unknown modes are refused."""
    rng = np.random.default_rng(5)
    q, _ = make(rng, (1, 2, 200, 64), torch.float32, dev)
    k, _ = make(rng, (1, 2, 200, 64), torch.float32, dev)
    v, _ = make(rng, (1, 2, 200, 64), torch.float32, dev)
    with nnop.float32_attention_precision("bf16x6"):
        assert nnop.get_float32_attention_precision() == "bf16x6"
        qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
        nnop.flash_attention(qa, ka, va, causal=True).sum().backward()
    assert nnop.get_float32_attention_precision() == "float32"
    qb, kb, vb = (t.clone().requires_grad_(True) for t in (q, k, v))
    nnop.flash_attention(qb, kb, vb, causal=True).sum().backward()
    torch.cuda.synchronize()
    for a, b in ((qa.grad, qb.grad), (ka.grad, kb.grad), (va.grad, vb.grad)):
        assert rel_err(host(a), host(b)) <= 1e-5
    with pytest.raises(ValueError, match="bf16x6"):
        nnop.set_float32_attention_precision("tf32")


@pytest.mark.parametrize("E", [64, 128])
def test_bf16x6_fused_rope_backward(dev, E):
    """The fused ∇llama_rope backward under bf16x6 equals the unfused composition under
    bf16x6 (dv bit for bit), and both stay within 1e-5 of the float64 oracle."""
    rng = np.random.default_rng(21)
    B, QH, KH, L = 2, 4, 2, 200
    q, _ = make(rng, (B, QH, L, E), torch.float32, dev)
    k, _ = make(rng, (B, KH, L, E), torch.float32, dev)
    v, vn = make(rng, (B, KH, L, E), torch.float32, dev)
    do, don = make(rng, (B, QH, L, E), torch.float32, dev)
    pos = torch.arange(L, dtype=torch.float32, device=dev)[None].expand(B, L).contiguous()
    cos, sin = nnop.LlamaRotaryEmbedding(E)(pos)
    print(f"bf16x6 fused rope E={E}", flush=True)
    with nnop.float32_attention_precision("bf16x6"):
        qr, kr = nnop._llama_rope(q, k, cos, sin, bwd=False)
        o, ms, ls = nnop._flash_attention(qr, kr, v, causal=True)
        dq, dk, dv, _ = nnop.grad_flash_attention_rope(do, o, ms, ls, qr, kr, v, cos, sin, causal=True,
                                                       qk_fp16=False)
        dqr2, dkr2, dv2, _ = nnop.grad_flash_attention(do, o, ms, ls, qr, kr, v, causal=True, qk_fp16=False)
        dq2, dk2 = nnop.grad_llama_rope(dqr2, dkr2, cos=cos, sin=sin)
    torch.cuda.synchronize()
    assert torch.equal(dv, dv2)
    assert rel_err(host(dq), host(dq2)) <= 1e-6 and rel_err(host(dk), host(dk2)) <= 1e-6
    scale = nnop.attention_scale(E, torch.float32)
    dqr_r, dkr_r, dv_r, _ = oracle.attn_bwd(don, host(qr), host(kr), vn, None, None, True, scale)
    dq_r, dk_r = oracle.llama_rope(dqr_r, dkr_r, host(cos), host(sin), sin_sign=-1.0)
    errs = {"dq": rel_err(host(dq), dq_r), "dk": rel_err(host(dk), dk_r), "dv": rel_err(host(dv), dv_r)}
    assert all(e <= 1e-5 for e in errs.values()), errs


def test_bf16x6_masked_edges(dev):
    """Edge cases of the masks under bf16x6: a batch whose keys are all padded (o = 0,
    ms = -Inf, ls = 0, finite gradients), whole padded key blocks next to partial ones,
    and a single key (o = v exactly: P = 1 is exact in every split)."""
    kpad = np.ones((2, 130), dtype=bool)
    kpad[1, :] = False
    kpad2 = np.ones((2, 200), dtype=bool)
    kpad2[0, 64:160] = False
    kpad2[1, 150:] = False
    with nnop.float32_attention_precision("bf16x6"):
        run_case(dev, "f32", 32, 70, 130, 2, 2, 2, False, True, True, seed=5, kpad=kpad)
        for causal in (False, True):
            run_case(dev, "f32", 64, 180, 200, 4, 2, 2, causal, False, True, seed=11, kpad=kpad2)
        rng = np.random.default_rng(1)
        q, _ = make(rng, (2, 2, 1, 64), torch.float32, dev)
        k, _ = make(rng, (2, 2, 1, 64), torch.float32, dev)
        v, _ = make(rng, (2, 2, 1, 64), torch.float32, dev)
        o, ms, ls = nnop._flash_attention(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o, v)
    assert torch.all(ls == 1.0)
