"""GPU parity of flash attention over packed variable-length sequences.

Every sequence of the packed batch is checked against the oracle run on that sequence
alone (float64 on the same rounded values): o, ms, ls, dq, dk, dv.  Lengths include
empty and single-row sequences, ragged tiles, GQA, causal and not.  Tolerance as for the
dense kernels: norm-wise relative error <= 1e-5 (float32), <= 2e-2 (float16, bfloat16).
"""
import numpy as np
import pytest
import torch

import nnop
import oracle
from helpers import DTYPES, TOL, host, make, rel_err

pytestmark = pytest.mark.gpu


def run_varlen(dev, dt, E, QH, KH, qlens, klens, causal, seed, tail=0):
    dtype = DTYPES[dt]
    rng = np.random.default_rng(seed)
    cq = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    ck = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    Tq, Tk = int(cq[-1]) + tail, int(ck[-1]) + tail  # `tail` packed rows in no sequence
    q, qn = make(rng, (QH, Tq, E), dtype, dev)
    k, kn = make(rng, (KH, Tk, E), dtype, dev)
    v, vn = make(rng, (KH, Tk, E), dtype, dev)
    do, don = make(rng, (QH, Tq, E), dtype, dev)
    cu_q, cu_k = torch.from_numpy(cq).to(dev), torch.from_numpy(ck).to(dev)
    mq, mk = max(max(qlens), 1), max(max(klens), 1)
    print(f"varlen {dt} E={E} QH={QH} KH={KH} qlens={list(qlens)} klens={list(klens)} causal={causal} "
          f"seed={seed}", flush=True)
    o, ms, ls = nnop._flash_attention_varlen(q, k, v, cu_q, cu_k, mq, mk, causal=causal)
    dq, dk, dv = nnop.grad_flash_attention_varlen(do, o, ms, ls, q, k, v, cu_q, cu_k, mq, mk, causal=causal,
                                                  qk_fp16=False)
    torch.cuda.synchronize()
    scale = nnop.attention_scale(E, dtype)
    o, ms, ls, dq, dk, dv = (host(t) for t in (o, ms, ls, dq, dk, dv))
    tol = TOL[dtype]
    for b in range(len(qlens)):
        q0, q1, k0, k1 = cq[b], cq[b + 1], ck[b], ck[b + 1]
        if q1 == q0 and k1 == k0:
            continue
        sq = lambda a: a[:, q0:q1][None]  # (1, H, len, E)
        sk = lambda a: a[:, k0:k1][None]
        o_r, ms_r, ls_r = oracle.attn_fwd(sq(qn), sk(kn), sk(vn), None, None, causal, scale)
        dq_r, dk_r, dv_r, _ = oracle.attn_bwd(sq(don), sq(qn), sk(kn), sk(vn), None, None, causal, scale)
        errs = {}
        nv = np.linalg.norm(dv_r)

        def grad_err(a, r):  # an exactly zero dq / dk (one key per row): round-off against dv
            if np.linalg.norm(r) == 0.0 and nv > 0.0:
                return float(np.linalg.norm(np.asarray(a, dtype=np.float64)) / nv)
            return rel_err(a, r)

        if q1 > q0:
            errs["o"] = rel_err(o[:, q0:q1], o_r[0])
            errs["dq"] = grad_err(dq[:, q0:q1], dq_r[0])
            errs["ls"] = rel_err(ls[:, q0:q1], ls_r[0])
            fin = np.isfinite(ms_r[0])
            if fin.any():
                errs["ms"] = rel_err(ms[:, q0:q1][fin], ms_r[0][fin])
        if k1 > k0:
            errs["dk"] = grad_err(dk[:, k0:k1], dk_r[0])
            errs["dv"] = rel_err(dv[:, k0:k1], dv_r[0])
        bad = {n: e for n, e in errs.items() if not e <= tol}
        assert not bad, f"sequence {b}: tolerance {tol}: {bad} (all: {errs})"


CASES = [
    # dt, E, QH, KH, qlens, klens, causal
    ("bf16", 64, 4, 4, [300, 1, 64, 129, 0, 257], [300, 1, 64, 129, 0, 257], True),
    ("bf16", 64, 4, 2, [500, 37, 1000], [500, 37, 1000], False),
    ("bf16", 128, 8, 2, [255, 512, 33], [255, 512, 33], True),
    ("f16", 128, 4, 4, [40, 300, 97], [260, 5, 97], False),
    ("f16", 32, 2, 2, [100, 200, 3], [150, 7, 300], False),
    ("f16", 64, 2, 1, [63, 65, 1, 128], [63, 65, 1, 128], True),
    ("f32", 64, 2, 2, [70, 0, 190], [70, 0, 190], True),
    ("f32", 16, 2, 2, [50, 17], [33, 80], False),
    ("f32", 128, 4, 2, [129, 64], [129, 64], True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-E{c[1]}-{c[2]}x{c[3]}-{len(c[4])}seq-c{int(c[6])}")
def test_varlen_parity(dev, case):
    dt, E, QH, KH, qlens, klens, causal = case
    run_varlen(dev, dt, E, QH, KH, qlens, klens, causal, seed=sum(qlens) % 997)


def test_varlen_rows_outside_sequences_untouched(dev):
    """Packed rows past the last sequence are neither read into a result nor written."""
    run_varlen(dev, "bf16", 64, 2, 2, [130, 70], [130, 70], True, seed=5, tail=40)
    dtype = torch.bfloat16
    QH, E = 2, 64
    q = torch.randn((QH, 240, E), device=dev).to(dtype)
    k = torch.randn((QH, 240, E), device=dev).to(dtype)
    v = torch.randn((QH, 240, E), device=dev).to(dtype)
    cu = torch.tensor([0, 130, 200], dtype=torch.int32, device=dev)
    o = torch.full_like(q, 7.0)
    ms = torch.full((QH, 240), 7.0, device=dev)
    ls = torch.full((QH, 240), 7.0, device=dev)
    L = nnop.lib()
    from nnop._util import ptr, stream_of
    nnop._lib.check(L.onionop_flash_attn_varlen_fwd(stream_of(q), 2, E, 240, 240, QH, QH, 2, ptr(cu), ptr(cu),
                                                    130, 130, ptr(q), ptr(k), ptr(v), 1,
                                                    nnop.attention_scale(E, dtype), ptr(o), ptr(ms), ptr(ls)))
    torch.cuda.synchronize()
    assert torch.all(o[:, 200:] == 7.0) and torch.all(ms[:, 200:] == 7.0) and torch.all(ls[:, 200:] == 7.0)


def test_varlen_matches_dense_without_padding(dev):
    """Equal lengths: the packed call equals the dense call on the same data."""
    rng = np.random.default_rng(11)
    B, QH, L, E = 3, 4, 200, 64
    q, _ = make(rng, (B, QH, L, E), torch.bfloat16, dev)
    k, _ = make(rng, (B, QH, L, E), torch.bfloat16, dev)
    v, _ = make(rng, (B, QH, L, E), torch.bfloat16, dev)
    o, ms, ls = nnop._flash_attention(q, k, v, causal=True)
    pk = lambda t: t.permute(1, 0, 2, 3).reshape(QH, B * L, E).contiguous()
    cu = torch.arange(0, (B + 1) * L, L, dtype=torch.int32, device=dev)
    o2, ms2, ls2 = nnop._flash_attention_varlen(pk(q), pk(k), pk(v), cu, cu, L, L, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(pk(o), o2)
    assert torch.equal(ms.permute(1, 0, 2).reshape(QH, B * L), ms2)


def test_varlen_autograd(dev):
    rng = np.random.default_rng(3)
    QH, E = 2, 64
    lens = [90, 40]
    cu = torch.tensor([0, 90, 130], dtype=torch.int32, device=dev)
    q, qn = make(rng, (QH, 130, E), torch.float32, dev)
    k, kn = make(rng, (QH, 130, E), torch.float32, dev)
    v, vn = make(rng, (QH, 130, E), torch.float32, dev)
    q.requires_grad_(True)
    o = nnop.flash_attention_varlen(q, k, v, cu, cu, 90, 90, causal=True, qk_fp16=False)
    o.sum().backward()
    torch.cuda.synchronize()
    scale = nnop.attention_scale(E, torch.float32)
    for b, (s0, s1) in enumerate(((0, 90), (90, 130))):
        sl = lambda a: a[:, s0:s1][None]
        dq_r = oracle.attn_bwd(np.ones_like(sl(qn)), sl(qn), sl(kn), sl(vn), None, None, True, scale)[0]
        assert rel_err(host(q.grad)[:, s0:s1], dq_r[0]) <= 1e-5


def test_varlen_autograd_tail_rows(dev):
    """A packing buffer longer than its sequences (40 tail rows in no sequence): the
    output and gradient rows the kernels never visit are exactly zero, in o, q, k and v."""
    rng = np.random.default_rng(4)
    QH, KH, E, T = 4, 2, 64, 210
    cu = torch.tensor([0, 100, 170], dtype=torch.int32, device=dev)
    q, qn = make(rng, (QH, T, E), torch.bfloat16, dev)
    k, kn = make(rng, (KH, T, E), torch.bfloat16, dev)
    v, vn = make(rng, (KH, T, E), torch.bfloat16, dev)
    for t in (q, k, v):
        t.requires_grad_(True)
    print("varlen autograd: 40 tail rows, bf16 E=64 4:2 causal", flush=True)
    o = nnop.flash_attention_varlen(q, k, v, cu, cu, 100, 100, causal=True)
    o.float().sum().backward()
    torch.cuda.synchronize()
    for name, t in (("o", o), ("dq", q.grad), ("dk", k.grad), ("dv", v.grad)):
        a = host(t)
        assert np.isfinite(a).all(), name
        assert (a[:, 170:] == 0).all(), f"{name}: rows in no sequence must be zero"
    scale = nnop.attention_scale(E, torch.bfloat16)
    for s0, s1 in ((0, 100), (100, 170)):
        sl = lambda a: a[:, s0:s1][None]
        dq_r, dk_r, dv_r, _ = oracle.attn_bwd(np.ones((1, QH, s1 - s0, E)), sl(qn), sl(kn), sl(vn), None, None,
                                              True, scale)
        for name, got, ref in (("dq", q.grad, dq_r), ("dk", k.grad, dk_r), ("dv", v.grad, dv_r)):
            assert rel_err(host(got)[:, s0:s1], ref[0]) <= 2e-2, name


def test_varlen_errors(dev):
    q = torch.zeros((2, 10, 64), dtype=torch.bfloat16, device=dev)
    cu = torch.tensor([0, 10], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        nnop._flash_attention_varlen(q, q, q, cu.to(torch.int64), cu, 10, 10, causal=True)
    with pytest.raises(ValueError, match="divisible"):
        nnop._flash_attention_varlen(torch.zeros((3, 10, 64), dtype=torch.bfloat16, device=dev), q, q, cu, cu,
                                     10, 10, causal=True)


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_four_wave_groups(dev, causal):
    """Packed sequences on a grid large enough for the four-wave forward and dQ groups at
    E = 128 (at least 256 workgroups of 128 queries): bf16, 16:4 heads, lengths
    [700, 1025, 300, 513].  Sequences and heads are independent, so sequences 1 and 3 of
    kv head 1 (q heads 4..7) are exact sub-problems for the oracle."""
    rng = np.random.default_rng(31)
    E, QH, KH = 128, 16, 4
    lens = [700, 1025, 300, 513]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q, qn = make(rng, (QH, T, E), torch.bfloat16, dev)
    k, kn = make(rng, (KH, T, E), torch.bfloat16, dev)
    v, vn = make(rng, (KH, T, E), torch.bfloat16, dev)
    do, don = make(rng, (QH, T, E), torch.bfloat16, dev)
    cut = torch.from_numpy(cu).to(dev)
    mx = max(lens)
    print(f"varlen four-wave groups: bf16 E=128 16:4 lens={lens} causal={causal}", flush=True)
    o, ms, ls = nnop._flash_attention_varlen(q, k, v, cut, cut, mx, mx, causal=causal)
    dq, dk, dv = nnop.grad_flash_attention_varlen(do, o, ms, ls, q, k, v, cut, cut, mx, mx, causal=causal,
                                                  qk_fp16=False)
    torch.cuda.synchronize()
    scale = nnop.attention_scale(E, torch.bfloat16)
    o, dq, dk, dv = (host(t) for t in (o, dq, dk, dv))
    errs = {}
    for s in (1, 3):
        a, b = cu[s], cu[s + 1]
        sq = lambda x: x[4:8, a:b][None]
        sk = lambda x: x[1:2, a:b][None]
        o_r, _, _ = oracle.attn_fwd(sq(qn), sk(kn), sk(vn), None, None, causal, scale)
        dq_r, dk_r, dv_r, _ = oracle.attn_bwd(sq(don), sq(qn), sk(kn), sk(vn), None, None, causal, scale)
        errs.update({f"o{s}": rel_err(o[4:8, a:b], o_r[0]), f"dq{s}": rel_err(dq[4:8, a:b], dq_r[0]),
                     f"dk{s}": rel_err(dk[1:2, a:b], dk_r[0]), f"dv{s}": rel_err(dv[1:2, a:b], dv_r[0])})
    assert all(e <= TOL[torch.bfloat16] for e in errs.values()), errs
