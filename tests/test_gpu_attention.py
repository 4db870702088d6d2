"""GPU parity of flash attention (fwd + bwd) against the oracle.

Cases follow the reference sweeps (test/attention_tests.jl:6-18,
test/causal_attention_tests.jl:6-16, test/gqa_attention_tests.jl:6-18): ragged and
aligned lengths (255/256/257/511/512/1024), E in {16, 32, 64, 128}, pair bias, key
padding with the last 11 keys of the last batch masked, GQA, causal.  Inputs are seeded
N(0, 1) rounded to the dtype; the oracle runs in float64 on the same rounded values.
Tolerance: norm-wise relative error <= 1e-5 (float32), <= 2e-2 (float16, bfloat16).
"""
import zlib

import numpy as np
import pytest
import torch

import nnop
import oracle
from helpers import DTYPES, TOL, host, make, rel_err

pytestmark = pytest.mark.gpu


def run_case(dev, dt, E, QL, KL, QH, KH, B, causal, use_pair, use_kpad, seed, qk16=False, kpad=None):
    dtype = DTYPES[dt]
    rng = np.random.default_rng(seed)
    q, qn = make(rng, (B, QH, QL, E), dtype, dev)
    k, kn = make(rng, (B, KH, KL, E), dtype, dev)
    v, vn = make(rng, (B, KH, KL, E), dtype, dev)
    do, don = make(rng, (B, QH, QL, E), dtype, dev)
    pair = pairn = None
    if use_pair:
        pair, pairn = make(rng, (B, KL, QL, QH), dtype, dev)
    kp = None
    if use_kpad and kpad is None:
        kpad = np.ones((B, KL), dtype=bool)
        kpad[-1, -11:] = False
    if kpad is not None:
        kp = torch.from_numpy(kpad).to(dev)
    print(f"case {dt} E={E} QL={QL} KL={KL} QH={QH} KH={KH} B={B} causal={causal} pair={use_pair} "
          f"kpad={kpad is not None} seed={seed} qk16={qk16}", flush=True)
    o, ms, ls = nnop._flash_attention(q, k, v, pair, causal=causal, kpad_mask=kp)
    dq, dk, dv, dpair = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, pair, causal=causal, kpad_mask=kp,
                                                  qk_fp16=qk16)
    torch.cuda.synchronize()
    scale = nnop.attention_scale(E, dtype)
    o_r, ms_r, ls_r = oracle.attn_fwd(qn, kn, vn, pairn, kpad, causal, scale)
    dq_r, dk_r, dv_r, dp_r = oracle.attn_bwd(don, qn, kn, vn, pairn, kpad, causal, scale,
                                            qk_fp16=qk16 and dtype == torch.float32)
    tol = TOL[dtype]

    def grad_err(a, r):
        # When every row's softmax sees at most one key, dS = P (dP - delta) is exactly zero
        # and so are dq, dk and dpair; the kernel's values are then the float round-off of
        # dP - delta, bounded against dv, a gradient of the same magnitude that does not
        # cancel.
        nv = np.linalg.norm(dv_r)
        if np.linalg.norm(r) == 0.0 and nv > 0.0:
            return float(np.linalg.norm(np.asarray(a, dtype=np.float64)) / nv)
        return rel_err(a, r)

    errs = {"o": rel_err(host(o), o_r), "dq": grad_err(host(dq), dq_r), "dk": grad_err(host(dk), dk_r),
            "dv": rel_err(host(dv), dv_r)}
    if use_pair:
        errs["dpair"] = grad_err(host(dpair), dp_r)
    fin = np.isfinite(ms_r)
    errs["ms"] = rel_err(host(ms)[fin], ms_r[fin]) if fin.any() else 0.0
    errs["ls"] = rel_err(host(ls), ls_r)
    assert np.all(host(ms)[~fin] == -np.inf) and np.all(host(ls)[~fin] == 0)
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"tolerance {tol}: {bad} (all: {errs})"
    return errs


CASES = [
    # dt, E, QL, KL, QH, KH, B, causal, pair, kpad
    ("f32", 16, 255, 255, 2, 2, 3, False, False, False),
    ("f32", 32, 256, 511, 2, 2, 3, False, True, True),
    ("f32", 64, 512, 256, 2, 2, 3, False, True, False),
    ("f32", 64, 1024, 1024, 2, 2, 1, False, False, True),
    ("f32", 128, 257, 257, 4, 2, 2, True, False, False),
    ("f32", 64, 511, 511, 2, 2, 3, True, True, True),
    # float32 on a small grid: two-wave dK/dV and one-wave dQ, four groups each, with
    # causal GQA, key padding and QL != KL
    ("f32", 64, 300, 200, 3, 1, 2, True, False, True),
    ("f16", 16, 256, 256, 2, 2, 3, False, True, True),
    ("f16", 32, 511, 255, 2, 2, 3, False, False, True),
    ("f16", 64, 512, 512, 2, 2, 3, True, True, False),
    ("f16", 64, 1024, 1024, 2, 2, 2, True, False, True),
    ("f16", 128, 255, 512, 2, 2, 2, False, False, False),
    ("bf16", 16, 255, 511, 2, 2, 3, False, True, False),
    ("bf16", 32, 768, 768, 8, 8, 2, False, True, False),
    # MQA at E >= 128 on small grids: the two-wave dK/dV's iterations split over workgroups
    ("bf16", 128, 300, 300, 8, 1, 2, True, False, True),
    ("f16", 128, 200, 333, 8, 1, 1, False, False, False),
    ("bf16", 256, 130, 130, 8, 1, 1, True, False, False),
    ("bf16", 64, 1024, 1024, 4, 4, 2, True, False, False),
    ("bf16", 64, 256, 256, 2, 2, 3, True, True, True),
    ("bf16", 128, 512, 512, 4, 1, 2, True, False, False),
    ("bf16", 128, 257, 257, 8, 2, 2, False, False, True),
    # 16-bit E = 128 dK / dV on two waves per key slice: causal with QL != KL and key
    # padding; a single partial key tile with more queries than keys
    ("bf16", 128, 200, 333, 4, 2, 2, True, False, True),
    ("f16", 128, 96, 64, 2, 1, 3, True, False, False),
    # 16-bit bias, QH % 4 == 0 and >= 192 four-head forward workgroups (q tiles x QH/4 x B):
    # four heads per forward workgroup, bias records staged through LDS
    ("bf16", 64, 64, 257, 32, 8, 24, True, True, True),
    ("f16", 16, 100, 300, 16, 16, 24, False, True, False),
    ("bf16", 32, 130, 129, 12, 4, 22, False, True, True),
    # ... and QH == KH: four kv heads per dK/dV workgroup as well
    ("bf16", 32, 200, 257, 8, 8, 24, True, True, True),
    ("f16", 64, 128, 130, 4, 4, 64, True, True, False),
    # the same kind of bias with fewer workgroups: one head per workgroup
    ("bf16", 64, 511, 257, 4, 2, 2, True, True, True),
    ("bf16", 32, 200, 200, 12, 4, 1, False, True, False),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_attention_parity(dev, case):
    dt, E, QL, KL, QH, KH, B, causal, pair, kpad = case
    run_case(dev, dt, E, QL, KL, QH, KH, B, causal, pair, kpad, seed=zlib.crc32(repr(case).encode()) % 1000)


GQA = [(QH, KH, causal, E, L) for QH, KH in ((4, 1), (6, 2), (8, 2)) for causal in (False, True)
       for E, L in ((32, 255), (64, 257))]


@pytest.mark.parametrize("case", GQA, ids=lambda c: "-".join(map(str, c)))
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_gqa_parity(dev, dt, case):
    QH, KH, causal, E, L = case
    run_case(dev, dt, E, L, L, QH, KH, 2, causal, False, False, seed=7)


@pytest.mark.parametrize("causal", [False, True])
def test_fp32_qk_fp16_mode(dev, causal):
    """The reference backward's Float16 Q/K (src/attention_bwd.jl:20-21), reproduced."""
    run_case(dev, "f32", 64, 300, 300, 2, 2, 2, causal, True, False, seed=3, qk16=True)


@pytest.mark.parametrize("causal", [False, True])
def test_fp32_qk_fp16_mode_no_bias(dev, causal):
    """The same without a bias: the two-wave dK/dV and one-wave dQ kernels round Q/K too."""
    run_case(dev, "f32", 64, 300, 300, 2, 2, 2, causal, False, False, seed=5, qk16=True)


# E = 256 (the largest head dim the reference's group-size search admits on a 64 KiB-LDS
# device, src/attention.jl:213-225): one wave per SIMD; float32 and the bias paths use
# scratch for part of their registers.  The 16-bit causal cases without a bias run the
# backward's key- and query-range splits (small grids), with ranges of odd tile counts.
@pytest.mark.parametrize("case", [
    ("bf16", 256, 130, 130, 2, 2, 1, True, False, False),
    ("f16", 256, 200, 200, 2, 2, 1, True, False, True),
    ("bf16", 256, 300, 300, 4, 2, 1, True, False, False),
    ("bf16", 256, 257, 200, 4, 2, 2, False, False, True),
    ("f16", 256, 100, 100, 2, 1, 1, True, True, False),
    ("f32", 256, 70, 70, 2, 2, 1, False, True, True),
    ("f32", 256, 96, 96, 2, 2, 1, True, False, False),
], ids=lambda c: "-".join(map(str, c)))
def test_head_dim_256(dev, case):
    dt, E, QL, KL, QH, KH, B, causal, pair, kpad = case
    run_case(dev, dt, E, QL, KL, QH, KH, B, causal, pair, kpad, seed=zlib.crc32(repr(case).encode()) % 1000)


def test_fully_masked_rows(dev):
    """A batch whose keys are all padded: o = 0, ms = -Inf, ls = 0 and finite gradients
    (the reference gives NaN there)."""
    kpad = np.ones((2, 130), dtype=bool)
    kpad[1, :] = False
    for dt in ("f32", "bf16"):
        run_case(dev, dt, 32, 70, 130, 2, 2, 2, False, True, True, seed=5, kpad=kpad)


@pytest.mark.parametrize("dt,E", [("f32", 64), ("bf16", 128), ("bf16", 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_padded_key_blocks(dev, dt, E, causal):
    """Whole 32- and 64-key blocks of padding (workgroups whose every key is padded write
    zero dK / dV without computing), next to partly padded blocks."""
    kpad = np.ones((2, 200), dtype=bool)
    kpad[0, 64:160] = False
    kpad[1, 150:] = False
    run_case(dev, dt, E, 180, 200, 4, 2, 2, causal, False, True, seed=11, kpad=kpad)


@pytest.mark.parametrize("dt,E,causal", [("bf16", 64, True), ("f16", 64, False), ("bf16", 64, False),
                                         ("bf16", 128, True), ("f16", 128, False)])
def test_four_wave_groups(dev, dt, E, causal):
    """16-bit attention without a bias on grids of at least 256 workgroups of 128 keys (or
    queries) takes the four-wave groups: dK/dV at E = 64, the forward and dQ at E = 128, the
    forward at E = 64 without the causal mask.  (E, 1024, 16:KH, 4), GQA, with key padding
    that leaves one whole 128-key block of batch 1 padded (its workgroups write zero dK / dV
    without computing) and the last keys of batch 2 padded.  Heads are independent, so one
    batch's kv group is an exact sub-problem for the oracle: batches 1 and 2, the kv head of
    q head 10 with every q head of its group."""
    dtype = DTYPES[dt]
    B, QH, L = 4, 16, 1024
    KH = 8 if E == 64 else 4
    rng = np.random.default_rng(21)
    q, qn = make(rng, (B, QH, L, E), dtype, dev)
    k, kn = make(rng, (B, KH, L, E), dtype, dev)
    v, vn = make(rng, (B, KH, L, E), dtype, dev)
    do, don = make(rng, (B, QH, L, E), dtype, dev)
    kpad = np.ones((B, L), dtype=bool)
    kpad[1, 256:384] = False
    kpad[2, -77:] = False
    kp = torch.from_numpy(kpad).to(dev)
    print(f"four-wave groups: {dt} ({E},1024,16:{KH},4) causal={causal} key padding", flush=True)
    o, ms, ls = nnop._flash_attention(q, k, v, causal=causal, kpad_mask=kp)
    dq, dk, dv, _ = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, causal=causal, kpad_mask=kp)
    torch.cuda.synchronize()
    scale = nnop.attention_scale(E, dtype)
    errs = {}
    for b in (1, 2):
        rep = QH // KH
        kvh = 10 // rep  # the kv head of q head 10, and all q heads of its group
        sq, sk = (slice(b, b + 1), slice(kvh * rep, (kvh + 1) * rep)), (slice(b, b + 1), slice(kvh, kvh + 1))
        o_r, _, _ = oracle.attn_fwd(qn[sq], kn[sk], vn[sk], None, kpad[b:b + 1], causal, scale)
        dq_r, dk_r, dv_r, _ = oracle.attn_bwd(don[sq], qn[sq], kn[sk], vn[sk], None, kpad[b:b + 1], causal, scale)
        errs.update({f"o{b}": rel_err(host(o[sq]), o_r), f"dq{b}": rel_err(host(dq[sq]), dq_r),
                     f"dk{b}": rel_err(host(dk[sk]), dk_r), f"dv{b}": rel_err(host(dv[sk]), dv_r)})
    assert all(e <= TOL[dtype] for e in errs.values()), errs
    # padded keys get exactly zero gradients, whole padded blocks included
    assert torch.count_nonzero(dk[1, :, 256:384]) == 0 and torch.count_nonzero(dv[1, :, 256:384]) == 0
    assert torch.count_nonzero(dk[2, :, -77:]) == 0 and torch.count_nonzero(dv[2, :, -77:]) == 0


def test_single_key(dev):
    """L = 1: o = v exactly, whatever q."""
    rng = np.random.default_rng(1)
    q, _ = make(rng, (2, 2, 1, 64), torch.float32, dev)
    k, _ = make(rng, (2, 2, 1, 64), torch.float32, dev)
    v, _ = make(rng, (2, 2, 1, 64), torch.float32, dev)
    o, ms, ls = nnop._flash_attention(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.allclose(o, v, rtol=1e-6, atol=1e-6)
    assert torch.all(ls == 1.0)


def test_autograd_matches_launchers(dev):
    rng = np.random.default_rng(11)
    q, _ = make(rng, (1, 4, 200, 64), torch.bfloat16, dev)
    k, _ = make(rng, (1, 2, 200, 64), torch.bfloat16, dev)
    v, _ = make(rng, (1, 2, 200, 64), torch.bfloat16, dev)
    qq, kk, vv = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o = nnop.flash_attention(qq, kk, vv, causal=True)
    o.sum().backward()
    o2, ms, ls = nnop._flash_attention(q, k, v, causal=True)
    dq, dk, dv, _ = nnop.grad_flash_attention(torch.ones_like(o2), o2, ms, ls, q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    assert torch.equal(qq.grad, dq) and torch.equal(kk.grad, dk) and torch.equal(vv.grad, dv)


def test_errors_match_reference_messages(dev):
    q = torch.zeros((1, 3, 8, 64), device=dev)
    k = torch.zeros((1, 2, 8, 64), device=dev)
    with pytest.raises(ValueError, match="Number of query heads `3` must be divisible by number of KV heads `2`."):
        nnop.flash_attention(q, k, k, causal=False)
    with pytest.raises(ValueError, match="Only power-of-2 embedding dims are supported."):
        x = torch.zeros((1, 2, 8, 48), device=dev)
        nnop.flash_attention(x, x, x, causal=False)
    with pytest.raises(ValueError, match="must be the same as of K"):
        nnop.flash_attention(torch.zeros((1, 2, 8, 32), device=dev), k, k, causal=False)
    with pytest.raises(nnop.NNopError, match="embedding dim 512 not supported"):
        x = torch.zeros((1, 2, 8, 512), device=dev)
        nnop.flash_attention(x, x, x, causal=False)


@pytest.mark.parametrize("dt,E,L,QH,KH,causal,use_pair,use_kpad", [
    ("bf16", 64, 300, 4, 2, True, False, False),
    ("f16", 128, 257, 2, 2, True, False, True),
    ("f32", 32, 200, 4, 4, False, True, True),
    ("bf16", 256, 300, 4, 2, True, False, False),  # dQ key- and dK/dV query-range splits
    ("bf16", 32, 256, 8, 8, False, True, False),   # the four-head bias kernels' splits
])
def test_staged_backward_matches_combined(dev, dt, E, L, QH, KH, causal, use_pair, use_kpad):
    """The staged entry points (preprocess, dK/dV, dQ) and the combined backward (dQ with
    the preprocess fused, then dK/dV) compute the same gradients."""
    from nnop import _lib
    from nnop._util import ptr

    dtype = DTYPES[dt]
    rng = np.random.default_rng(7)
    B = 2
    q, _ = make(rng, (B, QH, L, E), dtype, dev)
    k, _ = make(rng, (B, KH, L, E), dtype, dev)
    v, _ = make(rng, (B, KH, L, E), dtype, dev)
    do, _ = make(rng, (B, QH, L, E), dtype, dev)
    pair = make(rng, (B, L, L, QH), dtype, dev)[0] if use_pair else None
    kp = None
    if use_kpad:
        kpad = np.ones((B, L), dtype=bool)
        kpad[-1, -11:] = False
        kp = torch.from_numpy(kpad).to(dev)
    o, ms, ls = nnop._flash_attention(q, k, v, pair, causal=causal, kpad_mask=kp)
    dq, dk, dv, dpair = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, pair, causal=causal, kpad_mask=kp)
    L_ = _lib.lib()
    dtc = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dtype]
    dims = (E, L, L, QH, KH, B)
    wsb = int(L_.onionop_flash_attn_bwd_workspace(dtc, *dims))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    sc = nnop.attention_scale(E, dtype)
    dq2, dk2, dv2 = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dpair2 = None if pair is None else torch.empty_like(pair)
    _lib.check(L_.onionop_flash_attn_bwd_preprocess(s, dtc, E, L, QH, B, ptr(do), ptr(o), ptr(ms), ptr(ls),
                                                    ptr(ws), wsb))
    _lib.check(L_.onionop_flash_attn_bwd_dkdv(s, dtc, *dims, ptr(do), ptr(q), ptr(k), ptr(v), ptr(pair), ptr(kp),
                                              int(causal), sc, 1, ptr(dk2), ptr(dv2), ptr(ws), wsb))
    _lib.check(L_.onionop_flash_attn_bwd_dq(s, dtc, *dims, ptr(do), ptr(q), ptr(k), ptr(v), ptr(pair), ptr(kp),
                                            int(causal), sc, 1, ptr(dq2), ptr(dpair2), ptr(ws), wsb))
    torch.cuda.synchronize()
    # delta is summed in a different order by the two paths: agreement to a few ulps
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    pairs = {"dq": (dq, dq2), "dk": (dk, dk2), "dv": (dv, dv2)}
    if use_pair:
        pairs["dpair"] = (dpair, dpair2)
    errs = {n: rel_err(host(a), host(b)) for n, (a, b) in pairs.items()}
    assert all(e <= tol for e in errs.values()), errs


@pytest.mark.parametrize("dt,E,L,QH,KH,B,causal,use_kpad", [
    ("bf16", 32, 768, 8, 8, 2, False, False),   # config 4's shape: 5 key and 5 query ranges
    ("f16", 64, 300, 4, 2, 1, True, True),      # GQA (dQ split only), causal, key padding
    ("f16", 64, 300, 4, 4, 1, True, True),      # both splits, causal, key padding, ragged
    ("bf16", 16, 130, 8, 4, 1, False, False),   # E = 16, short keys: 2 key ranges
])
def test_pair_range_splits(dev, dt, E, L, QH, KH, B, causal, use_kpad):
    """On small grids, a 16-bit pair-biased backward splits the dQ's key range (and, with
    QH = KH, the dK / dV's query range) over several four-head workgroups and sums their
    float32 partials in range order, when the workspace has the full size
    onionop_flash_attn_bwd_workspace reports; with only the lse / delta part it runs
    unsplit.  Both agree with the oracle; dq, dk and dv differ only in summation order,
    and dpair = dS only in its rounding: the two dQ kernels (four heads per workgroup or
    one) may round an element of float16 dS once from an exact fused multiply-add or via
    float32 (one unit in the last place)."""
    from nnop import _lib
    from nnop._util import ptr

    dtype = DTYPES[dt]
    rng = np.random.default_rng(11)
    q, qn = make(rng, (B, QH, L, E), dtype, dev)
    k, kn = make(rng, (B, KH, L, E), dtype, dev)
    v, vn = make(rng, (B, KH, L, E), dtype, dev)
    do, don = make(rng, (B, QH, L, E), dtype, dev)
    pair, pairn = make(rng, (B, L, L, QH), dtype, dev)
    kpad = kp = None
    if use_kpad:
        kpad = np.ones((B, L), dtype=bool)
        kpad[-1, -11:] = False
        kp = torch.from_numpy(kpad).to(dev)
    print(f"dq key split: {dt} E={E} L={L} QH={QH} KH={KH} B={B} causal={causal} kpad={use_kpad}", flush=True)
    o, ms, ls = nnop._flash_attention(q, k, v, pair, causal=causal, kpad_mask=kp)
    L_ = _lib.lib()
    dtc = {torch.float16: 1, torch.bfloat16: 2}[dtype]
    dims = (E, L, L, QH, KH, B)
    full = int(L_.onionop_flash_attn_bwd_workspace(dtc, *dims))
    base = 2 * B * QH * L * 4 + 256  # the lse2 / delta rows alone
    assert full > base, (full, base)
    s = torch.cuda.current_stream().cuda_stream
    sc = nnop.attention_scale(E, dtype)
    outs = {}
    for name, wsb in (("split", full), ("unsplit", base)):
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        g = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(pair)]
        _lib.check(L_.onionop_flash_attn_bwd(s, dtc, *dims, ptr(do), ptr(o), ptr(ms), ptr(ls), ptr(q), ptr(k),
                                             ptr(v), ptr(pair), ptr(kp), int(causal), sc, 1, ptr(g[0]), ptr(g[1]),
                                             ptr(g[2]), ptr(g[3]), ptr(ws), wsb))
        outs[name] = g
    torch.cuda.synchronize()
    a, b = outs["split"], outs["unsplit"]
    for j in (1, 2):  # dk, dv
        assert rel_err(host(a[j]), host(b[j])) <= 1e-2
    ia, ib = a[3].view(torch.int16).int(), b[3].view(torch.int16).int()
    ia = torch.where(ia < 0, -(ia & 0x7FFF), ia)  # sign-magnitude to a monotone integer
    ib = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    assert int((ia - ib).abs().max()) <= 1, "dpair beyond one unit in the last place"
    assert rel_err(host(a[0]), host(b[0])) <= 1e-2
    dq_r, dk_r, dv_r, dp_r = oracle.attn_bwd(don, qn, kn, vn, pairn, kpad, causal, sc)
    for name, g in outs.items():
        errs = {"dq": rel_err(host(g[0]), dq_r), "dk": rel_err(host(g[1]), dk_r), "dv": rel_err(host(g[2]), dv_r),
                "dpair": rel_err(host(g[3]), dp_r)}
        assert all(e <= TOL[dtype] for e in errs.values()), (name, errs)


def test_shared_memory_query(dev):
    """NNop.shared_memory (src/NNop.jl:27-30, ext/NNopAMDGPUExt.jl:6-9): the LDS bytes per
    workgroup of the device, as hipDeviceProp_t.sharedMemPerBlock reports it (torch reads
    the same property), cached per device."""
    expect = torch.cuda.get_device_properties(0).shared_memory_per_block
    got = nnop.shared_memory(0)
    assert got == expect
    assert nnop.shared_memory(0) == got  # memoised value
    # every attention kernel's static LDS fits in it (the largest uses 133120 bytes)
    assert got >= 133120
