"""onionop_flash_attn_bwd_noalloc: the attention backward without a workspace argument,
whose workspace is the library's own 16 MiB device array, against onionop_flash_attn_bwd
with a caller-allocated workspace of the same 16 MiB.  Both then run the same kernels on
the same inputs (a workspace decides which range splits the backward may use), so the
gradients must be identical bit for bit; against the full workspace the query reports
they agree to the element type's tolerance (splits change only the summation order).
Two calls in a row, the second on a smaller problem (the array keeps the first call's
contents), then a request beyond the array's size, which must be refused before anything
is enqueued.
"""
import numpy as np
import pytest
import torch

import nnop
from helpers import TOL, host, make, rel_err

pytestmark = pytest.mark.gpu


def backward_both_ways(dev, dt, B, QH, KH, L, E, causal, with_pair, seed):
    rng = np.random.default_rng(seed)
    q, _ = make(rng, (B, QH, L, E), dt, dev)
    k, _ = make(rng, (B, KH, L, E), dt, dev)
    v, _ = make(rng, (B, KH, L, E), dt, dev)
    do, _ = make(rng, (B, QH, L, E), dt, dev)
    pair = make(rng, (B, L, L, QH), dt, dev)[0] if with_pair else None
    print(f"no-alloc backward: {dt} B={B} QH={QH} KH={KH} L={L} E={E} causal={causal} pair={with_pair}", flush=True)
    o, ms, ls = nnop._flash_attention(q, k, v, pair, causal=causal)
    full = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, pair, causal=causal)  # full workspace
    L_ = nnop.lib()
    from nnop._util import dtype_code, ptr, stream_of

    dtc, sc = dtype_code(q, "test"), nnop.attention_scale(E, dt)
    ws = torch.empty(16 << 20, dtype=torch.uint8, device=dev)  # the library array's size
    ref = [torch.full_like(q, 5.0), torch.full_like(k, 5.0), torch.full_like(v, 5.0)]
    ref.append(torch.full_like(pair, 5.0) if with_pair else None)
    nnop._lib.check(L_.onionop_flash_attn_bwd(
        stream_of(q), dtc, E, L, L, QH, KH, B, ptr(do), ptr(o), ptr(ms), ptr(ls), ptr(q), ptr(k), ptr(v), ptr(pair),
        None, int(causal), sc, 1, ptr(ref[0]), ptr(ref[1]), ptr(ref[2]), ptr(ref[3]), ptr(ws), ws.numel()))
    dq, dk, dv = torch.full_like(q, 3.0), torch.full_like(k, 3.0), torch.full_like(v, 3.0)
    dpair = torch.full_like(pair, 3.0) if with_pair else None
    st = L_.onionop_flash_attn_bwd_noalloc(
        stream_of(q), dtc, E, L, L, QH, KH, B, ptr(do), ptr(o), ptr(ms), ptr(ls), ptr(q), ptr(k),
        ptr(v), ptr(pair), None, int(causal), sc, 1, ptr(dq), ptr(dk), ptr(dv), ptr(dpair))
    nnop._lib.check(st)
    torch.cuda.synchronize()
    for name, a, b, c in (("dq", dq, ref[0], full[0]), ("dk", dk, ref[1], full[1]), ("dv", dv, ref[2], full[2])):
        assert torch.equal(a, b), name
        assert rel_err(host(a), host(c)) <= TOL[dt], name
    if with_pair:
        assert torch.equal(dpair, ref[3]), "dpair"
        assert rel_err(host(dpair), host(full[3])) <= TOL[dt], "dpair"


def test_noalloc_backward_matches_workspace_backward(dev):
    backward_both_ways(dev, torch.bfloat16, 2, 8, 2, 1000, 64, True, False, seed=1)
    backward_both_ways(dev, torch.float16, 1, 4, 4, 300, 32, False, True, seed=2)


def test_noalloc_backward_head_dim_256(dev):
    """E = 256 on a small causal grid: the dQ key-range and dK/dV query-range partials
    (about 9 MB) fit the array, so both entry points take the same splits."""
    backward_both_ways(dev, torch.bfloat16, 1, 2, 2, 300, 256, True, False, seed=3)


def test_noalloc_backward_refuses_oversized_requests(dev):
    L_ = nnop.lib()
    # 4 x 64 x 8192 query rows need 16 MiB + 256 bytes: more than the array holds
    st = L_.onionop_flash_attn_bwd_noalloc(None, 2, 64, 8192, 8192, 64, 64, 4, 16, 16, 16, 16, 16, 16, 16, None,
                                           None, 1, 0.125, 1, 16, 16, 16, None)
    assert st == -3 and b"scratch" in L_.onionop_last_error()
