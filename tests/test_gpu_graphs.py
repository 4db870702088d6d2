"""The library under HIP graph capture (torch.cuda.CUDAGraph is a hipGraph on ROCm).

An attention fwd+bwd step, the allocation-free attention backward, softmax, both norms and
RoPE are recorded into graphs and replayed.  The library enqueues nothing but kernel
launches (no memsets, allocations or synchronisations; zero fills are kernels), so every
replay must reproduce the eager results bit for bit.  Between replays the inputs are
refilled by eager work and the process synchronises; every replay is checked.
"""
import pytest
import torch

import nnop
from nnop._util import dtype_code, ptr, stream_of

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _graph(fn):
    """Warm fn up eagerly on a side stream (lazy one-time set-up happens outside the capture),
    then capture it; returns (graph, static outputs)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    torch.cuda.synchronize()
    return g, outs


def _replay_and_check(g, outs, fn, refill, what):
    for rep in range(REPLAYS):
        refill(rep)              # eager work between replays: new input values
        eager = fn()             # the same ops, eagerly, into fresh buffers
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), f"{what}: replay {rep}, output {i} differs from the eager result"


def _fill(t, gen):
    t.copy_(torch.randn(t.shape, generator=gen, device=t.device, dtype=torch.float32).to(t.dtype))


@pytest.mark.parametrize("dt,causal,with_kpad", [(torch.bfloat16, True, True), (torch.float32, False, False)])
def test_attention_step_in_a_graph(dev, dt, causal, with_kpad):
    B, QH, KH, L, E = 2, 4, 2, 384, 64
    gen = torch.Generator(device=dev).manual_seed(3)
    q, do = (torch.empty((B, QH, L, E), dtype=dt, device=dev) for _ in range(2))
    k, v = (torch.empty((B, KH, L, E), dtype=dt, device=dev) for _ in range(2))
    for t in (q, k, v, do):
        _fill(t, gen)
    kp = None
    if with_kpad:
        kp = torch.ones((B, L), dtype=torch.bool, device=dev)
        kp[-1, -37:] = False
    print(f"graph: attention step {dt} causal={causal} kpad={with_kpad}", flush=True)

    def step():
        o, ms, ls = nnop._flash_attention(q, k, v, causal=causal, kpad_mask=kp)
        dq, dk, dv, _ = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, causal=causal, kpad_mask=kp)
        return o, ms, ls, dq, dk, dv

    g, outs = _graph(step)
    _replay_and_check(g, outs, step, lambda rep: [_fill(t, gen) for t in (q, k, v, do)], "attention step")


def test_noalloc_backward_in_a_graph(dev):
    """The allocation-free backward is meant for captured code: its workspace is the
    library's own device array, so the graph holds no workspace allocation at all."""
    B, QH, KH, L, E = 2, 8, 2, 500, 64
    dt = torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(4)
    q, do = (torch.empty((B, QH, L, E), dtype=dt, device=dev) for _ in range(2))
    k, v = (torch.empty((B, KH, L, E), dtype=dt, device=dev) for _ in range(2))
    for t in (q, k, v, do):
        _fill(t, gen)
    o, ms, ls = nnop._flash_attention(q, k, v, causal=True)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    L_ = nnop.lib()
    print("graph: no-alloc backward", flush=True)

    def bwd():
        nnop._lib.check(L_.onionop_flash_attn_bwd_noalloc(
            stream_of(q), dtype_code(q, "test"), E, L, L, QH, KH, B, ptr(do), ptr(o), ptr(ms), ptr(ls), ptr(q),
            ptr(k), ptr(v), None, None, 1, nnop.attention_scale(E, dt), 1, ptr(dq), ptr(dk), ptr(dv), None))
        return dq, dk, dv

    dq2, dk2, dv2 = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)

    def eager():  # the same entry point (the same library array), outside the graph
        nnop._lib.check(L_.onionop_flash_attn_bwd_noalloc(
            stream_of(q), dtype_code(q, "test"), E, L, L, QH, KH, B, ptr(do), ptr(o), ptr(ms), ptr(ls), ptr(q),
            ptr(k), ptr(v), None, None, 1, nnop.attention_scale(E, dt), 1, ptr(dq2), ptr(dk2), ptr(dv2), None))
        return dq2, dk2, dv2

    g, outs = _graph(bwd)

    def refill(rep):
        _fill(do, gen)

    for rep in range(REPLAYS):
        refill(rep)
        ref = eager()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, ref)):
            assert torch.equal(a, b), f"no-alloc backward: replay {rep}, output {i}"


def test_rowwise_ops_in_a_graph(dev):
    """Softmax (fwd, bwd), RMS and layer norm (fwd, bwd with the column-sum launch) and RoPE
    (fwd) in one graph."""
    gen = torch.Generator(device=dev).manual_seed(5)
    x = torch.empty((300, 1024), dtype=torch.float32, device=dev)
    dy = torch.empty_like(x)
    xn = torch.empty((64, 4096), dtype=torch.bfloat16, device=dev)
    gn = torch.empty_like(xn)
    w = torch.empty((4096,), dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(w)
    q = torch.empty((2, 4, 200, 128), dtype=torch.bfloat16, device=dev)
    k = torch.empty((2, 2, 200, 128), dtype=torch.bfloat16, device=dev)
    cos, sin = nnop.LlamaRotaryEmbedding(128)(torch.arange(200, dtype=torch.float32, device=dev)[None].expand(2, 200))
    ins = (x, dy, xn, gn, w, b, q, k)
    for t in ins:
        _fill(t, gen)
    print("graph: softmax, norms, rope", flush=True)

    def ops():
        y = nnop.online_softmax(x)
        dx = nnop.grad_online_softmax(dy, y)
        yr, rstd = nnop._rms_norm(xn, w)
        dxr, dwr = nnop.grad_rms_norm(gn, rstd, xn, w)
        yl, mu, rs = nnop._layer_norm(xn, w, b)
        dxl, dwl, dbl = nnop.grad_layer_norm(gn, mu, rs, xn, w)
        qr, kr = nnop._llama_rope(q, k, cos, sin, bwd=False)
        return y, dx, yr, rstd, dxr, dwr, yl, mu, rs, dxl, dwl, dbl, qr, kr

    g, outs = _graph(ops)
    _replay_and_check(g, outs, ops, lambda rep: [_fill(t, gen) for t in ins], "row-wise ops")
