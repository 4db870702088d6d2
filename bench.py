#!/usr/bin/env python3
"""Benchmark of NNop's fused-kernel hot path on one MI355X.

Headline workload (the `value`): flash attention forward + backward, bfloat16,
(E, L, H, B) = (64, 4096, 4, 4), causal, q/k/v ~ N(0,1)/sqrt(E), dO = 1 (loss = sum(o)).
One step = _flash_attention + ∇flash_attention through the C ABI (3 kernels: forward, dQ with
the backward preprocess fused, dK/dV), inputs resident in HBM.  FLOPs per step use the flash-attention convention
14 B H L^2 E / 2 (forward 4, backward 10, causal halves).

Also reported (`memory_bound`): HBM GB/s of online softmax (f32, 8192 x 1024), RMS norm
and layer norm fwd/bwd (bf16, emb 4096 x 16384), Llama RoPE fwd (bf16, q (128,8192,32,4),
k (128,8192,8,4)), each over a rotating set of buffers larger than the 256 MB
Infinity Cache, with algorithmic bytes (one read / write of each API tensor).

Also reported (`workloads`): the other attention workloads at full size, timed through the
C ABI (float32 (64,1024,4,2); bf16 pair bias (32,768,8,2); llama_rope + causal GQA
(128,8192,32:8,4) with per-sequence lengths, as a key mask and packed).

Before the counted warmup a settle phase runs the step until the GPU's clocks are steady
(the clocks need ~30 ms of this load to ramp); its length is reported as settle_ms.

`roofline` is the slowest kernel of the step, timed alone with HIP events on the stream
the library launches on.  `cpu_baseline` is the oracle's float32 restatement of the
reference algorithm (oracle/oracle.c, FAITHFUL mode) on the host cores this job may use.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "onionop.jl_amd"))
sys.path.insert(0, ROOT)

MI355X_BF16_DENSE_TFLOPS = 2500.0   # dense bf16/fp16 MFMA peak
MI355X_HBM_GBS = 8000.0             # HBM3E peak
MI355X_FP32_MFMA_TFLOPS = 157.3     # dense fp32 MFMA peak

METRIC = "flash-attn fwd+bwd TFLOP/s (bf16, L=4096) + norm/softmax HBM GB/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def attention_setup(torch, nnop, dev, E=64, L=4096, H=4, B=4, seed=2):
    g = torch.Generator(device="cpu").manual_seed(seed)
    s = 1.0 / math.sqrt(E)
    q, k, v = [(torch.randn((B, H, L, E), generator=g) * s).to(torch.bfloat16).to(dev) for _ in range(3)]
    do = torch.ones((B, H, L, E), dtype=torch.bfloat16, device=dev)
    return q, k, v, do


class AttnStep:
    """One fwd+bwd step through the C ABI, with buffers allocated once.

    q (B, QH, QL, E), k / v (B, KH, KL, E); pair (B, KL, QL, QH) and kpad (B, KL) bool are
    optional.  qk16 is the backward's Float16 Q/K flag (float32 only)."""

    def __init__(self, torch, nnop, q, k, v, do, causal=True, pair=None, kpad=None, qk16=0, dt=None):
        from nnop import _lib
        from nnop._util import dtype_code, ptr

        self.torch, self.L, self.ptr = torch, _lib.lib(), ptr
        self.q, self.k, self.v, self.do, self.pair, self.kpad = q, k, v, do, pair, kpad
        B, H, QL, E = q.shape
        self.dt = dtype_code(q, "bench") if dt is None else dt  # 3: float32 through bf16x6 MFMA
        self.dims = (E, QL, k.shape[2], H, k.shape[1], B)
        self.causal, self.qk16 = int(causal), int(qk16)
        self.scale = nnop.attention_scale(E, q.dtype)
        self.o = torch.empty_like(q)
        self.ms = torch.empty((B, H, QL), dtype=torch.float32, device=q.device)
        self.ls = torch.empty_like(self.ms)
        self.dq, self.dk, self.dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        self.dpair = None if pair is None else torch.empty_like(pair)
        self.wsb = int(self.L.onionop_flash_attn_bwd_workspace(self.dt, *self.dims))
        self.ws = torch.empty(max(self.wsb, 1), dtype=torch.uint8, device=q.device)
        self.stream = torch.cuda.current_stream().cuda_stream
        self.chk = _lib.check

    def fwd(self):
        p = self.ptr
        self.chk(self.L.onionop_flash_attn_fwd(self.stream, self.dt, *self.dims, p(self.q), p(self.k), p(self.v),
                                               p(self.pair), p(self.kpad), self.causal, self.scale, p(self.o),
                                               p(self.ms), p(self.ls)))

    def pre(self):
        p = self.ptr
        E, QL, KL, QH, KH, B = self.dims
        self.chk(self.L.onionop_flash_attn_bwd_preprocess(self.stream, self.dt, E, QL, QH, B, p(self.do), p(self.o),
                                                          p(self.ms), p(self.ls), p(self.ws), self.wsb))

    def dkdv(self):
        p = self.ptr
        self.chk(self.L.onionop_flash_attn_bwd_dkdv(self.stream, self.dt, *self.dims, p(self.do), p(self.q),
                                                    p(self.k), p(self.v), p(self.pair), p(self.kpad), self.causal,
                                                    self.scale, self.qk16, p(self.dk), p(self.dv), p(self.ws),
                                                    self.wsb))

    def dq_(self):
        p = self.ptr
        self.chk(self.L.onionop_flash_attn_bwd_dq(self.stream, self.dt, *self.dims, p(self.do), p(self.q), p(self.k),
                                                  p(self.v), p(self.pair), p(self.kpad), self.causal, self.scale,
                                                  self.qk16, p(self.dq), p(self.dpair), p(self.ws), self.wsb))

    def bwd(self):
        """The combined backward (the entry point the drop-in's rrule calls): dQ with the
        preprocess fused, then dK/dV."""
        p = self.ptr
        self.chk(self.L.onionop_flash_attn_bwd(self.stream, self.dt, *self.dims, p(self.do), p(self.o), p(self.ms),
                                               p(self.ls), p(self.q), p(self.k), p(self.v), p(self.pair),
                                               p(self.kpad), self.causal, self.scale, self.qk16, p(self.dq),
                                               p(self.dk), p(self.dv), p(self.dpair), p(self.ws), self.wsb))

    def bwd_rope(self, cos, sin):
        """The combined backward with ∇llama_rope fused into the dQ / dK epilogues (q, k are
        the rotated tensors; dq, dk come out w.r.t. the tensors before the rotation)."""
        p = self.ptr
        self.chk(self.L.onionop_flash_attn_bwd_rope(self.stream, self.dt, *self.dims, p(self.do), p(self.o),
                                                    p(self.ms), p(self.ls), p(self.q), p(self.k), p(self.v),
                                                    p(self.pair), p(self.kpad), p(cos), p(sin), self.causal,
                                                    self.scale, self.qk16, p(self.dq), p(self.dk), p(self.dv),
                                                    p(self.dpair), p(self.ws), self.wsb))

    def step(self):
        self.fwd()
        self.bwd()


class VarlenStep:
    """One packed variable-length fwd+bwd step through the C ABI (buffers allocated once):
    q (QH, Tq, E), k / v (KH, Tk, E), sequences at the int32 offsets cu."""

    def __init__(self, torch, nnop, q, k, v, do, cu, max_len, causal=True):
        from nnop import _lib
        from nnop._util import dtype_code, ptr

        self.L, self.ptr, self.chk = _lib.lib(), ptr, _lib.check
        self.q, self.k, self.v, self.do, self.cu = q, k, v, do, cu
        QH, Tq, E = q.shape
        KH, Tk, _ = k.shape
        self.dt = dtype_code(q, "bench")
        self.dims = (E, Tq, Tk, QH, KH, cu.shape[0] - 1)
        self.max_len, self.causal = int(max_len), int(causal)
        self.scale = nnop.attention_scale(E, q.dtype)
        self.o = torch.zeros_like(q)
        self.ms = torch.zeros((QH, Tq), dtype=torch.float32, device=q.device)
        self.ls = torch.zeros_like(self.ms)
        self.dq, self.dk, self.dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
        self.wsb = int(self.L.onionop_flash_attn_varlen_bwd_workspace(self.dt, E, Tq, QH))
        self.ws = torch.empty(max(self.wsb, 1), dtype=torch.uint8, device=q.device)
        self.stream = torch.cuda.current_stream().cuda_stream

    def step(self):
        p, m = self.ptr, self.max_len
        self.chk(self.L.onionop_flash_attn_varlen_fwd(self.stream, self.dt, *self.dims, p(self.cu), p(self.cu), m, m,
                                                      p(self.q), p(self.k), p(self.v), self.causal, self.scale,
                                                      p(self.o), p(self.ms), p(self.ls)))
        self.chk(self.L.onionop_flash_attn_varlen_bwd(self.stream, self.dt, *self.dims, p(self.cu), p(self.cu), m, m,
                                                      p(self.do), p(self.o), p(self.ms), p(self.ls), p(self.q),
                                                      p(self.k), p(self.v), self.causal, self.scale, 0, p(self.dq),
                                                      p(self.dk), p(self.dv), p(self.ws), self.wsb))

    def step_rope(self, cos, sin):
        """step() with ∇llama_rope fused into the backward (cos / sin one row per packed position)."""
        p, m = self.ptr, self.max_len
        self.chk(self.L.onionop_flash_attn_varlen_fwd(self.stream, self.dt, *self.dims, p(self.cu), p(self.cu), m, m,
                                                      p(self.q), p(self.k), p(self.v), self.causal, self.scale,
                                                      p(self.o), p(self.ms), p(self.ls)))
        self.chk(self.L.onionop_flash_attn_varlen_bwd_rope(self.stream, self.dt, *self.dims, p(self.cu), p(self.cu),
                                                           m, m, p(self.do), p(self.o), p(self.ms), p(self.ls),
                                                           p(self.q), p(self.k), p(self.v), p(cos), p(sin),
                                                           self.causal, self.scale, 0, p(self.dq), p(self.dk),
                                                           p(self.dv), p(self.ws), self.wsb))


def time_region(torch, fn, iters):
    """Average ms of fn() over `iters` calls, HIP events on the current stream."""
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    st.record()
    for _ in range(iters):
        fn()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) / iters


def settle(torch, fn, min_ms=100.0, max_ms=500.0, chunk=20):
    """Run fn() until the GPU has reached its steady clocks, before the counted warmup.

    Under this load the MI355X needs some 30 ms to ramp its clocks (the first 50 steps of
    the headline workload average ~1.8x the steady step time).  Chunks of `chunk` calls are
    timed with HIP events for at least min_ms of wall time and until two successive chunks
    agree within 2%, or for at most max_ms.  Returns (wall ms, calls); both are reported."""
    t0 = time.perf_counter()
    calls, prev = 0, None
    while True:
        t = time_region(torch, fn, chunk)
        calls += chunk
        el = (time.perf_counter() - t0) * 1e3
        if el >= max_ms or (el >= min_ms and prev is not None and abs(t - prev) <= 0.02 * prev):
            return el, calls
        prev = t


def stage_times(torch, step, iters):
    """Per-kernel average ms: HIP events around `iters` back-to-back launches of each
    stage on the library's stream.  Every launch of a stage reads the same inputs and
    rewrites the same outputs, so each does the step's work; one event pair per stage
    keeps the events' own cost out of the per-launch figure."""
    stages = (("attn_fwd", step.fwd), ("attn_bwd_pre", step.pre), ("attn_bwd_dkdv", step.dkdv),
              ("attn_bwd_dq", step.dq_))
    out = {}
    for name, fn in stages:
        fn()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        st.record()
        for _ in range(iters):
            fn()
        en.record()
        en.synchronize()
        out[name] = st.elapsed_time(en) / iters
    return out


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` at this workload from the copy-calibrated
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes recorded in profiles/hbm_traffic.json
    (bench.py cannot read hardware counters itself); None when not recorded."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)["kernels"].get(kernel)
    except (OSError, ValueError, KeyError):
        return None
    return None if rec is None else int(rec["bytes"])


def memory_bound(torch, nnop, dev, reps=30):
    """GB/s of the HBM-bound kernels over buffer sets rotated past the 256 MB MALL."""
    from nnop import _lib
    from nnop._util import ptr

    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    g = torch.Generator(device="cpu").manual_seed(1)

    def rot(n_sets, make):
        return [make() for _ in range(n_sets)]

    def measure(name, sets, call, nbytes):
        for _ in range(5):  # warm (the first launches of a kernel run slower)
            for s in sets:
                call(s)
        torch.cuda.synchronize()
        i = [0]

        def one():
            call(sets[i[0] % len(sets)])
            i[0] += 1

        ms = time_region(torch, one, reps * len(sets))
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"GB/s": round(gbs, 1), "frac": round(gbs / MI355X_HBM_GBS, 3), "us": round(ms * 1e3, 2),
                     "bytes": int(nbytes)}
        log(f"  {name}: {ms * 1e3:.1f} us  {gbs:.0f} GB/s")

    # online softmax f32 (8192, 1024): Julia (N=8192, M=1024) -> torch (1024, 8192)
    M, N = 1024, 8192
    sets = rot(8, lambda: (torch.randn((M, N), generator=g).to(dev), torch.empty((M, N), device=dev),
                           torch.empty((M, N), device=dev)))
    measure("softmax_fwd_f32_8192x1024", sets,
            lambda s: _lib.check(L.onionop_softmax_fwd(stream, 0, N, M, ptr(s[0]), ptr(s[1]))), 2 * M * N * 4)
    measure("softmax_bwd_f32_8192x1024", sets,
            lambda s: _lib.check(L.onionop_softmax_bwd(stream, 0, N, M, ptr(s[0]), ptr(s[1]), ptr(s[2]))),
            3 * M * N * 4)
    del sets
    # second-order pullback: reads g, dy, y; writes d_dy, d_y
    sets = rot(6, lambda: tuple(torch.randn((M, N), generator=g).to(dev) for _ in range(5)))
    measure("softmax_bwd_bwd_f32_8192x1024", sets,
            lambda s: _lib.check(L.onionop_softmax_bwd_bwd(stream, 0, N, M, ptr(s[0]), ptr(s[1]), ptr(s[2]),
                                                           ptr(s[3]), ptr(s[4]))), 5 * M * N * 4)
    del sets

    # rms / layer norm bf16, Julia x (4096, 16384) -> torch (16384, 4096)
    emb, n = 4096, 16384
    w = (1 + 0.02 * torch.randn(emb, generator=g)).to(torch.bfloat16).to(dev)
    b = (0.02 * torch.randn(emb, generator=g)).to(torch.bfloat16).to(dev)
    wsb = int(L.onionop_layer_norm_bwd_workspace(emb, n))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    st1 = torch.empty(n, device=dev)
    st2 = torch.empty(n, device=dev)
    dwf = torch.empty(emb, device=dev)
    dwb = torch.empty(emb, dtype=torch.bfloat16, device=dev)
    dbb = torch.empty(emb, dtype=torch.bfloat16, device=dev)
    sets = rot(3, lambda: (torch.randn((n, emb), generator=g).to(torch.bfloat16).to(dev),
                           torch.randn((n, emb), generator=g).to(torch.bfloat16).to(dev),
                           torch.empty((n, emb), dtype=torch.bfloat16, device=dev)))
    xb = n * emb * 2
    measure("rms_norm_fwd_bf16_4096x16384", sets,
            lambda s: _lib.check(L.onionop_rms_norm_fwd(stream, 2, 2, emb, n, ptr(s[0]), ptr(w), 1e-6, 0.0,
                                                        ptr(s[2]), ptr(st1))), 2 * xb + emb * 2 + n * 4)
    measure("rms_norm_bwd_bf16_4096x16384", sets,
            lambda s: _lib.check(L.onionop_rms_norm_bwd(stream, 2, 2, emb, n, ptr(s[1]), ptr(st1), ptr(s[0]), ptr(w),
                                                        0.0, ptr(s[2]), ptr(dwf), ptr(ws), wsb)),
            3 * xb + emb * 2 + n * 4 + emb * 4)
    measure("layer_norm_fwd_bf16_4096x16384", sets,
            lambda s: _lib.check(L.onionop_layer_norm_fwd(stream, 2, 2, emb, n, ptr(s[0]), ptr(w), ptr(b), 1e-6,
                                                          ptr(s[2]), ptr(st1), ptr(st2))), 2 * xb + 2 * emb * 2 + 2 * n * 4)
    measure("layer_norm_bwd_bf16_4096x16384", sets,
            lambda s: _lib.check(L.onionop_layer_norm_bwd(stream, 2, 2, emb, n, ptr(s[1]), ptr(st1), ptr(st2),
                                                          ptr(s[0]), ptr(w), ptr(s[2]), ptr(dwb), ptr(dbb), ptr(ws),
                                                          wsb)), 3 * xb + emb * 2 + 2 * n * 4 + 2 * emb * 2)
    del sets

    # Llama RoPE bf16: q (128, 8192, 32, 4), k (128, 8192, 8, 4) -> torch (4, 32, 8192, 128), (4, 8, 8192, 128)
    E, Lr, QH, KH, Br = 128, 8192, 32, 8, 4
    cos, sin = nnop.LlamaRotaryEmbedding(E)(torch.arange(Lr, dtype=torch.float32)[None].expand(Br, Lr))
    cos, sin = cos.to(dev), sin.to(dev)
    sets = rot(2, lambda: (torch.randn((Br, QH, Lr, E), generator=g).to(torch.bfloat16).to(dev),
                           torch.randn((Br, KH, Lr, E), generator=g).to(torch.bfloat16).to(dev)))
    outs = (torch.empty((Br, QH, Lr, E), dtype=torch.bfloat16, device=dev),
            torch.empty((Br, KH, Lr, E), dtype=torch.bfloat16, device=dev))
    qk_bytes = (QH + KH) * Br * Lr * E * 2
    measure("llama_rope_fwd_bf16_128x8192x32+8x4", sets,
            lambda s: _lib.check(L.onionop_llama_rope(stream, 2, E, Lr, QH, KH, Br, ptr(s[0]), ptr(s[1]), ptr(cos),
                                                      ptr(sin), 1.0, ptr(outs[0]), ptr(outs[1]))),
            2 * qk_bytes + 2 * Br * Lr * (E // 2) * 4)
    return out


def host_threads():
    """Host cores this process may use: OMP_NUM_THREADS when set (the GPU host sets it to
    this job's CPU share), else every core in the process's affinity mask."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(E=64, L=4096, H=4, B=4, threads=None):
    """The oracle's float32 restatement of the reference tile algorithm on the host."""
    import numpy as np

    import oracle

    if threads is None:
        threads = host_threads()
    n = oracle.set_threads(threads)
    rng = np.random.default_rng(2)
    s = 1.0 / math.sqrt(E)
    q, k, v = [oracle.round_to("bf16", rng.standard_normal((B, H, L, E)) * s) for _ in range(3)]
    do = np.ones((B, H, L, E))
    t0 = time.perf_counter()
    o, ms, ls = oracle.attn_fwd(q, k, v, causal=True, scale=s, mode=oracle.FAITHFUL, gsz=64)
    oracle.attn_bwd(do, q, k, v, causal=True, scale=s, mode=oracle.FAITHFUL, o=o, ms=ms, ls=ls, gsz=64,
                    qk_fp16=True)
    dt = time.perf_counter() - t0
    flops = 14 * B * H * L * L * E / 2
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": n, "kind": "port",
            "nproc": os.cpu_count(), "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "sample": f"one full fwd+bwd step of the headline workload (E,L,H,B)=({E},{L},{H},{B}) causal, "
                      f"float32 tile algorithm of the reference (gsz 64, Float16 Q/K in the backward), "
                      f"{dt:.1f} s"}


def workloads(torch, nnop, dev):
    """The other attention workloads at full size, timed through the C ABI with buffers
    allocated once (settled clocks, then HIP events on the library's stream):
      f32     flash attention f32 (64,1024,4,2) non-causal, q,k,v ~ U[0,1), dO = 1, with the
              reference's Float16 Q/K backward (default) and with exact float32 Q/K, on float32
              MFMA and with the bf16x6 products (element type code 3);
      pair    bf16 (32,768,8,2) non-causal with a pair bias (8,768,768,2), gradients incl. the
              bias: FLOP rate and algorithmic HBM rate (inputs not rotated: the 18.9 MB bias
              can sit in the 256 MB MALL);
      gqa     llama_rope + causal GQA flash attention bf16 (128,8192,32:8,4) with per-sequence
              lengths U[1024,8192] (seed 4) as a key-padding mask + llama_rope backward, and the
              same sequences packed (variable-length entry points, RoPE positions per sequence);
              each also with ∇llama_rope fused into the attention backward (…_fused_rope_bwd).
    Rates of the GQA lines count valid work only (7 QH E sum(len^2))."""
    import numpy as np
    from nnop import _lib
    from nnop._util import ptr

    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    g = torch.Generator(device=dev).manual_seed(0)

    def timed(fn, iters):
        settle(torch, fn, min_ms=60.0, max_ms=300.0, chunk=max(1, iters // 2))
        return time_region(torch, fn, iters) * 1e3  # us

    E, QL, H, B = 64, 1024, 4, 2
    q, k, v = [torch.rand((B, H, QL, E), generator=g, device=dev) for _ in range(3)]
    do = torch.ones_like(q)
    fl = 14 * B * H * QL * QL * E
    for x6 in (False, True):  # float32 MFMA, then every product as six bf16 MFMA products
        for qk16 in (1, 0):
            st = AttnStep(torch, nnop, q, k, v, do, causal=False, qk16=qk16, dt=3 if x6 else None)
            t = timed(st.step, 50)
            key = "f32_64x1024x4x2" + ("_bf16x6" if x6 else "") + ("_qk16" if qk16 else "_exact")
            out[key] = {"us": round(t, 1), "TFLOP/s": round(fl / t / 1e6, 1),
                        "frac_of_fp32_mfma": round(fl / t / 1e6 / MI355X_FP32_MFMA_TFLOPS, 3)}
            if x6:  # issued bf16 MFMA work: six products per float32 product
                out[key]["frac_of_bf16_mfma_issued"] = round(6 * fl / t / 1e6 / MI355X_BF16_DENSE_TFLOPS, 3)
            log(f"  {key}: {t:.1f} us  {fl / t / 1e6:.1f} TFLOP/s")
            del st
    del q, k, v, do

    E, QL, H, B = 32, 768, 8, 2
    q, k, v, do = [torch.randn((B, H, QL, E), generator=g, device=dev).to(torch.bfloat16) for _ in range(4)]
    pair = torch.randn((B, QL, QL, H), generator=g, device=dev).to(torch.bfloat16)
    st = AttnStep(torch, nnop, q, k, v, do, causal=False, pair=pair)
    t = timed(st.step, 100)
    fl = 14 * B * H * QL * QL * E
    # bias read by the forward, dQ and dK/dV, dpair written; q,k,v,o,dO,dq,dk,dv once, o re-read
    byt = 4 * pair.numel() * 2 + 9 * q.numel() * 2
    out["pair_bf16_32x768x8x2"] = {"us": round(t, 1), "TFLOP/s": round(fl / t / 1e6, 1),
                                   "GB/s": round(byt / t / 1e3, 1), "algorithmic_bytes": byt,
                                   "frac_of_hbm": round(byt / t / 1e3 / MI355X_HBM_GBS, 3),
                                   "frac_of_bf16_mfma": round(fl / t / 1e6 / MI355X_BF16_DENSE_TFLOPS, 4)}
    log(f"  pair_bf16_32x768x8x2: {t:.1f} us  {fl / t / 1e6:.1f} TFLOP/s  {byt / t / 1e3:.0f} GB/s")
    del st, q, k, v, do, pair

    B, QH, KH, QL, E = 4, 32, 8, 8192, 128
    lens = np.random.default_rng(4).integers(1024, QL + 1, size=B)
    fl = 7 * QH * E * sum(int(n) ** 2 for n in lens)
    rope = nnop.LlamaRotaryEmbedding(E)
    cos, sin = rope(torch.arange(QL, dtype=torch.float32)[None].expand(B, QL))
    cos, sin = cos.to(dev), sin.to(dev)
    q = torch.randn((B, QH, QL, E), generator=g, device=dev).to(torch.bfloat16)
    k, v = [torch.randn((B, KH, QL, E), generator=g, device=dev).to(torch.bfloat16) for _ in range(2)]
    kp = torch.from_numpy(np.arange(QL)[None, :] < lens[:, None]).to(dev)
    do = (torch.randn((B, QH, QL, E), generator=g, device=dev) * kp[:, None, :, None]).to(torch.bfloat16)
    qr, kr = torch.empty_like(q), torch.empty_like(k)
    st = AttnStep(torch, nnop, qr, kr, v, do, causal=True, kpad=kp)
    dqr, dkr = torch.empty_like(q), torch.empty_like(k)

    def gqa_step():
        _lib.check(L.onionop_llama_rope(stream, 2, E, QL, QH, KH, B, ptr(q), ptr(k), ptr(cos), ptr(sin), 1.0,
                                        ptr(qr), ptr(kr)))
        st.step()
        _lib.check(L.onionop_llama_rope(stream, 2, E, QL, QH, KH, B, ptr(st.dq), ptr(st.dk), ptr(cos), ptr(sin),
                                        -1.0, ptr(dqr), ptr(dkr)))

    t = timed(gqa_step, 6)
    out["gqa_rope_bf16_128x8192x32:8x4_keymask"] = {
        "lens": lens.tolist(), "us": round(t), "TFLOP/s_valid_work": round(fl / t / 1e6, 1),
        "frac_of_bf16_mfma": round(fl / t / 1e6 / MI355X_BF16_DENSE_TFLOPS, 4)}
    log(f"  gqa keymask: {t:.0f} us  {fl / t / 1e6:.0f} TFLOP/s (valid work)")

    def gqa_step_fused():  # the same step, ∇llama_rope fused into the attention backward
        _lib.check(L.onionop_llama_rope(stream, 2, E, QL, QH, KH, B, ptr(q), ptr(k), ptr(cos), ptr(sin), 1.0,
                                        ptr(qr), ptr(kr)))
        st.fwd()
        st.bwd_rope(cos, sin)

    t = timed(gqa_step_fused, 6)
    out["gqa_rope_bf16_128x8192x32:8x4_keymask_fused_rope_bwd"] = {
        "us": round(t), "TFLOP/s_valid_work": round(fl / t / 1e6, 1),
        "frac_of_bf16_mfma": round(fl / t / 1e6 / MI355X_BF16_DENSE_TFLOPS, 4)}
    log(f"  gqa keymask, fused rope bwd: {t:.0f} us  {fl / t / 1e6:.0f} TFLOP/s (valid work)")
    del st, qr, kr, dqr, dkr

    # the same sequences packed: (QH, sum(len), E); RoPE positions restart per sequence
    pk = lambda x: torch.cat([x[b, :, :int(n)] for b, n in enumerate(lens)], dim=1).contiguous()
    qp, kpk, vp, dop = pk(q), pk(k), pk(v), pk(do)
    del q, k, v, do, kp
    Tq = int(sum(lens))
    pos = torch.cat([torch.arange(int(n), dtype=torch.float32) for n in lens])[None]
    cosp, sinp = [c.to(dev).contiguous() for c in rope(pos)]
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)).to(dev)
    qrp, krp = torch.empty_like(qp), torch.empty_like(kpk)
    vst = VarlenStep(torch, nnop, qrp, krp, vp, dop, cu, int(max(lens)), causal=True)
    dqp, dkp = torch.empty_like(qp), torch.empty_like(kpk)

    def packed_step():
        _lib.check(L.onionop_llama_rope(stream, 2, E, Tq, QH, KH, 1, ptr(qp), ptr(kpk), ptr(cosp), ptr(sinp), 1.0,
                                        ptr(qrp), ptr(krp)))
        vst.step()
        _lib.check(L.onionop_llama_rope(stream, 2, E, Tq, QH, KH, 1, ptr(vst.dq), ptr(vst.dk), ptr(cosp),
                                        ptr(sinp), -1.0, ptr(dqp), ptr(dkp)))

    t = timed(packed_step, 6)
    out["gqa_rope_bf16_128x8192x32:8x4_packed"] = {
        "lens": lens.tolist(), "us": round(t), "TFLOP/s_valid_work": round(fl / t / 1e6, 1),
        "frac_of_bf16_mfma": round(fl / t / 1e6 / MI355X_BF16_DENSE_TFLOPS, 4)}
    log(f"  gqa packed: {t:.0f} us  {fl / t / 1e6:.0f} TFLOP/s (valid work)")

    def packed_step_fused():
        _lib.check(L.onionop_llama_rope(stream, 2, E, Tq, QH, KH, 1, ptr(qp), ptr(kpk), ptr(cosp), ptr(sinp), 1.0,
                                        ptr(qrp), ptr(krp)))
        vst.step_rope(cosp, sinp)

    t = timed(packed_step_fused, 6)
    out["gqa_rope_bf16_128x8192x32:8x4_packed_fused_rope_bwd"] = {
        "us": round(t), "TFLOP/s_valid_work": round(fl / t / 1e6, 1),
        "frac_of_bf16_mfma": round(fl / t / 1e6 / MI355X_BF16_DENSE_TFLOPS, 4)}
    log(f"  gqa packed, fused rope bwd: {t:.0f} us  {fl / t / 1e6:.0f} TFLOP/s (valid work)")
    return out


SWEEP = [  # (E, L, H, KH, B, causal): bf16 attention fwd+bwd shapes around the headline
    (64, 1024, 16, 16, 4, True), (64, 2048, 8, 8, 4, True), (64, 4096, 4, 4, 4, True), (64, 8192, 4, 4, 2, True),
    (64, 16384, 4, 4, 1, True), (64, 4096, 4, 4, 4, False), (64, 4096, 16, 4, 4, True), (64, 4096, 16, 16, 4, True),
    (128, 1024, 16, 16, 4, True), (128, 4096, 4, 4, 4, True), (128, 4096, 32, 8, 1, True),
    (128, 8192, 8, 2, 2, True), (128, 4096, 4, 4, 4, False), (32, 4096, 8, 8, 4, True), (16, 4096, 8, 8, 4, True),
    (256, 2048, 4, 4, 2, True), (256, 4096, 8, 8, 1, True), (64, 4096, 32, 8, 1, True), (64, 4096, 8, 1, 4, True),
    (128, 2048, 32, 8, 2, True), (128, 4096, 8, 1, 4, True), (128, 4096, 32, 8, 4, True),
]


def sweep(torch, nnop, dev):
    """bf16 flash attention fwd+bwd over SWEEP's shapes (q, k, v ~ N(0,1)/sqrt(E), dO = 1),
    timed as the headline: settled clocks, then HIP events; FLOPs 14 B H L^2 E (x 1/2 causal)."""
    out = []
    for E, L, H, KH, B, causal in SWEEP:
        g = torch.Generator(device="cpu").manual_seed(5)
        s = 1.0 / math.sqrt(E)
        q = (torch.randn((B, H, L, E), generator=g) * s).to(torch.bfloat16).to(dev)
        k, v = [(torch.randn((B, KH, L, E), generator=g) * s).to(torch.bfloat16).to(dev) for _ in range(2)]
        do = torch.ones_like(q)
        st = AttnStep(torch, nnop, q, k, v, do, causal=causal)
        fl = 14 * B * H * L * L * E / (2 if causal else 1)
        settle(torch, st.step, min_ms=60.0, max_ms=300.0, chunk=5)
        t = time_region(torch, st.step, 20) * 1e3
        rec = {"E": E, "L": L, "H": H, "KH": KH, "B": B, "causal": causal, "us": round(t, 1),
               "TFLOP/s": round(fl / t / 1e6, 1), "frac_of_bf16_mfma": round(fl / t / 1e6 / MI355X_BF16_DENSE_TFLOPS, 3)}
        log(f"  sweep {rec}")
        out.append(rec)
        del q, k, v, do, st
    return out


def counter_summary(paths, last=20):
    """Per-kernel averages of rocprofv3 --pmc counter CSVs (the last `last` dispatches of each
    kernel, i.e. the timed steps), with the derived utilisations:
      mfma_busy  = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 * 1024)
                   (MFMA-busy cycles summed over the 1024 SIMDs, over the kernel's active
                   cycles; rocprofv3 sums GRBM_GUI_ACTIVE over the 8 XCDs)
      valu_busy  = 4 * SQ_ACTIVE_INST_VALU / (GRBM_GUI_ACTIVE / 8 * 1024)   (quad-cycles)
      coexec     = SQ_VALU_MFMA_COEXEC_CYCLES / (GRBM_GUI_ACTIVE / 8 * 1024)
      lds_active = SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE / 8 * 256)          (per CU)
      bank_conflict_share = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE
      valu_per_mfma = SQ_INSTS_VALU / SQ_INSTS_MFMA"""
    import csv

    def short(mangled):  # last name of an Itanium nested name: _ZN7onionop20attn_fwd_pipe_kernelI...
        if not mangled.startswith("_ZN"):
            return None  # torch's own kernels
        pos, last = 3, None
        while pos < len(mangled) and mangled[pos].isdigit():
            end = pos
            while mangled[end].isdigit():
                end += 1
            n = int(mangled[pos:end])
            last = mangled[end:end + n]
            pos = end + n
        args = mangled[pos:].split("EEEv")[0] if pos < len(mangled) else ""
        args = args[1:] if args.startswith("I") else args  # "I" opens the template arguments
        return f"{last}<{args}>" if args else last  # template arguments keep instantiations apart

    acc = {}
    for path in paths:
        for r in csv.DictReader(open(path)):
            name = short(r["Kernel_Name"])
            if name is None:  # torch's own kernels
                continue
            acc.setdefault(name, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    out = {}
    for name, cs in acc.items():
        avg = {c: sum(v[-last:]) / len(v[-last:]) for c, v in cs.items()}
        d = {c: round(x, 1) for c, x in sorted(avg.items())}
        gui = avg.get("GRBM_GUI_ACTIVE")
        if gui:
            simd = gui / 8 * 1024
            if "SQ_VALU_MFMA_BUSY_CYCLES" in avg:
                d["mfma_busy"] = round(avg["SQ_VALU_MFMA_BUSY_CYCLES"] / simd, 4)
            if "SQ_ACTIVE_INST_VALU" in avg:
                d["valu_busy"] = round(4 * avg["SQ_ACTIVE_INST_VALU"] / simd, 4)
            if "SQ_VALU_MFMA_COEXEC_CYCLES" in avg:
                d["coexec"] = round(avg["SQ_VALU_MFMA_COEXEC_CYCLES"] / simd, 4)
            if "SQ_LDS_IDX_ACTIVE" in avg:
                d["lds_active"] = round(avg["SQ_LDS_IDX_ACTIVE"] / (gui / 8 * 256), 4)
        if avg.get("SQ_LDS_IDX_ACTIVE") and "SQ_LDS_BANK_CONFLICT" in avg:
            d["bank_conflict_share"] = round(avg["SQ_LDS_BANK_CONFLICT"] / avg["SQ_LDS_IDX_ACTIVE"], 4)
        if avg.get("SQ_INSTS_MFMA") and "SQ_INSTS_VALU" in avg:
            d["valu_per_mfma"] = round(avg["SQ_INSTS_VALU"] / avg["SQ_INSTS_MFMA"], 2)
        out[name] = d
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # Counted warmup steps; before them a settle phase (reported as settle_ms / settle_steps)
    # runs the step until the GPU's clocks are steady (see settle()).
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-memory", action="store_true", help="skip the HBM-bound kernel set")
    ap.add_argument("--no-workloads", action="store_true", help="skip the other attention workloads")
    ap.add_argument("--workloads", action="store_true",
                    help="only time the other attention workloads (float32, pair bias, RoPE + GQA key mask "
                         "and packed) and print them as one JSON line")
    ap.add_argument("--sweep", action="store_true",
                    help="only time bf16 attention fwd+bwd over a list of shapes around the headline "
                         "and print them as one JSON line")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run 3 plain device copies of MIB MiB (a known-size kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--counter-summary", nargs="+", metavar="CSV",
                    help="summarise rocprofv3 --pmc counter CSVs per kernel (no GPU needed) and exit")
    args = ap.parse_args()
    if args.counter_summary:
        print(json.dumps(counter_summary(args.counter_summary), indent=1))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (run with --gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch

    import nnop

    dev = torch.device("cuda:0")
    if args.workloads:
        print(json.dumps(workloads(torch, nnop, dev)), flush=True)
        return
    if args.sweep:
        print(json.dumps({"sweep": sweep(torch, nnop, dev)}), flush=True)
        return
    E, L, H, B = 64, 4096, 4, 4
    q, k, v, do = attention_setup(torch, nnop, dev, E, L, H, B)
    step = AttnStep(torch, nnop, q, k, v, do, causal=True)
    settle_ms, settle_steps = settle(torch, step.step)
    log(f"bench: flash attention fwd+bwd bf16 (E,L,H,B)=({E},{L},{H},{B}) causal; settled clocks in "
        f"{settle_ms:.0f} ms ({settle_steps} steps); warmup {args.warmup}")
    for _ in range(args.warmup):
        step.step()
    torch.cuda.synchronize()
    ms = time_region(torch, step.step, args.steps)
    flops = 14 * B * H * L * L * E / 2
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"  step {ms * 1e3:.1f} us -> {tflops:.1f} TFLOP/s")

    stages = stage_times(torch, step, max(10, args.steps // 2))
    unit = B * H * L * L * E / 2  # 2*B*H*L^2*E/2 flops per causal GEMM
    stage_flops = {"attn_fwd": 4 * unit, "attn_bwd_dkdv": 8 * unit, "attn_bwd_dq": 2 * unit, "attn_bwd_pre": 0}
    dom = max((n for n in stages if stage_flops[n] > 0), key=lambda n: stages[n])
    ach = stage_flops[dom] / (stages[dom] * 1e-3) / 1e12
    log("  kernels (us): " + ", ".join(f"{n} {t * 1e3:.1f}" for n, t in stages.items()))
    roofline = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 1), "peak": MI355X_BF16_DENSE_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / MI355X_BF16_DENSE_TFLOPS, 4),
                "traffic": measured_traffic(dom), "avg_us": round(stages[dom] * 1e3, 2),
                "kernel_us": {n: round(t * 1e3, 2) for n, t in stages.items()}}

    result = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_ms": round(settle_ms, 1), "settle_steps": settle_steps,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1)/sqrt(E) q,k,v; dO = 1)",
        "config": {"workload": "flash_attention fwd+bwd bf16 (E,L,H,B)=(64,4096,4,4) causal",
                   "E": E, "L": L, "H": H, "B": B, "causal": True, "flops_per_step": flops,
                   "flop_convention": "14*B*H*L^2*E/2"},
        "roofline": roofline,
    }
    if args.calibrate_copy > 0:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: calibration copies of {args.calibrate_copy} MiB done")
        del src, dst
    if not args.no_memory:
        log("bench: HBM-bound kernels")
        result["memory_bound"] = memory_bound(torch, nnop, dev)
    if not args.no_workloads:
        log("bench: other attention workloads")
        del q, k, v, do, step
        result["workloads"] = workloads(torch, nnop, dev)
    if not args.no_cpu:
        log("bench: CPU baseline (oracle port, float32)")
        result["cpu_baseline"] = cpu_baseline(E, L, H, B)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
