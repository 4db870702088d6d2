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

`roofline` is the slowest kernel of the step, timed alone with HIP events on the stream
the library launches on.  `cpu_baseline` is the oracle's float32 restatement of the
reference algorithm (oracle/oracle.c, FAITHFUL mode) on the host cores.
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
    """One fwd+bwd step through the C ABI, with buffers allocated once."""

    def __init__(self, torch, nnop, q, k, v, do, causal=True):
        from nnop import _lib
        from nnop._util import ptr

        self.torch, self.L, self.ptr = torch, _lib.lib(), ptr
        self.q, self.k, self.v, self.do = q, k, v, do
        B, H, QL, E = q.shape
        self.dims = (E, QL, k.shape[2], H, k.shape[1], B)
        self.causal = int(causal)
        self.scale = nnop.attention_scale(E, q.dtype)
        self.o = torch.empty_like(q)
        self.ms = torch.empty((B, H, QL), dtype=torch.float32, device=q.device)
        self.ls = torch.empty_like(self.ms)
        self.dq, self.dk, self.dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        self.wsb = int(self.L.onionop_flash_attn_bwd_workspace(2, *self.dims))
        self.ws = torch.empty(self.wsb, dtype=torch.uint8, device=q.device)
        self.stream = torch.cuda.current_stream().cuda_stream
        self.chk = _lib.check

    def fwd(self):
        p = self.ptr
        self.chk(self.L.onionop_flash_attn_fwd(self.stream, 2, *self.dims, p(self.q), p(self.k), p(self.v), None,
                                               None, self.causal, self.scale, p(self.o), p(self.ms), p(self.ls)))

    def pre(self):
        p = self.ptr
        E, QL, KL, QH, KH, B = self.dims
        self.chk(self.L.onionop_flash_attn_bwd_preprocess(self.stream, 2, E, QL, QH, B, p(self.do), p(self.o),
                                                          p(self.ms), p(self.ls), p(self.ws), self.wsb))

    def dkdv(self):
        p = self.ptr
        self.chk(self.L.onionop_flash_attn_bwd_dkdv(self.stream, 2, *self.dims, p(self.do), p(self.q), p(self.k),
                                                    p(self.v), None, None, self.causal, self.scale, 0, p(self.dk),
                                                    p(self.dv), p(self.ws), self.wsb))

    def dq_(self):
        p = self.ptr
        self.chk(self.L.onionop_flash_attn_bwd_dq(self.stream, 2, *self.dims, p(self.do), p(self.q), p(self.k),
                                                  p(self.v), None, None, self.causal, self.scale, 0, p(self.dq),
                                                  None, p(self.ws), self.wsb))

    def bwd(self):
        """The combined backward (the entry point the drop-in's rrule calls): dQ with the
        preprocess fused, then dK/dV."""
        p = self.ptr
        self.chk(self.L.onionop_flash_attn_bwd(self.stream, 2, *self.dims, p(self.do), p(self.o), p(self.ms),
                                               p(self.ls), p(self.q), p(self.k), p(self.v), None, None, self.causal,
                                               self.scale, 0, p(self.dq), p(self.dk), p(self.dv), None, p(self.ws),
                                               self.wsb))

    def step(self):
        self.fwd()
        self.bwd()


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


def stage_times(torch, step, iters):
    """Per-kernel average ms: events between the four launches of each step."""
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(iters)]
    torch.cuda.synchronize()
    for i in range(iters):
        e = ev[i]
        e[0].record()
        step.fwd()
        e[1].record()
        step.pre()
        e[2].record()
        step.dkdv()
        e[3].record()
        step.dq_()
        e[4].record()
    torch.cuda.synchronize()
    names = ["attn_fwd", "attn_bwd_pre", "attn_bwd_dkdv", "attn_bwd_dq"]
    return {n: sum(ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(iters)) / iters for j, n in enumerate(names)}


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


def cpu_baseline(E=64, L=4096, H=4, B=4, threads=None):
    """The oracle's float32 restatement of the reference tile algorithm on the host."""
    import numpy as np

    import oracle

    if threads is None:
        threads = min(16, os.cpu_count() or 1)
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
            "sample": f"one full fwd+bwd step of the headline workload (E,L,H,B)=({E},{L},{H},{B}) causal, "
                      f"float32 tile algorithm of the reference (gsz 64, Float16 Q/K in the backward), "
                      f"{dt:.1f} s"}


def workload_timings(torch, nnop, dev):
    """Steady-state fwd+bwd times of the three other attention workloads at full size, through
    the nnop API (0.3 s warm, then HIP events): float32 (64,1024,4,2) non-causal with the
    Float16 Q/K backward, bf16 pair bias (32,768,8,2), and RoPE + causal GQA (128,8192,32:8,4)
    with per-sequence lengths in [1024, 8192] as a key mask, plus the RoPE backward.
    One JSON line each; inputs are not rotated (the 18.9 MB bias can sit in the MALL)."""
    import numpy as np

    def steady(f, iters):
        t0 = time.time()
        while time.time() - t0 < 0.3:
            f()
        torch.cuda.synchronize()
        return time_region(torch, f, iters) * 1e3  # us

    g = torch.Generator(device="cpu").manual_seed(0)
    E, L, H, B = 64, 1024, 4, 2
    q, k, v = [torch.rand((B, H, L, E), generator=g).to(dev) for _ in range(3)]
    do = torch.ones_like(q)

    def f32_step():
        o, ms, ls = nnop._flash_attention(q, k, v, causal=False)
        nnop.grad_flash_attention(do, o, ms, ls, q, k, v, causal=False, qk_fp16=True)

    t = steady(f32_step, 50)
    fl = 14 * B * H * L * L * E
    print(json.dumps({"workload": "flash_attention fwd+bwd f32 (64,1024,4,2) non-causal, Float16 Q/K backward",
                      "us": round(t, 1), "TFLOP/s": round(fl / t / 1e6, 1),
                      "frac_of_fp32_mfma": round(fl / t / 1e6 / MI355X_FP32_MFMA_TFLOPS, 3)}), flush=True)

    E, L, H, B = 32, 768, 8, 2
    q, k, v, do = [torch.randn((B, H, L, E), generator=g).to(torch.bfloat16).to(dev) for _ in range(4)]
    pair = torch.randn((B, L, L, H), generator=g).to(torch.bfloat16).to(dev)

    def pair_step():
        o, ms, ls = nnop._flash_attention(q, k, v, pair, causal=False)
        nnop.grad_flash_attention(do, o, ms, ls, q, k, v, pair, causal=False)

    t = steady(pair_step, 50)
    fl = 14 * B * H * L * L * E
    # bias read by the forward and dK/dV, read and dpair written by dQ; q,k,v,o,dO,dq,dk,dv, o re-read
    byt = 3 * pair.numel() * 2 + 9 * q.numel() * 2
    print(json.dumps({"workload": "flash_attention fwd+bwd bf16 (32,768,8,2) non-causal, pair bias, grads incl. bias",
                      "us": round(t, 1), "TFLOP/s": round(fl / t / 1e6, 1), "GB/s": round(byt / t / 1e3),
                      "algorithmic_MB": round(byt / 1e6, 1)}), flush=True)

    B, QH, KH, L, E = 4, 32, 8, 8192, 128
    lens = np.random.default_rng(4).integers(1024, L + 1, size=B)
    q = torch.randn((B, QH, L, E), generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn((B, KH, L, E), generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn((B, KH, L, E), generator=g).to(torch.bfloat16).to(dev)
    cos, sin = nnop.LlamaRotaryEmbedding(E)(torch.arange(L, dtype=torch.float32)[None].expand(B, L))
    cos, sin = cos.to(dev), sin.to(dev)
    kp = torch.from_numpy(np.arange(L)[None, :] < lens[:, None]).to(dev)
    do = torch.randn_like(q) * kp[:, None, :, None]

    def gqa_step():
        qr, kr = nnop._llama_rope(q, k, cos, sin, bwd=False)
        o, ms, ls = nnop._flash_attention(qr, kr, v, causal=True, kpad_mask=kp)
        dq, dk, dv, _ = nnop.grad_flash_attention(do, o, ms, ls, qr, kr, v, causal=True, kpad_mask=kp)
        nnop._llama_rope(dq, dk, cos, sin, bwd=True)

    t = steady(gqa_step, 5)
    fl = 7 * QH * E * sum(int(n) ** 2 for n in lens)  # causal fwd+bwd over each sequence's valid keys
    print(json.dumps({"workload": "llama_rope + flash_attention fwd+bwd bf16 (128,8192,32:8,4) causal GQA, "
                      "key mask from per-sequence lengths, + llama_rope bwd", "lens": lens.tolist(),
                      "us": round(t), "TFLOP/s_valid_work": round(fl / t / 1e6),
                      "frac_of_bf16_peak": round(fl / t / 1e6 / MI355X_BF16_DENSE_TFLOPS, 3)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # The GPU reaches its steady clocks only after some 30 ms of this load (the first 50
    # steps average ~1.8x the steady step time), so the default warmup is 200 steps (~40 ms).
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-memory", action="store_true", help="skip the HBM-bound kernel set")
    ap.add_argument("--workloads", action="store_true",
                    help="instead of the bench line, time the other attention workloads (float32, "
                         "pair bias, RoPE + GQA) and print one JSON line each")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run 3 plain device copies of MIB MiB (a known-size kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch

    import nnop

    dev = torch.device("cuda:0")
    if args.workloads:
        workload_timings(torch, nnop, dev)
        return
    E, L, H, B = 64, 4096, 4, 4
    q, k, v, do = attention_setup(torch, nnop, dev, E, L, H, B)
    step = AttnStep(torch, nnop, q, k, v, do, causal=True)
    log(f"bench: flash attention fwd+bwd bf16 (E,L,H,B)=({E},{L},{H},{B}) causal; warmup {args.warmup}")
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
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
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
    if not args.no_cpu:
        log("bench: CPU baseline (oracle port, float32)")
        result["cpu_baseline"] = cpu_baseline(E, L, H, B)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
