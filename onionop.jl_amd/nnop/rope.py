"""Llama rotary embedding: LlamaRotaryEmbedding, llama_rope and its rrule.

q (B, QH, L, E) == Julia (E, L, QH, B); k (B, KH, L, E); cos, sin (B, L, E) float32
== Julia (E, L, B).
"""
from __future__ import annotations

import torch

from . import _lib
from ._util import device_tensor, dtype_code, ptr, stream_of


class LlamaRotaryEmbedding:
    """LlamaRotaryEmbedding (src/rope/llama_rope.jl:1-22): cos/sin tables (input generator).

    inv_freq = 1 ./ base .^ ((0:2:dim-1) ./ dim) in float32; called on position ids (B, L)
    it returns cos, sin of vcat(freqs, freqs), shape (B, L, dim) float32.
    """

    def __init__(self, dim: int, base: int = 10000, device=None):
        ids = torch.arange(0, dim, 2, dtype=torch.float32, device=device) / float(dim)
        self.inv_freq = 1.0 / (float(base) ** ids)
        self.dim = dim
        self.base = base

    def __call__(self, position_ids: torch.Tensor):
        pos = position_ids.to(torch.float32)
        if pos.dim() == 1:
            pos = pos[None]
        if pos.is_cuda:  # on the device: the library's table kernel
            return rotary_tables(pos, self.dim, self.base)
        freqs = pos[..., None] * self.inv_freq.to(pos.device)[None, None, :]
        freqs = torch.cat([freqs, freqs], dim=-1)
        return torch.cos(freqs).contiguous(), torch.sin(freqs).contiguous()


def rotary_tables(positions: torch.Tensor, dim: int, base: int = 10000):
    """cos, sin (B, L, dim) float32 of LlamaRotaryEmbedding(dim; base) at device positions
    (B, L) (src/rope/llama_rope.jl:1-22), computed by the library on the positions' device."""
    pos = device_tensor(positions, "LlamaRotaryEmbedding").to(torch.float32).contiguous()
    if pos.dim() != 2:
        raise ValueError("LlamaRotaryEmbedding: positions must be (seq, batch) == torch (B, L)")
    B, L = pos.shape
    cos = torch.empty((B, L, dim), dtype=torch.float32, device=pos.device)
    sin = torch.empty_like(cos)
    _lib.check(_lib.lib().onionop_llama_rotary_embedding(stream_of(pos), int(dim), L, B, int(base), ptr(pos),
                                                         ptr(cos), ptr(sin)))
    return cos, sin


def _llama_rope(q, k, cos, sin, *, bwd: bool):
    """_llama_rope (src/rope/llama_rope.jl:69-89), out of place: returns (q', k')."""
    q = device_tensor(q, "llama_rope")
    k = device_tensor(k, "llama_rope")
    cos = device_tensor(cos, "llama_rope").to(torch.float32)
    sin = device_tensor(sin, "llama_rope").to(torch.float32)
    if q.dim() != 4 or k.dim() != 4:
        raise ValueError("llama_rope: q and k must be (E, L, H, B) arrays")
    B, QH, L, E = q.shape
    KB, KH, KL, KE = k.shape
    # @assert checks of src/rope/llama_rope.jl:70-72
    if KE != E:
        raise ValueError("AssertionError: size(q, 1) == size(k, 1)")
    if KL != L:
        raise ValueError("AssertionError: size(q, 2) == size(k, 2)")
    if KB != B:
        raise ValueError("AssertionError: size(q, 4) == size(k, 4)")
    if cos.shape != (B, L, E) or sin.shape != (B, L, E):
        raise ValueError(f"llama_rope: cos/sin must have Julia shape {(E, L, B)}")
    if k.dtype != q.dtype:
        raise TypeError("llama_rope: q and k must share one element type")
    qo = torch.empty_like(q)
    ko = torch.empty_like(k)
    _lib.check(_lib.lib().onionop_llama_rope(stream_of(q), dtype_code(q, "llama_rope"), E, L, QH, KH, B, ptr(q),
                                             ptr(k), ptr(cos), ptr(sin), -1.0 if bwd else 1.0, ptr(qo), ptr(ko)))
    return qo, ko


def grad_llama_rope(dq, dk, *, cos, sin):
    """∇llama_rope (src/rope/llama_rope.jl:92)."""
    return _llama_rope(dq, dk, cos, sin, bwd=True)


class _LlamaRopeFn(torch.autograd.Function):
    """rrule(llama_rope) (src/rope/llama_rope.jl:94-98)."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        qo, ko = _llama_rope(q, k, cos, sin, bwd=False)
        ctx.save_for_backward(cos, sin)
        ctx.q_meta = (q.shape, q.dtype, q.device)
        ctx.k_meta = (k.shape, k.dtype, k.device)
        return qo, ko

    @staticmethod
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        if dq is None:
            dq = torch.zeros(ctx.q_meta[0], dtype=ctx.q_meta[1], device=ctx.q_meta[2])
        if dk is None:
            dk = torch.zeros(ctx.k_meta[0], dtype=ctx.k_meta[1], device=ctx.k_meta[2])
        gq, gk = grad_llama_rope(dq.contiguous(), dk.contiguous(), cos=cos, sin=sin)
        return gq, gk, None, None


def llama_rope(q, k, *, cos, sin):
    """NNop.llama_rope (src/rope/llama_rope.jl:91): rotate-half RoPE of q and k."""
    return _LlamaRopeFn.apply(q, k, cos, sin)
