"""Flash attention: the host side of NNop.flash_attention over libonionop_hip.so.

Shapes are the reference's column-major Julia arrays read as row-major torch tensors:
  q (B, QH, QL, E)      == Julia (E, QL, QH, B)
  k, v (B, KH, KL, E)   == Julia (E, KL, KH, B)
  pair (B, KL, QL, QH)  == Julia (QH, QL, KL, B)   (additive bias, after the scale)
  kpad_mask (B, KL)     == Julia (KL, B) Bool      (False = masked key)
  ms, ls (B, QH, QL)    == Julia (QL, QH, B), float32
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from ._util import _F32_ATTN, attn_dtype_code, device_tensor, jdims, ptr, round_scalar, stream_of


def _check_shapes(q, k, v, pair, kpad_mask):
    """Validation of _flash_attention / ∇flash_attention (src/attention.jl:150-156,
    src/attention_bwd.jl:221-227), with the reference's messages."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k and v must be 4-dimensional (E, L, H, B) arrays")
    B, QH, QL, QE = q.shape
    KB, KH, KL, KE = k.shape
    if QE != KE:
        raise ValueError(f"Embedding dim of Q `{QE}` must be the same as of K `{KE}`.")
    if k.shape != v.shape:
        raise ValueError(f"Shapes of K `{jdims(k)}` and V `{jdims(v)}` must be the same.")
    if QE <= 0 or (QE & (QE - 1)) != 0:
        raise ValueError("Only power-of-2 embedding dims are supported.")
    if KH == 0 or QH % KH != 0:
        raise ValueError(f"Number of query heads `{QH}` must be divisible by number of KV heads `{KH}`.")
    if KB != B:
        raise ValueError(f"Batch of Q `{B}` must be the same as of K `{KB}`.")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k and v must share one element type")
    if pair is not None:
        if tuple(pair.shape) != (B, KL, QL, QH):
            raise ValueError(f"pair must have Julia shape {(QH, QL, KL, B)}, got {jdims(pair)}")
        if pair.dtype != q.dtype:
            raise TypeError("pair must have the element type of q")
    if kpad_mask is not None:
        if kpad_mask.dtype != torch.bool or tuple(kpad_mask.shape) != (B, KL):
            raise ValueError(f"kpad_mask must be a Bool array of Julia shape {(KL, B)}")
    return B, QH, QL, QE, KH, KL


def set_float32_attention_precision(mode: str) -> None:
    """Precision of float32 flash attention for this process.

    "float32" (default): float32 MFMA products, as the reference's float32 FMAs.
    "bf16x6": each float32 operand is split exactly into three bf16 parts and every product
    is accumulated in float32 from the six part products above 2^-23 relative size, on the
    bf16 matrix cores (element type code ONIONOP_F32_BF16X6).  Softmax, masks and all sums
    stay float32.  No counterpart in the reference."""
    if mode not in ("float32", "bf16x6"):
        raise ValueError(f"float32 attention precision must be 'float32' or 'bf16x6', got {mode!r}")
    _F32_ATTN[0] = mode


def get_float32_attention_precision() -> str:
    return _F32_ATTN[0]


class float32_attention_precision:
    """Context manager: `with nnop.float32_attention_precision("bf16x6"): ...`."""

    def __init__(self, mode: str):
        self.mode, self.prev = mode, None

    def __enter__(self):
        self.prev = _F32_ATTN[0]
        set_float32_attention_precision(self.mode)
        return self

    def __exit__(self, *exc):
        _F32_ATTN[0] = self.prev
        return False


def attention_scale(E: int, dtype: torch.dtype) -> float:
    """T(1/sqrt(E)) (src/attention.jl:166)."""
    return round_scalar(1.0 / math.sqrt(E), dtype)


def _flash_attention(q, k, v, pair=None, *, causal: bool, kpad_mask=None):
    """Forward launcher; returns (o, ms, ls) like `_flash_attention` (src/attention.jl:145-197)."""
    q = device_tensor(q, "flash_attention")
    k = device_tensor(k, "flash_attention")
    v = device_tensor(v, "flash_attention")
    pair = None if pair is None else device_tensor(pair, "flash_attention")
    kpad_mask = None if kpad_mask is None else device_tensor(kpad_mask, "flash_attention")
    B, QH, QL, E, KH, KL = _check_shapes(q, k, v, pair, kpad_mask)
    dt = attn_dtype_code(q, "flash_attention")
    o = torch.empty_like(q)
    ms = torch.empty((B, QH, QL), dtype=torch.float32, device=q.device)
    ls = torch.empty((B, QH, QL), dtype=torch.float32, device=q.device)
    _lib.check(_lib.lib().onionop_flash_attn_fwd(
        stream_of(q), dt, E, QL, KL, QH, KH, B, ptr(q), ptr(k), ptr(v), ptr(pair), ptr(kpad_mask),
        int(bool(causal)), attention_scale(E, q.dtype), ptr(o), ptr(ms), ptr(ls)))
    return o, ms, ls


def grad_flash_attention(do, o, ms, ls, q, k, v, pair=None, *, causal: bool, kpad_mask=None,
                         qk_fp16: bool = True):
    """Backward launcher ∇flash_attention (src/attention_bwd.jl:213-303).

    Returns (dq, dk, dv, dpair or None).  qk_fp16=True rounds Q and K to Float16 in every
    product, as the reference does for every element type (src/attention_bwd.jl:20-21);
    it only affects float32 inputs.
    """
    q = device_tensor(q, "∇flash_attention")
    k = device_tensor(k, "∇flash_attention")
    v = device_tensor(v, "∇flash_attention")
    do = device_tensor(do, "∇flash_attention").to(q.dtype)
    o = device_tensor(o, "∇flash_attention")
    ms = device_tensor(ms, "∇flash_attention")
    ls = device_tensor(ls, "∇flash_attention")
    pair = None if pair is None else device_tensor(pair, "∇flash_attention")
    kpad_mask = None if kpad_mask is None else device_tensor(kpad_mask, "∇flash_attention")
    B, QH, QL, E, KH, KL = _check_shapes(q, k, v, pair, kpad_mask)
    if do.shape != q.shape or o.shape != q.shape:
        raise ValueError("Δ and o must have the shape of q")
    dt = attn_dtype_code(q, "∇flash_attention")
    L = _lib.lib()
    ws_bytes = L.onionop_flash_attn_bwd_workspace(dt, E, QL, KL, QH, KH, B)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=q.device)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dpair = None if pair is None else torch.empty_like(pair)
    _lib.check(L.onionop_flash_attn_bwd(
        stream_of(q), dt, E, QL, KL, QH, KH, B, ptr(do), ptr(o), ptr(ms), ptr(ls), ptr(q), ptr(k), ptr(v),
        ptr(pair), ptr(kpad_mask), int(bool(causal)), attention_scale(E, q.dtype), int(bool(qk_fp16)), ptr(dq),
        ptr(dk), ptr(dv), ptr(dpair), ptr(ws), int(ws_bytes)))
    return dq, dk, dv, dpair


class _FlashAttentionFn(torch.autograd.Function):
    """The rrule of _flash_attention (src/attention_crc.jl:16-31)."""

    @staticmethod
    def forward(ctx, q, k, v, pair, kpad_mask, causal, qk_fp16):
        o, ms, ls = _flash_attention(q, k, v, pair, causal=causal, kpad_mask=kpad_mask)
        ctx.save_for_backward(q, k, v, pair, kpad_mask, o, ms, ls)
        ctx.causal = causal
        ctx.qk_fp16 = qk_fp16
        ctx.mark_non_differentiable(ms, ls)
        return o, ms, ls

    @staticmethod
    def backward(ctx, do, _dms, _dls):
        q, k, v, pair, kpad_mask, o, ms, ls = ctx.saved_tensors
        if do is None:
            do = torch.zeros_like(o)
        dq, dk, dv, dpair = grad_flash_attention(do.contiguous(), o, ms, ls, q, k, v, pair, causal=ctx.causal,
                                                 kpad_mask=kpad_mask, qk_fp16=ctx.qk_fp16)
        return dq, dk, dv, dpair, None, None, None


def flash_attention(q, k, v, pair: Optional[torch.Tensor] = None, *, causal: bool,
                    kpad_mask: Optional[torch.Tensor] = None, qk_fp16: bool = True):
    """NNop.flash_attention (src/attention_crc.jl:4-14): softmax(scale K^T Q + pair + masks) V.

    Differentiable with torch autograd in q, k, v and pair; GQA when QH is a multiple of KH.
    """
    o, _, _ = _FlashAttentionFn.apply(q, k, v, pair, kpad_mask, bool(causal), bool(qk_fp16))
    return o


# ---------------------------------------------------------------- packed variable length
#
# Packed sequences (no padding): q (QH, Tq, E) == Julia (E, Tq, QH), k / v (KH, Tk, E);
# sequence b is rows cu_seqlens_q[b]:cu_seqlens_q[b+1] of q (and cu_seqlens_k of k / v);
# ms, ls (QH, Tq).  The reference has only kpad_mask for variable lengths
# (src/attention.jl:16,83-89); this form skips padded queries as well as padded keys.

def _check_varlen(q, k, v, cu_q, cu_k):
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("packed q, k and v must be 3-dimensional (E, T, H) arrays")
    QH, Tq, E = q.shape
    KH, Tk, KE = k.shape
    if E != KE:
        raise ValueError(f"Embedding dim of Q `{E}` must be the same as of K `{KE}`.")
    if k.shape != v.shape:
        raise ValueError(f"Shapes of K `{jdims(k)}` and V `{jdims(v)}` must be the same.")
    if E <= 0 or (E & (E - 1)) != 0:
        raise ValueError("Only power-of-2 embedding dims are supported.")
    if KH == 0 or QH % KH != 0:
        raise ValueError(f"Number of query heads `{QH}` must be divisible by number of KV heads `{KH}`.")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k and v must share one element type")
    for name, cu in (("cu_seqlens_q", cu_q), ("cu_seqlens_k", cu_k)):
        if cu.dtype != torch.int32 or cu.dim() != 1 or cu.device != q.device:
            raise ValueError(f"{name} must be a 1-dimensional int32 tensor on the device of q")
    if cu_q.shape != cu_k.shape:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must have the same length (B + 1)")
    return QH, Tq, E, KH, Tk, cu_q.shape[0] - 1


def _flash_attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, max_seqlen_k: int, *,
                            causal: bool):
    """Forward over packed sequences; returns (o, ms, ls)."""
    q, k, v = (device_tensor(t, "flash_attention (varlen)") for t in (q, k, v))
    QH, Tq, E, KH, Tk, B = _check_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k)
    dt = attn_dtype_code(q, "flash_attention (varlen)")
    # Rows in no sequence (a packing buffer's tail, rows past max_seqlen_q) are not
    # written by the kernels: they start at zero (ls = 0 marks them as empty rows).
    o = torch.zeros_like(q)
    ms = torch.zeros((QH, Tq), dtype=torch.float32, device=q.device)
    ls = torch.zeros((QH, Tq), dtype=torch.float32, device=q.device)
    _lib.check(_lib.lib().onionop_flash_attn_varlen_fwd(
        stream_of(q), dt, E, Tq, Tk, QH, KH, B, ptr(cu_seqlens_q), ptr(cu_seqlens_k), int(max_seqlen_q),
        int(max_seqlen_k), ptr(q), ptr(k), ptr(v), int(bool(causal)), attention_scale(E, q.dtype), ptr(o), ptr(ms),
        ptr(ls)))
    return o, ms, ls


def grad_flash_attention_varlen(do, o, ms, ls, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int,
                                max_seqlen_k: int, *, causal: bool, qk_fp16: bool = True):
    """Backward over packed sequences; returns (dq, dk, dv)."""
    q, k, v, o = (device_tensor(t, "∇flash_attention (varlen)") for t in (q, k, v, o))
    do = device_tensor(do, "∇flash_attention (varlen)").to(q.dtype)
    QH, Tq, E, KH, Tk, B = _check_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k)
    if do.shape != q.shape or o.shape != q.shape:
        raise ValueError("Δ and o must have the shape of q")
    dt = attn_dtype_code(q, "∇flash_attention (varlen)")
    L = _lib.lib()
    ws_bytes = L.onionop_flash_attn_varlen_bwd_workspace(dt, E, Tq, QH)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=q.device)
    # Gradient rows of queries / keys in no sequence are not written: they are zero.
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    _lib.check(L.onionop_flash_attn_varlen_bwd(
        stream_of(q), dt, E, Tq, Tk, QH, KH, B, ptr(cu_seqlens_q), ptr(cu_seqlens_k), int(max_seqlen_q),
        int(max_seqlen_k), ptr(do), ptr(o), ptr(ms), ptr(ls), ptr(q), ptr(k), ptr(v), int(bool(causal)),
        attention_scale(E, q.dtype), int(bool(qk_fp16)), ptr(dq), ptr(dk), ptr(dv), ptr(ws), int(ws_bytes)))
    return dq, dk, dv


class _FlashAttentionVarlenFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu_q, cu_k, max_q, max_k, causal, qk_fp16):
        o, ms, ls = _flash_attention_varlen(q, k, v, cu_q, cu_k, max_q, max_k, causal=causal)
        ctx.save_for_backward(q, k, v, cu_q, cu_k, o, ms, ls)
        ctx.max_q, ctx.max_k, ctx.causal, ctx.qk_fp16 = max_q, max_k, causal, qk_fp16
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, cu_q, cu_k, o, ms, ls = ctx.saved_tensors
        dq, dk, dv = grad_flash_attention_varlen(do.contiguous(), o, ms, ls, q, k, v, cu_q, cu_k, ctx.max_q,
                                                 ctx.max_k, causal=ctx.causal, qk_fp16=ctx.qk_fp16)
        return dq, dk, dv, None, None, None, None, None, None


def flash_attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, max_seqlen_k: int, *,
                           causal: bool, qk_fp16: bool = True):
    """Flash attention over packed variable-length sequences (differentiable in q, k, v)."""
    return _FlashAttentionVarlenFn.apply(q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q),
                                         int(max_seqlen_k), bool(causal), bool(qk_fp16))


# ---------------------------------------------------------------- fused RoPE backward
#
# flash_attention(llama_rope(q, k; cos, sin)..., v): the forward runs llama_rope then the
# attention forward (the rotated q, k are kept for the backward, as the two rrules keep
# them); the backward is one launch sequence whose dQ and dK kernels apply ∇llama_rope to
# their float32 accumulators before storing, so no pass over dq and dk follows
# (onionop_flash_attn_bwd_rope).  The reference composes the two rrules
# (src/attention_crc.jl:16-31, src/rope/llama_rope.jl:94-98).

def grad_flash_attention_rope(do, o, ms, ls, qr, kr, v, cos, sin, pair=None, *, causal: bool, kpad_mask=None,
                              qk_fp16: bool = True):
    """Gradients (dq, dk, dv, dpair) w.r.t. q, k before the rotation; qr, kr are the rotated tensors."""
    qr, kr, v, o = (device_tensor(t, "∇flash_attention ∘ ∇llama_rope") for t in (qr, kr, v, o))
    do = device_tensor(do, "∇flash_attention ∘ ∇llama_rope").to(qr.dtype)
    ms, ls = (device_tensor(t, "∇flash_attention ∘ ∇llama_rope") for t in (ms, ls))
    cos = device_tensor(cos, "∇flash_attention ∘ ∇llama_rope").to(torch.float32).contiguous()
    sin = device_tensor(sin, "∇flash_attention ∘ ∇llama_rope").to(torch.float32).contiguous()
    pair = None if pair is None else device_tensor(pair, "∇flash_attention ∘ ∇llama_rope")
    kpad_mask = None if kpad_mask is None else device_tensor(kpad_mask, "∇flash_attention ∘ ∇llama_rope")
    B, QH, QL, E, KH, KL = _check_shapes(qr, kr, v, pair, kpad_mask)
    if cos.shape != (B, QL, E) or sin.shape != (B, QL, E):
        raise ValueError(f"cos/sin must have Julia shape {(E, QL, B)}")
    dt = attn_dtype_code(qr, "∇flash_attention ∘ ∇llama_rope")
    L = _lib.lib()
    ws_bytes = L.onionop_flash_attn_bwd_workspace(dt, E, QL, KL, QH, KH, B)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=qr.device)
    dq, dk, dv = torch.empty_like(qr), torch.empty_like(kr), torch.empty_like(v)
    dpair = None if pair is None else torch.empty_like(pair)
    _lib.check(L.onionop_flash_attn_bwd_rope(
        stream_of(qr), dt, E, QL, KL, QH, KH, B, ptr(do), ptr(o), ptr(ms), ptr(ls), ptr(qr), ptr(kr), ptr(v),
        ptr(pair), ptr(kpad_mask), ptr(cos), ptr(sin), int(bool(causal)), attention_scale(E, qr.dtype),
        int(bool(qk_fp16)), ptr(dq), ptr(dk), ptr(dv), ptr(dpair), ptr(ws), int(ws_bytes)))
    return dq, dk, dv, dpair


class _FlashAttentionRopeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cos, sin, pair, kpad_mask, causal, qk_fp16):
        from .rope import _llama_rope

        qr, kr = _llama_rope(q, k, cos, sin, bwd=False)
        o, ms, ls = _flash_attention(qr, kr, v, pair, causal=causal, kpad_mask=kpad_mask)
        ctx.save_for_backward(qr, kr, v, cos, sin, pair, kpad_mask, o, ms, ls)
        ctx.causal, ctx.qk_fp16 = causal, qk_fp16
        return o

    @staticmethod
    def backward(ctx, do):
        qr, kr, v, cos, sin, pair, kpad_mask, o, ms, ls = ctx.saved_tensors
        dq, dk, dv, dpair = grad_flash_attention_rope(do.contiguous(), o, ms, ls, qr, kr, v, cos, sin, pair,
                                                      causal=ctx.causal, kpad_mask=kpad_mask, qk_fp16=ctx.qk_fp16)
        return dq, dk, dv, None, None, dpair, None, None, None


def flash_attention_rope(q, k, v, cos, sin, pair: Optional[torch.Tensor] = None, *, causal: bool,
                         kpad_mask: Optional[torch.Tensor] = None, qk_fp16: bool = True):
    """flash_attention(llama_rope(q, k; cos, sin)..., v, pair; causal, kpad_mask), differentiable in
    q, k, v and pair, with ∇llama_rope fused into the attention backward."""
    return _FlashAttentionRopeFn.apply(q, k, v, cos, sin, pair, kpad_mask, bool(causal), bool(qk_fp16))


def grad_flash_attention_varlen_rope(do, o, ms, ls, qr, kr, v, cos, sin, cu_seqlens, max_seqlen: int, *,
                                     causal: bool, qk_fp16: bool = True):
    """Packed-sequence backward with the fused ∇llama_rope (q and k packed alike; cos / sin
    (Tq, E) float32, one row per packed position)."""
    what = "∇flash_attention ∘ ∇llama_rope (varlen)"
    qr, kr, v, o = (device_tensor(t, what) for t in (qr, kr, v, o))
    do = device_tensor(do, what).to(qr.dtype)
    ms, ls = device_tensor(ms, what), device_tensor(ls, what)
    cos = device_tensor(cos, what).to(torch.float32).contiguous()
    sin = device_tensor(sin, what).to(torch.float32).contiguous()
    QH, Tq, E, KH, Tk, B = _check_varlen(qr, kr, v, cu_seqlens, cu_seqlens)
    # one table row per packed position: (Tq, E), or (1, Tq, E) as LlamaRotaryEmbedding returns it
    if cos.numel() != Tq * E or sin.numel() != Tq * E or cos.shape[-2:] != (Tq, E) or sin.shape[-2:] != (Tq, E):
        raise ValueError(f"cos/sin must have Julia shape {(E, Tq)}")
    dt = attn_dtype_code(qr, what)
    L = _lib.lib()
    ws_bytes = L.onionop_flash_attn_varlen_bwd_workspace(dt, E, Tq, QH)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=qr.device)
    dq, dk, dv = torch.zeros_like(qr), torch.zeros_like(kr), torch.zeros_like(v)
    _lib.check(L.onionop_flash_attn_varlen_bwd_rope(
        stream_of(qr), dt, E, Tq, Tk, QH, KH, B, ptr(cu_seqlens), ptr(cu_seqlens), int(max_seqlen), int(max_seqlen),
        ptr(do), ptr(o), ptr(ms), ptr(ls), ptr(qr), ptr(kr), ptr(v), ptr(cos), ptr(sin), int(bool(causal)),
        attention_scale(E, qr.dtype), int(bool(qk_fp16)), ptr(dq), ptr(dk), ptr(dv), ptr(ws), int(ws_bytes)))
    return dq, dk, dv
