"""RMS norm and layer norm over the first Julia dimension, with their rrules.

x (n, emb) row-major == Julia (emb, n); w, b (emb).  Statistics (rstd, mu) are float32.
"""
from __future__ import annotations

import torch

from . import _lib
from ._util import device_tensor, dtype_code, ptr, stream_of


def _check_xw(x, w, what):
    if x.dim() != 2:
        raise ValueError(f"{what}: x must be a matrix (emb, n)")
    emb = x.shape[1]
    if w.dim() != 1 or w.shape[0] != emb:
        raise ValueError(f"{what}: weight length {tuple(w.shape)} does not match emb {emb}")
    return x.shape[0], emb


def _rms_norm(x, w, *, eps: float = 1e-6, offset: float = 0.0):
    """_rms_norm (src/rms_norm.jl:117-137) -> (y, rstd)."""
    x = device_tensor(x, "rms_norm")
    w = device_tensor(w, "rms_norm")
    n, emb = _check_xw(x, w, "rms_norm")
    y = torch.empty_like(x)
    rstd = torch.empty(n, dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().onionop_rms_norm_fwd(stream_of(x), dtype_code(x, "rms_norm"), dtype_code(w, "rms_norm"),
                                               emb, n, ptr(x), ptr(w), float(eps), float(offset), ptr(y),
                                               ptr(rstd)))
    return y, rstd


def grad_rms_norm(dy, rstd, x, w, *, offset: float = 0.0):
    """∇rms_norm (src/rms_norm.jl:139-169) -> (dx, dw) with dw float32."""
    x = device_tensor(x, "∇rms_norm")
    w = device_tensor(w, "∇rms_norm")
    dy = device_tensor(dy, "∇rms_norm").to(x.dtype)
    rstd = device_tensor(rstd, "∇rms_norm")
    n, emb = _check_xw(x, w, "∇rms_norm")
    L = _lib.lib()
    ws_bytes = int(L.onionop_rms_norm_bwd_workspace(emb, n))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    dx = torch.empty_like(x)
    dw = torch.empty(emb, dtype=torch.float32, device=x.device)
    _lib.check(L.onionop_rms_norm_bwd(stream_of(x), dtype_code(x, "∇rms_norm"), dtype_code(w, "∇rms_norm"), emb, n,
                                      ptr(dy), ptr(rstd), ptr(x), ptr(w), float(offset), ptr(dx), ptr(dw), ptr(ws),
                                      ws_bytes))
    return dx, dw


class _RmsNormFn(torch.autograd.Function):
    """rrule(_rms_norm) (src/rms_norm.jl:178-185)."""

    @staticmethod
    def forward(ctx, x, w, eps, offset):
        y, rstd = _rms_norm(x, w, eps=eps, offset=offset)
        ctx.save_for_backward(x, w, rstd)
        ctx.offset = offset
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, rstd = ctx.saved_tensors
        dx, dw = grad_rms_norm(dy.contiguous(), rstd, x, w, offset=ctx.offset)
        return dx, dw.to(w.dtype), None, None


def rms_norm(x, w, *, eps: float = 1e-6, offset: float = 0.0):
    """NNop.rms_norm (src/rms_norm.jl:171-176): (offset + w) .* x ./ sqrt.(mean(x.^2) .+ eps)."""
    return _RmsNormFn.apply(x, w, float(eps), float(offset))


def _layer_norm(x, w, b, *, eps: float = 1e-6):
    """_layer_norm (src/layer_norm.jl:150-170) -> (y, mu, rstd)."""
    x = device_tensor(x, "layer_norm")
    w = device_tensor(w, "layer_norm")
    b = device_tensor(b, "layer_norm").to(w.dtype)
    n, emb = _check_xw(x, w, "layer_norm")
    if b.shape != w.shape:
        raise ValueError("layer_norm: bias must have the shape of the weight")
    y = torch.empty_like(x)
    mu = torch.empty(n, dtype=torch.float32, device=x.device)
    rstd = torch.empty(n, dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().onionop_layer_norm_fwd(stream_of(x), dtype_code(x, "layer_norm"),
                                                 dtype_code(w, "layer_norm"), emb, n, ptr(x), ptr(w), ptr(b),
                                                 float(eps), ptr(y), ptr(mu), ptr(rstd)))
    return y, mu, rstd


def grad_layer_norm(dy, mu, rstd, x, w, b=None):
    """∇layer_norm (src/layer_norm.jl:172-204) -> (dx, dw, db), dw/db in w's element type."""
    x = device_tensor(x, "∇layer_norm")
    w = device_tensor(w, "∇layer_norm")
    dy = device_tensor(dy, "∇layer_norm").to(x.dtype)
    mu = device_tensor(mu, "∇layer_norm")
    rstd = device_tensor(rstd, "∇layer_norm")
    n, emb = _check_xw(x, w, "∇layer_norm")
    L = _lib.lib()
    ws_bytes = int(L.onionop_layer_norm_bwd_workspace(emb, n))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    db = torch.empty_like(w)
    _lib.check(L.onionop_layer_norm_bwd(stream_of(x), dtype_code(x, "∇layer_norm"), dtype_code(w, "∇layer_norm"),
                                        emb, n, ptr(dy), ptr(mu), ptr(rstd), ptr(x), ptr(w), ptr(dx), ptr(dw),
                                        ptr(db), ptr(ws), ws_bytes))
    return dx, dw, db


class _LayerNormFn(torch.autograd.Function):
    """rrule(_layer_norm) (src/layer_norm.jl:213-220)."""

    @staticmethod
    def forward(ctx, x, w, b, eps):
        y, mu, rstd = _layer_norm(x, w, b, eps=eps)
        ctx.save_for_backward(x, w, mu, rstd)
        ctx.b_dtype = b.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, mu, rstd = ctx.saved_tensors
        dx, dw, db = grad_layer_norm(dy.contiguous(), mu, rstd, x, w)
        return dx, dw, db.to(ctx.b_dtype), None


def layer_norm(x, w, b, *, eps: float = 1e-6):
    """NNop.layer_norm (src/layer_norm.jl:206-211): (x .- mu) ./ sqrt.(var .+ eps) .* w .+ b."""
    return _LayerNormFn.apply(x, w, b, float(eps))
