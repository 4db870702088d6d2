"""Online softmax over the first Julia dimension: NNop.online_softmax and its rrule.

x (M, N) row-major == Julia (N, M); the softmax runs along N for each of the M columns.
"""
from __future__ import annotations

import torch

from . import _lib
from ._util import device_tensor, dtype_code, ptr, stream_of


def _as_matrix(x):
    if x.dim() == 1:
        return x.reshape(1, -1)
    return x.reshape(-1, x.shape[-1])


def _online_softmax(x):
    """online_softmax (src/softmax.jl:60-68); y has x's element type."""
    x = device_tensor(x, "online_softmax")
    dt = dtype_code(x, "online_softmax")
    xm = _as_matrix(x)
    y = torch.empty_like(x)
    M, N = xm.shape
    _lib.check(_lib.lib().onionop_softmax_fwd(stream_of(x), dt, N, M, ptr(x), ptr(y)))
    return y


def grad_online_softmax(dy, y):
    """∇online_softmax (src/softmax.jl:70-80): dy .* y - y .* sum(dy .* y; dims=1)."""
    y = device_tensor(y, "∇online_softmax")
    dy = device_tensor(dy, "∇online_softmax").to(y.dtype)
    if dy.shape != y.shape:
        raise ValueError("Δ must have the shape of y")
    dt = dtype_code(y, "∇online_softmax")
    M, N = _as_matrix(y).shape
    dx = torch.empty_like(y)
    _lib.check(_lib.lib().onionop_softmax_bwd(stream_of(y), dt, N, M, ptr(dy), ptr(y), ptr(dx)))
    return dx


def grad_online_softmax_pullback(g, dy, y):
    """Pullback of ∇online_softmax for second derivatives (the reference keeps them through
    its within_gradient branch, src/softmax.jl:71-74): for g = dL/d(dx),
    returns (d_dy, d_y) = (y (g - u), g (dy - s) - dy u), s = sum(dy y), u = sum(g y)."""
    y = device_tensor(y, "∇online_softmax pullback")
    dy = device_tensor(dy, "∇online_softmax pullback").to(y.dtype)
    g = device_tensor(g, "∇online_softmax pullback").to(y.dtype)
    if dy.shape != y.shape or g.shape != y.shape:
        raise ValueError("g and Δ must have the shape of y")
    dt = dtype_code(y, "∇online_softmax pullback")
    M, N = _as_matrix(y).shape
    d_dy, d_y = torch.empty_like(y), torch.empty_like(y)
    _lib.check(_lib.lib().onionop_softmax_bwd_bwd(stream_of(y), dt, N, M, ptr(g), ptr(dy), ptr(y), ptr(d_dy),
                                                  ptr(d_y)))
    return d_dy, d_y


class _GradOnlineSoftmaxFn(torch.autograd.Function):
    """∇online_softmax as a differentiable operation (its own pullback on the GPU)."""

    @staticmethod
    def forward(ctx, dy, y):
        ctx.save_for_backward(dy, y)
        return grad_online_softmax(dy, y)

    @staticmethod
    def backward(ctx, g):
        dy, y = ctx.saved_tensors
        return grad_online_softmax_pullback(g.contiguous(), dy, y)


class _OnlineSoftmaxFn(torch.autograd.Function):
    """rrule(online_softmax) (src/softmax.jl:82-86); its backward is itself differentiable."""

    @staticmethod
    def forward(ctx, x):
        y = _online_softmax(x)
        ctx.save_for_backward(y)
        return y

    @staticmethod
    def backward(ctx, dy):
        (y,) = ctx.saved_tensors
        return _GradOnlineSoftmaxFn.apply(dy.contiguous(), y)


def online_softmax(x):
    """NNop.online_softmax: softmax over the contiguous (Julia first) dimension."""
    return _OnlineSoftmaxFn.apply(x)
