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


class _OnlineSoftmaxFn(torch.autograd.Function):
    """rrule(online_softmax) (src/softmax.jl:82-86)."""

    @staticmethod
    def forward(ctx, x):
        y = _online_softmax(x)
        ctx.save_for_backward(y)
        return y

    @staticmethod
    def backward(ctx, dy):
        (y,) = ctx.saved_tensors
        return grad_online_softmax(dy.contiguous(), y)


def online_softmax(x):
    """NNop.online_softmax: softmax over the contiguous (Julia first) dimension."""
    return _OnlineSoftmaxFn.apply(x)
