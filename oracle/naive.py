"""numpy restatements of the reference's *test-side* naive formulas -- TEST INFRASTRUCTURE.

These are the reference's own definition of "correct" (it compares every fused op to
them), written independently of ``oracle.c`` so the two can pin each other.  Same array
convention as the ``oracle`` package (row-major memory == the Julia column-major arrays).
"""
from __future__ import annotations

import numpy as np


def softmax(x, axis=-1):
    """naive_softmax (test/softmax_tests.jl:6-10, test/attention_testsetup.jl:10-14)."""
    mx = np.max(x, axis=axis, keepdims=True)
    t = np.exp(x - mx)
    return t / np.sum(t, axis=axis, keepdims=True)


def attention(q, k, v, pair=None, kpad=None, causal=False, scale=None):
    """naive_attention (test/attention_testsetup.jl:21-45).

    q (B, QH, QL, E), k/v (B, KH, KL, E), pair (B, KL, QL, QH), kpad (B, KL) bool.
    GQA repeats each kv head QH/KH times (:23-30); the causal mask keeps key <= query
    (NNlib.make_causal_mask); kpad adds log(mask) (:16-19); pair is added after the
    scale (:41-43).  Masks are -inf, so fully masked rows give NaN as in the reference.
    """
    B, QH, QL, E = q.shape
    KH, KL = k.shape[1], k.shape[2]
    if QH != KH:
        rep = QH // KH
        k = np.repeat(k, rep, axis=1)
        v = np.repeat(v, rep, axis=1)
    if scale is None:
        scale = 1.0 / np.sqrt(E)
    a = np.einsum("bhie,bhje->bhij", q, k) * scale
    if causal:
        i = np.arange(QL)[:, None]
        j = np.arange(KL)[None, :]
        a = np.where(j <= i, a, -np.inf)
    if kpad is not None:
        with np.errstate(divide="ignore"):
            a = a + np.log(np.asarray(kpad, dtype=np.float64))[:, None, None, :]
    if pair is not None:
        a = a + np.transpose(pair, (0, 3, 2, 1))
    with np.errstate(invalid="ignore"):
        p = softmax(a, axis=-1)
    return np.einsum("bhij,bhje->bhie", p, v)


def rms_norm(x, w, offset=0.0, eps=1e-6):
    """naive_rms_norm (test/rmsnorm_tests.jl:7-9); x (n, emb)."""
    return (w + offset) * x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def layer_norm(x, w, b, eps=1e-6):
    """naive_layer_norm (test/layernorm_tests.jl:7-11), biased variance; x (n, emb)."""
    mu = np.mean(x, axis=-1, keepdims=True)
    var = np.mean((x - mu) ** 2, axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def rotate_half(x):
    """rotate_half (test/rope_tests.jl:6-11): vcat(-x2, x1) along the embedding axis."""
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def llama_rope(q, k, cos, sin):
    """naive_llama_rope (test/rope_tests.jl:13-19); q (B, QH, L, E), cos/sin (B, L, E)."""
    c = cos[:, None]
    s = sin[:, None]
    return q * c + rotate_half(q) * s, k * c + rotate_half(k) * s
