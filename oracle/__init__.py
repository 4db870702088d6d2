"""CPU oracle for NNop's fused-kernel hot path -- TEST INFRASTRUCTURE ONLY.

Only tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this package, and only to check results against.  The product (``nnop`` and
``libonionop_hip.so``) never calls it.

Two layers:
  * ``liboracle.so`` (``oracle.c``): C restatement of the reference algorithms, in an
    EXACT float64 mode and a FAITHFUL float32 mode that replays the reference's own
    tiling and rounding (see the header of ``oracle.c``).
  * ``naive``: numpy restatements of the reference *test-side* naive formulas
    (test/attention_testsetup.jl:10-45, test/softmax_tests.jl:6-10,
    test/rmsnorm_tests.jl:7-9, test/layernorm_tests.jl:7-11, test/rope_tests.jl:6-19),
    used to cross-check the C oracle.

Array convention: every function takes and returns numpy arrays in row-major order
whose memory equals the reference's column-major Julia arrays, i.e. a Julia array
(E, L, H, B) is a numpy array of shape (B, H, L, E).  In that order:
  q (B, QH, QL, E); k, v (B, KH, KL, E); pair (B, KL, QL, QH); kpad (B, KL) bool;
  ms, ls (B, QH, QL); softmax x (M, N) reduced over the last axis; norm x (n, emb);
  rope q (B, QH, L, E), cos/sin (B, L, E).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import naive  # noqa: F401  (re-exported)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

EXACT, FAITHFUL = 0, 1

_dp = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile beside this file."""
    import subprocess

    args = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_round_f16.restype = ctypes.c_float
        L.orc_round_f16.argtypes = [ctypes.c_float]
        L.orc_round_bf16.restype = ctypes.c_float
        L.orc_round_bf16.argtypes = [ctypes.c_float]
        L.orc_round_array.argtypes = [ctypes.c_int, _i64, _dp, _dp]
        L.orc_softmax_fwd.argtypes = [ctypes.c_int, _i64, _i64, _dp, _dp]
        L.orc_softmax_bwd.argtypes = [ctypes.c_int, _i64, _i64, _dp, _dp, _dp]
        L.orc_softmax_bwd_bwd.argtypes = [_i64, _i64, _dp, _dp, _dp, _dp, _dp]
        L.orc_rms_fwd.argtypes = [ctypes.c_int, _i64, _i64, _dp, _dp, ctypes.c_double,
                                  ctypes.c_double, _dp, _dp]
        L.orc_rms_bwd.argtypes = [ctypes.c_int, _i64, _i64, _dp, _dp, _dp, _dp,
                                  ctypes.c_double, _dp, _dp]
        L.orc_ln_fwd.argtypes = [ctypes.c_int, _i64, _i64, _dp, _dp, _dp, ctypes.c_double,
                                 _dp, _dp, _dp]
        L.orc_ln_bwd.argtypes = [ctypes.c_int, _i64, _i64, _dp, _dp, _dp, _dp, _dp,
                                 _dp, _dp, _dp]
        L.orc_rotary_embedding.argtypes = [ctypes.c_int, _i64, ctypes.c_double, _i64, _i64,
                                           _dp, _dp, _dp]
        L.orc_rope.argtypes = [ctypes.c_int, _i64, _i64, _i64, _i64, _i64, _dp, _dp, _dp,
                               _dp, ctypes.c_double, _dp, _dp]
        L.orc_attn_fwd.argtypes = [ctypes.c_int, _i64, _i64, _i64, _i64, _i64, _i64, _dp, _dp,
                                   _dp, _dp, _u8p, ctypes.c_int, ctypes.c_double, ctypes.c_int,
                                   _dp, _dp, _dp]
        L.orc_attn_bwd.argtypes = [ctypes.c_int, _i64, _i64, _i64, _i64, _i64, _i64, _dp, _dp,
                                   _dp, _dp, _dp, _dp, _dp, _dp, _u8p, ctypes.c_int,
                                   ctypes.c_double, ctypes.c_int, ctypes.c_int, _dp, _dp, _dp,
                                   _dp]
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_get_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _d(a):
    """Contiguous float64 copy (or view) and its ctypes pointer."""
    a = np.ascontiguousarray(a, dtype=np.float64)
    return a, a.ctypes.data_as(_dp)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_dp)


def set_threads(n: int) -> int:
    lib().orc_set_threads(int(n))
    return lib().orc_get_threads()


def round_to(kind: str, x):
    """Round values to float32 / float16 / bfloat16 (ties to even), returned as float64."""
    code = {"f32": 0, "f16": 1, "bf16": 2}[kind]
    x, px = _d(x)
    out = np.empty_like(x)
    lib().orc_round_array(code, x.size, px, out.ctypes.data_as(_dp))
    return out


# ------------------------------------------------------------------ softmax

def softmax_fwd(x, mode=EXACT):
    x, px = _d(x)
    M, N = (1, x.shape[0]) if x.ndim == 1 else x.shape
    y = np.empty_like(x)
    lib().orc_softmax_fwd(mode, N, M, px, _ptr(y))
    return y


def softmax_bwd(dy, y, mode=EXACT):
    dy, pdy = _d(dy)
    y, py = _d(y)
    M, N = (1, y.shape[0]) if y.ndim == 1 else y.shape
    dx = np.empty_like(y)
    lib().orc_softmax_bwd(mode, N, M, pdy, py, _ptr(dx))
    return dx


def softmax_bwd_bwd(g, dy, y):
    """Pullback of softmax_bwd(dy, y) for upstream gradient g: (d_dy, d_y), float64."""
    g, pg = _d(g)
    dy, pdy = _d(dy)
    y, py = _d(y)
    M, N = (1, y.shape[0]) if y.ndim == 1 else y.shape
    d_dy, d_y = np.empty_like(y), np.empty_like(y)
    lib().orc_softmax_bwd_bwd(N, M, pg, pdy, py, _ptr(d_dy), _ptr(d_y))
    return d_dy, d_y


# ------------------------------------------------------------------ norms

def rms_norm_fwd(x, w, eps=1e-6, offset=0.0, mode=EXACT):
    x, px = _d(x)
    w, pw = _d(w)
    n, emb = x.shape
    y = np.empty_like(x)
    rstd = np.empty(n)
    lib().orc_rms_fwd(mode, emb, n, px, pw, eps, offset, _ptr(y), _ptr(rstd))
    return y, rstd


def rms_norm_bwd(dy, rstd, x, w, offset=0.0, mode=EXACT):
    dy, pdy = _d(dy)
    rstd, pr = _d(rstd)
    x, px = _d(x)
    w, pw = _d(w)
    n, emb = x.shape
    dx = np.empty_like(x)
    dw = np.empty(emb)
    lib().orc_rms_bwd(mode, emb, n, pdy, pr, px, pw, offset, _ptr(dx), _ptr(dw))
    return dx, dw


def layer_norm_fwd(x, w, b, eps=1e-6, mode=EXACT):
    x, px = _d(x)
    w, pw = _d(w)
    b, pb = _d(b)
    n, emb = x.shape
    y = np.empty_like(x)
    mu = np.empty(n)
    rstd = np.empty(n)
    lib().orc_ln_fwd(mode, emb, n, px, pw, pb, eps, _ptr(y), _ptr(mu), _ptr(rstd))
    return y, mu, rstd


def layer_norm_bwd(dy, mu, rstd, x, w, mode=EXACT):
    dy, pdy = _d(dy)
    mu, pm = _d(mu)
    rstd, pr = _d(rstd)
    x, px = _d(x)
    w, pw = _d(w)
    n, emb = x.shape
    dx = np.empty_like(x)
    dw = np.empty(emb)
    db = np.empty(emb)
    lib().orc_ln_bwd(mode, emb, n, pdy, pm, pr, px, pw, _ptr(dx), _ptr(dw), _ptr(db))
    return dx, dw, db


# ------------------------------------------------------------------ RoPE

def rotary_embedding(dim, positions, base=10000.0, mode=FAITHFUL):
    """LlamaRotaryEmbedding(dim)(positions): positions (B, L) -> cos, sin (B, L, dim)."""
    pos, pp = _d(positions)
    if pos.ndim == 1:
        pos = pos[None, :]
        pos, pp = _d(pos)
    B, L = pos.shape
    c = np.empty((B, L, dim))
    s = np.empty((B, L, dim))
    lib().orc_rotary_embedding(mode, dim, base, L, B, pp, _ptr(c), _ptr(s))
    return c, s


def llama_rope(q, k, cos, sin, sin_sign=1.0, mode=EXACT):
    q, pq = _d(q)
    k, pk = _d(k)
    cos, pc = _d(cos)
    sin, ps = _d(sin)
    B, QH, L, E = q.shape
    KH = k.shape[1]
    qo = np.empty_like(q)
    ko = np.empty_like(k)
    lib().orc_rope(mode, E, L, QH, KH, B, pq, pk, pc, ps, sin_sign, _ptr(qo), _ptr(ko))
    return qo, ko


# ------------------------------------------------------------------ attention

def _kpad(kpad):
    if kpad is None:
        return None, None
    kp = np.ascontiguousarray(kpad, dtype=np.uint8)
    return kp, kp.ctypes.data_as(_u8p)


def attn_fwd(q, k, v, pair=None, kpad=None, causal=False, scale=None, mode=EXACT, gsz=64):
    """Returns (o, ms, ls) with o (B, QH, QL, E), ms/ls (B, QH, QL)."""
    q, pq = _d(q)
    k, pk = _d(k)
    v, pv = _d(v)
    B, QH, QL, E = q.shape
    KH, KL = k.shape[1], k.shape[2]
    if scale is None:
        scale = 1.0 / np.sqrt(E)
    pr = None
    if pair is not None:
        pair, pr = _d(pair)
    kp, pkp = _kpad(kpad)
    o = np.empty_like(q)
    ms = np.empty((B, QH, QL))
    ls = np.empty((B, QH, QL))
    lib().orc_attn_fwd(mode, E, QL, KL, QH, KH, B, pq, pk, pv, pr, pkp, int(causal),
                       float(scale), int(gsz), _ptr(o), _ptr(ms), _ptr(ls))
    return o, ms, ls


def attn_bwd(dO, q, k, v, pair=None, kpad=None, causal=False, scale=None, mode=EXACT,
             o=None, ms=None, ls=None, gsz=64, qk_fp16=False):
    """Returns (dq, dk, dv, dpair|None).  FAITHFUL mode needs o, ms, ls of a FAITHFUL fwd."""
    dO, pdo = _d(dO)
    q, pq = _d(q)
    k, pk = _d(k)
    v, pv = _d(v)
    B, QH, QL, E = q.shape
    KH, KL = k.shape[1], k.shape[2]
    if scale is None:
        scale = 1.0 / np.sqrt(E)
    pr = None
    if pair is not None:
        pair, pr = _d(pair)
    kp, pkp = _kpad(kpad)
    po = pms = pls = None
    if mode == FAITHFUL:
        o, po = _d(o)
        ms, pms = _d(ms)
        ls, pls = _d(ls)
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dv = np.empty_like(v)
    dpair = np.empty_like(pair) if pair is not None else None
    lib().orc_attn_bwd(mode, E, QL, KL, QH, KH, B, pdo, po, pms, pls, pq, pk, pv, pr, pkp,
                       int(causal), float(scale), int(gsz), int(qk_fp16), _ptr(dq), _ptr(dk),
                       _ptr(dv), _ptr(dpair))
    return dq, dk, dv, dpair
