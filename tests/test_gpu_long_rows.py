"""GPU parity of softmax and the norms on rows longer than a workgroup's registers hold.

The reference loops over any reduction length (n_loop_iters, src/softmax.jl:204-253;
src/rms_norm.jl:3-38,43-115; src/layer_norm.jl:8-63,65-148).  Rows beyond 16384 float32 /
32768 16-bit elements (16-byte aligned rows), or beyond 4096 elements when rows are not
16-byte aligned, run on the streaming kernels; the lengths here sit on both sides of those
limits, at vocabulary sizes (32000, 50257, 128256), and with whole -inf chunks at the start
of a row (the online (max, sum) merge must ignore them).  Checked against the oracle in
float64 on the same rounded values: norm-wise relative error <= 1e-5 (float32),
<= 2e-2 (float16, bfloat16).
"""
import numpy as np
import pytest
import torch

import nnop
import oracle
from helpers import DTYPES, TOL, host, make, rel_err

pytestmark = pytest.mark.gpu


def check(errs, tol):
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"tolerance {tol}: {bad} (all: {errs})"


def tol_of(dtype):
    return 1e-5 if dtype == torch.float32 else TOL[dtype]


SOFTMAX_CASES = [
    ("f32", 16384), ("f32", 16385), ("f32", 32000), ("f32", 50257), ("bf16", 4097), ("bf16", 32768),
    ("bf16", 32776), ("bf16", 50257), ("bf16", 128256), ("f16", 128256), ("f16", 40001),
]


@pytest.mark.parametrize("dt,n", SOFTMAX_CASES, ids=lambda c: str(c))
def test_softmax_long(dev, dt, n):
    dtype = DTYPES[dt]
    rng = np.random.default_rng(n)
    rows = 3
    print(f"softmax long rows: {dt} n={n} rows={rows}", flush=True)
    x, xn = make(rng, (rows, n), dtype, dev, scale=3.0)
    g, gn = make(rng, (rows, n), dtype, dev)
    gg, ggn = make(rng, (rows, n), dtype, dev)
    y = nnop._online_softmax(x)
    dx = nnop.grad_online_softmax(g, y)
    d_dy, d_y = nnop.grad_online_softmax_pullback(gg, g, y)
    torch.cuda.synchronize()
    yh = host(y)
    y_r = oracle.softmax_fwd(xn)
    r_dy, r_y = oracle.softmax_bwd_bwd(ggn, gn, yh)
    check({"y": rel_err(yh, y_r), "dx": rel_err(host(dx), oracle.softmax_bwd(gn, yh)),
           "d_dy": rel_err(host(d_dy), r_dy), "d_y": rel_err(host(d_y), r_y)}, tol_of(dtype))
    assert np.allclose(yh.sum(-1), 1.0, atol=1e-4 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_softmax_long_masked_prefix(dev, dt):
    """Rows whose first chunks are all -inf (masked logits), then finite values."""
    dtype = DTYPES[dt]
    n = 70000
    rng = np.random.default_rng(5)
    x64 = rng.standard_normal((2, n)) * 2.0
    x64[0, :20000] = -np.inf
    x64[1, 1::2] = -np.inf
    x = torch.from_numpy(x64).to(dtype).to(dev)
    y = nnop._online_softmax(x)
    torch.cuda.synchronize()
    xr = x.double().cpu().numpy()
    check({"y": rel_err(host(y), oracle.softmax_fwd(xr))}, tol_of(dtype))
    assert (host(y)[0, :20000] == 0).all()


NORM_CASES = [
    # dt, emb, n: in-register (5000 bf16 is 16-byte aligned) and streaming (the rest)
    ("bf16", 5000, 33), ("bf16", 5001, 33), ("bf16", 40000, 9), ("f32", 16385, 7), ("f32", 20000, 7),
    ("f16", 4100, 13), ("bf16", 32776, 5),
]


@pytest.mark.parametrize("dt,emb,n", NORM_CASES, ids=lambda c: str(c))
def test_norms_long(dev, dt, emb, n):
    dtype = DTYPES[dt]
    rng = np.random.default_rng(emb + n)
    print(f"norms long rows: {dt} emb={emb} n={n}", flush=True)
    x, xn = make(rng, (n, emb), dtype, dev)
    w, wn = make(rng, (emb,), dtype, dev, scale=0.02, offset=1.0)
    b, bn = make(rng, (emb,), dtype, dev, scale=0.02)
    dy, dyn = make(rng, (n, emb), dtype, dev)
    y, rstd = nnop._rms_norm(x, w, offset=0.5)
    dx, dw = nnop.grad_rms_norm(dy, rstd, x, w, offset=0.5)
    torch.cuda.synchronize()
    y_r, r_r = oracle.rms_norm_fwd(xn, wn, 1e-6, 0.5)
    dx_r, dw_r = oracle.rms_norm_bwd(dyn, r_r, xn, wn, 0.5)
    tol = tol_of(dtype)
    check({"rms y": rel_err(host(y), y_r), "rms rstd": rel_err(host(rstd), r_r), "rms dx": rel_err(host(dx), dx_r),
           "rms dw": rel_err(host(dw), dw_r)}, tol)
    y, mu, rstd = nnop._layer_norm(x, w, b)
    dx, dw, db = nnop.grad_layer_norm(dy, mu, rstd, x, w, b)
    torch.cuda.synchronize()
    y_r, mu_r, r_r = oracle.layer_norm_fwd(xn, wn, bn)
    dx_r, dw_r, db_r = oracle.layer_norm_bwd(dyn, mu_r, r_r, xn, wn)
    check({"ln y": rel_err(host(y), y_r), "ln mu": rel_err(host(mu), mu_r), "ln rstd": rel_err(host(rstd), r_r),
           "ln dx": rel_err(host(dx), dx_r), "ln dw": rel_err(host(dw), dw_r), "ln db": rel_err(host(db), db_r)},
          tol)


def test_norms_long_weight_dtype(dev):
    """bf16 rows with float32 weights on the streaming path (the weight type is separate)."""
    rng = np.random.default_rng(9)
    emb, n = 33000, 4
    x, xn = make(rng, (n, emb), torch.bfloat16, dev)
    w, wn = make(rng, (emb,), torch.float32, dev, scale=0.02, offset=1.0)
    dy, dyn = make(rng, (n, emb), torch.bfloat16, dev)
    y, rstd = nnop._rms_norm(x, w)
    dx, dw = nnop.grad_rms_norm(dy, rstd, x, w)
    torch.cuda.synchronize()
    y_r, r_r = oracle.rms_norm_fwd(xn, wn)
    dx_r, dw_r = oracle.rms_norm_bwd(dyn, r_r, xn, wn)
    check({"y": rel_err(host(y), y_r), "dx": rel_err(host(dx), dx_r), "dw": rel_err(host(dw), dw_r)}, 2e-2)
