"""Seeded random sweep of the row kernels (softmax forward / backward / pullback, RMS norm
and layer norm forward / backward) against the oracle: row lengths at and around the
vector, workgroup and register-resident limits (and 1), ragged lengths that are not a
multiple of the 16-byte vector, vocabulary-sized rows, random row counts, float32 or
16-bit weights, RMS offsets, and rows with a large mean.  Every case prints its
parameters before it runs.  Tolerance: 1e-5 (float32), 2e-2 (16-bit) norm-wise relative
error against the float64 oracle.
"""
import numpy as np
import pytest
import torch

import nnop
import oracle
from helpers import DTYPES, TOL, host, make, rel_err

pytestmark = pytest.mark.gpu

EDGE = [1, 7, 8, 9, 255, 256, 257, 2047, 2048, 2049, 4095, 4096, 4097, 8191, 8192, 8193, 16383, 16384,
        16385, 32767, 32768, 32769, 50257]


def row_case(i):
    rng = np.random.default_rng(3000 + i)
    dt = ["f32", "f16", "bf16"][i % 3]
    n = int(rng.choice(EDGE)) if rng.random() < 0.6 else int(rng.integers(1, 70001))
    rows = int(rng.integers(1, max(2, min(40, 2_000_000 // n)) + 1))
    op = ["softmax", "rms", "ln"][(i // 3) % 3]
    if op == "rms" and n == 1:
        # one element: dx = rstd dy w eps / (x^2 + eps) exactly, but every float32 evaluation
        # (the reference's too) forms it as a difference of two terms equal to within
        # eps / x^2, so it is round-off; one element per row is covered by the layer norm
        n = 2
    wdt = "f32" if rng.random() < 0.3 else dt
    offset = float(rng.choice([0.0, 1.0])) if op == "rms" else 0.0
    shift = float(rng.choice([0.0, 0.0, 50.0])) if op == "ln" and dt == "f32" else 0.0
    return op, dt, wdt, n, rows, offset, shift, 3000 + i


CASES = [row_case(i) for i in range(90)]


def check(errs, tol):
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"tolerance {tol}: {bad} (all: {errs})"


@pytest.mark.parametrize("case", CASES, ids=lambda c: "{}-{}-w{}-n{}-r{}{}{}".format(
    c[0], c[1], c[2], c[3], c[4], f"-off{c[5]:g}" if c[5] else "", f"-shift{c[6]:g}" if c[6] else ""))
def test_random_rows(dev, case):
    op, dt, wdt, n, rows, offset, shift, seed = case
    dtype, wdtype = DTYPES[dt], DTYPES[wdt]
    tol = 1e-5 if dtype == torch.float32 else TOL[dtype]
    rng = np.random.default_rng(seed)
    print(f"rows {op} {dt} w={wdt} n={n} rows={rows} offset={offset} shift={shift} seed={seed}", flush=True)
    if op == "softmax":
        x, xn = make(rng, (rows, n), dtype, dev, scale=3.0)
        g, gn = make(rng, (rows, n), dtype, dev)
        gg, ggn = make(rng, (rows, n), dtype, dev)
        y = nnop._online_softmax(x)
        dx = nnop.grad_online_softmax(g, y)
        d_dy, d_y = nnop.grad_online_softmax_pullback(gg, g, y)
        torch.cuda.synchronize()
        yh = host(y)
        r_dy, r_y = oracle.softmax_bwd_bwd(ggn, gn, yh)
        check({"y": rel_err(yh, oracle.softmax_fwd(xn)), "dx": rel_err(host(dx), oracle.softmax_bwd(gn, yh)),
               "d_dy": rel_err(host(d_dy), r_dy), "d_y": rel_err(host(d_y), r_y)}, tol)
        return
    x, xn = make(rng, (rows, n), dtype, dev, offset=shift)
    w, wn = make(rng, (n,), wdtype, dev, scale=0.02, offset=1.0)
    g, gn = make(rng, (rows, n), dtype, dev)
    if op == "rms":
        y, rstd = nnop._rms_norm(x, w, offset=offset)
        dx, dw = nnop.grad_rms_norm(g, rstd, x, w, offset=offset)
        torch.cuda.synchronize()
        y_r, r_r = oracle.rms_norm_fwd(xn, wn, 1e-6, offset)
        dx_r, dw_r = oracle.rms_norm_bwd(gn, r_r, xn, wn, offset)
        check({"y": rel_err(host(y), y_r), "rstd": rel_err(host(rstd), r_r), "dx": rel_err(host(dx), dx_r),
               "dw": rel_err(host(dw), dw_r)}, tol)
        return
    b, bn = make(rng, (n,), wdtype, dev, scale=0.02)
    y, mu, rstd = nnop._layer_norm(x, w, b)
    dx, dw, db = nnop.grad_layer_norm(g, mu, rstd, x, w)
    torch.cuda.synchronize()
    y_r, mu_r, r_r = oracle.layer_norm_fwd(xn, wn, bn)
    dx_r, dw_r, db_r = oracle.layer_norm_bwd(gn, mu_r, r_r, xn, wn)
    # a large mean: x - mu carries the float32 rounding of mu (as in the large-mean test)
    ytol = 1e-3 if shift else tol
    check({"mu": rel_err(host(mu), mu_r), "rstd": rel_err(host(rstd), r_r), "dw": rel_err(host(dw), dw_r),
           "db": rel_err(host(db), db_r)}, tol if not shift else 1e-4)
    check({"y": rel_err(host(y), y_r), "dx": rel_err(host(dx), dx_r)}, ytol)
