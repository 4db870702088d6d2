"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every committed fixture (regression pin).
GPU: the HIP kernels reproduce the committed expected outputs at the dtype tolerance.
"""
import glob
import os

import numpy as np
import pytest

import oracle
from helpers import rel_err

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATTN = sorted(glob.glob(os.path.join(GOLDEN, "attn_*.npz")))
TOLS = {"f32": 1e-5, "f16": 2e-2, "bf16": 2e-2}


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _attn_args(g):
    B, QH, KH, QL, KL, E, causal = (int(x) for x in g["meta"])
    return dict(pair=g.get("pair"), kpad=g.get("kpad"), causal=bool(causal), scale=float(g["scale"][0]))


def test_fixtures_present():
    assert len(ATTN) == 4
    for n in ("softmax_bf16", "rms_norm_bf16", "layer_norm_bf16", "llama_rope_bf16"):
        assert os.path.exists(os.path.join(GOLDEN, n + ".npz"))


@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_oracle_reproduces_attention_fixture(path):
    g = load(path)
    a = _attn_args(g)
    o, ms, ls = oracle.attn_fwd(g["q"], g["k"], g["v"], a["pair"], a["kpad"], a["causal"], a["scale"])
    dq, dk, dv, dp = oracle.attn_bwd(g["do"], g["q"], g["k"], g["v"], a["pair"], a["kpad"], a["causal"], a["scale"])
    for got, name in ((o, "o"), (ls, "ls"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert rel_err(got, g[name]) < 1e-6, name
    if dp is not None:
        assert rel_err(dp, g["dpair"]) < 1e-6


def test_oracle_reproduces_rowwise_fixtures():
    s = load(os.path.join(GOLDEN, "softmax_bf16.npz"))
    assert rel_err(oracle.softmax_fwd(s["x"]), s["y"]) < 1e-6
    assert rel_err(oracle.softmax_bwd(s["dy"], s["y"]), s["dx"]) < 1e-6
    r = load(os.path.join(GOLDEN, "rms_norm_bf16.npz"))
    y, rs = oracle.rms_norm_fwd(r["x"], r["w"])
    dx, dw = oracle.rms_norm_bwd(r["dy"], r["rstd"], r["x"], r["w"])
    assert max(rel_err(y, r["y"]), rel_err(rs, r["rstd"]), rel_err(dx, r["dx"]), rel_err(dw, r["dw"])) < 1e-6
    n = load(os.path.join(GOLDEN, "layer_norm_bf16.npz"))
    y, mu, rs = oracle.layer_norm_fwd(n["x"], n["w"], n["b"])
    dx, dw, db = oracle.layer_norm_bwd(n["dy"], n["mu"], n["rstd"], n["x"], n["w"])
    assert max(rel_err(y, n["y"]), rel_err(dx, n["dx"]), rel_err(dw, n["dw"]), rel_err(db, n["db"])) < 1e-6
    p = load(os.path.join(GOLDEN, "llama_rope_bf16.npz"))
    c, s_ = oracle.rotary_embedding(64, p["pos"], mode=oracle.FAITHFUL)
    assert np.abs(c - p["cos"]).max() < 1e-6 and np.abs(s_ - p["sin"]).max() < 1e-6
    qo, ko = oracle.llama_rope(p["q"], p["k"], p["cos"], p["sin"], 1.0)
    assert rel_err(qo, p["qo"]) < 1e-6 and rel_err(ko, p["ko"]) < 1e-6


# ------------------------------------------------------------------ GPU

def _dev(a, dtype, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_gpu_attention_fixture(dev, path):
    import torch

    import nnop

    g = load(path)
    dt = str(g["dtype"][0])
    dtype = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dt]
    a = _attn_args(g)
    q, k, v, do = (_dev(g[n], dtype, dev) for n in ("q", "k", "v", "do"))
    pair = _dev(a["pair"], dtype, dev) if a["pair"] is not None else None
    kpad = torch.from_numpy(a["kpad"]).to(dev) if a["kpad"] is not None else None
    print(f"fixture {os.path.basename(path)}", flush=True)
    o, ms, ls = nnop._flash_attention(q, k, v, pair, causal=a["causal"], kpad_mask=kpad)
    dq, dk, dv, dp = nnop.grad_flash_attention(do, o, ms, ls, q, k, v, pair, causal=a["causal"], kpad_mask=kpad,
                                               qk_fp16=False)
    torch.cuda.synchronize()
    tol = TOLS[dt]
    h = lambda t: t.double().cpu().numpy()  # noqa: E731
    errs = {n: rel_err(h(t), g[n]) for n, t in (("o", o), ("ls", ls), ("dq", dq), ("dk", dk), ("dv", dv))}
    if dp is not None:
        errs["dpair"] = rel_err(h(dp), g["dpair"])
    assert all(e <= tol for e in errs.values()), errs


@pytest.mark.gpu
def test_gpu_rowwise_fixtures(dev):
    import torch

    import nnop

    bf = torch.bfloat16
    h = lambda t: t.double().cpu().numpy()  # noqa: E731
    s = load(os.path.join(GOLDEN, "softmax_bf16.npz"))
    y = nnop._online_softmax(_dev(s["x"], bf, dev))
    dx = nnop.grad_online_softmax(_dev(s["dy"], bf, dev), y)
    r = load(os.path.join(GOLDEN, "rms_norm_bf16.npz"))
    yr, rs = nnop._rms_norm(_dev(r["x"], bf, dev), _dev(r["w"], bf, dev))
    dxr, dwr = nnop.grad_rms_norm(_dev(r["dy"], bf, dev), rs, _dev(r["x"], bf, dev), _dev(r["w"], bf, dev))
    n = load(os.path.join(GOLDEN, "layer_norm_bf16.npz"))
    yl, mu, rl = nnop._layer_norm(_dev(n["x"], bf, dev), _dev(n["w"], bf, dev), _dev(n["b"], bf, dev))
    dxl, dwl, dbl = nnop.grad_layer_norm(_dev(n["dy"], bf, dev), mu, rl, _dev(n["x"], bf, dev),
                                         _dev(n["w"], bf, dev))
    p = load(os.path.join(GOLDEN, "llama_rope_bf16.npz"))
    qo, ko = nnop._llama_rope(_dev(p["q"], bf, dev), _dev(p["k"], bf, dev), _dev(p["cos"], torch.float32, dev),
                              _dev(p["sin"], torch.float32, dev), bwd=False)
    torch.cuda.synchronize()
    errs = {"softmax_y": rel_err(h(y), s["y"]), "softmax_dx": rel_err(h(dx), s["dx"]),
            "rms_y": rel_err(h(yr), r["y"]), "rms_dx": rel_err(h(dxr), r["dx"]), "rms_dw": rel_err(h(dwr), r["dw"]),
            "ln_y": rel_err(h(yl), n["y"]), "ln_dx": rel_err(h(dxl), n["dx"]), "ln_dw": rel_err(h(dwl), n["dw"]),
            "ln_db": rel_err(h(dbl), n["db"]), "rope_q": rel_err(h(qo), p["qo"]), "rope_k": rel_err(h(ko), p["ko"])}
    assert all(e <= 2e-2 for e in errs.values()), errs
