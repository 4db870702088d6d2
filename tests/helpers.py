"""Shared test helpers: seeded inputs rounded to a dtype, and norm-wise relative error."""
from __future__ import annotations

import numpy as np
import torch

TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}
DTYPES = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def make(rng, shape, dtype, dev, kind="normal", scale=1.0, offset=0.0):
    """Seeded input: (device tensor of `dtype`, the same values as float64 numpy)."""
    x = rng.standard_normal(shape) if kind == "normal" else rng.random(shape)
    x = x * scale + offset
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dtype)
    return (t.to(dev) if dev is not None else t), t.double().numpy()


def host(t):
    return t.detach().double().cpu().numpy()


def rel_err(a, b):
    """||a - b|| / ||b|| over all elements (both as float64 arrays)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    nb = np.linalg.norm(b)
    if nb == 0.0:
        return float(np.linalg.norm(a))
    return float(np.linalg.norm(a - b) / nb)
