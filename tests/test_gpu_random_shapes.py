"""Seeded random sweep of attention shapes against the oracle, to reach combinations the
fixed sweeps do not list: lengths at and around the 32 / 64 / 128-row tile edges (and 1),
query and key lengths that differ, GQA ratios, random key-padding masks (including a
batch whose keys are all masked), pair bias, causal, Float16 Q/K in the float32
backward, float32 through bf16x6 products, E = 256, pair-biased calls on grids small
enough for the backward's range splits, and packed sequences with empty ones.  Every case prints its parameters before it runs.  Tolerance as everywhere: 1e-5 (float32), 2e-2 (16-bit) norm-wise relative
error against the float64 oracle.
"""
import contextlib

import numpy as np
import pytest

import nnop
from test_gpu_attention import run_case
from test_gpu_varlen import run_varlen

pytestmark = pytest.mark.gpu

EDGE_LENGTHS = [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257]


def length(rng):
    return int(rng.choice(EDGE_LENGTHS)) if rng.random() < 0.6 else int(rng.integers(1, 401))


def dense_case(i):
    rng = np.random.default_rng(1000 + i)
    dt = ["f32", "f16", "bf16", "f32x6"][i % 4]
    E = int(rng.choice([16, 32, 64, 128, 256] if dt in ("f16", "bf16") else [16, 32, 64, 128]))
    KH = int(rng.choice([1, 2]))
    QH = KH * int(rng.choice([1, 2]))
    B = int(rng.choice([1, 2]))
    QL, KL = length(rng), length(rng)
    causal = bool(rng.random() < 0.5)
    pair = bool(rng.random() < 0.3)
    kpad = None
    if rng.random() < 0.4:
        kpad = rng.random((B, KL)) < 0.8
        if B > 1 and rng.random() < 0.3:
            kpad[0] = False  # every key of one batch masked: its rows give m = -inf, l = 0
    qk16 = dt in ("f32", "f32x6") and bool(rng.random() < 0.5)
    return dt, E, QL, KL, QH, KH, B, causal, pair, kpad, 1000 + i, qk16


DENSE = [dense_case(i) for i in range(96)]


@pytest.mark.parametrize("case", DENSE, ids=lambda c: "{}-E{}-{}x{}-h{}:{}-b{}{}{}{}{}".format(
    c[0], c[1], c[2], c[3], c[4], c[5], c[6], "-causal" if c[7] else "", "-pair" if c[8] else "",
    "-kpad" if c[9] is not None else "", "-qk16" if c[11] else ""))
def test_random_dense(dev, case):
    dt, E, QL, KL, QH, KH, B, causal, pair, kpad, seed, qk16 = case
    # "f32x6": float32 tensors through the bf16x6 kernels, held to the float32 bar
    mode = nnop.float32_attention_precision("bf16x6") if dt == "f32x6" else contextlib.nullcontext()
    with mode:
        run_case(dev, "f32" if dt == "f32x6" else dt, E, QL, KL, QH, KH, B, causal, pair, kpad is not None, seed,
                 qk16=qk16, kpad=kpad)


def split_case(i):
    """16-bit pair-biased calls on small grids, where the dQ splits its key range and, with
    QH = KH, the dK / dV their query range over several four-head workgroups."""
    rng = np.random.default_rng(4000 + i)
    dt = ["f16", "bf16"][i % 2]
    E = int(rng.choice([16, 32, 64]))
    QH = int(rng.choice([4, 8]))
    KH = QH if rng.random() < 0.7 else QH // 2
    B = int(rng.choice([1, 2]))
    QL, KL = length(rng) + 64, length(rng) + 64  # at least four 32-key tiles: two ranges
    causal = bool(rng.random() < 0.4)
    kpad = None
    if rng.random() < 0.4:
        kpad = rng.random((B, KL)) < 0.85
    return dt, E, QL, KL, QH, KH, B, causal, True, kpad, 4000 + i, False


SPLITS = [split_case(i) for i in range(24)]


@pytest.mark.parametrize("case", SPLITS, ids=lambda c: "{}-E{}-{}x{}-h{}:{}-b{}{}{}".format(
    c[0], c[1], c[2], c[3], c[4], c[5], c[6], "-causal" if c[7] else "", "-kpad" if c[9] is not None else ""))
def test_random_pair_splits(dev, case):
    dt, E, QL, KL, QH, KH, B, causal, pair, kpad, seed, qk16 = case
    run_case(dev, dt, E, QL, KL, QH, KH, B, causal, pair, kpad is not None, seed, qk16=qk16, kpad=kpad)


def varlen_case(i):
    rng = np.random.default_rng(2000 + i)
    dt = ["f32", "f16", "bf16"][i % 3]
    E = int(rng.choice([32, 64, 128]))
    KH = int(rng.choice([1, 2]))
    QH = KH * int(rng.choice([1, 2, 4]))
    n = int(rng.integers(1, 5))
    qlens = [0 if rng.random() < 0.15 else length(rng) for _ in range(n)]
    if sum(qlens) == 0:
        qlens[0] = length(rng)
    causal = bool(rng.random() < 0.5)
    # causal sequences keep equal lengths; an empty sequence is empty on both sides
    klens = list(qlens) if causal or rng.random() < 0.5 else [length(rng) if ql else 0 for ql in qlens]
    return dt, E, QH, KH, qlens, klens, causal, 2000 + i


VARLEN = [varlen_case(i) for i in range(32)]


@pytest.mark.parametrize("case", VARLEN, ids=lambda c: "{}-E{}-h{}:{}-{}-{}{}".format(
    c[0], c[1], c[2], c[3], "_".join(map(str, c[4])), "_".join(map(str, c[5])), "-causal" if c[6] else ""))
def test_random_varlen(dev, case):
    dt, E, QH, KH, qlens, klens, causal, seed = case
    run_varlen(dev, dt, E, QH, KH, qlens, klens, causal, seed)
