"""The C ABI library and the host-side logic, without a GPU.

* libonionop_hip.so loads and exports every entry point include/onionop.h declares,
  with the ABI version the header states (no compute call is made here);
* the Python signatures cover the same set;
* host validation raises the reference's messages before any launch, and there is no
  CPU fallback (host tensors are rejected).
"""
import ctypes
import os
import re

import pytest
import torch

import nnop
from nnop import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "onionop.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(onionop_\w+)\s*\(", text)))


def test_header_declares_the_hot_path():
    fns = header_functions()
    for must in ("onionop_flash_attn_fwd", "onionop_flash_attn_bwd", "onionop_softmax_fwd", "onionop_softmax_bwd",
                 "onionop_rms_norm_fwd", "onionop_rms_norm_bwd", "onionop_layer_norm_fwd", "onionop_layer_norm_bwd",
                 "onionop_llama_rope"):
        assert must in fns


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [f for f in header_functions() if not hasattr(lib, f)]
    assert not missing, missing
    assert set(header_functions()) == set(_lib.SIGNATURES)


def test_abi_version_matches_header():
    m = re.search(r"#define ONIONOP_ABI_VERSION (\d+)", open(HEADER).read())
    assert int(m.group(1)) == nnop.lib().onionop_abi_version() == _lib.ABI_VERSION


def test_workspace_queries_are_host_only():
    L = nnop.lib()
    assert L.onionop_flash_attn_bwd_workspace(2, 64, 4096, 4096, 4, 4, 4) >= 2 * 4096 * 16 * 4
    assert L.onionop_flash_attn_bwd_workspace(2, 64, 0, 4096, 4, 4, 4) == 0
    # rows of 4096 elements: 256 float32 partial rows; rows of 512 elements: 1024
    assert L.onionop_rms_norm_bwd_workspace(4096, 16384) == 256 * 4096 * 4
    assert L.onionop_rms_norm_bwd_workspace(512, 16384) == 1024 * 512 * 4
    assert L.onionop_layer_norm_bwd_workspace(4096, 3) == 2 * 3 * 4096 * 4


def test_c_abi_validation_errors():
    """Status codes and messages come back without touching a device (checks run first)."""
    L = nnop.lib()
    st = L.onionop_flash_attn_fwd(None, 2, 48, 8, 8, 2, 2, 1, None, None, None, None, None, 0, 1.0, None, None, None)
    assert st == -1 and L.onionop_last_error() == b"Only power-of-2 embedding dims are supported."
    st = L.onionop_flash_attn_fwd(None, 2, 64, 8, 8, 3, 2, 1, None, None, None, None, None, 0, 1.0, None, None, None)
    assert st == -1 and b"must be divisible by number of KV heads" in L.onionop_last_error()
    st = L.onionop_flash_attn_fwd(None, 7, 64, 8, 8, 2, 2, 1, None, None, None, None, None, 0, 1.0, None, None, None)
    assert st == -2
    # code 3 (float32 through bf16x6 MFMA products) is an attention element type: it passes
    # the type check and meets the NULL tensors; the row-wise ops refuse it
    st = L.onionop_flash_attn_fwd(None, 3, 64, 8, 8, 2, 2, 1, None, None, None, None, None, 0, 1.0, None, None, None)
    assert st == -5
    st = L.onionop_softmax_fwd(None, 3, 64, 4, 16, 16)
    assert st == -2
    # head dims 16..256 are built (E = 256 passes the shape checks, then meets the NULL
    # tensors); 512 and 8 are not
    st = L.onionop_flash_attn_fwd(None, 2, 256, 8, 8, 2, 2, 1, None, None, None, None, None, 0, 1.0, None, None, None)
    assert st == -5
    for e in (512, 8):
        st = L.onionop_flash_attn_fwd(None, 2, e, 8, 8, 2, 2, 1, None, None, None, None, None, 0, 1.0, None, None,
                                      None)
        assert st == -3 and b"embedding dim" in L.onionop_last_error()
    st = L.onionop_flash_attn_fwd(None, 2, 64, 8, 8, 2, 2, 1, None, None, None, None, None, 0, 1.0, None, None, None)
    assert st == -5
    st = L.onionop_flash_attn_bwd(None, 2, 64, 8, 8, 2, 2, 1, 16, 16, 16, 16, 16, 16, 16, 16, None, 0, 1.0, 0,
                                  16, 16, 16, None, None, 0)
    assert st == -5 and b"dpair" in L.onionop_last_error()
    st = L.onionop_flash_attn_bwd(None, 2, 64, 8, 8, 2, 2, 1, 16, 16, 16, 16, 16, 16, 16, None, None, 0, 1.0, 0,
                                  16, 16, 16, None, 16, 8)
    assert st == -6
    # a bias slice whose 64-key-row span needs offsets of 2^32 bytes or more
    st = L.onionop_flash_attn_fwd(None, 0, 16, 1 << 20, 8, 64, 64, 1, 16, 16, 16, 16, None, 0, 1.0, 16, 16, 16)
    assert st == -3 and b"pair bias too large" in L.onionop_last_error()
    st = L.onionop_llama_rope(None, 2, 15, 4, 1, 1, 1, 16, 16, 16, 16, 1.0, 16, 16)
    assert st == -1
    # rows of any length run (streaming kernels past the register-resident size), up to
    # the 32-bit row offsets
    st = L.onionop_softmax_fwd(None, 0, 1 << 29, 4, 16, 16)
    assert st == -3 and b"reduction length" in L.onionop_last_error()
    st = L.onionop_rms_norm_fwd(None, 2, 2, 1 << 29, 4, 16, 16, 1e-6, 0.0, 16, 16)
    assert st == -3


def test_host_checks_use_reference_messages():
    q = torch.zeros((1, 3, 8, 64))
    k = torch.zeros((1, 2, 8, 64))
    from nnop.attention import _check_shapes

    with pytest.raises(ValueError, match=r"Number of query heads `3` must be divisible by number of KV heads `2`\."):
        _check_shapes(q, k, k, None, None)
    with pytest.raises(ValueError, match=r"Embedding dim of Q `32` must be the same as of K `64`\."):
        _check_shapes(torch.zeros((1, 2, 8, 32)), k, k, None, None)
    with pytest.raises(ValueError, match=r"Shapes of K `\(64, 8, 2, 1\)` and V `\(64, 9, 2, 1\)` must be the same\."):
        _check_shapes(torch.zeros((1, 2, 8, 64)), k, torch.zeros((1, 2, 9, 64)), None, None)
    with pytest.raises(ValueError, match=r"Only power-of-2 embedding dims are supported\."):
        x = torch.zeros((1, 2, 8, 48))
        _check_shapes(x, x, x, None, None)


def test_no_cpu_fallback():
    x = torch.zeros((4, 64))
    with pytest.raises(ValueError, match="no CPU path"):
        nnop.online_softmax(x)
    with pytest.raises(ValueError, match="no CPU path"):
        nnop.rms_norm(x, torch.ones(64))
    q = torch.zeros((1, 2, 8, 64))
    with pytest.raises(ValueError, match="no CPU path"):
        nnop.flash_attention(q, q, q, causal=True)


def test_lds_query_errors():
    """onionop_device_lds_bytes (the shared_memory query, src/NNop.jl:27-30) rejects a NULL
    output and a device index outside the cache before touching a device."""
    L = nnop.lib()
    assert L.onionop_device_lds_bytes(0, None) == -5
    out = ctypes.c_size_t(7)
    assert L.onionop_device_lds_bytes(-1, ctypes.byref(out)) == -1
    assert L.onionop_device_lds_bytes(64, ctypes.byref(out)) == -1
    assert out.value == 7


def test_llama_rotary_embedding_tables():
    """nnop.LlamaRotaryEmbedding (src/rope/llama_rope.jl:1-22) against the oracle's float32
    restatement (FAITHFUL) and the float64 closed form cos/sin(p / base^(2i/dim)), for the
    headline GQA workload's table: dim 128, positions 0..8191, 4 sequences."""
    import numpy as np

    import oracle

    dim, L, B = 128, 8192, 4
    pos = torch.arange(L, dtype=torch.float32)[None].expand(B, L)
    c, s = nnop.LlamaRotaryEmbedding(dim)(pos)
    assert tuple(c.shape) == (B, L, dim) and c.dtype == torch.float32
    c, s = c.double().numpy(), s.double().numpy()
    # first and second halves repeat (vcat(freqs, freqs))
    assert np.array_equal(c[..., :64], c[..., 64:]) and np.array_equal(s[..., :64], s[..., 64:])
    cf, sf = oracle.rotary_embedding(dim, pos.double().numpy(), mode=oracle.FAITHFUL)
    assert np.abs(c - cf).max() <= 2e-7 and np.abs(s - sf).max() <= 2e-7
    # closed form in float64; the float32 angle p * inv_freq carries up to ~L ulp(1) of
    # error at the largest positions, which bounds the distance
    i = np.arange(0, dim, 2) / dim
    ang = np.arange(L)[:, None] / 10000.0 ** i[None, :]
    ang = np.concatenate([ang, ang], axis=1)[None]
    assert np.abs(c - np.cos(ang)).max() <= L * 2.0 ** -23 and np.abs(s - np.sin(ang)).max() <= L * 2.0 ** -23
    ce, se = oracle.rotary_embedding(dim, pos.double().numpy(), mode=oracle.EXACT)
    assert np.abs(ce - np.cos(ang)).max() <= 1e-12 and np.abs(se - np.sin(ang)).max() <= 1e-12
    # positions as a vector give the table of one sequence
    c1, _ = nnop.LlamaRotaryEmbedding(dim)(torch.arange(L, dtype=torch.float32))
    assert np.array_equal(c1.double().numpy()[0], c[0])
