"""ctypes binding of libonionop_hip.so (the C ABI in include/onionop.h).

There is no CPU fallback: if the library is missing or a tensor is not on a ROCm device,
the call raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# The in-tree build; ONIONOP_LIB may name another build of the same library.
LIB_PATH = os.environ.get("ONIONOP_LIB") or os.path.normpath(os.path.join(_HERE, "..", "lib", "libonionop_hip.so"))

F32, F16, BF16 = 0, 1, 2
F32_BF16X6 = 3  # float32 tensors, attention products on bf16 MFMA (six-term split)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f = ctypes.c_float
_i = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes); must match include/onionop.h
SIGNATURES = {
    "onionop_last_error": (ctypes.c_char_p, []),
    "onionop_abi_version": (_i, []),
    "onionop_device_lds_bytes": (_i, [_i, ctypes.POINTER(_sz)]),
    "onionop_flash_attn_fwd": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i,
                                    _f, _vp, _vp, _vp]),
    "onionop_flash_attn_bwd_workspace": (_sz, [_i, _i64, _i64, _i64, _i64, _i64, _i64]),
    "onionop_flash_attn_bwd": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                                    _vp, _vp, _vp, _i, _f, _i, _vp, _vp, _vp, _vp, _vp, _sz]),
    "onionop_flash_attn_bwd_rope": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                                         _vp, _vp, _vp, _vp, _vp, _i, _f, _i, _vp, _vp, _vp, _vp, _vp, _sz]),
    "onionop_flash_attn_bwd_noalloc": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _vp, _i, _f, _i, _vp, _vp, _vp, _vp]),
    "onionop_flash_attn_bwd_preprocess": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _sz]),
    "onionop_flash_attn_bwd_dkdv": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
                                         _vp, _i, _f, _i, _vp, _vp, _vp, _sz]),
    "onionop_flash_attn_bwd_dq": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
                                       _vp, _i, _f, _i, _vp, _vp, _vp, _sz]),
    "onionop_flash_attn_varlen_fwd": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i64,
                                           _vp, _vp, _vp, _i, _f, _vp, _vp, _vp]),
    "onionop_flash_attn_varlen_bwd_workspace": (_sz, [_i, _i64, _i64, _i64]),
    "onionop_flash_attn_varlen_bwd": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i64,
                                           _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _f, _i, _vp, _vp, _vp, _vp,
                                           _sz]),
    "onionop_flash_attn_varlen_bwd_rope": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i64,
                                                _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _f, _i, _vp, _vp,
                                                _vp, _vp, _sz]),
    "onionop_softmax_fwd": (_i, [_vp, _i, _i64, _i64, _vp, _vp]),
    "onionop_softmax_bwd": (_i, [_vp, _i, _i64, _i64, _vp, _vp, _vp]),
    "onionop_softmax_bwd_bwd": (_i, [_vp, _i, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "onionop_rms_norm_fwd": (_i, [_vp, _i, _i, _i64, _i64, _vp, _vp, _f, _f, _vp, _vp]),
    "onionop_rms_norm_bwd_workspace": (_sz, [_i64, _i64]),
    "onionop_rms_norm_bwd": (_i, [_vp, _i, _i, _i64, _i64, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _sz]),
    "onionop_layer_norm_fwd": (_i, [_vp, _i, _i, _i64, _i64, _vp, _vp, _vp, _f, _vp, _vp, _vp]),
    "onionop_layer_norm_bwd_workspace": (_sz, [_i64, _i64]),
    "onionop_layer_norm_bwd": (_i, [_vp, _i, _i, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz]),
    "onionop_llama_rope": (_i, [_vp, _i, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _f, _vp, _vp]),
    "onionop_llama_rotary_embedding": (_i, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
}

ABI_VERSION = 2


class NNopError(RuntimeError):
    """A failed library call; the message is the library's (the reference's where it has one)."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_lib = None


def lib():
    """Load libonionop_hip.so once (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libonionop_hip.so not found at {LIB_PATH}; build it with `make -C onionop.jl_amd` "
                "(or __graft_entry__.build()). There is no CPU fallback.")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        v = L.onionop_abi_version()
        if v != ABI_VERSION:
            raise ImportError(f"libonionop_hip.so ABI version {v}, expected {ABI_VERSION}")
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        msg = lib().onionop_last_error().decode("utf-8", "replace")
        raise NNopError(status, msg)
