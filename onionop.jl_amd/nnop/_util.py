"""Tensor plumbing shared by the op modules: dtype codes, device checks, stream handle."""
from __future__ import annotations

import torch

from ._lib import BF16, F16, F32, F32_BF16X6

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}


def dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported element type {t.dtype} (float32, float16, bfloat16)") from None


# Precision of float32 attention: "float32" (float32 MFMA) or "bf16x6" (every product as six
# bf16 MFMA products of an exact three-way split).  Process-wide, like torch's
# set_float32_matmul_precision.
_F32_ATTN = ["float32"]


def attn_dtype_code(t: torch.Tensor, what: str) -> int:
    """Element type code of an attention call: F32_BF16X6 for float32 under "bf16x6"."""
    dt = dtype_code(t, what)
    return F32_BF16X6 if dt == F32 and _F32_ATTN[0] == "bf16x6" else dt


def device_tensor(t: torch.Tensor, what: str) -> torch.Tensor:
    """Dense, 16-byte aligned device tensor (the reference's dense arrays); no host fallback
    exists.  The library's kernels use 16-byte vector accesses and reject pointers that are
    not 16-byte aligned; a view that starts inside its storage (a slice of a larger array,
    the counterpart of a Julia `view`) is copied into a fresh allocation here, as the Julia
    binding does for misaligned arrays."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{what}: expected a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{what}: tensor must be on a ROCm device (got {t.device}); there is no CPU path")
    t = t.contiguous()
    if t.data_ptr() % 16 != 0:
        t = t.clone()
    return t


def ptr(t):
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


def jdims(t: torch.Tensor) -> tuple:
    """Shape as the reference's column-major Julia array would print it."""
    return tuple(reversed(t.shape))


def round_scalar(x: float, dtype: torch.dtype) -> float:
    """x rounded to `dtype`, as the reference's T(x)."""
    return float(torch.tensor(x, dtype=torch.float64).to(dtype).item())
