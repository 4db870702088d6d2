"""nnop -- host side of NNop's fused-kernel hot path on MI355X (gfx950).

Mirrors the reference package's API (MurrellGroup/ONIONop.jl, module NNop) over
torch-ROCm device tensors; every op runs in libonionop_hip.so through its C ABI
(include/onionop.h).  Public functions are differentiable with torch autograd, the
way the reference's ChainRules rrules make them differentiable under Zygote.

Array convention: a Julia column-major array (d1, d2, d3, d4) is the row-major torch
tensor of shape (d4, d3, d2, d1) -- the same memory, no copies.

Reference names -> here:
  NNop.flash_attention / _flash_attention / ∇flash_attention
      -> flash_attention / _flash_attention / grad_flash_attention
  NNop.online_softmax / ∇online_softmax -> online_softmax / grad_online_softmax
  (second order, the within_gradient branch of ∇online_softmax) -> grad_online_softmax_pullback
  NNop.rms_norm / _rms_norm / ∇rms_norm -> rms_norm / _rms_norm / grad_rms_norm
  NNop.layer_norm / _layer_norm / ∇layer_norm -> layer_norm / _layer_norm / grad_layer_norm
  NNop.llama_rope / _llama_rope / ∇llama_rope / LlamaRotaryEmbedding -> same names
  (LlamaRotaryEmbedding on device positions: rotary_tables, the library's table kernel)
  flash_attention(llama_rope(q, k)..., v) with the RoPE backward fused into the attention
  backward -> flash_attention_rope / grad_flash_attention_rope (+ _varlen_rope)
  float32 attention on the bf16 matrix cores (six-term exact split; no reference
  counterpart) -> set_float32_attention_precision("bf16x6") / float32_attention_precision
"""
from ._lib import LIB_PATH, NNopError, lib
from .attention import (_flash_attention, _flash_attention_varlen, attention_scale, flash_attention,
                        flash_attention_rope, flash_attention_varlen, float32_attention_precision,
                        get_float32_attention_precision, grad_flash_attention, grad_flash_attention_rope,
                        grad_flash_attention_varlen, grad_flash_attention_varlen_rope,
                        set_float32_attention_precision)
from .norms import _layer_norm, _rms_norm, grad_layer_norm, grad_rms_norm, layer_norm, rms_norm
from .rope import LlamaRotaryEmbedding, _llama_rope, grad_llama_rope, llama_rope, rotary_tables
from .softmax import _online_softmax, grad_online_softmax, grad_online_softmax_pullback, online_softmax

__all__ = [
    "LIB_PATH", "NNopError", "lib",
    "flash_attention", "_flash_attention", "grad_flash_attention", "attention_scale",
    "flash_attention_varlen", "_flash_attention_varlen", "grad_flash_attention_varlen",
    "flash_attention_rope", "grad_flash_attention_rope", "grad_flash_attention_varlen_rope",
    "set_float32_attention_precision", "get_float32_attention_precision", "float32_attention_precision",
    "online_softmax", "_online_softmax", "grad_online_softmax", "grad_online_softmax_pullback",
    "rms_norm", "_rms_norm", "grad_rms_norm",
    "layer_norm", "_layer_norm", "grad_layer_norm",
    "llama_rope", "_llama_rope", "grad_llama_rope", "LlamaRotaryEmbedding", "rotary_tables",
    "shared_memory",
]


def shared_memory(device: int = 0) -> int:
    """LDS bytes per workgroup of `device` (NNop.shared_memory, src/NNop.jl:27-30)."""
    import ctypes

    from ._lib import check

    out = ctypes.c_size_t(0)
    check(lib().onionop_device_lds_bytes(int(device), ctypes.byref(out)))
    return int(out.value)
