# NNopAMDGPUExt.jl -- the AMDGPU package extension of NNop with every launcher of the hot
# path bound to libonionop_hip.so through `ccall` (C ABI: include/onionop.h).
#
# It replaces the reference's ext/NNopAMDGPUExt.jl.  The public functions of NNop
# (flash_attention, online_softmax, rms_norm, layer_norm, llama_rope) and their
# ChainRules rrules stay as they are; the methods below are ROCArray specialisations of the
# host launchers they call, so KernelAbstractions keeps serving every other backend:
#   NNop._shared_memory        src/NNop.jl:27-30, ext/NNopAMDGPUExt.jl:6-9
#   NNop._flash_attention      src/attention.jl:145-197
#   NNop.∇flash_attention      src/attention_bwd.jl:213-303 (with the preprocess, :177-211)
#   NNop.online_softmax        src/softmax.jl:60-68
#   NNop.∇online_softmax       src/softmax.jl:70-80 (second order through its own rrule)
#   NNop._rms_norm             src/rms_norm.jl:117-137
#   NNop.∇rms_norm             src/rms_norm.jl:139-169
#   NNop._layer_norm           src/layer_norm.jl:150-170
#   NNop.∇layer_norm           src/layer_norm.jl:172-204
#   NNop._llama_rope           src/rope/llama_rope.jl:69-89 (llama_rope and ∇llama_rope)
# plus flash_attention_varlen (packed sequences), which the reference does not have.
#
# Differences a caller can see, all documented in include/onionop.h:
#  * ms / ls of attention are Float32 for every element type (the reference stores them
#    as T); they only travel from the forward to its pullback.
#  * BFloat16 attention is accepted (the reference restricts T to Float16 / Float32).
#  * Rows whose keys are all masked give o = 0 instead of NaN.
#  * The float32 backward rounds Q and K to Float16 like the reference
#    (src/attention_bwd.jl:20-21); set ONIONOP_EXACT_QK=1 for exact float32 Q / K.
#  * Arrays must be dense; the kernels use 16-byte vector accesses, so an array whose
#    pointer is not 16-byte aligned (a view into a larger array) is copied first.
#
# Project.toml of NNop: AMDGPU and BFloat16s under [weakdeps], and
#   [extensions] NNopAMDGPUExt = ["AMDGPU", "BFloat16s"]
# The library is built from onionop.jl_amd/ (`make -C onionop.jl_amd`) and shipped as an
# Artifact; ONIONOP_LIB overrides its path.
module NNopAMDGPUExt

using AMDGPU
using BFloat16s: BFloat16
using NNop
import ChainRulesCore as CRC

const libonionop = get(ENV, "ONIONOP_LIB", joinpath(@__DIR__, "..", "lib", "libonionop_hip.so"))
const ABI_VERSION = 2

const HipFloat = Union{Float32, Float16, BFloat16}

_dt(::Type{Float32}) = Cint(0)
_dt(::Type{Float16}) = Cint(1)
_dt(::Type{BFloat16}) = Cint(2)

# Precision of Float32 attention: :float32 (Float32 MFMA products, the default) or :bf16x6
# (every product as the six bf16 MFMA products of an exact three-way split, accumulated in
# Float32: element type code ONIONOP_F32_BF16X6).  Set with
# `NNopAMDGPUExt.FLOAT32_ATTENTION[] = :bf16x6`.
const FLOAT32_ATTENTION = Ref(:float32)
_attn_dt(::Type{T}) where {T} = T === Float32 && FLOAT32_ATTENTION[] === :bf16x6 ? Cint(3) : _dt(T)

_ptr(::Nothing) = C_NULL
_ptr(x::ROCArray) = pointer(x)
_stream() = AMDGPU.stream().stream

# 16-byte aligned dense device array with x's values (a copy only when needed).
_aligned(x::ROCArray) = UInt(pointer(x)) % 16 == 0 ? x : copyto!(similar(x, eltype(x), size(x)), x)
# A cotangent as a dense, aligned ROCArray shaped like `like` (Zygote may hand a Fill or
# another lazy array).
_dense(Δ::ROCArray, like) = _aligned(Δ)
_dense(Δ, like) = copyto!(similar(like), Δ)

function _check(status::Cint)
    status == 0 && return nothing
    msg = unsafe_string(ccall((:onionop_last_error, libonionop), Cstring, ()))
    error(msg)
end

_exact_qk() = get(ENV, "ONIONOP_EXACT_QK", "0") == "1"

function __init__()
    v = ccall((:onionop_abi_version, libonionop), Cint, ())
    v == ABI_VERSION || @warn "libonionop_hip.so ABI version $v, expected $ABI_VERSION"
end

# ------------------------------------------------------------------------ LDS query

function NNop._shared_memory(::ROCBackend, device_id::Integer)
    out = Ref{Csize_t}(0)
    # AMDGPU numbers devices from 1, HIP from 0.
    _check(ccall((:onionop_device_lds_bytes, libonionop), Cint, (Cint, Ptr{Csize_t}), device_id - 1, out))
    return UInt64(out[])
end

# ------------------------------------------------------------------------ attention

_attn_scale(::Type{T}, E) where {T} = Float32(T(inv(sqrt(E))))

function NNop._flash_attention(
    q::ROCArray{T,4}, k::ROCArray{T,4}, v::ROCArray{T,4},
    pair::Union{Nothing,ROCArray{T,4}} = nothing;
    causal::Bool, kpad_mask::Union{Nothing,ROCMatrix{Bool}} = nothing,
) where {T <: HipFloat}
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    QE, QL, QH, B = size(q)
    KE, KL, KH, _ = size(k)
    o = similar(q)
    ms = ROCArray{Float32}(undef, QL, QH, B)
    ls = ROCArray{Float32}(undef, QL, QH, B)
    _check(ccall((:onionop_flash_attn_fwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Int64, Int64, Int64, Int64, Int64, Int64,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{UInt8}, Cint, Cfloat,
         Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cfloat}),
        _stream(), _attn_dt(T), QE, QL, KL, QH, KH, B,
        q, k, v, _ptr(pair), _ptr(kpad_mask), Cint(causal), _attn_scale(T, QE), o, ms, ls))
    return o, ms, ls
end

function NNop.∇flash_attention(
    Δ::ROCArray{T,4}, o::ROCArray{T,4}, ms::ROCArray{Float32,3}, ls::ROCArray{Float32,3},
    q::ROCArray{T,4}, k::ROCArray{T,4}, v::ROCArray{T,4},
    pair::Union{Nothing,ROCArray{T,4}} = nothing;
    causal::Bool, kpad_mask::Union{Nothing,ROCMatrix{Bool}} = nothing,
) where {T <: HipFloat}
    Δ, o, q, k, v = _aligned(Δ), _aligned(o), _aligned(q), _aligned(k), _aligned(v)
    QE, QL, QH, B = size(q)
    KE, KL, KH, _ = size(k)
    ws_bytes = ccall((:onionop_flash_attn_bwd_workspace, libonionop), Csize_t,
                     (Cint, Int64, Int64, Int64, Int64, Int64, Int64), _attn_dt(T), QE, QL, KL, QH, KH, B)
    ws = ROCArray{UInt8}(undef, max(ws_bytes, 1))
    dq, dk, dv = similar(q), similar(k), similar(v)
    dpair = pair === nothing ? nothing : similar(pair)
    _check(ccall((:onionop_flash_attn_bwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Int64, Int64, Int64, Int64, Int64, Int64,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
         Ptr{Cvoid}, Ptr{UInt8}, Cint, Cfloat, Cint,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Csize_t),
        _stream(), _attn_dt(T), QE, QL, KL, QH, KH, B,
        Δ, o, ms, ls, q, k, v, _ptr(pair), _ptr(kpad_mask), Cint(causal), _attn_scale(T, QE),
        Cint(!_exact_qk()),   # Float16 Q / K in the backward, as src/attention_bwd.jl:20-21
        dq, dk, dv, _ptr(dpair), ws, ws_bytes))
    return dq, dk, dv, dpair
end

# The reference rrule (src/attention_crc.jl:16-31): under AD the primal is o alone
# (flash_attention returns it as is when within_gradient holds), and the cotangent is
# materialised as a dense ROCArray before the backward launcher sees it.
function CRC.rrule(::typeof(NNop._flash_attention),
    q::ROCArray{T,4}, k::ROCArray{T,4}, v::ROCArray{T,4},
    pair::Union{Nothing,ROCArray{T,4}} = nothing;
    causal::Bool, kpad_mask::Union{Nothing,ROCMatrix{Bool}} = nothing,
) where {T <: HipFloat}
    o, ms, ls = NNop._flash_attention(q, k, v, pair; causal, kpad_mask)
    function _pullback(Δ)
        dq, dk, dv, dpair = NNop.∇flash_attention(
            _dense(CRC.unthunk(Δ), o), o, ms, ls, q, k, v, pair; causal, kpad_mask)
        return CRC.NoTangent(), dq, dk, dv, dpair
    end
    return o, _pullback
end

# Packed variable-length sequences: q (E, Tq, QH), k / v (E, Tk, KH), sequence b at rows
# cu_q[b]+1 : cu_q[b+1] (Int32 offsets on the device); max_q / max_k bound the lengths.
function flash_attention_varlen_fwd(q::ROCArray{T,3}, k::ROCArray{T,3}, v::ROCArray{T,3},
                                    cu_q::ROCVector{Int32}, cu_k::ROCVector{Int32}, max_q::Integer, max_k::Integer;
                                    causal::Bool) where {T <: HipFloat}
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    E, Tq, QH = size(q)
    _, Tk, KH = size(k)
    B = length(cu_q) - 1
    # rows in no sequence are not written: they start at zero
    o = AMDGPU.zeros(T, size(q))
    ms = AMDGPU.zeros(Float32, Tq, QH)
    ls = AMDGPU.zeros(Float32, Tq, QH)
    _check(ccall((:onionop_flash_attn_varlen_fwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Int64, Int64, Int64, Int64, Int64, Int64, Ptr{Int32}, Ptr{Int32}, Int64, Int64,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Cint, Cfloat, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cfloat}),
        _stream(), _attn_dt(T), E, Tq, Tk, QH, KH, B, cu_q, cu_k, max_q, max_k, q, k, v, Cint(causal),
        _attn_scale(T, E), o, ms, ls))
    return o, ms, ls
end

function flash_attention_varlen_bwd(Δ::ROCArray{T,3}, o::ROCArray{T,3}, ms::ROCMatrix{Float32},
                                    ls::ROCMatrix{Float32}, q::ROCArray{T,3}, k::ROCArray{T,3}, v::ROCArray{T,3},
                                    cu_q::ROCVector{Int32}, cu_k::ROCVector{Int32}, max_q::Integer, max_k::Integer;
                                    causal::Bool) where {T <: HipFloat}
    Δ, o, q, k, v = _aligned(Δ), _aligned(o), _aligned(q), _aligned(k), _aligned(v)
    E, Tq, QH = size(q)
    _, Tk, KH = size(k)
    B = length(cu_q) - 1
    ws_bytes = ccall((:onionop_flash_attn_varlen_bwd_workspace, libonionop), Csize_t,
                     (Cint, Int64, Int64, Int64), _attn_dt(T), E, Tq, QH)
    ws = ROCArray{UInt8}(undef, max(ws_bytes, 1))
    # gradient rows of queries / keys in no sequence are not written: they are zero
    dq, dk, dv = AMDGPU.zeros(T, size(q)), AMDGPU.zeros(T, size(k)), AMDGPU.zeros(T, size(v))
    _check(ccall((:onionop_flash_attn_varlen_bwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Int64, Int64, Int64, Int64, Int64, Int64, Ptr{Int32}, Ptr{Int32}, Int64, Int64,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Cint, Cfloat, Cint,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Csize_t),
        _stream(), _attn_dt(T), E, Tq, Tk, QH, KH, B, cu_q, cu_k, max_q, max_k, Δ, o, ms, ls, q, k, v,
        Cint(causal), _attn_scale(T, E), Cint(!_exact_qk()), dq, dk, dv, ws, ws_bytes))
    return dq, dk, dv
end

"""
    flash_attention_varlen(q, k, v, cu_q, cu_k, max_q, max_k; causal)

Flash attention over packed sequences (no padding rows are read or computed).
Differentiable in q, k and v.
"""
function flash_attention_varlen(q, k, v, cu_q, cu_k, max_q, max_k; causal::Bool)
    return first(flash_attention_varlen_fwd(q, k, v, cu_q, cu_k, max_q, max_k; causal))
end

function CRC.rrule(::typeof(flash_attention_varlen), q, k, v, cu_q, cu_k, max_q, max_k; causal::Bool)
    o, ms, ls = flash_attention_varlen_fwd(q, k, v, cu_q, cu_k, max_q, max_k; causal)
    function _pullback(Δ)
        dq, dk, dv = flash_attention_varlen_bwd(_dense(CRC.unthunk(Δ), o), o, ms, ls, q, k, v,
                                                cu_q, cu_k, max_q, max_k; causal)
        nt = CRC.NoTangent()
        return nt, dq, dk, dv, nt, nt, nt, nt
    end
    return o, _pullback
end

# flash_attention(llama_rope(q, k; cos, sin)..., v) with ∇llama_rope fused into the attention
# backward: the library rotates the float32 dQ / dK accumulators before it stores them, so the
# pullback of the composition (src/attention_crc.jl:16-31 then src/rope/llama_rope.jl:94-98)
# runs no separate ∇llama_rope pass.  qr, kr are the rotated tensors the forward used (the
# output of llama_rope); dq, dk come back w.r.t. q, k before the rotation.  cos, sin
# (E, L, B) Float32 as LlamaRotaryEmbedding returns them.
function ∇flash_attention_rope(
    Δ::ROCArray{T,4}, o::ROCArray{T,4}, ms::ROCArray{Float32,3}, ls::ROCArray{Float32,3},
    qr::ROCArray{T,4}, kr::ROCArray{T,4}, v::ROCArray{T,4}, cos::ROCArray{Float32,3}, sin::ROCArray{Float32,3},
    pair::Union{Nothing,ROCArray{T,4}} = nothing;
    causal::Bool, kpad_mask::Union{Nothing,ROCMatrix{Bool}} = nothing,
) where {T <: HipFloat}
    Δ, o, qr, kr, v = _aligned(Δ), _aligned(o), _aligned(qr), _aligned(kr), _aligned(v)
    QE, QL, QH, B = size(qr)
    KE, KL, KH, _ = size(kr)
    ws_bytes = ccall((:onionop_flash_attn_bwd_workspace, libonionop), Csize_t,
                     (Cint, Int64, Int64, Int64, Int64, Int64, Int64), _attn_dt(T), QE, QL, KL, QH, KH, B)
    ws = ROCArray{UInt8}(undef, max(ws_bytes, 1))
    dq, dk, dv = similar(qr), similar(kr), similar(v)
    dpair = pair === nothing ? nothing : similar(pair)
    _check(ccall((:onionop_flash_attn_bwd_rope, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Int64, Int64, Int64, Int64, Int64, Int64,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
         Ptr{Cvoid}, Ptr{UInt8}, Ptr{Cfloat}, Ptr{Cfloat}, Cint, Cfloat, Cint,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Csize_t),
        _stream(), _attn_dt(T), QE, QL, KL, QH, KH, B,
        Δ, o, ms, ls, qr, kr, v, _ptr(pair), _ptr(kpad_mask), cos, sin, Cint(causal), _attn_scale(T, QE),
        Cint(!_exact_qk()), dq, dk, dv, _ptr(dpair), ws, ws_bytes))
    return dq, dk, dv, dpair
end

"""
    flash_attention_rope(q, k, v, cos, sin, pair = nothing; causal, kpad_mask = nothing)

`flash_attention(llama_rope(q, k; cos, sin)..., v, pair; causal, kpad_mask)` whose pullback
fuses ∇llama_rope into the attention backward.  Differentiable in q, k, v and pair.
"""
function flash_attention_rope(q, k, v, cos, sin, pair = nothing; causal::Bool, kpad_mask = nothing)
    qr, kr = NNop.llama_rope(q, k; cos, sin)
    return first(NNop._flash_attention(qr, kr, v, pair; causal, kpad_mask))
end

function CRC.rrule(::typeof(flash_attention_rope), q, k, v, cos, sin, pair = nothing;
                   causal::Bool, kpad_mask = nothing)
    qr, kr = NNop.llama_rope(q, k; cos, sin)
    o, ms, ls = NNop._flash_attention(qr, kr, v, pair; causal, kpad_mask)
    function _pullback(Δ)
        dq, dk, dv, dpair = ∇flash_attention_rope(_dense(CRC.unthunk(Δ), o), o, ms, ls, qr, kr, v, cos, sin, pair;
                                                  causal, kpad_mask)
        nt = CRC.NoTangent()
        # one tangent per argument passed: pair only when it was given
        return pair === nothing ? (nt, dq, dk, dv, nt, nt) : (nt, dq, dk, dv, nt, nt, dpair)
    end
    return o, _pullback
end

# Packed sequences with the fused ∇llama_rope: q and k packed alike (cu_q == cu_k);
# cos, sin (E, Tq) Float32, one column per packed position.
function flash_attention_varlen_bwd_rope(Δ::ROCArray{T,3}, o::ROCArray{T,3}, ms::ROCMatrix{Float32},
                                         ls::ROCMatrix{Float32}, qr::ROCArray{T,3}, kr::ROCArray{T,3},
                                         v::ROCArray{T,3}, cos::ROCMatrix{Float32}, sin::ROCMatrix{Float32},
                                         cu::ROCVector{Int32}, max_len::Integer; causal::Bool) where {T <: HipFloat}
    Δ, o, qr, kr, v = _aligned(Δ), _aligned(o), _aligned(qr), _aligned(kr), _aligned(v)
    E, Tq, QH = size(qr)
    _, Tk, KH = size(kr)
    B = length(cu) - 1
    ws_bytes = ccall((:onionop_flash_attn_varlen_bwd_workspace, libonionop), Csize_t,
                     (Cint, Int64, Int64, Int64), _attn_dt(T), E, Tq, QH)
    ws = ROCArray{UInt8}(undef, max(ws_bytes, 1))
    dq, dk, dv = AMDGPU.zeros(T, size(qr)), AMDGPU.zeros(T, size(kr)), AMDGPU.zeros(T, size(v))
    _check(ccall((:onionop_flash_attn_varlen_bwd_rope, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Int64, Int64, Int64, Int64, Int64, Int64, Ptr{Int32}, Ptr{Int32}, Int64, Int64,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
         Ptr{Cfloat}, Ptr{Cfloat}, Cint, Cfloat, Cint,
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Csize_t),
        _stream(), _attn_dt(T), E, Tq, Tk, QH, KH, B, cu, cu, max_len, max_len, Δ, o, ms, ls, qr, kr, v,
        cos, sin, Cint(causal), _attn_scale(T, E), Cint(!_exact_qk()), dq, dk, dv, ws, ws_bytes))
    return dq, dk, dv
end

# ------------------------------------------------------------------------ softmax

function NNop.online_softmax(x::ROCMatrix{T}) where {T <: HipFloat}
    x = _aligned(x)
    y = similar(x)
    N, M = size(x)
    _check(ccall((:onionop_softmax_fwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}), _stream(), _dt(T), N, M, x, y))
    return y
end

# dx = Δ .* y .- y .* sum(Δ .* y; dims=1).  The kernel serves first and second order: the
# reference's `within_gradient` branch (src/softmax.jl:71-74) keeps the broadcasts
# differentiable; here the rrule below differentiates the kernel instead.
function NNop.∇online_softmax(Δ::ROCMatrix{T}, y::ROCMatrix{T}) where {T <: HipFloat}
    Δ, y = _aligned(Δ), _aligned(y)
    dx = similar(y)
    N, M = size(y)
    _check(ccall((:onionop_softmax_bwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}), _stream(), _dt(T), N, M, Δ, y, dx))
    return dx
end

# Pullback of ∇online_softmax: for g = dL/d(dx), s = sum(Δ .* y), u = sum(g .* y),
#   d_Δ = y .* (g .- u),   d_y = g .* (Δ .- s) .- Δ .* u.
function CRC.rrule(::typeof(NNop.∇online_softmax), Δ::ROCMatrix{T}, y::ROCMatrix{T}) where {T <: HipFloat}
    dx = NNop.∇online_softmax(Δ, y)
    function ∇online_softmax_pullback(g)
        g = _dense(CRC.unthunk(g), y)
        Δa, ya = _aligned(Δ), _aligned(y)
        dΔ, dy = similar(y), similar(y)
        N, M = size(y)
        _check(ccall((:onionop_softmax_bwd_bwd, libonionop), Cint,
            (Ptr{Cvoid}, Cint, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}),
            _stream(), _dt(T), N, M, g, Δa, ya, dΔ, dy))
        return CRC.NoTangent(), dΔ, dy
    end
    return dx, ∇online_softmax_pullback
end

# ------------------------------------------------------------------------ RMS norm

function NNop._rms_norm(x::ROCMatrix{T}, w::ROCVector{W}; ϵ::Float32, offset::Float32 = 0f0) where {T <: HipFloat, W <: HipFloat}
    emb, n = size(x)
    @assert emb == length(w)
    x = _aligned(x)
    y = similar(x)
    rstd = ROCArray{Float32}(undef, n)
    _check(ccall((:onionop_rms_norm_fwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Cint, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Cfloat, Cfloat, Ptr{Cvoid}, Ptr{Cfloat}),
        _stream(), _dt(T), _dt(W), emb, n, x, w, ϵ, offset, y, rstd))
    return y, rstd
end

function NNop.∇rms_norm(Δ, rstd::ROCVector{Float32}, x::ROCMatrix{T}, w::ROCVector{W}; offset::Float32) where {T <: HipFloat, W <: HipFloat}
    emb, n = size(x)
    x = _aligned(x)
    Δ = _dense(Δ, x)
    ws_bytes = ccall((:onionop_rms_norm_bwd_workspace, libonionop), Csize_t, (Int64, Int64), emb, n)
    ws = ROCArray{UInt8}(undef, max(ws_bytes, 1))
    dx = similar(x)
    dw = ROCArray{Float32}(undef, emb)   # the reference returns Float32 dw
    _check(ccall((:onionop_rms_norm_bwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Cint, Int64, Int64, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid}, Cfloat,
         Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cvoid}, Csize_t),
        _stream(), _dt(T), _dt(W), emb, n, Δ, rstd, x, w, offset, dx, dw, ws, ws_bytes))
    return dx, dw
end

# ------------------------------------------------------------------------ layer norm

function NNop._layer_norm(x::ROCMatrix{T}, w::ROCVector{W}, b::ROCVector{W}; ϵ::Float32 = 1f-6) where {T <: HipFloat, W <: HipFloat}
    emb, n = size(x)
    x = _aligned(x)
    y = similar(x)
    μ = ROCArray{Float32}(undef, n)
    rstd = ROCArray{Float32}(undef, n)
    _check(ccall((:onionop_layer_norm_fwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Cint, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Cfloat, Ptr{Cvoid},
         Ptr{Cfloat}, Ptr{Cfloat}),
        _stream(), _dt(T), _dt(W), emb, n, x, w, b, ϵ, y, μ, rstd))
    return y, μ, rstd
end

function NNop.∇layer_norm(Δ, μ::ROCVector{Float32}, rstd::ROCVector{Float32}, x::ROCMatrix{T}, w::ROCVector{W},
                          b::ROCVector{W}) where {T <: HipFloat, W <: HipFloat}
    emb, n = size(x)
    x = _aligned(x)
    Δ = _dense(Δ, x)
    ws_bytes = ccall((:onionop_layer_norm_bwd_workspace, libonionop), Csize_t, (Int64, Int64), emb, n)
    ws = ROCArray{UInt8}(undef, max(ws_bytes, 1))
    dx = similar(x)
    dw, db = similar(w), similar(b)   # eltype(w), eltype(b), as the reference
    _check(ccall((:onionop_layer_norm_bwd, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Cint, Int64, Int64, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid},
         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Csize_t),
        _stream(), _dt(T), _dt(W), emb, n, Δ, μ, rstd, x, w, dx, dw, db, ws, ws_bytes))
    return dx, dw, db
end

# ------------------------------------------------------------------------ RoPE

# LlamaRotaryEmbedding on device positions (src/rope/llama_rope.jl:14-22): the tables come
# from the library's kernel, in the reference's Float32 arithmetic, each value rounded once.
function (emb::NNop.LlamaRotaryEmbedding)(position_ids::ROCMatrix{Float32})
    L, B = size(position_ids)
    c = ROCArray{Float32}(undef, emb.dim, L, B)
    s = ROCArray{Float32}(undef, emb.dim, L, B)
    _check(ccall((:onionop_llama_rotary_embedding, libonionop), Cint,
        (Ptr{Cvoid}, Int64, Int64, Int64, Int64, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cfloat}),
        _stream(), emb.dim, L, B, emb.base, position_ids, c, s))
    return c, s
end

# q (E, L, QH, B), k (E, L, KH, B); cos, sin (E, L, B) Float32 (rows 1..E/2 are read).
function NNop._llama_rope(q::ROCArray{T,4}, k::ROCArray{T,4}, cos::ROCArray{Float32,3}, sin::ROCArray{Float32,3};
                          bwd::Bool) where {T <: HipFloat}
    @assert size(q, 1) == size(k, 1)
    @assert size(q, 2) == size(k, 2)
    @assert size(q, 4) == size(k, 4)
    q, k = _aligned(q), _aligned(k)
    E, L, QH, B = size(q)
    KH = size(k, 3)
    qo, ko = similar(q), similar(k)   # out of place, as the reference's copies
    _check(ccall((:onionop_llama_rope, libonionop), Cint,
        (Ptr{Cvoid}, Cint, Int64, Int64, Int64, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cfloat},
         Cfloat, Ptr{Cvoid}, Ptr{Cvoid}),
        _stream(), _dt(T), E, L, QH, KH, B, q, k, cos, sin, bwd ? -1f0 : 1f0, qo, ko))
    return qo, ko
end

end
