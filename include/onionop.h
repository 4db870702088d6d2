/*
 * onionop.h -- C ABI of libonionop_hip.so, the gfx950 (MI355X) implementation of
 * NNop's fused-kernel hot path: flash attention (causal, pair bias, GQA, key padding),
 * online softmax, RMS norm, layer norm and Llama RoPE, forward and backward.
 *
 * Every entry point replaces the body of one host launcher of the reference package
 * (MurrellGroup/ONIONop.jl, Julia module NNop); the reference file:line is given at
 * each declaration.  The public Julia functions and their ChainRules rrules stay as
 * they are and call these through `ccall`.
 *
 * Conventions
 *  - Arrays are dense and column-major, exactly as the Julia arrays they replace:
 *    an array documented as (d1, d2, d3, d4) has d1 contiguous.  (The same memory is
 *    a row-major C/torch tensor of shape (d4, d3, d2, d1).)
 *  - Dimensions are int64_t.  Element types are given by the ONIONOP_F32/F16/BF16
 *    codes below; statistics that travel from a forward to its backward (ms, ls,
 *    rstd, mu) are always float32.
 *  - `stream` is a hipStream_t (NULL = the default stream).  Every call only
 *    enqueues work on it; nothing synchronises, nothing allocates device memory.
 *    Workspace, where needed, is passed in by the caller; its size comes from the
 *    matching *_workspace() query.
 *  - Every call returns ONIONOP_OK (0) or a negative ONIONOP_E_* status.  The text
 *    of the last error of the calling thread is returned by onionop_last_error().
 *    Shape errors carry the reference's own messages.
 *  - All pointers are device pointers, except where stated.
 *  - Alignment: q, k, v, o, dO, dq, dk, dv, x, y, dx, dy, g and the RoPE in/outputs must
 *    be 16-byte aligned (the kernels use 16-byte vector accesses); a misaligned pointer
 *    returns ONIONOP_E_SHAPE before anything is enqueued.  Allocations are; a view that
 *    starts inside its allocation (a Julia `view`, an offset pointer) may not be, and the
 *    binding copies such an array into a fresh one first.  Weights, biases, statistics,
 *    the pair bias and the key mask have no alignment requirement (the four-head bias
 *    path is only taken when pair / dpair are 8-byte aligned).
 */
#ifndef ONIONOP_H
#define ONIONOP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * ONIONOP_F32_BF16X6 (attention entry points only): float32 tensors, exactly as
 * ONIONOP_F32, with every matrix product of the attention kernels computed on the bf16
 * matrix cores.  Each float32 operand is split exactly into three bf16 parts
 * (x = hi + mid + lo), and a product a b is accumulated in float32 from the six part
 * products a_i b_j of order up to 2^-16 |a b|; the dropped ones are below 2^-23 |a b|,
 * the size of one float32 rounding.  Softmax, scaling, masks and all accumulation stay
 * float32.  No counterpart in the reference (its Float32 path uses float32 FMAs); it
 * trades nothing measurable in accuracy for the bf16 matrix-core rate.
 */
enum onionop_dtype { ONIONOP_F32 = 0, ONIONOP_F16 = 1, ONIONOP_BF16 = 2, ONIONOP_F32_BF16X6 = 3 };

enum onionop_status {
    ONIONOP_OK = 0,
    ONIONOP_E_SHAPE = -1,        /* shape / size mismatch (reference `error(...)`, `@assert`) */
    ONIONOP_E_DTYPE = -2,        /* unknown or unsupported element type                       */
    ONIONOP_E_UNSUPPORTED = -3,  /* valid request the library has no kernel for (e.g. E=512) */
    ONIONOP_E_HIP = -4,          /* a HIP runtime call failed                                  */
    ONIONOP_E_NULL = -5,         /* a required pointer is NULL                                 */
    ONIONOP_E_WORKSPACE = -6     /* workspace missing or smaller than the *_workspace() size   */
};

/* Message of the last failed call on this thread ("" if none).  Host pointer, owned
 * by the library, valid until the next call on the same thread. */
const char* onionop_last_error(void);

/* ABI revision of this header (bumped on any signature change). */
int onionop_abi_version(void);
#define ONIONOP_ABI_VERSION 2

/* LDS bytes per workgroup of `device` (cached once per device).
 * Replaces NNop.shared_memory / _shared_memory(::ROCBackend)
 * (src/NNop.jl:27-30, ext/NNopAMDGPUExt.jl:6-9). */
int onionop_device_lds_bytes(int device, size_t* bytes_out /* host pointer */);

/* ------------------------------------------------------------------ attention */

/*
 * Flash attention forward.  Replaces the body of `_flash_attention`
 * (src/attention.jl:145-197) and its kernel `_flash_attention_fwd!`
 * (src/attention.jl:8-143).
 *   q    (E, QL, QH, B)        dtype
 *   k, v (E, KL, KH, B)        dtype
 *   pair (QH, QL, KL, B)       dtype, nullable: additive bias after scaling
 *   kpad (KL, B)               uint8 (Julia Bool), nullable: 0 = masked key
 *   o    (E, QL, QH, B)        dtype, output, normalised
 *   ms, ls (QL, QH, B)         float32 outputs: running row max and row denominator of
 *                              the online softmax, carried to the backward
 * scale multiplies Q.K before the bias; the reference passes T(1/sqrt(E))
 * (src/attention.jl:166).  E must be a power of two in {16, 32, 64, 128, 256};
 * QH % KH == 0 (q head j uses kv head j / (QH/KH), src/attention.jl:36).
 * Limits of the library (ONIONOP_E_UNSUPPORTED beyond them): L * E * sizeof(T) < 2^31
 * bytes per (head, batch) slice of q/k/v, and with a bias 64 * QL * QH * sizeof(T) < 2^32
 * (the kernels address 64 key rows of one bias slice with 32-bit offsets).
 * Rows whose keys are all masked give o = 0, ms = -Inf, ls = 0 (the reference
 * produces NaN there).
 */
int onionop_flash_attn_fwd(void* stream, int dtype,
                           int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH, int64_t B,
                           const void* q, const void* k, const void* v,
                           const void* pair, const uint8_t* kpad,
                           int causal, float scale,
                           void* o, float* ms, float* ls);

/* Bytes of workspace the backward entry points use for these sizes: the log-sum-exp and
 * rowsum(dO o) of every query row, and, for 16-bit calls on small grids (with a pair
 * bias, GQA, or E = 256), float32 partial rows of the range splits that spread a dQ's
 * keys or a dK / dV's queries over several workgroups.  A workspace of only 8 bytes per
 * query row plus 256 also works; the kernels then run unsplit (same results to rounding). */
size_t onionop_flash_attn_bwd_workspace(int dtype, int64_t E, int64_t QL, int64_t KL,
                                        int64_t QH, int64_t KH, int64_t B);

/*
 * Flash attention backward.  Replaces the body of `∇flash_attention`
 * (src/attention_bwd.jl:213-303) with its kernels `_flash_attention_bwd_preprocess!`
 * (src/attention_bwd.jl:177-211) and `_flash_attention_bwd!` (src/attention_bwd.jl:1-175).
 *   dO   (E, QL, QH, B)        dtype, cotangent of o (dense)
 *   o, ms, ls                  as produced by onionop_flash_attn_fwd
 *   q, k, v, pair, kpad, causal, scale  as given to the forward
 *   dq   (E, QL, QH, B), dk, dv (E, KL, KH, B)   dtype outputs (overwritten)
 *   dpair (QH, QL, KL, B)      dtype output, required iff pair != NULL (overwritten;
 *                              entries of causally masked pairs are 0)
 * qk_fp16 != 0 rounds Q and K to float16 before every product that uses them, as the
 * reference backward does for every element type (src/attention_bwd.jl:20-21,
 * src/attention.jl:219); it only changes results for dtype F32.  GQA gradients are
 * summed over the q heads of a group without atomics (deterministic).
 */
int onionop_flash_attn_bwd(void* stream, int dtype,
                           int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH, int64_t B,
                           const void* dO, const void* o, const float* ms, const float* ls,
                           const void* q, const void* k, const void* v,
                           const void* pair, const uint8_t* kpad,
                           int causal, float scale, int qk_fp16,
                           void* dq, void* dk, void* dv, void* dpair,
                           void* workspace, size_t workspace_bytes);

/*
 * onionop_flash_attn_bwd without a workspace argument and without any allocation.
 * No counterpart in the reference: this entry point is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as onionop_flash_attn_bwd; the workspace is a
 * device array the library owns, 16 MiB on each GPU it runs on, held until the process
 * ends, so B * QH * QL may be at most 2097120 query rows (8 bytes each); larger calls
 * return ONIONOP_E_UNSUPPORTED without enqueueing anything.  Every call on one GPU uses
 * that GPU's array: calls whose kernels overlap on one GPU (on different streams, or from
 * several threads) race and give wrong results, so serialise them.  Nothing in the array
 * needs to be zero between calls.
 */
int onionop_flash_attn_bwd_noalloc(void* stream, int dtype,
                                   int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH, int64_t B,
                                   const void* dO, const void* o, const float* ms, const float* ls,
                                   const void* q, const void* k, const void* v,
                                   const void* pair, const uint8_t* kpad,
                                   int causal, float scale, int qk_fp16,
                                   void* dq, void* dk, void* dv, void* dpair);

/*
 * The three stages onionop_flash_attn_bwd runs, callable one by one (same arguments,
 * same workspace; call them in this order on one stream).
 *  _preprocess: delta = rowsum(dO .* o) and the log-sum-exp of every query row into the
 *               workspace.  Replaces `_flash_attention_bwd_preprocess!`
 *               (src/attention_bwd.jl:177-211).
 *  _dkdv:       dk, dv.  With _dq, replaces `_flash_attention_bwd!`
 *               (src/attention_bwd.jl:1-175).
 *  _dq:         dq and dpair.
 */
int onionop_flash_attn_bwd_preprocess(void* stream, int dtype, int64_t E, int64_t QL, int64_t QH, int64_t B,
                                      const void* dO, const void* o, const float* ms, const float* ls,
                                      void* workspace, size_t workspace_bytes);
int onionop_flash_attn_bwd_dkdv(void* stream, int dtype,
                                int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH, int64_t B,
                                const void* dO, const void* q, const void* k, const void* v,
                                const void* pair, const uint8_t* kpad, int causal, float scale, int qk_fp16,
                                void* dk, void* dv, void* workspace, size_t workspace_bytes);
int onionop_flash_attn_bwd_dq(void* stream, int dtype,
                              int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH, int64_t B,
                              const void* dO, const void* q, const void* k, const void* v,
                              const void* pair, const uint8_t* kpad, int causal, float scale, int qk_fp16,
                              void* dq, void* dpair, void* workspace, size_t workspace_bytes);

/* ------------------------------------------- attention, packed variable-length sequences */

/*
 * Flash attention over B packed sequences of different lengths, with no padding
 * anywhere.  The reference expresses variable lengths only through `kpad_mask`
 * (src/attention.jl:16,83-89), which still computes every padded query row and reads
 * every padded key; here sequence b is rows cu_seqlens_q[b] .. cu_seqlens_q[b+1] of
 * q (E, Tq, QH) (row-major (QH, Tq, E)) and rows cu_seqlens_k[b] .. cu_seqlens_k[b+1]
 * of k, v (E, Tk, KH), and only those rows are read or computed.  Causal masking is
 * within each sequence, aligned at its first row (key j <= query i).
 *   cu_seqlens_q, cu_seqlens_k: B + 1 nondecreasing int32 device offsets, [0] = 0,
 *     [B] <= Tq (Tk).  max_seqlen_q / max_seqlen_k bound every length (host values:
 *     they size the launch; longer sequences are cut to them).  Offsets outside
 *     [0, Tq] ([0, Tk]) are clamped into it.
 *   o like q; ms, ls (Tq, QH) (row-major (QH, Tq)).  Rows not in any sequence are not
 *     written.  No pair bias or key mask (use the dense entry points for those).
 */
int onionop_flash_attn_varlen_fwd(void* stream, int dtype,
                                  int64_t E, int64_t Tq, int64_t Tk, int64_t QH, int64_t KH, int64_t B,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int64_t max_seqlen_q, int64_t max_seqlen_k,
                                  const void* q, const void* k, const void* v, int causal, float scale,
                                  void* o, float* ms, float* ls);

/* Bytes of workspace onionop_flash_attn_varlen_bwd needs. */
size_t onionop_flash_attn_varlen_bwd_workspace(int dtype, int64_t E, int64_t Tq, int64_t QH);

/*
 * Backward of onionop_flash_attn_varlen_fwd: dq, dk, dv in the packed layouts of q, k,
 * v (dk / dv rows of keys in no sequence are not written).  Same conventions as
 * onionop_flash_attn_bwd otherwise (qk_fp16 for Float32).
 */
int onionop_flash_attn_varlen_bwd(void* stream, int dtype,
                                  int64_t E, int64_t Tq, int64_t Tk, int64_t QH, int64_t KH, int64_t B,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int64_t max_seqlen_q, int64_t max_seqlen_k,
                                  const void* dO, const void* o, const float* ms, const float* ls,
                                  const void* q, const void* k, const void* v, int causal, float scale, int qk_fp16,
                                  void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes);

/*
 * ∇flash_attention followed by ∇llama_rope in one backward: the pullback of
 * flash_attention(llama_rope(q, k; cos, sin)..., v) for the rrules of both
 * (src/attention_crc.jl:16-31, src/rope/llama_rope.jl:94-98).  Arguments as
 * onionop_flash_attn_bwd, with q and k the rotated tensors the forward used (the output of
 * onionop_llama_rope), and cos / sin (B, L, E) float32 the tables of that rotation
 * (QL == KL == L); dq and dk come out w.r.t. the tensors before the rotation, as the
 * reference's ∇llama_rope (sin_sign = -1) would give them.  The rotation is applied to the
 * float32 dQ / dK accumulators before they are stored, so no separate pass over dq and dk
 * runs.  No counterpart launcher in the reference: it composes the two rrules.
 */
int onionop_flash_attn_bwd_rope(void* stream, int dtype,
                                int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH, int64_t B,
                                const void* dO, const void* o, const float* ms, const float* ls,
                                const void* q, const void* k, const void* v,
                                const void* pair, const uint8_t* kpad,
                                const float* cos, const float* sin,
                                int causal, float scale, int qk_fp16,
                                void* dq, void* dk, void* dv, void* dpair,
                                void* workspace, size_t workspace_bytes);

/*
 * The same for packed sequences: onionop_flash_attn_varlen_bwd with the fused ∇llama_rope.
 * q and k must be packed alike (cu_seqlens_q == cu_seqlens_k, Tq == Tk); cos / sin are
 * (Tq, E) float32, one row per packed position (positions restart per sequence).
 */
int onionop_flash_attn_varlen_bwd_rope(void* stream, int dtype,
                                       int64_t E, int64_t Tq, int64_t Tk, int64_t QH, int64_t KH, int64_t B,
                                       const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                       int64_t max_seqlen_q, int64_t max_seqlen_k,
                                       const void* dO, const void* o, const float* ms, const float* ls,
                                       const void* q, const void* k, const void* v,
                                       const float* cos, const float* sin,
                                       int causal, float scale, int qk_fp16,
                                       void* dq, void* dk, void* dv,
                                       void* workspace, size_t workspace_bytes);

/* -------------------------------------------------------------------- softmax */

/*
 * Online softmax over dim 1 of x (N, M): y[:, j] = exp(x[:, j] - max) / sum.
 * Replaces `online_softmax` (src/softmax.jl:60-68) and its kernel
 * `online_softmax!` (src/softmax.jl:19-58).  Computed in float32; y has x's dtype.
 * Any N up to 2^29 - 1: rows a workgroup's registers cannot hold (N > 16384 float32 /
 * 32768 16-bit, or N > 4096 when N * sizeof(T) is not a multiple of 16) are streamed with
 * the online (max, sum) merge of the reference's md_reduce (src/softmax.jl:1-16,204-253).
 * The same row-length rule holds for the softmax backward and the norms below.
 */
int onionop_softmax_fwd(void* stream, int dtype, int64_t N, int64_t M,
                        const void* x, void* y);

/*
 * Softmax backward: dx = y .* dy - y .* sum(y .* dy; dims=1).
 * Replaces `∇online_softmax` (src/softmax.jl:70-80), which the reference runs as
 * broadcasts plus a reduction.  dy, y, dx share `dtype`.
 */
int onionop_softmax_bwd(void* stream, int dtype, int64_t N, int64_t M,
                        const void* dy, const void* y, void* dx);

/*
 * Pullback of the softmax backward, for second derivatives: given g = dL/d(dx) of
 * dx = onionop_softmax_bwd(dy, y), with s = sum(dy .* y) and u = sum(g .* y) per column,
 *   d_dy = y .* (g - u),   d_y = g .* (dy - s) - dy .* u.
 * Replaces the reference's second-order path, the `within_gradient` branch of
 * `∇online_softmax` (src/softmax.jl:71-74), which keeps the backward as differentiable
 * broadcasts for the AD system.  All five tensors share `dtype`.
 */
int onionop_softmax_bwd_bwd(void* stream, int dtype, int64_t N, int64_t M,
                            const void* g, const void* dy, const void* y,
                            void* d_dy, void* d_y);

/* ------------------------------------------------------------------- RMS norm */

/*
 * y = (offset + w) .* x .* rstd, rstd = 1/sqrt(mean(x.^2; dims=1) + eps).
 * Replaces `_rms_norm` (src/rms_norm.jl:117-137) and `_rms_norm!` (src/rms_norm.jl:3-38).
 *   x (emb, n) dtype_x, w (emb) dtype_w, y (emb, n) dtype_x, rstd (n) float32.
 */
int onionop_rms_norm_fwd(void* stream, int dtype_x, int dtype_w, int64_t emb, int64_t n,
                         const void* x, const void* w, float eps, float offset,
                         void* y, float* rstd);

size_t onionop_rms_norm_bwd_workspace(int64_t emb, int64_t n);

/*
 * RMS norm backward.  Replaces `∇rms_norm` (src/rms_norm.jl:139-169) and
 * `_∇rms_norm!` (src/rms_norm.jl:43-115), including the column sum of the dw
 * partials (src/rms_norm.jl:162-167), which runs here as a second fused kernel.
 *   dy (emb, n) dtype_x, rstd (n) f32, x, w as forward.
 *   dx (emb, n) dtype_x, dw (emb) float32 (the reference returns Float32 dw).
 */
int onionop_rms_norm_bwd(void* stream, int dtype_x, int dtype_w, int64_t emb, int64_t n,
                         const void* dy, const float* rstd, const void* x, const void* w,
                         float offset, void* dx, float* dw,
                         void* workspace, size_t workspace_bytes);

/* ----------------------------------------------------------------- layer norm */

/*
 * y = (x - mu) .* rstd .* w .+ b with biased variance, two-pass.
 * Replaces `_layer_norm` (src/layer_norm.jl:150-170) and `_layer_norm!`
 * (src/layer_norm.jl:8-63).
 *   x (emb, n) dtype_x; w, b (emb) dtype_w; y (emb, n) dtype_x; mu, rstd (n) float32.
 */
int onionop_layer_norm_fwd(void* stream, int dtype_x, int dtype_w, int64_t emb, int64_t n,
                           const void* x, const void* w, const void* b, float eps,
                           void* y, float* mu, float* rstd);

size_t onionop_layer_norm_bwd_workspace(int64_t emb, int64_t n);

/*
 * Layer norm backward.  Replaces `∇layer_norm` (src/layer_norm.jl:172-204) and
 * `_∇layer_norm!` (src/layer_norm.jl:65-148), including the partial sums
 * (src/layer_norm.jl:197-202), accumulated here in float32 and rounded once.
 *   dx (emb, n) dtype_x; dw, db (emb) dtype_w.
 */
int onionop_layer_norm_bwd(void* stream, int dtype_x, int dtype_w, int64_t emb, int64_t n,
                           const void* dy, const float* mu, const float* rstd,
                           const void* x, const void* w,
                           void* dx, void* dw, void* db,
                           void* workspace, size_t workspace_bytes);

/* ----------------------------------------------------------------------- RoPE */

/*
 * Llama (rotate-half, non-interleaved) rotary embedding of q and k, out of place.
 * Replaces `_llama_rope` (src/rope/llama_rope.jl:69-89) and `llama_rope!`
 * (src/rope/llama_rope.jl:24-65); `llama_rope` is sin_sign = +1, `∇llama_rope`
 * is sin_sign = -1 (src/rope/llama_rope.jl:86,91-92).
 *   q (E, L, QH, B), k (E, L, KH, B) dtype; cos, sin (E, L, B) float32, of which
 *   rows 1..E/2 are read; q_out, k_out like q, k (may alias q, k).
 * For i < E/2, j = i + E/2:  out_i = x_i c - x_j s,  out_j = x_j c + x_i s,
 * with c = cos[i], s = sin_sign * sin[i].
 */
int onionop_llama_rope(void* stream, int dtype, int64_t E, int64_t L,
                       int64_t QH, int64_t KH, int64_t B,
                       const void* q, const void* k, const float* cos, const float* sin,
                       float sin_sign, void* q_out, void* k_out);

/*
 * LlamaRotaryEmbedding(dim; base)(positions) on the device (src/rope/llama_rope.jl:1-22):
 * positions (L, B) float32 (row-major (B, L)); cos, sin (dim, L, B) float32 outputs
 * (row-major (B, L, dim)): inv_freq = 1 ./ base .^ ((0:2:dim-1) ./ dim) and
 * freqs = inv_freq .* positions in float32 as the reference computes them, then
 * cos / sin of vcat(freqs, freqs), each correctly rounded to float32.  dim must be even.
 */
int onionop_llama_rotary_embedding(void* stream, int64_t dim, int64_t L, int64_t B, int64_t base,
                                   const float* positions, float* cos, float* sin);

#ifdef __cplusplus
}
#endif

#endif /* ONIONOP_H */
