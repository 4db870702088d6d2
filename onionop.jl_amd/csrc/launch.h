// launch.h -- internal launcher interface between the C ABI (abi.cpp) and the kernels.
// Every launcher only enqueues on `s` and returns false for a configuration it has no
// kernel for; validation happens in abi.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace onionop {

struct AttnArgs {
    int64_t E, QL, KL, QH, KH, B;
    const void *q, *k, *v, *pair;
    const uint8_t* kpad;
    int causal;
    float scale;
    // forward
    void* o;
    float *ms, *ls;
    // backward
    const void *dO, *o_in;
    const float *ms_in, *ls_in;
    int qk_fp16;
    void *dq, *dk, *dv, *dpair;
    float *lse2, *delta;  // workspace: log2-domain log-sum-exp and rowsum(dO o), (B, QH, QL)
    // Fused ∇llama_rope (backward only; nullptr: none): dq and dk come out w.r.t. q and k
    // before the rotation.  cos / sin are (rope_rows, E) float32, one row per (batch,
    // position) -- b L + pos for dense tensors (QL == KL), the packed row for packed ones
    // (cu_q == cu_k).
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    int64_t rope_rows = 0;
    // Packed variable-length sequences (cu_q == nullptr: dense).  With them, B counts
    // the sequences, QL / KL are the longest lengths (they size the grids), tensors are
    // (QH, Tq, E) / (KH, Tk, E), statistics (QH, Tq), and cu_q / cu_k hold B + 1 offsets.
    const int *cu_q = nullptr, *cu_k = nullptr;
    int64_t Tq = 0, Tk = 0;
    // Key-range split of the four-head bias dQ (dq_splits > 1): float32 partial rows in
    // the workspace, dq_splits x (B, QH, QL, E).
    float* dq_part = nullptr;
    int dq_splits = 1;
    // Query-range split of the dK / dV (kv_splits > 1; four-head bias or GQA): float32
    // partial rows, 2 x kv_splits x (B, KH, KL, E) (dK partials, then dV).
    float* kv_part = nullptr;
    int kv_splits = 1;
};

bool launch_attn_fwd(hipStream_t s, int dt, const AttnArgs& a);
// stages: bit 0 = preprocess, bit 1 = dK/dV, bit 2 = dQ (+ dpair).
enum { kBwdPre = 1, kBwdDkDv = 2, kBwdDq = 4, kBwdAll = 7 };
bool launch_attn_bwd(hipStream_t s, int dt, const AttnArgs& a, int stages);

bool launch_softmax_fwd(hipStream_t s, int dt, int64_t n, int64_t rows, const void* x, void* y);
bool launch_softmax_bwd(hipStream_t s, int dt, int64_t n, int64_t rows, const void* dy, const void* y, void* dx);
bool launch_softmax_bwd_bwd(hipStream_t s, int dt, int64_t n, int64_t rows, const void* g, const void* dy,
                            const void* y, void* d_dy, void* d_y);
bool launch_rms_fwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* x, const void* w,
                    float eps, float offset, void* y, float* rstd);
bool launch_rms_bwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* dy, const float* rstd,
                    const void* x, const void* w, float offset, void* dx, float* dw, float* ws);
bool launch_ln_fwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* x, const void* w,
                   const void* b, float eps, void* y, float* mu, float* rstd);
bool launch_ln_bwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* dy, const float* mu,
                   const float* rstd, const void* x, const void* w, void* dx, void* dw, void* db, float* ws);
bool launch_rope_table(hipStream_t s, int64_t dim, int64_t rows, float base, const float* pos, float* cosv,
                       float* sinv);
bool launch_rope(hipStream_t s, int dt, int64_t E, int64_t L, int64_t QH, int64_t KH, int64_t B, const void* q,
                 const void* k, const float* cosv, const float* sinv, float sign, void* qo, void* ko);

// Compute units of the current device (cached per device; 0 if the query fails).
int device_cu_count();
// Key ranges the dQ of a 16-bit call spreads over (1: none), a function of the shape only:
// with a pair bias, four-head workgroups on a grid of fewer than 192 of them take enough
// ranges to make about 256 workgroups; at E = 256 without one (causal), a grid of at most
// 256 workgroups takes enough to make about 512.  At most 8 ranges, each of at least two
// 32-key tiles.
int dq_key_splits(int dt, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t B);
// Query ranges the dK / dV spreads over (1: none), a function of the shape only: with a
// pair bias (QH = KH) by the same rule as the dQ (four kv heads per workgroup); without
// one, for GQA (QH > KH) on grids of fewer than 1024 one-wave dK/dV workgroups, towards
// 1024 of them over the rep q heads' query tiles; at E >= 128 (the two-wave kernel) for
// 8 or more q heads per kv head, and at E = 256 on grids of at most 256 workgroups
// (towards 512).  Ranges hold at least two tiles.
int kv_query_splits(int dt, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH, int64_t B);

// Longest row (elements) the row-wise kernels keep in registers for dtype dt.
int64_t max_row_elems(int dt);
// Number of workgroups (= float32 partial rows in the workspace) of the norm backward.
int64_t norm_bwd_groups(int64_t rows, int64_t n);
// float32 workspace elements per weight gradient of the norm backward (partial rows).
int64_t norm_bwd_ws_floats(int64_t rows, int64_t n);

}  // namespace onionop
