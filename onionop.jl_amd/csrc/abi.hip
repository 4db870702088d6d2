// abi.hip -- the extern "C" entry points of libonionop_hip.so declared in
// include/onionop.h: argument validation (with the reference's error messages),
// workspace sizing, and dispatch to the kernel launchers.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/onionop.h"
#include "launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = 0;
    return ONIONOP_OK;
}

// Status of the launches just enqueued on this thread.
int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ONIONOP_E_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

bool valid_dt(int dt) { return dt == ONIONOP_F32 || dt == ONIONOP_F16 || dt == ONIONOP_BF16; }
// attention also takes float32 computed with bf16x6 MFMA products
bool valid_attn_dt(int dt) { return valid_dt(dt) || dt == ONIONOP_F32_BF16X6; }
size_t dt_size(int dt) { return dt == ONIONOP_F32 || dt == ONIONOP_F32_BF16X6 ? 4 : 2; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

const char* dt_name(int dt) {
    return dt == 0 ? "Float32" : dt == 1 ? "Float16" : dt == 2 ? "BFloat16" : dt == 3 ? "Float32 (bf16x6)" : "?";
}

// Shape checks of _flash_attention / ∇flash_attention (src/attention.jl:153-156,
// src/attention_bwd.jl:224-227) plus what the library supports.
int check_attn(int dtype, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH, int64_t B) {
    if (!valid_attn_dt(dtype)) return fail(ONIONOP_E_DTYPE, "flash_attention: unsupported element type code %d", dtype);
    if (E < 0 || QL < 0 || KL < 0 || QH < 0 || KH < 0 || B < 0)
        return fail(ONIONOP_E_SHAPE, "flash_attention: negative dimension");
    if (!is_pow2(E)) return fail(ONIONOP_E_SHAPE, "Only power-of-2 embedding dims are supported.");
    if (KH == 0 || QH % KH != 0)
        return fail(ONIONOP_E_SHAPE, "Number of query heads `%lld` must be divisible by number of KV heads `%lld`.",
                    (long long)QH, (long long)KH);
    if (E < 16 || E > 256)
        return fail(ONIONOP_E_UNSUPPORTED,
                    "flash_attention: embedding dim %lld not supported (16, 32, 64, 128 or 256)", (long long)E);
    if (QL > (1LL << 30) || KL > (1LL << 30) || QH > 65535 || B > 65535)
        return fail(ONIONOP_E_UNSUPPORTED, "flash_attention: dimensions too large");
    // The kernels address one (head, batch) slice of q/k/v with 32-bit byte offsets.
    if ((QL > KL ? QL : KL) * E * (int64_t)dt_size(dtype) >= (1LL << 31))
        return fail(ONIONOP_E_UNSUPPORTED, "flash_attention: sequence too long (L*E*sizeof(T) must be below 2^31 bytes)");
    return ok();
}

// The bias kernels address 64 key rows of one (batch, head) bias slice with 32-bit byte
// offsets.
int check_pair(const void* pair, int dtype, int64_t QL, int64_t QH) {
    if (pair != nullptr && 64 * QL * QH * (int64_t)dt_size(dtype) >= (1LL << 32))
        return fail(ONIONOP_E_UNSUPPORTED,
                    "flash_attention: pair bias too large (64*QL*QH*sizeof(T) must be below 2^32 bytes)");
    return ok();
}

std::mutex g_lds_mu;
size_t g_lds[64];
bool g_lds_set[64];

}  // namespace

// Scratch of onionop_flash_attn_bwd_noalloc: the backward's workspace (per query row, the
// log2-sum-exp and delta, 8 bytes, written by the dQ kernel before the dK/dV kernel reads
// them) in a device array the library owns, so that entry point allocates nothing.  Each
// GPU the library runs on holds its own copy until the process ends.  In host code the
// array's name is not a device address: the address is looked up once per device with
// hipGetSymbolAddress and only that pointer is used.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[64];  // device address of `scratch` on device d, once looked up

// The scratch array's address on the current device (looked up on the first call there).
int scratch_on_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(ONIONOP_E_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= 64) return fail(ONIONOP_E_HIP, "device ordinal %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return fail(ONIONOP_E_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return ONIONOP_OK;
}

}  // namespace

extern "C" {

const char* onionop_last_error(void) { return g_err; }

int onionop_abi_version(void) { return ONIONOP_ABI_VERSION; }

int onionop_device_lds_bytes(int device, size_t* bytes_out) {
    if (bytes_out == nullptr) return fail(ONIONOP_E_NULL, "onionop_device_lds_bytes: bytes_out is NULL");
    if (device < 0 || device >= 64) return fail(ONIONOP_E_SHAPE, "onionop_device_lds_bytes: bad device %d", device);
    std::lock_guard<std::mutex> lock(g_lds_mu);
    if (!g_lds_set[device]) {
        hipDeviceProp_t prop;
        const hipError_t e = hipGetDeviceProperties(&prop, device);
        if (e != hipSuccess) return fail(ONIONOP_E_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
        g_lds[device] = prop.sharedMemPerBlock;
        g_lds_set[device] = true;
    }
    *bytes_out = g_lds[device];
    return ok();
}

// ------------------------------------------------------------------ attention

int onionop_flash_attn_fwd(void* stream, int dtype, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH,
                           int64_t B, const void* q, const void* k, const void* v, const void* pair,
                           const uint8_t* kpad, int causal, float scale, void* o, float* ms, float* ls) {
    int st = check_attn(dtype, E, QL, KL, QH, KH, B);
    if (st) return st;
    if ((st = check_pair(pair, dtype, QL, QH))) return st;
    const bool any_q = QL * QH * B > 0, any_k = KL * KH * B > 0;
    if ((any_q && (!q || !o || !ms || !ls)) || (any_q && any_k && (!k || !v)))
        return fail(ONIONOP_E_NULL, "flash_attention: NULL tensor pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return fail(ONIONOP_E_SHAPE, "flash_attention: q, k, v and o must be 16-byte aligned");
    onionop::AttnArgs a{};
    a.E = E; a.QL = QL; a.KL = KL; a.QH = QH; a.KH = KH; a.B = B;
    a.q = q; a.k = k; a.v = v; a.pair = pair; a.kpad = kpad; a.causal = causal != 0; a.scale = scale;
    a.o = o; a.ms = ms; a.ls = ls;
    if (!onionop::launch_attn_fwd((hipStream_t)stream, dtype, a))
        return fail(ONIONOP_E_UNSUPPORTED, "flash_attention: no kernel for %s E=%lld", dt_name(dtype), (long long)E);
    return check_launch("flash_attention");
}

// The part of the backward workspace every call needs: lse2 and delta per query row.
static size_t bwd_ws_base(int64_t QL, int64_t QH, int64_t B) {
    if (QL <= 0 || QH <= 0 || B <= 0) return 0;
    const size_t rows = (size_t)QL * (size_t)QH * (size_t)B;
    return 2 * rows * sizeof(float) + 256;  // lse2 and delta, each 256-byte aligned
}

// Layout of the range splits' partial rows after lse2 / delta (offsets from the 256-byte
// aligned start, each 256-byte aligned): the dK / dV query ranges' rows, then the dQ key
// ranges' rows (pair bias only, so last: a workspace that holds only the first part still
// serves the GQA dK/dV split); bytes 0 where a shape takes no split.
struct BwdSplitLayout {
    size_t dq_off, dq_bytes, kv_off, kv_bytes;
};
static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
static BwdSplitLayout bwd_split_layout(int dtype, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH,
                                       int64_t B) {
    BwdSplitLayout l{};
    if (QL <= 0 || QH <= 0 || B <= 0) return l;
    const size_t rows = (size_t)QL * (size_t)QH * (size_t)B, rows_k = (size_t)KL * (size_t)KH * (size_t)B;
    const int nq = onionop::dq_key_splits(dtype, E, QL, KL, QH, B);
    const int nk = onionop::kv_query_splits(dtype, E, QL, KL, QH, KH, B);
    l.kv_off = align256(2 * rows * sizeof(float));
    l.kv_bytes = nk > 1 ? 2 * (size_t)nk * rows_k * (size_t)E * sizeof(float) : 0;
    l.dq_off = align256(l.kv_off + l.kv_bytes);
    l.dq_bytes = nq > 1 ? (size_t)nq * rows * (size_t)E * sizeof(float) : 0;
    return l;
}

size_t onionop_flash_attn_bwd_workspace(int dtype, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH,
                                        int64_t B) {
    const size_t base = bwd_ws_base(QL, QH, B);
    const BwdSplitLayout l = bwd_split_layout(dtype, E, QL, KL, QH, KH, B);
    if (base == 0 || (l.dq_bytes == 0 && l.kv_bytes == 0)) return base;
    return 256 + (l.dq_bytes > 0 ? l.dq_off + l.dq_bytes : l.kv_off + l.kv_bytes);
}

// Shared body of the backward entry points; `stages` selects which kernels run.
static int attn_bwd_common(const char* what, int stages, void* stream, int dtype, int64_t E, int64_t QL, int64_t KL,
                           int64_t QH, int64_t KH, int64_t B, const void* dO, const void* o, const float* ms,
                           const float* ls, const void* q, const void* k, const void* v, const void* pair,
                           const uint8_t* kpad, int causal, float scale, int qk_fp16, void* dq, void* dk, void* dv,
                           void* dpair, void* workspace, size_t workspace_bytes, const float* rope_cos = nullptr,
                           const float* rope_sin = nullptr) {
    int st = check_attn(dtype, E, QL, KL, QH, KH, B);
    if (st) return st;
    if ((st = check_pair(pair, dtype, QL, QH))) return st;
    const bool any_q = QL * QH * B > 0, any_k = KL * KH * B > 0;
    if (stages & onionop::kBwdPre) {
        if (any_q && (!dO || !o || !ms || !ls)) return fail(ONIONOP_E_NULL, "%s: NULL tensor pointer", what);
        if (!aligned16(dO) || !aligned16(o)) return fail(ONIONOP_E_SHAPE, "%s: tensors must be 16-byte aligned", what);
    }
    if (stages & (onionop::kBwdDkDv | onionop::kBwdDq)) {
        if ((any_q && (!dO || !q)) || (any_k && (!k || !v)))
            return fail(ONIONOP_E_NULL, "%s: NULL tensor pointer", what);
        if (!aligned16(dO) || !aligned16(q) || !aligned16(k) || !aligned16(v))
            return fail(ONIONOP_E_SHAPE, "%s: tensors must be 16-byte aligned", what);
    }
    if (stages & onionop::kBwdDkDv) {
        if (any_k && (!dk || !dv)) return fail(ONIONOP_E_NULL, "%s: NULL tensor pointer", what);
        if (!aligned16(dk) || !aligned16(dv)) return fail(ONIONOP_E_SHAPE, "%s: tensors must be 16-byte aligned", what);
    }
    if (stages & onionop::kBwdDq) {
        if ((pair == nullptr) != (dpair == nullptr))
            return fail(ONIONOP_E_NULL, "%s: dpair must be given exactly when pair is given", what);
        if (any_q && !dq) return fail(ONIONOP_E_NULL, "%s: NULL tensor pointer", what);
        if (!aligned16(dq)) return fail(ONIONOP_E_SHAPE, "%s: tensors must be 16-byte aligned", what);
    }
    // Calls need the lse2 / delta rows; the dQ of a pair-biased small grid uses the rest of
    // the full size for its key-range split when it is given (else it runs unsplit).
    const size_t need = bwd_ws_base(QL, QH, B);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(ONIONOP_E_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", what,
                    onionop_flash_attn_bwd_workspace(dtype, E, QL, KL, QH, KH, B), workspace_bytes);
    onionop::AttnArgs a{};
    a.E = E; a.QL = QL; a.KL = KL; a.QH = QH; a.KH = KH; a.B = B;
    a.q = q; a.k = k; a.v = v; a.pair = pair; a.kpad = kpad; a.causal = causal != 0; a.scale = scale;
    a.dO = dO; a.o_in = o; a.ms_in = ms; a.ls_in = ls; a.qk_fp16 = qk_fp16 != 0;
    a.dq = dq; a.dk = dk; a.dv = dv; a.dpair = dpair;
    if (rope_cos != nullptr || rope_sin != nullptr) {
        if (rope_cos == nullptr || rope_sin == nullptr) return fail(ONIONOP_E_NULL, "%s: NULL cos / sin table", what);
        if (QL != KL)
            return fail(ONIONOP_E_SHAPE, "%s: the rotary embedding needs q and k of one length (%lld != %lld)", what,
                        (long long)QL, (long long)KL);
        if (B * QL * E * 4 >= (1LL << 32))
            return fail(ONIONOP_E_UNSUPPORTED, "%s: cos / sin tables too large (B*L*E*4 must be below 2^32)", what);
        a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.rope_rows = B * QL;
    }
    if (need > 0) {
        uintptr_t base = (reinterpret_cast<uintptr_t>(workspace) + 255) & ~uintptr_t(255);
        const size_t rows = (size_t)QL * (size_t)QH * (size_t)B;
        a.lse2 = reinterpret_cast<float*>(base);
        a.delta = a.lse2 + rows;
        // The range splits (pair-biased dQ and dK/dV, GQA dK/dV, E = 256 dQ and dK/dV), each
        // where the workspace holds it; with the fused RoPE only the GQA dK/dV one (its
        // kernel rotates dK before writing the partials).
        {
            const BwdSplitLayout l = bwd_split_layout(dtype, E, QL, KL, QH, KH, B);
            const size_t lead = base - reinterpret_cast<uintptr_t>(workspace);
            if ((pair != nullptr || E >= 256) && rope_cos == nullptr && (stages & onionop::kBwdDq) && l.dq_bytes > 0 &&
                lead + l.dq_off + l.dq_bytes <= workspace_bytes) {
                a.dq_part = reinterpret_cast<float*>(base + l.dq_off);
                a.dq_splits = onionop::dq_key_splits(dtype, E, QL, KL, QH, B);
            }
            if ((stages & onionop::kBwdDkDv) && (rope_cos == nullptr || QH > KH) && l.kv_bytes > 0 &&
                lead + l.kv_off + l.kv_bytes <= workspace_bytes) {
                a.kv_part = reinterpret_cast<float*>(base + l.kv_off);
                a.kv_splits = onionop::kv_query_splits(dtype, E, QL, KL, QH, KH, B);
            }
        }
    }
    if (!onionop::launch_attn_bwd((hipStream_t)stream, dtype, a, stages))
        return fail(ONIONOP_E_UNSUPPORTED, "%s: no kernel for %s E=%lld", what, dt_name(dtype), (long long)E);
    return check_launch(what);
}

int onionop_flash_attn_bwd(void* stream, int dtype, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH,
                           int64_t B, const void* dO, const void* o, const float* ms, const float* ls,
                           const void* q, const void* k, const void* v, const void* pair, const uint8_t* kpad,
                           int causal, float scale, int qk_fp16, void* dq, void* dk, void* dv, void* dpair,
                           void* workspace, size_t workspace_bytes) {
    return attn_bwd_common("∇flash_attention", onionop::kBwdAll, stream, dtype, E, QL, KL, QH, KH, B, dO, o, ms, ls,
                           q, k, v, pair, kpad, causal, scale, qk_fp16, dq, dk, dv, dpair, workspace,
                           workspace_bytes);
}

int onionop_flash_attn_bwd_rope(void* stream, int dtype, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH,
                                int64_t B, const void* dO, const void* o, const float* ms, const float* ls,
                                const void* q, const void* k, const void* v, const void* pair, const uint8_t* kpad,
                                const float* cos, const float* sin, int causal, float scale, int qk_fp16, void* dq,
                                void* dk, void* dv, void* dpair, void* workspace, size_t workspace_bytes) {
    const char* what = "∇flash_attention ∘ ∇llama_rope";
    if (cos == nullptr || sin == nullptr) return fail(ONIONOP_E_NULL, "%s: NULL cos / sin table", what);
    return attn_bwd_common(what, onionop::kBwdAll, stream, dtype, E, QL, KL, QH, KH, B, dO, o, ms, ls, q, k, v, pair,
                           kpad, causal, scale, qk_fp16, dq, dk, dv, dpair, workspace, workspace_bytes, cos, sin);
}

int onionop_flash_attn_bwd_noalloc(void* stream, int dtype, int64_t E, int64_t QL, int64_t KL, int64_t QH,
                                   int64_t KH, int64_t B, const void* dO, const void* o, const float* ms,
                                   const float* ls, const void* q, const void* k, const void* v, const void* pair,
                                   const uint8_t* kpad, int causal, float scale, int qk_fp16, void* dq, void* dk,
                                   void* dv, void* dpair) {
    const char* what = "∇flash_attention (no allocation)";
    int st = check_attn(dtype, E, QL, KL, QH, KH, B);
    if (st) return st;
    const size_t need = bwd_ws_base(QL, QH, B);  // the key-range split is used when it fits too
    if (need > kScratchBytes)
        return fail(ONIONOP_E_UNSUPPORTED,
                    "%s: needs %zu bytes of scratch (8 per query row), the library holds %zu "
                    "(at most %zu query rows B*QH*QL); use onionop_flash_attn_bwd with a workspace",
                    what, need, kScratchBytes, (kScratchBytes - 256) / 8);
    void* ws = nullptr;
    if (need > 0 && (st = scratch_on_current_device(&ws))) return st;
    // Nothing in the scratch has to start at zero: every value the dK/dV kernel reads is
    // written first by the dQ kernel of the same call.
    return attn_bwd_common(what, onionop::kBwdAll, stream, dtype, E, QL, KL, QH, KH, B, dO, o, ms, ls, q, k, v, pair,
                           kpad, causal, scale, qk_fp16, dq, dk, dv, dpair, ws, need > 0 ? kScratchBytes : 0);
}

int onionop_flash_attn_bwd_preprocess(void* stream, int dtype, int64_t E, int64_t QL, int64_t QH, int64_t B,
                                      const void* dO, const void* o, const float* ms, const float* ls,
                                      void* workspace, size_t workspace_bytes) {
    return attn_bwd_common("∇flash_attention preprocess", onionop::kBwdPre, stream, dtype, E, QL, 0, QH, QH, B, dO,
                           o, ms, ls, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 1.0f, 0, nullptr, nullptr,
                           nullptr, nullptr, workspace, workspace_bytes);
}

int onionop_flash_attn_bwd_dkdv(void* stream, int dtype, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH,
                                int64_t B, const void* dO, const void* q, const void* k, const void* v,
                                const void* pair, const uint8_t* kpad, int causal, float scale, int qk_fp16,
                                void* dk, void* dv, void* workspace, size_t workspace_bytes) {
    return attn_bwd_common("∇flash_attention dK/dV", onionop::kBwdDkDv, stream, dtype, E, QL, KL, QH, KH, B, dO,
                           nullptr, nullptr, nullptr, q, k, v, pair, kpad, causal, scale, qk_fp16, nullptr, dk, dv,
                           nullptr, workspace, workspace_bytes);
}

int onionop_flash_attn_bwd_dq(void* stream, int dtype, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH,
                              int64_t B, const void* dO, const void* q, const void* k, const void* v,
                              const void* pair, const uint8_t* kpad, int causal, float scale, int qk_fp16,
                              void* dq, void* dpair, void* workspace, size_t workspace_bytes) {
    return attn_bwd_common("∇flash_attention dQ", onionop::kBwdDq, stream, dtype, E, QL, KL, QH, KH, B, dO, nullptr,
                           nullptr, nullptr, q, k, v, pair, kpad, causal, scale, qk_fp16, dq, nullptr, nullptr,
                           dpair, workspace, workspace_bytes);
}

// ------------------------------------------------------ attention, packed variable length

// Extra checks of the packed entry points: per-sequence limits as in check_attn (with the
// longest lengths), offsets present, packed lengths within the 32-bit offsets.
static int check_varlen(const char* what, int dtype, int64_t E, int64_t Tq, int64_t Tk, int64_t QH, int64_t KH,
                        int64_t B, const int32_t* cu_q, const int32_t* cu_k, int64_t max_q, int64_t max_k) {
    int st = check_attn(dtype, E, max_q, max_k, QH, KH, B);
    if (st) return st;
    if (Tq < 0 || Tk < 0) return fail(ONIONOP_E_SHAPE, "%s: negative dimension", what);
    if (Tq >= (1LL << 31) || Tk >= (1LL << 31)) return fail(ONIONOP_E_UNSUPPORTED, "%s: too many packed rows", what);
    if (B > 0 && (!cu_q || !cu_k)) return fail(ONIONOP_E_NULL, "%s: NULL sequence offsets", what);
    return ok();
}

static onionop::AttnArgs varlen_args(int64_t E, int64_t Tq, int64_t Tk, int64_t QH, int64_t KH, int64_t B,
                                     const int32_t* cu_q, const int32_t* cu_k, int64_t max_q, int64_t max_k,
                                     const void* q, const void* k, const void* v, int causal, float scale) {
    onionop::AttnArgs a{};
    a.E = E; a.QL = max_q; a.KL = max_k; a.QH = QH; a.KH = KH; a.B = B;
    a.q = q; a.k = k; a.v = v; a.pair = nullptr; a.kpad = nullptr; a.causal = causal != 0; a.scale = scale;
    a.cu_q = cu_q; a.cu_k = cu_k; a.Tq = Tq; a.Tk = Tk;
    return a;
}

int onionop_flash_attn_varlen_fwd(void* stream, int dtype, int64_t E, int64_t Tq, int64_t Tk, int64_t QH,
                                  int64_t KH, int64_t B, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int64_t max_seqlen_q, int64_t max_seqlen_k, const void* q, const void* k,
                                  const void* v, int causal, float scale, void* o, float* ms, float* ls) {
    const char* what = "flash_attention (varlen)";
    int st = check_varlen(what, dtype, E, Tq, Tk, QH, KH, B, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k);
    if (st) return st;
    const bool any_q = Tq * QH > 0, any_k = Tk * KH > 0;
    if ((any_q && (!q || !o || !ms || !ls)) || (any_q && any_k && (!k || !v)))
        return fail(ONIONOP_E_NULL, "%s: NULL tensor pointer", what);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return fail(ONIONOP_E_SHAPE, "%s: q, k, v and o must be 16-byte aligned", what);
    onionop::AttnArgs a = varlen_args(E, Tq, Tk, QH, KH, B, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                      q, k, v, causal, scale);
    a.o = o; a.ms = ms; a.ls = ls;
    if (!onionop::launch_attn_fwd((hipStream_t)stream, dtype, a))
        return fail(ONIONOP_E_UNSUPPORTED, "%s: no kernel for %s E=%lld", what, dt_name(dtype), (long long)E);
    return check_launch(what);
}

size_t onionop_flash_attn_varlen_bwd_workspace(int dtype, int64_t E, int64_t Tq, int64_t QH) {
    (void)dtype; (void)E;
    if (Tq <= 0 || QH <= 0) return 0;
    return 2 * (size_t)Tq * (size_t)QH * sizeof(float) + 256;  // lse2 and delta per packed query row
}

static int varlen_bwd_common(const char* what, void* stream, int dtype, int64_t E, int64_t Tq, int64_t Tk,
                             int64_t QH, int64_t KH, int64_t B, const int32_t* cu_seqlens_q,
                             const int32_t* cu_seqlens_k, int64_t max_seqlen_q, int64_t max_seqlen_k, const void* dO,
                             const void* o, const float* ms, const float* ls, const void* q, const void* k,
                             const void* v, const float* rope_cos, const float* rope_sin, int causal, float scale,
                             int qk_fp16, void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes) {
    int st = check_varlen(what, dtype, E, Tq, Tk, QH, KH, B, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k);
    if (st) return st;
    const bool any_q = Tq * QH > 0, any_k = Tk * KH > 0;
    if ((any_q && (!dO || !o || !ms || !ls || !q || !dq)) || (any_k && (!k || !v || !dk || !dv)))
        return fail(ONIONOP_E_NULL, "%s: NULL tensor pointer", what);
    if (!aligned16(dO) || !aligned16(o) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dq) ||
        !aligned16(dk) || !aligned16(dv))
        return fail(ONIONOP_E_SHAPE, "%s: tensors must be 16-byte aligned", what);
    const size_t need = onionop_flash_attn_varlen_bwd_workspace(dtype, E, Tq, QH);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(ONIONOP_E_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", what, need, workspace_bytes);
    onionop::AttnArgs a = varlen_args(E, Tq, Tk, QH, KH, B, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                      q, k, v, causal, scale);
    a.dO = dO; a.o_in = o; a.ms_in = ms; a.ls_in = ls; a.qk_fp16 = qk_fp16 != 0;
    a.dq = dq; a.dk = dk; a.dv = dv; a.dpair = nullptr;
    if (rope_cos != nullptr || rope_sin != nullptr) {
        if (rope_cos == nullptr || rope_sin == nullptr) return fail(ONIONOP_E_NULL, "%s: NULL cos / sin table", what);
        if (cu_seqlens_q != cu_seqlens_k || Tq != Tk)
            return fail(ONIONOP_E_SHAPE, "%s: the rotary embedding needs q and k packed alike (one cu_seqlens)", what);
        if (Tq * E * 4 >= (1LL << 32))
            return fail(ONIONOP_E_UNSUPPORTED, "%s: cos / sin tables too large (Tq*E*4 must be below 2^32)", what);
        a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.rope_rows = Tq;
    }
    if (need > 0) {
        uintptr_t base = (reinterpret_cast<uintptr_t>(workspace) + 255) & ~uintptr_t(255);
        a.lse2 = reinterpret_cast<float*>(base);
        a.delta = a.lse2 + (size_t)Tq * (size_t)QH;
    }
    if (!onionop::launch_attn_bwd((hipStream_t)stream, dtype, a, onionop::kBwdAll))
        return fail(ONIONOP_E_UNSUPPORTED, "%s: no kernel for %s E=%lld", what, dt_name(dtype), (long long)E);
    return check_launch(what);
}

int onionop_flash_attn_varlen_bwd(void* stream, int dtype, int64_t E, int64_t Tq, int64_t Tk, int64_t QH,
                                  int64_t KH, int64_t B, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int64_t max_seqlen_q, int64_t max_seqlen_k, const void* dO, const void* o,
                                  const float* ms, const float* ls, const void* q, const void* k, const void* v,
                                  int causal, float scale, int qk_fp16, void* dq, void* dk, void* dv, void* workspace,
                                  size_t workspace_bytes) {
    return varlen_bwd_common("∇flash_attention (varlen)", stream, dtype, E, Tq, Tk, QH, KH, B, cu_seqlens_q,
                             cu_seqlens_k, max_seqlen_q, max_seqlen_k, dO, o, ms, ls, q, k, v, nullptr, nullptr, causal,
                             scale, qk_fp16, dq, dk, dv, workspace, workspace_bytes);
}

int onionop_flash_attn_varlen_bwd_rope(void* stream, int dtype, int64_t E, int64_t Tq, int64_t Tk, int64_t QH,
                                       int64_t KH, int64_t B, const int32_t* cu_seqlens_q,
                                       const int32_t* cu_seqlens_k, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                       const void* dO, const void* o, const float* ms, const float* ls, const void* q,
                                       const void* k, const void* v, const float* cos, const float* sin, int causal,
                                       float scale, int qk_fp16, void* dq, void* dk, void* dv, void* workspace,
                                       size_t workspace_bytes) {
    const char* what = "∇flash_attention ∘ ∇llama_rope (varlen)";
    if (cos == nullptr || sin == nullptr) return fail(ONIONOP_E_NULL, "%s: NULL cos / sin table", what);
    return varlen_bwd_common(what, stream, dtype, E, Tq, Tk, QH, KH, B, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                             max_seqlen_k, dO, o, ms, ls, q, k, v, cos, sin, causal, scale, qk_fp16, dq, dk, dv,
                             workspace, workspace_bytes);
}

// -------------------------------------------------------------------- softmax

static int check_rows(const char* what, int dtype, int64_t n, int64_t rows) {
    if (!valid_dt(dtype)) return fail(ONIONOP_E_DTYPE, "%s: unsupported element type code %d", what, dtype);
    if (n < 0 || rows < 0) return fail(ONIONOP_E_SHAPE, "%s: negative dimension", what);
    const int64_t lim = onionop::max_row_elems(dtype);
    if (n > lim)
        return fail(ONIONOP_E_UNSUPPORTED, "%s: reduction length %lld exceeds the supported %lld", what,
                    (long long)n, (long long)lim);
    return ok();
}

int onionop_softmax_fwd(void* stream, int dtype, int64_t N, int64_t M, const void* x, void* y) {
    int st = check_rows("online_softmax", dtype, N, M);
    if (st) return st;
    if (N * M > 0 && (!x || !y)) return fail(ONIONOP_E_NULL, "online_softmax: NULL tensor pointer");
    if (!aligned16(x) || !aligned16(y)) return fail(ONIONOP_E_SHAPE, "online_softmax: tensors must be 16-byte aligned");
    if (!onionop::launch_softmax_fwd((hipStream_t)stream, dtype, N, M, x, y))
        return fail(ONIONOP_E_UNSUPPORTED, "online_softmax: no kernel for N=%lld", (long long)N);
    return check_launch("online_softmax");
}

int onionop_softmax_bwd(void* stream, int dtype, int64_t N, int64_t M, const void* dy, const void* y, void* dx) {
    int st = check_rows("∇online_softmax", dtype, N, M);
    if (st) return st;
    if (N * M > 0 && (!dy || !y || !dx)) return fail(ONIONOP_E_NULL, "∇online_softmax: NULL tensor pointer");
    if (!aligned16(dy) || !aligned16(y) || !aligned16(dx))
        return fail(ONIONOP_E_SHAPE, "∇online_softmax: tensors must be 16-byte aligned");
    if (!onionop::launch_softmax_bwd((hipStream_t)stream, dtype, N, M, dy, y, dx))
        return fail(ONIONOP_E_UNSUPPORTED, "∇online_softmax: no kernel for N=%lld", (long long)N);
    return check_launch("∇online_softmax");
}

int onionop_softmax_bwd_bwd(void* stream, int dtype, int64_t N, int64_t M, const void* g, const void* dy,
                            const void* y, void* d_dy, void* d_y) {
    const char* what = "∇online_softmax pullback";
    int st = check_rows(what, dtype, N, M);
    if (st) return st;
    if (N * M > 0 && (!g || !dy || !y || !d_dy || !d_y)) return fail(ONIONOP_E_NULL, "%s: NULL tensor pointer", what);
    if (!aligned16(g) || !aligned16(dy) || !aligned16(y) || !aligned16(d_dy) || !aligned16(d_y))
        return fail(ONIONOP_E_SHAPE, "%s: tensors must be 16-byte aligned", what);
    if (!onionop::launch_softmax_bwd_bwd((hipStream_t)stream, dtype, N, M, g, dy, y, d_dy, d_y))
        return fail(ONIONOP_E_UNSUPPORTED, "%s: no kernel for N=%lld", what, (long long)N);
    return check_launch(what);
}

// ------------------------------------------------------------------- RMS norm

int onionop_rms_norm_fwd(void* stream, int dtype_x, int dtype_w, int64_t emb, int64_t n, const void* x,
                         const void* w, float eps, float offset, void* y, float* rstd) {
    int st = check_rows("rms_norm", dtype_x, emb, n);
    if (st) return st;
    if (!valid_dt(dtype_w)) return fail(ONIONOP_E_DTYPE, "rms_norm: unsupported weight type code %d", dtype_w);
    if (emb * n > 0 && (!x || !w || !y || !rstd)) return fail(ONIONOP_E_NULL, "rms_norm: NULL tensor pointer");
    if (n > 0 && emb > 0 && (!aligned16(x) || !aligned16(y)))
        return fail(ONIONOP_E_SHAPE, "rms_norm: x and y must be 16-byte aligned");
    if (n > 0 && emb == 0) return fail(ONIONOP_E_SHAPE, "rms_norm: empty embedding dimension");
    if (!onionop::launch_rms_fwd((hipStream_t)stream, dtype_x, dtype_w, emb, n, x, w, eps, offset, y, rstd))
        return fail(ONIONOP_E_UNSUPPORTED, "rms_norm: no kernel for emb=%lld", (long long)emb);
    return check_launch("rms_norm");
}

size_t onionop_rms_norm_bwd_workspace(int64_t emb, int64_t n) {
    if (emb <= 0 || n <= 0) return 0;
    return (size_t)onionop::norm_bwd_ws_floats(n, emb) * sizeof(float);
}

int onionop_rms_norm_bwd(void* stream, int dtype_x, int dtype_w, int64_t emb, int64_t n, const void* dy,
                         const float* rstd, const void* x, const void* w, float offset, void* dx, float* dw,
                         void* workspace, size_t workspace_bytes) {
    int st = check_rows("∇rms_norm", dtype_x, emb, n);
    if (st) return st;
    if (!valid_dt(dtype_w)) return fail(ONIONOP_E_DTYPE, "∇rms_norm: unsupported weight type code %d", dtype_w);
    if ((emb * n > 0 && (!dy || !rstd || !x || !dx)) || (emb > 0 && (!w || !dw)))
        return fail(ONIONOP_E_NULL, "∇rms_norm: NULL tensor pointer");
    if (n > 0 && emb > 0 && (!aligned16(dy) || !aligned16(x) || !aligned16(dx)))
        return fail(ONIONOP_E_SHAPE, "∇rms_norm: dy, x and dx must be 16-byte aligned");
    const size_t need = onionop_rms_norm_bwd_workspace(emb, n);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
        return fail(ONIONOP_E_WORKSPACE, "∇rms_norm: 16-byte aligned workspace of %zu bytes needed, %zu given", need,
                    workspace_bytes);
    if (!onionop::launch_rms_bwd((hipStream_t)stream, dtype_x, dtype_w, emb, n, dy, rstd, x, w, offset, dx, dw,
                                 (float*)workspace))
        return fail(ONIONOP_E_UNSUPPORTED, "∇rms_norm: no kernel for emb=%lld", (long long)emb);
    return check_launch("∇rms_norm");
}

// ----------------------------------------------------------------- layer norm

int onionop_layer_norm_fwd(void* stream, int dtype_x, int dtype_w, int64_t emb, int64_t n, const void* x,
                           const void* w, const void* b, float eps, void* y, float* mu, float* rstd) {
    int st = check_rows("layer_norm", dtype_x, emb, n);
    if (st) return st;
    if (!valid_dt(dtype_w)) return fail(ONIONOP_E_DTYPE, "layer_norm: unsupported weight type code %d", dtype_w);
    if (emb * n > 0 && (!x || !w || !b || !y || !mu || !rstd))
        return fail(ONIONOP_E_NULL, "layer_norm: NULL tensor pointer");
    if (n > 0 && emb > 0 && (!aligned16(x) || !aligned16(y)))
        return fail(ONIONOP_E_SHAPE, "layer_norm: x and y must be 16-byte aligned");
    if (n > 0 && emb == 0) return fail(ONIONOP_E_SHAPE, "layer_norm: empty embedding dimension");
    if (!onionop::launch_ln_fwd((hipStream_t)stream, dtype_x, dtype_w, emb, n, x, w, b, eps, y, mu, rstd))
        return fail(ONIONOP_E_UNSUPPORTED, "layer_norm: no kernel for emb=%lld", (long long)emb);
    return check_launch("layer_norm");
}

size_t onionop_layer_norm_bwd_workspace(int64_t emb, int64_t n) {
    if (emb <= 0 || n <= 0) return 0;
    return 2 * (size_t)onionop::norm_bwd_ws_floats(n, emb) * sizeof(float);
}

int onionop_layer_norm_bwd(void* stream, int dtype_x, int dtype_w, int64_t emb, int64_t n, const void* dy,
                           const float* mu, const float* rstd, const void* x, const void* w, void* dx, void* dw,
                           void* db, void* workspace, size_t workspace_bytes) {
    int st = check_rows("∇layer_norm", dtype_x, emb, n);
    if (st) return st;
    if (!valid_dt(dtype_w)) return fail(ONIONOP_E_DTYPE, "∇layer_norm: unsupported weight type code %d", dtype_w);
    if ((emb * n > 0 && (!dy || !mu || !rstd || !x || !dx)) || (emb > 0 && (!w || !dw || !db)))
        return fail(ONIONOP_E_NULL, "∇layer_norm: NULL tensor pointer");
    if (n > 0 && emb > 0 && (!aligned16(dy) || !aligned16(x) || !aligned16(dx)))
        return fail(ONIONOP_E_SHAPE, "∇layer_norm: dy, x and dx must be 16-byte aligned");
    const size_t need = onionop_layer_norm_bwd_workspace(emb, n);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
        return fail(ONIONOP_E_WORKSPACE, "∇layer_norm: 16-byte aligned workspace of %zu bytes needed, %zu given",
                    need, workspace_bytes);
    if (!onionop::launch_ln_bwd((hipStream_t)stream, dtype_x, dtype_w, emb, n, dy, mu, rstd, x, w, dx, dw, db,
                                (float*)workspace))
        return fail(ONIONOP_E_UNSUPPORTED, "∇layer_norm: no kernel for emb=%lld", (long long)emb);
    return check_launch("∇layer_norm");
}

// ----------------------------------------------------------------------- RoPE

int onionop_llama_rotary_embedding(void* stream, int64_t dim, int64_t L, int64_t B, int64_t base,
                                   const float* positions, float* cos, float* sin) {
    const char* what = "LlamaRotaryEmbedding";
    if (dim < 0 || L < 0 || B < 0) return fail(ONIONOP_E_SHAPE, "%s: negative dimension", what);
    if (dim % 2 != 0) return fail(ONIONOP_E_SHAPE, "%s: dim %lld must be even", what, (long long)dim);
    if (base <= 0) return fail(ONIONOP_E_SHAPE, "%s: base must be positive", what);
    if (dim * L * B > 0 && (!positions || !cos || !sin)) return fail(ONIONOP_E_NULL, "%s: NULL tensor pointer", what);
    if (dim * L * B >= (1LL << 31))
        return fail(ONIONOP_E_UNSUPPORTED, "%s: table too large (dim * L * B must be below 2^31)", what);
    if (!onionop::launch_rope_table((hipStream_t)stream, dim, L * B, (float)base, positions, cos, sin))
        return fail(ONIONOP_E_UNSUPPORTED, "%s: no kernel", what);
    return check_launch(what);
}

int onionop_llama_rope(void* stream, int dtype, int64_t E, int64_t L, int64_t QH, int64_t KH, int64_t B,
                       const void* q, const void* k, const float* cos, const float* sin, float sin_sign,
                       void* q_out, void* k_out) {
    if (!valid_dt(dtype)) return fail(ONIONOP_E_DTYPE, "llama_rope: unsupported element type code %d", dtype);
    if (E < 0 || L < 0 || QH < 0 || KH < 0 || B < 0) return fail(ONIONOP_E_SHAPE, "llama_rope: negative dimension");
    if (E % 2 != 0) return fail(ONIONOP_E_SHAPE, "llama_rope: head dim %lld must be even", (long long)E);
    if (E > 512) return fail(ONIONOP_E_UNSUPPORTED, "llama_rope: head dim %lld > 512", (long long)E);
    // The kernel addresses one (head, batch) slice with 32-bit byte offsets.
    if (L * E * (int64_t)dt_size(dtype) >= (1LL << 31))
        return fail(ONIONOP_E_UNSUPPORTED, "llama_rope: sequence too long (L*E*sizeof(T) must be below 2^31 bytes)");
    if (E * L * B == 0 || (QH == 0 && KH == 0)) return ok();
    if (!cos || !sin || (QH > 0 && (!q || !q_out)) || (KH > 0 && (!k || !k_out)))
        return fail(ONIONOP_E_NULL, "llama_rope: NULL tensor pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(q_out) || !aligned16(k_out))
        return fail(ONIONOP_E_SHAPE, "llama_rope: q, k and outputs must be 16-byte aligned");
    if (!onionop::launch_rope((hipStream_t)stream, dtype, E, L, QH, KH, B, q, k, cos, sin, sin_sign, q_out, k_out))
        return fail(ONIONOP_E_UNSUPPORTED, "llama_rope: no kernel for E=%lld", (long long)E);
    return check_launch("llama_rope");
}

}  // extern "C"
