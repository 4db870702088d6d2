// attn_dispatch.hip -- element-type dispatch of the attention launchers.
#include <atomic>

#include "launch.h"

// float32 through bf16x6 MFMA products (attn_f32x6.hip)
namespace onionop_x6 {
bool fwd_f32x6(hipStream_t s, const onionop::AttnArgs& a);
bool bwd_f32x6(hipStream_t s, const onionop::AttnArgs& a, int stages);
}  // namespace onionop_x6

namespace onionop {

typedef __bf16 bf16;
typedef _Float16 f16;

template <typename T> bool fwd_dispatch(hipStream_t s, const AttnArgs& a);
template <typename T, bool QK16> bool bwd_dispatch(hipStream_t s, const AttnArgs& a, int stages);

extern template bool fwd_dispatch<float>(hipStream_t, const AttnArgs&);
extern template bool fwd_dispatch<f16>(hipStream_t, const AttnArgs&);
extern template bool fwd_dispatch<bf16>(hipStream_t, const AttnArgs&);
extern template bool bwd_dispatch<float, false>(hipStream_t, const AttnArgs&, int);
extern template bool bwd_dispatch<float, true>(hipStream_t, const AttnArgs&, int);
extern template bool bwd_dispatch<f16, false>(hipStream_t, const AttnArgs&, int);
extern template bool bwd_dispatch<bf16, false>(hipStream_t, const AttnArgs&, int);

static __global__ void zero_bytes_kernel(void* p, int64_t bytes) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    unsigned char* c = reinterpret_cast<unsigned char*>(p);
    for (int j = 0; j < 4; ++j)
        if (i + j < bytes) c[i + j] = 0;
}

// Ranges of `tiles` tiles: at most `want` and 8, each of at least two tiles, and no empty
// one (ranges are runs of ceil(tiles / n) tiles).
static int split_count(int64_t want, int64_t tiles) {
    int64_t n = want < 8 ? want : 8;
    if (n > tiles / 2) n = tiles / 2;
    if (n <= 1) return 1;
    const int64_t per = (tiles + n - 1) / n;
    return (int)((tiles + per - 1) / per);
}

int dq_key_splits(int dt, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t B) {
    if ((dt != 1 && dt != 2) || QL <= 0 || KL <= 0 || QH <= 0 || B <= 0) return 1;
    if (E >= 256) {  // without a bias: one workgroup per CU, a grid that fills the chip at most once
        const int64_t nwg = ((QL + 63) / 64) * QH * B;
        return nwg > 256 ? 1 : split_count(512 / nwg, (KL + 31) / 32);
    }
    if (E > 64 || QH % 4 != 0) return 1;
    const int64_t nwg4 = ((QL + 63) / 64) * (QH / 4) * B;
    if (nwg4 >= 192) return 1;  // the unsplit four-head grid already fills the chip
    const int64_t tiles = (KL + 31) / 32;
    return split_count(256 / nwg4, tiles);
}

int kv_query_splits(int dt, int64_t E, int64_t QL, int64_t KL, int64_t QH, int64_t KH, int64_t B) {
    if ((dt != 1 && dt != 2) || KH <= 0 || QH % KH != 0 || QL <= 0 || KL <= 0 || B <= 0) return 1;
    if (E >= 128) {  // the two-wave kernel: 64 keys per workgroup, 32-query tiles
        const int64_t nws = ((KL + 63) / 64) * KH * B, tiles = (QH / KH) * ((QL + 31) / 32);
        // GQA of 8 or more q heads per kv head; fewer take two query-range groups
        if (QH / KH >= 8) return nws > 512 ? 1 : split_count(1024 / nws, tiles);
        // E = 256 (one workgroup per CU) on a grid that fills the chip at most once
        if (E >= 256 && nws <= 256) return split_count(512 / nws, tiles);
        return 1;
    }
    if (QH == KH) {  // pair bias, four kv heads per workgroup
        if (KH % 4 != 0) return 1;
        const int64_t nwg4 = ((KL + 63) / 64) * (KH / 4) * B;
        if (nwg4 >= 192) return 1;
        const int64_t bq = E >= 64 ? 32 : 64;  // the bias kernel's query tile
        return split_count(256 / nwg4, (QL + bq - 1) / bq);
    }
    // GQA without a bias: the one-wave dK/dV grid (8-wave workgroups of 128 keys at E = 64
    // while they make 256, one per CU; else 4-wave workgroups of 64 keys, two per CU),
    // split towards 1024 workgroups over the rep q heads' 64-query tiles when it fills
    // the chip at most once.
    const int64_t nwg = ((KL + 63) / 64) * KH * B, nwg4 = ((KL + 127) / 128) * KH * B;
    const bool wide = E == 64 && nwg4 >= 256;
    const int64_t g = wide ? nwg4 : nwg;
    if (g > (wide ? 256 : 512)) return 1;
    return split_count(1024 / g, (QH / KH) * ((QL + 63) / 64));
}

int device_cu_count() {
    static std::atomic<int> cache[64];  // 0: not queried yet, -1: query failed
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        int n = 0;
        v = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : -1;
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v > 0 ? v : 0;
}

bool launch_attn_fwd(hipStream_t s, int dt, const AttnArgs& a) {
    if (a.QL == 0 || a.QH == 0 || a.B == 0) return true;
    switch (dt) {
        case 0: return fwd_dispatch<float>(s, a);
        case 1: return fwd_dispatch<f16>(s, a);
        case 2: return fwd_dispatch<bf16>(s, a);
        case 3: return onionop_x6::fwd_f32x6(s, a);
    }
    return false;
}

bool launch_attn_bwd(hipStream_t s, int dt, const AttnArgs& a, int stages) {
    if (a.B == 0 || a.QH == 0) return true;
    if (a.QL == 0) {  // no queries: dk = dv = 0
        if (!(stages & kBwdDkDv)) return true;
        const int64_t krows = a.cu_q ? a.KH * a.Tk : a.KL * a.KH * a.B;
        const int64_t bytes = (dt == 0 || dt == 3 ? 4 : 2) * a.E * krows;
        if (bytes > 0) {
            zero_bytes_kernel<<<dim3((unsigned)((bytes + 1023) / 1024)), dim3(256), 0, s>>>(a.dk, bytes);
            zero_bytes_kernel<<<dim3((unsigned)((bytes + 1023) / 1024)), dim3(256), 0, s>>>(a.dv, bytes);
        }
        return true;
    }
    switch (dt) {
        case 0: return a.qk_fp16 ? bwd_dispatch<float, true>(s, a, stages) : bwd_dispatch<float, false>(s, a, stages);
        case 1: return bwd_dispatch<f16, false>(s, a, stages);
        case 2: return bwd_dispatch<bf16, false>(s, a, stages);
        case 3: return onionop_x6::bwd_f32x6(s, a, stages);
    }
    return false;
}

}  // namespace onionop
