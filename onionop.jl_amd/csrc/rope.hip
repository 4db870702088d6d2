// rope.hip -- Llama rotate-half rotary embedding of q and k, out of place
// (llama_rope!, src/rope/llama_rope.jl:24-65).
//
// Layout: q (B, QH, L, E) and k (B, KH, L, E) row-major (Julia (E, L, H, B)); cos/sin
// (B, L, E) float32 of which the first E/2 entries of a row are read.
// A workgroup owns (batch b, a block of positions) and loops over every q and k head,
// so each cos/sin value is read from HBM once and reused from registers for all
// QH + KH heads; q/k rows of one head are contiguous across the block, so loads and
// stores are 16-byte and coalesced.  Arithmetic is float32, rounded once on store.
#include "common.h"
#include "launch.h"

namespace onionop {

template <typename T, int VP>
__device__ __forceinline__ void load_n(const T* __restrict__ p, float* out) {
    if constexpr (VP == Vec<T>::N) load_vec<T>(p, out);
    else {
#pragma unroll
        for (int j = 0; j < VP; ++j) out[j] = to_f32(p[j]);
    }
}
template <typename T, int VP>
__device__ __forceinline__ void store_n(T* __restrict__ p, const float* in) {
    if constexpr (VP == Vec<T>::N) store_vec<T>(p, in);
    else {
#pragma unroll
        for (int j = 0; j < VP; ++j) p[j] = from_f32<T>(in[j]);
    }
}

// One thread = VP consecutive rotation pairs (i, i + E/2) of one position.
template <typename T, int VP>
__global__ __launch_bounds__(256) void rope_kernel(const T* q, const T* k, const float* __restrict__ cosv,
                                                   const float* __restrict__ sinv, float sin_sign, T* qo, T* ko,
                                                   int64_t E, int64_t L, int64_t QH, int64_t KH, int64_t rows_per_wg,
                                                   int64_t tpr) {
    const int64_t half = E / 2;
    const int64_t b = blockIdx.y;
    const int64_t l = (int64_t)blockIdx.x * rows_per_wg + threadIdx.x / tpr;
    const int64_t i0 = (threadIdx.x % tpr) * VP;
    if (threadIdx.x >= rows_per_wg * tpr || l >= L) return;
    float c[VP], s[VP];
    const int64_t cs = (b * L + l) * E + i0;
#pragma unroll
    for (int j = 0; j < VP; ++j) {
        c[j] = cosv[cs + j];
        s[j] = sinv[cs + j] * sin_sign;
    }
    const int64_t H = QH > KH ? QH : KH;
#pragma unroll 2
    for (int64_t h = 0; h < H; ++h) {
        if (h < QH) {
            const int64_t base = ((b * QH + h) * L + l) * E + i0;
            float x1[VP], x2[VP], y1[VP], y2[VP];
            load_n<T, VP>(q + base, x1);
            load_n<T, VP>(q + base + half, x2);
#pragma unroll
            for (int j = 0; j < VP; ++j) {
                y1[j] = x1[j] * c[j] - x2[j] * s[j];
                y2[j] = x2[j] * c[j] + x1[j] * s[j];
            }
            store_n<T, VP>(qo + base, y1);
            store_n<T, VP>(qo + base + half, y2);
        }
        if (h < KH) {
            const int64_t base = ((b * KH + h) * L + l) * E + i0;
            float x1[VP], x2[VP], y1[VP], y2[VP];
            load_n<T, VP>(k + base, x1);
            load_n<T, VP>(k + base + half, x2);
#pragma unroll
            for (int j = 0; j < VP; ++j) {
                y1[j] = x1[j] * c[j] - x2[j] * s[j];
                y2[j] = x2[j] * c[j] + x1[j] * s[j];
            }
            store_n<T, VP>(ko + base, y1);
            store_n<T, VP>(ko + base + half, y2);
        }
    }
}

template <typename T, int VP>
static void rope_launch(hipStream_t s, const void* q, const void* k, const float* cosv, const float* sinv,
                        float sign, void* qo, void* ko, int64_t E, int64_t L, int64_t QH, int64_t KH, int64_t B) {
    const int64_t tpr = (E / 2) / VP;  // threads per position
    const int64_t rows_per_wg = 256 / tpr;
    const dim3 grid((unsigned)((L + rows_per_wg - 1) / rows_per_wg), (unsigned)B);
    rope_kernel<T, VP><<<grid, dim3(256), 0, s>>>((const T*)q, (const T*)k, cosv, sinv, sign, (T*)qo, (T*)ko, E,
                                                 L, QH, KH, rows_per_wg, tpr);
}

bool launch_rope(hipStream_t s, int dt, int64_t E, int64_t L, int64_t QH, int64_t KH, int64_t B, const void* q,
                 const void* k, const float* cosv, const float* sinv, float sign, void* qo, void* ko) {
    if (L == 0 || B == 0 || (QH == 0 && KH == 0)) return true;
    const int64_t half = E / 2;
    switch (dt) {
        case 0:
            if (half % 4 == 0 && half / 4 <= 256) rope_launch<float, 4>(s, q, k, cosv, sinv, sign, qo, ko, E, L, QH, KH, B);
            else if (half <= 256) rope_launch<float, 1>(s, q, k, cosv, sinv, sign, qo, ko, E, L, QH, KH, B);
            else return false;
            return true;
        case 1:
            if (half % 8 == 0 && half / 8 <= 256) rope_launch<f16, 8>(s, q, k, cosv, sinv, sign, qo, ko, E, L, QH, KH, B);
            else if (half <= 256) rope_launch<f16, 1>(s, q, k, cosv, sinv, sign, qo, ko, E, L, QH, KH, B);
            else return false;
            return true;
        case 2:
            if (half % 8 == 0 && half / 8 <= 256) rope_launch<bf16, 8>(s, q, k, cosv, sinv, sign, qo, ko, E, L, QH, KH, B);
            else if (half <= 256) rope_launch<bf16, 1>(s, q, k, cosv, sinv, sign, qo, ko, E, L, QH, KH, B);
            else return false;
            return true;
    }
    return false;
}

}  // namespace onionop
