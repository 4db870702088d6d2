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

// Rotates heads [0, H) of one position for one thread: x1 = x[i0 .. i0+VP),
// x2 = x[half + i0 ..), with the loads of kU heads issued before any of their math so
// that each thread keeps 2 kU 16-byte requests in flight.  Each (batch, head) slice is a
// buffer resource of L*E elements (offsets fit 32 bits; heads past H read zero and drop
// their stores, so the unrolled tail needs no branch).
template <typename T, int VP>
__device__ __forceinline__ void rope_heads(const T* x, T* xo, int64_t H, int64_t b, int64_t l, int64_t i0,
                                           int64_t E, int64_t L, const float* c, const float* s) {
    constexpr int kU = 4;
    const int64_t half = E / 2;
    const uint32_t slice = (uint32_t)(L * E * (int64_t)sizeof(T));
    const uint32_t o1 = (uint32_t)((l * E + i0) * (int64_t)sizeof(T));
    const uint32_t o2 = o1 + (uint32_t)(half * (int64_t)sizeof(T));
    for (int64_t h0 = 0; h0 < H; h0 += kU) {
        u32x4 a[kU], bb[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const bool ok = h0 + u < H;
            const rsrc_t r = make_rsrc(x + ((b * H + (ok ? h0 + u : 0)) * L) * E, ok ? slice : 0u);
            if constexpr (VP == Vec<T>::N) {
                a[u] = bload16_nt(r, o1);
                bb[u] = bload16_nt(r, o2);
            }
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const bool ok = h0 + u < H;
            const int64_t base = ((b * H + (ok ? h0 + u : 0)) * L + l) * E + i0;
            float x1[VP], x2[VP], y1[VP], y2[VP];
            if constexpr (VP == Vec<T>::N) {
                union { u32x4 v; T e[VP]; } u1, u2;
                u1.v = a[u];
                u2.v = bb[u];
#pragma unroll
                for (int j = 0; j < VP; ++j) { x1[j] = to_f32(u1.e[j]); x2[j] = to_f32(u2.e[j]); }
            } else {
                if (!ok) continue;
                load_n<T, VP>(x + base, x1);
                load_n<T, VP>(x + base + half, x2);
            }
#pragma unroll
            for (int j = 0; j < VP; ++j) {
                y1[j] = x1[j] * c[j] - x2[j] * s[j];
                y2[j] = x2[j] * c[j] + x1[j] * s[j];
            }
            if constexpr (VP == Vec<T>::N) {
                const rsrc_t r = make_rsrc(xo + ((b * H + (ok ? h0 + u : 0)) * L) * E, ok ? slice : 0u);
                union { u32x4 v; T e[VP]; } w1, w2;
#pragma unroll
                for (int j = 0; j < VP; ++j) { w1.e[j] = from_f32<T>(y1[j]); w2.e[j] = from_f32<T>(y2[j]); }
                bstore16_nt(w1.v, r, o1);
                bstore16_nt(w2.v, r, o2);
            } else {
                store_n<T, VP>(xo + base, y1);
                store_n<T, VP>(xo + base + half, y2);
            }
        }
    }
}

// One thread = VP consecutive rotation pairs (i, i + E/2) of one position, for every q
// head and then every k head.
template <typename T, int VP>
__global__ __launch_bounds__(256) void rope_kernel(const T* q, const T* k, const float* __restrict__ cosv,
                                                   const float* __restrict__ sinv, float sin_sign, T* qo, T* ko,
                                                   int64_t E, int64_t L, int64_t QH, int64_t KH, int64_t rows_per_wg,
                                                   int64_t tpr) {
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
    rope_heads<T, VP>(q, qo, QH, b, l, i0, E, L, c, s);
    rope_heads<T, VP>(k, ko, KH, b, l, i0, E, L, c, s);
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

// cos / sin tables of LlamaRotaryEmbedding(dim; base) at float32 positions (B, L)
// (src/rope/llama_rope.jl:1-22): inv_freq[i] = 1 / base^(2i / dim) and freqs = inv_freq pos
// in float32 as the reference computes them; cos / sin of freqs, written at i and again at
// i + dim/2 (vcat(freqs, freqs)).  The power and the cos / sin are evaluated in float64 and
// rounded once, so each table value is the correctly rounded float32 of its float32
// argument.  One thread per (row, i < dim/2).
__global__ __launch_bounds__(256) void rope_table_kernel(const float* __restrict__ pos, float* __restrict__ cosv,
                                                         float* __restrict__ sinv, int64_t dim, int64_t rows,
                                                         float base) {
    const int64_t half = dim / 2;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= rows * half) return;
    const int64_t r = t / half, i = t - r * half;
    const float id = (float)(2 * i) / (float)dim;
    const float p = (float)pow((double)base, (double)id);
    const float inv_freq = 1.0f / p;
    const float f = inv_freq * pos[r];
    const float c = (float)cos((double)f), sn = (float)sin((double)f);
    cosv[r * dim + i] = c;
    cosv[r * dim + i + half] = c;
    sinv[r * dim + i] = sn;
    sinv[r * dim + i + half] = sn;
}

bool launch_rope_table(hipStream_t s, int64_t dim, int64_t rows, float base, const float* pos, float* cosv,
                       float* sinv) {
    const int64_t n = rows * (dim / 2);
    if (n == 0) return true;
    rope_table_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(pos, cosv, sinv, dim, rows, base);
    return true;
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
