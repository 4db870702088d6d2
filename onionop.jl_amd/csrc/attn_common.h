// attn_common.h -- MFMA fragment conventions shared by the attention kernels.
//
// All attention GEMMs use the 32x32 MFMA family of gfx950 (CDNA4):
//   16-bit inputs: v_mfma_f32_32x32x16_{bf16,f16}   (K = 16 per instruction)
//   float32:       v_mfma_f32_32x32x2f32             (K = 2 per instruction)
// Operand layouts (lane l in 0..63, h = l / 32):
//   A (32 x K):  lane l holds row l % 32, k = KE*h + [0, KE)      (KE = K/2 elements)
//   B (K x 32):  lane l holds column l % 32, k = KE*h + [0, KE)
//   C (32 x 32): lane l holds column l % 32; accumulator register r holds row
//                crow(r, h) = 8*(r/4) + 4*h + r%4.
// The contraction index may be permuted freely as long as A and B agree.  A C tile is
// reused as the B operand of the next product ("P^T as B") by taking chunk c from
// registers r = KE*c + j, j in [0, KE), which stand for rows crow(KE*c + j, h); the
// matching A operand is then read at those same k positions (kperm below).
#pragma once

#include "common.h"

namespace onionop {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ int crow(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

template <typename T> struct Mfma;

template <> struct Mfma<bf16> {
    static constexpr int KC = 16, KE = 8;
    typedef bf16x8 frag;
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<f16> {
    static constexpr int KC = 16, KE = 8;
    typedef f16x8 frag;
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<float> {
    static constexpr int KC = 2, KE = 1;
    typedef float frag;
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

// KE consecutive elements starting at p (LDS or global) as a fragment.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag load_frag(const T* p) {
    if constexpr (Mfma<T>::KE == 8) {
        return *reinterpret_cast<const typename Mfma<T>::frag*>(p);
    } else {
        return *p;
    }
}

// Fragment at k positions kperm(c, h, j) = crow(KE*c + j, h) of a row stored contiguously
// along k (row points at k = 0).  For KE = 8 these are two runs of 4: 16c + 4h + [0,4)
// and 16c + 8 + 4h + [0,4); for KE = 1 it is the single element crow(c, h).
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag load_frag_kperm(const T* row, int c, int h) {
    if constexpr (Mfma<T>::KE == 8) {
        typedef T t4 __attribute__((ext_vector_type(4)));
        const t4 lo = *reinterpret_cast<const t4*>(row + 16 * c + 4 * h);
        const t4 hi = *reinterpret_cast<const t4*>(row + 16 * c + 8 + 4 * h);
        typename Mfma<T>::frag f;
        f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
        f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
        return f;
    } else {
        return row[crow(c, h)];
    }
}

// Chunk c of a C tile (registers KE*c .. KE*c+KE-1) converted to a B fragment.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag c_to_frag(const f32x16& acc, int c) {
    if constexpr (Mfma<T>::KE == 8) {
        typename Mfma<T>::frag f;
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = (T)acc[8 * c + j];
        return f;
    } else {
        return acc[c];
    }
}

// Element type helpers for the float16-rounded Q/K of the reference backward.
template <typename T, bool QK16>
__device__ __forceinline__ T qk_round(T x) {
    if constexpr (QK16 && sizeof(T) == 4) return round_f16(x);
    else return x;
}

}  // namespace onionop
