// attn_tiles.h -- global -> register -> LDS staging of (rows x E) tiles for the attention
// kernels.  A tile of consecutive rows of one head is a contiguous chunk of global
// memory, so threads read consecutive 16-byte vectors (fully coalesced) and keep them in
// registers until the LDS buffer they go to is free (software pipelining).
#pragma once

#include "attn_common.h"

namespace onionop {

// LDS row stride (elements) of a natural (rows x EO) tile.  16-bit: 16 bytes of padding,
// keeping rows 16-byte aligned for ds_read_b128 / b128 stores.  float32: one element,
// making the column reads of the float32 MFMA operands conflict-free.
template <typename T, int EO> struct TileCfg { static constexpr int DS = EO + 8; };
template <int EO> struct TileCfg<float, EO> { static constexpr int DS = EO + 1; };

template <typename T, int NR, int E, int NT>
struct TileRegs {
    static constexpr int VN = 16 / (int)sizeof(T);  // elements per 16-byte vector
    static constexpr int VPR = E / VN;              // vectors per row
    static constexpr int NV = (NR * VPR + NT - 1) / NT;
    u32x4 r[NV];

    // Rows [r0, r0 + NR) of src (row length E); rows at or past nrows read as zero.
    template <bool QK16 = false>
    __device__ __forceinline__ void load(const T* __restrict__ src, int r0, int nrows) {
        // Rows r0 .. r0 + NR - 1 are one contiguous run of NR * E elements; a tile wholly
        // inside [0, nrows) (uniform across the workgroup) loads without per-vector checks.
        const bool full = r0 + NR <= nrows;
        const T* tile = src + (int64_t)r0 * E;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vi = threadIdx.x + i * NT;
            const int row = vi / VPR;
            const bool in_tile = (NR * VPR) % NT == 0 || vi < NR * VPR;
            if (full && in_tile) r[i] = *reinterpret_cast<const u32x4*>(tile + vi * VN);
            else if (in_tile && r0 + row < nrows) r[i] = *reinterpret_cast<const u32x4*>(tile + vi * VN);
            else r[i] = u32x4{0u, 0u, 0u, 0u};
            if constexpr (QK16 && sizeof(T) == 4) {
                union { u32x4 v; float f[4]; } u;
                u.v = r[i];
#pragma unroll
                for (int j = 0; j < 4; ++j) u.f[j] = round_f16(u.f[j]);
                r[i] = u.v;
            }
        }
    }
    // Write the tile to LDS dst[row * DS + e].
    __device__ __forceinline__ void store(T* dst, int DS) const {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vi = threadIdx.x + i * NT;
            if (vi >= NR * VPR) continue;
            const int row = vi / VPR, e0 = (vi % VPR) * VN;
            if constexpr (sizeof(T) == 2) {
                *reinterpret_cast<u32x4*>(dst + row * DS + e0) = r[i];
            } else {
                union { u32x4 v; float f[4]; } u;
                u.v = r[i];
#pragma unroll
                for (int j = 0; j < 4; ++j) dst[row * DS + e0 + j] = u.f[j];
            }
        }
    }
};

// Zero columns [E, DS) of two NR-row LDS tiles (the padding read as rows E..31 of a 32-row
// MFMA block when E = 16).
template <typename T, int NR, int E, int DS, int NT>
__device__ __forceinline__ void zero_pad_cols(T* a, T* b) {
    for (int i = threadIdx.x; i < NR * (DS - E); i += NT) {
        const int row = i / (DS - E), col = E + i % (DS - E);
        a[row * DS + col] = (T)0.f;
        b[row * DS + col] = (T)0.f;
    }
}

}  // namespace onionop
