// attn_tiles.h -- global -> register -> LDS staging of (rows x E) tiles for the attention
// kernels.  A tile of consecutive rows of one head is a contiguous chunk of global
// memory, so threads read consecutive 16-byte vectors (fully coalesced) and keep them in
// registers until the LDS buffer they go to is free (software pipelining).
#pragma once

#include "attn_common.h"

namespace onionop {

// LDS row stride (elements) of a natural (rows x EO) tile.  16-bit: 16 bytes of padding,
// keeping rows 16-byte aligned for ds_read_b128 / b128 stores; WIDE: 32 bytes, with which
// the transposed reads (ds_read_b64_tr_b16: each 16-lane group reads 4 rows x 32 bytes)
// hit every LDS bank exactly twice, the minimum for 512 bytes over 64 four-byte banks,
// while 16 bytes of padding give 3 (E = 32, 64) or 4 (E = 128) reads on the busiest bank.
// float32: one element, making the column reads of the float32 MFMA operands
// conflict-free.
template <typename T, int EO, bool WIDE = false> struct TileCfg { static constexpr int DS = EO + (WIDE ? 16 : 8); };
// bf16x6 float32 (ONIONOP_X6): rows stay 16-byte aligned for the natural fragment reads.
// WIDE: 8 floats, with which the two row halves of a transposed read (rows 4 apart) land
// 32 banks apart; otherwise 4 (2-way conflicts on those reads), which keeps four
// query-range groups of the float32 dK/dV kernel within the CU's LDS at E = 64.
#if ONIONOP_X6
template <int EO, bool WIDE> struct TileCfg<float, EO, WIDE> { static constexpr int DS = EO + (WIDE ? 8 : 4); };
#else
template <int EO, bool WIDE> struct TileCfg<float, EO, WIDE> { static constexpr int DS = EO + 1; };
#endif

// Waits until every outstanding vector-memory load has returned (s_waitcnt vmcnt(0)).
// Issued once after the loads that precede a software-pipelined loop, so the compiler's
// wait insertion does not carry them as possibly pending into the loop, where it would
// otherwise wait on the loop's own prefetches before each use of those registers.
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Resource over rows [0, nrows) of a row-major (rows x E) slice of T.
template <typename T, int E>
__device__ __forceinline__ rsrc_t slice_rsrc(const T* base, int nrows) {
    return make_rsrc(base, (uint32_t)nrows * (uint32_t)(E * sizeof(T)));
}
// An MFMA fragment (KE consecutive elements) at element offset `elem` of a slice
// resource; zero past the end of the slice.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag bload_frag(rsrc_t r, uint32_t elem) {
#if ONIONOP_X6
    if constexpr (sizeof(T) == 4) {
        union { u32x4 v; float f[4]; } a, b;
        a.v = bload16(r, elem * 4u);
        b.v = bload16(r, elem * 4u + 16u);
        const float x[8] = {a.f[0], a.f[1], a.f[2], a.f[3], b.f[0], b.f[1], b.f[2], b.f[3]};
        return split_f32x8(x);
    } else
#endif
    if constexpr (Mfma<T>::KE == 8) {
        union { u32x4 v; typename Mfma<T>::frag f; } u;
        u.v = bload16(r, elem * (uint32_t)sizeof(T));
        return u.f;
    } else {
        return bload_f32(r, elem * 4u);
    }
}

template <typename T, int NR, int E, int NT>
struct TileRegs {
    static constexpr int VN = 16 / (int)sizeof(T);  // elements per 16-byte vector
    static constexpr int VPR = E / VN;              // vectors per row
    static constexpr int NV = (NR * VPR + NT - 1) / NT;
    u32x4 r[NV];

    // Rows [r0, r0 + NR) of the slice behind `rs` (row length E); rows past the end of
    // the slice read as zero.  Rows r0 .. r0 + NR - 1 are one contiguous run of NR * E
    // elements, read as consecutive 16-byte vectors by consecutive threads.
    // `t` is this thread's index among the NT threads that share the tile.
    template <bool QK16 = false>
    __device__ __forceinline__ void load(rsrc_t rs, int r0, int t) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vi = t + i * NT;
            const int vc = (NR * VPR) % NT == 0 || vi < NR * VPR ? vi : 0;  // idle threads re-read vector 0
            r[i] = bload16(rs, ((uint32_t)r0 * E + (uint32_t)vc * VN) * (uint32_t)sizeof(T));
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
    __device__ __forceinline__ void store(T* dst, int DS, int t) const {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int vi = t + i * NT;
            if constexpr ((NR * VPR) % NT != 0) {
                if (vi >= NR * VPR) continue;
            }
            const int row = vi / VPR, e0 = (vi % VPR) * VN;
            if constexpr (sizeof(T) == 2 || ONIONOP_X6) {  // 16-byte aligned rows
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

// Direct global -> LDS staging of a 16-bit tile (buffer_load_dwordx4 ... lds): each
// lane's 16 bytes land at the wave's LDS base + 16 * lane, so one instruction fills 64
// consecutive 16-byte slots and no registers hold the tile in transit.  The padded layout
// is kept (row stride DS elements = SPR 16-byte slots, CPR of them data): a lane whose slot is a row's
// padding chunk, or whose row is past the slice, uses an offset past the resource's end
// and so writes zeros without touching memory.  Completion is tracked by the vector-
// memory counter: the waiting wave issues s_waitcnt vmcnt before the barrier that
// publishes the tile.
template <typename T, int NR, int E, int NT, int DS = TileCfg<T, E>::DS>
struct TileDMA {
    // 16-bit rows of E elements at an LDS row stride of DS elements (padding chunks >= 1)
    static constexpr bool kOK = sizeof(T) == 2 && DS > E && (DS - E) % 8 == 0;
    static constexpr int CPR = E * 2 / 16;  // data chunks per row
    static constexpr int SPR = DS * 2 / 16; // LDS slots per row (data + padding)
    static constexpr int NS = NR * SPR;     // slots per tile
    static constexpr int NI = (NS + NT - 1) / NT;

    // Rows [r0, r0 + NR) of the slice behind `rs` into the LDS tile at dst; t is the
    // thread's index among the NT threads that share the tile, wave = t / 64 (uniform).
    __device__ __forceinline__ static void load(rsrc_t rs, int r0, T* dst, int t, int wave) {
        static_assert(kOK, "16-bit tiles with one padding chunk per row");
        typedef __attribute__((address_space(3))) void lds_void;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int slot0 = i * NT + wave * 64;  // wave-uniform first slot of this instruction
            if constexpr (NS % NT != 0) {
                if (slot0 >= NS) continue;
            }
            const int slot = slot0 + (t & 63);
            const int row = slot / SPR, ch = slot - row * SPR;
            const uint32_t off = ch < CPR ? ((uint32_t)(r0 + row) * (uint32_t)(E * 2) + (uint32_t)ch * 16u) : 0xFFFFFFF0u;
            lds_void* base = (lds_void*)(dst + slot0 * 8);
            if constexpr (NS % 64 != 0) {
                if (slot >= NS) continue;  // partial last instruction: its lanes past the tile stay idle
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, base, 16, (int)off, 0, 0, 0);
        }
    }

    // The same loads with the per-lane byte offsets (relative to the tile's first row)
    // computed once, outside the tile loop: a tile then costs only scalar work to build a
    // resource that starts at its first row and ends at the slice's end, so rows past the
    // slice still read zeros, and no vector instructions go to address arithmetic.
    struct Offs { uint32_t o[NI]; };
    __device__ __forceinline__ static Offs offsets(int t, int wave) {
        Offs r;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int slot = i * NT + wave * 64 + (t & 63);
            const int row = slot / SPR, ch = slot - row * SPR;
            r.o[i] = ch < CPR ? (uint32_t)row * (uint32_t)(E * 2) + (uint32_t)ch * 16u : 0xFFFFFFF0u;
        }
        return r;
    }
    // Rows [r0, r0 + NR) of the slice of `nrows` rows at `slice` into the LDS tile at dst.
    __device__ __forceinline__ static void load(const T* slice, int nrows, int r0, const Offs& off, T* dst, int t,
                                                int wave) {
        static_assert(kOK, "16-bit tiles with one padding chunk per row");
        typedef __attribute__((address_space(3))) void lds_void;
        const rsrc_t rs = make_rsrc(slice + (int64_t)r0 * E, nrows > r0 ? (uint32_t)(nrows - r0) * (uint32_t)(E * 2) : 0u);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int slot0 = i * NT + wave * 64;
            if constexpr (NS % NT != 0) {
                if (slot0 >= NS) continue;
            }
            if constexpr (NS % 64 != 0) {
                if (slot0 + (t & 63) >= NS) continue;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + slot0 * 8), 16, (int)off.o[i], 0, 0, 0);
        }
    }
};

// Zero columns [E, DS) of two NR-row LDS tiles (the padding read as rows E..31 of a 32-row
// MFMA block when E = 16); `t` is this thread's index among the NT threads that share them.
template <typename T, int NR, int E, int DS, int NT>
__device__ __forceinline__ void zero_pad_cols(T* a, T* b, int t) {
    for (int i = t; i < NR * (DS - E); i += NT) {
        const int row = i / (DS - E), col = E + i % (DS - E);
        a[row * DS + col] = (T)0.f;
        b[row * DS + col] = (T)0.f;
    }
}

}  // namespace onionop
