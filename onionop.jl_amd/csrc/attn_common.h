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
#ifndef ONIONOP_X6
#define ONIONOP_X6 0
#endif
#if ONIONOP_X6
// float32 through bf16 MFMA ("bf16x6"; the translation unit attn_f32x6.hip compiles the
// float32 kernels with this policy in namespace onionop_x6).  A float32 x is split
// exactly into three bf16 values, x = hi + mid + lo: hi is x with its low 16 bits cleared
// (its top 8 significand bits), mid the same of r = x - hi (exact, at most 16 significant
// bits), and lo = r - mid (exact, at most 8 significant bits, so a bf16 value).  A product
// a b is the six terms a_i b_j with i + j <= 2 (in units of 8 bits), each exact in the
// float32 accumulator; the three dropped terms are below 2^-23 |a b| together, about the
// rounding of one float32 operation.  Fragments cover KC = 16 contraction positions like
// the 16-bit types, so a float32 dot product of 16 terms costs 6 MFMAs of 32 cycles
// instead of 8 float32 MFMAs of 64.
struct f32x6_frag {
    bf16x8 hi, mid, lo;
};
template <> struct Mfma<float> {
    static constexpr int KC = 16, KE = 8;
    typedef f32x6_frag frag;
    static __device__ __forceinline__ f32x16 mma(const frag& a, const frag& b, f32x16 c) {
        // smallest terms first
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.lo, b.hi, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.hi, b.lo, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.mid, b.mid, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.mid, b.hi, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.hi, b.mid, c, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.hi, b.hi, c, 0, 0, 0);
    }
};
// The split of 8 floats: element j of each plane is the bf16 part of x[j].
__device__ __forceinline__ f32x6_frag split_f32x8(const float (&x)[8]) {
    union { uint32_t u[4]; bf16x8 f; } H, Mi, L;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t a = __float_as_uint(x[2 * j]), b = __float_as_uint(x[2 * j + 1]);
        const float ra = x[2 * j] - __uint_as_float(a & 0xFFFF0000u);
        const float rb = x[2 * j + 1] - __uint_as_float(b & 0xFFFF0000u);
        const uint32_t ua = __float_as_uint(ra), ub = __float_as_uint(rb);
        const float la = ra - __uint_as_float(ua & 0xFFFF0000u);
        const float lb = rb - __uint_as_float(ub & 0xFFFF0000u);
        H.u[j] = (a >> 16) | (b & 0xFFFF0000u);
        Mi.u[j] = (ua >> 16) | (ub & 0xFFFF0000u);
        L.u[j] = (__float_as_uint(la) >> 16) | (__float_as_uint(lb) & 0xFFFF0000u);
    }
    f32x6_frag f;
    f.hi = H.f;
    f.mid = Mi.f;
    f.lo = L.f;
    return f;
}
// The 8 floats a fragment stands for (hi + mid + lo is exact in float32).
__device__ __forceinline__ void join_f32x8(const f32x6_frag& f, float (&x)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = ((float)f.lo[j] + (float)f.mid[j]) + (float)f.hi[j];
}
// The fragment of the float16-rounded values (the reference's Float16 Q/K).
__device__ __forceinline__ f32x6_frag round_f16(const f32x6_frag& f) {
    float x[8];
    join_f32x8(f, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = round_f16(x[j]);
    return split_f32x8(x);
}
#else
template <> struct Mfma<float> {
    static constexpr int KC = 2, KE = 1;
    typedef float frag;
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};
#endif

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

// KE consecutive elements starting at p (LDS or global) as a fragment.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag load_frag(const T* p) {
#if ONIONOP_X6
    if constexpr (sizeof(T) == 4) {  // 16-byte aligned: two 16-byte LDS reads, then the split
        const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
        const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        return split_f32x8(x);
    } else
#endif
    if constexpr (Mfma<T>::KE == 8) {
        return *reinterpret_cast<const typename Mfma<T>::frag*>(p);
    } else {
        return *p;
    }
}

// A fragment whose contraction index runs along the ROWS of a tile stored naturally,
// X[k][m] (m contiguous, row stride S elements): the fragment holds rows m0 + l%32 of
// X^T and k positions kb + kperm(c, h, j) = kb + crow(KE*c + j, h), the positions a C
// tile reused as a B operand stands for.
// 16-bit: two ds_read_b64_tr_b16.  Within each group of 16 lanes the instruction returns
// to lane i the elements d[4r + i/4][i%4], r = 0..3, where d[j] are the four 16-bit values
// at lane j's address; pointing lane 4r + q at X[k0 + r][mb + 4q] therefore gives lane i
// the four consecutive k values X[k0 .. k0+3][mb + i].  Lane groups g = l/16 cover
// m = m0 + 16*(g%2) + [0,16) and half h = g/2; the two reads fetch k0 = kb + 16c + 4h and
// kb + 16c + 8 + 4h, matching kperm.  X must be in LDS and 8-byte aligned at each address.
// float32: one element X[kb + crow(c, h)][m0 + l%32].
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag load_frag_tr(const T* X, int S, int m0, int kb, int c, int lane) {
#if ONIONOP_X6
    if constexpr (sizeof(T) == 4) {  // the 8 k positions of kperm, one float each
        const int h = lane >> 5;
        const T* p = X + (kb + 16 * c + 4 * h) * S + m0 + (lane & 31);
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = p[((j & 3) + 8 * (j >> 2)) * S];
        return split_f32x8(x);
    } else
#endif
    if constexpr (Mfma<T>::KE == 8) {
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
        const int g = lane >> 4, r = (lane >> 2) & 3, q = lane & 3, h = lane >> 5;
        const int mb = m0 + 16 * (g & 1) + 4 * q;
        const int k0 = kb + 16 * c + 4 * h + r;
        const T* p0 = X + k0 * S + mb;
        const T* p1 = p0 + 8 * S;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1));
        union { s16x4 s[2]; typename Mfma<T>::frag f; } u;
        u.s[0] = lo;
        u.s[1] = hi;
        return u.f;
    } else {
        return X[(kb + crow(c, lane >> 5)) * S + m0 + (lane & 31)];
    }
}

// Chunk c of a C tile (registers KE*c .. KE*c+KE-1) converted to a B fragment.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag c_to_frag(const f32x16& acc, int c) {
#if ONIONOP_X6
    if constexpr (sizeof(T) == 4) {
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = acc[8 * c + j];
        return split_f32x8(x);
    } else
#endif
    if constexpr (Mfma<T>::KE == 8) {
        typename Mfma<T>::frag f;
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = (T)acc[8 * c + j];
        return f;
    } else {
        return acc[c];
    }
}

// Sum of the elements a fragment stands for.  For bf16x6 fragments, the sum of the hi
// parts only (the float32 centring below needs some constant vector close to the mean of
// K, not the exact mean).
template <typename T>
__device__ __forceinline__ float frag_sum(const typename Mfma<T>::frag& f) {
#if ONIONOP_X6
    if constexpr (sizeof(T) == 4) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) s += (float)f.hi[j];
        return s;
    } else
#endif
    if constexpr (Mfma<T>::KE == 8) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) s += to_f32(f[j]);
        return s;
    } else {
        return f;
    }
}

// Key-padding bytes of the keys one lane holds in a 32-key C-tile block (rows
// crow(r, h)): keys kb0 + 8 rg + 4 h + [0, 4), rg = 0..3, are 4 consecutive bytes, so
// four dword loads cover them (past KL the resource, of KL bytes, reads 0 = padded).
// A dword that straddles KL would read as zero as a whole, so rows whose length is not
// a multiple of 4 load the bytes one by one (uniform branch).
struct KpadBlock {
    uint32_t d[4];
    __device__ __forceinline__ void load(rsrc_t r, int kb0, int h, int KL) {
        if ((KL & 3) == 0) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg)
                d[rg] = __builtin_amdgcn_raw_buffer_load_b32(r, kb0 + 8 * rg + 4 * h, 0, 0);
        } else {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                uint32_t x = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    x |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, kb0 + 8 * rg + 4 * h + j, 0, 0) << (8 * j);
                d[rg] = x;
            }
        }
    }
    // key of register r is a real key (non-zero byte)
    __device__ __forceinline__ bool ok(int r) const { return ((d[r >> 2] >> (8 * (r & 3))) & 0xFFu) != 0u; }
    // every key of this lane's 16 is real / none is
    __device__ __forceinline__ bool all() const {
        bool z = false;
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) z |= ((d[rg] - 0x01010101u) & ~d[rg] & 0x80808080u) != 0u;  // has a zero byte
        return !z;
    }
    __device__ __forceinline__ bool none() const { return (d[0] | d[1] | d[2] | d[3]) == 0u; }
};

// ---------------------------------------------------------------- pair bias
// The bias tensor is (B, KL, QL, QH) row-major == Julia (QH, QL, KL, B): element
// (b, key, query, head) at ((b KL + key) QL + query) QH + head.  The heads of one
// (key, query) are adjacent, so no two elements a lane needs are: every element is its
// own 16/32-bit buffer access.  The loads are unconditional (offsets past the resource
// read 0) and keep raw bits in registers until the scores use them, so a block's loads
// issue back to back and are prefetched a tile ahead.  Offsets are 32-bit: the host
// requires 64 QL QH sizeof(T) < 2^32 (a resource spans at most 64 key rows).

// Raw bits of the element of type T at byte offset off (0 past the resource).
template <typename T>
__device__ __forceinline__ uint32_t bload_bits(rsrc_t r, uint32_t off) {
    if constexpr (sizeof(T) == 4) return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
    else return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
template <typename T>
__device__ __forceinline__ float bits_f32(uint32_t u) {
    if constexpr (sizeof(T) == 4) return __uint_as_float(u);
    else if constexpr (__is_same(T, bf16)) return __uint_as_float(u << 16);
    else return (float)__builtin_bit_cast(f16, (unsigned short)u);
}
// Store x as T at byte offset off (dropped past the resource).
template <typename T>
__device__ __forceinline__ void bstore_elem(rsrc_t r, uint32_t off, float x) {
    if constexpr (sizeof(T) == 4) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, (int)off, 0, 0);
    } else {
        const T t = from_f32<T>(x);
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, t), r, (int)off, 0, 0);
    }
}

// Resource over the bias of rows [k0, k0 + nrows) of batch b, head `head`: the byte
// offset of (key k0 + i, query j) is (i QL + j) QH sizeof(T).  Rows past KL read 0.
template <typename T>
__device__ __forceinline__ rsrc_t pair_rsrc(const T* pair, int b, int k0, int nrows, int KL, int QL, int QH, int head) {
    const int rows = max(0, min(nrows, KL - k0));
    const uint32_t bytes = rows > 0 ? ((uint32_t)rows * (uint32_t)QL * (uint32_t)QH - (uint32_t)head) * sizeof(T) : 0u;
    return make_rsrc(pair + (((int64_t)b * KL + k0) * QL) * QH + head, bytes);
}

// Byte offsets of one lane's 16 elements of a 32 x 32 C block, rows crow(r, h):
//  query lane (S^T tiles: lane = query q, rows = keys kbl + crow(r, h) of the resource)
//    ((kbl + crow(r, h)) QL + q) QH sizeof(T);
//  key lane (S tiles: lane = key kl of the resource, rows = queries qb + crow(r, h))
//    (kl QL + qb + crow(r, h)) QH sizeof(T).
template <typename T>
__device__ __forceinline__ uint32_t pair_off_q(int kbl, int r, int q, int h, int QL, int QH) {
    return ((uint32_t)(kbl + crow(r, h)) * (uint32_t)QL + (uint32_t)q) * (uint32_t)QH * sizeof(T);
}
template <typename T>
__device__ __forceinline__ uint32_t pair_off_k(int kl, int qb, int r, int h, int QL, int QH) {
    return ((uint32_t)kl * (uint32_t)QL + (uint32_t)(qb + crow(r, h))) * (uint32_t)QH * sizeof(T);
}

// The bias bits of one lane's 16 rows of a 32 x 32 block.
template <typename T>
struct PairBlock {
    uint32_t u[16];
    __device__ __forceinline__ void load_q(rsrc_t rs, int kbl, int q, int h, int QL, int QH) {
#pragma unroll
        for (int r = 0; r < 16; ++r) u[r] = bload_bits<T>(rs, pair_off_q<T>(kbl, r, q, h, QL, QH));
    }
    __device__ __forceinline__ void load_k(rsrc_t rs, int kl, int qb, int h, int QL, int QH) {
#pragma unroll
        for (int r = 0; r < 16; ++r) u[r] = bload_bits<T>(rs, pair_off_k<T>(kl, qb, r, h, QL, QH));
    }
    __device__ __forceinline__ float get(int r) const { return bits_f32<T>(u[r]); }
};

// Workgroups are dispatched round-robin over the 8 XCDs (block x runs on XCD x % 8),
// and each XCD has its own L2.  xcd_group renumbers the n blocks of a grid so that G
// consecutive logical indices run on one XCD and successive groups of G on successive
// XCDs; a tail of fewer than 8 G blocks keeps the plain order.  With G = the heads of
// one (batch, tile), the heads that share every bias cache line share one L2.
__device__ __forceinline__ int xcd_group(int x, int G, int n) {
    const int round = 8 * G, full = n - n % round;
    if (x >= full) return x;
    const int j = x >> 3;
    return (j / G) * round + (x & 7) * G + j % G;
}

// (rank, batch, q head) of block x of a query-tile grid of ranks x NB x QH blocks.  Plain
// order: the rank varies slowest, (batch, q head) fastest.  With GQA (rep = QH / KH > 1)
// and NB KH a multiple of 8, each XCD (block x runs on XCD x % 8) instead takes whole
// (batch, kv head) pairs, the rep q heads of a pair next to each other, still rank by
// rank: an XCD's L2 then serves the K/V of NB KH / 8 pairs to all their q heads, instead
// of the K/V of up to 8 times as many pairs to one q head each.
struct QBlock {
    int rank, b, qh;
};
__device__ __forceinline__ QBlock qblock_map(int x, int QH, int KH, int NB) {
    QBlock r;
    const int rep = QH / KH, pairs = NB * KH;
    if (rep > 1 && (pairs & 7) == 0) {
        const int xcd = x & 7, j = x >> 3, per = pairs >> 3;
        const int jq = j % rep, t = j / rep;
        const int p = (t % per) * 8 + xcd;
        r.rank = t / per;
        r.b = p / KH;
        r.qh = (p % KH) * rep + jq;
    } else {
        const int BH = QH * NB, bh = x % BH;
        r.rank = x / BH;
        r.b = bh / QH;
        r.qh = bh % QH;
    }
    return r;
}

// (rank, batch, q head) of block x of a grid of n = nq NB QH blocks (nq ranks, nq % 4 == 0)
// that is resident all at once, four blocks per CU, with blocks x, x + n/4, x + n/2 and
// x + 3n/4 on one CU (the dispatcher fills the CUs round by round).  The plain order gives
// CU c the ranks k, k + nq/4, k + nq/2, k + 3nq/4 (k = c / (NB QH)), whose causal work
// falls with k; here the four slots take ranks k, nq/2 - 1 - k, nq/2 + k and nq - 1 - k,
// whose work sums to the same for every CU, and the longest ranks still start first.
__device__ __forceinline__ QBlock qblock_balanced(int x, int n, int nq, int QH, int NB) {
    const int q4 = nq / 4, quarter = n / 4, slot = x / quarter, c = x % quarter;
    const int BH = QH * NB, k = c / BH, bh = c % BH;
    QBlock r;
    r.rank = slot == 0 ? k : slot == 1 ? 2 * q4 - 1 - k : slot == 2 ? 2 * q4 + k : 4 * q4 - 1 - k;
    r.b = bh / QH;
    r.qh = bh % QH;
    return r;
}

// Packed variable-length sequences: sequence b is rows cu_q[b] .. cu_q[b+1] of every q
// head's (Tq x E) slab (and of the per-query statistics), rows cu_k[b] .. cu_k[b+1] of
// every k / v head's (Tk x E) slab.  cu_q == nullptr: dense (B, H, L, E) tensors.
struct VarLen {
    const int* cu_q;
    const int* cu_k;
    int Tq, Tk;
};

// Where the attention problem of sequence (batch) b sits: q rows of head h start at
// qbase + h * qhs, k rows of head h at kbase + h * khs; QL / KL are its lengths.  Grids
// are sized for the maxima QLmax / KLmax (the dense lengths); varlen offsets are clamped
// into their tensors, so malformed offsets cannot move an access outside them.
struct SeqRows {
    int64_t qbase, kbase, qhs, khs;
    int QL, KL;
    __device__ __forceinline__ int64_t qrow(int h) const { return qbase + (int64_t)h * qhs; }
    __device__ __forceinline__ int64_t krow(int h) const { return kbase + (int64_t)h * khs; }
};
__device__ __forceinline__ SeqRows seq_rows(const VarLen& vl, int b, int QH, int KH, int QLmax, int KLmax) {
    SeqRows s;
    if (vl.cu_q == nullptr) {
        s.qbase = (int64_t)b * QH * QLmax;
        s.kbase = (int64_t)b * KH * KLmax;
        s.qhs = QLmax;
        s.khs = KLmax;
        s.QL = QLmax;
        s.KL = KLmax;
    } else {
        const int q0 = min(max(vl.cu_q[b], 0), vl.Tq), q1 = min(max(vl.cu_q[b + 1], q0), vl.Tq);
        const int k0 = min(max(vl.cu_k[b], 0), vl.Tk), k1 = min(max(vl.cu_k[b + 1], k0), vl.Tk);
        s.qbase = __builtin_amdgcn_readfirstlane(q0);
        s.kbase = __builtin_amdgcn_readfirstlane(k0);
        s.qhs = vl.Tq;
        s.khs = vl.Tk;
        s.QL = __builtin_amdgcn_readfirstlane(min(q1 - q0, QLmax));
        s.KL = __builtin_amdgcn_readfirstlane(min(k1 - k0, KLmax));
    }
    return s;
}

// The pullback of the Llama rotate-half rotation (∇llama_rope, src/rope/llama_rope.jl:24-65
// with sin_sign = -1) applied to one row of a gradient held as C-tile registers: this
// lane's row (a query in dQ, a key in dK) has column e = 32 eb + 8 gg + 4 h + j in register
// acc[eb][4 gg + j].  For i < E/2, with c = cos[i], s = sin[i] of the row's position:
//   g_i <- g_i c + g_{i+E/2} s,   g_{i+E/2} <- g_{i+E/2} c - g_i s.
// Both columns of a pair sit in this lane (E/2 is a multiple of 8, so column i + E/2 is
// register ((i + E/2) / 32, ((i + E/2) % 32) / 8) with the same h and j), so the rotation
// needs no exchange.  ctab / stab are resources over the cos / sin tables (float32, E per
// row, the first E/2 used) and row_off the byte offset of this row in them.
template <int E, int NEB>
__device__ __forceinline__ void rope_bwd_row(f32x16 (&acc)[NEB], rsrc_t ctab, rsrc_t stab, uint32_t row_off, int h) {
    constexpr int HALF = E / 2;
    static_assert(HALF % 8 == 0, "rotation pairs in whole 8-column groups");
#pragma unroll
    for (int eb = 0; eb < NEB; ++eb)
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
            if (32 * eb + 8 * gg >= HALF) continue;  // compile time: this group's columns are >= E/2
            const int e0 = 32 * eb + 8 * gg;
            const int eb2 = (e0 + HALF) / 32, gg2 = ((e0 + HALF) % 32) / 8;
            const uint32_t off = row_off + (uint32_t)(e0 + 4 * h) * 4u;
            const u32x4 cr = bload16(ctab, off), sr = bload16(stab, off);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float c = __uint_as_float(cr[j]), sn = __uint_as_float(sr[j]);
                const float a = acc[eb][4 * gg + j], b2 = acc[eb2][4 * gg2 + j];
                acc[eb][4 * gg + j] = fmaf(a, c, b2 * sn);
                acc[eb2][4 * gg2 + j] = fmaf(b2, c, -(a * sn));
            }
        }
}

// Tables of the fused rotation (nullptr: none): cos / sin (rows x E) float32, a row per
// (batch, position) -- row b L + pos for dense tensors, the packed row for packed sequences.
struct RopeTab {
    const float* cos;
    const float* sin;
    int64_t rows;
};

// The reduction range of a four-head bias kernel spread over n workgroups (n > 1): keys
// for dQ, queries for dK / dV.  Range r writes float32 partial rows to part[r][row][E]
// (rows in the output's order; dK / dV: the n dK partials, then the n dV partials), and a
// second launch sums the n partials in range order into the outputs.  n <= 1: direct.
struct RangeSplit {
    float* part;
    int n;
};

// Element type helpers for the float16-rounded Q/K of the reference backward.
template <typename T, bool QK16>
__device__ __forceinline__ T qk_round(T x) {
    if constexpr (QK16 && sizeof(T) == 4) return round_f16(x);
    else return x;
}

}  // namespace onionop
