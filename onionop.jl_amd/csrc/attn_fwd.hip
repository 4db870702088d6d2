// attn_fwd.hip -- flash attention forward on gfx950 MFMA
// (replaces _flash_attention_fwd!, src/attention.jl:8-143).
//
// Layout: q (B, QH, QL, E), k/v (B, KH, KL, E) row-major == Julia (E, L, H, B);
// pair (B, KL, QL, QH) == Julia (QH, QL, KL, B); kpad (B, KL) bytes; ms/ls (B, QH, QL).
//
// A workgroup is 4 waves and owns BQ = 128 queries of one (q head, batch); wave w owns
// queries q0 + 32w + [0, 32).  Per key tile of BK = 64 keys:
//   S^T (keys x queries) = K Q^T     A = K tile from LDS (rows = keys), B = Q fragments
//                                    kept in registers for the whole kernel;
//   online softmax per query column: the C layout puts one query per lane, so the row
//   max / sum is a loop over registers plus one cross-half shuffle (lane ^ 32);
//   O^T (E x queries) += V^T P^T     A = V^T tile from LDS (stored transposed),
//                                    B = P^T taken straight from the S^T registers.
// Scores live in log2 units (scale * log2 e folded in), exp is exp2.  The bias is added
// after scaling, then causal and key-padding masks, as in the reference
// (src/attention.jl:63-89).  Causal workgroups stop at the diagonal tile and waves skip
// tiles entirely above their queries; heavy (late) q tiles are scheduled first.
#include "attn_common.h"
#include "launch.h"

namespace onionop {

template <typename T> struct Pad { static constexpr int V = 16 / (int)sizeof(T); };
template <> struct Pad<float> { static constexpr int V = 1; };

// Cooperative load of rows [r0, r0 + NR) (NR x E elements, contiguous in global memory)
// into LDS, natural (dst[r][e], stride DS) and/or transposed (dst_t[e][r], stride DTS).
// Rows at or past `nrows` are zero.  If QK16 the values are rounded to float16 (float T).
template <typename T, int E, int NR, bool NAT, bool TRN, bool QK16>
__device__ __forceinline__ void tile_to_lds(const T* __restrict__ src, int r0, int nrows, T* dst, int DS, T* dst_t,
                                            int DTS) {
    constexpr int VN = 16 / (int)sizeof(T);
    constexpr int VPR = E / VN;  // vectors per row
    constexpr int NVEC = NR * VPR;
    for (int vi = threadIdx.x; vi < NVEC; vi += 256) {
        const int r = vi / VPR, e0 = (vi % VPR) * VN;
        union { u32x4 v; T e[VN]; } u;
        if (r0 + r < nrows) u.v = *reinterpret_cast<const u32x4*>(src + (int64_t)(r0 + r) * E + e0);
        else u.v = u32x4{0u, 0u, 0u, 0u};
        if constexpr (QK16) {
#pragma unroll
            for (int j = 0; j < VN; ++j) u.e[j] = qk_round<T, true>(u.e[j]);
        }
        if constexpr (NAT) {
            if constexpr (sizeof(T) == 2) *reinterpret_cast<u32x4*>(dst + r * DS + e0) = u.v;
            else {
#pragma unroll
                for (int j = 0; j < VN; ++j) dst[r * DS + e0 + j] = u.e[j];
            }
        }
        if constexpr (TRN) {
#pragma unroll
            for (int j = 0; j < VN; ++j) dst_t[(e0 + j) * DTS + r] = u.e[j];
        }
    }
}

template <typename T, int E, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                       const T* __restrict__ v, const T* __restrict__ pair,
                                                       const uint8_t* __restrict__ kpad, T* __restrict__ o,
                                                       float* __restrict__ ms, float* __restrict__ ls, int QL,
                                                       int KL, int QH, int KH, float scale) {
    typedef Mfma<T> M;
    constexpr int BQ = 128, BK = 64;
    constexpr int EO = E < 32 ? 32 : E;  // O^T rows, padded to a full 32-row MFMA block
    constexpr int PAD = Pad<T>::V;
    constexpr int KS = E + PAD;    // K tile row stride
    constexpr int VTS = BK + PAD;  // V^T tile row stride
    __shared__ __attribute__((aligned(16))) T Ks[BK * KS];
    __shared__ __attribute__((aligned(16))) T Vt[EO * VTS];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
    const int b = blockIdx.z, qh = blockIdx.y;
    const int qt = CAUSAL ? (int)(gridDim.x - 1 - blockIdx.x) : (int)blockIdx.x;
    const int kh = qh / (QH / KH);
    const int q0 = qt * BQ, qw0 = q0 + 32 * w, myq = qw0 + l32;
    const bool q_ok = myq < QL;

    const T* qp = q + (int64_t)(b * QH + qh) * QL * E;
    const T* kp = k + (int64_t)(b * KH + kh) * KL * E;
    const T* vp = v + (int64_t)(b * KH + kh) * KL * E;

    if constexpr (EO > E) {  // zero the padding rows of V^T once
        for (int i = tid; i < (EO - E) * VTS; i += 256) Vt[E * VTS + i] = (T)0.f;
    }

    typename M::frag qf[E / M::KC];
#pragma unroll
    for (int c = 0; c < E / M::KC; ++c) {
        if (q_ok) qf[c] = load_frag<T>(qp + (int64_t)myq * E + c * M::KC + h * M::KE);
        else qf[c] = typename M::frag{};
    }

    f32x16 oacc[EO / 32];
#pragma unroll
    for (int i = 0; i < EO / 32; ++i) oacc[i] = zero16();
    float m2 = -INFINITY, lsum = 0.f;
    const float sl2 = scale * kLog2e;

    int nkt = (KL + BK - 1) / BK;
    if (CAUSAL) {
        const int last = min(q0 + BQ, QL) - 1;  // largest query of the tile
        nkt = min(nkt, last / BK + 1);
    }
    for (int kt = 0; kt < nkt; ++kt) {
        const int k0 = kt * BK;
        __syncthreads();
        tile_to_lds<T, E, BK, true, false, false>(kp, k0, KL, Ks, KS, nullptr, 0);
        tile_to_lds<T, E, BK, false, true, false>(vp, k0, KL, nullptr, 0, Vt, VTS);
        __syncthreads();
        if (CAUSAL && k0 > qw0 + 31) continue;  // every key of the tile is after every query of the wave

        f32x16 sacc[BK / 32];
#pragma unroll
        for (int kb = 0; kb < BK / 32; ++kb) {
            sacc[kb] = zero16();
            const T* arow = Ks + (32 * kb + l32) * KS + h * M::KE;
#pragma unroll
            for (int c = 0; c < E / M::KC; ++c) sacc[kb] = M::mma(load_frag<T>(arow + c * M::KC), qf[c], sacc[kb]);
        }
        // scale, bias, masks; tile max
        float tmax = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 32 * kb + crow(r, h);
                float s = sacc[kb][r] * sl2;
                bool masked = key >= KL || (CAUSAL && key > myq);
                if (pair != nullptr && !masked && q_ok)
                    s += to_f32(pair[(((int64_t)b * KL + key) * QL + myq) * QH + qh]) * kLog2e;
                if (kpad != nullptr && !masked) masked = kpad[(int64_t)b * KL + key] == 0;
                s = masked ? -INFINITY : s;
                sacc[kb][r] = s;
                tmax = fmaxf(tmax, s);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(m2, tmax);
        const float muse = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = exp2f(m2 - muse);
        float psum = 0.f;
#pragma unroll
        for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = exp2f(sacc[kb][r] - muse);
                sacc[kb][r] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 32, 64);
        lsum = lsum * alpha + psum;
        m2 = mnew;
#pragma unroll
        for (int eb = 0; eb < EO / 32; ++eb)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[eb][r] *= alpha;
        // O^T += V^T P^T
#pragma unroll
        for (int eb = 0; eb < EO / 32; ++eb) {
            const T* arow = Vt + (32 * eb + l32) * VTS;
#pragma unroll
            for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
                for (int c = 0; c < 32 / M::KC; ++c)
                    oacc[eb] = M::mma(load_frag_kperm<T>(arow + 32 * kb, c, h), c_to_frag<T>(sacc[kb], c), oacc[eb]);
        }
    }

    if (!q_ok) return;
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    T* op = o + ((int64_t)(b * QH + qh) * QL + myq) * E;
#pragma unroll
    for (int eb = 0; eb < EO / 32; ++eb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int e = 32 * eb + 8 * g + 4 * h;
            if (e < E) {
                typedef T t4 __attribute__((ext_vector_type(4)));
                t4 val;
#pragma unroll
                for (int j = 0; j < 4; ++j) val[j] = from_f32<T>(oacc[eb][4 * g + j] * inv);
                *reinterpret_cast<t4*>(op + e) = val;
            }
        }
    if (h == 0) {
        const int64_t si = (int64_t)(b * QH + qh) * QL + myq;
        ms[si] = lsum > 0.f ? m2 * kLn2 : -INFINITY;
        ls[si] = lsum;
    }
}

template <typename T, int E, bool CAUSAL>
static void fwd_launch(hipStream_t s, const AttnArgs& a) {
    const dim3 grid((unsigned)((a.QL + 127) / 128), (unsigned)a.QH, (unsigned)a.B);
    attn_fwd_kernel<T, E, CAUSAL><<<grid, dim3(256), 0, s>>>(
        (const T*)a.q, (const T*)a.k, (const T*)a.v, (const T*)a.pair, a.kpad, (T*)a.o, a.ms, a.ls, (int)a.QL,
        (int)a.KL, (int)a.QH, (int)a.KH, a.scale);
}

template <typename T>
static bool fwd_dispatch(hipStream_t s, const AttnArgs& a) {
#define ONIONOP_FWD_E(EE)                                          \
    case EE:                                                       \
        if (a.causal) fwd_launch<T, EE, true>(s, a);               \
        else fwd_launch<T, EE, false>(s, a);                       \
        return true;
    switch (a.E) {
        ONIONOP_FWD_E(16)
        ONIONOP_FWD_E(32)
        ONIONOP_FWD_E(64)
        ONIONOP_FWD_E(128)
    }
#undef ONIONOP_FWD_E
    return false;
}

bool launch_attn_fwd(hipStream_t s, int dt, const AttnArgs& a) {
    if (a.QL == 0 || a.QH == 0 || a.B == 0) return true;
    switch (dt) {
        case 0: return fwd_dispatch<float>(s, a);
        case 1: return fwd_dispatch<f16>(s, a);
        case 2: return fwd_dispatch<bf16>(s, a);
    }
    return false;
}

}  // namespace onionop
