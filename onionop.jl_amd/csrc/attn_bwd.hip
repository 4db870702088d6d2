// attn_bwd.hip -- flash attention backward on gfx950 MFMA
// (replaces _flash_attention_bwd_preprocess!, src/attention_bwd.jl:177-211, and
// _flash_attention_bwd!, src/attention_bwd.jl:1-175).
//
// With P = exp(S - m) / l from the forward's (m, l) = (ms, ls) and S = scale q.k + bias
// + masks, the gradients are
//   delta = rowsum(dO o),  dP = dO V^T,  dS = P (dP - delta),
//   dV = P^T dO,  dK = scale dS^T Q,  dQ = scale dS K,  dpair = dS,
// the reference's formulas with its dO/l and delta/l folded into P
// (src/attention_bwd.jl:88-92,125-139,196-210).
//
// Three kernels, no atomics (results are deterministic):
//  1. preprocess: delta and lse2 = log2(l) + m log2(e) per query row (B, QH, QL).
//  2. dK/dV: a workgroup owns 128 keys of one (kv head, batch), wave w owns 32 of them
//     with their K and V fragments in registers; it walks every q head of the GQA group
//     and every 64-query tile (from the diagonal when causal), accumulating dV^T and
//     dK^T in registers:  S = Q K^T and dP = dO V^T (A = Q, dO tiles from LDS),
//     P and dS in the C layout (key per lane), then dV^T += dO^T P and dK^T += Q^T dS
//     with A read from transposed LDS copies of dO and Q and B = P, dS from registers.
//  3. dQ: a workgroup owns 128 queries (32 per wave, Q and dO fragments in registers)
//     and walks the key tiles: S^T = K Q^T, dP^T = V dO^T, dS^T, dQ^T += K^T dS^T;
//     it also writes dpair, whose (QH, QL, KL, B) layout puts consecutive queries of a
//     head QH elements apart, and zeroes dpair above the causal diagonal.
#include "attn_common.h"
#include "launch.h"

namespace onionop {

template <typename T> struct BPad { static constexpr int V = 16 / (int)sizeof(T); };
template <> struct BPad<float> { static constexpr int V = 1; };

// Same cooperative global -> LDS tile copy as the forward (natural and/or transposed).
template <typename T, int E, int NR, bool NAT, bool TRN, bool QK16>
__device__ __forceinline__ void btile_to_lds(const T* __restrict__ src, int r0, int nrows, T* dst, int DS, T* dst_t,
                                             int DTS) {
    constexpr int VN = 16 / (int)sizeof(T);
    constexpr int VPR = E / VN;
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

// Fragment of a row of global memory, optionally rounded to float16 values.
template <typename T, bool QK16>
__device__ __forceinline__ typename Mfma<T>::frag gload_frag(const T* p) {
    typename Mfma<T>::frag f = load_frag<T>(p);
    if constexpr (QK16 && sizeof(T) == 4) f = round_f16(f);
    return f;
}

// ------------------------------------------------------------------ preprocess
template <typename T, int E>
__global__ __launch_bounds__(256) void attn_bwd_pre_kernel(const T* __restrict__ dO, const T* __restrict__ o,
                                                           const float* __restrict__ ms, const float* __restrict__ ls,
                                                           float* __restrict__ lse2, float* __restrict__ delta,
                                                           int64_t rows) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    constexpr int VN = 16 / (int)sizeof(T);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < E; e += VN) {
        float a[VN], c[VN];
        load_vec<T>(dO + r * E + e, a);
        load_vec<T>(o + r * E + e, c);
#pragma unroll
        for (int j = 0; j < VN; ++j) d = fmaf(a[j], c[j], d);
    }
    delta[r] = d;
    const float l = ls[r];
    lse2[r] = l > 0.f ? ms[r] * kLog2e + log2f(l) : INFINITY;  // fully masked row: P = 0
}

// ------------------------------------------------------------------ dK / dV
template <typename T, int E, bool CAUSAL, bool QK16>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(
    const T* __restrict__ dO, const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ pair, const uint8_t* __restrict__ kpad, const float* __restrict__ lse2,
    const float* __restrict__ delta, T* __restrict__ dk, T* __restrict__ dv, int QL, int KL, int QH, int KH,
    float scale) {
    typedef Mfma<T> M;
    constexpr int BKK = 128, BQQ = 64;
    constexpr int EO = E < 32 ? 32 : E;
    constexpr int PAD = BPad<T>::V;
    constexpr int QS = E + PAD;     // natural Q / dO tile stride
    constexpr int TS = BQQ + PAD;   // transposed Q / dO tile stride
    __shared__ __attribute__((aligned(16))) T Qs[BQQ * QS];
    __shared__ __attribute__((aligned(16))) T dOs[BQQ * QS];
    __shared__ __attribute__((aligned(16))) T Qt[EO * TS];
    __shared__ __attribute__((aligned(16))) T dOt[EO * TS];
    __shared__ __attribute__((aligned(16))) float Ls[BQQ];
    __shared__ __attribute__((aligned(16))) float Ds[BQQ];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
    const int b = blockIdx.z, kh = blockIdx.y;
    const int k0 = blockIdx.x * BKK, kw0 = k0 + 32 * w, mykey = kw0 + l32;
    const bool k_ok = mykey < KL;
    const int rep = QH / KH;
    const float sl2 = scale * kLog2e;

    if constexpr (EO > E) {
        for (int i = tid; i < (EO - E) * TS; i += 256) {
            Qt[E * TS + i] = (T)0.f;
            dOt[E * TS + i] = (T)0.f;
        }
    }

    const T* kp = k + (int64_t)(b * KH + kh) * KL * E;
    const T* vp = v + (int64_t)(b * KH + kh) * KL * E;
    typename M::frag kf[E / M::KC], vf[E / M::KC];
#pragma unroll
    for (int c = 0; c < E / M::KC; ++c) {
        if (k_ok) {
            kf[c] = gload_frag<T, QK16>(kp + (int64_t)mykey * E + c * M::KC + h * M::KE);
            vf[c] = gload_frag<T, false>(vp + (int64_t)mykey * E + c * M::KC + h * M::KE);
        } else {
            kf[c] = typename M::frag{};
            vf[c] = typename M::frag{};
        }
    }
    const bool kp_ok = kpad == nullptr || !k_ok || kpad[(int64_t)b * KL + mykey] != 0;

    f32x16 dkacc[EO / 32], dvacc[EO / 32];
#pragma unroll
    for (int i = 0; i < EO / 32; ++i) { dkacc[i] = zero16(); dvacc[i] = zero16(); }

    const int qstart = CAUSAL ? (k0 / BQQ) * BQQ : 0;
    for (int hq = kh * rep; hq < (kh + 1) * rep; ++hq) {
        const T* qp = q + (int64_t)(b * QH + hq) * QL * E;
        const T* dop = dO + (int64_t)(b * QH + hq) * QL * E;
        const float* lp = lse2 + (int64_t)(b * QH + hq) * QL;
        const float* dp = delta + (int64_t)(b * QH + hq) * QL;
        for (int q0 = qstart; q0 < QL; q0 += BQQ) {
            __syncthreads();
            btile_to_lds<T, E, BQQ, true, true, QK16>(qp, q0, QL, Qs, QS, Qt, TS);
            btile_to_lds<T, E, BQQ, true, true, false>(dop, q0, QL, dOs, QS, dOt, TS);
            if (tid < BQQ) {
                const int qi = q0 + tid;
                Ls[tid] = qi < QL ? lp[qi] : INFINITY;
                Ds[tid] = qi < QL ? dp[qi] : 0.f;
            }
            __syncthreads();
            if (CAUSAL && q0 + BQQ - 1 < kw0) continue;
#pragma unroll
            for (int qb = 0; qb < BQQ / 32; ++qb) {
                if (CAUSAL && q0 + 32 * qb + 31 < kw0) continue;
                f32x16 sacc = zero16(), pacc = zero16();
                const T* qrow = Qs + (32 * qb + l32) * QS + h * M::KE;
                const T* drow = dOs + (32 * qb + l32) * QS + h * M::KE;
#pragma unroll
                for (int c = 0; c < E / M::KC; ++c) {
                    sacc = M::mma(load_frag<T>(qrow + c * M::KC), kf[c], sacc);
                    pacc = M::mma(load_frag<T>(drow + c * M::KC), vf[c], pacc);
                }
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int ql = 32 * qb + 8 * g + 4 * h;  // local query of registers 4g..4g+3
                    const f32x4 lse4 = *reinterpret_cast<const f32x4*>(Ls + ql);
                    const f32x4 del4 = *reinterpret_cast<const f32x4*>(Ds + ql);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int r = 4 * g + j, qi = q0 + ql + j;
                        float s = sacc[r] * sl2;
                        bool masked = !k_ok || !kp_ok || qi >= QL || (CAUSAL && mykey > qi);
                        if (pair != nullptr && !masked)
                            s += to_f32(pair[(((int64_t)b * KL + mykey) * QL + qi) * QH + hq]) * kLog2e;
                        const float p = masked ? 0.f : exp2f(s - lse4[j]);
                        sacc[r] = p;
                        pacc[r] = p * (pacc[r] - del4[j]);
                    }
                }
#pragma unroll
                for (int eb = 0; eb < EO / 32; ++eb) {
                    const T* orow = dOt + (32 * eb + l32) * TS + 32 * qb;
                    const T* trow = Qt + (32 * eb + l32) * TS + 32 * qb;
#pragma unroll
                    for (int c = 0; c < 32 / M::KC; ++c) {
                        dvacc[eb] = M::mma(load_frag_kperm<T>(orow, c, h), c_to_frag<T>(sacc, c), dvacc[eb]);
                        dkacc[eb] = M::mma(load_frag_kperm<T>(trow, c, h), c_to_frag<T>(pacc, c), dkacc[eb]);
                    }
                }
            }
        }
    }

    if (!k_ok) return;
    T* dkp = dk + ((int64_t)(b * KH + kh) * KL + mykey) * E;
    T* dvp = dv + ((int64_t)(b * KH + kh) * KL + mykey) * E;
    typedef T t4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int eb = 0; eb < EO / 32; ++eb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int e = 32 * eb + 8 * g + 4 * h;
            if (e < E) {
                t4 a, c;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    a[j] = from_f32<T>(dkacc[eb][4 * g + j] * scale);
                    c[j] = from_f32<T>(dvacc[eb][4 * g + j]);
                }
                *reinterpret_cast<t4*>(dkp + e) = a;
                *reinterpret_cast<t4*>(dvp + e) = c;
            }
        }
}

// ------------------------------------------------------------------ dQ (+ dpair)
template <typename T, int E, bool CAUSAL, bool QK16>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(
    const T* __restrict__ dO, const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ pair, const uint8_t* __restrict__ kpad, const float* __restrict__ lse2,
    const float* __restrict__ delta, T* __restrict__ dq, T* __restrict__ dpair, int QL, int KL, int QH, int KH,
    float scale) {
    typedef Mfma<T> M;
    constexpr int BQ = 128, BK = 64;
    constexpr int EO = E < 32 ? 32 : E;
    constexpr int PAD = BPad<T>::V;
    constexpr int KS = E + PAD;
    constexpr int KTS = BK + PAD;
    __shared__ __attribute__((aligned(16))) T Ks[BK * KS];
    __shared__ __attribute__((aligned(16))) T Vs[BK * KS];
    __shared__ __attribute__((aligned(16))) T Kt[EO * KTS];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
    const int b = blockIdx.z, qh = blockIdx.y;
    const int qt = CAUSAL ? (int)(gridDim.x - 1 - blockIdx.x) : (int)blockIdx.x;
    const int kh = qh / (QH / KH);
    const int q0 = qt * BQ, qw0 = q0 + 32 * w, myq = qw0 + l32;
    const bool q_ok = myq < QL;
    const float sl2 = scale * kLog2e;

    if constexpr (EO > E) {
        for (int i = tid; i < (EO - E) * KTS; i += 256) Kt[E * KTS + i] = (T)0.f;
    }

    const T* qp = q + (int64_t)(b * QH + qh) * QL * E;
    const T* dop = dO + (int64_t)(b * QH + qh) * QL * E;
    const T* kp = k + (int64_t)(b * KH + kh) * KL * E;
    const T* vp = v + (int64_t)(b * KH + kh) * KL * E;
    typename M::frag qf[E / M::KC], df[E / M::KC];
#pragma unroll
    for (int c = 0; c < E / M::KC; ++c) {
        if (q_ok) {
            qf[c] = gload_frag<T, QK16>(qp + (int64_t)myq * E + c * M::KC + h * M::KE);
            df[c] = gload_frag<T, false>(dop + (int64_t)myq * E + c * M::KC + h * M::KE);
        } else {
            qf[c] = typename M::frag{};
            df[c] = typename M::frag{};
        }
    }
    const int64_t srow = (int64_t)(b * QH + qh) * QL + myq;
    const float lse_me = q_ok ? lse2[srow] : INFINITY;
    const float del_me = q_ok ? delta[srow] : 0.f;

    f32x16 dqacc[EO / 32];
#pragma unroll
    for (int i = 0; i < EO / 32; ++i) dqacc[i] = zero16();

    const int nkt_all = (KL + BK - 1) / BK;
    int nkt = nkt_all;
    if (CAUSAL) nkt = min(nkt, (min(q0 + BQ, QL) - 1) / BK + 1);
    T* dpp = dpair != nullptr ? dpair + ((int64_t)b * KL * QL + myq) * QH + qh : nullptr;  // + key * QL * QH

    for (int kt = 0; kt < nkt; ++kt) {
        const int k0 = kt * BK;
        __syncthreads();
        btile_to_lds<T, E, BK, true, true, QK16>(kp, k0, KL, Ks, KS, Kt, KTS);
        btile_to_lds<T, E, BK, true, false, false>(vp, k0, KL, Vs, KS, nullptr, 0);
        __syncthreads();
        if (CAUSAL && k0 > qw0 + 31) {  // tile entirely above this wave's queries
            if (dpp != nullptr && q_ok)
                for (int j = 0; j < BK / 2; ++j) {
                    const int key = k0 + 32 * h + j;
                    if (key < KL) dpp[(int64_t)key * QL * QH] = (T)0.f;
                }
            continue;
        }
#pragma unroll
        for (int kb = 0; kb < BK / 32; ++kb) {
            f32x16 sacc = zero16(), pacc = zero16();
            const T* krow = Ks + (32 * kb + l32) * KS + h * M::KE;
            const T* vrow = Vs + (32 * kb + l32) * KS + h * M::KE;
#pragma unroll
            for (int c = 0; c < E / M::KC; ++c) {
                sacc = M::mma(load_frag<T>(krow + c * M::KC), qf[c], sacc);
                pacc = M::mma(load_frag<T>(vrow + c * M::KC), df[c], pacc);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 32 * kb + crow(r, h);
                float s = sacc[r] * sl2;
                bool masked = !q_ok || key >= KL || (CAUSAL && key > myq);
                if (kpad != nullptr && !masked) masked = kpad[(int64_t)b * KL + key] == 0;
                if (pair != nullptr && !masked)
                    s += to_f32(pair[(((int64_t)b * KL + key) * QL + myq) * QH + qh]) * kLog2e;
                const float p = masked ? 0.f : exp2f(s - lse_me);
                const float ds = p * (pacc[r] - del_me);
                pacc[r] = ds;
                if (dpp != nullptr && q_ok && key < KL) dpp[(int64_t)key * QL * QH] = from_f32<T>(ds);
            }
#pragma unroll
            for (int eb = 0; eb < EO / 32; ++eb) {
                const T* arow = Kt + (32 * eb + l32) * KTS + 32 * kb;
#pragma unroll
                for (int c = 0; c < 32 / M::KC; ++c)
                    dqacc[eb] = M::mma(load_frag_kperm<T>(arow, c, h), c_to_frag<T>(pacc, c), dqacc[eb]);
            }
        }
    }
    if (CAUSAL && dpp != nullptr && q_ok) {  // zero dpair for the key tiles past the diagonal
        for (int key = nkt * BK + h; key < KL; key += 2) dpp[(int64_t)key * QL * QH] = (T)0.f;
    }

    if (!q_ok) return;
    T* dqp = dq + srow * E;
    typedef T t4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int eb = 0; eb < EO / 32; ++eb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int e = 32 * eb + 8 * g + 4 * h;
            if (e < E) {
                t4 a;
#pragma unroll
                for (int j = 0; j < 4; ++j) a[j] = from_f32<T>(dqacc[eb][4 * g + j] * scale);
                *reinterpret_cast<t4*>(dqp + e) = a;
            }
        }
}

// ------------------------------------------------------------------ launch

template <typename T, int E, bool CAUSAL, bool QK16>
static void bwd_launch(hipStream_t s, const AttnArgs& a, int stages) {
    const int64_t rows = a.B * a.QH * a.QL;
    if (stages & kBwdPre)
        attn_bwd_pre_kernel<T, E><<<dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s>>>(
            (const T*)a.dO, (const T*)a.o_in, a.ms_in, a.ls_in, a.lse2, a.delta, rows);
    if ((stages & kBwdDkDv) && a.KL > 0) {
        const dim3 g1((unsigned)((a.KL + 127) / 128), (unsigned)a.KH, (unsigned)a.B);
        attn_bwd_dkdv_kernel<T, E, CAUSAL, QK16><<<g1, dim3(256), 0, s>>>(
            (const T*)a.dO, (const T*)a.q, (const T*)a.k, (const T*)a.v, (const T*)a.pair, a.kpad, a.lse2, a.delta,
            (T*)a.dk, (T*)a.dv, (int)a.QL, (int)a.KL, (int)a.QH, (int)a.KH, a.scale);
    }
    if (!(stages & kBwdDq)) return;
    const dim3 g2((unsigned)((a.QL + 127) / 128), (unsigned)a.QH, (unsigned)a.B);
    attn_bwd_dq_kernel<T, E, CAUSAL, QK16><<<g2, dim3(256), 0, s>>>(
        (const T*)a.dO, (const T*)a.q, (const T*)a.k, (const T*)a.v, (const T*)a.pair, a.kpad, a.lse2, a.delta,
        (T*)a.dq, (T*)a.dpair, (int)a.QL, (int)a.KL, (int)a.QH, (int)a.KH, a.scale);
}

template <typename T, bool QK16>
static bool bwd_dispatch(hipStream_t s, const AttnArgs& a, int stages) {
#define ONIONOP_BWD_E(EE)                                          \
    case EE:                                                       \
        if (a.causal) bwd_launch<T, EE, true, QK16>(s, a, stages); \
        else bwd_launch<T, EE, false, QK16>(s, a, stages);         \
        return true;
    switch (a.E) {
        ONIONOP_BWD_E(16)
        ONIONOP_BWD_E(32)
        ONIONOP_BWD_E(64)
        ONIONOP_BWD_E(128)
    }
#undef ONIONOP_BWD_E
    return false;
}

bool launch_attn_bwd(hipStream_t s, int dt, const AttnArgs& a, int stages) {
    if (a.B == 0 || a.QH == 0) return true;
    if (a.QL == 0) {  // no queries: dk = dv = 0
        if (!(stages & kBwdDkDv)) return true;
        const int64_t bytes = (dt == 0 ? 4 : 2) * a.E * a.KL * a.KH * a.B;
        if (bytes > 0) {
            fill_zero_kernel<<<dim3((unsigned)((bytes + 1023) / 1024)), dim3(256), 0, s>>>(a.dk, bytes);
            fill_zero_kernel<<<dim3((unsigned)((bytes + 1023) / 1024)), dim3(256), 0, s>>>(a.dv, bytes);
        }
        return true;
    }
    switch (dt) {
        case 0: return a.qk_fp16 ? bwd_dispatch<float, true>(s, a, stages) : bwd_dispatch<float, false>(s, a, stages);
        case 1: return bwd_dispatch<f16, false>(s, a, stages);
        case 2: return bwd_dispatch<bf16, false>(s, a, stages);
    }
    return false;
}

}  // namespace onionop
