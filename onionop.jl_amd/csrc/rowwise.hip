// rowwise.hip -- HBM-bound kernels that reduce along the contiguous dimension:
// online softmax fwd/bwd, RMS norm fwd/bwd, layer norm fwd/bwd.
//
// Layout: a Julia (N, M) column-major matrix is M contiguous rows of N elements here.
// One 256-thread workgroup owns one row at a time and keeps the whole row in registers
// (NV 16-byte vectors per thread), so every element is read from HBM once and written
// once; reductions are wave64 shuffles plus one LDS exchange (one barrier) across the
// 4 waves.  Workgroups are persistent over rows and software-pipelined: the loads of a
// workgroup's next rows (the next two row blocks in the norm backward) are in flight
// while it reduces and stores the current ones, so reads and writes of neighbouring rows
// overlap.  Per-element weights stay in registers across rows, and the
// backward's weight-gradient partials accumulate in registers, one float32 partial row
// per workgroup, summed by one column-reduction launch with a fixed order.
// All row accesses are buffer loads / stores over a resource that ends at the row's
// last element: tails read zero and drop their stores without branches.
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace onionop {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// Row I/O for VEC elements of T per slot: slot i of thread t covers elements
// [VEC (t + 256 i), +VEC).  VEC is 16 / sizeof(T) (one 16-byte vector) or 1.
template <typename T, int VEC>
struct RowIO {
    typedef typename std::conditional<VEC == 1, uint32_t, u32x4>::type raw;
    static __device__ __forceinline__ uint32_t off(int i) {
        return (uint32_t)(VEC * (threadIdx.x + i * kThreads)) * (uint32_t)sizeof(T);
    }
    // the slot at byte offset o of the resource
    static __device__ __forceinline__ raw load_at(rsrc_t r, uint32_t o) {
        if constexpr (VEC != 1) return bload16_nt(r, o);
        else if constexpr (sizeof(T) == 4) return __builtin_amdgcn_raw_buffer_load_b32(r, (int)o, 0, kNT);
        else return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)o, 0, kNT);
    }
    static __device__ __forceinline__ raw load(rsrc_t r, int i) { return load_at(r, off(i)); }
    static __device__ __forceinline__ void to_float(raw v, float* out) {
        if constexpr (VEC != 1) {
            union { u32x4 v; T e[VEC]; } u;
            u.v = v;
#pragma unroll
            for (int j = 0; j < VEC; ++j) out[j] = to_f32(u.e[j]);
        } else if constexpr (sizeof(T) == 4) {
            out[0] = __uint_as_float(v);
        } else {
            union { uint16_t s; T e; } u;
            u.s = (uint16_t)v;
            out[0] = to_f32(u.e);
        }
    }
    static __device__ __forceinline__ void store_at(rsrc_t r, uint32_t o, const float* in) {
        if constexpr (VEC != 1) {
            union { u32x4 v; T e[VEC]; } u;
#pragma unroll
            for (int j = 0; j < VEC; ++j) u.e[j] = from_f32<T>(in[j]);
            bstore16_nt(u.v, r, o);
        } else if constexpr (sizeof(T) == 4) {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(in[0]), r, (int)o, 0, kNT);
        } else {
            union { uint16_t s; T e; } u;
            u.e = from_f32<T>(in[0]);
            __builtin_amdgcn_raw_buffer_store_b16(u.s, r, (int)o, 0, kNT);
        }
    }
    static __device__ __forceinline__ void store(rsrc_t r, int i, const float* in) { store_at(r, off(i), in); }
};

// Resource over row r of a (rows x n) matrix; an empty one for r >= rows (its loads
// read zero), so the prefetch of a row past the end needs no branch.
template <typename T>
__device__ __forceinline__ rsrc_t row_rsrc(const T* base, int64_t r, int64_t rows, int64_t n) {
    const bool ok = r < rows;
    return make_rsrc(base + (ok ? r : 0) * n, ok ? (uint32_t)(n * (int64_t)sizeof(T)) : 0u);
}

template <int VEC>
__device__ __forceinline__ bool slot_valid(int64_t n, int i) {
    return (int64_t)VEC * (threadIdx.x + (int64_t)i * kThreads) < n;
}

// Weight vector of runtime dtype `dt` (F32/F16/BF16): VEC consecutive values as float.
template <int VEC>
__device__ __forceinline__ void load_w(const void* __restrict__ w, int dt, int64_t n, int i, float* out) {
    const int64_t e0 = (int64_t)VEC * (threadIdx.x + (int64_t)i * kThreads);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
        const int64_t e = e0 + j;
        float v = 0.f;
        if (e < n) {
            if (dt == 0) v = reinterpret_cast<const float*>(w)[e];
            else if (dt == 1) v = to_f32(reinterpret_cast<const f16*>(w)[e]);
            else v = to_f32(reinterpret_cast<const bf16*>(w)[e]);
        }
        out[j] = v;
    }
}

// Dtype code of T (F32 = 0, F16 = 1, BF16 = 2), the codes of the weight dtype `dtw`.
template <typename T>
constexpr int dt_code() { return sizeof(T) == 4 ? 0 : __is_same(T, f16) ? 1 : 2; }

// A norm's per-thread weights, held for the whole kernel.  PACKED (16-bit weights of the
// row's own dtype in 16-byte slots) keeps the raw slots, half the registers of floats, and
// widens them where used; otherwise floats of any weight dtype.
template <typename T, int VEC, int NV, bool PACKED>
struct RowWeights {
    float v[NV][VEC];
    __device__ __forceinline__ void load(const void* __restrict__ w, int dt, int64_t n) {
#pragma unroll
        for (int i = 0; i < NV; ++i) load_w<VEC>(w, dt, n, i, v[i]);
    }
    __device__ __forceinline__ void get(int i, float* out) const {
#pragma unroll
        for (int j = 0; j < VEC; ++j) out[j] = v[i][j];
    }
};
template <typename T, int VEC, int NV>
struct RowWeights<T, VEC, NV, true> {
    static_assert(sizeof(T) == 2 && VEC != 1, "packed weights are 16-bit 16-byte slots");
    typename RowIO<T, VEC>::raw v[NV];
    __device__ __forceinline__ void load(const void* __restrict__ w, int, int64_t n) {
        const rsrc_t r = make_rsrc(w, (uint32_t)(n * 2));  // slots past the end read 0
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = bload16(r, RowIO<T, VEC>::off(i));
    }
    __device__ __forceinline__ void get(int i, float* out) const { RowIO<T, VEC>::to_float(v[i], out); }
};

// Rows handled together per loop iteration: short rows (NV < 4 vectors per thread) are
// processed R at a time, which halves (or quarters) the barriers per row and keeps more
// bytes in flight per thread.
template <int NV> struct RowsPerIter { static constexpr int R = NV >= 4 ? 1 : 4 / NV; };

// Block-wide sums / max of K values with one barrier: the LDS slot alternates between
// consecutive reductions (`par`), so a slot is rewritten only after every thread has
// passed the barrier of the reduction in between, i.e. after it finished reading the
// slot.  `red` holds 2 * kWaves * K floats.
template <int K, bool MAX>
__device__ __forceinline__ void block_reduce_n(float (&v)[K], float* red, int& par) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = MAX ? wave_max(v[k]) : wave_sum(v[k]);
    float* slot = red + par * kWaves * K;
    par ^= 1;
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < K; ++k) slot[k * kWaves + wid] = v[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; ++k) {
        float t = slot[k * kWaves];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) t = MAX ? fmaxf(t, slot[k * kWaves + i]) : t + slot[k * kWaves + i];
        v[k] = t;
    }
}

// Loads rows rb R + k (k < R) of a (rows x n) matrix as raw slots (zero past the end).
template <typename T, int VEC, int NV, int R>
__device__ __forceinline__ void load_rows(const T* base, int64_t rb, int64_t rows, int64_t n,
                                          typename RowIO<T, VEC>::raw (&out)[R][NV]) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const rsrc_t rs = row_rsrc(base, rb * R + k, rows, n);
#pragma unroll
        for (int i = 0; i < NV; ++i) out[k][i] = RowIO<T, VEC>::load(rs, i);
    }
}

// Calls step(slot, rb) for this workgroup's row blocks rb = blockIdx.x + j gridDim.x, in
// order, with slot = j % D a compile-time constant: D register slots of prefetched rows
// are then addressed statically (moving an in-flight load's registers would wait for it).
template <int S, int D, typename F>
__device__ __forceinline__ bool run_slots(int64_t& rb, int64_t nblk, F& step) {
    if constexpr (S == D) {
        return true;
    } else {
        if (rb >= nblk) return false;
        step(std::integral_constant<int, S>(), rb);
        rb += gridDim.x;
        return run_slots<S + 1, D>(rb, nblk, step);
    }
}
template <int D, typename F>
__device__ __forceinline__ void for_row_blocks(int64_t nblk, F&& step) {
    int64_t rb = blockIdx.x;
    while (run_slots<0, D>(rb, nblk, step)) {}
}

// ------------------------------------------------------------------ softmax
// y = exp(x - max) / sum(exp(x - max)) per row (online_softmax!, src/softmax.jl:19-58).
template <typename T, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void softmax_fwd_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                                int64_t n, int64_t rows) {
    typedef RowIO<T, VEC> IO;
    constexpr int R = RowsPerIter<NV>::R;
    __shared__ float red[2 * kWaves * R];
    int par = 0;
    const int64_t nblk = (rows + R - 1) / R;
    typename IO::raw cur[R][NV], nxt[R][NV];
    load_rows<T, VEC, NV, R>(x, blockIdx.x, rows, n, cur);
    for (int64_t rb = blockIdx.x; rb < nblk; rb += gridDim.x) {
        load_rows<T, VEC, NV, R>(x, rb + gridDim.x, rows, n, nxt);
        float v[R][NV][VEC], m[R], sm[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            m[k] = -INFINITY;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                IO::to_float(cur[k][i], v[k][i]);
                if (slot_valid<VEC>(n, i))
#pragma unroll
                    for (int j = 0; j < VEC; ++j) m[k] = fmaxf(m[k], v[k][i][j]);
            }
        }
        block_reduce_n<R, true>(m, red, par);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const float m2 = m[k] * kLog2e;
            sm[k] = 0.f;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const bool ok = slot_valid<VEC>(n, i);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    v[k][i][j] = fast_exp2(fmaf(v[k][i][j], kLog2e, -m2));
                    if (ok) sm[k] += v[k][i][j];
                }
            }
        }
        block_reduce_n<R, false>(sm, red, par);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const float inv = 1.0f / sm[k];
            const rsrc_t ry = row_rsrc(y, rb * R + k, rows, n);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) v[k][i][j] *= inv;
                IO::store(ry, i, v[k][i]);
            }
        }
#pragma unroll
        for (int k = 0; k < R; ++k)
#pragma unroll
            for (int i = 0; i < NV; ++i) cur[k][i] = nxt[k][i];
    }
}

// dx = y (dy - sum(y dy)) per row (∇online_softmax, src/softmax.jl:70-80).
template <typename T, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void softmax_bwd_kernel(const T* __restrict__ dy, const T* __restrict__ y,
                                                                T* __restrict__ dx, int64_t n, int64_t rows) {
    typedef RowIO<T, VEC> IO;
    constexpr int R = RowsPerIter<NV>::R;
    __shared__ float red[2 * kWaves * R];
    int par = 0;
    const int64_t nblk = (rows + R - 1) / R;
    typename IO::raw cg[R][NV], cy[R][NV], ng[R][NV], ny[R][NV];
    load_rows<T, VEC, NV, R>(dy, blockIdx.x, rows, n, cg);
    load_rows<T, VEC, NV, R>(y, blockIdx.x, rows, n, cy);
    for (int64_t rb = blockIdx.x; rb < nblk; rb += gridDim.x) {
        load_rows<T, VEC, NV, R>(dy, rb + gridDim.x, rows, n, ng);
        load_rows<T, VEC, NV, R>(y, rb + gridDim.x, rows, n, ny);
        float g[R][NV][VEC], yv[R][NV][VEC], sd[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            sd[k] = 0.f;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                IO::to_float(cg[k][i], g[k][i]);
                IO::to_float(cy[k][i], yv[k][i]);
#pragma unroll
                for (int j = 0; j < VEC; ++j) sd[k] = fmaf(g[k][i][j], yv[k][i][j], sd[k]);
            }
        }
        block_reduce_n<R, false>(sd, red, par);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const rsrc_t rx = row_rsrc(dx, rb * R + k, rows, n);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) g[k][i][j] = yv[k][i][j] * (g[k][i][j] - sd[k]);
                IO::store(rx, i, g[k][i]);
            }
        }
#pragma unroll
        for (int k = 0; k < R; ++k)
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                cg[k][i] = ng[k][i];
                cy[k][i] = ny[k][i];
            }
    }
}

// Pullback of the softmax backward (second order; src/softmax.jl:70-80, the
// within_gradient branch at :71-74): for dx = y (dy - s), s = sum(dy y), and upstream
// G = dL/d(dx), with u = sum(G y):  d_dy = y (G - u),  d_y = G (dy - s) - dy u.
template <typename T, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void softmax_bwd2_kernel(const T* __restrict__ g, const T* __restrict__ dy,
                                                                 const T* __restrict__ y, T* __restrict__ d_dy,
                                                                 T* __restrict__ d_y, int64_t n, int64_t rows) {
    typedef RowIO<T, VEC> IO;
    constexpr int R = RowsPerIter<NV>::R;
    __shared__ float red[2 * kWaves * 2 * R];
    int par = 0;
    const int64_t nblk = (rows + R - 1) / R;
    typename IO::raw cg[R][NV], cd[R][NV], cy[R][NV], ng[R][NV], nd[R][NV], ny[R][NV];
    load_rows<T, VEC, NV, R>(g, blockIdx.x, rows, n, cg);
    load_rows<T, VEC, NV, R>(dy, blockIdx.x, rows, n, cd);
    load_rows<T, VEC, NV, R>(y, blockIdx.x, rows, n, cy);
    for (int64_t rb = blockIdx.x; rb < nblk; rb += gridDim.x) {
        load_rows<T, VEC, NV, R>(g, rb + gridDim.x, rows, n, ng);
        load_rows<T, VEC, NV, R>(dy, rb + gridDim.x, rows, n, nd);
        load_rows<T, VEC, NV, R>(y, rb + gridDim.x, rows, n, ny);
        float gv[R][NV][VEC], dv[R][NV][VEC], yv[R][NV][VEC], su[2 * R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            su[2 * k] = su[2 * k + 1] = 0.f;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                IO::to_float(cg[k][i], gv[k][i]);
                IO::to_float(cd[k][i], dv[k][i]);
                IO::to_float(cy[k][i], yv[k][i]);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {  // elements past n read 0 and add nothing
                    su[2 * k] = fmaf(dv[k][i][j], yv[k][i][j], su[2 * k]);
                    su[2 * k + 1] = fmaf(gv[k][i][j], yv[k][i][j], su[2 * k + 1]);
                }
            }
        }
        block_reduce_n<2 * R, false>(su, red, par);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const float sk = su[2 * k], uk = su[2 * k + 1];
            const rsrc_t ra = row_rsrc(d_dy, rb * R + k, rows, n);
            const rsrc_t rc = row_rsrc(d_y, rb * R + k, rows, n);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                float a[VEC], c[VEC];
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    a[j] = yv[k][i][j] * (gv[k][i][j] - uk);
                    c[j] = gv[k][i][j] * (dv[k][i][j] - sk) - dv[k][i][j] * uk;
                }
                IO::store(ra, i, a);
                IO::store(rc, i, c);
            }
        }
#pragma unroll
        for (int k = 0; k < R; ++k)
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                cg[k][i] = ng[k][i];
                cd[k][i] = nd[k][i];
                cy[k][i] = ny[k][i];
            }
    }
}

// Marks raw row slots as rewritten (an empty asm), so that a second pass over them widens
// them again instead of keeping the first pass's floats live across a reduction: the
// floats of a 16-bit row take twice the registers of its raw slots.
template <int R, int NV, typename Raw>
__device__ __forceinline__ void reload_barrier(Raw (&a)[R][NV], Raw (&b)[R][NV]) {
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
        for (int i = 0; i < NV; ++i) asm volatile("" : "+v"(a[k][i]), "+v"(b[k][i]));
}

// ------------------------------------------------------------------ RMS norm
// rstd = 1/sqrt(mean(x^2) + eps); y = (offset + w) x rstd (_rms_norm!, src/rms_norm.jl:3-38).
template <typename T, int VEC, int NV, int D, bool PW>
__global__ __launch_bounds__(kThreads) void rms_fwd_kernel(const T* __restrict__ x, const void* __restrict__ w, int dtw,
                                                            T* __restrict__ y, float* __restrict__ rstd,
                                                            int64_t n, int64_t rows, float eps, float offset) {
    typedef RowIO<T, VEC> IO;
    constexpr int R = RowsPerIter<NV>::R;
    __shared__ float red[2 * kWaves * R];
    int par = 0;
    RowWeights<T, VEC, NV, PW> wv;
    wv.load(w, dtw, n);
    const float inv_n = 1.0f / (float)n;
    const int64_t nblk = (rows + R - 1) / R;
    typename IO::raw buf[D][R][NV];
#pragma unroll
    for (int d = 0; d < D; ++d) load_rows<T, VEC, NV, R>(x, blockIdx.x + (int64_t)d * gridDim.x, rows, n, buf[d]);
    for_row_blocks<D>(nblk, [&](auto slot, int64_t rb) {
        constexpr int sl = decltype(slot)::value;
        float v[R][NV][VEC], ss[R];
#pragma unroll
        for (int k = 0; k < R; ++k)
#pragma unroll
            for (int i = 0; i < NV; ++i) IO::to_float(buf[sl][k][i], v[k][i]);
        load_rows<T, VEC, NV, R>(x, rb + (int64_t)D * gridDim.x, rows, n, buf[sl]);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            ss[k] = 0.f;
#pragma unroll
            for (int i = 0; i < NV; ++i)
#pragma unroll
                for (int j = 0; j < VEC; ++j) ss[k] = fmaf(v[k][i][j], v[k][i][j], ss[k]);
        }
        block_reduce_n<R, false>(ss, red, par);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const int64_t r = rb * R + k;
            const float rs = 1.0f / sqrtf(ss[k] * inv_n + eps);
            if (threadIdx.x == 0 && r < rows) rstd[r] = rs;
            const rsrc_t ry = row_rsrc(y, r, rows, n);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                float wf[VEC];
                wv.get(i, wf);
#pragma unroll
                for (int j = 0; j < VEC; ++j) v[k][i][j] = (wf[j] + offset) * v[k][i][j] * rs;
                IO::store(ry, i, v[k][i]);
            }
        }
    });
}

// Float32 per-row statistic of rows rb R + k (0 past the end).
template <int R>
__device__ __forceinline__ void load_stats(const float* p, int64_t rb, int64_t rows, float (&out)[R]) {
    const rsrc_t r = make_rsrc(p, (uint32_t)(rows * 4));
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int64_t row = rb * R + k;
        out[k] = bload_f32(r, row < rows ? (uint32_t)row * 4u : 0xFFFFFFF0u);
    }
}

// Per row: dd = sum(dy (w+off) x); dx = rstd dy (w+off) - rstd^3 dd x / n; the dw partial
// sum(dy x rstd) over this workgroup's rows goes to ws[blockIdx.x, :]
// (_∇rms_norm!, src/rms_norm.jl:43-115).
template <typename T, int VEC, int NV, int D, bool PW>
__global__ __launch_bounds__(kThreads) void rms_bwd_kernel(const T* __restrict__ dy, const float* __restrict__ rstd,
                                                            const T* __restrict__ x, const void* __restrict__ w, int dtw,
                                                            float offset, T* __restrict__ dx, float* __restrict__ ws,
                                                            int64_t n, int64_t rows) {
    typedef RowIO<T, VEC> IO;
    constexpr int R = RowsPerIter<NV>::R;
    __shared__ float red[2 * kWaves * R];
    int par = 0;
    RowWeights<T, VEC, NV, PW> wv;
    wv.load(w, dtw, n);
    float dw[NV][VEC];
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) dw[i][j] = 0.f;
    const float inv_n = 1.0f / (float)n;
    const int64_t nblk = (rows + R - 1) / R;
    typename IO::raw bg[D][R][NV], bx[D][R][NV];
    float brs[D][R];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const int64_t b0 = blockIdx.x + (int64_t)d * gridDim.x;
        load_rows<T, VEC, NV, R>(dy, b0, rows, n, bg[d]);
        load_rows<T, VEC, NV, R>(x, b0, rows, n, bx[d]);
        load_stats<R>(rstd, b0, rows, brs[d]);
    }
    for_row_blocks<D>(nblk, [&](auto slot, int64_t rb) {
        constexpr int sl = decltype(slot)::value;
        // The current rows stay in their raw slots and are widened in each of the two
        // passes (half the registers of floats for 16-bit rows).
        typename IO::raw cg[R][NV], cx[R][NV];
        float dd[R], crs[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            crs[k] = brs[sl][k];
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                cg[k][i] = bg[sl][k][i];
                cx[k][i] = bx[sl][k][i];
            }
        }
        const int64_t nb = rb + (int64_t)D * gridDim.x;
        load_rows<T, VEC, NV, R>(dy, nb, rows, n, bg[sl]);
        load_rows<T, VEC, NV, R>(x, nb, rows, n, bx[sl]);
        load_stats<R>(rstd, nb, rows, brs[sl]);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            dd[k] = 0.f;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                float g[VEC], xv[VEC], wf[VEC];
                IO::to_float(cg[k][i], g);
                IO::to_float(cx[k][i], xv);
                wv.get(i, wf);
#pragma unroll
                for (int j = 0; j < VEC; ++j) dd[k] = fmaf(g[j] * (wf[j] + offset), xv[j], dd[k]);
            }
        }
        block_reduce_n<R, false>(dd, red, par);
        reload_barrier<R, NV>(cg, cx);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const float rs = crs[k];  // 0 for rows past the end, whose g and x are 0 too
            const float c3 = rs * rs * rs * dd[k] * inv_n;
            const rsrc_t rx = row_rsrc(dx, rb * R + k, rows, n);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                float g[VEC], xv[VEC], wf[VEC];
                IO::to_float(cg[k][i], g);
                IO::to_float(cx[k][i], xv);
                wv.get(i, wf);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    dw[i][j] = fmaf(g[j], xv[j] * rs, dw[i][j]);
                    g[j] = rs * g[j] * (wf[j] + offset) - c3 * xv[j];
                }
                IO::store(rx, i, g);
            }
        }
    });
    const rsrc_t rw = make_rsrc(ws + (int64_t)blockIdx.x * n, (uint32_t)(n * 4));
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dw[i][j]), rw,
                                                  (int)(((uint32_t)VEC * (threadIdx.x + i * kThreads) + j) * 4u), 0, 0);
}

// ------------------------------------------------------------------ layer norm
// mu = mean(x); rstd = 1/sqrt(mean((x-mu)^2) + eps); y = (x-mu) rstd w + b
// (_layer_norm!, src/layer_norm.jl:8-63).
template <typename T, int VEC, int NV, int D, bool PW>
__global__ __launch_bounds__(kThreads) void ln_fwd_kernel(const T* __restrict__ x, const void* __restrict__ w,
                                                           const void* __restrict__ b, int dtw, T* __restrict__ y,
                                                           float* __restrict__ mu, float* __restrict__ rstd,
                                                           int64_t n, int64_t rows, float eps) {
    typedef RowIO<T, VEC> IO;
    constexpr int R = RowsPerIter<NV>::R;
    __shared__ float red[2 * kWaves * R];
    int par = 0;
    RowWeights<T, VEC, NV, PW> wv, bv;
    wv.load(w, dtw, n);
    bv.load(b, dtw, n);
    const float inv_n = 1.0f / (float)n;
    const int64_t nblk = (rows + R - 1) / R;
    typename IO::raw buf[D][R][NV];
#pragma unroll
    for (int d = 0; d < D; ++d) load_rows<T, VEC, NV, R>(x, blockIdx.x + (int64_t)d * gridDim.x, rows, n, buf[d]);
    for_row_blocks<D>(nblk, [&](auto slot, int64_t rb) {
        constexpr int sl = decltype(slot)::value;
        float v[R][NV][VEC], m[R], q[R];
#pragma unroll
        for (int k = 0; k < R; ++k)
#pragma unroll
            for (int i = 0; i < NV; ++i) IO::to_float(buf[sl][k][i], v[k][i]);
        load_rows<T, VEC, NV, R>(x, rb + (int64_t)D * gridDim.x, rows, n, buf[sl]);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            m[k] = 0.f;
#pragma unroll
            for (int i = 0; i < NV; ++i)
#pragma unroll
                for (int j = 0; j < VEC; ++j) m[k] += v[k][i][j];
        }
        block_reduce_n<R, false>(m, red, par);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            m[k] *= inv_n;
            q[k] = 0.f;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const bool ok = slot_valid<VEC>(n, i);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    const int64_t e = (int64_t)VEC * (threadIdx.x + (int64_t)i * kThreads) + j;
                    const float c = v[k][i][j] - m[k];
                    if (ok && e < n) q[k] = fmaf(c, c, q[k]);
                }
            }
        }
        block_reduce_n<R, false>(q, red, par);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const int64_t r = rb * R + k;
            const float rs = 1.0f / sqrtf(q[k] * inv_n + eps);
            if (threadIdx.x == 0 && r < rows) { mu[r] = m[k]; rstd[r] = rs; }
            const rsrc_t ry = row_rsrc(y, r, rows, n);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                float wf[VEC], bf[VEC];
                wv.get(i, wf);
                bv.get(i, bf);
#pragma unroll
                for (int j = 0; j < VEC; ++j) v[k][i][j] = fmaf((v[k][i][j] - m[k]) * rs, wf[j], bf[j]);
                IO::store(ry, i, v[k][i]);
            }
        }
    });
}

// Per row: xn = (x-mu) rstd; c1 = mean(w dy xn); c2 = mean(w dy);
// dx = (w dy - (xn c1 + c2)) rstd; partials of dw = sum dy xn and db = sum dy go to
// ws[blockIdx.x, :] and ws[grid + blockIdx.x, :] (_∇layer_norm!, src/layer_norm.jl:65-148).
template <typename T, int VEC, int NV, int D, bool PW>
__global__ __launch_bounds__(kThreads) void ln_bwd_kernel(const T* __restrict__ dy, const float* __restrict__ mu,
                                                           const float* __restrict__ rstd, const T* __restrict__ x,
                                                           const void* __restrict__ w, int dtw, T* __restrict__ dx,
                                                           float* __restrict__ ws, int64_t n, int64_t rows) {
    typedef RowIO<T, VEC> IO;
    constexpr int R = RowsPerIter<NV>::R;
    __shared__ float red[2 * kWaves * 2 * R];
    int par = 0;
    RowWeights<T, VEC, NV, PW> wv;
    wv.load(w, dtw, n);
    float dw[NV][VEC], db[NV][VEC];
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) dw[i][j] = db[i][j] = 0.f;
    const float inv_n = 1.0f / (float)n;
    const int64_t nblk = (rows + R - 1) / R;
    typename IO::raw bg[D][R][NV], bx[D][R][NV];
    float bm[D][R], brs[D][R];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const int64_t b0 = blockIdx.x + (int64_t)d * gridDim.x;
        load_rows<T, VEC, NV, R>(dy, b0, rows, n, bg[d]);
        load_rows<T, VEC, NV, R>(x, b0, rows, n, bx[d]);
        load_stats<R>(mu, b0, rows, bm[d]);
        load_stats<R>(rstd, b0, rows, brs[d]);
    }
    for_row_blocks<D>(nblk, [&](auto slot, int64_t rb) {
        constexpr int sl = decltype(slot)::value;
        // The current rows stay in their raw slots (half the registers of floats for
        // 16-bit rows) and are widened, xn = (x-mu) rstd too, in each of the two passes.
        typename IO::raw cg[R][NV], cx[R][NV];
        float c12[2 * R], cm[R], crs[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            cm[k] = bm[sl][k];
            crs[k] = brs[sl][k];
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                cg[k][i] = bg[sl][k][i];
                cx[k][i] = bx[sl][k][i];
            }
        }
        const int64_t nb = rb + (int64_t)D * gridDim.x;
        load_rows<T, VEC, NV, R>(dy, nb, rows, n, bg[sl]);
        load_rows<T, VEC, NV, R>(x, nb, rows, n, bx[sl]);
        load_stats<R>(mu, nb, rows, bm[sl]);
        load_stats<R>(rstd, nb, rows, brs[sl]);
        auto widen = [&](int k, int i, float* g, float* xn) {
            IO::to_float(cg[k][i], g);
            IO::to_float(cx[k][i], xn);
#pragma unroll
            for (int j = 0; j < VEC; ++j) xn[j] = (xn[j] - cm[k]) * crs[k];
        };
#pragma unroll
        for (int k = 0; k < R; ++k) {
            c12[2 * k] = c12[2 * k + 1] = 0.f;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                float g[VEC], xn[VEC], wf[VEC];
                widen(k, i, g, xn);
                wv.get(i, wf);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {  // zero-padded slots give g = 0
                    const float wdy = wf[j] * g[j];
                    c12[2 * k] = fmaf(wdy, xn[j], c12[2 * k]);
                    c12[2 * k + 1] += wdy;
                }
            }
        }
        block_reduce_n<2 * R, false>(c12, red, par);
        reload_barrier<R, NV>(cg, cx);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const float c1 = c12[2 * k] * inv_n, c2 = c12[2 * k + 1] * inv_n, rs = crs[k];
            const rsrc_t rx = row_rsrc(dx, rb * R + k, rows, n);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                float o[VEC], g[VEC], xn[VEC], wf[VEC];
                widen(k, i, g, xn);
                wv.get(i, wf);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    o[j] = (wf[j] * g[j] - fmaf(xn[j], c1, c2)) * rs;
                    dw[i][j] = fmaf(g[j], xn[j], dw[i][j]);
                    db[i][j] += g[j];
                }
                IO::store(rx, i, o);
            }
        }
    });
    const rsrc_t rw = make_rsrc(ws + (int64_t)blockIdx.x * n, (uint32_t)(n * 4));
    const rsrc_t rb = make_rsrc(ws + ((int64_t)gridDim.x + blockIdx.x) * n, (uint32_t)(n * 4));
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const int off = (int)(((uint32_t)VEC * (threadIdx.x + i * kThreads) + j) * 4u);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dw[i][j]), rw, off, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(db[i][j]), rb, off, 0, 0);
        }
}

// ------------------------------------------------------------------ column sums
// The weight gradients are column sums of `groups` (at most 1024) float32 partial rows,
// one matrix per gradient, `count` of them.  One launch: block (x, y) owns 64 columns of
// matrix y; thread (column c, row group rg < 16) sums partial rows rg, rg + 16, ... in
// order, sixteen loads in flight per batch, and the 16 row-group sums of a column then
// combine in LDS by a fixed pairwise tree.  Blocking and order are fixed, so the bits do
// not depend on the device.
constexpr int kColRG = 16;

__global__ __launch_bounds__(1024) void colsum_kernel(const float* __restrict__ ws, int64_t groups, int64_t n,
                                                      void* __restrict__ out0, void* __restrict__ out1, int dt) {
    __shared__ float part[kColRG][64];
    const int c = threadIdx.x & 63, rg = threadIdx.x >> 6;
    const int64_t e = (int64_t)blockIdx.x * 64 + c;
    const rsrc_t r = make_rsrc(ws + (int64_t)blockIdx.y * groups * n, (uint32_t)(groups * n * 4));
    float s = 0.f;
    for (int64_t g0 = rg; g0 < groups; g0 += kColRG * 16) {
        float v[16];  // partial rows g0 + 16 j; rows past `groups` or columns past n read 0
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int64_t row = g0 + 16 * j;
            const bool ok = row < groups && e < n;
            v[j] = bload_f32(r, ok ? (uint32_t)(row * n + e) * 4u : 0xFFFFFFF0u);
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) s += v[j];
    }
    part[rg][c] = s;
    __syncthreads();
#pragma unroll
    for (int w = 1; w < kColRG; w *= 2) {
        if (rg % (2 * w) == 0) part[rg][c] += part[rg + w][c];
        __syncthreads();
    }
    if (rg != 0 || e >= n) return;
    s = part[0][c];
    void* out = blockIdx.y == 0 ? out0 : out1;
    if (dt == 0) reinterpret_cast<float*>(out)[e] = s;
    else if (dt == 1) reinterpret_cast<f16*>(out)[e] = from_f32<f16>(s);
    else reinterpret_cast<bf16*>(out)[e] = from_f32<bf16>(s);
}

#include "rowwise_long.inc"

// ------------------------------------------------------------------ dispatch

// Row blocks in flight ahead of the one being computed by the norm backward: two while
// a register slot (dy and x of R rows) is at most 4 vectors per tensor per thread.  The
// forward kernels keep one: a second measured slower there.
template <int NV> struct BwdDepth { static constexpr int D = RowsPerIter<NV>::R * NV <= 4 ? 2 : 1; };

static int num_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
            cus = prop.multiProcessorCount;
        else
            cus = 256;
    }
    return cus;
}

// Picks (VEC, NV) for a row of n elements of T: 16-byte vectors when rows stay 16-byte
// aligned, else scalars; NV = smallest power of two <= 16 covering the row.
template <typename T, template <typename, int, int> class K, typename... Args>
static bool dispatch_row(int64_t n, Args&&... args) {
    constexpr int V = Vec<T>::N;
    const bool vec_ok = (n % V) == 0;
    const int64_t per = vec_ok ? (int64_t)V * kThreads : kThreads;
    const int64_t nv = (n + per - 1) / per;
    if (vec_ok) {
        if (nv <= 1) return K<T, V, 1>::run(args...);
        if (nv <= 2) return K<T, V, 2>::run(args...);
        if (nv <= 4) return K<T, V, 4>::run(args...);
        if (nv <= 8) return K<T, V, 8>::run(args...);
        if (nv <= 16) return K<T, V, 16>::run(args...);
    } else {
        if (nv <= 1) return K<T, 1, 1>::run(args...);
        if (nv <= 2) return K<T, 1, 2>::run(args...);
        if (nv <= 4) return K<T, 1, 4>::run(args...);
        if (nv <= 8) return K<T, 1, 8>::run(args...);
        if (nv <= 16) return K<T, 1, 16>::run(args...);
    }
    return false;  // row longer than 16 vectors per thread: not supported
}

// Workgroups of kThreads threads of kernel `k` that fit on one CU at once.
template <typename Kern>
static int fit_per_cu(Kern k) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k, kThreads, 0) != hipSuccess || nb < 1) nb = 1;
    return nb;
}

// Persistent grid over `blocks` row blocks whose iteration loads `iter_bytes` bytes.
// Few long-lived workgroups stream best on MI355X: about 32 KiB of loads in flight per
// CU (2 to 8 workgroups per CU, no more than fit at once, so none waits for a slot), and
// the row blocks split evenly, so every workgroup runs the same number of iterations.
static int64_t grid_rows(int64_t blocks, int64_t iter_bytes, int fit) {
    int64_t wpc = (32 * 1024) / (iter_bytes > 0 ? iter_bytes : 1);
    wpc = wpc < 2 ? 2 : wpc > 8 ? 8 : wpc;
    if (wpc > fit) wpc = fit;
    const int64_t g = wpc * num_cus();
    if (blocks <= g) return blocks;
    const int64_t it = (blocks + g - 1) / g;
    return (blocks + it - 1) / it;
}

// Grid over row blocks of R rows of n elements of T, `ins` input rows each, for a
// kernel of which `fit` workgroups fit on a CU.
template <typename T, int NV>
static unsigned grid_blocks(int fit, int64_t rows, int64_t n, int ins) {
    constexpr int R = RowsPerIter<NV>::R;
    return (unsigned)grid_rows((rows + R - 1) / R, (int64_t)ins * R * n * (int64_t)sizeof(T), fit);
}

template <typename T, int VEC, int NV>
struct SoftmaxFwd {
    static bool run(hipStream_t s, const void* x, void* y, int64_t n, int64_t rows) {
        const auto k = softmax_fwd_kernel<T, VEC, NV>;
        static const int fit = fit_per_cu(k);
        k<<<dim3(grid_blocks<T, NV>(fit, rows, n, 1)), dim3(kThreads), 0, s>>>(
            (const T*)x, (T*)y, n, rows);
        return true;
    }
};
template <typename T, int VEC, int NV>
struct SoftmaxBwd {
    static bool run(hipStream_t s, const void* dy, const void* y, void* dx, int64_t n, int64_t rows) {
        const auto k = softmax_bwd_kernel<T, VEC, NV>;
        static const int fit = fit_per_cu(k);
        k<<<dim3(grid_blocks<T, NV>(fit, rows, n, 2)), dim3(kThreads), 0, s>>>(
            (const T*)dy, (const T*)y, (T*)dx, n, rows);
        return true;
    }
};
template <typename T, int VEC, int NV>
struct SoftmaxBwd2 {
    static bool run(hipStream_t s, const void* g, const void* dy, const void* y, void* d_dy, void* d_y, int64_t n,
                    int64_t rows) {
        const auto k = softmax_bwd2_kernel<T, VEC, NV>;
        static const int fit = fit_per_cu(k);
        k<<<dim3(grid_blocks<T, NV>(fit, rows, n, 3)), dim3(kThreads), 0, s>>>(
            (const T*)g, (const T*)dy, (const T*)y, (T*)d_dy, (T*)d_y, n, rows);
        return true;
    }
};
// Calls f(std::true_type) when a norm's weights (w, and b if not NULL) can be held packed:
// 16-bit weights of the row's own dtype, read as 16-byte slots, so 16-byte aligned.
// Else f(std::false_type).
template <typename T, int VEC, typename F>
static void with_weights(int dtw, const void* w, const void* b, F&& f) {
    if constexpr (sizeof(T) == 2 && VEC != 1) {
        if (dtw == dt_code<T>() && ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(b)) & 15u) == 0) {
            f(std::true_type());
            return;
        }
    }
    f(std::false_type());
}

template <typename T, int VEC, int NV>
struct RmsFwd {
    static bool run(hipStream_t s, const void* x, const void* w, int dtw, void* y, float* rstd, int64_t n,
                    int64_t rows, float eps, float offset) {
        with_weights<T, VEC>(dtw, w, nullptr, [&](auto pw) {
            const auto k = rms_fwd_kernel<T, VEC, NV, 1, decltype(pw)::value>;
            static const int fit = fit_per_cu(k);
            k<<<dim3(grid_blocks<T, NV>(fit, rows, n, 1)), dim3(kThreads), 0, s>>>(
                (const T*)x, w, dtw, (T*)y, rstd, n, rows, eps, offset);
        });
        return true;
    }
};
template <typename T, int VEC, int NV>
struct RmsBwd {
    static bool run(hipStream_t s, const void* dy, const float* rstd, const void* x, const void* w, int dtw,
                    float offset, void* dx, float* ws, int64_t groups, int64_t n, int64_t rows) {
        with_weights<T, VEC>(dtw, w, nullptr, [&](auto pw) {
            rms_bwd_kernel<T, VEC, NV, BwdDepth<NV>::D, decltype(pw)::value>
                <<<dim3((unsigned)groups), dim3(kThreads), 0, s>>>((const T*)dy, rstd, (const T*)x, w, dtw, offset,
                                                                   (T*)dx, ws, n, rows);
        });
        return true;
    }
};
template <typename T, int VEC, int NV>
struct LnFwd {
    static bool run(hipStream_t s, const void* x, const void* w, const void* b, int dtw, void* y, float* mu,
                    float* rstd, int64_t n, int64_t rows, float eps) {
        with_weights<T, VEC>(dtw, w, b, [&](auto pw) {
            const auto k = ln_fwd_kernel<T, VEC, NV, 1, decltype(pw)::value>;
            static const int fit = fit_per_cu(k);
            k<<<dim3(grid_blocks<T, NV>(fit, rows, n, 1)), dim3(kThreads), 0, s>>>(
                (const T*)x, w, b, dtw, (T*)y, mu, rstd, n, rows, eps);
        });
        return true;
    }
};
template <typename T, int VEC, int NV>
struct LnBwd {
    static bool run(hipStream_t s, const void* dy, const float* mu, const float* rstd, const void* x,
                    const void* w, int dtw, void* dx, float* ws, int64_t groups, int64_t n, int64_t rows) {
        with_weights<T, VEC>(dtw, w, nullptr, [&](auto pw) {
            ln_bwd_kernel<T, VEC, NV, BwdDepth<NV>::D, decltype(pw)::value>
                <<<dim3((unsigned)groups), dim3(kThreads), 0, s>>>((const T*)dy, mu, rstd, (const T*)x, w, dtw,
                                                                   (T*)dx, ws, n, rows);
        });
        return true;
    }
};

// Rows the register-resident kernels cannot hold: the streaming kernels of
// rowwise_long.inc, 16-byte vectors when rows stay 16-byte aligned, else scalars.
template <typename T, template <typename, int> class K, typename... Args>
static bool dispatch_long(int64_t n, Args&&... args) {
    if (n % Vec<T>::N == 0) return K<T, Vec<T>::N>::run(args...);
    return K<T, 1>::run(args...);
}

// Persistent grid of a streaming kernel: up to 8 workgroups per CU (no more than fit).
template <typename Kern>
static unsigned grid_long(Kern k, int64_t rows) {
    int fit = fit_per_cu(k);
    fit = fit > 8 ? 8 : fit;
    const int64_t g = (int64_t)fit * num_cus();
    return (unsigned)(rows < g ? rows : g);
}

template <typename T, int VEC>
struct SoftmaxFwdLong {
    static bool run(hipStream_t s, const void* x, void* y, int64_t n, int64_t rows) {
        const auto k = softmax_fwd_long_kernel<T, VEC>;
        k<<<dim3(grid_long(k, rows)), dim3(kThreads), 0, s>>>((const T*)x, (T*)y, n, rows);
        return true;
    }
};
template <typename T, int VEC>
struct SoftmaxBwdLong {
    static bool run(hipStream_t s, const void* dy, const void* y, void* dx, int64_t n, int64_t rows) {
        const auto k = softmax_bwd_long_kernel<T, VEC>;
        k<<<dim3(grid_long(k, rows)), dim3(kThreads), 0, s>>>((const T*)dy, (const T*)y, (T*)dx, n, rows);
        return true;
    }
};
template <typename T, int VEC>
struct SoftmaxBwd2Long {
    static bool run(hipStream_t s, const void* g, const void* dy, const void* y, void* d_dy, void* d_y, int64_t n,
                    int64_t rows) {
        const auto k = softmax_bwd2_long_kernel<T, VEC>;
        k<<<dim3(grid_long(k, rows)), dim3(kThreads), 0, s>>>((const T*)g, (const T*)dy, (const T*)y, (T*)d_dy,
                                                              (T*)d_y, n, rows);
        return true;
    }
};
template <typename T, int VEC>
struct RmsFwdLong {
    static bool run(hipStream_t s, const void* x, const void* w, int dtw, void* y, float* rstd, int64_t n,
                    int64_t rows, float eps, float offset) {
        const auto k = rms_fwd_long_kernel<T, VEC>;
        k<<<dim3(grid_long(k, rows)), dim3(kThreads), 0, s>>>((const T*)x, w, dtw, (T*)y, rstd, n, rows, eps,
                                                              offset);
        return true;
    }
};
template <typename T, int VEC>
struct RmsBwdLong {
    static bool run(hipStream_t s, const void* dy, const float* rstd, const void* x, const void* w, int dtw,
                    float offset, void* dx, float* ws, int64_t groups, int64_t n, int64_t rows) {
        rms_bwd_long_kernel<T, VEC><<<dim3((unsigned)groups), dim3(kThreads), 0, s>>>(
            (const T*)dy, rstd, (const T*)x, w, dtw, offset, (T*)dx, ws, n, rows);
        return true;
    }
};
template <typename T, int VEC>
struct LnFwdLong {
    static bool run(hipStream_t s, const void* x, const void* w, const void* b, int dtw, void* y, float* mu,
                    float* rstd, int64_t n, int64_t rows, float eps) {
        const auto k = ln_fwd_long_kernel<T, VEC>;
        k<<<dim3(grid_long(k, rows)), dim3(kThreads), 0, s>>>((const T*)x, w, b, dtw, (T*)y, mu, rstd, n, rows,
                                                              eps);
        return true;
    }
};
template <typename T, int VEC>
struct LnBwdLong {
    static bool run(hipStream_t s, const void* dy, const float* mu, const float* rstd, const void* x,
                    const void* w, int dtw, void* dx, float* ws, int64_t groups, int64_t n, int64_t rows) {
        ln_bwd_long_kernel<T, VEC><<<dim3((unsigned)groups), dim3(kThreads), 0, s>>>(
            (const T*)dy, mu, rstd, (const T*)x, w, dtw, (T*)dx, ws, n, rows);
        return true;
    }
};

#define ONIONOP_DT_SWITCH(dt, T, ...)                    \
    switch (dt) {                                        \
        case 0: { typedef float T; __VA_ARGS__; } break; \
        case 1: { typedef f16 T; __VA_ARGS__; } break;   \
        case 2: { typedef bf16 T; __VA_ARGS__; } break;  \
        default: return false;                           \
    }

// Longest row: the kernels address a row (and a partial row of the norm backward) with
// 32-bit byte offsets.
int64_t max_row_elems(int dt) {
    (void)dt;
    return (1LL << 29) - 1;
}

// Partial-row groups (= workgroups) of the norm backward for rows of n elements.  A
// function of the shape only, so the workspace size and the summation order, hence the
// bits of dw/db, do not depend on the GPU model.  Rows of 4096 or more elements take 256
// groups (one long-lived workgroup per CU of an MI355X, which streams best), shorter rows
// 512 or 1024, keeping the loads in flight per CU about the same.
int64_t norm_bwd_groups(int64_t rows, int64_t n) {
    int64_t per = n > 0 ? 4096 / n : 4;
    per = per < 1 ? 1 : per > 4 ? 4 : per;
    const int64_t g = 256 * per;
    return rows < g ? rows : g;
}

int64_t norm_bwd_ws_floats(int64_t rows, int64_t n) { return norm_bwd_groups(rows, n) * n; }

// Column sums of `count` partial matrices at ws ([count][groups][n]) into out0 / out1.
static void colsum(hipStream_t s, float* ws, int64_t groups, int64_t n, int count, void* out0, void* out1,
                   int dt) {
    colsum_kernel<<<dim3((unsigned)((n + 63) / 64), (unsigned)count), dim3(1024), 0, s>>>(ws, groups, n, out0, out1,
                                                                                         dt);
}

bool launch_softmax_fwd(hipStream_t s, int dt, int64_t n, int64_t rows, const void* x, void* y) {
    if (rows == 0 || n == 0) return true;
    ONIONOP_DT_SWITCH(dt, T, return dispatch_row<T, SoftmaxFwd>(n, s, x, y, n, rows) ||
                                    dispatch_long<T, SoftmaxFwdLong>(n, s, x, y, n, rows));
    return true;
}
bool launch_softmax_bwd(hipStream_t s, int dt, int64_t n, int64_t rows, const void* dy, const void* y, void* dx) {
    if (rows == 0 || n == 0) return true;
    ONIONOP_DT_SWITCH(dt, T, return dispatch_row<T, SoftmaxBwd>(n, s, dy, y, dx, n, rows) ||
                                    dispatch_long<T, SoftmaxBwdLong>(n, s, dy, y, dx, n, rows));
    return true;
}
bool launch_softmax_bwd_bwd(hipStream_t s, int dt, int64_t n, int64_t rows, const void* g, const void* dy,
                            const void* y, void* d_dy, void* d_y) {
    if (rows == 0 || n == 0) return true;
    ONIONOP_DT_SWITCH(dt, T, return dispatch_row<T, SoftmaxBwd2>(n, s, g, dy, y, d_dy, d_y, n, rows) ||
                                    dispatch_long<T, SoftmaxBwd2Long>(n, s, g, dy, y, d_dy, d_y, n, rows));
    return true;
}
bool launch_rms_fwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* x, const void* w,
                    float eps, float offset, void* y, float* rstd) {
    if (rows == 0) return true;
    ONIONOP_DT_SWITCH(dt, T, return dispatch_row<T, RmsFwd>(n, s, x, w, dtw, y, rstd, n, rows, eps, offset) ||
                                    dispatch_long<T, RmsFwdLong>(n, s, x, w, dtw, y, rstd, n, rows, eps, offset));
    return true;
}
bool launch_rms_bwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* dy, const float* rstd,
                    const void* x, const void* w, float offset, void* dx, float* dw, float* ws) {
    const int64_t groups = norm_bwd_groups(rows, n);
    if (rows > 0) {
        bool ok = false;
        ONIONOP_DT_SWITCH(dt, T,
                          ok = dispatch_row<T, RmsBwd>(n, s, dy, rstd, x, w, dtw, offset, dx, ws, groups, n, rows) ||
                               dispatch_long<T, RmsBwdLong>(n, s, dy, rstd, x, w, dtw, offset, dx, ws, groups, n,
                                                            rows));
        if (!ok) return false;
    }
    if (n == 0) return true;
    if (rows == 0) {  // no rows: dw = 0
        fill_zero_kernel<<<dim3((unsigned)((n * 4 + 1023) / 1024)), dim3(256), 0, s>>>(dw, n * 4);
        return true;
    }
    colsum(s, ws, groups, n, 1, dw, nullptr, 0);
    return true;
}
bool launch_ln_fwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* x, const void* w,
                   const void* b, float eps, void* y, float* mu, float* rstd) {
    if (rows == 0) return true;
    ONIONOP_DT_SWITCH(dt, T, return dispatch_row<T, LnFwd>(n, s, x, w, b, dtw, y, mu, rstd, n, rows, eps) ||
                                    dispatch_long<T, LnFwdLong>(n, s, x, w, b, dtw, y, mu, rstd, n, rows, eps));
    return true;
}
bool launch_ln_bwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* dy, const float* mu,
                   const float* rstd, const void* x, const void* w, void* dx, void* dw, void* db, float* ws) {
    const int64_t groups = norm_bwd_groups(rows, n);
    if (n == 0) return true;
    if (rows == 0) {
        const int64_t bytes = (dtw == 0 ? 4 : 2) * n;
        fill_zero_kernel<<<dim3((unsigned)((bytes + 1023) / 1024)), dim3(256), 0, s>>>(dw, bytes);
        fill_zero_kernel<<<dim3((unsigned)((bytes + 1023) / 1024)), dim3(256), 0, s>>>(db, bytes);
        return true;
    }
    bool ok = false;
    ONIONOP_DT_SWITCH(dt, T, ok = dispatch_row<T, LnBwd>(n, s, dy, mu, rstd, x, w, dtw, dx, ws, groups, n, rows) ||
                                  dispatch_long<T, LnBwdLong>(n, s, dy, mu, rstd, x, w, dtw, dx, ws, groups, n,
                                                              rows));
    if (!ok) return false;
    colsum(s, ws, groups, n, 2, dw, db, dtw);
    return true;
}

}  // namespace onionop
