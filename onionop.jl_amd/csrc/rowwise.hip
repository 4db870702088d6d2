// rowwise.hip -- HBM-bound kernels that reduce along the contiguous dimension:
// online softmax fwd/bwd, RMS norm fwd/bwd, layer norm fwd/bwd.
//
// Layout: a Julia (N, M) column-major matrix is M contiguous rows of N elements here.
// One 256-thread workgroup owns one row at a time and keeps the whole row in registers
// (NV 16-byte vectors per thread), so every element is read from HBM once and written
// once; reductions are wave64 shuffles plus one LDS exchange across the 4 waves.
// Workgroups are persistent over rows (grid = min(rows, 8 x CUs)), so per-element
// weights stay in registers and the backward's weight-gradient partials accumulate in
// registers, one float32 partial row per workgroup, summed by a second small kernel.
#include "common.h"
#include "launch.h"

namespace onionop {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// Element e of the row handled by (thread t, slot i) with VEC elements per vector:
// vector index t + i*256 covers elements [VEC*(t + i*256), +VEC).
template <typename T, int VEC>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int64_t n, int i, float* out) {
    const int64_t e0 = (int64_t)VEC * (threadIdx.x + (int64_t)i * kThreads);
    if constexpr (VEC == Vec<T>::N) {
        if (e0 < n) load_vec<T>(row + e0, out);
        else {
#pragma unroll
            for (int j = 0; j < VEC; ++j) out[j] = 0.f;
        }
    } else {
        static_assert(VEC == 1, "scalar path");
        out[0] = e0 < n ? to_f32(row[e0]) : 0.f;
    }
}
template <typename T, int VEC>
__device__ __forceinline__ void store_row(T* __restrict__ row, int64_t n, int i, const float* in) {
    const int64_t e0 = (int64_t)VEC * (threadIdx.x + (int64_t)i * kThreads);
    if (e0 >= n) return;
    if constexpr (VEC == Vec<T>::N) store_vec<T>(row + e0, in);
    else row[e0] = from_f32<T>(in[0]);
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
template <int VEC>
__device__ __forceinline__ void store_w(void* __restrict__ w, int dt, int64_t n, int i, const float* in) {
    const int64_t e0 = (int64_t)VEC * (threadIdx.x + (int64_t)i * kThreads);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
        const int64_t e = e0 + j;
        if (e < n) {
            if (dt == 0) reinterpret_cast<float*>(w)[e] = in[j];
            else if (dt == 1) reinterpret_cast<f16*>(w)[e] = from_f32<f16>(in[j]);
            else reinterpret_cast<bf16*>(w)[e] = from_f32<bf16>(in[j]);
        }
    }
}

// ------------------------------------------------------------------ softmax
// y = exp(x - max) / sum(exp(x - max)) per row (online_softmax!, src/softmax.jl:19-58).
template <typename T, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void softmax_fwd_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                                int64_t n, int64_t rows) {
    __shared__ float red[kWaves];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const T* xr = x + r * n;
        float v[NV][VEC];
#pragma unroll
        for (int i = 0; i < NV; ++i) load_row<T, VEC>(xr, n, i, v[i]);
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (slot_valid<VEC>(n, i))
#pragma unroll
                for (int j = 0; j < VEC; ++j) m = fmaxf(m, v[i][j]);
        m = block_max<kWaves>(m, red);
        const float m2 = m * kLog2e;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const bool ok = slot_valid<VEC>(n, i);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                v[i][j] = fast_exp2(fmaf(v[i][j], kLog2e, -m2));
                if (ok) s += v[i][j];
            }
        }
        s = block_sum<kWaves>(s, red);
        const float inv = 1.0f / s;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) v[i][j] *= inv;
            store_row<T, VEC>(y + r * n, n, i, v[i]);
        }
    }
}

// dx = y (dy - sum(y dy)) per row (∇online_softmax, src/softmax.jl:70-80).
template <typename T, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void softmax_bwd_kernel(const T* __restrict__ dy, const T* __restrict__ y,
                                                                T* __restrict__ dx, int64_t n, int64_t rows) {
    __shared__ float red[kWaves];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        float g[NV][VEC], yv[NV][VEC];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            load_row<T, VEC>(dy + r * n, n, i, g[i]);
            load_row<T, VEC>(y + r * n, n, i, yv[i]);
        }
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int j = 0; j < VEC; ++j) s = fmaf(g[i][j], yv[i][j], s);
        s = block_sum<kWaves>(s, red);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) g[i][j] = yv[i][j] * (g[i][j] - s);
            store_row<T, VEC>(dx + r * n, n, i, g[i]);
        }
    }
}

// ------------------------------------------------------------------ RMS norm
// rstd = 1/sqrt(mean(x^2) + eps); y = (offset + w) x rstd (_rms_norm!, src/rms_norm.jl:3-38).
template <typename T, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void rms_fwd_kernel(const T* __restrict__ x, const void* __restrict__ w, int dtw,
                                                            T* __restrict__ y, float* __restrict__ rstd,
                                                            int64_t n, int64_t rows, float eps, float offset) {
    __shared__ float red[kWaves];
    float wv[NV][VEC];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        load_w<VEC>(w, dtw, n, i, wv[i]);
#pragma unroll
        for (int j = 0; j < VEC; ++j) wv[i][j] += offset;
    }
    const float inv_n = 1.0f / (float)n;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        float v[NV][VEC];
#pragma unroll
        for (int i = 0; i < NV; ++i) load_row<T, VEC>(x + r * n, n, i, v[i]);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int j = 0; j < VEC; ++j) s = fmaf(v[i][j], v[i][j], s);
        s = block_sum<kWaves>(s, red);
        const float rs = 1.0f / sqrtf(s * inv_n + eps);
        if (threadIdx.x == 0) rstd[r] = rs;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) v[i][j] = wv[i][j] * v[i][j] * rs;
            store_row<T, VEC>(y + r * n, n, i, v[i]);
        }
    }
}

// Per row: dd = sum(dy (w+off) x); dx = rstd dy (w+off) - rstd^3 dd x / n; the dw partial
// sum(dy x rstd) over this workgroup's rows goes to ws[blockIdx.x, :]
// (_∇rms_norm!, src/rms_norm.jl:43-115).
template <typename T, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void rms_bwd_kernel(const T* __restrict__ dy, const float* __restrict__ rstd,
                                                            const T* __restrict__ x, const void* __restrict__ w, int dtw,
                                                            float offset, T* __restrict__ dx, float* __restrict__ ws,
                                                            int64_t n, int64_t rows) {
    __shared__ float red[kWaves];
    float wv[NV][VEC], dw[NV][VEC];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        load_w<VEC>(w, dtw, n, i, wv[i]);
#pragma unroll
        for (int j = 0; j < VEC; ++j) { wv[i][j] += offset; dw[i][j] = 0.f; }
    }
    const float inv_n = 1.0f / (float)n;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        float g[NV][VEC], xv[NV][VEC];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            load_row<T, VEC>(dy + r * n, n, i, g[i]);
            load_row<T, VEC>(x + r * n, n, i, xv[i]);
        }
        const float rs = rstd[r];
        float dd = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int j = 0; j < VEC; ++j) dd = fmaf(g[i][j] * wv[i][j], xv[i][j], dd);
        dd = block_sum<kWaves>(dd, red);
        const float c = rs * rs * rs * dd * inv_n;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                dw[i][j] = fmaf(g[i][j], xv[i][j] * rs, dw[i][j]);
                g[i][j] = rs * g[i][j] * wv[i][j] - c * xv[i][j];
            }
            store_row<T, VEC>(dx + r * n, n, i, g[i]);
        }
    }
    float* wsr = ws + (int64_t)blockIdx.x * n;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int64_t e0 = (int64_t)VEC * (threadIdx.x + (int64_t)i * kThreads);
#pragma unroll
        for (int j = 0; j < VEC; ++j)
            if (e0 + j < n) wsr[e0 + j] = dw[i][j];
    }
}

// ------------------------------------------------------------------ layer norm
// mu = mean(x); rstd = 1/sqrt(mean((x-mu)^2) + eps); y = (x-mu) rstd w + b
// (_layer_norm!, src/layer_norm.jl:8-63).
template <typename T, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void ln_fwd_kernel(const T* __restrict__ x, const void* __restrict__ w,
                                                           const void* __restrict__ b, int dtw, T* __restrict__ y,
                                                           float* __restrict__ mu, float* __restrict__ rstd,
                                                           int64_t n, int64_t rows, float eps) {
    __shared__ float red[kWaves];
    float wv[NV][VEC], bv[NV][VEC];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        load_w<VEC>(w, dtw, n, i, wv[i]);
        load_w<VEC>(b, dtw, n, i, bv[i]);
    }
    const float inv_n = 1.0f / (float)n;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        float v[NV][VEC];
#pragma unroll
        for (int i = 0; i < NV; ++i) load_row<T, VEC>(x + r * n, n, i, v[i]);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int j = 0; j < VEC; ++j) s += v[i][j];
        const float m = block_sum<kWaves>(s, red) * inv_n;
        float q = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const bool ok = slot_valid<VEC>(n, i);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const int64_t e = (int64_t)VEC * (threadIdx.x + (int64_t)i * kThreads) + j;
                const float c = v[i][j] - m;
                if (ok && e < n) q = fmaf(c, c, q);
            }
        }
        const float rs = 1.0f / sqrtf(block_sum<kWaves>(q, red) * inv_n + eps);
        if (threadIdx.x == 0) { mu[r] = m; rstd[r] = rs; }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) v[i][j] = fmaf((v[i][j] - m) * rs, wv[i][j], bv[i][j]);
            store_row<T, VEC>(y + r * n, n, i, v[i]);
        }
    }
}

// Per row: xn = (x-mu) rstd; c1 = mean(w dy xn); c2 = mean(w dy);
// dx = (w dy - (xn c1 + c2)) rstd; partials of dw = sum dy xn and db = sum dy go to
// ws[blockIdx.x, :] and ws[grid + blockIdx.x, :] (_∇layer_norm!, src/layer_norm.jl:65-148).
template <typename T, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void ln_bwd_kernel(const T* __restrict__ dy, const float* __restrict__ mu,
                                                           const float* __restrict__ rstd, const T* __restrict__ x,
                                                           const void* __restrict__ w, int dtw, T* __restrict__ dx,
                                                           float* __restrict__ ws, int64_t n, int64_t rows) {
    __shared__ float red[2 * kWaves];
    float wv[NV][VEC], dw[NV][VEC], db[NV][VEC];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        load_w<VEC>(w, dtw, n, i, wv[i]);
#pragma unroll
        for (int j = 0; j < VEC; ++j) dw[i][j] = db[i][j] = 0.f;
    }
    const float inv_n = 1.0f / (float)n;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        float g[NV][VEC], xv[NV][VEC];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            load_row<T, VEC>(dy + r * n, n, i, g[i]);
            load_row<T, VEC>(x + r * n, n, i, xv[i]);
        }
        const float m = mu[r], rs = rstd[r];
        float c1 = 0.f, c2 = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                xv[i][j] = (xv[i][j] - m) * rs;  // xn (zero-padded slots give g = 0)
                const float wdy = wv[i][j] * g[i][j];
                c1 = fmaf(wdy, xv[i][j], c1);
                c2 += wdy;
            }
        c1 = wave_sum(c1);
        c2 = wave_sum(c2);
        if (lane == 0) { red[wid] = c1; red[kWaves + wid] = c2; }
        __syncthreads();
        c1 = 0.f;
        c2 = 0.f;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) { c1 += red[i]; c2 += red[kWaves + i]; }
        __syncthreads();
        c1 *= inv_n;
        c2 *= inv_n;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            float o[VEC];
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                o[j] = (wv[i][j] * g[i][j] - fmaf(xv[i][j], c1, c2)) * rs;
                dw[i][j] = fmaf(g[i][j], xv[i][j], dw[i][j]);
                db[i][j] += g[i][j];
            }
            store_row<T, VEC>(dx + r * n, n, i, o);
        }
    }
    float* wsw = ws + (int64_t)blockIdx.x * n;
    float* wsb = ws + ((int64_t)gridDim.x + blockIdx.x) * n;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int64_t e0 = (int64_t)VEC * (threadIdx.x + (int64_t)i * kThreads);
#pragma unroll
        for (int j = 0; j < VEC; ++j)
            if (e0 + j < n) { wsw[e0 + j] = dw[i][j]; wsb[e0 + j] = db[i][j]; }
    }
}

// out[e] = sum_g ws[g, e] for e < n (column sums of the [groups, n] partials), written
// as float32 or as dtype `dt`; `count` partial matrices are reduced (dw, then db).
__global__ __launch_bounds__(256) void colsum_kernel(const float* __restrict__ ws, int64_t groups, int64_t n,
                                                     void* __restrict__ out0, void* __restrict__ out1, int dt) {
    const int64_t e = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
    const int part = threadIdx.x >> 6;  // 4 waves split the groups
    const int which = blockIdx.y;
    __shared__ float red[4][64];
    float s = 0.f;
    if (e < n) {
        const float* base = ws + (int64_t)which * groups * n;
        for (int64_t g = part; g < groups; g += 4) s += base[g * n + e];
    }
    red[part][threadIdx.x & 63] = s;
    __syncthreads();
    if (part == 0 && e < n) {
        s = red[0][threadIdx.x] + red[1][threadIdx.x] + red[2][threadIdx.x] + red[3][threadIdx.x];
        void* out = which == 0 ? out0 : out1;
        if (dt == 0) reinterpret_cast<float*>(out)[e] = s;
        else if (dt == 1) reinterpret_cast<f16*>(out)[e] = from_f32<f16>(s);
        else reinterpret_cast<bf16*>(out)[e] = from_f32<bf16>(s);
    }
}

// ------------------------------------------------------------------ dispatch

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

static inline int64_t grid_rows(int64_t rows) {
    const int64_t g = 8LL * num_cus();
    return rows < g ? rows : g;
}

template <typename T, int VEC, int NV>
struct SoftmaxFwd {
    static bool run(hipStream_t s, const void* x, void* y, int64_t n, int64_t rows) {
        softmax_fwd_kernel<T, VEC, NV><<<dim3((unsigned)grid_rows(rows)), dim3(kThreads), 0, s>>>(
            (const T*)x, (T*)y, n, rows);
        return true;
    }
};
template <typename T, int VEC, int NV>
struct SoftmaxBwd {
    static bool run(hipStream_t s, const void* dy, const void* y, void* dx, int64_t n, int64_t rows) {
        softmax_bwd_kernel<T, VEC, NV><<<dim3((unsigned)grid_rows(rows)), dim3(kThreads), 0, s>>>(
            (const T*)dy, (const T*)y, (T*)dx, n, rows);
        return true;
    }
};
template <typename T, int VEC, int NV>
struct RmsFwd {
    static bool run(hipStream_t s, const void* x, const void* w, int dtw, void* y, float* rstd, int64_t n,
                    int64_t rows, float eps, float offset) {
        rms_fwd_kernel<T, VEC, NV><<<dim3((unsigned)grid_rows(rows)), dim3(kThreads), 0, s>>>(
            (const T*)x, w, dtw, (T*)y, rstd, n, rows, eps, offset);
        return true;
    }
};
template <typename T, int VEC, int NV>
struct RmsBwd {
    static bool run(hipStream_t s, const void* dy, const float* rstd, const void* x, const void* w, int dtw,
                    float offset, void* dx, float* ws, int64_t groups, int64_t n, int64_t rows) {
        rms_bwd_kernel<T, VEC, NV><<<dim3((unsigned)groups), dim3(kThreads), 0, s>>>(
            (const T*)dy, rstd, (const T*)x, w, dtw, offset, (T*)dx, ws, n, rows);
        return true;
    }
};
template <typename T, int VEC, int NV>
struct LnFwd {
    static bool run(hipStream_t s, const void* x, const void* w, const void* b, int dtw, void* y, float* mu,
                    float* rstd, int64_t n, int64_t rows, float eps) {
        ln_fwd_kernel<T, VEC, NV><<<dim3((unsigned)grid_rows(rows)), dim3(kThreads), 0, s>>>(
            (const T*)x, w, b, dtw, (T*)y, mu, rstd, n, rows, eps);
        return true;
    }
};
template <typename T, int VEC, int NV>
struct LnBwd {
    static bool run(hipStream_t s, const void* dy, const float* mu, const float* rstd, const void* x,
                    const void* w, int dtw, void* dx, float* ws, int64_t groups, int64_t n, int64_t rows) {
        ln_bwd_kernel<T, VEC, NV><<<dim3((unsigned)groups), dim3(kThreads), 0, s>>>(
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

int64_t max_row_elems(int dt) {
    const int es = dt == 0 ? 4 : 2;
    return 16LL * kThreads * (16 / es);
}

// Fixed (device-independent) so the workspace size and the summation order, hence the
// bits of dw/db, do not depend on the GPU model.
int64_t norm_bwd_groups(int64_t rows) { return rows < 1024 ? rows : 1024; }

bool launch_softmax_fwd(hipStream_t s, int dt, int64_t n, int64_t rows, const void* x, void* y) {
    if (rows == 0 || n == 0) return true;
    ONIONOP_DT_SWITCH(dt, T, return dispatch_row<T, SoftmaxFwd>(n, s, x, y, n, rows));
    return true;
}
bool launch_softmax_bwd(hipStream_t s, int dt, int64_t n, int64_t rows, const void* dy, const void* y, void* dx) {
    if (rows == 0 || n == 0) return true;
    ONIONOP_DT_SWITCH(dt, T, return dispatch_row<T, SoftmaxBwd>(n, s, dy, y, dx, n, rows));
    return true;
}
bool launch_rms_fwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* x, const void* w,
                    float eps, float offset, void* y, float* rstd) {
    if (rows == 0) return true;
    ONIONOP_DT_SWITCH(dt, T, return dispatch_row<T, RmsFwd>(n, s, x, w, dtw, y, rstd, n, rows, eps, offset));
    return true;
}
bool launch_rms_bwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* dy, const float* rstd,
                    const void* x, const void* w, float offset, void* dx, float* dw, float* ws) {
    const int64_t groups = norm_bwd_groups(rows);
    if (rows > 0) {
        bool ok = false;
        ONIONOP_DT_SWITCH(dt, T,
                          ok = dispatch_row<T, RmsBwd>(n, s, dy, rstd, x, w, dtw, offset, dx, ws, groups, n, rows));
        if (!ok) return false;
    }
    if (n == 0) return true;
    if (rows == 0) {  // no rows: dw = 0
        fill_zero_kernel<<<dim3((unsigned)((n * 4 + 1023) / 1024)), dim3(256), 0, s>>>(dw, n * 4);
        return true;
    }
    colsum_kernel<<<dim3((unsigned)((n + 63) / 64), 1), dim3(256), 0, s>>>(ws, groups, n, dw, nullptr, 0);
    return true;
}
bool launch_ln_fwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* x, const void* w,
                   const void* b, float eps, void* y, float* mu, float* rstd) {
    if (rows == 0) return true;
    ONIONOP_DT_SWITCH(dt, T, return dispatch_row<T, LnFwd>(n, s, x, w, b, dtw, y, mu, rstd, n, rows, eps));
    return true;
}
bool launch_ln_bwd(hipStream_t s, int dt, int dtw, int64_t n, int64_t rows, const void* dy, const float* mu,
                   const float* rstd, const void* x, const void* w, void* dx, void* dw, void* db, float* ws) {
    const int64_t groups = norm_bwd_groups(rows);
    if (n == 0) return true;
    if (rows == 0) {
        const int64_t bytes = (dtw == 0 ? 4 : 2) * n;
        fill_zero_kernel<<<dim3((unsigned)((bytes + 1023) / 1024)), dim3(256), 0, s>>>(dw, bytes);
        fill_zero_kernel<<<dim3((unsigned)((bytes + 1023) / 1024)), dim3(256), 0, s>>>(db, bytes);
        return true;
    }
    bool ok = false;
    ONIONOP_DT_SWITCH(dt, T, ok = dispatch_row<T, LnBwd>(n, s, dy, mu, rstd, x, w, dtw, dx, ws, groups, n, rows));
    if (!ok) return false;
    colsum_kernel<<<dim3((unsigned)((n + 63) / 64), 2), dim3(256), 0, s>>>(ws, groups, n, dw, db, dtw);
    return true;
}

}  // namespace onionop
