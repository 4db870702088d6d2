// common.h -- shared device helpers for libonionop_hip.so (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace onionop {

typedef __bf16 bf16;
typedef _Float16 f16;

// 16-byte vector used for every coalesced global load / store.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }

// float -> nearest float16 value, kept as float (used for the reference's Float16 Q/K).
__device__ __forceinline__ float round_f16(float x) { return (float)(f16)x; }

// Number of T elements in one 16-byte vector.
template <typename T> struct Vec { static constexpr int N = 16 / sizeof(T); };

// Load / store N = 16/sizeof(T) consecutive elements as float (16-byte aligned).
template <typename T>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, float* out) {
    union { u32x4 v; T e[Vec<T>::N]; } u;
    u.v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < Vec<T>::N; ++i) out[i] = to_f32(u.e[i]);
}
template <typename T>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const float* in) {
    union { u32x4 v; T e[Vec<T>::N]; } u;
#pragma unroll
    for (int i = 0; i < Vec<T>::N; ++i) u.e[i] = from_f32<T>(in[i]);
    *reinterpret_cast<u32x4*>(p) = u.v;
}

// Buffer resource over `bytes` bytes at `base`.  A buffer load whose VGPR byte offset
// (plus the instruction offset) is at or past `bytes` returns zeros without touching
// memory, and such a store is dropped, so tails need no branches: every access is
// unconditional, which also keeps the compiler's memory-counter waits exact across
// software-pipelined loops.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ float bload_f32(rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ void bstore16(u32x4 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, 0);
}
// Streaming (non-temporal) variants for data touched exactly once: the cache-policy
// operand 2 marks the access non-temporal, which lets a read+write stream run close to
// 6 TB/s on MI355X instead of about 5.5 TB/s.
constexpr int kNT = 2;
__device__ __forceinline__ u32x4 bload16_nt(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kNT);
}
__device__ __forceinline__ void bstore16_nt(u32x4 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, kNT);
}

// Zero `bytes` bytes at p (any alignment); used instead of hipMemsetAsync so that the
// library records only kernels when a caller captures it into a HIP graph.
static __global__ void fill_zero_kernel(void* p, int64_t bytes) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    unsigned char* b = reinterpret_cast<unsigned char*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (i + j < bytes) b[i + j] = 0;
}

// 2^x by the hardware instruction (v_exp_f32), without the range reduction exp2f adds
// for results below 2^-126; those may come back as 0, which softmax weights tolerate.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max(a, b) as one v_max_f32.  fmaxf of values the compiler cannot prove canonical (MFMA
// results, values read across lanes, loop-carried values) costs two extra canonicalising
// v_max_f32 under IEEE mode; the operands here are never signalling NaNs.  Not volatile,
// so the scheduler still moves it.
__device__ __forceinline__ float fmax2(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// max / sum over lanes l and l ^ 32, by v_permlane32_swap (no LDS round trip).  With
// x in both operands the swap returns the low half broadcast to both halves and the
// high half broadcast to both halves; every lane combines the two.
__device__ __forceinline__ float pair32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// max of three floats as one v_max3_f32 (scores are never NaN here).
__device__ __forceinline__ float max3f(float a, float b, float c) {
    float r;
    asm volatile("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// ---------------------------------------------------------------- reductions
// Wave-wide sum / max with the result in every lane, all in VALU (no LDS crossbar round
// trips): DPP lane permutations within rows of 16 -- quad_perm [1,0,3,2] (lane ^ 1),
// quad_perm [2,3,0,1] (lane ^ 2), row_half_mirror (lane i with 7 - i of each 8, which after
// the two quad steps pairs the two quads of every 8) and row_mirror (i with 15 - i: the two
// halves of every 16) -- then v_permlane16_swap (the two rows of every 32) and
// v_permlane32_swap (the two halves of the wave).  Each step combines two equal partial
// results in an order that is the same in every lane, so all lanes end bit-identical.
// Every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_perm(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float pair16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_perm<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_perm<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_perm<0x141>(v);  // row_half_mirror
    v += dpp_perm<0x140>(v);  // row_mirror
    return pair32_sum(pair16_sum(v));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_perm<0xB1>(v));
    v = fmaxf(v, dpp_perm<0x4E>(v));
    v = fmaxf(v, dpp_perm<0x141>(v));
    v = fmaxf(v, dpp_perm<0x140>(v));
    return pair32_max(pair16_max(v));
}

// Block-wide sum of up to 16 waves; every thread gets the result.  `red` must hold
// blockDim/64 floats of LDS.  Ends with the LDS free for reuse after the next barrier.
template <int NWAVES>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    if (NWAVES == 1) return v;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NWAVES; ++i) t += red[i];
    __syncthreads();
    return t;
}
template <int NWAVES>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    if (NWAVES == 1) return v;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float t = -INFINITY;
#pragma unroll
    for (int i = 0; i < NWAVES; ++i) t = fmaxf(t, red[i]);
    __syncthreads();
    return t;
}

}  // namespace onionop
