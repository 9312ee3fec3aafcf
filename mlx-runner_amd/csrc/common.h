// Shared device/host helpers for the gfx950 kernels of libmlxr.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define MLXR_WAVE 64
#define MLXR_PAGE 64          // KV-cache page: positions per page (power of two)
#define MLXR_PAGE_SHIFT 6

// bf16 / f16 storage <-> fp32 --------------------------------------------------
__device__ __host__ __forceinline__ float bf16_to_f32(uint16_t u) {
    const uint32_t b = (uint32_t)u << 16;
    float f; __builtin_memcpy(&f, &b, 4); return f;
}
__device__ __host__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t b; __builtin_memcpy(&b, &f, 4);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}
// Global-memory access through a global-address-space pointer. A plain (generic) pointer makes a
// flat access, which also counts in the LDS counter: every later wait for LDS traffic (each
// barrier) would then wait for that memory round trip as well.
template <typename T>
__device__ __forceinline__ T gload(const T* p) { return *(const __attribute__((address_space(1))) T*)p; }
template <typename T>
__device__ __forceinline__ void gstore(T* p, T v) { *(__attribute__((address_space(1))) T*)p = v; }
__device__ __forceinline__ float4 gload4(const float* p) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v v = gload(reinterpret_cast<const f4v*>(p));
    return float4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float f16_to_f32(uint16_t u) {
    _Float16 h; __builtin_memcpy(&h, &u, 2); return (float)h;
}
// Scale/bias storage types: 0 = bf16, 1 = f16.
template <int ST> __device__ __forceinline__ float ld_scale(const uint16_t* p) {
    return ST == 0 ? bf16_to_f32(*p) : f16_to_f32(*p);
}

// Cross-lane reductions (64 lanes) without LDS: DPP within rows of 16 lanes, then the gfx950
// permlane swaps across rows. Every lane receives the result.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_sum(float v) {   // lanes 4q .. 4q + 3
    v += dpp<0xB1>(v);            // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);            // quad_perm [2,3,0,1]
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
    v = quad_sum(v);
    v += dpp<0x141>(v);           // row_half_mirror: 8-lane sums
    v += dpp<0x140>(v);           // row_mirror: 16-lane sums
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}
// v[l] (+) v[l ^ 16] and v[l] (+) v[l ^ 32]: the swap returns (own row pair, partner row pair).
__device__ __forceinline__ float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_sum(float v) { return xor32_sum(xor16_sum(row16_sum(v))); }

// Workgroup barrier for LDS traffic only. __syncthreads() also waits for every global load and store
// the wave has in flight (vmcnt 0: a weight prefetch, tagged write-backs); this waits for the wave's
// LDS (and scalar) accesses alone, so those stay in flight across it. The asm statements keep the
// compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);     // lgkmcnt(0); vmcnt and expcnt at their maxima (no wait)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
__device__ __forceinline__ float wave_max(float v) { return xor32_max(xor16_max(row16_max(v))); }

// KV cache addressing: layer cache [n_pages][nKV][PAGE][D] bf16; pt maps logical page -> physical.
__device__ __forceinline__ int64_t kv_row(const int* __restrict__ pt, int nKV, int kvh, int pos) {
    int page = pt[pos >> MLXR_PAGE_SHIFT];
    return ((int64_t)page * nKV + kvh) * MLXR_PAGE + (pos & (MLXR_PAGE - 1));
}

// Device-side step parameters read by captured decode graphs (position moves per step).
struct StepParams {
    int pos;          // position of the token this step processes
    int pad[15];
};
