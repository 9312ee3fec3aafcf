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
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float f16_to_f32(uint16_t u) {
    _Float16 h; __builtin_memcpy(&h, &u, 2); return (float)h;
}
// Scale/bias storage types: 0 = bf16, 1 = f16.
template <int ST> __device__ __forceinline__ float ld_scale(const uint16_t* p) {
    return ST == 0 ? bf16_to_f32(*p) : f16_to_f32(*p);
}

// Wave reductions (64 lanes) ---------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

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
