// Prefill quantized GEMM on gfx950 bf16 MFMA: Y[T][O] = X[T][K] * W[O][K]^T (+ bias).
//
// Semantics: the reference's prefill tiles (Kernels.swift:785-851, `qgemm`) compute the same
// product with fp32 operands. Here (the build's declared precision) X is rounded once to bf16 and
// each weight is dequantized in fp32 (`s * q + b`) then rounded to bf16; products accumulate in
// fp32 on the matrix cores (v_mfma_f32_16x16x32_bf16).
//
// Tiling: a 256-thread workgroup owns a 128-token x 128-row output tile; each wave a 64 x 64
// quarter (4 x 4 MFMA tiles of 16 x 16). K advances 64 at a time: the X tile (bf16) and the
// dequantized W tile are staged in LDS with a padded row stride (72 bf16) so the 16-byte fragment
// reads of 16 consecutive rows fall in different banks.
#include "kernels.h"

namespace mlxr {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int GB_M = 128, GB_N = 128, GB_K = 64, GB_LD = GB_K + 8;

__global__ __launch_bounds__(256) void to_bf16_kernel(const float* x, int xs, int K, int T, uint16_t* out) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const int64_t n = (int64_t)T * K;
    if (i >= n) return;
    const int t = (int)(i / K), k = (int)(i % K);
    const float4 v = *reinterpret_cast<const float4*>(x + (int64_t)t * xs + k);
    uint2 o;
    o.x = (uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16);
    o.y = (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16);
    *reinterpret_cast<uint2*>(out + i) = o;
}

struct QGemmDev {
    const uint8_t* w; const uint16_t* s; const uint16_t* b; const uint16_t* bias;
    int K, gs, O, T, ys;
    const uint16_t* xbf; float* y;
};

template <int BITS>
__device__ __forceinline__ void load_codes32(const uint8_t* p, uint32_t* w) {
    if constexpr (BITS == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (BITS == 8) {
        const uint4 a = reinterpret_cast<const uint4*>(p)[0], b = reinterpret_cast<const uint4*>(p)[1];
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < BITS; i++) w[i] = reinterpret_cast<const uint32_t*>(p)[i];
    }
}
template <int BITS>
__device__ __forceinline__ uint32_t code_of(const uint32_t* w, int j) {
    constexpr uint32_t M = (1u << BITS) - 1u;
    const int bit = j * BITS, wi = bit >> 5, off = bit & 31;
    if (off + BITS <= 32) return (w[wi] >> off) & M;
    return ((w[wi] >> off) | (w[wi + 1] << (32 - off))) & M;
}

template <int BITS, int ST>
__global__ __launch_bounds__(256) void qgemm_kernel(QGemmDev a) {
    __shared__ __attribute__((aligned(16))) uint16_t Xs[GB_M * GB_LD];
    __shared__ __attribute__((aligned(16))) uint16_t Ws[GB_N * GB_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * GB_N, m0 = blockIdx.y * GB_M;
    const int wm = wave >> 1, wn = wave & 1;
    const int K = a.K, gpr = K / a.gs;
    const int64_t rowBytes = (int64_t)K * BITS / 8;
    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // per-thread load roles
    const int lr = tid >> 1, lh = tid & 1;          // tile row, half (32 of the 64 k)
    const int xm = m0 + lr;
    const uint16_t* xrow = a.xbf + (int64_t)(xm < a.T ? xm : a.T - 1) * K + lh * 32;
    const int wrow = n0 + lr < a.O ? n0 + lr : a.O - 1;
    const uint8_t* wptr = a.w + wrow * rowBytes + lh * (4 * BITS);
    const uint16_t* sp = a.s + (int64_t)wrow * gpr;
    const uint16_t* bp = a.b + (int64_t)wrow * gpr;
    const bool xvalid = xm < a.T;
    for (int k0 = 0; k0 < K; k0 += GB_K) {
        // X tile
        {
            const uint4* src = reinterpret_cast<const uint4*>(xrow + k0);
            uint4* dst = reinterpret_cast<uint4*>(Xs + lr * GB_LD + lh * 32);
#pragma unroll
            for (int v = 0; v < 4; v++) dst[v] = xvalid ? src[v] : uint4{0, 0, 0, 0};
        }
        // W tile: 32 codes of row lr, dequantized in fp32, rounded to bf16
        {
            uint32_t w[BITS];
            load_codes32<BITS>(wptr + (int64_t)(k0 / 32) * (4 * BITS), w);
            const int g = (k0 + lh * 32) / a.gs;
            const float s = ld_scale<ST>(sp + g), b = ld_scale<ST>(bp + g);
            uint32_t packed[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float v0 = (float)code_of<BITS>(w, 2 * j) * s + b;
                const float v1 = (float)code_of<BITS>(w, 2 * j + 1) * s + b;
                packed[j] = (uint32_t)f32_to_bf16(v0) | ((uint32_t)f32_to_bf16(v1) << 16);
            }
            uint4* dst = reinterpret_cast<uint4*>(Ws + lr * GB_LD + lh * 32);
#pragma unroll
            for (int v = 0; v < 4; v++) dst[v] = uint4{packed[4 * v], packed[4 * v + 1], packed[4 * v + 2], packed[4 * v + 3]};
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            bf16x8_t af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                af[i] = *reinterpret_cast<const bf16x8_t*>(Xs + (wm * 64 + i * 16 + (lane & 15)) * GB_LD + kk * 32 + (lane >> 4) * 8);
#pragma unroll
            for (int j = 0; j < 4; j++)
                bf[j] = *reinterpret_cast<const bf16x8_t*>(Ws + (wn * 64 + j * 16 + (lane & 15)) * GB_LD + kk * 32 + (lane >> 4) * 8);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + wn * 64 + j * 16 + (lane & 15);
            if (n >= a.O) continue;
            const float bias = a.bias ? ld_scale<ST>(a.bias + n) : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
                if (m < a.T) a.y[(int64_t)m * a.ys + n] = acc[i][j][r] + bias;
            }
        }
}

hipError_t launch_qgemm(const QGemmArgs& a, hipStream_t s) {
    const int64_t n = (int64_t)a.T * a.K;
    hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, a.x, a.x_stride, a.K, a.T, a.xbf);
    QGemmDev d{a.m.w, a.m.s, a.m.b, a.m.bias, a.K, a.gs, a.O, a.T, a.y_stride, a.xbf, a.y};
    dim3 grid((a.O + GB_N - 1) / GB_N, (a.T + GB_M - 1) / GB_M);
#define GEMM_CASE(B) case B: \
    if (a.st == 0) hipLaunchKernelGGL((qgemm_kernel<B, 0>), grid, dim3(256), 0, s, d); \
    else hipLaunchKernelGGL((qgemm_kernel<B, 1>), grid, dim3(256), 0, s, d); \
    return hipGetLastError();
    switch (a.bits) { GEMM_CASE(2) GEMM_CASE(3) GEMM_CASE(4) GEMM_CASE(5) GEMM_CASE(6) GEMM_CASE(8) }
#undef GEMM_CASE
    return hipErrorInvalidValue;
}

}  // namespace mlxr
