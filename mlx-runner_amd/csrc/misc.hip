// Embedding lookup, RMSNorm, fused q/k-norm + RoPE + KV append, SiLU gate, and token selection.
#include "kernels.h"

namespace mlxr {

// ---- embedding (Kernels.swift:1002-1023, `qembed`): one thread per 8 values of a row ----
template <int BITS, int ST>
__global__ void qembed_kernel(QMat m, int K, int gs, const int* hist, const int* dpos, int T, float* out) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    if (c >= K / 8 || t >= T) return;
    const int row = hist[*dpos + t];
    const int64_t rowBytes = (int64_t)K * BITS / 8;
    const uint8_t* p = m.w + row * rowBytes + (int64_t)c * BITS;
    uint64_t v = 0;
#pragma unroll
    for (int i = 0; i < BITS; i++) v |= (uint64_t)p[i] << (8 * i);
    const int g = (c * 8) / gs, gpr = K / gs;
    const float s = ld_scale<ST>(m.s + (int64_t)row * gpr + g), b = ld_scale<ST>(m.b + (int64_t)row * gpr + g);
    float* o = out + (int64_t)t * K + c * 8;
    constexpr uint64_t M = (1ull << BITS) - 1ull;
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = (float)((v >> (j * BITS)) & M) * s + b;
}

hipError_t launch_qembed(const QMat& m, int K, int bits, int gs, int st, const int* hist, const int* dpos, int T,
                         float* out, hipStream_t s) {
    const int n = K / 8, bs = n < 256 ? n : 256;
    dim3 grid((n + bs - 1) / bs, T);
#define EMB(B) case B: if (st == 0) hipLaunchKernelGGL((qembed_kernel<B, 0>), grid, dim3(bs), 0, s, m, K, gs, hist, dpos, T, out); \
                       else hipLaunchKernelGGL((qembed_kernel<B, 1>), grid, dim3(bs), 0, s, m, K, gs, hist, dpos, T, out); break;
    switch (bits) { EMB(2) EMB(3) EMB(4) EMB(5) EMB(6) EMB(8) default: return hipErrorInvalidValue; }
#undef EMB
    return hipGetLastError();
}

// ---- RMSNorm (Kernels.swift:1037-1070, 1141-1175) ----
__device__ __forceinline__ float block_sum_256(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += red[i];
    return t;
}

__global__ __launch_bounds__(256) void rms_norm_kernel(const float* x, float* y, const float* w, int dim, int row_stride,
                                                       float eps, int add, float* h, const float* r) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    float ss = 0.0f;
    if (add) {
        float* hr = h + (int64_t)row * row_stride;
        const float* rr = r + (int64_t)row * row_stride;
        for (int i = threadIdx.x * 4; i < dim; i += 1024) {
            float4 v = *reinterpret_cast<float4*>(hr + i);
            const float4 u = *reinterpret_cast<const float4*>(rr + i);
            v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
            *reinterpret_cast<float4*>(hr + i) = v;
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        x = h;
    } else {
        const float* xr = x + (int64_t)row * row_stride;
        for (int i = threadIdx.x * 4; i < dim; i += 1024) {
            const float4 v = *reinterpret_cast<const float4*>(xr + i);
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    }
    ss = block_sum_256(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    const float* xr = x + (int64_t)row * row_stride;
    float* yr = y + (int64_t)row * row_stride;
    for (int i = threadIdx.x * 4; i < dim; i += 1024) {
        const float4 v = *reinterpret_cast<const float4*>(xr + i);
        const float4 ww = *reinterpret_cast<const float4*>(w + i);
        float4 o; o.x = v.x * inv * ww.x; o.y = v.y * inv * ww.y; o.z = v.z * inv * ww.z; o.w = v.w * inv * ww.w;
        *reinterpret_cast<float4*>(yr + i) = o;
    }
}

// RMSNorm (optionally after h += r) whose output is the 4-bit GEMM's f16 operand instead of fp32:
// the normalised row (the same fp32 values rms_norm_kernel stores) scaled by the power of two that
// puts its max |y| in [2^13, 2^14), rounded to f16, each 8-group stored as 0,4,1,5,2,6,3,7;
// inv[row] = the inverse scale (x_to_f16_kernel's format).
__global__ __launch_bounds__(256) void rms_norm_f16_kernel(const float* x, const float* w, int dim, int row_stride,
                                                           float eps, int add, float* h, const float* r, uint16_t* xh,
                                                           float* invs) {
    __shared__ float red[4];
    const int row = blockIdx.x, ng = dim >> 3;
    float ss = 0.0f;
    const float* xr = (add ? h : x) + (int64_t)row * row_stride;
    for (int gi = threadIdx.x; gi < ng; gi += 256) {
        float4 a = *reinterpret_cast<const float4*>(xr + 8 * gi), b = *reinterpret_cast<const float4*>(xr + 8 * gi + 4);
        if (add) {
            const float* rr = r + (int64_t)row * row_stride + 8 * gi;
            const float4 ua = *reinterpret_cast<const float4*>(rr), ub = *reinterpret_cast<const float4*>(rr + 4);
            a.x += ua.x; a.y += ua.y; a.z += ua.z; a.w += ua.w;
            b.x += ub.x; b.y += ub.y; b.z += ub.z; b.w += ub.w;
            float* hr = h + (int64_t)row * row_stride + 8 * gi;
            *reinterpret_cast<float4*>(hr) = a;
            *reinterpret_cast<float4*>(hr + 4) = b;
        }
        ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w + b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w;
    }
    ss = block_sum_256(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    auto norm8 = [&](int gi, float* o) {
        const float4 a = *reinterpret_cast<const float4*>(xr + 8 * gi), b = *reinterpret_cast<const float4*>(xr + 8 * gi + 4);
        const float4 wa = *reinterpret_cast<const float4*>(w + 8 * gi), wb = *reinterpret_cast<const float4*>(w + 8 * gi + 4);
        o[0] = a.x * inv * wa.x; o[1] = a.y * inv * wa.y; o[2] = a.z * inv * wa.z; o[3] = a.w * inv * wa.w;
        o[4] = b.x * inv * wb.x; o[5] = b.y * inv * wb.y; o[6] = b.z * inv * wb.z; o[7] = b.w * inv * wb.w;
    };
    float mx = 0.0f;
    for (int gi = threadIdx.x; gi < ng; gi += 256) {
        float o[8];
        norm8(gi, o);
        for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(o[e]));
    }
    __syncthreads();   // red is reused
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e2 = 0;
    if (mx > 0.0f && mx <= 3.0e38f) { frexpf(mx, &e2); e2 = 14 - e2; e2 = e2 < -126 ? -126 : (e2 > 126 ? 126 : e2); }
    const float sc = ldexpf(1.0f, e2);
    if (threadIdx.x == 0) invs[row] = ldexpf(1.0f, -e2);
    for (int gi = threadIdx.x; gi < ng; gi += 256) {
        float o[8];
        norm8(gi, o);
        uint4 q;
        q.x = (uint32_t)f32_to_f16(o[0] * sc) | ((uint32_t)f32_to_f16(o[4] * sc) << 16);
        q.y = (uint32_t)f32_to_f16(o[1] * sc) | ((uint32_t)f32_to_f16(o[5] * sc) << 16);
        q.z = (uint32_t)f32_to_f16(o[2] * sc) | ((uint32_t)f32_to_f16(o[6] * sc) << 16);
        q.w = (uint32_t)f32_to_f16(o[3] * sc) | ((uint32_t)f32_to_f16(o[7] * sc) << 16);
        reinterpret_cast<uint4*>(xh + (int64_t)row * dim)[gi] = q;
    }
}

// Single-pass form of the f16-operand producers above (x_to_f16_kernel in gemm.hip, and
// rms_norm_f16_kernel with or without the residual add) for rows of up to 2048 NG values: each
// thread loads its 8-groups g = tid + 256 i (i < NG) once, all loads in flight together, and keeps
// them in registers through the reductions; the arithmetic per value is the same as those kernels'.
// MODE 0: y = x; 1: y = RMSNorm(x) * w; 2: h += r, then y = RMSNorm(h) * w.
template <int NG, int MODE>
__global__ __launch_bounds__(256) void row_f16_kernel(const float* x, int row_stride, const float* w, int dim, float eps,
                                                      float* h, const float* r, uint16_t* xh, float* invs) {
    __shared__ float red[4];
    const int row = blockIdx.x, ng = dim >> 3, tid = threadIdx.x;
    const float* xr = (MODE == 2 ? h : x) + (int64_t)row * row_stride;
    float4 v[NG][2], u[MODE == 2 ? NG : 1][2];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = tid + 256 * i;
        v[i][0] = v[i][1] = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (g < ng) {
            v[i][0] = *reinterpret_cast<const float4*>(xr + 8 * g);
            v[i][1] = *reinterpret_cast<const float4*>(xr + 8 * g + 4);
            if constexpr (MODE == 2) {
                const float* rr = r + (int64_t)row * row_stride + 8 * g;
                u[i][0] = *reinterpret_cast<const float4*>(rr);
                u[i][1] = *reinterpret_cast<const float4*>(rr + 4);
            }
        }
    }
    if constexpr (MODE == 2) {
#pragma unroll
        for (int i = 0; i < NG; i++) {
            const int g = tid + 256 * i;
            if (g >= ng) continue;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                v[i][c].x += u[i][c].x; v[i][c].y += u[i][c].y; v[i][c].z += u[i][c].z; v[i][c].w += u[i][c].w;
            }
            float* hr = h + (int64_t)row * row_stride + 8 * g;
            *reinterpret_cast<float4*>(hr) = v[i][0];
            *reinterpret_cast<float4*>(hr + 4) = v[i][1];
        }
    }
    if constexpr (MODE != 0) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < NG; i++) {
            const float4 a = v[i][0], b = v[i][1];
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w + b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w;
        }
        ss = block_sum_256(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
        for (int i = 0; i < NG; i++) {
            const int g = tid + 256 * i;
            if (g >= ng) continue;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const float4 ww = *reinterpret_cast<const float4*>(w + 8 * g + 4 * c);
                float4& a = v[i][c];
                a.x = a.x * inv * ww.x; a.y = a.y * inv * ww.y; a.z = a.z * inv * ww.z; a.w = a.w * inv * ww.w;
            }
        }
        __syncthreads();   // red is reused
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < NG; i++)
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const float4 a = v[i][c];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        }
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e2 = 0;
    if (mx > 0.0f && mx <= 3.0e38f) { frexpf(mx, &e2); e2 = 14 - e2; e2 = e2 < -126 ? -126 : (e2 > 126 ? 126 : e2); }
    const float sc = ldexpf(1.0f, e2);
    if (tid == 0) invs[row] = ldexpf(1.0f, -e2);
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = tid + 256 * i;
        if (g >= ng) continue;
        const float4 a = v[i][0], b = v[i][1];
        uint4 q;
        q.x = (uint32_t)f32_to_f16(a.x * sc) | ((uint32_t)f32_to_f16(b.x * sc) << 16);
        q.y = (uint32_t)f32_to_f16(a.y * sc) | ((uint32_t)f32_to_f16(b.y * sc) << 16);
        q.z = (uint32_t)f32_to_f16(a.z * sc) | ((uint32_t)f32_to_f16(b.z * sc) << 16);
        q.w = (uint32_t)f32_to_f16(a.w * sc) | ((uint32_t)f32_to_f16(b.w * sc) << 16);
        reinterpret_cast<uint4*>(xh + (int64_t)row * dim)[g] = q;
    }
}

template <int MODE>
static bool row_f16_launch(const float* x, int row_stride, const float* w, int dim, int rows, float eps, float* h,
                           const float* r, uint16_t* xh, float* inv, hipStream_t s) {
    const int per = (dim / 8 + 255) / 256;
#define MLXR_ROW_F16(NG)                                                                                         \
    hipLaunchKernelGGL((row_f16_kernel<NG, MODE>), dim3(rows), dim3(256), 0, s, x, row_stride, w, dim, eps, h, r, xh, inv)
    if (per <= 2) MLXR_ROW_F16(2);
    else if (per <= 4) MLXR_ROW_F16(4);
    else if (per <= 8) MLXR_ROW_F16(8);
    else if (per <= 16) MLXR_ROW_F16(16);
    else return false;
#undef MLXR_ROW_F16
    return true;
}

bool launch_row_f16(const float* x, int xs, int K, int T, uint16_t* out, float* inv, hipStream_t s) {
    return row_f16_launch<0>(x, xs, nullptr, K, T, 0.0f, nullptr, nullptr, out, inv, s);
}

hipError_t launch_rms_norm_f16(const float* x, const float* w, int dim, int rows, int row_stride, float eps, uint16_t* xh,
                               float* inv, hipStream_t s) {
    if (dim % 8 || row_stride % 4) return hipErrorInvalidValue;
    if (row_f16_launch<1>(x, row_stride, w, dim, rows, eps, nullptr, nullptr, xh, inv, s)) return hipGetLastError();
    hipLaunchKernelGGL(rms_norm_f16_kernel, dim3(rows), dim3(256), 0, s, x, w, dim, row_stride, eps, 0, (float*)nullptr,
                       (const float*)nullptr, xh, inv);
    return hipGetLastError();
}
hipError_t launch_add_rms_norm_f16(float* h, const float* r, const float* w, int dim, int rows, float eps, uint16_t* xh,
                                   float* inv, hipStream_t s) {
    if (dim % 8) return hipErrorInvalidValue;
    if (row_f16_launch<2>(h, dim, w, dim, rows, eps, h, r, xh, inv, s)) return hipGetLastError();
    hipLaunchKernelGGL(rms_norm_f16_kernel, dim3(rows), dim3(256), 0, s, (const float*)h, w, dim, dim, eps, 1, h, r, xh, inv);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float* x, float* y, const float* w, int dim, int rows, int row_stride, float eps,
                           hipStream_t s) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), 0, s, x, y, w, dim, row_stride, eps, 0, (float*)nullptr,
                       (const float*)nullptr);
    return hipGetLastError();
}
hipError_t launch_add_rms_norm(float* h, const float* r, float* y, const float* w, int dim, int rows, float eps,
                               hipStream_t s) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), 0, s, (const float*)h, y, w, dim, dim, eps, 1, h, r);
    return hipGetLastError();
}

// ---- fused q/k norm + RoPE + KV append (Kernels.swift:1081-1138, `qkv_post`) ----
// One workgroup of D threads per (head, token); heads [0, nH) are queries, then nKV keys, nKV values.
__global__ __launch_bounds__(256) void qkv_post_kernel(QkvPostArgs a) {
    __shared__ float buf[256];
    __shared__ float red[4];
    const int h = blockIdx.x, t = blockIdx.y, i = threadIdx.x, D = a.D;
    float* base = a.qkv + (int64_t)t * a.row_stride + (int64_t)h * D;
    const int pos = *a.dpos + a.pos_add + t;
    float v = base[i];
    if (h >= a.nH + a.nKV) {   // value head: straight to the cache
        const int kvh = h - a.nH - a.nKV;
        a.vc[kv_row(a.pt, a.nKV, kvh, pos) * D + i] = f32_to_bf16(v);
        return;
    }
    const bool isQ = h < a.nH;
    if (a.qn) {
        float ss = wave_sum(v * v);
        if ((i & 63) == 0) red[i >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int s = 0; s < D / 64; s++) tot += red[s];
        v = v * (1.0f / sqrtf(tot / (float)D + a.eps)) * (isQ ? a.qn[i] : a.kn[i]);
    }
    buf[i] = v;
    __syncthreads();
    float out = v;
    if (i < a.rot_dim) {
        const int half = a.rot_dim / 2;
        int fi, partner; bool first;
        if (a.traditional) { fi = i / 2; partner = i ^ 1; first = (i & 1) == 0; }
        else { fi = i % half; first = i < half; partner = first ? i + half : i - half; }
        const float ang = (float)pos * a.inv_freq[fi];
        const float c = cosf(ang), sn = sinf(ang);
        out = first ? v * c - buf[partner] * sn : v * c + buf[partner] * sn;
    }
    if (isQ) { base[i] = out; return; }
    const int kvh = h - a.nH;
    const uint16_t kb = f32_to_bf16(out);
    a.kc[kv_row(a.pt, a.nKV, kvh, pos) * D + i] = kb;
    if (a.idx && a.T == 1 && (pos & 3) == 3) {
        // the block of keys pos - 3 .. pos is complete: its index row is the bf16 mean of the four
        // keys, summed in position order as sparse_index_kernel does
        float sum = 0.0f;
        for (int j = pos - 3; j < pos; j++) sum += bf16_to_f32(a.kc[kv_row(a.pt, a.nKV, kvh, j) * D + i]);
        sum += bf16_to_f32(kb);
        a.idx[((int64_t)(pos >> 2) * a.nKV + kvh) * D + i] = f32_to_bf16(sum / 4.0f);
    }
}

// The same for D = rot_dim = 128, one wave per (head, token) and no workgroup barrier: lane l holds
// dims (l, l + 64), or (2 l, 2 l + 1) for traditional RoPE, which are each other's rotation
// partners (angle index l for both), so the norm is one wave sum and the rotation needs no exchange.
__global__ __launch_bounds__(256) void qkv_post_wave_kernel(QkvPostArgs a) {
    const int NHT = a.nH + 2 * a.nKV;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (item >= NHT * a.T) return;
    const int h = item % NHT, t = item / NHT;
    const int d0 = a.traditional ? 2 * l : l, d1 = a.traditional ? 2 * l + 1 : l + 64;
    float* base = a.qkv + (int64_t)t * a.row_stride + (int64_t)h * 128;
    const int pos = *a.dpos + a.pos_add + t;
    float v0 = base[d0], v1 = base[d1];
    if (h >= a.nH + a.nKV) {   // value head: straight to the cache
        const int64_t row = kv_row(a.pt, a.nKV, h - a.nH - a.nKV, pos) * 128;
        a.vc[row + d0] = f32_to_bf16(v0);
        a.vc[row + d1] = f32_to_bf16(v1);
        return;
    }
    const bool isQ = h < a.nH;
    const float* nw = isQ ? a.qn : a.kn;
    if (nw) {
        const float r = 1.0f / sqrtf(wave_sum(v0 * v0 + v1 * v1) / 128.0f + a.eps);
        v0 = v0 * r * nw[d0];
        v1 = v1 * r * nw[d1];
    }
    const float ang = (float)pos * a.inv_freq[l];
    const float c = cosf(ang), sn = sinf(ang);
    const float o0 = v0 * c - v1 * sn, o1 = v1 * c + v0 * sn;
    if (isQ) { base[d0] = o0; base[d1] = o1; return; }
    const int kvh = h - a.nH;
    const int64_t row = kv_row(a.pt, a.nKV, kvh, pos) * 128;
    const uint16_t k0 = f32_to_bf16(o0), k1 = f32_to_bf16(o1);
    a.kc[row + d0] = k0;
    a.kc[row + d1] = k1;
    if (a.idx && a.T == 1 && (pos & 3) == 3) {
        // the block of keys pos - 3 .. pos is complete: its index row is the bf16 mean of the four
        // keys, summed in position order as sparse_index_kernel does
        float s0 = 0.0f, s1 = 0.0f;
        for (int j = pos - 3; j < pos; j++) {
            const int64_t rj = kv_row(a.pt, a.nKV, kvh, j) * 128;
            s0 += bf16_to_f32(a.kc[rj + d0]);
            s1 += bf16_to_f32(a.kc[rj + d1]);
        }
        s0 += bf16_to_f32(k0);
        s1 += bf16_to_f32(k1);
        uint16_t* ir = a.idx + ((int64_t)(pos >> 2) * a.nKV + kvh) * 128;
        ir[d0] = f32_to_bf16(s0 / 4.0f);
        ir[d1] = f32_to_bf16(s1 / 4.0f);
    }
}

hipError_t launch_qkv_post(const QkvPostArgs& a, hipStream_t s) {
    if (a.D == 128 && a.rot_dim == 128) {
        const int items = (a.nH + 2 * a.nKV) * a.T;
        hipLaunchKernelGGL(qkv_post_wave_kernel, dim3((items + 3) / 4), dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL(qkv_post_kernel, dim3(a.nH + 2 * a.nKV, a.T), dim3(a.D), 0, s, a);
    }
    return hipGetLastError();
}

// ---- SiLU gate (Kernels.swift:2004-2013): out[t][i] = silu(gu[t][i]) * gu[t][I + i] ----
__global__ void silu_mul_kernel(const float* gu, float* out, int I) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    if (i >= I) return;
    const float g = gu[(int64_t)t * 2 * I + i], u = gu[(int64_t)t * 2 * I + I + i];
    out[(int64_t)t * I + i] = (g / (1.0f + expf(-g))) * u;
}
hipError_t launch_silu_mul(const float* gu, float* out, int I, int T, hipStream_t s) {
    hipLaunchKernelGGL(silu_mul_kernel, dim3((I + 255) / 256, T), dim3(256), 0, s, gu, out, I);
    return hipGetLastError();
}

// ---- token selection (semantics: Kernels.swift:2362-2619, Engine.swift:112-173) ----
//
// Every comparison goes through one 64-bit selection key per logit: the value's order-preserving
// bits in the high word (NaN mapped below every number, so it is never selected while any number
// is present) and the complement of the index in the low word, so the larger key is the larger
// value and, among equal values, the lower index. A maximum over keys is therefore the argmax with
// the lowest index on ties, and keys are distinct, so a sort by key is a strict total order.
constexpr int SEL_SPAN = 256;     // logits per span of the first pass (one wave, 4 per lane)
constexpr int SEL_POOL = 1024;    // exact top-k limit (and the candidate pool of the sampled path)

__device__ __forceinline__ uint32_t sel_order(float v) {
    if (v != v) return 0u;
    const uint32_t u = __float_as_uint(v);
    return (u >> 31) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint64_t sel_key(float v, int i) { return ((uint64_t)sel_order(v) << 32) | (uint32_t)~(uint32_t)i; }
__device__ __forceinline__ float sel_value(uint64_t k) {
    const uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o >> 31) ? (o & 0x7fffffffu) : ~o);
}
__device__ __forceinline__ int sel_index(uint64_t k) { return (int)~(uint32_t)k; }
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t p = __shfl_xor(k, o, 64);
        k = p > k ? p : k;
    }
    return k;
}
// span b's maximum key, the whole wave (lanes read 4 consecutive logits)
__device__ __forceinline__ uint64_t span_max_key(const float* logits, int V, int b, int lane) {
    const int i = b * SEL_SPAN + 4 * lane;
    uint64_t k = 0;
    if (i + 4 <= V) {
        const float4 v = *reinterpret_cast<const float4*>(logits + i);
        k = max(max(sel_key(v.x, i), sel_key(v.y, i + 1)), max(sel_key(v.z, i + 2), sel_key(v.w, i + 3)));
    } else {
        for (int j = i; j < V; j++) k = max(k, sel_key(logits[j], j));
    }
    return wave_max_key(k);
}
__device__ __forceinline__ void span_store(const SampleArgs& a, int b, uint64_t k) {
    a.bmax[b] = sel_value(k); a.barg[b] = sel_index(k);
}

__global__ __launch_bounds__(256) void sample_blocks_kernel(SampleArgs a) {
    const int nb = (a.V + SEL_SPAN - 1) / SEL_SPAN, b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nb) return;
    const uint64_t k = span_max_key(a.logits, a.V, b, threadIdx.x & 63);
    if ((threadIdx.x & 63) == 0) span_store(a, b, k);
}

__device__ __forceinline__ void emit_token(const SampleArgs& a, int pos, int tok, int st) {
    a.hist[pos + 1] = tok; a.status[pos + 1] = st;
    if (a.host_tok) { a.host_tok[(pos + 1) & a.ring_mask] = tok; a.host_status[(pos + 1) & a.ring_mask] = st; }
    if (a.dpos_next) *a.dpos_next = pos + 1;
}

constexpr int SEL_STAGE = 2048;   // penalised tokens staged per round
constexpr int SEL_MAXSPANS = 1024;

// Repetition penalty over the distinct tokens among hist[pos - window + 1 .. pos]: v > 0 -> v / p,
// else v * p, once per token. Every occurrence of a token computes the same new value from the
// same old one, so the round reads all its tokens' logits before any is written, and duplicates
// within a round then write identical values; a token already seen in an earlier round (windows
// longer than one round) is skipped. The spans holding penalised tokens are marked in a bitmap and
// their maxima recomputed once each.
__device__ void apply_penalty(const SampleArgs& a, int pos, int* tok, float* nval, uint32_t* touched) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6, V = a.V;
    const int n = min(a.window, pos + 1), nb = (V + SEL_SPAN - 1) / SEL_SPAN;
    for (int i = tid; i < SEL_MAXSPANS / 32; i += blockDim.x) touched[i] = 0u;
    for (int r0 = 0; r0 < n; r0 += SEL_STAGE) {
        const int r1 = min(n, r0 + SEL_STAGE);
        for (int j = r0 + tid; j < r1; j += blockDim.x) {
            const int t = a.hist[pos - j];
            bool fresh = t >= 0 && t < V;
            for (int e = 0; fresh && e < r0; e++) fresh = a.hist[pos - e] != t;   // seen in an earlier round
            tok[j - r0] = fresh ? t : -1;
            if (fresh) {
                const float v = a.logits[t];
                nval[j - r0] = v > 0.0f ? v / a.penalty : v * a.penalty;
                atomicOr(&touched[(t / SEL_SPAN) >> 5], 1u << ((t / SEL_SPAN) & 31));
            }
        }
        __syncthreads();
        for (int j = tid; j < r1 - r0; j += blockDim.x)
            if (tok[j] >= 0) a.logits[tok[j]] = nval[j];
        __threadfence_block();
        __syncthreads();
    }
    // one wave per touched span
    for (int w = 0; w < (nb + 31) / 32; w++) {
        uint32_t bits = touched[w];
        int q = 0;
        while (bits) {
            const int bit = __builtin_ctz(bits);
            bits &= bits - 1;
            if (q++ % nw != wave) continue;
            const uint64_t k = span_max_key(a.logits, V, 32 * w + bit, lane);
            if (lane == 0) span_store(a, 32 * w + bit, k);
        }
    }
    __threadfence_block();
    __syncthreads();
}

// Descending bitonic sort of 64 keys across the lanes of a wave (lane i ends with rank i).
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t k, int lane) {
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
        for (int d = size >> 1; d > 0; d >>= 1) {
            const uint64_t p = __shfl_xor(k, d, 64);
            // the lower lane of a pair keeps the larger key in a descending run, the smaller in an
            // ascending one; runs alternate direction until the last stage
            const bool lower = (lane & d) == 0, desc = size == 64 || (lane & size) == 0;
            k = (lower == desc) ? (p > k ? p : k) : (p < k ? p : k);
        }
    return k;
}

// The sampled draw over the sorted top n (keys[0] the largest): probabilities exp((v - M) / T),
// min-p then top-p cuts, one xorshift64 draw r = (s >> 40) / 2^24 walked down the kept mass. The
// sums run sequentially in rank order (the reference's rounding, hence its draws for a seed).
__device__ int draw_token(const SampleArgs& a, const uint64_t* keys, const float* prob, int n, int minp_cut) {
    float mass = 0.0f;
    for (int i = 0; i < n; i++) mass += prob[i];
    int keep = minp_cut;
    if (a.top_p < 1.0f) {
        float run = 0.0f;
        int i = 0;
        while (i < keep) {
            run += prob[i] / mass;
            i++;
            if (run >= a.top_p) { keep = i; break; }
        }
    }
    keep = keep < 1 ? 1 : keep;
    float kept = 0.0f;
    for (int i = 0; i < keep; i++) kept += prob[i];
    uint64_t st = a.rng[0];
    st ^= st << 13; st ^= st >> 7; st ^= st << 17;
    a.rng[0] = st;
    float r = (float)(st >> 40) * (1.0f / 16777216.0f);
    for (int i = 0; i < keep; i++) {
        r -= prob[i] / kept;
        if (r <= 0.0f) return sel_index(keys[i]);
    }
    return sel_index(keys[keep - 1]);
}

// One workgroup of 1024 threads: penalty, the maximum over the span maxima, then the greedy token
// (temperature <= 0.001) or the sampled one.
__global__ __launch_bounds__(1024) void sample_token_kernel(SampleArgs a) {
    __shared__ uint64_t red[16];
    __shared__ uint32_t hist_cnt[256];
    __shared__ uint32_t pick[2];
    __shared__ uint64_t pool[SEL_POOL];
    __shared__ uint64_t ranked[SEL_POOL];
    __shared__ float prob[SEL_POOL];
    __shared__ int tokbuf[SEL_STAGE];
    __shared__ float valbuf[SEL_STAGE];
    __shared__ uint32_t touched[SEL_MAXSPANS / 32];
    __shared__ uint32_t sgt[16], seq_[16];
    __shared__ int minp_first, nfin;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int V = a.V, pos = *a.dpos;
    const float* logits = a.logits;
    const int nb = (V + SEL_SPAN - 1) / SEL_SPAN;
    if (a.penalty != 1.0f && a.window > 0) apply_penalty(a, pos, tokbuf, valbuf, touched);
    uint64_t best = 0;
    for (int b = tid; b < nb; b += blockDim.x) best = max(best, sel_key(a.bmax[b], a.barg[b]));
    best = wave_max_key(best);
    if (lane == 0) red[wave] = best;
    __syncthreads();
    uint64_t top = 0;
    for (int w = 0; w < nw; w++) top = max(top, red[w]);
    const float M = sel_value(top);
    if ((uint32_t)(top >> 32) == 0u || !isfinite(M)) {
        if (tid == 0) emit_token(a, pos, 0, 1);
        return;
    }
    if (a.temperature <= 0.001f) {
        if (tid == 0) emit_token(a, pos, sel_index(top), 0);
        return;
    }
    // Sampled: exact top-k (k <= SEL_POOL, lowest index first among equal values) by an 8-bit radix
    // select of the k-th largest order key over all V logits, then a stable gather.
    const int k = min(a.top_k > 0 ? min(a.top_k, V) : min(512, V), SEL_POOL);
    uint32_t prefix = 0, mask = 0, want = (uint32_t)k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += blockDim.x) hist_cnt[i] = 0;
        __syncthreads();
        for (int n = tid; n < V; n += blockDim.x) {
            const uint32_t key = sel_order(logits[n]);
            if ((key & mask) == prefix) atomicAdd(&hist_cnt[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t acc = 0;
            for (int bin = 255; bin >= 0; bin--) {
                if (acc + hist_cnt[bin] >= want) { pick[0] = (uint32_t)bin; pick[1] = want - acc; break; }
                acc += hist_cnt[bin];
            }
        }
        __syncthreads();
        prefix |= pick[0] << shift; mask |= 255u << shift; want = pick[1];
        __syncthreads();
    }
    // gather: keys > prefix all kept; of keys == prefix the first `want` by index.
    const int chunk = (V + blockDim.x - 1) / blockDim.x;
    const int n0 = min(V, tid * chunk), n1 = min(V, n0 + chunk);
    uint32_t gt = 0, eq = 0;
    for (int n = n0; n < n1; n++) { const uint32_t key = sel_order(logits[n]); gt += key > prefix; eq += key == prefix; }
    // exclusive scans over threads (wave scan then across waves)
    uint32_t gx = gt, ex = eq;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t g2 = __shfl_up(gx, o, 64), e2 = __shfl_up(ex, o, 64);
        if (lane >= o) { gx += g2; ex += e2; }
    }
    if (lane == 63) { sgt[wave] = gx; seq_[wave] = ex; }
    __syncthreads();
    uint32_t gbase = 0, ebase = 0;
    for (int w = 0; w < wave; w++) { gbase += sgt[w]; ebase += seq_[w]; }
    uint32_t gtot = 0; for (int w = 0; w < nw; w++) gtot += sgt[w];
    uint32_t gb = gbase + gx - gt, eb = ebase + ex - eq;
    for (int i = tid; i < SEL_POOL; i += blockDim.x) pool[i] = 0;   // padding: below every real key
    __syncthreads();
    for (int n = n0; n < n1; n++) {
        const float v = logits[n];
        const uint32_t key = sel_order(v);
        int slot = -1;
        if (key > prefix) slot = (int)(gb++);
        else if (key == prefix) { if (eb < want) slot = (int)(gtot + eb); eb++; }
        if (slot >= 0 && slot < SEL_POOL) pool[slot] = sel_key(v, n);
    }
    if (tid == 0) { minp_first = k; nfin = k; }
    __syncthreads();
    // sort: each wave sorts its 64 keys in registers, then every key's rank is its place in its
    // own run plus, for every other run, how many of that run's keys are larger (binary search)
    const uint64_t mine = wave_sort_desc(pool[tid], lane);
    __syncthreads();
    pool[tid] = mine;
    __syncthreads();
    int rank = lane;
    for (int w = 0; w < nw; w++) {
        if (w == wave) continue;
        const uint64_t* run = pool + 64 * w;
        int lo = 0, hi = 64;
        while (lo < hi) { const int mid = (lo + hi) >> 1; if (run[mid] > mine) lo = mid + 1; else hi = mid; }
        rank += lo;
    }
    if (rank < k) ranked[rank] = mine;
    __syncthreads();
    // candidates end at the first non-finite value (NaN or -inf: never drawn)
    if (tid < k && !isfinite(sel_value(ranked[tid]))) atomicMin(&nfin, tid);
    __syncthreads();
    const int n = nfin;
    const float invT = 1.0f / a.temperature;
    if (tid < n) prob[tid] = expf((sel_value(ranked[tid]) - M) * invT);
    __syncthreads();
    // min-p: the first rank whose probability falls below min_p * prob[0]
    if (a.min_p > 0.0f && tid < n && prob[tid] < a.min_p * prob[0]) atomicMin(&minp_first, tid);
    __syncthreads();
    if (tid == 0) {
        const int chosen = draw_token(a, ranked, prob, n, min(minp_first, n));
        if (a.diag) { a.diag[0] = n; a.diag[1] = 1; }
        emit_token(a, pos, chosen, 0);
    }
}

hipError_t launch_sample(const SampleArgs& a, hipStream_t s) {
    const int nb = (a.V + SEL_SPAN - 1) / SEL_SPAN;
    if (nb > SEL_MAXSPANS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(sample_blocks_kernel, dim3((nb + 3) / 4), dim3(256), 0, s, a);
    hipLaunchKernelGGL(sample_token_kernel, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace mlxr
