// Decode matvec (T == 1) and small-batch matmul (T = 2..8) over MLX affine-quantized weights.
//
// Semantics follow the reference's fused decode kernel (Kernels.swift:204-318, `qmv`) and its
// generic `qmm` (Kernels.swift:60-113): y[o] = sum over groups of s * (sum_j q_j x_j) + b * (sum_j x_j),
// fp32 accumulation, rows of up to three matrices [A | B | C] concatenated, optional per-row bias.
//
// MI355X layout: a 256-thread workgroup (4 waves of 64) owns ROWS rows per wave; for inputs of at
// least 64 chunks per wave (K >= 8192, below 8 bits) the four waves share the same ROWS rows and take a quarter of
// K each instead (so short-N, long-K projections still spread over many workgroups, and each
// wave's chain of loads is a quarter as long), their partial sums meeting in LDS, added in wave
// order. A lane
// consumes one 32-code chunk of a row per step (4*BITS bytes: one 16-byte load at 4 bits), so a
// wave streams a contiguous 64*4*BITS-byte span of the row per load instruction (fully coalesced),
// and every row reuses the lane's 32 x values. Codes are extracted without shifts where possible: at
// 4 bits the dword is split into low/high nibbles of its four bytes and each byte converted with the
// byte-to-float conversion. The workgroup can normalise x itself (RMSNorm of the residual stream
// times the norm weight, written to LDS) so the norm needs no kernel of its own.
#include "kernels.h"

namespace mlxr {

constexpr int QMV_WAVES = 4;
constexpr int QMV_ROWS = 4;   // rows per wave
constexpr int QMV_KS_ROWS = 8;   // rows of a split-K workgroup (its waves share them, so x is read once per 8 rows)

struct QmvDev {
    const uint8_t* w[3]; const uint16_t* s[3]; const uint16_t* b[3]; const uint16_t* bias[3];
    int o1, o2;               // rows of A, B (C gets the rest)
    int K, gs, O, epi, hasBias;
    const float* x; const float* norm_w; float eps; float* y;
};

// 32 codes of one chunk (BITS dwords) dotted with 32 x values.
template <int BITS>
__device__ __forceinline__ float chunk_dot(const uint32_t* w, const float* x) {
    float d = 0.0f;
    if constexpr (BITS == 4) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
            const float* xp = x + 8 * i;
            d = fmaf((float)(lo & 0xFFu), xp[0], d);
            d = fmaf((float)(hi & 0xFFu), xp[1], d);
            d = fmaf((float)((lo >> 8) & 0xFFu), xp[2], d);
            d = fmaf((float)((hi >> 8) & 0xFFu), xp[3], d);
            d = fmaf((float)((lo >> 16) & 0xFFu), xp[4], d);
            d = fmaf((float)((hi >> 16) & 0xFFu), xp[5], d);
            d = fmaf((float)(lo >> 24), xp[6], d);
            d = fmaf((float)(hi >> 24), xp[7], d);
        }
    } else if constexpr (BITS == 8) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float* xp = x + 4 * i;
            d = fmaf((float)(w[i] & 0xFFu), xp[0], d);
            d = fmaf((float)((w[i] >> 8) & 0xFFu), xp[1], d);
            d = fmaf((float)((w[i] >> 16) & 0xFFu), xp[2], d);
            d = fmaf((float)(w[i] >> 24), xp[3], d);
        }
    } else {
        constexpr uint32_t M = (1u << BITS) - 1u;
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const int bit = j * BITS, wi = bit >> 5, off = bit & 31;
            uint32_t q;
            if (off + BITS <= 32) q = (w[wi] >> off) & M;
            else q = ((w[wi] >> off) | (w[wi + 1] << (32 - off))) & M;
            d = fmaf((float)q, x[j], d);
        }
    }
    return d;
}

template <int BITS>
__device__ __forceinline__ void load_chunk(const uint8_t* p, uint32_t* w) {
    if constexpr (BITS == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (BITS == 8) {
        const uint4 a = reinterpret_cast<const uint4*>(p)[0], b = reinterpret_cast<const uint4*>(p)[1];
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
        for (int i = 0; i < BITS; i++) w[i] = q[i];
    }
}

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// XNORM: x is normalised into LDS by the workgroup (K floats). XCOPY: x is copied into LDS as it is
// (the four waves then read it from there: each wave's x would otherwise come through L2 once per
// four rows, more bytes than its weights). KS: the waves split K over the same rows.
template <int BITS, int ST, bool XNORM, bool KS, bool XCOPY = false>
__global__ __launch_bounds__(256) void qmv_kernel(QmvDev a) {
    constexpr int R = KS ? QMV_KS_ROWS : QMV_ROWS;   // rows per wave (split K: per workgroup)
    extern __shared__ __attribute__((aligned(16))) float xs_lds[];
    __shared__ float red[QMV_WAVES];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = a.K;
    const float* xsrc = a.x;
    if constexpr (XNORM) {
        float ss = 0.0f;
        for (int i = threadIdx.x * 4; i < K; i += 256 * 4) {
            const float4 v = *reinterpret_cast<const float4*>(a.x + i);
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        const float tot = red[0] + red[1] + red[2] + red[3];
        const float inv = 1.0f / sqrtf(tot / (float)K + a.eps);
        for (int i = threadIdx.x * 4; i < K; i += 256 * 4) {
            const float4 v = *reinterpret_cast<const float4*>(a.x + i);
            const float4 w = *reinterpret_cast<const float4*>(a.norm_w + i);
            float4 o; o.x = v.x * inv * w.x; o.y = v.y * inv * w.y; o.z = v.z * inv * w.z; o.w = v.w * inv * w.w;
            *reinterpret_cast<float4*>(xs_lds + i) = o;
        }
        __syncthreads();
        xsrc = xs_lds;
    }
    if constexpr (XCOPY && !XNORM) {
        for (int i = threadIdx.x * 4; i < K; i += 256 * 4)
            *reinterpret_cast<float4*>(xs_lds + i) = *reinterpret_cast<const float4*>(a.x + i);
        __syncthreads();
        xsrc = xs_lds;
    }
    const bool gated = a.epi == EPI_GATED;
    const int rows_per_wave = R;
    const int slot0 = (KS ? blockIdx.x : blockIdx.x * QMV_WAVES + wave) * (gated ? rows_per_wave / 2 : rows_per_wave);
    if (!KS && slot0 >= a.O) return;
    const int64_t rowBytes = (int64_t)K * BITS / 8;
    const int gpr = K / a.gs;
    const uint8_t* wp[R]; const uint16_t* sp[R]; const uint16_t* bp[R];
    bool valid[R];
    int outIdx[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int part, row;
        if (gated) {
            const int o = slot0 + (r % (R / 2));
            part = r < R / 2 ? 0 : 1; row = o; valid[r] = o < a.O; outIdx[r] = o;
        } else {
            const int gr = slot0 + r;
            valid[r] = gr < a.O; outIdx[r] = gr;
            if (gr < a.o1) { part = 0; row = gr; }
            else if (gr < a.o1 + a.o2) { part = 1; row = gr - a.o1; }
            else { part = 2; row = gr - a.o1 - a.o2; }
        }
        if (!valid[r]) { part = 0; row = 0; }
        wp[r] = a.w[part] + row * rowBytes;
        sp[r] = a.s[part] + (int64_t)row * gpr;
        bp[r] = a.b[part] + (int64_t)row * gpr;
        // bias pointer reuse: keep per-row bias in outIdx decode below
        outIdx[r] = valid[r] ? outIdx[r] : -1;
        (void)part;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    const int nchunks = K >> 5;
    const int cq0 = KS ? nchunks * wave / QMV_WAVES : 0, cq1 = KS ? nchunks * (wave + 1) / QMV_WAVES : nchunks;
    for (int c = cq0 + lane; c < cq1; c += 64) {
        const int k0 = c << 5;
        uint32_t w[R][BITS];
#pragma unroll
        for (int r = 0; r < R; r++) load_chunk<BITS>(wp[r] + (int64_t)c * (4 * BITS), w[r]);
        float x[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 v = *reinterpret_cast<const float4*>(xsrc + k0 + 4 * i);
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
        float xsum = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; j++) xsum += x[j];
        const int g = k0 / a.gs;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float s = ld_scale<ST>(sp[r] + g), b = ld_scale<ST>(bp[r] + g);
            const float d = chunk_dot<BITS>(w[r], x);
            acc[r] += s * d + b * xsum;
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
    if constexpr (KS) {
        __shared__ float wred[QMV_WAVES][R];
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++) wred[wave][r] = acc[r];
        }
        __syncthreads();
        if (wave != 0 || slot0 >= a.O) return;
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = ((wred[0][r] + wred[1][r]) + wred[2][r]) + wred[3][r];
    }
    if (lane != 0) return;
    if (gated) {
#pragma unroll
        for (int r = 0; r < R / 2; r++) {
            const int o = outIdx[r];
            if (o < 0) continue;
            float g = acc[r], u = acc[r + R / 2];
            if (a.hasBias) { g += ld_scale<ST>(a.bias[0] + o); u += ld_scale<ST>(a.bias[1] + o); }
            a.y[o] = silu_mul(g, u);
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int gr = outIdx[r];
        if (gr < 0) continue;
        float v = acc[r];
        if (a.hasBias) {
            int part, row;
            if (gr < a.o1) { part = 0; row = gr; }
            else if (gr < a.o1 + a.o2) { part = 1; row = gr - a.o1; }
            else { part = 2; row = gr - a.o1 - a.o2; }
            v += ld_scale<ST>(a.bias[part] + row);
        }
        if (a.epi == EPI_ADD) a.y[gr] += v; else a.y[gr] = v;
    }
}

template <int BITS, int ST, bool XNORM>
static hipError_t qmv_launch(const QmvDev& d, bool ks, int grid, size_t lds, hipStream_t s) {
    // x staged in LDS where it fits the default 64 KiB (XNORM stages it anyway), not when the waves
    // split K (each reads a quarter of it), and at 8 bits only over many rounds of workgroups
    // (measured on the sweep cells: 4096 -> 14336 rows 13.0 -> 10.9 us at 4 bits but 20.2 -> 22.1 at 8
    // bits; the 151936-row head 120 -> 87 us at 4 bits, 211 -> 171 at 8; the split-K 14336-input cells
    // 13-19 -> 15-21 us)
    const bool xc = !XNORM && !ks && (size_t)d.K * sizeof(float) <= 65536 && (BITS < 8 || grid >= 2048);
    if (xc) lds = (size_t)d.K * sizeof(float);
    if (ks) {
        if (xc) hipLaunchKernelGGL((qmv_kernel<BITS, ST, XNORM, true, true>), dim3(grid), dim3(256), lds, s, d);
        else hipLaunchKernelGGL((qmv_kernel<BITS, ST, XNORM, true>), dim3(grid), dim3(256), lds, s, d);
    } else {
        if (xc) hipLaunchKernelGGL((qmv_kernel<BITS, ST, XNORM, false, true>), dim3(grid), dim3(256), lds, s, d);
        else hipLaunchKernelGGL((qmv_kernel<BITS, ST, XNORM, false>), dim3(grid), dim3(256), lds, s, d);
    }
    return hipGetLastError();
}

template <int BITS>
static hipError_t qmv_dispatch_st(const QmvDev& d, int st, bool xn, bool ks, int grid, size_t lds, hipStream_t s) {
    if (st == 0) return xn ? qmv_launch<BITS, 0, true>(d, ks, grid, lds, s) : qmv_launch<BITS, 0, false>(d, ks, grid, lds, s);
    return xn ? qmv_launch<BITS, 1, true>(d, ks, grid, lds, s) : qmv_launch<BITS, 1, false>(d, ks, grid, lds, s);
}

hipError_t launch_qmv(const QmvArgs& a, hipStream_t s) {
    QmvDev d{};
    for (int i = 0; i < 3; i++) {
        const QMat& m = a.part[i < a.nparts ? i : a.nparts - 1];
        d.w[i] = m.w; d.s[i] = m.s; d.b[i] = m.b; d.bias[i] = m.bias;
    }
    d.o1 = a.part[0].O; d.o2 = a.nparts > 1 ? a.part[1].O : 0;
    d.K = a.K; d.gs = a.gs; d.O = a.O; d.epi = a.epi; d.hasBias = a.part[0].bias != nullptr;
    d.x = a.x; d.norm_w = a.norm_w; d.eps = a.eps; d.y = a.y;
    // measured on the 14336-input sweep cells: 3 / 4 / 6 bits 19.3 / 18.9 / 21.1 -> 12.9 / 13.5 / 15.6 us;
    // 8-bit rows (twice the bytes per chunk, each wave's loads already busy) 18.6 -> 21.9, so not those
    const bool ks = (a.K >> 5) >= 64 * QMV_WAVES && a.bits < 8;
    const int rows = ks ? QMV_KS_ROWS : QMV_ROWS;
    const int per_wg = (ks ? 1 : QMV_WAVES) * (a.epi == EPI_GATED ? rows / 2 : rows);
    const int grid = (a.O + per_wg - 1) / per_wg;
    const bool xn = a.norm_w != nullptr;
    const size_t lds = xn ? (size_t)a.K * sizeof(float) : 0;
    switch (a.bits) {
        case 2: return qmv_dispatch_st<2>(d, a.st, xn, ks, grid, lds, s);
        case 3: return qmv_dispatch_st<3>(d, a.st, xn, ks, grid, lds, s);
        case 4: return qmv_dispatch_st<4>(d, a.st, xn, ks, grid, lds, s);
        case 5: return qmv_dispatch_st<5>(d, a.st, xn, ks, grid, lds, s);
        case 6: return qmv_dispatch_st<6>(d, a.st, xn, ks, grid, lds, s);
        case 8: return qmv_dispatch_st<8>(d, a.st, xn, ks, grid, lds, s);
    }
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------------
// Small batch (T = 2..8) on the fp32 vector units (code widths other than 4 and 8, or callers
// without the pre-pass scratch; widths 4 and 8 run on the matrix cores: qmmx_kernel). A lane holds x of its 32-code chunk for up to QMM_TP tokens in registers
// and reuses it for QMM_R rows (each row's codes converted once and dotted with every token), so x
// is loaded once per chunk per pass instead of once per row and token. More than QMM_TP tokens take
// a second pass over the same rows (their weights then come from the caches). For inputs of at
// least 64 chunks per wave the four waves split K over the same rows (partial sums added in LDS in
// wave order), else each wave takes its own rows.
constexpr int QMM_TT = 8;    // tokens (max)
constexpr int QMM_TP = 4;    // tokens per pass
constexpr int QMM_R = 8;     // rows per wave

struct QmmDev {
    const uint8_t* w[3]; const uint16_t* s[3]; const uint16_t* b[3]; const uint16_t* bias[3];
    int o1, o2, K, gs, O, T, hasBias, xs, ys;
    const float* x; float* y;
};

template <int BITS>
__device__ __forceinline__ void unpack_chunk(const uint32_t* w, float* q) {
    if constexpr (BITS == 4) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
            q[8 * i + 0] = (float)(lo & 0xFFu);         q[8 * i + 1] = (float)(hi & 0xFFu);
            q[8 * i + 2] = (float)((lo >> 8) & 0xFFu);  q[8 * i + 3] = (float)((hi >> 8) & 0xFFu);
            q[8 * i + 4] = (float)((lo >> 16) & 0xFFu); q[8 * i + 5] = (float)((hi >> 16) & 0xFFu);
            q[8 * i + 6] = (float)(lo >> 24);           q[8 * i + 7] = (float)(hi >> 24);
        }
    } else if constexpr (BITS == 8) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            q[4 * i + 0] = (float)(w[i] & 0xFFu);         q[4 * i + 1] = (float)((w[i] >> 8) & 0xFFu);
            q[4 * i + 2] = (float)((w[i] >> 16) & 0xFFu); q[4 * i + 3] = (float)(w[i] >> 24);
        }
    } else {
        constexpr uint32_t M = (1u << BITS) - 1u;
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const int bit = j * BITS, wi = bit >> 5, off = bit & 31;
            uint32_t c;
            if (off + BITS <= 32) c = (w[wi] >> off) & M;
            else c = ((w[wi] >> off) | (w[wi + 1] << (32 - off))) & M;
            q[j] = (float)c;
        }
    }
}

template <int BITS, int ST, bool KS>
__global__ __launch_bounds__(256) void qmm_small_kernel(QmmDev a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gr0 = (KS ? blockIdx.x : blockIdx.x * QMV_WAVES + wave) * QMM_R;
    if (!KS && gr0 >= a.O) return;
    const int K = a.K;
    const int64_t rowBytes = (int64_t)K * BITS / 8;
    const int gpr = K / a.gs;
    const uint8_t* wp[QMM_R]; const uint16_t* sp[QMM_R]; const uint16_t* bp[QMM_R]; int gr[QMM_R];
#pragma unroll
    for (int r = 0; r < QMM_R; r++) {
        int g = gr0 + r; gr[r] = g < a.O ? g : -1; if (g >= a.O) g = min(gr0, a.O - 1);
        int part, row;
        if (g < a.o1) { part = 0; row = g; } else if (g < a.o1 + a.o2) { part = 1; row = g - a.o1; } else { part = 2; row = g - a.o1 - a.o2; }
        wp[r] = a.w[part] + row * rowBytes; sp[r] = a.s[part] + (int64_t)row * gpr; bp[r] = a.b[part] + (int64_t)row * gpr;
    }
    const int nchunks = K >> 5;
    const int cq0 = KS ? nchunks * wave / QMV_WAVES : 0, cq1 = KS ? nchunks * (wave + 1) / QMV_WAVES : nchunks;
    __shared__ float wred[QMV_WAVES][QMM_R][QMM_TP];
    for (int t0 = 0; t0 < a.T; t0 += QMM_TP) {
        const int nt = min(QMM_TP, a.T - t0);
        float acc[QMM_R][QMM_TP];
#pragma unroll
        for (int r = 0; r < QMM_R; r++)
#pragma unroll
            for (int t = 0; t < QMM_TP; t++) acc[r][t] = 0.0f;
        for (int c = cq0 + lane; c < cq1; c += 64) {
            const int k0 = c << 5, g = k0 / a.gs;
            float x[QMM_TP][32], xsum[QMM_TP];
#pragma unroll
            for (int t = 0; t < QMM_TP; t++) {
                const float* xp = a.x + (int64_t)(t0 + min(t, nt - 1)) * a.xs + k0;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float4 v = *reinterpret_cast<const float4*>(xp + 4 * i);
                    x[t][4 * i] = v.x; x[t][4 * i + 1] = v.y; x[t][4 * i + 2] = v.z; x[t][4 * i + 3] = v.w;
                }
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < 32; j++) sum += x[t][j];
                xsum[t] = sum;
            }
#pragma unroll
            for (int r = 0; r < QMM_R; r++) {
                uint32_t w[BITS];
                load_chunk<BITS>(wp[r] + (int64_t)c * (4 * BITS), w);
                const float sc = ld_scale<ST>(sp[r] + g), bi = ld_scale<ST>(bp[r] + g);
                float q[32];
                unpack_chunk<BITS>(w, q);
#pragma unroll
                for (int t = 0; t < QMM_TP; t++) {
                    float d = 0.0f;
#pragma unroll
                    for (int j = 0; j < 32; j++) d = fmaf(q[j], x[t][j], d);
                    acc[r][t] += sc * d + bi * xsum[t];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < QMM_R; r++)
#pragma unroll
            for (int t = 0; t < QMM_TP; t++) acc[r][t] = wave_sum(acc[r][t]);
        if constexpr (KS) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < QMM_R; r++)
#pragma unroll
                    for (int t = 0; t < QMM_TP; t++) wred[wave][r][t] = acc[r][t];
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < QMM_R; r++)
#pragma unroll
                for (int t = 0; t < QMM_TP; t++) acc[r][t] = ((wred[0][r][t] + wred[1][r][t]) + wred[2][r][t]) + wred[3][r][t];
            __syncthreads();   // wred is reused by the next pass
        }
        if (lane == 0 && (!KS || wave == 0)) {
#pragma unroll
            for (int r = 0; r < QMM_R; r++) {
                if (gr[r] < 0) continue;
                float bv = 0.0f;
                if (a.hasBias) {
                    const int g = gr[r]; int part, row;
                    if (g < a.o1) { part = 0; row = g; } else if (g < a.o1 + a.o2) { part = 1; row = g - a.o1; } else { part = 2; row = g - a.o1 - a.o2; }
                    bv = ld_scale<ST>(a.bias[part] + row);
                }
#pragma unroll
                for (int t = 0; t < QMM_TP; t++)
                    if (t < nt) a.y[(int64_t)(t0 + t) * a.ys + gr[r]] = acc[r][t] + bv;
            }
        }
    }
}

hipError_t launch_qmm_small(const QmmSmallArgs& a, hipStream_t s) {
    if (a.T < 1 || a.T > QMM_TT) return hipErrorInvalidValue;
    if (a.xbf && qmmx_supported(a.K, a.bits, a.gs)) return launch_qmmx(a, s);
    QmmDev d{};
    for (int i = 0; i < 3; i++) {
        const QMat& m = a.part[i < a.nparts ? i : a.nparts - 1];
        d.w[i] = m.w; d.s[i] = m.s; d.b[i] = m.b; d.bias[i] = m.bias;
    }
    d.o1 = a.part[0].O; d.o2 = a.nparts > 1 ? a.part[1].O : 0;
    d.K = a.K; d.gs = a.gs; d.O = a.O; d.T = a.T; d.hasBias = a.part[0].bias != nullptr;
    d.xs = a.x_stride; d.ys = a.y_stride; d.x = a.x; d.y = a.y;
    const bool ks = (a.K >> 5) >= 64 * QMV_WAVES;
    const int per_wg = (ks ? 1 : QMV_WAVES) * QMM_R;
    const int grid = (a.O + per_wg - 1) / per_wg;
#define QMM_CASE(B) case B: \
    if (ks) { if (a.st == 0) hipLaunchKernelGGL((qmm_small_kernel<B, 0, true>), dim3(grid), dim3(256), 0, s, d); \
              else hipLaunchKernelGGL((qmm_small_kernel<B, 1, true>), dim3(grid), dim3(256), 0, s, d); } \
    else { if (a.st == 0) hipLaunchKernelGGL((qmm_small_kernel<B, 0, false>), dim3(grid), dim3(256), 0, s, d); \
           else hipLaunchKernelGGL((qmm_small_kernel<B, 1, false>), dim3(grid), dim3(256), 0, s, d); } \
    return hipGetLastError();
    switch (a.bits) { QMM_CASE(2) QMM_CASE(3) QMM_CASE(4) QMM_CASE(5) QMM_CASE(6) QMM_CASE(8) }
#undef QMM_CASE
    return hipErrorInvalidValue;
}

}  // namespace mlxr
