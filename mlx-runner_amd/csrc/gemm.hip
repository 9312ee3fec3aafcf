// Prefill quantized GEMM over the MLX affine layout, every code width: Y[T][O] = X[T][K] W[O][K]^T
// (+ bias), the reference's `qgemm` tiles (Kernels.swift:785-851) with fp32-level results.
//
// Arithmetic (w = s q + b per group of gs inputs):
//   y[m][n] = sum_g ( s[n][g] * sum_{k in g} q[n][k] x[m][k]  +  b[n][g] * sum_{k in g} x[m][k] )
// - The codes enter the matrix cores exactly: code q as the f16 subnormal with bit pattern q, i.e.
//   q * 2^-24 (q < 256 for every width), so no dequantization rounds anything.
// - x: each token row is multiplied by the power of two 2^e that puts max|x| in [2^13, 2^14)
//   (exact) and split into f16 hi + lo (x 2^e = hi + lo to ~2^-22 relative). Both enter the same
//   accumulator (v_mfma_f32_32x32x16_f16), so sum q x is fp32 accumulation of near-exact products.
//   A tile whose rows all have lo == 0 (inputs that are bf16 values, e.g.) skips the lo products:
//   they would add exact zeros.
// - Each quantization group accumulates in its own registers; at the group's end every output
//   takes  tot = fma(s * 2^24, acc, fma(b, xsum, tot))  in fp32, with xsum = sum of the group's
//   scaled x (the pre-pass writes it), and the row is multiplied back by 2^-e at the end.
//
// Tiling: a 256-thread workgroup owns 128 tokens x 128 rows; wave (wm, wn) the 64 x 64 quarter as
// 2 x 2 tiles of 32 x 32. K advances 64 at a time: X hi / lo and the codes (as f16) are staged in
// LDS (rows padded to 72 halves so that 32 lanes reading 16 bytes of consecutive rows spread over
// the banks), the next block's global loads are in registers while this block's MFMAs run.
// Tiles are ordered so the token tiles of one weight tile run on the same XCD (its L2).
#include "kernels.h"

namespace mlxr {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

constexpr int GX_M = 128, GX_N = 128, GX_K = 64, GX_LD = GX_K + 8;

// Pre-pass: row t of x -> hi / lo (f16, [T][K]), gsum[t][g] (sum of the scaled group, fp32, summed
// in k order per 8-chunk and chunks in order), inv[t] = 2^-e, nz[t] = any lo != 0.
__global__ __launch_bounds__(256) void x_split_kernel(const float* __restrict__ x, int xs, int K, int gs, uint16_t* __restrict__ hi,
                                                      uint16_t* __restrict__ lo, float* __restrict__ gsum, float* __restrict__ inv,
                                                      int* __restrict__ nz) {
    extern __shared__ float xsp_part[];   // K / 8 chunk sums
    __shared__ float red[4];
    __shared__ int anyl;
    const int t = blockIdx.x, tid = threadIdx.x;
    const float* row = x + (int64_t)t * xs;
    if (tid == 0) anyl = 0;
    float mx = 0.0f;
    for (int c = tid; c < K / 8; c += 256) {
        const float4 a = reinterpret_cast<const float4*>(row)[2 * c], b = reinterpret_cast<const float4*>(row)[2 * c + 1];
        mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                             fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)))));
    }
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.0f && mx <= 3.0e38f) { frexpf(mx, &e); e = 14 - e; e = e < -126 ? -126 : (e > 126 ? 126 : e); }
    const float sc = ldexpf(1.0f, e);
    if (tid == 0) inv[t] = ldexpf(1.0f, -e);
    int any = 0;
    for (int c = tid; c < K / 8; c += 256) {
        const float4 a = reinterpret_cast<const float4*>(row)[2 * c], b = reinterpret_cast<const float4*>(row)[2 * c + 1];
        const float v[8] = {a.x * sc, a.y * sc, a.z * sc, a.w * sc, b.x * sc, b.y * sc, b.z * sc, b.w * sc};
        uint32_t h[4], l[4];
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint16_t h0 = f32_to_f16(v[2 * i]), h1 = f32_to_f16(v[2 * i + 1]);
            const uint16_t l0 = f32_to_f16(v[2 * i] - f16_to_f32(h0)), l1 = f32_to_f16(v[2 * i + 1] - f16_to_f32(h1));
            h[i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            l[i] = (uint32_t)l0 | ((uint32_t)l1 << 16);
            any |= (l[i] & 0x7FFF7FFFu) != 0;
        }
#pragma unroll
        for (int i = 0; i < 8; i++) sum += v[i];
        reinterpret_cast<uint4*>(hi + (int64_t)t * K)[c] = uint4{h[0], h[1], h[2], h[3]};
        reinterpret_cast<uint4*>(lo + (int64_t)t * K)[c] = uint4{l[0], l[1], l[2], l[3]};
        xsp_part[c] = sum;
    }
    if (any) anyl = 1;
    __syncthreads();
    const int cpg = gs >> 3, G = K / gs;
    for (int g = tid; g < G; g += 256) {
        float s = 0.0f;
        for (int c = 0; c < cpg; c++) s += xsp_part[g * cpg + c];
        gsum[(int64_t)t * G + g] = s;
    }
    if (tid == 0) nz[t] = anyl;
}

struct QGemmXDev {
    const uint8_t* w; const uint16_t* s; const uint16_t* b; const uint16_t* bias;
    int K, gs, O, T, ys, nT, ntiles;
    const uint16_t* xh; const uint16_t* xl; const float* gsum; const float* inv; const int* nz;
    float* y;
    float* split;             // split over K (gridDim.y slices): tile counters, then the slices' partial tiles
};

typedef uint32_t gx_u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 gload_u4(const void* p) {
    const gx_u4 v = gload(reinterpret_cast<const gx_u4*>(p));
    return uint4{v.x, v.y, v.z, v.w};
}
template <int BITS>
__device__ __forceinline__ void load_codes32(const uint8_t* p, uint32_t* w) {
    if constexpr (BITS == 4) {
        const uint4 v = gload_u4(p);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (BITS == 8) {
        const uint4 a = gload_u4(p), b = gload_u4(p + 16);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < BITS; i++) w[i] = gload(reinterpret_cast<const uint32_t*>(p) + i);
    }
}
// code j (0..31) of a 32-code run held in BITS words (little-endian bit stream)
template <int BITS>
__device__ __forceinline__ uint32_t code_of(const uint32_t* w, int j) {
    constexpr uint32_t M = (1u << BITS) - 1u;
    const int bit = j * BITS, wi = bit >> 5, off = bit & 31;
    if (off + BITS <= 32) return (w[wi] >> off) & M;
    return ((w[wi] >> off) | (w[wi + 1] << (32 - off))) & M;
}

// K slices: 4 fixed slices (whole blocks, at group boundaries) for inputs of at least 128 blocks
// whose group size divides 64 or is a multiple of it; 1 otherwise. The slice count depends on K and
// gs alone, so a token's result never depends on T or on how the slices are spread over workgroups.
__host__ __device__ constexpr int qgemm_slices(int K, int gs) {
    return (K / GX_K >= 128 && (64 % gs == 0 || gs % 64 == 0)) ? 4 : 1;
}

template <int BITS, int ST, int SF>
__global__ __launch_bounds__(256, 2) void qgemmx_kernel(QGemmXDev a) {
    __shared__ __attribute__((aligned(16))) uint16_t Xh[GX_M * GX_LD];
    __shared__ __attribute__((aligned(16))) uint16_t Xl[GX_M * GX_LD];
    __shared__ __attribute__((aligned(16))) uint16_t Wq[GX_N * GX_LD];
    __shared__ __attribute__((aligned(16))) float Gs[2][GX_M];
    __shared__ float Ss[2][GX_N], Bs[2][GX_N];   // [flush point][row]: s * 2^24, b
    __shared__ int lo_any;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // XCD x runs workgroups x, x + 8, ...: give it a contiguous run of tiles, token tiles fastest
    const int g = blockIdx.x, xcd = g & 7, per = a.ntiles >> 3, rem = a.ntiles & 7;
    const int tile = xcd * per + min(xcd, rem) + (g >> 3);
    const int ot = tile / a.nT, tt = tile - ot * a.nT;
    const int n0 = ot * GX_N, m0 = tt * GX_M;
    const int K = a.K, gs = a.gs, G = K / gs;
    const int64_t rowBytes = (int64_t)K * BITS / 8;
    if (tid == 0) lo_any = 0;
    __syncthreads();
    if (tid < GX_M && m0 + tid < a.T && gload(a.nz + m0 + tid)) lo_any = 1;
    __syncthreads();
    const bool has_lo = lo_any != 0;
    // load roles: row lr of the tile, half lh (32 of the block's 64 k)
    const int lr = tid >> 1, lh = tid & 1;
    const int xm = min(m0 + lr, a.T - 1);
    const bool xvalid = m0 + lr < a.T;
    const uint16_t* xhrow = a.xh + (int64_t)xm * K + lh * 32;
    const uint16_t* xlrow = a.xl + (int64_t)xm * K + lh * 32;
    const int wrow = min(n0 + lr, a.O - 1);
    const uint8_t* wptr = a.w + wrow * rowBytes + lh * (4 * BITS);
    // group-sum loads: token gt of the tile for flush point gf (the block's k = 32 or 64); the same
    // thread loads row gt's scale and bias of that group
    const int gt = tid & 127, gf = tid >> 7;
    const float* gsrow = a.gsum + (int64_t)min(m0 + gt, a.T - 1) * G;
    const int64_t srow = (int64_t)min(n0 + gt, a.O - 1) * G;

    f32x16_t acc[2][2], tot[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) { acc[i][j] = (f32x16_t)0.0f; tot[i][j] = (f32x16_t)0.0f; }

    const int nblk = K / GX_K;
    const int unit = gs > GX_K ? gs / GX_K : 1;      // slice boundaries fall on group boundaries
    const int nunits = nblk / unit, z = blockIdx.y, S = gridDim.y;
    const int sl0 = z * SF / S, sl1 = (z + 1) * SF / S;

    // block kb's global data in registers
    uint4 xhr[4], xlr[4];
    uint32_t wr[BITS];
    float gsr, ssr, bsr;
    auto fetch = [&](int kb) {
        const int k0 = kb * GX_K;
        const uint4* ph = reinterpret_cast<const uint4*>(xhrow + k0);
        const uint4* pl = reinterpret_cast<const uint4*>(xlrow + k0);
#pragma unroll
        for (int v = 0; v < 4; v++) xhr[v] = xvalid ? gload_u4(ph + v) : uint4{0, 0, 0, 0};
        if (has_lo) {
#pragma unroll
            for (int v = 0; v < 4; v++) xlr[v] = xvalid ? gload_u4(pl + v) : uint4{0, 0, 0, 0};
        }
        load_codes32<BITS>(wptr + (int64_t)kb * (8 * BITS), wr);
        const int kend = k0 + 32 * (gf + 1);
        if (kend % gs == 0) {
            const int gg = kend / gs - 1;
            gsr = gload(gsrow + gg);
            ssr = ld_scale<ST>(a.s + srow + gg) * 16777216.0f;
            bsr = ld_scale<ST>(a.b + srow + gg);
        }
    };
    for (int sl = sl0; sl < sl1; sl++) {
        const int kb0 = nunits * sl / SF * unit, kb1 = nunits * (sl + 1) / SF * unit;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) { acc[i][j] = (f32x16_t)0.0f; tot[i][j] = (f32x16_t)0.0f; }
        fetch(kb0);
        for (int kb = kb0; kb < kb1; kb++) {
            const int k0 = kb * GX_K;
            {
                uint4* dh = reinterpret_cast<uint4*>(Xh + lr * GX_LD + lh * 32);
#pragma unroll
                for (int v = 0; v < 4; v++) dh[v] = xhr[v];
                if (has_lo) {
                    uint4* dl = reinterpret_cast<uint4*>(Xl + lr * GX_LD + lh * 32);
#pragma unroll
                    for (int v = 0; v < 4; v++) dl[v] = xlr[v];
                }
                // the 32 codes as f16 bit patterns (subnormals q * 2^-24)
                uint32_t p[16];
#pragma unroll
                for (int j = 0; j < 16; j++) p[j] = code_of<BITS>(wr, 2 * j) | (code_of<BITS>(wr, 2 * j + 1) << 16);
                uint4* dw = reinterpret_cast<uint4*>(Wq + lr * GX_LD + lh * 32);
#pragma unroll
                for (int v = 0; v < 4; v++) dw[v] = uint4{p[4 * v], p[4 * v + 1], p[4 * v + 2], p[4 * v + 3]};
                Gs[gf][gt] = gsr;
                Ss[gf][gt] = ssr;
                Bs[gf][gt] = bsr;
            }
            __syncthreads();
            if (kb + 1 < kb1) fetch(kb + 1);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                __builtin_amdgcn_sched_barrier(0);   // one k-step's fragments live at a time
                const int ko = ks * 16 + 8 * (lane >> 5);
                half8_t ah[2], al[2], bw[2];
#pragma unroll
                for (int i = 0; i < 2; i++) ah[i] = *reinterpret_cast<const half8_t*>(Xh + (wm * 64 + i * 32 + (lane & 31)) * GX_LD + ko);
#pragma unroll
                for (int j = 0; j < 2; j++) bw[j] = *reinterpret_cast<const half8_t*>(Wq + (wn * 64 + j * 32 + (lane & 31)) * GX_LD + ko);
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bw[j], acc[i][j], 0, 0, 0);
                if (has_lo) {
#pragma unroll
                    for (int i = 0; i < 2; i++) al[i] = *reinterpret_cast<const half8_t*>(Xl + (wm * 64 + i * 32 + (lane & 31)) * GX_LD + ko);
#pragma unroll
                    for (int i = 0; i < 2; i++)
#pragma unroll
                        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bw[j], acc[i][j], 0, 0, 0);
                }
                if (ks & 1) {
                    const int f = ks >> 1;
                    if ((k0 + 32 * (f + 1)) % gs == 0) {
                        // group end: tot = fma(s 2^24, acc, fma(b, xsum, tot)); lane's token of
                        // register r in tile i: 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4
#pragma unroll
                        for (int i = 0; i < 2; i++) {
                            float4 xg[4];
#pragma unroll
                            for (int q = 0; q < 4; q++)
                                xg[q] = *reinterpret_cast<const float4*>(&Gs[f][wm * 64 + i * 32 + 8 * q + 4 * (lane >> 5)]);
#pragma unroll
                            for (int j = 0; j < 2; j++) {
                                const int nr = wn * 64 + j * 32 + (lane & 31);
                                const float sv = Ss[f][nr], bv = Bs[f][nr];
#pragma unroll
                                for (int r = 0; r < 16; r++) {
                                    const float xv = r % 4 == 0 ? xg[r / 4].x : r % 4 == 1 ? xg[r / 4].y : r % 4 == 2 ? xg[r / 4].z : xg[r / 4].w;
                                    tot[i][j][r] = fmaf(sv, acc[i][j][r], fmaf(bv, xv, tot[i][j][r]));
                                    acc[i][j][r] = 0.0f;
                                }
                            }
                        }
                    }
                }
            }
            __syncthreads();
        }
        if (sl1 - sl0 > 1) {
            // one workgroup walks several slices: the running sum of the finished slices waits in
            // the thread's own output elements (the same order of additions as the split launch).
            // The lane index is made opaque here so that the output addresses are computed in
            // place rather than kept live across the K loop.
            int ol = lane;
            asm volatile("" : "+v"(ol));
            const bool first = sl == sl0, lastsl = sl + 1 == sl1;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = n0 + wn * 64 + j * 32 + (ol & 31);
                if (n >= a.O) continue;
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (ol >> 5) + (r & 3);
                        if (m >= a.T) continue;
                        float* yp = a.y + (int64_t)m * a.ys + n;
                        if (!first) tot[i][j][r] = *yp + tot[i][j][r];
                        if (!lastsl) *yp = tot[i][j][r];
                    }
            }
        }
    }
    if (S > 1) {
        // this slice's partial tile (coherent stores), then the tile's counter; the last slice adds
        // the slices in order (deterministic) and writes the output
        unsigned* cnt = reinterpret_cast<unsigned*>(a.split);
        float* part = a.split + QGEMM_SPLIT_TILES;
        auto pidx = [&](int zz, int i, int j, int r) {   // [slice][tile][thread][64 values]
            return (((size_t)zz * a.ntiles + tile) * 256 + tid) * 64 + (i * 2 + j) * 16 + r;
        };
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) __hip_atomic_store(part + pidx(z, i, j, r), tot[i][j][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        __shared__ int last;
        if (tid == 0) last = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
        __syncthreads();
        if (!last) return;
        if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    float v = __hip_atomic_load(part + pidx(0, i, j, r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    for (int zz = 1; zz < S; zz++) v += __hip_atomic_load(part + pidx(zz, i, j, r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    tot[i][j][r] = v;
                }
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        if (n >= a.O) continue;
        const float bias = a.bias ? ld_scale<ST>(a.bias + n) : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < a.T) a.y[(int64_t)m * a.ys + n] = tot[i][j][r] * a.inv[m] + bias;
            }
    }
}

// ---------------------------------------------------------------------------------------------
// The tile GEMM's operand pre-pass (f16, per-row power-of-two scale; used by ptile.hip's launcher).
__global__ __launch_bounds__(256) void x_to_f16_kernel(const float* x, int xs, int K, uint16_t* out, float* inv) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float* row = x + (int64_t)t * xs;
    float mx = 0.0f;
    for (int g = tid; g < K / 8; g += 256) {
        const float4 a = reinterpret_cast<const float4*>(row)[2 * g], b = reinterpret_cast<const float4*>(row)[2 * g + 1];
        mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                             fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)))));
    }
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.0f && mx <= 3.0e38f) { frexpf(mx, &e); e = 14 - e; e = e < -126 ? -126 : (e > 126 ? 126 : e); }
    const float sc = ldexpf(1.0f, e);
    if (tid == 0) inv[t] = ldexpf(1.0f, -e);
    for (int g = tid; g < K / 8; g += 256) {
        const float4 a = reinterpret_cast<const float4*>(row)[2 * g], b = reinterpret_cast<const float4*>(row)[2 * g + 1];
        uint4 o;
        o.x = (uint32_t)f32_to_f16(a.x * sc) | ((uint32_t)f32_to_f16(b.x * sc) << 16);
        o.y = (uint32_t)f32_to_f16(a.y * sc) | ((uint32_t)f32_to_f16(b.y * sc) << 16);
        o.z = (uint32_t)f32_to_f16(a.z * sc) | ((uint32_t)f32_to_f16(b.z * sc) << 16);
        o.w = (uint32_t)f32_to_f16(a.w * sc) | ((uint32_t)f32_to_f16(b.w * sc) << 16);
        reinterpret_cast<uint4*>(out + (int64_t)t * K)[g] = o;
    }
}

hipError_t launch_x_to_f16(const float* x, int xs, int K, int T, uint16_t* out, float* inv, hipStream_t s) {
    if (K % 8 || xs % 4 || T < 1) return hipErrorInvalidValue;
    if (launch_row_f16(x, xs, K, T, out, inv, s)) return hipGetLastError();
    hipLaunchKernelGGL(x_to_f16_kernel, dim3(T), dim3(256), 0, s, x, xs, K, out, inv);
    return hipGetLastError();
}


hipError_t launch_qgemm(const QGemmArgs& a, hipStream_t s) {
    if (a.K % GX_K || a.gs % 32 || a.K % a.gs || a.T < 1 || !a.xbf || !a.xlo || !a.xgs || !a.xsc || !a.xnz) return hipErrorInvalidValue;
    if (!a.x_ready) {
        hipLaunchKernelGGL(x_split_kernel, dim3(a.T), dim3(256), (size_t)(a.K / 8) * 4, s, a.x, a.x_stride, a.K, a.gs, a.xbf,
                           a.xlo, a.xgs, a.xsc, a.xnz);
        if (hipError_t e = hipGetLastError()) return e;
    }
    const int nT = (a.T + GX_M - 1) / GX_M, nO = (a.O + GX_N - 1) / GX_N, tiles = nT * nO;
    QGemmXDev d{a.m.w, a.m.s, a.m.b, a.m.bias, a.K, a.gs, a.O, a.T, a.y_stride, nT, tiles,
                a.xbf, a.xlo, a.xgs, a.xsc, a.xnz, a.y, a.split};
    dim3 grid(tiles, 1);
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidDevice;
    }
    const int SF = qgemm_slices(a.K, a.gs);
    // under one round of workgroups (two per CU): the K slices on workgroups of their own, when a
    // scratch is given
    if (SF > 1 && tiles * SF <= 2 * cus && (size_t)tiles * SF <= QGEMM_SPLIT_TILES && a.split && a.split_floats >= QGEMM_SPLIT_FLOATS)
        grid.y = SF;
#define GEMM_CASE(B) case B: \
    if (SF == 4) { if (a.st == 0) hipLaunchKernelGGL((qgemmx_kernel<B, 0, 4>), grid, dim3(256), 0, s, d); \
                   else hipLaunchKernelGGL((qgemmx_kernel<B, 1, 4>), grid, dim3(256), 0, s, d); } \
    else { if (a.st == 0) hipLaunchKernelGGL((qgemmx_kernel<B, 0, 1>), grid, dim3(256), 0, s, d); \
           else hipLaunchKernelGGL((qgemmx_kernel<B, 1, 1>), grid, dim3(256), 0, s, d); } \
    return hipGetLastError();
    switch (a.bits) { GEMM_CASE(2) GEMM_CASE(3) GEMM_CASE(4) GEMM_CASE(5) GEMM_CASE(6) GEMM_CASE(8) }
#undef GEMM_CASE
    return hipErrorInvalidValue;
}

}  // namespace mlxr
