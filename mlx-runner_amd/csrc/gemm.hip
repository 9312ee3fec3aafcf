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
// reads of 16 consecutive rows fall in different banks; the next step's global loads are issued
// into registers before the current step's MFMAs.
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
    float* split;             // split over K (gridDim.z slices): tile counters, then the slices' partial tiles
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

// K slices of the bf16 GEMM: 4 (of at least 32 steps) for inputs of 8192 or more, else 1.
__host__ __device__ constexpr int qgemm_slices(int K) { return K / GB_K >= 128 ? 4 : 1; }

template <int BITS, int ST, int SF>
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
    // K in SF fixed slices (whole GB_K steps, SF set by K alone), each accumulated from zero and the
    // slices added in order: the same arithmetic whether one workgroup walks them in turn
    // (gridDim.z == 1) or SF workgroups take one each (gridDim.z == SF, the last adding the
    // partials), so a token's result never depends on T (nor on the launch's split)
    const int nsteps = K / GB_K, z = blockIdx.z, S = gridDim.z;
    const int sl0 = z * SF / S, sl1 = (z + 1) * SF / S;
    f32x4_t tot[4][4];
    // step k0's global data in registers: X (4 x 16 bytes), the row's 32 codes and their group's
    // scale / bias. The next step's loads are issued before this step's MFMAs, so their latency
    // hides behind the compute.
    uint4 xr[4];
    uint32_t wr[BITS];
    float sr, br;
    auto fetch = [&](int k0) {
        const uint4* src = reinterpret_cast<const uint4*>(xrow + k0);
#pragma unroll
        for (int v = 0; v < 4; v++) xr[v] = xvalid ? src[v] : uint4{0, 0, 0, 0};
        load_codes32<BITS>(wptr + (int64_t)(k0 / 32) * (4 * BITS), wr);
        const int g = (k0 + lh * 32) / a.gs;
        sr = ld_scale<ST>(sp + g); br = ld_scale<ST>(bp + g);
    };
    for (int sl = sl0; sl < sl1; sl++) {
        const int kb = nsteps * sl / SF * GB_K, ke = nsteps * (sl + 1) / SF * GB_K;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        fetch(kb);
        for (int k0 = kb; k0 < ke; k0 += GB_K) {
            // X tile
            {
                uint4* dst = reinterpret_cast<uint4*>(Xs + lr * GB_LD + lh * 32);
#pragma unroll
                for (int v = 0; v < 4; v++) dst[v] = xr[v];
            }
            // W tile: 32 codes of row lr, dequantized in fp32, rounded to bf16
            {
                uint32_t packed[16];
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const float v0 = (float)code_of<BITS>(wr, 2 * j) * sr + br;
                    const float v1 = (float)code_of<BITS>(wr, 2 * j + 1) * sr + br;
                    packed[j] = (uint32_t)f32_to_bf16(v0) | ((uint32_t)f32_to_bf16(v1) << 16);
                }
                uint4* dst = reinterpret_cast<uint4*>(Ws + lr * GB_LD + lh * 32);
#pragma unroll
                for (int v = 0; v < 4; v++) dst[v] = uint4{packed[4 * v], packed[4 * v + 1], packed[4 * v + 2], packed[4 * v + 3]};
            }
            __syncthreads();
            if (k0 + GB_K < ke) fetch(k0 + GB_K);
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
        if constexpr (SF > 1) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) tot[i][j] = sl == sl0 ? acc[i][j] : tot[i][j] + acc[i][j];
        }
    }
    if constexpr (SF > 1) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = tot[i][j];
    }
    if (S > 1) {
        // this slice's partial tile (coherent stores), then the tile's counter; the last slice adds
        // the slices in order (deterministic) and writes the output
        const int tile = blockIdx.y * gridDim.x + blockIdx.x, ntiles = gridDim.x * gridDim.y;
        unsigned* cnt = reinterpret_cast<unsigned*>(a.split);
        float* part = a.split + QGEMM_SPLIT_TILES;
        auto pidx = [&](int zz, int i, int j, int r) {   // [slice][tile][16 KB: this thread's 64 values]
            return (((size_t)zz * ntiles + tile) * 256 + tid) * 64 + (i * 4 + j) * 4 + r;
        };
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) __hip_atomic_store(part + pidx(z, i, j, r), acc[i][j][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        __shared__ int last;
        if (tid == 0) last = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
        __syncthreads();
        if (!last) return;
        if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float v = __hip_atomic_load(part + pidx(0, i, j, r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    for (int zz = 1; zz < S; zz++) v += __hip_atomic_load(part + pidx(zz, i, j, r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    acc[i][j][r] = v;
                }
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

// ---------------------------------------------------------------------------------------------
// 4-bit fast path (gs 32 / 64 / 128, K % 32 == 0): f16 operands on v_mfma_f32_16x16x32_f16.
//
// X pre-pass: each token row is multiplied by a power of two 2^e that puts its largest |x| in
// [2^13, 2^14) (exact), rounded once to f16 and stored with every 8-element group in the order
// [0,4,1,5,2,6,3,7]; the output row is multiplied back by 2^-e (exact).
// W: a 32-bit word of codes holds 8 consecutive 4-bit values (element i in bits 4i..4i+3), so
// ((w >> 4p) & 0x000F000F) | 0x64006400 is the f16 pair (1024 + q_p, 1024 + q_{p+4}); subtracting
// 1024 gives q exactly and one f16 FMA gives s*q + b (rounded once to f16). The pair order matches
// the X permutation, so the dot product is over the same k.
// Tile: a 256-thread workgroup owns 128 tokens x 256 output rows; wave w the rows 64w..64w+63
// (2 W fragments of 32 rows) against all 128 tokens (4 X fragments) on v_mfma_f32_32x32x16_f16
// (the 32x32 shape: one wave per SIMD keeps it near its peak, which the 16x16 shape does not),
// so each weight is dequantized once per workgroup. K advances 128 at a time: lane (r, kh) holds
// the 32 code bytes of k in [64kh, 64kh + 64) of its row and step s (16 k) uses code word s, so
// step s covers k = 64kh + 8s + (0..7) — the X fragment reads the same k from LDS. Operands reach
// LDS through buffer -> LDS copies (no registers): the X block (128 tokens x 128 k, f16, 16-byte
// chunks XOR-swizzled by (row & 15) so fragment reads are conflict-free), each wave's code chunks
// and scale / bias words; three pipeline stages keep two blocks in flight.
// Tiles are ordered so that the workgroups one XCD runs share W tiles (dispatch puts workgroup g
// on XCD g % 8).
constexpr int Q4_M = 128, Q4_N = 256, Q4_KB = 128, Q4_NST = 3;
typedef __attribute__((address_space(3))) void* q4_lptr;

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

struct QGemm4Dev {
    const uint8_t* w; const uint16_t* s; const uint16_t* b; const uint16_t* bias;
    int K, gsh, O, T, ys, nT, ntiles;
    const uint16_t* xh; const float* inv; float* y;
};

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(1))) uint8_t* q4_gptr;
typedef uint32_t q4_u4 __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int ST> __device__ __forceinline__ half2_t q4_half2(uint16_t v) {
    _Float16 h;
    if constexpr (ST == 0) h = (_Float16)bf16_to_f32(v);
    else h = __builtin_bit_cast(_Float16, v);
    return half2_t{h, h};
}

constexpr int Q4_RSRC_W3 = 0x00020000;   // raw buffer, 32-bit data format
// LDS per pipeline stage: X block (128 tokens x 128 k, f16, 32 KB), then per wave 4 KB of codes
// (fragment f: 64 lanes x 16 B) and 1 KB of scale / bias words (fragment f: 64 lanes x 4 B).
constexpr int Q4_XB = Q4_M * 256, Q4_WB = 4 * 4096, Q4_SB = 4 * 1024;
constexpr int Q4_STAGE = Q4_XB + Q4_WB + Q4_SB;
constexpr int Q4_LOADS = 4 + 2 + 2;   // buffer -> LDS copy instructions per wave per block

template <int ST>
__global__ __launch_bounds__(512, 1) void qgemm4_kernel(QGemm4Dev a) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t q4_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // wave (wq, kc): rows n0 + 64wq .. + 63, the half kc of every block's 8 MFMA steps; the two
    // waves of a pair run on one SIMD, so one issues MFMAs while the other waits on memory
    const int wq = wave & 3, kc = wave >> 2;
    // tile order: XCD x runs workgroups x, x + 8, ...; give it a contiguous run of tiles
    const int g = blockIdx.x, xcd = g & 7, per = a.ntiles >> 3, rem = a.ntiles & 7;
    const int tile = xcd * per + min(xcd, rem) + (g >> 3);
    const int ot = tile / a.nT, tt = tile - ot * a.nT;
    const int n0 = ot * Q4_N + wq * 64, m0 = tt * Q4_M;
    const int r32 = lane & 31, kh = lane >> 5, r16 = lane & 15, kq = lane >> 4;
    const int gpr = a.K >> a.gsh, nb = (a.K + Q4_KB - 1) / Q4_KB;
    const uint32_t rowb = (uint32_t)a.K >> 1;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)a.xh, 0, a.T * a.K * 2, Q4_RSRC_W3);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, 0, a.O * (int)rowb, Q4_RSRC_W3);
    // wave pair member kc copies the scales (kc = 0) or the biases (kc = 1) of its rows
    const __amdgpu_buffer_rsrc_t sbr = __builtin_amdgcn_make_buffer_rsrc((void*)(kc ? a.b : a.s), 0, a.O * gpr * 2,
                                                                          Q4_RSRC_W3);
    // W fragment f = rows n0 + 32f .. + 31 (rows >= O read as zeros); lane (r32, kh) owns the 64
    // codes k in [64kh, 64kh + 64) of each block (two 16-byte chunks; wave kc uses chunk kc) of row
    // n0 + 32f + r32
    const uint32_t wlane = (uint32_t)(n0 + r32) * rowb + 32 * kh + 16 * kc;
    // scale / bias word d = kh of row n0 + 32f + r32 (a word = the groups 2 (g0 / 2 + d), + 1)
    const uint32_t slane = (uint32_t)(n0 + r32) * gpr * 2;
    f32x16_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int f = 0; f < 2; f++) acc[i][f] = (f32x16_t)0.0f;

    // copy q (0..7) of block blk into its pipeline stage: 0-3 X (this wave's 4 KB: rows 16w ..
    // 16w + 15, 16-byte chunks swizzled by (row & 15)), 4-5 code chunk kc of fragment q - 4 (chunks
    // past K read out of range: zeros), 6-7 scale (kc = 0) / bias (kc = 1) words of fragment q - 6
    auto issue = [&](int blk, int q) {
        uint8_t* st = q4_lds + (blk % Q4_NST) * Q4_STAGE;
        if (q < 4) {
            const int qq = wave * 4 + q, r = 4 * qq + kq;
            const uint32_t off = (uint32_t)(m0 + r) * (uint32_t)a.K * 2u + blk * 256 + 16 * (r16 ^ (r & 15));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (q4_lptr)(st + qq * 1024), 16, off, 0, 0, 0);
        } else if (q < 6) {
            const int f = q - 4;
            const bool kok = blk * Q4_KB + 64 * kh + 32 * kc < a.K;
            const uint32_t wo = kok ? wlane + blk * 64 : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (q4_lptr)(st + Q4_XB + wq * 4096 + (2 * f + kc) * 1024), 16, wo,
                                                     32 * f * rowb, 0, 0);
        } else {
            const int f = q - 6;
            const int g0 = (blk * Q4_KB) >> a.gsh, gend = min(((blk + 1) * Q4_KB) >> a.gsh, gpr);
            const int wd = (g0 >> 1) + kh;
            const uint32_t so = 2 * wd < gend ? slane + 4 * wd : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sbr, (q4_lptr)(st + Q4_XB + Q4_WB + wq * 1024 + kc * 512 + f * 256), 4,
                                                     so, 32 * f * gpr * 2, 0, 0);
        }
    };

    // this wave's half of a 128-k block: steps s = 4kc .. 4kc + 3 of 16 k on
    // v_mfma_f32_32x32x16_f16; step s uses code word s & 3 of chunk kc, i.e. k = 64kh + 8s + (0..7),
    // and the X fragment reads the same k. Step s + 1's X fragments and dequantized W are produced
    // while step s's MFMAs run.
    auto compute = [&](int blk, int pf) {
        const uint8_t* st = q4_lds + (blk % Q4_NST) * Q4_STAGE;
        const uint8_t* wst = st + Q4_XB + wq * 4096;
        const uint8_t* sst = st + Q4_XB + Q4_WB + wq * 1024;
        q4_u4 c[2];
#pragma unroll
        for (int f = 0; f < 2; f++) c[f] = *reinterpret_cast<const q4_u4*>(wst + (2 * f + kc) * 1024 + lane * 16);
        // group of the lane's 32 codes: g = (blk * 128 + 64kh + 32kc) >> gsh, stored in word
        // (g >> 1) - (g0 >> 1), half g & 1
        const int g0 = (blk * Q4_KB) >> a.gsh, gg = (blk * Q4_KB + 64 * kh + 32 * kc) >> a.gsh;
        const int so = 128 * ((gg >> 1) - (g0 >> 1)) + 4 * r32 + 2 * (gg & 1);
        half2_t s2[2], b2[2];
#pragma unroll
        for (int f = 0; f < 2; f++) {
            s2[f] = q4_half2<ST>(*reinterpret_cast<const uint16_t*>(sst + f * 256 + so));
            b2[f] = q4_half2<ST>(*reinterpret_cast<const uint16_t*>(sst + 512 + f * 256 + so));
        }
        auto dequant = [&](int j, half8_t* wf) {
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const uint32_t wv = c[f][j];
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    // (w & 0x000F000F) | 0x64006400 as one three-input bit operation
                    const uint32_t t = __builtin_amdgcn_bitop3_b32(wv >> (4 * p), 0x000F000Fu, 0x64006400u, 0xEA);
                    const half2_t q = __builtin_bit_cast(half2_t, t) - half2_t{(_Float16)1024.0f, (_Float16)1024.0f};
                    const half2_t v = q * s2[f] + b2[f];
                    wf[f][2 * p] = v[0];
                    wf[f][2 * p + 1] = v[1];
                }
            }
        };
        auto xload = [&](int j, half8_t* xf) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                xf[i] = *reinterpret_cast<const half8_t*>(st + (32 * i + r32) * 256 + 16 * ((8 * kh + 4 * kc + j) ^ r16));
        };
        half8_t xf[2][4], wf[2][2];
        xload(0, xf[0]);
        dequant(0, wf[0]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            __builtin_amdgcn_sched_barrier(0);
            // two of block pf's copies per step: while this wave waits for the memory pipeline to
            // take them, the other wave on the SIMD issues MFMAs
            if (pf >= 0) { issue(pf, 2 * j); issue(pf, 2 * j + 1); }
            if (j < 3) { xload(j + 1, xf[(j + 1) & 1]); dequant(j + 1, wf[(j + 1) & 1]); }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int f = 0; f < 2; f++)
                    acc[i][f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[j & 1][f], xf[j & 1][i], acc[i][f], 0, 0, 0);
            // order within the step: the next step's LDS reads first (a full step of MFMAs hides
            // their latency), then each MFMA followed by a share of the next step's dequant
            if (j < 3) {
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // Q4_NST-stage pipeline: block b + Q4_NST - 1 is copied while block b is computed. vmcnt
    // completes in order, so leaving Q4_LOADS * (blocks issued after b) outstanding means block b's
    // own copies are done.
    static_assert(Q4_NST == 3, "the wait below assumes one block in flight after the current one");
    for (int u = 0; u < Q4_NST - 1 && u < nb; u++)
#pragma unroll
        for (int q = 0; q < Q4_LOADS; q++) issue(u, q);
    for (int blk = 0; blk < nb; blk++) {
        if (blk + 1 < nb) __builtin_amdgcn_s_waitcnt(0x0070 | (Q4_LOADS & 15) | ((Q4_LOADS >> 4) << 14));
        else __builtin_amdgcn_s_waitcnt(0);
        // every wave's copies of block blk landed; block blk - 1 is no longer read. A bare s_barrier:
        // __syncthreads' fence would also wait for the copies still in flight.
        __builtin_amdgcn_s_barrier();
        compute(blk, blk + Q4_NST - 1 < nb ? blk + Q4_NST - 1 : -1);
    }
    // the pair's partial sums: wave kc = 1 hands its accumulators to wave kc = 0 through LDS
    // (16 KB per fragment pair, lane-major so both sides access consecutive 16-byte chunks)
    __syncthreads();
    float* red = reinterpret_cast<float*>(q4_lds) + wq * (8 * 16 * 64);
    if (kc == 1) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int f = 0; f < 2; f++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    *reinterpret_cast<float4*>(red + (((i * 2 + f) * 4 + e) * 64 + lane) * 4) =
                        float4{acc[i][f][4 * e], acc[i][f][4 * e + 1], acc[i][f][4 * e + 2], acc[i][f][4 * e + 3]};
    }
    __syncthreads();
    if (kc == 1) return;
    // lane holds, for token m0 + 32i + r32, rows n0 + 32f + 8e + 4kh + (0..3) in acc[i][f][4e .. 4e + 3]
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int n = n0 + 32 * f + 8 * e + 4 * kh;
            if (n >= a.O) continue;
            float4 bias = {0.0f, 0.0f, 0.0f, 0.0f};
            if (a.bias) {
                bias.x = ld_scale<ST>(a.bias + n);
                if (n + 1 < a.O) bias.y = ld_scale<ST>(a.bias + n + 1);
                if (n + 2 < a.O) bias.z = ld_scale<ST>(a.bias + n + 2);
                if (n + 3 < a.O) bias.w = ld_scale<ST>(a.bias + n + 3);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 32 * i + r32;
                if (m >= a.T) continue;
                const float iv = a.inv[m];
                const float4 o = *reinterpret_cast<const float4*>(red + (((i * 2 + f) * 4 + e) * 64 + lane) * 4);
                float* yp = a.y + (int64_t)m * a.ys + n;
                const float4 v = {(acc[i][f][4 * e] + o.x) * iv + bias.x, (acc[i][f][4 * e + 1] + o.y) * iv + bias.y,
                                  (acc[i][f][4 * e + 2] + o.z) * iv + bias.z, (acc[i][f][4 * e + 3] + o.w) * iv + bias.w};
                if (n + 4 <= a.O && (reinterpret_cast<uintptr_t>(yp) & 15) == 0) *reinterpret_cast<float4*>(yp) = v;
                else {
                    yp[0] = v.x;
                    if (n + 1 < a.O) yp[1] = v.y;
                    if (n + 2 < a.O) yp[2] = v.z;
                    if (n + 3 < a.O) yp[3] = v.w;
                }
            }
        }
}

hipError_t launch_x_to_f16(const float* x, int xs, int K, int T, uint16_t* out, float* inv, hipStream_t s) {
    if (K % 8 || xs % 4 || T < 1) return hipErrorInvalidValue;
    if (launch_row_f16(x, xs, K, T, out, inv, s)) return hipGetLastError();
    hipLaunchKernelGGL(x_to_f16_kernel, dim3(T), dim3(256), 0, s, x, xs, K, out, inv);
    return hipGetLastError();
}

// The f16 path copies scale / bias words (4 bytes = 2 groups) and 16-byte code chunks straight into
// LDS, so rows must start 4- and 16-byte aligned: K / gs even, aligned bases.
static bool qgemm4_eligible(const QGemmArgs& a) {
    const uintptr_t sb = reinterpret_cast<uintptr_t>(a.m.s) | reinterpret_cast<uintptr_t>(a.m.b);
    return a.bits == 4 && a.xsc && (a.gs == 32 || a.gs == 64 || a.gs == 128) && a.K % 32 == 0 && (a.K / a.gs) % 2 == 0 &&
           (sb & 3) == 0 && (reinterpret_cast<uintptr_t>(a.m.w) & 15) == 0;
}

hipError_t launch_qgemm(const QGemmArgs& a, hipStream_t s) {
    if (qgemm4_eligible(a)) {
        if (!a.x_ready)
            if (hipError_t e = launch_x_to_f16(a.x, a.x_stride, a.K, a.T, a.xbf, a.xsc, s)) return e;
        const int nT = (a.T + Q4_M - 1) / Q4_M, nO = (a.O + Q4_N - 1) / Q4_N;
        QGemm4Dev d{a.m.w, a.m.s, a.m.b, a.m.bias, a.K, a.gs == 32 ? 5 : a.gs == 64 ? 6 : 7, a.O, a.T, a.y_stride,
                    nT, nT * nO, a.xbf, a.xsc, a.y};
        static bool attr = false;
        if (!attr) {
            hipFuncSetAttribute((const void*)qgemm4_kernel<0>, hipFuncAttributeMaxDynamicSharedMemorySize, Q4_NST * Q4_STAGE);
            hipFuncSetAttribute((const void*)qgemm4_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize, Q4_NST * Q4_STAGE);
            attr = true;
        }
        if (a.st == 0) hipLaunchKernelGGL((qgemm4_kernel<0>), dim3(nT * nO), dim3(512), Q4_NST * Q4_STAGE, s, d);
        else hipLaunchKernelGGL((qgemm4_kernel<1>), dim3(nT * nO), dim3(512), Q4_NST * Q4_STAGE, s, d);
        return hipGetLastError();
    }
    const int64_t n = (int64_t)a.T * a.K;
    hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, a.x, a.x_stride, a.K, a.T, a.xbf);
    QGemmDev d{a.m.w, a.m.s, a.m.b, a.m.bias, a.K, a.gs, a.O, a.T, a.y_stride, a.xbf, a.y, a.split};
    dim3 grid((a.O + GB_N - 1) / GB_N, (a.T + GB_M - 1) / GB_M);
    {   // under one round of workgroups: the K slices on workgroups of their own (at most two
        // workgroups per CU), when a scratch is given
        static int cus = 0;
        if (!cus) {
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
                return hipErrorInvalidDevice;
        }
        const int tiles = (int)(grid.x * grid.y), SF = qgemm_slices(a.K);
        if (SF > 1 && tiles * SF <= 2 * cus && (size_t)tiles * SF <= QGEMM_SPLIT_TILES && a.split && a.split_floats >= QGEMM_SPLIT_FLOATS)
            grid.z = SF;
    }
    const bool sf4 = qgemm_slices(a.K) == 4;
#define GEMM_CASE(B) case B: \
    if (sf4) { if (a.st == 0) hipLaunchKernelGGL((qgemm_kernel<B, 0, 4>), grid, dim3(256), 0, s, d); \
               else hipLaunchKernelGGL((qgemm_kernel<B, 1, 4>), grid, dim3(256), 0, s, d); } \
    else { if (a.st == 0) hipLaunchKernelGGL((qgemm_kernel<B, 0, 1>), grid, dim3(256), 0, s, d); \
           else hipLaunchKernelGGL((qgemm_kernel<B, 1, 1>), grid, dim3(256), 0, s, d); } \
    return hipGetLastError();
    switch (a.bits) { GEMM_CASE(2) GEMM_CASE(3) GEMM_CASE(4) GEMM_CASE(5) GEMM_CASE(6) GEMM_CASE(8) }
#undef GEMM_CASE
    return hipErrorInvalidValue;
}

}  // namespace mlxr
