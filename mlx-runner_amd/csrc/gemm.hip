// Prefill quantized GEMM over the MLX affine layout, every code width: Y[T][O] = X[T][K] W[O][K]^T
// (+ bias), the reference's `qgemm` tiles (Kernels.swift:785-851) with fp32-level results.
//
// Arithmetic (w = s q + b per group of gs inputs):
//   y[m][n] = sum_g ( s[n][g] * sum_{k in g} q[n][k] x[m][k]  +  b[n][g] * sum_{k in g} x[m][k] )
// - The codes enter the matrix cores exactly: code q as the f16 subnormal with bit pattern q, i.e.
//   q * 2^-24 (q < 256 for every width), so no dequantization rounds anything.
// - x: each token row is multiplied by the power of two 2^e that puts max|x| in [2^13, 2^14)
//   (exact) and split into f16 hi + lo (x 2^e = hi + lo to ~2^-22 relative). Both enter the same
//   accumulator (v_mfma_f32_32x32x16_f16). A tile whose rows all have lo == 0 (inputs that are
//   bf16 values, e.g.) skips the lo products: they would add exact zeros.
// - Each quantization group accumulates into one of two register sets (groups alternate); once the
//   next group's first products are issued, the finished one is folded in fp32,
//   tot = fma(s 2^24, acc, tot), so the matrix cores keep working meanwhile.
// - The bias terms sum_g b[n][g] xsum[m][g] (xsum: the group's sum of scaled x, from the pre-pass)
//   go through the matrix cores too, 4 groups at a time, straight into tot: xsum as three bf16
//   parts and b as one (bf16 biases) or two (f16) bf16 parts, every product exact in fp32.
// - The row is multiplied back by 2^-e at the end.
//
// Tiling: a 512-thread workgroup owns 128 tokens x 256 rows; wave (wm, wn) the 64 x 64 block
// (2 x 2 tiles of 32 x 32) of tokens 64 wm and rows 64 wn. K advances 64 at a time through three
// LDS stages filled by buffer -> LDS copies two blocks ahead (no registers hold the prefetch):
// X hi and lo (16-byte chunks XOR-swizzled by row, so 32 lanes reading 16 bytes of consecutive
// rows spread over the banks) and the raw code bytes of the 256 rows; the scales, biases and
// token group sums of 4 groups at a time (repacked by the pre-passes so that such a chunk is a few
// KB of consecutive bytes) into two more buffers. Tiles are ordered so the token tiles of one
// weight tile run on the same XCD (its L2).
#include "kernels.h"

namespace mlxr {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 gx_bf8 __attribute__((ext_vector_type(8)));
typedef uint32_t gx_u4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* gx_lptr;
__device__ __forceinline__ uint4 gload_u4(const void* p) {
    const gx_u4 v = gload(reinterpret_cast<const gx_u4*>(p));
    return uint4{v.x, v.y, v.z, v.w};
}

constexpr int GX_M = 128, GX_N = 256, GX_K = 64, GX_NST = 3;
constexpr int GX_RSRC_W3 = 0x00020000;   // raw buffer, 32-bit data format
// stage layout (bytes): X hi, X lo, codes (256 rows x 8 BITS); after the stages two chunk buffers:
// scales [256 rows][4] f16, biases [256 rows][4] f16, token group sums [4][128 tokens] f32
constexpr int GX_XB = GX_M * GX_K * 2;
constexpr int GX_CB = GX_N * 8 * 2 + GX_M * 16;
template <int BITS> constexpr int gx_wb() { return GX_N * 8 * BITS; }
template <int BITS> constexpr int gx_stage() { return 2 * GX_XB + gx_wb<BITS>(); }
template <int BITS> constexpr int gx_lds() { return GX_NST * gx_stage<BITS>() + 2 * GX_CB; }
// s_waitcnt vmcnt(n) (n < 64), expcnt and lgkmcnt not waited for
constexpr int gx_wait_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
// groups padded to a multiple of 4 (one chunk)
__host__ __device__ constexpr int gx_gpad(int G) { return (G + 3) / 4 * 4; }

// Pre-pass: row t of x -> hi / lo (f16, [T][K]); gsum[g][t] (each group's sum of the scaled x,
// summed in k order per 8-chunk and chunks in order; zero past G); inv[t] = 2^-e, nz[t] = any
// lo != 0.
__global__ __launch_bounds__(256) void x_split_kernel(const float* __restrict__ x, int xs, int K, int gs, int T, uint16_t* __restrict__ hi,
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
    const int cpg = gs >> 3, G = K / gs, Gp = gx_gpad(G);
    for (int g = tid; g < Gp; g += 256) {
        float s = 0.0f;
        if (g < G)
            for (int c = 0; c < cpg; c++) s += xsp_part[g * cpg + c];
        gsum[(int64_t)g * T + t] = s;
    }
    if (tid == 0) nz[t] = anyl;
}

// Pre-pass: the scales and biases repacked to [Gp / 4][O][4] (s, then b; their stored 16-bit words,
// zero past G), so that 4 groups of 256 consecutive rows are 2 KB of consecutive bytes. A workgroup
// moves 64 rows x 64 groups through LDS: row-contiguous reads, chunk-contiguous writes.
__global__ __launch_bounds__(256) void scale_repack_kernel(const uint16_t* __restrict__ s, const uint16_t* __restrict__ b, int O, int G,
                                                            uint16_t* __restrict__ out) {
    __shared__ uint16_t tile[2][64][66];
    const int Gp = gx_gpad(G), nc = Gp / 4, tid = threadIdx.x;
    const int n0 = blockIdx.x * 64, g0 = blockIdx.y * 64;
#pragma unroll 4
    for (int i = 0; i < 16; i++) {
        const int idx = i * 256 + tid, r = idx >> 6, gl = idx & 63, n = n0 + r, g = g0 + gl;
        const bool in = n < O && g < G;
        tile[0][r][gl] = in ? s[(int64_t)n * G + g] : 0;
        tile[1][r][gl] = in ? b[(int64_t)n * G + g] : 0;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int idx = i * 256 + tid, cl = idx >> 6, r = idx & 63, c = g0 / 4 + cl, n = n0 + r;
        if (c >= nc || n >= O) continue;
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const uint16_t* t = &tile[p][r][4 * cl];
            reinterpret_cast<uint2*>(out)[(int64_t)p * nc * O + (int64_t)c * O + n] =
                uint2{(uint32_t)t[0] | ((uint32_t)t[1] << 16), (uint32_t)t[2] | ((uint32_t)t[3] << 16)};
        }
    }
}

struct QGemmXDev {
    const uint8_t* w; const uint16_t* sb16; const uint16_t* bias; int st;
    int K, gs, O, T, ys, nT, ntiles;
    const uint16_t* xh; const uint16_t* xl; const float* gsum; const float* inv; const int* nz;
    float* y;
    float* split;             // split over K (gridDim.y slices): tile counters, then the slices' partial tiles
};

// K slices: 4 fixed slices (whole blocks, at group boundaries) for inputs of at least 128 blocks;
// 1 otherwise. The slice count depends on K alone, so a token's result never depends on T or on
// how the slices are spread over workgroups.
__host__ __device__ constexpr int qgemm_slices(int K) { return K / GX_K >= 128 ? 4 : 1; }

// A fragment's 8 codes (codes 8 u .. 8 u + 7 of a row's block, its 8 BITS raw bytes at `row`) as
// f16 subnormals, i.e. q * 2^-24 exactly.
template <int BITS>
__device__ __forceinline__ half8_t gx_codes(const uint8_t* row, int u) {
    const int byte = u * BITS, dw = byte >> 2, sh = (byte & 3) * 8;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(row) + dw;
    if constexpr (BITS == 4) {
        // even codes' bytes and odd codes' bytes, then byte permutes into (even, odd) 16-bit pairs
        const uint32_t ev = p[0] & 0x0F0F0F0Fu, od = (p[0] >> 4) & 0x0F0F0F0Fu;
        return __builtin_bit_cast(half8_t, gx_u4{__builtin_amdgcn_perm(od, ev, 0x0C040C00u), __builtin_amdgcn_perm(od, ev, 0x0C050C01u),
                                                 __builtin_amdgcn_perm(od, ev, 0x0C060C02u), __builtin_amdgcn_perm(od, ev, 0x0C070C03u)});
    } else if constexpr (BITS == 8) {
        const uint32_t a = p[0], b = p[1];
        return __builtin_bit_cast(half8_t, gx_u4{__builtin_amdgcn_perm(0u, a, 0x0C010C00u), __builtin_amdgcn_perm(0u, a, 0x0C030C02u),
                                                 __builtin_amdgcn_perm(0u, b, 0x0C010C00u), __builtin_amdgcn_perm(0u, b, 0x0C030C02u)});
    } else {
        uint64_t v = p[0];
        if constexpr (BITS != 2) v |= (uint64_t)p[1] << 32;   // 8 BITS bits from bit sh may cross into the next dword
        v >>= sh;
        constexpr uint32_t M = (1u << BITS) - 1u;
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            q[i] = (uint32_t)((v >> (2 * i * BITS)) & M) | ((uint32_t)((v >> ((2 * i + 1) * BITS)) & M) << 16);
        return __builtin_bit_cast(half8_t, gx_u4{q[0], q[1], q[2], q[3]});
    }
}

template <int BITS, int GS, int SF, bool LO>
__device__ __forceinline__ void qgemmx_body(const QGemmXDev& a, uint8_t* lds, int tile) {
    constexpr int STG = gx_stage<BITS>();
    constexpr int NCP = 2 + (LO ? 2 : 0) + BITS;   // copies a wave issues per block (a chunk adds 1 at its blocks)
    constexpr int BPC = 4 * GS / GX_K;              // blocks per chunk of 4 groups (2, 4 or 8)
    static_assert(NCP < 64 && BPC >= 2, "pipeline");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int ot = tile / a.nT, tt = tile - ot * a.nT;
    const int n0 = ot * GX_N, m0 = tt * GX_M;
    const int K = a.K, G = K / GS, Gp = gx_gpad(G);
    constexpr int NJ = 2;                                 // 32-row tiles per wave
    const uint32_t rowb = (uint32_t)(K / 8 * BITS);     // code bytes per row
    const __amdgpu_buffer_rsrc_t xhr = __builtin_amdgcn_make_buffer_rsrc((void*)a.xh, 0, a.T * K * 2, GX_RSRC_W3);
    const __amdgpu_buffer_rsrc_t xlr = __builtin_amdgcn_make_buffer_rsrc((void*)a.xl, 0, a.T * K * 2, GX_RSRC_W3);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, 0, (int)((uint32_t)a.O * rowb), GX_RSRC_W3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc((void*)a.sb16, 0, Gp * a.O * 4, GX_RSRC_W3);
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc((void*)a.gsum, 0, Gp * a.T * 4, GX_RSRC_W3);
    uint8_t* cbuf = lds + GX_NST * STG;

    // this wave's copies of block blk into its stage (every wave issues NCP of them, in this order)
    // per-lane parts of the copies' offsets (the rest is uniform): X row lane / 8 of a copy's 8 and
    // its XOR-swizzled 16-byte chunk; codes (widths whose rows tile a copy's 64 dwords): row lane /
    // (2 BITS) of the copy's rows, dword lane % (2 BITS). Rows past T or O read past the buffer's
    // end: zeros.
    constexpr bool WTILE = 64 % (2 * BITS) == 0;
    const uint32_t xl_off = (uint32_t)(lane >> 3) * (uint32_t)K * 2u + 16u * (uint32_t)((lane & 7) ^ ((lane >> 3) & 7));
    const uint32_t wl_off = WTILE ? (uint32_t)(lane / (2 * BITS)) * rowb + 4u * (uint32_t)(lane % (2 * BITS)) : 0u;
    // this wave's copies of block blk into its stage (every wave issues NCP of them, in this order)
    auto issue = [&](int blk) {
        uint8_t* st = lds + (blk % GX_NST) * STG;
        const uint32_t k0 = (uint32_t)blk * GX_K;
        // opaque copies: each offset is one add per copy here, not a register kept across the loop
        uint32_t xo = xl_off, wo = wl_off;
        int ln = lane;
        asm volatile("" : "+v"(xo), "+v"(wo), "+v"(ln));
        // X hi (and lo): 1 KB = 8 rows of 128 bytes per copy
#pragma unroll
        for (int h = 0; h < (LO ? 2 : 1); h++)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int q = 2 * wave + c;
                const uint32_t off = xo + (((uint32_t)(m0 + 8 * q) * (uint32_t)K + k0) * 2u);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(h ? xlr : xhr, (gx_lptr)(st + h * GX_XB + q * 1024), 16, off, 0, 0, 0);
            }
        // codes: 256 B per copy, the rows' 8 BITS bytes back to back (dword d of the block: row
        // d / (2 BITS), dword d % (2 BITS))
#pragma unroll
        for (int c = 0; c < BITS; c++) {
            const int q = wave * BITS + c;
            uint32_t off;
            if constexpr (WTILE) {
                off = wo + ((uint32_t)(n0 + q * 32 / BITS) * rowb + (uint32_t)blk * (8u * BITS));
            } else {
                const int d = q * 64 + ln, r = d / (2 * BITS), dw = d - r * 2 * BITS;
                off = (uint32_t)(n0 + r) * rowb + (uint32_t)blk * (8u * BITS) + 4u * dw;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (gx_lptr)(st + 2 * GX_XB + q * 256), 4, off, 0, 0, 0);
        }
    };
    // chunk ch (groups 4 ch .. 4 ch + 3) into buffer ch & 1: 2 KB of scales, 2 KB of biases (256
    // rows x 8 bytes), 2 KB of token group sums (4 groups x 128 tokens): six 1 KB copies, waves 6
    // and 7 repeating waves 0 and 1's (the same bytes to the same place)
    auto issue_chunk1 = [&](int ch, int q) {
        uint8_t* cb = cbuf + (ch & 1) * GX_CB;
        if (q < 4) {
            const int part = q >> 1, half = q & 1;                      // scales / biases, rows 128 half ..
            const uint32_t off = (uint32_t)part * (uint32_t)Gp * (uint32_t)a.O * 2u +
                                 ((uint32_t)ch * (uint32_t)a.O + (uint32_t)n0 + 128u * half) * 8u + 16u * lane;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (gx_lptr)(cb + part * 2048 + half * 1024), 16, off, 0, 0, 0);
        } else {
            // groups 4 ch + 2 (q - 4) + (lane >> 5), tokens m0 + 4 (lane & 31) .. + 3 (rows past T
            // read out of range or junk: never used)
            const int gg = 4 * ch + 2 * (q - 4) + (lane >> 5);
            const uint32_t off = ((uint32_t)gg * (uint32_t)a.T + (uint32_t)m0 + 4u * (lane & 31)) * 4u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(gr, (gx_lptr)(cb + 4096 + (q - 4) * 1024), 16, off, 0, 0, 0);
        }
    };
    auto issue_chunk = [&](int ch) { issue_chunk1(ch, wave < 6 ? wave : wave - 6); };

    f32x16_t acc[2][2][NJ], tot[2][NJ];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) { acc[0][i][j] = (f32x16_t)0.0f; acc[1][i][j] = (f32x16_t)0.0f; tot[i][j] = (f32x16_t)0.0f; }
    const int h = lane >> 5, l31 = lane & 31;

    // folds group g, held in register set SET (= g & 1), into tot: tot = fma(s 2^24, acc, tot)
    auto fold = [&](auto SETC, int g) {
        constexpr int SET = decltype(SETC)::value;
        const uint8_t* cb = cbuf + ((g >> 2) & 1) * GX_CB;
        const int gi = g & 3;
        float sv[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int rr = wn * 64 + j * 32 + l31;
            const uint16_t s16 = *reinterpret_cast<const uint16_t*>(cb + rr * 8 + gi * 2);
            sv[j] = (a.st == 0 ? bf16_to_f32(s16) : f16_to_f32(s16)) * 16777216.0f;
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) tot[i][j][r] = fmaf(sv[j], acc[SET][i][j][r], tot[i][j][r]);
    };

    // the bias terms of chunk ch's groups in [g0, g1) on the matrix cores: sum_g b[n][g] xsum[m][g]
    // with xsum split into bf16 hi + mid + lo (truncations; exact) and b into bf16 bhi + blo (blo = 0
    // for bf16 biases; 3 bits for f16 ones), every product exact and summed in fp32.
    // 32x32x16 bf16: k 0-3 hi * bhi, 4-7 mid * bhi, 8-11 lo * bhi, 12-15 hi * blo (4 groups each);
    // f16 biases add mid * blo and lo * blo in a second product.
    auto bias_terms = [&](int ch, int g0, int g1) {
        const uint8_t* cb = cbuf + (ch & 1) * GX_CB;
        const float* xs = reinterpret_cast<const float*>(cb + 4096);
        auto tr = [](float v) { return __uint_as_float(__float_as_uint(v) & 0xFFFF0000u); };
        auto bw = [](float v) { return (uint32_t)(__float_as_uint(v) >> 16); };
        const bool f16b = a.st != 0;
        gx_u4 A1[2], A2[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int mm = wm * 64 + i * 32 + l31;
            uint32_t hi[4], md[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int g = 4 * ch + q;
                const float v = (g >= g0 && g < g1) ? xs[q * GX_M + mm] : 0.0f;
                const float vh = tr(v), r1 = v - vh, vm = tr(r1), vl = r1 - vm;
                hi[q] = bw(vh); md[q] = bw(vm); lo[q] = bw(vl);
            }
            A1[i] = h == 0 ? gx_u4{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16), md[0] | (md[1] << 16), md[2] | (md[3] << 16)}
                           : gx_u4{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16), hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
            A2[i] = h == 0 ? gx_u4{md[0] | (md[1] << 16), md[2] | (md[3] << 16), lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)}
                           : gx_u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int rr = wn * 64 + j * 32 + l31;
            const uint2 b4 = *reinterpret_cast<const uint2*>(cb + 2048 + rr * 8);
            const uint16_t bb[4] = {(uint16_t)b4.x, (uint16_t)(b4.x >> 16), (uint16_t)b4.y, (uint16_t)(b4.y >> 16)};
            uint32_t bh[4], bl[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if (!f16b) { bh[q] = bb[q]; bl[q] = 0; }
                else { const float f = f16_to_f32(bb[q]), fh = tr(f); bh[q] = bw(fh); bl[q] = bw(f - fh); }
            }
            const uint32_t ph0 = bh[0] | (bh[1] << 16), ph1 = bh[2] | (bh[3] << 16);
            const uint32_t pl0 = bl[0] | (bl[1] << 16), pl1 = bl[2] | (bl[3] << 16);
            const gx_u4 B1 = h == 0 ? gx_u4{ph0, ph1, ph0, ph1} : gx_u4{ph0, ph1, pl0, pl1};
#pragma unroll
            for (int i = 0; i < 2; i++)
                tot[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gx_bf8, A1[i]), __builtin_bit_cast(gx_bf8, B1), tot[i][j], 0, 0, 0);
            if (f16b) {
                const gx_u4 B2 = h == 0 ? gx_u4{pl0, pl1, pl0, pl1} : gx_u4{0u, 0u, 0u, 0u};
#pragma unroll
                for (int i = 0; i < 2; i++)
                    tot[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gx_bf8, A2[i]), __builtin_bit_cast(gx_bf8, B2), tot[i][j], 0, 0, 0);
            }
        }
    };

    // block blk: group g accumulates into register set g & 1 (for gs 32, the block's two parts are
    // two groups; else the block lies in one group, SB = its set, FIRST = it starts the group), the
    // group's first k-step starting from zero. Once a group's first products are issued, the
    // previous group (the other set) is folded (not before the slice's first group).
    auto compute = [&](auto SBC, auto FIRSTC, int blk, int kbfirst) {
        constexpr int SB = decltype(SBC)::value;
        constexpr bool FIRST = decltype(FIRSTC)::value;
        int ln_ = threadIdx.x & 63;
        asm volatile("" : "+v"(ln_));
        const int h = ln_ >> 5, l31 = ln_ & 31;
        const uint8_t* st = lds + (blk % GX_NST) * STG;
        const int k0 = blk * GX_K;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            __builtin_amdgcn_sched_barrier(0);
            half8_t ah[2], bw[NJ];
            auto xfrag = [&](int part) {   // part 0: hi, 1: lo
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int r = wm * 64 + i * 32 + l31, c = 2 * ks + h;
                    ah[i] = *reinterpret_cast<const half8_t*>(st + part * GX_XB + r * 128 + 16 * (c ^ (r & 7)));
                }
            };
            xfrag(0);
#pragma unroll
            for (int j = 0; j < NJ; j++) bw[j] = gx_codes<BITS>(st + 2 * GX_XB + (wn * 64 + j * 32 + l31) * (8 * BITS), 2 * ks + h);
            // a group starts at this k-step: every part for gs 32, the block's first k-step else
            const bool gstart = GS == 32 ? (ks & 1) == 0 : (ks == 0 && FIRST);
            auto mm = [&](auto SC) {
                constexpr int S = decltype(SC)::value;
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        acc[S][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bw[j], gstart ? (f32x16_t)0.0f : acc[S][i][j], 0, 0, 0);
                if constexpr (LO) {
                    xfrag(1);
#pragma unroll
                    for (int i = 0; i < 2; i++)
#pragma unroll
                        for (int j = 0; j < NJ; j++) acc[S][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bw[j], acc[S][i][j], 0, 0, 0);
                }
                if (gstart && (ks > 0 || blk > kbfirst)) fold(std::integral_constant<int, 1 - S>{}, (k0 + 16 * ks) / GS - 1);
            };
            if (GS == 32 && ks >= 2) mm(std::integral_constant<int, 1>{});
            else mm(std::integral_constant<int, GS == 32 ? 0 : SB>{});
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    const int nblk = K / GX_K;
    const int unit = GS > GX_K ? GS / GX_K : 1;      // slice boundaries fall on group boundaries
    const int nunits = nblk / unit, z = blockIdx.y, S = gridDim.y;
    const int sl0 = z * SF / S, sl1 = (z + 1) * SF / S;
    for (int sl = sl0; sl < sl1; sl++) {
        const int kb0 = nunits * sl / SF * unit, kb1 = nunits * (sl + 1) / SF * unit;
        const int g0 = kb0 * GX_K / GS, g1 = kb1 * GX_K / GS;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++) tot[i][j] = (f32x16_t)0.0f;
        // every stage and chunk buffer of the previous slice has been read (its last fold plus this barrier)
        __syncthreads();
        issue_chunk(kb0 / BPC);
        issue(kb0);
        if (kb0 + 1 < kb1) issue(kb0 + 1);
        // block kb's step; SB, FIRST: as for compute (compile-time, so the loop is unrolled by the
        // period of the register sets: 1 block for gs 32, 2 for gs 64, 4 for gs 128)
        auto step = [&](int kb, auto SBC, auto FIRSTC) {
            // this wave's copies of block kb have landed (block kb + 1's may still be in flight) ...
            if (kb + 1 < kb1) __builtin_amdgcn_s_waitcnt(gx_wait_vm(NCP));
            else __builtin_amdgcn_s_waitcnt(gx_wait_vm(0));
            // ... and every wave's. Block kb - 1's stage, which block kb + 2 overwrites, is no longer
            // read; nor the chunk buffer that block kb + 1's chunk (if it starts one) overwrites:
            // the chunk two before it ended at block kb - 2 or earlier (chunks are >= 2 blocks); its
            // bias terms ran at its first block, and a group is folded in the block after its last,
            // so in block kb - 1 or earlier. The chunk's copies precede block kb + 2's, so the wait
            // before block kb + 1 covers them.
            __builtin_amdgcn_s_barrier();
            if (kb + 1 < kb1 && (kb + 1) % BPC == 0) issue_chunk((kb + 1) / BPC);
            if (kb + 2 < kb1) issue(kb + 2);
            compute(SBC, FIRSTC, kb, kb0);
            if (kb == kb0 || kb % BPC == 0) bias_terms(kb / BPC, g0, g1);
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using TT = std::true_type;
        using FF = std::false_type;
        // register set of group g: (g - g0) & 1
        if constexpr (GS == 32) {
            for (int kb = kb0; kb < kb1; kb++) step(kb, I0{}, TT{});
        } else if constexpr (GS == 64) {
            int kb = kb0;
            for (; kb + 1 < kb1; kb += 2) { step(kb, I0{}, TT{}); step(kb + 1, I1{}, TT{}); }
            if (kb < kb1) step(kb, I0{}, TT{});
        } else {
            int kb = kb0;   // slices hold whole groups: an even number of blocks
            for (; kb + 3 < kb1; kb += 4) { step(kb, I0{}, TT{}); step(kb + 1, I0{}, FF{}); step(kb + 2, I1{}, TT{}); step(kb + 3, I1{}, FF{}); }
            if (kb < kb1) { step(kb, I0{}, TT{}); step(kb + 1, I0{}, FF{}); }
        }
        // the slice's last group
        if (GS == 32 || ((g1 - 1 - g0) & 1)) fold(std::integral_constant<int, 1>{}, g1 - 1);
        else fold(std::integral_constant<int, 0>{}, g1 - 1);
        if (sl1 - sl0 > 1) {
            // one workgroup walks several slices: the running sum of the finished slices waits in
            // the thread's own output elements (the same order of additions as the split launch:
            // (slice 0 + slice 1) + slice 2 ...). The lane index is made opaque so the output
            // addresses are computed in place rather than kept live across the K loop.
            int ol = lane;
            asm volatile("" : "+v"(ol));
            const bool firstsl = sl == sl0, lastsl = sl + 1 == sl1;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int n = n0 + wn * 64 + j * 32 + (ol & 31);
                if (n >= a.O) continue;
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (ol >> 5) + (r & 3);
                        if (m >= a.T) continue;
                        float* yp = a.y + (int64_t)m * a.ys + n;
                        if (!firstsl) tot[i][j][r] = *yp + tot[i][j][r];
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
        auto pidx = [&](int zz, int i, int j, int r) {   // [slice][tile][64 values][thread]: a wave's accesses are contiguous
            return (((size_t)zz * a.ntiles + tile) * 64 + (i * NJ + j) * 16 + r) * 512 + tid;
        };
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) __hip_atomic_store(part + pidx(z, i, j, r), tot[i][j][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        __shared__ int last;
        if (tid == 0) last = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
        __syncthreads();
        if (!last) return;
        if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // slices in order ((s0 + s1) + s2 ...); this slice's own partial from registers, every other
        // slice's 64 values loaded at once
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++) acc[1][i][j] = tot[i][j];
#pragma unroll
        for (int zz = 0; zz < SF; zz++) {
            if (zz >= S) break;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        acc[0][i][j][r] = zz == z ? acc[1][i][j][r] : __hip_atomic_load(part + pidx(zz, i, j, r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++) tot[i][j] = zz == 0 ? acc[0][i][j] : tot[i][j] + acc[0][i][j];
        }
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        if (n >= a.O) continue;
        const float bias = a.bias ? (a.st == 0 ? ld_scale<0>(a.bias + n) : ld_scale<1>(a.bias + n)) : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < a.T) a.y[(int64_t)m * a.ys + n] = tot[i][j][r] * a.inv[m] + bias;
            }
    }
}

template <int BITS, int GS, int SF>
__global__ __launch_bounds__(512, 1) void qgemmx_kernel(QGemmXDev a) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t gx_lds_base[];
    __shared__ int lo_any;
    const int tid = threadIdx.x;
    // XCD x runs workgroups x, x + 8, ...: give it a contiguous run of tiles, token tiles fastest
    const int g = blockIdx.x, xcd = g & 7, per = a.ntiles >> 3, rem = a.ntiles & 7;
    const int tile = xcd * per + min(xcd, rem) + (g >> 3);
    const int m0 = (tile % a.nT) * GX_M;
    if (tid == 0) lo_any = 0;
    __syncthreads();
    if (tid < GX_M && m0 + tid < a.T && a.nz[m0 + tid]) lo_any = 1;
    __syncthreads();
    if (lo_any) qgemmx_body<BITS, GS, SF, true>(a, gx_lds_base, tile);
    else qgemmx_body<BITS, GS, SF, false>(a, gx_lds_base, tile);
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


bool qgemm_supported(int K, int gs) { return K % GX_K == 0 && (gs == 32 || gs == 64 || gs == 128) && K % gs == 0; }

hipError_t launch_qgemm(const QGemmArgs& a, hipStream_t s) {
    if (!qgemm_supported(a.K, a.gs) || a.T < 1 || !a.xbf || !a.xlo || !a.xgs || !a.xsc || !a.xnz || !a.wsb) return hipErrorInvalidValue;
    const int G = a.K / a.gs, Gp = gx_gpad(G);
    if (!a.x_ready) {
        hipLaunchKernelGGL(x_split_kernel, dim3(a.T), dim3(256), (size_t)(a.K / 8) * 4, s, a.x, a.x_stride, a.K, a.gs, a.T, a.xbf,
                           a.xlo, a.xgs, a.xsc, a.xnz);
        if (hipError_t e = hipGetLastError()) return e;
    }
    {
        hipLaunchKernelGGL(scale_repack_kernel, dim3((unsigned)((a.m.O + 63) / 64), (unsigned)((Gp + 63) / 64)), dim3(256), 0, s, a.m.s, a.m.b,
                           a.m.O, G, a.wsb);
        if (hipError_t e = hipGetLastError()) return e;
    }
    const int nT = (a.T + GX_M - 1) / GX_M, nO = (a.O + GX_N - 1) / GX_N, tiles = nT * nO;
    QGemmXDev d{a.m.w, a.wsb, a.m.bias, a.st, a.K, a.gs, a.O, a.T, a.y_stride, nT, tiles,
                a.xbf, a.xlo, a.xgs, a.xsc, a.xnz, a.y, a.split};
    dim3 grid(tiles, 1);
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidDevice;
    }
    const int SF = qgemm_slices(a.K);
    // under one round of workgroups (one per CU): the K slices on workgroups of their own, when a
    // scratch is given
    if (SF > 1 && tiles * SF <= cus && (size_t)tiles * SF <= QGEMM_SPLIT_TILES && a.split && a.split_floats >= QGEMM_SPLIT_FLOATS)
        grid.y = SF;
    static bool attr = false;
    if (!attr) {
#define GEMM_ATTR1(B, GS) \
        for (const void* f : {(const void*)qgemmx_kernel<B, GS, 1>, (const void*)qgemmx_kernel<B, GS, 4>}) \
            if (hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, gx_lds<B>())) return e;
#define GEMM_ATTR(B) GEMM_ATTR1(B, 32) GEMM_ATTR1(B, 64) GEMM_ATTR1(B, 128)
        GEMM_ATTR(2) GEMM_ATTR(3) GEMM_ATTR(4) GEMM_ATTR(5) GEMM_ATTR(6) GEMM_ATTR(8)
#undef GEMM_ATTR
#undef GEMM_ATTR1
        attr = true;
    }
    auto go = [&](auto kern, int lds) -> hipError_t {
        hipLaunchKernelGGL(kern, grid, dim3(512), (size_t)lds, s, d);
        return hipGetLastError();
    };
#define GEMM_GS(B, GS) if (a.gs == GS) return SF == 4 ? go(qgemmx_kernel<B, GS, 4>, gx_lds<B>()) : go(qgemmx_kernel<B, GS, 1>, gx_lds<B>());
#define GEMM_CASE(B) case B: GEMM_GS(B, 32) GEMM_GS(B, 64) GEMM_GS(B, 128) break;
    switch (a.bits) { GEMM_CASE(2) GEMM_CASE(3) GEMM_CASE(4) GEMM_CASE(5) GEMM_CASE(6) GEMM_CASE(8) }
#undef GEMM_CASE
#undef GEMM_GS
    return hipErrorInvalidValue;
}

// Scratch of the MLX-layout GEMM (per call): the x pre-pass' group sums (floats) and the repacked
// scales and biases (16-bit words).
size_t qgemm_gsum_floats(int T, int K, int gs) { return (size_t)T * gx_gpad(K / gs); }
size_t qgemm_scale_halves(int O, int K, int gs) { return (size_t)2 * gx_gpad(K / gs) * O; }


// ---------------------------------------------------------------------------------------------
// Small batch (T <= 8) on the matrix cores, code widths 4 and 8: the same arithmetic as the GEMM
// above (exact codes, x as f16 hi + lo with a per-token power of two, scale and bias per group in
// fp32), shaped for a few tokens. v_mfma_f32_16x16x32_f16 with the tokens as the 16 A rows (rows
// past T zero) and 16 weight rows as the B columns, so each lane's accumulator holds its own
// weight row (its scale and bias load with its codes) for tokens 4 (lane / 16) .. + 3.
// A 1024-thread workgroup owns 16 rows; its 16 waves take a sixteenth of the groups each and add
// their partial sums in wave order. Lane quarter q takes codes GS/4 q .. + GS/4 - 1 of every
// group (the k order inside a group is free: the same for codes and x), so its codes are one
// contiguous load per group.
struct QmmXDev {
    const uint8_t* w[3]; const uint16_t* s[3]; const uint16_t* b[3]; const uint16_t* bias[3];
    int o1, o2, K, O, T, ys;
    const uint16_t* xh; const uint16_t* xl; const float* gsum; const float* inv; const int* nz; float* y;
};
constexpr int QX_WAVES = 4;

template <int BITS, int GS, int ST>
__global__ __launch_bounds__(256) void qmmx_kernel(QmmXDev a) {
    __shared__ f32x4_t red[QX_WAVES][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q = lane >> 4, T = a.T;
    const int K = a.K, G = K / GS, g0 = G * wave / QX_WAVES, g1 = G * (wave + 1) / QX_WAVES;
    const int n = blockIdx.x * 16 + l16;   // the lane's weight row
    int row = min(n, a.O - 1), part = 0;
    if (row >= a.o1) {
        if (row < a.o1 + a.o2) { part = 1; row -= a.o1; }
        else { part = 2; row -= a.o1 + a.o2; }
    }
    const uint8_t* wp = a.w[part] + (int64_t)row * (K / 8 * BITS);
    const uint16_t* sp = a.s[part] + (int64_t)row * G;
    const uint16_t* bp = a.b[part] + (int64_t)row * G;
    const bool tok = l16 < T;                                   // A row l16: a token
    const int64_t xo = (int64_t)(tok ? l16 : 0) * K;
    // any token with lo parts (the loads issued together, not one round trip per token)
    int nzv[8];
#pragma unroll
    for (int t = 0; t < 8; t++) nzv[t] = a.nz[min(t, T - 1)];
    int lo = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) lo |= nzv[t];
    constexpr int CPL = GS / 4, NS = GS / 32, DW = CPL * BITS / 32;
    constexpr int QX_NB = GS == 128 ? 2 : 4;   // groups per batch of loads
    f32x4_t tot = {0.0f, 0.0f, 0.0f, 0.0f};
    // groups in batches of QX_NB: every load of a batch is issued before any is used, so a wave
    // pays one memory round trip per batch
    for (int gb = g0; gb < g1; gb += QX_NB) {
        uint32_t cw[QX_NB][DW];
        float sv[QX_NB], bv[QX_NB], xs[QX_NB][4];
        half8_t ah[QX_NB][NS];
#pragma unroll
        for (int u = 0; u < QX_NB; u++) {
            const int g = min(gb + u, g1 - 1), k0 = g * GS + CPL * q;
            const uint32_t* cp = reinterpret_cast<const uint32_t*>(wp + k0 / 8 * BITS);
            if constexpr (DW % 4 == 0) {
#pragma unroll
                for (int i = 0; i < DW / 4; i++) {
                    const uint4 v = gload_u4(cp + 4 * i);
                    cw[u][4 * i] = v.x; cw[u][4 * i + 1] = v.y; cw[u][4 * i + 2] = v.z; cw[u][4 * i + 3] = v.w;
                }
            } else if constexpr (DW == 2) {
                const uint2 v = *reinterpret_cast<const uint2*>(cp);
                cw[u][0] = v.x; cw[u][1] = v.y;
            } else {
                cw[u][0] = cp[0];
            }
            sv[u] = ld_scale<ST>(sp + g) * 16777216.0f;
            bv[u] = ld_scale<ST>(bp + g);
#pragma unroll
            for (int i = 0; i < 4; i++) xs[u][i] = 4 * q + i < T ? a.gsum[(int64_t)g * T + 4 * q + i] : 0.0f;
#pragma unroll
            for (int st = 0; st < NS; st++)
                ah[u][st] = tok ? __builtin_bit_cast(half8_t, gload_u4(a.xh + xo + k0 + 8 * st)) : (half8_t)0;
        }
#pragma unroll
        for (int u = 0; u < QX_NB; u++) {
            if (gb + u >= g1) break;
            const int k0 = (gb + u) * GS + CPL * q;
            f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < NS; st++) {
                half8_t bw;
                if constexpr (BITS == 4) {
                    const uint32_t ev = cw[u][st] & 0x0F0F0F0Fu, od = (cw[u][st] >> 4) & 0x0F0F0F0Fu;
                    bw = __builtin_bit_cast(half8_t, gx_u4{__builtin_amdgcn_perm(od, ev, 0x0C040C00u), __builtin_amdgcn_perm(od, ev, 0x0C050C01u),
                                                           __builtin_amdgcn_perm(od, ev, 0x0C060C02u), __builtin_amdgcn_perm(od, ev, 0x0C070C03u)});
                } else {
                    const uint32_t c0 = cw[u][2 * st], c1 = cw[u][2 * st + 1];
                    bw = __builtin_bit_cast(half8_t, gx_u4{__builtin_amdgcn_perm(0u, c0, 0x0C010C00u), __builtin_amdgcn_perm(0u, c0, 0x0C030C02u),
                                                           __builtin_amdgcn_perm(0u, c1, 0x0C010C00u), __builtin_amdgcn_perm(0u, c1, 0x0C030C02u)});
                }
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[u][st], bw, acc, 0, 0, 0);
                if (lo) {
                    const half8_t al = tok ? __builtin_bit_cast(half8_t, gload_u4(a.xl + xo + k0 + 8 * st)) : (half8_t)0;
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bw, acc, 0, 0, 0);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) tot[i] = fmaf(sv[u], acc[i], fmaf(bv[u], xs[u][i], tot[i]));
        }
    }
    red[wave][lane] = tot;
    __syncthreads();
    if (wave != 0 || n >= a.O) return;
    f32x4_t sum = red[0][lane];
#pragma unroll
    for (int w = 1; w < QX_WAVES; w++) sum += red[w][lane];
    const float bias = a.bias[part] ? ld_scale<ST>(a.bias[part] + row) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = 4 * q + i;
        if (t < T) a.y[(int64_t)t * a.ys + n] = sum[i] * a.inv[t] + bias;
    }
}

// Small batch over the MLX layout with wide code loads (widths 4 and 8, groups of 8 * gs | K):
// the same operands and arithmetic as qmmx_kernel, laid out so that each lane's code load is 16
// bytes. A "span" is 64 bytes of one weight row (4 lanes x 16 bytes, 128 / BITS codes per lane);
// lane quarter q holds span bytes 16 q .. 16 q + 15, and MFMA step j takes its codes 8 j .. 8 j + 7,
// matched in the A operand by the same tokens' x at the same k. A span may hold several
// quantization groups (4-bit gs 32 / 64: lanes of one group are q, or q / 2); each group then runs
// its own MFMAs with the x of the other groups' lanes zeroed, so every accumulator holds one
// group and is folded with that group's scale and bias in fp32 (y += s 2^24 acc + b sum x).
// A batch is QY_NG groups of a row: its spans' codes, the 16-byte runs of scales and biases and
// every span's x are loaded before any is used (one memory round trip per batch); the token
// group sums sit in LDS. The x of a batch reaches LDS by buffer -> LDS copies (1 KB of 4 tokens'
// chunks per copy at 32 codes per lane, of 8 tokens' at 16; no lane loading what another lane
// loads) and the A operands are read from there. 16 rows per workgroup, the four waves on a quarter of the batches each,
// partial sums added in wave order.
template <int BITS, int GS> struct QyShape {
    static constexpr int C = BITS == 8 ? 16 : 32;        // codes per lane per span
    static constexpr int NDW = C * BITS / 32;            // their dwords (2, 3, 4 or 6)
    static constexpr int SPAN = 4 * C;                   // codes of a row per span
    static constexpr int NG = GS == 128 ? 4 : 8;         // groups per batch
    static constexpr int SPB = NG * GS / SPAN;           // spans per batch
    static constexpr int NGS = SPAN / GS;                // groups per span
    static constexpr int LPG = GS / C;                   // lane quarters per group
    static constexpr int STEPS = C / 8;                  // MFMA steps per span
};

template <int BITS, int GS, int ST, int NW, bool PF>
__global__ __launch_bounds__(64 * NW) void qmmy_kernel(QmmXDev a) {
    using S = QyShape<BITS, GS>;
    static_assert(S::SPAN >= GS && S::SPB >= 1, "span shape");
    // dynamic LDS: [G][8] token group sums (zero past T), then (32 codes per lane) each wave's x
    // buffers: per span, TT = T rounded up to 4 token rows of 256 bytes, 16-byte chunk c of token t
    // at slot c ^ t (a B-operand read of 16 tokens' same chunk hits distinct banks)
    extern __shared__ __attribute__((aligned(16))) float qy_gsum[];
    __shared__ f32x4_t red[NW][64];
    constexpr bool XL = true;                                  // x through LDS
    constexpr int NBUF = PF ? 2 : 1;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q = lane >> 4, T = a.T;
    const int K = a.K, G = K / GS, NB = G / S::NG;
    // (a span's x per token: CPS chunks of 16 bytes, RB bytes; one copy carries TPI tokens)
    constexpr int CPS = S::SPAN / 8, TPI = 64 / CPS, RB = S::SPAN * 2;
    const int TT = (T + 3) & ~3, TTX = (T + TPI - 1) / TPI * TPI, XWB = S::SPB * TTX * RB;
    uint8_t* xlds = reinterpret_cast<uint8_t*>(qy_gsum) + (size_t)(K / GS) * 32;
    for (int i = tid; i < G * 8; i += 64 * NW) {
        const int g = i >> 3, t = i & 7;
        qy_gsum[i] = t < T ? a.gsum[(int64_t)g * T + t] : 0.0f;
    }
    const int n = blockIdx.x * 16 + l16;   // the lane's weight row
    int row = min(n, a.O - 1), part = 0;
    if (row >= a.o1) {
        if (row < a.o1 + a.o2) { part = 1; row -= a.o1; }
        else { part = 2; row -= a.o1 + a.o2; }
    }
    const uint8_t* wp = a.w[part] + (int64_t)row * (K / 8 * BITS) + 4 * S::NDW * q;
    const uint16_t* sp = a.s[part] + (int64_t)row * G;
    const uint16_t* bp = a.b[part] + (int64_t)row * G;
    const int TT0 = (T + 3) & ~3;
    const int64_t xo = (int64_t)min(S::NGS == 4 ? (int)(l16 % TT0) : l16, T - 1) * K + S::C * q;   // the token of A row l16
    int nzv[8];
#pragma unroll
    for (int t = 0; t < 8; t++) nzv[t] = a.nz[min(t, T - 1)];
    int lo = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) lo |= nzv[t];
    const int gq = q / S::LPG;                                  // the lane's group within a span
    __syncthreads();
    const int b0 = NB * wave / NW, b1 = NB * (wave + 1) / NW;
    f32x4_t tot = {0.0f, 0.0f, 0.0f, 0.0f};
    // codes and scales of batch bt (every load unconditional, indices clamped: a load issued in a
    // branch would make the compiler's later waits count from zero)
    uint32_t cw[S::SPB][S::NDW];
    uint32_t sw[S::NG / 2], bw[S::NG / 2];
    auto load_w = [&](int bt) {
        bt = max(0, min(bt, NB - 1));
        const int k0 = bt * S::NG * GS;
#pragma unroll
        for (int u = 0; u < S::SPB; u++) {
            const uint8_t* p = wp + (int64_t)(k0 + u * S::SPAN) / 8 * BITS;
            if constexpr (S::NDW == 4) {
                const uint4 v = gload_u4(p);
                cw[u][0] = v.x; cw[u][1] = v.y; cw[u][2] = v.z; cw[u][3] = v.w;
            } else {
                typedef const __attribute__((address_space(1))) uint32_t* gp32;
#pragma unroll
                for (int i = 0; i < S::NDW; i++) cw[u][i] = *((gp32)p + i);
            }
        }
        if constexpr (S::NG == 8) {
            const uint4 s4 = gload_u4(sp + S::NG * bt), b4 = gload_u4(bp + S::NG * bt);
            sw[0] = s4.x; sw[1] = s4.y; sw[2] = s4.z; sw[3] = s4.w;
            bw[0] = b4.x; bw[1] = b4.y; bw[2] = b4.z; bw[3] = b4.w;
        } else {
            const uint2 s2 = *reinterpret_cast<const uint2*>(sp + S::NG * bt), b2 = *reinterpret_cast<const uint2*>(bp + S::NG * bt);
            sw[0] = s2.x; sw[1] = s2.y; bw[0] = b2.x; bw[1] = b2.y;
        }
    };
    // x of batch bt into LDS buffer buf by buffer -> LDS copies: per span and 4 tokens one 1 KB copy,
    // lane i: token 4 tq + i / 16, chunk (i & 15) ^ token (rows past T repeat row T - 1, unread)
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.xh), 0, T * K * 2, 0x00020000);
    auto dma_x = [&](int bt, int buf) {
        bt = max(0, min(bt, NB - 1));
        const int k0 = bt * S::NG * GS;
        uint8_t* rb = xlds + (size_t)(wave * NBUF + buf) * XWB;
#pragma unroll
        for (int u = 0; u < S::SPB; u++)
            for (int tq = 0; tq < TTX / TPI; tq++) {
                const int t = TPI * tq + lane / CPS, c = (lane % CPS) ^ (t & (CPS - 1));
                const uint32_t off = (uint32_t)(min(t, T - 1) * K + k0 + u * S::SPAN + 8 * c) * 2u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)(rb + (u * TTX + TPI * tq) * RB), 16, off, 0, 0, 0);
            }
    };
    // A rows: NGP = 16 / TT group slots of TT token rows; row l16 is token ta of slot pa. D rows
    // 4 q .. 4 q + 3: tokens td0 .. td0 + 3 of slot pd. One MFMA set covers NGP groups of a span.
    // (PACK: spans of four groups; otherwise one slot: row l16 is token l16, D rows tokens 4 q ..)
    constexpr bool PACK = S::NGS == 4;
    const int NGP = PACK ? 16 / TT : 1, pa = PACK ? l16 / TT : 0, ta = PACK ? l16 % TT : l16;
    const int pd = PACK ? (4 * q) / TT : 0, td0 = PACK ? (4 * q) % TT : 4 * q;
    const bool tva = ta < T;
    const int mr = min(ta, TTX - 1);
    if constexpr (PF) {
        load_w(b0);
        if constexpr (XL) dma_x(b0, 0);
    }
    for (int bt = b0; bt < b1; bt++) {
        const int k0 = bt * S::NG * GS;
        if constexpr (!PF) {
            load_w(bt);
            if constexpr (XL) dma_x(bt, 0);
        }
        half8_t xv[S::SPB][S::STEPS];
        if constexpr (XL) {
            // this batch's copies (and codes) have landed
            __builtin_amdgcn_s_waitcnt(0x0F70);
            asm volatile("" ::: "memory");
            const uint8_t* rb = xlds + (size_t)(wave * NBUF + (PF ? (bt - b0) & 1 : 0)) * XWB;
#pragma unroll
            for (int u = 0; u < S::SPB; u++)
#pragma unroll
                for (int j = 0; j < S::STEPS; j++) {
                    const half8_t v = *reinterpret_cast<const half8_t*>(rb + (u * TTX + mr) * RB + (((S::C / 8) * q + j) ^ (mr & (CPS - 1))) * 16);
                    xv[u][j] = tva ? v : (half8_t)0;
                }
        } else {
#pragma unroll
            for (int u = 0; u < S::SPB; u++)
#pragma unroll
                for (int j = 0; j < S::STEPS; j++) {
                    const half8_t v = __builtin_bit_cast(half8_t, gload_u4(a.xh + xo + k0 + u * S::SPAN + 8 * j));
                    xv[u][j] = tva ? v : (half8_t)0;
                }
        }
        // this batch's codes and scales into their own registers; with PF (waves of three or more
        // batches) the next batch's stream in behind
        uint32_t cur[S::SPB][S::NDW];
        uint32_t scur[S::NG / 2], bcur[S::NG / 2];
#pragma unroll
        for (int u = 0; u < S::SPB; u++)
#pragma unroll
            for (int i = 0; i < S::NDW; i++) cur[u][i] = cw[u][i];
#pragma unroll
        for (int i = 0; i < S::NG / 2; i++) { scur[i] = sw[i]; bcur[i] = bw[i]; }
        if constexpr (PF) {
            load_w(bt + 1);
            if constexpr (XL) dma_x(bt + 1, (bt + 1 - b0) & 1);
        }
#pragma unroll
        for (int u = 0; u < S::SPB; u++) {
#define cd cur[u]
            half8_t wv[S::STEPS], xl[S::STEPS];
#pragma unroll
            for (int j = 0; j < S::STEPS; j++) {
                if constexpr (BITS == 4) {
                    const uint32_t ev = cd[j] & 0x0F0F0F0Fu, od = (cd[j] >> 4) & 0x0F0F0F0Fu;
                    wv[j] = __builtin_bit_cast(half8_t, gx_u4{__builtin_amdgcn_perm(od, ev, 0x0C040C00u), __builtin_amdgcn_perm(od, ev, 0x0C050C01u),
                                                              __builtin_amdgcn_perm(od, ev, 0x0C060C02u), __builtin_amdgcn_perm(od, ev, 0x0C070C03u)});
                } else if constexpr (BITS == 8) {
                    const uint32_t c0 = cd[2 * j], c1 = cd[2 * j + 1];
                    wv[j] = __builtin_bit_cast(half8_t, gx_u4{__builtin_amdgcn_perm(0u, c0, 0x0C010C00u), __builtin_amdgcn_perm(0u, c0, 0x0C030C02u),
                                                              __builtin_amdgcn_perm(0u, c1, 0x0C010C00u), __builtin_amdgcn_perm(0u, c1, 0x0C030C02u)});
                } else {
                    // codes 8 j .. 8 j + 7: bits 8 BITS j .. + 8 BITS of the lane's little-endian stream
                    const int b = 8 * BITS * j, i0 = b >> 5, sh = b & 31;
                    const uint64_t w = ((uint64_t)(i0 + 1 < S::NDW ? cd[i0 + 1] : 0u) << 32 | cd[i0]) >> sh;
                    constexpr uint32_t m = (1u << BITS) - 1;
                    uint32_t h[4];
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        h[e] = ((uint32_t)(w >> (2 * e * BITS)) & m) | (((uint32_t)(w >> ((2 * e + 1) * BITS)) & m) << 16);
                    wv[j] = __builtin_bit_cast(half8_t, gx_u4{h[0], h[1], h[2], h[3]});
                }
                xl[j] = (half8_t)0;
                if (lo && tva) xl[j] = __builtin_bit_cast(half8_t, gload_u4(a.xl + xo + k0 + u * S::SPAN + 8 * j));
            }
#undef cd
#pragma unroll
            for (int set = 0; set < S::NGS; set++) {
                if (PACK && set * NGP >= S::NGS) break;
                // A row l16 carries group set * NGP + pa: the x of the lanes holding that group's codes
                const bool mine = S::NGS == 1 || set * NGP + pa == gq;
                f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < S::STEPS; j++) {
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(mine ? xv[u][j] : (half8_t)0, wv[j], acc, 0, 0, 0);
                    if (lo) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(mine ? xl[j] : (half8_t)0, wv[j], acc, 0, 0, 0);
                }
                // this lane's D rows: group set * NGP + pd of the span, tokens td0 ..
                const int gs_ = set * NGP + pd;
                const bool live = !PACK || gs_ < S::NGS;
                const int gb = u * S::NGS + min(gs_, S::NGS - 1);   // group within the batch
                uint32_t sd = scur[0], bd = bcur[0];
                if constexpr (PACK) {
#pragma unroll
                    for (int i = 1; i < S::NG / 2; i++)
                        if ((gb >> 1) == i) { sd = scur[i]; bd = bcur[i]; }
                } else {
                    sd = scur[gb >> 1]; bd = bcur[gb >> 1];
                }
                const uint32_t sr = (sd >> (16 * (gb & 1))) & 0xFFFFu, br = (bd >> (16 * (gb & 1))) & 0xFFFFu;
                const float sv = live ? (ST == 0 ? __uint_as_float(sr << 16) : f16_to_f32((uint16_t)sr)) * 16777216.0f : 0.0f;
                const float bv = live ? (ST == 0 ? __uint_as_float(br << 16) : f16_to_f32((uint16_t)br)) : 0.0f;
                const f32x4_t xs = *reinterpret_cast<const f32x4_t*>(qy_gsum + (bt * S::NG + gb) * 8 + td0);
#pragma unroll
                for (int i = 0; i < 4; i++) tot[i] = fmaf(sv, acc[i], fmaf(bv, xs[i], tot[i]));
            }
        }
    }
    red[wave][lane] = tot;
    __syncthreads();
    // the lanes of slot 0 add every wave's and every slot's partial sums of their tokens, in order
    if (wave != 0 || pd != 0 || n >= a.O) return;
    f32x4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < NW; w++)
        for (int p = 0; p < NGP; p++) sum += red[w][lane + 16 * p * (TT / 4)];
    const float bias = a.bias[part] ? ld_scale<ST>(a.bias[part] + row) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = td0 + i;
        if (t < T) a.y[(int64_t)t * a.ys + n] = sum[i] * a.inv[t] + bias;
    }
}

// qmmy_kernel's shapes: widths 2 / 3 / 4 / 6 at gs 32 / 64 / 128, 8-bit at gs 32 / 64; K a multiple of
// a batch; the group sums' LDS within 64 KiB
static bool qmmy_supported(int K, int bits, int gs) {
    const bool b32 = bits == 2 || bits == 3 || bits == 4 || bits == 6;   // 32 codes per lane
    if (!((b32 && (gs == 32 || gs == 64 || gs == 128)) || (bits == 8 && (gs == 32 || gs == 64)))) return false;
    const int ng = gs == 128 ? 4 : 8;
    return K % (ng * gs) == 0 && (size_t)(K / gs) * 32 <= 65536;
}

bool qmmx_supported(int K, int bits, int gs) {
    if (qmmy_supported(K, bits, gs)) return true;
    return (bits == 4 || bits == 8) && (gs == 32 || gs == 64 || gs == 128) && K % gs == 0 && K % 32 == 0;
}

hipError_t launch_qmmx(const QmmSmallArgs& a, hipStream_t s) {
    if (!qmmx_supported(a.K, a.bits, a.gs) || a.T < 1 || a.T > 8 || !a.xbf || !a.xlo || !a.xgs || !a.xsc || !a.xnz)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(x_split_kernel, dim3(a.T), dim3(256), (size_t)(a.K / 8) * 4, s, a.x, a.x_stride, a.K, a.gs, a.T, a.xbf, a.xlo,
                       a.xgs, a.xsc, a.xnz);
    if (hipError_t e = hipGetLastError()) return e;
    QmmXDev d{};
    for (int i = 0; i < 3; i++) {
        const QMat& m = a.part[i < a.nparts ? i : a.nparts - 1];
        d.w[i] = m.w; d.s[i] = m.s; d.b[i] = m.b; d.bias[i] = m.bias;
    }
    d.o1 = a.part[0].O; d.o2 = a.nparts > 1 ? a.part[1].O : 0;
    d.K = a.K; d.O = a.O; d.T = a.T; d.ys = a.y_stride;
    d.xh = a.xbf; d.xl = a.xlo; d.gsum = a.xgs; d.inv = a.xsc; d.nz = a.xnz; d.y = a.y;
    const dim3 grid((unsigned)((a.O + 15) / 16));
    if (qmmy_supported(a.K, a.bits, a.gs)) {
        // eight waves (an eighth of the batches each) where a quarter of the batches would be a
        // long chain per wave; the next batch's loads in flight behind each batch where a wave has
        // three or more; LDS: group sums, then (32 codes per lane) every wave's x buffers
        const int ng = a.gs == 128 ? 4 : 8, nb = a.K / a.gs / ng;
        bool w8 = nb >= 16, pf = nb / (w8 ? 8 : 4) >= 3;
        const int C = a.bits == 8 ? 16 : 32, spb = ng * a.gs / (4 * C), tpi = 64 / (C / 2), tt = (a.T + tpi - 1) / tpi * tpi;
        auto lds_of = [&](bool w, bool p) {
            return (size_t)(a.K / a.gs) * 32 + (size_t)(w ? 8 : 4) * (p ? 2 : 1) * spb * tt * (8 * C);
        };
        // (160 KiB of LDS less the 8 KiB of the waves' partial sums)
        constexpr size_t QY_LDS_MAX = 152 * 1024;
        if (lds_of(w8, pf) > QY_LDS_MAX) w8 = pf = false;
        const size_t lds = lds_of(w8, pf);
        if (lds > QY_LDS_MAX) return hipErrorInvalidValue;
        static bool attr = false;
        if (!attr) {
#define QMMY_ATTR1(B, GS, ST) \
            for (const void* f : {(const void*)qmmy_kernel<B, GS, ST, 8, true>, (const void*)qmmy_kernel<B, GS, ST, 8, false>, \
                                  (const void*)qmmy_kernel<B, GS, ST, 4, false>}) \
                if (hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)QY_LDS_MAX)) return e;
#define QMMY_ATTR(B) QMMY_ATTR1(B, 32, 0) QMMY_ATTR1(B, 64, 0) QMMY_ATTR1(B, 128, 0) QMMY_ATTR1(B, 32, 1) QMMY_ATTR1(B, 64, 1) QMMY_ATTR1(B, 128, 1)
            QMMY_ATTR(2) QMMY_ATTR(3) QMMY_ATTR(4) QMMY_ATTR(6)
            QMMY_ATTR1(8, 32, 0) QMMY_ATTR1(8, 64, 0) QMMY_ATTR1(8, 32, 1) QMMY_ATTR1(8, 64, 1)
#undef QMMY_ATTR
#undef QMMY_ATTR1
            attr = true;
        }
#define QMMY_GO(B, GS) if (a.bits == B && a.gs == GS) { \
        if (w8 && pf) { \
            if (a.st == 0) hipLaunchKernelGGL((qmmy_kernel<B, GS, 0, 8, true>), grid, dim3(512), lds, s, d); \
            else hipLaunchKernelGGL((qmmy_kernel<B, GS, 1, 8, true>), grid, dim3(512), lds, s, d); \
        } else if (w8) { \
            if (a.st == 0) hipLaunchKernelGGL((qmmy_kernel<B, GS, 0, 8, false>), grid, dim3(512), lds, s, d); \
            else hipLaunchKernelGGL((qmmy_kernel<B, GS, 1, 8, false>), grid, dim3(512), lds, s, d); \
        } else { \
            if (a.st == 0) hipLaunchKernelGGL((qmmy_kernel<B, GS, 0, 4, false>), grid, dim3(256), lds, s, d); \
            else hipLaunchKernelGGL((qmmy_kernel<B, GS, 1, 4, false>), grid, dim3(256), lds, s, d); \
        } \
        return hipGetLastError(); }
        QMMY_GO(2, 32) QMMY_GO(2, 64) QMMY_GO(2, 128) QMMY_GO(3, 32) QMMY_GO(3, 64) QMMY_GO(3, 128)
        QMMY_GO(4, 32) QMMY_GO(4, 64) QMMY_GO(4, 128) QMMY_GO(6, 32) QMMY_GO(6, 64) QMMY_GO(6, 128)
        QMMY_GO(8, 32) QMMY_GO(8, 64)
#undef QMMY_GO
    }
#define QMMX_GO(B, GS) if (a.bits == B && a.gs == GS) { \
        if (a.st == 0) hipLaunchKernelGGL((qmmx_kernel<B, GS, 0>), grid, dim3(64 * QX_WAVES), 0, s, d); \
        else hipLaunchKernelGGL((qmmx_kernel<B, GS, 1>), grid, dim3(64 * QX_WAVES), 0, s, d); \
        return hipGetLastError(); }
    QMMX_GO(4, 32) QMMX_GO(4, 64) QMMX_GO(4, 128) QMMX_GO(8, 32) QMMX_GO(8, 64) QMMX_GO(8, 128)
#undef QMMX_GO
    return hipErrorInvalidValue;
}

}  // namespace mlxr
