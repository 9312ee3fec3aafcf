// Prefill GEMM over the repacked decode tiles (DPack): Y[T][rows] = X[T][K] * W^T, 4-bit, bf16
// scales, f16 operands on v_mfma_f32_16x16x32_f16.
//
// Semantics: the reference's prefill tiles (Kernels.swift:785-851, `qgemm`). Precision is the 4-bit
// GEMM path's (gemm.hip): x is scaled per row by the power of two 2^e that puts max|x| in
// [2^13, 2^14) and rounded to f16 (x_to_f16_kernel), each weight is f16(fma(s, q, b)), products
// accumulate in fp32 and the row is scaled back by 2^-e.
//
// Why the repacked tiles: a DPack code block is 1 KB of one 16-row tile x 128 k with each lane's 16
// bytes already in the MFMA A-operand layout (lane (r, kq), dword j: row r, k = 32 j + 8 kq + 0..7),
// and a scale block is 1 KB of (scale | bias << 16) for 16 rows x 16 groups. Every buffer -> LDS
// copy therefore reads 1 KB of consecutive bytes; copying the MLX layout instead (16-byte pieces of
// 32 rows, 4-byte scale words) costs about three times the L1 accesses, which bounded the GEMM.
//
// Tile: a 512-thread workgroup owns 128 tokens x 16 DPack tiles (256 rows). Wave (wq, kc) computes
// the tiles 4 wq + 2 kc, + 1 against all 128 tokens (8 X fragments x 2 W fragments = 16 MFMAs per
// 32-k step); two waves share each SIMD, so one issues MFMAs while the other waits on memory or
// dequantizes. The X block (128 tokens x 128 k, f16, 16-byte chunks XOR-swizzled by (row & 15),
// read by all eight waves), the 16 code blocks and the block's scale words are copied buffer -> LDS
// into three stages, two blocks ahead of the one being computed (one block ahead left about a third
// of the waves' time waiting for the copies). Gated phases (gate rows in tile rows 0-7, up rows in 8-15) finish with
// SiLU(gate) * up in the epilogue, so the MLP activation is written directly.
#include "decode.h"

namespace mlxr {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t q4u4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int PT_M = 128, PT_KB = 128;
constexpr int PT_XB = PT_M * 256;                   // X block
// RT row tiles per wave (16 RT per workgroup), NST stages: (2, 3) by default; (3, 2) where a
// launch of 16-tile workgroups would leave a round half empty (the q|k|v projection of the 8B
// models: 384 tiles)
template <int RT> constexpr int pt_stage() { return PT_XB + 8 * RT * 1024 + 8 * RT * 256; }
template <int RT, int NST> constexpr int pt_lds_bytes() { return NST * pt_stage<RT>(); }
// s_waitcnt vmcnt(n), expcnt and lgkmcnt not waited for: one block's n copies of a wave in flight
constexpr int pt_wait_vm(int n) { return 0x0F70 | n; }
constexpr int PT_RSRC_W3 = 0x00020000;              // raw buffer, 32-bit data format

struct TileGemmArgs {
    MvPhaseDesc p;
    const uint16_t* xh; const float* inv; float* y;
    int ys, T, nT, ntiles;
};

__device__ __forceinline__ half2_t bf16_half2(uint32_t raw16) {
    const _Float16 h = (_Float16)__uint_as_float(raw16 << 16);
    return half2_t{h, h};
}

template <int GATED, int RT, int NST>
__global__ __launch_bounds__(512, 1) void tile_gemm_kernel(TileGemmArgs a) {
    constexpr int PT_TILES = 8 * RT, PT_CB = PT_TILES * 1024, PT_STAGE = pt_stage<RT>();
    constexpr int NCP = 4 + RT + 1;                 // copies a wave issues per block
    static_assert(NCP < 16 && NST >= 2 && NST <= 3, "copy pipeline");
    extern __shared__ __attribute__((aligned(1024))) uint8_t pt_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // the wave's first tile within the workgroup's
    const int wt0 = RT == 2 ? 4 * (wave & 3) + 2 * (wave >> 2) : RT * wave;
    // tile order: XCD x runs workgroups x, x + 8, ...; give it a contiguous run of tiles, and
    // enumerate tiles in columns of 8 row-tiles so that the ~32 workgroups an XCD runs at once cover
    // 4 token tiles x 8 row tiles (X and W blocks each shared in its L2 by several workgroups)
    const int g = blockIdx.x, xcd = g & 7, per = a.ntiles >> 3, rem = a.ntiles & 7;
    const int tile = xcd * per + min(xcd, rem) + (g >> 3);
    const int nO = a.ntiles / a.nT, ob = tile / (8 * a.nT), ow = min(8, nO - 8 * ob), r8 = tile - ob * 8 * a.nT;
    const int tt = r8 / ow, ot = 8 * ob + (r8 - tt * ow);
    const int t0 = ot * PT_TILES, m0 = tt * PT_M;
    const int r16 = lane & 15, kq = lane >> 4;
    const int K = a.p.K, FB = a.p.gs >> 3, nb = K / PT_KB, NF = (nb + FB - 1) / FB;
    const uint32_t tile_bytes = (uint32_t)NF * (FB + 1) * 1024;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)a.xh, 0, a.T * K * 2, PT_RSRC_W3);
    // tiles past the matrix read out of range (zeros)
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void*)a.p.code, 0, (int)(a.p.tiles * tile_bytes),
                                                                         PT_RSRC_W3);
    f32x4_t acc[8][RT];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int u = 0; u < RT; u++) acc[i][u] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // this wave's copies of block blk (NCP per wave): X rows 16 w .. 16 w + 15 (4 x 1 KB), the code
    // blocks of workgroup tiles RT w .. RT w + RT - 1, and their scale words of the block's
    // 128 / gs groups (lanes 0 .. 16 RT - 1: tile RT w + (lane >> 4), 16-byte chunk (rows 4 rq ..
    // 4 rq + 3, group gl) with lane & 15 = 4 rq + gl; chunks past the block's groups are loaded and
    // never read)
    auto issue = [&](int blk) {
        uint8_t* st = pt_lds + (blk % NST) * PT_STAGE;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int qq = wave * 4 + q, r = 4 * qq + kq;
            const uint32_t off = (uint32_t)(m0 + r) * (uint32_t)K * 2u + blk * 256 + 16 * (r16 ^ (r & 15));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr_t)(st + qq * 1024), 16, off, 0, 0, 0);
        }
        const int f = blk / FB, bl = blk - f * FB;
#pragma unroll
        for (int c = 0; c < RT; c++) {
            const int tw = RT * wave + c;
            const uint32_t base = (uint32_t)(t0 + tw) * tile_bytes + (uint32_t)f * (FB + 1) * 1024 + lane * 16;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_ptr_t)(st + PT_XB + tw * 1024), 16, base + (bl + 1) * 1024, 0, 0, 0);
        }
        if (lane < 16 * RT) {
            const int tw = RT * wave + (lane >> 4), l = lane & 15;
            const uint32_t off = (uint32_t)(t0 + tw) * tile_bytes + (uint32_t)f * (FB + 1) * 1024 +
                                 ((l >> 2) * 16 + bl * (PT_KB / a.p.gs) + (l & 3)) * 16;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_ptr_t)(st + PT_XB + PT_CB + RT * wave * 256), 16, off, 0, 0, 0);
        }
    };

    // one 128-k block: step j uses code dword j of the lane's 16 bytes of each code block
    // (k = 32 j + 8 kq + 0..7) and the X fragment of the same k; step j + 1's X fragments and
    // dequantized W are produced while step j's MFMAs run.
    auto compute = [&](int blk, int pf) {
        const uint8_t* st = pt_lds + (blk % NST) * PT_STAGE;
        const uint8_t* sc = st + PT_XB + PT_CB;
        q4u4_t cw[RT];
#pragma unroll
        for (int u = 0; u < RT; u++) cw[u] = *reinterpret_cast<const q4u4_t*>(st + PT_XB + (wt0 + u) * 1024 + lane * 16);
        half2_t s2[4][RT], b2[4][RT];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int gl = (32 * j) / a.p.gs;                      // group within the block
            const int so = ((r16 >> 2) * 4 + gl) * 16 + (r16 & 3) * 4;
#pragma unroll
            for (int u = 0; u < RT; u++) {
                const uint32_t w = *reinterpret_cast<const uint32_t*>(sc + (wt0 + u) * 256 + so);
                s2[j][u] = bf16_half2(w & 0xFFFFu);
                b2[j][u] = bf16_half2(w >> 16);
            }
        }
        auto dequant = [&](int j, half8_t* wf) {
#pragma unroll
            for (int u = 0; u < RT; u++) {
                const uint32_t wv = cw[u][j];
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    // (w & 0x000F000F) | 0x64006400 = the f16 pair (1024 + q_p, 1024 + q_p+4)
                    const uint32_t t = __builtin_amdgcn_bitop3_b32(wv >> (4 * p), 0x000F000Fu, 0x64006400u, 0xEA);
                    const half2_t q = __builtin_bit_cast(half2_t, t) - half2_t{(_Float16)1024.0f, (_Float16)1024.0f};
                    const half2_t v = q * s2[j][u] + b2[j][u];
                    wf[u][2 * p] = v[0];
                    wf[u][2 * p + 1] = v[1];
                }
            }
        };
        auto xload = [&](int j, half8_t* xf) {
#pragma unroll
            for (int i = 0; i < 8; i++)
                xf[i] = *reinterpret_cast<const half8_t*>(st + (16 * i + r16) * 256 + 16 * ((4 * j + kq) ^ r16));
        };
        half8_t xf[2][8], wf[2][RT];
        xload(0, xf[0]);
        dequant(0, wf[0]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            __builtin_amdgcn_sched_barrier(0);
            if (pf >= 0 && j == 0) issue(pf);
            if (j < 3) { xload(j + 1, xf[(j + 1) & 1]); dequant(j + 1, wf[(j + 1) & 1]); }
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int u = 0; u < RT; u++)
                    acc[i][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[j & 1][u], xf[j & 1][i], acc[i][u], 0, 0, 0);
            if (j < 3) {
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
                for (int k = 0; k < 8 * RT; k++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    issue(0);
    if (NST == 3 && nb > 1) issue(1);
    for (int blk = 0; blk < nb; blk++) {
        // this wave's copies of block blk have landed (with three stages block blk + 1's may still
        // be in flight) ...
        if (NST == 3 && blk + 1 < nb) __builtin_amdgcn_s_waitcnt(pt_wait_vm(NCP));
        else __builtin_amdgcn_s_waitcnt(0);
        // ... and every wave's; block blk + 1 - NST's stage, which block blk + NST - 1 overwrites,
        // is no longer read. A bare s_barrier: __syncthreads' fence adds nothing here.
        __builtin_amdgcn_s_barrier();
        compute(blk, blk + NST - 1 < nb ? blk + NST - 1 : -1);
    }
    // lane holds, for token m0 + 16 i + r16, rows 4 kq .. 4 kq + 3 of tile t0 + wt0 + u
#pragma unroll
    for (int u = 0; u < RT; u++) {
        const int t = t0 + wt0 + u;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int m = m0 + 16 * i + r16;
            const float iv = m < a.T ? a.inv[m] : 0.0f;
            f32x4_t v = acc[i][u] * iv;
            if constexpr (GATED) {
                // lanes kq < 2: gate rows 8t + 4kq + r; lanes kq >= 2: the matching up rows
                const int n = 8 * t + 4 * (kq & 1);
                f32x4_t up;
#pragma unroll
                for (int r = 0; r < 4; r++) up[r] = __shfl_xor(v[r], 32);
                if (kq >= 2 || m >= a.T || n >= a.p.o1) continue;
                float* yp = a.y + (int64_t)m * a.ys + n;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float gt = v[r], ut = up[r];
                    if (n + r < a.p.o1) {
                        if (a.p.bias[0]) gt += bf16_to_f32(a.p.bias[0][n + r]);
                        if (a.p.bias[1]) ut += bf16_to_f32(a.p.bias[1][n + r]);
                        yp[r] = (gt / (1.0f + expf(-gt))) * ut;
                    }
                }
            } else {
                const int n = 16 * t + 4 * kq;
                if (m >= a.T || n >= a.p.rows) continue;
                float* yp = a.y + (int64_t)m * a.ys + n;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int nr = n + r;
                    const int part = nr < a.p.o1 ? 0 : nr < a.p.o1 + a.p.o2 ? 1 : 2;
                    const int row = nr - (part > 0 ? a.p.o1 : 0) - (part > 1 ? a.p.o2 : 0);
                    const uint16_t* bp = a.p.bias[part];
                    if (bp) v[r] += bf16_to_f32(bp[row]);
                }
                if (n + 4 <= a.p.rows && (reinterpret_cast<uintptr_t>(yp) & 15) == 0) *reinterpret_cast<f32x4_t*>(yp) = v;
                else
                    for (int r = 0; r < 4 && n + r < a.p.rows; r++) yp[r] = v[r];
            }
        }
    }
}

}  // namespace

bool tile_gemm_supported(const MvPhaseDesc& p) {
    return p.code && (p.gs == 32 || p.gs == 64) && p.K % PT_KB == 0 && p.tiles > 0;
}

template <int RT, int NST>
static hipError_t tile_gemm_launch(const TileGemmArgs& a0, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        for (const void* f : {(const void*)tile_gemm_kernel<0, RT, NST>, (const void*)tile_gemm_kernel<1, RT, NST>})
            if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, pt_lds_bytes<RT, NST>()) != hipSuccess)
                return hipErrorInvalidValue;
        attr = true;
    }
    TileGemmArgs a = a0;
    a.ntiles = a.nT * ((a.p.tiles + 8 * RT - 1) / (8 * RT));
    constexpr int lds = pt_lds_bytes<RT, NST>();
    if (a.p.gated) hipLaunchKernelGGL((tile_gemm_kernel<1, RT, NST>), dim3(a.ntiles), dim3(512), lds, s, a);
    else hipLaunchKernelGGL((tile_gemm_kernel<0, RT, NST>), dim3(a.ntiles), dim3(512), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_tile_gemm(const MvPhaseDesc& p, const uint16_t* xh, const float* inv, int T, float* y, int ys,
                            hipStream_t s) {
    if (!tile_gemm_supported(p) || T < 1) return hipErrorInvalidValue;
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidDevice;
    }
    TileGemmArgs a;
    a.p = p; a.xh = xh; a.inv = inv; a.y = y; a.ys = ys; a.T = T;
    a.nT = (T + PT_M - 1) / PT_M;
    // one workgroup per CU: rounds of workgroups x tiles per workgroup, the two-stage pipeline of the
    // 24-tile workgroups costing ~4% (measured on the 16-tile ones)
    auto cost = [&](int rt) {
        const long wgs = (long)a.nT * ((p.tiles + 8 * rt - 1) / (8 * rt));
        return (double)((wgs + cus - 1) / cus) * rt * (rt == 3 ? 1.04 : 1.0);
    };
    if (cost(3) < cost(2)) return tile_gemm_launch<3, 2>(a, s);
    return tile_gemm_launch<2, 3>(a, s);
}

}  // namespace mlxr
