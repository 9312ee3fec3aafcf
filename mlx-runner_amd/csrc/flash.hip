// Causal prefill attention on the matrix cores (flash attention over the bf16 paged KV cache).
//
// Semantics: the reference's flash_prefill (Kernels.swift:1839-2000): query t of the chunk sits at
// position pos0 + t and attends keys 0..pos0+t; scores s = (q * scale) . k, an online softmax over
// key tiles, out = sum p v / sum p, all in fp32 arithmetic. Here q and p enter the bf16 MFMA as a
// hi + lo pair of bf16 values (x = hi + lo exactly to ~2^-16), K and V are the bf16 cache itself,
// and every product accumulates in fp32, so the result matches fp32 arithmetic to ~1e-5 relative.
//
#include "kernels.h"

namespace mlxr {

typedef __bf16 fbf16x8_t __attribute__((ext_vector_type(8)));
typedef float ff32x4_t __attribute__((ext_vector_type(4)));

// MI355X layout: a 512-thread workgroup serves one KV head (up to 4 of its query heads; G > 4 takes
// ceil(G / 4) head groups) and two blocks of 32 queries, a light one (b) and its causal mirror
// (nb - 1 - b): waves 0-3 take the light block's heads, waves 4-7 the heavy block's,
// so every workgroup does the same work and the two waves on a SIMD hide each other's latency.
// Both blocks read the same K / V tiles, copied from the paged cache straight into LDS
// (buffer -> LDS, [key][128] bf16 with 16-byte chunks XOR-swizzled by (key & 15), two stages).
//   S^T = K Q^T   A = K rows (16-byte LDS reads), B = q * scale * log2(e) as bf16 hi + lo (registers)
//   softmax in base 2 (exp2), per query column (two lane exchanges)
//   O^T += V^T P^T  B = P^T from the S^T accumulators (hi + lo bf16: hardware conversions);
//                 A = V^T read with the LDS transpose read: lane j of a 16-lane group reads key
//                 base + (j >> 2), dims 4 (j & 3) .. + 3, and lane i receives dim i of the four
//                 keys base .. base + 3, so V needs no transposed copy.
typedef short fp_v4s __attribute__((ext_vector_type(4)));
typedef __bf16 fp_bf2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* fp_lptr;
typedef __attribute__((address_space(3))) fp_v4s* fp_lv4;
constexpr int F2_TILE = 64 * 256;                 // one K (or V) tile: 64 keys x 128 bf16

// (x0, x1) -> packed bf16 hi pair and lo pair, hi + lo = x to ~2^-16 relative
__device__ __forceinline__ void split2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
    const fp_bf2 h = {(__bf16)x0, (__bf16)x1};
    hi = __builtin_bit_cast(uint32_t, h);
    const float r0 = x0 - __uint_as_float(hi << 16), r1 = x1 - __uint_as_float(hi & 0xffff0000u);
    const fp_bf2 l = {(__bf16)r0, (__bf16)r1};
    lo = __builtin_bit_cast(uint32_t, l);
}

__global__ __launch_bounds__(512) void flash2_kernel(FlashArgs a, int nb, int ngroups) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t f2_lds[];   // [2 stages][K tile, V tile]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.nH / a.nKV, kvh = (int)blockIdx.y / ngroups, grp = (int)blockIdx.y - kvh * ngroups;
    const int gw = min(4, G - 4 * grp);                                  // heads of this group
    const int hh = wave & 3, half = wave >> 2;
    const int blight = (int)blockIdx.x, bheavy = nb - 1 - blight;
    const int blk = half ? bheavy : blight;
    const bool active = hh < gw && (half == 0 || bheavy != blight);
    const int h = kvh * G + 4 * grp + min(hh, gw - 1);
    const int pos0 = *a.dpos;
    const int q0 = blk * 32, nq = min(32, a.T - q0);
    const int kend = pos0 + q0 + nq;                                      // this wave's keys [0, kend)
    const int ntiles_wg = (pos0 + min(bheavy * 32 + 32, a.T) + 63) / 64;  // the heavy block's tiles
    const int ntiles = active ? (kend + 63) / 64 : 0;
    const int r16 = lane & 15, kq = lane >> 4;
    const float qscale = a.scale * 1.4426950408889634f;   // scores in base-2 units

    // copies of tile t: wave w takes 1-KB pieces 4w .. 4w + 3 of the 32 (K: 0-15, V: 16-31)
    auto issue = [&](int t) {
        const int page = a.pt[t];
        uint8_t* st = f2_lds + (t & 1) * 2 * F2_TILE;
        const size_t off = ((size_t)page * a.nKV + kvh) * (size_t)F2_TILE;
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)a.kc + off), 0, F2_TILE, 0x00020000);
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)a.vc + off), 0, F2_TILE, 0x00020000);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int piece = 4 * wave + i, q = piece & 15, key = 4 * q + kq;
            const uint32_t go = key * 256 + 16 * (r16 ^ (key & 15));
            if (piece < 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (fp_lptr)(st + q * 1024), 16, go, 0, 0, 0);
            else __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (fp_lptr)(st + F2_TILE + q * 1024), 16, go, 0, 0, 0);
        }
    };

    // q of this wave's head as B fragments [db][qb] x (hi, lo): dims 32 db + 8 kq .. +8, query 16 qb + r16
    fbf16x8_t qf[4][2][2];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const int t = min(q0 + 16 * qb + r16, a.T - 1);
        const float* qp = a.q + (size_t)t * a.q_stride + (size_t)h * 128;
#pragma unroll
        for (int db = 0; db < 4; db++) {
            const float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * db + 8 * kq);
            const float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * db + 8 * kq + 4);
            uint32_t hi[4], lo[4];
            split2(x0.x * qscale, x0.y * qscale, hi[0], lo[0]);
            split2(x0.z * qscale, x0.w * qscale, hi[1], lo[1]);
            split2(x1.x * qscale, x1.y * qscale, hi[2], lo[2]);
            split2(x1.z * qscale, x1.w * qscale, hi[3], lo[3]);
            qf[db][qb][0] = __builtin_bit_cast(fbf16x8_t, uint4{hi[0], hi[1], hi[2], hi[3]});
            qf[db][qb][1] = __builtin_bit_cast(fbf16x8_t, uint4{lo[0], lo[1], lo[2], lo[3]});
        }
    }
    ff32x4_t o[8][2];                            // O^T: dims 16 n + 4 kq + i, query 16 qb + r16
#pragma unroll
    for (int n = 0; n < 8; n++)
#pragma unroll
        for (int qb = 0; qb < 2; qb++) o[n][qb] = ff32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};

    issue(0);
    for (int t = 0; t < ntiles_wg; t++) {
        __builtin_amdgcn_s_waitcnt(0);       // this wave's copies of tile t landed ...
        __builtin_amdgcn_s_barrier();        // ... and every wave's; tile t - 1's stage is free
        if (t + 1 < ntiles_wg) issue(t + 1);
        if (t >= ntiles) continue;
        const uint8_t* ks = f2_lds + (t & 1) * 2 * F2_TILE;
        const uint8_t* vs = ks + F2_TILE;
        const int k0 = t * 64;

        // S^T tiles [kb][qb]: keys k0 + 16 kb + 4 kq + i, query 16 qb + r16
        ff32x4_t s[4][2];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            s[kb][0] = s[kb][1] = ff32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            const int key = 16 * kb + r16;
#pragma unroll
            for (int db = 0; db < 4; db++) {
                const fbf16x8_t ka = *reinterpret_cast<const fbf16x8_t*>(ks + key * 256 + 16 * ((4 * db + kq) ^ (key & 15)));
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    s[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[db][qb][0], s[kb][qb], 0, 0, 0);
                    s[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[db][qb][1], s[kb][qb], 0, 0, 0);
                }
            }
        }
        // causal mask (tiles reaching past the block's first query), base-2 online softmax
        const bool diag = k0 + 63 > pos0 + q0;
        uint32_t ph[2][2][4], pl[2][2][4];   // [st][qb] P^T fragments (hi, lo), 4 dwords each
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            const int qpos = pos0 + q0 + 16 * qb + r16;
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (diag && k0 + 16 * kb + 4 * kq + i > qpos) s[kb][qb][i] = -INFINITY;
                    mx = fmaxf(mx, s[kb][qb][i]);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = fmaxf(m[qb], mx);
            const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[qb] - mn);
            float p[4][4], sum = 0.0f;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    p[kb][i] = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[kb][qb][i] - mn);
                    sum += p[kb][i];
                }
            sum += __shfl_xor(sum, 16, 64);
            sum += __shfl_xor(sum, 32, 64);
            l[qb] = l[qb] * alpha + sum;
            m[qb] = mn;
#pragma unroll
            for (int n = 0; n < 8; n++) o[n][qb] *= alpha;
            // k-slots of PV step st: 0..3 = keys 16 (2 st) + 4 kq + i, 4..7 = keys 16 (2 st + 1) + 4 kq + i
#pragma unroll
            for (int st = 0; st < 2; st++) {
                split2(p[2 * st][0], p[2 * st][1], ph[st][qb][0], pl[st][qb][0]);
                split2(p[2 * st][2], p[2 * st][3], ph[st][qb][1], pl[st][qb][1]);
                split2(p[2 * st + 1][0], p[2 * st + 1][1], ph[st][qb][2], pl[st][qb][2]);
                split2(p[2 * st + 1][2], p[2 * st + 1][3], ph[st][qb][3], pl[st][qb][3]);
            }
        }
        // keys past the chunk's last key may hold anything: zero their V (their weight is 0, and
        // 0 * NaN is not)
        const bool tail = k0 + 64 > kend;
#pragma unroll
        for (int st = 0; st < 2; st++) {
            fbf16x8_t pb[2][2];
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                pb[qb][0] = __builtin_bit_cast(fbf16x8_t, uint4{ph[st][qb][0], ph[st][qb][1], ph[st][qb][2], ph[st][qb][3]});
                pb[qb][1] = __builtin_bit_cast(fbf16x8_t, uint4{pl[st][qb][0], pl[st][qb][1], pl[st][qb][2], pl[st][qb][3]});
            }
#pragma unroll
            for (int n = 0; n < 8; n++) {
                fp_v4s vv[2];
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const int key = 16 * (2 * st + r) + 4 * kq + (r16 >> 2);
                    const int c = 2 * n + ((r16 & 3) >> 1);
                    const uint8_t* ad = vs + key * 256 + 16 * (c ^ (key & 15)) + 8 * (r16 & 1);
                    vv[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fp_lv4)(ad));
                    if (tail) {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (k0 + 16 * (2 * st + r) + 4 * kq + e >= kend) vv[r][e] = 0;
                    }
                }
                const fbf16x8_t va = __builtin_bit_cast(fbf16x8_t, __builtin_shufflevector(vv[0], vv[1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    o[n][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[qb][0], o[n][qb], 0, 0, 0);
                    o[n][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[qb][1], o[n][qb], 0, 0, 0);
                }
            }
        }
    }
    if (!active) return;
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const int t = q0 + 16 * qb + r16;
        if (t >= a.T) continue;
        const float inv = 1.0f / l[qb];
        float* op = a.out + (size_t)t * a.out_stride + (size_t)h * 128 + 4 * kq;
#pragma unroll
        for (int n = 0; n < 8; n++)
            *reinterpret_cast<float4*>(op + 16 * n) = float4{o[n][qb][0] * inv, o[n][qb][1] * inv, o[n][qb][2] * inv, o[n][qb][3] * inv};
    }
}

hipError_t launch_flash_prefill(const FlashArgs& a, hipStream_t s) {
    if (a.D != 128 || a.nKV < 1 || a.nH % a.nKV || a.nH / a.nKV > 8 || a.T < 1) return hipErrorInvalidValue;
    const int G = a.nH / a.nKV, ngroups = (G + 3) / 4;
    const int nb = (a.T + 31) / 32, npair = (nb + 1) / 2;
    hipLaunchKernelGGL(flash2_kernel, dim3(npair, a.nKV * ngroups), dim3(512), 4 * F2_TILE, s, a, nb, ngroups);
    return hipGetLastError();
}

}  // namespace mlxr
