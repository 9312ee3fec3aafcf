// Decode attention over the bf16 paged KV cache (split over keys + ordered merge) and the sparse
// decode path (index, plan, block scores, exact top-p selection).
//
// Semantics: the reference's attention_split + attention_combine (Kernels.swift:1317-1374) and
// sparse kernels (Kernels.swift:1541-1756): scores s = (q * scale) . k in fp32, an online-softmax
// partial (max, sum, acc[D]) per key range, merged in range order. The key ranges here are
// contiguous (range r of `nsplit` holds keys r*c .. r*c+c-1, c = ceil(count/nsplit)), so with the
// list 0..L-1 the sparse path runs exactly the dense path's arithmetic.
//
// MI355X layout: one 256-thread workgroup per (KV head, token, key range); the G query heads of
// the KV head share every K/V read. Scores: 4 lanes per key, each reading 64 contiguous bytes of
// the key row (32 bf16), partial dots combined with two lane exchanges. Values: each wave takes a
// quarter of the range, lanes own 2 of the 128 dims, so a wave reads one 256-byte V row per key.
#include <algorithm>
#include "kernels.h"

namespace mlxr {

constexpr int ATT_D = 128;
constexpr int ATT_MAXG = 8;
constexpr int ATT_MAXC = 512;   // keys per workgroup (range size cap, checked on the host)

struct SparsePlanDev { int valid, b0, nb, p, sink_end, win_start, L, count; };

__device__ __forceinline__ void bf16x8_to_f32(const uint4 v, float* o) {
    o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
    o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
    o[4] = __uint_as_float(v.z << 16); o[5] = __uint_as_float(v.z & 0xffff0000u);
    o[6] = __uint_as_float(v.w << 16); o[7] = __uint_as_float(v.w & 0xffff0000u);
}

// grid (nKV * T, nsplit); block 256. Writes partials [t][h][split] = (m, l, acc[D]).
// Keys are taken 64 at a time; every thread's K (scores) and V (values) loads for a chunk are
// issued together, and the next chunk's before the current one is used, so a range costs about
// one memory round trip per pass rather than one per key. Row offsets (list and page table
// lookups) are resolved once into LDS.
constexpr int ATT_CH = 64;   // keys per chunk
__device__ __forceinline__ void att_ld4(const uint16_t* base, int row, int sub, uint4* o) {
    const uint4* p = reinterpret_cast<const uint4*>(base + (int64_t)row * ATT_D) + sub;
#pragma unroll
    for (int v = 0; v < 4; v++) o[v] = p[v];
}
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a, const SparsePlanDev* plan) {
    __shared__ float qs[ATT_MAXG][ATT_D];
    __shared__ float sc[ATT_MAXG][ATT_MAXC];
    __shared__ int rowi[ATT_MAXC];
    __shared__ float mx[ATT_MAXG], lsum[ATT_MAXG];
    __shared__ float accs[4][ATT_MAXG][ATT_D];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = blockIdx.x % a.nKV, t = blockIdx.x / a.nKV, split = blockIdx.y;
    const int G = a.nH / a.nKV, D = ATT_D;
    const int pos = *a.dpos + t, L = pos + 1;
    const bool sparse = a.lists != nullptr && plan != nullptr && plan->valid;
    const int count = sparse ? plan->count : L;
    const int* list = sparse ? a.lists + (int64_t)kvh * a.list_stride : nullptr;
    const int c = (count + a.nsplit - 1) / a.nsplit;
    const int n0 = min(count, split * c), n1 = min(count, n0 + c), nk = n1 - n0;
    {   // unrolled with guards: every load of the prologue in flight at once
        float qv[ATT_MAXG * ATT_D / 256];
#pragma unroll
        for (int r = 0; r < ATT_MAXG * ATT_D / 256; r++) {
            const int i = tid + 256 * r, g = i / D, d = i % D;
            qv[r] = i < G * D ? a.q[(int64_t)t * a.q_stride + (int64_t)(kvh * G + g) * D + d] : 0.0f;
        }
        int jv[ATT_MAXC / 256];
#pragma unroll
        for (int r = 0; r < ATT_MAXC / 256; r++) {
            const int kk = tid + 256 * r;
            int j = nk > 0 ? n0 + min(kk, nk - 1) : 0;
            if (sparse && nk > 0) j = list[j];
            j = j < 0 ? 0 : (j > L - 1 ? L - 1 : j);
            jv[r] = j;
        }
#pragma unroll
        for (int r = 0; r < ATT_MAXC / 256; r++) {
            const int kk = tid + 256 * r;
            const int64_t row = kv_row(a.pt, a.nKV, kvh, jv[r]);
            if (kk < nk) rowi[kk] = (int)row;
        }
#pragma unroll
        for (int r = 0; r < ATT_MAXG * ATT_D / 256; r++) {
            const int i = tid + 256 * r;
            if (i < G * D) qs[i / D][i % D] = qv[r] * a.scale;
        }
    }
    __syncthreads();
    const int nch = (nk + ATT_CH - 1) / ATT_CH;
    // V loads of the P V pass: thread = (key slot tid / 16: keys slot + 16 i of each chunk, dims
    // 8 (tid % 16) .. + 8); the first chunk's are issued with the first K loads
    const int ds = tid & 15, ks = tid >> 4;
    auto ldv = [&](int ch, uint4* o) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int kk = min(ch * ATT_CH + ks + 16 * i, nk - 1);
            o[i] = reinterpret_cast<const uint4*>(a.vc + (int64_t)rowi[kk] * ATT_D)[ds];
        }
    };
    uint4 vr[4];
    // scores: thread = (key tid / 4 of the chunk, quarter tid % 4 of the row)
    {
        const int qd = tid & 3, kq = tid >> 2;
        uint4 kr[4], kn[4];
        if (nch > 0) { att_ld4(a.kc, rowi[min(kq, nk - 1)], qd * 4, kr); ldv(0, vr); }
        for (int ch = 0; ch < nch; ch++) {
            if (ch + 1 < nch) att_ld4(a.kc, rowi[min((ch + 1) * ATT_CH + kq, nk - 1)], qd * 4, kn);
            float kf[32];
#pragma unroll
            for (int v = 0; v < 4; v++) bf16x8_to_f32(kr[v], kf + 8 * v);
            const int kk = ch * ATT_CH + kq;
            for (int g = 0; g < G; g++) {
                float s = 0.0f;
#pragma unroll
                for (int e = 0; e < 32; e++) s = fmaf(qs[g][qd * 32 + e], kf[e], s);
                s = quad_sum(s);
                if (kk < nk && qd == 0) sc[g][kk] = s;
            }
#pragma unroll
            for (int v = 0; v < 4; v++) kr[v] = kn[v];
        }
    }
    __syncthreads();
    // per-head max and exp
    for (int g = wave; g < G; g += 4) {
        float m = -1e30f;
        for (int i = lane; i < nk; i += 64) m = fmaxf(m, sc[g][i]);
        m = wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < nk; i += 64) { const float p = expf(sc[g][i] - m); sc[g][i] = p; l += p; }
        l = wave_sum(l);
        if (lane == 0) { mx[g] = m; lsum[g] = l; }
    }
    __syncthreads();
    // P V
    {
        float acc[ATT_MAXG][8];
#pragma unroll
        for (int g = 0; g < ATT_MAXG; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
        uint4 vn[4];
        for (int ch = 0; ch < nch; ch++) {
            if (ch + 1 < nch) ldv(ch + 1, vn);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kk = ch * ATT_CH + ks + 16 * i;
                if (kk < nk) {
                    float vf[8];
                    bf16x8_to_f32(vr[i], vf);
#pragma unroll
                    for (int g = 0; g < ATT_MAXG; g++) {
                        if (g < G) {
                            const float p = sc[g][kk];
#pragma unroll
                            for (int e = 0; e < 8; e++) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) vr[i] = vn[i];
        }
        // the wave's four key slots (lanes xor 16, 32), then the four waves through LDS
#pragma unroll
        for (int g = 0; g < ATT_MAXG; g++) {
            if (g < G) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    acc[g][e] = xor32_sum(xor16_sum(acc[g][e]));
                }
                if (lane < 16) {
#pragma unroll
                    for (int e = 0; e < 8; e++) accs[wave][g][8 * ds + e] = acc[g][e];
                }
            }
        }
    }
    __syncthreads();
    const int rows = a.nH * a.nsplit;
    float* pt_ = a.part + (int64_t)t * rows * (D + 2);
    for (int i = tid; i < G * D; i += 256) {
        const int g = i / D, d = i % D;
        const float v = ((accs[0][g][d] + accs[1][g][d]) + accs[2][g][d]) + accs[3][g][d];
        const int r = (kvh * G + g) * a.nsplit + split;
        pt_[2 * rows + (int64_t)r * D + d] = nk > 0 ? v : 0.0f;
        if (d == 0) { pt_[r] = nk > 0 ? mx[g] : -1e30f; pt_[rows + r] = nk > 0 ? lsum[g] : 0.0f; }
    }
}

// grid (nH, T); block D: merge the partials of one head in range order. The per-range weights
// exp(m_s - M) are computed once (one thread per range) into LDS; each thread then sums its
// dimension over the ranges with eight loads in flight.
constexpr int ATT_MAXS = 4096;   // key ranges per head (max, checked on the host)
__global__ __launch_bounds__(128) void attn_combine_kernel(AttnArgs a) {
    __shared__ float w[ATT_MAXS];
    __shared__ float red[2];
    const int h = blockIdx.x, t = blockIdx.y, d = threadIdx.x, D = ATT_D, NS = a.nsplit;
    const int rows = a.nH * NS;
    const float* pt_ = a.part + (int64_t)t * rows * (D + 2);
    const float* mrow = pt_ + h * NS;
    const float* lrow = pt_ + rows + h * NS;
    float M = -1e30f;
    for (int s = d; s < NS; s += 128) M = fmaxf(M, mrow[s]);
    M = wave_max(M);
    if ((d & 63) == 0) red[d >> 6] = M;
    __syncthreads();
    M = fmaxf(red[0], red[1]);
    for (int s = d; s < NS; s += 128) w[s] = expf(mrow[s] - M);
    __syncthreads();
    float Ls = 0.0f, o = 0.0f;
    const float* acc = pt_ + 2 * rows + (int64_t)h * NS * D + d;
    // 32 ranges' loads in flight per batch (each batch is a memory round trip: the partials come
    // from other XCDs), summed in range order
    constexpr int CB = 32;
    int s = 0;
    for (; s + CB <= NS; s += CB) {
        float v[CB], l[CB];
#pragma unroll
        for (int i = 0; i < CB; i++) { v[i] = acc[(int64_t)(s + i) * D]; l[i] = lrow[s + i]; }
#pragma unroll
        for (int i = 0; i < CB; i++) { Ls += l[i] * w[s + i]; o += v[i] * w[s + i]; }
    }
    for (; s < NS; s++) { Ls += lrow[s] * w[s]; o += acc[(int64_t)s * D] * w[s]; }
    a.out[(int64_t)t * a.out_stride + (int64_t)h * D + d] = o / Ls;
}

// Verify batch (T = 2..8 queries at positions *dpos .. *dpos + T - 1, dense keys): grid (nKV,
// nsplit); block 256. One workgroup per (KV head, key range) serves all G x T query rows of the head
// (row r = t G + g), so each K and V row is read from memory once for the whole batch rather than
// once per query. Every K and V load of the range is issued at once, after the row offsets (one
// memory round trip for the range), into LDS; each wave's q rows load straight
// into registers meanwhile. Both products run on the bf16 matrix cores
// (v_mfma_f32_16x16x32_bf16), 16 x 16 output tiles spread over the waves:
//   S^T = K Q^T    A = K rows, B = q * scale as bf16 hi + lo (the persistent decode step's split)
//   O = P V        A = P as three bf16 terms (hi + mid + lo = p to ~2^-24), B = V through the LDS
//                  transpose read (lane j of a 16-lane group reads key base + (j >> 2), dims
//                  4 (j & 3) .. + 3; lane i receives dim i of keys base .. base + 3)
// K and V are bf16 in the cache, so the only roundings are the splits'. Keys past a row's own
// position are masked (its softmax covers keys 0 .. *dpos + t). Rows and keys past the batch read
// copies of the last row / key (finite) and their results are dropped. Writes the same partials
// [t][h][split] as attn_split_kernel for attn_combine_kernel.
constexpr int ATT_MC = 128;                  // keys per workgroup (max; the host sets a.cap >= ceil(count / nsplit))
constexpr int ATT_VR = ATT_MC / 16;          // K / V staging: 16 rows per pass of 256 threads (16 bytes each)
constexpr int ATT_RS = ATT_D + 8;            // bf16 row stride of the K image (16 rows of a read: distinct banks)
typedef float f32x4_att __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_att __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4_att att_mfma(const uint4 a, const uint4 b, f32x4_att c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_att, a), __builtin_bit_cast(bf16x8_att, b), c, 0, 0, 0);
}
// The LDS layout of one workgroup (byte offsets, 16-byte aligned). The K image is dead once the
// scores are in, so the probabilities' bf16 terms take its place.
struct AttMultiLds {
    int GP, KQ, PS, scs;
    size_t ks, pb, vs, sc, rowi, ro, mx, ls, bytes;
    __host__ __device__ AttMultiLds(int GT, int cap) {
        GP = (GT + 15) / 16 * 16;            // query rows, padded to whole tiles
        KQ = (cap + 31) / 32 * 32;           // keys, padded to whole 32-key steps
        PS = KQ + 8; scs = KQ + 4;
        ks = pb = 0;                                     // [KQ][ATT_RS] bf16 K | [3][GP][PS] bf16 p terms
        const size_t kb = (size_t)KQ * ATT_RS * 2, pbb = (size_t)3 * GP * PS * 2;
        vs = kb > pbb ? kb : pbb;                        // [KQ][128] bf16 V, 16-byte chunk c of key k at c ^ (k & 15)
        sc = vs + (size_t)KQ * ATT_D * 2;                // [GP][scs] f32 scores
        rowi = sc + (size_t)GP * scs * 4;                // [KQ] cache rows
        ro = rowi + (size_t)KQ * 4;                      // [GP] int2: a row's token base and (head, split) row in the partials
        mx = ro + (size_t)GP * 8;                        // [GP] row max
        ls = mx + (size_t)GP * 4;                        // [GP] row sum
        bytes = ls + (size_t)GP * 4;
    }
};
// (x0, x1) -> packed bf16 pair (hardware round to nearest even)
__device__ __forceinline__ uint32_t att_pk(float x0, float x1) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    const bf2 h = {(__bf16)x0, (__bf16)x1};
    return __builtin_bit_cast(uint32_t, h);
}
typedef short att_v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) att_v4s* att_lv4;
__global__ __launch_bounds__(256) void attn_multi_kernel(AttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_b[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = blockIdx.x, split = blockIdx.y, D = ATT_D;
    const int G = a.nH / a.nKV, T = a.T, GT = G * T, cap = a.cap;
    const int pos0 = *a.dpos, count = pos0 + T;
    const int c = (count + a.nsplit - 1) / a.nsplit;
    const int n0 = min(count, split * c), n1 = min(count, n0 + min(c, cap)), nk = n1 - n0;
    const int rows = a.nH * a.nsplit;
    if (nk <= 0) {   // a range past the batch's last key: empty partials
        for (int r = wave; r < GT; r += 4) {
            const int t = r / G, g = r % G, rr = (kvh * G + g) * a.nsplit + split;
            float* pt_ = a.part + (int64_t)t * rows * (D + 2);
            *reinterpret_cast<float2*>(pt_ + 2 * rows + (int64_t)rr * D + 2 * lane) = float2{0.0f, 0.0f};
            if (lane == 0) { pt_[rr] = -1e30f; pt_[rows + rr] = 0.0f; }
        }
        return;
    }
    const AttMultiLds L(GT, cap);
    uint16_t* ks = reinterpret_cast<uint16_t*>(lds_b + L.ks);
    uint16_t* pb = reinterpret_cast<uint16_t*>(lds_b + L.pb);
    uint8_t* vs = lds_b + L.vs;
    float* sc = reinterpret_cast<float*>(lds_b + L.sc);
    int* rowi = reinterpret_cast<int*>(lds_b + L.rowi);
    int2* ro = reinterpret_cast<int2*>(lds_b + L.ro);
    float* mx = reinterpret_cast<float*>(lds_b + L.mx);
    float* lsum = reinterpret_cast<float*>(lds_b + L.ls);
    const int GP = L.GP, nkq = (nk + 31) / 32 * 32;
    const int l16 = lane & 15, l4 = lane >> 4;
    const int nrt = GP / 16, nkt = (nk + 15) / 16;
    // this wave's q rows (row tile rt: rows 16 rt + l16, dims 8 l4 + 32 s .. + 7) as the B operand,
    // scaled and split into bf16 hi + lo
    uint4 bh[4], bl[4];
    auto load_q = [&](int rt) {
        const int r = min(16 * rt + l16, GT - 1), t = r / G, g = r - t * G;
        const float* qr = a.q + (int64_t)t * a.q_stride + (int64_t)(kvh * G + g) * D + 8 * l4;
        float4 v[8];
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) { v[2 * s4] = *reinterpret_cast<const float4*>(qr + 32 * s4); v[2 * s4 + 1] = *reinterpret_cast<const float4*>(qr + 32 * s4 + 4); }
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
            const float x[8] = {v[2 * s4].x, v[2 * s4].y, v[2 * s4].z, v[2 * s4].w, v[2 * s4 + 1].x, v[2 * s4 + 1].y, v[2 * s4 + 1].z, v[2 * s4 + 1].w};
            uint32_t h[4], lo[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float x0 = x[2 * j] * a.scale, x1 = x[2 * j + 1] * a.scale;
                h[j] = att_pk(x0, x1);
                lo[j] = att_pk(x0 - __uint_as_float(h[j] << 16), x1 - __uint_as_float(h[j] & 0xffff0000u));
            }
            bh[s4] = uint4{h[0], h[1], h[2], h[3]}; bl[s4] = uint4{lo[0], lo[1], lo[2], lo[3]};
        }
    };
    int cur_rt = wave % nrt;
    load_q(cur_rt);
    if (tid < nk) rowi[tid] = (int)kv_row(a.pt, a.nKV, kvh, n0 + tid);   // nk <= ATT_MC <= 256 threads
    if (tid < GT) {   // partials of row r = t G + g: [t][(head, split)], below 2^31 floats
        const int t = tid / G, g = tid - t * G;
        ro[tid] = int2{t * rows * (D + 2), (kvh * G + g) * a.nsplit + split};
    }
    __syncthreads();
    {   // K and V rows to LDS: every load issued before the first store (unconditional: keys
        // past the range read the last key, and their rows, up to the image's edge, hold copies of it)
        const int vrow = tid >> 4, vd = tid & 15;
        uint4 kv[ATT_VR], vv[ATT_VR];
#pragma unroll
        for (int i = 0; i < ATT_VR; i++) {
            const int64_t row = rowi[min(vrow + 16 * i, nk - 1)];
            kv[i] = reinterpret_cast<const uint4*>(a.kc + row * D)[vd];
            vv[i] = reinterpret_cast<const uint4*>(a.vc + row * D)[vd];
        }
#pragma unroll
        for (int i = 0; i < ATT_VR; i++) {
            const int r = min(vrow + 16 * i, L.KQ - 1);
            *reinterpret_cast<uint4*>(ks + r * ATT_RS + 8 * vd) = kv[i];
            *reinterpret_cast<uint4*>(vs + r * 256 + 16 * (vd ^ (r & 15))) = vv[i];
        }
    }
    __syncthreads();
    // scores S^T: tile (kt, rt) = keys 16 kt.., rows 16 rt..; lane: keys 16 kt + 4 l4 + i, row l16
    for (int tI = wave; tI < nrt * nkt; tI += 4) {
        const int rt = tI % nrt, kt = tI / nrt;
        if (rt != cur_rt) { cur_rt = rt; load_q(rt); }
        const uint16_t* ka = ks + (16 * kt + l16) * ATT_RS + 8 * l4;
        uint4 av[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) av[s4] = *reinterpret_cast<const uint4*>(ka + 32 * s4);
        f32x4_att s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) { s0 = att_mfma(av[s4], bh[s4], s0); s1 = att_mfma(av[s4], bl[s4], s1); }
        const int r = 16 * rt + l16, key = 16 * kt + 4 * l4;
        if (r < GT) *reinterpret_cast<float4*>(sc + r * L.scs + key) = float4{s0[0] + s1[0], s0[1] + s1[1], s0[2] + s1[2], s0[3] + s1[3]};
    }
    __syncthreads();
    // per-row max and exp over the row's own keys (n0 .. min(n1, *dpos + t + 1)), lane: keys 2 lane,
    // 2 lane + 1 of each 128; p as three bf16 terms over the dead K image, zeros up to the 32-key
    // step edge. Padded rows stay as they are: an MFMA output row reads only its own A row.
    for (int r = wave; r < GT; r += 4) {
        const int nv = max(0, min(nk, pos0 + r / G + 1 - n0));
        float m = -1e30f;
        for (int k2 = 2 * lane; k2 < nkq; k2 += 128) {
            const float2 v = *reinterpret_cast<const float2*>(sc + r * L.scs + k2);
            m = fmaxf(m, fmaxf(k2 < nv ? v.x : -1e30f, k2 + 1 < nv ? v.y : -1e30f));
        }
        m = wave_max(m);
        float l = 0.0f;
        for (int k2 = 2 * lane; k2 < nkq; k2 += 128) {
            const float2 v = *reinterpret_cast<const float2*>(sc + r * L.scs + k2);
            const float p0 = k2 < nv ? expf(v.x - m) : 0.0f, p1 = k2 + 1 < nv ? expf(v.y - m) : 0.0f;
            l += p0 + p1;
            const uint32_t h = att_pk(p0, p1);
            const float r0 = p0 - __uint_as_float(h << 16), r1 = p1 - __uint_as_float(h & 0xffff0000u);
            const uint32_t md = att_pk(r0, r1);
            const uint32_t lo = att_pk(r0 - __uint_as_float(md << 16), r1 - __uint_as_float(md & 0xffff0000u));
            *reinterpret_cast<uint32_t*>(pb + r * L.PS + k2) = h;
            *reinterpret_cast<uint32_t*>(pb + (GP + r) * L.PS + k2) = md;
            *reinterpret_cast<uint32_t*>(pb + (2 * GP + r) * L.PS + k2) = lo;
        }
        l = wave_sum(l);
        if (lane == 0) { mx[r] = nv > 0 ? m : -1e30f; lsum[r] = l; }
    }
    __syncthreads();
    // O = P V: tile (rt, dt) = rows 16 rt.., dims 16 dt..; lane: row 16 rt + 4 l4 + i, dim 16 dt + l16
    for (int tI = wave; tI < nrt * (ATT_D / 16); tI += 4) {
        const int rt = tI >> 3, dt = tI & 7;
        // k-slots of a 32-key step: 0..3 = keys 4 l4 + (0..3), 4..7 = keys 16 + 4 l4 + (0..3) (the
        // transpose read's order), P read to match
        const uint16_t* p0 = pb + (16 * rt + l16) * L.PS + 4 * l4;
        const int c = 2 * dt + ((l16 & 3) >> 1);
        f32x4_att o0 = {0.0f, 0.0f, 0.0f, 0.0f}, o1 = {0.0f, 0.0f, 0.0f, 0.0f}, o2 = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = 0; k < nkq; k += 32) {
            att_v4s vv[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int key = k + 16 * h + 4 * l4 + (l16 >> 2);
                vv[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((att_lv4)(vs + key * 256 + 16 * (c ^ (key & 15)) + 8 * (l16 & 1)));
            }
            const uint4 bv = __builtin_bit_cast(uint4, __builtin_shufflevector(vv[0], vv[1], 0, 1, 2, 3, 4, 5, 6, 7));
            uint4 pt3[3];
#pragma unroll
            for (int tm = 0; tm < 3; tm++) {
                const uint2 x0 = *reinterpret_cast<const uint2*>(p0 + tm * GP * L.PS + k);
                const uint2 x1 = *reinterpret_cast<const uint2*>(p0 + tm * GP * L.PS + k + 16);
                pt3[tm] = uint4{x0.x, x0.y, x1.x, x1.y};
            }
            o0 = att_mfma(pt3[0], bv, o0); o1 = att_mfma(pt3[1], bv, o1); o2 = att_mfma(pt3[2], bv, o2);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 16 * rt + 4 * l4 + i;
            if (r >= GT) break;
            const int2 o = ro[r];
            const int rr = o.y;
            float* pt_ = a.part + o.x;
            const bool any = mx[r] > -1e30f;
            pt_[2 * rows + (int64_t)rr * D + 16 * dt + l16] = any ? (o0[i] + o1[i]) + o2[i] : 0.0f;
            if (dt == 0 && l16 == 0) { pt_[rr] = mx[r]; pt_[rows + rr] = any ? lsum[r] : 0.0f; }
        }
    }
}

hipError_t launch_attn_verify(const AttnArgs& a, hipStream_t s) {
    const int G = a.D == ATT_D && a.nKV > 0 && a.nH % a.nKV == 0 ? a.nH / a.nKV : 0, GT = G * a.T;
    if (G == 0 || a.T < 2 || GT > 64 || a.nsplit < 1 || a.nsplit > ATT_MAXS || a.lists || a.cap < 1 || a.cap > ATT_MC)
        return hipErrorInvalidValue;
    const AttMultiLds L(GT, a.cap);
    static bool attr = false;
    if (!attr) {
        if (hipFuncSetAttribute((const void*)attn_multi_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
            return hipErrorInvalidValue;
        attr = true;
    }
    if (L.bytes > 160 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_multi_kernel, dim3(a.nKV, a.nsplit), dim3(256), L.bytes, s, a);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nH, a.T), dim3(ATT_D), 0, s, a);
    return hipGetLastError();
}

static hipError_t attn_launch(const AttnArgs& a, const SparsePlanDev* plan, hipStream_t s) {
    if (a.D != ATT_D || a.nH % a.nKV || a.nH / a.nKV > ATT_MAXG || a.nsplit < 1 || a.nsplit > ATT_MAXS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_split_kernel, dim3(a.nKV * a.T, a.nsplit), dim3(256), 0, s, a, plan);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nH, a.T), dim3(ATT_D), 0, s, a);
    return hipGetLastError();
}
hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t s) {
    return attn_launch(a, reinterpret_cast<const SparsePlanDev*>(a.splan), s);
}

// ---------------------------------------------------------------------------------------------
// Sparse index (Kernels.swift:1545-1555): idx[b][kvh][d] = bf16(mean of the block's 4 keys), for
// the blocks completed by positions pos0 .. pos0+T-1 (b in [pos0/4, (pos0+T)/4)).
__global__ void sparse_index_kernel(const uint16_t* kc, const int* pt, uint16_t* idx, int nKV, int D,
                                    const int* dpos, int pos_add, int T) {
    const int pos0 = *dpos + pos_add;
    const int b0 = pos0 / 4, b1 = (pos0 + T) / 4;
    const int b = b0 + blockIdx.x, kvh = blockIdx.y, d = threadIdx.x;
    if (b >= b1) return;
    float s = 0.0f;
    for (int i = 0; i < 4; i++) s += bf16_to_f32(kc[kv_row(pt, nKV, kvh, b * 4 + i) * D + d]);
    idx[((int64_t)b * nKV + kvh) * D + d] = f32_to_bf16(s / 4.0f);
}
hipError_t launch_sparse_index(const uint16_t* kc, const int* pt, uint16_t* idx, int nKV, int D, const int* dpos,
                               int pos_add, int T, hipStream_t s) {
    hipLaunchKernelGGL(sparse_index_kernel, dim3(T / 4 + 1, nKV), dim3(D), 0, s, kc, pt, idx, nKV, D, dpos, pos_add, T);
    return hipGetLastError();
}

// Plan of the decode step at *dpos (SparseAttention.swift:80-94). One thread.
__global__ void sparse_plan_kernel(const int* dpos, int top_k, int window, int sink, int min_context, SparsePlanDev* o) {
    const int pool = 4, position = *dpos, L = position + 1;
    SparsePlanDev p{};
    p.valid = 0;
    if (position >= 0 && L >= min_context) {
        const int sinkEnd = (sink + pool - 1) / pool * pool;
        if (L - window > sinkEnd) {
            const int winStart = (L - window) / pool * pool;
            const int b0 = sinkEnd / pool, nb = winStart / pool - b0;
            if (nb > 0) {
                p.valid = 1; p.b0 = b0; p.nb = nb; p.p = min(top_k / pool, nb); p.sink_end = sinkEnd;
                p.win_start = winStart; p.L = L; p.count = sinkEnd + p.p * pool + (L - winStart);
            }
        }
    }
    *o = p;
}
hipError_t launch_sparse_plan(const SparseArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(sparse_plan_kernel, dim3(1), dim3(1), 0, s, a.dpos, a.top_k, a.window, a.sink, a.min_context,
                       reinterpret_cast<SparsePlanDev*>(a.dplan));
    return hipGetLastError();
}

// Block scores (Kernels.swift:1565-1612): qsum_kvh . idx[b0 + n][kvh] (qsum: the sum of the KV
// head's query rows), per KV head (rows == nKV) or summed over them (rows == 1). One wave per
// 4 blocks at a time: lane l holds dims 8 (l % 16) .. + 8 of KV heads l / 16 + 4 j, so the wave
// reads a block's whole index row (nKV * 256 bytes) in one 16-byte load per head pair, and all
// four blocks' loads are in flight together. D = 128, nKV <= 16.
constexpr int SCORE_BPW = 4;
__global__ __launch_bounds__(256) void sparse_score_kernel(const float* q, const uint16_t* idx, float* scores, int nH,
                                                           int nKV, int rows, int score_stride,
                                                           const SparsePlanDev* plan, int b0_, int nb_) {
    const int W = nKV * ATT_D, G = nH / nKV;
    int b0 = b0_, nb = nb_;
    if (plan) { if (!plan->valid) return; b0 = plan->b0; nb = plan->nb; }
    const int lane = threadIdx.x & 63, hq = lane >> 4, dq = lane & 15;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6), nw = gridDim.x * 4;
    // this wave's first blocks of the index (unconditional: rows clamped into the range, heads
    // past nKV read head 0), issued before the q loads so that their memory latencies overlap
    uint4 kv[SCORE_BPW][4];
    auto load_blocks = [&](int nbase) {
#pragma unroll
        for (int i = 0; i < SCORE_BPW; i++) {
            const int n = max(0, min(nbase + i, nb - 1));
            const uint4* row = reinterpret_cast<const uint4*>(idx + (int64_t)(b0 + n) * W);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int h = hq + 4 * j;
                kv[i][j] = row[(h < nKV ? h : 0) * 16 + dq];
            }
        }
    };
    load_blocks(gw * SCORE_BPW);
    // qsum of every KV head into LDS (unconditional loads, indices clamped: all in flight at once)
    __shared__ float qsum[16 * ATT_D];
#pragma unroll
    for (int r = 0; r < 16 * ATT_D / 256; r++) {
        const int i = threadIdx.x + 256 * r, h = i / ATT_D, d = i % ATT_D;
        float x[ATT_MAXG];
#pragma unroll
        for (int g = 0; g < ATT_MAXG; g++) x[g] = q[(int64_t)min(h * G + min(g, G - 1), nH - 1) * ATT_D + d];
        float sum = 0.0f;
#pragma unroll
        for (int g = 0; g < ATT_MAXG; g++) sum += g < G ? x[g] : 0.0f;
        if (i < W) qsum[i] = sum;
    }
    __syncthreads();
    float qv[4][8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int h = hq + 4 * j;
#pragma unroll
        for (int e = 0; e < 8; e++) qv[j][e] = h < nKV ? qsum[h * ATT_D + 8 * dq + e] : 0.0f;
    }
    for (int nbase = gw * SCORE_BPW; nbase < nb; nbase += nw * SCORE_BPW) {
        if (nbase != gw * SCORE_BPW) load_blocks(nbase);
#pragma unroll
        for (int i = 0; i < SCORE_BPW; i++) {
            const int n = nbase + i;
            float sj[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float f[8];
                bf16x8_to_f32(kv[i][j], f);
                float s = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) s = fmaf(qv[j][e], f[e], s);
                sj[j] = row16_sum(s);   // the head's 16 lanes
            }
            if (rows == 1) {
                const float tot = xor32_sum(xor16_sum((sj[0] + sj[1]) + (sj[2] + sj[3])));
                if (lane == 0 && n < nb) scores[n] = tot;
            } else if (dq == 0 && n < nb) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (hq + 4 * j < nKV) scores[(int64_t)(hq + 4 * j) * score_stride + n] = sj[j];
            }
        }
    }
}
static int score_grid(int nb) { return std::max(1, std::min((nb + 4 * SCORE_BPW - 1) / (4 * SCORE_BPW), 2048)); }
hipError_t launch_sparse_score(const SparseArgs& a, hipStream_t s) {
    if (a.D != ATT_D || a.nKV > 16 || a.nH % a.nKV || a.nH / a.nKV > ATT_MAXG) return hipErrorInvalidValue;
    hipLaunchKernelGGL(sparse_score_kernel, dim3(score_grid(a.max_blocks)), dim3(256), 0, s, a.q, (const uint16_t*)a.idx,
                       a.scores, a.nH, a.nKV, a.rows, a.max_blocks, reinterpret_cast<const SparsePlanDev*>(a.dplan), 0, 0);
    return hipGetLastError();
}
hipError_t launch_sparse_score_plan(const float* q, const uint16_t* idx, float* scores, int nH, int nKV, int D,
                                    int b0, int nb, int rows, hipStream_t s) {
    if (D != ATT_D || nKV > 16 || nH % nKV || nH / nKV > ATT_MAXG) return hipErrorInvalidValue;
    hipLaunchKernelGGL(sparse_score_kernel, dim3(score_grid(nb)), dim3(256), 0, s, q, idx, scores, nH, nKV, rows, nb,
                       (const SparsePlanDev*)nullptr, b0, nb);
    return hipGetLastError();
}

__device__ __forceinline__ uint32_t sparse_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exact selection (Kernels.swift:1628-1710): the p highest keys (ties: earlier block first), the
// attended positions written in ascending order. One 1024-thread workgroup per row.
// The row's keys are read once into LDS. Four 8-bit radix passes find the p-th largest key. The
// histogram has 16 copies (lane % 16 picks one), so lanes adding to the same bin, common in the
// leading passes, rarely hit the same LDS address; one wave sums the copies and scans the 256 bins
// with a lane prefix sum. A final
// pass counts, per thread's contiguous range, keys above the threshold and equal to it, and a
// workgroup scan gives each range its output slots.
constexpr int SEL_NT = 1024;
constexpr int SEL_MAXN = 32768;   // keys per row held in LDS (max; 128 KiB beside the 16 KiB histogram)
__global__ __launch_bounds__(SEL_NT) void sparse_select_kernel(const float* all_scores, int* all_lists, int list_stride,
                                                               int score_stride, const SparsePlanDev* plan,
                                                               SparsePlanDev fixed) {
    extern __shared__ uint32_t keys[];
    constexpr int HC = 16;                      // histogram copies
    __shared__ uint32_t hist[256 * HC];         // [bin][copy]
    __shared__ uint32_t pick[2];
    __shared__ uint32_t sgt[16], seq_[16];
    SparsePlanDev P = fixed;
    if (plan) { if (!plan->valid) return; P = *plan; }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int N = P.nb, row = blockIdx.x;
    const float* scores = all_scores + (int64_t)row * score_stride;
    int* list = all_lists + (int64_t)row * list_stride;
    for (int nb = 0; nb < N; nb += 8 * SEL_NT) {   // eight loads in flight per thread
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) { const int n = nb + i * SEL_NT + tid; v[i] = n < N ? scores[n] : 0.0f; }
#pragma unroll
        for (int i = 0; i < 8; i++) { const int n = nb + i * SEL_NT + tid; if (n < N) keys[n] = sparse_key(v[i]); }
    }
    uint32_t prefix = 0, mask = 0, want = (uint32_t)P.p;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256 * HC; i += SEL_NT) hist[i] = 0;
        __syncthreads();
        for (int n = tid; n < N; n += SEL_NT) {
            const uint32_t k = keys[n];
            if ((k & mask) == prefix) atomicAdd(&hist[((k >> shift) & 255u) * HC + (lane & (HC - 1))], 1u);
        }
        __syncthreads();
        if (wave == 0) {
            // lane l: bins 255 - 4l .. 252 - 4l (descending); inclusive prefix over lanes = keys in bins >= 252 - 4l
            uint32_t c[4], tot = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint4* h4 = reinterpret_cast<const uint4*>(hist + (255 - 4 * lane - i) * HC);
                uint32_t sum = 0;
#pragma unroll
                for (int q = 0; q < HC / 4; q++) { const uint4 v = h4[q]; sum += (v.x + v.y) + (v.z + v.w); }
                c[i] = sum; tot += sum;
            }
            uint32_t inc = tot;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t v = __shfl_up(inc, o, 64);
                if (lane >= o) inc += v;
            }
            const uint64_t hit = __ballot(inc >= want);
            const int first = __ffsll((long long)hit) - 1;   // exists: the last lane holds every candidate
            if (lane == first) {
                uint32_t acc = inc - tot;
                int i = 0;
                for (; i < 3; i++) {
                    if (acc + c[i] >= want) break;
                    acc += c[i];
                }
                pick[0] = (uint32_t)(255 - 4 * lane - i); pick[1] = want - acc;
            }
        }
        __syncthreads();
        prefix |= pick[0] << shift; mask |= 255u << shift; want = pick[1];
    }
    const int chunk = (N + SEL_NT - 1) / SEL_NT;
    const int n0 = min(N, tid * chunk), n1 = min(N, n0 + chunk);
    uint32_t gt = 0, eq = 0;
    for (int n = n0; n < n1; n++) { const uint32_t k = keys[n]; gt += k > prefix; eq += k == prefix; }
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
    const uint32_t gtB = gbase + gx - gt, eqB = ebase + ex - eq;
    uint32_t kept = gtB + min(eqB, want), tie = eqB;
    for (int n = n0; n < n1; n++) {
        const uint32_t k = keys[n];
        bool take = k > prefix;
        if (k == prefix) { take = tie < want; tie++; }
        if (take && kept < (uint32_t)P.p) {
            const int base = (P.b0 + n) * 4;
            int* o = list + P.sink_end + (int)kept * 4;
            if ((reinterpret_cast<uintptr_t>(o) & 15) == 0) *reinterpret_cast<int4*>(o) = int4{base, base + 1, base + 2, base + 3};
            else { o[0] = base; o[1] = base + 1; o[2] = base + 2; o[3] = base + 3; }
            kept++;
        }
    }
    for (int i = tid; i < P.sink_end; i += SEL_NT) list[i] = i;
    const int w0 = P.sink_end + P.p * 4;
    for (int i = tid; i < P.L - P.win_start; i += SEL_NT) list[w0 + i] = P.win_start + i;
}
static hipError_t select_launch(const float* scores, int* lists, int list_stride, int rows, int score_stride, int max_n,
                                const SparsePlanDev* plan, const SparsePlanDev& fixed, hipStream_t s) {
    if (max_n > SEL_MAXN) return hipErrorInvalidValue;
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute((const void*)sparse_select_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 SEL_MAXN * 4);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL(sparse_select_kernel, dim3(rows), dim3(SEL_NT), (size_t)std::max(max_n, 1) * 4, s, scores, lists, list_stride,
                       score_stride, plan, fixed);
    return hipGetLastError();
}
hipError_t launch_sparse_select(const SparseArgs& a, hipStream_t s) {
    return select_launch(a.scores, a.lists, a.list_stride, a.rows, a.max_blocks, a.max_blocks,
                         reinterpret_cast<const SparsePlanDev*>(a.dplan), SparsePlanDev{}, s);
}
hipError_t launch_sparse_select_plan(const float* scores, int* lists, int list_stride, int rows, int b0, int nb, int p,
                                     int sink_end, int win_start, int L, hipStream_t s) {
    SparsePlanDev P{1, b0, nb, p, sink_end, win_start, L, sink_end + p * 4 + (L - win_start)};
    return select_launch(scores, lists, list_stride, rows, nb, nb, nullptr, P, s);
}

}  // namespace mlxr
