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
    int s = 0;
    for (; s + 8 <= NS; s += 8) {
        float v[8], l[8];
#pragma unroll
        for (int i = 0; i < 8; i++) { v[i] = acc[(int64_t)(s + i) * D]; l[i] = lrow[s + i]; }
#pragma unroll
        for (int i = 0; i < 8; i++) { Ls += l[i] * w[s + i]; o += v[i] * w[s + i]; }
    }
    for (; s < NS; s++) { Ls += lrow[s] * w[s]; o += acc[(int64_t)s * D] * w[s]; }
    a.out[(int64_t)t * a.out_stride + (int64_t)h * D + d] = o / Ls;
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
    // qsum of every KV head into LDS (loads unrolled with guards: all in flight at once)
    __shared__ float qsum[16 * ATT_D];
#pragma unroll
    for (int r = 0; r < 16 * ATT_D / 256; r++) {
        const int i = threadIdx.x + 256 * r, h = i / ATT_D, d = i % ATT_D;
        float x[ATT_MAXG];
#pragma unroll
        for (int g = 0; g < ATT_MAXG; g++) x[g] = i < W && g < G ? q[(int64_t)(h * G + g) * ATT_D + d] : 0.0f;
        float sum = 0.0f;
#pragma unroll
        for (int g = 0; g < ATT_MAXG; g++) sum += x[g];
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
        uint4 kv[SCORE_BPW][4];
#pragma unroll
        for (int i = 0; i < SCORE_BPW; i++) {
            const int n = min(nbase + i, nb - 1);
            const uint4* row = reinterpret_cast<const uint4*>(idx + (int64_t)(b0 + n) * W);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int h = hq + 4 * j;
                kv[i][j] = h < nKV ? row[h * 16 + dq] : uint4{0u, 0u, 0u, 0u};
            }
        }
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
