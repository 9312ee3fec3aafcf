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
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a, const SparsePlanDev* plan) {
    __shared__ float qs[ATT_MAXG][ATT_D];
    __shared__ float sc[ATT_MAXG][ATT_MAXC];
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
    for (int i = tid; i < G * D; i += 256) {
        const int g = i / D, d = i % D;
        qs[g][d] = a.q[(int64_t)t * a.q_stride + (int64_t)(kvh * G + g) * D + d] * a.scale;
    }
    __syncthreads();
    // scores
    for (int base = 0; base < nk; base += 64) {
        const int kk = base + (tid >> 2), qd = tid & 3;
        const bool ok = kk < nk;
        int j = n0 + (ok ? kk : 0);
        if (sparse) { j = list[j]; j = j < 0 ? 0 : (j > L - 1 ? L - 1 : j); }
        const uint16_t* kp = a.kc + kv_row(a.pt, a.nKV, kvh, j) * D + qd * 32;
        float kf[32];
#pragma unroll
        for (int v = 0; v < 4; v++) bf16x8_to_f32(reinterpret_cast<const uint4*>(kp)[v], kf + 8 * v);
        for (int g = 0; g < G; g++) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 32; e++) s = fmaf(qs[g][qd * 32 + e], kf[e], s);
            s += __shfl_xor(s, 1, 64);
            s += __shfl_xor(s, 2, 64);
            if (ok && qd == 0) sc[g][kk] = s;
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
    // P V: wave w takes keys w, w+4, ...; lane owns dims 2*lane, 2*lane+1
    float acc[ATT_MAXG][2];
#pragma unroll
    for (int g = 0; g < ATT_MAXG; g++) { acc[g][0] = 0.0f; acc[g][1] = 0.0f; }
    for (int kk = wave; kk < nk; kk += 4) {
        int j = n0 + kk;
        if (sparse) { j = list[j]; j = j < 0 ? 0 : (j > L - 1 ? L - 1 : j); }
        const uint32_t vv = reinterpret_cast<const uint32_t*>(a.vc + kv_row(a.pt, a.nKV, kvh, j) * D)[lane];
        const float v0 = __uint_as_float(vv << 16), v1 = __uint_as_float(vv & 0xffff0000u);
#pragma unroll
        for (int g = 0; g < ATT_MAXG; g++) {
            if (g < G) { const float p = sc[g][kk]; acc[g][0] = fmaf(p, v0, acc[g][0]); acc[g][1] = fmaf(p, v1, acc[g][1]); }
        }
    }
#pragma unroll
    for (int g = 0; g < ATT_MAXG; g++)
        if (g < G) { accs[wave][g][2 * lane] = acc[g][0]; accs[wave][g][2 * lane + 1] = acc[g][1]; }
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

// grid (nH, T); block D: merge the partials of one head in range order.
__global__ __launch_bounds__(128) void attn_combine_kernel(AttnArgs a) {
    const int h = blockIdx.x, t = blockIdx.y, d = threadIdx.x, D = ATT_D;
    const int rows = a.nH * a.nsplit;
    const float* pt_ = a.part + (int64_t)t * rows * (D + 2);
    float M = -1e30f;
    for (int s = 0; s < a.nsplit; s++) M = fmaxf(M, pt_[h * a.nsplit + s]);
    float Ls = 0.0f, o = 0.0f;
    for (int s = 0; s < a.nsplit; s++) {
        const int r = h * a.nsplit + s;
        const float f = expf(pt_[r] - M);
        Ls += pt_[rows + r] * f;
        o += pt_[2 * rows + (int64_t)r * D + d] * f;
    }
    a.out[(int64_t)t * a.out_stride + (int64_t)h * D + d] = o / Ls;
}

static hipError_t attn_launch(const AttnArgs& a, const SparsePlanDev* plan, hipStream_t s) {
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

// Block scores (Kernels.swift:1565-1612): one thread per (row, block); q sums per KV head in LDS.
__global__ __launch_bounds__(256) void sparse_score_kernel(const float* q, const uint16_t* idx, float* scores, int nH,
                                                           int nKV, int D, int rows, int score_stride,
                                                           const SparsePlanDev* plan, int b0_, int nb_) {
    __shared__ float qsum[4096];
    const int W = nKV * D, G = nH / nKV;
    int b0 = b0_, nb = nb_;
    if (plan) { if (!plan->valid) return; b0 = plan->b0; nb = plan->nb; }
    for (int i = threadIdx.x; i < W; i += 256) {
        const int h = i / D, d = i % D;
        float s = 0.0f;
        for (int g = 0; g < G; g++) s += q[(int64_t)(h * G + g) * D + d];
        qsum[i] = s;
    }
    __syncthreads();
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= nb) return;
    const uint16_t* row = idx + (int64_t)(b0 + n) * W;
    float tot = 0.0f;
    for (int h = 0; h < nKV; h++) {
        float s = 0.0f;
        for (int d = 0; d < D; d += 8) {
            float f[8];
            bf16x8_to_f32(*reinterpret_cast<const uint4*>(row + h * D + d), f);
#pragma unroll
            for (int e = 0; e < 8; e++) s = fmaf(qsum[h * D + d + e], f[e], s);
        }
        if (rows == 1) tot += s; else scores[(int64_t)h * score_stride + n] = s;
    }
    if (rows == 1) scores[n] = tot;
}
hipError_t launch_sparse_score(const SparseArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(sparse_score_kernel, dim3((a.max_blocks + 255) / 256), dim3(256), 0, s, a.q, (const uint16_t*)a.idx,
                       a.scores, a.nH, a.nKV, a.D, a.rows, a.max_blocks, reinterpret_cast<const SparsePlanDev*>(a.dplan), 0, 0);
    return hipGetLastError();
}
hipError_t launch_sparse_score_plan(const float* q, const uint16_t* idx, float* scores, int nH, int nKV, int D,
                                    int b0, int nb, int rows, hipStream_t s) {
    hipLaunchKernelGGL(sparse_score_kernel, dim3((nb + 255) / 256), dim3(256), 0, s, q, idx, scores, nH, nKV, D, rows, nb,
                       (const SparsePlanDev*)nullptr, b0, nb);
    return hipGetLastError();
}

__device__ __forceinline__ uint32_t sparse_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exact selection (Kernels.swift:1628-1710): the p highest keys (ties: earlier block first), the
// attended positions written in ascending order. One 1024-thread workgroup per row.
__global__ __launch_bounds__(1024) void sparse_select_kernel(const float* all_scores, int* all_lists, int list_stride,
                                                             int score_stride, const SparsePlanDev* plan,
                                                             SparsePlanDev fixed) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t pick[2];
    __shared__ uint32_t sgt[16], seq_[16];
    SparsePlanDev P = fixed;
    if (plan) { if (!plan->valid) return; P = *plan; }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6, NT = blockDim.x;
    const int N = P.nb, row = blockIdx.x;
    const float* scores = all_scores + (int64_t)row * score_stride;
    int* list = all_lists + (int64_t)row * list_stride;
    uint32_t prefix = 0, mask = 0, want = (uint32_t)P.p;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += NT) hist[i] = 0;
        __syncthreads();
        for (int n = tid; n < N; n += NT) {
            const uint32_t k = sparse_key(scores[n]);
            if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t acc = 0;
            for (int bin = 255; bin >= 0; bin--) {
                if (acc + hist[bin] >= want) { pick[0] = (uint32_t)bin; pick[1] = want - acc; break; }
                acc += hist[bin];
            }
        }
        __syncthreads();
        prefix |= pick[0] << shift; mask |= 255u << shift; want = pick[1];
        __syncthreads();
    }
    const int chunk = (N + NT - 1) / NT;
    const int n0 = min(N, tid * chunk), n1 = min(N, n0 + chunk);
    uint32_t gt = 0, eq = 0;
    for (int n = n0; n < n1; n++) { const uint32_t k = sparse_key(scores[n]); gt += k > prefix; eq += k == prefix; }
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
    (void)nw;
    const uint32_t gtB = gbase + gx - gt, eqB = ebase + ex - eq;
    uint32_t kept = gtB + min(eqB, want), tie = eqB;
    for (int n = n0; n < n1; n++) {
        const uint32_t k = sparse_key(scores[n]);
        bool take = k > prefix;
        if (k == prefix) { take = tie < want; tie++; }
        if (take && kept < (uint32_t)P.p) {
            const int base = (P.b0 + n) * 4;
            int* o = list + P.sink_end + (int)kept * 4;
            o[0] = base; o[1] = base + 1; o[2] = base + 2; o[3] = base + 3;
            kept++;
        }
    }
    for (int i = tid; i < P.sink_end; i += NT) list[i] = i;
    const int w0 = P.sink_end + P.p * 4;
    for (int i = tid; i < P.L - P.win_start; i += NT) list[w0 + i] = P.win_start + i;
}
hipError_t launch_sparse_select(const SparseArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(sparse_select_kernel, dim3(a.rows), dim3(1024), 0, s, (const float*)a.scores, a.lists, a.list_stride,
                       a.max_blocks, reinterpret_cast<const SparsePlanDev*>(a.dplan), SparsePlanDev{});
    return hipGetLastError();
}
hipError_t launch_sparse_select_plan(const float* scores, int* lists, int list_stride, int rows, int b0, int nb, int p,
                                     int sink_end, int win_start, int L, hipStream_t s) {
    SparsePlanDev P{1, b0, nb, p, sink_end, win_start, L, sink_end + p * 4 + (L - win_start)};
    hipLaunchKernelGGL(sparse_select_kernel, dim3(rows), dim3(1024), 0, s, scores, lists, list_stride, nb,
                       (const SparsePlanDev*)nullptr, P);
    return hipGetLastError();
}

}  // namespace mlxr
