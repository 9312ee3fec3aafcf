// Persistent decode step: the whole batch-1 token step (every layer, lm_head and the greedy token)
// in ONE launch of exactly one 512-thread workgroup per CU.
//
// Why: a kernel-per-op step issues ~5 launches per layer, and each launch boundary on MI355X costs
// ~1.6 us of idle HBM inside a hipGraph, which alone caps an 8B decode near half of the bandwidth
// roofline. Here every workgroup, before it waits for a phase's input, issues the loads of its share
// of that phase's weights (and of its K/V rows: the cache up to the previous position does not
// depend on the current step), so HBM streams while the inputs are still being produced.
//
// Phases per layer; each hands its output to the next through a tagged vector (value, tag pairs:
// a reader polls the elements it needs until the producing phase's tag appears, one round trip
// instead of a grid barrier plus a fetch):
//   A  q|k|v matvec      x = RMSNorm(h) * input_norm (each workgroup normalises h itself)
//   B  attention         per (KV head, key range): q/k-norm + RoPE of its heads, K/V append by the
//                        range holding the new position, scores, softmax partial, P.V; the last
//                        range of a KV head to finish merges the partials in range order
//   C  o_proj            h += W_o attn
//   D  gate|up           mlp = silu(W_g x) * (W_u x), x = RMSNorm(h) * post_norm
//   E  down              h += W_d mlp
// then lm_head (x = RMSNorm(h) * final_norm) with a per-workgroup argmax; the last workgroup to
// finish reduces them (largest logit, lowest index on ties: Kernels.swift:2343-2356) and writes the
// token to hist[pos + 1] and the host ring, and advances *dpos.
//
// Semantics per phase are those of the separate kernels (qmv.hip, misc.hip, attn.hip): fp32
// activations and accumulation, bf16 K/V. Matvec phases run on the matrix cores over the repacked
// weight tiles (the matvec section below).
//
// Safety: every wait for a tagged value spins with a bounded count; on expiry it raises an abort
// flag (device and host-mapped) that every later wait honours, so every wave reaches the end of the
// kernel and the host reports an error.
#include "mv.h"

namespace mlxr {

constexpr int MK_MAXG = 8;
constexpr int MK_HOWN = 256;         // residual rows of one workgroup in an accumulate phase (max)
constexpr int MK_MERGE_L = 2;        // attention partials of one merged output per lane (nsplit <= 128)

// ------------------------------------------------------------------------------- coherence
// Data one workgroup writes and another reads within the launch (h, q|k|v, attention partials and
// output, mlp, argmax partials) moves with agent-scope loads and stores, which are coherent across
// the eight XCDs' L2 caches, so no L2 writeback / invalidate (an agent-scope fence, ~10 us here)
// is ever needed. Weights and the K/V rows read within a launch are never written in it.
__device__ __forceinline__ float ld_ag(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_ag(const int* p) {
    return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte device-coherent load (the SC1 cache-policy bit, as agent-scope atomics use): vectors of
// data written by other workgroups in this launch. Batches of these are issued before any is used,
// so a phase pays one memory round trip, not one per element.
typedef unsigned int coh_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_coh4(const float* base, int i, int n) {   // floats i..i+3 of base[0..n)
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, n * 4, 0x00020000);
    const coh_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, i * 4, 0, 16);
    return float4{__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
}
__device__ __forceinline__ float ld_coh1(const float* base, int i, int n) {
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, n * 4, 0x00020000);
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, i * 4, 0, 16));
}

__device__ __forceinline__ void st_ag(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_ag(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ unsigned ld_ag(unsigned* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ unsigned add_ag(unsigned* p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------------------- tagged exchange
// Phase outputs other workgroups read (h, q|k|v, attention output, SiLU(g)*u) are (value, tag)
// pairs, each written by one 8-byte agent-scope store, so a reader sees the value and its tag
// together. The tag names the launch and the phase that produced the value: (launch << 10) +
// phase index. A reader polls the elements it needs until their tags appear; that one round trip
// replaces a grid barrier plus the fetch after it. No buffer is overwritten while it can still be
// read: every phase's consumers depend (through the next layer's full-vector reads) on every
// workgroup having moved past the phase, and h alternates between two buffers.
__device__ __forceinline__ unsigned phase_tag(unsigned launch, int idx) { return (launch << 10) + (unsigned)idx; }
__device__ __forceinline__ void st_tag(uint2* p, float v, unsigned tag) {
    const unsigned long long w = (unsigned long long)__float_as_uint(v) | ((unsigned long long)tag << 32);
    __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
struct TagWait { MegaSync* sync; int* abort_host; unsigned limit; };
// Gives up after tw.limit polls: raises the abort flags (every later wait returns at once and the
// host reports the step as failed), so every wave still reaches the end of the kernel.
__device__ __forceinline__ bool tag_spin(const TagWait& tw, unsigned& spins) {
    if (ld_ag(&tw.sync->abort)) return false;
    __builtin_amdgcn_s_sleep(1);
    if (++spins > tw.limit) {
        __hip_atomic_store(&tw.sync->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(tw.abort_host, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return false;
    }
    return true;
}
// Pairs i, i + 1 (i even) of base[0..n): two values once both carry the tag.
__device__ __forceinline__ float2 ld_tag2(const uint2* base, int i, int n, unsigned tag, const TagWait& tw) {
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint2*>(base), 0, n * 8, 0x00020000);
    coh_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, i * 8, 0, 16);
    unsigned spins = 0;
    while ((v.y != tag || v.w != tag) && tag_spin(tw, spins)) v = __builtin_amdgcn_raw_buffer_load_b128(r, i * 8, 0, 16);
    return float2{__uint_as_float(v.x), __uint_as_float(v.z)};
}
// N tagged values base[idx[i]] in one round trip: every load issued, then polled together until
// all carry `tag` (the ones still missing reissued each round).
template <int N>
__device__ __forceinline__ void ld_tagN(const uint2* base, int n, const int* idx, unsigned tag, const TagWait& tw, float* out) {
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint2*>(base), 0, n * 8, 0x00020000);
    typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
    u32x2v v[N];
#pragma unroll
    for (int q = 0; q < N; q++) v[q] = __builtin_amdgcn_raw_buffer_load_b64(r, idx[q] * 8, 0, 16);
    for (unsigned spins = 0;;) {
        bool ready = true;
#pragma unroll
        for (int q = 0; q < N; q++) ready &= v[q].y == tag;
        if (ready || !tag_spin(tw, spins)) break;
#pragma unroll
        for (int q = 0; q < N; q++)
            if (v[q].y != tag) v[q] = __builtin_amdgcn_raw_buffer_load_b64(r, idx[q] * 8, 0, 16);
    }
#pragma unroll
    for (int q = 0; q < N; q++) out[q] = __uint_as_float(v[q].x);
}
__device__ __forceinline__ float ld_tag1(const uint2* base, int i, int n, unsigned tag, const TagWait& tw) {
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint2*>(base), 0, n * 8, 0x00020000);
    typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
    u32x2v v = __builtin_amdgcn_raw_buffer_load_b64(r, i * 8, 0, 16);
    unsigned spins = 0;
    while (v.y != tag && tag_spin(tw, spins)) v = __builtin_amdgcn_raw_buffer_load_b64(r, i * 8, 0, 16);
    return __uint_as_float(v.x);
}

// Every layer's descriptors are copied into LDS at the start of a launch and read from there: a
// global load of a descriptor field would make its wait also wait for every global load and store
// the wave has in flight (that counter completes in order), such as the next phase's weight
// prefetch or the tagged results just stored, at every phase boundary.

// Profile marks (optional): wall clock of phase boundaries, per workgroup.
__device__ __forceinline__ void prof_mark(unsigned long long* prof, int ev) {
    if (prof && threadIdx.x == 0 && ev < MEGA_PROF_EVENTS) prof[(size_t)blockIdx.x * MEGA_PROF_EVENTS + ev] = wall_clock64();
}

// After every wave's mv_run: combines the partials and writes the phase's outputs (coherent stores
// for data other workgroups read). ARGMAX returns the workgroup's largest row (lowest index among
// equals; NaN rows never win) to every thread.
template <int MODE, int FB, bool HALF = false>
__device__ __forceinline__ MvResult mv_finish(const MvPhase& p, float unscale, int wg, int nwg, const float* part, uint2* out,
                                              unsigned tag, float* logits, const float* hown, float* red, int* redi) {
    lds_barrier();
    MvGeom<FB> g = mv_geom<FB>(p, wg, nwg, 0);
    if (HALF) g.NF *= 2;                         // the waves' ranges count half scale groups
    const int nfw = g.nt * g.NF;
    MvResult res{-INFINITY, 0x7fffffff};
    if (MODE == OUT_GATED) {
        for (int i = threadIdx.x; i < g.nt * 8; i += MK_THREADS) {
            const int tl = i >> 3, j = i & 7, o = 8 * (g.t0 + tl) + j;
            if (o < p.o1) {
                const float gv = tile_row(part, tl, j, nfw, g.NF) * unscale;
                const float uv = tile_row(part, tl, j + 8, nfw, g.NF) * unscale;
                st_tag(out + o, (gv / (1.0f + expf(-gv))) * uv, tag);
            }
        }
        return res;
    }
    for (int i = threadIdx.x; i < g.nt * 16; i += MK_THREADS) {
        const int row = 16 * g.t0 + i;
        if (row >= p.rows) break;
        const float v = tile_row(part, i >> 4, i & 15, nfw, g.NF) * unscale + row_bias(p, row);
        if (MODE == OUT_STORE) st_tag(out + row, v, tag);
        else if (MODE == OUT_ADD) st_tag(out + row, hown[i] + v, tag);
        else {
            logits[row] = v;   // read by the host after the launch
            if (v > res.best) { res.best = v; res.best_idx = row; }
        }
    }
    if (MODE == OUT_ARGMAX) {
        // workgroup reduction: larger value, then lower index
        float m = res.best; int idx = res.best_idx;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float m2 = __shfl_xor(m, o, 64); const int i2 = __shfl_xor(idx, o, 64);
            if (m2 > m || (m2 == m && i2 < idx)) { m = m2; idx = i2; }
        }
        if ((threadIdx.x & 63) == 0) { red[threadIdx.x >> 6] = m; redi[threadIdx.x >> 6] = idx; }
        lds_barrier();
        res.best = -INFINITY; res.best_idx = 0x7fffffff;
        for (int w = 0; w < MK_WAVES; w++)
            if (red[w] > res.best || (red[w] == res.best && redi[w] < res.best_idx)) { res.best = red[w]; res.best_idx = redi[w]; }
    }
    return res;
}

// Loads the tagged vector src[0..K) (written by other workgroups) into xf (f32, contiguous):
// MK_LDB 16-byte loads (two pairs each) per thread in flight per batch, each polled until its tag
// appears; returns this thread's sum of squares and max |x|.
constexpr int MK_LDB = 4;
template <int NB = MK_LDB>
__device__ __forceinline__ float2 fetch_to_lds(const uint2* src, int K, unsigned tag, const TagWait& tw, float* xf) {
    float ss = 0.0f, mx = 0.0f;
    const int K2 = K >> 1;
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint2*>(src), 0, K * 8, 0x00020000);
    for (int base = 0; base < K2; base += MK_THREADS * NB) {
        coh_u32x4 v[NB];
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int i2 = min(base + j * MK_THREADS + (int)threadIdx.x, K2 - 1);
            v[j] = __builtin_amdgcn_raw_buffer_load_b128(r, i2 * 16, 0, 16);
        }
        // poll the batch: every round reissues all loads still missing their tag together
        for (unsigned spins = 0;;) {
            bool ready = true;
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const int i2 = base + j * MK_THREADS + (int)threadIdx.x;
                ready &= i2 >= K2 || (v[j].y == tag && v[j].w == tag);
            }
            if (ready || !tag_spin(tw, spins)) break;
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const int i2 = base + j * MK_THREADS + (int)threadIdx.x;
                if (i2 < K2 && (v[j].y != tag || v[j].w != tag)) v[j] = __builtin_amdgcn_raw_buffer_load_b128(r, i2 * 16, 0, 16);
            }
        }
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int i2 = base + j * MK_THREADS + (int)threadIdx.x;
            if (i2 < K2) {
                const float x0 = __uint_as_float(v[j].x), x1 = __uint_as_float(v[j].z);
                *reinterpret_cast<float2*>(xf + i2 * 2) = float2{x0, x1};
                ss += x0 * x0 + x1 * x1;
                mx = fmaxf(mx, fmaxf(fabsf(x0), fabsf(x1)));
            }
        }
    }
    return float2{ss, mx};
}

// Workgroup max of a non-negative per-thread value (red[8..15] as scratch; ends with a barrier).
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[8 + (threadIdx.x >> 6)] = v;
    lds_barrier();
    float m = 0.0f;
    for (int i = 0; i < MK_WAVES; i++) m = fmaxf(m, red[8 + i]);
    return m;
}


// A norm's weights as each thread uses them in norm_to_lds (float4 i = threadIdx.x + MK_THREADS j),
// loaded into registers before the phase's weight prefetch: issued later, they would complete
// behind it (the memory counter completes in order) and add a round trip after the input arrives.
constexpr int MK_NWR = 2;             // float4 per thread (norms of up to 4096 values)
struct NormW { float4 v[MK_NWR]; };
__device__ __forceinline__ NormW norm_w_load(const float* w, int K) {
    NormW r;
#pragma unroll
    for (int j = 0; j < MK_NWR; j++) {
        const int i = 4 * (threadIdx.x + MK_THREADS * j);
        r.v[j] = i < K ? gload4(w + i) : float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    return r;
}

// x := RMSNorm(src) * w, packed to the f16 matvec layout (every workgroup computes the same
// values). Returns the unscale factor of the packing. wr: norm_w_load(w, K) (K <= 4096); longer
// norms load w here.
__device__ __forceinline__ float norm_to_lds(const uint2* src, unsigned tag, const TagWait& tw, const float* w, const NormW& wr,
                                            int K, float eps, const MvLds& L, int gsh, float* red) {
    const float ss = wave_sum(fetch_to_lds(src, K, tag, tw, L.xf).x);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    lds_barrier();
    float tot = 0.0f;
    for (int i = 0; i < MK_WAVES; i++) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)K + eps);
    float mx = 0.0f;
    for (int i = threadIdx.x * 4, j = 0; i < K; i += MK_THREADS * 4, j++) {
        float4 v = *reinterpret_cast<float4*>(L.xf + i);
        float4 ww = wr.v[0];
#pragma unroll
        for (int q = 1; q < MK_NWR; q++)
            if (j == q) ww = wr.v[q];
        if (K > 4 * MK_THREADS * MK_NWR) ww = gload4(w + i);
        v.x = v.x * inv * ww.x; v.y = v.y * inv * ww.y; v.z = v.z * inv * ww.z; v.w = v.w * inv * ww.w;
        *reinterpret_cast<float4*>(L.xf + i) = v;
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    return pack_x16(L.xf, K, block_max(mx, red), L, gsh);
}

// x := src packed to the f16 matvec layout, plus this workgroup's residual rows h[row0 .. row1)
// into hown (for the accumulate epilogue, so no row needs its own round trip).
template <int NB = MK_LDB>
__device__ __forceinline__ float copy_to_lds(const uint2* src, unsigned tag, const TagWait& tw, int K, const MvLds& L, int gsh,
                                             const uint2* h, unsigned htag, int H, int row0, int row1, float* red) {
    const int n = row1 - row0;
    // the residual row was written phases ago: its load is issued first and checked only after the
    // input's loads, so it adds no round trip of its own
    const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint2*>(h), 0, H * 8, 0x00020000);
    typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
    const int hi = min(row0 + (int)threadIdx.x, H - 1);
    u32x2v hv = __builtin_amdgcn_raw_buffer_load_b64(hr, hi * 8, 0, 16);
    const float mx = fetch_to_lds<NB>(src, K, tag, tw, L.xf).y;
    if ((int)threadIdx.x < n) {
        for (unsigned spins = 0; hv.y != htag && tag_spin(tw, spins);) hv = __builtin_amdgcn_raw_buffer_load_b64(hr, hi * 8, 0, 16);
        L.hown[threadIdx.x] = __uint_as_float(hv.x);
    }
    return pack_x16(L.xf, K, block_max(mx, red), L, gsh);
}

// ------------------------------------------------------------------------------- attention phase
// K and V of one chunk of 128 keys held in registers: k[db] is the lane's A-operand slice of the
// wave's 16 keys (dims 32 db + 8 (lane >> 4) .. +8 of key 16 wave + (lane & 15)); v[r] is the
// thread's P.V slice (dims 4 (tid & 31) .. +4 of key 8 (tid >> 5) + r).
struct KVPrefetch { uint4 k[4]; uint2 v[8]; };

// The thread index, opaque to the compiler: offsets derived from it in the attention phase are
// recomputed where used instead of being hoisted out of the layer loop and held in scratch memory
// (a reload from scratch waits, in order, for every load issued before it, such as the K / V rows).
__device__ __forceinline__ int att_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Key range of attention item (kvh, split): [n0, n1) of the L = pos + 1 keys.
__device__ __forceinline__ void att_range(int L, int nsplit, int split, int& n0, int& n1) {
    const int c = (L + nsplit - 1) / nsplit;
    n0 = min(L, split * c); n1 = min(L, n0 + c);
}

// Loads chunk c of keys [n0, nf) (nf: the first key not yet final in the cache; keys past it are
// clamped to a final row and replaced or masked by the caller).
// Every path defines the registers, so no earlier value stays live across phases.
__device__ __forceinline__ void att_load_k(const MegaArgs& a, const LayerDev& ly, int kvh, int kb, int nf, int pg0, int e0, int e1,
                                           KVPrefetch& pf);
__device__ __forceinline__ void att_load_v(const MegaArgs& a, const LayerDev& ly, int kvh, int kb, int nf, int pg0, int e0, int e1,
                                           KVPrefetch& pf);
__device__ __forceinline__ void att_prefetch_k(const MegaArgs& a, const int* pt, const LayerDev& ly, int kvh, int n0, int nf, int c, KVPrefetch& pf) {
    if (nf <= n0) {
#pragma unroll
        for (int db = 0; db < 4; db++) pf.k[db] = uint4{0u, 0u, 0u, 0u};
        return;
    }
    const int t = att_tid(), lane = t & 63, wave = t >> 6;
    const int kb = n0 + 128 * c + 16 * wave;            // the wave's 16 keys span at most two pages
    const int jf = min(kb, nf - 1), jl = min(kb + 15, nf - 1);
    const int pg0 = jf >> MLXR_PAGE_SHIFT, e0 = pt[pg0], e1 = pt[jl >> MLXR_PAGE_SHIFT];
    att_load_k(a, ly, kvh, kb, nf, pg0, e0, e1, pf);
}
// K rows of the wave's 16 keys from kb, with the page entries of the first and last already loaded.
__device__ __forceinline__ void att_load_k(const MegaArgs& a, const LayerDev& ly, int kvh, int kb, int nf, int pg0, int e0, int e1,
                                           KVPrefetch& pf) {
    const int lane = att_tid() & 63;
    const int jk = min(kb + (lane & 15), nf - 1);
    const int64_t rk = ((int64_t)(((jk >> MLXR_PAGE_SHIFT) == pg0 ? e0 : e1) * a.nKV + kvh) * MLXR_PAGE + (jk & (MLXR_PAGE - 1))) * 128 +
                       8 * (lane >> 4);
#pragma unroll
    for (int db = 0; db < 4; db++) pf.k[db] = ld_stream16((gptr8)(ly.kc + rk + 32 * db));
}
__device__ __forceinline__ void att_prefetch_v(const MegaArgs& a, const int* pt, const LayerDev& ly, int kvh, int n0, int nf, int c, KVPrefetch& pf) {
    if (nf <= n0) {
#pragma unroll
        for (int r = 0; r < 8; r++) pf.v[r] = uint2{0u, 0u};
        return;
    }
    const int t = att_tid();
    const int kb = n0 + 128 * c + 8 * (t >> 5);          // the thread's 8 keys span at most two pages
    const int jf = min(kb, nf - 1), jl = min(kb + 7, nf - 1);
    const int pg0 = jf >> MLXR_PAGE_SHIFT, e0 = pt[pg0], e1 = pt[jl >> MLXR_PAGE_SHIFT];
    att_load_v(a, ly, kvh, kb, nf, pg0, e0, e1, pf);
}
// V slices of the thread's 8 keys from kb, with the page entries of the first and last already loaded.
__device__ __forceinline__ void att_load_v(const MegaArgs& a, const LayerDev& ly, int kvh, int kb, int nf, int pg0, int e0, int e1,
                                           KVPrefetch& pf) {
    const int t = att_tid();
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int jv = min(kb + r, nf - 1);
        const int64_t rv = ((int64_t)(((jv >> MLXR_PAGE_SHIFT) == pg0 ? e0 : e1) * a.nKV + kvh) * MLXR_PAGE + (jv & (MLXR_PAGE - 1))) * 128;
        typedef const __attribute__((address_space(1))) unsigned long long* gptr64;
        const unsigned long long v = *(gptr64)(ly.vc + rv + 4 * (t & 31));
        pf.v[r] = uint2{(uint32_t)v, (uint32_t)(v >> 32)};
    }
}
// Chunk 1 (keys n0 + 128 .. n0 + 255) of a range longer than 128 keys, copied by buffer->LDS DMA into
// kvl right after the q|k|v matvec: K rows [128][256 B] (16-byte piece j of row r stored at piece
// j ^ (r & 15), so the 16 rows a wave's A-operand load reads together fall in different LDS banks),
// then V rows. Keys at or past nf are clamped
// to a final row, and groups of 4 rows that start at or past nf are not copied (the caller replaces
// the new key and reads no row past the range). Each wave moves its
// 16 keys' K and V rows, 4 rows (1 KiB) per instruction. Byte offsets fit 32 bits (checked at setup).
typedef __attribute__((address_space(3))) void* att_lptr;
constexpr int ATT_KVL_OFF = 53248;
constexpr int ATT_PPS = 260;           // row stride (floats) of the attention phase's probabilities     // byte offset of the staged chunk in the workgroup's LDS
constexpr int ATT_KVL_BYTES = 65536;
__device__ __forceinline__ void att_stage1(const MegaArgs& a, const LayerDev& ly, int kvh, int kb, int nf, int pg0, int e0, int e1,
                                           uint8_t* kvl) {
    const int lane = att_tid() & 63, wave = att_tid() >> 6;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(ly.kc, 0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(ly.vc, 0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (kb + 4 * i >= nf) break;   // rows of keys past the cache's final ones are never read
        const int j = min(kb + 4 * i + (lane >> 4), nf - 1);
        const uint32_t row = (uint32_t)((((j >> MLXR_PAGE_SHIFT) == pg0 ? e0 : e1) * a.nKV + kvh) * MLXR_PAGE + (j & (MLXR_PAGE - 1))) * 256u;
        const uint32_t pk = (uint32_t)((lane & 15) ^ ((4 * i + (lane >> 4)) & 15));   // LDS row 16 wave + 4 i + (lane >> 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (att_lptr)(kvl + (16 * wave + 4 * i) * 256), 16, row + 16u * pk, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (att_lptr)(kvl + 32768 + (16 * wave + 4 * i) * 256), 16, row + 16u * (lane & 15), 0, 0, 0);
    }
}
// Start of the attention phase: chunk 0's K / V into registers and, for a staged range, chunk 1 into
// LDS; every page entry these need is loaded first, together (one round trip before the data loads).
__device__ __forceinline__ void att_begin(const MegaArgs& a, const int* pt, const LayerDev& ly, int kvh, int n0, int nf, bool staged,
                                          uint8_t* kvl, KVPrefetch& pf) {
    if (nf <= n0) {
#pragma unroll
        for (int db = 0; db < 4; db++) pf.k[db] = uint4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int r = 0; r < 8; r++) pf.v[r] = uint2{0u, 0u};
        return;
    }
    const int t = att_tid(), wave = t >> 6;
    const int kk = n0 + 16 * wave, kv = n0 + 8 * (t >> 5), ks = n0 + 128 + 16 * wave;
    const int pk = min(kk, nf - 1) >> MLXR_PAGE_SHIFT, pv = min(kv, nf - 1) >> MLXR_PAGE_SHIFT, ps = min(ks, nf - 1) >> MLXR_PAGE_SHIFT;
    const int ek0 = pt[pk], ek1 = pt[min(kk + 15, nf - 1) >> MLXR_PAGE_SHIFT];
    const int ev0 = pt[pv], ev1 = pt[min(kv + 7, nf - 1) >> MLXR_PAGE_SHIFT];
    const int es0 = pt[ps], es1 = pt[min(ks + 15, nf - 1) >> MLXR_PAGE_SHIFT];
    att_load_k(a, ly, kvh, kk, nf, pk, ek0, ek1, pf);
    att_load_v(a, ly, kvh, kv, nf, pv, ev0, ev1, pf);
    if (staged) att_stage1(a, ly, kvh, ks, nf, ps, es0, es1, kvl);
}

__device__ __forceinline__ void unpack_bf16x8(const uint4 v, float* o) {
    o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
    o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
    o[4] = __uint_as_float(v.z << 16); o[5] = __uint_as_float(v.z & 0xffff0000u);
    o[6] = __uint_as_float(v.w << 16); o[7] = __uint_as_float(v.w & 0xffff0000u);
}

// head vector (128, in LDS buf) -> per-head RMSNorm (optional) -> RoPE, 128 threads of one group
// nwi: the norm weight of dimension i (loaded by the caller); rope: cos / sin of pos * inv_freq[f]
// for f < rot_dim / 2 (LDS, computed once per launch).
__device__ __forceinline__ float head_norm_rope(float v, int i, bool norm, float nwi, float eps, const float2* rope,
                                                int rot_dim, int traditional, float* buf, float* red, int grp) {
    // grp: which 128-thread group (0..3) of the workgroup; red has 2 floats per group
    if (norm) {
        float ss = wave_sum(v * v);
        if ((i & 63) == 0) red[grp * 2 + (i >> 6)] = ss;
        lds_barrier();
        const float tot = red[grp * 2] + red[grp * 2 + 1];
        v = v * (1.0f / sqrtf(tot / 128.0f + eps)) * nwi;
    } else {
        lds_barrier();
    }
    buf[i] = v;
    lds_barrier();
    float out = v;
    if (i < rot_dim) {
        const int half = rot_dim / 2;
        int fi, partner; bool first;
        if (traditional) { fi = i / 2; partner = i ^ 1; first = (i & 1) == 0; }
        else { fi = i % half; first = i < half; partner = first ? i + half : i - half; }
        const float2 cs = rope[fi];
        out = first ? v * cs.x - buf[partner] * cs.y : v * cs.x + buf[partner] * cs.y;
    }
    lds_barrier();
    return out;
}

// ------------------------------------------------------------------------------- the kernel
// MAXG: the largest query-head group the attention phase's registers hold (4 or 8).
// FB: code blocks per scale group (4: group size 32, 8: group size 64).
template <int MAXG, int FB>
__global__ __launch_bounds__(MK_THREADS, 1) void decode_step_kernel(MegaArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ float red[64];
    __shared__ int flag;
    const int wg = blockIdx.x, nwg = gridDim.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: row ranges stay scalar
    const int pos = *a.dpos, L = pos + 1;
    const int H = a.H, D = 128, nH = a.nH, nKV = a.nKV, G = nH / nKV;
    const int Kmax = std::max(H, std::max(a.I, nH * D));
    // matvec LDS: what mv_finish reads (partials, residual rows) lies below ATT_KVL_OFF, so the
    // attention phase's staging DMA may start as soon as a workgroup leaves the q|k|v matvec
    MvLds ml;
    ml.part = lds;                                // per-tile partial row sums [MK_TPW][waves][16]
    ml.hown = ml.part + MK_TPW * MK_WAVES * 16;   // this workgroup's residual rows (up to MK_HOWN)
    ml.xf = ml.hown + MK_HOWN;                    // matvec input, f32 staging (Kmax floats)
    ml.xh = ml.xf + Kmax;                         // matvec input, f16 layout (Kmax / 32 chunks)
    ml.gsum = ml.xh + (Kmax >> 5) * XH_STRIDE;    // per-group sums of x (Kmax / 32 at most)
    ml.zero16 = ml.gsum + (((Kmax >> 5) + 3) & ~3);   // MV_ZERO floats of zeros (16-byte aligned)
    __shared__ int redi[MK_WAVES];
    Ring<FB> ring;
    KVPrefetch kvpf;

    const unsigned launch = ld_ag(&a.sync->launch);
    const TagWait tw{a.sync, a.abort_host, a.spin_limit};
    // tags: embedding 1; layer l: q|k|v 2 + 5l, attention 3 + 5l, h after o_proj 4 + 5l,
    // SiLU(g)*u 5 + 5l, h after down 6 + 5l
    auto tag_of = [&](int idx) { return phase_tag(launch, idx); };
    // embedding row of hist[pos] -> hA (each workgroup writes a slice), and the first prefetch
    {
        const int tok = a.hist[pos];
        const int gpr = H / a.embed_gs;
        for (int c = wg * MK_THREADS + tid; c < H / 8; c += nwg * MK_THREADS) {
            const uint32_t w = reinterpret_cast<const uint32_t*>(a.embed_w + (int64_t)tok * (H / 2))[c];
            const int g = (c * 8) / a.embed_gs;
            const float s = bf16_to_f32(a.embed_s[(int64_t)tok * gpr + g]), b = bf16_to_f32(a.embed_b[(int64_t)tok * gpr + g]);
#pragma unroll
            for (int j = 0; j < 8; j++) st_tag(a.hA + c * 8 + j, (float)((w >> (4 * j)) & 15u) * s + b, tag_of(1));
        }
    }
    // the layers' descriptors into LDS (read at every phase; see above)
    LayerDev* ldesc = reinterpret_cast<LayerDev*>(reinterpret_cast<uint8_t*>(lds) + a.desc_lds_off);
    {
        static_assert(sizeof(LayerDev) % 16 == 0, "descriptor copy in 16-byte units");
        typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
        const u32x4_t* src = reinterpret_cast<const u32x4_t*>(a.layers);
        u32x4_t* dst = reinterpret_cast<u32x4_t*>(ldesc);
        const int n = a.L * (int)(sizeof(LayerDev) / 16);
        for (int i = tid; i < n; i += MK_THREADS) dst[i] = gload(src + i);
    }
    // the page table too (the attention phase's row lookups must not wait on global traffic either)
    int* lpt = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(lds) + a.pt_lds_off);
    for (int i = tid; i < a.n_pages; i += MK_THREADS) lpt[i] = gload(a.pt + i);
    // RoPE cos / sin of this step's position (the angle of every layer's q and k)
    float2* rope = reinterpret_cast<float2*>(lpt + (a.n_pages + 3) / 4 * 4);
    if (tid < a.rot_dim / 2) {
        const float ang = (float)pos * gload(a.inv_freq + tid);
        rope[tid] = float2{cosf(ang), sinf(ang)};
    }
    lds_barrier();
    unsigned epoch = 0;                                   // phase boundaries of this launch (profile marks)
    prof_mark(a.prof, 0);
    prof_mark(a.prof, 2 * epoch); ++epoch;
    NormW nwr = norm_w_load(ldesc[0].in_norm, H);
    mvh_prefetch<FB>(ldesc[0].qkv, wg, nwg, wave, lane, ring);
    prof_mark(a.prof, 2 * epoch - 1);

    const int nsplit = nwg / nKV;
    for (int li = 0; li < a.L; li++) {
        // the step position, opaque per layer: what depends on it (the attention phase's key range,
        // page and row lookups) is computed in each layer where it is used, not once before the
        // loop and held (in scratch: there are not enough registers) across every phase
        int pos_l = pos;
        asm volatile("" : "+s"(pos_l));
        const LayerDev& ly = ldesc[li];
        // ---- A: q|k|v
        {
            unsigned itag = tag_of(li == 0 ? 1 : 6 + 5 * (li - 1));
            if (li == 0 && a.stall && wg == 0) itag ^= 0x80000000u;   // test hook: a tag no launch writes
            const float us = norm_to_lds(a.hA, itag, tw, ly.in_norm, nwr, H, a.eps, ml, FB == 4 ? 5 : 6, red);
            prof_mark(a.prof, 512 + 8 * li + 0);
            mvh_run<FB>(ly.qkv, ml.xh, ml.gsum, ml.zero16, wg, nwg, wave, lane, ring, ml.part);
            mv_finish<OUT_STORE, FB, true>(ly.qkv, us, wg, nwg, ml.part, a.qkvT, tag_of(2 + 5 * li), nullptr, nullptr, red, redi);
        }
        prof_mark(a.prof, 2 * epoch); ++epoch;
        // prefetch this workgroup's K/V rows (positions < pos are final)
        const int item = wg;                       // nwg == nKV * nsplit
        const int kvh = item / nsplit, split = item % nsplit;
        int n0, n1; att_range(pos_l + 1, nsplit, split, n0, n1);
        uint8_t* kvl = reinterpret_cast<uint8_t*>(lds) + ATT_KVL_OFF;
        const bool staged = a.kv_stage && n1 - n0 > 128;   // chunk 1 joins chunk 0's pass from LDS
        const int QKV = (nH + 2 * nKV) * D;
        // q / k norm + RoPE: with rot_dim 128 wave-local (lane l holds dims nd0, nd1 = (l, l + 64), or
        // (2 l, 2 l + 1) traditional; their norm weights load later, with the q / k values); else
        // one dim per thread (tid & 127), whose norm weights load here, before the K / V loads (the
        // memory counter completes in order: a load issued after them could only be used once
        // they are in)
        const bool wave_rope = a.rot_dim == 128;
        const int nd0 = wave_rope ? (a.traditional ? 2 * (tid & 63) : (tid & 63)) : (tid & 127);
        const int nd1 = a.traditional ? nd0 + 1 : nd0 + 64;
        const float qnw = ly.q_norm && !wave_rope ? gload(ly.q_norm + nd0) : 1.0f, knw = ly.k_norm && !wave_rope ? gload(ly.k_norm + nd0) : 1.0f;
        att_begin(a, lpt, ly, kvh, n0, min(n1, pos_l), staged, kvl, kvpf);
        prof_mark(a.prof, 2 * epoch - 1);

        // ---- B: attention for (kvh, split): scores on the matrix cores (K rows from the bf16 cache as
        // the A operand, q as bf16 hi + lo parts in B), softmax over chunks of 128 keys with running
        // max / sum, P.V on the vector units.
        typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
        const int nk = n1 - n0;
        const int prow = (kvh * G) * nsplit;             // partial rows: (head, split)
        // [2][16][128] bf16: q hi / lo; the 16-byte piece j of head row g at piece j ^ g, so the
        // 16 rows read together by a B-operand load fall in different LDS banks
        uint16_t* qb = reinterpret_cast<uint16_t*>(lds);
        uint16_t* kn16 = qb + 2 * 16 * 128;              // new key, bf16 [128]
        uint16_t* vn16 = kn16 + 128;                     // new value, bf16 [128]
        float* buf = reinterpret_cast<float*>(vn16 + 128);   // 4 x 128 rope scratch
        float* wred = buf + 4 * 128;                     // [2][waves][16] per-wave max, sum
        float* mls = wred + 2 * MK_WAVES * 16;           // [2][16] running max, sum per head
        // [MAXG][ATT_PPS] probabilities of the pass's 256 keys (rows padded so that the 16 heads'
        // 16-byte stores of one key quad fall in different LDS banks)
        float* pp = mls + 32;
        float* wacc = pp + MAXG * ATT_PPS;               // [waves][MAXG][128] P.V partials; merge scratch
        float* mrow = wacc + MK_WAVES * MAXG * 128;      // [MAXG] merge scale
        {
            const int tid = att_tid(), lane = tid & 63;
            const bool owns_new = pos_l >= n0 && pos_l < n1;
            const unsigned qtag = tag_of(2 + 5 * li);
            if (wave_rope) {
                // wave w takes item w (q head w < G, the new key at item G if this range holds pos);
                // a lane's two dims are each other's RoPE partners, so the norm is one wave sum and
                // the rotation needs no exchange
                const int wv = tid >> 6;
                const float2 cs = rope[lane];
                for (int it = wv; it < G + (owns_new ? 1 : 0); it += MK_WAVES) {
                    const bool isk = it == G;
                    const int col = isk ? (nH + kvh) * D : (kvh * G + it) * D;
                    // the norm weights load with the q / k values: both complete behind this range's
                    // K / V loads (issued first; the memory counter completes in order)
                    const float* nwp = isk ? ly.k_norm : ly.q_norm;
                    const float nw0 = nwp ? gload(nwp + nd0) : 1.0f, nw1 = nwp ? gload(nwp + nd1) : 1.0f;
                    // this item's two dims (and, for the new key, the value's two dims) in one round trip
                    const int vc = (nH + nKV + kvh) * D;
                    const int ix[4] = {col + nd0, col + nd1, isk ? vc + nd0 : col + nd0, isk ? vc + nd1 : col + nd1};
                    float got[4];
                    ld_tagN<4>(a.qkvT, QKV, ix, qtag, tw, got);
                    float v0 = got[0], v1 = got[1];
                    if (nwp) {
                        const float r = 1.0f / sqrtf(wave_sum(v0 * v0 + v1 * v1) / 128.0f + a.eps);
                        v0 = v0 * r * nw0;
                        v1 = v1 * r * nw1;
                    }
                    const float o0 = v0 * cs.x - v1 * cs.y, o1 = v1 * cs.x + v0 * cs.y;
                    if (isk) {
                        const uint16_t k0 = f32_to_bf16(o0), k1 = f32_to_bf16(o1);
                        const uint16_t w0 = f32_to_bf16(got[2]), w1 = f32_to_bf16(got[3]);
                        kn16[nd0] = k0; kn16[nd1] = k1; vn16[nd0] = w0; vn16[nd1] = w1;
                        const int64_t row = kv_row(lpt, nKV, kvh, pos_l) * 128;
                        gstore(ly.kc + row + nd0, k0); gstore(ly.kc + row + nd1, k1);
                        gstore(ly.vc + row + nd0, w0); gstore(ly.vc + row + nd1, w1);
                    } else {
                        const float q[2] = {o0 * a.scale, o1 * a.scale};
                        const int dd[2] = {nd0, nd1};
#pragma unroll
                        for (int e = 0; e < 2; e++) {
                            const uint16_t hi = f32_to_bf16(q[e]);
                            const int si = it * 128 + (((dd[e] >> 3) ^ it) << 3) + (dd[e] & 7);
                            qb[si] = hi;
                            qb[2048 + si] = f32_to_bf16(q[e] - bf16_to_f32(hi));
                        }
                    }
                }
            } else {
            // q heads (4 per pass of 512 threads), then the new k and v if this range holds pos
            const int grp = tid >> 7, i = tid & 127;
            // every value this workgroup needs from q|k|v, loaded at once
            const int ix[4] = {(kvh * G + min(grp, G - 1)) * D + i, (kvh * G + min(grp + 4, G - 1)) * D + i,
                               (nH + kvh) * D + i, (nH + nKV + kvh) * D + i};
            float got[4];
            ld_tagN<4>(a.qkvT, QKV, ix, qtag, tw, got);
            const float qv0 = got[0], qv1 = got[1], kraw = got[2], vraw = got[3];
            for (int base = 0; base < G; base += 4) {
                const int g = base + grp;
                const float v = g < G ? (base == 0 ? qv0 : qv1) : 0.0f;
                const float o = head_norm_rope(v, i, ly.q_norm != nullptr, qnw, a.eps, rope, a.rot_dim, a.traditional, buf + grp * 128, red, grp);
                if (g < G) {
                    const float q = o * a.scale;
                    const uint16_t hi = f32_to_bf16(q);
                    const int si = g * 128 + (((i >> 3) ^ g) << 3) + (i & 7);
                    qb[si] = hi;
                    qb[2048 + si] = f32_to_bf16(q - bf16_to_f32(hi));
                }
            }
            if (owns_new) {
                const float ko = head_norm_rope(tid < 128 ? kraw : 0.0f, i, ly.k_norm != nullptr, knw, a.eps, rope, a.rot_dim, a.traditional, buf + grp * 128, red, grp);
                if (tid < 128) {
                    const uint16_t kb = f32_to_bf16(ko), vb = f32_to_bf16(vraw);
                    kn16[i] = kb; vn16[i] = vb;
                    const int64_t row = kv_row(lpt, nKV, kvh, pos_l) * 128 + i;
                    gstore(ly.kc + row, kb); gstore(ly.vc + row, vb);
                }
            }
            }
            for (int e = tid; e < 2 * (16 - G) * 128; e += MK_THREADS) {   // unused head columns: zero
                const int hl = e / ((16 - G) * 128), r = e - hl * (16 - G) * 128;
                qb[hl * 2048 + G * 128 + r] = 0;
            }
            if (tid < 32) mls[tid] = tid < 16 ? -1e30f : 0.0f;
            lds_barrier();
            prof_mark(a.prof, 512 + 8 * li + 7);

            float acc[MAXG][4];
#pragma unroll
            for (int g = 0; g < MAXG; g++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[g][e] = 0.0f;
            const int hh = lane & 15, d4 = tid & 31, slice = tid >> 5;
            const int nchunks = (nk + 127) >> 7;
            const int nf = min(n1, pos_l);
            for (int c = 0; c < nchunks;) {
                asm volatile("" ::: "memory");   // keeps the q reads in the loop (no registers held across chunks)
                // a staged range takes chunks 0 and 1 in one pass (chunk 1 from LDS)
                const bool pair = staged && c == 0;
                const int cn = c + (pair ? 2 : 1);
                // scores S[key][head] of the wave's 16 keys (and its 16 keys of chunk 1)
                const int kbase = n0 + 128 * c + 16 * wave;
                uint4* kq = kvpf.k;
                if (owns_new && kbase + (lane & 15) == pos_l) {   // only the owner wrote kn16 / vn16
#pragma unroll
                    for (int db = 0; db < 4; db++) kq[db] = *reinterpret_cast<const uint4*>(kn16 + 32 * db + 8 * (lane >> 4));
                }
                f32x4_t sacc = {0.0f, 0.0f, 0.0f, 0.0f}, sacc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int db = 0; db < 4; db++)
#pragma unroll
                    for (int hl = 0; hl < 2; hl++) {
                        const uint4 bq = *reinterpret_cast<const uint4*>(qb + hl * 2048 + hh * 128 + 8 * ((4 * db + (lane >> 4)) ^ hh));
                        sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kq[db]), __builtin_bit_cast(bf16x8_t, bq), sacc, 0, 0, 0);
                    }
                if (pair) {
                    __builtin_amdgcn_s_waitcnt(0x0070);    // this wave's DMA (vmcnt 0), then every wave's
                    __builtin_amdgcn_s_barrier();
                    const bool newk = owns_new && kbase + 128 + (lane & 15) == pos_l;
#pragma unroll
                    for (int db = 0; db < 4 && kbase + 128 < n1; db++) {   // none of the wave's keys in range: masked anyway
                        const uint16_t* src = newk ? kn16 + 32 * db + 8 * (lane >> 4)
                                                   : reinterpret_cast<const uint16_t*>(kvl + (16 * wave + (lane & 15)) * 256) +
                                                         8 * ((4 * db + (lane >> 4)) ^ (lane & 15));
                        const uint4 k1 = *reinterpret_cast<const uint4*>(src);
#pragma unroll
                        for (int hl = 0; hl < 2; hl++) {
                            const uint4 bq = *reinterpret_cast<const uint4*>(qb + hl * 2048 + hh * 128 + 8 * ((4 * db + (lane >> 4)) ^ hh));
                            sacc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, k1), __builtin_bit_cast(bf16x8_t, bq), sacc1, 0, 0, 0);
                        }
                    }
                }
                float sv[4], sv1[4], mloc = -INFINITY;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const bool ok = kbase + 4 * (lane >> 4) + r < n1;
                    sv[r] = ok ? sacc[r] : -INFINITY;
                    mloc = fmaxf(mloc, sv[r]);
                    const bool ok1 = pair && kbase + 128 + 4 * (lane >> 4) + r < n1;
                    sv1[r] = ok1 ? sacc1[r] : -INFINITY;
                    mloc = fmaxf(mloc, sv1[r]);
                }
                mloc = xor32_max(xor16_max(mloc));
                if (lane < 16) wred[lane * MK_WAVES + wave] = mloc;
                lds_barrier();
                // new running max per head; probabilities of this lane's keys
                const float4 wa = *reinterpret_cast<const float4*>(wred + hh * MK_WAVES);
                const float4 wb = *reinterpret_cast<const float4*>(wred + hh * MK_WAVES + 4);
                const float mnew_h = fmaxf(mls[hh], fmaxf(fmaxf(fmaxf(wa.x, wa.y), fmaxf(wa.z, wa.w)), fmaxf(fmaxf(wb.x, wb.y), fmaxf(wb.z, wb.w))));
                float lsum = 0.0f;
                float pq[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    pq[r] = expf(sv[r] - mnew_h);
                    lsum += pq[r];
                }
                if (hh < MAXG)
                    *reinterpret_cast<float4*>(pp + hh * ATT_PPS + 16 * wave + 4 * (lane >> 4)) =
                        hh < G ? float4{pq[0], pq[1], pq[2], pq[3]} : float4{0.0f, 0.0f, 0.0f, 0.0f};
                if (pair) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        pq[r] = expf(sv1[r] - mnew_h);
                        lsum += pq[r];
                    }
                    if (hh < MAXG)
                        *reinterpret_cast<float4*>(pp + hh * ATT_PPS + 128 + 16 * wave + 4 * (lane >> 4)) =
                            hh < G ? float4{pq[0], pq[1], pq[2], pq[3]} : float4{0.0f, 0.0f, 0.0f, 0.0f};
                }
                lsum = xor32_sum(xor16_sum(lsum));
                if (lane < 16) wred[MK_WAVES * 16 + lane * MK_WAVES + wave] = lsum;
                float alpha[MAXG];
#pragma unroll
                for (int g = 0; g < MAXG; g++) {
                    const float4 ga = *reinterpret_cast<const float4*>(wred + g * MK_WAVES);
                    const float4 gb = *reinterpret_cast<const float4*>(wred + g * MK_WAVES + 4);
                    const float mn = fmaxf(mls[g], fmaxf(fmaxf(fmaxf(ga.x, ga.y), fmaxf(ga.z, ga.w)), fmaxf(fmaxf(gb.x, gb.y), fmaxf(gb.z, gb.w))));
                    alpha[g] = expf(mls[g] - mn);
                }
                if (cn < nchunks) att_prefetch_k(a, lpt, ly, kvh, n0, nf, cn, kvpf);   // while softmax and P.V run
                lds_barrier();
                // running sums (one thread per head), then P.V with the rescaled accumulators
                if (tid < G) {
                    const float4 ma = *reinterpret_cast<const float4*>(wred + tid * MK_WAVES);
                    const float4 mb = *reinterpret_cast<const float4*>(wred + tid * MK_WAVES + 4);
                    const float4 la = *reinterpret_cast<const float4*>(wred + MK_WAVES * 16 + tid * MK_WAVES);
                    const float4 lb = *reinterpret_cast<const float4*>(wred + MK_WAVES * 16 + tid * MK_WAVES + 4);
                    const float mn = fmaxf(mls[tid], fmaxf(fmaxf(fmaxf(ma.x, ma.y), fmaxf(ma.z, ma.w)), fmaxf(fmaxf(mb.x, mb.y), fmaxf(mb.z, mb.w))));
                    const float ls = ((((((la.x + la.y) + la.z) + la.w) + lb.x) + lb.y) + lb.z) + lb.w;
                    mls[16 + tid] = mls[16 + tid] * alpha[tid] + ls;
                    mls[tid] = mn;
                }
#pragma unroll
                for (int g = 0; g < MAXG; g++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[g][e] *= alpha[g];
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    // keys 8 slice + 4 half .. +4 of the chunk (probabilities of masked keys are 0)
                    float4 pr[MAXG];
#pragma unroll
                    for (int g = 0; g < MAXG; g++) pr[g] = *reinterpret_cast<const float4*>(pp + g * ATT_PPS + 8 * slice + 4 * half);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int r = 4 * half + q, j = n0 + 128 * c + 8 * slice + r;
                        uint2 vv = kvpf.v[r];
                        if (owns_new && j == pos_l) vv = *reinterpret_cast<const uint2*>(vn16 + 4 * d4);
                        const float vf[4] = {__uint_as_float(vv.x << 16), __uint_as_float(vv.x & 0xffff0000u),
                                             __uint_as_float(vv.y << 16), __uint_as_float(vv.y & 0xffff0000u)};
#pragma unroll
                        for (int g = 0; g < MAXG; g++) {
                            const float pg = q == 0 ? pr[g].x : q == 1 ? pr[g].y : q == 2 ? pr[g].z : pr[g].w;
#pragma unroll
                            for (int e = 0; e < 4; e++) acc[g][e] = fmaf(pg, vf[e], acc[g][e]);
                        }
                    }
                }
                if (pair && n0 + 128 + 16 * wave < n1) {   // the wave's 16 keys of chunk 1 (rows past n1 are not staged)
#pragma unroll
                    for (int half = 0; half < 2; half++) {
                        float4 pr[MAXG];
#pragma unroll
                        for (int g = 0; g < MAXG; g++) pr[g] = *reinterpret_cast<const float4*>(pp + g * ATT_PPS + 128 + 8 * slice + 4 * half);
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const int r = 4 * half + q, j = n0 + 128 + 8 * slice + r;
                            if (j >= n1) continue;
                            const uint16_t* src = owns_new && j == pos_l ? vn16 + 4 * d4
                                                                       : reinterpret_cast<const uint16_t*>(kvl + 32768 + (8 * slice + r) * 256) + 4 * d4;
                            const uint2 vv = *reinterpret_cast<const uint2*>(src);
                            const float vf[4] = {__uint_as_float(vv.x << 16), __uint_as_float(vv.x & 0xffff0000u),
                                                 __uint_as_float(vv.y << 16), __uint_as_float(vv.y & 0xffff0000u)};
#pragma unroll
                            for (int g = 0; g < MAXG; g++) {
                                const float pg = q == 0 ? pr[g].x : q == 1 ? pr[g].y : q == 2 ? pr[g].z : pr[g].w;
#pragma unroll
                                for (int e = 0; e < 4; e++) acc[g][e] = fmaf(pg, vf[e], acc[g][e]);
                            }
                        }
                    }
                }
                if (cn < nchunks) att_prefetch_v(a, lpt, ly, kvh, n0, nf, cn, kvpf);
                c = cn;
            }
            prof_mark(a.prof, 512 + 8 * li + 1);
            prof_mark(a.prof, 512 + 8 * li + 2);
            // reduce over the 2 slices of a wave (lanes l, l^32), then over waves via LDS
#pragma unroll
            for (int g = 0; g < MAXG; g++) {
                if (g < G) {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float v = xor32_sum(acc[g][e]);
                        if (lane < 32) wacc[(wave * MAXG + g) * 128 + lane * 4 + e] = v;
                    }
                }
            }
            lds_barrier();
            // partials: plain agent-scope stores, then (once they are complete) this range's ready tag
            const unsigned atag = tag_of(3 + 5 * li);
            const int P = nH * nsplit;
            float* pm = a.part; float* pl = a.part + P; float* pa = a.part + 2 * P;
            for (int idx = tid; idx < G * 128; idx += MK_THREADS) {
                const int g = idx >> 7, d = idx & 127;
                float v = 0.0f;
                for (int w = 0; w < MK_WAVES; w++) v += wacc[(w * MAXG + g) * 128 + d];
                const int r = prow + g * nsplit + split;
                st_ag(pa + (int64_t)r * 128 + d, nk > 0 ? v : 0.0f);
                if (d == 0) { st_ag(pm + r, nk > 0 ? mls[g] : -1e30f); st_ag(pl + r, nk > 0 ? mls[16 + g] : 0.0f); }
            }
            __builtin_amdgcn_s_waitcnt(0);
            lds_barrier();
            if (tid == 0) st_tag(a.part_ready + kvh * nsplit + split, 0.0f, atag);
            prof_mark(a.prof, 512 + 8 * li + 3);
            // every range of the KV head merges a slice of its G * 128 outputs once all the head's
            // ranges are stored: ceil(G * 128 / nsplit) outputs here, one wave per output, the
            // nsplit partials of an output over the wave's lanes (one round trip of small loads)
            if (tid < nsplit) ld_tag1(a.part_ready, kvh * nsplit + tid, nKV * nsplit, atag, tw);
            lds_barrier();
            {
                const int opw = (G * 128 + nsplit - 1) / nsplit;
                const int o0 = split * opw, o1 = min(G * 128, o0 + opw);
                for (int o = o0 + wave; o < o1; o += MK_WAVES) {
                    const int g = o >> 7, d = o & 127;
                    const int rb = prow + g * nsplit;
                    float mv[MK_MERGE_L], lv[MK_MERGE_L], av[MK_MERGE_L];
#pragma unroll
                    for (int q = 0; q < MK_MERGE_L; q++) {
                        const int sp = lane + 64 * q;
                        const bool ok = sp < nsplit;
                        const int r = rb + (ok ? sp : 0);
                        mv[q] = ok ? ld_coh1(pm, r, P) : -1e30f;
                        lv[q] = ok ? ld_coh1(pl, r, P) : 0.0f;
                        av[q] = ok ? ld_coh1(pa, r * 128 + d, P * 128) : 0.0f;
                    }
                    float M = mv[0];
#pragma unroll
                    for (int q = 1; q < MK_MERGE_L; q++) M = fmaxf(M, mv[q]);
                    M = wave_max(M);
                    float on = 0.0f, ls = 0.0f;
#pragma unroll
                    for (int q = 0; q < MK_MERGE_L; q++) {
                        const float f = expf(mv[q] - M);
                        on += av[q] * f;
                        ls += lv[q] * f;
                    }
                    on = wave_sum(on); ls = wave_sum(ls);
                    if (lane == 0) st_tag(a.attnT + (kvh * G + g) * 128 + d, on * (1.0f / ls), atag);
                }
            }
        }
        prof_mark(a.prof, 2 * epoch); ++epoch;
        mvh_prefetch<FB>(ly.o, wg, nwg, wave, lane, ring);
        prof_mark(a.prof, 2 * epoch - 1);

        // ---- C: o_proj, h += W_o attn
        {
            const MvGeom<FB> gg = mv_geom<FB>(ly.o, wg, nwg, 0);
            const float us = copy_to_lds(a.attnT, tag_of(3 + 5 * li), tw, nH * D, ml, FB == 4 ? 5 : 6, a.hA,
                                         tag_of(li == 0 ? 1 : 6 + 5 * (li - 1)), H, 16 * gg.t0, min(16 * (gg.t0 + gg.nt), H), red);
            prof_mark(a.prof, 512 + 8 * li + 4);
            mvh_run<FB>(ly.o, ml.xh, ml.gsum, ml.zero16, wg, nwg, wave, lane, ring, ml.part);
            mv_finish<OUT_ADD, FB, true>(ly.o, us, wg, nwg, ml.part, a.hB, tag_of(4 + 5 * li), nullptr, ml.hown, red, redi);
        }
        prof_mark(a.prof, 2 * epoch); ++epoch;
        nwr = norm_w_load(ly.post_norm, H);
        mv_prefetch<FB>(ly.gu, wg, nwg, wave, lane, ring);
        prof_mark(a.prof, 2 * epoch - 1);

        // ---- D: gate|up with SiLU
        {
            const float us = norm_to_lds(a.hB, tag_of(4 + 5 * li), tw, ly.post_norm, nwr, H, a.eps, ml, FB == 4 ? 5 : 6, red);
            prof_mark(a.prof, 512 + 8 * li + 5);
            mv_run<FB, true>(ly.gu, ml.xh, ml.gsum, ml.zero16, wg, nwg, wave, lane, ring, ml.part);
            mv_finish<OUT_GATED, FB>(ly.gu, us, wg, nwg, ml.part, a.mlpT, tag_of(5 + 5 * li), nullptr, nullptr, red, redi);
        }
        prof_mark(a.prof, 2 * epoch); ++epoch;
        mv_prefetch<FB>(ly.down, wg, nwg, wave, lane, ring);
        prof_mark(a.prof, 2 * epoch - 1);

        // ---- E: down, h += W_d mlp
        {
            const MvGeom<FB> gg = mv_geom<FB>(ly.down, wg, nwg, 0);
            // the intermediate vector in two round trips (12288 values: 8 loads per thread per batch; 12
            // would do it in one but spill)
            const float us = copy_to_lds<8>(a.mlpT, tag_of(5 + 5 * li), tw, a.I, ml, FB == 4 ? 5 : 6, a.hB, tag_of(4 + 5 * li), H,
                                         16 * gg.t0, min(16 * (gg.t0 + gg.nt), H), red);
            prof_mark(a.prof, 512 + 8 * li + 6);
            mv_run<FB, true>(ly.down, ml.xh, ml.gsum, ml.zero16, wg, nwg, wave, lane, ring, ml.part);
            mv_finish<OUT_ADD, FB>(ly.down, us, wg, nwg, ml.part, a.hA, tag_of(6 + 5 * li), nullptr, ml.hown, red, redi);
        }
        prof_mark(a.prof, 2 * epoch); ++epoch;
        nwr = norm_w_load(li + 1 < a.L ? ldesc[li + 1].in_norm : a.final_norm, H);
        if (li + 1 < a.L) mvh_prefetch<FB>(ldesc[li + 1].qkv, wg, nwg, wave, lane, ring);
        else mv_prefetch<FB>(a.head, wg, nwg, wave, lane, ring);
        prof_mark(a.prof, 2 * epoch - 1);
    }

    // ---- lm_head with the final norm, logits and the greedy token
    const float us = norm_to_lds(a.hA, tag_of(6 + 5 * (a.L - 1)), tw, a.final_norm, nwr, H, a.eps, ml, FB == 4 ? 5 : 6, red);
    mv_run<FB, true>(a.head, ml.xh, ml.gsum, ml.zero16, wg, nwg, wave, lane, ring, ml.part);
    const MvResult best = mv_finish<OUT_ARGMAX, FB>(a.head, us, wg, nwg, ml.part, nullptr, 0u, a.logits, nullptr, red, redi);
    prof_mark(a.prof, 2 * epoch);
    __shared__ float bv[MK_WAVES];
    __shared__ int bi[MK_WAVES];
    if (tid == 0) {
        st_ag(a.wg_best + wg, best.best); st_ag(a.wg_idx + wg, best.best_idx);
        __builtin_amdgcn_s_waitcnt(0);
        const unsigned done = add_ag(a.head_done, 1u);
        flag = done == (unsigned)nwg - 1;
        if (flag) {   // every workgroup has finished its phases: reset the counter, count the launch
            __hip_atomic_store(a.head_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.sync->launch, launch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();
    if (!flag || !a.select) return;
    // workgroups hold ascending row ranges: the largest value, lowest index among equals
    float m = -INFINITY; int idx = 0x7fffffff;
    if (tid < nwg) { m = ld_coh1(a.wg_best, tid, nwg); idx = __float_as_int(ld_coh1(reinterpret_cast<const float*>(a.wg_idx), tid, nwg)); }
    if (!(m == m)) m = -INFINITY;
    float wm = wave_max(m);
    int wi = m == wm ? idx : 0x7fffffff;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) wi = min(wi, __shfl_xor(wi, o, 64));
    if (lane == 0) { bv[wave] = wm; bi[wave] = wi; }
    __syncthreads();
    if (tid != 0) return;
    m = -INFINITY; idx = 0x7fffffff;
    for (int w = 0; w < MK_WAVES; w++)
        if (bv[w] > m || (bv[w] == m && bi[w] < idx)) { m = bv[w]; idx = bi[w]; }
    const int ok = isfinite(m) && !ld_ag(&a.sync->abort) ? 1 : 0;   // an aborted step's token is not valid
    const int tok = ok ? idx : 0;
    a.hist[pos + 1] = tok; a.status[pos + 1] = ok ? 0 : 1;
    if (a.ring_tok) { a.ring_tok[(pos + 1) & a.ring_mask] = tok; a.ring_status[(pos + 1) & a.ring_mask] = ok ? 0 : 1; }
    *a.dpos = pos + 1;
}

// ------------------------------------------------------------------------------- repack (load time)
// Virtual row vr of tile t, row r16 (0..15) -> (part, row), or part -1 past the matrix.
__device__ __forceinline__ void dpack_row(const DPackSrc& s, int t, int r16, int& part, int& row) {
    if (s.gated) {
        part = r16 < 8 ? 0 : 1; row = 8 * t + (r16 & 7);
        if (row >= s.o1) part = -1;
        return;
    }
    const int vr = 16 * t + r16;
    if (vr >= s.rows) { part = -1; row = 0; return; }
    const int a = vr >= s.o1 ? 1 : 0, b = vr >= s.o1 + s.o2 ? 1 : 0;
    part = a + b; row = vr - (a ? s.o1 : 0) - (b ? s.o2 : 0);
}

// One thread per output dword of the interleaved stream.
__global__ void dpack_kernel(DPackSrc s, uint32_t* out, int tiles) {
    const int KBT = s.K >> 7, gpr = s.K / s.gs, FB = s.gs >> 3, NF = (KBT + FB - 1) / FB, dpr = s.K >> 3;
    const int64_t n = (int64_t)tiles * NF * (FB + 1) * 256;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int dw = (int)(i & 3), l = (int)((i >> 2) & 63);
        const int64_t blk = i >> 8;
        const int pos = (int)(blk % (FB + 1));
        const int64_t tf = blk / (FB + 1);
        const int t = (int)(tf / NF), f = (int)(tf % NF);
        uint32_t v = 0;
        if (pos == 0) {                       // scales of rows 4 (l >> 4) + dw, group 16 f + (l & 15)
            const int g = 16 * f + (l & 15);
            int part, row; dpack_row(s, t, 4 * (l >> 4) + dw, part, row);
            if (part >= 0 && g < gpr) {
                const uint16_t* sc = part == 0 ? s.s[0] : part == 1 ? s.s[1] : s.s[2];
                const uint16_t* bi = part == 0 ? s.b[0] : part == 1 ? s.b[1] : s.b[2];
                v = (uint32_t)sc[(int64_t)row * gpr + g] | ((uint32_t)bi[(int64_t)row * gpr + g] << 16);
            }
        } else {                              // code block kb: row l & 15, dword 16 kb + 4 dw + (l >> 4)
            const int kb = f * FB + pos - 1;
            int part, row; dpack_row(s, t, l & 15, part, row);
            if (part >= 0 && kb < KBT) {
                const uint32_t* src = reinterpret_cast<const uint32_t*>(part == 0 ? s.w[0] : part == 1 ? s.w[1] : s.w[2]);
                v = src[(int64_t)row * dpr + 16 * kb + 4 * dw + (l >> 4)];
            }
        }
        out[i] = v;
    }
}

int dpack_tiles(const DPackSrc& s) { return s.gated ? (s.o1 + 7) / 8 : (s.rows + 15) / 16; }
size_t dpack_bytes(const DPackSrc& s) {
    const int FB = s.gs >> 3, NF = ((s.K >> 7) + FB - 1) / FB;
    return (size_t)dpack_tiles(s) * NF * (FB + 1) * 1024;
}
hipError_t launch_dpack(const DPackSrc& s, uint8_t* out, hipStream_t st) {
    hipLaunchKernelGGL(dpack_kernel, dim3(2048), dim3(256), 0, st, s, reinterpret_cast<uint32_t*>(out), dpack_tiles(s));
    return hipGetLastError();
}

size_t mega_lds_bytes(const MegaArgs& a, int max_keys_per_split) {
    const int G = a.nH / a.nKV;
    const size_t kmax = (size_t)std::max(a.H, std::max(a.I, a.nH * 128));
    size_t mv = (kmax + kmax / 32 * XH_STRIDE + (kmax / 32 + 3) / 4 * 4 + MV_ZERO + MK_HOWN + MK_TPW * MK_WAVES * 16) * 4;
    // attention: q hi/lo image, new k/v, rope scratch, exchanges, probabilities, P.V partials, merge scale
    size_t att = 2 * 16 * 128 * 2 + 2 * 128 * 2 + (size_t)(4 * 128 + 2 * MK_WAVES * 16 + 32 + MK_MAXG * ATT_PPS +
                 MK_WAVES * MK_MAXG * 128 + MK_MAXG) * 4;
    if (att > (size_t)ATT_KVL_OFF || (size_t)(MK_TPW * MK_WAVES * 16 + MK_HOWN) * 4 > (size_t)ATT_KVL_OFF) return (size_t)-1;
    if (a.kv_stage) att = ATT_KVL_OFF + ATT_KVL_BYTES;   // the staged second chunk of keys
    (void)max_keys_per_split; (void)G;
    // then every layer's descriptors and the page table (copied in at the start of the launch)
    // (and the RoPE table: 64 cos / sin pairs at most)
    return (std::max(mv, att) + 15) / 16 * 16 + (size_t)a.L * sizeof(LayerDev) + ((size_t)a.n_pages * 4 + 15) / 16 * 16 + 64 * 8;
}
size_t mega_desc_offset(const MegaArgs& a) {
    return mega_lds_bytes(a, 0) - (size_t)a.L * sizeof(LayerDev) - ((size_t)a.n_pages * 4 + 15) / 16 * 16 - 64 * 8;
}

// Every layer's matrices share the group size (checked at setup); a.head.gs selects the variant.
static const void* pick_kernel(const MegaArgs& a) {
    const bool g4 = a.nH / a.nKV <= 4, fb4 = a.head.gs == 32;
    return g4 ? (fb4 ? (const void*)decode_step_kernel<4, 4> : (const void*)decode_step_kernel<4, 8>)
              : (fb4 ? (const void*)decode_step_kernel<8, 4> : (const void*)decode_step_kernel<8, 8>);
}

// A plain launch on the model stream. Co-residency (the phases' hand-overs wait for other
// workgroups' results) rests on the setup's check that the grid fits the device at the step's LDS
// size (one workgroup per CU), and every wait is bounded: a grid that is only partly resident (the
// device shared with other work) ends through the abort path instead of stalling. A cooperative
// launch would give the same guarantee up front, but the runtime routes it through a queue of its
// own, ordered against the model stream by markers, and tears that queue down at process exit.
hipError_t launch_decode_step(const MegaArgs& a, int nwg, size_t lds, hipStream_t s) {
    MegaArgs args = a;
    void* kargs[] = {&args};
    return hipLaunchKernel(pick_kernel(a), dim3(nwg), dim3(MK_THREADS), kargs, lds, s);
}

int mega_blocks_per_cu(const MegaArgs& a, size_t lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, pick_kernel(a), MK_THREADS, lds) != hipSuccess) return 0;
    return n;
}

hipError_t mega_set_lds_limit(size_t lds) {
    const void* k[4] = {(const void*)decode_step_kernel<4, 4>, (const void*)decode_step_kernel<4, 8>,
                        (const void*)decode_step_kernel<8, 4>, (const void*)decode_step_kernel<8, 8>};
    for (const void* f : k) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

int mega_threads() { return MK_THREADS; }
int mega_tiles_per_wg_cap() { return MK_TPW; }
int mega_wg_row_cap() { return MK_HOWN; }
int mega_split_cap() { return 64 * MK_MERGE_L; }

}  // namespace mlxr
