// Standalone batch-1 matvec over the repacked weight tiles: one launch per projection of the
// kernel-per-op decode step. Kept in its own translation unit, apart from the persistent decode
// kernel: sharing that kernel's code object slowed it by ~70% (measured), so each gets its own.
#include <algorithm>
#include "mv.h"

namespace mlxr {

constexpr int DMV_MAX_K = 32768;     // input length of the standalone matvec (max)
constexpr int DMV_MAX_LDS = 160 * 1024;
constexpr int DMV_OUT_PARTIAL = 5;   // dmv_finish mode: plain store, coherent across the XCDs (an input slice's partial rows)

// The matvec over the packed input and the epilogue (y = v, y += v, or SiLU(gate) * up).
template <int FB, int MODE, bool TS>
__device__ __forceinline__ void dmv_finish(const MvPhaseDesc& p, const MvLds& L, int wg, int nwg, int wave, int lane,
                                           Ring<FB>& ring, float unscale, float* __restrict__ y) {
    mv_run<FB, false, TS>(p, L.xh, L.gsum, L.zero16, wg, nwg, wave, lane, ring, L.part);
    lds_barrier();
    const MvGeom<FB> g = mv_geom<FB>(p, wg, nwg, 0);
    const int nfw = g.nt * g.NF;
    if (MODE == OUT_GATED) {
        for (int i = threadIdx.x; i < g.nt * 8; i += MK_THREADS) {
            const int tl = i >> 3, j = i & 7, o = 8 * (g.t0 + tl) + j;
            if (o < p.o1) {
                const float gv = tile_row(L.part, tl, j, nfw, g.NF) * unscale;
                const float uv = tile_row(L.part, tl, j + 8, nfw, g.NF) * unscale;
                y[o] = (gv / (1.0f + expf(-gv))) * uv;
            }
        }
        return;
    }
    for (int i = threadIdx.x; i < g.nt * 16; i += MK_THREADS) {
        const int row = 16 * g.t0 + i;
        if (row >= p.rows) break;
        const float v = tile_row(L.part, i >> 4, i & 15, nfw, g.NF) * unscale + row_bias(p, row);
        if (MODE == OUT_ADD) y[row] += v;
        else if (MODE == DMV_OUT_PARTIAL) __hip_atomic_store(y + row, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else y[row] = v;
    }
}

// One projection of the kernel-per-op decode step (the path for steps the persistent kernel does
// not take: sparse attention, models outside its limits, decode mode 0) over the same repacked
// tiles: y = W x (+ bias), y += W x, or y = SiLU(W_g x) * (W_u x), x optionally RMSNorm(x) * w.
// Every workgroup issues its first scale group of weights (after x when x is held in registers)
// and packs x straight from global memory (the norm statistics and max |x| first, then the
// packing), so large inputs (K up to 32768) fit in LDS without an f32 copy.
template <int FB, int MODE, bool TS = false>
__device__ __forceinline__ void dmv_body(const MvPhaseDesc& p, const float* __restrict__ x, const float* __restrict__ nw, float eps,
                                         float* __restrict__ y, int tpw, int wg, int nwg) {
    constexpr int GSH = FB == 4 ? 5 : 6;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int K = p.K;
    MvLds L;
    L.xf = nullptr; L.hown = nullptr;
    L.xh = lds;
    L.gsum = L.xh + (K >> 5) * XH_STRIDE;
    L.zero16 = L.gsum + (((K >> GSH) + 3) & ~3);   // 16-byte aligned
    L.part = L.zero16 + MV_ZERO;
    float* red = L.part + tpw * MK_WAVES * 16;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    Ring<FB> ring;
    // statistics: sum of squares of x, max |x w| (max |x| without a norm). Inputs of up to
    // 8 * XR * MK_THREADS values are read once, 8-group t = tid + MK_THREADS i into registers, and
    // packed from there; longer ones are read again to pack, four 16-byte loads per thread in flight
    // (global address space: they cannot alias the LDS writes).
    typedef float f4v __attribute__((ext_vector_type(4)));
    typedef const __attribute__((address_space(1))) f4v* gf4p;
    auto gf4 = [](const float* p) { const f4v v = *(gf4p)p; return float4{v.x, v.y, v.z, v.w}; };
    constexpr int XR = 4;
    const bool inreg = K <= 8 * XR * MK_THREADS;
    float4 xv[XR][2];
    float ss = 0.0f, mx = 0.0f;
    if (inreg) {
        float4 wv[XR][2];
#pragma unroll
        for (int i = 0; i < XR; i++) {
            const int t = threadIdx.x + i * MK_THREADS;
#pragma unroll
            for (int c = 0; c < 2; c++) { xv[i][c] = float4{0.0f, 0.0f, 0.0f, 0.0f}; wv[i][c] = float4{1.0f, 1.0f, 1.0f, 1.0f}; }
            if (8 * t < K) {
                xv[i][0] = gf4(x + 8 * t); xv[i][1] = gf4(x + 8 * t + 4);
                if (nw) { wv[i][0] = gf4(nw + 8 * t); wv[i][1] = gf4(nw + 8 * t + 4); }
            }
        }
#pragma unroll
        for (int i = 0; i < XR; i++)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const float4 v = xv[i][c], w = wv[i][c];
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                const float4 a = float4{v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w};
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
            }
        // the weights' first scale group once x is in (the memory counter completes in order: a
        // prefetch issued before would make the statistics wait for it); it streams in during the
        // reductions and the packing. The empty asm takes the statistics as inputs and clobbers
        // memory, so neither the statistics nor the prefetch's loads move across it.
        asm volatile("" : : "v"(ss), "v"(mx) : "memory");
        mv_prefetch<FB, TS>(p, wg, nwg, wave, lane, ring);
        ss = wave_sum(ss); mx = wave_max(mx);
        if (lane == 0) { red[wave] = ss; red[8 + wave] = mx; }
        lds_barrier();
        float tot = 0.0f, gmax = 0.0f;
        for (int i = 0; i < MK_WAVES; i++) { tot += red[i]; gmax = fmaxf(gmax, red[8 + i]); }
        const float inv = nw ? 1.0f / sqrtf(tot / (float)K + eps) : 1.0f;
        if (nw) {
#pragma unroll
            for (int i = 0; i < XR; i++)
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    float4& v = xv[i][c];
                    const float4 w = wv[i][c];
                    v.x = v.x * inv * w.x; v.y = v.y * inv * w.y; v.z = v.z * inv * w.z; v.w = v.w * inv * w.w;
                }
        }
        // pack_x16_from visits t = tid + MK_THREADS i in order of i
        auto ld = [&](int t, float4& lo, float4& hi) {
            const int i = (t - (int)threadIdx.x) / MK_THREADS;
            lo = xv[0][0]; hi = xv[0][1];
#pragma unroll
            for (int k = 1; k < XR; k++)
                if (i == k) { lo = xv[k][0]; hi = xv[k][1]; }
        };
        const float unscale = pack_x16_from(ld, K, gmax * inv, L, GSH);
        dmv_finish<FB, MODE, TS>(p, L, wg, nwg, wave, lane, ring, unscale, y);
        return;
    }
    mv_prefetch<FB, TS>(p, wg, nwg, wave, lane, ring);
    for (int base = threadIdx.x * 4; base < K; base += MK_THREADS * 16) {
        float4 v[4], w[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = base + u * MK_THREADS * 4;
            v[u] = float4{0.0f, 0.0f, 0.0f, 0.0f}; w[u] = float4{1.0f, 1.0f, 1.0f, 1.0f};
            if (i < K) v[u] = gf4(x + i);
            if (nw && i < K) w[u] = gf4(nw + i);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            ss += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
            const float4 a = float4{v[u].x * w[u].x, v[u].y * w[u].y, v[u].z * w[u].z, v[u].w * w[u].w};
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        }
    }
    ss = wave_sum(ss); mx = wave_max(mx);
    if (lane == 0) { red[wave] = ss; red[8 + wave] = mx; }
    lds_barrier();
    float tot = 0.0f, gmax = 0.0f;
    for (int i = 0; i < MK_WAVES; i++) { tot += red[i]; gmax = fmaxf(gmax, red[8 + i]); }
    const float inv = nw ? 1.0f / sqrtf(tot / (float)K + eps) : 1.0f;
    float unscale;
    if (nw) {
        auto ld = [x, nw, inv, gf4](int t, float4& lo, float4& hi) {
            lo = gf4(x + 8 * t); hi = gf4(x + 8 * t + 4);
            const float4 wl = gf4(nw + 8 * t), wh = gf4(nw + 8 * t + 4);
            lo.x = lo.x * inv * wl.x; lo.y = lo.y * inv * wl.y; lo.z = lo.z * inv * wl.z; lo.w = lo.w * inv * wl.w;
            hi.x = hi.x * inv * wh.x; hi.y = hi.y * inv * wh.y; hi.z = hi.z * inv * wh.z; hi.w = hi.w * inv * wh.w;
        };
        unscale = pack_x16_from(ld, K, gmax * inv, L, GSH);
    } else {
        auto ld = [x, gf4](int t, float4& lo, float4& hi) { lo = gf4(x + 8 * t); hi = gf4(x + 8 * t + 4); };
        unscale = pack_x16_from(ld, K, gmax, L, GSH);
    }
    dmv_finish<FB, MODE, TS>(p, L, wg, nwg, wave, lane, ring, unscale, y);
}

template <int FB, int MODE>
__global__ void __launch_bounds__(MK_THREADS) dpack_mv_kernel(MvPhaseDesc p, const float* __restrict__ x,
                                                              const float* __restrict__ nw, float eps, float* __restrict__ y, int tpw) {
    dmv_body<FB, MODE>(p, x, nw, eps, y, tpw, blockIdx.x, gridDim.x);
}

// Split over the input (no norm, not gated): workgroup (w, s) computes the rows of its share of the
// tiles (as dpack_mv_kernel shares them over gridDim.x workgroups) over the s-th of gridDim.y
// contiguous runs of every tile's scale groups, from its own slice of x, into part[s][rows] with
// coherent stores; for each tile, the last slice to finish (per-tile counters in the scratch's fixed
// counter region, part after it, so that launches of other shapes and slice counts sharing the
// scratch never overwrite a counter; reset by that slice for the next launch) adds the slices in order,
// the bias and the output: deterministic, and no combine launch.
template <int FB>
__global__ void __launch_bounds__(MK_THREADS) dpack_mv_split_kernel(MvPhaseDesc p, const float* __restrict__ x, float* __restrict__ split,
                                                                    float* __restrict__ y, int accumulate, int tpw) {
    unsigned* cnt = reinterpret_cast<unsigned*>(split);
    float* part = split + DMV_SPLIT_CNT;
    const int w = blockIdx.x, nw = gridDim.x, sl = blockIdx.y, S = gridDim.y;
    const int NF = ((p.K >> 7) + FB - 1) / FB;
    const int fa = NF * sl / S, fb = NF * (sl + 1) / S;
    MvPhaseDesc q = p;
    q.code = p.code + (size_t)fa * ((FB + 1) * 1024);
    q.K = min(fb * FB * 128, p.K) - fa * FB * 128;
    q.tstride = NF;
    q.bias[0] = q.bias[1] = q.bias[2] = nullptr;
    dmv_body<FB, DMV_OUT_PARTIAL, true>(q, x + fa * FB * 128, nullptr, 0.0f, part + (size_t)sl * p.rows, tpw, w, nw);
    // the partial rows are stored (and visible at agent scope) before the tiles' counters move
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ int last[MK_TPW];
    const MvGeom<FB> g = mv_geom<FB>(q, w, nw, 0);
    if ((int)threadIdx.x < g.nt)
        last[threadIdx.x] = __hip_atomic_fetch_add(cnt + g.t0 + threadIdx.x, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
    __syncthreads();
    for (int i = threadIdx.x; i < g.nt * 16; i += MK_THREADS) {
        if (!last[i >> 4]) continue;
        const int r = 16 * g.t0 + i;
        if (r < p.rows) {
            float v = 0.0f;
            for (int k = 0; k < S; k++) v += __hip_atomic_load(part + (size_t)k * p.rows + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v += row_bias(p, r);
            y[r] = accumulate ? y[r] + v : v;
        }
        if ((i & 15) == 0) __hip_atomic_store(cnt + g.t0 + (i >> 4), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---------------------------------------------------------------------------------------------
// Small batch over the repacked tiles: Y[t] = W x[t] (+ bias), Y[t] += W x[t], or SiLU(gate) * up,
// for up to 8 tokens at once (the speculative verify batch), x optionally RMSNorm(x) * w first.
// The tokens ride in the MFMA B columns (token c & 7, its hi part in column c, lo part in column
// c + 8), so the A operands (codes) are built once for every token, and each quantization group of
// a scale group accumulates in its own registers and is scaled after its MFMAs (the decode matvec
// separates groups by column instead). x of each token is packed as the decode matvec packs it
// (its own power-of-two scale, f16 hi + lo), every token's statistics in one pass over registers.
// Inputs too long for every token's image in LDS run as S input slices (grid.y) of each tile, the
// slices' partial rows summed in slice order by the tile's last workgroup (per-tile counters), so
// the result does not depend on arrival order.
constexpr int DMM_TOK = 8;
// f(std::integral_constant<int, I>) for I = B .. E - 1, in order
template <int B, int E> struct StaticFor {
    template <typename F> __device__ __forceinline__ static void run(F& f) {
        if constexpr (B < E) { f(std::integral_constant<int, B>{}); StaticFor<B + 1, E>::run(f); }
    }
};
constexpr int DMM_MAX_S = 8;                               // input slices (max)
constexpr int DMM_XR = 2;                                  // 8-groups of x per thread and token (max: slices of <= 8192 values)
constexpr int DMM_SLOTS = MK_WAVES * 2 * 16 * DMM_TOK;     // floats: each wave's first and last tile rows, when shared
constexpr int DMM_RED = 2 * MK_WAVES * DMM_TOK + DMM_TOK;  // per-wave max |x w| and sum of squares per token; unscales

struct MmArgs {
    MvPhaseDesc p;                       // the whole phase (parts, bias, rows)
    const float* x; int xs;              // token t's input at x + t * xs
    const float* nw; float eps;          // optional RMSNorm weights
    float* y; int ys; int accumulate;    // token t's output at y + t * ys
    int t0, nt;                          // the launch's tokens
    unsigned* cnt; float* part;          // S > 1: tile counters (zero between launches), partials [S][nt][tiles * 16]
};

// Streams the wave's scale groups. A tile the wave covers whole goes to emit(tile, rows) at once
// (lane (c, q): token c & 7, rows 4q .. 4q + 3); the wave's first and last tile, when other waves
// share them, leave their rows in slots[wave][0 / 1][row][token].
template <int FB, bool TS, typename EMIT>
__device__ __forceinline__ void mvt_run(const MvPhase p, const float* xh, int img, const float* gsum, int gstride, int nt,
                                        int wg, int nwg, int wave, int lane, Ring<FB>& ring, float* slots, const EMIT& emit) {
    constexpr int GSH = FB == 4 ? 5 : 6, CPG = 1 << (GSH - 5);   // chunks of 32 per quantization group
    const MvGeom<FB> g = mv_geom<FB>(p, wg, nwg, wave);
    const int nfb = g.f1 - g.f0;
    if (nfb <= 0) return;
    const int gpr = p.K >> GSH;
    const gptr8 base = mv_base<FB, TS>(p, g, lane);
    const int col = lane & 15, tok = col & 7, kq = lane >> 4;
    // B operand: the token's image (image 0 for the unused columns: read, never written), hi or lo
    // slots, slot kq of each chunk
    const float* xb = xh + (tok < nt ? tok : 0) * img + kq * 4 + (col >= 8 ? XH_LO : 0);
    const float* gs_t = gsum + (tok < nt ? tok : 0) * gstride;
    // run: the tile rows' code sums, scale * D per column (hi and lo columns added at the tile's
    // end, the codes' 2^24 too); runb: bias * Xs, hi columns only (xs is zero on the lo lanes)
    f32x4_t run = {0.0f, 0.0f, 0.0f, 0.0f}, runb = {0.0f, 0.0f, 0.0f, 0.0f};
    int tile = g.f0 / g.NF, f = g.f0 - tile * g.NF;
    const int first = tile;
    bool fresh = f == 0;                 // the wave holds the tile from its first scale group
    gptr8 cur = base;
    for (int i = 0; i < nfb; i++) {
        const bool more = i + 1 < nfb;
        gptr8 nxt;
        if constexpr (TS) nxt = cur = cur + (int64_t)(f + 1 == g.NF ? p.tstride - g.NF + 1 : 1) * ((FB + 1) * 1024);
        else nxt = base + (int64_t)(i + 1) * ((FB + 1) * 1024);
        const uint4 sbr = ring.u[0];
        if (more) ring.u[0] = ld_stream16(nxt);
        f32x4_t acc[16];
#pragma unroll
        for (int q = 0; q < 16; q++) acc[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < FB; k++) {
            const uint4 unit = ring.u[k + 1];
            const uint32_t wd[4] = {unit.x, unit.y, unit.z, unit.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int chunk = (f * FB + k) * 4 + j;
                const f16x8_t bv = __builtin_bit_cast(f16x8_t, *reinterpret_cast<const uint4*>(xb + chunk * XH_STRIDE));
                const int gl = (4 * k + j) / CPG;
                acc[gl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_operand(wd[j]), bv, acc[gl], 0, 0, 0);
            }
            if (more) ring.u[k + 1] = ld_stream16(nxt + (k + 1) * 1024);
        }
        // each group: scale * D + bias * Xs with the group's word for this lane's rows (held by the
        // scale block's lane of column gl in the same row quarter: a row broadcast)
        const uint32_t sv[4] = {sbr.x, sbr.y, sbr.z, sbr.w};
        // (GUARD: the input's last scale group, some of whose groups lie past the input)
        auto epilogue = [&](auto guard) {
            constexpr bool GUARD = decltype(guard)::value;
            auto group = [&](auto glc) {
                constexpr int gl = decltype(glc)::value;
                const int gi = 16 * f + gl;
                const bool real = !GUARD || gi < gpr;
                const float xs = col < 8 ? gs_t[real ? gi : 0] : 0.0f;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t w = __float_as_uint(dpp<0x150 + gl>(__uint_as_float(sv[r])));
                    const float a1 = fmaf(__uint_as_float(w << 16), acc[gl][r], run[r]);
                    const float b1 = fmaf(__uint_as_float(w & 0xffff0000u), xs, runb[r]);
                    // a group past the input: its products may be anything (0 * NaN is not 0)
                    run[r] = GUARD && !real ? run[r] : a1;
                    runb[r] = GUARD && !real ? runb[r] : b1;
                }
            };
            StaticFor<0, 16>::run(group);
        };
        if (16 * f + 16 <= gpr) epilogue(std::false_type{});
        else epilogue(std::true_type{});
        if (f == g.NF - 1 || i == nfb - 1) {     // tile done (or the wave's range)
#pragma unroll
            for (int r = 0; r < 4; r++) {   // hi + lo columns (lane c ^ 8: row rotation by 8), codes' 2^24, bias
                const float v = run[r] + dpp<0x128>(run[r]), b = runb[r] + dpp<0x128>(runb[r]);
                run[r] = fmaf(v, 16777216.0f, b);
            }
            if (fresh && f == g.NF - 1) {
                emit(tile, run);
            } else if (col < DMM_TOK) {
                const int slot = tile == first ? 0 : 1;
#pragma unroll
                for (int r = 0; r < 4; r++) slots[((wave * 2 + slot) * 16 + 4 * kq + r) * DMM_TOK + col] = run[r];
            }
            run = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}; runb = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (++f == g.NF) { f = 0; tile++; fresh = true; }
    }
}

// grid (workgroups, S). Slice blockIdx.y of every tile: scale groups [NF y / S, NF (y + 1) / S).
// XR: 8-groups of x per thread and token (1: slices of <= 4096 values, half the registers).
template <int FB, bool TS, int XR>
__global__ void __launch_bounds__(MK_THREADS) dpack_mm_kernel(MmArgs a) {
    constexpr int GSH = FB == 4 ? 5 : 6;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const MvPhaseDesc& p = a.p;
    const int wg = blockIdx.x, nwg = gridDim.x, sl = blockIdx.y, S = gridDim.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int NF = ((p.K >> 7) + FB - 1) / FB;
    const int fa = NF * sl / S, fb = NF * (sl + 1) / S;
    const int k0 = fa * FB * 128, Ks = min(fb * FB * 128, p.K) - k0;
    MvPhaseDesc q = p;
    if constexpr (TS) { q.code = p.code + (size_t)fa * ((FB + 1) * 1024); q.K = Ks; q.tstride = NF; }
    const int nt = a.nt, img = Ks, gstride = ((Ks >> GSH) + 3) & ~3;
    float* xh = lds;                                        // nt images of Ks floats (hi + lo halves)
    float* gsum = xh + (size_t)nt * img;                    // nt x gstride group sums
    float* zero = gsum + (size_t)nt * gstride;              // MV_ZERO (the packing clears it)
    float* slots = zero + MV_ZERO;                          // DMM_SLOTS
    float* red = slots + DMM_SLOTS;                         // max [wave][tok], sum of squares [wave][tok], unscale [tok]
    typedef float f4v __attribute__((ext_vector_type(4)));
    typedef const __attribute__((address_space(1))) f4v* gf4p;
    auto gf4 = [](const float* v) { const f4v u = *(gf4p)v; return float4{u.x, u.y, u.z, u.w}; };
    // every token's slice of x (8-groups t = tid + MK_THREADS i) and the norm weights into registers,
    // then the weights' first scale group: the memory counter completes in order, so the statistics
    // wait for x alone while the weights stream in behind
    float4 xv[DMM_TOK][XR][2], wv[XR][2];
#pragma unroll
    for (int i = 0; i < XR; i++) {
        const int t = threadIdx.x + i * MK_THREADS;
        const bool in = 8 * t < Ks;
        {   // unconditional too (without a norm: a load of x, replaced by ones)
            const float* wp = (a.nw ? a.nw : a.x) + k0 + 8 * (in ? t : 0);
            const float4 w0 = gf4(wp), w1 = gf4(wp + 4), one = float4{1.0f, 1.0f, 1.0f, 1.0f};
            wv[i][0] = a.nw ? w0 : one; wv[i][1] = a.nw ? w1 : one;
        }
        // unconditional loads (tokens and 8-groups past the input clamped to the last ones): the
        // waits before their uses then count exactly the loads behind them (the weights' ring),
        // where a conditional load would make them wait for everything
#pragma unroll
        for (int tk = 0; tk < DMM_TOK; tk++) {
            const float* xt = a.x + (int64_t)(a.t0 + min(tk, nt - 1)) * a.xs + k0 + 8 * (in ? t : 0);
            xv[tk][i][0] = gf4(xt); xv[tk][i][1] = gf4(xt + 4);
        }
    }
    Ring<FB> ring;
    __builtin_amdgcn_sched_barrier(0);   // the weights' loads stay behind every x load
    mv_prefetch_all<FB, TS>(q, wg, nwg, wave, lane, ring);
    // every token slot's statistics without a branch (slots past nt hold copies of the last
    // token), so the 16 reductions interleave
#pragma unroll
    for (int tk = 0; tk < DMM_TOK; tk++) {
        float ss = 0.0f, mx = 0.0f;
#pragma unroll
        for (int i = 0; i < XR; i++)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const bool in = 8 * ((int)threadIdx.x + i * MK_THREADS) < Ks;   // past the input: a copy, not counted
                const float4 v = in ? xv[tk][i][c] : float4{0.0f, 0.0f, 0.0f, 0.0f}, w = wv[i][c];
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                const float4 u = float4{v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w};
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))));
            }
        if (a.nw && S > 1) {   // the norm's statistics cover the whole input, not the slice
            ss = 0.0f;
            const float* xt = a.x + (int64_t)(a.t0 + tk) * a.xs;
            for (int i = threadIdx.x * 4; i < p.K; i += MK_THREADS * 4) {
                const float4 v = gf4(xt + i);
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
        }
        ss = wave_sum(ss); mx = wave_max(mx);
        if (lane == 0) { red[wave * DMM_TOK + tk] = mx; red[(MK_WAVES + wave) * DMM_TOK + tk] = ss; }
    }
    lds_barrier();
    MvLds L;
    L.xf = nullptr; L.hown = nullptr; L.part = nullptr; L.zero16 = zero;
    // every token's norm scale and max, lane tk for token tk (one chain for all tokens), read
    // before any packing writes LDS (reads could not pass those writes)
    float linv, lmax;
    {
        const int tk = lane & (DMM_TOK - 1);
        float tot = 0.0f, gmax = 0.0f;
        for (int w = 0; w < MK_WAVES; w++) { tot += red[(MK_WAVES + w) * DMM_TOK + tk]; gmax = fmaxf(gmax, red[w * DMM_TOK + tk]); }
        linv = a.nw ? 1.0f / sqrtf(tot / (float)p.K + a.eps) : 1.0f;
        lmax = gmax;
    }
#pragma unroll
    for (int tk = 0; tk < DMM_TOK; tk++) {
        if (tk >= nt) break;
        const float inv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(linv), tk));
        const float gmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lmax), tk));
        if (a.nw) {
#pragma unroll
            for (int i = 0; i < XR; i++)
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    float4& v = xv[tk][i][c];
                    const float4 w = wv[i][c];
                    v.x = v.x * inv * w.x; v.y = v.y * inv * w.y; v.z = v.z * inv * w.z; v.w = v.w * inv * w.w;
                }
        }
        L.xh = xh + (size_t)tk * img; L.gsum = gsum + (size_t)tk * gstride;
        // the packing visits t = tid + MK_THREADS i in order of i
        auto ld = [&](int t, float4& lo, float4& hi) {
            const bool second = XR > 1 && t >= MK_THREADS;
            lo = second ? xv[tk][XR - 1][0] : xv[tk][0][0];
            hi = second ? xv[tk][XR - 1][1] : xv[tk][0][1];
        };
        const float us = pack_x16_from<decltype(ld), false>(ld, Ks, gmax * inv, L, GSH);
        if (threadIdx.x == 0) red[2 * MK_WAVES * DMM_TOK + tk] = us;
    }
    lds_barrier();
    const float* unscale = red + 2 * MK_WAVES * DMM_TOK;
    const MvGeom<FB> g0 = mv_geom<FB>(q, wg, nwg, 0);
    const int T0 = g0.t0, R = p.tiles * 16;
    const bool gated = p.gated != 0, direct = S == 1;
    // a finished row: to y (one slice) or to the slice's partials
    auto put = [&](int tl, int row, int tk, float v) {
        if (!direct) {
            __hip_atomic_store(a.part + ((size_t)sl * nt + tk) * R + 16 * (T0 + tl) + row, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        const int r = 16 * (T0 + tl) + row;
        if (r >= p.rows) return;
        float* yr = a.y + (int64_t)(a.t0 + tk) * a.ys + r;
        const float o = v + row_bias(p, r);
        *yr = a.accumulate ? *yr + o : o;
    };
    // tile rows 0-7: gate of outputs 8 t + row, rows 8-15 the matching up values
    auto put_gated = [&](int tl, int row, int tk, float gv, float uv) {
        const int o = 8 * (T0 + tl) + row;
        if (o >= p.o1) return;
        gv += p.bias[0] ? bf16_to_f32(p.bias[0][o]) : 0.0f;
        uv += p.bias[1] ? bf16_to_f32(p.bias[1][o]) : 0.0f;
        a.y[(int64_t)(a.t0 + tk) * a.ys + o] = (gv / (1.0f + expf(-gv))) * uv;
    };
    auto emit = [&](int tl, const f32x4_t& run) {   // the whole wave
        const int col = lane & 15, kq = lane >> 4;
        const float us = unscale[col & 7];
        if (gated && direct) {
            f32x4_t up;
#pragma unroll
            for (int r = 0; r < 4; r++) up[r] = __shfl_xor(run[r], 32, 64);
            if (col < nt && kq < 2)
#pragma unroll
                for (int r = 0; r < 4; r++) put_gated(tl, 4 * kq + r, col, run[r] * us, up[r] * us);
        } else if (col < nt) {
#pragma unroll
            for (int r = 0; r < 4; r++) put(tl, 4 * kq + r, col, run[r] * us);
        }
    };
    mvt_run<FB, TS>(q, xh, img, gsum, gstride, nt, wg, nwg, wave, lane, ring, slots, emit);
    lds_barrier();
    // tiles shared between waves: their slots summed in wave order
    const int nfw = g0.nt * g0.NF;
    for (int i = threadIdx.x; i < g0.nt * 16 * nt; i += MK_THREADS) {
        const int tk = i % nt, rr = i / nt, tl = rr >> 4, row = rr & 15;
        if (gated && direct && row >= 8) continue;
        const int lo = tl * g0.NF, hi = lo + g0.NF;
        float v = 0.0f, u = 0.0f;
        bool whole = false;
        for (int w = 0; w < MK_WAVES; w++) {
            const int f0 = (nfw * w) >> 3, f1 = (nfw * (w + 1)) >> 3;
            if (f1 <= f0 || f1 <= lo || f0 >= hi) continue;
            if (f0 <= lo && f1 >= hi) { whole = true; break; }
            const int slot = f0 / g0.NF == tl ? 0 : 1;
            v += slots[((w * 2 + slot) * 16 + row) * DMM_TOK + tk];
            if (gated && direct) u += slots[((w * 2 + slot) * 16 + row + 8) * DMM_TOK + tk];
        }
        if (whole) continue;
        if (gated && direct) put_gated(tl, row, tk, v * unscale[tk], u * unscale[tk]);
        else put(tl, row, tk, v * unscale[tk]);
    }
    if (direct) return;
    // the slices' partials are stored (and visible at agent scope) before the tiles' counters move;
    // the tile's last workgroup sums them in slice order
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int* last = reinterpret_cast<int*>(slots);
    if ((int)threadIdx.x < g0.nt)
        last[threadIdx.x] = __hip_atomic_fetch_add(a.cnt + T0 + threadIdx.x, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
    __syncthreads();
    auto partial = [&](int tl, int row, int tk) {
        float v = 0.0f;
        for (int k = 0; k < S; k++)
            v += __hip_atomic_load(a.part + ((size_t)k * nt + tk) * R + 16 * (T0 + tl) + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return v;
    };
    for (int i = threadIdx.x; i < g0.nt * 16 * nt; i += MK_THREADS) {
        const int tk = i % nt, rr = i / nt, tl = rr >> 4, row = rr & 15;
        if (!last[tl]) continue;
        if (gated) {
            if (row < 8) {
                const float gv = partial(tl, row, tk), uv = partial(tl, row + 8, tk);
                const int o = 8 * (T0 + tl) + row;
                if (o < p.o1) {
                    const float gb = gv + (p.bias[0] ? bf16_to_f32(p.bias[0][o]) : 0.0f);
                    const float ub = uv + (p.bias[1] ? bf16_to_f32(p.bias[1][o]) : 0.0f);
                    a.y[(int64_t)(a.t0 + tk) * a.ys + o] = (gb / (1.0f + expf(-gb))) * ub;
                }
            }
        } else {
            const int r = 16 * (T0 + tl) + row;
            if (r < p.rows) {
                float* yr = a.y + (int64_t)(a.t0 + tk) * a.ys + r;
                const float o = partial(tl, row, tk) + row_bias(p, r);
                *yr = a.accumulate ? *yr + o : o;
            }
        }
    }
    if ((int)threadIdx.x < g0.nt && last[threadIdx.x])
        __hip_atomic_store(a.cnt + T0 + threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int FB, int MODE>
static hipError_t dmv_launch(const MvPhaseDesc& p, const float* x, const float* nw, float eps, float* y, int nwg, int tpw,
                             size_t lds, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute((const void*)dpack_mv_kernel<FB, MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 DMV_MAX_LDS);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((dpack_mv_kernel<FB, MODE>), dim3(nwg), dim3(MK_THREADS), lds, s, p, x, nw, eps, y, tpw);
    return hipGetLastError();
}

bool dpack_mv_supported(const MvPhaseDesc& p) {
    return (p.gs == 32 || p.gs == 64) && p.K % 128 == 0 && p.K <= DMV_MAX_K && p.tiles > 0 && p.code;
}

hipError_t launch_dpack_mv(const MvPhaseDesc& p, const float* x, const float* norm_w, float eps, float* y, int mode,
                           hipStream_t s, float* split) {
    if (!dpack_mv_supported(p) || mode < 0 || mode > 2) return hipErrorInvalidValue;
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidDevice;
    }
    // workgroups per CU: 2 (what the registers let run at once), 1 for inputs over 16K values (their
    // f16 hi + lo image alone takes over half the LDS); more only queues extra rounds (measured on
    // the 32B projections: gate|up 43 -> 36 us at 2, down 48 -> 37 us at 1)
    const int nwg = std::min(p.tiles, (p.K > 16384 ? 1 : 2) * cus);
    const int tpw = (p.tiles + nwg - 1) / nwg;
    if (split && !norm_w && mode != OUT_GATED && p.tiles <= DMV_SPLIT_CNT) {
        // S input slices of every tile over nw = slots / S workgroups each (two per CU: a slice's
        // f16 image fits twice in LDS); the longest workgroup streams ceil(tiles / nw) tiles x
        // ceil(NF / S) scale groups over its 8 waves: take the S that makes the longest wave's chain
        // shortest, if shorter than unsplit (the fewest slices among equals: each slice repacks x)
        const int FB = p.gs >> 3, NF = ((p.K >> 7) + FB - 1) / FB;
        auto chain = [](long groups) { return (groups + MK_WAVES - 1) / MK_WAVES; };
        int best_s = 1, best_nw = nwg, best_tpw = tpw;
        long best = chain((long)tpw * NF);
        for (int S = 2; S <= DMV_MAX_SLICES; S++) {
            const int nw = std::min(p.tiles, 2 * cus / S), t = (p.tiles + nw - 1) / nw, fs = (NF + S - 1) / S;
            if (t > MK_TPW || (long)fs * FB * 128 * 4 > DMV_MAX_LDS / 2 - 8192) continue;
            if (chain((long)t * fs) < best) { best = chain((long)t * fs); best_s = S; best_nw = nw; best_tpw = t; }
        }
        if (best_s > 1) {
            const int kslice = (NF + best_s - 1) / best_s * FB * 128;
            const size_t lds = sizeof(float) * ((size_t)(kslice >> 5) * XH_STRIDE + ((kslice / p.gs + 3) & ~3) + MV_ZERO +
                                                (size_t)best_tpw * MK_WAVES * 16 + 16);
            static bool attr = false;
            if (!attr) {
                for (const void* f : {(const void*)dpack_mv_split_kernel<4>, (const void*)dpack_mv_split_kernel<8>})
                    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, DMV_MAX_LDS - 1024) != hipSuccess)   // beside its static LDS
                        return hipErrorInvalidValue;
                attr = true;
            }
            const int acc = mode == OUT_ADD ? 1 : 0;
            if (p.gs == 32)
                hipLaunchKernelGGL(dpack_mv_split_kernel<4>, dim3(best_nw, best_s), dim3(MK_THREADS), lds, s, p, x, split, y, acc, best_tpw);
            else
                hipLaunchKernelGGL(dpack_mv_split_kernel<8>, dim3(best_nw, best_s), dim3(MK_THREADS), lds, s, p, x, split, y, acc, best_tpw);
            return hipGetLastError();
        }
    }
    if (tpw > MK_TPW) return hipErrorInvalidValue;
    const size_t lds = sizeof(float) * ((size_t)(p.K >> 5) * XH_STRIDE + (((p.K / p.gs) + 3) & ~3) + MV_ZERO + (size_t)tpw * MK_WAVES * 16 + 16);
    if (lds > DMV_MAX_LDS) return hipErrorInvalidValue;
    const bool fb4 = p.gs == 32;
    switch (mode) {
        case OUT_STORE: return fb4 ? dmv_launch<4, OUT_STORE>(p, x, norm_w, eps, y, nwg, tpw, lds, s)
                                   : dmv_launch<8, OUT_STORE>(p, x, norm_w, eps, y, nwg, tpw, lds, s);
        case OUT_ADD: return fb4 ? dmv_launch<4, OUT_ADD>(p, x, norm_w, eps, y, nwg, tpw, lds, s)
                                 : dmv_launch<8, OUT_ADD>(p, x, norm_w, eps, y, nwg, tpw, lds, s);
        default: return fb4 ? dmv_launch<4, OUT_GATED>(p, x, norm_w, eps, y, nwg, tpw, lds, s)
                            : dmv_launch<8, OUT_GATED>(p, x, norm_w, eps, y, nwg, tpw, lds, s);
    }
}

// Input slices of a small-batch launch of nt tokens: the fewest whose nt images fit in LDS and
// whose longest slice fits one 8-group of x per thread (4096 values; the two-group variant needs
// twice the registers and ran slower, measured: the 8B down projection at T = 5 as 2 x 6144 took
// ~22 us), else the fewest that fit two; 0: none. *lds = the launch's dynamic LDS.
static int mm_slices(const MvPhaseDesc& p, int nt, size_t* lds) {
    const int FB = p.gs >> 3, GSH = FB == 4 ? 5 : 6, NF = ((p.K >> 7) + FB - 1) / FB;
    for (int xr = 1; xr <= DMM_XR; xr++)
        for (int S = 1; S <= DMM_MAX_S && S <= NF; S++) {
            int ks = 0;
            for (int sl = 0; sl < S; sl++)
                ks = std::max(ks, std::min(NF * (sl + 1) / S * FB * 128, p.K) - NF * sl / S * FB * 128);
            if (ks > xr * 8 * MK_THREADS) continue;
            const size_t b = sizeof(float) * ((size_t)nt * (ks + (((ks >> GSH) + 3) & ~3)) + MV_ZERO + DMM_SLOTS + DMM_RED);
            if (b <= (size_t)DMV_MAX_LDS) { *lds = b; return S; }
        }
    return 0;
}

size_t dpack_mm_split_floats(const MvPhaseDesc& p) {
    if (!dpack_mv_supported(p)) return 0;
    int S = 1;
    for (int nt = 1; nt <= DMM_TOK; nt++) { size_t lds = 0; S = std::max(S, mm_slices(p, nt, &lds)); }
    if (S <= 1) return 0;
    return (size_t)DMV_SPLIT_CNT + (size_t)S * DMM_TOK * 16 * p.tiles;
}

hipError_t launch_dpack_mm(const MvPhaseDesc& p, const float* x, int xs, const float* norm_w, float eps, float* y, int ys,
                           bool accumulate, int T, float* split, size_t split_floats, hipStream_t s) {
    if (!dpack_mv_supported(p) || T < 1 || T > DMM_TOK || (p.gated && accumulate)) return hipErrorInvalidValue;
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidDevice;
    }
    static bool attr = false;
    if (!attr) {
        for (const void* f : {(const void*)dpack_mm_kernel<4, false, 1>, (const void*)dpack_mm_kernel<8, false, 1>,
                              (const void*)dpack_mm_kernel<4, true, 1>, (const void*)dpack_mm_kernel<8, true, 1>,
                              (const void*)dpack_mm_kernel<4, false, 2>, (const void*)dpack_mm_kernel<8, false, 2>,
                              (const void*)dpack_mm_kernel<4, true, 2>, (const void*)dpack_mm_kernel<8, true, 2>})
            if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, DMV_MAX_LDS) != hipSuccess) return hipErrorInvalidValue;
        attr = true;
    }
    size_t lds = 0;
    const int S = mm_slices(p, T, &lds);
    if (S == 0) return hipErrorInvalidValue;
    if (S > 1 && (!split || p.tiles > DMV_SPLIT_CNT || split_floats < (size_t)DMV_SPLIT_CNT + (size_t)S * T * 16 * p.tiles))
        return hipErrorInvalidValue;
    MmArgs a;
    a.p = p; a.x = x; a.xs = xs; a.nw = norm_w; a.eps = eps; a.y = y; a.ys = ys; a.accumulate = accumulate ? 1 : 0;
    a.t0 = 0; a.nt = T;
    a.cnt = reinterpret_cast<unsigned*>(split); a.part = split ? split + DMV_SPLIT_CNT : nullptr;
    // one workgroup per CU over all slices (the images fill most of the LDS)
    const int nwg = std::min(p.tiles, std::max(1, cus / S));
    // the longest slice decides how many 8-groups of x each thread holds
    const int FBv = p.gs >> 3, NF = ((p.K >> 7) + FBv - 1) / FBv;
    int ks = 0;
    for (int sl = 0; sl < S; sl++) ks = std::max(ks, std::min(NF * (sl + 1) / S * FBv * 128, p.K) - NF * sl / S * FBv * 128);
    const bool xr1 = ks <= 8 * MK_THREADS;
    const dim3 grid(nwg, S);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(MK_THREADS), lds, s, a); };
    if (p.gs == 32) {
        if (S == 1) xr1 ? go(dpack_mm_kernel<4, false, 1>) : go(dpack_mm_kernel<4, false, 2>);
        else xr1 ? go(dpack_mm_kernel<4, true, 1>) : go(dpack_mm_kernel<4, true, 2>);
    } else {
        if (S == 1) xr1 ? go(dpack_mm_kernel<8, false, 1>) : go(dpack_mm_kernel<8, false, 2>);
        else xr1 ? go(dpack_mm_kernel<8, true, 1>) : go(dpack_mm_kernel<8, true, 2>);
    }
    return hipGetLastError();
}

}  // namespace mlxr
