// Persistent decode step: the whole batch-1 token step (every layer, lm_head and the greedy token)
// in ONE launch of exactly one 512-thread workgroup per CU, phases separated by grid barriers.
//
// Why: a kernel-per-op step issues ~5 launches per layer, and each launch boundary on MI355X costs
// ~1.6 us of idle HBM inside a hipGraph, which alone caps an 8B decode near half of the bandwidth
// roofline. Here every workgroup, before it waits at a barrier, issues the loads of its share of
// the NEXT phase's weights (and of its K/V rows: the cache up to the previous position does not
// depend on the current step), so HBM streams through the barrier.
//
// Phases per layer (one grid barrier after each):
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
// activations and accumulation, bf16 K/V. Matvec work unit: one 32-code chunk of one row per lane
// (16 bytes at 4 bits), a ring of DEPTH units in flight per lane.
//
// Safety: the grid barrier spins with a bounded count; on expiry it raises an abort flag that every
// later barrier honours, so every wave reaches the end of the kernel and the host reports an error.
#include "decode.h"

namespace mlxr {

constexpr int MK_THREADS = 512;
constexpr int MK_WAVES = MK_THREADS / 64;
#ifndef MLXR_MK_DEPTH
#define MLXR_MK_DEPTH 8
#endif
constexpr int MK_DEPTH = MLXR_MK_DEPTH;   // matvec units in flight per lane
constexpr int MK_KV_PF = 4;          // attention: K/V rounds (32 keys each) prefetched per thread
constexpr int MK_MAXG = 8;
constexpr int MK_HOWN = 1024;        // residual rows of one workgroup in an accumulate phase (max)
constexpr int MK_YCAP = 512;         // row results of one wave in a matvec phase (max)

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

// ------------------------------------------------------------------------------- grid barrier
// Split barrier. `arrive`: every wave waits for its own stores to complete, then one thread counts
// the workgroup into its XCD group's counter; the last of a group counts the group, and the last
// group publishes the epoch. The caller then issues its next-phase loads, and `wait` polls the
// epoch. (1.9 us measured for 256 workgroups, against ~14 us with agent-scope fences.)
// An expired wait sets `abort`, which every later wait honours, so every wave reaches the end.
__device__ __forceinline__ void prof_mark(unsigned long long* prof, int ev) {
    if (prof && threadIdx.x == 0 && ev < MEGA_PROF_EVENTS) prof[(size_t)blockIdx.x * MEGA_PROF_EVENTS + ev] = wall_clock64();
}

__device__ __forceinline__ void grid_arrive(MegaSync* sync, unsigned epoch) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int x = blockIdx.x & 7, nwg = gridDim.x;
        const unsigned per = (unsigned)((nwg - x + 7) / 8), groups = nwg < 8 ? (unsigned)nwg : 8u;
        if (add_ag(&sync->xcd[x][0], 1u) + 1 == epoch * per)
            if (add_ag(&sync->count, 1u) + 1 == epoch * groups)
                __hip_atomic_store(&sync->gen, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
__device__ __forceinline__ void grid_wait(MegaSync* sync, unsigned epoch) {
    if (threadIdx.x == 0) {
        unsigned spins = 0;
        while (ld_ag(&sync->gen) < epoch) {
            if (ld_ag(&sync->abort)) break;
            __builtin_amdgcn_s_sleep(1);
            if (++spins > (1u << 21)) {   // far beyond any phase: let every wave run to the end instead
                __hip_atomic_store(&sync->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------------------------- matvec phase
// MvPhaseDesc (decode.h): rows of up to three matrices; o1/o2 = rows of parts 0 and 1 (part 2 gets
// the rest); gated: virtual row 2o is gate row o (part 0), 2o+1 is up row o (part 1).
typedef MvPhaseDesc MvPhase;

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// Global-address-space pointers: loads through them are global (not flat) loads, which count on
// the memory counter only; a flat load also counts on the LDS counter, so every wait for an LDS
// read would wait for it too.
typedef const __attribute__((address_space(1))) uint8_t* gptr8;
typedef const __attribute__((address_space(1))) uint16_t* gptr16;
typedef const __attribute__((address_space(1))) u32x4_t* gptr128;
// 16-byte streaming load (data read once: the nontemporal hint keeps it from displacing activations)
__device__ __forceinline__ uint4 ld_stream16(gptr8 p) {
    const u32x4_t v = __builtin_nontemporal_load((gptr128)p);
    return uint4{v.x, v.y, v.z, v.w};
}

// Loaded units, kept exactly as loaded: no instruction touches a value before the unit is
// consumed, so the memory-counter wait for a slot never drains the loads issued after it.
struct Ring {
    uint4 code[MK_DEPTH];
    uint32_t s[MK_DEPTH], b[MK_DEPTH];   // bf16 scale / bias (zero-extended)
};

// Branch-free (the row may differ between the halves of a wave).
__device__ __forceinline__ void mv_locate(const MvPhase& p, int vr, int& part, int& row) {
    const int a = vr >= p.o1 ? 1 : 0, b = vr >= p.o1 + p.o2 ? 1 : 0;
    const int pn = a + b, rn = vr - (a ? p.o1 : 0) - (b ? p.o2 : 0);
    part = p.gated ? (vr & 1) : pn;
    row = p.gated ? (vr >> 1) : rn;
}

// Element `part` of a 3-array by selects (dynamic indexing would move the array to scratch memory).
// Mask arithmetic rather than a conditional, which the compiler turns into divergent branches.
template <typename T>
__device__ __forceinline__ T pick3(const T (&a)[3], int part) {
    const uint64_t m0 = 0ull - (uint64_t)(part == 0), m1 = 0ull - (uint64_t)(part == 1), m2 = 0ull - (uint64_t)(part == 2);
    return (T)(((uint64_t)a[0] & m0) | ((uint64_t)a[1] & m1) | ((uint64_t)a[2] & m2));
}

// Work split of a wave's rows [r0, r1): rows go in pairs, lanes 0-31 take the pair's first row and
// lanes 32-63 its second; a unit is one 32-code chunk per lane, (lane & 31) + 32 * ci. One pair
// takes nci = ceil(chunks / 32) units, so a wave load reads two runs of 512 contiguous bytes, and a
// row sum needs a 32-lane reduction once per nci units (DPP, no LDS round trip).
// Load cursor: per-lane pointers advance by 32 chunks per unit and are recomputed once per pair.
// Every unit issues its loads from a valid address (a lane past its row's last chunk, or on the
// missing second row of an odd tail, re-reads its row's first chunk and is zeroed when consumed),
// so the ring has no branches around loads and the memory-counter waits stay exact. Units past the
// wave's last re-read the last one.
struct Cursor {
    gptr8 w; gptr16 s; gptr16 b;   // this lane's unit pointers
    int pr, ci;                    // pair's first row, unit within the pair (wave-uniform)
};

__device__ __forceinline__ void cursor_pair(const MvPhase& p, int pr, int r1, int lane, int gsh, Cursor& c) {
    int part, row; mv_locate(p, min(pr + (lane >> 5), r1 - 1), part, row);
    const int gpr = p.K >> gsh, ch = lane & 31;
    c.w = (gptr8)pick3(p.w, part) + (int64_t)row * (p.K >> 1) + ch * 16;
    c.s = (gptr16)pick3(p.s, part) + (int64_t)row * gpr + ((ch << 5) >> gsh);
    c.b = (gptr16)pick3(p.b, part) + (int64_t)row * gpr + ((ch << 5) >> gsh);
    c.pr = pr; c.ci = 0;
}

// FULL: every row has a multiple of 32 chunks (no lane is ever past its row's end).
template <bool FULL>
__device__ __forceinline__ void cursor_load(const Cursor& c, int lane, int nch, int gsh, uint4& code, uint32_t& sv, uint32_t& bv) {
    if (FULL) { code = ld_stream16(c.w); sv = *c.s; bv = *c.b; return; }
    const int ch = (lane & 31) + 32 * c.ci;
    const bool ok = ch < nch;
    const int back = ok ? 0 : c.ci * 512;                      // re-read the lane's first unit of the row
    const int sback = ok ? 0 : ((c.ci * 1024) >> gsh);
    code = ld_stream16(c.w - back);
    sv = c.s[-sback]; bv = c.b[-sback];
}

// Whether the step to pair pr (from pr - 2) needs cursor_pair: a part boundary between a half's
// old and new row, or a missing second row (odd tail). Wave-uniform.
__device__ __forceinline__ bool pair_slow(const MvPhase& p, int pr, int r1) {
    if (pr + 1 >= r1) return true;
    if (p.gated) return false;
    const int b1 = p.o1, b2 = p.o1 + p.o2;
    return (b1 > pr - 2 && b1 <= pr + 1) || (b2 > pr - 2 && b2 <= pr + 1);
}

// Moves to the next unit unless `last` (stays on the wave's final unit). With FULL rows a pair's
// units advance each lane's pointers by exactly one row, which is the next pair's row in a gated
// phase (gate row o + 1, up row o + 1) and one row short of it otherwise.
template <bool FULL>
__device__ __forceinline__ void cursor_next(const MvPhase& p, int r1, int lane, int gsh, int nci, bool last, Cursor& c) {
    if (last) return;
    if (++c.ci == nci) {
        if (FULL && !pair_slow(p, c.pr + 2, r1)) {
            c.pr += 2; c.ci = 0;
            if (!p.gated) { c.w += p.K >> 1; c.s += p.K >> gsh; c.b += p.K >> gsh; }
            return;
        }
        cursor_pair(p, c.pr + 2, r1, lane, gsh, c);
        return;
    }
    c.w += 512; c.s += 1024 >> gsh; c.b += 1024 >> gsh;
}

// Sum over each half-wave (lanes 0-31, 32-63); the totals land in lanes 31 and 63.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ float half_wave_sum(float v) {
    v += dpp<0xB1>(v);            // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);            // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);           // row_half_mirror: 8-lane sums
    v += dpp<0x140>(v);           // row_mirror: 16-lane sums in every lane of a row
    v += dpp<0x142, 0xA>(v);      // row_bcast15: rows 1 and 3 add lane 15 of rows 0 and 2
    return v;
}

// LDS layout of the matvec input (f16): chunk c of 32 values at xh + 20 * c (80 bytes, so the
// 16-byte reads of 8 consecutive lanes fall in distinct banks). Dword i of a chunk's codes holds
// codes 8i..8i+7 (nibble j at bits 4j); its x slot (16 bytes) holds the f16 pairs
//   (x0, x4), (x1 / 16, x5 / 16), (x2, x6), (x3 / 16, x7 / 16)      (x of codes 8i..8i+7)
// after a power-of-two scaling of the whole vector, then the chunk's (Cs, Xs) at byte 64:
// Cs = 1024 * (sum of the chunk's 32 stored halves), Xs = sum of the chunk's scaled x.
constexpr int XH_STRIDE = 20;          // floats per chunk

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }

// One 32-code unit, s * sum_j q_j x_j + b * sum_j x_j (in the scaled x units). A nibble masked into
// the low mantissa bits of the f16 1024.0 is the half 1024 + q (bits 4..7: 1024 + 16 q, met by the
// x / 16 slots), so one AND-OR builds two operands of v_dot2_f32_f16 and
// sum (1024 + q) x = Cs + sum q x. Products of halves are exact in the f32 accumulation.
// (a & m) | c in one instruction; m and c are passed in VGPRs (a VOP3 takes one constant at most).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    uint32_t r; asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(c)); return r;
}

// Constants of unit_dot, held in VGPRs for the whole phase.
struct DotConsts { uint32_t m_lo, m_hi, magic; };   // magic: two halves of 1024.0
__device__ __forceinline__ DotConsts dot_consts() {
    DotConsts k;
    asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(k.m_lo));
    asm volatile("v_mov_b32 %0, 0x00F000F0" : "=v"(k.m_hi));
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(k.magic));
    return k;
}

// One chunk of x in registers.
struct XChunk { uint4 q[4]; float2 cx; };
__device__ __forceinline__ XChunk load_x(const float* xc) {
    XChunk x;
    const uint4* xq = reinterpret_cast<const uint4*>(xc);
#pragma unroll
    for (int i = 0; i < 4; i++) x.q[i] = xq[i];
    x.cx = *reinterpret_cast<const float2*>(xc + 16);
    return x;
}

__device__ __forceinline__ float unit_dot(const uint4 w, uint32_t s16, uint32_t b16, const XChunk& x, const DotConsts& k) {
    float d0 = 0.0f, d1 = 0.0f;
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 xv = x.q[i];
        const uint32_t a = ww[i], a8 = a >> 8;
        d0 = __builtin_amdgcn_fdot2(as_h2(and_or(a, k.m_lo, k.magic)), as_h2(xv.x), d0, false);
        d1 = __builtin_amdgcn_fdot2(as_h2(and_or(a, k.m_hi, k.magic)), as_h2(xv.y), d1, false);
        d0 = __builtin_amdgcn_fdot2(as_h2(and_or(a8, k.m_lo, k.magic)), as_h2(xv.z), d0, false);
        d1 = __builtin_amdgcn_fdot2(as_h2(and_or(a8, k.m_hi, k.magic)), as_h2(xv.w), d1, false);
    }
    const float sc = __uint_as_float(s16 << 16), bi = __uint_as_float(b16 << 16);
    return sc * ((d0 + d1) - x.cx.x) + bi * x.cx.y;
}

// Packs xf[0..K) (f32, contiguous; every thread's share already written, max |x| reduced by the
// caller into gmax) into the f16 layout above. Scale 2^e maps max |x| below 2^14, so every stored
// half is finite and (for all but values 2^28 below the maximum) normal. Returns 2^-e.
__device__ __forceinline__ float pack_x16(const float* xf, int K, float gmax, float* xh) {
    int ex = 0;
    if (gmax > 0.0f && gmax <= 3.0e38f) frexpf(gmax, &ex);
    const int e = min(max(14 - ex, -100), 100);
    const float up = ldexpf(1.0f, e);
    for (int t = threadIdx.x; t < (K >> 3); t += MK_THREADS) {   // t: 8 values; 4 consecutive t per chunk
        const float4 lo = *reinterpret_cast<const float4*>(xf + 8 * t);
        const float4 hi = *reinterpret_cast<const float4*>(xf + 8 * t + 4);
        const _Float16 h0 = (_Float16)(lo.x * up), h4 = (_Float16)(hi.x * up);
        const _Float16 h1 = (_Float16)(lo.y * up * 0.0625f), h5 = (_Float16)(hi.y * up * 0.0625f);
        const _Float16 h2 = (_Float16)(lo.z * up), h6 = (_Float16)(hi.z * up);
        const _Float16 h3 = (_Float16)(lo.w * up * 0.0625f), h7 = (_Float16)(hi.w * up * 0.0625f);
        uint4 o;
        o.x = __builtin_bit_cast(uint32_t, h2_t{h0, h4});
        o.y = __builtin_bit_cast(uint32_t, h2_t{h1, h5});
        o.z = __builtin_bit_cast(uint32_t, h2_t{h2, h6});
        o.w = __builtin_bit_cast(uint32_t, h2_t{h3, h7});
        const int c = t >> 2;
        *reinterpret_cast<uint4*>(xh + c * XH_STRIDE + (t & 3) * 4) = o;
        const float ev = (float)h0 + (float)h4 + (float)h2 + (float)h6;
        const float od = (float)h1 + (float)h5 + (float)h3 + (float)h7;
        float cs = ev + od, xsum = ev + 16.0f * od;
        cs += __shfl_xor(cs, 1, 64); cs += __shfl_xor(cs, 2, 64);
        xsum += __shfl_xor(xsum, 1, 64); xsum += __shfl_xor(xsum, 2, 64);
        if ((t & 3) == 0) *reinterpret_cast<float2*>(xh + c * XH_STRIDE + 16) = float2{1024.0f * cs, xsum};
    }
    __syncthreads();
    return 1.0f / up;
}

// Rows [r0, r1) of the phase assigned to this workgroup.
__device__ __forceinline__ void wg_rows(int rows, int wg, int nwg, int& r0, int& r1) {
    r0 = (int)((int64_t)rows * wg / nwg); r1 = (int)((int64_t)rows * (wg + 1) / nwg);
}

// Rows [r0, r1) of the phase assigned to this wave.
__device__ __forceinline__ void wave_rows(int rows, int wg, int nwg, int wave, bool pairs, int& r0, int& r1) {
    const int unit = pairs ? 2 : 1;
    const int n = rows / unit;
    const int a = (int)((int64_t)n * wg / nwg), b = (int)((int64_t)n * (wg + 1) / nwg);
    const int m = b - a;
    const int wa = a + m * wave / MK_WAVES, wb = a + m * (wave + 1) / MK_WAVES;
    r0 = wa * unit; r1 = wb * unit;
}

__device__ __forceinline__ int gshift(int gs) { return gs == 32 ? 5 : gs == 64 ? 6 : gs == 128 ? 7 : 8; }

// The phase descriptor is taken by value: held in registers, a row change reads no memory (a load
// there would make the ring's next memory-counter wait drain every unit in flight).
__device__ __forceinline__ int pair_units(const MvPhase& p) { return ((p.K >> 5) + 31) >> 5; }

template <bool FULL>
__device__ __forceinline__ void mv_prefetch_t(const MvPhase& p, int r0, int r1, int lane, Ring& ring) {
    const int nci = pair_units(p), nch = p.K >> 5, gsh = gshift(p.gs);
    const int n = ((r1 - r0 + 1) >> 1) * nci;
    if (n <= 0) return;
    Cursor c; cursor_pair(p, r0, r1, lane, gsh, c);
#pragma unroll
    for (int d = 0; d < MK_DEPTH; d++) {
        cursor_load<FULL>(c, lane, nch, gsh, ring.code[d], ring.s[d], ring.b[d]);
        cursor_next<FULL>(p, r1, lane, gsh, nci, d + 1 >= n, c);
    }
}
__device__ __forceinline__ bool mv_full(const MvPhase& p) { return ((p.K >> 5) & 31) == 0; }
__device__ __forceinline__ void mv_prefetch(const MvPhase p, int r0, int r1, int lane, Ring& ring) {
    if (mv_full(p)) mv_prefetch_t<true>(p, r0, r1, lane, ring);
    else mv_prefetch_t<false>(p, r0, r1, lane, ring);
}

enum MvOut { OUT_STORE = 0, OUT_ADD = 1, OUT_GATED = 2, OUT_ARGMAX = 3 };

struct MvResult { float best; int best_idx; };   // wave-uniform

__device__ __forceinline__ float row_bias(const MvPhase& p, int vr) {
    int part, row; mv_locate(p, vr, part, row);
    return bf16_to_f32(pick3(p.bias, part)[row]);
}

// Consumes the wave's units (the first DEPTH already in the ring) and writes row results.
// Gated phases have even r0 and r1, so a pair is (gate row, up row) of one output.
// Row results are collected in this wave's LDS slice `ybuf` and written to `out` once, after the
// last unit: a store between ring loads would hold back every later load's completion (vector
// memory operations count down in issue order, and an agent-scope store completes only at memory).
template <int MODE, bool FULL>
__device__ __forceinline__ MvResult mv_run_t(const MvPhase& p, const float* xh, float unscale, int r0, int r1, int lane, Ring& ring,
                                             float* out, const float* hown, int hrow0, float* ybuf) {
    const int nci = pair_units(p), nch = p.K >> 5, gsh = gshift(p.gs);
    const int n = ((r1 - r0 + 1) >> 1) * nci;
    MvResult res{-INFINITY, 0x7fffffff};
    int cpr = r0, cci = 0;                 // consume pointer
    // load cursor: unit DEPTH, clamped to the last unit n - 1
    Cursor lc; cursor_pair(p, r0, r1, lane, gsh, lc);
    for (int k = 0; k < MK_DEPTH && k + 1 < n; k++) cursor_next<FULL>(p, r1, lane, gsh, nci, false, lc);
    float acc = 0.0f;
    const DotConsts kc = dot_consts();
    const bool has_bias = p.bias[0] != nullptr;
    const float* xl = xh + (lane & 31) * XH_STRIDE;       // this lane's chunk of unit 0 of a pair
    for (int u = 0; u < n; u += MK_DEPTH) {
#pragma unroll
        for (int d = 0; d < MK_DEPTH; d++) {
            const bool valid = u + d < n;                       // wave-uniform
            const int ch = (lane & 31) + 32 * cci;
            float contrib = 0.0f;
            if (valid) contrib = unit_dot(ring.code[d], ring.s[d], ring.b[d], load_x(FULL ? xl + cci * 32 * XH_STRIDE
                                          : xh + min(ch, nch - 1) * XH_STRIDE), kc);
            const bool lane_ok = FULL || ch < nch;     // a missing second row is dropped at the pair's end
            // next unit for this slot (clamped to the last one: harmless reload, never consumed)
            cursor_load<FULL>(lc, lane, nch, gsh, ring.code[d], ring.s[d], ring.b[d]);
            cursor_next<FULL>(p, r1, lane, gsh, nci, u + d + MK_DEPTH + 1 >= n, lc);
            if (valid) {
                acc += FULL ? contrib : (lane_ok ? contrib : 0.0f);
                if (++cci == nci) {
                    const float t = half_wave_sum(acc);
                    acc = 0.0f;
                    const bool two = cpr + 1 < r1;
                    float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 31)) * unscale;
                    float v1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 63)) * unscale;
                    if (has_bias) { v0 += row_bias(p, cpr); if (two) v1 += row_bias(p, cpr + 1); }
                    if (MODE == OUT_GATED) {
                        if (lane == 0) ybuf[(cpr - r0) >> 1] = (v0 / (1.0f + expf(-v0))) * v1;
                    } else {
                        if (lane < 2 && (lane == 0 || two)) ybuf[cpr - r0 + lane] = lane ? v1 : v0;
                        if (MODE == OUT_ARGMAX) {
                            if (v0 > res.best) { res.best = v0; res.best_idx = cpr; }
                            if (two && v1 > res.best) { res.best = v1; res.best_idx = cpr + 1; }
                        }
                    }
                    cci = 0; cpr += 2;
                }
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
    const int o0 = MODE == OUT_GATED ? r0 >> 1 : r0, no = MODE == OUT_GATED ? (r1 - r0) >> 1 : r1 - r0;
    for (int i = lane; i < no; i += 64) {
        const float v = ybuf[i];
        if (MODE == OUT_ARGMAX) out[o0 + i] = v;   // logits: read by the host after the launch
        else st_ag(out + o0 + i, MODE == OUT_ADD ? hown[o0 + i - hrow0] + v : v);
    }
    return res;
}
template <int MODE>
__device__ __forceinline__ MvResult mv_run(const MvPhase p, const float* xh, float unscale, int r0, int r1, int lane, Ring& ring,
                                           float* ybuf, float* out, const float* hown = nullptr, int hrow0 = 0) {
    if (mv_full(p)) return mv_run_t<MODE, true>(p, xh, unscale, r0, r1, lane, ring, out, hown, hrow0, ybuf);
    return mv_run_t<MODE, false>(p, xh, unscale, r0, r1, lane, ring, out, hown, hrow0, ybuf);
}

// Loads src[0..K) (written by other workgroups) into xf (f32, contiguous): 8 coherent 16-byte loads
// per thread in flight per batch; returns this thread's sum of squares and max |x|.
constexpr int MK_LDB = 8;
__device__ __forceinline__ float2 fetch_to_lds(const float* src, int K, float* xf) {
    float ss = 0.0f, mx = 0.0f;
    const int K4 = K >> 2;
    for (int base = 0; base < K4; base += MK_THREADS * MK_LDB) {
        float4 v[MK_LDB];
#pragma unroll
        for (int j = 0; j < MK_LDB; j++) {
            const int i4 = min(base + j * MK_THREADS + (int)threadIdx.x, K4 - 1);
            v[j] = ld_coh4(src, i4 * 4, K);
        }
#pragma unroll
        for (int j = 0; j < MK_LDB; j++) {
            const int i4 = base + j * MK_THREADS + (int)threadIdx.x;
            if (i4 < K4) {
                *reinterpret_cast<float4*>(xf + i4 * 4) = v[j];
                ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
            }
        }
    }
    return float2{ss, mx};
}

// Workgroup max of a non-negative per-thread value (red[8..15] as scratch; ends with a barrier).
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[8 + (threadIdx.x >> 6)] = v;
    __syncthreads();
    float m = 0.0f;
    for (int i = 0; i < MK_WAVES; i++) m = fmaxf(m, red[8 + i]);
    return m;
}

// x := RMSNorm(src) * w, packed to the f16 matvec layout (every workgroup computes the same
// values). Returns the unscale factor of the packing.
__device__ __forceinline__ float norm_to_lds(const float* src, const float* w, int K, float eps, float* xf, float* xh, float* red) {
    const float ss = wave_sum(fetch_to_lds(src, K, xf).x);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < MK_WAVES; i++) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)K + eps);
    float mx = 0.0f;
    for (int i = threadIdx.x * 4; i < K; i += MK_THREADS * 4) {
        float4 v = *reinterpret_cast<float4*>(xf + i);
        const float4 ww = *reinterpret_cast<const float4*>(w + i);
        v.x = v.x * inv * ww.x; v.y = v.y * inv * ww.y; v.z = v.z * inv * ww.z; v.w = v.w * inv * ww.w;
        *reinterpret_cast<float4*>(xf + i) = v;
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    return pack_x16(xf, K, block_max(mx, red), xh);
}

// x := src packed to the f16 matvec layout, plus this workgroup's residual rows h[row0 .. row1)
// into hown (for the accumulate epilogue, so no row needs its own round trip).
__device__ __forceinline__ float copy_to_lds(const float* src, int K, float* xf, float* xh, const float* h, int H, int row0,
                                             int row1, float* hown, float* red) {
    const int n = row1 - row0;
    float hv = 0.0f;
    if ((int)threadIdx.x < n) hv = ld_coh1(h, row0 + threadIdx.x, H);
    const float mx = fetch_to_lds(src, K, xf).y;
    if ((int)threadIdx.x < n) hown[threadIdx.x] = hv;
    return pack_x16(xf, K, block_max(mx, red), xh);
}

// ------------------------------------------------------------------------------- attention phase
struct KVPrefetch { uint4 k[MK_KV_PF]; uint4 v[MK_KV_PF]; };

// Key range of attention item (kvh, split): [n0, n1) of the L = pos + 1 keys.
__device__ __forceinline__ void att_range(int L, int nsplit, int split, int& n0, int& n1) {
    const int c = (L + nsplit - 1) / nsplit;
    n0 = min(L, split * c); n1 = min(L, n0 + c);
}

__device__ __forceinline__ void att_prefetch(const MegaArgs& a, const LayerDev& ly, int kvh, int n0, int n1, KVPrefetch& pf) {
    const int t = threadIdx.x, slot = t >> 4, part = t & 15;   // 16 lanes per key row, 32 keys per round
#pragma unroll
    for (int r = 0; r < MK_KV_PF; r++) {
        const int j = n0 + r * 32 + slot;
        if (j < n1) {
            const int64_t row = kv_row(a.pt, a.nKV, kvh, j) * 128 + part * 8;
            pf.k[r] = ld_stream16((gptr8)(ly.kc + row));
            pf.v[r] = ld_stream16((gptr8)(ly.vc + row));
        }
    }
}

// Register array element r (r < MK_KV_PF) without dynamic indexing (a select chain).
__device__ __forceinline__ uint4 pick_pf(const uint4 (&a)[MK_KV_PF], int r) {
    uint4 v = a[0];
#pragma unroll
    for (int i = 1; i < MK_KV_PF; i++) if (r == i) v = a[i];
    return v;
}

__device__ __forceinline__ void unpack_bf16x8(const uint4 v, float* o) {
    o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
    o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
    o[4] = __uint_as_float(v.z << 16); o[5] = __uint_as_float(v.z & 0xffff0000u);
    o[6] = __uint_as_float(v.w << 16); o[7] = __uint_as_float(v.w & 0xffff0000u);
}

// head vector (128, in LDS buf) -> per-head RMSNorm (optional) -> RoPE, 128 threads of one group
__device__ __forceinline__ float head_norm_rope(float v, int i, const float* nw, float eps, const float* invf, int pos,
                                                int rot_dim, int traditional, float* buf, float* red, int grp) {
    // grp: which 128-thread group (0..3) of the workgroup; red has 2 floats per group
    if (nw) {
        float ss = wave_sum(v * v);
        if ((i & 63) == 0) red[grp * 2 + (i >> 6)] = ss;
        __syncthreads();
        const float tot = red[grp * 2] + red[grp * 2 + 1];
        v = v * (1.0f / sqrtf(tot / 128.0f + eps)) * nw[i];
    } else {
        __syncthreads();
    }
    buf[i] = v;
    __syncthreads();
    float out = v;
    if (i < rot_dim) {
        const int half = rot_dim / 2;
        int fi, partner; bool first;
        if (traditional) { fi = i / 2; partner = i ^ 1; first = (i & 1) == 0; }
        else { fi = i % half; first = i < half; partner = first ? i + half : i - half; }
        const float ang = (float)pos * invf[fi];
        const float c = cosf(ang), sn = sinf(ang);
        out = first ? v * c - buf[partner] * sn : v * c + buf[partner] * sn;
    }
    __syncthreads();
    return out;
}

// ------------------------------------------------------------------------------- the kernel
// MAXG: the largest query-head group the attention phase's registers hold (4 or 8).
template <int MAXG>
__global__ __launch_bounds__(MK_THREADS, 1) void decode_step_kernel(MegaArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ float red[64];
    __shared__ int flag;
    const int wg = blockIdx.x, nwg = gridDim.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: row ranges stay scalar
    const int pos = *a.dpos, L = pos + 1;
    const int H = a.H, D = 128, nH = a.nH, nKV = a.nKV, G = nH / nKV;
    const int Kmax = std::max(H, std::max(a.I, nH * D));
    float* xf = lds;                              // matvec input, f32 staging (Kmax floats)
    float* xh = lds + Kmax;                       // matvec input, f16 layout (Kmax / 32 chunks)
    float* hown = xh + (Kmax >> 5) * XH_STRIDE;   // this workgroup's residual rows (up to MK_HOWN)
    float* ybuf = hown + MK_HOWN + wave * MK_YCAP; // this wave's row results
    Ring ring;
    KVPrefetch kvpf;

    // embedding row of hist[pos] -> h (each workgroup writes a slice), and the first prefetch
    {
        const int tok = a.hist[pos];
        const int gpr = H / a.embed_gs;
        for (int c = wg * MK_THREADS + tid; c < H / 8; c += nwg * MK_THREADS) {
            const uint32_t w = reinterpret_cast<const uint32_t*>(a.embed_w + (int64_t)tok * (H / 2))[c];
            const int g = (c * 8) / a.embed_gs;
            const float s = bf16_to_f32(a.embed_s[(int64_t)tok * gpr + g]), b = bf16_to_f32(a.embed_b[(int64_t)tok * gpr + g]);
#pragma unroll
            for (int j = 0; j < 8; j++) st_ag(a.h + c * 8 + j, (float)((w >> (4 * j)) & 15u) * s + b);
        }
    }
    unsigned epoch = 0;
    prof_mark(a.prof, 0);
    int r0, r1;
    prof_mark(a.prof, 2 * epoch); grid_arrive(a.sync, ++epoch);
    wave_rows(a.layers[0].qkv.rows, wg, nwg, wave, false, r0, r1);
    mv_prefetch(a.layers[0].qkv, r0, r1, lane, ring);
    grid_wait(a.sync, epoch); prof_mark(a.prof, 2 * epoch - 1);

    const int nsplit = nwg / nKV;
    for (int li = 0; li < a.L; li++) {
        const LayerDev& ly = a.layers[li];
        // ---- A: q|k|v
        {
            const float us = norm_to_lds(a.h, ly.in_norm, H, a.eps, xf, xh, red);
            prof_mark(a.prof, 512 + 8 * li + 0);
            wave_rows(ly.qkv.rows, wg, nwg, wave, false, r0, r1);
            mv_run<OUT_STORE>(ly.qkv, xh, us, r0, r1, lane, ring, ybuf, a.qkv);
        }
        prof_mark(a.prof, 2 * epoch); grid_arrive(a.sync, ++epoch);
        // prefetch this workgroup's K/V rows (positions < pos are final)
        const int item = wg;                       // nwg == nKV * nsplit
        const int kvh = item / nsplit, split = item % nsplit;
        int n0, n1; att_range(L, nsplit, split, n0, n1);
        att_prefetch(a, ly, kvh, n0, min(n1, pos), kvpf);
        grid_wait(a.sync, epoch); prof_mark(a.prof, 2 * epoch - 1);

        // ---- B: attention for (kvh, split)
        {
            float* qs = lds;                        // [G][128] scaled queries
            float* kn = qs + MK_MAXG * 128;         // new key (bf16-rounded) [128]
            float* vn = kn + 128;                   // new value [128]
            float* buf = vn + 128;                  // 4 x 128 rope scratch
            float* sc = buf + 4 * 128;              // scores [G][nk]
            const int nk = n1 - n0;
            const bool owns_new = pos >= n0 && pos < n1;
            // q heads (4 per pass of 512 threads), then the new k and v if this range holds pos
            const int grp = tid >> 7, i = tid & 127;
            const int QKV = (nH + 2 * nKV) * D;
            // every value this workgroup needs from q|k|v, loaded at once
            const float qv0 = ld_coh1(a.qkv, (kvh * G + min(grp, G - 1)) * D + i, QKV);
            const float qv1 = ld_coh1(a.qkv, (kvh * G + min(grp + 4, G - 1)) * D + i, QKV);
            const float kraw = ld_coh1(a.qkv, (nH + kvh) * D + i, QKV);
            const float vraw = ld_coh1(a.qkv, (nH + nKV + kvh) * D + i, QKV);
            for (int base = 0; base < G; base += 4) {
                const int g = base + grp;
                const float v = g < G ? (base == 0 ? qv0 : qv1) : 0.0f;
                const float o = head_norm_rope(v, i, ly.q_norm, a.eps, a.inv_freq, pos, a.rot_dim, a.traditional, buf + grp * 128, red, grp);
                if (g < G) qs[g * 128 + i] = o * a.scale;
            }
            if (owns_new) {
                const float ko = head_norm_rope(tid < 128 ? kraw : 0.0f, i, ly.k_norm, a.eps, a.inv_freq, pos, a.rot_dim, a.traditional, buf + grp * 128, red, grp);
                if (tid < 128) {
                    const uint16_t kb = f32_to_bf16(ko), vb = f32_to_bf16(vraw);
                    kn[i] = bf16_to_f32(kb); vn[i] = bf16_to_f32(vb);
                    const int64_t row = kv_row(a.pt, nKV, kvh, pos) * 128 + i;
                    ly.kc[row] = kb; ly.vc[row] = vb;
                }
            }
            __syncthreads();
            // scores: 16 lanes per key (8 dims each), 32 keys per round
            const int slot = tid >> 4, part = tid & 15;
            const int rounds = (nk + 31) / 32;
            for (int r = 0; r < rounds; r++) {
                const int jj = r * 32 + slot, j = n0 + jj;
                float kf[8];
                if (j == pos) {
#pragma unroll
                    for (int e = 0; e < 8; e++) kf[e] = kn[part * 8 + e];
                } else if (jj < nk) {
                    uint4 kv = pick_pf(kvpf.k, r);
                    if (r >= MK_KV_PF) kv = *reinterpret_cast<const uint4*>(ly.kc + kv_row(a.pt, nKV, kvh, j) * 128 + part * 8);
                    unpack_bf16x8(kv, kf);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) kf[e] = 0.0f;
                }
                for (int g = 0; g < G; g++) {
                    float s = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; e++) s = fmaf(qs[g * 128 + part * 8 + e], kf[e], s);
                    s += __shfl_xor(s, 1, 64); s += __shfl_xor(s, 2, 64); s += __shfl_xor(s, 4, 64); s += __shfl_xor(s, 8, 64);
                    if (part == 0 && jj < nk) sc[g * nk + jj] = s;
                }
            }
            __syncthreads();
            prof_mark(a.prof, 512 + 8 * li + 1);
            // softmax partial per head (waves take heads)
            float* mrow = sc + G * (nk > 0 ? nk : 1);        // [G] max, [G] sum
            for (int g = wave; g < G; g += MK_WAVES) {
                float m = -1e30f;
                for (int k = lane; k < nk; k += 64) m = fmaxf(m, sc[g * nk + k]);
                m = wave_max(m);
                float l = 0.0f;
                for (int k = lane; k < nk; k += 64) { const float p = expf(sc[g * nk + k] - m); sc[g * nk + k] = p; l += p; }
                l = wave_sum(l);
                if (lane == 0) { mrow[g] = m; mrow[MK_MAXG + g] = l; }
            }
            __syncthreads();
            // P.V: thread owns 8 dims (part) of keys slot, slot+32, ...
            float acc[MAXG][8];
#pragma unroll
            for (int g = 0; g < MAXG; g++)
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
            for (int r = 0; r < rounds; r++) {
                const int jj = r * 32 + slot, j = n0 + jj;
                if (jj >= nk) continue;
                float vf[8];
                if (j == pos) {
#pragma unroll
                    for (int e = 0; e < 8; e++) vf[e] = vn[part * 8 + e];
                } else {
                    uint4 vv = pick_pf(kvpf.v, r);
                    if (r >= MK_KV_PF) vv = *reinterpret_cast<const uint4*>(ly.vc + kv_row(a.pt, nKV, kvh, j) * 128 + part * 8);
                    unpack_bf16x8(vv, vf);
                }
#pragma unroll
                for (int g = 0; g < MAXG; g++) {
                    if (g < G) {
                        const float p = sc[g * nk + jj];
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
                    }
                }
            }
            prof_mark(a.prof, 512 + 8 * li + 2);
            // reduce over the 4 slots of a wave (lanes l, l+16, l+32, l+48), then over waves via LDS
            float* wsum = mrow + 2 * MK_MAXG;                 // [waves][G][128]
#pragma unroll
            for (int g = 0; g < MAXG; g++) {
                if (g < G) {
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        float v = acc[g][e];
                        v += __shfl_xor(v, 16, 64); v += __shfl_xor(v, 32, 64);
                        if (lane < 16) wsum[(wave * G + g) * 128 + lane * 8 + e] = v;
                    }
                }
            }
            __syncthreads();
            const int prow = (kvh * G) * nsplit;             // partial rows: (head, split)
            float* pm = a.part; float* pl = a.part + nH * nsplit; float* pa = a.part + 2 * nH * nsplit;
            for (int idx = tid; idx < G * 128; idx += MK_THREADS) {
                const int g = idx >> 7, d = idx & 127;
                float v = 0.0f;
                for (int w = 0; w < MK_WAVES; w++) v += wsum[(w * G + g) * 128 + d];
                const int r = prow + g * nsplit + split;
                st_ag(pa + (int64_t)r * 128 + d, nk > 0 ? v : 0.0f);
                if (d == 0) { st_ag(pm + r, nk > 0 ? mrow[g] : -1e30f); st_ag(pl + r, nk > 0 ? mrow[MK_MAXG + g] : 0.0f); }
            }
            prof_mark(a.prof, 512 + 8 * li + 3);
            // the last range of this KV head to finish merges the partials in range order
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid == 0) {
                const unsigned done = add_ag(&a.kv_done[kvh * 32], 1u);
                flag = done == (unsigned)nsplit - 1;
                if (flag) __hip_atomic_store(&a.kv_done[kvh * 32], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            if (flag) {
                // merge: weights f_s = exp(m_s - M) and 1 / sum_s l_s f_s per head (m, l staged in LDS),
                // then every (head, dim) sums its nsplit partials, loaded 32 at a time
                const int P = nH * nsplit;
                float* wts = wsum;                                  // [G][nsplit] weights
                float* lsv = wsum + MK_MAXG * 64;                   // [G][nsplit] sums
                for (int idx = tid; idx < G * nsplit; idx += MK_THREADS) {
                    wts[idx] = ld_coh1(pm, prow + idx, P);
                    lsv[idx] = ld_coh1(pl, prow + idx, P);
                }
                __syncthreads();
                if (tid < G) {
                    float M = -1e30f;
                    for (int s = 0; s < nsplit; s++) M = fmaxf(M, wts[tid * nsplit + s]);
                    float Ls = 0.0f;
                    for (int s = 0; s < nsplit; s++) {
                        const float f = expf(wts[tid * nsplit + s] - M);
                        wts[tid * nsplit + s] = f;
                        Ls += lsv[tid * nsplit + s] * f;
                    }
                    mrow[tid] = 1.0f / Ls;
                }
                __syncthreads();
                for (int idx = tid; idx < G * 128; idx += MK_THREADS) {
                    const int g = idx >> 7, d = idx & 127;
                    const int rb = prow + g * nsplit;
                    float o = 0.0f;
                    for (int s0 = 0; s0 < nsplit; s0 += 32) {
                        float v[32];
#pragma unroll
                        for (int q = 0; q < 32; q++) v[q] = ld_coh1(pa, (rb + min(s0 + q, nsplit - 1)) * 128 + d, P * 128);
#pragma unroll
                        for (int q = 0; q < 32; q++) if (s0 + q < nsplit) o += v[q] * wts[g * nsplit + s0 + q];
                    }
                    st_ag(a.attn + (kvh * G + g) * 128 + d, o * mrow[g]);
                }
            }
        }
        prof_mark(a.prof, 2 * epoch); grid_arrive(a.sync, ++epoch);
        wave_rows(ly.o.rows, wg, nwg, wave, false, r0, r1);
        mv_prefetch(ly.o, r0, r1, lane, ring);
        grid_wait(a.sync, epoch); prof_mark(a.prof, 2 * epoch - 1);

        // ---- C: o_proj, h += W_o attn
        {
            int g0, g1; wg_rows(ly.o.rows, wg, nwg, g0, g1);
            const float us = copy_to_lds(a.attn, nH * D, xf, xh, a.h, H, g0, g1, hown, red);
            prof_mark(a.prof, 512 + 8 * li + 4);
            mv_run<OUT_ADD>(ly.o, xh, us, r0, r1, lane, ring, ybuf, a.h, hown, g0);
        }
        prof_mark(a.prof, 2 * epoch); grid_arrive(a.sync, ++epoch);
        wave_rows(ly.gu.rows, wg, nwg, wave, true, r0, r1);
        mv_prefetch(ly.gu, r0, r1, lane, ring);
        grid_wait(a.sync, epoch); prof_mark(a.prof, 2 * epoch - 1);

        // ---- D: gate|up with SiLU
        {
            const float us = norm_to_lds(a.h, ly.post_norm, H, a.eps, xf, xh, red);
            prof_mark(a.prof, 512 + 8 * li + 5);
            mv_run<OUT_GATED>(ly.gu, xh, us, r0, r1, lane, ring, ybuf, a.mlp);
        }
        prof_mark(a.prof, 2 * epoch); grid_arrive(a.sync, ++epoch);
        wave_rows(ly.down.rows, wg, nwg, wave, false, r0, r1);
        mv_prefetch(ly.down, r0, r1, lane, ring);
        grid_wait(a.sync, epoch); prof_mark(a.prof, 2 * epoch - 1);

        // ---- E: down, h += W_d mlp
        {
            int g0, g1; wg_rows(ly.down.rows, wg, nwg, g0, g1);
            const float us = copy_to_lds(a.mlp, a.I, xf, xh, a.h, H, g0, g1, hown, red);
            prof_mark(a.prof, 512 + 8 * li + 6);
            mv_run<OUT_ADD>(ly.down, xh, us, r0, r1, lane, ring, ybuf, a.h, hown, g0);
        }
        prof_mark(a.prof, 2 * epoch); grid_arrive(a.sync, ++epoch);
        if (li + 1 < a.L) {
            wave_rows(a.layers[li + 1].qkv.rows, wg, nwg, wave, false, r0, r1);
            mv_prefetch(a.layers[li + 1].qkv, r0, r1, lane, ring);
        } else {
            wave_rows(a.head.rows, wg, nwg, wave, false, r0, r1);
            mv_prefetch(a.head, r0, r1, lane, ring);
        }
        grid_wait(a.sync, epoch); prof_mark(a.prof, 2 * epoch - 1);
    }

    // ---- lm_head with the final norm, logits and the greedy token
    const float us = norm_to_lds(a.h, a.final_norm, H, a.eps, xf, xh, red);
    const MvResult best = mv_run<OUT_ARGMAX>(a.head, xh, us, r0, r1, lane, ring, ybuf, a.logits);
    prof_mark(a.prof, 2 * epoch);
    __shared__ float bv[MK_WAVES];
    __shared__ int bi[MK_WAVES];
    if (lane == 0) { bv[wave] = best.best; bi[wave] = best.best_idx; }
    __syncthreads();
    if (tid == 0) {
        float m = -INFINITY; int idx = 0x7fffffff;
        for (int w = 0; w < MK_WAVES; w++)   // waves hold ascending row ranges
            if (bv[w] > m) { m = bv[w]; idx = bi[w]; }
        st_ag(a.wg_best + wg, m); st_ag(a.wg_idx + wg, idx);
        __builtin_amdgcn_s_waitcnt(0);
        const unsigned done = add_ag(a.head_done, 1u);
        flag = done == (unsigned)nwg - 1;
        if (flag) {   // every workgroup is past its last barrier: reset the counters for the next launch
            __hip_atomic_store(a.head_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.sync->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.sync->gen, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int x = 0; x < 8; x++) __hip_atomic_store(&a.sync->xcd[x][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    const int ok = isfinite(m) ? 1 : 0;
    const int tok = ok ? idx : 0;
    a.hist[pos + 1] = tok; a.status[pos + 1] = ok ? 0 : 1;
    if (a.ring_tok) { a.ring_tok[(pos + 1) & a.ring_mask] = tok; a.ring_status[(pos + 1) & a.ring_mask] = ok ? 0 : 1; }
    *a.dpos = pos + 1;
}

size_t mega_lds_bytes(const MegaArgs& a, int max_keys_per_split) {
    const int G = a.nH / a.nKV;
    const size_t kmax = (size_t)std::max(a.H, std::max(a.I, a.nH * 128));
    size_t mv = (kmax + kmax / 32 * XH_STRIDE + MK_HOWN + MK_WAVES * MK_YCAP) * 4;
    size_t att = (size_t)(MK_MAXG * 128 + 256 + 512) * 4 + (size_t)G * max_keys_per_split * 4 + 2 * MK_MAXG * 4 +
                 (size_t)std::max(MK_WAVES * G * 128, 2 * MK_MAXG * 64) * 4;
    return std::max(mv, att);
}

hipError_t launch_decode_step(const MegaArgs& a, int nwg, size_t lds, hipStream_t s) {
    if (a.nH / a.nKV <= 4) hipLaunchKernelGGL(decode_step_kernel<4>, dim3(nwg), dim3(MK_THREADS), lds, s, a);
    else hipLaunchKernelGGL(decode_step_kernel<8>, dim3(nwg), dim3(MK_THREADS), lds, s, a);
    return hipGetLastError();
}

hipError_t mega_set_lds_limit(size_t lds) {
    hipError_t e = hipFuncSetAttribute((const void*)decode_step_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute((const void*)decode_step_kernel<8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

int mega_threads() { return MK_THREADS; }
int mega_wave_row_cap() { return MK_YCAP; }
int mega_wg_row_cap() { return MK_HOWN; }

}  // namespace mlxr
