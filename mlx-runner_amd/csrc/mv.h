// Matvec building blocks over the repacked weight tiles (DPack), shared by the persistent decode
// step (decode.hip) and the standalone per-projection matvec (dmv.hip).
#pragma once
#include <type_traits>
#include "decode.h"

namespace mlxr {

constexpr int MK_THREADS = 512;
constexpr int MK_WAVES = MK_THREADS / 64;
constexpr int MK_TPW = 40;           // 16-row tiles of one workgroup in a matvec phase (max; a 152K vocab over 256 CUs needs 38)

// ------------------------------------------------------------------------------- matvec phase
// Weights of the persistent step are a repacked copy (DPack, built once at load by dpack_kernel).
// A matrix is cut into tiles of 16 rows; a tile is a sequence of scale groups, each covering 16
// quantization groups (FB = gs / 8 code blocks of 128 codes) and stored as FB + 1 blocks of 1 KB
// (one 16-byte slice per lane):
//   block 0      (scale | bias << 16) of rows 4 (l >> 4) + i (i = slot dword), group 16 f + (l & 15):
//                the accumulator layout of v_mfma_f32_16x16x32_f16;
//   blocks 1..FB code block k: row 16 t + (l & 15), code dwords 16 kb + 4 j + (l >> 4) (j = slot
//                dword, one per MFMA), kb = FB f + k - 1: the A-operand layout.
// Gated phases put gate rows 8t..8t+7 in tile rows 0-7 and the matching up rows in rows 8-15.
// A wave streams whole scale groups, so its loads walk one contiguous range and every ring slot
// has a fixed role (slot 0: scales, slot k: code block k - 1).
//
// MFMA formulation: a code masked into the low mantissa bits of an f16 with a zero exponent is the
// subnormal q * 2^-24 (the nibble at bits 4..7 gives 16 q * 2^-24, met by x / 16 in the operand), so
// A is built with one AND per two codes and carries the codes exactly, with no offset. The input
// enters as two f16 parts, x = hi + lo (lo = f16(x - hi): ~22 significant bits, fp32 accuracy for
// the matvec). B holds the chunk's hi in the column of the chunk's group g and its lo in column
// g ^ 8, zeros elsewhere. Groups 0-7 of a scale group accumulate into one register set and groups
// 8-15 into another, so in each set columns c and c ^ 8 are the hi and lo sums of one group; one
// cross-lane add per set joins them:
//   D_rg = sum q (hi + lo) * 2^-24      (products exact, fp32 accumulation)
// and the scale and bias are applied once per scale group:
//   y_row += s_rg 2^24 D_rg + b_rg Xs_g,   Xs_g = sum of the group's x (fp32).
typedef MvPhaseDesc MvPhase;

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
// Global-address-space pointers: loads through them are global (not flat) loads, which count on
// the memory counter only; a flat load also counts on the LDS counter, so every wait for an LDS
// read would wait for it too.
typedef const __attribute__((address_space(1))) uint8_t* gptr8;
typedef const __attribute__((address_space(1))) u32x4_t* gptr128;
// 16-byte streaming load (data read once: the nontemporal hint keeps it from displacing activations)
__device__ __forceinline__ uint4 ld_stream16(gptr8 p) {
    const u32x4_t v = __builtin_nontemporal_load((gptr128)p);
    return uint4{v.x, v.y, v.z, v.w};
}

// One scale group in flight per lane (FB + 1 slices of 16 bytes), kept exactly as loaded: no
// instruction touches a slot before it is consumed, so the memory-counter wait for a slot never
// drains the loads after it.
template <int FB>
struct Ring { uint4 u[FB + 1]; };

// Geometry of a phase for this workgroup / wave.
template <int FB>
struct MvGeom {
    int KBT, NF;            // code blocks and scale groups per tile
    int t0, nt;             // this workgroup's tiles [t0, t0 + nt)
    int f0, f1;             // this wave's scale groups [f0, f1) in the workgroup's tile-major order
};
template <int FB>
__device__ __forceinline__ MvGeom<FB> mv_geom(const MvPhase& p, int wg, int nwg, int wave) {
    MvGeom<FB> g;
    g.KBT = p.K >> 7; g.NF = (g.KBT + FB - 1) / FB;
    // 32-bit: tiles * workgroups stays far below 2^31 (tiles <= 2^16, checked at setup)
    g.t0 = (int)((unsigned)(p.tiles * wg) / (unsigned)nwg);
    g.nt = (int)((unsigned)(p.tiles * (wg + 1)) / (unsigned)nwg) - g.t0;
    const int nfw = g.nt * g.NF;
    g.f0 = (nfw * wave) >> 3; g.f1 = (nfw * (wave + 1)) >> 3;   // MK_WAVES == 8
    static_assert(MK_WAVES == 8, "wave split");
    return g;
}
// This lane's slice of the wave's first scale group (TS: tiles p.tstride scale groups apart, the
// phase covering a run of each tile's scale groups).
template <int FB, bool TS = false>
__device__ __forceinline__ gptr8 mv_base(const MvPhase& p, const MvGeom<FB>& g, int lane) {
    if constexpr (TS) {
        const int tl = g.f0 / g.NF;
        return (gptr8)p.code + (size_t)(unsigned)((g.t0 + tl) * p.tstride + g.f0 - tl * g.NF) * ((FB + 1) * 1024) + lane * 16;
    }
    return (gptr8)p.code + (size_t)(unsigned)(g.t0 * g.NF + g.f0) * ((FB + 1) * 1024) + lane * 16;
}

template <int FB, bool TS = false>
__device__ __forceinline__ void mv_prefetch(const MvPhase p, int wg, int nwg, int wave, int lane, Ring<FB>& ring) {
    const MvGeom<FB> g = mv_geom<FB>(p, wg, nwg, wave);
    if (g.f1 <= g.f0) {   // every path defines the ring, so no earlier value stays live across phases
#pragma unroll
        for (int d = 0; d <= FB; d++) ring.u[d] = uint4{0u, 0u, 0u, 0u};
        return;
    }
    const gptr8 b = mv_base<FB, TS>(p, g, lane);
#pragma unroll
    for (int d = 0; d <= FB; d++) ring.u[d] = ld_stream16(b + d * 1024);
}

// mv_prefetch without a branch: a wave without scale groups reads its workgroup's last one, unused
// (the workgroup has at least one tile). Loads issued in a branch make every later wait on the
// memory counter count from zero, so a kernel that issues x before the weights and waits for x
// alone needs the weights' loads unconditional.
template <int FB, bool TS = false>
__device__ __forceinline__ void mv_prefetch_all(const MvPhase p, int wg, int nwg, int wave, int lane, Ring<FB>& ring) {
    MvGeom<FB> g = mv_geom<FB>(p, wg, nwg, wave);
    g.f0 = max(0, min(g.f0, g.nt * g.NF - 1));
    const gptr8 b = mv_base<FB, TS>(p, g, lane);
#pragma unroll
    for (int d = 0; d <= FB; d++) ring.u[d] = ld_stream16(b + d * 1024);
}

// A operand of one code dword: halves (n0, n4, 16 n1, 16 n5, n2, n6, 16 n3, 16 n7) * 2^-24 (subnormal).
// No inline assembly here: the compiler must see every VGPR write that feeds an MFMA operand to
// insert the wait states the matrix core requires.
__device__ __forceinline__ f16x8_t a_operand(uint32_t w) {
    const uint32_t w8 = w >> 8;
    const u32x4_t v = {w & 0x000F000Fu, w & 0x00F000F0u, w8 & 0x000F000Fu, w8 & 0x00F000F0u};
    return __builtin_bit_cast(f16x8_t, v);
}

// LDS layout of the matvec input (f16): chunk c of 32 values at xh + 32 * c (128 bytes); code dword i
// of the chunk (codes 8i..8i+7, nibble j at bits 4j) matched by the 16-byte slot i holding
//   (x0, x4), (x1 / 16, x5 / 16), (x2, x6), (x3 / 16, x7 / 16)      (hi parts of codes 8i..8i+7)
// after a power-of-two scaling of the whole vector, and slot 4 + i holding the lo parts in the same
// order. gsum[g] holds Xs, the sum of quantization group g's scaled x; zero16 is 16 bytes of zeros
// (the masked B operand).
constexpr int XH_STRIDE = 32;          // floats per chunk
constexpr int XH_LO = 16;              // floats from a chunk's hi slots to its lo slots
constexpr int MV_ZERO = 64;            // floats of zeros (a B operand read of any chunk of a group in it reads zeros)

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// Packs x[0..K) (f32, read through the loader; every value already final, max |x| reduced by the
// caller into gmax) into the f16 layout above and the group sums for group size 2^gsh. Scale 2^e
// maps max |x| below 2^14, so every stored half is finite and (for all but values 2^28 below the
// maximum) normal. Returns 2^-e.
// LDS of a matvec phase (the attention phase reuses the same memory, so every phase rebuilds it).
struct MvLds { float* xf; float* xh; float* gsum; float* zero16; float* hown; float* part; };

// LD(t, lo, hi) yields values 8t..8t+7 of x. BAR: end with a barrier (the packed x readable by
// every wave); without it the caller places one after packing several inputs.
template <typename LD, bool BAR = true>
__device__ __forceinline__ float pack_x16_from(const LD& ld, int K, float gmax, const MvLds& L, int gsh) {
    float* xh = L.xh; float* gsum = L.gsum;
    if (threadIdx.x < MV_ZERO) L.zero16[threadIdx.x] = 0.0f;
    int ex = 0;
    if (gmax > 0.0f && gmax <= 3.0e38f) frexpf(gmax, &ex);
    const int e = min(max(14 - ex, -100), 100);
    const float up = ldexpf(1.0f, e);
    for (int t = threadIdx.x; t < (K >> 3); t += MK_THREADS) {   // t: 8 values; 4 consecutive t per chunk
        float4 lo, hi;
        ld(t, lo, hi);
        // scaled values in slot order (x0, x4, x1 / 16, x5 / 16, x2, x6, x3 / 16, x7 / 16)
        const float v[8] = {lo.x * up, hi.x * up, lo.y * up * 0.0625f, hi.y * up * 0.0625f,
                            lo.z * up, hi.z * up, lo.w * up * 0.0625f, hi.w * up * 0.0625f};
        _Float16 hh[8], hl[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            hh[i] = (_Float16)v[i];
            hl[i] = (_Float16)(v[i] - (float)hh[i]);
        }
        uint4 o, ol;
        o.x = __builtin_bit_cast(uint32_t, h2_t{hh[0], hh[1]});
        o.y = __builtin_bit_cast(uint32_t, h2_t{hh[2], hh[3]});
        o.z = __builtin_bit_cast(uint32_t, h2_t{hh[4], hh[5]});
        o.w = __builtin_bit_cast(uint32_t, h2_t{hh[6], hh[7]});
        ol.x = __builtin_bit_cast(uint32_t, h2_t{hl[0], hl[1]});
        ol.y = __builtin_bit_cast(uint32_t, h2_t{hl[2], hl[3]});
        ol.z = __builtin_bit_cast(uint32_t, h2_t{hl[4], hl[5]});
        ol.w = __builtin_bit_cast(uint32_t, h2_t{hl[6], hl[7]});
        const int c = t >> 2;
        *reinterpret_cast<uint4*>(xh + c * XH_STRIDE + (t & 3) * 4) = o;
        *reinterpret_cast<uint4*>(xh + c * XH_STRIDE + XH_LO + (t & 3) * 4) = ol;
        // Xs of the quantization group: the 4 (gs 32) or 8 (gs 64) t of a group sit in consecutive
        // lanes of one wave (K is a multiple of 128, so whole groups are active)
        // (lane moves within rows of 16: quad swaps, then the half-row mirror, whose partner 7 - i
        // holds the same quad sum as i ^ 4)
        float xsum = ((lo.x + lo.y) + (lo.z + lo.w) + ((hi.x + hi.y) + (hi.z + hi.w))) * up;
        xsum = quad_sum(xsum);
        if (gsh == 6) xsum += dpp<0x141>(xsum);
        if ((t & ((1 << (gsh - 3)) - 1)) == 0) gsum[t >> (gsh - 3)] = xsum;
    }
    if constexpr (BAR) lds_barrier();
    return 1.0f / up;
}
__device__ __forceinline__ float pack_x16(const float* xf, int K, float gmax, const MvLds& L, int gsh) {
    auto ld = [xf](int t, float4& lo, float4& hi) {
        lo = *reinterpret_cast<const float4*>(xf + 8 * t);
        hi = *reinterpret_cast<const float4*>(xf + 8 * t + 4);
    };
    return pack_x16_from(ld, K, gmax, L, gsh);
}


// Streams the wave's scale groups (the first already in the ring), leaving per-tile partial row
// sums in part[(tile * MK_WAVES + wave) * 16 + row] (LDS) for mv_finish.
template <int FB, bool STRAIGHT = false, bool TS = false>
__device__ __forceinline__ void mv_run(const MvPhase p, const float* xh, const float* gsum, const float* zero16, int wg, int nwg,
                                       int wave, int lane, Ring<FB>& ring, float* part) {
    constexpr int GSH = FB == 4 ? 5 : 6;          // log2 of the group size
    const MvGeom<FB> g = mv_geom<FB>(p, wg, nwg, wave);
    const int nfb = g.f1 - g.f0;
    if (nfb <= 0) return;
    const int gpr = p.K >> GSH;                   // groups per row
    const gptr8 base = mv_base<FB, TS>(p, g, lane);
    const int col = lane & 15;
    f32x4_t run = {0.0f, 0.0f, 0.0f, 0.0f};
    int tile = g.f0 / g.NF, f = g.f0 - tile * g.NF;   // scale group within the tile
    gptr8 cur = base;                                 // TS: this scale group's address
    for (int i = 0; i < nfb; i++) {
        // the next scale group streams in behind this one (none after the last: no load is left in flight)
        const bool more = i + 1 < nfb;
        gptr8 nxt;
        if constexpr (TS) nxt = cur = cur + (int64_t)(f + 1 == g.NF ? p.tstride - g.NF + 1 : 1) * ((FB + 1) * 1024);
        else nxt = base + (int64_t)(i + 1) * ((FB + 1) * 1024);
        const uint4 sbr = ring.u[0];
        if (more) ring.u[0] = ld_stream16(nxt);
        const float* xb = xh + (lane >> 4) * 4 + f * (4 * FB) * XH_STRIDE;   // this lane's slot of the group's first chunk
        // groups 0-7 of the scale group accumulate in accA, 8-15 in accB; each split in two (even /
        // odd chunks) for half the dependent MFMA chain
        f32x4_t accA = {0.0f, 0.0f, 0.0f, 0.0f}, accA2 = {0.0f, 0.0f, 0.0f, 0.0f};
        f32x4_t accB = {0.0f, 0.0f, 0.0f, 0.0f}, accB2 = {0.0f, 0.0f, 0.0f, 0.0f};
        // one scale group: straight-line code when the reloads' condition is taken outside it
        // (STRAIGHT), so the compiler issues the B-operand LDS reads ahead of the MFMAs that use
        // them; with the condition inside, each slot's reload follows its MFMAs directly, which
        // keeps a long stream of groups fed (the standalone matvec)
        auto group = [&](auto reload) {
#pragma unroll
            for (int k = 0; k < FB; k++) {
                const uint4 unit = ring.u[k + 1];
                const uint32_t wd[4] = {unit.x, unit.y, unit.z, unit.w};
                f16x8_t b[4];
                constexpr int CPG = 1 << (GSH - 5);                            // chunks per group
                const bool high = (4 * k) / CPG >= 8;                          // groups 8-15 (accB)
                auto mfma = [&](int j, const f16x8_t& bj) {   // k and j are constants after unrolling
                    const f16x8_t av = a_operand(wd[j]);
                    if (high) {
                        if (j & 1) accB2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bj, accB2, 0, 0, 0);
                        else accB = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bj, accB, 0, 0, 0);
                    } else {
                        if (j & 1) accA2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bj, accA2, 0, 0, 0);
                        else accA = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bj, accA, 0, 0, 0);
                    }
                };
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    // one base per group (the j of a group share it), the chunk's place as a constant
                    // offset: the group's hi slots, its lo slots, or the zero region shifted back by
                    // the group's offset, so that every chunk of the group reads zeros there
                    const int gcol = (4 * k + j) / CPG;                        // the chunk's group column
                    const int g0 = gcol * CPG * XH_STRIDE;                    // the group's first chunk
                    const float* gb = col == gcol ? xb : col == (gcol ^ 8) ? xb + XH_LO : zero16 - g0;
                    const float* bp = gb + g0 + (4 * k + j - gcol * CPG) * XH_STRIDE;
                    b[j] = __builtin_bit_cast(f16x8_t, *reinterpret_cast<const uint4*>(bp));
                    if constexpr (!STRAIGHT) mfma(j, b[j]);   // each operand read right before its MFMA
                }
                if constexpr (STRAIGHT) {        // the four reads first, then the four MFMAs
#pragma unroll
                    for (int j = 0; j < 4; j++) mfma(j, b[j]);
                }
                if constexpr (!STRAIGHT) {
                    if (more) ring.u[k + 1] = ld_stream16(nxt + (k + 1) * 1024);
                } else if constexpr (decltype(reload)::value) {
                    ring.u[k + 1] = ld_stream16(nxt + (k + 1) * 1024);
                }
            }
        };
        if (!STRAIGHT || more) group(std::true_type{});
        else group(std::false_type{});
        // scales of the 16 groups (groups past the row's last are zero-scaled; their sums may be junk)
        const int gi = 16 * f + col;
        const bool real = gi < gpr;
        const float xs = gsum[real ? gi : 0];
        accA += accA2; accB += accB2;
        f32x4_t acc;
#pragma unroll
        for (int r = 0; r < 4; r++) {   // hi (column c) + lo (column c ^ 8) of each group
            const float sa = accA[r] + dpp<0x128>(accA[r]), sb = accB[r] + dpp<0x128>(accB[r]);   // lane c ^ 8: row rotation by 8
            acc[r] = col < 8 ? sa : sb;
        }
        const uint32_t sv[4] = {sbr.x, sbr.y, sbr.z, sbr.w};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float sc = __uint_as_float(sv[r] << 16) * 16777216.0f, bb = __uint_as_float(sv[r] & 0xffff0000u);
            const float t = sc * acc[r] + bb * xs;
            run[r] += real ? t : 0.0f;
        }
        if (f == g.NF - 1 || i == nfb - 1) {     // tile done (or the wave's range): row sums to LDS
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float v = row16_sum(run[r]);
                if (col == 0) part[(tile * MK_WAVES + wave) * 16 + 4 * (lane >> 4) + r] = v;
            }
            run = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (++f == g.NF) { f = 0; tile++; }
    }
}

enum MvOut { OUT_STORE = 0, OUT_ADD = 1, OUT_GATED = 2, OUT_ARGMAX = 3 };

struct MvResult { float best; int best_idx; };

// Branch-free (part, row) of a concatenated row (bias lookup).
__device__ __forceinline__ void mv_locate(const MvPhase& p, int vr, int& part, int& row) {
    const int a = vr >= p.o1 ? 1 : 0, b = vr >= p.o1 + p.o2 ? 1 : 0;
    part = a + b; row = vr - (a ? p.o1 : 0) - (b ? p.o2 : 0);
}
__device__ __forceinline__ float row_bias(const MvPhase& p, int vr) {
    if (!p.bias[0]) return 0.0f;
    int part, row; mv_locate(p, vr, part, row);
    const uint16_t* b = part == 0 ? p.bias[0] : part == 1 ? p.bias[1] : p.bias[2];
    return bf16_to_f32(gload(b + row));
}

// Half scale groups: for the phases with few scale groups per workgroup (q|k|v, o_proj: one per
// wave or fewer), each scale group is cut into two units, its first and its second half of code
// blocks (quantization groups 0-7 and 8-15), each with the group's scale block, so twice as many
// waves work and each wave's chain of dependent MFMAs is half as long (the scale block is read
// twice: 1 KB more per 9 KB). Unit u of the workgroup's tile-major order: group u >> 1, half u & 1.
template <int FB>
__device__ __forceinline__ void mvh_geom(const MvPhase& p, int wg, int nwg, int wave, int& NF, int& t0, int& nt, int& u0, int& u1) {
    NF = ((p.K >> 7) + FB - 1) / FB;
    t0 = (int)((unsigned)(p.tiles * wg) / (unsigned)nwg);
    nt = (int)((unsigned)(p.tiles * (wg + 1)) / (unsigned)nwg) - t0;
    const int nu = 2 * nt * NF;
    u0 = (nu * wave) >> 3; u1 = (nu * (wave + 1)) >> 3;
}
// Block b (0: scales, 1..FB/2: the half's code blocks) of unit u, this lane's 16 bytes.
template <int FB>
__device__ __forceinline__ gptr8 mvh_block(const MvPhase& p, int NF, int t0, int u, int b, int lane) {
    const int gi = u >> 1, h = u & 1;   // group in the workgroup's tile-major order, half
    const int blk = b == 0 ? 0 : 1 + h * (FB / 2) + (b - 1);
    return (gptr8)p.code + ((size_t)(unsigned)(t0 * NF + gi) * (FB + 1) + blk) * 1024 + lane * 16;
}
template <int FB>
__device__ __forceinline__ void mvh_prefetch(const MvPhase p, int wg, int nwg, int wave, int lane, Ring<FB>& ring) {
    int NF, t0, nt, u0, u1;
    mvh_geom<FB>(p, wg, nwg, wave, NF, t0, nt, u0, u1);
#pragma unroll
    for (int b = 0; b <= FB; b++) ring.u[b] = uint4{0u, 0u, 0u, 0u};
    if (u1 <= u0) return;
#pragma unroll
    for (int b = 0; b <= FB / 2; b++) ring.u[b] = ld_stream16(mvh_block<FB>(p, NF, t0, u0, b, lane));
}
// mv_run over half units (the first unit already in ring slots 0..FB/2). Partial row sums per
// tile as mv_run leaves them; mv_finish combines them with tile_row(.., 2 * nt * NF, 2 * NF).
template <int FB>
__device__ __forceinline__ void mvh_run(const MvPhase p, const float* xh, const float* gsum, const float* zero16, int wg, int nwg,
                                        int wave, int lane, Ring<FB>& ring, float* part) {
    constexpr int GSH = FB == 4 ? 5 : 6;
    constexpr int CPG = 1 << (GSH - 5);           // chunks per group
    constexpr int HB = FB / 2;                     // code blocks per half
    int NF, t0, nt, u0, u1;
    mvh_geom<FB>(p, wg, nwg, wave, NF, t0, nt, u0, u1);
    if (u1 <= u0) return;
    const int gpr = p.K >> GSH;
    const int col = lane & 15;
    f32x4_t run = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int u = u0; u < u1; u++) {
        const bool more = u + 1 < u1;
        const int gi = u >> 1, h = u & 1, tile = gi / NF, f = gi - tile * NF;
        const uint4 sbr = ring.u[0];
        if (more) ring.u[0] = ld_stream16(mvh_block<FB>(p, NF, t0, u + 1, 0, lane));
        const float* xb = xh + (lane >> 4) * 4 + f * (4 * FB) * XH_STRIDE;
        f32x4_t acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
        // code blocks H * HB .. of the group (H a constant in each copy of the body)
        auto body = [&](auto HC) {
            constexpr int H = decltype(HC)::value;
#pragma unroll
            for (int kl = 0; kl < HB; kl++) {
                const int k = H * HB + kl;                                 // block within the group
                const uint4 unit = ring.u[1 + kl];
                const uint32_t wd[4] = {unit.x, unit.y, unit.z, unit.w};
                f16x8_t b[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int gcol = (4 * k + j) / CPG;
                    const int g0 = gcol * CPG * XH_STRIDE;
                    const float* gb = col == gcol ? xb : col == (gcol ^ 8) ? xb + XH_LO : zero16 - g0;
                    const float* bp = gb + g0 + (4 * k + j - gcol * CPG) * XH_STRIDE;
                    b[j] = __builtin_bit_cast(f16x8_t, *reinterpret_cast<const uint4*>(bp));
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const f16x8_t av = a_operand(wd[j]);
                    if (j & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b[j], acc1, 0, 0, 0);
                    else acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b[j], acc0, 0, 0, 0);
                }
                if (more) ring.u[1 + kl] = ld_stream16(mvh_block<FB>(p, NF, t0, u + 1, 1 + kl, lane));
            }
        };
        if (h == 0) body(std::integral_constant<int, 0>{});
        else body(std::integral_constant<int, 1>{});
        acc0 += acc1;
        // this half's groups are columns 8h .. 8h + 7 (hi), their lo parts in the other eight
        const bool mine = (col >> 3) == h;
        const int gi16 = 16 * f + col;
        const bool real = mine && gi16 < gpr;
        const float xs = gsum[real ? gi16 : 0];
        const uint32_t sv[4] = {sbr.x, sbr.y, sbr.z, sbr.w};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float a = acc0[r] + dpp<0x128>(acc0[r]);   // lane c ^ 8: row rotation by 8
            const float sc = __uint_as_float(sv[r] << 16) * 16777216.0f, bb = __uint_as_float(sv[r] & 0xffff0000u);
            const float t = sc * a + bb * xs;
            run[r] += real ? t : 0.0f;
        }
        if ((f == NF - 1 && h == 1) || !more) {    // tile done (or the wave's range): row sums to LDS
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float v = row16_sum(run[r]);
                if (col == 0) part[(tile * MK_WAVES + wave) * 16 + 4 * (lane >> 4) + r] = v;
            }
            run = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
}

// Row r of tile tl of this workgroup: the partial sums of the waves whose ranges meet the tile, in
// wave order.
__device__ __forceinline__ float tile_row(const float* part, int tl, int r, int nfw, int NF) {
    float v[MK_WAVES];
#pragma unroll
    for (int w = 0; w < MK_WAVES; w++) v[w] = part[(tl * MK_WAVES + w) * 16 + r];   // all read at once, then masked
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < MK_WAVES; w++) {
        const int a = (nfw * w) >> 3, b = (nfw * (w + 1)) >> 3;
        if (a < b && a < (tl + 1) * NF && b > tl * NF) s += v[w];   // non-empty, meets the tile
    }
    return s;
}


}  // namespace mlxr
