// Persistent decode step (decode.hip): device-side descriptors.
#pragma once
#include <algorithm>
#include "kernels.h"

namespace mlxr {

// A matvec phase over a repacked (DPack) matrix: rows of up to three concatenated matrices (o1, o2:
// rows of parts 0 and 1), or gated (o1 = o2 = outputs; gate and up rows interleaved per tile).
struct MvPhaseDesc {
    const uint8_t* code;                      // DPack stream (scale groups of scale + code blocks)
    const uint16_t* bias[3];                  // optional per-row bias of each part (bf16)
    int o1, o2, rows, K, gs, gated, tiles;
    int tstride;   // scale groups from one tile's first to the next's when they are not contiguous (an input slice), else 0
};

// Source of a repack: the MLX layout (codes [O][K/2], bf16 scales / biases [O][K/gs]) of each part.
struct DPackSrc {
    const uint8_t* w[3]; const uint16_t* s[3]; const uint16_t* b[3];
    int o1, o2, rows, K, gs, gated;
};
int dpack_tiles(const DPackSrc& s);
size_t dpack_bytes(const DPackSrc& s);
hipError_t launch_dpack(const DPackSrc& s, uint8_t* out, hipStream_t st);

// Prefill GEMM over a repacked matrix (ptile.hip): y[T][rows] (gated: y[T][o1] = SiLU(gate) * up)
// from x already converted by the 4-bit GEMM pre-pass (xh: f16 rows scaled by 1 / inv[t]).
bool tile_gemm_supported(const MvPhaseDesc& p);
hipError_t launch_tile_gemm(const MvPhaseDesc& p, const uint16_t* xh, const float* inv, int T, float* y, int ys,
                            hipStream_t s);

// Batch-1 matvec over a repacked matrix (the kernel-per-op decode step): mode 0 y = W x (+ bias),
// 1 y += W x (+ bias), 2 y[o1] = SiLU(gate) * up; norm_w: x := RMSNorm(x) * norm_w first.
bool dpack_mv_supported(const MvPhaseDesc& p);
// split: optional scratch of dpack_mv_split_floats(rows) floats, zeroed once before its first use
// (its tile counters return to zero after every launch); with it, a projection without norm or
// gate whose tiles are too few to spread evenly over the CUs runs as up to DMV_MAX_SLICES input
// slices of every tile, the slices' partials combined in order by the last of them.
// Every split launch (this one and the small-batch launch below) keeps its per-tile counters in the
// first DMV_SPLIT_CNT words of the scratch and its partials after them, so launches of different
// tile counts sharing one scratch never write partials over another launch's counters.
constexpr int DMV_MAX_SLICES = 8;
constexpr int DMV_SPLIT_CNT = 16384;   // tiles of a split launch (max)
inline size_t dpack_mv_split_floats(int rows) { return (size_t)DMV_SPLIT_CNT + (size_t)DMV_MAX_SLICES * rows; }
hipError_t launch_dpack_mv(const MvPhaseDesc& p, const float* x, const float* norm_w, float eps, float* y, int mode,
                           hipStream_t s, float* split = nullptr);
// The same matrices for T = 1..8 tokens (x[t] at x + t * xs, y[t] at y + t * ys): y = W x (+ bias),
// y += W x (accumulate), or for a gated phase y[o1] = SiLU(gate) * up; x := RMSNorm(x) * norm_w
// first when norm_w is given. Inputs too long for all T tokens' images in LDS run in input slices
// and need `split`: dpack_mm_split_floats(p) floats, zeroed once before the first use (tile
// counters that every launch leaves at zero); launches sharing it must not overlap.
size_t dpack_mm_split_floats(const MvPhaseDesc& p);
hipError_t launch_dpack_mm(const MvPhaseDesc& p, const float* x, int xs, const float* norm_w, float eps, float* y, int ys,
                           bool accumulate, int T, float* split, size_t split_floats, hipStream_t s);

struct LayerDev {
    MvPhaseDesc qkv, o, gu, down;
    const float* in_norm; const float* post_norm; const float* q_norm; const float* k_norm;
    uint16_t* kc; uint16_t* vc;
};

// Launch state of the persistent step: the launch count (the high part of every exchange tag) and
// the abort flag a stalled wait raises. Phases hand data over through tagged vectors (MegaArgs).
constexpr int MEGA_MAX_WG = 1024;
struct MegaSync {
    unsigned launch;      // launches completed
    unsigned abort;       // set when a wait for a tagged value expires
    unsigned pad0[30];
};

struct MegaArgs {
    const LayerDev* layers; int L;
    MvPhaseDesc head;
    const uint8_t* embed_w; const uint16_t* embed_s; const uint16_t* embed_b; int embed_gs;
    const float* final_norm; const float* inv_freq;
    int H, nH, nKV, I, rot_dim, traditional;
    float eps, scale;
    const int* pt;
    int* hist; int* status; int* dpos;
    float *logits, *part;             // attention partials: max [nH * nsplit], sum [..], acc [..][128]
    uint2* part_ready;                // per (KV head, range): tagged once the range's partials are stored
    // Tagged exchange vectors: element i is (value bits, tag) written by one 8-byte store; a reader
    // polls until the tag of the phase that produces it appears (no grid barrier between phases).
    // hA: h after down (and the embedding), hB: h after o_proj; q|k|v; attention output; SiLU(g)*u.
    uint2 *hA, *hB, *qkvT, *attnT, *mlpT;
    float* wg_best; int* wg_idx;
    unsigned* kv_done; unsigned* head_done;
    MegaSync* sync;
    int* abort_host;                  // host-mapped copy of sync->abort (read by the host after a step)
    int select;                       // 1: greedy token selection fused (writes hist / ring, advances *dpos)
    int kv_stage;                     // 1: a range's second chunk of keys is staged in LDS (cache byte offsets < 2^31)
    int desc_lds_off;                 // byte offset of the layers' descriptors in the workgroup's LDS
    int n_pages, pt_lds_off;          // page table entries, byte offset of their LDS copy
    int* ring_tok; int* ring_status; int ring_mask;
    unsigned long long* prof;         // optional: per workgroup, wall-clock at every phase start / end
    unsigned spin_limit;              // polls of a wait before it gives up (MEGA_SPIN_LIMIT)
    int stall;                        // test hook, 1: workgroup 0's first wait asks for a tag no launch writes
};
constexpr unsigned MEGA_SPIN_LIMIT = 1u << 20;
constexpr int MEGA_PROF_EVENTS = 1024;

size_t mega_lds_bytes(const MegaArgs& a, int max_keys_per_split);   // a.L, a.kv_stage and the shape set
size_t mega_desc_offset(const MegaArgs& a);
hipError_t launch_decode_step(const MegaArgs& a, int nwg, size_t lds, hipStream_t s);
hipError_t mega_set_lds_limit(size_t lds);
int mega_blocks_per_cu(const MegaArgs& a, size_t lds);   // resident workgroups per CU at this LDS size (0: error)
int mega_threads();
int mega_tiles_per_wg_cap();   // 16-row tiles of one phase one workgroup may own
int mega_wg_row_cap();     // rows of an accumulate phase one workgroup may own
int mega_split_cap();      // key ranges per KV head (workgroups / KV heads) the attention merge handles

}  // namespace mlxr
