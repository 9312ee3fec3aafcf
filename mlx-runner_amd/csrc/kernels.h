// Host-side launchers of the gfx950 kernels (defined in the .hip files of this directory).
// All launchers validate nothing: the callers in model.cpp / capi.cpp check shapes first.
#pragma once
#include "common.h"

namespace mlxr {

// One quantized matrix on the device, MLX affine layout:
// w: [O][K*bits/8] codes (little-endian bit stream per row); s, b: [O][K/gs] scale/bias (bf16 or f16).
struct QMat {
    const uint8_t* w = nullptr;
    const uint16_t* s = nullptr;
    const uint16_t* b = nullptr;
    const uint16_t* bias = nullptr;   // optional per-row bias, same dtype as s
    int O = 0;
};

// Epilogues of the decode matvec.
enum QmvEpi { EPI_STORE = 0, EPI_ADD = 1, EPI_GATED = 2 };

struct QmvArgs {
    QMat part[3];
    int nparts = 1;
    int K = 0, bits = 4, gs = 64, st = 0;   // st: 0 bf16 scales, 1 f16
    int O = 0;                            // total rows (EPI_GATED: number of outputs = rows of one part)
    const float* x = nullptr;             // input vector (K floats)
    const float* norm_w = nullptr;        // if set: x := rmsnorm(x) * norm_w computed per workgroup
    float eps = 1e-6f;
    float* y = nullptr;                   // output (EPI_ADD: y[o] += result)
    int epi = EPI_STORE;
};
hipError_t launch_qmv(const QmvArgs& a, hipStream_t s);

// Small batch (2..8 tokens): y[t][o] = W x[t] (+bias) at fp32-level precision.
struct QmmSmallArgs {
    QMat part[3];
    int nparts = 1;
    int K = 0, bits = 4, gs = 64, st = 0, O = 0, T = 1;
    const float* x = nullptr; int x_stride = 0;
    float* y = nullptr; int y_stride = 0;
    // optional pre-pass scratch (as QGemmArgs'): with it, the shapes qmmx_supported accepts (widths
    // 2 / 3 / 4 / 6 / 8) run on the matrix cores (launch_qmmx); without it, or for other shapes, on
    // the fp32 vector path
    uint16_t* xbf = nullptr; uint16_t* xlo = nullptr; float* xgs = nullptr; float* xsc = nullptr; int* xnz = nullptr;
};
hipError_t launch_qmm_small(const QmmSmallArgs& a, hipStream_t s);
bool qmmx_supported(int K, int bits, int gs);
hipError_t launch_qmmx(const QmmSmallArgs& a, hipStream_t s);

// Prefill GEMM over the MLX layout, any code width: Y[T][O] = X[T][K] W[O][K]^T (+bias) with exact
// codes on the f16 matrix cores, x as f16 hi + lo (per-row power-of-two scale) and the group scale
// and bias applied in fp32 per group: fp32-level results. Needs qgemm_supported(K, gs).
struct QGemmArgs {
    QMat m;
    int K = 0, bits = 4, gs = 64, st = 0, O = 0, T = 0;
    const float* x = nullptr; int x_stride = 0;
    float* y = nullptr; int y_stride = 0;
    // pre-pass scratch: hi and lo (T*K 16-bit each), group sums (qgemm_gsum_floats), the rows' inverse
    // scales (T floats), lo-nonzero flags (T ints) and the repacked scales and biases
    // (qgemm_scale_halves 16-bit words)
    uint16_t* xbf = nullptr; uint16_t* xlo = nullptr; float* xgs = nullptr; float* xsc = nullptr; int* xnz = nullptr;
    uint16_t* wsb = nullptr;
    bool x_ready = false;                 // the scratch already holds this x (same K and gs): skip the pre-pass
    // optional scratch for the split over K when the grid is under one round:
    // QGEMM_SPLIT_FLOATS floats, zero before first use (its tile counters return to zero)
    float* split = nullptr; size_t split_floats = 0;
};
// tile counters for up to 256 tiles, then at most 256 partial 128 x 256 tiles (slices x tiles stay
// within one workgroup per CU of a 256-CU device)
constexpr size_t QGEMM_SPLIT_TILES = 256;
constexpr size_t QGEMM_SPLIT_FLOATS = QGEMM_SPLIT_TILES + QGEMM_SPLIT_TILES * 128 * 256;
hipError_t launch_qgemm(const QGemmArgs& a, hipStream_t s);
size_t qgemm_gsum_floats(int T, int K, int gs);
bool qgemm_supported(int K, int gs);   // K % 64 == 0, gs 32 / 64 / 128
size_t qgemm_scale_halves(int O, int K, int gs);
// The 4-bit GEMM pre-pass: row t of x scaled by the power of two that puts max|x| in [2^13, 2^14),
// rounded to f16 (each 8-group stored as 0,4,1,5,2,6,3,7), inv[t] = the inverse scale.
// launch_x_to_f16's single-pass kernel (misc.hip) for K <= 32768; false (nothing launched) above.
bool launch_row_f16(const float* x, int xs, int K, int T, uint16_t* out, float* inv, hipStream_t s);
hipError_t launch_x_to_f16(const float* x, int xs, int K, int T, uint16_t* out, float* inv, hipStream_t s);

// Embedding: out[t][k] = dequant(row ids[t]) (ids read from hist + *dpos + t0).
hipError_t launch_qembed(const QMat& m, int K, int bits, int gs, int st, const int* hist, const int* dpos, int T,
                         float* out, hipStream_t s);

// RMSNorm rows (weights fp32): y = x * rsqrt(mean(x^2)+eps) * w.  add: h += r first (add_rms_norm).
hipError_t launch_rms_norm(const float* x, float* y, const float* w, int dim, int rows, int row_stride, float eps,
                           hipStream_t s);
hipError_t launch_add_rms_norm(float* h, const float* r, float* y, const float* w, int dim, int rows, float eps,
                               hipStream_t s);
// The same with the output in the 4-bit GEMM's f16 operand format (launch_x_to_f16's xh / inv).
hipError_t launch_rms_norm_f16(const float* x, const float* w, int dim, int rows, int row_stride, float eps, uint16_t* xh,
                               float* inv, hipStream_t s);
hipError_t launch_add_rms_norm_f16(float* h, const float* r, const float* w, int dim, int rows, float eps, uint16_t* xh,
                                   float* inv, hipStream_t s);

// Fused post-projection: per-head q/k RMSNorm, RoPE, q in place, K/V appended to the bf16 paged cache.
struct QkvPostArgs {
    float* qkv = nullptr; int row_stride = 0;
    const float* inv_freq = nullptr;
    uint16_t* kc = nullptr; uint16_t* vc = nullptr; const int* pt = nullptr;
    const float* qn = nullptr; const float* kn = nullptr;   // per-head norm weights (nullptr: none)
    const uint16_t* q_bias = nullptr;   // unused (bias folded into the projection)
    int D = 128, nH = 0, nKV = 0, rot_dim = 128, traditional = 0, T = 1;
    const int* dpos = nullptr; int pos_add = 0;
    float eps = 1e-6f;
    uint16_t* idx = nullptr;            // sparse block index: written for a block the step completes (T == 1)
};
hipError_t launch_qkv_post(const QkvPostArgs& a, hipStream_t s);

// Decode attention (one query token per step, positions from *dpos + t): split over the keys,
// then an ordered merge. lists: optional sparse position lists (per KV head, list_stride apart).
struct AttnArgs {
    const float* q = nullptr; int q_stride = 0;   // q rows: token t at q + t*q_stride, head h at +h*D
    const uint16_t* kc = nullptr; const uint16_t* vc = nullptr; const int* pt = nullptr;
    float* out = nullptr; int out_stride = 0;
    float* part = nullptr;                        // partials [T][nH][nsplit][D+2]
    int D = 128, nH = 0, nKV = 0, T = 1, nsplit = 32;
    const int* dpos = nullptr;
    float scale = 1.0f;
    const int* lists = nullptr; int list_stride = 0;
    const int* splan = nullptr;                   // sparse plan (device, written by launch_sparse_plan)
    int cap = 0;                                  // verify batch: keys per range (max), >= ceil((*dpos + T) / nsplit), <= 128
};
hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t s);
// Verify batch (T = 2..8, G T <= 64, dense keys): one workgroup per (KV head, key range) for all T
// queries, each masked at its own position; a.cap >= ceil((*dpos + T) / nsplit), at most 128.
hipError_t launch_attn_verify(const AttnArgs& a, hipStream_t s);

// Causal prefill attention (flash, bf16 MFMA for QK^T and PV) over the cache (queries at
// positions *dpos + t for t < T, keys 0..pos).
struct FlashArgs {
    const float* q = nullptr; int q_stride = 0;
    const uint16_t* kc = nullptr; const uint16_t* vc = nullptr; const int* pt = nullptr;
    float* out = nullptr; int out_stride = 0;
    int D = 128, nH = 0, nKV = 0, T = 0;
    const int* dpos = nullptr;
    float scale = 1.0f;
};
hipError_t launch_flash_prefill(const FlashArgs& a, hipStream_t s);

hipError_t launch_silu_mul(const float* gu, float* out, int I, int T, hipStream_t s);

// Sparse decode attention.
struct SparseArgs {
    const uint16_t* kc = nullptr; const int* pt = nullptr;
    uint16_t* idx = nullptr;            // [max_blocks][nKV][D] bf16
    const float* q = nullptr;           // decode query row (RoPE applied)
    float* scores = nullptr;            // [rows][nb]
    int* lists = nullptr; int list_stride = 0;
    int nKV = 0, nH = 0, D = 128, rows = 1;
    int top_k = 2048, window = 512, sink = 4, min_context = 1;
    const int* dpos = nullptr; int max_blocks = 0;
    int* dplan = nullptr;               // device plan scratch [8]
};
hipError_t launch_sparse_index(const uint16_t* kc, const int* pt, uint16_t* idx, int nKV, int D, const int* dpos,
                               int pos_add, int T, hipStream_t s);
hipError_t launch_sparse_plan(const SparseArgs& a, hipStream_t s);
hipError_t launch_sparse_score(const SparseArgs& a, hipStream_t s);
hipError_t launch_sparse_select(const SparseArgs& a, hipStream_t s);
// Host-side variant for tests: fixed plan values.
hipError_t launch_sparse_select_plan(const float* scores, int* lists, int list_stride, int rows, int b0, int nb, int p,
                                     int sink_end, int win_start, int L, hipStream_t s);
hipError_t launch_sparse_score_plan(const float* q, const uint16_t* idx, float* scores, int nH, int nKV, int D,
                                    int b0, int nb, int rows, hipStream_t s);

// Token selection: block maxima, then one workgroup (greedy argmax or top-k/top-p/min-p draw).
struct SampleArgs {
    float* logits = nullptr; int V = 0;
    int* hist = nullptr; int* status = nullptr;
    uint64_t* rng = nullptr;            // [0] xorshift64 state, [1] float pool-width hint
    float* bmax = nullptr; int* barg = nullptr;
    const int* dpos = nullptr;          // pos of the token whose logits these are; writes hist[pos+1]
    int* dpos_next = nullptr;           // if set: *dpos_next = pos + 1 after selection
    int window = 0, top_k = 0; float penalty = 1, temperature = 0, top_p = 1, min_p = 0;
    int* diag = nullptr;
    int* host_tok = nullptr; int* host_status = nullptr; int ring_mask = 0;   // host-mapped token ring
};
hipError_t launch_sample(const SampleArgs& a, hipStream_t s);

}  // namespace mlxr
