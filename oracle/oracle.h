/*
 * CPU oracle: a plain-C restatement of the reference's token-loop semantics.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load this library, and only as the checker (or as the timed CPU baseline). The product
 * (libmlxr) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths under the reference tree
 * BackendStack21/mlx-runner). Where each function's result is pinned (golden vectors, closed
 * forms, invariants) is listed in tests/test_oracle.py; functions with no such pin say
 * "parity unpinned" below.
 *
 * Precision contract (the build's declared precision, mirrored here):
 *   - activations fp32, accumulation in double (the reference tests' Float64 references);
 *   - K/V cache entries rounded to bf16 (round-to-nearest-even) when appended;
 *   - optionally (orc_forward's small_t, a diagnostic) the 4-bit tile GEMM's f16 operand rounding
 *     on chunks of more than small_t tokens; every other product is fp32-level (double here).
 */
#ifndef MLXR_ORACLE_H
#define MLXR_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define ORC_SMALL_T 8

/* ---- number formats ---- */
float orc_bf16_to_f32(uint16_t u);
uint16_t orc_f32_to_bf16(float f);          /* RNE, NaN kept quiet (ModelConfig.swift:483-490) */
float orc_f16_to_f32(uint16_t h);           /* GPU.swift:171-184 */
uint16_t orc_f32_to_f16(float f);           /* RNE */
float orc_round_bf16(float f);

/* ---- MLX affine code packing (KernelTests.swift:34-43, Kernels.swift:34-55, SieveImport.swift:90-111) ---- */
void orc_pack(const uint32_t* codes, int64_t n, int bits, uint8_t* out);      /* out: (n*bits+7)/8 bytes, zeroed by caller */
void orc_unpack(const uint8_t* packed, int64_t n, int bits, uint32_t* codes);

/* ---- a quantized linear layer on host memory (Transformer.swift:40-111) ----
 * w: packed codes [O][K*bits/8]; scales/biases [O][K/gs] as float values (already converted
 * from their storage dtype); bias: optional per-row bias [O] (Qwen2 q/k/v). */
typedef struct {
    const uint8_t* w; const float* scales; const float* biases; const float* bias;
    int O, K, bits, gs;
} orc_qlinear;

/* y[t][o] = sum_k (s*q+b) * x[t][k] (+ bias[o]); double accumulation, the reference test's
 * QuantFixture.reference (KernelTests.swift:102-113). x row stride K, y row stride O. */
void orc_qlinear_f64(const orc_qlinear* l, const float* x, int T, float* y);
/* The 4-bit tile GEMM's operand rounding (f16 x with a per-row power-of-two scale, f16(fma(s, q, b))
 * weights), double accumulation. */
void orc_qlinear_f16(const orc_qlinear* l, const float* x, int T, float* y);
/* The model prefill's precision: orc_qlinear_f16 where the tile GEMM runs (4-bit, gs 32/64/128, an
 * even number of groups per row), orc_qlinear_f64 otherwise. */
void orc_qlinear_prefill(const orc_qlinear* l, const float* x, int T, float* y);
double orc_round_f16_d(double v);
/* One row of dequantized weights (fp32 `s*q+b`, SieveImport.swift:108). */
void orc_dequant_row(const orc_qlinear* l, int row, float* out);

/* ---- norms / RoPE / activation ---- */
/* y = x * 1/sqrt(mean(x^2)+eps) * w, per row of `dim` (Kernels.swift:1037-1070). */
void orc_rms_norm(const float* x, float* y, const float* w, int dim, int rows, float eps);
/* inverse RoPE frequencies, computed in double then cast (ModelConfig.swift:438-466; plain theta). */
void orc_inv_freq(double theta, int rot_dim, float* out);
/* in-place RoPE of one head, half-split (traditional=0) or interleaved (Kernels.swift:1124-1134). */
void orc_rope(float* v, int D, int rot_dim, int traditional, int pos, const float* inv_freq);
float orc_silu_mul(float g, float u);   /* Kernels.swift:126-130 */

/* ---- attention ----
 * q: [nH][D] one query row (already RoPE'd); caches: [nKV][max_seq][D] fp32 values of the
 * stored (bf16) entries. Attention of query position `pos` over keys 0..pos (softmax with a
 * max shift), the reference test's `reference` (KernelTests.swift:461-486). */
void orc_attention(const float* q, const float* kc, const float* vc, int D, int nH, int nKV, int max_seq,
                   int pos, float scale, float* out);
/* Over an explicit per-KV-head list of positions (SparseAttentionTests.swift:250-270).
 * lists: nKV lists of `count` entries, `list_stride` apart (0: one shared list). Entries are
 * clamped to [0, L-1] with L = pos + 1 (Kernels.swift:1745). */
void orc_attention_list(const float* q, const float* kc, const float* vc, int D, int nH, int nKV, int max_seq,
                        int pos, float scale, const int32_t* lists, int count, int list_stride, float* out);

/* ---- sparse decode attention (SparseAttention.swift:80-94, Kernels.swift:1541-1710) ---- */
typedef struct { int pool, b0, nb, p, sink_end, win_start, L, count; } orc_sparse_plan;
/* returns 1 with a plan, 0 when the step stays dense. */
int orc_sparse_make_plan(int top_k, int window, int sink, int min_context, int position, orc_sparse_plan* out);
/* normalise a budget as SparseAttention.init does (SparseAttention.swift:47-54). */
void orc_sparse_clamp(int* top_k, int* window, int* sink, int* min_context, int has_min_context);
/* idx[b][kvh][d] = mean of the block's pool keys (fp32 values of stored keys), result rounded to bf16. */
void orc_sparse_index(const float* kc, int nKV, int D, int max_seq, int pool, int b0, int nb, float* idx);
/* scores: per KV head (rows = nKV) or shared (rows = 1) (Kernels.swift:1565-1612). */
void orc_sparse_score(const float* q, const float* idx, int nH, int nKV, int D, int b0, int nb, int rows, float* scores);
uint32_t orc_sparse_key(float f);   /* Kernels.swift:1615-1618 */
/* exact top-p by key, ties to the earlier block, list in ascending position (Kernels.swift:1628-1710). */
void orc_sparse_select(const float* scores, int nb, const orc_sparse_plan* plan, int32_t* list);

/* ---- token selection ---- */
/* argmax, lowest index on ties; -1 if the maximum is not finite (Engine.swift:119-124, Kernels.swift:2343-2356). */
int orc_argmax(const float* logits, int V);
/* The CPU sampler's distribution (Engine.swift:112-160): in place penalty over `recent`
 * (n_recent entries), temperature, top-k, min-p, top-p. Writes up to max_out (id, p) pairs,
 * descending; returns the count, or -1 for non-finite logits. */
int orc_sample_distribution(float* logits, int V, const int32_t* recent, int n_recent, float temperature,
                            int top_k, float top_p, float min_p, float penalty, int32_t* ids, float* probs, int max_out);

/* ---- whole model (Transformer.swift:1323-1584, qwen3 / qwen2 / llama) ---- */
typedef struct orc_model orc_model;
/* Loads config.json + *.safetensors from dir with the oracle's own reader. NULL on error
 * (message via orc_last_error). */
orc_model* orc_model_load(const char* dir, int max_seq);
void orc_model_free(orc_model* m);
const char* orc_last_error(void);
int orc_model_vocab(const orc_model* m);
int orc_model_hidden(const orc_model* m);
/* Runs tokens at positions offset..offset+n-1 (KV appended), writes the last row's logits
 * (V floats) when logits != NULL. `small_t` (a diagnostic) mirrors the model prefill's kernel
 * choice: projections over more than small_t tokens use orc_qlinear_prefill. Returns 0 on success. */
int orc_forward(orc_model* m, const int32_t* tokens, int n, int offset, int small_t, float* logits);
/* Sparse decode attention for single-token steps (0/NULL: dense). */
void orc_model_set_sparse(orc_model* m, int enabled, int top_k, int window, int sink, int min_context, int per_head);
/* Host copies of the KV cache (fp32 values of the bf16 entries), layer-major
 * [layer][nKV][max_seq][D]; for loading a cache produced elsewhere. */
int orc_model_set_kv(orc_model* m, int layer, const float* k, const float* v, int rows);
int orc_model_threads(void);

#ifdef __cplusplus
}
#endif
#endif
