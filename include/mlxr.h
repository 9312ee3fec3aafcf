/*
 * mlxr.h — C ABI of libmlxr, the MI355X (gfx950) token loop.
 *
 * The reference (BackendStack21/mlx-runner) has no FFI layer: its engine boundary is the Swift
 * `Transformer` class (Sources/MLXEngine/Transformer.swift:642-1303), used by `InferenceEngine`
 * (Engine.swift:318-345, 549-813). Each model entry point below replaces one member of that
 * class (cited per function); a Swift shim binding these symbols is shown in INTEGRATION.md.
 *
 * Conventions: every function returns 0 (MLXR_OK) or a negative MLXR_E_* code; the message of the
 * last failure on the calling thread is mlxr_last_error(). Not thread-safe per model (the
 * reference serialises every call on one queue, Engine.swift:241). Token arrays belong to the
 * caller and are copied before the call returns. Pointers returned by the model stay valid until
 * the next call on it.
 *
 * The kernel-level entry points (mlxr_k_*) take DEVICE pointers (mlxr_dev_alloc) and run on the
 * library's stream; they mirror the reference's kernels by host name and exist for parity tests
 * and micro-benchmarks.
 */
#ifndef MLXR_H
#define MLXR_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* EngineError cases (GPU.swift:4-33) as status codes. */
enum {
    MLXR_OK = 0,
    MLXR_E_NO_DEVICE = -1,       /* noMetalDevice */
    MLXR_E_INVALID_FILE = -2,    /* invalidFile */
    MLXR_E_MISSING_TENSOR = -3,  /* missingTensor */
    MLXR_E_UNSUPPORTED = -4,     /* unsupported */
    MLXR_E_CONTEXT_FULL = -5,    /* contextFull */
    MLXR_E_OUT_OF_MEMORY = -6,   /* outOfMemory */
    MLXR_E_CANCELLED = -7,       /* cancelled */
    MLXR_E_INVALID_OUTPUT = -8,  /* invalidOutput */
    MLXR_E_GPU = -9,             /* gpuFailure */
    MLXR_E_INVALID_ARG = -10     /* caller error (bad pointer / size) */
};

typedef struct mlxr_model mlxr_model;

/* SparseAttention (SparseAttention.swift:29-54): budget of the sparse decode attention. */
typedef struct {
    int32_t top_k;        /* long-range keys kept per step (whole blocks of 4) */
    int32_t window;       /* most recent keys always attended */
    int32_t sink;         /* first keys always attended */
    int32_t min_context;  /* sparse from this context length (position + 1); <= 0: 2*(sink+top_k+window) */
    int32_t per_head;     /* 1: one selection per KV head (default); 0: one shared selection */
} mlxr_sparse_cfg;

/* SampleParams (GPU.swift:56-66), byte-compatible field order. V and pos are filled by the model. */
typedef struct {
    int32_t V, pos, window, top_k;
    float penalty, temperature, top_p, min_p;
} mlxr_sample_params;

/* A committed decode step (Transformer.DecodeStep, Transformer.swift:1267-1272). */
typedef struct {
    int64_t id;        /* internal slot */
    int32_t offset;    /* position of the token the step processed; its token lands at offset + 1 */
} mlxr_step;

/* ---------------------------------------------------------------- model lifecycle */
/* Transformer.init(directory:contextLength:sparse:sieve:) (Transformer.swift:854-1109).
 * sparse == NULL loads without the sparse index (dense decode). */
int mlxr_model_open(const char* dir, int context_len, const mlxr_sparse_cfg* sparse, mlxr_model** out);
void mlxr_model_close(mlxr_model* m);

/* Info getters (Transformer.swift:792-800, 875; Engine.swift:852-873 memoryNeed). */
int mlxr_vocab_size(const mlxr_model* m);
int mlxr_max_seq(const mlxr_model* m);
int mlxr_hidden_size(const mlxr_model* m);
int mlxr_num_layers(const mlxr_model* m);
int64_t mlxr_weight_bytes(const mlxr_model* m);
int64_t mlxr_device_bytes(const mlxr_model* m);
const char* mlxr_quant_description(const mlxr_model* m);   /* e.g. "q4g64" (Linear.description) */
int mlxr_sparse_available(const mlxr_model* m);            /* Transformer.sparseAvailable (:815) */
/* Transformer.sparseLayerCount (:818): layers that decode sparse (every layer when available). */
int mlxr_sparse_layer_count(const mlxr_model* m);
/* Transformer.sparseOffReason (:821, set at :1029-1031): why a model opened with sparse attention
 * decodes densely ("" otherwise); valid until the model closes. */
const char* mlxr_sparse_off_reason(const mlxr_model* m);
int mlxr_written_high(const mlxr_model* m);                /* Transformer.writtenHigh (:665) */
/* config.modelType (ModelConfig.swift:39, lower-cased); valid until the model closes. */
const char* mlxr_model_type(const mlxr_model* m);
/* config.eosTokenIds (ModelConfig.swift:284-291: config.json and generation_config.json, each a
 * number or a list, deduplicated; ascending here): copies up to cap ids to out, returns how many
 * there are. */
int mlxr_eos_token_ids(const mlxr_model* m, int32_t* out, int cap);
/* config.isHybrid (ModelConfig.swift:125): always 0, no linear-attention architecture loads. */
int mlxr_is_hybrid(const mlxr_model* m);
/* supportsBatchedVerify (Transformer.swift:842-847): 1 when a forward of 2..8 tokens with all
 * logits runs the batched verify pass (every projection of every loadable model does). */
int mlxr_supports_batched_verify(const mlxr_model* m);

/* ---------------------------------------------------------------- the step API */
/* The isCancelled closure of forward / prefill (Transformer.swift:1118,1224): called with `user`
 * between chunks (never before the first); nonzero stops the call with MLXR_E_CANCELLED. The rows
 * of the chunks already run stay in the KV cache, as in the reference. NULL: never cancelled. */
typedef int (*mlxr_cancel_fn)(void* user);
/* forward(_:offset:allLogits:dense:isCancelled:) (Transformer.swift:1117-1136): runs tokens at
 * offset..offset+n-1 in chunks of MLXR_PREFILL_CHUNK; *logits_out = last row's logits (V floats)
 * or, with all_logits (n <= 8), [n][V]. Owned by the model, valid until the next call. Like the
 * reference's forward it selects no token: the history past offset + n - 1 is left as it was. */
int mlxr_forward(mlxr_model* m, const int32_t* tokens, int n, int offset, int all_logits, int dense,
                 const float** logits_out, mlxr_cancel_fn is_cancelled, void* user);
/* prefill(_:offset:sample:isCancelled:) (Transformer.swift:1224-1249): token selected on the GPU
 * from the last row, stored at position offset + n. */
int mlxr_prefill(mlxr_model* m, const int32_t* tokens, int n, int offset, const mlxr_sample_params* sp,
                 int32_t* token_out, mlxr_cancel_fn is_cancelled, void* user);
/* Tokens per batched pass of forward / prefill: the reference's maxBatch is 512
 * (ModelConfig.swift); here 2048, so a cancel request is seen after at most one 2048-token chunk
 * (about 40 ms of an 8B prefill on one MI355X). */
#define MLXR_PREFILL_CHUNK 2048
/* Logits of the last decode step (V floats, the row its token was selected from), after its
 * finish and with no step in flight. Owned by the model, valid until the next call. No
 * counterpart in the reference, whose logits buffer the caller reads directly (Transformer.logits). */
int mlxr_step_logits(mlxr_model* m, const float** logits_out);
/* beginDecodeStep(offset:sample:) (Transformer.swift:1255-1264): commits the step for the token at
 * position offset (written by the previous step's sampler or by prefill) without waiting. Steps
 * must be begun and finished in position order, at most two in flight. */
int mlxr_begin_decode(mlxr_model* m, int offset, const mlxr_sample_params* sp, mlxr_step* out);
/* beginSteps(_:offset:sample:) (Transformer.swift:1265-1296): writes tokens to positions
 * offset..offset+n-1 and commits one step over them whose token (selected on the GPU from the
 * last row) lands at offset + n, without waiting. Nothing may be in flight; the returned step
 * (offset = offset + n - 1) counts as one for the in-flight limit and is finished with
 * mlxr_finish. Draft models use it to catch up on the tokens the target accepted. */
int mlxr_begin_steps(mlxr_model* m, const int32_t* tokens, int n, int offset, const mlxr_sample_params* sp, mlxr_step* out);
/* finish(_:) (Transformer.swift:1298-1303): waits and returns the token at offset + 1. */
int mlxr_finish(mlxr_model* m, const mlxr_step* step, int32_t* token_out);
/* reusablePrefix(_:previousLength:) (Transformer.swift:1193-1209). */
int mlxr_reusable_prefix(mlxr_model* m, int common, int previous_length);
/* resetWriteTracking() (Transformer.swift:1213). */
void mlxr_reset_write_tracking(mlxr_model* m);
/* seedSampler(_:) (Transformer.swift:1216-1219): seed 0 -> 0x9E3779B97F4A7C15. */
int mlxr_seed_sampler(mlxr_model* m, uint64_t seed);
/* `sparse` property (Transformer.swift:813): NULL turns sparse decode off. Takes effect only for
 * a model opened with sparse attention. */
int mlxr_set_sparse(mlxr_model* m, const mlxr_sparse_cfg* cfg);
/* lastGPUTime (Transformer.swift:788): seconds of the last completed step. */
double mlxr_last_gpu_time(const mlxr_model* m);
/* Host copies of one layer's KV cache, positions [0, rows): k/v as fp32 [nKV][rows][D]. */
int mlxr_read_kv(mlxr_model* m, int layer, int rows, float* k_out, float* v_out);
/* Times one decode kernel class on the model's weights (kind: "qkv", "o", "gateup", "down", "head",
 * "attn" at `context` keys; "step": the persistent whole-token decode kernel, greedy steps from
 * position context - 1, which overwrite the history after it): `iters` launches cycling through
 * the layers, HIP events around them on the model's stream. avg_ms: mean launch duration; bytes:
 * algorithmic bytes per launch. Profiling hook in the spirit of Transformer.profile()
 * (Transformer.swift:1696-1798). */
int mlxr_profile_kernel(mlxr_model* m, const char* kind, int iters, int context, double* avg_ms, int64_t* bytes);
/* Decode step implementation: 1 (default) = the persistent kernel (one launch per token, tagged
 * hand-over between phases) where the model allows it, 0 = one kernel per operation (projections
 * over the repacked weight tiles where the model has them), 2 = one kernel per operation on the
 * MLX weight layout. Fails while a step is in flight. */
int mlxr_set_decode_mode(mlxr_model* m, int mode);
/* Runs one persistent greedy decode step at `offset` with wall-clock marks at every phase boundary:
 * out[3e..3e+2] = mean start, mean end, latest end (us) of interval e over the workgroups
 * (intervals alternate phase work / barrier wait). Returns the interval count or an error.
 * max_intervals < 0: raw marks instead, out[w * 1024 + e] = time (us) of mark e of workgroup w
 * (-1 where unset; marks 512 + 8 * layer + k are sub-phase points), out sized for every
 * workgroup; returns the workgroup count. */
int mlxr_profile_decode_phases(mlxr_model* m, int offset, double* out, int max_intervals);
/* Test hook of the persistent step's failure path: the next persistent decode step's first input
 * wait (workgroup 0) asks for a tag no launch writes, with a short bound, so the wait expires, the
 * abort flag propagates and every wave still ends normally. That step's finish, and that of any
 * step queued behind it, return MLXR_E_GPU; the model falls back to the kernel-per-op step. No
 * counterpart in the reference. */
int mlxr_debug_stall_next_step(mlxr_model* m);
/* 1 when begin_decode runs the persistent kernel for dense steps. */
int mlxr_decode_mode(const mlxr_model* m);
/* Why dense steps do not run the persistent kernel ("" when they do); valid until the model closes. */
const char* mlxr_decode_mode_reason(const mlxr_model* m);
/* Decode steps with the whole step captured as a hipGraph (1, default) or launched kernel by kernel (0). */
int mlxr_set_graphs(mlxr_model* m, int enabled);

/* ---------------------------------------------------------------- synthetic models */
/* Writes an MLX-format model directory (config.json + model.safetensors) whose fp32 weights are
 * drawn N(0, std) from a seeded generator and affine-quantized (bits, group_size) with bf16
 * scale/bias; norm weights are 1. `config_json` is a Hugging Face config.json text plus
 * "quantization": {"bits", "group_size"}. Deterministic in (config, seed). */
int mlxr_synth_write(const char* config_json, uint64_t seed, float std, const char* dir);
/* Quantizes one row of fp32 weights exactly as mlxr_synth_write does (MLX affine: per group
 * scale = (max-min)/(2^bits-1), bias = min, both rounded to bf16; codes packed little-endian). */
int mlxr_quantize_row(const float* w, int K, int bits, int group_size, uint8_t* codes, uint16_t* scales_bf16,
                      uint16_t* biases_bf16);
/* One seeded synthetic matrix [O][K], drawn and quantized exactly as mlxr_synth_write draws tensor
 * number `tensor_id`: codes [O][K*bits/8], bf16 scales / biases [O][K/group_size] (host buffers).
 * Test and benchmark fixtures at real model shapes; no counterpart in the reference. */
int mlxr_synth_matrix(uint64_t seed, uint64_t tensor_id, int O, int K, int bits, int group_size, float std,
                      uint8_t* codes, uint16_t* scales_bf16, uint16_t* biases_bf16);

/* ---------------------------------------------------------------- device helpers */
int mlxr_device_count(void);
const char* mlxr_device_name(void);
int mlxr_dev_alloc(void** ptr, size_t bytes);
int mlxr_dev_free(void* ptr);
int mlxr_memcpy_h2d(void* dst, const void* src, size_t bytes);
int mlxr_memcpy_d2h(void* dst, const void* src, size_t bytes);
int mlxr_memset(void* dst, int value, size_t bytes);
int mlxr_synchronize(void);
const char* mlxr_last_error(void);
/* Timing of kernel-level calls: events recorded on the library stream (milliseconds). */
int mlxr_timer_start(void);
int mlxr_timer_stop(float* ms);

/* ---------------------------------------------------------------- kernels (device pointers) */
/* One quantized matrix: codes [O][K*bits/8], scales/biases [O][K/gs] (bf16: st 0, f16: st 1),
 * optional per-row bias [O] of the scales' dtype. */
typedef struct {
    const void* w; const void* scales; const void* biases; const void* bias;
    int32_t O;
} mlxr_qmat;

/* Fused decode matvec over up to three matrices [A|B|C] sharing K and quantization
 * (`qmv`, Kernels.swift:204-318). norm_w (fp32 [K], optional): x is first RMS-normalised and
 * scaled (the residual stream's norm, add_rms_norm Kernels.swift:1141-1175, fused).
 * epi: 0 store, 1 accumulate (y += Wx), 2 gated: parts A, B -> y[o] = silu(A x)[o] * (B x)[o]
 * (`qmv` MODE / silu_mul Kernels.swift:2004-2013). */
int mlxr_k_qmv(const mlxr_qmat* parts, int nparts, int K, int bits, int gs, int st, const float* x,
               const float* norm_w, float eps, float* y, int epi);
/* Small batch, T in 1..8 (`qmm` / `qmvx4`, Kernels.swift:60-113, 518-622). */
int mlxr_k_qmm(const mlxr_qmat* parts, int nparts, int K, int bits, int gs, int st, int T, const float* x,
               int x_stride, float* y, int y_stride);
/* Prefill GEMM on bf16 MFMA (`qgemm`, Kernels.swift:785-851), any T >= 1. */
int mlxr_k_qgemm(const mlxr_qmat* mat, int K, int bits, int gs, int st, int T, const float* x, int x_stride,
                 float* y, int y_stride);
/* The prefill GEMM over the repacked decode tiles that model prefill uses for 4-bit bf16-scale
 * models (`qgemm`, Kernels.swift:785-851): parts [A|B|C] as in mlxr_k_qmv, bits 4, bf16 scales,
 * gs 32/64, K % 128 == 0; gated (two parts of equal O): y[t][o] = silu(A x_t)[o] * (B x_t)[o]
 * (the MLP's gate|up, silu_mul Kernels.swift:2004-2013). Repacks into a temporary buffer per call. */
int mlxr_k_qgemm_tiles(const mlxr_qmat* parts, int nparts, int K, int gs, int gated, int T, const float* x,
                       int x_stride, float* y, int y_stride);
/* Batch-1 matvec over the repacked tiles, the kernel-per-op decode step's projection (`qmv` with
 * its fused epilogues, Kernels.swift:60-113, 1037-1070, 2004-2013): mode 0 y = W x (+ bias),
 * 1 y += W x (+ bias), 2 (two parts of equal O) y[o] = silu(A x)[o] * (B x)[o]; norm_w (or NULL)
 * first replaces x by RMSNorm(x) * norm_w (eps). Same quantization limits as mlxr_k_qgemm_tiles,
 * K <= 32768. `reps` launches back to back (timing; mode 1 then adds reps times). */
int mlxr_k_qmv_tiles(const mlxr_qmat* parts, int nparts, int K, int gs, int mode, const float* x, const float* norm_w,
                     float eps, float* y, int reps);
/* The small-batch form over the same tiles (the verify batch's projections, `qmm` / `qmvx4`,
 * Kernels.swift:60-113, 518-622): T = 1..8 tokens (x[t] at x + t * x_stride, y[t] at
 * y + t * y_stride), mode 0 y[t] = W x[t] (+ bias), 1 y[t] += W x[t] (+ bias), 2 (two parts of
 * equal O) y[t][o] = silu(A x_t)[o] * (B x_t)[o]; norm_w (or NULL) first replaces each x[t] by
 * RMSNorm(x[t]) * norm_w (eps). x and norm_w 16-byte aligned, x_stride a multiple of 4. Same
 * quantization limits as mlxr_k_qmv_tiles. */
int mlxr_k_qmm_tiles(const mlxr_qmat* parts, int nparts, int K, int gs, int mode, int T, const float* x, int x_stride,
                     const float* norm_w, float eps, float* y, int y_stride);
/* Quantized embedding rows (`qembed`, Kernels.swift:1002-1023): ids device int32 [T]. */
int mlxr_k_qembed(const mlxr_qmat* mat, int K, int bits, int gs, int st, const int32_t* ids, int T, float* out);
/* RMSNorm rows (`rms_norm`, Kernels.swift:1037-1070), fp32 weights; add_rms_norm with r != NULL. */
int mlxr_k_rms_norm(float* x_or_h, const float* r, float* y, const float* w, int dim, int rows, float eps);
/* `qkv_post` (Kernels.swift:1081-1138): per-head q/k RMSNorm (qn/kn fp32 [D] or NULL), RoPE
 * (half-split or traditional), K/V appended to the bf16 cache [nKV][max_seq][D] at positions
 * offset..offset+T-1. */
int mlxr_k_qkv_post(float* qkv, int row_stride, const float* inv_freq, void* kcache, void* vcache, int max_seq,
                    const float* qn, const float* kn, int D, int nH, int nKV, int rot_dim, int traditional,
                    int offset, int T, float eps);
/* Decode attention (`attention_split` + `attention_combine`, Kernels.swift:1317-1374) for T query
 * rows at positions offset+t over the bf16 cache [nKV][max_seq][D]; lists (device int32, per KV
 * head list_stride apart, or NULL) restrict the keys to `count` listed positions
 * (`attention_sparse`, Kernels.swift:1716-1756). */
int mlxr_k_attention(const float* q, int q_stride, const void* kcache, const void* vcache, int max_seq, int D,
                     int nH, int nKV, int offset, int T, float scale, float* out, int out_stride,
                     const int32_t* lists, int count, int list_stride, int nsplit);
/* Causal prefill attention (`flash_prefill`, Kernels.swift:1839-2000). */
int mlxr_k_flash_prefill(const float* q, int q_stride, const void* kcache, const void* vcache, int max_seq, int D,
                         int nH, int nKV, int offset, int T, float scale, float* out, int out_stride);
/* `sparse_index` (Kernels.swift:1545-1555): blocks completed by positions offset..offset+T-1. */
int mlxr_k_sparse_index(const void* kcache, int max_seq, int nKV, int D, int offset, int T, void* idx);
/* `sparse_score` (Kernels.swift:1565-1612): rows = nKV (per head) or 1 (shared). */
int mlxr_k_sparse_score(const float* q, const void* idx, int nH, int nKV, int D, int b0, int nb, int rows,
                        float* scores);
/* `sparse_select` (Kernels.swift:1628-1710): rows lists of sink_end + p*4 + (L - win_start). */
int mlxr_k_sparse_select(const float* scores, int rows, int b0, int nb, int p, int sink_end, int win_start, int L,
                         int32_t* lists, int list_stride);
/* `sample_blocks` + `sample_token` (Kernels.swift:2362-2619): logits device fp32 [V] (penalised in
 * place), hist device int32 (reads [pos-window+1, pos], writes [pos+1]), status int32 [pos+1],
 * rng device u64[2]. */
int mlxr_k_sample(float* logits, int V, int32_t* hist, int32_t* status, uint64_t* rng, int pos,
                  const mlxr_sample_params* sp);
/* mlxr_k_sample without any allocation: no counterpart in the reference. For callers that cannot
 * allocate device memory (code under stream capture, tight serving loops, harnesses that forbid
 * hipMalloc). The per-block partials and the position word live in a fixed 8.25 KiB device array
 * of the library (one copy per GPU, held until the process ends) instead of library-allocated
 * buffers; V <= 262144 (larger: MLXR_E_INVALID_ARG, nothing launched). Kernels go on `stream`
 * (a hipStream_t; NULL: the null stream) and the call returns without waiting. Every call on one GPU
 * shares its array: calls that overlap on one GPU race. Same results as mlxr_k_sample. */
int mlxr_k_sample_noalloc(float* logits, int V, int32_t* hist, int32_t* status, uint64_t* rng, int pos,
                          const mlxr_sample_params* sp, void* stream);

#ifdef __cplusplus
}
#endif
#endif
