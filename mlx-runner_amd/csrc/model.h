// Host runtime of the token loop: model configuration, MLX safetensors loading, device buffers and
// the step protocol of the reference's `Transformer` (Sources/MLXEngine/Transformer.swift).
#pragma once
#include <hip/hip_runtime.h>
#include <map>
#include <string>
#include <tuple>
#include <vector>
#include "kernels.h"
#include "decode.h"
#include "../../include/mlxr.h"

namespace mlxr {

int set_error(int code, const std::string& msg);
const char* last_error();

// ModelConfig subset for the qwen3 / qwen2 / llama / mistral families (ModelConfig.swift:149-307).
struct Config {
    std::string model_type;
    std::vector<int> eos;          // end-of-sequence ids (config.json + generation_config.json)
    int H = 0, L = 0, nH = 0, nKV = 0, D = 0, I = 0, V = 0, max_pos = 4096;
    float eps = 1e-6f;
    double theta = 10000;
    bool traditional = false, tie = false;
    int rot_dim = 0;
    float query_scale = 1.0f, rope_attention_factor = 1.0f;
    std::vector<float> inv_freq;
    int bits = 0, gs = 0;
};
int parse_config(const std::string& dir, Config& c);

struct Lin {
    QMat m;
    int K = 0, O = 0, bits = 0, gs = 0, st = 0;
    std::string desc;
};

struct Layer {
    Lin q, k, v, o, gate, up, down;
    float* in_norm = nullptr; float* post_norm = nullptr;
    float* q_norm = nullptr; float* k_norm = nullptr;
    uint16_t* kc = nullptr; uint16_t* vc = nullptr;   // [n_pages][nKV][PAGE][D] bf16
    uint16_t* idx = nullptr;                          // sparse index [max_seq/4][nKV][D] bf16
};

struct Model {
    Config cfg;
    int max_seq = 0, n_pages = 0;
    Lin embed, head;
    bool tied = false;
    float* final_norm = nullptr;
    float* inv_freq = nullptr;
    std::vector<Layer> layers;
    std::string quant_desc;
    int64_t weight_bytes = 0, device_bytes = 0;

    // device memory
    std::vector<void*> allocs;
    uint8_t* arena = nullptr;
    int* page_table = nullptr;
    int* hist = nullptr; int* status = nullptr; uint64_t* rng = nullptr;
    int* dpos = nullptr;                 // position of the step being processed (device)
    float *h = nullptr, *xn = nullptr, *tmp = nullptr, *qkv = nullptr, *attn = nullptr, *gu = nullptr, *mlp = nullptr;
    float* mm_split = nullptr;       // input-slice scratch of the verify batch's small-batch matvec (dpack_mm_split_floats)
    size_t mm_split_floats = 0;
    float* dmv_split = nullptr;      // [2][H] input-slice partials of the kernel-per-op down matvec (long inputs)
    float* logits = nullptr; float* part = nullptr; float* bmax = nullptr; int* barg = nullptr;
    float* qsplit = nullptr;            // the other widths' prefill GEMM split over K (QGEMM_SPLIT_FLOATS, counters at zero)
    uint16_t* xbf = nullptr; float* xsc = nullptr;
    uint16_t* xlo = nullptr; float* xgs = nullptr; int* xnz = nullptr;   // the MLX-layout GEMM's x lo part, group sums, lo flags
    uint16_t* wsb = nullptr;          // the MLX-layout GEMM's repacked scales
    int* diag = nullptr;
    // sparse
    bool sparse_alloc = false; bool sparse_on = false;
    std::string sparse_off;          // why a model opened with sparse attention decodes densely
    mlxr_sparse_cfg sparse{};
    float* sp_scores = nullptr; int* sp_lists = nullptr; int* sp_plan = nullptr; int sp_max_blocks = 0;
    // host staging
    int* h_tokens = nullptr;             // pinned [max_batch]
    int* h_pos = nullptr;                // pinned ring of position values
    int h_pos_i = 0;
    float* h_logits = nullptr;           // pinned [8][V]
    int* ring_tok = nullptr; int* ring_status = nullptr;   // host-mapped token ring
    int* ring_tok_dev = nullptr; int* ring_status_dev = nullptr;
    int* abort_host = nullptr; int* abort_host_dev = nullptr;   // host-mapped barrier-expiry flag
    static constexpr int RING = 64;

    hipStream_t stream = nullptr;
    int qkv_cols = 0, nsplit_dec = 32, nsplit_ver = 32;
    int max_batch = MLXR_PREFILL_CHUNK;                // prefill chunk (tokens per batched pass)
    int dev_pos_known = -1;              // value *dpos will hold once queued work completes
    int written_high = 0;
    bool use_graphs = true;
    // persistent decode step (decode.hip)
    bool mega_ok = false;            // the model fits the persistent kernel's constraints
    int decode_mode = 1;             // 1: persistent kernel when eligible, 0: kernel per op, 2: kernel per op on the MLX layout
    MegaArgs mega{};
    LayerDev* mega_layers = nullptr;
    std::vector<LayerDev> tile_layers;  // host copy of the repacked phases: the prefill GEMMs use them too
    MvPhaseDesc tile_head{};            // repacked lm_head (code == nullptr: none)
    int mega_nwg = 0; size_t mega_lds = 0;
    bool stall_next = false;         // test hook: the next persistent step's first wait expires
    std::string mega_reason;
    double last_gpu_time = 0;

    struct StepSlot { hipEvent_t start = nullptr, stop = nullptr; int offset = -1; bool busy = false, failed = false; };
    StepSlot slots[4];
    int next_slot = 0;

    struct GraphKey {
        int window, top_k, sparse; float penalty, temperature, top_p, min_p;
        bool operator<(const GraphKey& o) const {
            return std::tie(window, top_k, sparse, penalty, temperature, top_p, min_p) <
                   std::tie(o.window, o.top_k, o.sparse, o.penalty, o.temperature, o.top_p, o.min_p);
        }
    };
    std::map<GraphKey, hipGraphExec_t> graphs;
    std::vector<hipGraph_t> graph_defs;

    ~Model();
};

int model_open(const char* dir, int context_len, const mlxr_sparse_cfg* sparse, Model** out);
// The caller's isCancelled closure: polled between chunks.
struct Cancel {
    mlxr_cancel_fn fn; void* user;
    bool requested() const { return fn && fn(user) != 0; }
};
int model_forward(Model* m, const int32_t* tokens, int n, int offset, bool all_logits, bool dense, const float** out,
                  Cancel cancel = {});
int model_prefill(Model* m, const int32_t* tokens, int n, int offset, const mlxr_sample_params* sp, int32_t* tok,
                  Cancel cancel = {});
int model_step_logits(Model* m, const float** out);
int model_begin_decode(Model* m, int offset, const mlxr_sample_params* sp, mlxr_step* out);
int model_finish(Model* m, const mlxr_step* st, int32_t* tok);
int model_begin_steps(Model* m, const int32_t* tokens, int n, int offset, const mlxr_sample_params* sp, mlxr_step* out);
int model_reusable_prefix(Model* m, int common, int prev_len);
int model_stall_next_step(Model* m);
int model_seed(Model* m, uint64_t seed);
int model_set_sparse(Model* m, const mlxr_sparse_cfg* cfg);
int model_read_kv(Model* m, int layer, int rows, float* k, float* v);
void sparse_clamp(mlxr_sparse_cfg& c);
int model_set_decode_mode(Model* m, int mode);
int model_phase_times(Model* m, int offset, double* out, int max_intervals);
int model_profile(Model* m, const char* kind, int iters, int context, double* avg_ms, int64_t* bytes);

}  // namespace mlxr
