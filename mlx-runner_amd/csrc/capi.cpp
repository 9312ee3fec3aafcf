// extern "C" entry points of libmlxr (include/mlxr.h). Every kernel-level entry point checks its
// shapes on the host before anything is launched, so a bad call returns an error instead of
// reaching the GPU.
#include <cstring>
#include <mutex>
#include <string>
#include <vector>
#include "model.h"

namespace mlxr { int synth_write(const char* config_json, uint64_t seed, float std_, const char* dir); }

using namespace mlxr;

struct mlxr_model { Model* m; };

namespace {
std::mutex g_mu;
hipStream_t g_stream = nullptr;
int* g_pos = nullptr;          // device scalar for kernel-level calls
int* g_pt = nullptr;           // identity page table
int g_pt_pages = 0;
float* g_part = nullptr; size_t g_part_floats = 0;
float* g_qsplit = nullptr; size_t g_qsplit_floats = 0;   // the GEMM's split-over-K scratch (counters kept at zero)
float* g_split = nullptr; size_t g_split_floats = 0;   // the long-input split matvec's scratch
uint16_t* g_xbf = nullptr; size_t g_xbf_elems = 0;
float* g_xsc = nullptr; size_t g_xsc_elems = 0;
uint16_t* g_xlo = nullptr; size_t g_xlo_elems = 0;   // the MLX-layout GEMM's pre-pass: x lo part, group sums, lo flags
float* g_xgs = nullptr; size_t g_xgs_elems = 0;
int* g_xnz = nullptr; size_t g_xnz_elems = 0;
uint16_t* g_wsb = nullptr; size_t g_wsb_elems = 0;   // the MLX-layout GEMM's repacked scales
float* g_bmax = nullptr; int* g_barg = nullptr; int g_blocks = 0;
hipEvent_t g_t0 = nullptr, g_t1 = nullptr;

#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) return set_error(MLXR_E_GPU, std::string(#x) + ": " + hipGetErrorString(e_)); } while (0)

int ensure_stream() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return set_error(MLXR_E_NO_DEVICE, "no HIP GPU available");
    if (!g_stream) {
        CK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
        CK(hipMalloc(&g_pos, 256));
        CK(hipEventCreate(&g_t0)); CK(hipEventCreate(&g_t1));
    }
    return MLXR_OK;
}
int set_pos(int v) {
    CK(hipMemcpyAsync(g_pos, &v, 4, hipMemcpyHostToDevice, g_stream));
    CK(hipStreamSynchronize(g_stream));
    return MLXR_OK;
}
int ensure_pt(int max_seq) {
    const int pages = (max_seq + MLXR_PAGE - 1) / MLXR_PAGE;
    if (pages <= g_pt_pages) return MLXR_OK;
    if (g_pt) { hipStreamSynchronize(g_stream); hipFree(g_pt); }
    CK(hipMalloc(&g_pt, (size_t)pages * 4));
    std::vector<int> v(pages);
    for (int i = 0; i < pages; i++) v[i] = i;
    CK(hipMemcpy(g_pt, v.data(), (size_t)pages * 4, hipMemcpyHostToDevice));
    g_pt_pages = pages;
    return MLXR_OK;
}
template <typename T> int ensure_buf(T*& p, size_t& have, size_t need) {
    if (need <= have) return MLXR_OK;
    if (p) { hipStreamSynchronize(g_stream); hipFree(p); p = nullptr; }
    CK(hipMalloc(&p, need * sizeof(T)));
    have = need;
    return MLXR_OK;
}
bool bits_ok(int b) { return b == 2 || b == 3 || b == 4 || b == 5 || b == 6 || b == 8; }
int check_quant(int K, int bits, int gs, int st) {
    if (!bits_ok(bits)) return set_error(MLXR_E_UNSUPPORTED, "bits must be 2, 3, 4, 5, 6 or 8");
    if (gs <= 0 || gs % 32 || K <= 0 || K % gs || K % 64) return set_error(MLXR_E_UNSUPPORTED, "needs K % 64 == 0, group % 32 == 0, K % group == 0");
    if (st != 0 && st != 1) return set_error(MLXR_E_INVALID_ARG, "scale dtype must be 0 (bf16) or 1 (f16)");
    return MLXR_OK;
}
QMat qmat(const mlxr_qmat& q) {
    QMat m; m.w = (const uint8_t*)q.w; m.s = (const uint16_t*)q.scales; m.b = (const uint16_t*)q.biases;
    m.bias = (const uint16_t*)q.bias; m.O = q.O;
    return m;
}
int check_parts(const mlxr_qmat* parts, int n) {
    if (!parts || n < 1 || n > 3) return set_error(MLXR_E_INVALID_ARG, "1 to 3 matrices");
    for (int i = 0; i < n; i++) {
        if (!parts[i].w || !parts[i].scales || !parts[i].biases || parts[i].O <= 0) return set_error(MLXR_E_INVALID_ARG, "matrix pointers / rows");
        if ((parts[i].bias != nullptr) != (parts[0].bias != nullptr)) return set_error(MLXR_E_INVALID_ARG, "bias on every matrix or none");
    }
    return MLXR_OK;
}
int done(hipError_t e) {
    if (e != hipSuccess) return set_error(MLXR_E_GPU, hipGetErrorString(e));
    return MLXR_OK;
}
}  // namespace

extern "C" {

const char* mlxr_last_error(void) { return last_error(); }

int mlxr_model_open(const char* dir, int context_len, const mlxr_sparse_cfg* sparse, mlxr_model** out) {
    if (!dir || !out) return set_error(MLXR_E_INVALID_ARG, "null argument");
    *out = nullptr;
    Model* m = nullptr;
    if (int rc = model_open(dir, context_len, sparse, &m)) return rc;
    *out = new mlxr_model{m};
    return MLXR_OK;
}
void mlxr_model_close(mlxr_model* m) { if (m) { delete m->m; delete m; } }
int mlxr_vocab_size(const mlxr_model* m) { return m ? m->m->cfg.V : 0; }
int mlxr_max_seq(const mlxr_model* m) { return m ? m->m->max_seq : 0; }
int mlxr_hidden_size(const mlxr_model* m) { return m ? m->m->cfg.H : 0; }
int mlxr_num_layers(const mlxr_model* m) { return m ? m->m->cfg.L : 0; }
int64_t mlxr_weight_bytes(const mlxr_model* m) { return m ? m->m->weight_bytes : 0; }
int64_t mlxr_device_bytes(const mlxr_model* m) { return m ? m->m->device_bytes : 0; }
const char* mlxr_quant_description(const mlxr_model* m) { return m ? m->m->quant_desc.c_str() : ""; }
int mlxr_sparse_available(const mlxr_model* m) { return m && m->m->sparse_alloc ? 1 : 0; }
int mlxr_sparse_layer_count(const mlxr_model* m) { return m && m->m->sparse_alloc ? m->m->cfg.L : 0; }
const char* mlxr_sparse_off_reason(const mlxr_model* m) { return m ? m->m->sparse_off.c_str() : ""; }
int mlxr_written_high(const mlxr_model* m) { return m ? m->m->written_high : 0; }
const char* mlxr_model_type(const mlxr_model* m) { return m ? m->m->cfg.model_type.c_str() : ""; }
int mlxr_eos_token_ids(const mlxr_model* m, int32_t* out, int cap) {
    if (!m) return 0;
    const auto& e = m->m->cfg.eos;
    for (int i = 0; out && i < cap && i < (int)e.size(); i++) out[i] = e[i];
    return (int)e.size();
}
int mlxr_is_hybrid(const mlxr_model* m) { (void)m; return 0; }
int mlxr_supports_batched_verify(const mlxr_model* m) { return m ? 1 : 0; }

int mlxr_forward(mlxr_model* m, const int32_t* tokens, int n, int offset, int all_logits, int dense, const float** logits_out,
                 mlxr_cancel_fn is_cancelled, void* user) {
    if (!m || !logits_out) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return model_forward(m->m, tokens, n, offset, all_logits != 0, dense != 0, logits_out, Cancel{is_cancelled, user});
}
int mlxr_prefill(mlxr_model* m, const int32_t* tokens, int n, int offset, const mlxr_sample_params* sp, int32_t* token_out,
                 mlxr_cancel_fn is_cancelled, void* user) {
    if (!m || !token_out) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return model_prefill(m->m, tokens, n, offset, sp, token_out, Cancel{is_cancelled, user});
}
int mlxr_step_logits(mlxr_model* m, const float** logits_out) {
    if (!m || !logits_out) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return model_step_logits(m->m, logits_out);
}
int mlxr_begin_decode(mlxr_model* m, int offset, const mlxr_sample_params* sp, mlxr_step* out) {
    if (!m || !out) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return model_begin_decode(m->m, offset, sp, out);
}
int mlxr_begin_steps(mlxr_model* m, const int32_t* tokens, int n, int offset, const mlxr_sample_params* sp, mlxr_step* out) {
    if (!m || !out) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return model_begin_steps(m->m, tokens, n, offset, sp, out);
}
int mlxr_finish(mlxr_model* m, const mlxr_step* step, int32_t* token_out) {
    if (!m || !token_out) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return model_finish(m->m, step, token_out);
}
int mlxr_reusable_prefix(mlxr_model* m, int common, int previous_length) { return m ? model_reusable_prefix(m->m, common, previous_length) : 0; }
void mlxr_reset_write_tracking(mlxr_model* m) { if (m) m->m->written_high = 0; }
int mlxr_seed_sampler(mlxr_model* m, uint64_t seed) { return m ? model_seed(m->m, seed) : set_error(MLXR_E_INVALID_ARG, "null model"); }
int mlxr_set_sparse(mlxr_model* m, const mlxr_sparse_cfg* cfg) { return m ? model_set_sparse(m->m, cfg) : set_error(MLXR_E_INVALID_ARG, "null model"); }
double mlxr_last_gpu_time(const mlxr_model* m) { return m ? m->m->last_gpu_time : 0; }
int mlxr_read_kv(mlxr_model* m, int layer, int rows, float* k_out, float* v_out) {
    if (!m || !k_out || !v_out) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return model_read_kv(m->m, layer, rows, k_out, v_out);
}
int mlxr_profile_kernel(mlxr_model* m, const char* kind, int iters, int context, double* avg_ms, int64_t* bytes) {
    if (!m || !avg_ms || !bytes) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return model_profile(m->m, kind, iters, context, avg_ms, bytes);
}
int mlxr_set_decode_mode(mlxr_model* m, int mode) { return m ? model_set_decode_mode(m->m, mode) : set_error(MLXR_E_INVALID_ARG, "null model"); }
int mlxr_decode_mode(const mlxr_model* m) { return m && m->m->mega_ok && m->m->decode_mode == 1 ? 1 : 0; }
const char* mlxr_decode_mode_reason(const mlxr_model* m) {
    if (!m) return "null model";
    if (m->m->mega_ok && m->m->decode_mode == 1) return "";
    return m->m->mega_ok ? "decode mode set to the kernel-per-op step" : m->m->mega_reason.c_str();
}
int mlxr_profile_decode_phases(mlxr_model* m, int offset, double* out, int max_intervals) {
    if (!m || !out) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return model_phase_times(m->m, offset, out, max_intervals);
}
int mlxr_debug_stall_next_step(mlxr_model* m) { return m ? model_stall_next_step(m->m) : set_error(MLXR_E_INVALID_ARG, "null model"); }
int mlxr_set_graphs(mlxr_model* m, int enabled) { if (!m) return MLXR_E_INVALID_ARG; m->m->use_graphs = enabled != 0; return MLXR_OK; }

int mlxr_synth_write(const char* config_json, uint64_t seed, float std_, const char* dir) {
    if (!config_json || !dir) return set_error(MLXR_E_INVALID_ARG, "null argument");
    return synth_write(config_json, seed, std_, dir);
}

// ------------------------------------------------------------------------------ device helpers
int mlxr_device_count(void) { int n = 0; if (hipGetDeviceCount(&n) != hipSuccess) return 0; return n; }
const char* mlxr_device_name(void) {
    static std::string name;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) return "";
    name = p.gcnArchName;
    return name.c_str();
}
int mlxr_dev_alloc(void** ptr, size_t bytes) {
    if (!ptr) return MLXR_E_INVALID_ARG;
    if (int rc = ensure_stream()) return rc;
    hipError_t e = hipMalloc(ptr, bytes ? bytes : 16);
    return e == hipSuccess ? MLXR_OK : set_error(MLXR_E_OUT_OF_MEMORY, hipGetErrorString(e));
}
int mlxr_dev_free(void* ptr) { if (g_stream) hipStreamSynchronize(g_stream); return done(hipFree(ptr)); }
int mlxr_memcpy_h2d(void* dst, const void* src, size_t bytes) { if (g_stream) hipStreamSynchronize(g_stream); return done(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)); }
int mlxr_memcpy_d2h(void* dst, const void* src, size_t bytes) { if (g_stream) hipStreamSynchronize(g_stream); return done(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost)); }
int mlxr_memset(void* dst, int value, size_t bytes) { if (g_stream) hipStreamSynchronize(g_stream); return done(hipMemset(dst, value, bytes)); }
int mlxr_synchronize(void) {
    if (g_stream) { hipError_t e = hipStreamSynchronize(g_stream); if (e != hipSuccess) return set_error(MLXR_E_GPU, hipGetErrorString(e)); }
    return done(hipDeviceSynchronize());
}
int mlxr_timer_start(void) { if (int rc = ensure_stream()) return rc; return done(hipEventRecord(g_t0, g_stream)); }
int mlxr_timer_stop(float* ms) {
    if (!g_stream || !ms) return MLXR_E_INVALID_ARG;
    CK(hipEventRecord(g_t1, g_stream));
    CK(hipEventSynchronize(g_t1));
    return done(hipEventElapsedTime(ms, g_t0, g_t1));
}

// ------------------------------------------------------------------------------ kernels
int mlxr_k_qmv(const mlxr_qmat* parts, int nparts, int K, int bits, int gs, int st, const float* x, const float* norm_w,
               float eps, float* y, int epi) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (int rc = check_parts(parts, nparts)) return rc;
    if (int rc = check_quant(K, bits, gs, st)) return rc;
    if (!x || !y || epi < 0 || epi > 2) return set_error(MLXR_E_INVALID_ARG, "x / y / epi");
    if (epi == EPI_GATED && (nparts != 2 || parts[0].O != parts[1].O)) return set_error(MLXR_E_INVALID_ARG, "gated: two matrices of equal rows");
    if (norm_w && K > 16384) return set_error(MLXR_E_UNSUPPORTED, "normalised input wider than 16384");
    QmvArgs a; a.nparts = nparts; int O = 0;
    for (int i = 0; i < nparts; i++) { a.part[i] = qmat(parts[i]); O += parts[i].O; }
    a.K = K; a.bits = bits; a.gs = gs; a.st = st; a.O = epi == EPI_GATED ? parts[0].O : O;
    a.x = x; a.norm_w = norm_w; a.eps = eps; a.y = y; a.epi = epi;
    return done(launch_qmv(a, g_stream));
}

int mlxr_k_qmm(const mlxr_qmat* parts, int nparts, int K, int bits, int gs, int st, int T, const float* x, int x_stride,
               float* y, int y_stride) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (int rc = check_parts(parts, nparts)) return rc;
    if (int rc = check_quant(K, bits, gs, st)) return rc;
    int O = 0;
    for (int i = 0; i < nparts; i++) O += parts[i].O;
    if (T < 1 || T > 8 || !x || !y || x_stride < K || y_stride < O || x_stride % 4) return set_error(MLXR_E_INVALID_ARG, "T in 1..8, strides");
    QmmSmallArgs a; a.nparts = nparts;
    for (int i = 0; i < nparts; i++) a.part[i] = qmat(parts[i]);
    a.K = K; a.bits = bits; a.gs = gs; a.st = st; a.O = O; a.T = T; a.x = x; a.x_stride = x_stride; a.y = y; a.y_stride = y_stride;
    if (qmmx_supported(K, bits, gs)) {
        if (int rc = ensure_buf(g_xbf, g_xbf_elems, (size_t)T * K)) return rc;
        if (int rc = ensure_buf(g_xlo, g_xlo_elems, (size_t)T * K)) return rc;
        if (int rc = ensure_buf(g_xgs, g_xgs_elems, qgemm_gsum_floats(T, K, gs))) return rc;
        if (int rc = ensure_buf(g_xsc, g_xsc_elems, (size_t)T)) return rc;
        if (int rc = ensure_buf(g_xnz, g_xnz_elems, (size_t)T)) return rc;
        a.xbf = g_xbf; a.xlo = g_xlo; a.xgs = g_xgs; a.xsc = g_xsc; a.xnz = g_xnz;
    }
    return done(launch_qmm_small(a, g_stream));
}

int mlxr_k_qgemm(const mlxr_qmat* mat, int K, int bits, int gs, int st, int T, const float* x, int x_stride, float* y, int y_stride) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (int rc = check_parts(mat, 1)) return rc;
    if (int rc = check_quant(K, bits, gs, st)) return rc;
    if (T < 1 || !x || !y || x_stride < K || y_stride < mat->O || x_stride % 4) return set_error(MLXR_E_INVALID_ARG, "T / strides");
    if (int rc = ensure_buf(g_xbf, g_xbf_elems, (size_t)T * K)) return rc;
    if (int rc = ensure_buf(g_xsc, g_xsc_elems, (size_t)T)) return rc;
    if (int rc = ensure_buf(g_xlo, g_xlo_elems, (size_t)T * K)) return rc;
    if (int rc = ensure_buf(g_xgs, g_xgs_elems, qgemm_gsum_floats(T, K, gs))) return rc;
    if (int rc = ensure_buf(g_wsb, g_wsb_elems, qgemm_scale_halves(mat->O, K, gs))) return rc;
    if (int rc = ensure_buf(g_xnz, g_xnz_elems, (size_t)T)) return rc;
    if (!g_qsplit) {
        if (int rc = ensure_buf(g_qsplit, g_qsplit_floats, QGEMM_SPLIT_FLOATS)) return rc;
        CK(hipMemset(g_qsplit, 0, QGEMM_SPLIT_FLOATS * 4));
    }
    QGemmArgs a; a.m = qmat(*mat); a.K = K; a.bits = bits; a.gs = gs; a.st = st; a.O = mat->O; a.T = T;
    a.x = x; a.x_stride = x_stride; a.y = y; a.y_stride = y_stride; a.xbf = g_xbf; a.xsc = g_xsc;
    a.xlo = g_xlo; a.xgs = g_xgs; a.xnz = g_xnz; a.wsb = g_wsb;
    a.split = g_qsplit; a.split_floats = g_qsplit_floats;
    return done(launch_qgemm(a, g_stream));
}

// Repacks the parts into a temporary DPack (freed by the caller).
static int tiles_pack(const mlxr_qmat* parts, int nparts, int K, int gs, int gated, MvPhaseDesc& d, uint8_t*& code) {
    if (int rc = check_parts(parts, nparts)) return rc;
    if ((gs != 32 && gs != 64) || K % 128) return set_error(MLXR_E_INVALID_ARG, "repacked tiles need gs 32/64 and K % 128 == 0");
    if (gated && (nparts != 2 || parts[0].O != parts[1].O)) return set_error(MLXR_E_INVALID_ARG, "gated: two parts of equal O");
    DPackSrc src{};
    d = MvPhaseDesc{};
    int rows = 0;
    for (int i = 0; i < nparts; i++) rows += parts[i].O;
    for (int i = 0; i < 3; i++) {
        const mlxr_qmat& q = parts[i < nparts ? i : nparts - 1];
        src.w[i] = static_cast<const uint8_t*>(q.w);
        src.s[i] = static_cast<const uint16_t*>(q.scales); src.b[i] = static_cast<const uint16_t*>(q.biases);
        d.bias[i] = i < nparts ? static_cast<const uint16_t*>(q.bias) : nullptr;
    }
    d.o1 = src.o1 = parts[0].O; d.o2 = src.o2 = nparts > 1 ? parts[1].O : 0;
    d.rows = src.rows = rows; d.K = src.K = K; d.gs = src.gs = gs; d.gated = src.gated = gated ? 1 : 0;
    d.tiles = dpack_tiles(src);
    code = nullptr;
    CK(hipMalloc(&code, dpack_bytes(src)));
    d.code = code;
    const hipError_t e = launch_dpack(src, code, g_stream);
    if (e != hipSuccess) { hipFree(code); code = nullptr; return done(e); }
    return MLXR_OK;
}

int mlxr_k_qgemm_tiles(const mlxr_qmat* parts, int nparts, int K, int gs, int gated, int T, const float* x, int x_stride,
                       float* y, int y_stride) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    int rows = 0;
    for (int i = 0; i < nparts && parts; i++) rows += parts[i].O;
    const int out_cols = gated ? (parts ? parts[0].O : 0) : rows;
    if (T < 1 || !x || !y || x_stride < K || y_stride < out_cols || x_stride % 4) return set_error(MLXR_E_INVALID_ARG, "T / strides");
    MvPhaseDesc d; uint8_t* code;
    if (int rc = tiles_pack(parts, nparts, K, gs, gated, d, code)) return rc;
    if (int rc = ensure_buf(g_xbf, g_xbf_elems, (size_t)T * K)) { hipFree(code); return rc; }
    if (int rc = ensure_buf(g_xsc, g_xsc_elems, (size_t)T)) { hipFree(code); return rc; }
    hipError_t e = launch_x_to_f16(x, x_stride, K, T, g_xbf, g_xsc, g_stream);
    if (e == hipSuccess) e = launch_tile_gemm(d, g_xbf, g_xsc, T, y, y_stride, g_stream);
    const hipError_t e2 = hipStreamSynchronize(g_stream);
    hipFree(code);
    if (e == hipSuccess) e = e2;
    return done(e);
}

int mlxr_k_qmv_tiles(const mlxr_qmat* parts, int nparts, int K, int gs, int mode, const float* x, const float* norm_w, float eps,
                     float* y, int reps) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (mode < 0 || mode > 2 || !x || !y || reps < 1) return set_error(MLXR_E_INVALID_ARG, "mode / pointers / reps");
    MvPhaseDesc d; uint8_t* code;
    if (int rc = tiles_pack(parts, nparts, K, gs, mode == 2, d, code)) return rc;
    if (!dpack_mv_supported(d)) { hipFree(code); return set_error(MLXR_E_UNSUPPORTED, "matvec over repacked tiles: K too large"); }
    // the scratch of the input-sliced matvec, as the model's kernel-per-op step passes it
    const size_t sf = dpack_mv_split_floats(d.rows);
    if (sf > g_split_floats) {
        if (int rc = ensure_buf(g_split, g_split_floats, sf)) { hipFree(code); return rc; }
        CK(hipMemset(g_split, 0, sf * 4));   // tile counters start at zero and return to it
    }
    hipError_t e = hipSuccess;
    for (int r = 0; r < reps && e == hipSuccess; r++) e = launch_dpack_mv(d, x, norm_w, eps, y, mode, g_stream, g_split);
    const hipError_t e2 = hipStreamSynchronize(g_stream);
    hipFree(code);
    if (e == hipSuccess) e = e2;
    return done(e);
}

int mlxr_k_qmm_tiles(const mlxr_qmat* parts, int nparts, int K, int gs, int mode, int T, const float* x, int x_stride,
                     const float* norm_w, float eps, float* y, int y_stride) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (T < 1 || T > 8 || mode < 0 || mode > 2 || !x || !y || x_stride < K || x_stride % 4)
        return set_error(MLXR_E_INVALID_ARG, "T 1..8 / mode / pointers / strides");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(norm_w)) & 15)   // read as 16-byte vectors
        return set_error(MLXR_E_INVALID_ARG, "x and norm_w must be 16-byte aligned");
    MvPhaseDesc d; uint8_t* code;
    if (int rc = tiles_pack(parts, nparts, K, gs, mode == 2, d, code)) return rc;
    const int cols = mode == 2 ? d.o1 : d.rows;
    if (y_stride < cols) { hipFree(code); return set_error(MLXR_E_INVALID_ARG, "y_stride"); }
    // the input-slice scratch, as the model passes it (tile counters start at zero and return to it)
    const size_t sf = dpack_mm_split_floats(d);
    if (sf > g_split_floats) {
        if (int rc = ensure_buf(g_split, g_split_floats, sf)) { hipFree(code); return rc; }
        CK(hipMemset(g_split, 0, sf * 4));
    }
    hipError_t e = launch_dpack_mm(d, x, x_stride, norm_w, eps, y, y_stride, mode == 1, T, g_split, g_split_floats, g_stream);
    const hipError_t e2 = hipStreamSynchronize(g_stream);
    hipFree(code);
    if (e == hipSuccess) e = e2;
    if (e == hipErrorInvalidValue) return set_error(MLXR_E_UNSUPPORTED, "small-batch matvec over repacked tiles: shape");
    return done(e);
}

int mlxr_k_qembed(const mlxr_qmat* mat, int K, int bits, int gs, int st, const int32_t* ids, int T, float* out) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (int rc = check_parts(mat, 1)) return rc;
    if (!bits_ok(bits) || gs <= 0 || gs % 8 || K % gs || K % 8 || (st != 0 && st != 1)) return set_error(MLXR_E_UNSUPPORTED, "quantization");
    if (!ids || !out || T < 1) return set_error(MLXR_E_INVALID_ARG, "ids / out / T");
    std::vector<int32_t> h(T);
    CK(hipMemcpy(h.data(), ids, (size_t)T * 4, hipMemcpyDeviceToHost));
    for (int v : h) if (v < 0 || v >= mat->O) return set_error(MLXR_E_INVALID_FILE, "token id outside the embedding table");
    if (int rc = set_pos(0)) return rc;
    return done(launch_qembed(qmat(*mat), K, bits, gs, st, ids, g_pos, T, out, g_stream));
}

int mlxr_k_rms_norm(float* x_or_h, const float* r, float* y, const float* w, int dim, int rows, float eps) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (!x_or_h || !y || !w || dim <= 0 || dim % 4 || rows < 1) return set_error(MLXR_E_INVALID_ARG, "rms_norm arguments (dim % 4 == 0)");
    if (r) return done(launch_add_rms_norm(x_or_h, r, y, w, dim, rows, eps, g_stream));
    return done(launch_rms_norm(x_or_h, y, w, dim, rows, dim, eps, g_stream));
}

int mlxr_k_qkv_post(float* qkv, int row_stride, const float* inv_freq, void* kcache, void* vcache, int max_seq, const float* qn,
                    const float* kn, int D, int nH, int nKV, int rot_dim, int traditional, int offset, int T, float eps) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (!qkv || !inv_freq || !kcache || !vcache || D != 128 || nH < 1 || nKV < 1 || nH % nKV || rot_dim < 0 || rot_dim > D || rot_dim % 2 ||
        row_stride < (nH + 2 * nKV) * D || T < 1 || offset < 0 || offset + T > max_seq || max_seq % MLXR_PAGE || (qn == nullptr) != (kn == nullptr))
        return set_error(MLXR_E_INVALID_ARG, "qkv_post arguments (D 128, max_seq multiple of 64)");
    if (int rc = ensure_pt(max_seq)) return rc;
    if (int rc = set_pos(offset)) return rc;
    QkvPostArgs a; a.qkv = qkv; a.row_stride = row_stride; a.inv_freq = inv_freq; a.kc = (uint16_t*)kcache; a.vc = (uint16_t*)vcache;
    a.pt = g_pt; a.qn = qn; a.kn = kn; a.D = D; a.nH = nH; a.nKV = nKV; a.rot_dim = rot_dim; a.traditional = traditional; a.T = T;
    a.dpos = g_pos; a.eps = eps;
    return done(launch_qkv_post(a, g_stream));
}

int mlxr_k_attention(const float* q, int q_stride, const void* kcache, const void* vcache, int max_seq, int D, int nH, int nKV,
                     int offset, int T, float scale, float* out, int out_stride, const int32_t* lists, int count, int list_stride,
                     int nsplit) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (!q || !kcache || !vcache || !out || D != 128 || nH < 1 || nKV < 1 || nH % nKV || nH / nKV > 8 || T < 1 || offset < 0 ||
        offset + T > max_seq || max_seq % MLXR_PAGE || q_stride < nH * D || out_stride < nH * D)
        return set_error(MLXR_E_INVALID_ARG, "attention arguments (D 128, G <= 8, max_seq multiple of 64)");
    if (lists && (T != 1 || count < 1 || count > max_seq || list_stride < 0)) return set_error(MLXR_E_INVALID_ARG, "sparse lists: T 1, count");
    const int maxCount = lists ? count : offset + T;
    if (nsplit <= 0) nsplit = 32;
    // several dense queries share each key range (the verify batch's kernel: 128 keys per range at most)
    const bool multi = !lists && T > 1 && (nH / nKV) * T <= 64 && q_stride % 4 == 0;
    const int per = multi ? 128 : 512;
    if ((maxCount + nsplit - 1) / nsplit > per) nsplit = (maxCount + per - 1) / per;
    if (int rc = ensure_pt(max_seq)) return rc;
    if (int rc = ensure_buf(g_part, g_part_floats, (size_t)T * nH * nsplit * (D + 2))) return rc;
    if (int rc = set_pos(offset)) return rc;
    // the sparse plan only carries `count` to the kernel
    int* plan = nullptr;
    if (lists) {
        int p[8] = {1, 0, 0, 0, 0, 0, offset + 1, count};
        CK(hipMemcpy(g_pos + 16, p, sizeof p, hipMemcpyHostToDevice));
        plan = g_pos + 16;
    }
    AttnArgs a; a.q = q; a.q_stride = q_stride; a.kc = (const uint16_t*)kcache; a.vc = (const uint16_t*)vcache; a.pt = g_pt;
    a.out = out; a.out_stride = out_stride; a.part = g_part; a.D = D; a.nH = nH; a.nKV = nKV; a.T = T; a.nsplit = nsplit;
    a.dpos = g_pos; a.scale = scale; a.lists = lists; a.list_stride = list_stride; a.splan = plan;
    a.cap = (maxCount + nsplit - 1) / nsplit;
    return done(multi ? launch_attn_verify(a, g_stream) : launch_attn_decode(a, g_stream));
}

int mlxr_k_flash_prefill(const float* q, int q_stride, const void* kcache, const void* vcache, int max_seq, int D, int nH, int nKV,
                         int offset, int T, float scale, float* out, int out_stride) {
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (int rc = ensure_stream()) return rc;
        if (!q || !kcache || !vcache || !out || D != 128 || nH < 1 || nKV < 1 || nH % nKV || nH / nKV > 8 || T < 1 || offset < 0 ||
            offset + T > max_seq || max_seq % MLXR_PAGE || q_stride < nH * D || out_stride < nH * D)
            return set_error(MLXR_E_INVALID_ARG, "flash arguments (D 128, G <= 8, max_seq multiple of 64)");
        if (int rc = ensure_pt(max_seq)) return rc;
        if (int rc = set_pos(offset)) return rc;
        FlashArgs a; a.q = q; a.q_stride = q_stride; a.kc = (const uint16_t*)kcache; a.vc = (const uint16_t*)vcache; a.pt = g_pt;
        a.out = out; a.out_stride = out_stride; a.D = D; a.nH = nH; a.nKV = nKV; a.T = T; a.dpos = g_pos; a.scale = scale;
        return done(launch_flash_prefill(a, g_stream));
    }
}

int mlxr_k_sparse_index(const void* kcache, int max_seq, int nKV, int D, int offset, int T, void* idx) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (!kcache || !idx || D != 128 || nKV < 1 || T < 1 || offset < 0 || offset + T > max_seq || max_seq % MLXR_PAGE)
        return set_error(MLXR_E_INVALID_ARG, "sparse_index arguments");
    if (int rc = ensure_pt(max_seq)) return rc;
    if (int rc = set_pos(offset)) return rc;
    return done(launch_sparse_index((const uint16_t*)kcache, g_pt, (uint16_t*)idx, nKV, D, g_pos, 0, T, g_stream));
}

int mlxr_k_sparse_score(const float* q, const void* idx, int nH, int nKV, int D, int b0, int nb, int rows, float* scores) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (!q || !idx || !scores || nKV < 1 || nH % nKV || nKV * D > 4096 || D % 8 || b0 < 0 || nb < 1 || (rows != 1 && rows != nKV))
        return set_error(MLXR_E_INVALID_ARG, "sparse_score arguments");
    return done(launch_sparse_score_plan(q, (const uint16_t*)idx, scores, nH, nKV, D, b0, nb, rows, g_stream));
}

int mlxr_k_sparse_select(const float* scores, int rows, int b0, int nb, int p, int sink_end, int win_start, int L, int32_t* lists,
                         int list_stride) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    const int count = sink_end + p * 4 + (L - win_start);
    if (!scores || !lists || rows < 1 || nb < 1 || p < 1 || p > nb || sink_end != b0 * 4 || win_start != (b0 + nb) * 4 || L < win_start ||
        (rows > 1 && list_stride < count))
        return set_error(MLXR_E_INVALID_ARG, "sparse_select arguments (1 <= p <= nb, sink_end == b0*4, win_start == (b0+nb)*4)");
    return done(launch_sparse_select_plan(scores, lists, list_stride, rows, b0, nb, p, sink_end, win_start, L, g_stream));
}

int mlxr_k_sample(float* logits, int V, int32_t* hist, int32_t* status, uint64_t* rng, int pos, const mlxr_sample_params* sp) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (int rc = ensure_stream()) return rc;
    if (!logits || !hist || !status || !rng || !sp || V < 1 || pos < 0) return set_error(MLXR_E_INVALID_ARG, "sample arguments");
    const int blocks = (V + 255) / 256;
    if (blocks > g_blocks) {
        if (g_bmax) { hipStreamSynchronize(g_stream); hipFree(g_bmax); hipFree(g_barg); }
        CK(hipMalloc(&g_bmax, (size_t)blocks * 4)); CK(hipMalloc(&g_barg, (size_t)blocks * 4));
        g_blocks = blocks;
    }
    if (int rc = set_pos(pos)) return rc;
    SampleArgs a; a.logits = logits; a.V = V; a.hist = hist; a.status = status; a.rng = rng; a.bmax = g_bmax; a.barg = g_barg;
    a.dpos = g_pos; a.window = sp->window; a.top_k = sp->top_k; a.penalty = sp->penalty; a.temperature = sp->temperature;
    a.top_p = sp->top_p; a.min_p = sp->min_p;
    return done(launch_sample(a, g_stream));
}

}  // extern "C"
