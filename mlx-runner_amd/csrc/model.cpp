// Host runtime of the token loop (see model.h). Reference: Sources/MLXEngine/Transformer.swift,
// GPU.swift (safetensors), ModelConfig.swift (config), SparseAttention.swift (sparse plan budget).
#include "model.h"
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include "json.h"
#include <functional>

namespace mlxr {

static thread_local std::string g_err;
int set_error(int code, const std::string& msg) { g_err = msg; return code; }
const char* last_error() { return g_err.c_str(); }

#define HIPCHECK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) return set_error(e_ == hipErrorOutOfMemory ? MLXR_E_OUT_OF_MEMORY : MLXR_E_GPU, std::string(#x) + ": " + hipGetErrorString(e_)); } while (0)

static bool read_file(const std::string& path, std::string& out) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return false;
    fseek(f, 0, SEEK_END); long n = ftell(f); fseek(f, 0, SEEK_SET);
    if (n < 0 || n > (1 << 26)) { fclose(f); return false; }
    out.resize((size_t)n);
    bool ok = fread(&out[0], 1, (size_t)n, f) == (size_t)n;
    fclose(f);
    return ok;
}

// ------------------------------------------------------------------------------------ config
int parse_config(const std::string& dir, Config& c) {
    std::string text, err;
    if (!read_file(dir + "/config.json", text)) return set_error(MLXR_E_INVALID_FILE, "config.json not found or unreadable");
    Json o;
    if (!Json::parse(text.data(), text.size(), o, err) || o.t != Json::Obj) return set_error(MLXR_E_INVALID_FILE, "config.json: " + err);
    if (!o.get("hidden_size")) {   // multimodal exports nest the text model (ModelConfig.swift:163-165)
        if (const Json* tc = o.get("text_config")) for (auto& kv : tc->obj) o.obj.push_back(kv);
    }
    c.model_type = o.strOr("model_type", "");
    // end-of-sequence ids: config.json's eos_token_id (a number or a list), plus
    // generation_config.json's, deduplicated (ModelConfig.swift:284-291)
    {
        std::vector<int> eos;
        auto take = [&](const Json& root) {
            const Json* e = root.get("eos_token_id");
            if (!e) return;
            if (e->t == Json::Num) eos.push_back((int)e->num);
            else if (e->t == Json::Arr)
                for (const Json& v : e->arr) if (v.t == Json::Num) eos.push_back((int)v.num);
        };
        take(o);
        std::string gtext, gerr;
        Json g;
        if (read_file(dir + "/generation_config.json", gtext) && Json::parse(gtext.data(), gtext.size(), g, gerr) && g.t == Json::Obj) take(g);
        std::sort(eos.begin(), eos.end());
        eos.erase(std::unique(eos.begin(), eos.end()), eos.end());
        c.eos = eos;
    }
    for (auto& ch : c.model_type) ch = (char)tolower(ch);
    static const char* ok_types[] = {"qwen3", "qwen2", "llama", "mistral"};
    bool supported = false;
    for (auto t : ok_types) supported |= c.model_type == t;
    if (!supported) return set_error(MLXR_E_UNSUPPORTED, "architecture '" + c.model_type + "' is not supported (qwen3, qwen2, llama, mistral)");
    if (!o.get("hidden_size") || !o.get("num_hidden_layers") || !o.get("num_attention_heads"))
        return set_error(MLXR_E_INVALID_FILE, "config.json is missing core dimensions");
    c.H = (int)o.numOr("hidden_size", 0); c.L = (int)o.numOr("num_hidden_layers", 0); c.nH = (int)o.numOr("num_attention_heads", 0);
    c.I = (int)o.numOr("intermediate_size", 4.0 * c.H);
    c.nKV = (int)o.numOr("num_key_value_heads", c.nH);
    c.D = (int)o.numOr("head_dim", c.nH ? c.H / c.nH : 0);
    c.V = (int)o.numOr("vocab_size", 0);
    c.eps = (float)o.numOr("rms_norm_eps", 1e-6);
    c.theta = (double)(float)o.numOr("rope_theta", 10000);
    c.traditional = o.boolOr("rope_traditional", false);
    c.tie = o.boolOr("tie_word_embeddings", false);
    c.max_pos = (int)o.numOr("max_position_embeddings", 4096);
    const double partial = (float)o.numOr("partial_rotary_factor", 1.0);
    struct Range { const char* n; int v; int lo, hi; } dims[] = {
        {"hidden_size", c.H, 1, 65536}, {"intermediate_size", c.I, 1, 262144}, {"num_hidden_layers", c.L, 1, 512},
        {"num_attention_heads", c.nH, 1, 1024}, {"num_key_value_heads", c.nKV, 1, 1024}, {"head_dim", c.D, 1, 1024},
        {"max_position_embeddings", c.max_pos, 1, 1 << 24}};
    for (auto& d : dims)
        if (d.v < d.lo || d.v > d.hi) return set_error(MLXR_E_INVALID_FILE, std::string("config.json: ") + d.n + " = " + std::to_string(d.v) + " is out of range");
    if (c.nH % c.nKV) return set_error(MLXR_E_INVALID_FILE, "config.json: num_attention_heads must be a multiple of num_key_value_heads");
    if (!(c.eps > 0) || !std::isfinite(c.eps) || !(c.theta > 0) || !(partial > 0 && partial <= 1))
        return set_error(MLXR_E_INVALID_FILE, "config.json: invalid rms_norm_eps, rope_theta or partial_rotary_factor");
    c.query_scale = 1.0f / std::sqrt((float)c.D);
    c.rot_dim = (int)((float)c.D * (float)partial) / 2 * 2;
    // inverse frequencies (ModelConfig.swift:438-466), llama3 / linear scaling
    const int half = c.rot_dim / 2;
    std::vector<double> f(half);
    for (int i = 0; i < half; i++) f[i] = 1.0 / std::pow(c.theta, (double)(2 * i) / (double)c.rot_dim);
    if (const Json* rs = o.get("rope_scaling")) {
        if (rs->t == Json::Obj) {
            std::string type = rs->strOr("rope_type", rs->strOr("type", ""));
            double factor = rs->numOr("factor", 1);
            if (type == "llama3") {
                double low = rs->numOr("low_freq_factor", 1), high = rs->numOr("high_freq_factor", 4);
                double old = rs->numOr("original_max_position_embeddings", 8192);
                double lowW = old / low, highW = old / high;
                for (auto& x : f) {
                    double wl = 2 * M_PI / x;
                    if (wl < highW) continue;
                    if (wl > lowW) { x = x / factor; continue; }
                    double sm = (old / wl - low) / (high - low);
                    x = (1 - sm) * x / factor + sm * x;
                }
            } else if (type == "linear") {
                for (auto& x : f) x /= factor;
            } else if (!type.empty() && type != "default") {
                return set_error(MLXR_E_UNSUPPORTED, "rope_scaling type '" + type + "'");
            }
        }
    }
    c.inv_freq.resize(half);
    for (int i = 0; i < half; i++) c.inv_freq[i] = (float)f[i];
    const Json* q = o.get("quantization"); if (!q) q = o.get("quantization_config");
    if (q) { c.bits = (int)q->numOr("bits", 0); c.gs = (int)q->numOr("group_size", 0); }
    return MLXR_OK;
}

// ------------------------------------------------------------------------------ safetensors
enum DType { DT_U32, DT_BF16, DT_F16, DT_F32, DT_U8, DT_I32, DT_OTHER };
static int dtype_size(int d) { return d == DT_BF16 || d == DT_F16 ? 2 : d == DT_U8 ? 1 : 4; }
struct HostTensor { int dtype = DT_OTHER; std::vector<int64_t> shape; const uint8_t* data = nullptr; size_t nbytes = 0; };
struct Store {
    std::vector<std::pair<void*, size_t>> maps;
    std::map<std::string, HostTensor> t;
    ~Store() { for (auto& m : maps) munmap(m.first, m.second); }
    const HostTensor* get(const std::string& n) const { auto it = t.find(n); return it == t.end() ? nullptr : &it->second; }
};

// SafeTensorFile.init validation (GPU.swift:214-272).
static int load_safetensors(const std::string& path, Store& st) {
    const std::string file = path.substr(path.find_last_of('/') + 1);
    int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) return set_error(MLXR_E_INVALID_FILE, "cannot open " + file);
    struct stat sb;
    if (fstat(fd, &sb) != 0) { close(fd); return set_error(MLXR_E_INVALID_FILE, file); }
    const size_t size = (size_t)sb.st_size;
    if (size < 8) { close(fd); return set_error(MLXR_E_INVALID_FILE, file + " is truncated"); }
    void* p = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return set_error(MLXR_E_INVALID_FILE, "mmap failed for " + file);
    madvise(p, size, MADV_WILLNEED);
    st.maps.emplace_back(p, size);
    const uint8_t* base = (const uint8_t*)p;
    uint64_t hl; memcpy(&hl, base, 8);
    if (hl > std::min<uint64_t>(100ull << 20, size - 8)) return set_error(MLXR_E_INVALID_FILE, "bad header length in " + file);
    Json h; std::string err;
    if (!Json::parse((const char*)base + 8, (size_t)hl, h, err) || h.t != Json::Obj) return set_error(MLXR_E_INVALID_FILE, "bad header JSON in " + file);
    const size_t dstart = 8 + (size_t)hl, dsize = size - dstart;
    for (auto& kv : h.obj) {
        if (kv.first == "__metadata__") continue;
        const Json& e = kv.second;
        const Json* dt = e.get("dtype"); const Json* sh = e.get("shape"); const Json* of = e.get("data_offsets");
        if (!dt || dt->t != Json::Str) return set_error(MLXR_E_INVALID_FILE, "bad entry '" + kv.first + "' in " + file);
        int d = dt->str == "U32" ? DT_U32 : dt->str == "BF16" ? DT_BF16 : dt->str == "F16" ? DT_F16 : dt->str == "F32" ? DT_F32
              : dt->str == "U8" ? DT_U8 : dt->str == "I32" ? DT_I32 : DT_OTHER;
        if (d == DT_OTHER) continue;   // unused dtypes
        if (!sh || sh->t != Json::Arr || sh->arr.size() > 8 || !of || of->t != Json::Arr || of->arr.size() != 2)
            return set_error(MLXR_E_INVALID_FILE, "bad entry '" + kv.first + "' in " + file);
        HostTensor t; t.dtype = d;
        int64_t count = 1;
        for (auto& s : sh->arr) {
            if (s.t != Json::Num || s.num < 0 || s.num > 2147483647.0) return set_error(MLXR_E_INVALID_FILE, "tensor '" + kv.first + "' is out of bounds in " + file);
            const int64_t v = (int64_t)s.num;
            if (v && count > INT64_MAX / 8 / v) return set_error(MLXR_E_INVALID_FILE, "tensor '" + kv.first + "' is too large in " + file);
            count *= v; t.shape.push_back(v);
        }
        if (of->arr[0].t != Json::Num || of->arr[1].t != Json::Num) return set_error(MLXR_E_INVALID_FILE, "bad entry '" + kv.first + "'");
        const double a = of->arr[0].num, b = of->arr[1].num;
        if (!(a >= 0 && a <= b && b <= (double)dsize)) return set_error(MLXR_E_INVALID_FILE, "tensor '" + kv.first + "' is out of bounds in " + file);
        if ((double)count * dtype_size(d) != b - a) return set_error(MLXR_E_INVALID_FILE, "tensor '" + kv.first + "' size does not match its shape in " + file);
        t.data = base + dstart + (size_t)a; t.nbytes = (size_t)(b - a);
        st.t[kv.first] = t;
    }
    return MLXR_OK;
}

// WeightStore.shardFiles (GPU.swift:317-330).
static int load_store(const std::string& dir, Store& st) {
    std::vector<std::string> all;
    DIR* d = opendir(dir.c_str());
    if (!d) return set_error(MLXR_E_INVALID_FILE, "cannot list " + dir);
    while (dirent* e = readdir(d)) {
        std::string n = e->d_name;
        if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) all.push_back(n);
    }
    closedir(d);
    std::sort(all.begin(), all.end());
    std::string idx;
    if (read_file(dir + "/model.safetensors.index.json", idx)) {
        Json j; std::string err;
        if (Json::parse(idx.data(), idx.size(), j, err)) {
            if (const Json* wm = j.get("weight_map")) {
                std::vector<std::string> listed;
                for (auto& n : all) {
                    bool ref = false;
                    for (auto& kv : wm->obj) if (kv.second.t == Json::Str && kv.second.str == n) { ref = true; break; }
                    if (ref) listed.push_back(n);
                }
                if (!listed.empty()) all = listed;
            }
        }
    }
    if (all.empty()) return set_error(MLXR_E_INVALID_FILE, "no .safetensors files in " + dir);
    for (auto& n : all) if (int rc = load_safetensors(dir + "/" + n, st)) return rc;
    // multimodal aliases (GPU.swift:349-357)
    if (!st.get("model.embed_tokens.weight")) {
        const char* from[] = {"language_model.model.", "language_model.lm_head.", "model.language_model."};
        const char* to[] = {"model.", "lm_head.", "model."};
        std::vector<std::pair<std::string, HostTensor>> add;
        for (auto& kv : st.t)
            for (int i = 0; i < 3; i++)
                if (kv.first.rfind(from[i], 0) == 0) add.emplace_back(to[i] + kv.first.substr(strlen(from[i])), kv.second);
        for (auto& a : add) if (!st.get(a.first)) st.t[a.first] = a.second;
    }
    return MLXR_OK;
}

// ------------------------------------------------------------------------------------ model
Model::~Model() {
    if (stream) hipStreamSynchronize(stream);
    for (auto& g : graphs) hipGraphExecDestroy(g.second);
    for (auto g : graph_defs) hipGraphDestroy(g);
    for (auto& s : slots) { if (s.start) hipEventDestroy(s.start); if (s.stop) hipEventDestroy(s.stop); }
    for (void* p : allocs) hipFree(p);
    if (h_tokens) hipHostFree(h_tokens);
    if (h_pos) hipHostFree(h_pos);
    if (h_logits) hipHostFree(h_logits);
    if (ring_tok) hipHostFree(ring_tok);
    if (ring_status) hipHostFree(ring_status);
    if (abort_host) hipHostFree(abort_host);
    if (stream) hipStreamDestroy(stream);
}

namespace {
struct Arena {
    uint8_t* base = nullptr; size_t used = 0, cap = 0;
    void* take(size_t n) { size_t a = (used + 255) & ~(size_t)255; if (a + n > cap) return nullptr; used = a + n; return base + a; }
};

int dev_alloc(Model* m, void** p, size_t n) {
    hipError_t e = hipMalloc(p, n < 256 ? 256 : n);
    if (e != hipSuccess) return set_error(MLXR_E_OUT_OF_MEMORY, "could not allocate " + std::to_string(n >> 20) + " MiB on the GPU");
    m->allocs.push_back(*p);
    m->device_bytes += (int64_t)n;
    return MLXR_OK;
}
template <typename T> int dalloc(Model* m, T** p, size_t count) { return dev_alloc(m, reinterpret_cast<void**>(p), count * sizeof(T)); }

int upload(Arena& ar, const HostTensor& t, const void** out) {
    void* d = ar.take(t.nbytes);
    if (!d) return set_error(MLXR_E_OUT_OF_MEMORY, "weight arena exhausted");
    if (hipMemcpy(d, t.data, t.nbytes, hipMemcpyHostToDevice) != hipSuccess) return set_error(MLXR_E_GPU, "weight upload failed");
    *out = d;
    return MLXR_OK;
}

std::vector<float> floats_of(const HostTensor& t) {
    size_t n = t.nbytes / dtype_size(t.dtype);
    std::vector<float> v(n);
    for (size_t i = 0; i < n; i++) {
        uint16_t u;
        switch (t.dtype) {
            case DT_BF16: memcpy(&u, t.data + 2 * i, 2); v[i] = bf16_to_f32(u); break;
            case DT_F16: { memcpy(&u, t.data + 2 * i, 2); _Float16 hh; memcpy(&hh, &u, 2); v[i] = (float)hh; break; }
            case DT_F32: memcpy(&v[i], t.data + 4 * i, 4); break;
            default: v[i] = 0;
        }
    }
    return v;
}

// Linear.init validation (Transformer.swift:48-111).
int make_lin(const Store& st, Arena& ar, const std::string& prefix, int inDim, int expectOut, Lin& L) {
    const HostTensor* w = st.get(prefix + ".weight");
    const HostTensor* s = st.get(prefix + ".scales");
    const HostTensor* b = st.get(prefix + ".biases");
    const HostTensor* bias = st.get(prefix + ".bias");
    if (!w) return set_error(MLXR_E_MISSING_TENSOR, prefix + ".weight");
    if (s && !b) return set_error(MLXR_E_MISSING_TENSOR, prefix + ".biases");
    auto bad = [&](const std::string& what) { return set_error(MLXR_E_INVALID_FILE, prefix + ": " + what); };
    if (w->shape.size() != 2 || w->shape[0] <= 0 || w->shape[1] <= 0 || inDim <= 0) return bad("weight must be a 2-D tensor");
    if (expectOut > 0 && w->shape[0] != expectOut) return bad("expected " + std::to_string(expectOut) + " output rows, found " + std::to_string(w->shape[0]));
    if (!s) return set_error(MLXR_E_UNSUPPORTED, prefix + ": dense (unquantized) weights are not supported by this build");
    if (bias && (bias->shape.size() != 1 || bias->shape[0] != w->shape[0])) return bad("bias shape");
    if (s->shape.size() != 2 || s->shape[0] != w->shape[0] || s->shape[1] <= 0 || inDim % s->shape[1] != 0 || b->shape != s->shape ||
        (w->shape[1] * dtype_size(w->dtype) * 8) % inDim != 0)
        return bad("inconsistent quantization tensors");
    const int64_t packed = w->shape[1] * dtype_size(w->dtype);
    L.bits = (int)(packed * 8 / inDim);
    L.gs = inDim / (int)s->shape[1];
    if (!(L.bits == 2 || L.bits == 3 || L.bits == 4 || L.bits == 5 || L.bits == 6 || L.bits == 8) || L.gs % 8 != 0 || inDim % 8 != 0)
        return set_error(MLXR_E_UNSUPPORTED, prefix + ": " + std::to_string(L.bits) + "-bit / group " + std::to_string(L.gs) + " quantization");
    // This build's kernels take 32 codes per lane step within one group.
    if (inDim % 64 != 0 || L.gs % 32 != 0)
        return set_error(MLXR_E_UNSUPPORTED, prefix + ": input size " + std::to_string(inDim) + " / group " + std::to_string(L.gs) + " (needs K % 64 == 0, group % 32 == 0)");
    if (s->dtype != DT_BF16 && s->dtype != DT_F16) return set_error(MLXR_E_UNSUPPORTED, prefix + ": scales dtype");
    if (b->dtype != s->dtype || (bias && bias->dtype != s->dtype)) return set_error(MLXR_E_UNSUPPORTED, prefix + ": mixed quantization dtypes");
    L.st = s->dtype == DT_F16 ? 1 : 0;
    L.K = inDim; L.O = (int)w->shape[0]; L.m.O = L.O;
    const void* p;
    if (int rc = upload(ar, *w, &p)) return rc; L.m.w = (const uint8_t*)p;
    if (int rc = upload(ar, *s, &p)) return rc; L.m.s = (const uint16_t*)p;
    if (int rc = upload(ar, *b, &p)) return rc; L.m.b = (const uint16_t*)p;
    if (bias) { if (int rc = upload(ar, *bias, &p)) return rc; L.m.bias = (const uint16_t*)p; }
    L.desc = "q" + std::to_string(L.bits) + "g" + std::to_string(L.gs);
    return MLXR_OK;
}

int norm_weight(Model* m, const Store& st, const std::string& name, int dim, float** out) {
    const HostTensor* t = st.get(name);
    if (!t) return set_error(MLXR_E_MISSING_TENSOR, name);
    if (t->shape.size() != 1 || t->shape[0] != dim) return set_error(MLXR_E_INVALID_FILE, name + ": expected shape [" + std::to_string(dim) + "]");
    std::vector<float> v = floats_of(*t);
    if (int rc = dalloc(m, out, dim)) return rc;
    if (hipMemcpy(*out, v.data(), dim * 4, hipMemcpyHostToDevice) != hipSuccess) return set_error(MLXR_E_GPU, "upload " + name);
    return MLXR_OK;
}

size_t lin_bytes(const Store& st, const std::string& prefix) {
    size_t n = 0;
    for (const char* suf : {".weight", ".scales", ".biases", ".bias"})
        if (const HostTensor* t = st.get(prefix + suf)) n += (t->nbytes + 255) & ~(size_t)255;
    return n;
}
}  // namespace

void sparse_clamp(mlxr_sparse_cfg& c) {   // SparseAttention.init (SparseAttention.swift:47-54)
    const int p = 4;
    c.top_k = std::max(p, std::min(c.top_k, 1 << 22)) / p * p;
    c.window = std::max(p, std::min(c.window, 1 << 22));
    c.sink = std::max(0, std::min(c.sink, 1 << 16));
    int mc = c.min_context > 0 ? c.min_context : 2 * (c.sink + c.top_k + c.window);
    c.min_context = std::max(1, std::min(mc, 1 << 30));
    c.per_head = c.per_head ? 1 : 0;
}

// The persistent decode step (decode.hip) covers 4-bit bf16-scaled models with head_dim 128,
// at most 8 query heads per KV head and a KV-head count dividing the workgroup count.
// The repacked copy (DPack) of every layer's phases, built when every projection is 4-bit with
// bf16 scales, gs 32/64, K % 128 == 0 and each fused phase shares one group size. The prefill tile
// GEMMs read it; the persistent decode step (mega_setup) reads it too, plus a repacked lm_head.
static MvPhaseDesc repack_phase(Model* m, const Lin* parts, int n, bool gated, int& rc) {
    MvPhaseDesc d{};
    DPackSrc src{};
    for (int i = 0; i < 3; i++) {
        const Lin& l = parts[i < n ? i : n - 1];
        src.w[i] = reinterpret_cast<const uint8_t*>(l.m.w); src.s[i] = l.m.s; src.b[i] = l.m.b;
        d.bias[i] = i < n ? l.m.bias : nullptr;
    }
    d.o1 = src.o1 = parts[0].O; d.o2 = src.o2 = n > 1 ? parts[1].O : 0;
    int rows = 0; for (int i = 0; i < n; i++) rows += parts[i].O;
    d.rows = src.rows = rows; d.K = src.K = parts[0].K; d.gs = src.gs = parts[0].gs; d.gated = src.gated = gated ? 1 : 0;
    d.tiles = dpack_tiles(src);
    uint8_t* code = nullptr;
    if (rc == MLXR_OK) rc = dalloc(m, &code, dpack_bytes(src));
    if (rc == MLXR_OK && launch_dpack(src, code, m->stream) != hipSuccess) rc = set_error(MLXR_E_GPU, "repack launch");
    d.code = code;
    return d;
}
static bool repackable(const Lin& l) { return l.bits == 4 && l.st == 0 && l.K % 128 == 0 && (l.gs == 32 || l.gs == 64); }
static int tiles_setup(Model* m) {
    const Config& c = m->cfg;
    for (auto& ly : m->layers) {
        for (const Lin* l : {&ly.q, &ly.k, &ly.v, &ly.o, &ly.gate, &ly.up, &ly.down})
            if (!repackable(*l)) return MLXR_OK;
        if (ly.q.gs != ly.k.gs || ly.q.gs != ly.v.gs || ly.gate.gs != ly.up.gs) return MLXR_OK;
    }
    int rc = MLXR_OK;
    std::vector<LayerDev> host(c.L);
    for (int i = 0; i < c.L; i++) {
        const Layer& ly = m->layers[i];
        const Lin qkv[3] = {ly.q, ly.k, ly.v}, gu[2] = {ly.gate, ly.up};
        LayerDev& d = host[i];
        d.qkv = repack_phase(m, qkv, 3, false, rc); d.o = repack_phase(m, &ly.o, 1, false, rc);
        d.gu = repack_phase(m, gu, 2, true, rc); d.down = repack_phase(m, &ly.down, 1, false, rc);
        if (rc) return rc;
        d.in_norm = ly.in_norm; d.post_norm = ly.post_norm; d.q_norm = ly.q_norm; d.k_norm = ly.k_norm;
        d.kc = ly.kc; d.vc = ly.vc;
    }
    if (repackable(m->head)) m->tile_head = repack_phase(m, &m->head, 1, false, rc);
    if (rc) return rc;
    // the verify batch's input-slice scratch: the largest any phase needs (counters zeroed once)
    size_t mm = 0;
    for (const LayerDev& d : host)
        for (const MvPhaseDesc* p : {&d.qkv, &d.o, &d.gu, &d.down}) mm = std::max(mm, dpack_mm_split_floats(*p));
    if (m->tile_head.code) mm = std::max(mm, dpack_mm_split_floats(m->tile_head));
    if (mm) {
        if ((rc = dalloc(m, &m->mm_split, mm))) return rc;
        HIPCHECK(hipMemset(m->mm_split, 0, mm * 4));
        m->mm_split_floats = mm;
    }
    HIPCHECK(hipStreamSynchronize(m->stream));
    m->tile_layers = host;
    return MLXR_OK;
}

static int mega_setup(Model* m) {
    const Config& c = m->cfg;
    auto no = [&](const std::string& why) { m->mega_ok = false; m->mega_reason = why; return MLXR_OK; };
    auto four_bf16 = [&](const Lin& l) { return repackable(l) && l.gs == m->head.gs; };
    if (!four_bf16(m->embed) || !four_bf16(m->head)) return no("embedding / lm_head not 4-bit bf16");
    if ((int)m->tile_layers.size() != c.L) return no("projections not repackable (4-bit, bf16 scales, gs 32/64, K % 128)");
    for (auto& ly : m->layers)
        for (const Lin* l : {&ly.q, &ly.k, &ly.v, &ly.o, &ly.gate, &ly.up, &ly.down})
            if (!four_bf16(*l)) return no("a projection's group size differs from the lm_head's");
    if (c.D != 128 || c.nH / c.nKV > 8 || c.rot_dim > 128) return no("head shape");
    if (5 * c.L + 2 > 1023) return no("too many layers for the exchange tags");
    hipDeviceProp_t prop;
    HIPCHECK(hipGetDeviceProperties(&prop, 0));
    int cus = prop.multiProcessorCount;
    const int nwg = cus / c.nKV * c.nKV;
    if (nwg < c.nKV) return no("too few compute units");
    const int nsplit = nwg / c.nKV;
    const int max_keys = (m->max_seq + nsplit - 1) / nsplit;
    if ((c.nH / c.nKV) * nsplit > 512) return no("too many attention partials per KV head");
    if (nsplit > mega_split_cap()) return no("too many key ranges per KV head");
    {
        const int tmax = std::max({(c.V + 15) / 16, ((c.nH + 2 * c.nKV) * c.D + 15) / 16, (c.I + 7) / 8, (c.H + 15) / 16});
        if ((tmax + nwg - 1) / nwg > mega_tiles_per_wg_cap()) return no("too many row tiles per workgroup");
        if (16 * ((c.H + 15) / 16 + nwg - 1) / nwg > mega_wg_row_cap()) return no("too many residual rows per workgroup");
        for (auto& ly : m->layers)
            if (ly.q.gs != ly.k.gs || ly.q.gs != ly.v.gs || ly.gate.gs != ly.up.gs) return no("mixed group sizes in a fused phase");
    }
    MegaArgs& a = m->mega;
    a.H = c.H; a.nH = c.nH; a.nKV = c.nKV; a.I = c.I; a.rot_dim = c.rot_dim; a.traditional = c.traditional;
    // a layer's K (or V) cache in bytes: the LDS-staged chunk addresses it with 32-bit offsets
    a.kv_stage = (double)m->n_pages * c.nKV * MLXR_PAGE * c.D * 2 < 2147483648.0 ? 1 : 0;
    a.L = c.L; a.n_pages = m->n_pages;
    const size_t lds = mega_lds_bytes(a, max_keys);
    a.desc_lds_off = (int)mega_desc_offset(a);
    a.pt_lds_off = a.desc_lds_off + (int)(sizeof(LayerDev) * c.L);
    if (lds > 158 * 1024) return no("LDS need " + std::to_string(lds >> 10) + " KiB");
    if (mega_set_lds_limit(lds) != hipSuccess) return no("LDS attribute");
    if (nwg > MEGA_MAX_WG) return no("too many workgroups");
    // co-residency: the phases' hand-overs wait for other workgroups, so the whole grid must fit the
    // device at once (every wait is bounded, so a grid that still ends up partly resident aborts)
    a.head = m->tile_head;   // the kernel variant follows the group size
    const int per_cu = mega_blocks_per_cu(a, lds);
    if (per_cu < 1 || nwg > per_cu * cus)
        return no("the grid cannot be resident at once (" + std::to_string(per_cu) + " workgroups per CU)");
    // the layers' repacked phases (tiles_setup), plus the lm_head's
    int rc = MLXR_OK;
    if ((rc = dalloc(m, &m->mega_layers, c.L))) return rc;
    HIPCHECK(hipMemcpy(m->mega_layers, m->tile_layers.data(), sizeof(LayerDev) * c.L, hipMemcpyHostToDevice));
    a.layers = m->mega_layers; a.L = c.L;
    a.head = m->tile_head;
    a.embed_w = m->embed.m.w; a.embed_s = m->embed.m.s; a.embed_b = m->embed.m.b; a.embed_gs = m->embed.gs;
    a.final_norm = m->final_norm; a.inv_freq = m->inv_freq;
    a.eps = c.eps; a.scale = c.query_scale * c.rope_attention_factor * c.rope_attention_factor;
    a.pt = m->page_table; a.hist = m->hist; a.status = m->status; a.dpos = m->dpos;
    a.logits = m->logits;
    {   // tagged exchange vectors (zeroed: tag 0 names no phase)
        const size_t qkv_n = (size_t)(c.nH + 2 * c.nKV) * c.D;
        if ((rc = dalloc(m, &a.hA, (size_t)c.H)) || (rc = dalloc(m, &a.hB, (size_t)c.H)) || (rc = dalloc(m, &a.qkvT, qkv_n)) ||
            (rc = dalloc(m, &a.attnT, (size_t)c.nH * c.D)) || (rc = dalloc(m, &a.mlpT, (size_t)c.I)))
            return rc;
        HIPCHECK(hipMemset(a.hA, 0, sizeof(uint2) * c.H));
        HIPCHECK(hipMemset(a.hB, 0, sizeof(uint2) * c.H));
        HIPCHECK(hipMemset(a.qkvT, 0, sizeof(uint2) * qkv_n));
        HIPCHECK(hipMemset(a.attnT, 0, sizeof(uint2) * c.nH * c.D));
        HIPCHECK(hipMemset(a.mlpT, 0, sizeof(uint2) * c.I));
    }
    if ((rc = dalloc(m, &a.part, (size_t)c.nH * nsplit * (c.D + 2))) || (rc = dalloc(m, &a.part_ready, (size_t)c.nKV * nsplit)) ||
        (rc = dalloc(m, &a.wg_best, nwg)) ||
        (rc = dalloc(m, &a.wg_idx, nwg)) || (rc = dalloc(m, &a.kv_done, 64 * 32)) || (rc = dalloc(m, &a.head_done, 64)) ||
        (rc = dalloc(m, &a.sync, 1)))
        return rc;
    HIPCHECK(hipMemset(a.part_ready, 0, sizeof(uint2) * c.nKV * nsplit));
    HIPCHECK(hipMemset(a.kv_done, 0, 64 * 32 * 4));
    HIPCHECK(hipMemset(a.head_done, 0, 64 * 4));
    HIPCHECK(hipMemset(a.sync, 0, sizeof(MegaSync)));
    a.ring_tok = m->ring_tok_dev; a.ring_status = m->ring_status_dev; a.ring_mask = Model::RING - 1;
    *m->abort_host = 0;
    a.abort_host = m->abort_host_dev;
    a.spin_limit = MEGA_SPIN_LIMIT; a.stall = 0;
    m->mega_nwg = nwg; m->mega_lds = lds; m->mega_ok = true;
    return MLXR_OK;
}

int model_set_decode_mode(Model* m, int mode) {
    if (mode < 0 || mode > 2)
        return set_error(MLXR_E_INVALID_ARG, "decode mode: 0 (kernel per op), 1 (persistent) or 2 (kernel per op, MLX layout)");
    for (auto& s : m->slots)
        if (s.busy) return set_error(MLXR_E_INVALID_ARG, "decode mode change with a step in flight");
    if (mode != m->decode_mode) {   // captured steps hold the previous mode's kernels
        HIPCHECK(hipStreamSynchronize(m->stream));
        for (auto& g : m->graphs) hipGraphExecDestroy(g.second);
        m->graphs.clear();
    }
    m->decode_mode = mode;
    return MLXR_OK;
}

int model_open(const char* dir_c, int context_len, const mlxr_sparse_cfg* sparse, Model** out) {
    *out = nullptr;
    std::string dir = dir_c;
    auto m = new Model();
    auto fail = [&](int rc) { delete m; return rc; };
    if (int rc = parse_config(dir, m->cfg)) return fail(rc);
    Config& c = m->cfg;
    if (c.D != 128) return fail(set_error(MLXR_E_UNSUPPORTED, "head_dim " + std::to_string(c.D) + " (this build's attention kernels take 128)"));
    if (c.nH / c.nKV > 8) return fail(set_error(MLXR_E_UNSUPPORTED, "more than 8 query heads per KV head"));
    if (c.H % 64 || c.I % 64) return fail(set_error(MLXR_E_UNSUPPORTED, "hidden / intermediate sizes must be multiples of 64"));
    // Transformer.init: seq = max(256, min(contextLength, max(maxPositionEmbeddings, 256))), rounded up to whole pages
    int seq = std::max(256, std::min(context_len, std::max(c.max_pos, 256)));
    seq = (seq + MLXR_PAGE - 1) / MLXR_PAGE * MLXR_PAGE;
    m->max_seq = seq; m->n_pages = seq / MLXR_PAGE;
    Store st;
    if (int rc = load_store(dir, st)) return fail(rc);   // files are validated before any device work
    {
        std::vector<std::string> need = {"model.embed_tokens.weight", "model.embed_tokens.scales", "model.embed_tokens.biases", "model.norm.weight"};
        for (int i = 0; i < c.L; i++) {
            const std::string p = "model.layers." + std::to_string(i);
            for (const char* l : {".self_attn.q_proj", ".self_attn.k_proj", ".self_attn.v_proj", ".self_attn.o_proj", ".mlp.gate_proj", ".mlp.up_proj", ".mlp.down_proj"})
                for (const char* suf : {".weight", ".scales", ".biases"}) need.push_back(p + l + suf);
            need.push_back(p + ".input_layernorm.weight");
            need.push_back(p + ".post_attention_layernorm.weight");
        }
        for (auto& n : need) if (!st.get(n)) return fail(set_error(MLXR_E_MISSING_TENSOR, n));
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) return fail(set_error(MLXR_E_NO_DEVICE, "no HIP GPU available"));
    // weight arena
    size_t total = lin_bytes(st, "model.embed_tokens") + lin_bytes(st, "lm_head");
    for (int i = 0; i < c.L; i++) {
        std::string p = "model.layers." + std::to_string(i);
        for (const char* n : {".self_attn.q_proj", ".self_attn.k_proj", ".self_attn.v_proj", ".self_attn.o_proj", ".mlp.gate_proj", ".mlp.up_proj", ".mlp.down_proj"})
            total += lin_bytes(st, p + n);
    }
    if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) return fail(set_error(MLXR_E_GPU, "stream"));
    size_t freeB = 0, totalB = 0;
    hipMemGetInfo(&freeB, &totalB);
    const size_t kvBytes = (size_t)c.L * 2 * m->n_pages * c.nKV * MLXR_PAGE * c.D * 2;
    if (total + kvBytes > freeB) return fail(set_error(MLXR_E_OUT_OF_MEMORY, "the model needs " + std::to_string((total + kvBytes) >> 20) + " MiB; " + std::to_string(freeB >> 20) + " MiB free"));
    Arena ar;
    if (int rc = dev_alloc(m, (void**)&ar.base, total + 4096)) return fail(rc);
    ar.cap = total + 4096;
    m->arena = ar.base;
    if (int rc = make_lin(st, ar, "model.embed_tokens", c.H, 0, m->embed)) return fail(rc);
    if (c.V == 0) c.V = m->embed.O;
    if (st.get("lm_head.weight")) { if (int rc = make_lin(st, ar, "lm_head", c.H, 0, m->head)) return fail(rc); }
    else { m->head = m->embed; m->tied = true; }
    if (int rc = norm_weight(m, st, "model.norm.weight", c.H, &m->final_norm)) return fail(rc);
    m->layers.resize(c.L);
    const int kvBlk = c.nKV * MLXR_PAGE * c.D;
    for (int i = 0; i < c.L; i++) {
        Layer& ly = m->layers[i];
        std::string p = "model.layers." + std::to_string(i);
        int rc;
        if ((rc = make_lin(st, ar, p + ".self_attn.q_proj", c.H, c.nH * c.D, ly.q)) || (rc = make_lin(st, ar, p + ".self_attn.k_proj", c.H, c.nKV * c.D, ly.k)) ||
            (rc = make_lin(st, ar, p + ".self_attn.v_proj", c.H, c.nKV * c.D, ly.v)) || (rc = make_lin(st, ar, p + ".self_attn.o_proj", c.nH * c.D, c.H, ly.o)) ||
            (rc = make_lin(st, ar, p + ".mlp.gate_proj", c.H, c.I, ly.gate)) || (rc = make_lin(st, ar, p + ".mlp.up_proj", c.H, c.I, ly.up)) ||
            (rc = make_lin(st, ar, p + ".mlp.down_proj", c.I, c.H, ly.down)))
            return fail(rc);
        if (ly.q.bits != ly.k.bits || ly.q.bits != ly.v.bits || ly.q.gs != ly.k.gs || ly.q.gs != ly.v.gs || ly.q.st != ly.k.st || ly.q.st != ly.v.st ||
            (ly.q.m.bias != nullptr) != (ly.k.m.bias != nullptr) || (ly.q.m.bias != nullptr) != (ly.v.m.bias != nullptr))
            return fail(set_error(MLXR_E_UNSUPPORTED, p + ": q/k/v projections quantized differently"));
        if (ly.gate.bits != ly.up.bits || ly.gate.gs != ly.up.gs || ly.gate.st != ly.up.st || ly.gate.m.bias || ly.up.m.bias)
            return fail(set_error(MLXR_E_UNSUPPORTED, p + ": gate/up projections quantized differently"));
        if ((rc = norm_weight(m, st, p + ".input_layernorm.weight", c.H, &ly.in_norm)) ||
            (rc = norm_weight(m, st, p + ".post_attention_layernorm.weight", c.H, &ly.post_norm)))
            return fail(rc);
        const bool hq = st.get(p + ".self_attn.q_norm.weight") != nullptr, hk = st.get(p + ".self_attn.k_norm.weight") != nullptr;
        if (hq != hk) return fail(set_error(MLXR_E_INVALID_FILE, p + ": q_norm and k_norm must come together"));
        if (hq && ((rc = norm_weight(m, st, p + ".self_attn.q_norm.weight", c.D, &ly.q_norm)) || (rc = norm_weight(m, st, p + ".self_attn.k_norm.weight", c.D, &ly.k_norm))))
            return fail(rc);
        if ((rc = dalloc(m, &ly.kc, (size_t)m->n_pages * kvBlk)) || (rc = dalloc(m, &ly.vc, (size_t)m->n_pages * kvBlk))) return fail(rc);
    }
    m->quant_desc = m->layers[0].down.desc;
    m->weight_bytes = (int64_t)ar.used;
    std::vector<float> invf = c.inv_freq; invf.resize(std::max<size_t>(invf.size(), 1));
    if (int rc = dalloc(m, &m->inv_freq, invf.size())) return fail(rc);
    HIPCHECK(hipMemcpy(m->inv_freq, invf.data(), invf.size() * 4, hipMemcpyHostToDevice));
    // page table: identity over this sequence's pages
    std::vector<int> pt(m->n_pages);
    for (int i = 0; i < m->n_pages; i++) pt[i] = i;
    if (int rc = dalloc(m, &m->page_table, m->n_pages)) return fail(rc);
    HIPCHECK(hipMemcpy(m->page_table, pt.data(), pt.size() * 4, hipMemcpyHostToDevice));
    // scratch (Transformer.swift:906-930), sized for max_batch tokens
    const int B = m->max_batch, H = c.H, I = c.I, V = c.V;
    m->qkv_cols = (c.nH + 2 * c.nKV) * c.D;
    m->nsplit_dec = std::max((seq + 511) / 512, std::min(64, (512 + c.nKV - 1) / c.nKV));
    // verify batches: key ranges of at most 128 keys for the multi-query kernel
    m->nsplit_ver = std::max(m->nsplit_dec, (seq + 127) / 128);
    const size_t partFloats = (size_t)8 * c.nH * m->nsplit_ver * (c.D + 2);   // split-attention partials (T <= 8)
    int Kmax = std::max(c.I, std::max(c.H, c.nH * c.D));
    size_t wsb_halves = 0;   // the MLX-layout GEMM's repacked scales: the largest projection's
    for (auto& ly : m->layers)
        for (const Lin* l : {&ly.q, &ly.k, &ly.v, &ly.o, &ly.gate, &ly.up, &ly.down}) wsb_halves = std::max(wsb_halves, qgemm_scale_halves(l->O, l->K, l->gs));
    wsb_halves = std::max(wsb_halves, qgemm_scale_halves(m->head.O, m->head.K, m->head.gs));
    int rc;
    if ((rc = dalloc(m, &m->hist, seq + 1)) || (rc = dalloc(m, &m->status, seq + 1)) || (rc = dalloc(m, &m->rng, 2)) ||
        (rc = dalloc(m, &m->dpos, 64)) || (rc = dalloc(m, &m->h, (size_t)B * H)) || (rc = dalloc(m, &m->xn, (size_t)B * H)) ||
        (rc = dalloc(m, &m->tmp, (size_t)B * H)) || (rc = dalloc(m, &m->qkv, (size_t)B * m->qkv_cols)) ||
        (rc = dalloc(m, &m->attn, (size_t)B * c.nH * c.D)) || (rc = dalloc(m, &m->gu, (size_t)B * 2 * I)) ||
        (rc = dalloc(m, &m->mlp, (size_t)B * I)) || (rc = dalloc(m, &m->logits, (size_t)8 * V)) || (rc = dalloc(m, &m->dmv_split, dpack_mv_split_floats(H))) ||
        (rc = dalloc(m, &m->part, partFloats)) || (rc = dalloc(m, &m->qsplit, QGEMM_SPLIT_FLOATS)) || (rc = dalloc(m, &m->bmax, (V + 255) / 256)) ||
        (rc = dalloc(m, &m->barg, (V + 255) / 256)) || (rc = dalloc(m, &m->xbf, (size_t)B * Kmax)) || (rc = dalloc(m, &m->xsc, (size_t)B)) || (rc = dalloc(m, &m->diag, 8)) ||
        (rc = dalloc(m, &m->xlo, (size_t)B * Kmax)) || (rc = dalloc(m, &m->xgs, qgemm_gsum_floats(B, Kmax, 32))) || (rc = dalloc(m, &m->xnz, (size_t)B)) || (rc = dalloc(m, &m->wsb, wsb_halves)))
        return fail(rc);
    HIPCHECK(hipMemset(m->hist, 0, (seq + 1) * 4));
    HIPCHECK(hipMemset(m->dmv_split, 0, dpack_mv_split_floats(H) * 4));   // the split matvec's tile counters
    HIPCHECK(hipMemset(m->status, 0, (seq + 1) * 4));
    HIPCHECK(hipMemset(m->qsplit, 0, QGEMM_SPLIT_FLOATS * 4));
    HIPCHECK(hipMemset(m->dpos, 0, 64 * 4));
    // sparse index (Transformer.swift:1009-1063)
    if (sparse) {
        m->sparse = *sparse; sparse_clamp(m->sparse);
        if (seq < m->sparse.min_context)
            m->sparse_off = "the context length (" + std::to_string(seq) + ") is below " + std::to_string(m->sparse.min_context) +
                            " tokens, where it starts";
        if (seq >= m->sparse.min_context) {
            m->sparse_alloc = true; m->sparse_on = true;
            m->sp_max_blocks = seq / 4;
            for (auto& ly : m->layers) if ((rc = dalloc(m, &ly.idx, (size_t)m->sp_max_blocks * c.nKV * c.D))) return fail(rc);
            if ((rc = dalloc(m, &m->sp_scores, (size_t)c.nKV * m->sp_max_blocks)) || (rc = dalloc(m, &m->sp_lists, (size_t)c.nKV * seq)) ||
                (rc = dalloc(m, &m->sp_plan, 16)))
                return fail(rc);
        }
    }
    // host staging
    HIPCHECK(hipHostMalloc((void**)&m->h_tokens, (size_t)B * 4, 0));
    HIPCHECK(hipHostMalloc((void**)&m->h_pos, 64 * 4, 0));
    HIPCHECK(hipHostMalloc((void**)&m->h_logits, (size_t)8 * V * 4, 0));
    HIPCHECK(hipHostMalloc((void**)&m->ring_tok, Model::RING * 4, hipHostMallocMapped));
    HIPCHECK(hipHostMalloc((void**)&m->ring_status, Model::RING * 4, hipHostMallocMapped));
    HIPCHECK(hipHostGetDevicePointer((void**)&m->ring_tok_dev, m->ring_tok, 0));
    HIPCHECK(hipHostGetDevicePointer((void**)&m->ring_status_dev, m->ring_status, 0));
    HIPCHECK(hipHostMalloc((void**)&m->abort_host, 64, hipHostMallocMapped));
    HIPCHECK(hipHostGetDevicePointer((void**)&m->abort_host_dev, m->abort_host, 0));
    *m->abort_host = 0;
    for (auto& s : m->slots) { HIPCHECK(hipEventCreate(&s.start)); HIPCHECK(hipEventCreate(&s.stop)); }
    if ((rc = model_seed(m, 0))) return fail(rc);
    if ((rc = tiles_setup(m)) || (rc = mega_setup(m))) return fail(rc);
    *out = m;
    return MLXR_OK;
}

// ----------------------------------------------------------------------------- encoding
namespace {

QmvArgs qmv_args(const Lin* parts, int n, const float* x, const float* norm_w, float eps, float* y, int epi) {
    QmvArgs a;
    a.nparts = n;
    int O = 0;
    for (int i = 0; i < n; i++) { a.part[i] = parts[i].m; O += parts[i].O; }
    a.K = parts[0].K; a.bits = parts[0].bits; a.gs = parts[0].gs; a.st = parts[0].st;
    a.O = epi == EPI_GATED ? parts[0].O : O;
    a.x = x; a.norm_w = norm_w; a.eps = eps; a.y = y; a.epi = epi;
    return a;
}

// Writes `value` into *dpos through the stream (pinned ring slot, no allocation).
int set_dpos(Model* m, int value) {
    if (m->dev_pos_known == value) return MLXR_OK;
    int* slot = m->h_pos + (m->h_pos_i++ & 63);
    *slot = value;
    HIPCHECK(hipMemcpyAsync(m->dpos, slot, 4, hipMemcpyHostToDevice, m->stream));
    m->dev_pos_known = value;
    return MLXR_OK;
}

// Projection over T tokens: decode matvec (T == 1), small batch (T <= 8) or MFMA GEMM.
int project(Model* m, const Lin* parts, int n, const float* x, int xs, float* y, int ys, int T) {
    hipStream_t s = m->stream;
    if (T == 1) {
        QmvArgs a = qmv_args(parts, n, x, nullptr, 0, y, EPI_STORE);
        HIPCHECK(launch_qmv(a, s));
        return MLXR_OK;
    }
    if (T <= 8) {
        QmmSmallArgs a; a.nparts = n; int O = 0;
        for (int i = 0; i < n; i++) { a.part[i] = parts[i].m; O += parts[i].O; }
        a.K = parts[0].K; a.bits = parts[0].bits; a.gs = parts[0].gs; a.st = parts[0].st; a.O = O; a.T = T;
        a.x = x; a.x_stride = xs; a.y = y; a.y_stride = ys;
        a.xbf = m->xbf; a.xlo = m->xlo; a.xgs = m->xgs; a.xsc = m->xsc; a.xnz = m->xnz;
        HIPCHECK(launch_qmm_small(a, s));
        return MLXR_OK;
    }
    int col = 0;
    for (int i = 0; i < n; i++) {
        QGemmArgs g; g.m = parts[i].m; g.K = parts[i].K; g.bits = parts[i].bits; g.gs = parts[i].gs; g.st = parts[i].st;
        g.O = parts[i].O; g.T = T; g.x = x; g.x_stride = xs; g.y = y + col; g.y_stride = ys; g.xbf = m->xbf; g.xsc = m->xsc;
        g.xlo = m->xlo; g.xgs = m->xgs; g.xnz = m->xnz; g.wsb = m->wsb;
        g.split = m->qsplit; g.split_floats = QGEMM_SPLIT_FLOATS;
        g.x_ready = i > 0 && parts[i].K == parts[0].K && parts[i].bits == parts[0].bits && parts[i].gs == parts[0].gs;
        HIPCHECK(launch_qgemm(g, s));
        col += parts[i].O;
    }
    return MLXR_OK;
}

int encode_sample(Model* m, int V, const mlxr_sample_params* sp, bool advance) {
    SampleArgs a;
    a.logits = m->logits; a.V = V; a.hist = m->hist; a.status = m->status; a.rng = m->rng;
    a.bmax = m->bmax; a.barg = m->barg; a.dpos = m->dpos; a.dpos_next = advance ? m->dpos : nullptr;
    a.window = sp->window; a.top_k = sp->top_k; a.penalty = sp->penalty; a.temperature = sp->temperature;
    a.top_p = sp->top_p; a.min_p = sp->min_p; a.diag = m->diag;
    a.host_tok = m->ring_tok_dev; a.host_status = m->ring_status_dev; a.ring_mask = Model::RING - 1;
    HIPCHECK(launch_sample(a, m->stream));
    return MLXR_OK;
}

// One decode step (T == 1) at position *dpos: the token is read from hist[*dpos]. With `sp`, the
// token is selected into hist[*dpos + 1] and *dpos advanced (graph-replayable: nothing here
// depends on the position on the host).
int encode_decode(Model* m, const mlxr_sample_params* sp, bool sparse, bool logits) {
    const Config& c = m->cfg;
    hipStream_t s = m->stream;
    HIPCHECK(launch_qembed(m->embed.m, c.H, m->embed.bits, m->embed.gs, m->embed.st, m->hist, m->dpos, 1, m->h, s));
    if (sparse) {
        SparseArgs sa; sa.dpos = m->dpos; sa.top_k = m->sparse.top_k; sa.window = m->sparse.window; sa.sink = m->sparse.sink;
        sa.min_context = m->sparse.min_context; sa.dplan = m->sp_plan;
        HIPCHECK(launch_sparse_plan(sa, s));
    }
    // projections over the repacked tiles where the model has them (decode mode 2: the MLX layout)
    const bool dmv = m->decode_mode != 2 && (int)m->tile_layers.size() == c.L;
    for (int li = 0; li < c.L; li++) {
        Layer& ly = m->layers[li];
        const LayerDev* tl = dmv ? &m->tile_layers[li] : nullptr;
        const Lin qkvp[3] = {ly.q, ly.k, ly.v};
        if (tl) HIPCHECK(launch_dpack_mv(tl->qkv, m->h, ly.in_norm, c.eps, m->qkv, 0, s));
        else HIPCHECK(launch_qmv(qmv_args(qkvp, 3, m->h, ly.in_norm, c.eps, m->qkv, EPI_STORE), s));
        QkvPostArgs pa; pa.qkv = m->qkv; pa.row_stride = m->qkv_cols; pa.inv_freq = m->inv_freq; pa.kc = ly.kc; pa.vc = ly.vc;
        pa.pt = m->page_table; pa.qn = ly.q_norm; pa.kn = ly.k_norm; pa.D = c.D; pa.nH = c.nH; pa.nKV = c.nKV;
        pa.rot_dim = c.rot_dim; pa.traditional = c.traditional; pa.T = 1; pa.dpos = m->dpos; pa.eps = c.eps;
        pa.idx = m->sparse_alloc ? ly.idx : nullptr;   // the index row of a block this step completes
        HIPCHECK(launch_qkv_post(pa, s));
        AttnArgs aa; aa.q = m->qkv; aa.q_stride = m->qkv_cols; aa.kc = ly.kc; aa.vc = ly.vc; aa.pt = m->page_table;
        aa.out = m->attn; aa.out_stride = c.nH * c.D; aa.part = m->part; aa.D = c.D; aa.nH = c.nH; aa.nKV = c.nKV; aa.T = 1;
        aa.nsplit = m->nsplit_dec; aa.dpos = m->dpos; aa.scale = c.query_scale * c.rope_attention_factor * c.rope_attention_factor;
        if (sparse) {
            SparseArgs sa; sa.kc = ly.kc; sa.pt = m->page_table; sa.idx = ly.idx; sa.q = m->qkv; sa.scores = m->sp_scores;
            sa.lists = m->sp_lists; sa.list_stride = m->sparse.per_head ? m->max_seq : 0; sa.nKV = c.nKV; sa.nH = c.nH; sa.D = c.D;
            sa.rows = m->sparse.per_head ? c.nKV : 1; sa.dpos = m->dpos; sa.max_blocks = m->sp_max_blocks; sa.dplan = m->sp_plan;
            HIPCHECK(launch_sparse_score(sa, s));
            HIPCHECK(launch_sparse_select(sa, s));
            aa.lists = m->sp_lists; aa.list_stride = sa.list_stride; aa.splan = m->sp_plan;
        }
        HIPCHECK(launch_attn_decode(aa, s));
        const Lin gup[2] = {ly.gate, ly.up};
        if (tl) {
            HIPCHECK(launch_dpack_mv(tl->o, m->attn, nullptr, 0, m->h, 1, s));
            HIPCHECK(launch_dpack_mv(tl->gu, m->h, ly.post_norm, c.eps, m->mlp, 2, s));
            HIPCHECK(launch_dpack_mv(tl->down, m->mlp, nullptr, 0, m->h, 1, s, m->dmv_split));
        } else {
            HIPCHECK(launch_qmv(qmv_args(&ly.o, 1, m->attn, nullptr, 0, m->h, EPI_ADD), s));
            HIPCHECK(launch_qmv(qmv_args(gup, 2, m->h, ly.post_norm, c.eps, m->mlp, EPI_GATED), s));
            HIPCHECK(launch_qmv(qmv_args(&ly.down, 1, m->mlp, nullptr, 0, m->h, EPI_ADD), s));
        }
    }
    if (logits || sp) {
        if (dmv && m->tile_head.code) HIPCHECK(launch_dpack_mv(m->tile_head, m->h, m->final_norm, c.eps, m->logits, 0, s));
        else HIPCHECK(launch_qmv(qmv_args(&m->head, 1, m->h, m->final_norm, c.eps, m->logits, EPI_STORE), s));
    }
    if (sp) return encode_sample(m, c.V, sp, true);
    return MLXR_OK;
}

// A batch of T tokens (2..max_batch) at positions *dpos .. *dpos + T - 1 (prefill chunk / verify).
// all_logits: logits of every row ([T][V], T <= 8); else of the last row only.
// Prefill GEMM over a repacked phase: the f16 pre-pass of x (x == nullptr: the fused norm already
// wrote m->xbf / m->xsc), then the tile GEMM.
int project_tiles(Model* m, const MvPhaseDesc& p, const float* x, int xs, float* y, int ys, int T) {
    if (x) HIPCHECK(launch_x_to_f16(x, xs, p.K, T, m->xbf, m->xsc, m->stream));
    HIPCHECK(launch_tile_gemm(p, m->xbf, m->xsc, T, y, ys, m->stream));
    return MLXR_OK;
}

// Attention of a batch's T queries (positions *dpos .. *dpos + T - 1) after their q|k|v: QK norms,
// RoPE and the cache write, then flash attention (prefill chunks) or the split attention (verify
// batches, T <= 8).
int attend(Model* m, int li, int T) {
    const Config& c = m->cfg;
    hipStream_t s = m->stream;
    Layer& ly = m->layers[li];
    QkvPostArgs pa; pa.qkv = m->qkv; pa.row_stride = m->qkv_cols; pa.inv_freq = m->inv_freq; pa.kc = ly.kc; pa.vc = ly.vc;
    pa.pt = m->page_table; pa.qn = ly.q_norm; pa.kn = ly.k_norm; pa.D = c.D; pa.nH = c.nH; pa.nKV = c.nKV;
    pa.rot_dim = c.rot_dim; pa.traditional = c.traditional; pa.T = T; pa.dpos = m->dpos; pa.eps = c.eps;
    HIPCHECK(launch_qkv_post(pa, s));
    if (m->sparse_alloc) HIPCHECK(launch_sparse_index(ly.kc, m->page_table, ly.idx, c.nKV, c.D, m->dpos, 0, T, s));
    const float scale = c.query_scale * c.rope_attention_factor * c.rope_attention_factor;
    if (T > 8) {   // prefill chunk: flash attention on the matrix cores
        FlashArgs fa; fa.q = m->qkv; fa.q_stride = m->qkv_cols; fa.kc = ly.kc; fa.vc = ly.vc; fa.pt = m->page_table;
        fa.out = m->attn; fa.out_stride = c.nH * c.D; fa.D = c.D; fa.nH = c.nH; fa.nKV = c.nKV; fa.T = T;
        fa.dpos = m->dpos; fa.scale = scale;
        HIPCHECK(launch_flash_prefill(fa, s));
    } else {       // verify batch: every query of a KV head in one pass over each key range
        AttnArgs aa; aa.q = m->qkv; aa.q_stride = m->qkv_cols; aa.kc = ly.kc; aa.vc = ly.vc; aa.pt = m->page_table;
        aa.out = m->attn; aa.out_stride = c.nH * c.D; aa.part = m->part; aa.D = c.D; aa.nH = c.nH; aa.nKV = c.nKV; aa.T = T;
        aa.nsplit = T > 1 ? m->nsplit_ver : m->nsplit_dec; aa.dpos = m->dpos; aa.scale = scale;
        aa.cap = (m->max_seq + aa.nsplit - 1) / aa.nsplit;   // positions stay below the context length
        HIPCHECK(T > 1 ? launch_attn_verify(aa, s) : launch_attn_decode(aa, s));
    }
    return MLXR_OK;
}

// A verify batch (T <= 8) over the repacked tiles: every projection is one small-batch launch with
// the tokens in the matrix cores' columns, the RMSNorms fused into the launches that read the
// residual stream and the residual adds into the ones that write it (o_proj, down: h += W x).
int encode_verify(Model* m, int T, bool want_logits, bool all_logits) {
    const Config& c = m->cfg;
    hipStream_t s = m->stream;
    const int H = c.H, I = c.I;
    auto mm = [&](const MvPhaseDesc& p, const float* x, int xs, const float* nw, float* y, int ys, bool acc, int n) {
        return launch_dpack_mm(p, x, xs, nw, c.eps, y, ys, acc, n, m->mm_split, m->mm_split_floats, s);
    };
    for (int li = 0; li < c.L; li++) {
        const Layer& ly = m->layers[li];
        const LayerDev& d = m->tile_layers[li];
        HIPCHECK(mm(d.qkv, m->h, H, ly.in_norm, m->qkv, m->qkv_cols, false, T));
        if (int rc = attend(m, li, T)) return rc;
        HIPCHECK(mm(d.o, m->attn, c.nH * c.D, nullptr, m->h, H, true, T));
        HIPCHECK(mm(d.gu, m->h, H, ly.post_norm, m->mlp, I, false, T));   // SiLU(gate) * up
        HIPCHECK(mm(d.down, m->mlp, I, nullptr, m->h, H, true, T));
    }
    if (!want_logits) return MLXR_OK;
    const int r0 = all_logits ? 0 : T - 1, n = all_logits ? T : 1;
    if (m->tile_head.code) {
        HIPCHECK(mm(m->tile_head, m->h + (size_t)r0 * H, H, m->final_norm, m->logits, c.V, false, n));
        return MLXR_OK;
    }
    HIPCHECK(launch_rms_norm(m->h, m->xn, m->final_norm, H, T, H, c.eps, s));
    for (int t = 0; t < n; t++)
        HIPCHECK(launch_qmv(qmv_args(&m->head, 1, m->xn + (size_t)(r0 + t) * H, nullptr, 0, m->logits + (size_t)t * c.V, EPI_STORE), s));
    return MLXR_OK;
}

int encode_batch(Model* m, int T, bool want_logits, bool all_logits) {
    const Config& c = m->cfg;
    hipStream_t s = m->stream;
    const int H = c.H, I = c.I;
    // prefill chunks on the repacked tiles when the model has them (fused q|k|v and gate|up, SiLU
    // in the gate|up epilogue); verify batches (T <= 8) run the tiles' small-batch matvec (tokens in
    // the matrix cores' columns), else the MLX-layout small-batch kernels
    const bool tiles = T > 8 && (int)m->tile_layers.size() == c.L;
    const bool small_tiles = T <= 8 && (int)m->tile_layers.size() == c.L && m->decode_mode != 2;
    HIPCHECK(launch_qembed(m->embed.m, H, m->embed.bits, m->embed.gs, m->embed.st, m->hist, m->dpos, T, m->h, s));
    if (small_tiles) return encode_verify(m, T, want_logits, all_logits);
    if (tiles) HIPCHECK(launch_rms_norm_f16(m->h, m->layers[0].in_norm, H, T, H, c.eps, m->xbf, m->xsc, s));
    else HIPCHECK(launch_rms_norm(m->h, m->xn, m->layers[0].in_norm, H, T, H, c.eps, s));
    for (int li = 0; li < c.L; li++) {
        Layer& ly = m->layers[li];
        const Lin qkvp[3] = {ly.q, ly.k, ly.v};
        const LayerDev* tl = tiles ? &m->tile_layers[li] : nullptr;
        if (int rc = tl ? project_tiles(m, tl->qkv, nullptr, H, m->qkv, m->qkv_cols, T)
                        : project(m, qkvp, 3, m->xn, H, m->qkv, m->qkv_cols, T)) return rc;
        if (int rc = attend(m, li, T)) return rc;
        if (int rc = tl ? project_tiles(m, tl->o, m->attn, c.nH * c.D, m->tmp, H, T)
                        : project(m, &ly.o, 1, m->attn, c.nH * c.D, m->tmp, H, T)) return rc;
        if (tl) {
            HIPCHECK(launch_add_rms_norm_f16(m->h, m->tmp, ly.post_norm, H, T, c.eps, m->xbf, m->xsc, s));
            if (int rc = project_tiles(m, tl->gu, nullptr, H, m->mlp, I, T)) return rc;
        } else {
            HIPCHECK(launch_add_rms_norm(m->h, m->tmp, m->xn, ly.post_norm, H, T, c.eps, s));
            const Lin gup[2] = {ly.gate, ly.up};
            if (int rc = project(m, gup, 2, m->xn, H, m->gu, 2 * I, T)) return rc;
            HIPCHECK(launch_silu_mul(m->gu, m->mlp, I, T, s));
        }
        if (int rc = tl ? project_tiles(m, tl->down, m->mlp, I, m->tmp, H, T)
                        : project(m, &ly.down, 1, m->mlp, I, m->tmp, H, T)) return rc;
        const bool last = li + 1 == c.L;
        if (last && !want_logits) continue;
        if (tl && !last) HIPCHECK(launch_add_rms_norm_f16(m->h, m->tmp, m->layers[li + 1].in_norm, H, T, c.eps, m->xbf, m->xsc, s));
        else HIPCHECK(launch_add_rms_norm(m->h, m->tmp, m->xn, last ? m->final_norm : m->layers[li + 1].in_norm, H, T, c.eps, s));
    }
    if (!want_logits) return MLXR_OK;
    if (all_logits) {
        for (int t = 0; t < T; t++)
            HIPCHECK(launch_qmv(qmv_args(&m->head, 1, m->xn + (size_t)t * H, nullptr, 0, m->logits + (size_t)t * c.V, EPI_STORE), s));
    } else {
        HIPCHECK(launch_qmv(qmv_args(&m->head, 1, m->xn + (size_t)(T - 1) * H, nullptr, 0, m->logits, EPI_STORE), s));
    }
    return MLXR_OK;
}

int write_tokens(Model* m, const int32_t* tokens, int n, int at) {
    memcpy(m->h_tokens, tokens, (size_t)n * 4);
    HIPCHECK(hipMemcpyAsync(m->hist + at, m->h_tokens, (size_t)n * 4, hipMemcpyHostToDevice, m->stream));
    return MLXR_OK;
}

int check_tokens(Model* m, const int32_t* tokens, int n) {
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->embed.O)
            return set_error(MLXR_E_INVALID_FILE, "token id outside the embedding table (" + std::to_string(m->embed.O) + " rows)");
    return MLXR_OK;
}

int sync_stream(Model* m) {
    hipError_t e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return set_error(MLXR_E_GPU, std::string("GPU error: ") + hipGetErrorString(e));
    return MLXR_OK;
}

// Runs one chunk of n tokens at `at` (eager launches); the caller synchronises.
int run_chunk(Model* m, const int32_t* toks, int n, int at, bool logits, bool all_logits, bool dense) {
    if (int rc = set_dpos(m, at)) return rc;
    if (int rc = write_tokens(m, toks, n, at)) return rc;
    HIPCHECK(hipEventRecord(m->slots[0].start, m->stream));
    int rc = n == 1 ? encode_decode(m, nullptr, !dense && m->sparse_on, logits) : encode_batch(m, n, logits, all_logits);
    if (rc) return rc;
    HIPCHECK(hipEventRecord(m->slots[0].stop, m->stream));
    m->written_high = std::max(m->written_high, at + n);
    return MLXR_OK;
}

void record_gpu_time(Model* m, const Model::StepSlot& s) {
    float ms = 0;
    if (hipEventElapsedTime(&ms, s.start, s.stop) == hipSuccess) m->last_gpu_time = ms * 1e-3;
}
}  // namespace

static bool sparse_plan_valid(const mlxr_sparse_cfg& c, int position);

int model_forward(Model* m, const int32_t* tokens, int n, int offset, bool all_logits, bool dense, const float** out, Cancel cancel) {
    if (n <= 0 || !tokens) return set_error(MLXR_E_INVALID_ARG, "no tokens");
    if (all_logits && n > 8) return set_error(MLXR_E_INVALID_OUTPUT, "verify batch too large");
    if (offset < 0 || offset + n > m->max_seq) return set_error(MLXR_E_CONTEXT_FULL, "The context window is full.");
    if (int rc = check_tokens(m, tokens, n)) return rc;
    // one token whose step the persistent kernel takes (the decode loop's own step: speculative
    // decoding's steps without a draft): the token goes into the history and one persistent step runs
    // without token selection (select = 0: it writes neither hist[offset + 1] nor the ring and leaves
    // *dpos at offset, as the reference's forward leaves them); its logits are returned
    bool idle = true;
    for (auto& s : m->slots) idle = idle && !s.busy;
    if (n == 1 && idle && offset + 1 < m->max_seq && m->mega_ok && m->decode_mode == 1 &&
        !(m->sparse_on && sparse_plan_valid(m->sparse, offset))) {
        if (int rc = write_tokens(m, tokens, 1, offset)) return rc;
        if (int rc = set_dpos(m, offset)) return rc;
        HIPCHECK(hipEventRecord(m->slots[0].start, m->stream));
        MegaArgs a = m->mega;
        a.select = 0;
        HIPCHECK(launch_decode_step(a, m->mega_nwg, m->mega_lds, m->stream));
        if (m->sparse_alloc && (offset + 1) % 4 == 0)   // the sparse index row of the block this token completes
            for (auto& ly : m->layers)
                HIPCHECK(launch_sparse_index(ly.kc, m->page_table, ly.idx, m->cfg.nKV, m->cfg.D, m->dpos, 0, 1, m->stream));
        HIPCHECK(hipEventRecord(m->slots[0].stop, m->stream));
        m->written_high = std::max(m->written_high, offset + 1);
        if (int rc = sync_stream(m)) return rc;
        record_gpu_time(m, m->slots[0]);
        if (*(volatile int*)m->abort_host) {
            // a bounded wait expired: clear the flags and use the kernel-per-op step from now on
            HIPCHECK(hipMemsetAsync(&m->mega.sync->abort, 0, sizeof(unsigned), m->stream));
            HIPCHECK(hipMemsetAsync(m->mega.head_done, 0, sizeof(unsigned), m->stream));
            HIPCHECK(hipStreamSynchronize(m->stream));
            *(volatile int*)m->abort_host = 0;
            m->mega_ok = false;
            m->mega_reason = "a persistent step's bounded wait expired";
            return set_error(MLXR_E_GPU, "persistent decode step: a bounded wait expired (step result discarded)");
        }
        HIPCHECK(hipMemcpy(m->h_logits, m->logits, (size_t)m->cfg.V * 4, hipMemcpyDeviceToHost));
        *out = m->h_logits;
        return MLXR_OK;
    }
    for (int start = 0; start < n;) {
        if (start > 0 && cancel.requested()) return set_error(MLXR_E_CANCELLED, "cancelled");   // Transformer.swift:1127
        const int k = std::min(m->max_batch, n - start);
        const bool last = start + k == n;
        if (int rc = run_chunk(m, tokens + start, k, offset + start, last, last && all_logits, dense || n > 1)) return rc;
        if (int rc = sync_stream(m)) return rc;
        record_gpu_time(m, m->slots[0]);
        start += k;
    }
    const int V = m->cfg.V, rows = all_logits ? n : 1;
    HIPCHECK(hipMemcpy(m->h_logits, m->logits, (size_t)rows * V * 4, hipMemcpyDeviceToHost));
    *out = m->h_logits;
    return MLXR_OK;
}

static int check_sample(const mlxr_sample_params* sp) {
    if (!sp) return set_error(MLXR_E_INVALID_ARG, "sample params");
    if (!(sp->temperature >= 0) || !(sp->penalty > 0) || !(sp->top_p > 0 && sp->top_p <= 1) || !(sp->min_p >= 0 && sp->min_p <= 1) ||
        sp->top_k < 0 || sp->window < 0)
        return set_error(MLXR_E_INVALID_ARG, "sampling parameters out of range");
    return MLXR_OK;
}

static int read_ring(Model* m, int pos, int32_t* tok) {
    const int st = ((volatile int*)m->ring_status)[pos & (Model::RING - 1)];
    const int t = ((volatile int*)m->ring_tok)[pos & (Model::RING - 1)];
    if (st != 0) return set_error(MLXR_E_INVALID_OUTPUT, "non-finite logits");
    if (t < 0 || t >= m->embed.O) return set_error(MLXR_E_INVALID_OUTPUT, "sampled token " + std::to_string(t) + " outside the vocabulary");
    *tok = t;
    return MLXR_OK;
}

int model_prefill(Model* m, const int32_t* tokens, int n, int offset, const mlxr_sample_params* sp, int32_t* tok, Cancel cancel) {
    if (n <= 0 || !tokens || offset < 0 || offset + n >= m->max_seq) return set_error(MLXR_E_CONTEXT_FULL, "The context window is full.");
    if (int rc = check_sample(sp)) return rc;
    if (int rc = check_tokens(m, tokens, n)) return rc;
    for (int start = 0; start < n;) {
        if (start > 0 && cancel.requested()) return set_error(MLXR_E_CANCELLED, "cancelled");   // Transformer.swift:1233
        const int k = std::min(m->max_batch, n - start);
        const bool last = start + k == n;
        const int at = offset + start;
        if (int rc = run_chunk(m, tokens + start, k, at, last, false, true)) return rc;
        if (last) {
            if (k > 1) { if (int rc = set_dpos(m, at + k - 1)) return rc; }
            const int V = std::min(sp->V > 0 ? (int)sp->V : m->cfg.V, m->cfg.V);
            if (int rc = encode_sample(m, V, sp, true)) return rc;
            m->dev_pos_known = at + k;
            HIPCHECK(hipEventRecord(m->slots[0].stop, m->stream));
        }
        if (int rc = sync_stream(m)) return rc;
        record_gpu_time(m, m->slots[0]);
        start += k;
    }
    return read_ring(m, offset + n, tok);
}

int model_step_logits(Model* m, const float** out) {
    for (auto& s : m->slots)
        if (s.busy) return set_error(MLXR_E_INVALID_ARG, "a decode step is in flight");
    HIPCHECK(hipStreamSynchronize(m->stream));
    HIPCHECK(hipMemcpy(m->h_logits, m->logits, (size_t)m->cfg.V * 4, hipMemcpyDeviceToHost));
    *out = m->h_logits;
    return MLXR_OK;
}

// SparseAttention.plan(position:) != nil (SparseAttention.swift:80-94), on the host.
static bool sparse_plan_valid(const mlxr_sparse_cfg& c, int position) {
    const int pool = 4, L = position + 1;
    if (position < 0 || L < c.min_context) return false;
    const int sinkEnd = (c.sink + pool - 1) / pool * pool;
    if (!(L - c.window > sinkEnd)) return false;
    const int winStart = (L - c.window) / pool * pool;
    return winStart / pool - sinkEnd / pool > 0;
}

int model_begin_decode(Model* m, int offset, const mlxr_sample_params* sp, mlxr_step* out) {
    if (offset < 0 || offset + 1 >= m->max_seq) return set_error(MLXR_E_CONTEXT_FULL, "The context window is full.");
    if (int rc = check_sample(sp)) return rc;
    int busy = 0;
    for (auto& s : m->slots) busy += s.busy;
    if (busy >= 2) return set_error(MLXR_E_INVALID_ARG, "at most two decode steps may be in flight");
    Model::StepSlot& slot = m->slots[m->next_slot];
    if (slot.busy) return set_error(MLXR_E_INVALID_ARG, "decode steps must be finished in order");
    if (int rc = set_dpos(m, offset)) return rc;
    HIPCHECK(hipEventRecord(slot.start, m->stream));
    const bool sparse = m->sparse_on;
    const bool sparse_step = sparse && sparse_plan_valid(m->sparse, offset);
    if (m->mega_ok && m->decode_mode == 1 && !sparse_step) {
        const bool greedy = sp->temperature <= 0.001f && sp->penalty == 1.0f;
        MegaArgs a = m->mega;
        a.select = greedy ? 1 : 0;
        if (m->stall_next) {   // test hook: this step's first wait expires after a few polls
            a.stall = 1; a.spin_limit = 4096;
            m->stall_next = false;
        }
        HIPCHECK(launch_decode_step(a, m->mega_nwg, m->mega_lds, m->stream));
        if (!greedy) {
            const int V = std::min(sp->V > 0 ? (int)sp->V : m->cfg.V, m->cfg.V);
            if (int rc = encode_sample(m, V, sp, true)) return rc;
        }
        if (m->sparse_alloc && (offset + 1) % 4 == 0)   // keep the sparse index of completed blocks
            for (auto& ly : m->layers)
                HIPCHECK(launch_sparse_index(ly.kc, m->page_table, ly.idx, m->cfg.nKV, m->cfg.D, m->dpos, -1, 1, m->stream));
    } else if (m->use_graphs) {
        Model::GraphKey key{sp->window, sp->top_k, sparse ? 1 : 0, sp->penalty, sp->temperature, sp->top_p, sp->min_p};
        auto it = m->graphs.find(key);
        if (it == m->graphs.end()) {
            mlxr_sample_params p = *sp;
            HIPCHECK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
            int rc = encode_decode(m, &p, sparse, true);
            hipGraph_t g = nullptr;
            hipError_t e = hipStreamEndCapture(m->stream, &g);
            if (rc) { if (g) hipGraphDestroy(g); return rc; }
            if (e != hipSuccess) return set_error(MLXR_E_GPU, std::string("graph capture: ") + hipGetErrorString(e));
            hipGraphExec_t ex = nullptr;
            if (hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) != hipSuccess) { hipGraphDestroy(g); return set_error(MLXR_E_GPU, "graph instantiate"); }
            m->graph_defs.push_back(g);
            it = m->graphs.emplace(key, ex).first;
        }
        HIPCHECK(hipGraphLaunch(it->second, m->stream));
    } else {
        if (int rc = encode_decode(m, sp, sparse, true)) return rc;
    }
    HIPCHECK(hipEventRecord(slot.stop, m->stream));
    m->dev_pos_known = offset + 1;
    slot.busy = true; slot.offset = offset;
    out->id = m->next_slot; out->offset = offset;
    m->next_slot = (m->next_slot + 1) % 4;
    m->written_high = std::max(m->written_high, offset + 1);
    return MLXR_OK;
}

int model_finish(Model* m, const mlxr_step* st, int32_t* tok) {
    if (!st || st->id < 0 || st->id >= 4) return set_error(MLXR_E_INVALID_ARG, "bad step");
    Model::StepSlot& slot = m->slots[st->id];
    if (!slot.busy || slot.offset != st->offset) return set_error(MLXR_E_INVALID_ARG, "step is not in flight");
    hipError_t e = hipEventSynchronize(slot.stop);
    slot.busy = false;
    if (e != hipSuccess) return set_error(MLXR_E_GPU, std::string("GPU error: ") + hipGetErrorString(e));
    record_gpu_time(m, slot);
    if (slot.failed) {
        slot.failed = false;
        return set_error(MLXR_E_GPU, "decode step discarded: an earlier step in flight failed");
    }
    if (m->mega_ok && *(volatile int*)m->abort_host) {
        // A wait of the persistent step expired. Every kernel still ran to its end, but a step queued
        // behind this one ran with the abort flag raised: wait for it and fail it too.
        HIPCHECK(hipStreamSynchronize(m->stream));
        for (auto& other : m->slots)
            if (other.busy) other.failed = true;
        // clear the device abort flag (the launch counter keeps counting, so no later tag can match a
        // stale value) and the argmax counter, on the model stream; then fall back to the
        // kernel-per-op step for good
        HIPCHECK(hipMemsetAsync(&m->mega.sync->abort, 0, sizeof(unsigned), m->stream));
        HIPCHECK(hipMemsetAsync(m->mega.head_done, 0, sizeof(unsigned), m->stream));
        HIPCHECK(hipStreamSynchronize(m->stream));
        *(volatile int*)m->abort_host = 0;
        m->mega_ok = false;
        m->mega_reason = "a persistent step's bounded wait expired";
        m->dev_pos_known = -1;   // the failed steps advanced *dpos; the next step writes it again
        return set_error(MLXR_E_GPU, "persistent decode step: a bounded wait expired (step result discarded)");
    }
    return read_ring(m, st->offset + 1, tok);
}

// beginSteps (Transformer.swift:1265-1296): tokens[0 .. n) go to positions offset .. offset + n - 1
// and one step is committed over them whose token (at offset + n) is selected on the GPU, without
// waiting: the first n - 1 tokens run as one pass without logits (the small-batch matvecs, or the
// prefill GEMMs past 8 tokens), the last as a decode step. Nothing may be in flight; the returned
// step counts as one for the in-flight limit and is finished like any decode step.
int model_begin_steps(Model* m, const int32_t* tokens, int n, int offset, const mlxr_sample_params* sp, mlxr_step* out) {
    if (n <= 0 || !tokens || n > m->max_batch || offset < 0 || offset + n >= m->max_seq)
        return set_error(MLXR_E_CONTEXT_FULL, "The context window is full.");
    if (int rc = check_sample(sp)) return rc;
    if (int rc = check_tokens(m, tokens, n)) return rc;
    for (auto& s : m->slots)
        if (s.busy) return set_error(MLXR_E_INVALID_ARG, "begin_steps needs no step in flight");
    if (int rc = write_tokens(m, tokens, n, offset)) return rc;
    if (n > 1) {
        if (int rc = set_dpos(m, offset)) return rc;
        const int T = n - 1;
        if (int rc = T == 1 ? encode_decode(m, nullptr, m->sparse_on, false) : encode_batch(m, T, false, false)) return rc;
        m->dev_pos_known = -1;   // the pass leaves *dpos where it was; the step below writes it again
        m->written_high = std::max(m->written_high, offset + T);
    }
    return model_begin_decode(m, offset + n - 1, sp, out);
}

int model_stall_next_step(Model* m) {
    if (!m->mega_ok || m->decode_mode != 1) return set_error(MLXR_E_UNSUPPORTED, "the persistent decode step is not in use");
    m->stall_next = true;
    return MLXR_OK;
}

// reusablePrefix (Transformer.swift:1193-1209): every cache of this build holds the full context.
int model_reusable_prefix(Model* m, int common, int prev_len) {
    (void)prev_len;
    return std::max(0, std::min(common, m->max_seq));
}

int model_seed(Model* m, uint64_t seed) {
    uint64_t st[2];
    st[0] = seed == 0 ? 0x9E3779B97F4A7C15ull : seed;
    float hint = 8.0f; st[1] = 0; memcpy(&st[1], &hint, 4);
    HIPCHECK(hipStreamSynchronize(m->stream));
    HIPCHECK(hipMemcpy(m->rng, st, 16, hipMemcpyHostToDevice));
    return MLXR_OK;
}

int model_set_sparse(Model* m, const mlxr_sparse_cfg* cfg) {
    if (!cfg) { m->sparse_on = false; return MLXR_OK; }
    if (!m->sparse_alloc) return set_error(MLXR_E_UNSUPPORTED, "the model was not loaded with sparse attention");
    mlxr_sparse_cfg c = *cfg; sparse_clamp(c);
    m->sparse = c; m->sparse_on = true;
    for (auto& g : m->graphs) hipGraphExecDestroy(g.second);   // budgets are baked into captured graphs
    m->graphs.clear();
    return MLXR_OK;
}

int model_read_kv(Model* m, int layer, int rows, float* k, float* v) {
    const Config& c = m->cfg;
    if (layer < 0 || layer >= c.L || rows < 0 || rows > m->max_seq) return set_error(MLXR_E_INVALID_ARG, "layer / rows");
    HIPCHECK(hipStreamSynchronize(m->stream));
    const size_t blk = (size_t)c.nKV * MLXR_PAGE * c.D;
    std::vector<uint16_t> kh(blk * m->n_pages), vh(blk * m->n_pages);
    HIPCHECK(hipMemcpy(kh.data(), m->layers[layer].kc, kh.size() * 2, hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(vh.data(), m->layers[layer].vc, vh.size() * 2, hipMemcpyDeviceToHost));
    for (int h = 0; h < c.nKV; h++)
        for (int j = 0; j < rows; j++) {
            const size_t src = (((size_t)(j / MLXR_PAGE) * c.nKV + h) * MLXR_PAGE + (j % MLXR_PAGE)) * c.D;   // identity page table
            for (int d = 0; d < c.D; d++) {
                k[((size_t)h * rows + j) * c.D + d] = bf16_to_f32(kh[src + d]);
                v[((size_t)h * rows + j) * c.D + d] = bf16_to_f32(vh[src + d]);
            }
        }
    return MLXR_OK;
}

// Times one decode kernel class over the model's own weights, cycling through the layers so every
// launch streams its matrices from HBM (the whole model is far larger than the 256 MB MALL).
// Events are recorded on the model stream, around the launches only. `bytes`: algorithmic bytes
// of one launch (quantized weights + scales/biases + activations read and written).
int model_profile(Model* m, const char* kind_c, int iters, int context, double* avg_ms, int64_t* bytes) {
    const Config& c = m->cfg;
    const std::string kind = kind_c ? kind_c : "";
    if (iters < 1 || context < 1 || context > m->max_seq) return set_error(MLXR_E_INVALID_ARG, "iters / context");
    auto lin_bytes_of = [](const Lin& l) { return (int64_t)l.O * ((int64_t)l.K * l.bits / 8 + 2 * 2 * (l.K / l.gs)) + (l.m.bias ? (int64_t)l.O * 2 : 0); };
    std::function<int(int)> launch;
    int64_t b = 0;
    hipStream_t s = m->stream;
    if (kind == "qkv") {
        const Layer& l0 = m->layers[0];
        b = lin_bytes_of(l0.q) + lin_bytes_of(l0.k) + lin_bytes_of(l0.v) + (int64_t)c.H * 4 * 2 + (int64_t)m->qkv_cols * 4;
        launch = [&](int i) { const Layer& ly = m->layers[i % c.L]; const Lin p[3] = {ly.q, ly.k, ly.v};
            return (int)launch_qmv(qmv_args(p, 3, m->h, ly.in_norm, c.eps, m->qkv, EPI_STORE), s); };
    } else if (kind == "o") {
        b = lin_bytes_of(m->layers[0].o) + (int64_t)c.nH * c.D * 4 + (int64_t)c.H * 4 * 2;
        launch = [&](int i) { const Layer& ly = m->layers[i % c.L]; return (int)launch_qmv(qmv_args(&ly.o, 1, m->attn, nullptr, 0, m->tmp, EPI_ADD), s); };
    } else if (kind == "gateup") {
        const Layer& l0 = m->layers[0];
        b = lin_bytes_of(l0.gate) + lin_bytes_of(l0.up) + (int64_t)c.H * 4 * 2 + (int64_t)c.I * 4;
        launch = [&](int i) { const Layer& ly = m->layers[i % c.L]; const Lin p[2] = {ly.gate, ly.up};
            return (int)launch_qmv(qmv_args(p, 2, m->h, ly.post_norm, c.eps, m->mlp, EPI_GATED), s); };
    } else if (kind == "down") {
        b = lin_bytes_of(m->layers[0].down) + (int64_t)c.I * 4 + (int64_t)c.H * 4 * 2;
        launch = [&](int i) { const Layer& ly = m->layers[i % c.L]; return (int)launch_qmv(qmv_args(&ly.down, 1, m->mlp, nullptr, 0, m->tmp, EPI_ADD), s); };
    } else if (kind.size() > 1 && kind[0] == 't' && (kind == "tqkv" || kind == "to" || kind == "tgateup" || kind == "tdown") &&
               (int)m->tile_layers.size() == c.L) {
        // the same projections on the repacked-tile matvec of the kernel-per-op step (dpack_mv_kernel)
        const Layer& l0 = m->layers[0];
        const std::string k = kind.substr(1);
        b = k == "qkv" ? lin_bytes_of(l0.q) + lin_bytes_of(l0.k) + lin_bytes_of(l0.v) + (int64_t)c.H * 4 * 2 + (int64_t)m->qkv_cols * 4
          : k == "o" ? lin_bytes_of(l0.o) + (int64_t)c.nH * c.D * 4 + (int64_t)c.H * 4 * 2
          : k == "gateup" ? lin_bytes_of(l0.gate) + lin_bytes_of(l0.up) + (int64_t)c.H * 4 * 2 + (int64_t)c.I * 4
          : lin_bytes_of(l0.down) + (int64_t)c.I * 4 + (int64_t)c.H * 4 * 2;
        launch = [&, k](int i) {
            const LayerDev& t = m->tile_layers[i % c.L];
            const Layer& ly = m->layers[i % c.L];
            if (k == "qkv") return (int)launch_dpack_mv(t.qkv, m->h, ly.in_norm, c.eps, m->qkv, 0, s);
            if (k == "o") return (int)launch_dpack_mv(t.o, m->attn, nullptr, 0, m->tmp, 1, s);
            if (k == "gateup") return (int)launch_dpack_mv(t.gu, m->h, ly.post_norm, c.eps, m->mlp, 2, s);
            return (int)launch_dpack_mv(t.down, m->mlp, nullptr, 0, m->tmp, 1, s, m->dmv_split);
        };
    } else if (kind == "head") {
        b = lin_bytes_of(m->head) + (int64_t)c.H * 4 * 2 + (int64_t)c.V * 4;
        launch = [&](int) { return (int)launch_qmv(qmv_args(&m->head, 1, m->h, m->final_norm, c.eps, m->logits, EPI_STORE), s); };
    } else if (kind == "attn") {
        b = (int64_t)2 * c.nKV * context * c.D * 2 + (int64_t)c.nH * c.D * 4 * 2;
        if (int rc = set_dpos(m, context - 1)) return rc;
        launch = [&](int i) {
            const Layer& ly = m->layers[i % c.L];
            AttnArgs aa; aa.q = m->qkv; aa.q_stride = m->qkv_cols; aa.kc = ly.kc; aa.vc = ly.vc; aa.pt = m->page_table;
            aa.out = m->attn; aa.out_stride = c.nH * c.D; aa.part = m->part; aa.D = c.D; aa.nH = c.nH; aa.nKV = c.nKV; aa.T = 1;
            aa.nsplit = m->nsplit_dec; aa.dpos = m->dpos; aa.scale = c.query_scale;
            return (int)launch_attn_decode(aa, s);
        };
    } else if (kind == "step") {
        // the persistent decode step (one launch per token): greedy steps from position context - 1,
        // each advancing the device position; bytes = every weight byte read + K/V at the mean context
        if (!m->mega_ok) return set_error(MLXR_E_UNSUPPORTED, "persistent decode step not available: " + m->mega_reason);
        const int warm = std::min(iters, 4);
        if (context - 1 + warm + iters + 1 >= m->max_seq) return set_error(MLXR_E_CONTEXT_FULL, "context + iters");
        for (const Layer& ly : m->layers)
            for (const Lin* l : {&ly.q, &ly.k, &ly.v, &ly.o, &ly.gate, &ly.up, &ly.down}) b += lin_bytes_of(*l);
        b += lin_bytes_of(m->head) + (int64_t)c.H / 2 + 4 * (c.H / m->embed.gs);
        const double mean_ctx = context + warm + (iters - 1) / 2.0;
        b += (int64_t)(2.0 * c.L * c.nKV * mean_ctx * c.D * 2);
        if (int rc = set_dpos(m, context - 1)) return rc;
        launch = [&](int) {
            MegaArgs a = m->mega; a.select = 1;
            return (int)launch_decode_step(a, m->mega_nwg, m->mega_lds, s);
        };
        for (int i = 0; i < warm; i++) if (launch(i)) return set_error(MLXR_E_GPU, "launch");
        HIPCHECK(hipEventRecord(m->slots[0].start, s));
        for (int i = 0; i < iters; i++) if (launch(i)) return set_error(MLXR_E_GPU, "launch");
        HIPCHECK(hipEventRecord(m->slots[0].stop, s));
        HIPCHECK(hipEventSynchronize(m->slots[0].stop));
        m->dev_pos_known = context - 1 + warm + iters;
        float ms = 0;
        HIPCHECK(hipEventElapsedTime(&ms, m->slots[0].start, m->slots[0].stop));
        *avg_ms = ms / iters;
        *bytes = b;
        return MLXR_OK;
    } else {
        return set_error(MLXR_E_INVALID_ARG, "kind: qkv, o, gateup, down, head, attn, step");
    }
    for (int i = 0; i < std::min(iters, 4); i++) if (launch(i)) return set_error(MLXR_E_GPU, "launch");
    HIPCHECK(hipEventRecord(m->slots[0].start, s));
    for (int i = 0; i < iters; i++) if (launch(i)) return set_error(MLXR_E_GPU, "launch");
    HIPCHECK(hipEventRecord(m->slots[0].stop, s));
    HIPCHECK(hipEventSynchronize(m->slots[0].stop));
    float ms = 0;
    HIPCHECK(hipEventElapsedTime(&ms, m->slots[0].start, m->slots[0].stop));
    *avg_ms = ms / iters;
    *bytes = b;
    return MLXR_OK;
}

// Runs one persistent decode step at `offset` (greedy, token from hist[offset]) with per-phase
// wall-clock marks: out[e * 3 + 0..2] = mean start, mean end, max end over workgroups of event
// interval e, in microseconds from the earliest kernel start. Returns the number of intervals.
int model_phase_times(Model* m, int offset, double* out, int max_intervals) {
    if (!m->mega_ok) return set_error(MLXR_E_UNSUPPORTED, "persistent decode step not available: " + m->mega_reason);
    if (offset < 0 || offset + 1 >= m->max_seq) return set_error(MLXR_E_CONTEXT_FULL, "context");
    const int nwg = m->mega_nwg;
    unsigned long long* prof = nullptr;
    HIPCHECK(hipMalloc(&prof, (size_t)nwg * MEGA_PROF_EVENTS * 8));
    HIPCHECK(hipMemset(prof, 0, (size_t)nwg * MEGA_PROF_EVENTS * 8));
    if (int rc = set_dpos(m, offset)) { hipFree(prof); return rc; }
    MegaArgs a = m->mega; a.select = 1; a.prof = prof;
    HIPCHECK(launch_decode_step(a, nwg, m->mega_lds, m->stream));
    m->dev_pos_known = offset + 1;
    HIPCHECK(hipStreamSynchronize(m->stream));
    std::vector<unsigned long long> h((size_t)nwg * MEGA_PROF_EVENTS);
    HIPCHECK(hipMemcpy(h.data(), prof, h.size() * 8, hipMemcpyDeviceToHost));
    hipFree(prof);
    int nev = 0;
    while (nev < MEGA_PROF_EVENTS && h[nev]) nev++;
    unsigned long long t0 = ~0ull;
    for (int w = 0; w < nwg; w++) if (h[(size_t)w * MEGA_PROF_EVENTS]) t0 = std::min(t0, h[(size_t)w * MEGA_PROF_EVENTS]);
    if (max_intervals < 0) {
        for (size_t i = 0; i < h.size(); i++) out[i] = h[i] ? (double)(h[i] - t0) * 0.01 : -1.0;
        return nwg;
    }
    int n = 0;
    for (int e = 0; e + 1 < nev && n < max_intervals; e++, n++) {
        double s0 = 0, s1 = 0, mx = 0;
        for (int w = 0; w < nwg; w++) {
            const double a0 = (double)(h[(size_t)w * MEGA_PROF_EVENTS + e] - t0) * 0.01;   // 100 MHz clock
            const double a1 = (double)(h[(size_t)w * MEGA_PROF_EVENTS + e + 1] - t0) * 0.01;
            s0 += a0; s1 += a1; mx = std::max(mx, a1);
        }
        out[n * 3] = s0 / nwg; out[n * 3 + 1] = s1 / nwg; out[n * 3 + 2] = mx;
    }
    return n;
}

}  // namespace mlxr
