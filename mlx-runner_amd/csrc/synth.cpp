// Seeded synthetic MLX-format models: fp32 weights N(0, std) from a counter-seeded xorshift64
// stream per row (Box-Muller), MLX affine quantization with bf16 scale/bias, written as
// config.json + model.safetensors. Deterministic in (config, seed) and independent of the thread
// count. Norm weights are 1.0 (bf16); Qwen2 q/k/v biases are drawn N(0, std) in bf16.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>
#include <sys/stat.h>
#include "json.h"
#include "model.h"

namespace mlxr {
namespace {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
inline uint64_t xorshift64(uint64_t& s) { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return s; }

// Row `row` of tensor `tid`: K normal values (K even).
void gen_row(uint64_t seed, uint64_t tid, int64_t row, int K, float std_, float* out) {
    uint64_t s = splitmix64(seed ^ splitmix64(tid * 0x100000001B3ull + (uint64_t)row));
    if (!s) s = 0x9E3779B97F4A7C15ull;
    for (int k = 0; k < K; k += 2) {
        const double u1 = ((double)(xorshift64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        const double u2 = ((double)(xorshift64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        const double r = std::sqrt(-2.0 * std::log(u1)), a = 6.283185307179586 * u2;
        out[k] = (float)(r * std::cos(a)) * std_;
        if (k + 1 < K) out[k + 1] = (float)(r * std::sin(a)) * std_;
    }
}

template <typename F> void parallel_rows(int64_t n, F f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 4;
    if (nt > 64) nt = 64;
    if (n < 64) nt = 1;
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; t++)
        th.emplace_back([&, t] { for (int64_t r = t; r < n; r += nt) f(r); });
    for (auto& x : th) x.join();
}

struct TensorOut { std::string name, dtype; std::vector<int64_t> shape; std::vector<uint8_t> data; };

void quant_tensor(uint64_t seed, uint64_t tid, int O, int K, int bits, int gs, float std_, TensorOut& w, TensorOut& s, TensorOut& b) {
    const int64_t rowBytes = (int64_t)K * bits / 8, groups = K / gs;
    w.dtype = "U32"; w.shape = {O, rowBytes / 4}; w.data.assign((size_t)O * rowBytes, 0);
    s.dtype = "BF16"; s.shape = {O, groups}; s.data.assign((size_t)O * groups * 2, 0);
    b.dtype = "BF16"; b.shape = {O, groups}; b.data.assign((size_t)O * groups * 2, 0);
    parallel_rows(O, [&](int64_t r) {
        std::vector<float> row(K);
        gen_row(seed, tid, r, K, std_, row.data());
        mlxr_quantize_row(row.data(), K, bits, gs, w.data.data() + r * rowBytes, (uint16_t*)(s.data.data() + r * groups * 2),
                          (uint16_t*)(b.data.data() + r * groups * 2));
    });
}

void vec_tensor(const std::string& name, int n, float value, std::vector<TensorOut>& out) {
    TensorOut t; t.name = name; t.dtype = "BF16"; t.shape = {n}; t.data.resize((size_t)n * 2);
    const uint16_t v = f32_to_bf16(value);
    for (int i = 0; i < n; i++) memcpy(&t.data[2 * i], &v, 2);
    out.push_back(std::move(t));
}

void rand_vec_tensor(const std::string& name, uint64_t seed, uint64_t tid, int n, float std_, std::vector<TensorOut>& out) {
    TensorOut t; t.name = name; t.dtype = "BF16"; t.shape = {n}; t.data.resize((size_t)n * 2);
    std::vector<float> v(n + 1);
    gen_row(seed, tid, 0, (n + 1) / 2 * 2, std_, v.data());
    for (int i = 0; i < n; i++) { const uint16_t u = f32_to_bf16(v[i]); memcpy(&t.data[2 * i], &u, 2); }
    out.push_back(std::move(t));
}

}  // namespace

int synth_write(const char* config_json, uint64_t seed, float std_, const char* dir) {
    Json cfg; std::string err;
    if (!Json::parse(config_json, strlen(config_json), cfg, err) || cfg.t != Json::Obj) return set_error(MLXR_E_INVALID_ARG, "config: " + err);
    {   // mkdir -p
        std::string path = dir;
        for (size_t i = 1; i <= path.size(); i++)
            if (i == path.size() || path[i] == '/') mkdir(path.substr(0, i).c_str(), 0755);
    }
    {
        FILE* f = fopen((std::string(dir) + "/config.json").c_str(), "wb");
        if (!f) return set_error(MLXR_E_INVALID_FILE, std::string("cannot write ") + dir);
        fwrite(config_json, 1, strlen(config_json), f);
        fclose(f);
    }
    Config c;
    if (int rc = parse_config(dir, c)) return rc;
    if (c.bits == 0 || c.gs == 0) return set_error(MLXR_E_INVALID_ARG, "config has no quantization {bits, group_size}");
    if (c.V <= 0) return set_error(MLXR_E_INVALID_ARG, "config has no vocab_size");
    const int bits = c.bits, gs = c.gs;
    const bool qwen2 = c.model_type == "qwen2", qk_norm = c.model_type == "qwen3";
    // Tensor specs first (sizes known up front), then generated and written one at a time so the
    // host holds at most one tensor.
    struct Spec { std::string name, dtype; std::vector<int64_t> shape; size_t bytes; int kind; uint64_t tid; int O, K; float value; };
    std::vector<Spec> specs;
    uint64_t tid = 1;
    auto qlin = [&](const std::string& prefix, int O, int K) {
        const int64_t rowBytes = (int64_t)K * bits / 8, groups = K / gs;
        const uint64_t t = tid++;
        specs.push_back({prefix + ".weight", "U32", {O, rowBytes / 4}, (size_t)O * rowBytes, 0, t, O, K, 0});
        specs.push_back({prefix + ".scales", "BF16", {O, groups}, (size_t)O * groups * 2, 1, t, O, K, 0});
        specs.push_back({prefix + ".biases", "BF16", {O, groups}, (size_t)O * groups * 2, 2, t, O, K, 0});
    };
    auto vec = [&](const std::string& name, int n, float value) { specs.push_back({name, "BF16", {n}, (size_t)n * 2, 3, 0, n, 0, value}); };
    auto rvec = [&](const std::string& name, int n) { specs.push_back({name, "BF16", {n}, (size_t)n * 2, 4, tid++, n, 0, 0}); };
    qlin("model.embed_tokens", c.V, c.H);
    for (int i = 0; i < c.L; i++) {
        const std::string p = "model.layers." + std::to_string(i);
        qlin(p + ".self_attn.q_proj", c.nH * c.D, c.H);
        qlin(p + ".self_attn.k_proj", c.nKV * c.D, c.H);
        qlin(p + ".self_attn.v_proj", c.nKV * c.D, c.H);
        if (qwen2) {
            rvec(p + ".self_attn.q_proj.bias", c.nH * c.D);
            rvec(p + ".self_attn.k_proj.bias", c.nKV * c.D);
            rvec(p + ".self_attn.v_proj.bias", c.nKV * c.D);
        }
        qlin(p + ".self_attn.o_proj", c.H, c.nH * c.D);
        qlin(p + ".mlp.gate_proj", c.I, c.H);
        qlin(p + ".mlp.up_proj", c.I, c.H);
        qlin(p + ".mlp.down_proj", c.H, c.I);
        vec(p + ".input_layernorm.weight", c.H, 1.0f);
        vec(p + ".post_attention_layernorm.weight", c.H, 1.0f);
        if (qk_norm) {
            vec(p + ".self_attn.q_norm.weight", c.D, 1.0f);
            vec(p + ".self_attn.k_norm.weight", c.D, 1.0f);
        }
    }
    vec("model.norm.weight", c.H, 1.0f);
    if (!c.tie) qlin("lm_head", c.V, c.H);
    // safetensors: header (padded with spaces to 8 bytes) then the tensors in order
    std::string hdr = "{\"__metadata__\":{\"format\":\"mlx\"}";
    size_t off = 0;
    for (auto& t : specs) {
        hdr += ",\"" + t.name + "\":{\"dtype\":\"" + t.dtype + "\",\"shape\":[";
        for (size_t i = 0; i < t.shape.size(); i++) hdr += (i ? "," : "") + std::to_string(t.shape[i]);
        hdr += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + t.bytes) + "]}";
        off += t.bytes;
    }
    hdr += "}";
    while ((8 + hdr.size()) % 8) hdr += ' ';
    FILE* f = fopen((std::string(dir) + "/model.safetensors").c_str(), "wb");
    if (!f) return set_error(MLXR_E_INVALID_FILE, "cannot write model.safetensors");
    uint64_t hl = hdr.size();
    bool ok = fwrite(&hl, 8, 1, f) == 1 && fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size();
    TensorOut w, sc, bi;
    for (size_t i = 0; i < specs.size() && ok; i++) {
        const Spec& t = specs[i];
        if (t.kind == 0) {   // weight: generate the matrix once, emit codes / scales / biases in turn
            quant_tensor(seed, t.tid, t.O, t.K, bits, gs, std_, w, sc, bi);
            ok = fwrite(w.data.data(), 1, w.data.size(), f) == w.data.size();
        } else if (t.kind == 1) {
            ok = fwrite(sc.data.data(), 1, sc.data.size(), f) == sc.data.size();
        } else if (t.kind == 2) {
            ok = fwrite(bi.data.data(), 1, bi.data.size(), f) == bi.data.size();
            w = TensorOut(); sc = TensorOut(); bi = TensorOut();
        } else {
            std::vector<TensorOut> one;
            if (t.kind == 3) vec_tensor(t.name, t.O, t.value, one); else rand_vec_tensor(t.name, seed, t.tid, t.O, std_, one);
            ok = fwrite(one[0].data.data(), 1, one[0].data.size(), f) == one[0].data.size();
        }
    }
    ok = fclose(f) == 0 && ok;
    if (!ok) return set_error(MLXR_E_INVALID_FILE, "short write of model.safetensors");
    return MLXR_OK;
}

}  // namespace mlxr

extern "C" int mlxr_quantize_row(const float* w, int K, int bits, int gs, uint8_t* codes, uint16_t* sc, uint16_t* bi) {
    if (!w || !codes || !sc || !bi || K <= 0 || gs <= 0 || K % gs || bits < 1 || bits > 8) return MLXR_E_INVALID_ARG;
    const int nb = (1 << bits) - 1;
    memset(codes, 0, (size_t)K * bits / 8);
    for (int g = 0; g < K / gs; g++) {
        float lo = w[g * gs], hi = w[g * gs];
        for (int j = 1; j < gs; j++) { lo = fminf(lo, w[g * gs + j]); hi = fmaxf(hi, w[g * gs + j]); }
        const uint16_t sb = f32_to_bf16((hi - lo) / (float)nb), bb = f32_to_bf16(lo);
        sc[g] = sb; bi[g] = bb;
        const float s = bf16_to_f32(sb), b = bf16_to_f32(bb);
        for (int j = 0; j < gs; j++) {
            int q = s > 0 ? (int)std::nearbyint((w[g * gs + j] - b) / s) : 0;
            q = q < 0 ? 0 : (q > nb ? nb : q);
            const int64_t bit = (int64_t)(g * gs + j) * bits;
            for (int i = 0; i < bits; i++)
                if ((q >> i) & 1) codes[(bit + i) >> 3] |= (uint8_t)(1u << ((bit + i) & 7));
        }
    }
    return MLXR_OK;
}

extern "C" int mlxr_synth_matrix(uint64_t seed, uint64_t tid, int O, int K, int bits, int gs, float std_, uint8_t* codes,
                                 uint16_t* sc, uint16_t* bi) {
    if (!codes || !sc || !bi || O <= 0 || K <= 0 || K % 2 || gs <= 0 || K % gs || bits < 1 || bits > 8 || (int64_t)K * bits % 8)
        return MLXR_E_INVALID_ARG;
    const int64_t rowBytes = (int64_t)K * bits / 8, groups = K / gs;
    mlxr::parallel_rows(O, [&](int64_t r) {
        std::vector<float> row(K);
        mlxr::gen_row(seed, tid, r, K, std_, row.data());
        mlxr_quantize_row(row.data(), K, bits, gs, codes + r * rowBytes, sc + r * groups, bi + r * groups);
    });
    return MLXR_OK;
}
