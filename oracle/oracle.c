/*
 * CPU oracle: plain-C restatement of the reference's token-loop semantics.
 * TEST INFRASTRUCTURE ONLY (see oracle.h): never linked, loaded or called by the product.
 */
#define _GNU_SOURCE
#include "oracle.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <stdarg.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <fcntl.h>
#include <unistd.h>
#include <dirent.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[512];
static void set_err(const char* fmt, ...) {
    va_list ap; va_start(ap, fmt); vsnprintf(g_err, sizeof g_err, fmt, ap); va_end(ap);
}
const char* orc_last_error(void) { return g_err; }
int orc_model_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ formats */
float orc_bf16_to_f32(uint16_t u) { uint32_t b = (uint32_t)u << 16; float f; memcpy(&f, &b, 4); return f; }
uint16_t orc_f32_to_bf16(float f) {
    uint32_t b; memcpy(&b, &f, 4);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40);   /* quiet NaN */
    b = b + 0x7fffu + ((b >> 16) & 1u);                                          /* ModelConfig.swift:486-488 */
    return (uint16_t)(b >> 16);
}
float orc_round_bf16(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }
/* GPU.swift:171-184 */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, fr = h & 0x3ffu, bits;
    if (e == 0) {
        if (fr == 0) bits = sign;
        else { int ex = 127 - 15 + 1; while (!(fr & 0x400u)) { fr <<= 1; ex--; } bits = sign | ((uint32_t)ex << 23) | ((fr & 0x3ffu) << 13); }
    } else if (e == 31) bits = sign | 0x7f800000u | (fr << 13);
    else bits = sign | ((e + 127 - 15) << 23) | (fr << 13);
    float f; memcpy(&f, &bits, 4); return f;
}
uint16_t orc_f32_to_f16(float f) {
    uint32_t b; memcpy(&b, &f, 4);
    uint32_t sign = (b >> 16) & 0x8000u; int e = (int)((b >> 23) & 0xff); uint32_t m = b & 0x7fffffu;
    if (e == 255) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0));
    int ne = e - 127 + 15;
    if (ne >= 31) return (uint16_t)(sign | 0x7c00u);
    if (ne <= 0) {
        if (ne < -10) return (uint16_t)sign;
        m |= 0x800000u; int shift = 14 - ne; uint32_t hm = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = m >> 13, rem = m & 0x1fffu;
    uint32_t out = sign | ((uint32_t)ne << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1))) out++;
    return (uint16_t)out;
}

/* ------------------------------------------------------------------ packing */
/* KernelTests.swift:34-43: bit b of value i goes to stream bit i*bits+b, little-endian bytes. */
void orc_pack(const uint32_t* codes, int64_t n, int bits, uint8_t* out) {
    for (int64_t i = 0; i < n; i++)
        for (int b = 0; b < bits; b++)
            if ((codes[i] >> b) & 1u) { int64_t bit = i * bits + b; out[bit >> 3] |= (uint8_t)(1u << (bit & 7)); }
}
/* SieveImport.swift:104-108: code j at bit j*bits, read from one or two bytes. */
void orc_unpack(const uint8_t* p, int64_t n, int bits, uint32_t* codes) {
    uint32_t mask = (1u << bits) - 1u;
    for (int64_t j = 0; j < n; j++) {
        int64_t bit = j * bits, at = bit >> 3; int sh = (int)(bit & 7);
        uint32_t v = p[at];
        if (sh + bits > 8) v |= (uint32_t)p[at + 1] << 8;
        codes[j] = (v >> sh) & mask;
    }
}

/* ------------------------------------------------------------------ linear */
static inline uint32_t code_at(const uint8_t* row, int64_t j, int bits) {
    int64_t bit = j * bits, at = bit >> 3; int sh = (int)(bit & 7);
    uint32_t v = row[at];
    if (sh + bits > 8) v |= (uint32_t)row[at + 1] << 8;
    return (v >> sh) & ((1u << bits) - 1u);
}
void orc_dequant_row(const orc_qlinear* l, int r, float* out) {
    const int64_t rowBytes = (int64_t)l->K * l->bits / 8; const int groups = l->K / l->gs;
    const uint8_t* row = l->w + (int64_t)r * rowBytes;
    const float* s = l->scales + (int64_t)r * groups; const float* b = l->biases + (int64_t)r * groups;
    if (l->bits == 4) {
        for (int k = 0; k < l->K; k += 2) {
            uint8_t byte = row[k >> 1];
            float sg = s[k / l->gs], bg = b[k / l->gs];
            out[k] = (float)(byte & 15) * sg + bg;
            out[k + 1] = (float)(byte >> 4) * sg + bg;
        }
        return;
    }
    for (int k = 0; k < l->K; k++) out[k] = (float)code_at(row, k, l->bits) * s[k / l->gs] + b[k / l->gs];
}
/* Round a double to the nearest f16 value (ties to even; subnormals kept), returned as double. */
double orc_round_f16_d(double v) {
    if (v == 0.0 || !isfinite(v)) return v;
    int e; frexp(v, &e);                       /* |v| in [2^(e-1), 2^e) */
    const int q = e - 11 < -24 ? -24 : e - 11; /* ulp exponent: 11 significant bits, floor 2^-24 */
    const double r = ldexp(nearbyint(ldexp(v, -q)), q);
    return fabs(r) > 65504.0 ? copysign(INFINITY, v) : r;
}
/* The 4-bit model prefill's tile GEMM precision (mlx-runner_amd/csrc/ptile.hip): each token row
 * is scaled by the power of two 2^e that puts max|x| in [2^13, 2^14) and rounded to f16; each weight
 * is f16(fma(s16, q, b16)) with s, b converted to f16; products accumulate exactly here (f32 on the
 * GPU) and the row is scaled back by 2^-e. */
static int f16_mode(const orc_qlinear* l) {
    return l->bits == 4 && (l->gs == 32 || l->gs == 64 || l->gs == 128) && (l->K / l->gs) % 2 == 0;
}
/* sum_k w[k] x[k] in double precision: four interleaved partial sums (k mod 4), added at the end. */
typedef double orc_v4d __attribute__((vector_size(32)));
static double dot_f64(const float* w, const float* x, int K) {
    orc_v4d acc = {0, 0, 0, 0};
    int k = 0;
    for (; k + 4 <= K; k += 4) {
        const orc_v4d a = {w[k], w[k + 1], w[k + 2], w[k + 3]}, b = {x[k], x[k + 1], x[k + 2], x[k + 3]};
        acc += a * b;
    }
    double s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    for (; k < K; k++) s += (double)w[k] * (double)x[k];
    return s;
}
static void qlinear_impl(const orc_qlinear* l, const float* x, int T, float* y, int mode) {
    float* xr = NULL;
    double* inv = NULL;
    if (mode == 2) {
        xr = (float*)malloc((size_t)T * l->K * sizeof(float));
        inv = (double*)malloc((size_t)T * sizeof(double));
        for (int t = 0; t < T; t++) {
            const float* xt = x + (int64_t)t * l->K;
            float mx = 0.0f;
            for (int k = 0; k < l->K; k++) mx = fmaxf(mx, fabsf(xt[k]));
            int e = 0;
            if (mx > 0.0f && mx <= 3.0e38f) { frexpf(mx, &e); e = 14 - e; e = e < -126 ? -126 : (e > 126 ? 126 : e); }
            inv[t] = ldexp(1.0, -e);
            for (int k = 0; k < l->K; k++) xr[(int64_t)t * l->K + k] = (float)orc_round_f16_d((double)ldexpf(xt[k], e));
        }
        x = xr;
    }
    const int groups = l->K / l->gs;
    #pragma omp parallel
    {
        float* w = (float*)malloc((size_t)l->K * sizeof(float));
        #pragma omp for schedule(static)
        for (int o = 0; o < l->O; o++) {
            if (mode == 2) {
                const uint8_t* row = l->w + (int64_t)o * (l->K / 2);
                for (int k = 0; k < l->K; k++) {
                    const double sg = orc_round_f16_d(l->scales[(int64_t)o * groups + k / l->gs]);
                    const double bg = orc_round_f16_d(l->biases[(int64_t)o * groups + k / l->gs]);
                    const int q = (row[k >> 1] >> ((k & 1) * 4)) & 15;
                    w[k] = (float)orc_round_f16_d(sg * q + bg);
                }
            } else {
                orc_dequant_row(l, o, w);
            }
            for (int t = 0; t < T; t++) {
                const float* xt = x + (int64_t)t * l->K;
                double acc = dot_f64(w, xt, l->K);
                if (mode == 2) acc *= inv[t];
                y[(int64_t)t * l->O + o] = (float)acc + (l->bias ? l->bias[o] : 0.0f);
            }
        }
        free(w);
    }
    free(xr);
    free(inv);
}
void orc_qlinear_f64(const orc_qlinear* l, const float* x, int T, float* y) { qlinear_impl(l, x, T, y, 0); }
void orc_qlinear_f16(const orc_qlinear* l, const float* x, int T, float* y) { qlinear_impl(l, x, T, y, 2); }
/* The model prefill's precision (T > 8 tokens): the tile GEMM's f16 operands for 4-bit with gs
 * 32/64/128 and an even number of groups per row; the MLX-layout GEMM's fp32-level products (exact
 * codes, x as f16 hi + lo, scale and bias per group in fp32: modelled as exact) otherwise. */
void orc_qlinear_prefill(const orc_qlinear* l, const float* x, int T, float* y) { qlinear_impl(l, x, T, y, f16_mode(l) ? 2 : 0); }

/* ------------------------------------------------------------------ norms, RoPE */
void orc_rms_norm(const float* x, float* y, const float* w, int dim, int rows, float eps) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (int64_t)r * dim; float* yr = y + (int64_t)r * dim;
        double ss = 0;
        for (int i = 0; i < dim; i++) ss += (double)xr[i] * xr[i];
        float inv = 1.0f / sqrtf((float)(ss / dim) + eps);
        for (int i = 0; i < dim; i++) yr[i] = xr[i] * inv * (w ? w[i] : 1.0f);
    }
}
/* ModelConfig.swift:438-443: 1 / theta^(2i/rotDim) in double, then Float. */
void orc_inv_freq(double theta, int rot_dim, float* out) {
    for (int i = 0; i < rot_dim / 2; i++) out[i] = (float)(1.0 / pow(theta, (double)(2 * i) / (double)rot_dim));
}
/* Kernels.swift:1124-1134 */
void orc_rope(float* v, int D, int rot_dim, int traditional, int pos, const float* inv_freq) {
    float buf[1024];
    memcpy(buf, v, sizeof(float) * D);
    int half = rot_dim / 2;
    for (int i = 0; i < rot_dim; i++) {
        int fi, partner, first;
        if (traditional) { fi = i / 2; partner = i ^ 1; first = (i & 1) == 0; }
        else { fi = i % half; first = i < half; partner = first ? i + half : i - half; }
        float ang = (float)pos * inv_freq[fi];
        float c = cosf(ang), s = sinf(ang);
        v[i] = first ? buf[i] * c - buf[partner] * s : buf[i] * c + buf[partner] * s;
    }
}
float orc_silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

/* ------------------------------------------------------------------ attention */
static void attend(const float* qh, const float* kb, const float* vb, int D, const int32_t* pos_list, int n,
                   float scale, float* out) {
    double* s = (double*)malloc(sizeof(double) * (n > 0 ? n : 1));
    double m = -1e300;
    for (int i = 0; i < n; i++) {
        const float* k = kb + (int64_t)pos_list[i] * D;
        double d = 0;
        for (int e = 0; e < D; e++) d += (double)(qh[e] * scale) * k[e];
        s[i] = d; if (d > m) m = d;
    }
    double z = 0;
    for (int i = 0; i < n; i++) { s[i] = exp(s[i] - m); z += s[i]; }
    for (int e = 0; e < D; e++) {
        double acc = 0;
        for (int i = 0; i < n; i++) acc += s[i] * vb[(int64_t)pos_list[i] * D + e];
        out[e] = (float)(acc / z);
    }
    free(s);
}
void orc_attention(const float* q, const float* kc, const float* vc, int D, int nH, int nKV, int max_seq,
                   int pos, float scale, float* out) {
    int L = pos + 1;
    int32_t* list = (int32_t*)malloc(sizeof(int32_t) * L);
    for (int j = 0; j < L; j++) list[j] = j;
    for (int h = 0; h < nH; h++) {
        int kvh = h / (nH / nKV);
        attend(q + (int64_t)h * D, kc + (int64_t)kvh * max_seq * D, vc + (int64_t)kvh * max_seq * D, D, list, L, scale,
               out + (int64_t)h * D);
    }
    free(list);
}
void orc_attention_list(const float* q, const float* kc, const float* vc, int D, int nH, int nKV, int max_seq,
                        int pos, float scale, const int32_t* lists, int count, int list_stride, float* out) {
    int L = pos + 1;
    int32_t* cl = (int32_t*)malloc(sizeof(int32_t) * (count > 0 ? count : 1));
    for (int h = 0; h < nH; h++) {
        int kvh = h / (nH / nKV);
        const int32_t* li = lists + (int64_t)kvh * list_stride;
        for (int i = 0; i < count; i++) { int j = li[i]; cl[i] = j < 0 ? 0 : (j > L - 1 ? L - 1 : j); }
        attend(q + (int64_t)h * D, kc + (int64_t)kvh * max_seq * D, vc + (int64_t)kvh * max_seq * D, D, cl, count, scale,
               out + (int64_t)h * D);
    }
    free(cl);
}

/* ------------------------------------------------------------------ sparse */
void orc_sparse_clamp(int* top_k, int* window, int* sink, int* min_context, int has_min) {
    const int p = 4;
    int t = *top_k < (1 << 22) ? *top_k : (1 << 22); if (t < p) t = p; *top_k = t / p * p;
    int w = *window < (1 << 22) ? *window : (1 << 22); if (w < p) w = p; *window = w;
    int s = *sink < (1 << 16) ? *sink : (1 << 16); if (s < 0) s = 0; *sink = s;
    int mc = has_min ? *min_context : 2 * (*sink + *top_k + *window);
    if (mc > (1 << 30)) mc = 1 << 30; if (mc < 1) mc = 1; *min_context = mc;
}
/* SparseAttention.swift:80-94 */
int orc_sparse_make_plan(int top_k, int window, int sink, int min_context, int position, orc_sparse_plan* o) {
    const int pool = 4; int L = position + 1;
    if (position < 0 || L < min_context) return 0;
    int sinkEnd = (sink + pool - 1) / pool * pool;
    if (!(L - window > sinkEnd)) return 0;
    int winStart = (L - window) / pool * pool;
    int b0 = sinkEnd / pool, nb = winStart / pool - b0;
    if (nb <= 0) return 0;
    int p = top_k / pool < nb ? top_k / pool : nb;
    o->pool = pool; o->b0 = b0; o->nb = nb; o->p = p; o->sink_end = sinkEnd; o->win_start = winStart; o->L = L;
    o->count = sinkEnd + p * pool + (L - winStart);
    return 1;
}
/* Kernels.swift:1545-1555 (mean of the pool keys in fp32, stored in the index dtype: bf16 here) */
void orc_sparse_index(const float* kc, int nKV, int D, int max_seq, int pool, int b0, int nb, float* idx) {
    for (int b = b0; b < b0 + nb; b++)
        for (int h = 0; h < nKV; h++)
            for (int d = 0; d < D; d++) {
                float s = 0;
                for (int i = 0; i < pool; i++) s += kc[((int64_t)h * max_seq + (int64_t)b * pool + i) * D + d];
                idx[((int64_t)b * nKV + h) * D + d] = orc_round_bf16(s / (float)pool);
            }
}
/* Kernels.swift:1565-1612: per KV head qsum_kvh . idx[b0+n][kvh], or the sum over KV heads. */
void orc_sparse_score(const float* q, const float* idx, int nH, int nKV, int D, int b0, int nb, int rows, float* scores) {
    int G = nH / nKV, W = nKV * D;
    float* qs = (float*)malloc(sizeof(float) * W);
    for (int h = 0; h < nKV; h++)
        for (int d = 0; d < D; d++) { float s = 0; for (int g = 0; g < G; g++) s += q[(int64_t)(h * G + g) * D + d]; qs[h * D + d] = s; }
    for (int n = 0; n < nb; n++) {
        const float* row = idx + (int64_t)(b0 + n) * W;
        double tot = 0;
        for (int h = 0; h < nKV; h++) {
            double s = 0;
            for (int d = 0; d < D; d++) s += (double)qs[h * D + d] * row[h * D + d];
            if (rows == 1) tot += s; else scores[(int64_t)h * nb + n] = (float)s;
        }
        if (rows == 1) scores[n] = (float)tot;
    }
    free(qs);
}
uint32_t orc_sparse_key(float f) { uint32_t u; memcpy(&u, &f, 4); return (u & 0x80000000u) ? ~u : (u | 0x80000000u); }
/* SparseAttentionTests.swift:141-149: highest key first, earlier block first among equals, then
 * back in position order; list = sink, kept blocks' keys, window. */
void orc_sparse_select(const float* scores, int nb, const orc_sparse_plan* pl, int32_t* list) {
    int32_t* order = (int32_t*)malloc(sizeof(int32_t) * nb);
    uint32_t* keys = (uint32_t*)malloc(sizeof(uint32_t) * nb);
    for (int i = 0; i < nb; i++) { order[i] = i; keys[i] = orc_sparse_key(scores[i]); }
    /* partial selection: p passes would be O(p*nb); a plain insertion sort on (key desc, idx asc) is fine for tests */
    /* use a merge sort for large nb */
    int32_t* tmp = (int32_t*)malloc(sizeof(int32_t) * nb);
    for (int w = 1; w < nb; w *= 2) {
        for (int lo = 0; lo < nb; lo += 2 * w) {
            int mid = lo + w < nb ? lo + w : nb, hi = lo + 2 * w < nb ? lo + 2 * w : nb, a = lo, b = mid, k = lo;
            while (a < mid && b < hi) {
                int ia = order[a], ib = order[b];
                int takeA = keys[ia] != keys[ib] ? keys[ia] > keys[ib] : ia < ib;
                tmp[k++] = takeA ? order[a++] : order[b++];
            }
            while (a < mid) tmp[k++] = order[a++];
            while (b < hi) tmp[k++] = order[b++];
        }
        memcpy(order, tmp, sizeof(int32_t) * nb);
    }
    char* kept = (char*)calloc(nb, 1);
    for (int i = 0; i < pl->p; i++) kept[order[i]] = 1;
    int c = 0;
    for (int i = 0; i < pl->sink_end; i++) list[c++] = i;
    for (int n = 0; n < nb; n++) if (kept[n]) for (int i = 0; i < pl->pool; i++) list[c++] = (pl->b0 + n) * pl->pool + i;
    for (int j = pl->win_start; j < pl->L; j++) list[c++] = j;
    free(order); free(keys); free(tmp); free(kept);
}

/* ------------------------------------------------------------------ sampling */
int orc_argmax(const float* l, int V) {
    int best = 0; float bv = -INFINITY;
    for (int i = 0; i < V; i++) if (l[i] > bv) { bv = l[i]; best = i; }
    return isfinite(bv) ? best : -1;
}
/* Engine.swift:112-160 */
int orc_sample_distribution(float* logits, int V, const int32_t* recent, int n_recent, float temperature, int top_k,
                            float top_p, float min_p, float penalty, int32_t* ids, float* probs, int max_out) {
    if (penalty != 1.0f && n_recent > 0) {
        for (int i = 0; i < n_recent; i++) {
            int t = recent[i], dup = 0;
            for (int j = 0; j < i; j++) if (recent[j] == t) { dup = 1; break; }
            if (dup || t < 0 || t >= V) continue;
            logits[t] = logits[t] > 0 ? logits[t] / penalty : logits[t] * penalty;
        }
    }
    if (temperature <= 0.001f) {
        int b = orc_argmax(logits, V);
        if (b < 0) return -1;
        ids[0] = b; probs[0] = 1.0f; return 1;
    }
    int k = top_k > 0 ? (top_k < V ? top_k : V) : (512 < V ? 512 : V);
    /* stable descending order by value, earlier index first among equals (the partial selection
       keeps the first-seen of equal values ahead: binary insertion after equals) */
    int32_t* cand = (int32_t*)malloc(sizeof(int32_t) * (k + 1)); int n = 0;
    for (int i = 0; i < V; i++) {
        float v = logits[i];
        if (n < k) {
            int pos = n; while (pos > 0 && logits[cand[pos - 1]] < v) { cand[pos] = cand[pos - 1]; pos--; }
            cand[pos] = i; n++;
        } else if (v > logits[cand[k - 1]]) {
            int pos = k - 1; while (pos > 0 && logits[cand[pos - 1]] < v) { cand[pos] = cand[pos - 1]; pos--; }
            cand[pos] = i;
        }
    }
    float maxV = logits[cand[0]];
    if (!isfinite(maxV)) { free(cand); return -1; }
    float invT = 1.0f / temperature;
    float* p = (float*)malloc(sizeof(float) * n);
    float total = 0;
    for (int i = 0; i < n; i++) { p[i] = expf((logits[cand[i]] - maxV) * invT); total += p[i]; }
    int cut = n;
    if (min_p > 0) { float th = min_p * p[0]; for (int i = 0; i < n; i++) if (p[i] < th) { cut = i; break; } }
    if (top_p < 1) { float acc = 0; for (int i = 0; i < cut; i++) { acc += p[i] / total; if (acc >= top_p) { cut = i + 1; break; } } }
    if (cut < 1) cut = 1;
    float tot = 0; for (int i = 0; i < cut; i++) tot += p[i];
    int out = cut < max_out ? cut : max_out;
    for (int i = 0; i < out; i++) { ids[i] = cand[i]; probs[i] = p[i] / tot; }
    free(cand); free(p);
    return out;
}

/* ------------------------------------------------------------------ JSON (minimal) */
typedef enum { J_NULL, J_BOOL, J_NUM, J_STR, J_ARR, J_OBJ } jtype;
typedef struct jval { jtype t; double num; char* str; int n; struct jval* items; char** keys; } jval;
static const char* jskip(const char* p) { while (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t') p++; return p; }
static const char* jparse(const char* p, jval* v, int depth);
static const char* jstr(const char* p, char** out) {
    if (*p != '"') return NULL; p++;
    size_t cap = 32, n = 0; char* s = (char*)malloc(cap);
    while (*p && *p != '"') {
        char c = *p++;
        if (c == '\\') { c = *p++; if (c == 'n') c = '\n'; else if (c == 't') c = '\t'; else if (c == 'u') { p += 4; c = '?'; } else if (!c) break; }
        if (n + 2 > cap) { cap *= 2; s = (char*)realloc(s, cap); }
        s[n++] = c;
    }
    if (*p != '"') { free(s); return NULL; }
    s[n] = 0; *out = s; return p + 1;
}
static const char* jparse(const char* p, jval* v, int depth) {
    memset(v, 0, sizeof *v);
    if (depth > 64) return NULL;
    p = jskip(p);
    if (*p == '{') {
        v->t = J_OBJ; p = jskip(p + 1);
        if (*p == '}') return p + 1;
        for (;;) {
            char* k; p = jstr(jskip(p), &k); if (!p) return NULL;
            p = jskip(p); if (*p != ':') return NULL;
            v->items = (jval*)realloc(v->items, sizeof(jval) * (v->n + 1));
            v->keys = (char**)realloc(v->keys, sizeof(char*) * (v->n + 1));
            v->keys[v->n] = k;
            p = jparse(p + 1, &v->items[v->n], depth + 1); if (!p) return NULL;
            v->n++; p = jskip(p);
            if (*p == ',') { p++; continue; }
            if (*p == '}') return p + 1;
            return NULL;
        }
    }
    if (*p == '[') {
        v->t = J_ARR; p = jskip(p + 1);
        if (*p == ']') return p + 1;
        for (;;) {
            v->items = (jval*)realloc(v->items, sizeof(jval) * (v->n + 1));
            p = jparse(p, &v->items[v->n], depth + 1); if (!p) return NULL;
            v->n++; p = jskip(p);
            if (*p == ',') { p++; continue; }
            if (*p == ']') return p + 1;
            return NULL;
        }
    }
    if (*p == '"') { v->t = J_STR; return jstr(p, &v->str); }
    if (!strncmp(p, "true", 4)) { v->t = J_BOOL; v->num = 1; return p + 4; }
    if (!strncmp(p, "false", 5)) { v->t = J_BOOL; v->num = 0; return p + 5; }
    if (!strncmp(p, "null", 4)) { v->t = J_NULL; return p + 4; }
    char* end; v->num = strtod(p, &end); if (end == p) return NULL; v->t = J_NUM; return end;
}
static void jfree(jval* v) {
    for (int i = 0; i < v->n; i++) { jfree(&v->items[i]); if (v->keys) free(v->keys[i]); }
    free(v->items); free(v->keys); free(v->str);
}
static const jval* jget(const jval* o, const char* k) {
    if (!o || o->t != J_OBJ) return NULL;
    for (int i = 0; i < o->n; i++) if (!strcmp(o->keys[i], k)) return &o->items[i];
    return NULL;
}
static double jnum(const jval* o, const char* k, double def) { const jval* v = jget(o, k); return v && (v->t == J_NUM || v->t == J_BOOL) ? v->num : def; }

/* ------------------------------------------------------------------ safetensors */
typedef struct { char* name; int dtype; int64_t shape[8]; int ndim; uint8_t* data; int64_t nbytes; } stensor;
enum { DT_U32 = 1, DT_BF16, DT_F16, DT_F32, DT_OTHER };
typedef struct { stensor* t; int n; void** maps; size_t* maplens; int nmaps; } sstore;
static int load_file(sstore* st, const char* path) {
    int fd = open(path, O_RDONLY); if (fd < 0) { set_err("cannot open %s", path); return -1; }
    struct stat sb; fstat(fd, &sb); size_t size = (size_t)sb.st_size;
    if (size < 8) { close(fd); set_err("%s truncated", path); return -1; }
    uint8_t* base = (uint8_t*)mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0); close(fd);
    if (base == MAP_FAILED) { set_err("mmap %s", path); return -1; }
    st->maps = (void**)realloc(st->maps, sizeof(void*) * (st->nmaps + 1));
    st->maplens = (size_t*)realloc(st->maplens, sizeof(size_t) * (st->nmaps + 1));
    st->maps[st->nmaps] = base; st->maplens[st->nmaps++] = size;
    uint64_t hl; memcpy(&hl, base, 8);
    if (hl > size - 8) { set_err("bad header length"); return -1; }
    char* hdr = (char*)malloc(hl + 1); memcpy(hdr, base + 8, hl); hdr[hl] = 0;
    jval root; if (!jparse(hdr, &root, 0) || root.t != J_OBJ) { free(hdr); set_err("bad header json"); return -1; }
    free(hdr);
    uint8_t* data = base + 8 + hl; int64_t dsize = (int64_t)(size - 8 - hl);
    for (int i = 0; i < root.n; i++) {
        if (!strcmp(root.keys[i], "__metadata__")) continue;
        const jval* e = &root.items[i]; const jval* dt = jget(e, "dtype"), *sh = jget(e, "shape"), *of = jget(e, "data_offsets");
        if (!dt || !sh || !of || dt->t != J_STR || sh->t != J_ARR || of->t != J_ARR || of->n != 2) { set_err("bad entry"); jfree(&root); return -1; }
        stensor t; memset(&t, 0, sizeof t);
        t.name = strdup(root.keys[i]);
        t.dtype = !strcmp(dt->str, "U32") ? DT_U32 : !strcmp(dt->str, "BF16") ? DT_BF16 : !strcmp(dt->str, "F16") ? DT_F16 : !strcmp(dt->str, "F32") ? DT_F32 : DT_OTHER;
        t.ndim = sh->n; for (int d = 0; d < sh->n && d < 8; d++) t.shape[d] = (int64_t)sh->items[d].num;
        int64_t a = (int64_t)of->items[0].num, b = (int64_t)of->items[1].num;
        if (a < 0 || b < a || b > dsize) { set_err("tensor %s out of bounds", t.name); jfree(&root); return -1; }
        t.data = data + a; t.nbytes = b - a;
        st->t = (stensor*)realloc(st->t, sizeof(stensor) * (st->n + 1)); st->t[st->n++] = t;
    }
    jfree(&root);
    return 0;
}
static const stensor* sget(const sstore* st, const char* name) {
    for (int i = 0; i < st->n; i++) if (!strcmp(st->t[i].name, name)) return &st->t[i];
    return NULL;
}
static float* to_floats(const stensor* t) {
    int64_t n = 1; for (int d = 0; d < t->ndim; d++) n *= t->shape[d];
    float* out = (float*)malloc(sizeof(float) * (n > 0 ? n : 1));
    for (int64_t i = 0; i < n; i++) {
        uint16_t u;
        switch (t->dtype) {
            case DT_BF16: memcpy(&u, t->data + 2 * i, 2); out[i] = orc_bf16_to_f32(u); break;
            case DT_F16: memcpy(&u, t->data + 2 * i, 2); out[i] = orc_f16_to_f32(u); break;
            case DT_F32: memcpy(&out[i], t->data + 4 * i, 4); break;
            default: out[i] = 0;
        }
    }
    return out;
}

/* ------------------------------------------------------------------ model */
typedef struct { orc_qlinear l; float* s; float* b; float* bias; } olin;
typedef struct {
    olin q, k, v, o, gate, up, down;
    float *in_norm, *post_norm, *q_norm, *k_norm;
    float *kc, *vc;   /* [nKV][max_seq][D] fp32 values of bf16 entries */
    float *idx;       /* sparse index [max_seq/4][nKV][D] */
} olayer;
struct orc_model {
    int H, L, nH, nKV, D, I, V, max_seq, rot_dim, traditional;
    float eps, scale; double theta;
    float* inv_freq;
    olin embed, head; int tied;
    float* final_norm;
    olayer* layers;
    sstore st;
    int sparse_on, sp_topk, sp_window, sp_sink, sp_min, sp_perhead;
};
static int make_lin(sstore* st, const char* prefix, int K, olin* out) {
    char nm[256];
    snprintf(nm, sizeof nm, "%s.weight", prefix); const stensor* w = sget(st, nm);
    snprintf(nm, sizeof nm, "%s.scales", prefix); const stensor* s = sget(st, nm);
    snprintf(nm, sizeof nm, "%s.biases", prefix); const stensor* b = sget(st, nm);
    snprintf(nm, sizeof nm, "%s.bias", prefix); const stensor* bias = sget(st, nm);
    if (!w || !s || !b) { set_err("missing tensor %s", prefix); return -1; }
    memset(out, 0, sizeof *out);
    int O = (int)w->shape[0];
    int64_t packedBytes = w->shape[1] * 4;
    int bits = (int)(packedBytes * 8 / K);
    int gs = K / (int)s->shape[1];
    out->s = to_floats(s); out->b = to_floats(b); out->bias = bias ? to_floats(bias) : NULL;
    out->l.w = w->data; out->l.scales = out->s; out->l.biases = out->b; out->l.bias = out->bias;
    out->l.O = O; out->l.K = K; out->l.bits = bits; out->l.gs = gs;
    return 0;
}
static float* req_floats(sstore* st, const char* name) {
    const stensor* t = sget(st, name); if (!t) { set_err("missing tensor %s", name); return NULL; }
    return to_floats(t);
}
orc_model* orc_model_load(const char* dir, int max_seq) {
    char path[1024];
    snprintf(path, sizeof path, "%s/config.json", dir);
    FILE* f = fopen(path, "rb"); if (!f) { set_err("config.json not found"); return NULL; }
    fseek(f, 0, SEEK_END); long n = ftell(f); fseek(f, 0, SEEK_SET);
    char* txt = (char*)malloc(n + 1); if (fread(txt, 1, n, f) != (size_t)n) { fclose(f); free(txt); return NULL; } txt[n] = 0; fclose(f);
    jval cfg; if (!jparse(txt, &cfg, 0)) { free(txt); set_err("bad config.json"); return NULL; } free(txt);
    orc_model* m = (orc_model*)calloc(1, sizeof *m);
    m->H = (int)jnum(&cfg, "hidden_size", 0); m->L = (int)jnum(&cfg, "num_hidden_layers", 0);
    m->nH = (int)jnum(&cfg, "num_attention_heads", 0); m->nKV = (int)jnum(&cfg, "num_key_value_heads", m->nH);
    m->D = (int)jnum(&cfg, "head_dim", m->H / (m->nH ? m->nH : 1)); m->I = (int)jnum(&cfg, "intermediate_size", 4 * m->H);
    m->eps = (float)jnum(&cfg, "rms_norm_eps", 1e-6); m->theta = (float)jnum(&cfg, "rope_theta", 10000);
    m->traditional = (int)jnum(&cfg, "rope_traditional", 0);
    m->rot_dim = m->D; m->scale = 1.0f / sqrtf((float)m->D);   /* ModelConfig.swift:246 */
    jfree(&cfg);
    m->max_seq = max_seq;
    m->inv_freq = (float*)malloc(sizeof(float) * m->D);
    /* rope_theta is parsed as Float then widened (ModelConfig.swift:226, :443) */
    orc_inv_freq((double)(float)m->theta, m->rot_dim, m->inv_freq);
    DIR* dd = opendir(dir); if (!dd) { set_err("cannot list %s", dir); free(m); return NULL; }
    struct dirent* de;
    char names[64][256]; int nf = 0;
    while ((de = readdir(dd)) && nf < 64) {
        size_t ln = strlen(de->d_name);
        if (ln > 12 && !strcmp(de->d_name + ln - 12, ".safetensors")) snprintf(names[nf++], 256, "%s", de->d_name);
    }
    closedir(dd);
    for (int i = 0; i < nf; i++) { snprintf(path, sizeof path, "%s/%s", dir, names[i]); if (load_file(&m->st, path)) { orc_model_free(m); return NULL; } }
    if (make_lin(&m->st, "model.embed_tokens", m->H, &m->embed)) { orc_model_free(m); return NULL; }
    m->V = m->embed.l.O;
    if (sget(&m->st, "lm_head.weight")) { if (make_lin(&m->st, "lm_head", m->H, &m->head)) { orc_model_free(m); return NULL; } }
    else { m->head = m->embed; m->tied = 1; }
    if (!(m->final_norm = req_floats(&m->st, "model.norm.weight"))) { orc_model_free(m); return NULL; }
    m->layers = (olayer*)calloc(m->L, sizeof(olayer));
    for (int i = 0; i < m->L; i++) {
        olayer* ly = &m->layers[i]; char p[256], nm[300];
        snprintf(p, sizeof p, "model.layers.%d", i);
#define LIN(field, sub, K) do { snprintf(nm, sizeof nm, "%s.%s", p, sub); if (make_lin(&m->st, nm, K, &ly->field)) { orc_model_free(m); return NULL; } } while (0)
        LIN(q, "self_attn.q_proj", m->H); LIN(k, "self_attn.k_proj", m->H); LIN(v, "self_attn.v_proj", m->H);
        LIN(o, "self_attn.o_proj", m->nH * m->D);
        LIN(gate, "mlp.gate_proj", m->H); LIN(up, "mlp.up_proj", m->H); LIN(down, "mlp.down_proj", m->I);
#undef LIN
        snprintf(nm, sizeof nm, "%s.input_layernorm.weight", p); if (!(ly->in_norm = req_floats(&m->st, nm))) { orc_model_free(m); return NULL; }
        snprintf(nm, sizeof nm, "%s.post_attention_layernorm.weight", p); if (!(ly->post_norm = req_floats(&m->st, nm))) { orc_model_free(m); return NULL; }
        snprintf(nm, sizeof nm, "%s.self_attn.q_norm.weight", p);
        if (sget(&m->st, nm)) {
            ly->q_norm = req_floats(&m->st, nm);
            snprintf(nm, sizeof nm, "%s.self_attn.k_norm.weight", p); if (!(ly->k_norm = req_floats(&m->st, nm))) { orc_model_free(m); return NULL; }
        }
        ly->kc = (float*)calloc((size_t)m->nKV * max_seq * m->D, sizeof(float));
        ly->vc = (float*)calloc((size_t)m->nKV * max_seq * m->D, sizeof(float));
        ly->idx = (float*)calloc((size_t)(max_seq / 4 + 1) * m->nKV * m->D, sizeof(float));
    }
    return m;
}
static void free_lin(olin* l) { free(l->s); free(l->b); free(l->bias); }
void orc_model_free(orc_model* m) {
    if (!m) return;
    if (m->layers) for (int i = 0; i < m->L; i++) {
        olayer* ly = &m->layers[i];
        free_lin(&ly->q); free_lin(&ly->k); free_lin(&ly->v); free_lin(&ly->o); free_lin(&ly->gate); free_lin(&ly->up); free_lin(&ly->down);
        free(ly->in_norm); free(ly->post_norm); free(ly->q_norm); free(ly->k_norm); free(ly->kc); free(ly->vc); free(ly->idx);
    }
    free(m->layers);
    free_lin(&m->embed); if (!m->tied) free_lin(&m->head);
    free(m->final_norm); free(m->inv_freq);
    for (int i = 0; i < m->st.n; i++) free(m->st.t[i].name);
    free(m->st.t);
    for (int i = 0; i < m->st.nmaps; i++) munmap(m->st.maps[i], m->st.maplens[i]);
    free(m->st.maps); free(m->st.maplens);
    free(m);
}
int orc_model_vocab(const orc_model* m) { return m->V; }
int orc_model_hidden(const orc_model* m) { return m->H; }
void orc_model_set_sparse(orc_model* m, int enabled, int top_k, int window, int sink, int min_context, int per_head) {
    m->sparse_on = enabled; m->sp_topk = top_k; m->sp_window = window; m->sp_sink = sink; m->sp_min = min_context; m->sp_perhead = per_head;
}
int orc_model_set_kv(orc_model* m, int layer, const float* k, const float* v, int rows) {
    if (layer < 0 || layer >= m->L || rows > m->max_seq) return -1;
    olayer* ly = &m->layers[layer];
    for (int h = 0; h < m->nKV; h++) {
        memcpy(ly->kc + (size_t)h * m->max_seq * m->D, k + (size_t)h * rows * m->D, sizeof(float) * rows * m->D);
        memcpy(ly->vc + (size_t)h * m->max_seq * m->D, v + (size_t)h * rows * m->D, sizeof(float) * rows * m->D);
    }
    /* rebuild the sparse index over the rows given */
    orc_sparse_index(ly->kc, m->nKV, m->D, m->max_seq, 4, 0, rows / 4, ly->idx);
    return 0;
}

static void lin_apply(const olin* l, const float* x, int T, float* y, int bf16) {
    if (bf16) orc_qlinear_prefill(&l->l, x, T, y); else orc_qlinear_f64(&l->l, x, T, y);
}
/* Transformer.swift:1323-1584 for qwen3 / qwen2 / llama layers (no sliding window, no gates). */
int orc_forward(orc_model* m, const int32_t* tokens, int n, int offset, int small_t, float* logits) {
    if (n <= 0 || offset < 0 || offset + n > m->max_seq) { set_err("context full"); return -1; }
    for (int i = 0; i < n; i++) if (tokens[i] < 0 || tokens[i] >= m->V) { set_err("token id outside the embedding table"); return -1; }
    const int H = m->H, D = m->D, nH = m->nH, nKV = m->nKV, I = m->I;
    const int qkvCols = (nH + 2 * nKV) * D;
    const int bf = n > small_t;
    float* h = (float*)malloc(sizeof(float) * n * H);
    float* xn = (float*)malloc(sizeof(float) * n * H);
    float* q = (float*)malloc(sizeof(float) * n * nH * D);
    float* kk = (float*)malloc(sizeof(float) * n * nKV * D);
    float* vv = (float*)malloc(sizeof(float) * n * nKV * D);
    float* attn = (float*)malloc(sizeof(float) * n * nH * D);
    float* tmp = (float*)malloc(sizeof(float) * n * H);
    float* g = (float*)malloc(sizeof(float) * n * I);
    float* u = (float*)malloc(sizeof(float) * n * I);
    (void)qkvCols;
    for (int t = 0; t < n; t++) orc_dequant_row(&m->embed.l, tokens[t], h + (int64_t)t * H);   /* qembed Kernels.swift:1002-1023 */
    orc_rms_norm(h, xn, m->layers[0].in_norm, H, n, m->eps);
    orc_sparse_plan plan; int sparse = 0;
    if (n == 1 && m->sparse_on) sparse = orc_sparse_make_plan(m->sp_topk, m->sp_window, m->sp_sink, m->sp_min, offset, &plan);
    for (int li = 0; li < m->L; li++) {
        olayer* ly = &m->layers[li];
        lin_apply(&ly->q, xn, n, q, bf); lin_apply(&ly->k, xn, n, kk, bf); lin_apply(&ly->v, xn, n, vv, bf);
        /* qkv_post (Kernels.swift:1081-1138) */
        for (int t = 0; t < n; t++) {
            int pos = offset + t;
            for (int hh = 0; hh < nH + nKV; hh++) {
                float* v = hh < nH ? q + ((int64_t)t * nH + hh) * D : kk + ((int64_t)t * nKV + (hh - nH)) * D;
                if (ly->q_norm) orc_rms_norm(v, v, hh < nH ? ly->q_norm : ly->k_norm, D, 1, m->eps);
                orc_rope(v, D, m->rot_dim, m->traditional, pos, m->inv_freq);
            }
            for (int kv = 0; kv < nKV; kv++)
                for (int e = 0; e < D; e++) {
                    ly->kc[((int64_t)kv * m->max_seq + pos) * D + e] = orc_round_bf16(kk[((int64_t)t * nKV + kv) * D + e]);
                    ly->vc[((int64_t)kv * m->max_seq + pos) * D + e] = orc_round_bf16(vv[((int64_t)t * nKV + kv) * D + e]);
                }
        }
        /* sparse index of the blocks completed by this step (Transformer.swift:1394-1405) */
        { int b0 = offset / 4, b1 = (offset + n) / 4; if (b1 > b0) orc_sparse_index(ly->kc, nKV, D, m->max_seq, 4, b0, b1 - b0, ly->idx); }
        if (sparse) {
            int rows = m->sp_perhead ? nKV : 1;
            float* scores = (float*)malloc(sizeof(float) * rows * plan.nb);
            int32_t* lists = (int32_t*)malloc(sizeof(int32_t) * rows * plan.count);
            orc_sparse_score(q, ly->idx, nH, nKV, D, plan.b0, plan.nb, rows, scores);
            for (int r = 0; r < rows; r++) orc_sparse_select(scores + (int64_t)r * plan.nb, plan.nb, &plan, lists + (int64_t)r * plan.count);
            orc_attention_list(q, ly->kc, ly->vc, D, nH, nKV, m->max_seq, offset, m->scale, lists, plan.count,
                               rows == 1 ? 0 : plan.count, attn);
            free(scores); free(lists);
        } else {
            #pragma omp parallel for schedule(dynamic)
            for (int t = 0; t < n; t++)
                orc_attention(q + (int64_t)t * nH * D, ly->kc, ly->vc, D, nH, nKV, m->max_seq, offset + t, m->scale, attn + (int64_t)t * nH * D);
        }
        lin_apply(&ly->o, attn, n, tmp, bf);
        for (int64_t i = 0; i < (int64_t)n * H; i++) h[i] += tmp[i];
        orc_rms_norm(h, xn, ly->post_norm, H, n, m->eps);
        lin_apply(&ly->gate, xn, n, g, bf); lin_apply(&ly->up, xn, n, u, bf);
        for (int64_t i = 0; i < (int64_t)n * I; i++) g[i] = orc_silu_mul(g[i], u[i]);
        lin_apply(&ly->down, g, n, tmp, bf);
        for (int64_t i = 0; i < (int64_t)n * H; i++) h[i] += tmp[i];
        const float* nw = li + 1 < m->L ? m->layers[li + 1].in_norm : m->final_norm;
        orc_rms_norm(h, xn, nw, H, n, m->eps);
    }
    /* lm_head on the last row only (Transformer.swift:1573-1575); a single row uses the decode precision */
    if (logits) orc_qlinear_f64(&m->head.l, xn + (int64_t)(n - 1) * H, 1, logits);
    free(h); free(xn); free(q); free(kk); free(vv); free(attn); free(tmp); free(g); free(u);
    return 0;
}
