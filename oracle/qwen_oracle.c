/*
 * CPU oracle for the Qwen2 decode path -- TEST INFRASTRUCTURE ONLY.
 * Never linked into the product. Interface and provenance: qwen_oracle.h.
 *
 * Built with -std=c11 -O2 -ffp-contract=off (oracle/Makefile) so that float
 * expressions round exactly as the reference's ISO C++20 build does.
 */
#define _GNU_SOURCE
#include "qwen_oracle.h"

#include <math.h>
#include <stdio.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ codecs
 * backends/cpu/cpu_backend.cpp:8-97 */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_bf16_to_f32(uint16_t v) { return u2f((uint32_t)v << 16); }

uint16_t orc_f32_to_bf16(float v) {
    uint32_t bits = f2u(v);
    if (isnan(v)) return (uint16_t)((bits >> 16) | 0x0040u);
    /* round half to even on the dropped 16 bits */
    uint32_t bias = 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + bias) >> 16);
}

float orc_f16_to_f32(uint16_t v) {
    uint32_t sign = (uint32_t)(v & 0x8000u) << 16;
    uint32_t e = (v >> 10) & 0x1Fu;
    uint32_t m = v & 0x3FFu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal half: shift the mantissa up until the implicit bit */
        int shift = 0;
        while ((m & 0x400u) == 0) { m <<= 1; ++shift; }
        return u2f(sign | (uint32_t)(113 - shift) << 23 | ((m & 0x3FFu) << 13));
    }
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t orc_f32_to_f16(float value) {
    uint32_t bits = f2u(value);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    uint32_t fexp = (bits >> 23) & 0xFFu;
    uint32_t mant = bits & 0x7FFFFFu;
    if (fexp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    int32_t e = (int32_t)fexp - 112; /* rebias 127 -> 15 */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return sign;
        /* result is a subnormal half: keep 24-bit significand, shift, RNE */
        uint32_t full = mant | 0x800000u;
        uint32_t sh = (uint32_t)(14 - e);
        uint32_t q = full >> sh;
        uint32_t rem = full & ((1u << sh) - 1u);
        uint32_t half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = mant >> 13;
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) {
        if (++q == 0x400u) {
            q = 0;
            if (++e >= 31) return (uint16_t)(sign | 0x7C00u);
        }
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | q);
}

void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}
void orc_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}

static float round_f16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

/* -------------------------------------------------------------- quantizers */

uint16_t orc_quant_scale_f16(float absmax, float qmax) {
    /* s = absmax / qmax in fp32, rounded to fp16; an all-zero group (or one
     * whose scale underflows fp16) uses 1.0, one that overflows uses the
     * largest finite half. */
    if (!(absmax > 0.0f)) return 0x3C00u;
    uint16_t h = orc_f32_to_f16(absmax / qmax);
    if ((h & 0x7FFFu) == 0) return 0x3C00u;
    if ((h & 0x7C00u) == 0x7C00u) return 0x7BFFu;
    return h;
}

static int8_t quant_one(float w, float s, float lo, float hi) {
    float r = roundf(w / s); /* ties away from zero, as std::round */
    if (r < lo) r = lo;
    if (r > hi) r = hi;
    return (int8_t)r;
}

void orc_q4_quantize(const float* w, int64_t n, int64_t k, int8_t* codes,
                     uint16_t* scales) {
    const int64_t groups = (k + 31) / 32;
    for (int64_t r = 0; r < n; ++r) {
        const float* row = w + r * k;
        for (int64_t g = 0; g < groups; ++g) {
            int64_t k0 = g * 32, k1 = k0 + 32 < k ? k0 + 32 : k;
            float absmax = 0.0f;
            for (int64_t i = k0; i < k1; ++i) {
                float a = fabsf(row[i]);
                if (a > absmax) absmax = a;
            }
            uint16_t sh = orc_quant_scale_f16(absmax, 7.0f);
            scales[r * groups + g] = sh;
            float s = orc_f16_to_f32(sh);
            for (int64_t i = k0; i < k1; ++i)
                codes[r * k + i] = quant_one(row[i], s, -8.0f, 7.0f);
        }
    }
}

void orc_q4_dequantize(const int8_t* codes, const uint16_t* scales, int64_t n,
                       int64_t k, float* w) {
    const int64_t groups = (k + 31) / 32;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i)
            w[r * k + i] = (float)codes[r * k + i] *
                           orc_f16_to_f32(scales[r * groups + i / 32]);
}

void orc_q8_quantize(const float* w, int64_t n, int64_t k, int8_t* codes,
                     uint16_t* scales) {
    for (int64_t r = 0; r < n; ++r) {
        const float* row = w + r * k;
        float absmax = 0.0f;
        for (int64_t i = 0; i < k; ++i) {
            float a = fabsf(row[i]);
            if (a > absmax) absmax = a;
        }
        uint16_t sh = orc_quant_scale_f16(absmax, 127.0f);
        scales[r] = sh;
        float s = orc_f16_to_f32(sh);
        for (int64_t i = 0; i < k; ++i)
            codes[r * k + i] = quant_one(row[i], s, -127.0f, 127.0f);
    }
}

void orc_q8_dequantize(const int8_t* codes, const uint16_t* scales, int64_t n,
                       int64_t k, float* w) {
    for (int64_t r = 0; r < n; ++r) {
        float s = orc_f16_to_f32(scales[r]);
        for (int64_t i = 0; i < k; ++i) w[r * k + i] = (float)codes[r * k + i] * s;
    }
}

/* -------------------------------------------------------------- primitives */

void orc_matvec(const float* w, const float* bias, const float* x,
                int64_t in_dim, int64_t out_dim, float* out) {
    /* qwen_model.cpp:21-31: acc starts at the bias, adds w*x in index order */
    for (int64_t o = 0; o < out_dim; ++o) {
        const float* row = w + o * in_dim;
        float acc = bias ? bias[o] : 0.0f;
        for (int64_t i = 0; i < in_dim; ++i) acc += row[i] * x[i];
        out[o] = acc;
    }
}

/* The same sum with the products added in descending index order: a second,
 * equally valid fp32 order (not the reference's), for measuring how much a
 * result depends on summation order alone. */
static void matvec_descending(const float* w, const float* bias, const float* x,
                              int64_t in_dim, int64_t out_dim, float* out) {
    for (int64_t o = 0; o < out_dim; ++o) {
        const float* row = w + o * in_dim;
        float acc = bias ? bias[o] : 0.0f;
        for (int64_t i = in_dim; i-- > 0;) acc += row[i] * x[i];
        out[o] = acc;
    }
}

typedef struct {
    const float *w, *bias, *x;
    int64_t in_dim, r0, r1;
    float* out;
    int descending;
} mv_job;

static void* mv_worker(void* p) {
    mv_job* j = (mv_job*)p;
    (j->descending ? matvec_descending : orc_matvec)(j->w + j->r0 * j->in_dim,
                                                     j->bias ? j->bias + j->r0 : NULL, j->x,
                                                     j->in_dim, j->r1 - j->r0, j->out + j->r0);
    return NULL;
}

static void matvec_rows(const float* w, const float* bias, const float* x, int64_t in_dim,
                        int64_t out_dim, float* out, int threads, int descending);

void orc_matvec_mt(const float* w, const float* bias, const float* x,
                   int64_t in_dim, int64_t out_dim, float* out, int threads) {
    matvec_rows(w, bias, x, in_dim, out_dim, out, threads, 0);
}

static void matvec_rows(const float* w, const float* bias, const float* x, int64_t in_dim,
                        int64_t out_dim, float* out, int threads, int descending) {
    if (threads <= 1 || out_dim * in_dim < (1 << 18)) {
        (descending ? matvec_descending : orc_matvec)(w, bias, x, in_dim, out_dim, out);
        return;
    }
    if (threads > 64) threads = 64;
    pthread_t tid[64];
    int spawned[64] = {0};
    mv_job jobs[64];
    for (int t = 0; t < threads; ++t) {
        jobs[t].w = w; jobs[t].bias = bias; jobs[t].x = x;
        jobs[t].in_dim = in_dim; jobs[t].out = out;
        jobs[t].r0 = out_dim * t / threads;
        jobs[t].r1 = out_dim * (t + 1) / threads;
        jobs[t].descending = descending;
    }
    for (int t = 1; t < threads; ++t)
        spawned[t] = pthread_create(&tid[t], NULL, mv_worker, &jobs[t]) == 0;
    mv_worker(&jobs[0]);
    for (int t = 1; t < threads; ++t) {
        if (spawned[t]) pthread_join(tid[t], NULL);
        else mv_worker(&jobs[t]); /* could not spawn: run it here */
    }
}

void orc_rmsnorm(const float* x, const float* weight, float eps, int64_t dim,
                 float* out) {
    /* qwen_model.cpp:33-39 */
    float ss = 0.0f;
    for (int64_t i = 0; i < dim; ++i) ss += x[i] * x[i];
    float scale = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int64_t i = 0; i < dim; ++i) out[i] = x[i] * scale * weight[i];
}

void orc_rope(float* vec, uint32_t head_dim, uint32_t pos, float theta) {
    /* qwen_model.cpp:41-54, rotate-half */
    uint32_t half = head_dim / 2;
    for (uint32_t i = 0; i < half; ++i) {
        float freq = powf(theta, -2.0f * (float)i / (float)head_dim);
        float angle = (float)pos * freq;
        float c = cosf(angle), s = sinf(angle);
        float a = vec[i], b = vec[i + half];
        vec[i] = a * c - b * s;
        vec[i + half] = b * c + a * s;
    }
}

/* Query heads [h0, h1) of orc_attention. */
static void attention_heads(const float* q, const float* keys, const float* values,
                            uint32_t context, uint32_t heads, uint32_t kv_heads,
                            uint32_t head_dim, uint32_t h0, uint32_t h1, float* out) {
    /* qwen_model.cpp:255-287 */
    const uint32_t group = heads / kv_heads;
    const size_t stride = (size_t)kv_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* scores = (float*)malloc(sizeof(float) * (context ? context : 1));
    for (uint32_t h = h0; h < h1; ++h) {
        const uint32_t kvh = h / group;
        const float* qh = q + (size_t)h * head_dim;
        float mx = -INFINITY;
        for (uint32_t t = 0; t < context; ++t) {
            const float* kt = keys + t * stride + (size_t)kvh * head_dim;
            float dot = 0.0f;
            for (uint32_t d = 0; d < head_dim; ++d) dot += qh[d] * kt[d];
            scores[t] = dot * scale;
            if (scores[t] > mx) mx = scores[t];
        }
        float denom = 0.0f;
        for (uint32_t t = 0; t < context; ++t) {
            scores[t] = expf(scores[t] - mx);
            denom += scores[t];
        }
        float* o = out + (size_t)h * head_dim;
        for (uint32_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
        for (uint32_t t = 0; t < context; ++t) {
            const float wgt = scores[t] / denom;
            const float* vt = values + t * stride + (size_t)kvh * head_dim;
            for (uint32_t d = 0; d < head_dim; ++d) o[d] += wgt * vt[d];
        }
    }
    free(scores);
}

void orc_attention(const float* q, const float* keys, const float* values,
                   uint32_t context, uint32_t heads, uint32_t kv_heads,
                   uint32_t head_dim, float* out) {
    attention_heads(q, keys, values, context, heads, kv_heads, head_dim, 0, heads, out);
}

typedef struct {
    const float *q, *keys, *values;
    uint32_t context, heads, kv_heads, head_dim, h0, h1;
    float* out;
} att_job;

static void* att_worker(void* p) {
    const att_job* j = (const att_job*)p;
    attention_heads(j->q, j->keys, j->values, j->context, j->heads, j->kv_heads,
                    j->head_dim, j->h0, j->h1, j->out);
    return NULL;
}

void orc_attention_mt(const float* q, const float* keys, const float* values,
                      uint32_t context, uint32_t heads, uint32_t kv_heads,
                      uint32_t head_dim, float* out, int threads) {
    /* each head is computed by the same code whatever thread runs it */
    if (threads > (int)heads) threads = (int)heads;
    if (threads > 64) threads = 64;
    if (threads <= 1 || (uint64_t)context * heads * head_dim < (1u << 18)) {
        orc_attention(q, keys, values, context, heads, kv_heads, head_dim, out);
        return;
    }
    pthread_t tid[64];
    int spawned[64] = {0};
    att_job jobs[64];
    for (int t = 0; t < threads; ++t) {
        att_job j = {q, keys, values, context, heads, kv_heads, head_dim,
                     (uint32_t)((uint64_t)heads * t / threads),
                     (uint32_t)((uint64_t)heads * (t + 1) / threads), out};
        jobs[t] = j;
    }
    for (int t = 1; t < threads; ++t)
        spawned[t] = pthread_create(&tid[t], NULL, att_worker, &jobs[t]) == 0;
    att_worker(&jobs[0]);
    for (int t = 1; t < threads; ++t) {
        if (spawned[t]) pthread_join(tid[t], NULL);
        else att_worker(&jobs[t]);
    }
}

/* ------------------------------------------------------------------- model */

struct orc_model {
    orc_config c;
    float* model_t[ORC_T_COUNT];      /* model-level tensors */
    float** layer_t[ORC_T_COUNT];     /* per-layer tensors */
    int threads;
    int f16_mirror;
    int descending;   /* forward matvecs add products in descending index order */
};

struct orc_seq {
    uint32_t max_tokens, length, kv_dim, layers;
    float** keys;   /* [layer] -> [max_tokens][kv_dim] */
    float** values;
    float* hidden;
};

static int is_layer_kind(int kind) {
    return kind >= ORC_T_INPUT_NORM && kind <= ORC_T_DOWN_W;
}

static uint64_t kind_numel(const orc_config* c, int kind) {
    const uint64_t h = c->hidden_size;
    const uint64_t q = (uint64_t)c->num_heads * c->head_dim;
    const uint64_t kv = (uint64_t)c->num_kv_heads * c->head_dim;
    const uint64_t I = c->intermediate_size, V = c->vocab_size;
    switch (kind) {
        case ORC_T_EMBED: return V * h;
        case ORC_T_INPUT_NORM: case ORC_T_POST_NORM: case ORC_T_FINAL_NORM: return h;
        case ORC_T_Q_W: return q * h;
        case ORC_T_Q_B: return q;
        case ORC_T_K_W: case ORC_T_V_W: return kv * h;
        case ORC_T_K_B: case ORC_T_V_B: return kv;
        case ORC_T_O_W: return h * q;
        case ORC_T_GATE_W: case ORC_T_UP_W: case ORC_T_DOWN_W: return I * h;
        case ORC_T_LM_HEAD: return c->tie_word_embeddings ? 0 : V * h;
    }
    return 0;
}

orc_model* orc_model_new(const orc_config* c) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    if (!m) return NULL;
    m->c = *c;
    m->threads = 1;
    for (int k = 0; k < ORC_T_COUNT; ++k) {
        uint64_t n = kind_numel(c, k);
        if (is_layer_kind(k)) {
            m->layer_t[k] = (float**)calloc(c->num_layers, sizeof(float*));
            for (uint32_t l = 0; l < c->num_layers; ++l) {
                m->layer_t[k][l] = (float*)calloc(n, sizeof(float));
                if (!m->layer_t[k][l]) { orc_model_free(m); return NULL; }
            }
        } else if (n) {
            m->model_t[k] = (float*)calloc(n, sizeof(float));
            if (!m->model_t[k]) { orc_model_free(m); return NULL; }
        }
    }
    return m;
}

void orc_model_free(orc_model* m) {
    if (!m) return;
    for (int k = 0; k < ORC_T_COUNT; ++k) {
        free(m->model_t[k]);
        if (m->layer_t[k]) {
            for (uint32_t l = 0; l < m->c.num_layers; ++l) free(m->layer_t[k][l]);
            free(m->layer_t[k]);
        }
    }
    free(m);
}

float* orc_model_tensor(orc_model* m, int kind, uint32_t layer) {
    if (kind < 0 || kind >= ORC_T_COUNT) return NULL;
    if (is_layer_kind(kind))
        return layer < m->c.num_layers ? m->layer_t[kind][layer] : NULL;
    return m->model_t[kind];
}

uint64_t orc_model_tensor_numel(const orc_model* m, int kind) {
    return kind_numel(&m->c, kind);
}

void orc_model_set_threads(orc_model* m, int threads) {
    m->threads = threads < 1 ? 1 : threads;
}

void orc_model_set_f16_mirror(orc_model* m, int on) { m->f16_mirror = on; }

void orc_model_set_descending_sums(orc_model* m, int on) { m->descending = on; }

orc_seq* orc_seq_new(const orc_model* m, uint32_t max_tokens) {
    orc_seq* s = (orc_seq*)calloc(1, sizeof(orc_seq));
    s->max_tokens = max_tokens;
    s->layers = m->c.num_layers;
    s->kv_dim = m->c.num_kv_heads * m->c.head_dim;
    s->keys = (float**)calloc(s->layers, sizeof(float*));
    s->values = (float**)calloc(s->layers, sizeof(float*));
    for (uint32_t l = 0; l < s->layers; ++l) {
        s->keys[l] = (float*)calloc((size_t)max_tokens * s->kv_dim + 1, sizeof(float));
        s->values[l] = (float*)calloc((size_t)max_tokens * s->kv_dim + 1, sizeof(float));
    }
    s->hidden = (float*)calloc(m->c.hidden_size, sizeof(float));
    return s;
}

void orc_seq_free(orc_seq* s) {
    if (!s) return;
    for (uint32_t l = 0; l < s->layers; ++l) { free(s->keys[l]); free(s->values[l]); }
    free(s->keys); free(s->values); free(s->hidden); free(s);
}

uint32_t orc_seq_length(const orc_seq* s) { return s->length; }
const float* orc_seq_hidden(const orc_seq* s) { return s->hidden; }

static void mirror_round(const orc_model* m, float* v, size_t n) {
    if (!m->f16_mirror) return;
    for (size_t i = 0; i < n; ++i) v[i] = round_f16(v[i]);
}

/* qwen_model.cpp:212-308 */
static void forward_token(const orc_model* m, orc_seq* s, uint32_t token,
                          uint32_t pos) {
    const orc_config* c = &m->c;
    const size_t h = c->hidden_size;
    const size_t qd = (size_t)c->num_heads * c->head_dim;
    const size_t kvd = (size_t)c->num_kv_heads * c->head_dim;
    const size_t I = c->intermediate_size;
    const int T = m->threads;
    float* hidden = s->hidden;
    memcpy(hidden, m->model_t[ORC_T_EMBED] + (size_t)token * h, h * sizeof(float));

    float* normed = (float*)malloc(h * sizeof(float));
    float* q = (float*)malloc(qd * sizeof(float));
    float* attn = (float*)malloc(qd * sizeof(float));
    float* proj = (float*)malloc(h * sizeof(float));
    float* gate = (float*)malloc(I * sizeof(float));
    float* up = (float*)malloc(I * sizeof(float));

    for (uint32_t l = 0; l < c->num_layers; ++l) {
#define LT(kind) (m->layer_t[kind][l])
        orc_rmsnorm(hidden, LT(ORC_T_INPUT_NORM), c->rms_norm_eps, h, normed);
        mirror_round(m, normed, h);
        matvec_rows(LT(ORC_T_Q_W), LT(ORC_T_Q_B), normed, h, qd, q, T, m->descending);
        float* k = s->keys[l] + (size_t)pos * kvd;
        float* v = s->values[l] + (size_t)pos * kvd;
        matvec_rows(LT(ORC_T_K_W), LT(ORC_T_K_B), normed, h, kvd, k, T, m->descending);
        matvec_rows(LT(ORC_T_V_W), LT(ORC_T_V_B), normed, h, kvd, v, T, m->descending);
        for (uint32_t hh = 0; hh < c->num_heads; ++hh)
            orc_rope(q + (size_t)hh * c->head_dim, c->head_dim, pos, c->rope_theta);
        for (uint32_t hh = 0; hh < c->num_kv_heads; ++hh)
            orc_rope(k + (size_t)hh * c->head_dim, c->head_dim, pos, c->rope_theta);
        mirror_round(m, k, kvd);
        mirror_round(m, v, kvd);
        orc_attention_mt(q, s->keys[l], s->values[l], pos + 1, c->num_heads,
                         c->num_kv_heads, c->head_dim, attn, T);
        mirror_round(m, attn, qd);
        matvec_rows(LT(ORC_T_O_W), NULL, attn, qd, h, proj, T, m->descending);
        for (size_t i = 0; i < h; ++i) hidden[i] += proj[i];

        orc_rmsnorm(hidden, LT(ORC_T_POST_NORM), c->rms_norm_eps, h, normed);
        mirror_round(m, normed, h);
        matvec_rows(LT(ORC_T_GATE_W), NULL, normed, h, I, gate, T, m->descending);
        matvec_rows(LT(ORC_T_UP_W), NULL, normed, h, I, up, T, m->descending);
        for (size_t i = 0; i < I; ++i) {
            const float x = gate[i];
            const float silu = x / (1.0f + expf(-x));
            gate[i] = silu * up[i];
        }
        mirror_round(m, gate, I);
        matvec_rows(LT(ORC_T_DOWN_W), NULL, gate, I, h, proj, T, m->descending);
        for (size_t i = 0; i < h; ++i) hidden[i] += proj[i];
#undef LT
    }
    free(normed); free(q); free(attn); free(proj); free(gate); free(up);
}

/* qwen_model.cpp:310-331 */
static int logits_from_hidden(const orc_model* m, const float* hidden,
                              float* logits) {
    const orc_config* c = &m->c;
    float* normed = (float*)malloc(c->hidden_size * sizeof(float));
    orc_rmsnorm(hidden, m->model_t[ORC_T_FINAL_NORM], c->rms_norm_eps,
                c->hidden_size, normed);
    mirror_round(m, normed, c->hidden_size);
    const float* head = c->tie_word_embeddings ? m->model_t[ORC_T_EMBED]
                                               : m->model_t[ORC_T_LM_HEAD];
    matvec_rows(head, NULL, normed, c->hidden_size, c->vocab_size, logits,
                m->threads, m->descending);
    free(normed);
    for (uint32_t i = 0; i < c->vocab_size; ++i)
        if (!isfinite(logits[i])) return ORC_INFERENCE_FAILED;
    return ORC_OK;
}

int orc_prefill(const orc_model* m, orc_seq* s, const uint32_t* tokens,
                size_t n, float* logits) {
    /* qwen_model.cpp:333-360 */
    if (n == 0) return ORC_INVALID_REQUEST;
    if (s->length != 0) return ORC_INTERNAL_ERROR;
    if (n > s->max_tokens) return ORC_CONTEXT_LENGTH_EXCEEDED;
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= m->c.vocab_size) return ORC_INVALID_REQUEST;
    for (size_t i = 0; i < n; ++i) {
        forward_token(m, s, tokens[i], (uint32_t)i);
        s->length += 1;
    }
    return logits_from_hidden(m, s->hidden, logits);
}

int orc_decode(const orc_model* m, orc_seq* s, uint32_t token, float* logits) {
    /* qwen_model.cpp:398-412 */
    if (token >= m->c.vocab_size) return ORC_INVALID_REQUEST;
    if (s->length >= s->max_tokens) return ORC_CONTEXT_LENGTH_EXCEEDED;
    forward_token(m, s, token, s->length);
    s->length += 1;
    return logits_from_hidden(m, s->hidden, logits);
}

/* ------------------------------------------------------------ tiny weights
 * tests/testutil/tiny_model.cpp:14-24 (LCG) and 52-116 (tensors written in
 * std::map order, i.e. byte-lexicographic names; "norm" tensors are 1.0). */

typedef struct { const char* suffix; int kind; } tiny_name;

static int name_cmp(const void* a, const void* b) {
    return strcmp(*(const char* const*)a, *(const char* const*)b);
}

void orc_fill_tiny_weights(orc_model* m, uint64_t seed) {
    static const tiny_name layer_names[] = {
        {"input_layernorm.weight", ORC_T_INPUT_NORM},
        {"self_attn.q_proj.weight", ORC_T_Q_W},
        {"self_attn.q_proj.bias", ORC_T_Q_B},
        {"self_attn.k_proj.weight", ORC_T_K_W},
        {"self_attn.k_proj.bias", ORC_T_K_B},
        {"self_attn.v_proj.weight", ORC_T_V_W},
        {"self_attn.v_proj.bias", ORC_T_V_B},
        {"self_attn.o_proj.weight", ORC_T_O_W},
        {"post_attention_layernorm.weight", ORC_T_POST_NORM},
        {"mlp.gate_proj.weight", ORC_T_GATE_W},
        {"mlp.up_proj.weight", ORC_T_UP_W},
        {"mlp.down_proj.weight", ORC_T_DOWN_W},
    };
    const uint32_t L = m->c.num_layers;
    const size_t count = 2 + (size_t)L * 12;
    char** names = (char**)malloc(count * sizeof(char*));
    size_t n = 0;
    names[n++] = strdup("model.embed_tokens.weight");
    names[n++] = strdup("model.norm.weight");
    for (uint32_t l = 0; l < L; ++l)
        for (size_t j = 0; j < 12; ++j) {
            char buf[128];
            snprintf(buf, sizeof buf, "model.layers.%u.%s", l, layer_names[j].suffix);
            names[n++] = strdup(buf);
        }
    qsort(names, n, sizeof(char*), name_cmp);

    uint64_t state = seed;
    for (size_t i = 0; i < n; ++i) {
        float* dst = NULL;
        uint64_t numel = 0;
        int is_norm = strstr(names[i], "norm") != NULL;
        if (strcmp(names[i], "model.embed_tokens.weight") == 0) {
            dst = m->model_t[ORC_T_EMBED]; numel = kind_numel(&m->c, ORC_T_EMBED);
        } else if (strcmp(names[i], "model.norm.weight") == 0) {
            dst = m->model_t[ORC_T_FINAL_NORM]; numel = m->c.hidden_size;
        } else {
            unsigned l = 0;
            int off = 0;
            sscanf(names[i], "model.layers.%u.%n", &l, &off);
            for (size_t j = 0; j < 12; ++j)
                if (strcmp(names[i] + off, layer_names[j].suffix) == 0) {
                    dst = m->layer_t[layer_names[j].kind][l];
                    numel = kind_numel(&m->c, layer_names[j].kind);
                }
        }
        for (uint64_t e = 0; e < numel; ++e) {
            float v = 1.0f;
            if (!is_norm) {
                state = state * 6364136223846793005ULL + 1442695040888963407ULL;
                v = ((float)(state >> 40) / (float)(1 << 24) - 0.5f) * 0.2f;
            }
            dst[e] = v;
        }
        free(names[i]);
    }
    free(names);
}

/* ----------------------------------------------------------------- sampler */

void orc_mt64_seed(orc_mt64* g, uint64_t seed) {
    g->mt[0] = seed;
    for (int i = 1; i < 312; ++i)
        g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
    g->idx = 312;
}

uint64_t orc_mt64_next(orc_mt64* g) {
    const uint64_t upper = 0xFFFFFFFF80000000ULL, lower = 0x7FFFFFFFULL;
    if (g->idx >= 312) {
        for (int i = 0; i < 312; ++i) {
            uint64_t y = (g->mt[i] & upper) | (g->mt[(i + 1) % 312] & lower);
            uint64_t v = g->mt[(i + 156) % 312] ^ (y >> 1);
            if (y & 1) v ^= 0xB5026F5AA96619E9ULL;
            g->mt[i] = v;
        }
        g->idx = 0;
    }
    uint64_t x = g->mt[g->idx++];
    x ^= (x >> 29) & 0x5555555555555555ULL;
    x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
    x ^= (x << 37) & 0xFFF7EEE000000000ULL;
    x ^= x >> 43;
    return x;
}

double orc_mt64_canonical(orc_mt64* g) {
    /* generate_canonical<double, 53> with a 64-bit engine: one draw, divided
     * by 2^64, values rounding up to 1.0 replaced by the largest double < 1 */
    double r = (double)orc_mt64_next(g) / 18446744073709551616.0;
    if (r >= 1.0) r = nextafter(1.0, 0.0);
    return r;
}

struct orc_sampler {
    float temperature, top_p;
    uint32_t top_k;
    orc_mt64 rng;
};

orc_sampler* orc_sampler_new(float temperature, float top_p, uint32_t top_k,
                             uint64_t seed) {
    orc_sampler* s = (orc_sampler*)calloc(1, sizeof(orc_sampler));
    s->temperature = temperature;
    s->top_p = top_p;
    s->top_k = top_k;
    orc_mt64_seed(&s->rng, seed);
    return s;
}

void orc_sampler_free(orc_sampler* s) { free(s); }

uint32_t orc_argmax(const float* logits, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
        if (logits[best] < logits[i]) best = i;
    return (uint32_t)best;
}

/* Stable descending order by logit: merge sort on indices. */
static void sort_desc(uint32_t* idx, uint32_t* tmp, const float* l, size_t n) {
    if (n < 2) return;
    size_t h = n / 2;
    sort_desc(idx, tmp, l, h);
    sort_desc(idx + h, tmp, l, n - h);
    size_t a = 0, b = h, o = 0;
    while (a < h && b < n) {
        /* take from the right run only when strictly greater (stability) */
        if (l[idx[b]] > l[idx[a]]) tmp[o++] = idx[b++];
        else tmp[o++] = idx[a++];
    }
    while (a < h) tmp[o++] = idx[a++];
    while (b < n) tmp[o++] = idx[b++];
    memcpy(idx, tmp, n * sizeof(uint32_t));
}

int orc_sample(orc_sampler* s, const float* logits, size_t n, uint32_t* out) {
    if (n == 0) return ORC_INFERENCE_FAILED;
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(logits[i])) return ORC_INFERENCE_FAILED;
    if (s->temperature == 0.0f) {
        *out = orc_argmax(logits, n);
        return ORC_OK;
    }
    uint32_t* idx = (uint32_t*)malloc(n * sizeof(uint32_t));
    uint32_t* tmp = (uint32_t*)malloc(n * sizeof(uint32_t));
    for (size_t i = 0; i < n; ++i) idx[i] = (uint32_t)i;
    sort_desc(idx, tmp, logits, n);
    size_t cand = n;
    if (s->top_k > 0 && s->top_k < cand) cand = s->top_k;
    const float inv_temp = 1.0f / s->temperature;
    const float mx = logits[idx[0]];
    double* probs = (double*)malloc(cand * sizeof(double));
    double denom = 0.0;
    for (size_t i = 0; i < cand; ++i) {
        probs[i] = exp((double)(logits[idx[i]] - mx) * inv_temp);
        denom += probs[i];
    }
    size_t nucleus = cand;
    if (s->top_p < 1.0f) {
        double cum = 0.0;
        for (size_t i = 0; i < cand; ++i) {
            cum += probs[i] / denom;
            if (cum >= (double)s->top_p) { nucleus = i + 1; break; }
        }
    }
    double mass = 0.0;
    for (size_t i = 0; i < nucleus; ++i) mass += probs[i];
    double r = orc_mt64_canonical(&s->rng) * (mass - 0.0) + 0.0;
    double acc = 0.0;
    uint32_t tok = idx[nucleus - 1];
    for (size_t i = 0; i < nucleus; ++i) {
        acc += probs[i];
        if (r <= acc) { tok = idx[i]; break; }
    }
    *out = tok;
    free(idx); free(tmp); free(probs);
    return ORC_OK;
}

/* ------------------------------------------------------- synthetic weights */

static uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

void orc_synth_normal(uint64_t seed, uint64_t stream_id, uint64_t first,
                      uint64_t count, float sigma, float* out) {
    /* Box-Muller on pairs: element 2p uses the cosine branch, 2p+1 the sine
     * branch of pair p; each pair takes two splitmix64 outputs. */
    const uint64_t key = splitmix64(seed ^ splitmix64(stream_id));
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t e = first; e < first + count; ++e) {
        uint64_t p = e >> 1;
        uint64_t a = splitmix64(key + 2 * p), b = splitmix64(key + 2 * p + 1);
        double u1 = (double)((a >> 11) + 1) * (1.0 / 9007199254740992.0);
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        double rad = sqrt(-2.0 * log(u1));
        double z = (e & 1) ? rad * sin(two_pi * u2) : rad * cos(two_pi * u2);
        out[e - first] = (float)(z * (double)sigma);
    }
}

void orc_synth_tokens(uint64_t seed, uint64_t stream_id, uint64_t count,
                      uint32_t n, uint32_t* out) {
    const uint64_t key = splitmix64(seed ^ splitmix64(stream_id));
    for (uint64_t i = 0; i < count; ++i) {
        uint64_t u = splitmix64(key + i) >> 32;
        out[i] = (uint32_t)((u * (uint64_t)n) >> 32);
    }
}
