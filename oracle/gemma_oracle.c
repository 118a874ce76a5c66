/*
 * gemma_oracle.c -- CPU restatement of gemma.hs's GPU decode step.
 *
 * TEST INFRASTRUCTURE ONLY (see gemma_oracle.h).  Built with
 * -ffp-contract=off so that "sum + w*x" rounds twice, as the WGSL source
 * reads.  All arithmetic is f32 unless a function says otherwise.
 *
 * Pinning (what fixes each function besides this restatement itself; the
 * checks live in tests/test_oracle.py):
 *   orc_f16_to_f32 / orc_q4_0_dequant : exhaustive over all 65536 fp16 bit
 *       patterns against numpy float16->float32 with FTZ applied, plus
 *       hand-built blocks -- pinned.
 *   orc_q4_0_matvec, orc_f32_matvec    : brute-force fp64 dot products and the
 *       reference's golden linear_* fixture -- pinned.
 *   orc_rmsnorm_tree / _seq / qk_norm  : golden rmsnorm_* fixture and the
 *       closed form [1,2,3,4] -> [0.3651,...] of test/GemmaSpec.hs:176-190 --
 *       pinned.
 *   orc_rope                            : closed forms (pos 0 identity, a
 *       single pair rotated by a known angle, norm preservation) -- pinned.
 *       The reference fixture rope_output_pos1 is interleaved RoPE and does
 *       not apply to the split-half shader.
 *   orc_attention                       : golden attention_* fixture, Leff=1
 *       => o = V, brute-force softmax in fp64 -- pinned.
 *   orc_gelu_tanh / orc_geglu           : closed form of the tanh formula in
 *       fp64, and the golden gelu_output within the +-2e-4 bound the
 *       reference itself allows (the fixture is erf-GELU) -- pinned.
 *   orc_argmax                          : numpy.argmax (first max) -- pinned.
 *   orc_softcap                         : the reference's runMatmulQ4_0DSL
 *       body is absent, so the Gemma-2 form cap*tanh(y/cap) is pinned by the
 *       properties that fix it: odd, |f| < cap and |f(y)| <= |y|, the Taylor
 *       terms y - y^3/(3cap^2) at 0, saturation at +-cap, monotone, and
 *       f(cap*atanh(1/2)) = cap/2; planted wrong forms fail them -- pinned.
 *   orc_philox4x32_10                   : the published Random123
 *       known-answer vectors for philox4x32-10 -- pinned.
 *   orc_sample                          : inversion sampling; pinned by the
 *       closed forms of equal logits (index = floor(u n)) and of a single
 *       dominant logit, and by frequencies against softmax on small n.
 *       There is no reference counterpart: the reference's temperature
 *       path is an argmax (app/Main.hs:505-507).
 *   orc_sample_top_k                    : the same draw over the k largest
 *       logits in rank order; pinned by k = 1 (the first maximum for every
 *       u), equal logits (index floor(u k)), k = n on logits that decrease
 *       with the index (orc_sample's pick for every u), the picked value's
 *       invariance under a permutation of distinct logits, and frequencies
 *       against a numpy top-k softmax.  No reference counterpart.
 *   orc_step / orc_generate             : composition of the above; checked
 *       against an independent float64 numpy restatement in the tests.
 */
#include "gemma_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* IEEE binary16 -> binary32.  Subnormal inputs flush to a signed zero when
 * ftz != 0, as src/Gemma/GGUF.hs:797-820 (halfToFloat) does; with ftz == 0
 * they are decoded exactly (IEEE mode). */
float orc_f16_to_f32(uint16_t h, int ftz) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (m == 0 || ftz) {
            bits = sign;
        } else {
            /* exact subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-08f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* Q4_0 block = {f16 d (LE), qs[16]}; element e<16 -> qs[e]&0xF, e>=16 ->
 * qs[e-16]>>4; value (q - 8) * d.  src/Gemma/GGUF.hs:726-760 (loadQ4_0Tensor),
 * block size 18 from src/Gemma/GGUF.hs:881. */
static inline float q4_elem(const uint8_t* blk, int e, float d) {
    uint8_t b = blk[2 + (e & 15)];
    int q = (e < 16) ? (b & 0x0F) : (b >> 4);
    return ((float)q - 8.0f) * d;
}

static inline float q4_scale(const uint8_t* blk, int ftz) {
    uint16_t h = (uint16_t)(blk[0] | (blk[1] << 8));
    return orc_f16_to_f32(h, ftz);
}

void orc_q4_0_dequant(const uint8_t* raw, size_t n_blocks, int ftz, float* out) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = raw + b * 18;
        float d = q4_scale(blk, ftz);
        for (int e = 0; e < 32; ++e) out[b * 32 + e] = q4_elem(blk, e, d);
    }
}

/* y = W x with W in GGUF Q4_0 rows (cols/32 blocks per row): each row is
 * dequantised element by element and accumulated sequentially in f32, the
 * order of the reference's fp32 matvec shaders (qkvProjectionShader,
 * src/Gemma/Layers/AttentionGPU.hs:143-195; linearKernelFP32,
 * src/Gemma/Layers/LinearDSL.hs:217-278) applied to the dequantised weights
 * of loadQ4_0Tensor.  The API mirrors runLinearQ4
 * (src/Gemma/Layers/LinearQ4.hs:41-48). */
void orc_q4_0_matvec(const uint8_t* raw, const float* x, int rows, int cols, int ftz, float* y) {
    int nb = cols / 32;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const uint8_t* row = raw + (size_t)r * nb * 18;
        float sum = 0.0f;
        for (int b = 0; b < nb; ++b) {
            const uint8_t* blk = row + (size_t)b * 18;
            float d = q4_scale(blk, ftz);
            for (int e = 0; e < 32; ++e) {
                float w = q4_elem(blk, e, d);
                sum = sum + w * x[b * 32 + e];
            }
        }
        y[r] = sum;
    }
}

/* fp64 accumulation of the same products, plus sum |w x| for error bounds. */
void orc_q4_0_matvec_f64(const uint8_t* raw, const float* x, int rows, int cols, int ftz,
                         double* y, double* abs_y) {
    int nb = cols / 32;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const uint8_t* row = raw + (size_t)r * nb * 18;
        double sum = 0.0, asum = 0.0;
        for (int b = 0; b < nb; ++b) {
            const uint8_t* blk = row + (size_t)b * 18;
            float d = q4_scale(blk, ftz);
            for (int e = 0; e < 32; ++e) {
                double p = (double)q4_elem(blk, e, d) * (double)x[b * 32 + e];
                sum += p;
                asum += fabs(p);
            }
        }
        y[r] = sum;
        if (abs_y) abs_y[r] = asum;
    }
}

/* Sequential f32 matvec, src/Gemma/Layers/AttentionGPU.hs:143-195 and
 * :445-471 (outputProjectionShader), src/Gemma/Layers/LinearDSL.hs:217-278
 * (scalar path). */
void orc_f32_matvec(const float* w, const float* x, int rows, int cols, float* y) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* wr = w + (size_t)r * cols;
        float sum = 0.0f;
        for (int i = 0; i < cols; ++i) sum = sum + wr[i] * x[i];
        y[r] = sum;
    }
}

/* Standalone RMSNorm, src/Gemma/Layers/RMSNorm.hs:45-154 (scalar path):
 * 256 strided partial sums of x^2, LDS tree reduction with halving stride,
 * rms = sqrt(sum/n + eps), y = (x / rms) * (1 + w) (zero-centred) or
 * (x / rms) * w. */
void orc_rmsnorm_tree(const float* x, const float* w, int n, float eps, int zc, float* y) {
    float part[256];
    for (int t = 0; t < 256; ++t) {
        float s = 0.0f;
        for (int i = t; i < n; i += 256) s = s + x[i] * x[i];
        part[t] = s;
    }
    for (int stride = 128; stride > 0; stride /= 2)
        for (int t = 0; t < stride; ++t) part[t] = part[t] + part[t + stride];
    float mean_sq = part[0] / (float)n;
    float rms = sqrtf(mean_sq + eps);
    for (int i = 0; i < n; ++i) y[i] = zc ? (x[i] / rms) * (1.0f + w[i]) : (x[i] / rms) * w[i];
}

/* RMS computed sequentially inside the fused kernels:
 * rmsNormGateUpFusedShader (src/Gemma/Layers/MLP.hs:507-622, scalar path
 * 553-558) and rmsNormLinearFusedShader (src/Gemma/Layers/RMSNorm.hs:343-386).
 * rms = sqrt(sum/n + eps); normalized = (x / rms) * (1 + w). */
void orc_rmsnorm_seq(const float* x, const float* w, int n, float eps, int zc, float* y) {
    float s = 0.0f;
    for (int i = 0; i < n; ++i) s = s + x[i] * x[i];
    float rms = sqrtf(s / (float)n + eps);
    for (int i = 0; i < n; ++i) y[i] = zc ? (x[i] / rms) * (1.0f + w[i]) : (x[i] / rms) * w[i];
}

/* Per-head RMSNorm over head_dim, src/Gemma/Layers/AttentionGPU.hs:218-257
 * (qkNormShader).  Applied to the n_heads actually present (quirk Q1: the
 * reference runs the Q-head shader over the K buffer; the out-of-range heads
 * are not a parity target). */
void orc_qk_norm(const float* x, const float* w, int n_heads, int hd, float eps, int zc, float* y) {
    for (int h = 0; h < n_heads; ++h) {
        const float* xh = x + h * hd;
        float s = 0.0f;
        for (int i = 0; i < hd; ++i) s = s + xh[i] * xh[i];
        float rms = sqrtf(s / (float)hd + eps);
        for (int i = 0; i < hd; ++i)
            y[h * hd + i] = zc ? (xh[i] / rms) * (1.0f + w[i]) : (xh[i] / rms) * w[i];
    }
}

/* Split-half RoPE, src/Gemma/Layers/AttentionGPU.hs:68-115 (ropeShader):
 * for i < hd/2: f = 1/pow(theta, f32(2i)/f32(hd)), a = pos * f,
 * y_i = x_i cos a - x_{i+hd/2} sin a, y_{i+hd/2} = x_i sin a + x_{i+hd/2} cos a.
 * Safe in place (x == y). */
void orc_rope(const float* x, int n_heads, int hd, float theta, int pos, float* y) {
    int half = hd / 2;
    for (int h = 0; h < n_heads; ++h) {
        for (int i = 0; i < half; ++i) {
            int idx = h * hd + i;
            float a = x[idx], b = x[idx + half];
            float freq_exp = (float)(i * 2) / (float)hd;
            float freq = 1.0f / powf(theta, freq_exp);
            float ang = (float)pos * freq;
            float c = cosf(ang), s = sinf(ang);
            y[idx] = a * c - b * s;
            y[idx + half] = a * s + b * c;
        }
    }
}

/* Cached GQA attention for one query token,
 * src/Gemma/Layers/AttentionGPU.hs:292-352 (attentionScoresShader) and
 * :382-423 (attentionOutputShader): kv head = h / (nq/nkv);
 * s_p = (q_h . K_p) * (1/sqrt(hd)) for p in [p_begin, p_end); softmax with
 * max initialised to -1e9, exp(s - max), sum, divide; o = sum_p s_p V_p
 * accumulated over p in order.  Cache layout [pos][nkv][hd]. */
void orc_attention(const float* q, const float* k_cache, const float* v_cache, int nq, int nkv,
                   int hd, int p_begin, int p_end, float* out) {
    int n = p_end - p_begin;
    float scale = 1.0f / sqrtf((float)hd);
    float* sc = (float*)malloc(sizeof(float) * (n > 0 ? n : 1));
    int grp = nq / nkv;
    for (int h = 0; h < nq; ++h) {
        int g = h / grp;
        const float* qh = q + h * hd;
        float mx = -1e9f;
        for (int j = 0; j < n; ++j) {
            const float* kp = k_cache + ((size_t)(p_begin + j) * nkv + g) * hd;
            float dot = 0.0f;
            for (int i = 0; i < hd; ++i) dot = dot + qh[i] * kp[i];
            float s = dot * scale;
            sc[j] = s;
            mx = fmaxf(mx, s);
        }
        float se = 0.0f;
        for (int j = 0; j < n; ++j) {
            float e = expf(sc[j] - mx);
            sc[j] = e;
            se = se + e;
        }
        for (int j = 0; j < n; ++j) sc[j] = sc[j] / se;
        for (int d = 0; d < hd; ++d) {
            float s = 0.0f;
            for (int j = 0; j < n; ++j) {
                const float* vp = v_cache + ((size_t)(p_begin + j) * nkv + g) * hd;
                s = s + sc[j] * vp[d];
            }
            out[h * hd + d] = s;
        }
    }
    free(sc);
}

/* GELU(tanh) with the +-10 clamp, src/Gemma/Layers/MLP.hs:384-447
 * (geluMultiplyFusedShader, scalar path): x * 0.5 * (1 + tanh(clamp(
 * 0.7978845608 * (x + 0.044715 * x^3), -10, 10))). */
float orc_gelu_tanh(float x) {
    float x3 = x * x * x;
    float t = 0.7978845608f * (x + 0.044715f * x3);
    if (t < -10.0f) t = -10.0f;
    if (t > 10.0f) t = 10.0f;
    return x * 0.5f * (1.0f + tanhf(t));
}

void orc_geglu(const float* g, const float* u, int n, float* h) {
    for (int i = 0; i < n; ++i) h[i] = orc_gelu_tanh(g[i]) * u[i];
}

/* Greedy sampling: first maximum, app/Main.hs:488-507 (sampleToken /
 * sampleWithTemperature, which also returns the argmax). */
int32_t orc_argmax(const float* v, int n) {
    int32_t best = 0;
    for (int i = 1; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

/* Gemma-2 style soft-cap cap*tanh(y/cap); the runLinearQ4 flag
 * (src/Gemma/Layers/LinearQ4.hs:37-48).  Pinned by its invariants (see the
 * header comment). */
void orc_softcap(float* y, int n, float cap) {
    for (int i = 0; i < n; ++i) y[i] = cap * tanhf(y[i] / cap);
}

/* ------------------------------------------------------------------ */
/* Whole-model restatement: runGemmaInferenceCached,
 * src/Gemma/Model.hs:1313-1437, and the block
 * src/Gemma/Layers/TransformerBlockGPU.hs:92-461. */

typedef struct {
    int dtype;
    size_t nbytes;
    void* data;
} orc_tensor;

enum {
    T_ATTN_NORM,
    T_Q,
    T_K,
    T_V,
    T_QN,
    T_KN,
    T_O,
    T_POST_ATTN,
    T_FFN_NORM,
    T_GATE,
    T_UP,
    T_DOWN,
    T_POST_FFN,
    T_NLAYER
};

static const char* k_layer_names[T_NLAYER] = {
    "attn_norm.weight",   "attn_q.weight",        "attn_k.weight",     "attn_v.weight",
    "attn_q_norm.weight", "attn_k_norm.weight",   "attn_output.weight", "post_attention_norm.weight",
    "ffn_norm.weight",    "ffn_gate.weight",      "ffn_up.weight",     "ffn_down.weight",
    "post_ffw_norm.weight"};

struct orc_model {
    orc_config c;
    orc_tensor embd, out_norm;
    orc_tensor lm;  /* output.weight: untied LM head (optional) */
    orc_tensor* lt; /* [n_layers][T_NLAYER] */
    float* kc;      /* [n_layers][max_seq][nkv][hd] */
    float* vc;
};

orc_model* orc_model_create(const orc_config* cfg) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->c = *cfg;
    m->lt = (orc_tensor*)calloc((size_t)cfg->n_layers * T_NLAYER, sizeof(orc_tensor));
    size_t kv = (size_t)cfg->n_layers * cfg->max_seq * cfg->n_kv_heads * cfg->head_dim;
    m->kc = (float*)calloc(kv, sizeof(float));
    m->vc = (float*)calloc(kv, sizeof(float));
    return m;
}

static void free_tensor(orc_tensor* t) {
    free(t->data);
    t->data = NULL;
}

void orc_model_destroy(orc_model* m) {
    if (!m) return;
    free_tensor(&m->embd);
    free_tensor(&m->out_norm);
    free_tensor(&m->lm);
    for (int i = 0; i < m->c.n_layers * T_NLAYER; ++i) free_tensor(&m->lt[i]);
    free(m->lt);
    free(m->kc);
    free(m->vc);
    free(m);
}

void orc_model_reset(orc_model* m) {
    size_t kv = (size_t)m->c.n_layers * m->c.max_seq * m->c.n_kv_heads * m->c.head_dim;
    memset(m->kc, 0, kv * sizeof(float));
    memset(m->vc, 0, kv * sizeof(float));
}

int orc_model_set_kv(orc_model* m, int layer, int n_pos, const float* k, const float* v) {
    const orc_config* c = &m->c;
    if (layer < 0 || layer >= c->n_layers || n_pos < 0 || n_pos > c->max_seq) return -1;
    const size_t row = (size_t)c->n_kv_heads * c->head_dim, kv_layer = (size_t)c->max_seq * row;
    memcpy(m->kc + layer * kv_layer, k, sizeof(float) * row * n_pos);
    memcpy(m->vc + layer * kv_layer, v, sizeof(float) * row * n_pos);
    return 0;
}

int orc_model_set_tensor(orc_model* m, const char* name, int dtype, const void* data, size_t nbytes) {
    orc_tensor* t = NULL;
    if (strcmp(name, "token_embd.weight") == 0) {
        t = &m->embd;
    } else if (strcmp(name, "output_norm.weight") == 0) {
        t = &m->out_norm;
    } else if (strcmp(name, "output.weight") == 0) {
        t = &m->lm;
    } else if (strncmp(name, "blk.", 4) == 0) {
        char* end = NULL;
        long l = strtol(name + 4, &end, 10);
        if (!end || *end != '.' || l < 0 || l >= m->c.n_layers) return -1;
        for (int k = 0; k < T_NLAYER; ++k)
            if (strcmp(end + 1, k_layer_names[k]) == 0) t = &m->lt[l * T_NLAYER + k];
    }
    if (!t) return -2;
    free_tensor(t);
    t->data = malloc(nbytes);
    memcpy(t->data, data, nbytes);
    t->nbytes = nbytes;
    t->dtype = dtype;
    return 0;
}

static int ftz_of(const orc_model* m) { return (m->c.flags & ORC_IEEE_SCALES) ? 0 : 1; }

static void matvec_t(const orc_model* m, const orc_tensor* t, const float* x, int rows, int cols,
                     float* y) {
    if (t->dtype == ORC_Q4_0)
        orc_q4_0_matvec((const uint8_t*)t->data, x, rows, cols, ftz_of(m), y);
    else
        orc_f32_matvec((const float*)t->data, x, rows, cols, y);
}

static int layer_is_global(const orc_config* c, int l) {
    if (c->global_every <= 0) return 1;
    return ((l + 1) % c->global_every) == 0;
}

int orc_step(orc_model* m, int32_t token, int32_t pos, float* logits, float* layer_out) {
    const orc_config* c = &m->c;
    int H = c->hidden, nq = c->n_heads, nkv = c->n_kv_heads, hd = c->head_dim, F = c->ffn;
    int zc = (c->flags & ORC_ZERO_CENTERED) ? 1 : 0;
    float eps = c->rms_eps;
    if (token < 0 || token >= c->vocab || pos < 0 || pos >= c->max_seq) return -1;
    if (!m->embd.data || !m->out_norm.data) return -2;

    float* x = (float*)malloc(sizeof(float) * H);
    float* xn = (float*)malloc(sizeof(float) * H);
    float* x1 = (float*)malloc(sizeof(float) * H);
    float* a = (float*)malloc(sizeof(float) * H);
    float* q = (float*)malloc(sizeof(float) * nq * hd);
    float* k = (float*)malloc(sizeof(float) * nkv * hd);
    float* v = (float*)malloc(sizeof(float) * nkv * hd);
    float* o = (float*)malloc(sizeof(float) * nq * hd);
    float* g = (float*)malloc(sizeof(float) * F);
    float* u = (float*)malloc(sizeof(float) * F);
    float* hh = (float*)malloc(sizeof(float) * F);
    float* lg = logits ? logits : (float*)malloc(sizeof(float) * c->vocab);

    /* embedding (src/Gemma/Layers/Embedding.hs:30-64) then the host-side
     * f32 scale by sqrt(H) (src/Gemma/Model.hs:1357-1361) */
    float escale = sqrtf((float)H);
    if (m->embd.dtype == ORC_Q4_0)
        orc_q4_0_dequant((const uint8_t*)m->embd.data + (size_t)token * (H / 32) * 18, H / 32,
                         ftz_of(m), x);
    else
        memcpy(x, (const float*)m->embd.data + (size_t)token * H, sizeof(float) * H);
    for (int i = 0; i < H; ++i) x[i] = x[i] * escale;

    size_t kv_layer = (size_t)c->max_seq * nkv * hd;
    for (int l = 0; l < c->n_layers; ++l) {
        orc_tensor* T = &m->lt[l * T_NLAYER];
        int global = layer_is_global(c, l);
        float theta;
        int p_begin = 0, p_end = pos + 1;
        if (c->mode == ORC_MODE_REF) {
            /* quirks Q2/Q3: one theta; window = first min(len, W) positions
             * (src/Gemma/Model.hs:1380-1384, TransformerBlockGPU.hs:236-240) */
            theta = c->rope_theta_global;
            if (c->sliding_window > 0 && p_end > c->sliding_window) p_end = c->sliding_window;
        } else {
            theta = global ? c->rope_theta_global : c->rope_theta_local;
            if (!global && c->sliding_window > 0 && p_end - c->sliding_window > 0)
                p_begin = p_end - c->sliding_window;
        }
        /* TBG:110 pre-attention norm */
        orc_rmsnorm_tree(x, (const float*)T[T_ATTN_NORM].data, H, eps, zc, xn);
        /* QKV */
        matvec_t(m, &T[T_Q], xn, nq * hd, H, q);
        matvec_t(m, &T[T_K], xn, nkv * hd, H, k);
        matvec_t(m, &T[T_V], xn, nkv * hd, H, v);
        /* TBG:171-179 QK-norm */
        if ((c->flags & ORC_QK_NORM) && T[T_QN].data && T[T_KN].data) {
            orc_qk_norm(q, (const float*)T[T_QN].data, nq, hd, eps, zc, q);
            orc_qk_norm(k, (const float*)T[T_KN].data, nkv, hd, eps, zc, k);
        }
        /* RoPE on q and k */
        orc_rope(q, nq, hd, theta, pos, q);
        orc_rope(k, nkv, hd, theta, pos, k);
        /* appendKVCacheShader (AttentionGPU.hs:502-534) */
        memcpy(m->kc + l * kv_layer + (size_t)pos * nkv * hd, k, sizeof(float) * nkv * hd);
        memcpy(m->vc + l * kv_layer + (size_t)pos * nkv * hd, v, sizeof(float) * nkv * hd);
        orc_attention(q, m->kc + l * kv_layer, m->vc + l * kv_layer, nq, nkv, hd, p_begin, p_end, o);
        /* O projection, post-attention norm, residual (TBG:305-343) */
        matvec_t(m, &T[T_O], o, H, nq * hd, a);
        if ((c->flags & ORC_POST_ATTN_NORM) && T[T_POST_ATTN].data)
            orc_rmsnorm_tree(a, (const float*)T[T_POST_ATTN].data, H, eps, zc, a);
        for (int i = 0; i < H; ++i) x1[i] = x[i] + a[i];
        /* fused pre-FFN norm + gate/up (MLP.hs:507-622); pre-FFN weight is
         * ffn_norm, else post_attention_norm (src/Gemma/Model.hs:337-339) */
        const float* wffn = T[T_FFN_NORM].data ? (const float*)T[T_FFN_NORM].data
                                                : (const float*)T[T_POST_ATTN].data;
        orc_rmsnorm_seq(x1, wffn, H, eps, zc, xn);
        matvec_t(m, &T[T_GATE], xn, F, H, g);
        matvec_t(m, &T[T_UP], xn, F, H, u);
        orc_geglu(g, u, F, hh);
        /* down, post-FFN norm, residual (TBG:413-444) */
        matvec_t(m, &T[T_DOWN], hh, H, F, a);
        if ((c->flags & ORC_POST_FFN_NORM) && T[T_POST_FFN].data)
            orc_rmsnorm_tree(a, (const float*)T[T_POST_FFN].data, H, eps, zc, a);
        for (int i = 0; i < H; ++i) x[i] = x1[i] + a[i];
        if (layer_out) memcpy(layer_out + (size_t)l * H, x, sizeof(float) * H);
    }
    /* fused final norm + LM head (RMSNorm.hs:343-386): lm_head.weight when
     * the model has one, else the tied embedding table
     * (src/Gemma/Model.hs:412-414; GGUF output.weight, Model.hs:988) */
    orc_rmsnorm_seq(x, (const float*)m->out_norm.data, H, eps, zc, xn);
    const orc_tensor* head = m->lm.data ? &m->lm : &m->embd;
    if (head->dtype == ORC_Q4_0)
        orc_q4_0_matvec((const uint8_t*)head->data, xn, c->vocab, H, ftz_of(m), lg);
    else
        orc_f32_matvec((const float*)head->data, xn, c->vocab, H, lg);
    int32_t best = orc_argmax(lg, c->vocab);

    free(x); free(xn); free(x1); free(a); free(q); free(k); free(v); free(o);
    free(g); free(u); free(hh);
    if (!logits) free(lg);
    return best;
}

int orc_generate(orc_model* m, const int32_t* prompt, int n_prompt, int n_gen, int32_t* ids_out,
                 float* margin_out) {
    if (n_prompt < 1 || n_prompt + n_gen > m->c.max_seq + 1) return -1;
    float* lg = (float*)malloc(sizeof(float) * m->c.vocab);
    int32_t tok = prompt[0];
    int pos = 0;
    int produced = 0;
    int rc = 0;
    /* app/Main.hs:426-448: prompt fed one token per step, then greedy */
    while (produced < n_gen) {
        int best = orc_step(m, tok, pos, lg, NULL);
        if (best < 0) { rc = best; break; }
        ++pos;
        if (pos < n_prompt) {
            tok = prompt[pos];
            continue;
        }
        ids_out[produced] = best;
        if (margin_out) {
            float top1 = lg[best], top2 = -INFINITY;
            for (int i = 0; i < m->c.vocab; ++i)
                if (i != best && lg[i] > top2) top2 = lg[i];
            margin_out[produced] = top1 - top2;
        }
        ++produced;
        tok = best;
    }
    free(lg);
    return rc;
}

/* Philox4x32-10 (J. Salmon, M. Moraes, R. Dror, D. Shaw, "Parallel random
 * numbers: as easy as 1, 2, 3", SC'11): ten rounds of
 *   (c0..c3) -> (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0))
 * with the key bumped by the Weyl constants between rounds. */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        if (r) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
        c0 = n0;
        c1 = n1;
        c2 = n2;
        c3 = n3;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

float orc_philox_uniform(uint64_t seed, uint64_t counter) {
    const uint32_t ctr[4] = {(uint32_t)counter, (uint32_t)(counter >> 32), 0u, 0u};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    orc_philox4x32_10(ctr, key, o);
    return (float)(o[0] >> 8) * (1.0f / 16777216.0f);
}

int32_t orc_sample(const float* logits, int n, float temperature, float u, double* margin_out) {
    double m = -INFINITY;
    for (int i = 0; i < n; ++i)
        if (logits[i] > m) m = logits[i];
    double z = 0.0;
    for (int i = 0; i < n; ++i) z += exp(((double)logits[i] - m) / temperature);
    const double target = (double)u * z;
    double acc = 0.0, margin = INFINITY;
    int32_t pick = -1, last = 0;
    for (int i = 0; i < n; ++i) {
        const double w = exp(((double)logits[i] - m) / temperature);
        if (w > 0.0) last = i;
        if (fabs(acc - target) < margin) margin = fabs(acc - target);
        if (pick < 0 && acc + w > target && w > 0.0) pick = i;
        acc += w;
    }
    if (fabs(acc - target) < margin) margin = fabs(acc - target);
    if (margin_out) *margin_out = margin / z;
    return pick >= 0 ? pick : last;
}

/* Inversion draw of u from softmax(logits / T) restricted to the k largest
 * logits, ranked by value descending then index ascending, walked in rank
 * order; margin as orc_sample's, over the restricted total. */
int32_t orc_sample_top_k(const float* logits, int n, float temperature, int k, float u, double* margin_out) {
    if (k > n) k = n;
    if (k < 1) k = 1;
    int32_t* idx = (int32_t*)malloc((size_t)k * sizeof(int32_t));
    int have = 0;
    for (int i = 0; i < n; ++i) { /* insertion into the ranked prefix; ties keep the earlier index first */
        const float v = logits[i];
        if (have == k && !(v > logits[idx[k - 1]])) continue;
        int j = have < k ? have++ : k - 1;
        while (j > 0 && v > logits[idx[j - 1]]) {
            idx[j] = idx[j - 1];
            --j;
        }
        idx[j] = i;
    }
    const double m = logits[idx[0]];
    double z = 0.0;
    for (int j = 0; j < k; ++j) z += exp(((double)logits[idx[j]] - m) / temperature);
    const double target = (double)u * z;
    double acc = 0.0, margin = INFINITY;
    int pick = -1, last = 0;
    for (int j = 0; j < k; ++j) {
        const double w = exp(((double)logits[idx[j]] - m) / temperature);
        if (w > 0.0) last = j;
        if (fabs(acc - target) < margin) margin = fabs(acc - target);
        if (pick < 0 && acc + w > target && w > 0.0) pick = j;
        acc += w;
    }
    if (fabs(acc - target) < margin) margin = fabs(acc - target);
    if (margin_out) *margin_out = margin / z;
    const int32_t row = idx[pick >= 0 ? pick : last];
    free(idx);
    return row;
}
