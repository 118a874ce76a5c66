/*
 * gemma_oracle.h -- CPU restatement of gemma.hs's per-token decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or, in bench.py, as the timed CPU baseline).  The product path
 * (libgemma_hip) never links, loads or calls it.
 *
 * Every function restates one reference shader / Haskell function in plain C
 * with the reference's f32 operation order; the citation is on each
 * definition in gemma_oracle.c.  Pinning status of each function (which
 * golden vector, closed form or brute-force check fixes it) is listed in the
 * header comment of gemma_oracle.c.
 */
#ifndef GEMMA_ORACLE_H
#define GEMMA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes (same values as the product's GH_DTYPE_*) */
#define ORC_F32 0
#define ORC_Q4_0 2

/* config.mode */
#define ORC_MODE_GEMMA3 0 /* trailing window on local layers, per-type theta */
#define ORC_MODE_REF 1    /* reference quirks Q2/Q3: one theta, prefix window */

/* config.flags */
#define ORC_QK_NORM 1
#define ORC_POST_ATTN_NORM 2
#define ORC_POST_FFN_NORM 4
#define ORC_ZERO_CENTERED 8
#define ORC_IEEE_SCALES 16 /* keep fp16 subnormal scales (default: FTZ) */

typedef struct orc_config {
    int32_t vocab, hidden, n_layers, n_heads, n_kv_heads, head_dim, ffn;
    int32_t max_seq;
    int32_t sliding_window; /* 0 = no window */
    int32_t global_every;   /* layer i is global iff (i+1) % global_every == 0; 0 = all global */
    float rope_theta_local, rope_theta_global;
    float rms_eps;
    int32_t mode;
    int32_t flags;
} orc_config;

/* ---- primitive ops ---- */
float orc_f16_to_f32(uint16_t h, int ftz);
void orc_q4_0_dequant(const uint8_t* raw, size_t n_blocks, int ftz, float* out);
void orc_q4_0_matvec(const uint8_t* raw, const float* x, int rows, int cols, int ftz, float* y);
void orc_q4_0_matvec_f64(const uint8_t* raw, const float* x, int rows, int cols, int ftz,
                         double* y, double* abs_y);
void orc_f32_matvec(const float* w, const float* x, int rows, int cols, float* y);
void orc_rmsnorm_tree(const float* x, const float* w, int n, float eps, int zc, float* y);
void orc_rmsnorm_seq(const float* x, const float* w, int n, float eps, int zc, float* y);
void orc_qk_norm(const float* x, const float* w, int n_heads, int hd, float eps, int zc, float* y);
void orc_rope(const float* x, int n_heads, int hd, float theta, int pos, float* y);
void orc_attention(const float* q, const float* k_cache, const float* v_cache, int nq, int nkv,
                   int hd, int p_begin, int p_end, float* out);
float orc_gelu_tanh(float x);
void orc_geglu(const float* g, const float* u, int n, float* h);
int32_t orc_argmax(const float* v, int n);
void orc_softcap(float* y, int n, float cap);
/* Philox4x32-10 (Salmon et al., SC'11) and the sampler's uniform: top 24
 * bits of the first output word for counter (lo, hi, 0, 0), key = seed. */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float orc_philox_uniform(uint64_t seed, uint64_t counter);
/* Draw from softmax(logits / temperature) by inversion of u in double
 * precision: the first index whose running sum of exp((l - max) / T)
 * exceeds u * total.  margin_out (may be NULL): distance of u * total to
 * the nearest running-sum boundary, relative to the total. */
int32_t orc_sample(const float* logits, int n, float temperature, float u, double* margin_out);
int32_t orc_sample_top_k(const float* logits, int n, float temperature, int k, float u, double* margin_out);

/* ---- whole model ---- */
typedef struct orc_model orc_model;
orc_model* orc_model_create(const orc_config* cfg);
void orc_model_destroy(orc_model* m);
/* name: GGUF tensor name (token_embd.weight, blk.N.attn_q.weight, ...) */
int orc_model_set_tensor(orc_model* m, const char* name, int dtype, const void* data, size_t nbytes);
void orc_model_reset(orc_model* m);
/* Positions [0, n_pos) of layer `layer`'s K and V cache ([n_pos][nkv*hd]
 * each): a prefilled context (the checker's copy of gh_kv_synth). */
int orc_model_set_kv(orc_model* m, int layer, int n_pos, const float* k, const float* v);
/* One decode step at position pos (= current cache length).  logits [vocab]
 * and layer_out [n_layers*hidden] may be NULL.  Returns argmax or <0. */
int orc_step(orc_model* m, int32_t token, int32_t pos, float* logits, float* layer_out);
/* Greedy generation: prompt steps then n_gen generated tokens.
 * ids_out[n_gen]; margin_out[n_gen] (top1-top2 logit, may be NULL). */
int orc_generate(orc_model* m, const int32_t* prompt, int n_prompt, int n_gen, int32_t* ids_out,
                 float* margin_out);
void orc_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
