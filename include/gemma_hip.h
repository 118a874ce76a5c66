/*
 * gemma_hip.h -- C ABI of libgemma_hip, the MI355X (gfx950) replacement for
 * the Dawn/WebGPU Graphics layer under gemma.hs's per-token decode loop.
 *
 * Conventions
 *  - Every function returns int: GH_OK (0) or a negative GH_ERR_* code, and
 *    on failure sets a thread-local message readable with gh_last_error().
 *  - Host pointers are borrowed for the duration of the call (the Haskell
 *    side passes Storable.unsafeWith pointers); the library copies what it
 *    keeps.  Device memory is owned by the library (contexts, models,
 *    caches, gh_q4 tensors and gh_buf_alloc buffers).
 *  - One HIP stream per context; calls on one context are serialised by a
 *    mutex, so a Haskell RTS running with -N may call from any thread.
 *  - Handles (gh_ctx, gh_model, gh_kv, gh_q4) may be destroyed in any
 *    order, as garbage-collector finalisers run them: destroying a context
 *    or model that still has open handles made from it only releases it,
 *    and the library frees it with the last of them.  A call on a handle
 *    already destroyed returns GH_ERR_STATE without touching its memory
 *    (unless the address was since reused by a new handle).  The
 *    gh_*_release functions are void-typed destroys for finalisers
 *    (Foreign.ForeignPtr's FinalizerPtr).
 *  - Plain C types only: no HIP or torch types cross this boundary.
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the reference repository root).
 */
#ifndef GEMMA_HIP_H
#define GEMMA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes ---- */
#define GH_OK 0
#define GH_ERR_INVALID (-1)   /* bad argument / shape */
#define GH_ERR_HIP (-2)       /* HIP runtime failure (incl. no device) */
#define GH_ERR_OOM (-3)       /* device or host allocation failed */
#define GH_ERR_STATE (-4)     /* model incomplete / wrong object state */
#define GH_ERR_RANGE (-5)     /* position >= max_seq (KV cache full) */
#define GH_ERR_NAN (-6)       /* NaN in logits */
#define GH_ERR_FORMAT (-7)    /* malformed GGUF file */
#define GH_ERR_NOT_FOUND (-8) /* missing tensor / unknown tensor name */

/* ---- tensor dtypes ---- */
#define GH_DTYPE_F32 0
#define GH_DTYPE_F16 1
#define GH_DTYPE_Q4_0 2 /* raw GGUF Q4_0 bytes: 18-byte blocks along the row */

/* ---- gh_config.mode ---- */
#define GH_MODE_GEMMA3 0 /* local layers attend to the last W positions; per-type theta */
#define GH_MODE_REF 1    /* the reference's quirks Q2/Q3: one theta, prefix window */

/* ---- gh_config.flags ---- */
#define GH_FLAG_QK_NORM 1
#define GH_FLAG_POST_ATTN_NORM 2
#define GH_FLAG_POST_FFN_NORM 4
#define GH_FLAG_ZERO_CENTERED 8
/* keep fp16 subnormals: Q4_0 scales and F16 tensor values (default: flush
 * them to zero, as halfToFloat does, src/Gemma/GGUF.hs:797-820) */
#define GH_FLAG_IEEE_SCALES 16

const char* gh_last_error(void);
/* Library version string. */
const char* gh_version(void);

/* ================================================================
 * Context: replaces Graphics.WebGPU.Dawn createContext / waitAll
 * (used at src/Gemma/Model.hs:419 and src/Gemma/Model.hs:1432).
 * ================================================================ */
typedef struct gh_ctx gh_ctx;
int gh_device_count(int* n_out);
int gh_ctx_create(int device, gh_ctx** out);
/* Releases the context: models, caches and Q4_0 tensors made on it stay
 * usable, and the context is freed with the last of them. */
int gh_ctx_destroy(gh_ctx* ctx);
void gh_ctx_release(gh_ctx* ctx); /* gh_ctx_destroy for finalisers */
/* waitAll (src/Gemma/Model.hs:1432) */
int gh_ctx_sync(gh_ctx* ctx);
/* Event timer on the context stream (replaces the wall-clock timing of
 * examples/BenchmarkKVCache.hs:186-210): start records an event, stop
 * records a second one, waits for it and returns the elapsed ms. */
int gh_timer_start(gh_ctx* ctx);
int gh_timer_stop(gh_ctx* ctx, float* ms_out);
/* Graph timing of op-level calls (no reference counterpart; used by the
 * matvec and attention microbenchmarks): after gh_capture_begin the
 * launch-only op calls (gh_q4_0_matvec, gh_attention_decode, gh_rmsnorm,
 * gh_qk_norm, gh_gelu_mul, gh_q4_0_dequant) enqueue without
 * synchronising; gh_capture_replay ends the capture, replays the graph
 * n_replays times between two events and returns the ms per replay. */
int gh_capture_begin(gh_ctx* ctx);
int gh_capture_replay(gh_ctx* ctx, int32_t n_replays, float* ms_per_replay_out);

/* ================================================================
 * Buffers: replace createTensor / createTensorWithData / fromGPU
 * (e.g. src/Gemma/Model.hs:588-616, src/Gemma/Model.hs:1435).
 * ================================================================ */
int gh_buf_alloc(gh_ctx* ctx, size_t bytes, void** dev_out);
int gh_buf_free(gh_ctx* ctx, void* dev);
int gh_buf_upload(gh_ctx* ctx, void* dev, const void* host, size_t bytes);
int gh_buf_download(gh_ctx* ctx, void* host, const void* dev, size_t bytes);

/* ================================================================
 * GGUF Q4_0 tensors.  Replaces Gemma.GGUF.loadQ4_0Tensor's dequant
 * (src/Gemma/GGUF.hs:726-760) and Gemma.Layers.LinearQ4.runLinearQ4
 * (src/Gemma/Layers/LinearQ4.hs:41-48, body runMatmulQ4_0DSL).
 * ================================================================ */
typedef struct gh_q4 gh_q4;
/* raw: rows*cols/32 GGUF blocks of 18 bytes, row-major, cols % 32 == 0.
 * flags: GH_FLAG_IEEE_SCALES or 0.  The bytes are repacked on upload into
 * the device tile layout; dequantised values are bit-identical. */
int gh_q4_0_upload(gh_ctx* ctx, const void* raw, int64_t rows, int64_t cols, int flags, gh_q4** out);
int gh_q4_0_free(gh_q4* t);
void gh_q4_0_release(gh_q4* t); /* gh_q4_0_free for finalisers */
/* out_dev: rows*cols f32, row-major (loadQ4_0Tensor's result). */
int gh_q4_0_dequant(gh_q4* t, float* out_dev);
/* y_dev[rows] = W x_dev[cols]; softcap != 0 applies cap*tanh(y/cap). */
int gh_q4_0_matvec(gh_q4* t, const float* x_dev, float* y_dev, int softcap, float cap);
/* runLinearQ4 signature: raw GGUF bytes packed little-endian into 32-bit
 * words (a block straddles words), host x[cols] -> host y[rows]. */
int gh_linear_q4(gh_ctx* ctx, const uint32_t* raw_words, size_t n_words, const float* x, int rows,
                 int cols, int softcap, float cap, float* y);

/* ================================================================
 * Op-level entry points on device pointers (parity hooks for the
 * individual shaders of the step).
 * ================================================================ */
/* rmsNormShader, src/Gemma/Layers/RMSNorm.hs:45-154 */
int gh_rmsnorm(gh_ctx* ctx, const float* x, const float* w, int n, float eps, int zero_centered,
               float* y);
/* qkNormShader, src/Gemma/Layers/AttentionGPU.hs:218-257 */
int gh_qk_norm(gh_ctx* ctx, const float* x, const float* w, int n_heads, int head_dim, float eps,
               int zero_centered, float* y);
/* ropeShader, src/Gemma/Layers/AttentionGPU.hs:68-115 (in place) */
int gh_rope(gh_ctx* ctx, float* x, int n_heads, int head_dim, float theta, int pos);
/* attentionScoresShader + attentionOutputShader,
 * src/Gemma/Layers/AttentionGPU.hs:292-352,382-423: one query token over
 * cache rows [p_begin, p_end) of a [pos][nkv][hd] f32 cache.  n_splits = 0
 * picks the split count. */
int gh_attention_decode(gh_ctx* ctx, const float* q, const float* k_cache, const float* v_cache,
                        int nq, int nkv, int head_dim, int p_begin, int p_end, int n_splits,
                        float* out);
/* gh_attention_decode that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * The split-K chunk states go to a static per-GPU array of 4 MiB instead of
 * the context's scratch; a call that needs more, nkv * n_splits *
 * (nq / nkv) * (head_dim + 2) floats > 2^20, returns GH_ERR_RANGE.  The
 * array keeps the last call's contents; calls that overlap on one GPU (on
 * different contexts or threads) share it and race. */
int gh_attention_decode_noalloc(gh_ctx* ctx, const float* q, const float* k_cache, const float* v_cache,
                                int nq, int nkv, int head_dim, int p_begin, int p_end, int n_splits,
                                float* out);
/* geluMultiplyFusedShader, src/Gemma/Layers/MLP.hs:384-447 */
int gh_gelu_mul(gh_ctx* ctx, const float* g, const float* u, int n, float* h);
/* sampleToken / sampleWithTemperature, app/Main.hs:488-507 (first max) */
int gh_argmax(gh_ctx* ctx, const float* v, int n, int32_t* idx_out);
/* Op-level draw from softmax(logits[n] / temperature) with Philox4x32-10
 * (key = seed, counter = counter); temperature 0 is gh_argmax.  Same
 * device code as the step's sampler. */
int gh_sample_logits(gh_ctx* ctx, const float* logits, int n, float temperature, uint64_t seed, uint64_t counter,
                     int32_t* token_out);
/* Top-k variant, no reference counterpart (the reference's sampler is an
 * argmax, app/Main.hs:505-507): the draw is restricted to the top_k largest
 * logits (value descending, then lower index) and made by inversion in that
 * rank order; top_k 0 is gh_sample_logits, 1..GH_TOP_K_MAX (64) restricts,
 * anything else is GH_ERR_RANGE.  Same device code as the step's sampler. */
#define GH_TOP_K_MAX 64
int gh_sample_logits_top_k(gh_ctx* ctx, const float* logits, int n, float temperature, int32_t top_k,
                           uint64_t seed, uint64_t counter, int32_t* token_out);


/* ================================================================
 * Model: replaces GemmaConfig / loadGemmaModel / loadGemmaModelFromGGUF
 * (src/Gemma/Model.hs:106-129, 276, 908) and the per-token step
 * runGemmaInferenceCached (src/Gemma/Model.hs:1313-1437).
 * ================================================================ */
typedef struct gh_config {
    int32_t vocab, hidden, n_layers, n_heads, n_kv_heads, head_dim, ffn;
    int32_t max_seq;        /* default KV capacity (reference: 2048) */
    int32_t sliding_window; /* 0 = none */
    int32_t global_every;   /* layer i global iff (i+1) % global_every == 0; 0 = all global */
    float rope_theta_local, rope_theta_global;
    float rms_eps;
    int32_t mode;  /* GH_MODE_* */
    int32_t flags; /* GH_FLAG_* */
} gh_config;

/* Presets: name in {"tiny", "gemma3-1b", "gemma3-4b"}. */
int gh_config_preset(const char* name, gh_config* out);

typedef struct gh_model gh_model;
/* GH_ERR_INVALID for shapes the kernels do not support: head_dim other than
 * 32/128/256, n_heads/n_kv_heads other than 1/2/4/8, hidden above 3072,
 * hidden/ffn/n_heads*head_dim not multiples of 32; and for a negative
 * window or global period, RoPE theta not finite and > 0, rms_eps negative
 * or not finite. */
int gh_model_create(gh_ctx* ctx, const gh_config* cfg, gh_model** out);
int gh_model_destroy(gh_model* m);
void gh_model_release(gh_model* m); /* gh_model_destroy for finalisers */
/* name: GGUF tensor name (token_embd.weight, output_norm.weight,
 * output.weight, blk.N.{attn_norm,attn_q,attn_k,attn_v,attn_q_norm,
 * attn_k_norm,attn_output,post_attention_norm,ffn_norm,ffn_gate,ffn_up,
 * ffn_down,post_ffw_norm}.weight).  dtype GH_DTYPE_F32 / F16 / Q4_0 (raw
 * bytes).  The projections share one format (Q4_0, or f32 from F32/F16);
 * the embedding and output.weight may each have their own.
 * output.weight [vocab x hidden] is an untied LM head: the model uses it
 * instead of the embedding (the reference's lm_head.weight when present,
 * src/Gemma/Model.hs:412-414, and the GGUF output.weight,
 * src/Gemma/Model.hs:988).  It is optional and must be set before the
 * model's first step (GH_ERR_STATE after). */
int gh_model_set_tensor(gh_model* m, const char* name, int dtype, const void* data, size_t nbytes);
/* 0 when every tensor the config needs is present. */
int gh_model_check(gh_model* m);
int gh_model_config(gh_model* m, gh_config* out);
/* The kernel plan the model's decode step runs (no reference counterpart:
 * the reference compiles one fixed set of shaders).  A one-line text of
 * space-separated key=value items: the step mode (graph, eager or
 * persistent; GH_NO_GRAPH is read at every step, so eager reflects it now),
 * then per matvec phase (qkv, o_proj, gate_up, down, lm_head) its column
 * splits S, rows per lane rl, work items per workgroup ni, dot-product unit
 * (valu or mfma) and in_first when every wave's input loads are issued before
 * any weight load, the attention chunks per kv head, the LM head (tied
 * or untied), and env= with every GH_* environment variable that was set
 * when the plan was made and can change what runs (the tuning and study
 * switches GH_PLAN_*, GH_Q4_*, GH_ATTN_*, GH_PERSISTENT, GH_NO_GRAPH), or
 * env=none.  The plan is fixed at the model's first step; before it, this
 * reports the plan that step will choose.  Writes at most cap bytes including the terminating NUL;
 * *len_out (may be NULL) receives the full length without it. */
int gh_model_plan(gh_model* m, char* buf, size_t cap, size_t* len_out);
/* loadGemmaModelFromGGUF (src/Gemma/Model.hs:908-1234) + configFromGGUF
 * (src/Gemma/Model.hs:843-902): parse a GGUF v3 file, build the config from
 * its metadata (vocab from the token_embd shape) and upload every tensor.
 * Tensor types: F32, F16, Q4_0, and Q4_1, which is dequantised to f32 on the
 * host in the reference's element order (src/Gemma/GGUF.hs:762-795). */
int gh_model_load_gguf(gh_ctx* ctx, const char* path, int32_t max_seq, gh_model** out);
/* configFromGGUF alone (src/Gemma/Model.hs:843-902): parse the header,
 * metadata and tensor infos of a GGUF v3 file into a config; no device. */
int gh_gguf_inspect(const char* path, gh_config* out);

/* ================================================================
 * KV cache handle: replaces Gemma.KVCache (src/Gemma/KVCache.hs:20-35,
 * initKVCache 78-82, cacheLength 146-147).  Device K/V of shape
 * [n_layers][max_seq][n_kv_heads][head_dim] f32.
 * ================================================================ */
typedef struct gh_kv gh_kv;
int gh_kv_create(gh_model* m, int32_t max_seq, gh_kv** out);
int gh_kv_destroy(gh_kv* kv);
void gh_kv_release(gh_kv* kv); /* gh_kv_destroy for finalisers */
int gh_kv_reset(gh_kv* kv);
int gh_kv_length(gh_kv* kv, int32_t* len_out);
/* Rewind to the first n positions (0 <= n <= length; GH_ERR_RANGE
 * otherwise): the next step runs at position n.  The reference's KVCache
 * is a persistent value whose layer-0 cacheLen is the next position
 * (src/Gemma/Model.hs:1332-1334, src/Gemma/KVCache.hs:146-147), so stepping
 * an older cache value continues from its own length. */
int gh_kv_truncate(gh_kv* kv, int32_t n);
/* Benchmark set-up with no reference counterpart: fill positions
 * [0, n_pos) of every layer's K and V with seeded N(0, sigma) values
 * (gh_synth_kv, generated on the host and uploaded) and set the cache
 * length to n_pos, standing in for a prefilled context. */
int gh_kv_synth(gh_kv* kv, uint64_t seed, int32_t n_pos, float sigma);
/* Sampling of the next token for this cache's steps: temperature 0 is
 * greedy (the reference's sampleToken / sampleWithTemperature, which is an
 * argmax at any temperature: app/Main.hs:488-507); temperature > 0 draws
 * from softmax(logits / T) with Philox4x32-10 keyed by `seed`, counter =
 * the step's position, so a generation is reproducible. */
int gh_kv_set_sampling(gh_kv* kv, float temperature, uint64_t seed);
/* Top-k restriction of that draw for this cache's steps (no reference
 * counterpart): 0 = every logit (the default), 1..GH_TOP_K_MAX = the top_k
 * largest, as gh_sample_logits_top_k; it has no effect at temperature 0. */
int gh_kv_set_top_k(gh_kv* kv, int32_t top_k);

/* runGemmaInferenceCached (src/Gemma/Model.hs:1313-1437) and its layer-0
 * variant runGemmaInferenceCachedWithLayer0 (src/Gemma/Model.hs:1441):
 * one token at position = cache length; the cache grows by one.
 * logits[vocab], layer_out[n_layers*hidden] (hidden state after each
 * layer) may be NULL; argmax_out receives the greedy next token. */
int gh_step(gh_model* m, gh_kv* kv, int32_t token, float* logits, float* layer_out,
            int32_t* argmax_out);

/* The generation loop of app/Main.hs:372-463 / examples/BenchmarkKVCache.hs
 * :166-220 (prompt one token per step, then greedy), run on device with no
 * host round trip per token: ids_out[n_gen]. */
int gh_generate(gh_model* m, gh_kv* kv, const int32_t* prompt, int32_t n_prompt, int32_t n_gen,
                int32_t* ids_out);

/* Batched prompt prefill.  It replaces the token-by-token prompt loop
 * `goPrompt` (app/Main.hs:426-436), which calls runGemmaInferenceCached
 * once per token; the reference itself rejects more than one token per
 * call (src/Gemma/Model.hs:1321-1324).
 * The n tokens run at the cache's next positions in one pass per layer:
 * the projections are Q4_0 (or f32) GEMMs on MFMA, attention is causal
 * over the cache, and K/V are appended.  Passes hold up to 512 tokens.
 * The cache then holds n more positions.  logits[vocab], layer_out
 * [n_layers*hidden] (may be NULL) and next_out (greedy, or sampled per
 * gh_kv_set_sampling) are those of the last token: what gh_step on that
 * token would return after the others. */
int gh_prefill(gh_model* m, gh_kv* kv, const int32_t* tokens, int32_t n, float* logits, float* layer_out,
               int32_t* next_out);

/* gh_generate with the prompt fed by gh_prefill: ids_out[0] is the
 * prefill's next token, then n_gen - 1 decode steps on device. */
int gh_generate_prefill(gh_model* m, gh_kv* kv, const int32_t* prompt, int32_t n_prompt, int32_t n_gen,
                        int32_t* ids_out);

/* Decode benchmark (examples/BenchmarkKVCache.hs:56-165): feeds the prompt,
 * runs n_warmup greedy steps, then times n_steps greedy steps with HIP
 * events.  ids_out[n_warmup + n_steps + 1] may be NULL. */
int gh_bench_decode(gh_model* m, gh_kv* kv, const int32_t* prompt, int32_t n_prompt,
                    int32_t n_warmup, int32_t n_steps, float* ms_out, int32_t* ids_out);

/* ================================================================
 * Profiling: replaces the gpu_print_profile_stats /
 * gpu_reset_profile_stats hooks (examples/BenchmarkKVCache.hs:38-42).
 * Runs n_steps greedy steps, launched eagerly in the step's order, and
 * reports per-kernel-kind statistics of every kernel's execution time: the
 * begin and end timestamps of its own dispatch (hipExtLaunchKernel's start
 * and stop events), which is what a kernel trace reports, measured inside
 * real decode steps (each layer's weights cold, as in the decode loop).
 * ================================================================ */
typedef struct gh_kernel_stat {
    char name[32];
    int32_t launches;   /* launches over the n_steps steps */
    double total_ms;    /* summed event durations */
    double bytes;       /* algorithmic bytes per launch, averaged */
} gh_kernel_stat;
int gh_profile_steps(gh_model* m, gh_kv* kv, int32_t n_steps, gh_kernel_stat* stats,
                     int32_t max_stats, int32_t* n_stats_out);
/* gh_prefill of n tokens with HIP events around every kernel: the same
 * per-kernel-kind statistics (no reference counterpart: the reference has
 * no prefill).  The cache advances by n as with gh_prefill. */
int gh_prefill_profile(gh_model* m, gh_kv* kv, const int32_t* tokens, int32_t n, gh_kernel_stat* stats,
                       int32_t max_stats, int32_t* n_stats_out);
/* Kernel timing for the roofline: replays only the step kernels named
 * `name` ("qkv", "attention", "o_proj", "gate_up", "down", "final_norm",
 * "lm_head") of one step at the cache's current position, n_reps times
 * back to back on the context stream between two HIP events, and returns
 * the average duration per launch, the algorithmic HBM bytes per launch
 * and the launches per step.  The n_reps passes run as one captured graph
 * (the way the decode loop runs them), or as eager launches when
 * GH_NO_GRAPH=1.  The replayed kernels are idempotent (same
 * inputs, same outputs), so the model and cache state are unchanged.
 * Also replaces the gpu_print_profile_stats hook (BenchmarkKVCache.hs:38-42). */
int gh_time_kernel(gh_model* m, gh_kv* kv, const char* name, int32_t n_reps, double* avg_us_out,
                   double* bytes_per_launch_out, int32_t* launches_per_step_out);
/* Measured stream-read peak of the device (no reference counterpart: a
 * measurement helper for the roofline): allocates `bytes` (a multiple of
 * 16, below 2 GiB) on the context's device, reads every byte once per launch with
 * non-temporal 16-byte loads, 4096 workgroups each streaming one
 * contiguous chunk (the access shape of a matvec tile), n_reps launches back
 * to back after one warm-up, and returns the average duration per launch.
 * bytes / duration is the practical HBM read bandwidth the hot path's
 * weight streaming is measured against beside the nominal 8 TB/s. */
int gh_time_stream_read(gh_ctx* ctx, size_t bytes, int32_t n_reps, double* avg_us_out);
/* All-to-all exchange cost (no reference counterpart; the measurement
 * behind the persistent step): `rounds` exchanges of one self-validating
 * 64-bit word per workgroup among n_wg co-resident workgroups (one kernel,
 * agent-scope relaxed stores and polled loads).  *us_out = microseconds per
 * exchange (workgroup 0's clock over all rounds).  GH_ERR_RANGE for n_wg
 * outside 1 .. min(256, CUs); GH_ERR_STATE if a bounded wait timed out. */
int gh_time_exchange(gh_ctx* ctx, int32_t n_wg, int32_t rounds, double* us_out);

/* ================================================================
 * Seeded synthetic weights (SplitMix64 + Box-Muller), identical on every
 * host, so a GPU box can regenerate the exact bytes of a test model.
 * ================================================================ */
/* N(0, sigma) f32 values for tensor `name`. */
int gh_synth_f32(uint64_t seed, const char* name, float sigma, float* out, size_t n);
/* GGUF Q4_0 raw blocks: codes uniform in [0,15], scale |N(0,scale_sigma)|
 * rounded to fp16 (round to nearest even). */
int gh_synth_q4_0(uint64_t seed, const char* name, float scale_sigma, int64_t rows, int64_t cols,
                  uint8_t* out);
/* K and V rows of one layer of gh_kv_synth: positions [0, n_pos), `width`
 * (= n_kv_heads * head_dim) N(0, sigma) values per position each, one
 * stream per (layer, K or V, position); k_out / v_out [n_pos * width]. */
int gh_synth_kv(uint64_t seed, int32_t layer, int32_t n_pos, int32_t width, float sigma, float* k_out,
                float* v_out);
/* token ids uniform in [0, vocab) */
int gh_synth_tokens(uint64_t seed, const char* name, int32_t n, int32_t vocab, int32_t* out);
/* Populate every tensor of `m` from the seed (Q4_0 projections and
 * embedding when q4 != 0, else f32; norm weights f32 N(0, norm_sigma)). */
int gh_synth_model(gh_model* m, uint64_t seed, int q4, float w_sigma, float scale_sigma,
                   float norm_sigma);

#ifdef __cplusplus
}
#endif
#endif /* GEMMA_HIP_H */
