// Host-side shared definitions of libgemma_hip: handles, device matrix
// descriptors, error helpers.  Included by both the host .cpp files and the
// .hip kernel file.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/gemma_hip.h"

namespace gh {

int set_error(int code, const char* fmt, ...);

#define GH_HIP(expr)                                                                   \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess)                                                          \
            return ::gh::set_error(GH_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

#define GH_CHECK(expr)            \
    do {                          \
        int rc_ = (expr);         \
        if (rc_ != GH_OK) return rc_; \
    } while (0)

uint16_t f32_to_f16_rne(float f);
float f16_to_f32(uint16_t h, bool ftz);

// Matrix storage formats on the device.  FMT_Q4M is not a storage format:
// it names the kernels' compute mode for Q4_0 matrices whose dot products
// run on the int8 matrix cores (Plan::mfma).
enum Fmt : int { FMT_Q4 = 0, FMT_F32 = 1, FMT_Q4M = 2 };

// Rows per tile of the device layout.  A tile stores, for every column
// block kb, the 16-byte payloads of its 128 rows contiguously:
//   payload[tile][kb][row 0..127]   (Q4_0: 16 code bytes = 32 weights;
//                                    F32: 4 floats = 4 weights)
//   scale  [tile][kb][row 0..127]   (Q4_0 only: fp16 d, FTZ applied)
// so a wavefront reading block kb of rows lane and lane+64 issues two
// contiguous 1 KB loads.
constexpr int TILE_ROWS = 128;

struct DMat {
    const void* codes = nullptr;
    const uint16_t* scales = nullptr;
    int fmt = FMT_F32;
    int rows = 0;   // logical rows
    int cols = 0;   // logical columns
    int nblk = 0;   // column blocks (cols/32 for Q4_0, cols/4 for F32)
    int tiles = 0;  // ceil(rows / 128)
    int order_in = 0;  // matvec: a barrier between the input loads and the weight loads
};

inline int block_cols(int fmt) { return fmt == FMT_F32 ? 4 : 32; }
inline int pad_rows(int r) { return (r + TILE_ROWS - 1) / TILE_ROWS * TILE_ROWS; }

// Device-side per-sequence step state (one per KV handle).
struct StepState {
    int32_t pos;        // position of the token being processed
    int32_t token;      // token being processed
    int32_t last;       // argmax of the last finished step
    int32_t start;      // position of prompt[0] (device-fed generation)
    int32_t n_prompt;   // prompt length (device-fed generation)
    int32_t nan_flag;   // set when a logit is NaN
    int32_t gen_count;  // generated ids written so far
    int32_t gen_cap;    // capacity of the ids buffer
    float inv_temp;     // 1/temperature; 0 = greedy
    uint32_t seed_lo, seed_hi;  // Philox key of the sampler
    int32_t xchg_err;   // persistent step: an exchange wait timed out
    int32_t top_k;      // sampler: draw among the top_k largest logits (0 = all)
    unsigned long long keys[2];  // argmax keys, slot pos & 1
};

// Work split of one matvec phase: S column splits per 128-row tile, each
// wave of a 4-wave workgroup covering at most `kbw` column blocks in one
// register batch.
struct Plan {
    int S = 1;
    int kbw = 1;
    int rl = 2;  // rows per lane: 2 = 128-row workgroups, 1 = 64-row workgroups
    int mfma = 0;  // Q4_0: dot products on the int8 matrix cores (1) or the VALU (0)
    int ni = 1;    // work items per workgroup (1 or 2; 4 waves each, one prologue)
    int order_in = 1;  // every wave's input loads issue before any wave's weight loads
    int rg16 = 0;      // op level: rows per workgroup (4, 8, 16) over all columns (k_mq_rows); 0 = off
    int row_tiles(int tiles) const { return rl == 2 ? tiles : 2 * tiles; }
};

// float4 groups per thread (256 threads) of the widest column split of a
// matrix under plan p: the GeGLU prologue of the down projection holds
// gm x (gate/up splits) partial groups, at most 8.
inline int geglu_groups(const DMat& w, const Plan& p) {
    const int cols = (w.nblk + p.S - 1) / p.S * block_cols(w.fmt);
    return (cols / 4 + 255) / 256;
}

struct LayerDev {
    DMat qkv, o, gu, down;
    float* attn_norm = nullptr;
    float* q_norm = nullptr;
    float* k_norm = nullptr;
    float* post_attn = nullptr;
    float* ffn_norm = nullptr;
    float* post_ffw = nullptr;
    bool global = true;
    int p_codes[4] = {0, 0, 0, 0};  // bitmask of sub-tensors uploaded
};

// Allocation with a byte count, freed by the owner.
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
};

}  // namespace gh

struct gh_model;
struct gh_q4;

struct gh_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::recursive_mutex mu;
    std::vector<void*> bufs;  // gh_buf_alloc allocations
    hipEvent_t t0 = nullptr, t1 = nullptr;  // gh_timer_start / gh_timer_stop
    void* scratch = nullptr;                // op-level temporaries
    size_t scratch_bytes = 0;
    // open handles created on this context; a context whose destroy was
    // called (released) is freed when the last of them is destroyed
    std::vector<gh_model*> models;
    std::vector<gh_q4*> q4s;
    bool released = false;
    bool dying = false;  // chosen for freeing (by the one thread that saw it collectable)
};

struct gh_q4 {
    gh_ctx* ctx = nullptr;
    gh::DMat m;
    void* codes = nullptr;
    uint16_t* scales = nullptr;
    gh::Plan plan;
    float* part = nullptr;  // [S][rows_pad] partial sums
    ~gh_q4();               // frees the device buffers
};

struct gh_kv;

namespace gh {

// Kernel arguments kept alive for a graph node; ptrs is the kernelParams array.
struct NodeArgsBase {
    virtual ~NodeArgsBase() = default;
    std::vector<void*> ptrs;
};

// A graph kernel node whose position-dependent arguments are rewritten
// before each replay (the position is host-known: one step = one position);
// `set` updates the node's argument blob for a position.
struct PosPatch {
    hipGraphNode_t node;
    hipKernelNodeParams params;
    std::function<void(int)> set;
};

struct Profiler;

// Where enqueue_step puts its kernels: a stream (eager, optionally event
// profiled) or a graph under construction (linear chain of kernel nodes).
struct Sink {
    hipStream_t s = nullptr;
    Profiler* prof = nullptr;
    hipGraph_t g = nullptr;
    hipGraphNode_t last = nullptr;
    std::vector<std::unique_ptr<NodeArgsBase>>* store = nullptr;
    std::vector<PosPatch>* patches = nullptr;
    const char* only = nullptr;  // launch only the kernels of this name (timing)
    int launched = 0;            // kernels enqueued
    double bytes = 0.0;          // their algorithmic bytes
};

// Buffers of the batched prompt prefill (per model, grown on demand).
struct PfBufs {
    int cap = 0;                 // token rows (multiple of 64) the row buffers hold
    float* x = nullptr;          // [cap][H] residual after attention / after the layer
    float* x1 = nullptr;         // [cap][H] residual after attention
    void* a = nullptr;           // [2][cap][Kmax] fp16 (Q4_0 weights) or [cap][Kmax] f32: GEMM operand
    float* ascale = nullptr;     // [cap] inverse row scales of the fp16 operand
    float* q = nullptr;          // [cap][nq * hd] normed + roped queries
    float* st = nullptr;         // [cap][nkv][PF_ATTN_NC][G][hd + 2] attention chunk states per token
    int32_t* tok = nullptr;      // [cap] token ids of the chunk
    float* part = nullptr;       // split-K GEMM partials
    size_t part_floats = 0;
};

}  // namespace gh

struct gh_model {
    gh_ctx* ctx = nullptr;
    gh_config cfg{};
    int fmt = -1;  // projection format, fixed by the first projection upload
    std::vector<gh::LayerDev> layers;
    std::vector<gh::DevBuf> owned;
    gh::DMat embd;  // token_embd (also the LM head when no output.weight is set: tied)
    gh::DMat lm;    // output.weight, an untied LM head (valid when has_lm)
    float* out_norm = nullptr;
    std::vector<float> inv_freq;  // [2][head_dim/2]: local, global (host)
    // rows of the fused QKV matrix: [q (nq*hd) | k | v], each padded to 128
    int q_rows_pad = 0, kv_rows_pad = 0;
    int f_pad = 0;  // padded ffn rows (gate block, then up block)
    // plans
    gh::Plan pa, pc, pd, pe, plm;
    std::string plan_env;  // the GH_* switches set when the plans were made
    int attn_nc = 16;  // attention chunks per kv head
    int attn_xcd = 1;  // a chunk's attention workgroups on one XCD (groups of 4+ q heads)
    // scratch
    float* x_res = nullptr;
    float* x1 = nullptr;
    float* part_qkv = nullptr;
    float* part_o = nullptr;
    float* part_gu = nullptr;
    float* part_d = nullptr;
    float* attn_part = nullptr;
    float* logits = nullptr;
    float* layer_out = nullptr;
    float* xn_final = nullptr;               // final-norm output, input of the LM head
    unsigned long long* lm_cand = nullptr;   // per-workgroup argmax keys of the LM head
    float* lm_m = nullptr;                   // per-workgroup max logit (sampling)
    float* lm_s = nullptr;                   // per-workgroup sum of exp((l - max) / T) (sampling)
    // presence tracking
    bool has_embd = false, has_out_norm = false, has_lm = false;
    std::vector<uint32_t> present;  // per layer bitmask of tensor kinds
    std::vector<gh_kv*> kvs;  // open caches; a released model is freed when the last goes
    bool released = false;    // gh_model_destroy was called
    // persistent step (GH_PERSISTENT=1): exchange words, launch counter,
    // grid, the interleaved gate/up matrices and the number of down partials
    int persistent = 0;
    uint64_t* w_qkv = nullptr;   // q | k | v rows
    uint64_t* w_attn = nullptr;  // attention chunk states
    uint64_t* w_o = nullptr;     // merged attention output
    uint64_t* w_a = nullptr;     // O-projection rows
    uint64_t* w_p = nullptr;     // down partials [p_np][H]
    uint64_t* w_down = nullptr;  // down rows
    uint32_t p_tick = 0;
    int p_grid = 0;
    int p_np = 0;
    std::vector<gh::DMat> p_gi;  // per layer: gate/up in 64-row chunks of 32 gate + 32 up rows
    bool p_gi_ok = false;        // p_gi matches the uploaded gate/up weights
    // batched prompt prefill
    gh::PfBufs pf;
};

struct gh_kv {
    gh_model* m = nullptr;
    int max_seq = 0;
    int len = 0;
    float* k = nullptr;  // [n_layers][max_seq][nkv][hd]
    float* v = nullptr;
    gh::StepState* st = nullptr;
    float* rope = nullptr;        // [2 (local, global)][max_seq][head_dim/2] (cos, sin) pairs
    int32_t* d_prompt = nullptr;  // [max_seq]
    int32_t* d_ids = nullptr;     // [max_seq]
    float inv_temp = 0.0f;        // sampler: 1/temperature (0 = greedy)
    uint64_t seed = 0;            // sampler: Philox key
    int top_k = 0;                // sampler: candidates (0 = every logit)
    gh::StepState* h_st = nullptr;  // pinned staging
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    std::vector<std::unique_ptr<gh::NodeArgsBase>> graph_args;
    std::vector<gh::PosPatch> patches;
    void* d_players = nullptr;  // persistent step: per-layer pointer table
    ~gh_kv();                   // frees the device buffers and the graph
};

namespace gh {

// The LM head matrix: output.weight when the model has one, else the tied
// token embedding (src/Gemma/Model.hs:412-414).
inline const DMat& lm_mat(const gh_model* m) { return m->has_lm ? m->lm : m->embd; }

// Per-kernel event timing used by gh_profile_steps.
struct Profiler {
    struct Rec {
        int kind;
        double bytes;
        hipEvent_t a, b;
    };
    std::vector<Rec> recs;
    std::vector<std::string> names;
    // events created before the launches (reserve), so that the enqueue
    // loop only launches and keeps ahead of the GPU; the timed kernels then
    // run back to back as in a graph replay
    std::vector<hipEvent_t> pool;
    int kind_of(const char* name);
    int reserve(size_t n_events);
    void release_pool();
    Profiler() = default;
    Profiler(const Profiler&) = delete;  // owns the pooled events
    Profiler& operator=(const Profiler&) = delete;
    ~Profiler() { release_pool(); }
};

// kernels.hip: one decode step at position `pos` (patched per replay in graphs)
int enqueue_step(gh_model* m, gh_kv* kv, Sink& sink, int pos);
int persistent_supported(const gh_model* m);
size_t persistent_land(const gh_model* m);  // floats of the persistent step's landing area
int launch_interleave_gu(const DMat& gu, int f_pad, int F, const DMat& gi, hipStream_t s);
int enqueue_persistent(gh_model* m, gh_kv* kv, Sink& sink, int pos);
// kernels.hip: batched prefill of n tokens (ids in m->pf.tok) at positions
// pos0 .. pos0+n-1; with `head`, also the final norm, LM head and next-token
// selection of the last of them (position pos0+n-1).
constexpr int PF_MAX_TOKENS = 512;  // tokens per prefill pass
constexpr int PF_ATTN_NC = 16;      // attention chunks per token and kv head in the prefill
int pf_splits(const DMat& w, int Pp, int* kb_per);
int enqueue_prefill(gh_model* m, gh_kv* kv, Sink& sink, int n, int pos0, bool head);
int launch_q4_dequant(const DMat& w, float* out, hipStream_t s);
int launch_matvec_plain(const DMat& w, const Plan& p, const float* x, float* part, float* y,
                        int softcap, float cap, hipStream_t s);
int launch_rmsnorm(const float* x, const float* w, int n, float eps, int zc, float* y, hipStream_t s);
int launch_qk_norm(const float* x, const float* w, int n_heads, int hd, float eps, int zc, float* y,
                   hipStream_t s);
int launch_rope(float* x, int n_heads, int hd, const float* cs_dev, hipStream_t s);
int launch_attention(const float* q, const float* kc, const float* vc, int nq, int nkv, int hd,
                     int p_begin, int p_end, int n_splits, float* part, float* out, hipStream_t s);
int launch_gelu_mul(const float* g, const float* u, int n, float* h, hipStream_t s);
int launch_argmax(const float* v, int n, unsigned long long* key, hipStream_t s);
int launch_stream_read(const void* p, size_t bytes, float* sink, hipStream_t s);
int launch_xchg_probe(uint64_t* words, int n_wg, int rounds, int* err, unsigned long long* stamps, hipStream_t s);
constexpr int GH_ATTN_OP_MAX_NC = 256;  // chunks per kv head of the op-level attention
// Capacity (floats) of the static chunk-state array of
// gh_attention_decode_noalloc: nkv * n_splits * (nq / nkv) * (head_dim + 2)
// floats per call; 1 Mi floats = 4 MiB (C4: 264,192; 4B shapes: 528,384).
constexpr size_t ATTN_NOALLOC_SCRATCH_FLOATS = size_t(1) << 20;
// this device's address of that array (hipGetSymbolAddress, once per device)
int attn_noalloc_scratch(float** out);
// top_k 0: every logit; 1..GH_TOP_K_MAX (gemma_hip.h): the top_k largest
int launch_sample_logits(const float* logits, int n, float inv_temp, int top_k, uint64_t seed, uint64_t counter,
                         float* scratch, int32_t* token_dev, hipStream_t s);

// repack.cpp
void repack_q4_0(const uint8_t* raw, int64_t rows, int64_t cols, bool ftz, uint8_t* codes,
                 uint16_t* scales, int64_t tiles);
void repack_f32(const float* src, int64_t rows, int64_t cols, float* dst, int64_t tiles);
Plan choose_plan(int fmt, int tiles, int nblk, int target_wgs, int max_s = 8);
int kbw_for(int fmt, int per_wave);
// cos/sin of pos * inv_freq[i] in f32, as ropeShader computes the angle
void rope_table(const float* inv_freq, int half, int pos0, int n_pos, float* out);

}  // namespace gh
