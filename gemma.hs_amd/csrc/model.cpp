// Host side of the C ABI: contexts, buffers, Q4_0 tensors, op-level entry
// points, the model / KV-cache handles and the step/generate drivers.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>

#include "common.h"

using namespace gh;

namespace {

using Lock = std::lock_guard<std::recursive_mutex>;

// ---------------------------------------------------------------------
// Handle lifetimes.  Every handle the ABI returns is registered until its
// destroy call.  A destroy (or any other call) on a handle that is not
// registered -- destroyed already, or never returned -- is GH_ERR_STATE and
// touches no memory.  A context or model whose destroy is called while
// handles created from it are still open is only released: it stays alive
// (stream, device memory) until the last of them is destroyed, so handles
// may be destroyed in any order, as finalisers run them.
//
// Locking.  The registry mutex is a leaf: it is held only for one map
// operation (handle_add / handle_live / handle_take) and nothing else is
// locked or waited for while it is held.  Everything else about a handle --
// its parent's lists of children, the released flags, device memory -- is
// guarded by its context's mutex (gh_ctx::mu), and the decision to free a
// released context or model is taken under that mutex together with the
// state change that makes it collectable, so exactly one thread frees it.
// A finaliser destroying one handle while another thread steps on the same
// context therefore waits for the step and cannot deadlock with it.
// ---------------------------------------------------------------------
enum HandleKind { HK_CTX = 1, HK_MODEL, HK_KV, HK_Q4 };
std::mutex& handles_mu() {
    static auto* m = new std::mutex();  // never destroyed, as the map below
    return *m;
}
std::unordered_map<const void*, int>& handles() {
    static auto* h = new std::unordered_map<const void*, int>();  // never destroyed: finalisers may run at exit
    return *h;
}
void handle_add(const void* h, int kind) {
    std::lock_guard<std::mutex> g(handles_mu());
    handles()[h] = kind;
}
bool handle_live(const void* h, int kind) {
    std::lock_guard<std::mutex> g(handles_mu());
    auto it = handles().find(h);
    return it != handles().end() && it->second == kind;
}
// Unregisters an open handle of `kind`; false if it is not one.
bool handle_take(const void* h, int kind) {
    std::lock_guard<std::mutex> g(handles_mu());
    auto it = handles().find(h);
    if (it == handles().end() || it->second != kind) return false;
    handles().erase(it);
    return true;
}
const char* kind_name(int kind) {
    return kind == HK_CTX ? "context" : kind == HK_MODEL ? "model" : kind == HK_KV ? "KV cache" : "Q4_0 tensor";
}
int dead_handle(const char* fn, int kind) {
    return set_error(GH_ERR_STATE, "%s: not an open %s handle (destroyed already or never created)", fn, kind_name(kind));
}
#define GH_LIVE(h, kind)                                                  \
    do {                                                                  \
        if (!(h)) return set_error(GH_ERR_INVALID, "%s: null handle", __func__); \
        if (!handle_live((h), (kind))) return dead_handle(__func__, (kind)); \
    } while (0)

// Entry points taking a context handle: it must be open.
int ctx_bind(gh_ctx* ctx) {
    if (!ctx) return set_error(GH_ERR_INVALID, "null context");
    if (!handle_live(ctx, HK_CTX)) return dead_handle("context", HK_CTX);
    GH_HIP(hipSetDevice(ctx->device));
    return GH_OK;
}

// Entry points taking a model / cache / tensor handle (checked open by the
// caller): its context is alive, released or not.
int dev_bind(gh_ctx* ctx) {
    GH_HIP(hipSetDevice(ctx->device));
    return GH_OK;
}

template <class T>
int dev_alloc(gh_model* m, T** out, size_t count) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(count * sizeof(T), 16);
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return set_error(GH_ERR_OOM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    m->owned.push_back({p, bytes});
    *out = (T*)p;
    return GH_OK;
}

int upload(gh_ctx* ctx, void* dst, const void* src, size_t bytes) {
    GH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    GH_HIP(hipStreamSynchronize(ctx->stream));
    return GH_OK;
}

// Allocate a device matrix in tile layout.
int alloc_mat(gh_model* m, DMat& d, int fmt, int rows, int cols) {
    d.fmt = fmt;
    d.rows = rows;
    d.cols = cols;
    d.nblk = cols / block_cols(fmt);
    d.tiles = (rows + TILE_ROWS - 1) / TILE_ROWS;
    const size_t nb = (size_t)d.tiles * d.nblk * TILE_ROWS;
    uint8_t* codes = nullptr;
    GH_CHECK(dev_alloc(m, &codes, nb * 16));
    d.codes = codes;
    if (fmt == FMT_Q4) {
        uint16_t* sc = nullptr;
        GH_CHECK(dev_alloc(m, &sc, nb));
        d.scales = sc;
    }
    return GH_OK;
}

// Upload host rows [rows x cols] of `dtype` into the device matrix at a row
// offset that is a multiple of TILE_ROWS.
int upload_rows(gh_ctx* ctx, const DMat& d, int row_off, int dtype, const void* data, size_t nbytes,
                int rows, int cols, bool ftz) {
    if (row_off % TILE_ROWS) return set_error(GH_ERR_INVALID, "internal: unaligned row offset");
    const int64_t tiles = (rows + TILE_ROWS - 1) / TILE_ROWS;
    const int64_t t0 = row_off / TILE_ROWS;
    if (d.fmt == FMT_Q4) {
        if (dtype != GH_DTYPE_Q4_0) return set_error(GH_ERR_INVALID, "projection dtype differs from model format (Q4_0)");
        if (cols % 32) return set_error(GH_ERR_INVALID, "Q4_0 tensor with cols %% 32 != 0");
        const size_t need = (size_t)rows * (cols / 32) * 18;
        if (nbytes != need) return set_error(GH_ERR_INVALID, "Q4_0 tensor has %zu bytes, expected %zu", nbytes, need);
        const size_t nb = (size_t)tiles * d.nblk * TILE_ROWS;
        std::vector<uint8_t> codes(nb * 16);
        std::vector<uint16_t> sc(nb);
        repack_q4_0((const uint8_t*)data, rows, cols, ftz, codes.data(), sc.data(), tiles);
        const size_t off = (size_t)t0 * d.nblk * TILE_ROWS;
        GH_CHECK(upload(ctx, (uint8_t*)d.codes + off * 16, codes.data(), codes.size()));
        GH_CHECK(upload(ctx, (uint16_t*)d.scales + off, sc.data(), sc.size() * 2));
    } else {
        std::vector<float> f32;
        const float* src = (const float*)data;
        if (dtype == GH_DTYPE_F16) {
            if (nbytes != (size_t)rows * cols * 2) return set_error(GH_ERR_INVALID, "F16 tensor size mismatch");
            f32.resize((size_t)rows * cols);
            for (size_t i = 0; i < f32.size(); ++i) f32[i] = f16_to_f32(((const uint16_t*)data)[i], ftz);
            src = f32.data();
        } else if (dtype == GH_DTYPE_F32) {
            if (nbytes != (size_t)rows * cols * 4) return set_error(GH_ERR_INVALID, "F32 tensor size mismatch");
        } else {
            return set_error(GH_ERR_INVALID, "projection dtype differs from model format (F32)");
        }
        if (cols % 4) return set_error(GH_ERR_INVALID, "F32 matrix with cols %% 4 != 0");
        std::vector<float> tiled((size_t)tiles * d.nblk * TILE_ROWS * 4);
        repack_f32(src, rows, cols, tiled.data(), tiles);
        const size_t off = (size_t)t0 * d.nblk * TILE_ROWS * 4;
        GH_CHECK(upload(ctx, (float*)d.codes + off, tiled.data(), tiled.size() * 4));
    }
    return GH_OK;
}

int vec_to_f32(int dtype, const void* data, size_t nbytes, int n, bool ftz, std::vector<float>& out) {
    out.resize(n);
    if (dtype == GH_DTYPE_F32 && nbytes == (size_t)n * 4) {
        std::memcpy(out.data(), data, nbytes);
    } else if (dtype == GH_DTYPE_F16 && nbytes == (size_t)n * 2) {
        for (int i = 0; i < n; ++i) out[i] = f16_to_f32(((const uint16_t*)data)[i], ftz);
    } else {
        return set_error(GH_ERR_INVALID, "vector tensor: dtype %d with %zu bytes, expected %d elements", dtype, nbytes, n);
    }
    return GH_OK;
}

enum Kind {
    K_ATTN_NORM, K_Q, K_K, K_V, K_QN, K_KN, K_O, K_POST_ATTN, K_FFN_NORM, K_GATE, K_UP, K_DOWN, K_POST_FFN, K_N
};
const char* kKindNames[K_N] = {"attn_norm.weight",   "attn_q.weight",      "attn_k.weight",
                               "attn_v.weight",      "attn_q_norm.weight", "attn_k_norm.weight",
                               "attn_output.weight", "post_attention_norm.weight",
                               "ffn_norm.weight",    "ffn_gate.weight",    "ffn_up.weight",
                               "ffn_down.weight",    "post_ffw_norm.weight"};

uint32_t required_mask(const gh_config& c) {
    uint32_t m = (1u << K_ATTN_NORM) | (1u << K_Q) | (1u << K_K) | (1u << K_V) | (1u << K_O) |
                 (1u << K_GATE) | (1u << K_UP) | (1u << K_DOWN);
    if (c.flags & GH_FLAG_QK_NORM) m |= (1u << K_QN) | (1u << K_KN);
    if (c.flags & GH_FLAG_POST_ATTN_NORM) m |= 1u << K_POST_ATTN;
    if (c.flags & GH_FLAG_POST_FFN_NORM) m |= 1u << K_POST_FFN;
    return m;
}

int env_int(const char* name, int def) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : def;
}

// The GH_* environment switches that can change what the library runs, as
// "NAME=value,..." for those set ("" if none).
std::string env_switches() {
    static const char* vars[] = {
        "GH_PLAN_A_S", "GH_PLAN_C_S", "GH_PLAN_D_S", "GH_PLAN_E_S", "GH_PLAN_A_RL", "GH_PLAN_C_RL", "GH_PLAN_D_RL",
        "GH_PLAN_E_RL", "GH_PLAN_LM_RL", "GH_PLAN_A_NI", "GH_PLAN_C_NI", "GH_PLAN_D_NI", "GH_PLAN_E_NI",
        "GH_PLAN_A_MFMA", "GH_PLAN_C_MFMA", "GH_PLAN_D_MFMA", "GH_PLAN_E_MFMA", "GH_PLAN_LM_MFMA", "GH_PLAN_ORDER_IN", "GH_ATTN_NC", "GH_ATTN_HSPLIT",
        "GH_ATTN_XCD", "GH_PERSISTENT", "GH_NO_GRAPH", "GH_Q4_TARGET", "GH_Q4_MAXS", "GH_Q4_RL", "GH_Q4_MFMA", "GH_Q4_ORDER_IN", "GH_Q4_RG16"};
    std::string env;
    for (const char* v : vars) {
        const char* val = std::getenv(v);
        if (val && *val) env += (env.empty() ? "" : ",") + std::string(v) + "=" + val;
    }
    return env;
}

// Work-split plans, overridable for tuning sweeps with GH_PLAN_{A,C,D,E}_S.
void make_plans(gh_model* m) {
    m->plan_env = env_switches();
    const LayerDev& L = m->layers[0];
    // Measured on MI355X (sweeps of S x RL on the gemma3-1b and gemma3-4b
    // shapes): qkv, o_proj, down and the LM head run fastest as 64-row
    // work items (RL 1), qkv, o_proj and down with 8 splits (4B qkv, paired
    // on the matrix cores: 805 tok/s against 798 as 128-row items, which
    // won on the VALU, 6.3 vs 7.0 us; 1B 1734 against 1712); gate/up as 128-row work items with about 288 / tiles splits (1B: 3,
    // 4B: 2, raised to 3 below); with paired items 1B runs 5.38 us at 3
    // splits against 5.45 at 4 (1560 vs 1556 tok/s).
    m->pa = choose_plan(m->fmt, L.qkv.tiles, L.qkv.nblk, 256);
    m->pc = choose_plan(m->fmt, L.o.tiles, L.o.nblk, 256);
    m->pd = choose_plan(m->fmt, L.gu.tiles, L.gu.nblk, std::max(1, (288 + L.gu.tiles / 2) / L.gu.tiles) * L.gu.tiles);
    // gate/up: more splits until a wave's share of a split fits one register
    // batch of at most 9 blocks of its two rows per lane; a second batch's
    // loads wait for the first's dot products, and a 10-block batch of two
    // rows spills (4B: 2 -> 3 splits, gate/up 14.3 -> 11.9 us, 651 -> 690 tok/s)
    while (m->fmt == FMT_Q4 && m->pd.S < 8 && ((L.gu.nblk + m->pd.S - 1) / m->pd.S + 3) / 4 > 9) ++m->pd.S;
    m->pe = choose_plan(m->fmt, L.down.tiles, L.down.nblk, 8 * L.down.tiles);
    m->plm = choose_plan(lm_mat(m).fmt, lm_mat(m).tiles, lm_mat(m).nblk, 1);
    m->pa.rl = m->pc.rl = m->pe.rl = m->plm.rl = 1;
    auto over = [&](Plan& p, const char* env, const DMat& d) {
        int s = env_int(env, 0);
        if (s > 0) {
            Plan q = choose_plan(m->fmt, d.tiles, d.nblk, 1);
            q.S = std::min(s, d.nblk);
            p = q;
        }
    };
    auto capped = [](Plan& p) { p.S = std::min(p.S, 8); };
    over(m->pa, "GH_PLAN_A_S", L.qkv);
    over(m->pc, "GH_PLAN_C_S", L.o);
    over(m->pd, "GH_PLAN_D_S", L.gu);
    over(m->pe, "GH_PLAN_E_S", L.down);
    // rows per lane (2: 128-row workgroups, 1: 64-row workgroups)
    // Q4_0 dot products on the matrix cores: the LM head only.  They shorten
    // the dot phase of every work item, but their input limbs lengthen each
    // workgroup's prologue, and the per-layer kernels are prologue-bound:
    // measured on MI355X with every phase on the matrix cores, 1B decode
    // 1420 vs 1452 tok/s and 4B 580 vs 650 tok/s.
    m->plm.mfma = env_int("GH_PLAN_LM_MFMA", 1);
    m->pa.rl = env_int("GH_PLAN_A_RL", m->pa.rl);
    m->pc.rl = env_int("GH_PLAN_C_RL", m->pc.rl);
    m->pd.rl = env_int("GH_PLAN_D_RL", m->pd.rl);
    m->pe.rl = env_int("GH_PLAN_E_RL", m->pe.rl);
    m->plm.rl = env_int("GH_PLAN_LM_RL", m->plm.rl);
    for (Plan* p : {&m->pa, &m->pc, &m->pd, &m->pe, &m->plm}) p->rl = p->rl == 1 ? 1 : 2;
    capped(m->pe);
    // the down projection's GeGLU prologue holds gm float4 groups of each
    // gate/up split: gm * S <= 8 (gm <= 2 up to 2048 columns per split)
    m->pd.S = std::max(1, std::min(m->pd.S, 8 / std::max(1, std::min(2, geglu_groups(L.down, m->pe)))));
    for (Plan* p : {&m->pa, &m->pc, &m->pd, &m->pe}) {
        capped(*p);
        const DMat& d = p == &m->pa ? L.qkv : p == &m->pc ? L.o : p == &m->pd ? L.gu : L.down;
        p->kbw = kbw_for(m->fmt, ((d.nblk + p->S - 1) / p->S + 3) / 4);
    }
    // work items per workgroup: where a phase has at least as many work
    // items as the device has CUs, two items share one 8-wave workgroup and
    // so one prologue, which is what bounds these items.  Measured on
    // MI355X: 1B gate/up 432 -> 216 workgroups, 6.15 -> 5.5 us; 4B gate/up
    // 11.6 -> 10.7 us and down (320 items) 793 -> 820 tok/s; 4B qkv (256
    // items, with the inputs ordered ahead of the weights) 785 -> 792 tok/s.
    // Below the CU count pairing only halves the CUs in use (1B down, 144
    // items: 1538 -> 1501 tok/s; 1B qkv, 192 items: 1670 -> 1652); four
    // items per 16-wave workgroup leave 128 VGPRs a lane and spill.
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m->ctx->device) != hipSuccess || cus <= 0)
        cus = 256;
    // The O projection stays at one item: its attention-merge prologue
    // paired measured 4.25 -> 4.29 us on 4B.
    for (Plan* p : {&m->pa, &m->pd, &m->pe}) {
        const DMat& d = p == &m->pa ? L.qkv : p == &m->pd ? L.gu : L.down;
        p->ni = (long long)p->row_tiles(d.tiles) * p->S >= cus ? 2 : 1;
    }
    m->pa.ni = env_int("GH_PLAN_A_NI", m->pa.ni);
    m->pc.ni = env_int("GH_PLAN_C_NI", m->pc.ni);
    m->pd.ni = env_int("GH_PLAN_D_NI", m->pd.ni);
    m->pe.ni = env_int("GH_PLAN_E_NI", m->pe.ni);
    for (Plan* p : {&m->pa, &m->pc, &m->pd, &m->pe}) p->ni = p->ni == 2 ? 2 : 1;
    // Paired items run their dot products on the matrix cores: the lead
    // waves then build int8 limbs of the slice (a longer prologue) and the
    // dot phase shrinks.  Measured on MI355X, models differing only in this
    // choice alternating in one process: 1B gate/up (12 blocks per split)
    // 5.96 -> 5.74 us, 1618 -> 1632 tok/s; 4B 751 -> 773 tok/s (gate/up)
    // and 762 -> 773 (down); 4B qkv, paired, 791.6 -> 792.5.  The down
    // projection takes the matrix cores as single items too (its VALU dot
    // phase was 1.4 us of a 3 us chain on 1B): 1B 1678 -> 1728 tok/s once
    // the inputs were ordered ahead of the weights (1618 -> 1615 before).
    // Single-item qkv and o_proj stay on the VALU: 1B 1674 and 1670 against
    // 1678, 4B o_proj 790 against 796.
    for (Plan* p : {&m->pa, &m->pd, &m->pe}) p->mfma = m->fmt == FMT_Q4 && p->ni == 2 ? 1 : 0;
    if (m->fmt == FMT_Q4) m->pe.mfma = 1;
    m->pa.mfma = env_int("GH_PLAN_A_MFMA", m->pa.mfma);
    m->pc.mfma = m->fmt == FMT_Q4 ? env_int("GH_PLAN_C_MFMA", m->pc.mfma) : 0;
    m->pd.mfma = env_int("GH_PLAN_D_MFMA", m->pd.mfma);
    m->pe.mfma = env_int("GH_PLAN_E_MFMA", m->pe.mfma);
    m->attn_nc = std::max(1, std::min(64, env_int("GH_ATTN_NC", 64)));
    m->attn_xcd = env_int("GH_ATTN_XCD", 1) ? 1 : 0;
    // A barrier after the input loads, so that every wave's input loads
    // (the prologue's) go out before any wave's weight loads: without it a
    // CU's later waves queue their inputs behind the earlier waves' weights
    // and the norm, which needs all of them, waits for most of the stream.
    // Bits: 1 qkv, 2 o_proj, 4 gate/up, 8 down, 16 LM head.  Measured on
    // MI355X, models differing only in this alternating in one process
    // (three rounds each): 1B 1657 (none) / 1680 (matvec phases) / 1684
    // (and the LM head) tok/s, 4B 773 / 786 / 788.  The same barrier in
    // the step attention, between its prologue and its K/V loads, gained
    // nothing (1B 1678, 4B 784 with it).
    {
        const int oi = env_int("GH_PLAN_ORDER_IN", 31);
        m->pa.order_in = oi & 1;
        m->pc.order_in = (oi >> 1) & 1;
        m->pd.order_in = (oi >> 2) & 1;
        m->pe.order_in = (oi >> 3) & 1;
        m->plm.order_in = (oi >> 4) & 1;
    }
}

int ensure_scratch(gh_model* m) {
    if (m->x_res) return GH_OK;
    const gh_config& c = m->cfg;
    const LayerDev& L = m->layers[0];
    make_plans(m);
    const int G = c.n_heads / c.n_kv_heads;
    GH_CHECK(dev_alloc(m, &m->x_res, c.hidden));
    GH_CHECK(dev_alloc(m, &m->x1, c.hidden));
    GH_CHECK(dev_alloc(m, &m->part_qkv, (size_t)m->pa.S * L.qkv.tiles * TILE_ROWS));
    GH_CHECK(dev_alloc(m, &m->part_o, (size_t)m->pc.S * L.o.tiles * TILE_ROWS));
    GH_CHECK(dev_alloc(m, &m->part_gu, (size_t)m->pd.S * L.gu.tiles * TILE_ROWS));
    GH_CHECK(dev_alloc(m, &m->part_d, (size_t)m->pe.S * L.down.tiles * TILE_ROWS));
    GH_CHECK(dev_alloc(m, &m->attn_part, (size_t)c.n_kv_heads * m->attn_nc * G * (c.head_dim + 2)));
    GH_CHECK(dev_alloc(m, &m->logits, (size_t)m->embd.tiles * TILE_ROWS));
    GH_CHECK(dev_alloc(m, &m->layer_out, (size_t)c.n_layers * c.hidden));
    GH_CHECK(dev_alloc(m, &m->xn_final, c.hidden));
    // per LM-head workgroup (at most 2 per tile: 64-row workgroups)
    GH_CHECK(dev_alloc(m, &m->lm_cand, 2 * (size_t)m->embd.tiles));
    GH_CHECK(dev_alloc(m, &m->lm_m, 2 * (size_t)m->embd.tiles));
    GH_CHECK(dev_alloc(m, &m->lm_s, 2 * (size_t)m->embd.tiles));
    // persistent step: exchange words (GH_PERSISTENT=1 on a supported shape)
    m->persistent = env_int("GH_PERSISTENT", 0) && persistent_supported(m);
    if (m->persistent) {
        int cus = 0;
        GH_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m->ctx->device));
        if (cus <= 0) {
            m->persistent = 0;
        } else {
            m->p_grid = cus;
            m->p_np = std::min(c.ffn / 32, cus);
            const size_t nw[] = {(size_t)L.qkv.tiles * TILE_ROWS,
                                 (size_t)c.n_kv_heads * m->attn_nc * G * (c.head_dim + 2),
                                 (size_t)c.n_heads * c.head_dim, (size_t)c.hidden, (size_t)m->p_np * c.hidden,
                                 (size_t)c.hidden};
            uint64_t** ws[] = {&m->w_qkv, &m->w_attn, &m->w_o, &m->w_a, &m->w_p, &m->w_down};
            for (int i = 0; i < 6; ++i) {
                GH_CHECK(dev_alloc(m, ws[i], nw[i]));
                // epoch 0 everywhere: no published word matches before its phase
                GH_HIP(hipMemset(*ws[i], 0, nw[i] * sizeof(uint64_t)));
            }
            m->p_gi.resize(c.n_layers);
            for (int l = 0; l < c.n_layers; ++l) GH_CHECK(alloc_mat(m, m->p_gi[l], FMT_Q4, 2 * c.ffn, c.hidden));
        }
    }
    return GH_OK;
}

void free_prefill(gh_model* m) {
    PfBufs& B = m->pf;
    for (void* p : {(void*)B.x, (void*)B.x1, B.a, (void*)B.ascale, (void*)B.q, (void*)B.st, (void*)B.tok, (void*)B.part})
        if (p) hipFree(p);
    B = PfBufs{};
}

// Prefill buffers for passes of up to n tokens (rows rounded up to 64).
int prefill_reserve(gh_model* m, int n) {
    const gh_config& c = m->cfg;
    const int cap = (n + 63) / 64 * 64;
    if (cap > PF_MAX_TOKENS) return set_error(GH_ERR_INVALID, "internal: prefill pass of %d tokens", n);
    if (m->pf.cap >= cap) return GH_OK;
    GH_HIP(hipStreamSynchronize(m->ctx->stream));
    free_prefill(m);
    const LayerDev& L = m->layers[0];
    const int H = c.hidden, nq = c.n_heads, hd = c.head_dim;
    const size_t kmax = std::max({(size_t)H, (size_t)nq * hd, (size_t)c.ffn});
    size_t part = 0;
    for (const DMat* w : {&L.qkv, &L.o, &L.gu, &L.down})
        for (int pp = 64; pp <= cap; pp += 64)
            part = std::max(part, (size_t)pf_splits(*w, pp, nullptr) * pp * w->tiles * TILE_ROWS);
    PfBufs& B = m->pf;
    auto get = [&](void** p, size_t bytes) -> int {
        hipError_t e = hipMalloc(p, std::max<size_t>(bytes, 16));
        if (e != hipSuccess) {
            free_prefill(m);
            return set_error(GH_ERR_OOM, "prefill: hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
        }
        return GH_OK;
    };
    GH_CHECK(get((void**)&B.x, sizeof(float) * cap * H));
    GH_CHECK(get((void**)&B.x1, sizeof(float) * cap * H));
    GH_CHECK(get(&B.a, sizeof(float) * cap * kmax));  // 2 fp16 parts or 1 f32
    GH_CHECK(get((void**)&B.ascale, sizeof(float) * cap));
    GH_CHECK(get((void**)&B.q, sizeof(float) * cap * nq * hd));
    GH_CHECK(get((void**)&B.st, sizeof(float) * cap * nq * PF_ATTN_NC * (hd + 2)));
    GH_CHECK(get((void**)&B.tok, sizeof(int32_t) * cap));
    GH_CHECK(get((void**)&B.part, sizeof(float) * part));
    B.part_floats = part;
    B.cap = cap;
    return GH_OK;
}

int model_check(const gh_model* m);

// Called with the context mutex held, on a handle the caller checked open.
int model_ready(gh_model* m) {
    if (!m) return set_error(GH_ERR_INVALID, "null model");
    GH_CHECK(model_check(m));
    GH_CHECK(ensure_scratch(m));
    if (m->persistent && !m->p_gi_ok) {  // the persistent step's gate/up layout, from the uploaded weights
        for (int l = 0; l < m->cfg.n_layers; ++l)
            GH_CHECK(launch_interleave_gu(m->layers[l].gu, m->f_pad, m->cfg.ffn, m->p_gi[l], m->ctx->stream));
        GH_HIP(hipStreamSynchronize(m->ctx->stream));
        m->p_gi_ok = true;
    }
    return GH_OK;
}

// The step as a graph: a linear chain of kernel nodes built explicitly, so
// the nodes whose arguments hold the position can be patched per replay.
int kv_graph(gh_kv* kv) {
    if (kv->graph_exec) return GH_OK;
    gh_model* m = kv->m;
    hipGraph_t g = nullptr;
    GH_HIP(hipGraphCreate(&g, 0));
    Sink sink;
    sink.g = g;
    sink.store = &kv->graph_args;
    sink.patches = &kv->patches;
    kv->graph_args.clear();
    kv->patches.clear();
    int rc = m->persistent ? enqueue_persistent(m, kv, sink, 0) : enqueue_step(m, kv, sink, 0);
    if (rc != GH_OK) {
        hipGraphDestroy(g);
        return rc;
    }
    hipError_t e = hipGraphInstantiate(&kv->graph_exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        hipGraphDestroy(g);
        return set_error(GH_ERR_HIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
    }
    kv->graph = g;
    return GH_OK;
}

// One step at position `pos` on the stream: graph replay with the position
// patched into its nodes (default), or eager launches (GH_NO_GRAPH=1).
int launch_step(gh_kv* kv, int pos) {
    hipStream_t s = kv->m->ctx->stream;
    if (env_int("GH_NO_GRAPH", 0)) {
        Sink sink;
        sink.s = s;
        return kv->m->persistent ? enqueue_persistent(kv->m, kv, sink, pos) : enqueue_step(kv->m, kv, sink, pos);
    }
    GH_CHECK(kv_graph(kv));
    for (auto& p : kv->patches) {
        p.set(pos);
        GH_HIP(hipGraphExecKernelNodeSetParams(kv->graph_exec, p.node, &p.params));
    }
    GH_HIP(hipGraphLaunch(kv->graph_exec, s));
    return GH_OK;
}

// Host -> device step state (everything but the argmax keys).
int put_state(gh_kv* kv, int pos, int token, int start, int n_prompt, int gen_cap) {
    StepState* h = kv->h_st;
    h->pos = pos;
    h->token = token;
    h->last = -1;
    h->start = start;
    h->n_prompt = n_prompt;
    h->nan_flag = 0;
    h->gen_count = 0;
    h->gen_cap = gen_cap;
    h->inv_temp = kv->inv_temp;
    h->seed_lo = (uint32_t)kv->seed;
    h->seed_hi = (uint32_t)(kv->seed >> 32);
    h->xchg_err = 0;
    h->top_k = kv->top_k;
    GH_HIP(hipMemcpyAsync(kv->st, h, offsetof(StepState, keys), hipMemcpyHostToDevice, kv->m->ctx->stream));
    return GH_OK;
}

int get_state(gh_kv* kv) {
    GH_HIP(hipMemcpyAsync(kv->h_st, kv->st, sizeof(StepState), hipMemcpyDeviceToHost, kv->m->ctx->stream));
    return GH_OK;
}

}  // namespace

// =====================================================================
// context and buffers
// =====================================================================
extern "C" int gh_device_count(int* n) {
    if (!n) return set_error(GH_ERR_INVALID, "null output");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) c = 0;
    *n = c;
    return GH_OK;
}

extern "C" int gh_ctx_create(int device, gh_ctx** out) {
    if (!out) return set_error(GH_ERR_INVALID, "null output");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return set_error(GH_ERR_HIP, "no HIP device available");
    if (device < 0 || device >= n) return set_error(GH_ERR_INVALID, "device %d out of range (%d devices)", device, n);
    GH_HIP(hipSetDevice(device));
    std::unique_ptr<gh_ctx> c(new gh_ctx);
    c->device = device;
    GH_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    *out = c.release();
    handle_add(*out, HK_CTX);
    return GH_OK;
}

// Lifetime helpers.  ctx_dead and model_collect_locked run with the
// context mutex held; ctx_free runs after it is released.
namespace {

// True when a released context has no open model or Q4_0 tensor left; the
// caller that sees this (once: `dying` is set) frees it with ctx_free.
bool ctx_dead(gh_ctx* ctx) {
    if (ctx->dying || !ctx->released || !ctx->models.empty() || !ctx->q4s.empty()) return false;
    ctx->dying = true;
    return true;
}

// Frees a context that ctx_dead selected.  No other thread holds a handle
// made from it, so nothing else can be waiting on its mutex.
void ctx_free(gh_ctx* ctx) {
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    for (void* p : ctx->bufs) hipFree(p);
    if (ctx->scratch) hipFree(ctx->scratch);
    if (ctx->t0) hipEventDestroy(ctx->t0);
    if (ctx->t1) hipEventDestroy(ctx->t1);
    hipStreamDestroy(ctx->stream);
    delete ctx;
}

// Frees a released model that has no open KV cache left (context mutex
// held); returns whether its context is now to be freed.
bool model_collect_locked(gh_model* m) {
    gh_ctx* ctx = m->ctx;
    if (!m->released || !m->kvs.empty()) return false;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    free_prefill(m);
    for (auto& b : m->owned) hipFree(b.p);
    auto& v = ctx->models;
    v.erase(std::remove(v.begin(), v.end(), m), v.end());
    delete m;
    return ctx_dead(ctx);
}

}  // namespace

extern "C" int gh_ctx_destroy(gh_ctx* ctx) {
    if (!ctx) return GH_OK;
    if (!handle_take(ctx, HK_CTX)) return dead_handle("gh_ctx_destroy", HK_CTX);
    bool dead = false;
    {
        Lock lk(ctx->mu);
        ctx->released = true;
        dead = ctx_dead(ctx);
    }
    if (dead) ctx_free(ctx);
    return GH_OK;
}

extern "C" int gh_timer_start(gh_ctx* ctx) {
    GH_CHECK(ctx_bind(ctx));
    Lock lk(ctx->mu);
    if (!ctx->t0) GH_HIP(hipEventCreate(&ctx->t0));
    if (!ctx->t1) GH_HIP(hipEventCreate(&ctx->t1));
    GH_HIP(hipEventRecord(ctx->t0, ctx->stream));
    return GH_OK;
}

extern "C" int gh_timer_stop(gh_ctx* ctx, float* ms_out) {
    if (!ms_out) return set_error(GH_ERR_INVALID, "null output");
    GH_CHECK(ctx_bind(ctx));
    Lock lk(ctx->mu);
    if (!ctx->t0 || !ctx->t1) return set_error(GH_ERR_STATE, "gh_timer_stop without gh_timer_start");
    GH_HIP(hipEventRecord(ctx->t1, ctx->stream));
    GH_HIP(hipEventSynchronize(ctx->t1));
    GH_HIP(hipEventElapsedTime(ms_out, ctx->t0, ctx->t1));
    return GH_OK;
}

extern "C" int gh_capture_begin(gh_ctx* ctx) {
    GH_CHECK(ctx_bind(ctx));
    Lock lk(ctx->mu);
    GH_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return GH_OK;
}

extern "C" int gh_capture_replay(gh_ctx* ctx, int32_t n_replays, float* ms_per_replay_out) {
    GH_CHECK(ctx_bind(ctx));
    Lock lk(ctx->mu);
    hipGraph_t g = nullptr;
    GH_HIP(hipStreamEndCapture(ctx->stream, &g));
    if (n_replays <= 0 || !ms_per_replay_out) {
        hipGraphDestroy(g);
        return set_error(GH_ERR_INVALID, "bad arguments");
    }
    hipGraphExec_t ge = nullptr;
    int rc = GH_OK;
    hipEvent_t a = nullptr, b = nullptr;
    if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipGraphInstantiate failed");
    if (rc == GH_OK && (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess))
        rc = set_error(GH_ERR_HIP, "hipEventCreate failed");
    if (rc == GH_OK && hipGraphLaunch(ge, ctx->stream) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipGraphLaunch failed");
    if (rc == GH_OK && hipEventRecord(a, ctx->stream) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventRecord failed");
    for (int i = 0; i < n_replays && rc == GH_OK; ++i)
        if (hipGraphLaunch(ge, ctx->stream) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipGraphLaunch failed");
    float ms = 0.0f;
    if (rc == GH_OK && hipEventRecord(b, ctx->stream) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventRecord failed");
    if (rc == GH_OK && hipEventSynchronize(b) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventSynchronize failed");
    if (rc == GH_OK && hipEventElapsedTime(&ms, a, b) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventElapsedTime failed");
    if (a) hipEventDestroy(a);
    if (b) hipEventDestroy(b);
    if (ge) hipGraphExecDestroy(ge);
    hipGraphDestroy(g);
    GH_CHECK(rc);
    *ms_per_replay_out = ms / n_replays;
    return GH_OK;
}

extern "C" int gh_ctx_sync(gh_ctx* ctx) {
    GH_CHECK(ctx_bind(ctx));
    GH_HIP(hipStreamSynchronize(ctx->stream));
    return GH_OK;
}

extern "C" int gh_buf_alloc(gh_ctx* ctx, size_t bytes, void** dev) {
    GH_CHECK(ctx_bind(ctx));
    if (!dev) return set_error(GH_ERR_INVALID, "null output");
    Lock lk(ctx->mu);
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, std::max<size_t>(bytes, 16));
    if (e != hipSuccess) return set_error(GH_ERR_OOM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    ctx->bufs.push_back(p);
    *dev = p;
    return GH_OK;
}

extern "C" int gh_buf_free(gh_ctx* ctx, void* dev) {
    GH_CHECK(ctx_bind(ctx));
    Lock lk(ctx->mu);
    auto it = std::find(ctx->bufs.begin(), ctx->bufs.end(), dev);
    if (it == ctx->bufs.end()) return set_error(GH_ERR_INVALID, "buffer not owned by this context");
    GH_HIP(hipStreamSynchronize(ctx->stream));
    GH_HIP(hipFree(dev));
    ctx->bufs.erase(it);
    return GH_OK;
}

extern "C" int gh_buf_upload(gh_ctx* ctx, void* dev, const void* host, size_t bytes) {
    GH_CHECK(ctx_bind(ctx));
    Lock lk(ctx->mu);
    GH_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, ctx->stream));
    GH_HIP(hipStreamSynchronize(ctx->stream));
    return GH_OK;
}

extern "C" int gh_buf_download(gh_ctx* ctx, void* host, const void* dev, size_t bytes) {
    GH_CHECK(ctx_bind(ctx));
    Lock lk(ctx->mu);
    GH_HIP(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
    GH_HIP(hipStreamSynchronize(ctx->stream));
    return GH_OK;
}

// =====================================================================
// Q4_0 tensors
// =====================================================================
extern "C" int gh_q4_0_upload(gh_ctx* ctx, const void* raw, int64_t rows, int64_t cols, int flags, gh_q4** out) {
    GH_CHECK(ctx_bind(ctx));
    if (!raw || !out || rows <= 0 || cols <= 0 || cols % 32 || rows > (1 << 30) || cols > (1 << 24))
        return set_error(GH_ERR_INVALID, "gh_q4_0_upload: bad shape %lld x %lld (cols %% 32 must be 0)", (long long)rows, (long long)cols);
    Lock lk(ctx->mu);
    std::unique_ptr<gh_q4> t(new gh_q4);
    t->ctx = ctx;
    DMat& d = t->m;
    d.fmt = FMT_Q4;
    d.rows = (int)rows;
    d.cols = (int)cols;
    d.nblk = (int)(cols / 32);
    d.tiles = (int)((rows + TILE_ROWS - 1) / TILE_ROWS);
    const size_t nb = (size_t)d.tiles * d.nblk * TILE_ROWS;
    std::vector<uint8_t> codes(nb * 16);
    std::vector<uint16_t> sc(nb);
    repack_q4_0((const uint8_t*)raw, rows, cols, !(flags & GH_FLAG_IEEE_SCALES), codes.data(), sc.data(), d.tiles);
    GH_HIP(hipMalloc(&t->codes, codes.size()));
    GH_HIP(hipMalloc((void**)&t->scales, sc.size() * 2));
    d.codes = t->codes;
    d.scales = t->scales;
    GH_CHECK(upload(ctx, t->codes, codes.data(), codes.size()));
    GH_CHECK(upload(ctx, t->scales, sc.data(), sc.size() * 2));
    // 64-row workgroups.  One column split, so one kernel with no
    // partial-sum pass, where the rows alone give at least 96 workgroups;
    // otherwise about 512 workgroups with up to 16 column splits.  An
    // MI355X sweep of the C2 shapes over rotating cold copies: 6912x1152
    // 4.42 us with one split against 5.42 us with 8 and the partial-sum
    // kernel; 1152x6912 (18 row items) 5.85 us at 16 splits, 18.2 at one.
    const int max_s = env_int("GH_Q4_MAXS", 2 * d.tiles >= 96 ? 1 : 16);
    t->plan = choose_plan(FMT_Q4, d.tiles, d.nblk, env_int("GH_Q4_TARGET", 512), max_s);
    t->plan.rl = env_int("GH_Q4_RL", 1) == 2 ? 2 : 1;
    // dot products on the matrix cores: over cold copies on MI355X,
    // 262144 x 1152 29.5 us against 34.5 on the VALU, 6912 x 1152 4.01
    // against 4.41, 1152 x 6912 5.76 against 5.87
    t->plan.mfma = env_int("GH_Q4_MFMA", 1);
    t->plan.order_in = env_int("GH_Q4_ORDER_IN", 1) ? 1 : 0;
    // A split plan with at most 5120 columns on the matrix cores runs as
    // one kernel instead, one workgroup per 16 rows over all the columns
    // (k_mq_rows).  Over rotating cold copies on MI355X: 1536 x 1152 4.70
    // -> 3.53 us, 1152 x 1024 4.50 -> 3.48, 1024 x 2560 4.84 -> 4.02,
    // 4096 x 2560 5.93 -> 4.63, 2560 x 5120 6.25 -> 6.08; with longer rows
    // each workgroup's input prologue costs more than the split saves
    // (1152 x 6912 5.70 -> 6.49, 2560 x 8192 6.91 -> 8.59).  8 or 4 rows per
    // workgroup were slower at every shape but 640 x 4096 (4.57 vs 4.78).
    {
        const int R = env_int("GH_Q4_RG16", cols <= 5120 ? 16 : 0);
        t->plan.rg16 = t->plan.mfma && t->plan.S > 1 && cols <= 8192 && (R == 4 || R == 8 || R == 16) ? R : 0;
    }
    if (t->plan.S > 1 && !t->plan.rg16)
        GH_HIP(hipMalloc((void**)&t->part, sizeof(float) * t->plan.S * d.tiles * TILE_ROWS));
    ctx->q4s.push_back(t.get());
    *out = t.release();
    handle_add(*out, HK_Q4);
    return GH_OK;
}

gh_q4::~gh_q4() {
    if (codes) hipFree(codes);
    if (scales) hipFree(scales);
    if (part) hipFree(part);
}

extern "C" int gh_q4_0_free(gh_q4* t) {
    if (!t) return GH_OK;
    if (!handle_take(t, HK_Q4)) return dead_handle("gh_q4_0_free", HK_Q4);
    gh_ctx* ctx = t->ctx;
    bool dead = false;
    {
        Lock lk(ctx->mu);
        hipSetDevice(ctx->device);
        hipStreamSynchronize(ctx->stream);
        auto& v = ctx->q4s;
        v.erase(std::remove(v.begin(), v.end(), t), v.end());
        delete t;
        dead = ctx_dead(ctx);
    }
    if (dead) ctx_free(ctx);
    return GH_OK;
}

// Op-level calls are synchronous, except while the context stream is being
// captured (gh_capture_begin): then they only enqueue.
static int op_sync(gh_ctx* ctx) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    GH_HIP(hipStreamIsCapturing(ctx->stream, &st));
    if (st == hipStreamCaptureStatusNone) GH_HIP(hipStreamSynchronize(ctx->stream));
    return GH_OK;
}

// Per-context device scratch for op-level temporaries; grows outside capture.
static int ctx_scratch(gh_ctx* ctx, size_t bytes, void** out) {
    if (bytes > ctx->scratch_bytes) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        GH_HIP(hipStreamIsCapturing(ctx->stream, &st));
        if (st != hipStreamCaptureStatusNone)
            return set_error(GH_ERR_STATE, "op needs %zu B of scratch while capturing; run it once before capture", bytes);
        GH_HIP(hipStreamSynchronize(ctx->stream));
        if (ctx->scratch) GH_HIP(hipFree(ctx->scratch));
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
        GH_HIP(hipMalloc(&ctx->scratch, bytes));
        ctx->scratch_bytes = bytes;
    }
    *out = ctx->scratch;
    return GH_OK;
}

extern "C" int gh_q4_0_dequant(gh_q4* t, float* out) {
    GH_LIVE(t, HK_Q4);
    if (!t || !out) return set_error(GH_ERR_INVALID, "null argument");
    GH_CHECK(dev_bind(t->ctx));
    Lock lk(t->ctx->mu);
    GH_CHECK(launch_q4_dequant(t->m, out, t->ctx->stream));
    GH_CHECK(op_sync(t->ctx));
    return GH_OK;
}

extern "C" int gh_q4_0_matvec(gh_q4* t, const float* x, float* y, int softcap, float cap) {
    GH_LIVE(t, HK_Q4);
    if (!t || !x || !y) return set_error(GH_ERR_INVALID, "null argument");
    if (softcap && !(cap > 0.0f)) return set_error(GH_ERR_INVALID, "soft-cap value must be > 0");
    GH_CHECK(dev_bind(t->ctx));
    Lock lk(t->ctx->mu);
    GH_CHECK(launch_matvec_plain(t->m, t->plan, x, t->part, y, softcap, cap, t->ctx->stream));
    GH_CHECK(op_sync(t->ctx));
    return GH_OK;
}

extern "C" int gh_linear_q4(gh_ctx* ctx, const uint32_t* raw_words, size_t n_words, const float* x, int rows,
                            int cols, int softcap, float cap, float* y) {
    GH_CHECK(ctx_bind(ctx));
    if (!raw_words || !x || !y || rows <= 0 || cols <= 0 || cols % 32)
        return set_error(GH_ERR_INVALID, "gh_linear_q4: bad arguments (cols %% 32 must be 0)");
    const size_t need = (size_t)rows * (cols / 32) * 18;
    if (n_words * 4 < need) return set_error(GH_ERR_INVALID, "gh_linear_q4: %zu words hold fewer than %zu bytes", n_words, need);
    gh_q4* t = nullptr;
    GH_CHECK(gh_q4_0_upload(ctx, raw_words, rows, cols, 0, &t));
    float *dx = nullptr, *dy = nullptr;
    int rc = GH_OK;
    if (hipMalloc((void**)&dx, sizeof(float) * cols) != hipSuccess || hipMalloc((void**)&dy, sizeof(float) * rows) != hipSuccess) {
        rc = set_error(GH_ERR_OOM, "gh_linear_q4: allocation failed");
    }
    if (rc == GH_OK) rc = upload(ctx, dx, x, sizeof(float) * cols);
    if (rc == GH_OK) rc = gh_q4_0_matvec(t, dx, dy, softcap, cap);
    if (rc == GH_OK && hipMemcpy(y, dy, sizeof(float) * rows, hipMemcpyDeviceToHost) != hipSuccess)
        rc = set_error(GH_ERR_HIP, "gh_linear_q4: download failed");
    if (dx) hipFree(dx);
    if (dy) hipFree(dy);
    gh_q4_0_free(t);
    return rc;
}

// =====================================================================
// op-level entry points (device pointers)
// =====================================================================
#define OP_ENTER(ctx)             \
    GH_CHECK(ctx_bind(ctx));      \
    Lock lk((ctx)->mu)

extern "C" int gh_rmsnorm(gh_ctx* ctx, const float* x, const float* w, int n, float eps, int zc, float* y) {
    OP_ENTER(ctx);
    if (!x || !w || !y || n <= 0) return set_error(GH_ERR_INVALID, "gh_rmsnorm: bad arguments");
    GH_CHECK(launch_rmsnorm(x, w, n, eps, zc, y, ctx->stream));
    GH_CHECK(op_sync(ctx));
    return GH_OK;
}

extern "C" int gh_qk_norm(gh_ctx* ctx, const float* x, const float* w, int n_heads, int hd, float eps, int zc, float* y) {
    OP_ENTER(ctx);
    if (!x || !w || !y || n_heads <= 0) return set_error(GH_ERR_INVALID, "gh_qk_norm: bad arguments");
    GH_CHECK(launch_qk_norm(x, w, n_heads, hd, eps, zc, y, ctx->stream));
    GH_CHECK(op_sync(ctx));
    return GH_OK;
}

extern "C" int gh_rope(gh_ctx* ctx, float* x, int n_heads, int hd, float theta, int pos) {
    OP_ENTER(ctx);
    if (!x || n_heads <= 0 || pos < 0 || hd <= 0 || hd % 2) return set_error(GH_ERR_INVALID, "gh_rope: bad arguments");
    const int half = hd / 2;
    std::vector<float> f(half), tab((size_t)half * 2);
    for (int i = 0; i < half; ++i) f[i] = 1.0f / powf(theta, (float)(i * 2) / (float)hd);
    rope_table(f.data(), half, pos, 1, tab.data());
    float* d = nullptr;
    GH_HIP(hipMalloc((void**)&d, tab.size() * sizeof(float)));
    int rc = upload(ctx, d, tab.data(), tab.size() * sizeof(float));
    if (rc == GH_OK) rc = launch_rope(x, n_heads, hd, d, ctx->stream);
    if (rc == GH_OK) rc = op_sync(ctx);
    hipFree(d);
    return rc;
}

extern "C" int gh_attention_decode(gh_ctx* ctx, const float* q, const float* kc, const float* vc, int nq, int nkv,
                                   int hd, int p_begin, int p_end, int n_splits, float* out) {
    OP_ENTER(ctx);
    if (!q || !kc || !vc || !out || nkv <= 0 || nq % nkv || p_begin < 0 || p_end <= p_begin)
        return set_error(GH_ERR_INVALID, "gh_attention_decode: bad arguments");
    const int n_pos = p_end - p_begin;
    // default: 32-position chunks, at most GH_ATTN_OP_MAX_NC (256) per kv
    // head; an MI355X sweep of the chunk count with the single-round-trip
    // merge: 8192 positions 8.7 us at 256 chunks vs 10.3 at 128, 32768
    // 18.6 us at 256 vs 22.9 at 128, the last 512 7.3 us at 16 vs 9.6 at 8
    if (n_splits <= 0) n_splits = std::max(1, std::min((n_pos + 31) / 32, GH_ATTN_OP_MAX_NC));
    n_splits = std::min(std::min(n_splits, n_pos), GH_ATTN_OP_MAX_NC);
    void* part = nullptr;
    const int G = nq / nkv;
    GH_CHECK(ctx_scratch(ctx, sizeof(float) * nkv * n_splits * G * (hd + 2), &part));
    GH_CHECK(launch_attention(q, kc, vc, nq, nkv, hd, p_begin, p_end, n_splits, (float*)part, out, ctx->stream));
    return op_sync(ctx);
}

extern "C" int gh_attention_decode_noalloc(gh_ctx* ctx, const float* q, const float* kc, const float* vc, int nq,
                                           int nkv, int hd, int p_begin, int p_end, int n_splits, float* out) {
    OP_ENTER(ctx);
    if (!q || !kc || !vc || !out || nkv <= 0 || nq <= 0 || nq % nkv || p_begin < 0 || p_end <= p_begin)
        return set_error(GH_ERR_INVALID, "gh_attention_decode_noalloc: bad arguments");
    const int n_pos = p_end - p_begin;
    if (n_splits <= 0) n_splits = std::max(1, std::min((n_pos + 31) / 32, GH_ATTN_OP_MAX_NC));
    n_splits = std::min(std::min(n_splits, n_pos), GH_ATTN_OP_MAX_NC);
    const size_t need = (size_t)nkv * n_splits * (nq / nkv) * ((size_t)hd + 2);
    if (need > ATTN_NOALLOC_SCRATCH_FLOATS)
        return set_error(GH_ERR_RANGE,
                         "gh_attention_decode_noalloc: %zu floats of chunk states exceed the static %zu-float "
                         "scratch (fewer splits or gh_attention_decode)", need, ATTN_NOALLOC_SCRATCH_FLOATS);
    float* part = nullptr;
    GH_CHECK(attn_noalloc_scratch(&part));
    GH_CHECK(launch_attention(q, kc, vc, nq, nkv, hd, p_begin, p_end, n_splits, part, out, ctx->stream));
    return op_sync(ctx);
}

extern "C" int gh_gelu_mul(gh_ctx* ctx, const float* g, const float* u, int n, float* h) {
    OP_ENTER(ctx);
    if (!g || !u || !h || n <= 0) return set_error(GH_ERR_INVALID, "gh_gelu_mul: bad arguments");
    GH_CHECK(launch_gelu_mul(g, u, n, h, ctx->stream));
    GH_CHECK(op_sync(ctx));
    return GH_OK;
}

static int argmax_locked(gh_ctx* ctx, const float* v, int n, int32_t* idx);

extern "C" int gh_sample_logits(gh_ctx* ctx, const float* logits, int n, float temperature, uint64_t seed,
                                uint64_t counter, int32_t* token_out) {
    return gh_sample_logits_top_k(ctx, logits, n, temperature, 0, seed, counter, token_out);
}

extern "C" int gh_sample_logits_top_k(gh_ctx* ctx, const float* logits, int n, float temperature, int32_t top_k,
                                      uint64_t seed, uint64_t counter, int32_t* token_out) {
    OP_ENTER(ctx);
    if (!logits || !token_out || n <= 0) return set_error(GH_ERR_INVALID, "gh_sample_logits: bad arguments");
    if (!(temperature >= 0.0f) || std::isinf(temperature))
        return set_error(GH_ERR_INVALID, "temperature must be finite and >= 0");
    if (top_k < 0 || top_k > GH_TOP_K_MAX)
        return set_error(GH_ERR_RANGE, "top_k %d outside [0, %d]", top_k, GH_TOP_K_MAX);
    if (temperature == 0.0f) return argmax_locked(ctx, logits, n, token_out);
    const int nblk = (n + 63) / 64;
    void* scratch = nullptr;
    GH_CHECK(ctx_scratch(ctx, sizeof(float) * (2 * (size_t)nblk + 4), &scratch));
    float* sc = (float*)scratch;
    int32_t* tok_dev = (int32_t*)(sc + 2 * (size_t)nblk);
    GH_CHECK(launch_sample_logits(logits, n, 1.0f / temperature, top_k, seed, counter, sc, tok_dev, ctx->stream));
    int32_t tok = -1;
    GH_HIP(hipMemcpyAsync(&tok, tok_dev, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
    GH_CHECK(op_sync(ctx));
    *token_out = tok;
    return GH_OK;
}

extern "C" int gh_argmax(gh_ctx* ctx, const float* v, int n, int32_t* idx) {
    OP_ENTER(ctx);
    return argmax_locked(ctx, v, n, idx);
}

// gh_argmax on a bound context whose mutex the caller holds.
static int argmax_locked(gh_ctx* ctx, const float* v, int n, int32_t* idx) {
    if (!v || !idx || n <= 0) return set_error(GH_ERR_INVALID, "gh_argmax: bad arguments");
    unsigned long long* key = nullptr;  // [0] result, [1..1024] per-block keys
    GH_HIP(hipMallocAsync((void**)&key, 8 * 1025, ctx->stream));
    int rc = launch_argmax(v, n, key, ctx->stream);
    unsigned long long h = 0;
    if (rc == GH_OK) {
        GH_HIP(hipMemcpyAsync(&h, key, 8, hipMemcpyDeviceToHost, ctx->stream));
    }
    hipFreeAsync(key, ctx->stream);
    GH_CHECK(op_sync(ctx));
    if (rc == GH_OK) *idx = (int32_t)(0xFFFFFFFFu - (uint32_t)(h & 0xFFFFFFFFull));
    return rc;
}

// =====================================================================
// configs and models
// =====================================================================
extern "C" int gh_config_preset(const char* name, gh_config* out) {
    if (!name || !out) return set_error(GH_ERR_INVALID, "null argument");
    gh_config c{};
    c.rms_eps = 1e-6f;
    c.mode = GH_MODE_GEMMA3;
    c.flags = GH_FLAG_QK_NORM | GH_FLAG_POST_ATTN_NORM | GH_FLAG_POST_FFN_NORM | GH_FLAG_ZERO_CENTERED;
    if (!std::strcmp(name, "tiny")) {
        c.vocab = 1024; c.hidden = 128; c.n_layers = 2; c.n_heads = 4; c.n_kv_heads = 1;
        c.head_dim = 32; c.ffn = 512; c.max_seq = 2048; c.sliding_window = 0; c.global_every = 0;
        c.rope_theta_local = 10000.0f; c.rope_theta_global = 10000.0f;
    } else if (!std::strcmp(name, "gemma3-1b")) {
        // src/Gemma/Model.hs:213-237 plus the Gemma-3 5:1 local/global layout
        c.vocab = 262144; c.hidden = 1152; c.n_layers = 26; c.n_heads = 4; c.n_kv_heads = 1;
        c.head_dim = 256; c.ffn = 6912; c.max_seq = 2048; c.sliding_window = 512; c.global_every = 6;
        c.rope_theta_local = 10000.0f; c.rope_theta_global = 1000000.0f;
    } else if (!std::strcmp(name, "gemma3-4b")) {
        c.vocab = 262144; c.hidden = 2560; c.n_layers = 34; c.n_heads = 8; c.n_kv_heads = 4;
        c.head_dim = 256; c.ffn = 10240; c.max_seq = 8192; c.sliding_window = 1024; c.global_every = 6;
        c.rope_theta_local = 10000.0f; c.rope_theta_global = 1000000.0f;
    } else {
        return set_error(GH_ERR_NOT_FOUND, "unknown preset '%s'", name);
    }
    *out = c;
    return GH_OK;
}

extern "C" int gh_model_create(gh_ctx* ctx, const gh_config* cfg, gh_model** out) {
    GH_CHECK(ctx_bind(ctx));
    if (!cfg || !out) return set_error(GH_ERR_INVALID, "null argument");
    const gh_config& c = *cfg;
    if (c.vocab <= 0 || c.hidden <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.ffn <= 0 ||
        c.head_dim <= 0 || c.max_seq <= 0)
        return set_error(GH_ERR_INVALID, "config: dimensions must be positive");
    if (c.n_heads % c.n_kv_heads) return set_error(GH_ERR_INVALID, "config: n_heads %% n_kv_heads != 0");
    const int G = c.n_heads / c.n_kv_heads;
    if (!(c.head_dim == 32 || c.head_dim == 128 || c.head_dim == 256) || !(G == 1 || G == 2 || G == 4 || G == 8))
        return set_error(GH_ERR_INVALID, "config: head_dim %d / group %d not supported", c.head_dim, G);
    if (c.hidden % 32 || c.ffn % 32 || (c.n_heads * c.head_dim) % 32)
        return set_error(GH_ERR_INVALID, "config: hidden, ffn and n_heads*head_dim must be multiples of 32");
    if (c.mode != GH_MODE_GEMMA3 && c.mode != GH_MODE_REF) return set_error(GH_ERR_INVALID, "config: bad mode");
    // the residual prologues hold at most 3 float4 groups of the hidden
    // vector per thread of a 256-thread workgroup
    if (c.hidden > 3072) return set_error(GH_ERR_INVALID, "config: hidden %d above 3072", c.hidden);
    if (c.sliding_window < 0 || c.global_every < 0)
        return set_error(GH_ERR_INVALID, "config: sliding_window and global_every must be >= 0");
    if (!(c.rope_theta_local > 0.0f) || !(c.rope_theta_global > 0.0f) || std::isinf(c.rope_theta_local) ||
        std::isinf(c.rope_theta_global))
        return set_error(GH_ERR_INVALID, "config: RoPE theta must be finite and > 0");
    if (!(c.rms_eps >= 0.0f) || std::isinf(c.rms_eps))
        return set_error(GH_ERR_INVALID, "config: rms_eps must be finite and >= 0");
    Lock lk(ctx->mu);
    std::unique_ptr<gh_model> m(new gh_model);
    m->ctx = ctx;
    m->cfg = c;
    m->layers.resize(c.n_layers);
    m->present.assign(c.n_layers, 0);
    m->q_rows_pad = pad_rows(c.n_heads * c.head_dim);
    m->kv_rows_pad = pad_rows(c.n_kv_heads * c.head_dim);
    m->f_pad = pad_rows(c.ffn);
    for (int l = 0; l < c.n_layers; ++l)
        m->layers[l].global = c.global_every <= 0 || ((l + 1) % c.global_every) == 0;
    // RoPE inverse frequencies, ropeShader's formula (AttentionGPU.hs:98-99)
    m->inv_freq.resize(c.head_dim);
    for (int i = 0; i < c.head_dim / 2; ++i) {
        const float e = (float)(i * 2) / (float)c.head_dim;
        m->inv_freq[i] = 1.0f / powf(c.rope_theta_local, e);
        m->inv_freq[c.head_dim / 2 + i] = 1.0f / powf(c.rope_theta_global, e);
    }
    ctx->models.push_back(m.get());
    *out = m.release();
    handle_add(*out, HK_MODEL);
    return GH_OK;
}

extern "C" int gh_model_destroy(gh_model* m) {
    if (!m) return GH_OK;
    if (!handle_take(m, HK_MODEL)) return dead_handle("gh_model_destroy", HK_MODEL);
    gh_ctx* ctx = m->ctx;
    bool dead = false;
    {
        Lock lk(ctx->mu);
        m->released = true;
        dead = model_collect_locked(m);
    }
    if (dead) ctx_free(ctx);
    return GH_OK;
}

// The projections share one format (Q4_0 or f32), set by the first one
// uploaded; the embedding (the tied LM head) has its own, so a Q4_0 model
// can carry an embedding the GGUF loader dequantised (Q4_1).
static int ensure_fmt(gh_model* m, int dtype) {
    const int want = dtype == GH_DTYPE_Q4_0 ? FMT_Q4 : FMT_F32;
    if (m->fmt < 0) {
        m->fmt = want;
        const gh_config& c = m->cfg;
        for (auto& L : m->layers) {
            GH_CHECK(alloc_mat(m, L.qkv, want, m->q_rows_pad + 2 * m->kv_rows_pad, c.hidden));
            GH_CHECK(alloc_mat(m, L.o, want, c.hidden, c.n_heads * c.head_dim));
            GH_CHECK(alloc_mat(m, L.gu, want, 2 * m->f_pad, c.hidden));
            GH_CHECK(alloc_mat(m, L.down, want, c.hidden, c.ffn));
        }
    } else if (m->fmt != want) {
        return set_error(GH_ERR_INVALID, "all projections must share one format");
    }
    return GH_OK;
}

static int ensure_embd_fmt(gh_model* m, int dtype) {
    const int want = dtype == GH_DTYPE_Q4_0 ? FMT_Q4 : FMT_F32;
    if (!m->embd.codes) return alloc_mat(m, m->embd, want, m->cfg.vocab, m->cfg.hidden);
    if (m->embd.fmt != want) return set_error(GH_ERR_INVALID, "token_embd.weight was uploaded in another format");
    return GH_OK;
}

extern "C" int gh_model_set_tensor(gh_model* m, const char* name, int dtype, const void* data, size_t nbytes) {
    GH_LIVE(m, HK_MODEL);
    if (!m || !name || !data) return set_error(GH_ERR_INVALID, "null argument");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    const gh_config& c = m->cfg;
    const bool ftz = !(c.flags & GH_FLAG_IEEE_SCALES);
    std::vector<float> v;
    if (!std::strcmp(name, "token_embd.weight")) {
        GH_CHECK(ensure_embd_fmt(m, dtype));
        GH_CHECK(upload_rows(m->ctx, m->embd, 0, dtype, data, nbytes, c.vocab, c.hidden, ftz));
        m->has_embd = true;
        return GH_OK;
    }
    if (!std::strcmp(name, "output.weight")) {
        // untied LM head (src/Gemma/Model.hs:412-414 lm_head.weight; GGUF
        // output.weight, src/Gemma/Model.hs:988), in its own format; the
        // step's plans and graphs are built from it at the first step
        if (m->x_res) return set_error(GH_ERR_STATE, "output.weight must be set before the model's first step");
        const int want = dtype == GH_DTYPE_Q4_0 ? FMT_Q4 : FMT_F32;
        if (!m->lm.codes) GH_CHECK(alloc_mat(m, m->lm, want, c.vocab, c.hidden));
        else if (m->lm.fmt != want) return set_error(GH_ERR_INVALID, "output.weight was uploaded in another format");
        GH_CHECK(upload_rows(m->ctx, m->lm, 0, dtype, data, nbytes, c.vocab, c.hidden, ftz));
        m->has_lm = true;
        return GH_OK;
    }
    if (!std::strcmp(name, "output_norm.weight")) {
        GH_CHECK(vec_to_f32(dtype, data, nbytes, c.hidden, ftz, v));
        if (!m->out_norm) GH_CHECK(dev_alloc(m, &m->out_norm, c.hidden));
        GH_CHECK(upload(m->ctx, m->out_norm, v.data(), v.size() * 4));
        m->has_out_norm = true;
        return GH_OK;
    }
    if (std::strncmp(name, "blk.", 4))
        return set_error(GH_ERR_NOT_FOUND, "unknown tensor '%s'", name);
    char* end = nullptr;
    long l = std::strtol(name + 4, &end, 10);
    if (!end || *end != '.' || l < 0 || l >= c.n_layers) return set_error(GH_ERR_NOT_FOUND, "bad layer in '%s'", name);
    int kind = -1;
    for (int k = 0; k < K_N; ++k)
        if (!std::strcmp(end + 1, kKindNames[k])) kind = k;
    if (kind < 0) return set_error(GH_ERR_NOT_FOUND, "unknown tensor '%s'", name);
    LayerDev& L = m->layers[l];
    const int H = c.hidden, hd = c.head_dim;
    auto vec = [&](float*& dst, int n) -> int {
        GH_CHECK(vec_to_f32(dtype, data, nbytes, n, ftz, v));
        if (!dst) GH_CHECK(dev_alloc(m, &dst, n));
        return upload(m->ctx, dst, v.data(), (size_t)n * 4);
    };
    switch (kind) {
        case K_ATTN_NORM: GH_CHECK(vec(L.attn_norm, H)); break;
        case K_QN: GH_CHECK(vec(L.q_norm, hd)); break;
        case K_KN: GH_CHECK(vec(L.k_norm, hd)); break;
        case K_POST_ATTN: GH_CHECK(vec(L.post_attn, H)); break;
        case K_FFN_NORM: GH_CHECK(vec(L.ffn_norm, H)); break;
        case K_POST_FFN: GH_CHECK(vec(L.post_ffw, H)); break;
        case K_Q:
            GH_CHECK(ensure_fmt(m, dtype));
            GH_CHECK(upload_rows(m->ctx, L.qkv, 0, dtype, data, nbytes, c.n_heads * hd, H, ftz));
            break;
        case K_K:
            GH_CHECK(ensure_fmt(m, dtype));
            GH_CHECK(upload_rows(m->ctx, L.qkv, m->q_rows_pad, dtype, data, nbytes, c.n_kv_heads * hd, H, ftz));
            break;
        case K_V:
            GH_CHECK(ensure_fmt(m, dtype));
            GH_CHECK(upload_rows(m->ctx, L.qkv, m->q_rows_pad + m->kv_rows_pad, dtype, data, nbytes, c.n_kv_heads * hd, H, ftz));
            break;
        case K_O:
            GH_CHECK(ensure_fmt(m, dtype));
            GH_CHECK(upload_rows(m->ctx, L.o, 0, dtype, data, nbytes, H, c.n_heads * hd, ftz));
            break;
        case K_GATE:
            m->p_gi_ok = false;
            GH_CHECK(ensure_fmt(m, dtype));
            GH_CHECK(upload_rows(m->ctx, L.gu, 0, dtype, data, nbytes, c.ffn, H, ftz));
            break;
        case K_UP:
            m->p_gi_ok = false;
            GH_CHECK(ensure_fmt(m, dtype));
            GH_CHECK(upload_rows(m->ctx, L.gu, m->f_pad, dtype, data, nbytes, c.ffn, H, ftz));
            break;
        case K_DOWN:
            GH_CHECK(ensure_fmt(m, dtype));
            GH_CHECK(upload_rows(m->ctx, L.down, 0, dtype, data, nbytes, H, c.ffn, ftz));
            break;
    }
    m->present[l] |= 1u << kind;
    return GH_OK;
}

extern "C" int gh_model_check(gh_model* m) {
    GH_LIVE(m, HK_MODEL);
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    return model_check(m);
}

namespace {
int model_check(const gh_model* m) {
    if (!m->has_embd) return set_error(GH_ERR_NOT_FOUND, "missing tensor token_embd.weight");
    if (!m->has_out_norm) return set_error(GH_ERR_NOT_FOUND, "missing tensor output_norm.weight");
    const uint32_t need = required_mask(m->cfg);
    for (int l = 0; l < m->cfg.n_layers; ++l) {
        const uint32_t miss = need & ~m->present[l];
        if (miss) {
            for (int k = 0; k < K_N; ++k)
                if (miss & (1u << k)) return set_error(GH_ERR_NOT_FOUND, "missing tensor blk.%d.%s", l, kKindNames[k]);
        }
        if (!m->layers[l].ffn_norm && !m->layers[l].post_attn)
            return set_error(GH_ERR_NOT_FOUND, "missing tensor blk.%d.ffn_norm.weight", l);
    }
    return GH_OK;
}
}  // namespace

extern "C" int gh_model_plan(gh_model* m, char* buf, size_t cap, size_t* len_out) {
    GH_LIVE(m, HK_MODEL);
    if (!buf && cap) return set_error(GH_ERR_INVALID, "null buffer with a non-zero capacity");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    GH_CHECK(model_check(m));
    if (!m->x_res) make_plans(m);  // what ensure_scratch will choose at the first step
    const bool persistent = m->x_res ? m->persistent != 0 : env_int("GH_PERSISTENT", 0) && persistent_supported(m);
    std::string s = std::string("step=") + (persistent ? "persistent" : env_int("GH_NO_GRAPH", 0) ? "eager" : "graph");
    auto phase = [&](const char* name, const Plan& p) {
        char t[96];
        std::snprintf(t, sizeof t, " %s=S%d,rl%d,ni%d,%s%s", name, p.S, p.rl, p.ni, p.mfma ? "mfma" : "valu",
                      p.order_in ? ",in_first" : "");
        s += t;
    };
    phase("qkv", m->pa);
    phase("o_proj", m->pc);
    phase("gate_up", m->pd);
    phase("down", m->pe);
    phase("lm_head", m->plm);
    s += " attn_chunks=" + std::to_string(m->attn_nc) + (m->attn_xcd ? "" : ",xcd_off");
    s += std::string(" lm=") + (m->has_lm ? "untied" : "tied");
    s += " env=" + (m->plan_env.empty() ? std::string("none") : m->plan_env);
    if (len_out) *len_out = s.size();
    if (cap) {
        const size_t n = std::min(cap - 1, s.size());
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return GH_OK;
}

extern "C" int gh_model_config(gh_model* m, gh_config* out) {
    GH_LIVE(m, HK_MODEL);
    if (!m || !out) return set_error(GH_ERR_INVALID, "null argument");
    *out = m->cfg;
    return GH_OK;
}

// =====================================================================
// KV cache handle
// =====================================================================
extern "C" int gh_kv_create(gh_model* m, int32_t max_seq, gh_kv** out) {
    GH_LIVE(m, HK_MODEL);
    if (!m || !out) return set_error(GH_ERR_INVALID, "null argument");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    if (max_seq <= 0) max_seq = m->cfg.max_seq;
    const gh_config& c = m->cfg;
    // the kernels address one layer's K (or V) through a buffer view of at
    // most 2^31 - 1 bytes
    if ((uint64_t)max_seq * c.n_kv_heads * c.head_dim * 4 > 0x7fffffffull)
        return set_error(GH_ERR_RANGE, "max_seq %d: one layer's K cache would exceed 2 GiB", max_seq);
    std::unique_ptr<gh_kv> kv(new gh_kv);
    kv->m = m;
    kv->max_seq = max_seq;
    const size_t n = (size_t)c.n_layers * max_seq * c.n_kv_heads * c.head_dim;
    hipError_t e1 = hipMalloc((void**)&kv->k, n * 4);
    hipError_t e2 = hipMalloc((void**)&kv->v, n * 4);
    if (e1 != hipSuccess || e2 != hipSuccess)
        return set_error(GH_ERR_OOM, "KV cache of %zu bytes does not fit", 2 * n * 4);
    GH_HIP(hipMalloc((void**)&kv->st, sizeof(StepState)));
    {
        // (cos, sin) of pos * inv_freq for both layer types, positions [0, max_seq)
        const int half = c.head_dim / 2;
        std::vector<float> tab((size_t)2 * max_seq * half * 2);
        rope_table(m->inv_freq.data(), half, 0, max_seq, tab.data());
        rope_table(m->inv_freq.data() + half, half, 0, max_seq, tab.data() + (size_t)max_seq * half * 2);
        GH_HIP(hipMalloc((void**)&kv->rope, tab.size() * sizeof(float)));
        GH_HIP(hipMemcpy(kv->rope, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice));
    }
    GH_HIP(hipMalloc((void**)&kv->d_prompt, sizeof(int32_t) * max_seq));
    GH_HIP(hipMalloc((void**)&kv->d_ids, sizeof(int32_t) * max_seq));
    GH_HIP(hipHostMalloc((void**)&kv->h_st, sizeof(StepState), hipHostMallocDefault));
    std::memset(kv->h_st, 0, sizeof(StepState));
    GH_HIP(hipMemcpy(kv->st, kv->h_st, sizeof(StepState), hipMemcpyHostToDevice));
    m->kvs.push_back(kv.release());
    *out = m->kvs.back();
    handle_add(*out, HK_KV);
    return GH_OK;
}

gh_kv::~gh_kv() {
    if (graph_exec) hipGraphExecDestroy(graph_exec);
    if (graph) hipGraphDestroy(graph);
    for (void* p : {(void*)k, (void*)v, (void*)st, (void*)rope, (void*)d_prompt, (void*)d_ids, d_players})
        if (p) hipFree(p);
    if (h_st) hipHostFree(h_st);
}

extern "C" int gh_kv_destroy(gh_kv* kv) {
    if (!kv) return GH_OK;
    if (!handle_take(kv, HK_KV)) return dead_handle("gh_kv_destroy", HK_KV);
    gh_model* m = kv->m;
    gh_ctx* ctx = m->ctx;
    bool dead = false;
    {
        Lock lk(ctx->mu);
        hipSetDevice(ctx->device);
        hipStreamSynchronize(ctx->stream);
        m->kvs.erase(std::remove(m->kvs.begin(), m->kvs.end(), kv), m->kvs.end());
        delete kv;
        dead = model_collect_locked(m);
    }
    if (dead) ctx_free(ctx);
    return GH_OK;
}

extern "C" void gh_ctx_release(gh_ctx* ctx) { (void)gh_ctx_destroy(ctx); }
extern "C" void gh_model_release(gh_model* m) { (void)gh_model_destroy(m); }
extern "C" void gh_kv_release(gh_kv* kv) { (void)gh_kv_destroy(kv); }
extern "C" void gh_q4_0_release(gh_q4* t) { (void)gh_q4_0_free(t); }

// The cache's host fields are read and written under its context's mutex,
// so these calls are ordered with a step, generation or prefill running on
// the same cache from another thread.
extern "C" int gh_kv_reset(gh_kv* kv) {
    GH_LIVE(kv, HK_KV);
    Lock lk(kv->m->ctx->mu);
    kv->len = 0;
    return GH_OK;
}

extern "C" int gh_kv_length(gh_kv* kv, int32_t* len) {
    GH_LIVE(kv, HK_KV);
    if (!len) return set_error(GH_ERR_INVALID, "null argument");
    Lock lk(kv->m->ctx->mu);
    *len = kv->len;
    return GH_OK;
}

extern "C" int gh_kv_truncate(gh_kv* kv, int32_t n) {
    GH_LIVE(kv, HK_KV);
    Lock lk(kv->m->ctx->mu);
    if (n < 0 || n > kv->len) return set_error(GH_ERR_RANGE, "gh_kv_truncate: %d outside [0, %d]", n, kv->len);
    kv->len = n;
    return GH_OK;
}

extern "C" int gh_kv_set_sampling(gh_kv* kv, float temperature, uint64_t seed) {
    GH_LIVE(kv, HK_KV);
    if (!(temperature >= 0.0f) || std::isinf(temperature))
        return set_error(GH_ERR_INVALID, "temperature must be finite and >= 0");
    Lock lk(kv->m->ctx->mu);
    kv->inv_temp = temperature > 0.0f ? 1.0f / temperature : 0.0f;
    kv->seed = seed;
    return GH_OK;
}

extern "C" int gh_kv_set_top_k(gh_kv* kv, int32_t top_k) {
    GH_LIVE(kv, HK_KV);
    if (top_k < 0 || top_k > GH_TOP_K_MAX)
        return set_error(GH_ERR_RANGE, "top_k %d outside [0, %d]", top_k, GH_TOP_K_MAX);
    Lock lk(kv->m->ctx->mu);
    kv->top_k = top_k;
    return GH_OK;
}

extern "C" int gh_kv_synth(gh_kv* kv, uint64_t seed, int32_t n_pos, float sigma) {
    GH_LIVE(kv, HK_KV);
    if (!kv) return set_error(GH_ERR_INVALID, "null kv");
    if (n_pos < 0 || n_pos > kv->max_seq) return set_error(GH_ERR_RANGE, "n_pos %d outside [0, %d]", n_pos, kv->max_seq);
    gh_model* m = kv->m;
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    const gh_config& c = m->cfg;
    const int width = c.n_kv_heads * c.head_dim;
    const size_t per_layer = (size_t)kv->max_seq * width;
    const size_t n = (size_t)n_pos * width;
    // generated on the host (gh_synth_kv: the bytes a CPU checker can
    // regenerate), one layer at a time
    std::vector<float> hk(n), hv(n);
    GH_HIP(hipStreamSynchronize(m->ctx->stream));
    for (int l = 0; l < c.n_layers; ++l) {
        GH_CHECK(gh_synth_kv(seed, l, n_pos, width, sigma, hk.data(), hv.data()));
        GH_HIP(hipMemcpy(kv->k + l * per_layer, hk.data(), n * sizeof(float), hipMemcpyHostToDevice));
        GH_HIP(hipMemcpy(kv->v + l * per_layer, hv.data(), n * sizeof(float), hipMemcpyHostToDevice));
    }
    kv->len = n_pos;
    return GH_OK;
}

// =====================================================================
// step / generate / bench / profile
// =====================================================================
extern "C" int gh_step(gh_model* m, gh_kv* kv, int32_t token, float* logits, float* layer_out, int32_t* argmax_out) {
    GH_LIVE(m, HK_MODEL);
    GH_LIVE(kv, HK_KV);
    if (!m || !kv || kv->m != m) return set_error(GH_ERR_INVALID, "model / kv mismatch");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    GH_CHECK(model_ready(m));
    const gh_config& c = m->cfg;
    if (token < 0 || token >= c.vocab) return set_error(GH_ERR_INVALID, "token %d outside [0, %d)", token, c.vocab);
    if (kv->len >= kv->max_seq) return set_error(GH_ERR_RANGE, "KV cache full (%d positions)", kv->max_seq);
    hipStream_t s = m->ctx->stream;
    GH_CHECK(put_state(kv, kv->len, token, kv->len, 0, 0));
    GH_CHECK(launch_step(kv, kv->len));
    GH_CHECK(get_state(kv));
    if (logits) GH_HIP(hipMemcpyAsync(logits, m->logits, sizeof(float) * c.vocab, hipMemcpyDeviceToHost, s));
    if (layer_out)
        GH_HIP(hipMemcpyAsync(layer_out, m->layer_out, sizeof(float) * c.n_layers * c.hidden, hipMemcpyDeviceToHost, s));
    GH_HIP(hipStreamSynchronize(s));
    kv->len += 1;
    if (argmax_out) *argmax_out = kv->h_st->last;
    if (kv->h_st->xchg_err) return set_error(GH_ERR_STATE, "persistent step: a phase exchange timed out");
    if (kv->h_st->nan_flag) return set_error(GH_ERR_NAN, "NaN in logits at position %d", kv->len - 1);
    return GH_OK;
}

static int run_device_fed(gh_model* m, gh_kv* kv, const int32_t* prompt, int32_t n_prompt, int32_t n_before,
                          int32_t n_timed, int32_t gen_cap, float* ms_out, int32_t* ids_out) {
    const gh_config& c = m->cfg;
    if (!prompt || n_prompt <= 0) return set_error(GH_ERR_INVALID, "empty prompt");
    for (int i = 0; i < n_prompt; ++i)
        if (prompt[i] < 0 || prompt[i] >= c.vocab) return set_error(GH_ERR_INVALID, "prompt token %d out of range", prompt[i]);
    const long long steps = (long long)n_before + n_timed;
    if (kv->len + steps > kv->max_seq)
        return set_error(GH_ERR_RANGE, "generation needs %lld positions from %d; KV holds %d", steps, kv->len, kv->max_seq);
    hipStream_t s = m->ctx->stream;
    GH_HIP(hipMemcpyAsync(kv->d_prompt, prompt, sizeof(int32_t) * n_prompt, hipMemcpyHostToDevice, s));
    GH_CHECK(put_state(kv, kv->len, prompt[0], kv->len, n_prompt, gen_cap));
    const int pos0 = kv->len;
    for (int i = 0; i < n_before; ++i) GH_CHECK(launch_step(kv, pos0 + i));
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (ms_out) {
        GH_HIP(hipStreamSynchronize(s));
        GH_HIP(hipDeviceSynchronize());
        GH_HIP(hipEventCreate(&e0));
        GH_HIP(hipEventCreate(&e1));
        GH_HIP(hipEventRecord(e0, s));
    }
    for (int i = 0; i < n_timed; ++i) GH_CHECK(launch_step(kv, pos0 + n_before + i));
    if (ms_out) GH_HIP(hipEventRecord(e1, s));
    GH_CHECK(get_state(kv));
    GH_HIP(hipStreamSynchronize(s));
    if (ms_out) {
        GH_HIP(hipDeviceSynchronize());
        float ms = 0.0f;
        GH_HIP(hipEventElapsedTime(&ms, e0, e1));
        *ms_out = ms;
        hipEventDestroy(e0);
        hipEventDestroy(e1);
    }
    kv->len += (int)steps;
    const int got = kv->h_st->gen_count;
    if (ids_out && got > 0) GH_HIP(hipMemcpy(ids_out, kv->d_ids, sizeof(int32_t) * got, hipMemcpyDeviceToHost));
    if (kv->h_st->xchg_err) return set_error(GH_ERR_STATE, "persistent step: a phase exchange timed out");
    if (kv->h_st->nan_flag) return set_error(GH_ERR_NAN, "NaN in logits during generation");
    if (got != gen_cap) return set_error(GH_ERR_STATE, "generated %d ids, expected %d", got, gen_cap);
    return GH_OK;
}

extern "C" int gh_generate(gh_model* m, gh_kv* kv, const int32_t* prompt, int32_t n_prompt, int32_t n_gen,
                           int32_t* ids_out) {
    GH_LIVE(m, HK_MODEL);
    GH_LIVE(kv, HK_KV);
    if (!m || !kv || kv->m != m) return set_error(GH_ERR_INVALID, "model / kv mismatch");
    if (n_gen <= 0 || !ids_out) return set_error(GH_ERR_INVALID, "n_gen must be > 0 with an output buffer");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    GH_CHECK(model_ready(m));
    return run_device_fed(m, kv, prompt, n_prompt, n_prompt + n_gen - 1, 0, n_gen, nullptr, ids_out);
}

extern "C" int gh_bench_decode(gh_model* m, gh_kv* kv, const int32_t* prompt, int32_t n_prompt, int32_t n_warmup,
                               int32_t n_steps, float* ms_out, int32_t* ids_out) {
    GH_LIVE(m, HK_MODEL);
    GH_LIVE(kv, HK_KV);
    if (!m || !kv || kv->m != m || !ms_out) return set_error(GH_ERR_INVALID, "bad arguments");
    if (n_warmup < 0 || n_steps <= 0) return set_error(GH_ERR_INVALID, "bad step counts");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    GH_CHECK(model_ready(m));
    return run_device_fed(m, kv, prompt, n_prompt, n_prompt + n_warmup, n_steps, n_warmup + n_steps + 1, ms_out,
                          ids_out);
}

// Per-kernel-kind totals of a profiled run; releases the events.
int Profiler::reserve(size_t n_events) {
    pool.reserve(pool.size() + n_events);
    for (size_t i = 0; i < n_events; ++i) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) {
            release_pool();
            return set_error(GH_ERR_HIP, "hipEventCreate failed");
        }
        pool.push_back(e);
    }
    return GH_OK;
}

void Profiler::release_pool() {
    for (hipEvent_t e : pool) (void)hipEventDestroy(e);
    pool.clear();
}

static int collect_stats(Profiler& prof, gh_kernel_stat* stats, int32_t max_stats, int32_t* n_stats) {
    std::vector<double> tot(prof.names.size(), 0.0), bytes(prof.names.size(), 0.0);
    std::vector<int> cnt(prof.names.size(), 0);
    for (auto& r : prof.recs) {
        float ms = 0.0f;
        hipEventElapsedTime(&ms, r.a, r.b);
        tot[r.kind] += ms;
        bytes[r.kind] += r.bytes;
        cnt[r.kind] += 1;
        hipEventDestroy(r.a);
        hipEventDestroy(r.b);
    }
    prof.recs.clear();
    prof.release_pool();
    const int n = std::min<int>((int)prof.names.size(), max_stats);
    for (int i = 0; i < n; ++i) {
        std::memset(&stats[i], 0, sizeof(gh_kernel_stat));
        std::snprintf(stats[i].name, sizeof(stats[i].name), "%s", prof.names[i].c_str());
        stats[i].launches = cnt[i];
        stats[i].total_ms = tot[i];
        stats[i].bytes = cnt[i] ? bytes[i] / cnt[i] : 0.0;
    }
    *n_stats = n;
    return GH_OK;
}

// Batched prefill of n tokens at the cache's next positions, in passes of
// up to PF_MAX_TOKENS; the last token's logits, layer outputs and next token
// are those of gh_step at that position.
static int prefill_run(gh_model* m, gh_kv* kv, const int32_t* tokens, int32_t n, float* logits, float* layer_out,
                       int32_t* next_out, Profiler* prof = nullptr) {
    const gh_config& c = m->cfg;
    if (!tokens || n <= 0) return set_error(GH_ERR_INVALID, "prefill: empty token list");
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= c.vocab)
            return set_error(GH_ERR_INVALID, "prefill: token %d outside [0, %d)", tokens[i], c.vocab);
    if ((long long)kv->len + n > kv->max_seq)
        return set_error(GH_ERR_RANGE, "prefill of %d tokens from position %d; KV holds %d", n, kv->len, kv->max_seq);
    hipStream_t s = m->ctx->stream;
    GH_CHECK(prefill_reserve(m, std::min(n, PF_MAX_TOKENS)));
    GH_CHECK(put_state(kv, kv->len + n - 1, tokens[n - 1], kv->len, 0, 0));
    Sink sink;
    sink.s = s;
    sink.prof = prof;
    for (int done = 0; done < n;) {
        const int k = std::min(PF_MAX_TOKENS, n - done);
        GH_HIP(hipMemcpyAsync(m->pf.tok, tokens + done, sizeof(int32_t) * k, hipMemcpyHostToDevice, s));
        GH_CHECK(enqueue_prefill(m, kv, sink, k, kv->len + done, done + k == n));
        done += k;
    }
    GH_CHECK(get_state(kv));
    if (logits) GH_HIP(hipMemcpyAsync(logits, m->logits, sizeof(float) * c.vocab, hipMemcpyDeviceToHost, s));
    if (layer_out)
        GH_HIP(hipMemcpyAsync(layer_out, m->layer_out, sizeof(float) * c.n_layers * c.hidden, hipMemcpyDeviceToHost, s));
    GH_HIP(hipStreamSynchronize(s));
    kv->len += n;
    if (next_out) *next_out = kv->h_st->last;
    if (kv->h_st->nan_flag) return set_error(GH_ERR_NAN, "NaN in logits at position %d", kv->len - 1);
    return GH_OK;
}

extern "C" int gh_prefill(gh_model* m, gh_kv* kv, const int32_t* tokens, int32_t n, float* logits, float* layer_out,
                          int32_t* next_out) {
    GH_LIVE(m, HK_MODEL);
    GH_LIVE(kv, HK_KV);
    if (!m || !kv || kv->m != m) return set_error(GH_ERR_INVALID, "model / kv mismatch");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    GH_CHECK(model_ready(m));
    return prefill_run(m, kv, tokens, n, logits, layer_out, next_out);
}

extern "C" int gh_generate_prefill(gh_model* m, gh_kv* kv, const int32_t* prompt, int32_t n_prompt, int32_t n_gen,
                                   int32_t* ids_out) {
    GH_LIVE(m, HK_MODEL);
    GH_LIVE(kv, HK_KV);
    if (!m || !kv || kv->m != m) return set_error(GH_ERR_INVALID, "model / kv mismatch");
    if (n_gen <= 0 || !ids_out) return set_error(GH_ERR_INVALID, "n_gen must be > 0 with an output buffer");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    GH_CHECK(model_ready(m));
    if (prompt && n_prompt > 0 && (long long)kv->len + n_prompt + n_gen - 1 > kv->max_seq)
        return set_error(GH_ERR_RANGE, "generation needs %d positions from %d; KV holds %d", n_prompt + n_gen - 1,
                         kv->len, kv->max_seq);
    int32_t next = 0;
    GH_CHECK(prefill_run(m, kv, prompt, n_prompt, nullptr, nullptr, &next));
    ids_out[0] = next;
    if (n_gen == 1) return GH_OK;
    return run_device_fed(m, kv, &next, 1, n_gen - 1, 0, n_gen - 1, nullptr, ids_out + 1);
}

extern "C" int gh_profile_steps(gh_model* m, gh_kv* kv, int32_t n_steps, gh_kernel_stat* stats, int32_t max_stats,
                                int32_t* n_stats) {
    GH_LIVE(m, HK_MODEL);
    GH_LIVE(kv, HK_KV);
    if (!m || !kv || kv->m != m || !stats || !n_stats || n_steps <= 0)
        return set_error(GH_ERR_INVALID, "bad arguments");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    GH_CHECK(model_ready(m));
    if (kv->len + n_steps > kv->max_seq) return set_error(GH_ERR_RANGE, "KV cache full");
    hipStream_t s = m->ctx->stream;
    int tok = kv->h_st->last >= 0 && kv->h_st->last < m->cfg.vocab ? kv->h_st->last : 0;
    GH_CHECK(put_state(kv, kv->len, tok, kv->len, 0, 0));
    Profiler prof;
    // two events per launch of the graph step (5 per layer + final norm, LM
    // head, finish; the persistent step launches fewer)
    GH_CHECK(prof.reserve(2 * (size_t)n_steps * (5 * (size_t)m->cfg.n_layers + 3)));
    Sink sink;
    sink.s = s;
    sink.prof = &prof;
    int rc = GH_OK;
    for (int i = 0; i < n_steps && rc == GH_OK; ++i) {
        rc = enqueue_step(m, kv, sink, kv->len);
        kv->len += 1;
    }
    GH_CHECK(get_state(kv));
    GH_HIP(hipStreamSynchronize(s));
    const int rc2 = collect_stats(prof, stats, max_stats, n_stats);
    return rc != GH_OK ? rc : rc2;
}

extern "C" int gh_prefill_profile(gh_model* m, gh_kv* kv, const int32_t* tokens, int32_t n, gh_kernel_stat* stats,
                                  int32_t max_stats, int32_t* n_stats) {
    GH_LIVE(m, HK_MODEL);
    GH_LIVE(kv, HK_KV);
    if (!m || !kv || kv->m != m || !stats || !n_stats) return set_error(GH_ERR_INVALID, "bad arguments");
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    GH_CHECK(model_ready(m));
    Profiler prof;
    const int rc = prefill_run(m, kv, tokens, n, nullptr, nullptr, nullptr, &prof);
    GH_HIP(hipStreamSynchronize(m->ctx->stream));
    const int rc2 = collect_stats(prof, stats, max_stats, n_stats);
    return rc != GH_OK ? rc : rc2;
}

extern "C" int gh_time_kernel(gh_model* m, gh_kv* kv, const char* name, int32_t n_reps, double* avg_us_out,
                              double* bytes_per_launch_out, int32_t* launches_per_step_out) {
    GH_LIVE(m, HK_MODEL);
    GH_LIVE(kv, HK_KV);
    if (!m || !kv || kv->m != m || !name || n_reps <= 0 || !avg_us_out)
        return set_error(GH_ERR_INVALID, "bad arguments");
    static const char* kinds[] = {"qkv", "attention", "o_proj", "gate_up", "down", "final_norm", "lm_head"};
    bool known = false;
    for (const char* k : kinds) known = known || std::strcmp(k, name) == 0;
    if (!known) return set_error(GH_ERR_INVALID, "gh_time_kernel: unknown or non-idempotent kernel '%s'", name);
    GH_CHECK(dev_bind(m->ctx));
    Lock lk(m->ctx->mu);
    GH_CHECK(model_ready(m));
    if (kv->len >= kv->max_seq) return set_error(GH_ERR_RANGE, "KV cache full");
    hipStream_t s = m->ctx->stream;
    gh::Sink sink;
    sink.s = s;
    sink.only = name;
    GH_CHECK(enqueue_step(m, kv, sink, kv->len));  // warm-up
    const int per_step = sink.launched;
    const double bytes = per_step ? sink.bytes / per_step : 0.0;
    // Graph mode (default): the n_reps passes are built into one graph and
    // replayed once, so the launches run back to back as the decode graph
    // runs them, with no host work between them.  GH_NO_GRAPH=1: eager
    // launches, one host pass of the step per repetition.
    const bool use_graph = !env_int("GH_NO_GRAPH", 0);
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    std::vector<std::unique_ptr<gh::NodeArgsBase>> store;
    std::vector<gh::PosPatch> patches;
    hipEvent_t a = nullptr, b = nullptr;
    int rc = GH_OK;
    if (use_graph) {
        if (hipGraphCreate(&g, 0) != hipSuccess) return set_error(GH_ERR_HIP, "hipGraphCreate failed");
        gh::Sink gs;
        gs.g = g;
        gs.only = name;
        gs.store = &store;
        gs.patches = &patches;
        for (int i = 0; i < n_reps && rc == GH_OK; ++i) rc = enqueue_step(m, kv, gs, kv->len);
        if (rc == GH_OK && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess)
            rc = set_error(GH_ERR_HIP, "hipGraphInstantiate failed");
        if (rc == GH_OK && hipGraphLaunch(ge, s) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipGraphLaunch failed");
    }
    if (rc == GH_OK && (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess))
        rc = set_error(GH_ERR_HIP, "hipEventCreate failed");
    if (rc == GH_OK && hipEventRecord(a, s) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventRecord failed");
    if (use_graph) {
        if (rc == GH_OK && hipGraphLaunch(ge, s) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipGraphLaunch failed");
    } else {
        for (int i = 0; i < n_reps && rc == GH_OK; ++i) rc = enqueue_step(m, kv, sink, kv->len);
    }
    float ms = 0.0f;
    if (rc == GH_OK && hipEventRecord(b, s) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventRecord failed");
    if (rc == GH_OK && hipEventSynchronize(b) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventSynchronize failed");
    if (rc == GH_OK && hipEventElapsedTime(&ms, a, b) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventElapsedTime failed");
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (ge) (void)hipGraphExecDestroy(ge);
    if (g) (void)hipGraphDestroy(g);
    GH_CHECK(rc);
    *avg_us_out = per_step ? 1e3 * ms / ((double)n_reps * per_step) : 0.0;
    if (bytes_per_launch_out) *bytes_per_launch_out = bytes;
    if (launches_per_step_out) *launches_per_step_out = per_step;
    return GH_OK;
}

extern "C" int gh_time_stream_read(gh_ctx* ctx, size_t bytes, int32_t n_reps, double* avg_us_out) {
    if (!ctx || bytes < 16 || bytes % 16 || bytes > (1u << 31) - 16u || n_reps <= 0 || !avg_us_out)
        return set_error(GH_ERR_INVALID, "gh_time_stream_read: bytes must be a multiple of 16 in [16, 2 GiB)");
    GH_CHECK(ctx_bind(ctx));
    Lock lk(ctx->mu);
    hipStream_t s = ctx->stream;
    void* buf = nullptr;
    float* sink = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    float ms = 0.0f;
    int rc = GH_OK;
    if (hipMalloc(&buf, bytes) != hipSuccess || hipMalloc((void**)&sink, 4096 * sizeof(float)) != hipSuccess)
        rc = set_error(GH_ERR_OOM, "gh_time_stream_read: hipMalloc of %zu bytes failed", bytes);
    // zeros: the kernel's guarded store never fires
    if (rc == GH_OK && hipMemsetAsync(buf, 0, bytes, s) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipMemsetAsync failed");
    if (rc == GH_OK) rc = gh::launch_stream_read(buf, bytes, sink, s);  // warm-up
    if (rc == GH_OK && (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess))
        rc = set_error(GH_ERR_HIP, "hipEventCreate failed");
    if (rc == GH_OK && hipEventRecord(a, s) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventRecord failed");
    for (int i = 0; i < n_reps && rc == GH_OK; ++i) rc = gh::launch_stream_read(buf, bytes, sink, s);
    if (rc == GH_OK && hipEventRecord(b, s) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventRecord failed");
    if (rc == GH_OK && hipEventSynchronize(b) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventSynchronize failed");
    if (rc == GH_OK && hipEventElapsedTime(&ms, a, b) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipEventElapsedTime failed");
    (void)hipStreamSynchronize(s);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (sink) (void)hipFree(sink);
    if (buf) (void)hipFree(buf);
    GH_CHECK(rc);
    *avg_us_out = 1e3 * ms / n_reps;
    return GH_OK;
}

extern "C" int gh_time_exchange(gh_ctx* ctx, int32_t n_wg, int32_t rounds, double* us_out) {
    if (!ctx || !us_out || rounds < 1 || rounds > 1000000)
        return set_error(GH_ERR_INVALID, "gh_time_exchange: rounds must be in [1, 1000000]");
    GH_CHECK(ctx_bind(ctx));
    int cus = 0;
    GH_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device));
    if (n_wg < 1 || n_wg > 256 || n_wg > cus)
        return set_error(GH_ERR_RANGE, "gh_time_exchange: %d workgroups (1 .. min(256, %d CUs))", n_wg, cus);
    Lock lk(ctx->mu);
    hipStream_t s = ctx->stream;
    void* dev = nullptr;
    const size_t words = 2 * sizeof(uint64_t) * (size_t)n_wg;
    const size_t bytes = words + 64 + 2 * sizeof(unsigned long long);
    int rc = GH_OK;
    if (hipMalloc(&dev, bytes) != hipSuccess) rc = set_error(GH_ERR_OOM, "gh_time_exchange: hipMalloc failed");
    // zeros: epoch 0 is never a round's
    if (rc == GH_OK && hipMemsetAsync(dev, 0, bytes, s) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipMemsetAsync failed");
    uint64_t* w = (uint64_t*)dev;
    int* err = (int*)((char*)dev + words);
    unsigned long long* stamps = (unsigned long long*)((char*)dev + words + 64);
    if (rc == GH_OK) rc = gh::launch_xchg_probe(w, n_wg, rounds, err, stamps, s);
    int herr = 0;
    unsigned long long hs[2] = {0, 0};
    if (rc == GH_OK && hipMemcpyAsync(&herr, err, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess)
        rc = set_error(GH_ERR_HIP, "hipMemcpyAsync failed");
    if (rc == GH_OK && hipMemcpyAsync(hs, stamps, sizeof(hs), hipMemcpyDeviceToHost, s) != hipSuccess)
        rc = set_error(GH_ERR_HIP, "hipMemcpyAsync failed");
    if (rc == GH_OK && hipStreamSynchronize(s) != hipSuccess) rc = set_error(GH_ERR_HIP, "hipStreamSynchronize failed");
    (void)hipStreamSynchronize(s);
    if (dev) (void)hipFree(dev);
    GH_CHECK(rc);
    if (herr) return set_error(GH_ERR_STATE, "gh_time_exchange: a wait timed out (workgroups not co-resident?)");
    *us_out = (double)(hs[1] - hs[0]) * 0.01 / rounds;  // s_memrealtime ticks at 100 MHz
    return GH_OK;
}

// =====================================================================
// synthetic model
// =====================================================================
extern "C" int gh_synth_model(gh_model* m, uint64_t seed, int q4, float w_sigma, float scale_sigma, float norm_sigma) {
    GH_LIVE(m, HK_MODEL);
    if (!m) return set_error(GH_ERR_INVALID, "null model");
    const gh_config& c = m->cfg;
    const int H = c.hidden, hd = c.head_dim, F = c.ffn;
    auto mat = [&](const std::string& name, int rows, int cols) -> int {
        if (q4) {
            std::vector<uint8_t> raw((size_t)rows * (cols / 32) * 18);
            GH_CHECK(gh_synth_q4_0(seed, name.c_str(), scale_sigma, rows, cols, raw.data()));
            return gh_model_set_tensor(m, name.c_str(), GH_DTYPE_Q4_0, raw.data(), raw.size());
        }
        std::vector<float> w((size_t)rows * cols);
        GH_CHECK(gh_synth_f32(seed, name.c_str(), w_sigma, w.data(), w.size()));
        return gh_model_set_tensor(m, name.c_str(), GH_DTYPE_F32, w.data(), w.size() * 4);
    };
    auto vec = [&](const std::string& name, int n) -> int {
        std::vector<float> w(n);
        GH_CHECK(gh_synth_f32(seed, name.c_str(), norm_sigma, w.data(), n));
        return gh_model_set_tensor(m, name.c_str(), GH_DTYPE_F32, w.data(), w.size() * 4);
    };
    GH_CHECK(mat("token_embd.weight", c.vocab, H));
    GH_CHECK(vec("output_norm.weight", H));
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        GH_CHECK(vec(p + "attn_norm.weight", H));
        GH_CHECK(mat(p + "attn_q.weight", c.n_heads * hd, H));
        GH_CHECK(mat(p + "attn_k.weight", c.n_kv_heads * hd, H));
        GH_CHECK(mat(p + "attn_v.weight", c.n_kv_heads * hd, H));
        GH_CHECK(vec(p + "attn_q_norm.weight", hd));
        GH_CHECK(vec(p + "attn_k_norm.weight", hd));
        GH_CHECK(mat(p + "attn_output.weight", H, c.n_heads * hd));
        GH_CHECK(vec(p + "post_attention_norm.weight", H));
        GH_CHECK(vec(p + "ffn_norm.weight", H));
        GH_CHECK(mat(p + "ffn_gate.weight", F, H));
        GH_CHECK(mat(p + "ffn_up.weight", F, H));
        GH_CHECK(mat(p + "ffn_down.weight", H, F));
        GH_CHECK(vec(p + "post_ffw_norm.weight", H));
    }
    return GH_OK;
}
