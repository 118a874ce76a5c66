// gfx950 kernels of the batch-1 decode step and the op-level entry points.
//
// Every matvec-shaped kernel follows one pattern (k_matvec):
//   1. each wave issues the loads of its weight blocks into registers
//      (two rows per lane: lane and lane+64 of a 128-row tile; one 1 KB
//      contiguous wave load per row and column block),
//   2. the prologue builds the input-vector slice the workgroup needs in LDS
//      (residual + RMSNorm, attention combine, GeGLU, ...) while those loads
//      are in flight,
//   3. dequant-dot: nibbles -> f32 via byte conversions, x broadcast from
//      LDS, f32 accumulation, scale applied once per 32-weight block,
//   4. the four waves' row partials are summed in LDS and the epilogue
//      writes a split partial (summed by the next kernel's prologue) or the
//      logits plus a grid-wide argmax key.
// No MFMA: batch-1 decode is HBM-bound (3.5 flop/byte for Q4_0).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>

#include "common.h"

namespace gh {

constexpr int NT = 256;  // threads per workgroup (4 wave64)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------
// reductions
// ------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over the 256 threads; `red` holds 4 floats of LDS.  Every thread gets
// the result.  Contains two barriers; call from uniform control flow.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int o) {
    unsigned lo = (unsigned)v, hi = (unsigned)(v >> 32);
    lo = __shfl_xor(lo, o, 64);
    hi = __shfl_xor(hi, o, 64);
    return ((unsigned long long)hi << 32) | lo;
}

// Order-preserving argmax key: larger value wins, then lower index.
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    unsigned b = __float_as_uint(v);
    unsigned ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned)(0xFFFFFFFFu - (unsigned)idx);
}

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// GELU(tanh) with the +-10 clamp of src/Gemma/Layers/MLP.hs:384-447.
__device__ __forceinline__ float gelu_tanh(float x) {
    float x3 = x * x * x;
    float t = 0.7978845608f * (x + 0.044715f * x3);
    t = fminf(fmaxf(t, -10.0f), 10.0f);
    return x * 0.5f * (1.0f + tanhf(t));
}

// Element (r, c) of a tiled matrix, dequantised exactly: (q - 8) * d.
__device__ __forceinline__ float dq_elem(const DMat& w, int r, int c) {
    const int t = r >> 7, lr = r & 127;
    if (w.fmt == FMT_Q4) {
        const int b = c >> 5, e = c & 31;
        const size_t idx = ((size_t)t * w.nblk + b) * TILE_ROWS + lr;
        const uint8_t byte = ((const uint8_t*)w.codes)[idx * 16 + (e & 15)];
        const int q = (e < 16) ? (byte & 15) : (byte >> 4);
        return ((float)q - 8.0f) * h2f(w.scales[idx]);
    }
    const size_t idx = ((size_t)t * w.nblk + (c >> 2)) * TILE_ROWS + lr;
    return ((const float*)w.codes)[idx * 4 + (c & 3)];
}

// RMS of a vector held in LDS (or any memory), block-wide; zero-centred
// norm weight gives (x / rms) * (1 + w) as the reference's shaders do.
__device__ __forceinline__ float block_rms(const float* v, int n, float eps, float* red) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += NT) ss += v[i] * v[i];
    ss = block_sum(ss, red);
    return sqrtf(ss / (float)n + eps);
}

__device__ __forceinline__ float norm_apply(float x, float rms, float w, int zc) {
    return zc ? (x / rms) * (1.0f + w) : (x / rms) * w;
}

// ------------------------------------------------------------------
// matvec core
// ------------------------------------------------------------------
template <int FMT>
struct Blk;
template <>
struct Blk<FMT_Q4> {
    static constexpr int BK = 32;
};
template <>
struct Blk<FMT_F32> {
    static constexpr int BK = 4;
};

template <int FMT, int KBW>
struct WRegs {
    u32x4 c0[KBW], c1[KBW];
    uint16_t s0[KBW], s1[KBW];
};

template <int FMT, int KBW>
__device__ __forceinline__ void mv_load(WRegs<FMT, KBW>& r, const DMat& w, int tile, int base,
                                        int kw1) {
    const int lane = threadIdx.x & 63;
    const u32x4* cp = (const u32x4*)w.codes + (size_t)tile * w.nblk * TILE_ROWS;
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
        const int kb = base + i;
        if (kb < kw1) {
            r.c0[i] = __builtin_nontemporal_load(cp + (size_t)kb * TILE_ROWS + lane);
            r.c1[i] = __builtin_nontemporal_load(cp + (size_t)kb * TILE_ROWS + 64 + lane);
            if (FMT == FMT_Q4) {
                const uint16_t* sp = w.scales + (size_t)tile * w.nblk * TILE_ROWS;
                r.s0[i] = __builtin_nontemporal_load(sp + (size_t)kb * TILE_ROWS + lane);
                r.s1[i] = __builtin_nontemporal_load(sp + (size_t)kb * TILE_ROWS + 64 + lane);
            }
        }
    }
}

__device__ __forceinline__ float dot_q4_word(uint32_t w, float4 xl, float4 xh) {
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    float d = (float)(lo & 0xFF) * xl.x;
    d += (float)((lo >> 8) & 0xFF) * xl.y;
    d += (float)((lo >> 16) & 0xFF) * xl.z;
    d += (float)(lo >> 24) * xl.w;
    d += (float)(hi & 0xFF) * xh.x;
    d += (float)((hi >> 8) & 0xFF) * xh.y;
    d += (float)((hi >> 16) & 0xFF) * xh.z;
    d += (float)(hi >> 24) * xh.w;
    return d;
}

// Accumulate the dot products of one register batch.  xs/sxs index the
// LDS slice starting at column block kb0.
template <int FMT, int KBW>
__device__ __forceinline__ void mv_compute(const WRegs<FMT, KBW>& r, int base, int kw1, int kb0,
                                           const float* xs, const float* sxs, float& acc0,
                                           float& acc1) {
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
        const int kb = base + i;
        if (kb < kw1) {
            if (FMT == FMT_Q4) {
                const float4* xv = (const float4*)(xs + (kb - kb0) * 32);
                // element e<16 <- low nibble of byte e, e>=16 <- high nibble of byte e-16
                float d0 = 0.0f, d1 = 0.0f;
                const uint32_t w0[4] = {r.c0[i].x, r.c0[i].y, r.c0[i].z, r.c0[i].w};
                const uint32_t w1[4] = {r.c1[i].x, r.c1[i].y, r.c1[i].z, r.c1[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 xl = xv[j], xh = xv[4 + j];
                    d0 += dot_q4_word(w0[j], xl, xh);
                    d1 += dot_q4_word(w1[j], xl, xh);
                }
                // sum (q-8) x = sum q x - 8 sum x ; sxs holds sum x per block
                const float sx8 = 8.0f * sxs[kb - kb0];
                acc0 += h2f(r.s0[i]) * (d0 - sx8);
                acc1 += h2f(r.s1[i]) * (d1 - sx8);
            } else {
                const float4 x = *(const float4*)(xs + (kb - kb0) * 4);
                const f32x4 a = __builtin_bit_cast(f32x4, r.c0[i]);
                const f32x4 b = __builtin_bit_cast(f32x4, r.c1[i]);
                acc0 += a.x * x.x + a.y * x.y + a.z * x.z + a.w * x.w;
                acc1 += b.x * x.x + b.y * x.y + b.z * x.z + b.w * x.w;
            }
        }
    }
}

// LDS layout of k_matvec (floats):
//   red [512] | misc [64] | xs [per_split*BK] | sxs [per_split] | tmp [...]
struct MvLds {
    float* red;
    float* misc;
    float* xs;
    float* sxs;
    float* tmp;
};

inline size_t mv_lds_bytes(int fmt, int per_split, int tmp_floats) {
    const int bk = block_cols(fmt);
    size_t f = 512 + 64 + (size_t)per_split * bk + (((size_t)per_split + 3) & ~(size_t)3) + tmp_floats;
    return f * sizeof(float);
}

// Sum of x over each 32-element block of the slice (Q4_0 only).
template <int FMT>
__device__ __forceinline__ void fill_block_sums(const MvLds& L, int nk) {
    if (FMT == FMT_Q4) {
        __syncthreads();
        for (int b = threadIdx.x; b < nk; b += NT) {
            const float* x = L.xs + b * 32;
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 32; ++e) s += x[e];
            L.sxs[b] = s;
        }
    }
}

template <int FMT, int KBW, class Pro, class Epi>
__global__ __launch_bounds__(NT) void k_matvec(DMat w, int S, Pro pro, Epi epi) {
    extern __shared__ float lds[];
    constexpr int BK = Blk<FMT>::BK;
    const int tile = blockIdx.x / S, s = blockIdx.x % S;
    const int nb = w.nblk;
    const int per_split = (nb + S - 1) / S;
    const int kb0 = min(nb, s * per_split), kb1 = min(nb, kb0 + per_split);
    const int nk = kb1 - kb0;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int per_wave = (nk + 3) >> 2;
    const int kw0 = min(kb1, kb0 + wave * per_wave), kw1 = min(kb1, kw0 + per_wave);

    MvLds L;
    L.red = lds;
    L.misc = lds + 512;
    L.xs = lds + 576;
    L.sxs = L.xs + per_split * BK;
    L.tmp = L.sxs + ((per_split + 3) & ~3);

    // 1. weights of the first batch in flight
    WRegs<FMT, KBW> r;
    mv_load<FMT, KBW>(r, w, tile, kw0, kw1);
    // 2. input slice [kb0*BK, kb1*BK) into LDS
    pro(L, kb0 * BK, nk * BK);
    fill_block_sums<FMT>(L, nk);
    __syncthreads();
    // 3. dot products
    float acc0 = 0.0f, acc1 = 0.0f;
    mv_compute<FMT, KBW>(r, kw0, kw1, kb0, L.xs, L.sxs, acc0, acc1);
    for (int base = kw0 + KBW; base < kw1; base += KBW) {
        mv_load<FMT, KBW>(r, w, tile, base, kw1);
        mv_compute<FMT, KBW>(r, base, kw1, kb0, L.xs, L.sxs, acc0, acc1);
    }
    // 4. reduce the four waves
    L.red[wave * TILE_ROWS + lane] = acc0;
    L.red[wave * TILE_ROWS + 64 + lane] = acc1;
    __syncthreads();
    float y = 0.0f;
    const int t = threadIdx.x;
    if (t < TILE_ROWS) y = (L.red[t] + L.red[TILE_ROWS + t]) + (L.red[2 * TILE_ROWS + t] + L.red[3 * TILE_ROWS + t]);
    epi(L, tile, s, t, y);
}

// ------------------------------------------------------------------
// prologues: build xs[0 .. n) = input[c0 .. c0+n)
// ------------------------------------------------------------------
struct ProPlain {
    const float* x;
    __device__ void operator()(const MvLds& L, int c0, int n) const {
        for (int i = threadIdx.x; i < n; i += NT) L.xs[i] = x[c0 + i];
    }
};

// Residual stream entering a layer (or the final norm) followed by RMSNorm:
//   layer 0 : x = E[token] * sqrt(H)  (src/Gemma/Model.hs:1346-1361)
//   else    : x = x1 + postnorm(sum_s d_s)  (TBG:413-444)
//   xs      = norm(x) with w_norm  (TBG:110, or the final norm RMSNorm.hs:343-386)
// Block 0 stores x (the residual input of this layer) and, when asked, the
// hidden state after the previous layer.
struct ProResidNorm {
    int from_embedding;
    DMat embd;
    const StepState* st;
    float escale;
    const float* x1;
    const float* part_d;
    int Sd, ld_d;
    const float* w_post;  // nullable
    const float* w_norm;
    float eps;
    int zc, H;
    float* x_res;          // nullable
    float* layer_out_row;  // nullable
    __device__ void operator()(const MvLds& L, int c0, int n) const {
        float* x = L.tmp;
        if (from_embedding) {
            // the host validates tokens; the clamp keeps a corrupted state in bounds
            const int tok = min(max(st->token, 0), embd.rows - 1);
            for (int i = threadIdx.x; i < H; i += NT) x[i] = dq_elem(embd, tok, i) * escale;
        } else {
            for (int i = threadIdx.x; i < H; i += NT) {
                float a = 0.0f;
                for (int s = 0; s < Sd; ++s) a += part_d[(size_t)s * ld_d + i];
                x[i] = a;
            }
            if (w_post) {
                const float rms = block_rms(x, H, eps, L.misc);
                for (int i = threadIdx.x; i < H; i += NT) x[i] = x1[i] + norm_apply(x[i], rms, w_post[i], zc);
            } else {
                for (int i = threadIdx.x; i < H; i += NT) x[i] = x1[i] + x[i];
            }
        }
        if (blockIdx.x == 0) {
            for (int i = threadIdx.x; i < H; i += NT) {
                if (x_res) x_res[i] = x[i];
                if (layer_out_row) layer_out_row[i] = x[i];
            }
        }
        const float rms = block_rms(x, H, eps, L.misc);  // has barriers: x complete
        for (int i = threadIdx.x; i < n; i += NT) L.xs[i] = norm_apply(x[c0 + i], rms, w_norm[c0 + i], zc);
    }
};

// Attention window of the current token (see k_attn).
__device__ __forceinline__ void attn_window(int pos, int global, int window, int mode, int& pb, int& pe) {
    pb = 0;
    pe = pos + 1;
    if (window > 0) {
        if (mode == GH_MODE_REF) {
            if (pe > window) pe = window;  // quirk Q3: first min(len, W) positions
        } else if (!global) {
            if (pe > window) pb = pe - window;  // last W positions
        }
    }
}

__device__ __forceinline__ void attn_chunks(int n_pos, int nc, int& ch, int& n_used) {
    ch = (n_pos + nc - 1) / nc;
    n_used = (n_pos + ch - 1) / ch;
}

// Merge the split-K attention partials {m[G], l[G], o[G][HD]} of kv group g.
__device__ __forceinline__ float attn_merge(const float* part, int nc, int n_used, int G, int HD,
                                            int g, int hl, int d) {
    const int stride = G * (HD + 2);
    const float* base = part + (size_t)g * nc * stride;
    float M = -INFINITY;
    for (int j = 0; j < n_used; ++j) M = fmaxf(M, base[(size_t)j * stride + hl]);
    float den = 0.0f, num = 0.0f;
    for (int j = 0; j < n_used; ++j) {
        const float* p = base + (size_t)j * stride;
        const float wgt = expf(p[hl] - M);
        den += p[G + hl] * wgt;
        num += p[2 * G + hl * HD + d] * wgt;
    }
    return num / den;
}

// O-projection input: the merged attention output of the slice.
struct ProAttnCombine {
    const float* part;
    const StepState* st;
    int nc, G, HD;
    int global, window, mode;
    __device__ void operator()(const MvLds& L, int c0, int n) const {
        int pb, pe, ch, n_used;
        attn_window(st->pos, global, window, mode, pb, pe);
        attn_chunks(pe - pb, nc, ch, n_used);
        for (int i = threadIdx.x; i < n; i += NT) {
            const int c = c0 + i;
            const int h = c / HD, d = c % HD;
            L.xs[i] = attn_merge(part, nc, n_used, G, HD, h / G, h % G, d);
        }
    }
};

// Gate/up input: x1 = x + postnorm(sum_s o_s) (TBG:305-343), then the
// pre-FFN norm (MLP.hs:507-622).  Block 0 stores x1.
struct ProPostAttn {
    const float* part_o;
    int So, ld_o;
    const float* w_post;  // nullable
    const float* x_res;
    float* x1_out;
    const float* w_ffn;
    float eps;
    int zc, H;
    __device__ void operator()(const MvLds& L, int c0, int n) const {
        float* x = L.tmp;
        for (int i = threadIdx.x; i < H; i += NT) {
            float a = 0.0f;
            for (int s = 0; s < So; ++s) a += part_o[(size_t)s * ld_o + i];
            x[i] = a;
        }
        if (w_post) {
            const float rms = block_rms(x, H, eps, L.misc);
            for (int i = threadIdx.x; i < H; i += NT) x[i] = x_res[i] + norm_apply(x[i], rms, w_post[i], zc);
        } else {
            for (int i = threadIdx.x; i < H; i += NT) x[i] = x_res[i] + x[i];
        }
        if (blockIdx.x == 0)
            for (int i = threadIdx.x; i < H; i += NT) x1_out[i] = x[i];
        const float rms = block_rms(x, H, eps, L.misc);
        for (int i = threadIdx.x; i < n; i += NT) L.xs[i] = norm_apply(x[c0 + i], rms, w_ffn[c0 + i], zc);
    }
};

// Down-projection input: h = gelu_tanh(sum_s g_s) * sum_s u_s (MLP.hs:384-447).
struct ProGeglu {
    const float* part_gu;
    int Sg, ld_g, up_off;
    __device__ void operator()(const MvLds& L, int c0, int n) const {
        for (int i = threadIdx.x; i < n; i += NT) {
            const int c = c0 + i;
            float g = 0.0f, u = 0.0f;
            for (int s = 0; s < Sg; ++s) {
                g += part_gu[(size_t)s * ld_g + c];
                u += part_gu[(size_t)s * ld_g + up_off + c];
            }
            L.xs[i] = gelu_tanh(g) * u;
        }
    }
};

// ------------------------------------------------------------------
// epilogues (called by all threads; t < 128 hold row sums)
// ------------------------------------------------------------------
struct EpiPartial {
    float* part;
    int ld;
    __device__ void operator()(const MvLds&, int tile, int s, int t, float y) const {
        if (t < TILE_ROWS) part[(size_t)s * ld + tile * TILE_ROWS + t] = y;
    }
};

struct EpiOut {
    float* y;
    int rows, softcap;
    float cap;
    __device__ void operator()(const MvLds&, int tile, int, int t, float v) const {
        const int row = tile * TILE_ROWS + t;
        if (t < TILE_ROWS && row < rows) y[row] = softcap ? cap * tanhf(v / cap) : v;
    }
};

// Logits + grid-wide greedy argmax (first maximum) into st->keys[pos & 1].
struct EpiLogits {
    float* logits;  // nullable
    int V;
    StepState* st;
    __device__ void operator()(const MvLds& L, int tile, int, int t, float y) const {
        const int row = tile * TILE_ROWS + t;
        unsigned long long key = 0ull;
        if (t < TILE_ROWS && row < V) {
            if (logits) logits[row] = y;
            key = argmax_key(y, row);
            if (isnan(y)) atomicOr(&st->nan_flag, 1);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long k2 = shfl_xor_u64(key, o);
            key = k2 > key ? k2 : key;
        }
        unsigned long long* sk = (unsigned long long*)L.misc;
        __syncthreads();
        if ((t & 63) == 0) sk[t >> 6] = key;
        __syncthreads();
        if (t == 0) {
            unsigned long long b = sk[0];
            for (int i = 1; i < 4; ++i) b = sk[i] > b ? sk[i] : b;
            atomicMax(&st->keys[st->pos & 1], b);
        }
    }
};

template <class Pro, class Epi>
static int launch_mv(const DMat& w, const Plan& p, const Pro& pro, const Epi& epi, int tmp_floats,
                     hipStream_t s) {
    const int per_split = (w.nblk + p.S - 1) / p.S;
    const size_t lds = mv_lds_bytes(w.fmt, per_split, tmp_floats);
    const dim3 grid(w.tiles * p.S), block(NT);
    if (w.fmt == FMT_Q4) {
        switch (p.kbw) {
            case 1: hipLaunchKernelGGL((k_matvec<FMT_Q4, 1, Pro, Epi>), grid, block, lds, s, w, p.S, pro, epi); break;
            case 2: hipLaunchKernelGGL((k_matvec<FMT_Q4, 2, Pro, Epi>), grid, block, lds, s, w, p.S, pro, epi); break;
            case 3: hipLaunchKernelGGL((k_matvec<FMT_Q4, 3, Pro, Epi>), grid, block, lds, s, w, p.S, pro, epi); break;
            case 4: hipLaunchKernelGGL((k_matvec<FMT_Q4, 4, Pro, Epi>), grid, block, lds, s, w, p.S, pro, epi); break;
            case 6: hipLaunchKernelGGL((k_matvec<FMT_Q4, 6, Pro, Epi>), grid, block, lds, s, w, p.S, pro, epi); break;
            case 9: hipLaunchKernelGGL((k_matvec<FMT_Q4, 9, Pro, Epi>), grid, block, lds, s, w, p.S, pro, epi); break;
            default: return set_error(GH_ERR_INVALID, "unsupported register batch %d", p.kbw);
        }
    } else {
        hipLaunchKernelGGL((k_matvec<FMT_F32, 8, Pro, Epi>), grid, block, lds, s, w, p.S, pro, epi);
    }
    GH_HIP(hipGetLastError());
    return GH_OK;
}

// ------------------------------------------------------------------
// attention (split-K over cache positions, one kv head per group)
// ------------------------------------------------------------------
struct AttnArgs {
    // step mode: q/k/v come from the QKV partials and are normed + roped here
    const float* part_qkv;
    int Sa, ld_qkv, q_off, k_off, v_off;
    const float* q_norm;
    const float* k_norm;
    int use_qk_norm, zc;
    float eps;
    const float* inv_freq;  // [HD/2]
    const StepState* st;
    int global, window, mode;
    // raw mode: q given, window given
    const float* q;
    int p_begin, p_end;
    // common
    float* kc;
    float* vc;
    int nkv;
    float scale;
    float* part;
    int nc;
};

// In-place per-vector RMSNorm by one wave (qkNormShader semantics).
template <int HD>
__device__ __forceinline__ void wave_head_norm(float* p, const float* w, float eps, int zc) {
    const int lane = threadIdx.x & 63;
    float ss = 0.0f;
    for (int i = lane; i < HD; i += 64) ss += p[i] * p[i];
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)HD + eps);
    for (int i = lane; i < HD; i += 64) p[i] = norm_apply(p[i], rms, w[i], zc);
}

// In-place split-half RoPE of one head vector by one wave (ropeShader).
template <int HD>
__device__ __forceinline__ void wave_head_rope(float* p, const float* inv_freq, int pos) {
    const int lane = threadIdx.x & 63;
    for (int i = lane; i < HD / 2; i += 64) {
        const float ang = (float)pos * inv_freq[i];
        float sn, cs;
        sincosf(ang, &sn, &cs);
        const float a = p[i], b = p[i + HD / 2];
        p[i] = a * cs - b * sn;
        p[i + HD / 2] = a * sn + b * cs;
    }
}

template <int HD, int G, bool STEP>
__global__ __launch_bounds__(NT) void k_attn(AttnArgs a) {
    constexpr int LP = HD / 4;    // lanes per position (each lane owns 4 dims)
    constexpr int PPW = 64 / LP;  // positions per wave step
    constexpr int NS = 4 * PPW;   // softmax states per workgroup
    __shared__ float qs[G * HD], ks[HD], vs[HD];
    __shared__ float sm[NS][G], sl[NS][G];
    __shared__ float so[NS][G * HD];

    const int g = blockIdx.x / a.nc, j = blockIdx.x % a.nc;
    int pos = -1, pb, pe;
    if (STEP) {
        pos = a.st->pos;
        attn_window(pos, a.global, a.window, a.mode, pb, pe);
    } else {
        pb = a.p_begin;
        pe = a.p_end;
    }
    int ch, n_used;
    attn_chunks(pe - pb, a.nc, ch, n_used);
    if (j >= n_used) return;  // uniform per workgroup
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

    if (STEP) {
        for (int i = tid; i < (G + 2) * HD; i += NT) {
            int row;
            float* dst;
            if (i < G * HD) {
                row = a.q_off + g * G * HD + i;
                dst = &qs[i];
            } else if (i < (G + 1) * HD) {
                row = a.k_off + g * HD + (i - G * HD);
                dst = &ks[i - G * HD];
            } else {
                row = a.v_off + g * HD + (i - (G + 1) * HD);
                dst = &vs[i - (G + 1) * HD];
            }
            float v = 0.0f;
            for (int s = 0; s < a.Sa; ++s) v += a.part_qkv[(size_t)s * a.ld_qkv + row];
            *dst = v;
        }
        __syncthreads();
        // QK-norm (TBG:171-179), then RoPE, on the G q heads and the k head
        for (int vec = wave; vec < G + 1; vec += 4) {
            float* p = vec < G ? qs + vec * HD : ks;
            if (a.use_qk_norm) wave_head_norm<HD>(p, vec < G ? a.q_norm : a.k_norm, a.eps, a.zc);
            wave_head_rope<HD>(p, a.inv_freq, pos);
        }
        __syncthreads();
        if (j == 0) {  // appendKVCacheShader (AttentionGPU.hs:502-534)
            for (int i = tid; i < HD; i += NT) {
                a.kc[((size_t)pos * a.nkv + g) * HD + i] = ks[i];
                a.vc[((size_t)pos * a.nkv + g) * HD + i] = vs[i];
            }
        }
    } else {
        for (int i = tid; i < G * HD; i += NT) qs[i] = a.q[(size_t)g * G * HD + i];
        __syncthreads();
    }

    const int c0 = pb + j * ch, c1 = min(pe, c0 + ch);
    const int grp = lane / LP, lp = lane % LP;
    float q[G][4], m[G], l[G], acc[G][4];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float4 qq = *(const float4*)&qs[h * HD + 4 * lp];
        q[h][0] = qq.x; q[h][1] = qq.y; q[h][2] = qq.z; q[h][3] = qq.w;
        m[h] = -INFINITY;
        l[h] = 0.0f;
        acc[h][0] = acc[h][1] = acc[h][2] = acc[h][3] = 0.0f;
    }
    const size_t pstride = (size_t)a.nkv * HD;
    const float* kb = a.kc + (size_t)g * HD + 4 * lp;
    const float* vb = a.vc + (size_t)g * HD + 4 * lp;
    for (int p0 = c0 + wave * PPW; p0 < c1; p0 += 4 * PPW) {
        const int p = p0 + grp;
        const bool valid = p < c1;
        float4 kk = make_float4(0.f, 0.f, 0.f, 0.f), vv = kk;
        if (valid) {
            if (STEP && p == pos) {
                kk = *(const float4*)&ks[4 * lp];
                vv = *(const float4*)&vs[4 * lp];
            } else {
                kk = *(const float4*)(kb + (size_t)p * pstride);
                vv = *(const float4*)(vb + (size_t)p * pstride);
            }
        }
        float sc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) sc[h] = q[h][0] * kk.x + q[h][1] * kk.y + q[h][2] * kk.z + q[h][3] * kk.w;
#pragma unroll
        for (int o = LP / 2; o > 0; o >>= 1)
#pragma unroll
            for (int h = 0; h < G; ++h) sc[h] += __shfl_xor(sc[h], o, 64);
        if (valid) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float s = sc[h] * a.scale;
                const float mn = fmaxf(m[h], s);
                const float corr = expf(m[h] - mn);
                const float pe_ = expf(s - mn);
                l[h] = l[h] * corr + pe_;
                acc[h][0] = acc[h][0] * corr + pe_ * vv.x;
                acc[h][1] = acc[h][1] * corr + pe_ * vv.y;
                acc[h][2] = acc[h][2] * corr + pe_ * vv.z;
                acc[h][3] = acc[h][3] * corr + pe_ * vv.w;
                m[h] = mn;
            }
        }
    }
    const int si = wave * PPW + grp;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        if (lp == 0) {
            sm[si][h] = m[h];
            sl[si][h] = l[h];
        }
        *(float4*)&so[si][h * HD + 4 * lp] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    }
    __syncthreads();
    float* out = a.part + ((size_t)g * a.nc + j) * (G * (HD + 2));
    for (int idx = tid; idx < G * HD; idx += NT) {
        const int h = idx / HD;
        float M = -INFINITY;
        for (int s2 = 0; s2 < NS; ++s2) M = fmaxf(M, sm[s2][h]);
        float Lsum = 0.0f, O = 0.0f;
        for (int s2 = 0; s2 < NS; ++s2) {
            const float wgt = expf(sm[s2][h] - M);  // empty states: exp(-inf) = 0
            Lsum += sl[s2][h] * wgt;
            O += so[s2][idx] * wgt;
        }
        out[2 * G + idx] = O;
        if (idx % HD == 0) {
            out[h] = M;
            out[G + h] = Lsum;
        }
    }
}

template <bool STEP>
static int launch_attn_t(int hd, int G, const AttnArgs& a, int nkv, hipStream_t s) {
    const dim3 grid(nkv * a.nc), block(NT);
#define GH_ATTN_CASE(HD_, G_)                                                         \
    if (hd == HD_ && G == G_) {                                                       \
        hipLaunchKernelGGL((k_attn<HD_, G_, STEP>), grid, block, 0, s, a);            \
        GH_HIP(hipGetLastError());                                                    \
        return GH_OK;                                                                 \
    }
    GH_ATTN_CASE(256, 1) GH_ATTN_CASE(256, 2) GH_ATTN_CASE(256, 4) GH_ATTN_CASE(256, 8)
    GH_ATTN_CASE(128, 1) GH_ATTN_CASE(128, 2) GH_ATTN_CASE(128, 4) GH_ATTN_CASE(128, 8)
    GH_ATTN_CASE(32, 1) GH_ATTN_CASE(32, 2) GH_ATTN_CASE(32, 4) GH_ATTN_CASE(32, 8)
#undef GH_ATTN_CASE
    return set_error(GH_ERR_INVALID, "attention: unsupported head_dim %d / group %d", hd, G);
}

__global__ void k_attn_combine(const float* part, int nc, int n_used, int G, int HD, int nq, float* out) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nq * HD) return;
    const int h = idx / HD, d = idx % HD;
    out[idx] = attn_merge(part, nc, n_used, G, HD, h / G, h % G, d);
}

// ------------------------------------------------------------------
// step epilogue: next token, position, argmax slot reset
// ------------------------------------------------------------------
__global__ void k_step_finish(StepState* st, const int32_t* prompt, int32_t* ids) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const int pos = st->pos;
    const unsigned long long key = st->keys[pos & 1];
    const int tok = (int)(0xFFFFFFFFu - (unsigned)(key & 0xFFFFFFFFull));
    st->last = tok;
    const int rel = pos + 1 - st->start;
    int next = tok;
    if (prompt && rel < st->n_prompt) {
        next = prompt[rel];
    } else if (ids && st->gen_count < st->gen_cap) {
        ids[st->gen_count] = tok;
        st->gen_count = st->gen_count + 1;
    }
    st->token = next;
    st->keys[(pos + 1) & 1] = 0ull;
    st->pos = pos + 1;
}

// ------------------------------------------------------------------
// the decode step: 5 kernels per layer + LM head + finish
// ------------------------------------------------------------------
int Profiler::kind_of(const char* name) {
    for (size_t i = 0; i < names.size(); ++i)
        if (names[i] == name) return (int)i;
    names.emplace_back(name);
    return (int)names.size() - 1;
}

namespace {
struct ProfScope {
    Profiler* p;
    hipStream_t s;
    int idx = -1;
    ProfScope(Profiler* p_, hipStream_t s_, const char* name, double bytes) : p(p_), s(s_) {
        if (!p) return;
        Profiler::Rec r;
        r.kind = p->kind_of(name);
        r.bytes = bytes;
        hipEventCreate(&r.a);
        hipEventCreate(&r.b);
        hipEventRecord(r.a, s);
        p->recs.push_back(r);
        idx = (int)p->recs.size() - 1;
    }
    ~ProfScope() {
        if (p && idx >= 0) hipEventRecord(p->recs[idx].b, s);
    }
};

double mat_bytes(const DMat& w) {
    const double wb = w.fmt == FMT_Q4 ? (double)w.rows * w.cols / 32.0 * 18.0 : (double)w.rows * w.cols * 4.0;
    return wb + 4.0 * w.cols + 4.0 * w.rows;
}
}  // namespace

int enqueue_step(gh_model* m, gh_kv* kv, hipStream_t s, Profiler* prof) {
    const gh_config& c = m->cfg;
    const int H = c.hidden, nq = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    const int G = nq / nkv;
    const int zc = (c.flags & GH_FLAG_ZERO_CENTERED) ? 1 : 0;
    const float eps = c.rms_eps;
    const size_t kv_layer = (size_t)kv->max_seq * nkv * hd;
    const int n_pos_host = std::min(kv->len + 1, kv->max_seq);  // for profiling byte counts only

    for (int li = 0; li < c.n_layers; ++li) {
        LayerDev& L = m->layers[li];
        const LayerDev* P = li > 0 ? &m->layers[li - 1] : nullptr;
        // A: residual + pre-attention norm + fused QKV matvec
        {
            ProResidNorm pro;
            pro.from_embedding = li == 0;
            pro.embd = m->embd;
            pro.st = kv->st;
            pro.escale = sqrtf((float)H);
            pro.x1 = m->x1;
            pro.part_d = m->part_d;
            pro.Sd = m->pe.S;
            pro.ld_d = P ? P->down.tiles * TILE_ROWS : 0;
            pro.w_post = P && (c.flags & GH_FLAG_POST_FFN_NORM) ? P->post_ffw : nullptr;
            pro.w_norm = L.attn_norm;
            pro.eps = eps;
            pro.zc = zc;
            pro.H = H;
            pro.x_res = m->x_res;
            pro.layer_out_row = li > 0 ? m->layer_out + (size_t)(li - 1) * H : nullptr;
            EpiPartial epi{m->part_qkv, L.qkv.tiles * TILE_ROWS};
            ProfScope ps(prof, s, "qkv", mat_bytes(L.qkv));
            GH_CHECK(launch_mv(L.qkv, m->pa, pro, epi, H, s));
        }
        // B: QK-norm + RoPE + KV append + split-K attention
        {
            AttnArgs a{};
            a.part_qkv = m->part_qkv;
            a.Sa = m->pa.S;
            a.ld_qkv = L.qkv.tiles * TILE_ROWS;
            a.q_off = 0;
            a.k_off = m->q_rows_pad;
            a.v_off = m->q_rows_pad + m->kv_rows_pad;
            a.q_norm = L.q_norm;
            a.k_norm = L.k_norm;
            a.use_qk_norm = (c.flags & GH_FLAG_QK_NORM) && L.q_norm && L.k_norm;
            a.zc = zc;
            a.eps = eps;
            const bool global = c.mode == GH_MODE_REF ? true : L.global;
            a.inv_freq = m->inv_freq + (global ? hd / 2 : 0);
            a.st = kv->st;
            a.global = L.global;
            a.window = c.sliding_window;
            a.mode = c.mode;
            a.kc = kv->k + li * kv_layer;
            a.vc = kv->v + li * kv_layer;
            a.nkv = nkv;
            a.scale = 1.0f / sqrtf((float)hd);
            a.part = m->attn_part;
            a.nc = m->attn_nc;
            ProfScope ps(prof, s, "attention", 2.0 * 4.0 * hd * nkv * n_pos_host);
            GH_CHECK(launch_attn_t<true>(hd, G, a, nkv, s));
        }
        // C: attention merge + O projection
        {
            ProAttnCombine pro{m->attn_part, kv->st, m->attn_nc, G, hd, L.global ? 1 : 0,
                               c.sliding_window, c.mode};
            EpiPartial epi{m->part_o, L.o.tiles * TILE_ROWS};
            ProfScope ps(prof, s, "o_proj", mat_bytes(L.o));
            GH_CHECK(launch_mv(L.o, m->pc, pro, epi, 0, s));
        }
        // D: post-attention norm + residual + pre-FFN norm + gate/up matvec
        {
            ProPostAttn pro;
            pro.part_o = m->part_o;
            pro.So = m->pc.S;
            pro.ld_o = L.o.tiles * TILE_ROWS;
            pro.w_post = (c.flags & GH_FLAG_POST_ATTN_NORM) ? L.post_attn : nullptr;
            pro.x_res = m->x_res;
            pro.x1_out = m->x1;
            pro.w_ffn = L.ffn_norm ? L.ffn_norm : L.post_attn;
            pro.eps = eps;
            pro.zc = zc;
            pro.H = H;
            EpiPartial epi{m->part_gu, L.gu.tiles * TILE_ROWS};
            ProfScope ps(prof, s, "gate_up", mat_bytes(L.gu));
            GH_CHECK(launch_mv(L.gu, m->pd, pro, epi, H, s));
        }
        // E: GeGLU + down projection
        {
            ProGeglu pro{m->part_gu, m->pd.S, L.gu.tiles * TILE_ROWS, m->f_pad};
            EpiPartial epi{m->part_d, L.down.tiles * TILE_ROWS};
            ProfScope ps(prof, s, "down", mat_bytes(L.down));
            GH_CHECK(launch_mv(L.down, m->pe, pro, epi, 0, s));
        }
    }
    // final norm + LM head + argmax
    {
        const LayerDev& P = m->layers[c.n_layers - 1];
        ProResidNorm pro;
        pro.from_embedding = 0;
        pro.embd = m->embd;
        pro.st = kv->st;
        pro.escale = 1.0f;
        pro.x1 = m->x1;
        pro.part_d = m->part_d;
        pro.Sd = m->pe.S;
        pro.ld_d = P.down.tiles * TILE_ROWS;
        pro.w_post = (c.flags & GH_FLAG_POST_FFN_NORM) ? P.post_ffw : nullptr;
        pro.w_norm = m->out_norm;
        pro.eps = eps;
        pro.zc = zc;
        pro.H = H;
        pro.x_res = nullptr;
        pro.layer_out_row = m->layer_out + (size_t)(c.n_layers - 1) * H;
        EpiLogits epi{m->logits, c.vocab, kv->st};
        ProfScope ps(prof, s, "lm_head", mat_bytes(m->embd));
        GH_CHECK(launch_mv(m->embd, m->plm, pro, epi, H, s));
    }
    {
        ProfScope ps(prof, s, "finish", 0.0);
        hipLaunchKernelGGL(k_step_finish, dim3(1), dim3(64), 0, s, kv->st, kv->d_prompt, kv->d_ids);
        GH_HIP(hipGetLastError());
    }
    return GH_OK;
}

// ------------------------------------------------------------------
// op-level kernels
// ------------------------------------------------------------------
__global__ void k_q4_dequant(DMat w, float* out) {
    const long long blk = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long nblk_total = (long long)w.rows * w.nblk;
    if (blk >= nblk_total) return;
    const int r = (int)(blk / w.nblk), b = (int)(blk % w.nblk);
    float* o = out + (size_t)r * w.cols + (size_t)b * 32;
    for (int e = 0; e < 32; ++e) o[e] = dq_elem(w, r, b * 32 + e);
}

int launch_q4_dequant(const DMat& w, float* out, hipStream_t s) {
    const long long n = (long long)w.rows * w.nblk;
    hipLaunchKernelGGL(k_q4_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w, out);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

__global__ void k_sum_partials(const float* part, int S, int ld, int rows, int softcap, float cap,
                               float* y) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float a = 0.0f;
    for (int s = 0; s < S; ++s) a += part[(size_t)s * ld + r];
    y[r] = softcap ? cap * tanhf(a / cap) : a;
}

int launch_matvec_plain(const DMat& w, const Plan& p, const float* x, float* part, float* y,
                        int softcap, float cap, hipStream_t s) {
    ProPlain pro{x};
    if (p.S == 1) {
        EpiOut epi{y, w.rows, softcap, cap};
        return launch_mv(w, p, pro, epi, 0, s);
    }
    EpiPartial epi{part, w.tiles * TILE_ROWS};
    GH_CHECK(launch_mv(w, p, pro, epi, 0, s));
    hipLaunchKernelGGL(k_sum_partials, dim3((w.rows + 255) / 256), dim3(256), 0, s, part, p.S,
                       w.tiles * TILE_ROWS, w.rows, softcap, cap, y);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

__global__ __launch_bounds__(NT) void k_rmsnorm(const float* x, const float* w, int n, float eps, int zc,
                                                float* y) {
    __shared__ float red[4];
    const float rms = block_rms(x, n, eps, red);
    for (int i = threadIdx.x; i < n; i += NT) y[i] = norm_apply(x[i], rms, w[i], zc);
}

int launch_rmsnorm(const float* x, const float* w, int n, float eps, int zc, float* y, hipStream_t s) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(NT), 0, s, x, w, n, eps, zc, y);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

// one wave per head, in global memory
template <int HD>
__global__ void k_qk_norm(const float* x, const float* w, int n_heads, float eps, int zc, float* y) {
    const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (h >= n_heads) return;
    const int lane = threadIdx.x & 63;
    for (int i = lane; i < HD; i += 64) y[h * HD + i] = x[h * HD + i];
    __builtin_amdgcn_wave_barrier();
    wave_head_norm<HD>(y + h * HD, w, eps, zc);
}

int launch_qk_norm(const float* x, const float* w, int n_heads, int hd, float eps, int zc, float* y,
                   hipStream_t s) {
    const dim3 grid((n_heads + 3) / 4), block(NT);
    if (hd == 256) hipLaunchKernelGGL(k_qk_norm<256>, grid, block, 0, s, x, w, n_heads, eps, zc, y);
    else if (hd == 128) hipLaunchKernelGGL(k_qk_norm<128>, grid, block, 0, s, x, w, n_heads, eps, zc, y);
    else if (hd == 32) hipLaunchKernelGGL(k_qk_norm<32>, grid, block, 0, s, x, w, n_heads, eps, zc, y);
    else return set_error(GH_ERR_INVALID, "qk_norm: unsupported head_dim %d", hd);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

template <int HD>
__global__ void k_rope(float* x, int n_heads, const float* inv_freq, int pos) {
    const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (h >= n_heads) return;
    wave_head_rope<HD>(x + h * HD, inv_freq, pos);
}

int launch_rope(float* x, int n_heads, int hd, float theta, int pos, hipStream_t s) {
    // inverse frequencies computed on the host with ropeShader's formula
    std::vector<float> f(hd / 2);
    for (int i = 0; i < hd / 2; ++i) f[i] = 1.0f / powf(theta, (float)(i * 2) / (float)hd);
    float* d = nullptr;
    GH_HIP(hipMallocAsync((void**)&d, sizeof(float) * f.size(), s));
    GH_HIP(hipMemcpyAsync(d, f.data(), sizeof(float) * f.size(), hipMemcpyHostToDevice, s));
    const dim3 grid((n_heads + 3) / 4), block(NT);
    if (hd == 256) hipLaunchKernelGGL(k_rope<256>, grid, block, 0, s, x, n_heads, d, pos);
    else if (hd == 128) hipLaunchKernelGGL(k_rope<128>, grid, block, 0, s, x, n_heads, d, pos);
    else if (hd == 32) hipLaunchKernelGGL(k_rope<32>, grid, block, 0, s, x, n_heads, d, pos);
    else {
        hipFreeAsync(d, s);
        return set_error(GH_ERR_INVALID, "rope: unsupported head_dim %d", hd);
    }
    GH_HIP(hipGetLastError());
    GH_HIP(hipStreamSynchronize(s));  // f is a host temporary
    GH_HIP(hipFreeAsync(d, s));
    return GH_OK;
}

int launch_attention(const float* q, const float* kc, const float* vc, int nq, int nkv, int hd,
                     int p_begin, int p_end, int n_splits, float* part, float* out, hipStream_t s) {
    AttnArgs a{};
    a.q = q;
    a.p_begin = p_begin;
    a.p_end = p_end;
    a.kc = const_cast<float*>(kc);
    a.vc = const_cast<float*>(vc);
    a.nkv = nkv;
    a.scale = 1.0f / sqrtf((float)hd);
    a.part = part;
    a.nc = n_splits;
    GH_CHECK(launch_attn_t<false>(hd, nq / nkv, a, nkv, s));
    int n_pos = p_end - p_begin, ch = (n_pos + n_splits - 1) / n_splits;
    int n_used = (n_pos + ch - 1) / ch;
    hipLaunchKernelGGL(k_attn_combine, dim3((nq * hd + 255) / 256), dim3(256), 0, s, part, n_splits,
                       n_used, nq / nkv, hd, nq, out);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

__global__ void k_gelu_mul(const float* g, const float* u, int n, float* h) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = gelu_tanh(g[i]) * u[i];
}

int launch_gelu_mul(const float* g, const float* u, int n, float* h, hipStream_t s) {
    hipLaunchKernelGGL(k_gelu_mul, dim3((n + 255) / 256), dim3(256), 0, s, g, u, n, h);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

__global__ void k_fill_u64(unsigned long long* p, unsigned long long v) { *p = v; }

__global__ __launch_bounds__(NT) void k_argmax(const float* v, int n, unsigned long long* key) {
    __shared__ unsigned long long sk[4];
    unsigned long long best = 0ull;
    for (int i = blockIdx.x * NT + threadIdx.x; i < n; i += gridDim.x * NT) {
        const unsigned long long k = argmax_key(v[i], i);
        best = k > best ? k : best;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long k2 = shfl_xor_u64(best, o);
        best = k2 > best ? k2 : best;
    }
    if ((threadIdx.x & 63) == 0) sk[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < 4; ++i) best = sk[i] > best ? sk[i] : best;
        best = sk[0] > best ? sk[0] : best;
        atomicMax(key, best);
    }
}

int launch_argmax(const float* v, int n, unsigned long long* key, hipStream_t s) {
    hipLaunchKernelGGL(k_fill_u64, dim3(1), dim3(1), 0, s, key, 0ull);
    const int blocks = std::max(1, std::min(1024, (n + NT - 1) / NT));
    hipLaunchKernelGGL(k_argmax, dim3(blocks), dim3(NT), 0, s, v, n, key);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

}  // namespace gh
