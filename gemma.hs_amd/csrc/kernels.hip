// gfx950 kernels of the batch-1 decode step and the op-level entry points.
//
// The step is 5 kernels per layer + final norm + LM head + finish, replayed
// from one hipGraph.  On MI355X a graph kernel boundary costs ~1.6 us while a
// correct chip-wide barrier inside a persistent kernel costs more (agent-scope
// fences serialise per XCD), so the design minimises the latency *inside*
// each kernel: one global round trip per prologue, DPP/readlane reductions,
// weights in flight before the prologue starts.
//
// Every matvec-shaped kernel follows one pattern (k_matvec):
//   1. each wave issues the loads of its weight blocks into registers
//      (two rows per lane: lane and lane+64 of a 128-row tile; one 1 KB
//      contiguous wave load per row and column block),
//   2. the prologue builds the input-vector slice of the workgroup in LDS
//      (residual + RMSNorm, attention merge, GeGLU, ...) while those loads
//      are in flight,
//   3. dequant-dot: nibbles -> f32 with byte conversions, x broadcast from
//      LDS, f32 accumulation, block scale applied once per 32 weights,
//   4. the four waves' row partials are summed in LDS; the epilogue writes a
//      split partial (summed by the next kernel's prologue) or the logits
//      and a per-tile argmax key.
// Where a phase has more work items than the device has CUs, two items of
// one column split share an 8-wave workgroup and its prologue
// (k_matvec_multi).  Batch-1 decode is HBM-bound (3.5 flop/byte for Q4_0),
// so the matrix cores are not needed for the flops; where the VALU
// dequant-dot itself costs time (the LM head, large op-level matvecs,
// paired items with wide column splits) the dot products run on the int8
// matrix cores instead (FMT_Q4M, mq_item_v, mq_item_multi_v).
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "common.h"

// The library compiles this file as several translation units in parallel
// (GH_TU = 1 step, 2 persistent step, 3 prefill, 4 op level, 5-7 the step's
// matvec phases by prologue); each defines
// its own host entry points and so instantiates only the kernels they
// launch.  Kernels launched from several units are templates, whose
// symbols are merged at link time.  GH_TU = 0 (the default) is everything.
#ifndef GH_TU
#define GH_TU 0
#endif
#define GH_IN_TU(n) (GH_TU == 0 || GH_TU == (n))

// Phase timestamp hook for latency studies; compiles to nothing unless a
// timing harness defines it before including this file.
#ifndef GH_MARK
#define GH_MARK(slot)
#endif
#ifndef GH_MARK_END
#define GH_MARK_END()
#endif

namespace gh {

constexpr int NT = 256;  // threads per workgroup (4 wave64)
constexpr int MAXS = 8;  // max column splits reduced by a prologue in one round trip

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------
// cross-lane reductions (DPP within 16-lane rows, row broadcasts + readlane across rows)
// ------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int DPP_ROW_ROR4 = 0x124;
constexpr int DPP_ROW_ROR8 = 0x128;
constexpr int DPP_ROW_HALF_MIRROR = 0x141;

__device__ __forceinline__ float readlane(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// every lane of a 16-lane row gets the row sum
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<DPP_QUAD_XOR1>(v);
    v += dpp<DPP_QUAD_XOR2>(v);
    v += dpp<DPP_ROW_ROR4>(v);
    v += dpp<DPP_ROW_ROR8>(v);
    return v;
}

// Combine the four 16-lane rows (each already holding its row result in
// every lane): row_bcast:15 folds row 0 into row 1 and row 2 into row 3,
// row_bcast:31 folds row 1 into rows 2-3, so lane 63 holds the result,
// which readlane makes wave-uniform.  (gfx950's permlane16/32_swap would
// avoid the SGPR, but the ROCm 7.2 compiler returns the first swap output
// for both halves of the builtin's result, so they are not used.)
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_rows(float old, float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                                 CTRL, ROW_MASK, 0xF, false));
}
constexpr int DPP_ROW_BCAST15 = 0x142;
constexpr int DPP_ROW_BCAST31 = 0x143;

template <class Op>
__device__ __forceinline__ float rows_combine(float v, float ident, Op op) {
    v = op(v, dpp_rows<DPP_ROW_BCAST15, 0xA>(ident, v));
    v = op(v, dpp_rows<DPP_ROW_BCAST31, 0xC>(ident, v));
    return readlane(v, 63);
}

// wave-uniform sum of the 64 lanes
__device__ __forceinline__ float wave_sum(float v) {
    return rows_combine(row16_sum(v), 0.0f, [](float x, float y) { return x + y; });
}

__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp<DPP_ROW_ROR4>(v));
    v = fmaxf(v, dpp<DPP_ROW_ROR8>(v));
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    return rows_combine(row16_max(v), -INFINITY, [](float x, float y) { return fmaxf(x, y); });
}

// wave-uniform max of a value that is already uniform within aligned groups
// of 8 lanes (one DPP step instead of four inside each row)
__device__ __forceinline__ float wave_max_g8(float v) {
    return rows_combine(fmaxf(v, dpp<DPP_ROW_ROR8>(v)), -INFINITY, [](float x, float y) { return fmaxf(x, y); });
}

// sum over aligned groups of LP lanes (result in every lane of the group)
template <int LP>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (LP == 64) {
        return wave_sum(v);
    } else if constexpr (LP == 32) {
        v = row16_sum(v);
        return v + __shfl_xor(v, 16, 64);
    } else if constexpr (LP == 16) {
        return row16_sum(v);
    } else {
        static_assert(LP == 8, "lanes per position must be 8, 16, 32 or 64");
        v += dpp<DPP_QUAD_XOR1>(v);
        v += dpp<DPP_QUAD_XOR2>(v);
        return v + dpp<DPP_ROW_HALF_MIRROR>(v);
    }
}

// max over aligned groups of 8 lanes (result in every lane of the group)
__device__ __forceinline__ float group_max8(float v) {
    v = fmaxf(v, dpp<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp<DPP_QUAD_XOR2>(v));
    return fmaxf(v, dpp<DPP_ROW_HALF_MIRROR>(v));
}

// Sum over the 256 threads, one barrier; `slot` (4 floats of LDS) must not
// be reused before every thread has returned.
__device__ __forceinline__ float block_sum(float v, float* slot) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = v;
    __syncthreads();
    return (slot[0] + slot[1]) + (slot[2] + slot[3]);
}

// Max over the 256 threads, one barrier (same slot rules as block_sum).
__device__ __forceinline__ float block_max(float v, float* slot) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(slot[0], slot[1]), fmaxf(slot[2], slot[3]));
}

// Four sums over the 256 threads with one barrier (`slot`: 16 floats of LDS,
// same reuse rule as block_sum).
__device__ __forceinline__ float4 block_sum4(float4 v, float* slot) {
    v.x = wave_sum(v.x);
    v.y = wave_sum(v.y);
    v.z = wave_sum(v.z);
    v.w = wave_sum(v.w);
    if ((threadIdx.x & 63) == 0) ((float4*)slot)[threadIdx.x >> 6] = v;
    __syncthreads();
    const float4 a = ((const float4*)slot)[0], b = ((const float4*)slot)[1];
    const float4 c = ((const float4*)slot)[2], d = ((const float4*)slot)[3];
    return make_float4((a.x + b.x) + (c.x + d.x), (a.y + b.y) + (c.y + d.y), (a.z + b.z) + (c.z + d.z),
                       (a.w + b.w) + (c.w + d.w));
}

// Order-preserving argmax key: larger value wins, then lower index.
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    unsigned b = __float_as_uint(v);
    unsigned ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned)(0xFFFFFFFFu - (unsigned)idx);
}

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int o) {
    unsigned lo = (unsigned)v, hi = (unsigned)(v >> 32);
    lo = __shfl_xor(lo, o, 64);
    hi = __shfl_xor(hi, o, 64);
    return ((unsigned long long)hi << 32) | lo;
}

// block-wide max key (one barrier), result valid in every thread
__device__ __forceinline__ unsigned long long block_max_key(unsigned long long k, unsigned long long* slot) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) k = umax64(k, shfl_xor_u64(k, o));
    if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = k;
    __syncthreads();
    return umax64(umax64(slot[0], slot[1]), umax64(slot[2], slot[3]));
}

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// ------------------------------------------------------------------
// Raw buffer views.  A load whose byte offset lies outside the view returns
// zeros without touching memory (the buffer range check of CDNA), so
// optional, ragged and split-count-dependent loads need neither a branch
// nor a clamp: every load of a prologue or weight batch is straight-line
// code, and the compiler's s_waitcnt counts stay exact (a prologue waits
// for its own inputs, not for the weight loads issued after them).
// ------------------------------------------------------------------
constexpr uint32_t OOB = 0x80000000u;  // past the end of every view (views are < 2 GiB)
#ifndef GH_CP_WEIGHTS
#define GH_CP_WEIGHTS 2
#endif
constexpr int CP_NT = GH_CP_WEIGHTS;  // cache policy of streamed weights (2: non-temporal)

struct BufView {
    __amdgpu_buffer_rsrc_t r;
    // bytes = 0 (or p = nullptr with bytes = 0): every load reads zeros.
    // p and bytes must be the same in every lane of the wave (the descriptor
    // is a scalar operand): they are taken from the first active lane, so
    // that the compiler keeps the descriptor in SGPRs.  Where it cannot prove
    // a base uniform (loop-carried layer tables, SGPR pressure) it would
    // otherwise wrap each load in a waterfall loop.
    __device__ __forceinline__ BufView(const void* p, size_t bytes) {
        const uint64_t a = (uint64_t)p;
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
        const int n = __builtin_amdgcn_readfirstlane((int)(bytes < 0x7fffffffu ? bytes : 0x7fffffffu));
        r = __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, n, 0x00020000);
    }
    template <int CP = 0>
    __device__ __forceinline__ float4 f4(uint32_t off) const {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP));
    }
    template <int CP = 0>
    __device__ __forceinline__ u32x4 u4(uint32_t off) const {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP));
    }
    template <int CP = 0>
    __device__ __forceinline__ u32x2 u2(uint32_t off) const {
        return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CP));
    }
    template <int CP = 0>
    __device__ __forceinline__ float f1(uint32_t off) const {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CP));
    }
    template <int CP = 0>
    __device__ __forceinline__ uint16_t h1(uint32_t off) const {
        return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, CP);
    }
};

// wave index as a wave-uniform (scalar) value
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// GELU(tanh) with the +-10 clamp of src/Gemma/Layers/MLP.hs:384-447.
__device__ __forceinline__ float gelu_tanh(float x) {
    float x3 = x * x * x;
    float t = 0.7978845608f * (x + 0.044715f * x3);
    t = fminf(fmaxf(t, -10.0f), 10.0f);
    return x * 0.5f * (1.0f + tanhf(t));
}

__device__ __forceinline__ float norm_apply(float x, float rms, float w, int zc) {
    return zc ? (x / rms) * (1.0f + w) : (x / rms) * w;
}

__device__ __forceinline__ float4 operator+(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float dot4(float4 a, float4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }
// The step's norms scale by one reciprocal of the RMS per vector instead of
// dividing every element: (x * (1/rms)) differs from x / rms by at most an
// ulp or so, far inside the 1e-4 activation tolerance, and it takes the
// divide sequence off the latency chain of every prologue.
__device__ __forceinline__ float norm_apply_inv(float x, float inv, float w, int zc) {
    return zc ? (x * inv) * (1.0f + w) : (x * inv) * w;
}
__device__ __forceinline__ float4 norm4i(float4 x, float inv, float4 w, int zc) {
    return make_float4(norm_apply_inv(x.x, inv, w.x, zc), norm_apply_inv(x.y, inv, w.y, zc),
                       norm_apply_inv(x.z, inv, w.z, zc), norm_apply_inv(x.w, inv, w.w, zc));
}
__device__ __forceinline__ float4 norm4(float4 x, float rms, float4 w, int zc) {
    return make_float4(norm_apply(x.x, rms, w.x, zc), norm_apply(x.y, rms, w.y, zc), norm_apply(x.z, rms, w.z, zc),
                       norm_apply(x.w, rms, w.w, zc));
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

// Elements c..c+3 (c % 4 == 0) of row r, dequantised exactly.
__device__ __forceinline__ float4 dq_elem4(const DMat& w, int r, int c) {
    const int t = r >> 7, lr = r & 127;
    if (w.fmt == FMT_Q4) {
        const int b = c >> 5, e = c & 31;
        const size_t idx = ((size_t)t * w.nblk + b) * TILE_ROWS + lr;
        const uint32_t word = ((const uint32_t*)w.codes)[idx * 4 + ((e & 15) >> 2)];
        const uint32_t q = (e < 16) ? (word & 0x0F0F0F0Fu) : ((word >> 4) & 0x0F0F0F0Fu);
        const float d = h2f(w.scales[idx]);
        return make_float4(((float)(q & 0xFF) - 8.0f) * d, ((float)((q >> 8) & 0xFF) - 8.0f) * d,
                           ((float)((q >> 16) & 0xFF) - 8.0f) * d, ((float)(q >> 24) - 8.0f) * d);
    }
    const size_t idx = ((size_t)t * w.nblk + (c >> 2)) * TILE_ROWS + lr;
    return ((const float4*)w.codes)[idx];
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
struct Blk<FMT_Q4M> {
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

// Views of a tiled matrix: the codes (16 B per row and column block) and,
// for Q4_0, the fp16 scales (2 B per row and block).
struct MatViews {
    BufView codes, scales;
    __device__ __forceinline__ explicit MatViews(const DMat& w)
        : codes(w.codes, (size_t)w.tiles * w.nblk * TILE_ROWS * 16),
          scales(w.scales, w.fmt == FMT_Q4 ? (size_t)w.tiles * w.nblk * TILE_ROWS * 2 : 0) {}
};

// Loads of one register batch: rows rbase+lane (and rbase+lane+64 when a
// lane holds RL = 2 rows) of column blocks base .. base+KBW-1 of row tile
// `tile`; blocks at or past kw1 (wave-uniform) read zeros from an
// out-of-range offset, so the batch is straight-line code.
template <int FMT, int KBW, int RL>
__device__ __forceinline__ void mv_load(WRegs<FMT, KBW>& r, const DMat& w, const MatViews& v, int tile, int rbase,
                                        int base, int kw1) {
    const int lane = threadIdx.x & 63;
    const uint32_t row0 = (uint32_t)tile * (uint32_t)w.nblk * TILE_ROWS + (uint32_t)(rbase + lane);
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
        const bool ok = base + i < kw1;
        const uint32_t e = row0 + (uint32_t)(base + i) * TILE_ROWS;  // element (row, block) index
        r.c0[i] = v.codes.template u4<CP_NT>(ok ? e * 16u : OOB);
        if (RL == 2) r.c1[i] = v.codes.template u4<CP_NT>(ok ? (e + 64u) * 16u : OOB);
        if (FMT == FMT_Q4) {
            r.s0[i] = v.scales.template h1<CP_NT>(ok ? e * 2u : OOB);
            if (RL == 2) r.s1[i] = v.scales.template h1<CP_NT>(ok ? (e + 64u) * 2u : OOB);
        }
    }
}

// Opaque nibble masks: hiding the AND from the optimiser keeps each byte
// conversion a single v_cvt_f32_ubyteN (it would otherwise fold the mask
// into a 4-bit v_bfe_u32 plus v_cvt_f32_ubyte0).
__device__ __forceinline__ uint32_t mask_lo(uint32_t w) {
    uint32_t r;
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(w));
    return r;
}
__device__ __forceinline__ uint32_t mask_hi(uint32_t w) {
    uint32_t r;
    asm("v_and_b32 %0, 0xf0f0f0f0, %1" : "=v"(r) : "v"(w));
    return r;
}

// acc + sum_e q_e x_e over one 32-bit word of codes.  Bytes of `lo` are
// elements 4j..4j+3 (low nibbles, value q); bytes of `hi` are elements
// 16+4j.. (high nibbles kept in place, value 16q) and meet x/16, which the
// prologue stores for the upper half of every block: 16q * (x/16) == q x.
__device__ __forceinline__ float dot_q4_word(uint32_t w, float4 xl, float4 xh, float acc) {
    const uint32_t lo = mask_lo(w), hi = mask_hi(w);
    acc = fmaf((float)(lo & 0xFF), xl.x, acc);
    acc = fmaf((float)((lo >> 8) & 0xFF), xl.y, acc);
    acc = fmaf((float)((lo >> 16) & 0xFF), xl.z, acc);
    acc = fmaf((float)(lo >> 24), xl.w, acc);
    acc = fmaf((float)(hi & 0xFF), xh.x, acc);
    acc = fmaf((float)((hi >> 8) & 0xFF), xh.y, acc);
    acc = fmaf((float)((hi >> 16) & 0xFF), xh.z, acc);
    acc = fmaf((float)(hi >> 24), xh.w, acc);
    return acc;
}

template <int FMT, int KBW, int RL>
__device__ __forceinline__ void mv_block(const WRegs<FMT, KBW>& r, int i, int kb, int kb0, const float* xs,
                                         const float* sxs, float& acc0, float& acc1) {
    if (FMT == FMT_Q4) {
        const float4* xv = (const float4*)(xs + (kb - kb0) * 32);
        float d0 = 0.0f, d1 = 0.0f;
        const uint32_t w0[4] = {r.c0[i].x, r.c0[i].y, r.c0[i].z, r.c0[i].w};
        const uint32_t w1[4] = {r.c1[i].x, r.c1[i].y, r.c1[i].z, r.c1[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 xl = xv[j], xh = xv[4 + j];
            d0 = dot_q4_word(w0[j], xl, xh, d0);
            if (RL == 2) d1 = dot_q4_word(w1[j], xl, xh, d1);
        }
        // sum (q-8) x = sum q x - 8 sum x ; sxs holds sum x per block
        const float sx8 = 8.0f * sxs[kb - kb0];
        acc0 = fmaf(h2f(r.s0[i]), d0 - sx8, acc0);
        if (RL == 2) acc1 = fmaf(h2f(r.s1[i]), d1 - sx8, acc1);
    } else {
        const float4 x = *(const float4*)(xs + (kb - kb0) * 4);
        const f32x4 a = __builtin_bit_cast(f32x4, r.c0[i]);
        acc0 += a.x * x.x + a.y * x.y + a.z * x.z + a.w * x.w;
        if (RL == 2) {
            const f32x4 b = __builtin_bit_cast(f32x4, r.c1[i]);
            acc1 += b.x * x.x + b.y * x.y + b.z * x.z + b.w * x.w;
        }
    }
}

template <int FMT, int KBW, int RL>
__device__ __forceinline__ void mv_compute(const WRegs<FMT, KBW>& r, int base, int kw1, int kb0, const float* xs,
                                           const float* sxs, float& acc0, float& acc1) {
    if (base + KBW <= kw1) {  // full batch: no per-block predication (kw1 is wave-uniform)
#pragma unroll
        for (int i = 0; i < KBW; ++i) mv_block<FMT, KBW, RL>(r, i, base + i, kb0, xs, sxs, acc0, acc1);
    } else {
#pragma unroll
        for (int i = 0; i < KBW; ++i)
            if (base + i < kw1) mv_block<FMT, KBW, RL>(r, i, base + i, kb0, xs, sxs, acc0, acc1);
    }
}

// LDS layout of k_matvec (floats), with P = per_split rounded up to 4 blocks:
//   red [512] | misc [64] | xs [P*BK] | sxs [P] | zero [4] | tmp [...]
// xs/sxs hold the input slice: floats and per-block sums (F32, VALU Q4_0)
// or int8 limbs and per-block multipliers (Q4_0 on the matrix cores);
// zero is a 16-byte zero operand.
struct MvLds {
    float* red;
    float* misc;  // 16 slots of 4 floats for block reductions
    float* xs;
    float* sxs;
    float* zero;
    float* tmp;
};

inline size_t mv_lds_floats(int fmt, int per_split, int tmp_floats) {
    const size_t p4 = ((size_t)per_split + 3) & ~(size_t)3;
    return 512 + 64 + p4 * block_cols(fmt) + p4 + 4 + (size_t)tmp_floats;
}
inline size_t mv_lds_bytes(int fmt, int per_split, int tmp_floats) {
    return mv_lds_floats(fmt, per_split, tmp_floats) * sizeof(float);
}

// LDS carve-up of one matvec work item (floats from `lds`).
template <int FMT>
__device__ __forceinline__ MvLds mv_lds(float* lds, int per_split) {
    constexpr int BK = Blk<FMT>::BK;
    const int p4 = (per_split + 3) & ~3;
    MvLds L;
    L.red = lds;
    L.misc = lds + 512;
    L.xs = lds + 576;
    L.sxs = L.xs + p4 * BK;
    L.zero = L.sxs + p4;
    L.tmp = L.zero + 4;
    return L;
}

// One matvec work item: 64*RL rows (one or both halves of 128-row tile
// `tile`, starting at row rbase of it) x column split s of S.  Rows: lane
// (RL 1) or lane and lane+64 (RL 2); the four waves split the split's
// column blocks evenly.  `rt` is the item's row-tile index for the
// epilogue, which wave 0 runs on the summed rows.
//
// A prologue may define load_v<V>() and variant(): the waves whose share of
// the input loads is all out of range (a partial last round of float4
// groups, or no groups at all) take the variant V = 0 that does not issue
// those loads, since each load instruction costs its CU's address unit the
// same time whether or not its offset is in range.  The variant is chosen
// before any load, so each variant's s_waitcnt counts stay exact.
template <class P, class = void>
struct HasSettle : std::false_type {};
template <class P>
struct HasSettle<P, std::void_t<decltype(&P::template settle<1>)>> : std::true_type {};

template <class P, class = void>
struct HasFinishBarriers : std::false_type {};
template <class P>
struct HasFinishBarriers<P, std::void_t<decltype(P::kFinishBarriers)>> : std::true_type {};

template <class P, class = void>
struct HasLoadVariants : std::false_type {};
template <class P>
struct HasLoadVariants<P, std::void_t<decltype(&P::template load_v<0>)>> : std::true_type {};

template <int FMT, int KBW, int RL, int V, class Pro, class Epi>
__device__ __forceinline__ void mv_item_v(const DMat& w, int rt, int s, int S, const Pro& pro, const Epi& epi,
                                          const MvLds& L);

template <int FMT, int KBW, int RL, class Pro, class Epi>
__device__ __forceinline__ void mv_item(const DMat& w, int rt, int s, int S, const Pro& pro, const Epi& epi,
                                        const MvLds& L) {
    if constexpr (HasLoadVariants<Pro>::value) {
        constexpr int BK = Blk<FMT>::BK;
        const int per_split = (w.nblk + S - 1) / S;
        const int kb0 = min(w.nblk, s * per_split), nk = min(w.nblk, kb0 + per_split) - kb0;
        if (pro.variant(kb0 * BK, nk * BK)) mv_item_v<FMT, KBW, RL, 1>(w, rt, s, S, pro, epi, L);
        else mv_item_v<FMT, KBW, RL, 0>(w, rt, s, S, pro, epi, L);
    } else {
        mv_item_v<FMT, KBW, RL, 1>(w, rt, s, S, pro, epi, L);
    }
}

// ------------------------------------------------------------------
// Q4_0 matvec on the int8 matrix cores (v_mfma_i32_16x16x64_i8)
// ------------------------------------------------------------------
// A wave takes 16-row groups; one MFMA pair covers a group's rows x a quad
// of 4 column blocks:
//   B (64 x 16): lane m + 16g holds the 16 code bytes of row m, block
//     4q+g; their low nibbles feed the first MFMA and the high ones the
//     second, each as the int8 16*(q-8) (q ^ 8 is q-8 as a signed nibble);
//   A (16 x 64): row n = 4*b + limb; lane n + 16g holds limb n%4 of
//     elements 0..15 (first MFMA) or 16..31 (second) of block 4q+g when
//     n/4 == g, and zeros otherwise;
//   D[n][m] = 16 * sum_p (q_mp - 8) * limb_{n%4}(X_p) over block 4q + n/4,
//     exact in int32 (|D| < 2^19); lane L holds D[4(L/16)+i][L%16], i.e.
//     row L%16, block 4q + L/16, limbs 0..3.
// Each lane combines its four limbs (X = L0 + 2^7 L1 + 2^14 L2 + 2^21 L3),
// scales by the row's fp16 block scale and the block multiplier, and
// accumulates in f32; the four blocks of a quad meet in a cross-row sum.
template <int QB, int RL>
struct QRegs {
    u32x4 c[RL][QB];     // codes: row (lane & 15) of the row group, block 4q + lane/16
    uint16_t s[RL][QB];  // fp16 scale of the same row and block
};

// Loads of one register batch: quads q0 .. q0+QB-1 (first block kq) of the
// wave's RL row groups; blocks at or past kb1 read zeros.
template <int QB, int RL>
__device__ __forceinline__ void mq_load(QRegs<QB, RL>& r, const DMat& w, const MatViews& v, int tile, int rbase,
                                        int kq, int kb1, int wave) {
    const int lane = threadIdx.x & 63;
    const uint32_t tb = (uint32_t)tile * (uint32_t)w.nblk * TILE_ROWS;
#pragma unroll
    for (int j = 0; j < RL; ++j) {
        const int r16 = rbase + 16 * (wave * RL + j);
#pragma unroll
        for (int i = 0; i < QB; ++i) {
            const int ka = kq + 4 * i + (lane >> 4);
            const uint32_t ea = tb + (uint32_t)ka * TILE_ROWS + (uint32_t)(r16 + (lane & 15));
            r.c[j][i] = v.codes.template u4<CP_NT>(ka < kb1 ? ea * 16u : OOB);
            r.s[j][i] = v.scales.template h1<CP_NT>(ka < kb1 ? ea * 2u : OOB);
        }
    }
}

// The MFMA pairs of quad i of a register batch; bl = first block of the quad
// within the slice.
template <int QB, int RL>
__device__ __forceinline__ void mq_quad(const QRegs<QB, RL>& r, int i, int bl, const MvLds& L, float (&acc)[RL]) {
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const bool act = (n >> 2) == g;
    // 16-byte limb chunks: block * 8 + half * 4 + limb
    const i32x4* lb = (const i32x4*)L.xs + ((bl + g) * 8 + (n & 3));
    const i32x4* zero = (const i32x4*)L.zero;
    const i32x4 b0 = *(act ? lb : zero), b1 = *(act ? lb + 4 : zero);
    const float mq = L.sxs[bl + g];
#pragma unroll
    for (int j = 0; j < RL; ++j) {
        const u32x4 c = r.c[j][i];
        i32x4 alo, ahi;
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // 16 * (q - 8) as int8: q ^ 8 is q - 8 as a signed nibble
            ahi[k] = (int)((c[k] ^ 0x80808080u) & 0xF0F0F0F0u);
            alo[k] = (int)(((c[k] << 4) ^ 0x80808080u) & 0xF0F0F0F0u);
        }
        i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(b0, alo, (i32x4){0, 0, 0, 0}, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(b1, ahi, d, 0, 0, 0);
        // limbs 0+1 and 2+3 exactly in int32 (|D| < 2^19), then in f32
        const int lo01 = d[0] + d[1] * 128, hi23 = d[2] + d[3] * 128;
        const float x = fmaf((float)hi23, 16384.0f, (float)lo01);
        acc[j] = fmaf(x, h2f(r.s[j][i]) * mq, acc[j]);
    }
}

// The MFMA pairs of quads q0 .. min(q0+QB, nq)-1 (quad q: blocks 4q.. of the slice).
template <int QB, int RL>
__device__ __forceinline__ void mq_compute(const QRegs<QB, RL>& r, int q0, int nq, const MvLds& L,
                                           float (&acc)[RL]) {
    if (q0 + QB <= nq) {  // full batch: straight-line (nq is wave-uniform)
#pragma unroll
        for (int i = 0; i < QB; ++i) mq_quad<QB, RL>(r, i, 4 * (q0 + i), L, acc);
    } else {
#pragma unroll
        for (int i = 0; i < QB; ++i)
            if (q0 + i < nq) mq_quad<QB, RL>(r, i, 4 * (q0 + i), L, acc);
    }
}

// One Q4_0 work item on the matrix cores (same contract as mv_item_v): wave
// w takes row groups w*RL .. w*RL+RL-1 over all of the split's blocks, in
// register batches of QB quads.
template <int QB, int RL, int V, class Pro, class Epi>
__device__ __forceinline__ void mq_item_v(const DMat& w, int rt, int s, int S, const Pro& pro, const Epi& epi,
                                          const MvLds& L) {
    const int tile = RL == 2 ? rt : rt >> 1, rbase = RL == 2 ? 0 : (rt & 1) * 64;
    const int nb = w.nblk;
    const int per_split = (nb + S - 1) / S;
    // uniform: readfirstlane as in mv_item_valu
    const int kb0 = __builtin_amdgcn_readfirstlane(min(nb, s * per_split));
    const int kb1 = __builtin_amdgcn_readfirstlane(min(nb, kb0 + per_split));
    const int nk = kb1 - kb0, nq = (nk + 3) >> 2;
    const int wave = wave_id(), lane = threadIdx.x & 63;

    GH_MARK(0);
    typename Pro::Regs pr;
    if constexpr (HasLoadVariants<Pro>::value) pro.template load_v<V>(pr, kb0 * 32, nk * 32);
    else pro.load(pr, kb0 * 32, nk * 32);
    typename Epi::Regs er;
    epi.load(er);
    __builtin_amdgcn_sched_barrier(0);
    if (w.order_in) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const MatViews mv(w);
    QRegs<QB, RL> r;
    mq_load<QB, RL>(r, w, mv, tile, rbase, kb0, kb1, wave);
    __builtin_amdgcn_sched_barrier(0);
    pro.template finish<FMT_Q4M>(L, pr, kb0 * 32, nk * 32);
    if (threadIdx.x < 4) L.zero[threadIdx.x] = 0.0f;
    GH_MARK(1);
    __syncthreads();
    GH_MARK(2);
    float acc[RL];
#pragma unroll
    for (int j = 0; j < RL; ++j) acc[j] = 0.0f;
    mq_compute<QB, RL>(r, 0, nq, L, acc);
    for (int q0 = QB; q0 < nq; q0 += QB) {
        mq_load<QB, RL>(r, w, mv, tile, rbase, kb0 + 4 * q0, kb1, wave);
        mq_compute<QB, RL>(r, q0, nq, L, acc);
    }
    GH_MARK(3);
    // sum the four blocks of each row; lane m < 16 then holds row m
#pragma unroll
    for (int j = 0; j < RL; ++j) {
        acc[j] += __shfl_xor(acc[j], 32, 64);
        acc[j] += __shfl_xor(acc[j], 16, 64);
    }
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < RL; ++j) L.red[16 * (wave * RL + j) + lane] = acc[j];
    }
    __syncthreads();
    GH_MARK(4);
    if (wave == 0) {
        const float y0 = L.red[lane], y1 = RL == 2 ? L.red[64 + lane] : 0.0f;
        epi.template run<RL>(L, er, rt, tile * TILE_ROWS + rbase + lane, s, y0, y1);
    }
    GH_MARK(5);
    GH_MARK_END();
}

template <int FMT, int KBW, int RL, int V, class Pro, class Epi>
__device__ __forceinline__ void mv_item_valu(const DMat& w, int rt, int s, int S, const Pro& pro, const Epi& epi,
                                             const MvLds& L);

template <int FMT, int KBW, int RL, int V, class Pro, class Epi>
__device__ __forceinline__ void mv_item_v(const DMat& w, int rt, int s, int S, const Pro& pro, const Epi& epi,
                                          const MvLds& L) {
    if constexpr (FMT == FMT_Q4M) {
        mq_item_v<KBW, RL, V>(w, rt, s, S, pro, epi, L);
    } else {
        mv_item_valu<FMT, KBW, RL, V>(w, rt, s, S, pro, epi, L);
    }
}

// One work item with the dot products on the VALU (F32, Q4_0).
template <int FMT, int KBW, int RL, int V, class Pro, class Epi>
__device__ __forceinline__ void mv_item_valu(const DMat& w, int rt, int s, int S, const Pro& pro, const Epi& epi,
                                             const MvLds& L) {
    constexpr int BK = Blk<FMT>::BK;
    const int tile = RL == 2 ? rt : rt >> 1, rbase = RL == 2 ? 0 : (rt & 1) * 64;
    const int nb = w.nblk;
    const int per_split = (nb + S - 1) / S;
    // uniform; the readfirstlane keeps the split bounds, and so the buffer
    // bases and loop bounds derived from them, in SGPRs (without it some
    // instances compute them on the VALU and wrap loads in waterfall loops)
    const int kb0 = __builtin_amdgcn_readfirstlane(min(nb, s * per_split));
    const int kb1 = __builtin_amdgcn_readfirstlane(min(nb, kb0 + per_split));
    const int nk = kb1 - kb0;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int kw0 = kb0 + (nk * wave >> 2), kw1 = kb0 + (nk * (wave + 1) >> 2);

    // 1. the prologue's input loads go out first (they are waited on first),
    // 2. then the epilogue's and the weights of the first register batch,
    // 3. the prologue builds the input slice [kb0*BK, kb1*BK) in LDS.
    GH_MARK(0);
    typename Pro::Regs pr;
    if constexpr (HasLoadVariants<Pro>::value) pro.template load_v<V>(pr, kb0 * BK, nk * BK);
    else pro.load(pr, kb0 * BK, nk * BK);
    typename Epi::Regs er;
    epi.load(er);
    // the scheduler may not interleave the three groups: a prologue add
    // hoisted above a weight load would make that load wait for the inputs
    __builtin_amdgcn_sched_barrier(0);
    if (w.order_in) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const MatViews mv(w);
    WRegs<FMT, KBW> r;
    mv_load<FMT, KBW, RL>(r, w, mv, tile, rbase, kw0, kw1);
    __builtin_amdgcn_sched_barrier(0);
    pro.template finish<FMT>(L, pr, kb0 * BK, nk * BK);
    GH_MARK(1);
    __syncthreads();
    GH_MARK(2);
    // 4. dot products
    float acc0 = 0.0f, acc1 = 0.0f;
    mv_compute<FMT, KBW, RL>(r, kw0, kw1, kb0, L.xs, L.sxs, acc0, acc1);
    for (int base = kw0 + KBW; base < kw1; base += KBW) {
        mv_load<FMT, KBW, RL>(r, w, mv, tile, rbase, base, kw1);
        mv_compute<FMT, KBW, RL>(r, base, kw1, kb0, L.xs, L.sxs, acc0, acc1);
    }
    // 5. reduce the four waves; wave 0 finishes the item
    GH_MARK(3);
    L.red[wave * TILE_ROWS + lane] = acc0;
    if (RL == 2) L.red[wave * TILE_ROWS + 64 + lane] = acc1;
    __syncthreads();
    GH_MARK(4);
    if (wave == 0) {
        const float y0 = (L.red[lane] + L.red[TILE_ROWS + lane]) + (L.red[2 * TILE_ROWS + lane] + L.red[3 * TILE_ROWS + lane]);
        float y1 = 0.0f;
        if (RL == 2)
            y1 = (L.red[64 + lane] + L.red[TILE_ROWS + 64 + lane]) +
                 (L.red[2 * TILE_ROWS + 64 + lane] + L.red[3 * TILE_ROWS + 64 + lane]);
        epi.template run<RL>(L, er, rt, tile * TILE_ROWS + rbase + lane, s, y0, y1);
    }
    GH_MARK(5);
    GH_MARK_END();
}

// NI work items of one column split per workgroup of NI x 4 waves: waves
// 0-3 build the split's input slice once for all NI items and take item
// NI*q, waves 4i .. 4i+3 take item NI*q + i and meet the prologue's
// barriers (Pro::kFinishBarriers of them) without issuing its loads.  A CU
// then runs one prologue where NI 4-wave workgroups would run NI; the
// prologue is what bounds these latency-bound items.
template <int FMT, int KBW, int RL, int V, class Pro, class Epi>
__device__ __forceinline__ void mv_item_multi_v(const DMat& w, int it, int s, int S, const Pro& pro, const Epi& epi,
                                                const MvLds& L, float* red) {
    constexpr int BK = Blk<FMT>::BK;
    const int lead = wave_id() < 4, wave = wave_id() & 3, lane = threadIdx.x & 63;
    const int tile = RL == 2 ? it : it >> 1, rbase = RL == 2 ? 0 : (it & 1) * 64;
    const bool live = tile < w.tiles;
    const int nb = w.nblk;
    const int per_split = (nb + S - 1) / S;
    // uniform: readfirstlane as in mv_item_valu
    const int kb0 = __builtin_amdgcn_readfirstlane(min(nb, s * per_split));
    const int kb1 = __builtin_amdgcn_readfirstlane(min(nb, kb0 + per_split));
    const int nk = kb1 - kb0;
    const int kw0 = kb0 + (nk * wave >> 2);
    // an item past the last row tile loads nothing and writes nothing
    const int kw1 = live ? kb0 + (nk * (wave + 1) >> 2) : kw0;
    GH_MARK(0);
    typename Pro::Regs pr;
    if (lead) {
        if constexpr (HasLoadVariants<Pro>::value) pro.template load_v<V>(pr, kb0 * BK, nk * BK);
        else pro.load(pr, kb0 * BK, nk * BK);
    }
    typename Epi::Regs er;
    epi.load(er);
    __builtin_amdgcn_sched_barrier(0);
    if (w.order_in) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const MatViews mv(w);
    WRegs<FMT, KBW> r;
    mv_load<FMT, KBW, RL>(r, w, mv, tile, rbase, kw0, kw1);
    __builtin_amdgcn_sched_barrier(0);
    if (lead) {
        pro.template finish<FMT>(L, pr, kb0 * BK, nk * BK);
    } else {
#pragma unroll
        for (int i = 0; i < Pro::kFinishBarriers; ++i) __syncthreads();
    }
    GH_MARK(1);
    __syncthreads();
    GH_MARK(2);
    float acc0 = 0.0f, acc1 = 0.0f;
    mv_compute<FMT, KBW, RL>(r, kw0, kw1, kb0, L.xs, L.sxs, acc0, acc1);
    for (int base = kw0 + KBW; base < kw1; base += KBW) {
        mv_load<FMT, KBW, RL>(r, w, mv, tile, rbase, base, kw1);
        mv_compute<FMT, KBW, RL>(r, base, kw1, kb0, L.xs, L.sxs, acc0, acc1);
    }
    GH_MARK(3);
    red[wave * TILE_ROWS + lane] = acc0;
    if (RL == 2) red[wave * TILE_ROWS + 64 + lane] = acc1;
    __syncthreads();
    GH_MARK(4);
    if (wave == 0 && live) {
        const float y0 = (red[lane] + red[TILE_ROWS + lane]) + (red[2 * TILE_ROWS + lane] + red[3 * TILE_ROWS + lane]);
        float y1 = 0.0f;
        if (RL == 2)
            y1 = (red[64 + lane] + red[TILE_ROWS + 64 + lane]) + (red[2 * TILE_ROWS + 64 + lane] + red[3 * TILE_ROWS + 64 + lane]);
        epi.template run<RL>(L, er, it, tile * TILE_ROWS + rbase + lane, s, y0, y1);
    }
    GH_MARK(5);
    GH_MARK_END();
}

// The same on the matrix cores (mq_item_v's dot products): the lead waves'
// prologue builds the int8 limbs of the slice once for both items.
template <int QB, int RL, int V, class Pro, class Epi>
__device__ __forceinline__ void mq_item_multi_v(const DMat& w, int it, int s, int S, const Pro& pro, const Epi& epi,
                                                const MvLds& L, float* red) {
    const int lead = wave_id() < 4, wave = wave_id() & 3, lane = threadIdx.x & 63;
    const int tile = RL == 2 ? it : it >> 1, rbase = RL == 2 ? 0 : (it & 1) * 64;
    const bool live = tile < w.tiles;
    const int nb = w.nblk;
    const int per_split = (nb + S - 1) / S;
    // uniform: readfirstlane as in mv_item_valu
    const int kb0 = __builtin_amdgcn_readfirstlane(min(nb, s * per_split));
    const int kb1 = __builtin_amdgcn_readfirstlane(min(nb, kb0 + per_split));
    const int nk = kb1 - kb0;
    // an item past the last row tile loads nothing and writes nothing
    const int kl = live ? kb1 : kb0, nq = live ? (nk + 3) >> 2 : 0;
    GH_MARK(0);
    typename Pro::Regs pr;
    if (lead) {
        if constexpr (HasLoadVariants<Pro>::value) pro.template load_v<V>(pr, kb0 * 32, nk * 32);
        else pro.load(pr, kb0 * 32, nk * 32);
    }
    typename Epi::Regs er;
    epi.load(er);
    __builtin_amdgcn_sched_barrier(0);
    if (w.order_in) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const MatViews mv(w);
    QRegs<QB, RL> r;
    mq_load<QB, RL>(r, w, mv, tile, rbase, kb0, kl, wave);
    __builtin_amdgcn_sched_barrier(0);
    if (lead) {
        pro.template finish<FMT_Q4M>(L, pr, kb0 * 32, nk * 32);
        if (threadIdx.x < 4) L.zero[threadIdx.x] = 0.0f;
    } else {
#pragma unroll
        for (int i = 0; i < Pro::kFinishBarriers; ++i) __syncthreads();
    }
    GH_MARK(1);
    __syncthreads();
    GH_MARK(2);
    float acc[RL];
#pragma unroll
    for (int j = 0; j < RL; ++j) acc[j] = 0.0f;
    mq_compute<QB, RL>(r, 0, nq, L, acc);
    for (int q0 = QB; q0 < nq; q0 += QB) {
        mq_load<QB, RL>(r, w, mv, tile, rbase, kb0 + 4 * q0, kl, wave);
        mq_compute<QB, RL>(r, q0, nq, L, acc);
    }
    GH_MARK(3);
    // sum the four blocks of each row; lane m < 16 then holds row m
#pragma unroll
    for (int j = 0; j < RL; ++j) {
        acc[j] += __shfl_xor(acc[j], 32, 64);
        acc[j] += __shfl_xor(acc[j], 16, 64);
    }
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < RL; ++j) red[16 * (wave * RL + j) + lane] = acc[j];
    }
    __syncthreads();
    GH_MARK(4);
    if (wave == 0 && live) {
        const float y0 = red[lane], y1 = RL == 2 ? red[64 + lane] : 0.0f;
        epi.template run<RL>(L, er, it, tile * TILE_ROWS + rbase + lane, s, y0, y1);
    }
    GH_MARK(5);
    GH_MARK_END();
}

// grid = ceil(items / NI) x S, NI x 256 threads; LDS: k_matvec's carve-up
// (red_off floats), then the reduction areas of items 1 .. NI-1 (512 floats
// each)
template <int FMT, int KBW, int RL, int NI, class Pro, class Epi>
__global__ __launch_bounds__(NI * NT) void k_matvec_multi(DMat w, int S, Pro pro, Epi epi, int red_off) {
    extern __shared__ float lds[];
    const int per_split = (w.nblk + S - 1) / S;
    const MvLds L = mv_lds<FMT>(lds, per_split);
    const int i = wave_id() >> 2;
    float* red = i == 0 ? L.red : lds + red_off + (i - 1) * 512;
    const int it = blockIdx.x / S * NI + i, s = blockIdx.x % S;
    auto item = [&](auto v) {
        constexpr int V = decltype(v)::value;
        if constexpr (FMT == FMT_Q4M) mq_item_multi_v<KBW, RL, V>(w, it, s, S, pro, epi, L, red);
        else mv_item_multi_v<FMT, KBW, RL, V>(w, it, s, S, pro, epi, L, red);
    };
    if constexpr (HasLoadVariants<Pro>::value) {
        constexpr int BK = Blk<FMT>::BK;
        const int kb0 = min(w.nblk, s * per_split), nk = min(w.nblk, kb0 + per_split) - kb0;
        if (i == 0 && pro.variant(kb0 * BK, nk * BK)) item(std::integral_constant<int, 1>{});
        else item(std::integral_constant<int, 0>{});
    } else {
        item(std::integral_constant<int, 1>{});
    }
}

// One workgroup per work item: grid = row tiles x S.
template <int FMT, int KBW, int RL, class Pro, class Epi>
__global__ __launch_bounds__(NT) void k_matvec(DMat w, int S, Pro pro, Epi epi) {
    extern __shared__ float lds[];
    const int per_split = (w.nblk + S - 1) / S;
    mv_item<FMT, KBW, RL>(w, blockIdx.x / S, blockIdx.x % S, S, pro, epi, mv_lds<FMT>(lds, per_split));
}

constexpr int RG16_QB = 14;  // quads per register batch: a wave's share of 224 blocks in one batch

// Q4_0 matvec for matrices of few rows (the op level's 1536 x 1152): one
// workgroup per group of R rows (16, 8 or 4; R divides 128) over all the
// columns, on the matrix cores.  Lane l's MFMA row is row (l & 15) of the
// group; rows past R load nothing (their products are zeros and are not
// stored).  The four waves split the quads and add their dot products in
// LDS: one kernel and no split partials, where 64-row items need up to 16
// column splits and a partial-sum kernel to fill the device.  As the step's
// qkv (the residual prologue then lays out the whole vector once per 16
// rows, and attention reads one vector instead of 8 split partials) it was
// slower on MI355X: 1B 1673 -> 1598 tok/s, 4B 796 -> 768.
template <class Pro, class Epi>
__global__ __launch_bounds__(NT) void k_mq_rows(DMat w, int R, Pro pro, Epi epi) {
    extern __shared__ float lds[];
    const int nb = w.nblk;
    const MvLds L = mv_lds<FMT_Q4M>(lds, nb);
    const int row0 = blockIdx.x * R, tile = row0 / TILE_ROWS, rt0 = row0 % TILE_ROWS;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int nq = (nb + 3) >> 2;
    const int q_lo = __builtin_amdgcn_readfirstlane(nq * wave >> 2);
    const int q_hi = __builtin_amdgcn_readfirstlane(nq * (wave + 1) >> 2);
    const int kb1 = min(nb, 4 * q_hi);  // blocks of later waves read zeros
    const bool row_ok = (lane & 15) < R;
    typename Pro::Regs pr;
    pro.load(pr, 0, nb * 32);
    typename Epi::Regs er;
    epi.load(er);
    __builtin_amdgcn_sched_barrier(0);
    if (w.order_in) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const MatViews mv(w);
    const uint32_t tb = (uint32_t)tile * (uint32_t)nb * TILE_ROWS + (uint32_t)(rt0 + (lane & 15));
    QRegs<RG16_QB, 1> r;
    auto load = [&](int kq) {
#pragma unroll
        for (int i = 0; i < RG16_QB; ++i) {
            const int ka = kq + 4 * i + (lane >> 4);
            const uint32_t ea = tb + (uint32_t)ka * TILE_ROWS;
            const bool ok = row_ok && ka < kb1;
            r.c[0][i] = mv.codes.template u4<CP_NT>(ok ? ea * 16u : OOB);
            r.s[0][i] = mv.scales.template h1<CP_NT>(ok ? ea * 2u : OOB);
        }
    };
    load(4 * q_lo);
    __builtin_amdgcn_sched_barrier(0);
    pro.template finish<FMT_Q4M>(L, pr, 0, nb * 32);
    if (threadIdx.x < 4) L.zero[threadIdx.x] = 0.0f;
    __syncthreads();
    float acc[1] = {0.0f};
    mq_compute<RG16_QB, 1>(r, q_lo, q_hi, L, acc);
    for (int q0 = q_lo + RG16_QB; q0 < q_hi; q0 += RG16_QB) {
        load(4 * q0);
        mq_compute<RG16_QB, 1>(r, q0, q_hi, L, acc);
    }
    // the four blocks of each row, then the four waves; lane m < R holds row m
    acc[0] += __shfl_xor(acc[0], 32, 64);
    acc[0] += __shfl_xor(acc[0], 16, 64);
    if (lane < 16) L.red[16 * wave + lane] = acc[0];
    __syncthreads();
    if (wave == 0 && lane < R) {
        const float y = (L.red[lane] + L.red[16 + lane]) + (L.red[32 + lane] + L.red[48 + lane]);
        epi.template run<1>(L, er, blockIdx.x, row0 + lane, 0, y, 0.0f);
    }
}

// ------------------------------------------------------------------
// prologues: load() issues the global loads of the input, finish<FMT>()
// builds xs[0 .. n) = input[c0 .. c0+n) in LDS through emit_x4
// ------------------------------------------------------------------
__device__ __forceinline__ float4 fma4(float w, float4 o, float4 acc) {
    return make_float4(acc.x + w * o.x, acc.y + w * o.y, acc.z + w * o.z, acc.w + w * o.w);
}
__device__ __forceinline__ float4 f4z() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// 7-bit field of X starting at bit 7*l, as an int8 byte (l = 3: the signed top limb)
template <int l>
__device__ __forceinline__ uint32_t limb_byte(int X) {
    return __builtin_amdgcn_ubfe((uint32_t)X, 7 * l, l == 3 ? 8 : 7);
}

// Store float4 group gi (< ng) of the input slice.  For Q4_0 the 8 groups of
// a 32-element block sit in 8 consecutive lanes.  Called by every thread of
// the workgroup with gi = base + threadIdx.x (base uniform, a multiple of NT).
//
// FMT_Q4M (Q4_0 on the matrix cores): the block's lanes find its largest |x| < 2^e and
// write X = rint(x * 2^(27-e)) (|X| <= 2^27; the rounding error is at most
// 2^(e-28), i.e. 2^-27 of the block's largest element) as four int8 limbs
//   X = L0 + 2^7 L1 + 2^14 L2 + 2^21 L3   (L0..L2 in [0, 127], L3 in [-64, 64])
// at limbs[block][half][limb][16 bytes] (byte p: element 16*half + p), and
// the block multiplier 2^(e-31) = 2^-(27-e) * 2^-4 (the 4 undoes the x16 of
// the signed nibbles; NaN when the block holds an Inf or NaN, so it
// propagates).  Groups from ng up to the next 4-block boundary are zeros.
//
// FMT_Q4 (Q4_0 on the VALU): the lanes sum the block (sxs, for the -8 * sum(x) term)
// and scale elements 16..31 by 1/16 (exact) for the high-nibble products of
// dot_q4_word.
template <int FMT>
__device__ __forceinline__ void emit_x4(const MvLds& L, int gi, int ng, float4 v) {
    if constexpr (FMT == FMT_Q4M) {
        const int ngp = (ng + 31) & ~31;
        if (__builtin_amdgcn_readfirstlane(gi - (int)(threadIdx.x & 63)) >= ngp) return;  // no group of this wave
        if (gi >= ng) v = f4z();
        // an Inf or NaN element makes the block maximum Inf (fmaxf drops NaNs)
        const float fin = (v.x - v.x) + (v.y - v.y) + (v.z - v.z) + (v.w - v.w);
        const float a4 = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        const float amax = group_max8(fin == 0.0f ? a4 : INFINITY);
        const int e = __builtin_amdgcn_frexp_expf(amax);  // amax < 2^e (0 for 0)
        const int sh = 27 - e;
        const int X0 = (int)rintf(ldexpf(v.x, sh)), X1 = (int)rintf(ldexpf(v.y, sh));
        const int X2 = (int)rintf(ldexpf(v.z, sh)), X3 = (int)rintf(ldexpf(v.w, sh));
        auto pack = [&](auto l) {
            constexpr int L_ = decltype(l)::value;
            return limb_byte<L_>(X0) | limb_byte<L_>(X1) << 8 | limb_byte<L_>(X2) << 16 | limb_byte<L_>(X3) << 24;
        };
        if (gi < ngp) {
            uint32_t* d = (uint32_t*)L.xs + (gi >> 3) * 32 + ((gi & 7) >> 2) * 16 + (gi & 3);
            d[0] = pack(std::integral_constant<int, 0>{});
            d[4] = pack(std::integral_constant<int, 1>{});
            d[8] = pack(std::integral_constant<int, 2>{});
            d[12] = pack(std::integral_constant<int, 3>{});
            if ((gi & 7) == 0) L.sxs[gi >> 3] = amax <= 3.4028235e38f ? ldexpf(1.0f, e - 31) : __builtin_nanf("");
        }
    } else if constexpr (FMT == FMT_Q4) {
        const float bs = group_sum<8>((v.x + v.y) + (v.z + v.w));
        if ((gi & 7) >= 4) v = make_float4(v.x * 0.0625f, v.y * 0.0625f, v.z * 0.0625f, v.w * 0.0625f);
        if (gi < ng) {
            ((float4*)L.xs)[gi] = v;
            if ((gi & 7) == 0) L.sxs[gi >> 3] = bs;
        }
    } else {
        if (gi < ng) ((float4*)L.xs)[gi] = v;
    }
}

// sum over s < S of the float4 group g of part[s][ld]: all loads issued
// before the first add, so the sum costs one round trip.
__device__ __forceinline__ float4 sum_splits4(const float* part, int S, int ld, int g) {
    float4 v[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; ++s) v[s] = s < S ? ((const float4*)(part + (size_t)s * ld))[g] : f4z();
    float4 r = v[0];
#pragma unroll
    for (int s = 1; s < MAXS; ++s)
        if (s < S) r = r + v[s];
    return r;
}

// A vector already in global memory (2 float4 per thread prefetched).
// (no kFinishBarriers: the LM head measured slower with paired items, 28 ->
// 31 us on 1B, its many one-item workgroups already overlapping each
// other's prologues with streaming)
struct ProPlain {
    const float* x;
    struct Regs {
        float4 v[2];
    };
    __device__ void load(Regs& r, int c0, int n) const {
        const BufView X(x + c0, (size_t)n * 4);
#pragma unroll
        for (int k = 0; k < 2; ++k) r.v[k] = X.f4(16u * (threadIdx.x + k * NT));
    }
    template <int FMT>
    __device__ void finish(const MvLds& L, Regs& r, int c0, int n) const {
        const int ng = n >> 2;
#pragma unroll
        for (int k = 0; k < 2; ++k)
            if (k * NT < ng) emit_x4<FMT>(L, threadIdx.x + k * NT, ng, r.v[k]);
        for (int base = 2 * NT; base < ng; base += NT) {
            const int gi = base + threadIdx.x;
            emit_x4<FMT>(L, gi, ng, gi < ng ? ((const float4*)(x + c0))[gi] : f4z());
        }
    }
};

// Residual stream update followed by an RMSNorm (MG = float4 groups per thread):
//   x  = base + postnorm(sum_s part_s)        (residual add, TBG:305-343 / TBG:413-444)
//     or E[token] * sqrt(H) for layer 0        (src/Gemma/Model.hs:1346-1361)
//   xs = norm(x) with w_norm                   (TBG:110, MLP.hs:507-622, RMSNorm.hs:343-386)
// Thread t, round k holds float4 group (c0/4 + t + k*256) mod H/4 of the
// vector: the groups are rotated so that each thread's first groups are the
// workgroup's own slice, which it then lays out from registers.  Both RMS
// values come from one block reduction of four sums: with d the split sum,
// e = d * (1 + w_post) and c = 1/rms(d), x = b + c * e, so
//   sum x^2 = sum b^2 + 2 c sum b e + c^2 sum e^2.
// Block 0 stores x to x_out and, when asked, to layer_out_row.  All split
// partials (S <= MAXS), the residual and both norm weights are loaded in one
// round trip, as straight-line buffer loads (absent splits read zeros).
// EMB: layer 0 (x is the token's embedding row); a separate instance, so
// that in the other layers the compiler keeps every prologue load ahead of
// the weight loads (a runtime branch lets it sink them into the branch).
struct ResidFields {
    int from_embedding;  // must equal EMB
    DMat embd;
    const StepState* st;
    float escale;
    const float* base;
    const float* part;
    int S, ld;
    const float* w_post;  // nullable
    const float* w_norm;
    float eps;
    int zc, H;
    float* x_out;          // nullable
    float* layer_out_row;  // nullable
};

template <int MG, bool EMB = false>
struct ProResid : ResidFields {
    static constexpr int kFinishBarriers = 1;  // finish<>() holds one __syncthreads
    struct Regs {
        float4 pv[MAXS][MG];
        float4 bv[MG], wp[MG];
        float4 wn[MG];  // norm weights of this thread's groups of the slice
    };
    // group of thread t in round k, rotated to start at the slice's first group
    __device__ static int group(int g0, int t, int k, int NG) {
        const int g = g0 + t + k * NT;
        return g >= NG ? g - NG : g;
    }
    // variant 1: this wave has groups in the last round of the H/4 groups
    __device__ int variant(int, int) const { return wave_id() * 64 + (MG - 1) * NT < (H >> 2); }
    template <int V>
    __device__ void load_v(Regs& r, int c0, int n) const {
        constexpr int RR = MG > 1 && V == 0 ? MG - 1 : MG;  // rounds this wave loads
        const int NG = H >> 2, tid = threadIdx.x, g0 = c0 >> 2;
        const BufView WN(w_norm + c0, (size_t)n * 4);
#pragma unroll
        for (int k = 0; k < MG; ++k) r.wn[k] = k < RR ? WN.f4(16u * (tid + k * NT)) : f4z();
        if constexpr (!EMB) {
            const BufView P(part, (size_t)S * ld * 4), B(base, (size_t)H * 4), WP(w_post, w_post ? (size_t)H * 4 : 0);
#pragma unroll
            for (int k = 0; k < MG; ++k) {
                const int g = group(g0, tid, k, NG);
                const bool in = tid + k * NT < NG;
                const uint32_t o = in ? 16u * g : OOB;
                r.bv[k] = k < RR ? B.f4(o) : f4z();
                r.wp[k] = k < RR ? WP.f4(o) : f4z();
#pragma unroll
                for (int s = 0; s < MAXS; ++s)
                    r.pv[s][k] = k < RR ? P.f4(in ? 4u * (uint32_t)(s * ld) + 16u * g : OOB) : f4z();
            }
        }
    }
    __device__ void load(Regs& r, int c0, int n) const { load_v<1>(r, c0, n); }
    template <int FMT>
    __device__ void finish(const MvLds& L, Regs& r, int c0, int n) const {
        const int NG = H >> 2, tid = threadIdx.x, g0 = c0 >> 2;
        float4 xv[MG];
        float inv;  // 1 / rms(x)
        if constexpr (EMB) {
            // the host validates tokens; the clamp keeps a corrupted state in bounds
            const int tok = min(max(st->token, 0), embd.rows - 1);
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < MG; ++k) {
                xv[k] = f4z();
                if (tid + k * NT < NG) {
                    const float4 e = dq_elem4(embd, tok, 4 * group(g0, tid, k, NG));
                    xv[k] = make_float4(e.x * escale, e.y * escale, e.z * escale, e.w * escale);
                }
                ss += dot4(xv[k], xv[k]);
            }
            inv = 1.0f / sqrtf(block_sum(ss, L.misc) / (float)H + eps);
        } else {
            // absent splits and groups past H were read as zeros
            float4 dv[MG], ev[MG];
            float dd = 0.0f, bb = 0.0f, be = 0.0f, ee = 0.0f;
#pragma unroll
            for (int k = 0; k < MG; ++k) {
                dv[k] = r.pv[0][k];
#pragma unroll
                for (int s = 1; s < MAXS; ++s) dv[k] = dv[k] + r.pv[s][k];
                const float4 w1 = zc ? make_float4(1.0f + r.wp[k].x, 1.0f + r.wp[k].y, 1.0f + r.wp[k].z, 1.0f + r.wp[k].w)
                                     : r.wp[k];
                ev[k] = w_post ? make_float4(dv[k].x * w1.x, dv[k].y * w1.y, dv[k].z * w1.z, dv[k].w * w1.w) : dv[k];
                dd += dot4(dv[k], dv[k]);
                bb += dot4(r.bv[k], r.bv[k]);
                be += dot4(r.bv[k], ev[k]);
                ee += dot4(ev[k], ev[k]);
            }
            const float4 t = block_sum4(make_float4(dd, bb, be, ee), L.misc + 16);
            const float c = w_post ? 1.0f / sqrtf(t.x / (float)H + eps) : 1.0f;
            GH_MARK(6);
#pragma unroll
            for (int k = 0; k < MG; ++k) xv[k] = r.bv[k] + (w_post ? norm4i(dv[k], c, r.wp[k], zc) : dv[k]);
            const float sxx = fmaxf(t.y + 2.0f * c * t.z + c * c * t.w, 0.0f);
            inv = 1.0f / sqrtf(sxx / (float)H + eps);
        }
        if (blockIdx.x == 0 && (x_out || layer_out_row)) {
#pragma unroll
            for (int k = 0; k < MG; ++k) {
                if (tid + k * NT < NG) {
                    const int g = group(g0, tid, k, NG);
                    if (x_out) ((float4*)x_out)[g] = xv[k];
                    if (layer_out_row) ((float4*)layer_out_row)[g] = xv[k];
                }
            }
        }
        GH_MARK(7);
        // this thread's groups of the slice are its first ones (rotation)
        const int ng = n >> 2;
#pragma unroll
        for (int k = 0; k < MG; ++k) {
            const int gi = tid + k * NT;
            if (k * NT < ng) emit_x4<FMT>(L, gi, ng, gi < ng ? norm4i(xv[k], inv, r.wn[k], zc) : f4z());
        }
    }
};

// Attention window of the current token.
__host__ __device__ __forceinline__ void attn_window(int pos, int global, int window, int mode, int& pb, int& pe) {
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

constexpr int ATTN_SUB = 32;      // positions per attention sub-chunk
constexpr int ATTN_MAX_NC = 64;   // chunks per kv head

// Chunking of n_pos positions over at most nc workgroups: chunk length is a
// multiple of ATTN_SUB, n_used chunks are non-empty.
__host__ __device__ __forceinline__ void attn_chunks(int n_pos, int nc, int& ch, int& n_used) {
    const int per = (n_pos + nc - 1) / nc;
    ch = (per + ATTN_SUB - 1) / ATTN_SUB * ATTN_SUB;
    n_used = (n_pos + ch - 1) / ch;
}

// O-projection input: merge the split-K attention partials {m[G], l[G],
// o[G][HD]} of every chunk for the slice [c0, c0+n) of o = [nq][hd].
struct ProAttnCombine {
    static constexpr int kFinishBarriers = 1;
    const float* part;
    int pos;  // current position (patched per step with set_pos)
    int nc, G, HD;
    int global, window, mode;
    int n_used;  // chunks of this position, derived on the host
    int nkv;
    __host__ __device__ void set_pos(int p) {
        int pb, pe, ch;
        pos = p;
        attn_window(p, global, window, mode, pb, pe);
        attn_chunks(pe - pb, nc, ch, n_used);
    }
    static constexpr int PRE = 16;  // chunk states loaded by load()
    struct Regs {
        float4 ov[PRE];
        float mj, lj;
    };
    // variant 1: this wave holds column groups of the slice
    __device__ int variant(int, int n) const { return wave_id() * 64 < (n >> 2); }
    template <int V>
    __device__ void load_v(Regs& r, int c0, int n) const {
        const int stride = G * (HD + 2), tid = threadIdx.x;
        const BufView P(part, (size_t)nkv * nc * stride * 4);
        // this thread's column group (one per thread up to 1024 columns)
        const int c = c0 + 4 * tid, h = c / HD, d = c % HD;
        const uint32_t ob = 4u * (uint32_t)((h / G) * nc * stride + 2 * G + (h % G) * HD + d);
        const bool in = tid < (n >> 2);
#pragma unroll
        for (int j = 0; j < PRE; ++j)
            r.ov[j] = V ? P.f4(in && j < n_used ? ob + 4u * (uint32_t)(j * stride) : OOB) : f4z();
        // (m, l) of chunk j = lane for head h0 + wave
        const int h0 = c0 / HD, nh = (c0 + n - 1) / HD - h0 + 1;
        const int hh = tid >> 6, j = tid & 63;
        const bool ok = hh < nh && j < n_used;
        const int hg = h0 + hh;
        const uint32_t bj = 4u * (uint32_t)(((hg / G) * nc + j) * stride + hg % G);
        r.mj = ok ? P.f1(bj) : -INFINITY;
        r.lj = P.f1(ok ? bj + 4u * G : OOB);
    }
    __device__ void load(Regs& r, int c0, int n) const { load_v<1>(r, c0, n); }
    template <int FMT>
    __device__ void finish(const MvLds& L, Regs& r, int c0, int n) const {
        const int stride = G * (HD + 2), tid = threadIdx.x;
        const int h0 = c0 / HD, nh = (c0 + n - 1) / HD - h0 + 1;
        float* wts = L.tmp;  // [nh][ATTN_MAX_NC] merge weights exp(m_j - M) / sum_j l_j exp(m_j - M)
        const int j = tid & 63;
        auto weights = [&](int hh, float mj, float lj) {
            const float M = wave_max(mj);
            const float e = j < n_used ? expf(mj - M) : 0.0f;
            const float den = wave_sum(lj * e);
            wts[hh * ATTN_MAX_NC + j] = e / den;
        };
        // straight-line first pass on the prefetched (m, l); heads beyond the
        // slice's first four (slices of more than 4 heads) load theirs here
        const int w0 = wave_id();
        if (w0 < nh) weights(w0, r.mj, r.lj);
        for (int hh = w0 + 4; hh < nh; hh += 4) {
            const int hg = h0 + hh;
            const float* bj = part + ((size_t)(hg / G) * nc + j) * stride;
            weights(hh, j < n_used ? bj[hg % G] : -INFINITY, j < n_used ? bj[G + hg % G] : 0.0f);
        }
        __syncthreads();
        const int ng = n >> 2;
        auto group = [&](int gi, const float4* pre) {
            float4 acc = f4z();
            if (gi < ng) {
                const int c = c0 + 4 * gi, h = c / HD, d = c % HD;
                const float* pbase = part + (size_t)(h / G) * nc * stride + 2 * G + (h % G) * HD + d;
                const float* wv = wts + (h - h0) * ATTN_MAX_NC;
                int jj = 0;
                if (pre) {  // chunks 0..PRE-1 were loaded by load() (zeros past n_used)
#pragma unroll
                    for (int q = 0; q < PRE; ++q)
                        if (q < n_used) acc = fma4(wv[q], pre[q], acc);
                    jj = PRE;
                }
                for (; jj < n_used; ++jj) acc = fma4(wv[jj], *(const float4*)(pbase + (size_t)jj * stride), acc);
            }
            emit_x4<FMT>(L, gi, ng, acc);
        };
        group(tid, r.ov);
        for (int base = NT; base < ng; base += NT) group(base + tid, nullptr);
    }
};

// Down-projection input: h = gelu_tanh(sum_s g_s) * sum_s u_s (MLP.hs:384-447).
// The gate/up split partials of the slice are loaded in one round trip:
// gm (1 or 2) float4 groups per thread, register slot i < NS holding split
// i / gm of group i % gm (the host keeps Sg * gm <= NS; NS is 3, 4 or 8, so
// no load instruction is spent on absent splits beyond the next of those).
template <int NS>
struct ProGeglu {
    static constexpr int kFinishBarriers = 0;
    const float* part_gu;
    int Sg, ld_g, up_off;
    int gm;
    struct Regs {
        float4 g[NS], u[NS];
    };
    __device__ void load(Regs& r, int c0, int n) const {
        const BufView P(part_gu, (size_t)Sg * ld_g * 4);
        const int ng = n >> 2;
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int s = gm == 2 ? i >> 1 : i, gi = threadIdx.x + (gm == 2 ? (i & 1) * NT : 0);
            const bool ok = s < Sg && gi < ng;
            const uint32_t o = 4u * (uint32_t)(s * ld_g + c0 + 4 * gi);
            r.g[i] = P.f4(ok ? o : OOB);
            r.u[i] = P.f4(ok ? o + 4u * (uint32_t)up_off : OOB);
        }
    }
    template <int FMT>
    __device__ void finish(const MvLds& L, Regs& r, int c0, int n) const {
        const int ng = n >> 2;
        auto emit = [&](int gi, float4 gs, float4 us) {
            float4 h = f4z();
            if (gi < ng)
                h = make_float4(gelu_tanh(gs.x) * us.x, gelu_tanh(gs.y) * us.y, gelu_tanh(gs.z) * us.z,
                                gelu_tanh(gs.w) * us.w);
            emit_x4<FMT>(L, gi, ng, h);
        };
        if (gm == 1) {
            float4 gs = r.g[0], us = r.u[0];
#pragma unroll
            for (int s = 1; s < NS; ++s) {
                gs = gs + r.g[s];
                us = us + r.u[s];
            }
            emit(threadIdx.x, gs, us);
        } else {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                float4 gs = r.g[k], us = r.u[k];
#pragma unroll
                for (int s = 1; s < NS / 2; ++s) {
                    gs = gs + r.g[2 * s + k];
                    us = us + r.u[2 * s + k];
                }
                if (k * NT < ng) emit(threadIdx.x + k * NT, gs, us);
            }
        }
    }
};

// ------------------------------------------------------------------
// word exchange of the persistent step: a phase publishes its outputs as
// 64-bit words (epoch << 32 | float bits) with relaxed agent-scope stores
// (written through to memory); a consumer polls each word with relaxed
// agent-scope loads (L2 bypassed) until its epoch matches.  A word is
// single-copy atomic, so it validates itself: no fences are needed.  Every
// wait is bounded; on timeout the step's error flag is set and all later
// waits give up at once, so the kernel always finishes.
// ------------------------------------------------------------------
constexpr int XCHG_SPIN = 1 << 18;

// (global address space: vector-memory instructions only, so LDS waits
// never wait for a word in flight)
typedef __attribute__((address_space(1))) uint64_t gword;
__device__ __forceinline__ void st_word(uint64_t* p, uint32_t epoch, float v) {
    __hip_atomic_store((gword*)p, ((uint64_t)epoch << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t ld_word(const uint64_t* p) {
    return __hip_atomic_load((gword*)const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// Input slice already in LDS from the previous item of the same matrix.
struct ProKeep {
    struct Regs {};
    __device__ void load(Regs&, int, int) const {}
    template <int FMT>
    __device__ void finish(const MvLds&, Regs&, int, int) const {}
};

// ------------------------------------------------------------------
// epilogues: load() runs at kernel start (its global loads go out with the
// prologue's); run<RL>() is called by the 64 lanes of wave 0 with the sums
// of rows row0 = (item's first row) + lane and, when RL = 2, row0 + 64.
// No epilogue may use a workgroup barrier.
// ------------------------------------------------------------------
struct EpiPartial {
    float* part;
    int ld;
    struct Regs {};
    __device__ void load(Regs&) const {}
    template <int RL>
    __device__ void run(const MvLds&, const Regs&, int, int row0, int s, float y0, float y1) const {
        part[(size_t)s * ld + row0] = y0;
        if (RL == 2) part[(size_t)s * ld + row0 + 64] = y1;
    }
};

struct EpiOut {
    float* y;
    int rows, softcap;
    float cap;
    struct Regs {};
    __device__ void load(Regs&) const {}
    template <int RL>
    __device__ void run(const MvLds&, const Regs&, int, int row0, int, float y0, float y1) const {
        if (row0 < rows) y[row0] = softcap ? cap * tanhf(y0 / cap) : y0;
        if (RL == 2 && row0 + 64 < rows) y[row0 + 64] = softcap ? cap * tanhf(y1 / cap) : y1;
    }
};

// Logits + this item's greedy argmax key (first maximum); the finish kernel
// reduces the per-item keys (no same-address atomics on the step path).
// When sampling, also the item's max logit and sum of exp((l - max) / T).
struct EpiLogits {
    float* logits;  // nullable
    int V;
    unsigned long long* cand;
    StepState* st;
    float* bm;  // per-item max logit (written when sampling)
    float* bs;  // per-item sum of exp((l - max) / T)
    struct Regs {
        float inv_t;
    };
    __device__ void load(Regs& r) const { r.inv_t = st->inv_temp; }
    template <int RL>
    __device__ void run(const MvLds&, const Regs& r, int rt, int row0, int, float y0, float y1) const {
        const int lane = threadIdx.x & 63;
        const bool in0 = row0 < V, in1 = RL == 2 && row0 + 64 < V;
        if (logits) {
            if (in0) logits[row0] = y0;
            if (in1) logits[row0 + 64] = y1;
        }
        if ((in0 && isnan(y0)) || (in1 && isnan(y1))) atomicOr(&st->nan_flag, 1);
        // first maximum: the wave's max value, then the lowest row holding it
        // (every row of the lower half precedes every row of the upper half)
        const float v0 = in0 ? y0 : -INFINITY, v1 = in1 ? y1 : -INFINITY;
        const float M = wave_max(fmaxf(v0, v1));
        const unsigned long long b0 = __ballot(in0 && v0 == M);
        const unsigned long long b1 = __ballot(in1 && v1 == M);
        const int first = row0 - lane;
        unsigned long long key = 0ull;
        if (b0) key = argmax_key(M, first + __builtin_ctzll(b0));
        else if (b1) key = argmax_key(M, first + 64 + __builtin_ctzll(b1));
        if (lane == 0) cand[rt] = key;
        if (r.inv_t > 0.0f) {  // temperature sampling: softmax statistics of the item's rows
            const float e = (in0 ? expf((y0 - M) * r.inv_t) : 0.0f) + (in1 ? expf((y1 - M) * r.inv_t) : 0.0f);
            const float sb = wave_sum(e);
            if (lane == 0) {
                bm[rt] = M;
                bs[rt] = sb;
            }
        }
    }
};

// ------------------------------------------------------------------
// launching into a Sink (stream or graph)
// ------------------------------------------------------------------
template <class... P>
struct NodeArgs : NodeArgsBase {
    std::tuple<P...> t;
    explicit NodeArgs(P... a) : t(a...) {
        std::apply([this](auto&... x) { ptrs = {(void*)&x...}; }, t);
    }
};

namespace {
// Eager launch of fn; with a profiler, the launch carries a start and a stop
// event that hipExtLaunchKernel fills from the dispatch's own begin and end
// timestamps, so the recorded duration is the kernel's execution (what a
// kernel trace reports), without the queue gaps around it.
static int profiled_launch(Profiler* p, hipStream_t s, const char* name, double bytes, const void* fn, dim3 grid,
                           dim3 block, void** args, size_t lds) {
    if (!p) {
        GH_HIP(hipLaunchKernel(fn, grid, block, args, lds, s));
        return GH_OK;
    }
    Profiler::Rec r;
    r.kind = p->kind_of(name);
    r.bytes = bytes;
    if (p->pool.size() >= 2) {
        r.b = p->pool.back();
        p->pool.pop_back();
        r.a = p->pool.back();
        p->pool.pop_back();
    } else {
        GH_HIP(hipEventCreate(&r.a));
        if (hipEventCreate(&r.b) != hipSuccess) {
            (void)hipEventDestroy(r.a);
            return set_error(GH_ERR_HIP, "hipEventCreate failed");
        }
    }
    p->recs.push_back(r);
    GH_HIP(hipExtLaunchKernel(fn, grid, block, args, lds, s, r.a, r.b, 0));
    return GH_OK;
}

// Setter of the position-dependent argument I: an int, or a struct with
// set_pos(int) that also recomputes what derives from the position.
template <int I, class Tup>
std::function<void(int)> pos_setter(Tup& t) {
    auto* a = &std::get<I>(t);
    if constexpr (std::is_same_v<std::decay_t<decltype(*a)>, int>) return [a](int pos) { *a = pos; };
    else return [a](int pos) { a->set_pos(pos); };
}
}  // namespace

// Launch fn<<<grid, block, lds>>>(args...) on the sink.  POS_ARG >= 0 names
// the argument holding the step position (an int, or a struct with
// set_pos), which graph replays rewrite per step.
template <int POS_ARG = -1, class... P>
static int sink_launch(Sink& k, const char* name, double bytes, void (*fn)(P...), dim3 grid, dim3 block, size_t lds,
                       P... args) {
    if (k.only && std::strcmp(k.only, name) != 0) return GH_OK;
    k.launched += 1;
    k.bytes += bytes;
    auto blob = std::make_unique<NodeArgs<P...>>(args...);
    if (k.g) {
        hipKernelNodeParams prm{};
        prm.func = (void*)fn;
        prm.gridDim = grid;
        prm.blockDim = block;
        prm.sharedMemBytes = (unsigned)lds;
        prm.kernelParams = blob->ptrs.data();
        prm.extra = nullptr;
        hipGraphNode_t node;
        GH_HIP(hipGraphAddKernelNode(&node, k.g, k.last ? &k.last : nullptr, k.last ? 1 : 0, &prm));
        k.last = node;
        if constexpr (POS_ARG >= 0) k.patches->push_back({node, prm, pos_setter<POS_ARG>(blob->t)});
        k.store->push_back(std::move(blob));
        return GH_OK;
    }
    return profiled_launch(k.prof, k.s, name, bytes, (const void*)fn, grid, block, blob->ptrs.data(), lds);
}

template <int POS_ARG = -1, class Pro, class Epi>
static int launch_mv(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const Pro& pro,
                     const Epi& epi, int tmp_floats) {
    const int per_split = (w.nblk + p.S - 1) / p.S;
    // items per workgroup: NI > 1 only on the VALU Q4_0 path, for prologues
    // that declare their barriers
    int ni = 1;
    if constexpr (HasFinishBarriers<Pro>::value)
        if (w.fmt == FMT_Q4) ni = p.ni;
    if (ni != 1 && ni != 2) return set_error(GH_ERR_INVALID, "unsupported items per workgroup %d", ni);
    const size_t lds = mv_lds_bytes(w.fmt, per_split, tmp_floats) + (size_t)(ni - 1) * 512 * sizeof(float);
    const dim3 grid((p.row_tiles(w.tiles) + ni - 1) / ni * p.S), block(ni * NT);
    // POS_ARG counts kernel arguments (DMat, S, Pro, Epi): the prologue is 2
    DMat wk = w;
    wk.order_in = p.order_in;
    auto go = [&](void (*fn)(DMat, int, Pro, Epi)) {
        return sink_launch<POS_ARG>(k, name, bytes, fn, grid, block, lds, wk, p.S, pro, epi);
    };
    const int red_off = (int)mv_lds_floats(w.fmt, per_split, tmp_floats);
    auto go_multi = [&](void (*fn)(DMat, int, Pro, Epi, int)) {
        return sink_launch<POS_ARG>(k, name, bytes, fn, grid, block, lds, wk, p.S, pro, epi, red_off);
    };
    auto by_rl = [&](auto kbw) -> int {
        constexpr int KBW = decltype(kbw)::value;
        if constexpr (HasFinishBarriers<Pro>::value) {
            if (ni == 2 && p.mfma)
                return p.rl == 2 ? go_multi(k_matvec_multi<FMT_Q4M, KBW, 2, 2, Pro, Epi>)
                                 : go_multi(k_matvec_multi<FMT_Q4M, KBW, 1, 2, Pro, Epi>);
            if (ni == 2)
                return p.rl == 2 ? go_multi(k_matvec_multi<FMT_Q4, KBW, 2, 2, Pro, Epi>)
                                 : go_multi(k_matvec_multi<FMT_Q4, KBW, 1, 2, Pro, Epi>);
        }
        // one item per workgroup on the matrix cores: the LM head and the
        // op-level matvecs by default
        if (p.mfma)
            return p.rl == 2 ? go(k_matvec<FMT_Q4M, KBW, 2, Pro, Epi>) : go(k_matvec<FMT_Q4M, KBW, 1, Pro, Epi>);
        return p.rl == 2 ? go(k_matvec<FMT_Q4, KBW, 2, Pro, Epi>) : go(k_matvec<FMT_Q4, KBW, 1, Pro, Epi>);
    };
    if (p.rl != 1 && p.rl != 2) return set_error(GH_ERR_INVALID, "unsupported rows per lane %d", p.rl);
    if (w.fmt != FMT_Q4)
        return p.rl == 2 ? go(k_matvec<FMT_F32, 8, 2, Pro, Epi>) : go(k_matvec<FMT_F32, 8, 1, Pro, Epi>);
    switch (p.kbw) {
        case 1: return by_rl(std::integral_constant<int, 1>{});
        case 2: return by_rl(std::integral_constant<int, 2>{});
        case 3: return by_rl(std::integral_constant<int, 3>{});
        case 4: return by_rl(std::integral_constant<int, 4>{});
        case 6: return by_rl(std::integral_constant<int, 6>{});
        case 7: return by_rl(std::integral_constant<int, 7>{});
        case 9: return by_rl(std::integral_constant<int, 9>{});
        case 10: return by_rl(std::integral_constant<int, 10>{});
        default: return set_error(GH_ERR_INVALID, "unsupported register batch %d", p.kbw);
    }
}

// float4 groups per thread of the residual prologue: ceil(H / 1024)
template <class F>
static int with_mg(int H, F&& f) {
    const int mg = (H / 4 + NT - 1) / NT;
    switch (mg) {
        case 1: return f(std::integral_constant<int, 1>{});
        case 2: return f(std::integral_constant<int, 2>{});
        case 3: return f(std::integral_constant<int, 3>{});
        default: return set_error(GH_ERR_INVALID, "hidden size %d above 3072", H);
    }
}

// Final norm (once per step): xn = norm(x1 + postnorm(sum_s d_s), w_out).
template <int MG>
__global__ __launch_bounds__(NT) void k_final_norm(ProResid<MG> pro, float* xn) {
    extern __shared__ float lds[];
    MvLds L;
    L.red = lds;
    L.misc = lds + 512;
    L.xs = lds + 576;
    L.sxs = L.xs + pro.H;
    L.tmp = L.sxs;
    typename ProResid<MG>::Regs r;
    pro.load(r, 0, pro.H);
    pro.template finish<FMT_F32>(L, r, 0, pro.H);
    __syncthreads();
    for (int i = threadIdx.x; i < pro.H; i += NT) xn[i] = L.xs[i];
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
    const float* rope;  // [max_seq][HD/2] (cos, sin) of this layer type
    int pos;            // current position (patched per step with set_pos)
    int global, window, mode;
    // raw mode: q given
    const float* q;
    // common
    float* kc;
    float* vc;
    int nkv;
    float scale;
    float* part;
    int nc;
    int xcd;  // HSP > 1: a chunk's workgroups on one XCD (attn_wg)
    // attended positions [pb, pe) in chunks of ch, n_used of them (host-derived)
    int pb, pe, ch, n_used;
    __host__ __device__ void set_range(int b, int e) {
        pb = b;
        pe = e;
        attn_chunks(e - b, nc, ch, n_used);
    }
    __host__ __device__ void set_pos(int p) {
        int b, e;
        pos = p;
        attn_window(p, global, window, mode, b, e);
        set_range(b, e);
    }
};

// In-place per-vector RMSNorm by one wave (qkNormShader semantics).
template <int HD>
__device__ __forceinline__ void wave_head_norm(float* p, const float* w, float eps, int zc) {
    const int lane = threadIdx.x & 63;
    float ss = 0.0f;
    for (int i = lane; i < HD; i += 64) ss += p[i] * p[i];
    const float rms = sqrtf(wave_sum(ss) / (float)HD + eps);
    for (int i = lane; i < HD; i += 64) p[i] = norm_apply(p[i], rms, w[i], zc);
}

// In-place split-half RoPE of one head vector by one wave (ropeShader),
// cs = (cos, sin) of pos * f_i for i < HD/2.
template <int HD>
__device__ __forceinline__ void wave_head_rope(float* p, const float2* cs) {
    const int lane = threadIdx.x & 63;
    for (int i = lane; i < HD / 2; i += 64) {
        const float2 t = cs[i];
        const float a = p[i], b = p[i + HD / 2];
        p[i] = a * t.x - b * t.y;
        p[i + HD / 2] = a * t.y + b * t.x;
    }
}

// One query token over cache positions [pb, pe), split-K over chunks of
// ATTN_SUB-multiple length: workgroup (g, j) handles kv head g and chunk j
// and writes {m[G], l[G], o[G][HD]} (running max, sum of exp, unnormalised
// output) for the merge.
//
// Layout (flash-decoding): per sub-chunk of ATTN_SUB = 32 positions,
//   scores  8 lanes per position, each lane 16 B of every 128 B line of the
//           K row (one instruction reads 8 whole lines), q from LDS; one
//           3-step in-row DPP sum per score;
//   softmax wave w owns heads w, w+4: one wave max + one wave sum per head;
//   P.V     lane = 4 dims, the positions spread over NSLOT slots; the slot
//           partials are summed in LDS at the end.
// The K/V of the first sub-chunk are loaded at kernel start, with the QKV
// split partials (one global round trip); the next sub-chunk's K (V) is
// loaded as soon as the current one's K (V) registers are consumed.
// In step mode the prologue also applies QK-norm and RoPE to this token's
// q/k, appends k/v to the cache (appendKVCacheShader, AttentionGPU.hs:502-534)
// and uses them for the p == pos row.  The window and the chunking come from
// the host (AttnArgs::set_pos).
// Sources of the QKV vector: the split partials of the QKV matvec, or
// published words (persistent step).  g4(row) = float4 at fused-QKV row.
// issue() starts the loads of the float4 at fused-QKV row `row` (ok: the
// thread has one), get() returns it.
struct QkvPartials {
    const float* part;
    int S, ld;
    struct Pre {
        float4 v[MAXS];
    };
    __device__ void issue(Pre& p, int row, bool ok) const {
        const BufView P(part, (size_t)S * ld * 4);
#pragma unroll
        for (int s = 0; s < MAXS; ++s) p.v[s] = P.f4(ok ? 4u * (uint32_t)(s * ld + row) : OOB);
    }
    __device__ float4 get(const Pre& p, int) const {  // absent splits read zeros
        float4 r = p.v[0];
#pragma unroll
        for (int s = 1; s < MAXS; ++s) r = r + p.v[s];
        return r;
    }
};
// Sinks of the chunk state: plain floats or published words.
struct AttnOutPlain {
    float* part;
    __device__ void put(size_t i, float v) const { part[i] = v; }
};
struct AttnOutWords {
    uint64_t* w;
    uint32_t epoch;
    __device__ void put(size_t i, float v) const { st_word(w + i, epoch, v); }
};

template <int HD, int G, bool STEP, class In, class Out>
__device__ __forceinline__ void attn_item(const AttnArgs& a, int g, int j, const In& in, const Out& out) {
    constexpr int SUB = ATTN_SUB;
    constexpr int K4 = HD / 32;               // score phase: float4 per lane per position
    static_assert(SUB == 32, "one score round of 8 positions per wave");
    constexpr int LPV = HD / 4;               // P.V phase: lanes per position (4 dims each)
    constexpr int PGW = 64 / LPV;             // position groups per wave
    constexpr int NSLOT = 4 * PGW;            // position slots per workgroup
    constexpr int VPS = (SUB + NSLOT - 1) / NSLOT;  // positions per slot per sub-chunk
    constexpr int NG4 = (G + 2) * HD / 4;     // float4 groups of q|k|v
    constexpr int MG4 = (NG4 + NT - 1) / NT;  // per thread
    constexpr int NWR = (HD + 63) / 64;       // norm weights per lane
    constexpr int HPW = (G + 3) / 4;          // heads owned per wave in the softmax
    __shared__ __align__(16) float qs[G * HD];
    __shared__ __align__(16) float ks[HD];
    __shared__ __align__(16) float vs[HD];
    __shared__ __align__(16) float2 cs[HD / 2];
    __shared__ __align__(16) float sc[G][SUB];
    __shared__ __align__(16) float pr[SUB][G];
    __shared__ float corr_s[G];
    __shared__ __align__(16) float so[NSLOT][G * HD];

    GH_MARK(0);
    const int pos = STEP ? a.pos : -1;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c0 = a.pb + j * a.ch, c1 = min(a.pe, c0 + a.ch);
    const size_t pstride = (size_t)a.nkv * HD;
    const int pg = lane / LPV, dq = lane % LPV, slot = wave * PGW + pg;
    const int kq = lane & 7;                       // score phase: lane within the position's 8
    const int kp = wave * 8 + (lane >> 3);         // score phase: position within the sub-chunk
    // K/V rows [0, pe) as buffer views: vector-memory loads only, so the LDS
    // waits between them (lgkmcnt) never wait for the cache rows in flight
    const BufView KC(a.kc, (size_t)a.pe * pstride * 4), VC(a.vc, (size_t)a.pe * pstride * 4);
    const uint32_t kcol = 4u * (uint32_t)(g * HD + 4 * kq), vcol = 4u * (uint32_t)(g * HD + 4 * dq);

    // Loads are unconditional, from rows clamped into [c0, c1): rows past the
    // chunk are masked in the softmax / P.V, and row pos is replaced from LDS.
    float4 kr[K4], vr[VPS];
    auto load_k = [&](int s0) {
        const uint32_t ko = 4u * (uint32_t)min(s0 + kp, c1 - 1) * (uint32_t)pstride + kcol;
#pragma unroll
        for (int i = 0; i < K4; ++i) kr[i] = KC.f4(ko + 128u * i);
    };
    auto load_v = [&](int s0) {
#pragma unroll
        for (int k = 0; k < VPS; ++k) {
            const int pl = min(slot + k * NSLOT, SUB - 1);
            vr[k] = VC.f4(4u * (uint32_t)min(s0 + pl, c1 - 1) * (uint32_t)pstride + vcol);
        }
    };
    // 1. the QKV partials of this token (step mode), the QK-norm weights and
    //    the RoPE row go out first; then the K/V of the first sub-chunk (row
    //    pos comes from LDS below), so waiting for the prologue's inputs does
    //    not wait for the cache rows.
    if (STEP) {
        typename In::Pre pv[MG4];
        int rowv[MG4];
#pragma unroll
        for (int m = 0; m < MG4; ++m) {
            const int gi = tid + m * NT, i = 4 * gi;
            const int row = i < G * HD ? a.q_off + g * G * HD + i
                          : i < (G + 1) * HD ? a.k_off + g * HD + (i - G * HD)
                                             : a.v_off + g * HD + (i - (G + 1) * HD);
            rowv[m] = row;
            in.issue(pv[m], row, gi < NG4);
        }
        const BufView QN(a.q_norm, a.use_qk_norm ? HD * 4 : 0), KN(a.k_norm, a.use_qk_norm ? HD * 4 : 0);
        float wq[NWR], wk[NWR];
#pragma unroll
        for (int r = 0; r < NWR; ++r) {
            const uint32_t o = 4u * (lane + 64 * r);
            wq[r] = QN.f1(o);
            wk[r] = KN.f1(o);
        }
        const BufView CS(a.rope + (size_t)pos * HD, HD * 4);
        const float2 csv = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(CS.r, tid < HD / 2 ? 8u * tid : OOB, 0, 0));
        __builtin_amdgcn_sched_barrier(0);  // keep the cache-row loads behind the prologue's
        load_k(c0);
        load_v(c0);
        __builtin_amdgcn_sched_barrier(0);
        // a source whose words may still be in flight (persistent step)
        // waits for all of them here, the K/V loads already issued
        if constexpr (HasSettle<In>::value) in.template settle<MG4>(pv, rowv);
        GH_MARK(1);
        // 2. q, k, v of this token into LDS
#pragma unroll
        for (int m = 0; m < MG4; ++m) {
            const int gi = tid + m * NT;
            if (gi < NG4) {
                const int i = 4 * gi;
                const int row = i < G * HD ? a.q_off + g * G * HD + i
                              : i < (G + 1) * HD ? a.k_off + g * HD + (i - G * HD)
                                                 : a.v_off + g * HD + (i - (G + 1) * HD);
                float* dst = i < G * HD ? &qs[i] : i < (G + 1) * HD ? &ks[i - G * HD] : &vs[i - (G + 1) * HD];
                *(float4*)dst = in.get(pv[m], row);
            }
        }
        if (tid < HD / 2) cs[tid] = csv;
        __syncthreads();
        GH_MARK(2);
        // QK-norm (TBG:171-179), then RoPE, on the G q heads and the k head
        for (int vec = wave; vec < G + 1; vec += 4) {
            float* p = vec < G ? qs + vec * HD : ks;
            if (a.use_qk_norm) {
                float ss = 0.0f;
#pragma unroll
                for (int r = 0; r < NWR; ++r) {
                    const int i = lane + 64 * r;
                    if (i < HD) ss += p[i] * p[i];
                }
                const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)HD + a.eps);
#pragma unroll
                for (int r = 0; r < NWR; ++r) {
                    const int i = lane + 64 * r;
                    if (i < HD) p[i] = norm_apply_inv(p[i], inv, vec < G ? wq[r] : wk[r], a.zc);
                }
            }
            wave_head_rope<HD>(p, cs);
        }
        __syncthreads();
        GH_MARK(3);
        if (j == 0) {  // appendKVCacheShader (AttentionGPU.hs:502-534); global stores (no LDS counter)
            typedef __attribute__((address_space(1))) float gfloat;
            for (int i = tid; i < HD; i += NT) {
                ((gfloat*)a.kc)[((size_t)pos * a.nkv + g) * HD + i] = ks[i];
                ((gfloat*)a.vc)[((size_t)pos * a.nkv + g) * HD + i] = vs[i];
            }
        }
    } else {
        load_k(c0);
        load_v(c0);
        GH_MARK(1);
        for (int i = tid; i < G * HD; i += NT) qs[i] = a.q[(size_t)g * G * HD + i];
        __syncthreads();
    }

    float mrun[HPW], lrun[HPW];
#pragma unroll
    for (int hi = 0; hi < HPW; ++hi) {
        mrun[hi] = -INFINITY;
        lrun[hi] = 0.0f;
    }
    float4 acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h] = f4z();

    // one sub-chunk; `more` issues the next sub-chunk's loads as registers free up
    auto sub_chunk = [&](int s0, bool more) {
        if (STEP) {
            if (s0 + kp == pos) {
#pragma unroll
                for (int i = 0; i < K4; ++i) kr[i] = *(const float4*)&ks[32 * i + 4 * kq];
            }
#pragma unroll
            for (int k = 0; k < VPS; ++k)
                if (s0 + slot + k * NSLOT == pos) vr[k] = *(const float4*)&vs[4 * dq];
        }
        // 3. scores of this wave's 8 positions
        {
            float sv[G];
#pragma unroll
            for (int h = 0; h < G; ++h) sv[h] = 0.0f;
#pragma unroll
            for (int i = 0; i < K4; ++i) {
#pragma unroll
                for (int h = 0; h < G; ++h) sv[h] += dot4(*(const float4*)&qs[h * HD + 32 * i + 4 * kq], kr[i]);
            }
            if (more) load_k(s0 + SUB);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                sv[h] = group_sum<8>(sv[h]);
                if (kq == 0) sc[h][kp] = sv[h];
            }
        }
        __syncthreads();
        GH_MARK(8);
        // 4. softmax update of the heads this wave owns
        const bool valid = lane < SUB && s0 + lane < c1;
#pragma unroll
        for (int hi = 0; hi < HPW; ++hi) {
            const int h = wave + 4 * hi;
            if (h < G) {
                const float v = valid ? sc[h][lane] * a.scale : -INFINITY;
                const float mn = fmaxf(mrun[hi], wave_max(v));
                const float e = valid ? __expf(v - mn) : 0.0f;
                const float corr = mrun[hi] == -INFINITY ? 0.0f : __expf(mrun[hi] - mn);
                lrun[hi] = lrun[hi] * corr + wave_sum(e);
                mrun[hi] = mn;
                if (lane < SUB) pr[lane][h] = e;
                if (lane == 0) corr_s[h] = corr;
            }
        }
        __syncthreads();
        GH_MARK(9);
        // 5. P.V over this slot's positions
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float c = corr_s[h];
            acc[h] = make_float4(acc[h].x * c, acc[h].y * c, acc[h].z * c, acc[h].w * c);
        }
#pragma unroll
        for (int k = 0; k < VPS; ++k) {
            const int pl = slot + k * NSLOT;
            if (pl < SUB && s0 + pl < c1) {
                float pw[G];
                if constexpr (G >= 4) {
#pragma unroll
                    for (int h4 = 0; h4 < G; h4 += 4) {
                        const float4 t = *(const float4*)&pr[pl][h4];
                        pw[h4] = t.x; pw[h4 + 1] = t.y; pw[h4 + 2] = t.z; pw[h4 + 3] = t.w;
                    }
                } else {
#pragma unroll
                    for (int h = 0; h < G; ++h) pw[h] = pr[pl][h];
                }
#pragma unroll
                for (int h = 0; h < G; ++h) acc[h] = fma4(pw[h], vr[k], acc[h]);
            }
        }
        if (more) {
            load_v(s0 + SUB);
            __syncthreads();  // sc / pr of this sub-chunk consumed
        }
    };
    if (c1 - c0 <= SUB) {
        sub_chunk(c0, false);  // chunks up to 32 positions: straight-line code
    } else {
        for (int s0 = c0; s0 < c1; s0 += SUB) sub_chunk(s0, s0 + SUB < c1);
    }
    GH_MARK(4);
    // 6. sum the slot partials; write the chunk's state
#pragma unroll
    for (int h = 0; h < G; ++h) *(float4*)&so[slot][h * HD + 4 * dq] = acc[h];
    __syncthreads();
    GH_MARK(5);
    const size_t ob = ((size_t)g * a.nc + j) * (G * (HD + 2));
    for (int idx = tid; idx < G * HD; idx += NT) {
        float O = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < NSLOT; ++s2) O += so[s2][idx];
        out.put(ob + 2 * G + idx, O);
    }
#pragma unroll
    for (int hi = 0; hi < HPW; ++hi) {
        const int h = wave + 4 * hi;
        if (h < G && lane == 0) {
            out.put(ob + h, mrun[hi]);
            out.put(ob + G + h, lrun[hi]);
        }
    }
    GH_MARK(6);
    GH_MARK_END();
}

template <int HD, int G, bool STEP>
__global__ __launch_bounds__(NT) void k_attn(AttnArgs a) {
    const int g = blockIdx.x / a.nc, j = blockIdx.x % a.nc;
    if (j >= a.n_used) return;  // uniform per workgroup
    attn_item<HD, G, STEP>(a, g, j, QkvPartials{a.part_qkv, a.Sa, a.ld_qkv}, AttnOutPlain{a.part});
}

// One query token of the decode step over cache positions [pb, pe): split-K
// over chunks as attn_item (workgroup (g, j): kv head g, chunk j; the same
// {m[G], l[G], o[G][HD]} chunk state), with a short dependency chain:
//   prologue  the QKV split partials of this token are summed in registers,
//             one float4 group per lane, each q/k head vector held by
//             LPH = HD/4 consecutive lanes: QK-norm (TBG:171-179) is one
//             lane-group reduction, split-half RoPE (ropeShader) swaps with
//             the lane LPH/2 away; q, k, v go to LDS behind one barrier.
//             Only workgroup 0 (the KV append, appendKVCacheShader) and the
//             workgroup whose chunk holds `pos` load the k/v partials.
//   stream    wave w takes the chunk's rounds of 8 positions w, w+4, ...
//             with its own online softmax, K/V two rounds ahead, no
//             workgroup barrier: scores 8 lanes per position (lane kq holds
//             one 16 B piece of each 128 B line of the K row), one 3-step
//             DPP sum per score; P.V lane = 4 dims, weights by readlane.
//   merge     the four wave states, once, through LDS.
// PF: K/V rounds per wave loaded ahead (1 for chunks of up to 4 rounds, where
// each wave has at most one round; 2 otherwise).  SKIP: this wave's groups
// in the last prologue round are all k/v that its workgroup does not need,
// or past q|k|v, so it issues none of that round's loads (every load
// instruction costs its CU's address unit the same time, in range or not).
// The kernel picks the body before issuing any load, so each body's
// s_waitcnt counts stay exact.
// OPQ (the op-level entry point): the G query heads of kv head g come
// ready in a.q (normed and roped), K/V are complete in the cache; the
// prologue loads q only, and there is no current row to append or score.
template <int HD, int G>
struct AttnStepLds {
    float qs[G * HD];
    float ks[HD];
    float vs[HD];
    float ms[4][G], ls[4][G];
    float os[4][G * HD];
};

// GT: the kv group's q heads; this workgroup takes G of them, from head
// hs * G of the group (GT / G workgroups per chunk read the same K/V).
template <int HD, int G, int PF, bool SKIP, bool OPQ = false, int GT = G>
__device__ __forceinline__ void attn_step_body(const AttnArgs& a, int g, int j, AttnStepLds<HD, G>& S, int hs = 0) {
    constexpr int LPH = HD / 4;                  // lanes per head vector (one float4 each)
    constexpr int NG4 = (G + 2) * LPH;           // float4 groups of q | k | v
    constexpr int MG4 = (NG4 + NT - 1) / NT;     // groups per thread
    constexpr int K4 = HD / 32, RP = 8;          // score float4 per lane and position; positions per round
    static_assert(HD % 32 == 0 && LPH <= 64, "head_dim 32..256");
    float* qs = S.qs;
    float* ks = S.ks;
    float* vs = S.vs;
    auto& ms = S.ms;
    auto& ls = S.ls;
    auto& os = S.os;
    GH_MARK(0);
    const int pos = a.pos;
    const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63;
    const int c0 = a.pb + j * a.ch, c1 = min(a.pe, c0 + a.ch);
    const bool own = !OPQ && pos >= c0 && pos < c1;  // this chunk scores the current position
    const bool append = !OPQ && j == 0 && hs == 0;   // this workgroup appends k, v to the cache
    const bool need_kv = own || append;
    const int h0 = g * GT + hs * G;                  // first q head of this workgroup
    const size_t pstride = (size_t)a.nkv * HD;

    // 1. prologue loads: partials, QK-norm weights, RoPE row (straight-line)
    constexpr int QG4 = G * LPH, MQ4 = (QG4 + NT - 1) / NT;  // OPQ: float4 groups of q per thread
    float4 qv[MQ4];
    if constexpr (OPQ) {
        const BufView Q(a.q + (size_t)h0 * HD, (size_t)G * HD * 4);
#pragma unroll
        for (int m = 0; m < MQ4; ++m) qv[m] = Q.f4(16u * (uint32_t)(tid + m * NT));
    }
    const BufView P(a.part_qkv, OPQ ? 0 : (size_t)a.Sa * a.ld_qkv * 4);
    const BufView QN(a.q_norm, a.use_qk_norm ? HD * 4 : 0), KN(a.k_norm, a.use_qk_norm ? HD * 4 : 0);
    const BufView CS(OPQ ? nullptr : a.rope + (size_t)pos * HD, OPQ ? 0 : HD * 4);
    float4 pv[MG4][MAXS], wn[MG4], cs0[MG4], cs1[MG4];
#pragma unroll
    for (int m = 0; m < MG4; ++m) {
        if constexpr (OPQ) continue;
        if (SKIP && m == MG4 - 1) {
#pragma unroll
            for (int s = 0; s < MAXS; ++s) pv[m][s] = f4z();
            wn[m] = cs0[m] = cs1[m] = f4z();
            continue;
        }
        const int gi = tid + m * NT, vec = gi / LPH, d = 4 * (gi % LPH);  // vector (G q heads, k, v), first dim
        const int row = vec < G ? a.q_off + (h0 + vec) * HD + d : vec == G ? a.k_off + g * HD + d : a.v_off + g * HD + d;
        const bool ok = gi < NG4 && (vec < G || need_kv);
#pragma unroll
        for (int s = 0; s < MAXS; ++s) pv[m][s] = P.f4(ok ? 4u * (uint32_t)(s * a.ld_qkv + row) : OOB);
        const float4 wq = QN.f4(vec < G ? 4u * d : OOB), wk = KN.f4(vec == G ? 4u * d : OOB);
        wn[m] = vec < G ? wq : wk;
        const int i = d % (HD / 2);  // RoPE pair index of the first dim
        cs0[m] = CS.f4(vec <= G ? 8u * i : OOB);
        cs1[m] = CS.f4(vec <= G ? 8u * i + 16u : OOB);
    }
    __builtin_amdgcn_sched_barrier(0);
    // K/V rounds as buffer loads: rounds past the chunk's and positions past
    // its end read zeros without traffic (and are masked); row pos is
    // replaced from LDS (it is being appended)
    const int kq = lane & 7, kp = lane >> 3;
    const BufView KC(a.kc, (size_t)a.pe * pstride * 4), VC(a.vc, (size_t)a.pe * pstride * 4);
    const uint32_t kcol = 4u * (uint32_t)(g * HD + 4 * kq), vcol = 4u * (uint32_t)(g * HD + 4 * lane);
    const int nr = (c1 - c0 + RP - 1) / RP;
    const int rot = (j * 5) % nr;  // round order rotated per chunk (HBM channels), a permutation
    auto round_pos = [&](int r) { return c0 + RP * ((r + rot) % nr); };
    float4 kr[PF][K4], vr[PF][RP];
    auto load = [&](int u, int r) {
        const bool rok = r < nr;
        const int p0 = round_pos(rok ? r : 0);
        const uint32_t ko = rok && p0 + kp < c1 ? 4u * (uint32_t)(p0 + kp) * (uint32_t)pstride + kcol : OOB;
#pragma unroll
        for (int i = 0; i < K4; ++i) kr[u][i] = KC.f4(ko + 128u * i);
#pragma unroll
        for (int k = 0; k < RP; ++k)
            vr[u][k] = VC.f4(rok && p0 + k < c1 && lane < LPH ? 4u * (uint32_t)(p0 + k) * (uint32_t)pstride + vcol : OOB);
    };
    load(0, wave);
    if (PF == 2) load(PF - 1, wave + 4);
    __builtin_amdgcn_sched_barrier(0);
    GH_MARK(1);

    // 2. sums, QK-norm, RoPE in registers; q, k, v to LDS
    if constexpr (OPQ) {
#pragma unroll
        for (int m = 0; m < MQ4; ++m)
            if (tid + m * NT < QG4) *(float4*)&qs[4 * (tid + m * NT)] = qv[m];
    }
#pragma unroll
    for (int m = 0; m < MG4; ++m) {
        if constexpr (OPQ) continue;
        const int gi = tid + m * NT, vec = gi / LPH, d = 4 * (gi % LPH);
        float4 v = pv[m][0];
#pragma unroll
        for (int s = 1; s < MAXS; ++s) v = v + pv[m][s];  // absent splits read zeros
        if (m * NT < NG4) {  // uniform: some lane of the workgroup holds a group
            const bool qk = vec <= G;
            if (a.use_qk_norm) {
                const float ss = group_sum<LPH>(qk ? dot4(v, v) : 0.0f);
                const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
                if (qk) v = norm4i(v, inv, wn[m], a.zc);
            }
            // split-half RoPE: the partner dims d +- HD/2 sit LPH/2 lanes away
            float4 pr;
            pr.x = __shfl_xor(v.x, LPH / 2, 64);
            pr.y = __shfl_xor(v.y, LPH / 2, 64);
            pr.z = __shfl_xor(v.z, LPH / 2, 64);
            pr.w = __shfl_xor(v.w, LPH / 2, 64);
            if (qk) {
                const float c[4] = {cs0[m].x, cs0[m].z, cs1[m].x, cs1[m].z}, sn[4] = {cs0[m].y, cs0[m].w, cs1[m].y, cs1[m].w};
                const float x[4] = {v.x, v.y, v.z, v.w}, q[4] = {pr.x, pr.y, pr.z, pr.w};
                float y[4];
                const bool first = d < HD / 2;
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] = first ? x[e] * c[e] - q[e] * sn[e] : q[e] * sn[e] + x[e] * c[e];
                v = make_float4(y[0], y[1], y[2], y[3]);
            }
            if (gi < NG4) {
                float* dst = vec < G ? &qs[vec * HD + d] : vec == G ? &ks[d] : &vs[d];
                *(float4*)dst = v;
            }
        }
    }
    __syncthreads();
    GH_MARK(2);
    if (append) {  // appendKVCacheShader (AttentionGPU.hs:502-534)
        for (int i = tid; i < HD; i += NT) {
            a.kc[((size_t)pos * a.nkv + g) * HD + i] = ks[i];
            a.vc[((size_t)pos * a.nkv + g) * HD + i] = vs[i];
        }
    }

    // 3. stream the wave's rounds
    float mrun[G], lrun[G];
    float4 acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        mrun[h] = -INFINITY;
        lrun[h] = 0.0f;
        acc[h] = f4z();
    }
    for (int r = wave; r < nr; r += 4 * PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int rr = r + 4 * u;
            if (rr >= nr) break;  // uniform per wave
            const int p0 = round_pos(rr);
            if (own && pos >= p0 && pos < p0 + RP) {  // the current row comes from LDS
                if (p0 + kp == pos) {
#pragma unroll
                    for (int i = 0; i < K4; ++i) kr[u][i] = *(const float4*)&ks[32 * i + 4 * kq];
                }
#pragma unroll
                for (int k = 0; k < RP; ++k)
                    if (p0 + k == pos && lane < LPH) vr[u][k] = *(const float4*)&vs[4 * lane];
            }
            const bool valid = p0 + kp < c1;
            float pw[G];
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float sv = 0.0f;
#pragma unroll
                for (int i = 0; i < K4; ++i) sv += dot4(*(const float4*)&qs[h * HD + 32 * i + 4 * kq], kr[u][i]);
                sv = group_sum<8>(sv) * a.scale;
                sv = valid ? sv : -INFINITY;
                const float mn = fmaxf(mrun[h], wave_max_g8(sv));  // the round has a valid position: mn finite
                const float corr = __expf(mrun[h] - mn);             // mrun = -inf -> 0
                pw[h] = valid ? __expf(sv - mn) : 0.0f;
                // per-lane running sums (lanes kq == 0 hold their position's
                // terms), reduced once after the rounds
                lrun[h] = lrun[h] * corr + (kq == 0 ? pw[h] : 0.0f);
                mrun[h] = mn;
                acc[h] = make_float4(acc[h].x * corr, acc[h].y * corr, acc[h].z * corr, acc[h].w * corr);
            }
#pragma unroll
            for (int k = 0; k < RP; ++k) {
                if (p0 + k < c1) {  // uniform per wave
#pragma unroll
                    for (int h = 0; h < G; ++h) acc[h] = fma4(readlane(pw[h], 8 * k), vr[u][k], acc[h]);
                }
            }
            if (PF == 2) load(u, rr + 8);
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) lrun[h] = wave_sum(lrun[h]);
    GH_MARK(4);
    // 4. merge the four wave states; write the chunk's state
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            ms[wave][h] = mrun[h];
            ls[wave][h] = lrun[h];
        }
    }
    if (lane < LPH) {
#pragma unroll
        for (int h = 0; h < G; ++h) *(float4*)&os[wave][h * HD + 4 * lane] = acc[h];
    }
    __syncthreads();
    GH_MARK(5);
    const size_t ob = ((size_t)g * a.nc + j) * (GT * (HD + 2));
    // four consecutive outputs per thread (one head each: HD % 4 == 0)
    for (int q4 = tid; q4 < G * HD / 4; q4 += NT) {
        const int h = 4 * q4 / HD;
        const float m0 = ms[0][h], m1 = ms[1][h], m2 = ms[2][h], m3 = ms[3][h];
        const float M = fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
        const float e0 = __expf(m0 - M), e1 = __expf(m1 - M), e2 = __expf(m2 - M), e3 = __expf(m3 - M);
        const float4 o0 = *(const float4*)&os[0][4 * q4], o1 = *(const float4*)&os[1][4 * q4];
        const float4 o2 = *(const float4*)&os[2][4 * q4], o3 = *(const float4*)&os[3][4 * q4];
        float* dst = a.part + ob + 2 * GT + hs * G * HD + 4 * q4;
        dst[0] = ((e0 * o0.x + e1 * o1.x) + e2 * o2.x) + e3 * o3.x;
        dst[1] = ((e0 * o0.y + e1 * o1.y) + e2 * o2.y) + e3 * o3.y;
        dst[2] = ((e0 * o0.z + e1 * o1.z) + e2 * o2.z) + e3 * o3.z;
        dst[3] = ((e0 * o0.w + e1 * o1.w) + e2 * o2.w) + e3 * o3.w;
    }
    if (tid < G) {
        const float M = fmaxf(fmaxf(ms[0][tid], ms[1][tid]), fmaxf(ms[2][tid], ms[3][tid]));
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) L += __expf(ms[w][tid] - M) * ls[w][tid];
        a.part[ob + hs * G + tid] = M;
        a.part[ob + GT + hs * G + tid] = L;
    }
    GH_MARK(6);
    GH_MARK_END();
}

// Workgroup b of a launch runs on XCD b % 8.  With HSP > 1 workgroups per
// chunk (q heads split between them), chunk gj's workgroups are
// b = 8 * (HSP * (gj / 8) + hs) + gj % 8, all on XCD gj % 8, so that the
// chunk's K/V rows come into one L2 instead of HSP of them; the grid is
// rounded up to whole groups of 8 chunks (false: a workgroup past the last
// chunk).  AttnArgs::xcd = 0 keeps b = HSP * gj + hs.
template <int HSP>
__device__ __forceinline__ bool attn_wg(const AttnArgs& a, int& gj, int& hs) {
    if (HSP == 1 || !a.xcd) {
        hs = blockIdx.x % HSP;
        gj = blockIdx.x / HSP;
        return true;
    }
    const int r = blockIdx.x & 7, q = blockIdx.x >> 3;
    hs = q % HSP;
    gj = (q / HSP) * 8 + r;
    return gj < a.nkv * a.nc;
}

// HSP workgroups per chunk, each taking G / HSP of the group's q heads.
template <int HD, int G, int HSP = 1>
__global__ __launch_bounds__(NT) void k_attn_step(AttnArgs a) {
    constexpr int GW = G / HSP;
    int hs, gj;
    if (!attn_wg<HSP>(a, gj, hs)) return;
    const int g = gj / a.nc, j = gj % a.nc;
    if (j >= a.n_used) return;  // uniform per workgroup
    const int c0 = a.pb + j * a.ch, c1 = min(a.pe, c0 + a.ch);
    __shared__ __align__(16) AttnStepLds<HD, GW> lds;
    // the first vector of this wave's groups in the last prologue round
    constexpr int LPH = HD / 4, NG4 = (GW + 2) * LPH, MG4 = (NG4 + NT - 1) / NT;
    const int vec_lo = ((MG4 - 1) * NT + wave_id() * 64) / LPH;
    const int pos = a.pos;
    const bool need_kv = (pos >= c0 && pos < c1) || (j == 0 && hs == 0);
    const bool skip = vec_lo >= GW + 2 || (vec_lo >= GW && !need_kv);
    if (c1 - c0 <= 32) {
        if (skip) attn_step_body<HD, GW, 1, true, false, G>(a, g, j, lds, hs);
        else attn_step_body<HD, GW, 1, false, false, G>(a, g, j, lds, hs);
    } else {
        if (skip) attn_step_body<HD, GW, 2, true, false, G>(a, g, j, lds, hs);
        else attn_step_body<HD, GW, 2, false, false, G>(a, g, j, lds, hs);
    }
}

// Op-level attention of one query token over [pb, pe) of a complete cache
// (gh_attention_decode, head_dim 256): the step kernel's streaming body with
// q read ready-made (OPQ); workgroup (g, j) writes chunk j's state for
// k_attn_combine.
template <int HD, int G, int HSP = 1>
__global__ __launch_bounds__(NT) void k_attn_op(AttnArgs a) {
    constexpr int GW = G / HSP;
    int hs, gj;
    if (!attn_wg<HSP>(a, gj, hs)) return;
    const int g = gj / a.nc, j = gj % a.nc;
    if (j >= a.n_used) return;  // uniform per workgroup
    const int c0 = a.pb + j * a.ch, c1 = min(a.pe, c0 + a.ch);
    __shared__ __align__(16) AttnStepLds<HD, GW> lds;
    if (c1 - c0 <= 32) attn_step_body<HD, GW, 1, false, true, G>(a, g, j, lds, hs);
    else attn_step_body<HD, GW, 2, false, true, G>(a, g, j, lds, hs);
}

#if GH_IN_TU(1)
static int launch_attn_step(Sink& k, double bytes, int hd, int G, const AttnArgs& a, int nkv) {
    if (a.nc > ATTN_MAX_NC || a.nc < 1) return set_error(GH_ERR_INVALID, "attention: %d splits (1..%d)", a.nc, ATTN_MAX_NC);
    // groups of 4+ q heads: one workgroup per (chunk, q head), each reading
    // its head's q partials and the chunk's K/V rounds (read once per head).
    // Measured on MI355X, 1B (4 heads per kv head): attention 5.15 us with
    // one workgroup per chunk, 4.28 with two (two heads each), 3.91 with
    // four; 1450 -> 1495 -> 1511 tok/s.  With 2 heads per kv head (4B) one
    // head per workgroup is slower (4.33 -> 4.88 us; with a chunk's two
    // workgroups on one XCD, C5 740 vs 759 tok/s), so those stay whole.
    // A chunk's workgroups share one XCD (attn_wg): 1B 1632-1633 tok/s
    // against 1605-1606 with consecutive workgroups on different XCDs.
    static const char* hs_env = std::getenv("GH_ATTN_HSPLIT");  // 0: one workgroup per chunk
    const int hsp = G >= 4 && !(hs_env && *hs_env == '0') ? G : 1;
    const dim3 grid(hsp > 1 && a.xcd ? 8 * hsp * ((nkv * a.nc + 7) / 8) : nkv * a.nc * hsp), block(NT);
#define GH_ATTN_CASE(HD_, G_)                                                                                  \
    if (hd == HD_ && G == G_)                                                                                  \
        return hsp > 1 ? sink_launch<0>(k, "attention", bytes, k_attn_step<HD_, G_, (G_ >= 4 ? G_ : 1)>, grid,   \
                                         block, 0, a)                                                         \
                        : sink_launch<0>(k, "attention", bytes, k_attn_step<HD_, G_, 1>, grid, block, 0, a);
    GH_ATTN_CASE(256, 1) GH_ATTN_CASE(256, 2) GH_ATTN_CASE(256, 4) GH_ATTN_CASE(256, 8)
    GH_ATTN_CASE(128, 1) GH_ATTN_CASE(128, 2) GH_ATTN_CASE(128, 4) GH_ATTN_CASE(128, 8)
    GH_ATTN_CASE(32, 1) GH_ATTN_CASE(32, 2) GH_ATTN_CASE(32, 4) GH_ATTN_CASE(32, 8)
#undef GH_ATTN_CASE
    return set_error(GH_ERR_INVALID, "attention: unsupported head_dim %d / group %d", hd, G);
}
#endif

template <bool STEP>
static int launch_attn_t(Sink& k, double bytes, int hd, int G, const AttnArgs& a, int nkv) {
    const int max_nc = STEP ? ATTN_MAX_NC : GH_ATTN_OP_MAX_NC;
    if (a.nc > max_nc || a.nc < 1) return set_error(GH_ERR_INVALID, "attention: %d splits (1..%d)", a.nc, max_nc);
    const dim3 grid(nkv * a.nc), block(NT);
#define GH_ATTN_CASE(HD_, G_) \
    if (hd == HD_ && G == G_) return sink_launch<STEP ? 0 : -1>(k, "attention", bytes, k_attn<HD_, G_, STEP>, grid, block, 0, a);
    GH_ATTN_CASE(256, 1) GH_ATTN_CASE(256, 2) GH_ATTN_CASE(256, 4) GH_ATTN_CASE(256, 8)
    GH_ATTN_CASE(128, 1) GH_ATTN_CASE(128, 2) GH_ATTN_CASE(128, 4) GH_ATTN_CASE(128, 8)
    GH_ATTN_CASE(32, 1) GH_ATTN_CASE(32, 2) GH_ATTN_CASE(32, 4) GH_ATTN_CASE(32, 8)
#undef GH_ATTN_CASE
    return set_error(GH_ERR_INVALID, "attention: unsupported head_dim %d / group %d", hd, G);
}

// Merge of the split-K partials for the op-level entry point (the
// reference's softmax over all positions, combined from the chunk states
// {m_j, l_j, o_j}): workgroup (q head h, 32-dim slice); thread t holds chunk
// t's (m, l) and, as lane (c, q) = (t / 8, t % 8), dims 4q..4q+3 of chunks
// c, c + 32, ...  Every load is issued before the first use, as straight-line
// buffer loads (chunks past n_used read zeros), so the merge costs one round
// trip; the 32 chunk groups are added in LDS.  (64-dim slices, half the
// workgroups with twice the loads each: C4 8192 global 10.24 vs 10.11 us.)
// VEC: float4 loads of o (the state stride G*(HD+2) is a multiple of 4 when
// G is even), else 4 scalars.
#if GH_IN_TU(4)
constexpr int COMB_DIMS = 32, COMB_CG = NT / (COMB_DIMS / 4), COMB_PER = GH_ATTN_OP_MAX_NC / COMB_CG;
template <bool VEC>
__global__ __launch_bounds__(NT) void k_attn_combine(const float* part, int nc, int n_used, int G, int HD, float* out) {
    __shared__ float wj[GH_ATTN_OP_MAX_NC];
    __shared__ float slot[8];
    __shared__ __align__(16) float red[COMB_CG][COMB_DIMS];
    static_assert(GH_ATTN_OP_MAX_NC <= NT, "one chunk state per thread");
    const int nds = (HD + COMB_DIMS - 1) / COMB_DIMS;
    const int h = blockIdx.x / nds, d0 = (blockIdx.x % nds) * COMB_DIMS;
    const int g = h / G, hl = h % G, tid = threadIdx.x;
    const int dq = 4 * (tid % (COMB_DIMS / 4)), cg = tid / (COMB_DIMS / 4);
    const uint32_t stride = (uint32_t)(G * (HD + 2));
    const BufView P(part + (size_t)g * nc * stride, (size_t)n_used * stride * 4);
    const float m = P.f1(tid < n_used ? 4u * (tid * stride + hl) : OOB);
    const float l = P.f1(tid < n_used ? 4u * (tid * stride + G + hl) : OOB);
    const bool dok = d0 + dq < HD;  // HD is a multiple of 4
    float4 ov[COMB_PER];
#pragma unroll
    for (int k = 0; k < COMB_PER; ++k) {
        const int j = cg + COMB_CG * k;
        const uint32_t off = dok && j < n_used ? 4u * (j * stride + 2 * G + hl * HD + d0 + dq) : OOB;
        if (VEC) {
            ov[k] = P.f4(off);
        } else {
            const uint32_t o1 = off == OOB ? OOB : off + 4u, o2 = off == OOB ? OOB : off + 8u, o3 = off == OOB ? OOB : off + 12u;
            ov[k] = make_float4(P.f1(off), P.f1(o1), P.f1(o2), P.f1(o3));
        }
    }
    // block max of m over the chunks
    const float mx = wave_max(tid < n_used ? m : -INFINITY);
    if ((tid & 63) == 0) slot[tid >> 6] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(slot[0], slot[1]), fmaxf(slot[2], slot[3]));
    const float w = tid < n_used ? expf(m - M) : 0.0f;
    wj[tid] = w;
    const float den = block_sum(l * w, slot + 4);  // barrier: wj complete
    float4 num = f4z();
#pragma unroll
    for (int k = 0; k < COMB_PER; ++k) num = fma4(wj[cg + COMB_CG * k], ov[k], num);
    *(float4*)&red[cg][dq] = num;
    __syncthreads();
    if (tid < COMB_DIMS && d0 + tid < HD) {
        float t = 0.0f;
#pragma unroll
        for (int c = 0; c < COMB_CG; ++c) t += red[c][tid];
        out[(size_t)h * HD + d0 + tid] = t / den;
    }
}
#endif

// ------------------------------------------------------------------
// step epilogue: greedy token from the per-tile keys, next token, position
// ------------------------------------------------------------------
// Philox4x32-10 counter-based generator (Salmon, Moraes, Dror, Shaw,
// "Parallel random numbers: as easy as 1, 2, 3", SC'11): 10 rounds of the
// 4x32 round function with the published multipliers and Weyl key bumps.
struct PhiloxOut {
    uint32_t x, y, z, w;
};
__host__ __device__ inline PhiloxOut philox4x32_10(PhiloxOut c, uint32_t k0, uint32_t k1) {
    for (int r = 0; r < 10; ++r) {
        if (r) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c.x;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c.z;
        c = PhiloxOut{(uint32_t)(p1 >> 32) ^ c.y ^ k0, (uint32_t)p1, (uint32_t)(p0 >> 32) ^ c.w ^ k1, (uint32_t)p0};
    }
    return c;
}
// u in [0, 1) from Philox(counter = (lo, hi, 0, 0), key = seed): the top 24
// bits of the first output word.
__host__ __device__ inline float philox_uniform(uint64_t seed, uint64_t counter) {
    const PhiloxOut o = philox4x32_10(PhiloxOut{(uint32_t)counter, (uint32_t)(counter >> 32), 0u, 0u}, (uint32_t)seed,
                                      (uint32_t)(seed >> 32));
    return (float)(o.x >> 8) * (1.0f / 16777216.0f);
}

// ---- samplers ----
// Inversion draws: with weights w_i over an ordered set and u in [0, 1), the
// pick is the first element whose running sum of weights exceeds u * total
// (if rounding leaves none, the last element with a positive weight).

// inclusive running sum over the 64 lanes, lane order
__device__ __forceinline__ float wave_scan_incl(float v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(v, o, 64);
        if (lane >= o) v += y;
    }
    return v;
}

// One wave walks rows r0 .. r1-1 (64 at a time) for the first row whose
// running sum of exp((l - M) / T) exceeds `target`; all lanes return it.
__device__ __forceinline__ int wave_row_walk(const float* logits, int r0, int r1, float M, float inv_t, float target) {
    const int lane = threadIdx.x & 63;
    const BufView L(logits, (size_t)r1 * 4);
    float base = 0.0f;
    int last = r0;
    for (int s = r0; s < r1; s += 64) {
        const int r = s + lane;
        const float y = L.f1(r < r1 ? 4u * r : OOB);
        const float wt = r < r1 ? expf((y - M) * inv_t) : 0.0f;
        const float c = base + wave_scan_incl(wt);
        const unsigned long long hit = __ballot(wt > 0.0f && c > target);
        if (hit) return s + __builtin_ctzll(hit);
        const unsigned long long any = __ballot(wt > 0.0f);
        if (any) last = s + 63 - __builtin_clzll(any);
        base = readlane(c, 63);
    }
    return last;
}

// Categorical draw from softmax(l / T) over n logits in index order, given
// per-block statistics (block b = rows [b*R, b*R+R): max bm[b], sum bs[b] of
// exp((l - bm[b]) / T)):  M = max bm, W_b = bs[b] exp((bm[b] - M) / T),
// target = u * sum W.  Thread t holds the W of its `per` consecutive blocks
// and their sum; a block-wide running sum over the threads finds the thread,
// the thread's own running sum the block, and wave 0's running sum over the
// block's rows the row.  Called by all NT threads; returns the row in every
// thread.
__device__ __forceinline__ int sample_select(const float* bm, const float* bs, int nb, int R, const float* logits, int n, float inv_t,
                             float u) {
    constexpr int BPT = 16;  // blocks per thread kept in registers
    __shared__ float slot[8];
    __shared__ float wsum[4];
    __shared__ int hit_t[4], last_t[4];
    __shared__ int sel_b;
    __shared__ float sel_rem;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const BufView BM(bm, (size_t)nb * 4), BS(bs, (size_t)nb * 4);
    const int per = (nb + NT - 1) / NT, b0 = min(nb, tid * per), b1 = min(nb, b0 + per);
    // the thread's blocks as one batch of loads (per <= BPT), M, their weights
    float xb[BPT], sb[BPT], wb[BPT];
    float m = -INFINITY, part = 0.0f;
    if (per <= BPT) {
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            const int b = b0 + j;
            xb[j] = BM.f1(b < b1 ? 4u * b : OOB);
            sb[j] = BS.f1(b < b1 ? 4u * b : OOB);
        }
#pragma unroll
        for (int j = 0; j < BPT; ++j) m = b0 + j < b1 ? fmaxf(m, xb[j]) : m;
    } else {
        for (int b = b0; b < b1; ++b) m = fmaxf(m, bm[b]);
    }
    const float M = block_max(m, slot);
    if (per <= BPT) {
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            wb[j] = b0 + j < b1 ? sb[j] * expf((xb[j] - M) * inv_t) : 0.0f;
            part += wb[j];
        }
    } else {
        for (int b = b0; b < b1; ++b) part += bs[b] * expf((bm[b] - M) * inv_t);
    }
    // threads in order: the first whose running sum passes the target
    const float c = wave_scan_incl(part);
    if (lane == 63) wsum[w] = c;
    __syncthreads();
    float base = 0.0f, Z = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        base += i < w ? wsum[i] : 0.0f;
        Z += wsum[i];
    }
    const float target = u * Z, incl = base + c;
    const unsigned long long hit = __ballot(part > 0.0f && incl > target);
    const unsigned long long any = __ballot(part > 0.0f);
    if (lane == 0) {
        hit_t[w] = hit ? 64 * w + __builtin_ctzll(hit) : -1;
        last_t[w] = any ? 64 * w + 63 - __builtin_clzll(any) : -1;
    }
    __syncthreads();
    int t_sel = -1, t_last = -1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (t_sel < 0) t_sel = hit_t[i];
        t_last = max(t_last, last_t[i]);
    }
    if (t_sel < 0) t_sel = max(t_last, 0);  // rounding: the target landed past the total (NaN: none, row 0)
    if (tid == t_sel) {
        float rem = target - (incl - part), acc = 0.0f;
        int bsel = -1, blast = b0;
        if (per <= BPT) {
#pragma unroll
            for (int j = 0; j < BPT; ++j) {
                if (bsel < 0 && b0 + j < b1) {
                    if (wb[j] > 0.0f) blast = b0 + j;
                    if (acc + wb[j] > rem && wb[j] > 0.0f) bsel = b0 + j;
                    else acc += wb[j];
                }
            }
        } else {
            for (int b = b0; b < b1 && bsel < 0; ++b) {
                const float wj = bs[b] * expf((bm[b] - M) * inv_t);
                if (wj > 0.0f) blast = b;
                if (acc + wj > rem && wj > 0.0f) bsel = b;
                else acc += wj;
            }
        }
        sel_b = bsel >= 0 ? bsel : blast;
        // rounding past the thread's total: the last positive row of its last positive block
        sel_rem = bsel >= 0 ? rem - acc : INFINITY;
    }
    __syncthreads();
    __shared__ int chosen;
    if (w == 0) {
        const int r0 = sel_b * R;
        const int row = wave_row_walk(logits, r0, min(n, r0 + R), M, inv_t, sel_rem);
        if (lane == 0) chosen = row;
    }
    __syncthreads();
    return chosen;
}

// ---- top-k sampling ----
// Keys are argmax_key(value, index): a larger key is a larger value, then a
// lower index, and 0 is below every real key.  A wave keeps the 64 best keys
// it has seen as a list sorted in descending order across its lanes
// (GH_TOP_K_MAX = 64, one key per lane).

__device__ __forceinline__ unsigned long long umin64(unsigned long long a, unsigned long long b) {
    return a < b ? a : b;
}

__device__ __forceinline__ unsigned long long shfl_u64(unsigned long long v, int src) {
    const unsigned lo = __shfl((unsigned)v, src, 64), hi = __shfl((unsigned)(v >> 32), src, 64);
    return ((unsigned long long)hi << 32) | lo;
}

template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)v, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(v >> 32), CTRL, 0xF, 0xF, false);
    return ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo;
}

// the key of lane ^ S: DPP inside 16-lane rows (S = 4 as a half-row mirror,
// lane ^ 7, then a quad reversal, lane ^ 3), a permute across rows
template <int S>
__device__ __forceinline__ unsigned long long lane_xor_u64(unsigned long long v) {
    if constexpr (S == 1) {
        return dpp_u64<DPP_QUAD_XOR1>(v);
    } else if constexpr (S == 2) {
        return dpp_u64<DPP_QUAD_XOR2>(v);
    } else if constexpr (S == 4) {
        return dpp_u64<0x1B>(dpp_u64<DPP_ROW_HALF_MIRROR>(v));  // quad_perm [3,2,1,0]
    } else if constexpr (S == 8) {
        return dpp_u64<DPP_ROW_ROR8>(v);
    } else {
        return shfl_xor_u64(v, S);
    }
}

// compare-exchange steps STRIDE, STRIDE/2, .., 1 of a bitonic network whose
// blocks of SIZE lanes sort descending (ascending if ASC) when SIZE = 64 and
// alternate below
template <int SIZE, int STRIDE, bool ASC>
__device__ __forceinline__ unsigned long long bitonic_steps(unsigned long long key, int lane) {
    const unsigned long long o = lane_xor_u64<STRIDE>(key);
    const bool desc = ((lane & SIZE) == 0) != ASC;
    key = (((lane & STRIDE) == 0) == desc) ? umax64(key, o) : umin64(key, o);
    if constexpr (STRIDE > 1) return bitonic_steps<SIZE, STRIDE / 2, ASC>(key, lane);
    return key;
}

template <bool ASC, int SIZE = 2>
__device__ __forceinline__ unsigned long long wave_sort(unsigned long long key, int lane) {
    key = bitonic_steps<SIZE, SIZE / 2, ASC>(key, lane);
    if constexpr (SIZE < 64) return wave_sort<ASC, SIZE * 2>(key, lane);
    return key;
}

// the 64 best of a descending list and an ascending one: their lane-wise max
// is a bitonic sequence holding them, which one half-cleaner cascade sorts
__device__ __forceinline__ unsigned long long wave_merge(unsigned long long desc, unsigned long long asc, int lane) {
    return bitonic_steps<64, 32, false>(umax64(desc, asc), lane);
}

// Streaming top-k of one wave: keys that beat the list's k-th key gather in
// a 128-key LDS buffer; each 64 of them are sorted and merged into the list.
struct WaveTopK {
    unsigned long long list = 0ull;  // descending, lane j = rank j
    unsigned long long thr = 0ull;   // a key must exceed this to matter
    unsigned long long floor = 0ull; // thr never drops below this bound
    int count = 0;                   // keys in the buffer
    unsigned long long* buf;

    __device__ __forceinline__ void flush(int k, int lane) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const unsigned long long g = lane < count ? buf[lane] : 0ull;
        const unsigned long long rest = lane + 64 < count ? buf[lane + 64] : 0ull;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane + 64 < count) buf[lane] = rest;
        count = max(0, count - 64);
        list = wave_merge(list, wave_sort<true>(g, lane), lane);
        thr = umax64(floor, shfl_u64(list, k - 1));
    }
    __device__ __forceinline__ void push(unsigned long long key, int k, int lane) {
        const bool pass = key > thr;
        const unsigned long long m = __ballot(pass);
        if (!m) return;
        if (pass) buf[count + __builtin_popcountll(m & ((1ull << lane) - 1ull))] = key;
        count += __builtin_popcountll(m);
        if (count >= 64) flush(k, lane);
    }
};

// the four waves' lists merged (one barrier; `lds` holds 256 keys and must
// not be reused before every thread has returned); every wave gets the result
__device__ __forceinline__ unsigned long long block_merge(unsigned long long list, unsigned long long* lds) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    lds[64 * w + 63 - lane] = list;  // reversed: ascending
    __syncthreads();
    list = lds[63 - lane];
#pragma unroll
    for (int i = 1; i < 4; ++i) list = wave_merge(list, lds[64 * i + lane], lane);
    return list;
}

__device__ __forceinline__ float key_value(unsigned long long key) {
    const unsigned ord = (unsigned)(key >> 32);
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord);
}

// Keys at or above `floor` among each thread's `VPT` keys, appended to
// cand[] in thread order (one LDS atomic per wave); returns after a barrier
// with every thread seeing the count.  `cnt` must be zero on entry to the
// barrier before the first call and is left holding the count.
template <int VPT>
__device__ __forceinline__ int block_compact(const unsigned long long (&key)[VPT], unsigned long long floor,
                                             unsigned long long* cand, int* cnt) {
    const int lane = threadIdx.x & 63;
    int mine = 0;
#pragma unroll
    for (int j = 0; j < VPT; ++j) mine += key[j] != 0ull && key[j] >= floor;
    int incl = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    int base = 0;
    if (lane == 63 && incl) base = atomicAdd(cnt, incl);
    int at = __shfl(base, 63, 64) + incl - mine;
#pragma unroll
    for (int j = 0; j < VPT; ++j)
        if (key[j] != 0ull && key[j] >= floor) cand[at++] = key[j];
    __syncthreads();
    return *cnt;
}

// Draw from softmax(l / T) restricted to the k largest logits (k <= 64;
// value descending, then lower index) by inversion in that rank order:
// weights exp((l_j - l_0) / T).  bm[b] is the max over rows [b*R, b*R+R) (R
// a multiple of 64).
//   1. The k tiles with the largest (max, -tile): the k-th largest of the
//      threads' own best tile keys bounds them from below (k threads hold a
//      tile at or above it), so only tiles at or above it are kept, then
//      streamed through each wave's top-k and merged.
//   2. Those tiles hold the k largest logits: each holds a logit >= the k-th
//      largest tile max m, so the k-th largest logit is >= m, while a logit
//      outside them is <= m, and if equal to m it lies in a later tile than
//      every chosen tile of max m, so at a higher row than logits it ties
//      with.  Their rows at or above m are kept and streamed the same way.
// Values arrive as one batch of loads per 4096.  Called by all NT threads;
// returns the row in every thread.
__device__ __forceinline__ int sample_top_k(const float* bm, int nb, int R, const float* logits, int n, int k,
                                            float inv_t, float u) {
    constexpr int CH = 4096;  // values per pass
    constexpr int VPT = CH / NT;
    __shared__ unsigned long long cand[CH];
    __shared__ unsigned long long bufs[4][128];
    __shared__ unsigned long long lists[3][NT];
    __shared__ int tiles[GH_TOP_K_MAX];
    __shared__ int cnt;
    __shared__ int chosen;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    k = max(1, min(k, min(GH_TOP_K_MAX, n)));
    WaveTopK s;
    s.buf = bufs[w];
    // 1. the k tiles
    const BufView B(bm, (size_t)nb * 4);
    for (int c0 = 0; c0 < nb; c0 += CH) {
        if (c0) __syncthreads();  // the previous pass is consumed
        if (tid == 0) cnt = 0;
        const int cn = min(CH, nb - c0);
        float v[VPT];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int e = tid + NT * j;
            v[j] = B.f1(e < cn ? 4u * (c0 + e) : OOB);
        }
        unsigned long long key[VPT], tmax = 0ull;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int e = tid + NT * j;
            key[j] = e < cn ? argmax_key(v[j], c0 + e) : 0ull;
            tmax = umax64(tmax, key[j]);
        }
        const unsigned long long tm = block_merge(wave_sort<false>(tmax, lane), lists[0]);
        const int nc = block_compact(key, shfl_u64(tm, k - 1), cand, &cnt);
        for (int g = w; g * 64 < nc; g += 4) {
            const int e = g * 64 + lane;
            s.push(e < nc ? cand[e] : 0ull, k, lane);
        }
    }
    if (s.count) s.flush(k, lane);
    const unsigned long long tl = block_merge(s.list, lists[1]);
    if (w == 0) tiles[lane] = (int)(0xFFFFFFFFu - (unsigned)tl);
    // 2. the k best rows of those tiles, counting only rows at or above the
    // k-th tile max
    const unsigned kth_ord = (unsigned)(shfl_u64(tl, k - 1) >> 32);
    const unsigned long long floor = kth_ord ? (unsigned long long)kth_ord << 32 : 1ull;
    s.list = 0ull;
    s.floor = s.thr = floor - 1ull;
    s.count = 0;
    const BufView L(logits, (size_t)n * 4);
    const int total = k * R;
    for (int c0 = 0; c0 < total; c0 += CH) {
        __syncthreads();  // tiles written; the previous pass is consumed
        if (tid == 0) cnt = 0;
        __syncthreads();
        const int cn = min(CH, total - c0);
        float v[VPT];
        int row[VPT];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int e = tid + NT * j, slot = min((c0 + e) / R, GH_TOP_K_MAX - 1);
            row[j] = tiles[slot] * R + (c0 + e - slot * R);
            v[j] = L.f1(e < cn && (unsigned)row[j] < (unsigned)n ? 4u * row[j] : OOB);
        }
        // (slots past the tiles that exist hold tile -1: negative rows)
        unsigned long long key[VPT];
#pragma unroll
        for (int j = 0; j < VPT; ++j)
            key[j] = tid + NT * j < cn && (unsigned)row[j] < (unsigned)n ? argmax_key(v[j], row[j]) : 0ull;
        const int nc = block_compact(key, floor, cand, &cnt);
        for (int g = w; g * 64 < nc; g += 4) {
            const int e = g * 64 + lane;
            s.push(e < nc ? cand[e] : 0ull, k, lane);
        }
    }
    if (s.count) s.flush(k, lane);
    const unsigned long long best = block_merge(s.list, lists[2]);
    // 3. inversion over ranks 0..k-1 (wave 0)
    if (w == 0) {
        const float v = key_value(best), v0 = readlane(v, 0);
        const float wt = lane < k && best != 0ull ? expf((v - v0) * inv_t) : 0.0f;
        const float c = wave_scan_incl(wt);
        const float target = u * readlane(c, 63);
        const unsigned long long hit = __ballot(wt > 0.0f && c > target);
        const unsigned long long any = __ballot(wt > 0.0f);
        const int pick = hit ? __builtin_ctzll(hit) : (any ? 63 - __builtin_clzll(any) : 0);
        const unsigned row = 0xFFFFFFFFu - (unsigned)__builtin_amdgcn_readlane((int)(unsigned)best, pick);
        if (lane == 0) chosen = row < (unsigned)n ? (int)row : 0;
    }
    __syncthreads();
    return chosen;
}

// (a template so that every translation unit that launches it has its copy)
template <int = 0>
__global__ __launch_bounds__(NT) void k_step_finish(StepState* st, int pos, const unsigned long long* cand, int n_cand,
                                                    const float* bm, const float* bs, int rows_per_cand,
                                                    const float* logits, int V, const int32_t* prompt, int32_t* ids) {
    __shared__ unsigned long long slot[4];
    // the step state and the prompt token at pos + 1 are read up front, so
    // their round trips overlap the key reduction
    const float inv_t = st->inv_temp;
    const int start = st->start, n_prompt = st->n_prompt, gen_count = st->gen_count, gen_cap = st->gen_cap;
    const int rel = pos + 1 - start;
    const bool from_prompt = prompt && rel >= 0 && rel < n_prompt;
    const int ptok = from_prompt ? prompt[rel] : 0;
    int tok;
    if (inv_t > 0.0f) {  // temperature sampling with a Philox draw keyed by the seed, counter = position
        const uint64_t seed = ((uint64_t)st->seed_hi << 32) | st->seed_lo;
        const float u = philox_uniform(seed, (uint64_t)pos);
        const int top_k = st->top_k;
        tok = top_k > 0 ? sample_top_k(bm, n_cand, rows_per_cand, logits, V, top_k, inv_t, u)
                        : sample_select(bm, bs, n_cand, rows_per_cand, logits, V, inv_t, u);
    } else {  // greedy: first maximum (sampleGreedy, examples/BenchmarkKVCache.hs:223-224)
        // the per-item keys as one batch of straight-line buffer loads (keys
        // past n_cand read zero, which no real key loses to)
        constexpr int KPT = 16;  // keys per thread in one round trip: 4096 items
        const BufView C(cand, (size_t)n_cand * 8);
        unsigned long long k[KPT];
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(C.r, 8u * (threadIdx.x + i * NT), 0, 0));
            k[i] = ((unsigned long long)v.y << 32) | v.x;
        }
        unsigned long long best = 0ull;
#pragma unroll
        for (int i = 0; i < KPT; ++i) best = umax64(best, k[i]);
        for (int i = threadIdx.x + KPT * NT; i < n_cand; i += NT) best = umax64(best, cand[i]);
        best = block_max_key(best, slot);
        tok = (int)(0xFFFFFFFFu - (unsigned)(best & 0xFFFFFFFFull));
    }
    if (threadIdx.x != 0) return;
    st->last = tok;
    int next = tok;
    if (from_prompt) {
        next = ptok;
    } else if (ids && gen_count < gen_cap) {
        ids[gen_count] = tok;
        st->gen_count = gen_count + 1;
    }
    st->token = next;
    st->pos = pos + 1;
}

#if GH_IN_TU(2)
// ------------------------------------------------------------------
// Persistent step (GH_PERSISTENT=1): the layers of one token as one kernel
// of one workgroup per CU, then the LM head and the finish kernel.
//
// Phases of layer l and who does them (W = workgroups = CUs):
//   A  QKV: 8-row groups of the fused matrix, round-robin over the
//      workgroups.  Every workgroup first updates its own copy of the
//      residual stream x (x = x1 + postnorm(d), d from phase E) and norms it.
//   B  attention: chunk items (kv group, chunk) on workgroups 0.. (q/k/v of
//      the group from phase A; QK-norm, RoPE, KV append, split-K chunk state).
//   B2 merge: (q head, 64-dim slice) items on the last workgroups: the chunk
//      states of the head -> its attention output slice.
//   C  O projection: 8-row groups (input: the merged output).
//   D  every workgroup: x1 = x + postnorm(o) and n2 = norm(x1); the 64-row
//      chunks of the gate/up matrix interleaved as 32 gate + 32 up rows (so a
//      chunk yields 32 GeGLU values) go round-robin to the workgroups after
//      the attention items' (first chunk c0, then c0 + W, ...), each
//      multiplied into the matching 32-column block of the down matrix: one
//      down partial P_c0[H] per workgroup.  The first chunk's weights are
//      staged in LDS during phase C, and its gate/up rows run on the matrix
//      cores.
//   E  down reduction: 8-row groups of H summed over the partials.
// Phases exchange their outputs as self-validating 64-bit words (epoch <<
// 32 | float bits; st_word / ld_word): a consumer polls exactly the words
// it needs, all loads of a batch issued before any check (ps_poll), so an
// exchange costs about one round trip after the producer's store.  Each
// workgroup keeps x and x1 in LDS; what crosses workgroups per layer is
// q/k/v, the chunk states, the merged output, the O rows, the partials and
// the down rows.  A phase's buffer is rewritten one layer later, after a
// dependency chain through all of its readers.  Every wait is bounded
// (StepState::xchg_err; once set, every wait returns at once).
// ------------------------------------------------------------------
struct PLayer {
    DMat qkv, o, gi, down;  // gi: gate/up interleaved in 64-row chunks (32 gate, 32 up rows)
    const float* attn_norm;
    const float* q_norm;
    const float* k_norm;
    const float* post_attn;
    const float* ffn_norm;
    const float* post_ffw;
    float* kc;
    float* vc;
    int global;
    int pad;
};

struct PArgs {
    const PLayer* layers;
    DMat embd;
    const float* out_norm;
    StepState* st;
    int pos;
    uint32_t tick;  // epoch of layer l = tick * (L + 1) + l + 1
    const float* rope_local;
    const float* rope_global;
    uint64_t* w_qkv;  // [q_rows_pad + 2 kv_rows_pad] raw q | k | v rows
    uint64_t* w_st;   // [nkv][nc][G][HD + 2] chunk states
    uint64_t* w_o;    // [nq * HD] merged attention output
    uint64_t* w_a;    // [H] O-projection rows
    uint64_t* w_p;    // [np][H] down partials
    uint64_t* w_d;    // [H] down rows
    float* xn_final;  // [H] normed final state (plain stores; read by the LM head kernel)
    float* layer_out; // [L][H]
    int L, H, nq, nkv, q_rows_pad, kv_rows_pad, n_chunks, nc, np, land;
    int pf_gu, pf_down, pf_off;  // phase D weights staged in LDS (at float pf_off of the dynamic LDS)
    float eps, escale, scale;
    int zc, use_qk_norm, post_attn_norm, post_ffn_norm, mode, window;
    int pb[2], pe[2], ch[2], n_used[2];  // attention range at pos: [0] local, [1] global layer
    uint32_t* host_tick;                 // host-side launch counter (not used on the device)
    // position-dependent arguments of one replay: position, a fresh epoch
    // base, and the attention range of local and global layers
    void set_pos(int p) {
        pos = p;
        tick = ++*host_tick;
        for (int t = 0; t < 2; ++t) {
            AttnArgs r{};
            r.global = t;
            r.window = window;
            r.mode = mode;
            r.nc = nc;
            r.set_pos(p);
            pb[t] = r.pb;
            pe[t] = r.pe;
            ch[t] = r.ch;
            n_used[t] = r.n_used;
        }
    }
};

static int enqueue_head(gh_model* m, gh_kv* kv, Sink& sink, int pos);  // LM head + finish (below)

constexpr int PS_PW = 8;    // words per thread per poll batch
constexpr int PS_MAXP = 3;  // (block, row) pairs per thread of an 8-row group: K <= 3072
constexpr int PS_MG = 3;    // float4 groups per thread of an H-vector: H <= 3072
constexpr int PS_KR = 10;   // down-partial rows per thread: H <= 2560

__device__ __forceinline__ bool ps_failed(int* err) {
    return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// dst[i] <- the float of word addr(i), i < n, once that word carries epoch
// e.  Each thread issues the loads of its batch of PS_PW words before it
// checks any; stale words are polled again, all of them per round.  The
// caller synchronises before reading dst.
template <class Addr>
__device__ void ps_poll(int n, Addr addr, uint32_t e, float* dst, int* err) {
    for (int base = 0; base < n; base += PS_PW * NT) {
        uint64_t v[PS_PW];
#pragma unroll
        for (int k = 0; k < PS_PW; ++k) {
            const int i = base + (int)threadIdx.x + k * NT;
            v[k] = i < n ? ld_word(addr(i)) : (uint64_t)e << 32;
        }
        uint32_t pend = 0;
#pragma unroll
        for (int k = 0; k < PS_PW; ++k) {
            const int i = base + (int)threadIdx.x + k * NT;
            if ((uint32_t)(v[k] >> 32) == e) {
                if (i < n) dst[i] = __uint_as_float((uint32_t)v[k]);
            } else {
                pend |= 1u << k;
            }
        }
        for (int spin = 1; pend; ++spin) {
            if (spin >= XCHG_SPIN) {
                __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if ((spin & 63) == 0 && ps_failed(err)) break;
#pragma unroll
            for (int k = 0; k < PS_PW; ++k)
                if (pend >> k & 1u) v[k] = ld_word(addr(base + (int)threadIdx.x + k * NT));
#pragma unroll
            for (int k = 0; k < PS_PW; ++k) {
                if ((pend >> k & 1u) && (uint32_t)(v[k] >> 32) == e) {
                    dst[base + threadIdx.x + k * NT] = __uint_as_float((uint32_t)v[k]);
                    pend &= ~(1u << k);
                }
            }
        }
    }
}

// Sum of squares of LDS v[0, n) over the workgroup (one barrier; slot: 4 floats).
__device__ __forceinline__ float ps_sumsq(const float* v, int n, float* slot) {
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += NT) s += v[i] * v[i];
    return block_sum(s, slot);
}

// Residual add and the RMS of its result from one block reduction (the
// prologue ProResid's algebra): this thread's float4 groups t + 256 k of
// x = b + postnorm(d) into xv (b, d in LDS; the post-norm weight groups wp
// apply when pn), returning 1 / rms(x).  With e = d * w' and c = 1/rms(d):
// sum x^2 = sum b^2 + 2 c sum b e + c^2 sum e^2.  slot: 16 floats of LDS.
__device__ __forceinline__ float ps_resid_norm(const float* b, const float* d, const float4 (&wp)[PS_MG], bool pn,
                                               int H, float eps, int zc, float* slot, float4 (&xv)[PS_MG]) {
    const int ng4 = H >> 2;
    float4 dv[PS_MG];
    float dd = 0.0f, bb = 0.0f, be = 0.0f, ee = 0.0f;
#pragma unroll
    for (int k = 0; k < PS_MG; ++k) {
        const int gi = threadIdx.x + k * NT;
        dv[k] = f4z();
        xv[k] = f4z();
        if (gi < ng4) {
            dv[k] = ((const float4*)d)[gi];
            xv[k] = ((const float4*)b)[gi];
            const float4 w1 = zc ? make_float4(1.0f + wp[k].x, 1.0f + wp[k].y, 1.0f + wp[k].z, 1.0f + wp[k].w) : wp[k];
            const float4 ev = pn ? make_float4(dv[k].x * w1.x, dv[k].y * w1.y, dv[k].z * w1.z, dv[k].w * w1.w) : dv[k];
            dd += dot4(dv[k], dv[k]);
            bb += dot4(xv[k], xv[k]);
            be += dot4(xv[k], ev);
            ee += dot4(ev, ev);
        }
    }
    const float4 t = block_sum4(make_float4(dd, bb, be, ee), slot);
    const float c = pn ? 1.0f / sqrtf(t.x / (float)H + eps) : 1.0f;
#pragma unroll
    for (int k = 0; k < PS_MG; ++k) xv[k] = xv[k] + (pn ? norm4i(dv[k], c, wp[k], zc) : dv[k]);
    const float sxx = fmaxf(t.y + 2.0f * c * t.z + c * c * t.w, 0.0f);
    return 1.0f / sqrtf(sxx / (float)H + eps);
}

// xs/sxs <- src[0, K) (LDS), normed by inv and (1 + w) / w when w is given,
// in the VALU Q4_0 input format (emit_x4).
__device__ __forceinline__ void ps_emit(const MvLds& L, const float* src, int K, float inv, const float* w, int zc) {
    const int ng = K >> 2;
    for (int b = 0; b < ng; b += NT) {
        const int gi = b + threadIdx.x;
        float4 v = f4z();
        if (gi < ng) {
            v = ((const float4*)src)[gi];
            if (w) v = norm4i(v, inv, ((const float4*)w)[gi], zc);
        }
        emit_x4<FMT_Q4>(L, gi, ng, v);
    }
}

// Weights of 8-row group grp (rows 8 grp .. 8 grp + 7) of a tiled Q4_0
// matrix: thread t holds the pairs p = t + 256 k, block p / 8 of row p % 8
// (8 consecutive lanes read one 128-byte line); pairs past the matrix read
// zeros.
struct RowRegs {
    u32x4 c[PS_MAXP];
    uint16_t s[PS_MAXP];
};

__device__ __forceinline__ void rg_load(RowRegs& R, const DMat& W, const MatViews& V, int grp) {
    const int row0 = grp * 8;
    const uint32_t tb = (uint32_t)(row0 >> 7) * (uint32_t)W.nblk * TILE_ROWS + (uint32_t)(row0 & 127);
#pragma unroll
    for (int k = 0; k < PS_MAXP; ++k) {
        const int p = threadIdx.x + k * NT, kb = p >> 3;
        const uint32_t e = tb + (uint32_t)kb * TILE_ROWS + (uint32_t)(p & 7);
        const bool ok = kb < W.nblk;
        R.c[k] = V.codes.template u4<CP_NT>(ok ? e * 16u : OOB);
        R.s[k] = V.scales.template h1<CP_NT>(ok ? e * 2u : OOB);
    }
}

// The group's 8 dot products with the slice in xs/sxs; thread r < 8 returns
// row r's (the others return 0).  Two barriers (red: 32 floats of LDS).
__device__ __forceinline__ float rg_dot(const RowRegs& R, int nblk, const MvLds& L, float* red) {
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < PS_MAXP; ++k) {
        const int kb = (threadIdx.x + k * NT) >> 3;
        if (kb < nblk) {
            const float4* xv = (const float4*)(L.xs + kb * 32);
            const uint32_t w[4] = {R.c[k].x, R.c[k].y, R.c[k].z, R.c[k].w};
            float d = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) d = dot_q4_word(w[j], xv[j], xv[4 + j], d);
            acc = fmaf(h2f(R.s[k]), d - 8.0f * L.sxs[kb], acc);
        }
    }
    acc += __shfl_xor(acc, 8, 64);
    acc += __shfl_xor(acc, 16, 64);
    acc += __shfl_xor(acc, 32, 64);
    const int lane = threadIdx.x & 63;
    if (lane < 8) red[(threadIdx.x >> 6) * 8 + lane] = acc;
    __syncthreads();
    const float y = threadIdx.x < 8 ? (red[threadIdx.x] + red[8 + threadIdx.x]) + (red[16 + threadIdx.x] + red[24 + threadIdx.x])
                                    : 0.0f;
    __syncthreads();
    return y;
}

// q | k | v rows of this token as published words: issue() starts the
// loads of a float4 group's 4 words early (before the K/V loads), settle()
// waits until every group of the thread carries the step's epoch (stale
// words are polled again together, bounded), get() returns a group.
struct QkvPoll {
    const uint64_t* w;
    uint32_t e;
    int* err;
    struct Pre {
        uint64_t v[4];
    };
    __device__ void issue(Pre& p, int row, bool ok) const {
#pragma unroll
        for (int j = 0; j < 4; ++j) p.v[j] = ok ? ld_word(w + row + j) : (uint64_t)e << 32;
    }
    template <int M>
    __device__ void settle(Pre (&p)[M], const int (&row)[M]) const {
        uint32_t pend = 0;
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if ((uint32_t)(p[m].v[j] >> 32) != e) pend |= 1u << (4 * m + j);
        for (int spin = 1; pend; ++spin) {
            if (spin >= XCHG_SPIN) {
                __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if ((spin & 63) == 0 && ps_failed(err)) break;
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (pend >> (4 * m + j) & 1u) p[m].v[j] = ld_word(w + row[m] + j);
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if ((pend >> (4 * m + j) & 1u) && (uint32_t)(p[m].v[j] >> 32) == e) pend &= ~(1u << (4 * m + j));
        }
    }
    __device__ float4 get(const Pre& p, int) const {
        return make_float4(__uint_as_float((uint32_t)p.v[0]), __uint_as_float((uint32_t)p.v[1]),
                           __uint_as_float((uint32_t)p.v[2]), __uint_as_float((uint32_t)p.v[3]));
    }
};

// LDS scratch of the persistent step (floats after the matvec region).
struct PsLds {
    float* xr;    // [H] residual stream entering the layer
    float* x1;    // [H] residual after attention
    float* land;  // [a.land] polled words
    float* red;   // [64] reductions
    float* gu;    // [64] gate/up rows of a chunk
};

// Phase D input, run by every workgroup: poll the O rows, x1 = x +
// postnorm(o) (kept for the next layer), xs = norm(x1) with the pre-FFN
// weight (ffn_norm, else post_attention_norm: src/Gemma/Model.hs:337-339).
struct ProFfnPs {
    const uint64_t* w_a;
    const float* post_attn;  // nullable: no post-attention norm
    const float* ffn_w;      // pre-FFN norm weight
    PsLds S;
    uint32_t e;
    int* err;
    int H, zc;
    float eps;
    struct Regs {
        float4 wp[PS_MG], wf[PS_MG];
    };
    __device__ void load(Regs& r, int, int) const {
        const int ng4 = H >> 2;
        const BufView WP(post_attn, post_attn ? (size_t)H * 4 : 0), WF(ffn_w, (size_t)H * 4);
#pragma unroll
        for (int b = 0; b < PS_MG; ++b) {
            const int gi = threadIdx.x + b * NT;
            r.wp[b] = WP.f4(gi < ng4 ? 16u * gi : OOB);
            r.wf[b] = WF.f4(gi < ng4 ? 16u * gi : OOB);
        }
    }
    template <int FMT>
    __device__ void finish(const MvLds& L, Regs& r, int, int) const {
        const int ng4 = H >> 2;
        const uint64_t* wa = w_a;
        ps_poll(H, [=](int i) { return wa + i; }, e, S.land, err);
        __syncthreads();
        float4 xv[PS_MG];
        const float inv2 = ps_resid_norm(S.xr, S.land, r.wp, post_attn != nullptr, H, eps, zc, S.red + 48, xv);
#pragma unroll
        for (int b = 0; b < PS_MG; ++b) {
            const int gi = threadIdx.x + b * NT;
            if (gi < ng4) ((float4*)S.x1)[gi] = xv[b];
        }
#pragma unroll
        for (int b = 0; b < PS_MG; ++b) {
            const int gi = threadIdx.x + b * NT;
            emit_x4<FMT>(L, gi, ng4, gi < ng4 ? norm4i(xv[b], inv2, r.wf[b], zc) : f4z());
        }
    }
};

// Gate/up chunk output rows into LDS (64 rows: gate 0..31, up 32..63).
struct EpiLdsRows {
    float* y;
    struct Regs {};
    __device__ void load(Regs&) const {}
    template <int RL>
    __device__ void run(const MvLds&, const Regs&, int, int, int, float y0, float) const {
        y[threadIdx.x & 63] = y0;
    }
};

// Phase D weights staged in LDS ahead of the phase (floats from the region
// base): the gate/up chunk's codes [nb][64 rows][16 B] (gc) and scales
// [nb][64][2 B] (gs); with the down block, its codes [rows][16 B] (dc) and
// scales [rows][2 B] (ds).  Each part is whole 1 KiB wave loads.
struct PfLayout {
    int gc, gs, dc, ds, total;
};
__host__ __device__ inline PfLayout pf_layout(int nb, int down_tiles, bool down) {
    PfLayout p;
    p.gc = 0;
    p.gs = nb * 256;
    p.dc = p.gs + (nb + 7) / 8 * 256;
    p.ds = p.dc + (down ? 2 * down_tiles * 256 : 0);
    p.total = p.ds + (down ? (down_tiles + 3) / 4 * 256 : 0);
    return p;
}

// 16 bytes per lane from a buffer view straight into LDS: lane i's bytes
// land at dst + 16 i (dst wave-uniform); offsets outside the view write zeros.
__device__ __forceinline__ void lds_dma16(const BufView& v, uint32_t off, float* dst) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(v.r, (__attribute__((address_space(3))) void*)dst, 16, off, 0, 0, CP_NT);
}

// Issue the staging of chunk c (gate/up rows 64c .. 64c + 63 of the
// interleaved matrix: tile c / 2, half c % 2) and, with `down`, of column
// block c of the down matrix.  The loads are only issued here; the next
// wait on this workgroup's vector memory (the O-row poll) covers them.
__device__ void ps_prefetch(const PLayer& P, int c, float* pf, bool down) {
    const PfLayout Y = pf_layout(P.gi.nblk, P.down.tiles, down);
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const MatViews G(P.gi);
    const uint32_t nb = (uint32_t)P.gi.nblk, t = (uint32_t)(c >> 1), rh = (uint32_t)(c & 1) * 64u;
    for (int kb = wave; kb < (int)nb; kb += 4)
        lds_dma16(G.codes, ((t * nb + (uint32_t)kb) * TILE_ROWS + rh + (uint32_t)lane) * 16u, pf + Y.gc + kb * 256);
    for (int i = wave; i < ((int)nb + 7) / 8; i += 4) {
        const uint32_t kb = (uint32_t)(8 * i + (lane >> 3));
        lds_dma16(G.scales, kb < nb ? ((t * nb + kb) * TILE_ROWS + rh) * 2u + (uint32_t)(lane & 7) * 16u : OOB,
                  pf + Y.gs + i * 256);
    }
    if (down) {
        const MatViews D(P.down);
        const uint32_t nd = (uint32_t)P.down.nblk, td = (uint32_t)P.down.tiles, cc = (uint32_t)c;
        for (int j = wave; j < 2 * (int)td; j += 4)
            lds_dma16(D.codes, (((uint32_t)(j >> 1) * nd + cc) * TILE_ROWS + (uint32_t)(j & 1) * 64u + (uint32_t)lane) * 16u,
                      pf + Y.dc + j * 256);
        for (int i = wave; i < ((int)td + 3) / 4; i += 4) {
            const uint32_t tt = (uint32_t)(4 * i + (lane >> 4));
            lds_dma16(D.scales, tt < td ? (tt * nd + cc) * TILE_ROWS * 2u + (uint32_t)(lane & 15) * 16u : OOB,
                      pf + Y.ds + i * 256);
        }
    }
}

// The staged chunk's 64 gate/up rows on the int8 matrix cores, against the
// whole-row slice in xs/sxs in the FMT_Q4M limb format (L.zero cleared):
// wave w takes rows 16w .. 16w + 15, one MFMA pair per quad of column
// blocks with the operands and combination of mq_quad, the codes and
// scales read from the staged LDS copy (blocks past nb: zero codes and
// scales against zero limbs).
__device__ void ps_gu_lds_mfma(const float* pf, int nb, const MvLds& L, float* y) {
    const PfLayout Y = pf_layout(nb, 0, false);
    const int wave = wave_id(), lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4, r16 = 16 * wave;
    const u32x4* cw = (const u32x4*)(pf + Y.gc);
    const uint16_t* sw = (const uint16_t*)(pf + Y.gs);
    const bool act = (n >> 2) == g;
    const i32x4* zero = (const i32x4*)L.zero;
    float acc = 0.0f;
    const int nq = (nb + 3) >> 2;
    for (int q = 0; q < nq; ++q) {
        const int ka = 4 * q + g;
        const u32x4 c = ka < nb ? cw[ka * 64 + r16 + n] : (u32x4){0u, 0u, 0u, 0u};
        const uint16_t sc = ka < nb ? sw[ka * 64 + r16 + n] : (uint16_t)0;
        const i32x4* lb = (const i32x4*)L.xs + ((4 * q + g) * 8 + (n & 3));
        const i32x4 b0 = *(act ? lb : zero), b1 = *(act ? lb + 4 : zero);
        const float mq = L.sxs[4 * q + g];
        i32x4 alo, ahi;
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // 16 * (q - 8) as int8: q ^ 8 is q - 8 as a signed nibble
            ahi[k] = (int)((c[k] ^ 0x80808080u) & 0xF0F0F0F0u);
            alo[k] = (int)(((c[k] << 4) ^ 0x80808080u) & 0xF0F0F0F0u);
        }
        i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(b0, alo, (i32x4){0, 0, 0, 0}, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(b1, ahi, d, 0, 0, 0);
        const int lo01 = d[0] + d[1] * 128, hi23 = d[2] + d[3] * 128;
        acc = fmaf(fmaf((float)hi23, 16384.0f, (float)lo01), h2f(sc) * mq, acc);
    }
    // sum the four blocks of each row; lane m < 16 then holds row m
    acc += __shfl_xor(acc, 32, 64);
    acc += __shfl_xor(acc, 16, 64);
    if (lane < 16) L.red[r16 + lane] = acc;
    __syncthreads();
    if (wave == 0) y[lane] = L.red[lane];
}

template <int HD, int G, int KBW>
__global__ __launch_bounds__(NT) void k_step_ps(PArgs a) {
    extern __shared__ float lds[];
    const int nwg = gridDim.x, wg = blockIdx.x, tid = threadIdx.x;
    int* err = &a.st->xchg_err;
    const int H = a.H, QK = a.nq * HD;
    const int nbx = (H > QK ? H : QK) / 32;
    const MvLds L = mv_lds<FMT_Q4>(lds, nbx);
    PsLds S;
    S.xr = lds + 512 + 64 + ((nbx + 3) & ~3) * 33 + 4;  // after the matvec region (mv_lds_floats, Q4_0)
    S.x1 = S.xr + H;
    S.land = S.x1 + H;
    S.red = S.land + a.land;
    S.gu = S.red + 64;
    float* const pf = lds + a.pf_off;
    const float eps = a.eps;
    const int zc = a.zc;

    // layer-0 input, in every workgroup: x = E[token] * sqrt(H) (Embedding.hs:30-64, Model.hs:1357-1361)
    {
        const int tok = min(max(a.st->token, 0), a.embd.rows - 1);
        for (int i = 4 * tid; i < H; i += 4 * NT) {
            const float4 ev = dq_elem4(a.embd, tok, i);
            *(float4*)&S.xr[i] = make_float4(ev.x * a.escale, ev.y * a.escale, ev.z * a.escale, ev.w * a.escale);
        }
    }
    __syncthreads();

    const float* prev_post_ffw = nullptr;  // post-FFN norm weight of layer l - 1
    for (int l = 0; l < a.L; ++l) {
        const PLayer P = a.layers[l];  // one scalar-load burst, in flight with the layer's first wait
        // The exchange buffers' addresses are re-derived in every layer (the
        // empty asm hides that they do not change): per-thread addresses built
        // from them would otherwise be hoisted out of the layer loop and held
        // in registers for the whole kernel.
        uint64_t *w_qkv = a.w_qkv, *w_st = a.w_st, *w_o = a.w_o, *w_a = a.w_a, *w_p = a.w_p, *w_d = a.w_d;
        float* layer_out = a.layer_out;
        asm volatile("" : "+s"(w_qkv), "+s"(w_st), "+s"(w_o), "+s"(w_a), "+s"(w_p), "+s"(w_d), "+s"(layer_out));
        const uint32_t e = a.tick * (uint32_t)(a.L + 1) + (uint32_t)l + 1u;
        // ---------------- A: residual update, pre-attention norm, QKV rows
        {
            const int ngrp = P.qkv.tiles * (TILE_ROWS / 8);
            const MatViews V(P.qkv);
            RowRegs R;
            rg_load(R, P.qkv, V, wg);  // out of range: zeros, no traffic
            // the norm weights of this thread's float4 groups, in flight with the weights
            const int ng4 = H >> 2;
            const bool pn = l > 0 && a.post_ffn_norm && prev_post_ffw;
            const BufView WP(pn ? prev_post_ffw : nullptr, pn ? (size_t)H * 4 : 0), WN(P.attn_norm, (size_t)H * 4);
            float4 wpv[PS_MG], wnv[PS_MG];
#pragma unroll
            for (int b = 0; b < PS_MG; ++b) {
                const int gi = tid + b * NT;
                wpv[b] = WP.f4(gi < ng4 ? 16u * gi : OOB);
                wnv[b] = WN.f4(gi < ng4 ? 16u * gi : OOB);
            }
            float4 xv[PS_MG];
            float inv;  // 1 / rms of the layer's input x
            if (l > 0) {
                const uint64_t* wd = w_d;
                ps_poll(H, [=](int i) { return wd + i; }, e - 1u, S.land, err);
                __syncthreads();
                inv = ps_resid_norm(S.x1, S.land, wpv, pn, H, eps, zc, S.red + 48, xv);
#pragma unroll
                for (int b = 0; b < PS_MG; ++b) {
                    const int gi = tid + b * NT;
                    if (gi < ng4) {
                        ((float4*)S.xr)[gi] = xv[b];
                        if (wg == 0)
                            *(__attribute__((address_space(1))) f32x4*)(layer_out + (size_t)(l - 1) * H + 4 * gi) =
                                __builtin_bit_cast(f32x4, xv[b]);
                    }
                }
            } else {
                float ss = 0.0f;
#pragma unroll
                for (int b = 0; b < PS_MG; ++b) {
                    const int gi = tid + b * NT;
                    xv[b] = gi < ng4 ? ((const float4*)S.xr)[gi] : f4z();
                    ss += dot4(xv[b], xv[b]);
                }
                inv = 1.0f / sqrtf(block_sum(ss, S.red + 4) / (float)H + eps);
            }
#pragma unroll
            for (int b = 0; b < PS_MG; ++b) {
                const int gi = tid + b * NT;
                emit_x4<FMT_Q4>(L, gi, ng4, gi < ng4 ? norm4i(xv[b], inv, wnv[b], zc) : f4z());
            }
            __syncthreads();
            for (int grp = wg; grp < ngrp; grp += nwg) {
                if (grp != wg) rg_load(R, P.qkv, V, grp);
                const float y = rg_dot(R, P.qkv.nblk, L, S.red + 8);
                if (tid < 8) st_word(w_qkv + grp * 8 + tid, e, y);
            }
        }
        // ---------------- B: attention chunks
        const int gsel = P.global ? 1 : 0;
        const int nu = a.n_used[gsel];
        // FFN chunks start past the attention items' workgroups (chunk c on
        // workgroup (c + items) mod W), so that an attention workgroup's
        // staging loads do not delay its O-row poll; c0 = this workgroup's first
        const int n_att = a.nkv * nu;
        const int c0 = ((wg - n_att) % nwg + nwg) % nwg;
        const bool staged = a.pf_gu && c0 < a.n_chunks;  // chunk c0's phase D weights go through LDS
        {
            AttnArgs aa{};
            aa.q_off = 0;
            aa.k_off = a.q_rows_pad;
            aa.v_off = a.q_rows_pad + a.kv_rows_pad;
            aa.q_norm = P.q_norm;
            aa.k_norm = P.k_norm;
            aa.use_qk_norm = a.use_qk_norm && P.q_norm && P.k_norm;
            aa.zc = zc;
            aa.eps = eps;
            aa.rope = (a.mode == GH_MODE_REF || P.global) ? a.rope_global : a.rope_local;
            aa.pos = a.pos;
            aa.global = P.global;
            aa.window = a.window;
            aa.mode = a.mode;
            aa.kc = P.kc;
            aa.vc = P.vc;
            aa.nkv = a.nkv;
            aa.scale = a.scale;
            aa.nc = a.nc;
            aa.pb = a.pb[gsel];
            aa.pe = a.pe[gsel];
            aa.ch = a.ch[gsel];
            aa.n_used = nu;
            for (int it = wg; it < a.nkv * nu; it += nwg) {
                const int g = it / nu, j = it % nu;
                attn_item<HD, G, true>(aa, g, j, QkvPoll{w_qkv, e, err}, AttnOutWords{w_st, e});
                __syncthreads();
            }
        }
        // ---------------- B2: merge of the chunk states
        {
            constexpr int SL = HD < 64 ? HD : 64;
            const int nsl = HD / SL, nitem = a.nq * nsl;
            const size_t stride = (size_t)G * (HD + 2);
            for (int it = nwg - 1 - wg; it >= 0 && it < nitem; it += nwg) {
                const int h = it / nsl, d0 = (it % nsl) * SL, g = h / G, hl = h % G;
                const uint64_t* base = w_st + (size_t)g * a.nc * stride;
                // land: m[nu] | l[nu] | o[nu][SL]
                ps_poll(nu * (2 + SL), [=](int i) {
                    if (i < nu) return base + (size_t)i * stride + hl;
                    if (i < 2 * nu) return base + (size_t)(i - nu) * stride + G + hl;
                    const int j = (i - 2 * nu) / SL, d = (i - 2 * nu) % SL;
                    return base + (size_t)j * stride + 2 * G + (size_t)hl * HD + d0 + d;
                }, e, S.land, err);
                __syncthreads();
                if (tid < SL) {
                    float M = -INFINITY;
                    for (int j = 0; j < nu; ++j) M = fmaxf(M, S.land[j]);
                    float den = 0.0f, o = 0.0f;
                    for (int j = 0; j < nu; ++j) {
                        const float w = __expf(S.land[j] - M);
                        den += S.land[nu + j] * w;
                        o += w * S.land[2 * nu + j * SL + tid];
                    }
                    st_word(w_o + (size_t)h * HD + d0 + tid, e, o / den);
                }
                __syncthreads();
            }
        }
        // this workgroup's attention and merge waits are behind it: stage its
        // phase D weights now, so they stream during phase C
        if (staged) ps_prefetch(P, c0, pf, a.pf_down != 0);
        // ---------------- C: O projection rows
        {
            const int ngrp = H / 8;
            if (wg < ngrp) {
                const MatViews V(P.o);
                RowRegs R;
                rg_load(R, P.o, V, wg);
                const uint64_t* wo = w_o;
                ps_poll(QK, [=](int i) { return wo + i; }, e, S.land, err);
                __syncthreads();
                ps_emit(L, S.land, QK, 1.0f, nullptr, zc);
                __syncthreads();
                for (int grp = wg; grp < ngrp; grp += nwg) {
                    if (grp != wg) rg_load(R, P.o, V, grp);
                    const float y = rg_dot(R, P.o.nblk, L, S.red + 8);
                    if (tid < 8) st_word(w_a + grp * 8 + tid, e, y);
                }
            }
        }
        // ---------------- D: post-attention residual, pre-FFN norm, gate/up chunks, down partial
        {
            ProFfnPs pro{w_a, a.post_attn_norm ? P.post_attn : nullptr, P.ffn_norm ? P.ffn_norm : P.post_attn,
                         S, e, err, H, zc, eps};
            float part[PS_KR];  // this thread's rows t + 256 k of the down partial
#pragma unroll
            for (int k = 0; k < PS_KR; ++k) part[k] = 0.0f;
            const MatViews VD(P.down);
            u32x4 dw[PS_KR];
            uint16_t ds[PS_KR];
            // down-column block c of this thread's rows: issued before the gate/up item
            auto load_down = [&](int c) {
#pragma unroll
                for (int k = 0; k < PS_KR; ++k) {
                    const int r = tid + k * NT;
                    const uint32_t el = ((uint32_t)(r >> 7) * (uint32_t)P.down.nblk + (uint32_t)c) * TILE_ROWS + (uint32_t)(r & 127);
                    dw[k] = VD.codes.template u4<CP_NT>(r < H ? el * 16u : OOB);
                    ds[k] = VD.scales.template h1<CP_NT>(r < H ? el * 2u : OOB);
                }
            };
            bool built = false;
            for (int c = c0; c < a.n_chunks; c += nwg) {
                const bool from_lds = staged && c == c0, down_lds = from_lds && a.pf_down;
                if (!down_lds) load_down(c);
                if (from_lds) {
                    ProFfnPs::Regs r0;
                    pro.load(r0, 0, H);
                    pro.template finish<FMT_Q4M>(L, r0, 0, H);
                    if (tid < 4) L.zero[tid] = 0.0f;
                    __syncthreads();
                    ps_gu_lds_mfma(pf, P.gi.nblk, L, S.gu);
                    built = true;
                } else if (!built || staged) {
                    // first chunk, or one after the staged chunk, whose slice is in the
                    // limb format: the prologue (re)builds the VALU-format slice
                    mv_item_valu<FMT_Q4, KBW, 1, 1>(P.gi, c, 0, 1, pro, EpiLdsRows{S.gu}, L);
                    built = true;
                } else {
                    mv_item_valu<FMT_Q4, KBW, 1, 1>(P.gi, c, 0, 1, ProKeep{}, EpiLdsRows{S.gu}, L);
                }
                __syncthreads();
                if (down_lds) {  // the staged down block of this thread's rows
                    const PfLayout Y = pf_layout(P.gi.nblk, P.down.tiles, true);
#pragma unroll
                    for (int k = 0; k < PS_KR; ++k) {
                        const int r = tid + k * NT;
                        if (r < H) {
                            dw[k] = ((const u32x4*)(pf + Y.dc))[r];
                            ds[k] = ((const uint16_t*)(pf + Y.ds))[r];
                        }
                    }
                }
                // GeGLU of the chunk's 32 rows (MLP.hs:384-447) as a Q4_0 input block: h[0..31] in
                // the emit format (16..31 scaled by 1/16) and sum(h)
                float* hb = S.gu + 64;
                if (tid < 64) {  // wave 0, all lanes (the sum is a wave reduction)
                    const float hv = tid < 32 ? gelu_tanh(S.gu[tid]) * S.gu[32 + tid] : 0.0f;
                    const float hsum = wave_sum(hv);
                    if (tid < 32) hb[tid] = tid < 16 ? hv : hv * 0.0625f;
                    if (tid == 0) hb[32] = hsum;
                }
                __syncthreads();
                const float4* hv4 = (const float4*)hb;
                const float hs8 = 8.0f * hb[32];
#pragma unroll
                for (int k = 0; k < PS_KR; ++k) {
                    if (tid + k * NT < H) {
                        float d = 0.0f;
                        d = dot_q4_word(dw[k].x, hv4[0], hv4[4], d);
                        d = dot_q4_word(dw[k].y, hv4[1], hv4[5], d);
                        d = dot_q4_word(dw[k].z, hv4[2], hv4[6], d);
                        d = dot_q4_word(dw[k].w, hv4[3], hv4[7], d);
                        part[k] = fmaf(h2f(ds[k]), d - hs8, part[k]);
                    }
                }
                __syncthreads();
            }
            if (!built) {  // no chunk here: x1 and n2 are still this workgroup's to keep
                ProFfnPs::Regs r0;
                pro.load(r0, 0, H);
                pro.template finish<FMT_Q4>(L, r0, 0, H);
                __syncthreads();
            } else {  // partial slot c0 (< np: every slot below np has its first chunk)
                uint64_t* pw = w_p + (size_t)c0 * H;
#pragma unroll
                for (int k = 0; k < PS_KR; ++k) {
                    const int r = tid + k * NT;
                    if (r < H) st_word(pw + r, e, part[k]);
                }
            }
        }
        // ---------------- E: down rows = sum of the partials
        {
            const int ngrp = H / 8;
            for (int grp = wg; grp < ngrp; grp += nwg) {
                // land[p * 8 + r] = partial p of row 8 grp + r
                const uint64_t* wp = w_p + grp * 8;
                ps_poll(a.np * 8, [=](int i) { return wp + (size_t)(i >> 3) * H + (i & 7); }, e, S.land, err);
                __syncthreads();
                float s = 0.0f;
                for (int i = tid; i < a.np * 8; i += NT) s += S.land[i];  // row i & 7 == tid & 7
                s += __shfl_xor(s, 8, 64);
                s += __shfl_xor(s, 16, 64);
                s += __shfl_xor(s, 32, 64);
                if ((tid & 63) < 8) S.red[16 + (tid >> 6) * 8 + (tid & 7)] = s;
                __syncthreads();
                if (tid < 8)
                    st_word(w_d + grp * 8 + tid, e,
                            (S.red[16 + tid] + S.red[24 + tid]) + (S.red[32 + tid] + S.red[40 + tid]));
                __syncthreads();
            }
        }
        prev_post_ffw = P.post_ffw;
    }
    // final residual and norm (workgroup 0): layer_out[L-1], xn_final for the LM head
    if (wg == 0) {
        const PLayer& Q = a.layers[a.L - 1];
        const uint32_t e = a.tick * (uint32_t)(a.L + 1) + (uint32_t)a.L;
        const uint64_t* wd = a.w_d;
        ps_poll(H, [=](int i) { return wd + i; }, e, S.land, err);
        __syncthreads();
        float inv = 1.0f;
        const bool pn = a.post_ffn_norm && Q.post_ffw;
        if (pn) inv = 1.0f / sqrtf(ps_sumsq(S.land, H, S.red) / (float)H + eps);
        for (int i = tid; i < H; i += NT) S.xr[i] = S.x1[i] + (pn ? norm_apply_inv(S.land[i], inv, Q.post_ffw[i], zc) : S.land[i]);
        __syncthreads();
        const float inv2 = 1.0f / sqrtf(ps_sumsq(S.xr, H, S.red + 4) / (float)H + eps);
        for (int i = tid; i < H; i += NT) {
            a.layer_out[(size_t)(a.L - 1) * H + i] = S.xr[i];
            a.xn_final[i] = norm_apply(S.xr[i], 1.0f / inv2, a.out_norm[i], zc);
        }
    }
}

// Interleave a layer's [gate | up] matrix (f_pad rows each) into 64-row
// chunks of 32 gate rows and the 32 up rows of the same FFN indices.
__global__ void k_interleave_gu(DMat gu, int f_pad, int F, DMat gi) {
    const size_t n = (size_t)gi.tiles * gi.nblk * TILE_ROWS;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
        const int rr = (int)(idx % TILE_ROWS);
        const size_t tk = idx / TILE_ROWS;
        const int kb = (int)(tk % gi.nblk), t = (int)(tk / gi.nblk);
        const int r = t * TILE_ROWS + rr, c = r / 64, i = r % 64;
        const int f = 32 * c + (i & 31);
        u32x4 code = {0u, 0u, 0u, 0u};
        uint16_t sc = 0;
        if (f < F) {
            const int src = (i < 32 ? 0 : f_pad) + f;
            const size_t sidx = ((size_t)(src >> 7) * gu.nblk + kb) * TILE_ROWS + (src & 127);
            code = ((const u32x4*)gu.codes)[sidx];
            sc = gu.scales[sidx];
        }
        ((u32x4*)gi.codes)[idx] = code;
        ((uint16_t*)gi.scales)[idx] = sc;
    }
}

int launch_interleave_gu(const DMat& gu, int f_pad, int F, const DMat& gi, hipStream_t s) {
    if (gu.fmt != FMT_Q4 || gi.fmt != FMT_Q4 || gu.nblk != gi.nblk)
        return set_error(GH_ERR_INVALID, "internal: gate/up interleave needs two Q4_0 matrices of one width");
    const size_t n = (size_t)gi.tiles * gi.nblk * TILE_ROWS;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(k_interleave_gu, dim3(blocks), dim3(256), 0, s, gu, f_pad, F, gi);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

// Per-cache table of layer pointers for the persistent step.
static int persistent_layers(gh_model* m, gh_kv* kv) {
    if (kv->d_players) return GH_OK;
    const gh_config& c = m->cfg;
    const size_t kv_layer = (size_t)kv->max_seq * c.n_kv_heads * c.head_dim;
    std::vector<PLayer> h(c.n_layers);
    for (int i = 0; i < c.n_layers; ++i) {
        const LayerDev& L = m->layers[i];
        PLayer& p = h[i];
        p.qkv = L.qkv;
        p.o = L.o;
        p.gi = m->p_gi[i];
        p.down = L.down;
        p.attn_norm = L.attn_norm;
        p.q_norm = L.q_norm;
        p.k_norm = L.k_norm;
        p.post_attn = L.post_attn;
        p.ffn_norm = L.ffn_norm;
        p.post_ffw = L.post_ffw;
        p.kc = kv->k + i * kv_layer;
        p.vc = kv->v + i * kv_layer;
        p.global = L.global ? 1 : 0;
        p.pad = 0;
    }
    void* d = nullptr;
    GH_HIP(hipMalloc(&d, sizeof(PLayer) * h.size()));
    if (hipMemcpy(d, h.data(), sizeof(PLayer) * h.size(), hipMemcpyHostToDevice) != hipSuccess) {
        hipFree(d);
        return set_error(GH_ERR_HIP, "upload of the persistent layer table failed");
    }
    kv->d_players = d;
    return GH_OK;
}

// Shapes the persistent step is built for: Q4_0 weights, head_dim 32 with
// group 4 (tiny), head_dim 256 with group 2 or 4 (4B, 1B); every K of a
// row-group matvec within 3072 and H within the down partial's registers.
int persistent_supported(const gh_model* m) {
    const gh_config& c = m->cfg;
    const int G = c.n_heads / c.n_kv_heads;
    if (m->fmt != FMT_Q4) return 0;
    const bool shape = (c.head_dim == 32 && G == 4) || (c.head_dim == 256 && (G == 2 || G == 4));
    return shape && c.hidden <= 2560 && c.n_heads * c.head_dim <= 3072 && c.hidden % 8 == 0;
}

// Word buffers of the persistent step, in floats' worth of words.
size_t persistent_land(const gh_model* m) {
    const gh_config& c = m->cfg;
    const int SL = c.head_dim < 64 ? c.head_dim : 64;
    size_t f = (size_t)std::max(c.hidden, c.n_heads * c.head_dim);
    f = std::max(f, (size_t)(m->q_rows_pad + 2 * m->kv_rows_pad));
    f = std::max(f, (size_t)ATTN_MAX_NC * (2 + SL));
    f = std::max(f, (size_t)m->p_np * 8);
    return (f + 3) & ~(size_t)3;
}

// One decode step as the persistent kernel (one workgroup per CU) + the LM
// head and the finish kernel, into a sink (graph nodes or stream launches).
// The grid is the CU count at one workgroup per CU (the dynamic LDS keeps a
// second one off each CU), so all workgroups are resident; the bounded
// waits turn anything else into GH_ERR_STATE, not a hang.
int enqueue_persistent(gh_model* m, gh_kv* kv, Sink& sink, int pos) {
    const gh_config& c = m->cfg;
    if (!persistent_supported(m)) return set_error(GH_ERR_INVALID, "persistent step: unsupported shape");
    GH_CHECK(persistent_layers(m, kv));
    const int hd = c.head_dim, G = c.n_heads / c.n_kv_heads, H = c.hidden;
    PArgs a{};
    a.layers = (const PLayer*)kv->d_players;
    a.embd = m->embd;
    a.out_norm = m->out_norm;
    a.st = kv->st;
    a.rope_local = kv->rope;
    a.rope_global = kv->rope + (size_t)kv->max_seq * hd;
    a.w_qkv = m->w_qkv;
    a.w_st = m->w_attn;
    a.w_o = m->w_o;
    a.w_a = m->w_a;
    a.w_p = m->w_p;
    a.w_d = m->w_down;
    a.xn_final = m->xn_final;
    a.layer_out = m->layer_out;
    a.L = c.n_layers;
    a.H = H;
    a.nq = c.n_heads;
    a.nkv = c.n_kv_heads;
    a.q_rows_pad = m->q_rows_pad;
    a.kv_rows_pad = m->kv_rows_pad;
    a.n_chunks = c.ffn / 32;
    a.nc = m->attn_nc;
    a.np = m->p_np;
    a.land = (int)persistent_land(m);
    a.eps = c.rms_eps;
    a.escale = sqrtf((float)H);
    a.scale = 1.0f / sqrtf((float)hd);
    a.zc = (c.flags & GH_FLAG_ZERO_CENTERED) ? 1 : 0;
    a.use_qk_norm = (c.flags & GH_FLAG_QK_NORM) ? 1 : 0;
    a.post_attn_norm = (c.flags & GH_FLAG_POST_ATTN_NORM) ? 1 : 0;
    a.post_ffn_norm = (c.flags & GH_FLAG_POST_FFN_NORM) ? 1 : 0;
    a.mode = c.mode;
    a.window = c.sliding_window;
    a.host_tick = &m->p_tick;
    a.set_pos(pos);
    int kbw = kbw_for(FMT_Q4, (m->layers[0].qkv.nblk + 3) / 4);
    if (kbw == 7) kbw = 9;  // the persistent step is built for 1, 2, 3, 4, 6, 9, 10
    void (*fn)(PArgs) = nullptr;
    auto by_kbw = [&](auto hdc, auto gc) {
        constexpr int HD_ = decltype(hdc)::value, G_ = decltype(gc)::value;
        switch (kbw) {
            case 1: fn = k_step_ps<HD_, G_, 1>; break;
            case 2: fn = k_step_ps<HD_, G_, 2>; break;
            case 3: fn = k_step_ps<HD_, G_, 3>; break;
            case 4: fn = k_step_ps<HD_, G_, 4>; break;
            case 6: fn = k_step_ps<HD_, G_, 6>; break;
            case 9: fn = k_step_ps<HD_, G_, 9>; break;
            case 10: fn = k_step_ps<HD_, G_, 10>; break;
            default: break;
        }
    };
    auto pick = [&] {
        fn = nullptr;
        if (hd == 32) by_kbw(std::integral_constant<int, 32>{}, std::integral_constant<int, 4>{});
        else if (G == 4) by_kbw(std::integral_constant<int, 256>{}, std::integral_constant<int, 4>{});
        else by_kbw(std::integral_constant<int, 256>{}, std::integral_constant<int, 2>{});
        return fn != nullptr;
    };
    if (!pick()) return set_error(GH_ERR_INVALID, "persistent step: register batch %d", kbw);
    // dynamic LDS: the matvec slice, x, x1, the landing area, reductions and
    // the chunk rows, then the staged phase D weights where the CU's LDS
    // holds them beside the kernel's static arrays
    const int nbx = std::max(H, c.n_heads * hd) / 32;
    const size_t base = ((mv_lds_floats(FMT_Q4, nbx, 0) + 2 * (size_t)H + a.land + 64 + 128 + 3) & ~(size_t)3) * sizeof(float);
    hipFuncAttributes fa{};
    GH_HIP(hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(fn)));
    int dev_lds = 0;
    GH_HIP(hipDeviceGetAttribute(&dev_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, m->ctx->device));
    const size_t budget = (size_t)dev_lds > fa.sharedSizeBytes ? (size_t)dev_lds - fa.sharedSizeBytes : 0;
    const int nb_gu = m->p_gi[0].nblk, td = m->layers[0].down.tiles;
    const size_t with_down = (size_t)pf_layout(nb_gu, td, true).total * sizeof(float);
    const size_t gu_only = (size_t)pf_layout(nb_gu, td, false).total * sizeof(float);
    a.pf_off = (int)(base / sizeof(float));
    a.pf_gu = base + gu_only <= budget ? 1 : 0;
    a.pf_down = base + with_down <= budget ? 1 : 0;
    // every chunk staged: the register path (the only user of the batch
    // width) never runs, and the narrowest variant has the fewest registers
    if (a.pf_gu && a.n_chunks <= m->p_grid && kbw != 1) {
        kbw = 1;
        if (!pick()) return set_error(GH_ERR_INVALID, "persistent step: register batch %d", kbw);
        hipFuncAttributes f1{};
        GH_HIP(hipFuncGetAttributes(&f1, reinterpret_cast<const void*>(fn)));
        if (f1.sharedSizeBytes != fa.sharedSizeBytes) return set_error(GH_ERR_INVALID, "persistent step: static LDS differs by batch width");
    }
    const size_t need = base + (a.pf_down ? with_down : a.pf_gu ? gu_only : 0);
    const size_t lds = std::max<size_t>(need, 96 << 10);  // one workgroup per CU
    if (lds > budget) return set_error(GH_ERR_INVALID, "persistent step: %zu B of LDS exceed the device's %zu", lds, budget);
    GH_CHECK(sink_launch<0>(sink, "step", 0.0, fn, dim3(m->p_grid), dim3(NT), lds, a));
    return enqueue_head(m, kv, sink, pos);
}

#endif  // GH_IN_TU(2)

// ------------------------------------------------------------------
// the step's matvec phases, one translation unit per prologue family (their
// instances are most of the library's kernels): 5 residual + norm (qkv of
// layers 1.., gate/up), 6 the same from the token embedding (qkv of layer
// 0), 7 the attention merge (o_proj) and GeGLU (down)
// ------------------------------------------------------------------
int launch_resid_mv(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const ResidFields& f,
                    const EpiPartial& epi);
int launch_resid_emb_mv(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const ResidFields& f,
                        const EpiPartial& epi);
int launch_combine_mv(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const ProAttnCombine& pro,
                      const EpiPartial& epi);
int launch_geglu_mv(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const float* part_gu,
                    int Sg, int ld_g, int up_off, int gm, const EpiPartial& epi);

template <bool EMB>
static int launch_resid_t(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const ResidFields& f,
                          const EpiPartial& epi) {
    if ((f.from_embedding != 0) != EMB) return set_error(GH_ERR_INVALID, "residual prologue: embedding flag");
    return with_mg(f.H, [&](auto mg) {
        ProResid<decltype(mg)::value, EMB> pro;
        static_cast<ResidFields&>(pro) = f;
        return launch_mv(k, name, bytes, w, p, pro, epi, 0);
    });
}

#if GH_IN_TU(5)
int launch_resid_mv(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const ResidFields& f,
                    const EpiPartial& epi) {
    return launch_resid_t<false>(k, name, bytes, w, p, f, epi);
}
#endif

#if GH_IN_TU(6)
int launch_resid_emb_mv(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const ResidFields& f,
                        const EpiPartial& epi) {
    return launch_resid_t<true>(k, name, bytes, w, p, f, epi);
}
#endif

#if GH_IN_TU(7)
int launch_combine_mv(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const ProAttnCombine& pro,
                      const EpiPartial& epi) {
    const int per_split = (w.nblk + p.S - 1) / p.S * block_cols(w.fmt);
    return launch_mv<2>(k, name, bytes, w, p, pro, epi, (per_split / pro.HD + 2) * ATTN_MAX_NC);
}

int launch_geglu_mv(Sink& k, const char* name, double bytes, const DMat& w, const Plan& p, const float* part_gu,
                    int Sg, int ld_g, int up_off, int gm, const EpiPartial& epi) {
    // slots = gate/up splits x groups where possible: an absent split's
    // slot still issues its (out-of-range) loads
    if (gm * Sg == 3) return launch_mv(k, name, bytes, w, p, ProGeglu<3>{part_gu, Sg, ld_g, up_off, gm}, epi, 0);
    if (gm * Sg <= 4) return launch_mv(k, name, bytes, w, p, ProGeglu<4>{part_gu, Sg, ld_g, up_off, gm}, epi, 0);
    return launch_mv(k, name, bytes, w, p, ProGeglu<MAXS>{part_gu, Sg, ld_g, up_off, gm}, epi, 0);
}
#endif

// ------------------------------------------------------------------
// the decode step
// ------------------------------------------------------------------
#if GH_IN_TU(1)
int Profiler::kind_of(const char* name) {
    for (size_t i = 0; i < names.size(); ++i)
        if (names[i] == name) return (int)i;
    names.emplace_back(name);
    return (int)names.size() - 1;
}

#endif

namespace {
[[maybe_unused]] double mat_bytes(const DMat& w) {
    const double wb = w.fmt == FMT_Q4 ? (double)w.rows * w.cols / 32.0 * 18.0 : (double)w.rows * w.cols * 4.0;
    return wb + 4.0 * w.cols + 4.0 * w.rows;
}
}  // namespace

// LM head (output.weight, or the tied embedding) on m->xn_final with
// per-workgroup argmax keys and softmax statistics, then the next-token
// selection of position pos.
[[maybe_unused]] static int enqueue_head(gh_model* m, gh_kv* kv, Sink& sink, int pos) {
    const gh_config& c = m->cfg;
    const DMat& W = lm_mat(m);
    {
        ProPlain pro{m->xn_final};
        EpiLogits epi{m->logits, c.vocab, m->lm_cand, kv->st, m->lm_m, m->lm_s};
        GH_CHECK(launch_mv(sink, "lm_head", mat_bytes(W), W, m->plm, pro, epi, 0));
    }
    return sink_launch<1>(sink, "finish", 0.0, k_step_finish<0>, dim3(1), dim3(NT), 0, kv->st, pos,
                          (const unsigned long long*)m->lm_cand, m->plm.row_tiles(W.tiles), (const float*)m->lm_m,
                          (const float*)m->lm_s, 64 * m->plm.rl, (const float*)m->logits, c.vocab,
                          (const int32_t*)kv->d_prompt, kv->d_ids);
}

#if GH_IN_TU(1)
int enqueue_step(gh_model* m, gh_kv* kv, Sink& sink, int pos) {
    const gh_config& c = m->cfg;
    const int H = c.hidden, nkv = c.n_kv_heads, hd = c.head_dim;
    const int G = c.n_heads / nkv;
    const int zc = (c.flags & GH_FLAG_ZERO_CENTERED) ? 1 : 0;
    const float eps = c.rms_eps;
    const size_t kv_layer = (size_t)kv->max_seq * nkv * hd;

    for (int li = 0; li < c.n_layers; ++li) {
        LayerDev& L = m->layers[li];
        const LayerDev* P = li > 0 ? &m->layers[li - 1] : nullptr;
        // A: residual + pre-attention norm + fused QKV matvec
        {
            ResidFields f;
            f.from_embedding = li == 0;
            f.embd = m->embd;
            f.st = kv->st;
            f.escale = sqrtf((float)H);
            f.base = m->x1;
            f.part = m->part_d;
            f.S = m->pe.S;
            f.ld = P ? P->down.tiles * TILE_ROWS : 0;
            f.w_post = P && (c.flags & GH_FLAG_POST_FFN_NORM) ? P->post_ffw : nullptr;
            f.w_norm = L.attn_norm;
            f.eps = eps;
            f.zc = zc;
            f.H = H;
            f.x_out = m->x_res;
            f.layer_out_row = li > 0 ? m->layer_out + (size_t)(li - 1) * H : nullptr;
            EpiPartial epi{m->part_qkv, L.qkv.tiles * TILE_ROWS};
            GH_CHECK(li == 0 ? launch_resid_emb_mv(sink, "qkv", mat_bytes(L.qkv), L.qkv, m->pa, f, epi)
                             : launch_resid_mv(sink, "qkv", mat_bytes(L.qkv), L.qkv, m->pa, f, epi));
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
            const bool global_theta = c.mode == GH_MODE_REF ? true : L.global;
            a.rope = kv->rope + (global_theta ? (size_t)kv->max_seq * hd : 0);
            a.global = L.global;
            a.window = c.sliding_window;
            a.mode = c.mode;
            a.kc = kv->k + li * kv_layer;
            a.vc = kv->v + li * kv_layer;
            a.nkv = nkv;
            a.scale = 1.0f / sqrtf((float)hd);
            a.part = m->attn_part;
            a.nc = m->attn_nc;
            a.xcd = m->attn_xcd;
            a.set_pos(pos);
            GH_CHECK(launch_attn_step(sink, 2.0 * 4.0 * hd * nkv * (a.pe - a.pb), hd, G, a, nkv));
        }
        // C: attention merge + O projection
        {
            ProAttnCombine pro{m->attn_part, pos, m->attn_nc, G, hd, L.global ? 1 : 0, c.sliding_window, c.mode, 0, nkv};
            pro.set_pos(pos);
            EpiPartial epi{m->part_o, L.o.tiles * TILE_ROWS};
            GH_CHECK(launch_combine_mv(sink, "o_proj", mat_bytes(L.o), L.o, m->pc, pro, epi));
        }
        // D: post-attention norm + residual + pre-FFN norm + gate/up matvec
        {
            ResidFields f;
            f.from_embedding = 0;
            f.embd = m->embd;
            f.st = kv->st;
            f.escale = 1.0f;
            f.base = m->x_res;
            f.part = m->part_o;
            f.S = m->pc.S;
            f.ld = L.o.tiles * TILE_ROWS;
            f.w_post = (c.flags & GH_FLAG_POST_ATTN_NORM) ? L.post_attn : nullptr;
            f.w_norm = L.ffn_norm ? L.ffn_norm : L.post_attn;
            f.eps = eps;
            f.zc = zc;
            f.H = H;
            f.x_out = m->x1;
            f.layer_out_row = nullptr;
            EpiPartial epi{m->part_gu, L.gu.tiles * TILE_ROWS};
            GH_CHECK(launch_resid_mv(sink, "gate_up", mat_bytes(L.gu), L.gu, m->pd, f, epi));
        }
        // E: GeGLU + down projection
        {
            const int gm = geglu_groups(L.down, m->pe);
            if (gm > 2 || gm * m->pd.S > MAXS)
                return set_error(GH_ERR_INVALID, "down projection split of %d columns with %d gate/up splits",
                                 (L.down.nblk + m->pe.S - 1) / m->pe.S * block_cols(L.down.fmt), m->pd.S);
            EpiPartial epi{m->part_d, L.down.tiles * TILE_ROWS};
            GH_CHECK(launch_geglu_mv(sink, "down", mat_bytes(L.down), L.down, m->pe, m->part_gu, m->pd.S,
                                     L.gu.tiles * TILE_ROWS, m->f_pad, gm, epi));
        }
    }
    // final residual + norm, once
    {
        const LayerDev& P = m->layers[c.n_layers - 1];
        GH_CHECK(with_mg(H, [&](auto mg) {
            constexpr int MG = decltype(mg)::value;
            ProResid<MG> pro;
            pro.from_embedding = 0;
            pro.embd = m->embd;
            pro.st = kv->st;
            pro.escale = 1.0f;
            pro.base = m->x1;
            pro.part = m->part_d;
            pro.S = m->pe.S;
            pro.ld = P.down.tiles * TILE_ROWS;
            pro.w_post = (c.flags & GH_FLAG_POST_FFN_NORM) ? P.post_ffw : nullptr;
            pro.w_norm = m->out_norm;
            pro.eps = eps;
            pro.zc = zc;
            pro.H = H;
            pro.x_out = nullptr;
            pro.layer_out_row = m->layer_out + (size_t)(c.n_layers - 1) * H;
            const size_t lds = (576 + 2 * (size_t)H) * sizeof(float);
            return sink_launch(sink, "final_norm", 0.0, k_final_norm<MG>, dim3(1), dim3(NT), lds, pro, m->xn_final);
        }));
    }
    return enqueue_head(m, kv, sink, pos);
}
#endif  // GH_IN_TU(1)

#if GH_IN_TU(3)
// ------------------------------------------------------------------
// batched prompt prefill: n prompt tokens in one pass per layer, instead of
// the token-by-token prompt loop of app/Main.hs:426-436.  Per layer:
//   rows   residual update + norm of every token row -> GEMM operand A
//   GEMM   A [n x K] times the Q4_0 (or f32) weight rows on MFMA -> split-K partials
//   qkv    QK-norm + RoPE of each token's q/k, K/V append at its position
//   attn   causal attention of each token over the cache (attn_item, one chunk)
//   a_out  o / l per head -> GEMM operand A
//   geglu  gelu_tanh(g) * u -> GEMM operand A
// The arithmetic per token is the decode step's (TBG:92-461); only the
// matvecs become GEMMs.
// ------------------------------------------------------------------
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// GEMM operand A, [Pp][K] per part.
// With Q4_0 weights (split = 1), each token row t is first scaled by a power
// of two, so that its largest |x| lies in [2^14, 2^15); inv_scale[t] undoes it.
// The row is then stored as two fp16 parts hi + lo.  Per element the error
// |x - (hi + lo) / scale| is at most 2^-23 |x| + 2^-40 max|x|, which is below
// f32 rounding.  (q - 8) * part is exact in the MFMA's f32 products.
// The columns of every 32-column block are permuted to match the weight
// fragments: lane group g of an MFMA holds columns
// {4g, 4g+2, 4g+1, 4g+3, 16+4g, 16+4g+2, 16+4g+1, 16+4g+3}, the low and
// high nibbles of code bytes 4g..4g+3 as q4_f16_pair unpacks them.
// With f32 weights (split = 0): plain f32, unscaled.
struct PfA {
    void* p;
    int Pp, K;
    int split;
    float* inv_scale;  // [Pp] (split only)
    // columns k..k+3 (k a multiple of 4) of token row t, scaled by sc
    __device__ void put4(int t, int k, float4 v, float sc) const {
        if (!split) {
            *(float4*)((float*)p + (size_t)t * K + k) = v;
            return;
        }
        const int kk = k & 31;
        const size_t at = (size_t)t * K + (k & ~31) + (kk < 16 ? 2 * kk : 2 * kk - 28);
        const float x[4] = {v.x * sc, v.z * sc, v.y * sc, v.w * sc};  // stored order 0, 2, 1, 3
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const _Float16 h = (_Float16)x[e];
            hi[e] = __builtin_bit_cast(uint16_t, h);
            lo[e] = __builtin_bit_cast(uint16_t, (_Float16)(x[e] - (float)h));
        }
        uint16_t* base = (uint16_t*)p + at;
        *(uint2*)base = make_uint2(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16));
        *(uint2*)(base + (size_t)Pp * K) = make_uint2(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16));
    }
    // scale of a row whose largest |x| is m; thread 0 records its inverse
    __device__ float row_scale(int t, float m) const {
        if (!split) return 1.0f;
        int ex = 0;
        if (m > 0.0f && m < INFINITY) frexpf(m, &ex);
        ex = min(max(ex, -100), 100);
        if (threadIdx.x == 0) inv_scale[t] = ldexpf(1.0f, ex - 15);
        return ldexpf(1.0f, 15 - ex);
    }
};

__device__ __forceinline__ float amax4(float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); }

// Residual update + norm of token rows t0 + blockIdx.x (ProResid semantics):
//   x = E[token] * sqrt(H)                      (layer 0)
//     or base + postnorm(sum_s part_s)          (TBG:305-343, TBG:413-444)
//   A row = norm(x) with w_norm   (or xn_out = norm(x) for the final norm)
struct PfRows {
    const int32_t* tok;   // layer 0: token ids
    DMat embd;
    float escale;
    const float* base;    // else: residual rows [Pp][H]
    const float* part;    // split-K partials [S][Pp][ld]
    int S, ld, Pp;
    const float* w_post;  // nullable
    const float* w_norm;
    float eps;
    int zc, H;
    float* x_out;         // nullable: new residual rows [Pp][H]
    float* layer_out;     // nullable: receives row t_layer of x
    int t_layer;
    PfA a;
    float* xn_out;        // nullable: plain normed row (final norm of one row)
    int t0;
};

template <int MG>
__global__ __launch_bounds__(NT) void k_pf_rows(PfRows r) {
    __shared__ float slot[12];
    const int t = r.t0 + blockIdx.x, tid = threadIdx.x, NG = r.H >> 2;
    // The row's global loads (split partials, residual, both norm weights)
    // are issued here, before the first use, as straight-line buffer loads
    // (absent splits, groups past H and a null w_post read zeros): one round
    // trip instead of one per reduction.
    const BufView WN(r.w_norm, (size_t)r.H * 4);
    float4 wn[MG];
#pragma unroll
    for (int k = 0; k < MG; ++k) wn[k] = WN.f4(tid + k * NT < NG ? 16u * (uint32_t)(tid + k * NT) : OOB);
    float4 xv[MG];
    if (r.tok) {
        const int tk = min(max(r.tok[t], 0), r.embd.rows - 1);
#pragma unroll
        for (int k = 0; k < MG; ++k) {
            const int g = tid + k * NT;
            xv[k] = f4z();
            if (g < NG) {
                const float4 e = dq_elem4(r.embd, tk, 4 * g);
                xv[k] = make_float4(e.x * r.escale, e.y * r.escale, e.z * r.escale, e.w * r.escale);
            }
        }
    } else {
        const BufView P(r.part + (size_t)t * r.ld, ((size_t)(r.S - 1) * r.Pp * r.ld + r.H) * 4);
        const BufView B(r.base + (size_t)t * r.H, (size_t)r.H * 4);
        const BufView WP(r.w_post, r.w_post ? (size_t)r.H * 4 : 0);
        float4 pv[MG][MAXS], bv[MG], wp[MG];
#pragma unroll
        for (int k = 0; k < MG; ++k) {
            const int g = tid + k * NT;
            const bool ok = g < NG;
#pragma unroll
            for (int s = 0; s < MAXS; ++s)
                pv[k][s] = P.f4(ok && s < r.S ? 4u * (uint32_t)(s * r.Pp * r.ld) + 16u * (uint32_t)g : OOB);
            bv[k] = B.f4(ok ? 16u * (uint32_t)g : OOB);
            wp[k] = WP.f4(ok ? 16u * (uint32_t)g : OOB);
        }
        float4 dv[MG];
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < MG; ++k) {
            dv[k] = pv[k][0];
#pragma unroll
            for (int s = 1; s < MAXS; ++s) dv[k] = dv[k] + pv[k][s];  // absent splits read zeros
            ss += dot4(dv[k], dv[k]);
        }
        float rms = 1.0f;
        if (r.w_post) rms = sqrtf(block_sum(ss, slot) / (float)r.H + r.eps);
#pragma unroll
        for (int k = 0; k < MG; ++k)
            xv[k] = tid + k * NT < NG ? bv[k] + (r.w_post ? norm4(dv[k], rms, wp[k], r.zc) : dv[k]) : f4z();
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < MG; ++k) {
        const int g = tid + k * NT;
        if (g < NG) {
            ss += dot4(xv[k], xv[k]);
            if (r.x_out) ((float4*)(r.x_out + (size_t)t * r.H))[g] = xv[k];
            if (r.layer_out && t == r.t_layer) ((float4*)r.layer_out)[g] = xv[k];
        }
    }
    const float rms = sqrtf(block_sum(ss, slot + 4) / (float)r.H + r.eps);
    float4 y[MG];
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < MG; ++k) {
        const int g = tid + k * NT;
        y[k] = g < NG ? norm4(xv[k], rms, wn[k], r.zc) : f4z();
        mx = fmaxf(mx, amax4(y[k]));
    }
    if (r.xn_out) {
#pragma unroll
        for (int k = 0; k < MG; ++k) {
            const int g = tid + k * NT;
            if (g < NG) ((float4*)r.xn_out)[g] = y[k];
        }
        return;
    }
    const float sc = r.a.row_scale(t, r.a.split ? block_max(mx, slot + 8) : 0.0f);
#pragma unroll
    for (int k = 0; k < MG; ++k) {
        const int g = tid + k * NT;
        if (g < NG) r.a.put4(t, 4 * g, y[k], sc);
    }
}

// GEMM of the prefill: out[s][t][row] = sum over split s's column blocks of
// A[t][k] * W[row][k].
struct PfGemm {
    PfA a;
    DMat w;
    int kb_per;  // column blocks per split
    float* out;  // [S][Pp][ldo]
    int ldo;
    int X, Y, S;  // row groups, 64-token tiles, splits (the grid is 1-D, see pf_tile)
};

// XCD-aware workgroup order of the 1-D prefill GEMM grid.  Workgroups go to
// the 8 XCDs round-robin (XCD = id % 8), each XCD with its own L2.  Key =
// (row group x, split z) names the weight slice a workgroup reads; key k
// runs on XCD k % 8, and its Y token tiles run back to back there, so the
// slice is fetched from HBM once.  With 8 splits, split z lives on XCD z
// only, so its column slice of A is fetched by one L2 as well.  Ids past
// the last key return (fewer than 8 Y of them).
struct PfTile {
    int x, y, z;
};
__device__ __forceinline__ bool pf_tile(const PfGemm& g, PfTile& t) {
    const int b = blockIdx.x, xcd = b & 7, j = b >> 3;
    t.y = j % g.Y;
    const int key = (j / g.Y) * 8 + xcd;
    if (key >= g.X * g.S) return false;
    t.x = key / g.S;
    t.z = key % g.S;
    return true;
}
inline int pf_grid(int X, int Y, int S) { return (X * S + 7) / 8 * 8 * Y; }

// (q - 8) as fp16 for the two nibbles of w at bits [s, s+4) and [s+16, s+20):
// 1024 + q is 0x6400 | q in fp16, and 1024 + q - 1032 is exact.
__device__ __forceinline__ uint32_t q4_f16_pair(uint32_t w, int s) {
    const uint32_t v = ((w >> s) & 0x000F000Fu) | 0x64006400u;
    const f16x2_t h = __builtin_bit_cast(f16x2_t, v) - f16x2_t{(_Float16)1032.0f, (_Float16)1032.0f};
    return __builtin_bit_cast(uint32_t, h);
}

// The 8 fp16 weights of code dword w (bytes 4g..4g+3 of a row's block), in
// the order of the A column permutation.
__device__ __forceinline__ uint4 q4_f16_frag(uint32_t w) {
    return make_uint4(q4_f16_pair(w, 0), q4_f16_pair(w, 8), q4_f16_pair(w, 4), q4_f16_pair(w, 12));
}

constexpr int PF_DEPTH = 4;  // column blocks in flight per workgroup

// LDS slot of B-operand lane s (0..63) of a fragment: s ^ 4 * (s / 16).  The
// 16 lanes of a write phase (4 rows x the 4 k-groups of one code dword's
// row) and of a read phase (16 lanes of one k-group) then fall on 16
// different 16-byte bank groups (without it, a row's four k-groups sit
// 256 bytes apart: the same banks).
__device__ __forceinline__ int pf_swz(int s) { return s ^ ((s >> 4) << 2); }

// Q4_0 weights on v_mfma_f32_16x16x32_f16.  Workgroup = 64 token rows x
// 16*NS weight rows (NS = 8: one 128-row tile, NS = 4: half a tile) x one
// split; wave w owns token rows 16w..16w+15 and all NS row subtiles.
// Per 32-column block (one MFMA K step):
//   1. the workgroup unpacks the block's codes of its rows once into LDS as
//      fp16 fragments, and its scales as f32;
//   2. each wave runs 2 MFMAs (hi, lo parts of A) per row subtile into a
//      fresh accumulator, then adds d * that to the running sum.
// Codes, scales and A fragments are loaded PF_DEPTH blocks ahead.  The LDS
// fragments are double-buffered, with one barrier per block.
template <int NS>
__global__ __launch_bounds__(NT) void k_pf_gemm_q4(PfGemm g) {
    constexpr int R = 16 * NS;       // weight rows per workgroup
    constexpr int NI = R * 4 / NT;   // code dwords per thread per block
    static_assert(NI >= 1 && NI * NT == R * 4, "NS must be 4 or 8");
    __shared__ __align__(16) uint4 bs[2][NS][64];
    __shared__ float ss[2][R];
    PfTile pt;
    if (!pf_tile(g, pt)) return;  // uniform per workgroup
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = pt.x / (8 / NS), r0 = (pt.x % (8 / NS)) * R;
    const int t0 = pt.y * 64 + 16 * wave;
    const int kb0 = pt.z * g.kb_per, nk = min(g.w.nblk, kb0 + g.kb_per) - kb0;
    const int K = g.a.K;
    const size_t pstride = (size_t)g.a.Pp * K;
    const uint16_t* abase = (const uint16_t*)g.a.p + (size_t)(t0 + (lane & 15)) * K + 8 * (lane >> 4);
    const uint32_t* codes = (const uint32_t*)g.w.codes + ((size_t)tile * g.w.nblk + kb0) * TILE_ROWS * 4 + r0 * 4;
    const uint16_t* scales = g.w.scales + ((size_t)tile * g.w.nblk + kb0) * TILE_ROWS + r0;
    // code dword item = tid + NT*q of the block's R x 4 -> (row = item >> 2,
    // g = item & 3) -> LDS fragment (subtile row >> 4, lane (row & 15) + 16 g)
    uint4* frag[NI];
#pragma unroll
    for (int q = 0; q < NI; ++q) {
        const int item = tid + NT * q, row = item >> 2;
        frag[q] = &bs[0][row >> 4][pf_swz((row & 15) + 16 * (item & 3))];
    }
    uint32_t rb[PF_DEPTH][NI];
    uint16_t rs[PF_DEPTH];
    uint4 ra0[PF_DEPTH], ra1[PF_DEPTH];
    // Block i's loads into ring slot j.  Every call issues the same loads
    // (indices clamped into range, no branches), so the wait counts stay
    // static and the PF_DEPTH blocks in flight are not drained early.
    auto load = [&](int j, int i) {
        const int ic = min(i, nk - 1);
        const uint32_t* cb = codes + (size_t)ic * TILE_ROWS * 4;
#pragma unroll
        for (int q = 0; q < NI; ++q) rb[j][q] = cb[tid + NT * q];
        rs[j] = scales[(size_t)ic * TILE_ROWS + min(tid, R - 1)];
        const uint16_t* ap = abase + (size_t)(kb0 + ic) * 32;
        ra0[j] = *(const uint4*)ap;
        ra1[j] = *(const uint4*)(ap + pstride);
    };
    f32x4_t acc[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) acc[n] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < PF_DEPTH; ++j) load(j, j);
    for (int base = 0; base < nk; base += PF_DEPTH) {
#pragma unroll
        for (int j = 0; j < PF_DEPTH; ++j) {
            const int i = base + j;
            if (i >= nk) break;
            const int buf = j & 1;  // == i & 1: PF_DEPTH is even
#pragma unroll
            for (int q = 0; q < NI; ++q) frag[q][buf * NS * 64] = q4_f16_frag(rb[j][q]);
            if (tid < R) ss[buf][tid] = h2f(rs[j]);
            const f16x8_t a0 = __builtin_bit_cast(f16x8_t, ra0[j]);
            const f16x8_t a1 = __builtin_bit_cast(f16x8_t, ra1[j]);
            __syncthreads();
            load(j, i + PF_DEPTH);
#pragma unroll
            for (int n = 0; n < NS; ++n) {
                const f16x8_t b = __builtin_bit_cast(f16x8_t, bs[buf][n][pf_swz(lane)]);
                const float d = ss[buf][16 * n + (lane & 15)];
                f32x4_t c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b, c, 0, 0, 0);
                acc[n] += d * c;
            }
        }
    }
    // lane holds token rows 4*(lane>>4) .. +3 of the wave's 16, weight row
    // r0 + 16 n + (lane & 15) of the tile
    const int tr = t0 + 4 * (lane >> 4);
    float inv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) inv[r] = g.a.inv_scale[tr + r];
    float* o = g.out + ((size_t)pt.z * g.a.Pp + tr) * g.ldo + (size_t)tile * TILE_ROWS + r0 + (lane & 15);
#pragma unroll
    for (int n = 0; n < NS; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[(size_t)r * g.ldo + 16 * n] = acc[n][r] * inv[r];
}

// Row-subtiles per workgroup of a Q4_0 prefill GEMM: whole tiles, unless
// even 8 splits leave fewer than 512 workgroups; then half tiles.
static int pf_ns(const DMat& w, int Pp) { return w.tiles * (Pp / 64) * 8 >= 512 ? 8 : 4; }

// f32 weights on v_mfma_f32_16x16x4_f32: one 4-column block per MFMA.
__global__ __launch_bounds__(NT) void k_pf_gemm_f32(PfGemm g) {
    PfTile pt;
    if (!pf_tile(g, pt)) return;  // uniform per workgroup
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tile = pt.x >> 1;
    const int lr = (pt.x & 1) * 64 + wave * 16 + (lane & 15);
    const int t0 = pt.y * 64;
    const int kb0 = pt.z * g.kb_per, kb1 = min(g.w.nblk, kb0 + g.kb_per);
    const int kq = lane >> 4;
    const int K = g.a.K;
    const float* ab = (const float*)g.a.p + (size_t)(t0 + (lane & 15)) * K + kq;
    const float* wc = (const float*)g.w.codes;
    f32x4_t acc[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int kb = kb0; kb < kb1; ++kb) {
        const float bw = wc[(((size_t)tile * g.w.nblk + kb) * TILE_ROWS + lr) * 4 + kq];
#pragma unroll
        for (int m = 0; m < 4; ++m)
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(ab[(size_t)(16 * m) * K + 4 * kb], bw, acc[m], 0, 0, 0);
    }
    float* o = g.out + ((size_t)pt.z * g.a.Pp + t0 + 4 * kq) * g.ldo + (size_t)tile * TILE_ROWS + lr;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[(size_t)(16 * m + r) * g.ldo] = acc[m][r];
}

// q/k/v of token t, kv head g: sum of the QKV split partials, QK-norm
// (TBG:171-179), RoPE at the token's position, K/V append
// (appendKVCacheShader, AttentionGPU.hs:502-534); q goes to the query rows.
struct PfQkv {
    const float* part;
    int S, ld, Pp;
    int q_off, k_off, v_off;
    const float* q_norm;
    const float* k_norm;
    int use_qk_norm, zc;
    float eps;
    const float* rope;  // [max_seq][HD/2] (cos, sin) of this layer type
    int pos0, nkv;
    float* q;           // [Pp][nq * HD]
    float* kc;
    float* vc;
};

// One wave per (token, kv head, vector): the G q heads, k and v are
// independent until attention, so each vector's split sum, QK-norm and RoPE
// run on a workgroup of their own (6x the workgroups of one per (token, kv
// head) for G = 4: the per-token chains spread over the chip).
template <int HD, int G>
__global__ __launch_bounds__(64) void k_pf_qkv(PfQkv p) {
    __shared__ __align__(16) float buf[HD];
    const int vec = blockIdx.x % (G + 2), tg = blockIdx.x / (G + 2);
    const int t = tg / p.nkv, g = tg % p.nkv, lane = threadIdx.x;
    const int pos = p.pos0 + t;
    const int row0 = vec < G ? p.q_off + (g * G + vec) * HD : vec == G ? p.k_off + g * HD : p.v_off + g * HD;
    for (int i = 4 * lane; i < HD; i += 4 * 64)
        *(float4*)&buf[i] = sum_splits4(p.part + (size_t)t * p.ld, p.S, p.Pp * p.ld, (row0 + i) >> 2);
    __syncthreads();
    if (vec <= G) {
        if (p.use_qk_norm) wave_head_norm<HD>(buf, vec < G ? p.q_norm : p.k_norm, p.eps, p.zc);
        wave_head_rope<HD>(buf, (const float2*)p.rope + (size_t)pos * (HD / 2));
    }
    __syncthreads();
    float* dst = vec < G ? p.q + (size_t)t * p.nkv * G * HD + ((size_t)g * G + vec) * HD
               : (vec == G ? p.kc : p.vc) + ((size_t)pos * p.nkv + g) * HD;
    for (int i = lane; i < HD; i += 64) dst[i] = buf[i];
}

// Attention of token t (kv head g) over its window of the cache: the
// window is split into up to a.nc (<= PF_ATTN_NC, from the host: one per 128
// positions of the longest window) chunks of ATTN_SUB-multiple length, each
// a workgroup running the decode kernel's flash-decoding item; the chunk
// states {m, l, o} go to the token's slot of `state`.
template <int HD, int G>
__global__ __launch_bounds__(NT) void k_pf_attn(AttnArgs a, const float* q, int pos0, float* state) {
    const int j = blockIdx.x % a.nc, tg = blockIdx.x / a.nc;
    const int t = tg / a.nkv, g = tg % a.nkv;
    AttnArgs b = a;
    b.q = q + (size_t)t * a.nkv * G * HD;
    b.set_pos(pos0 + t);
    if (j >= b.n_used) return;  // uniform per workgroup
    attn_item<HD, G, false>(b, g, j, QkvPartials{nullptr, 0, 0},
                            AttnOutPlain{state + (size_t)t * a.nkv * PF_ATTN_NC * G * (HD + 2)});
}

// Causal attention of the prompt on the f32 matrix cores (head_dim 256,
// v_mfma_f32_16x16x4f32): workgroup (query tile, kv head g, key chunk j).
// A wave owns 16 query rows, (token, q head) pairs of 16 / G tokens, and the
// workgroup's 4 waves share every staged 16-key block of K and V in LDS
// (double-buffered, one barrier per block).  Per block and wave:
//   S^T = K Q^T: 64 MFMAs; lane i supplies K[key i%16][d] and
//     Q[row i%16][d] over the dims d = 16u + 4(i/16) + e (the sum runs over
//     every dim once, in this order), and holds S^T[key 4(i/16)+r][row i%16];
//   online softmax per row (its 4 lane copies reduced by xor 16, 32);
//   O^T += V^T P^T: 64 MFMAs; the K dimension of MFMA j is key 4(i/16) + j,
//     so lane i's own probabilities are its B operand, and output block
//     (gamma, b') holds the dims 64 gamma + 4m + b' of row i%16.
// Keys outside a row's window or past the chunk are masked.  The chunk's
// state {m, l, o} goes to slot j of the token's states, in the layout the
// merge (k_pf_attn_out) reads, for the rows whose window meets the chunk.
constexpr int FA_KB = 16;       // keys per staged block
constexpr int FA_LD = 256 + 4;  // LDS row stride (floats) of a staged K or V row
inline size_t pf_fa_lds_bytes() { return sizeof(float) * 2 * 2 * FA_KB * FA_LD; }
template <int G>
__global__ __launch_bounds__(NT) void k_pf_fa(AttnArgs a, const float* q, int pos0, int n, int nch, int ch,
                                              float* state) {
    constexpr int HD = 256, TPW = 16 / G, TPB = 4 * TPW;
    static_assert(G >= 1 && G <= 16 && 16 % G == 0, "16 query rows per wave");
    extern __shared__ __align__(16) float fa_lds[];
    const int j = blockIdx.x % nch, tg = blockIdx.x / nch, g = tg % a.nkv, tile = tg / a.nkv;
    const int wave = wave_id(), lane = threadIdx.x & 63, qr = lane & 15, kq = lane >> 4;
    const int t0 = tile * TPB, tl = min(t0 + TPB, n) - 1;  // the workgroup's tokens
    const int tw0 = t0 + wave * TPW, twl = min(tw0 + TPW, n) - 1;  // the wave's (tw0 > twl: none)
    const int t = tw0 + qr / G, hl = qr % G;  // this lane's query row
    const bool tok_ok = t < n;
    int pb = 0, pe = 0, wpb = 0, wpe = 0, dump = 0, vpb = 0, vpe = 0;
    if (tok_ok) attn_window(pos0 + t, a.global, a.window, a.mode, pb, pe);
    // windows are monotone in the position: the workgroup's union is
    // [pb(t0), pe(tl)), cut to chunk j
    attn_window(pos0 + t0, a.global, a.window, a.mode, wpb, dump);
    attn_window(pos0 + tl, a.global, a.window, a.mode, dump, wpe);
    const int k_lo = max(wpb, j * ch), k_hi = min(wpe, (j + 1) * ch);
    if (tw0 <= twl) {
        attn_window(pos0 + tw0, a.global, a.window, a.mode, vpb, dump);
        attn_window(pos0 + twl, a.global, a.window, a.mode, dump, vpe);
    }
    const size_t rs = (size_t)a.nkv * HD;  // cache row stride (floats)
    // this lane's q row, dims 16u + 4 kq .. + 3
    float4 qv[16];
    const float* qrow = q + (size_t)(tok_ok ? t : 0) * a.nkv * G * HD + (size_t)(g * G + hl) * HD;
#pragma unroll
    for (int u = 0; u < 16; ++u) qv[u] = tok_ok ? *(const float4*)(qrow + 16 * u + 4 * kq) : f4z();
    f32x4 acc[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[c][b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    // staging: thread -> key tid / 16, dims 16 (tid % 16) .. + 15; rows at or
    // past wpe read zeros (the views end there) and are masked
    const BufView KC(a.kc, (size_t)wpe * rs * 4), VC(a.vc, (size_t)wpe * rs * 4);
    float4 sk[4], sv[4];
    const int skey = threadIdx.x >> 4, sdim = 16 * (threadIdx.x & 15);
    auto stage_load = [&](int k0) {
        const uint32_t off = 4u * ((uint32_t)(k0 + skey) * (uint32_t)rs + (uint32_t)(g * HD + sdim));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sk[e] = KC.f4(off + 16u * e);
            sv[e] = VC.f4(off + 16u * e);
        }
    };
    auto slab = [&](int buf, int which) { return fa_lds + (size_t)((buf * 2 + which) * FA_KB) * FA_LD; };
    const int kb_lo = k_lo / FA_KB * FA_KB;
    if (k_lo < k_hi) stage_load(kb_lo);
    int buf = 0;
    for (int k0 = kb_lo; k0 < k_hi; k0 += FA_KB, buf ^= 1) {
        float* Ks = slab(buf, 0);
        float* Vs = slab(buf, 1);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            *(float4*)(Ks + skey * FA_LD + sdim + 4 * e) = sk[e];
            *(float4*)(Vs + skey * FA_LD + sdim + 4 * e) = sv[e];
        }
        __syncthreads();  // this block staged; the block two back no longer read
        if (k0 + FA_KB < k_hi) stage_load(k0 + FA_KB);
        if (tw0 > twl || k0 >= vpe || k0 + FA_KB <= vpb) continue;  // no row of this wave sees the block
        f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const float4 kv = *(const float4*)(Ks + qr * FA_LD + 16 * u + 4 * kq);
            sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qv[u].x, sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qv[u].y, sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qv[u].z, sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qv[u].w, sc, 0, 0, 0);
        }
        // row qr, keys k0 + 4 kq + r
        float p[4], bm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = k0 + 4 * kq + r;
            const bool ok = tok_ok && key >= pb && key < pe && key >= k_lo && key < k_hi;
            p[r] = ok ? sc[r] * a.scale : -INFINITY;
            bm = fmaxf(bm, p[r]);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        const float mn = fmaxf(m, bm);
        float corr = 1.0f;
        if (mn == -INFINITY) {
#pragma unroll
            for (int r = 0; r < 4; ++r) p[r] = 0.0f;
        } else {
            corr = m == -INFINITY ? 0.0f : __expf(m - mn);
#pragma unroll
            for (int r = 0; r < 4; ++r) p[r] = p[r] == -INFINITY ? 0.0f : __expf(p[r] - mn);
        }
        float ps = (p[0] + p[1]) + (p[2] + p[3]);
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        l = l * corr + ps;
        m = mn;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int b = 0; b < 4; ++b) acc[c][b] *= corr;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float4 vv = *(const float4*)(Vs + (4 * kq + jj) * FA_LD + 64 * c + 4 * qr);
                acc[c][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, p[jj], acc[c][0], 0, 0, 0);
                acc[c][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, p[jj], acc[c][1], 0, 0, 0);
                acc[c][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, p[jj], acc[c][2], 0, 0, 0);
                acc[c][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, p[jj], acc[c][3], 0, 0, 0);
            }
        }
    }
    // The state of a row whose window meets the chunk (the merge reads
    // exactly those): m and l from the row's first lane copy; o through LDS
    // (the K/V buffers, free once every wave is past the loop), so that each
    // row leaves as one contiguous 1 KB store of the wave.
    const size_t cs = (size_t)G * (HD + 2);
    const bool keep = tok_ok && max(pb, j * ch) < min(pe, (j + 1) * ch);
    if (keep && kq == 0) {
        float* st = state + (size_t)t * a.nkv * PF_ATTN_NC * cs + ((size_t)g * nch + j) * cs;
        st[hl] = m;
        st[G + hl] = l;
    }
    __syncthreads();
    float* ob = fa_lds + (size_t)wave * 16 * HD;  // this wave's 16 rows (64 KB for 4 waves)
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r)  // lane holds dims 64 c + 16 kq + 4 r + b of its row
            *(float4*)(ob + qr * HD + 64 * c + 16 * kq + 4 * r) =
                make_float4(acc[c][0][r], acc[c][1][r], acc[c][2][r], acc[c][3][r]);
    const unsigned long long kept = __ballot(keep);  // bit qr (lanes 0..15) = row qr kept
    for (int row = 0; row < 16; ++row) {
        if (!(kept >> row & 1ull)) continue;  // wave-uniform
        const int tr = tw0 + row / G, hr = row % G;
        float* st = state + (size_t)tr * a.nkv * PF_ATTN_NC * cs + ((size_t)g * nch + j) * cs;
        *(float4*)(st + 2 * G + hr * HD + 4 * lane) = *(const float4*)(ob + row * HD + 4 * lane);
    }
}

// Merge of token t's chunk states per head, o = sum_j w_j o_j / sum_j w_j l_j
// (fa_ch > 0: the prompt-wide k_pf_fa chunks of fa_ch positions that meet
// the token's window; else the token's own n_used chunks)
// with w_j = exp(m_j - max_j m_j), into GEMM operand A.  The row (all heads)
// is staged in dynamic LDS for its scale.
template <int HD, int G>
__global__ __launch_bounds__(NT) void k_pf_attn_out(AttnArgs a, int pos0, const float* state, PfA out,
                                                    int fa_ch) {
    extern __shared__ __align__(16) float rowbuf[];
    __shared__ float wj[8 * G][PF_ATTN_NC];
    __shared__ float den[8 * G];
    __shared__ float slot[4];
    const int t = blockIdx.x, nq = a.nkv * G, n = nq * HD, tid = threadIdx.x;
    AttnArgs b = a;
    b.set_pos(pos0 + t);
    // the token's chunks: its own n_used, or (fa_ch > 0) the k_pf_fa chunks of
    // fa_ch positions that meet its window
    int c_lo = 0, c_hi = b.n_used;
    if (fa_ch > 0) {
        int pb, pe;
        attn_window(pos0 + t, a.global, a.window, a.mode, pb, pe);
        c_lo = pb / fa_ch;
        c_hi = (pe - 1) / fa_ch + 1;
    }
    const size_t cstride = (size_t)G * (HD + 2);  // one chunk state
    const float* st = state + (size_t)t * a.nkv * PF_ATTN_NC * cstride;
    // chunk weights per head (nq <= 8 G heads, one thread per head)
    if (tid < nq) {
        const int g = tid / G, hl = tid % G;
        const float* sg = st + (size_t)g * a.nc * cstride;  // attn_item's layout: (g * nc + chunk)
        float M = -INFINITY;
        for (int c = c_lo; c < c_hi; ++c) M = fmaxf(M, sg[c * cstride + hl]);
        float dsum = 0.0f;
        for (int c = c_lo; c < c_hi; ++c) {
            const float w = expf(sg[c * cstride + hl] - M);
            wj[tid][c] = w;
            dsum += w * sg[c * cstride + G + hl];
        }
        den[tid] = dsum;
    }
    __syncthreads();
    float mx = 0.0f;
    for (int i = 4 * tid; i < n; i += 4 * NT) {
        const int h = i / HD, d = i % HD, g = h / G, hl = h % G;
        const float* o = st + (size_t)g * a.nc * cstride + 2 * G + hl * HD + d;
        float4 v = f4z();
        for (int c = c_lo; c < c_hi; ++c) {
            const float w = wj[h][c];
            const float* oc = o + c * cstride;
            v = make_float4(v.x + w * oc[0], v.y + w * oc[1], v.z + w * oc[2], v.w + w * oc[3]);
        }
        const float l = den[h];
        v = make_float4(v.x / l, v.y / l, v.z / l, v.w / l);
        *(float4*)&rowbuf[i] = v;
        mx = fmaxf(mx, amax4(v));
    }
    const float sc = out.row_scale(t, block_max(mx, slot));  // barrier: rowbuf complete
    for (int i = 4 * tid; i < n; i += 4 * NT) out.put4(t, i, *(const float4*)&rowbuf[i], sc);
}

// h = gelu_tanh(sum_s g_s) * sum_s u_s (MLP.hs:384-447) -> GEMM operand A.
// The row is staged in dynamic LDS (F floats) for its scale.
template <int S>
__global__ __launch_bounds__(NT) void k_pf_geglu(const float* part, int ld, int Pp, int F, int up_off, PfA a) {
    extern __shared__ __align__(16) float rowbuf[];
    __shared__ float slot[4];
    const int t = blockIdx.x;
    // the S split partials of gate and up for elements i..i+3, as
    // straight-line buffer loads (past F: zeros); the next group's loads go
    // out before this group's GELU, so a row costs one round trip, not one
    // per group
    const BufView P(part + (size_t)t * ld, ((size_t)(S - 1) * Pp * ld + up_off + F) * 4);
    const uint32_t ss = 4u * (uint32_t)(Pp * ld);
    float4 g[2][S], u[2][S];
    auto load = [&](int b, int i) {
        const bool ok = i < F;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            g[b][s] = P.f4(ok ? s * ss + 4u * (uint32_t)i : OOB);
            u[b][s] = P.f4(ok ? s * ss + 4u * (uint32_t)(up_off + i) : OOB);
        }
    };
    float mx = 0.0f;
    auto compute = [&](int b, int i) {
        float4 gs = g[b][0], us = u[b][0];
#pragma unroll
        for (int s = 1; s < S; ++s) {
            gs = gs + g[b][s];
            us = us + u[b][s];
        }
        const float4 h = make_float4(gelu_tanh(gs.x) * us.x, gelu_tanh(gs.y) * us.y, gelu_tanh(gs.z) * us.z,
                                     gelu_tanh(gs.w) * us.w);
        *(float4*)&rowbuf[i] = h;
        mx = fmaxf(mx, amax4(h));
    };
    int i = 4 * threadIdx.x;
    load(0, i);
    for (; i < F; i += 8 * NT) {
        load(1, i + 4 * NT);
        compute(0, i);
        if (i + 4 * NT >= F) break;
        load(0, i + 8 * NT);
        compute(1, i + 4 * NT);
    }
    const float sc = a.row_scale(t, block_max(mx, slot));  // barrier: rowbuf complete
    for (int k = 4 * threadIdx.x; k < F; k += 4 * NT) a.put4(t, k, *(const float4*)&rowbuf[k], sc);
}

// Split count of a prefill GEMM over Pp token rows, at most 8: enough for
// two workgroups per CU where the columns are many (K >= 4096: the FFN's
// down projection, whose workgroups' latency chain bounds it), one per CU
// otherwise (QKV, O: there the next kernel's reads of the partials cost
// more than the extra workgroups save).  Measured on MI355X, 512-token
// prefill: QKV 426 -> 355 us and O 302 -> 267 us at one workgroup per CU;
// down 831 -> 1048 us, so it keeps two.
int pf_splits(const DMat& w, int Pp, int* kb_per) {
    const int wgs = (w.fmt == FMT_Q4 ? w.tiles * (8 / pf_ns(w, Pp)) : 2 * w.tiles) * (Pp / 64);
    const int target = w.cols >= 4096 ? 512 : 256;
    int S = std::max(1, std::min(8, (target + wgs - 1) / wgs));
    S = std::min(S, w.nblk);
    const int per = (w.nblk + S - 1) / S;
    if (kb_per) *kb_per = per;
    return (w.nblk + per - 1) / per;
}

static double pf_gemm_bytes(const DMat& w, int n) {
    return mat_bytes(w) + 4.0 * (double)n * (w.cols + w.rows) - 4.0 * (w.cols + w.rows);
}

int enqueue_prefill(gh_model* m, gh_kv* kv, Sink& sink, int n, int pos0, bool head) {
    const gh_config& c = m->cfg;
    const PfBufs& B = m->pf;
    const int H = c.hidden, hd = c.head_dim, nkv = c.n_kv_heads, G = c.n_heads / nkv, F = c.ffn;
    const int Pp = (n + 63) / 64 * 64;
    if (n <= 0 || Pp > B.cap) return set_error(GH_ERR_INVALID, "internal: prefill of %d rows, buffers hold %d", n, B.cap);
    const int zc = (c.flags & GH_FLAG_ZERO_CENTERED) ? 1 : 0;
    const float eps = c.rms_eps;
    const size_t kv_layer = (size_t)kv->max_seq * nkv * hd;
    const int split = m->fmt == FMT_Q4 ? 1 : 0;
    auto A = [&](int K) { return PfA{B.a, Pp, K, split, B.ascale}; };
    if ((size_t)F * sizeof(float) > 65536 || (size_t)c.n_heads * hd * sizeof(float) > 65536 || nkv > 8)
        return set_error(GH_ERR_INVALID, "prefill: ffn %d / heads x head_dim %d above 16384 or %d kv heads above 8", F,
                         c.n_heads * hd, nkv);
    // GEMM of operand A (K columns) with w into the partials; returns S
    auto gemm = [&](const char* name, const DMat& w, int* S_out) -> int {
        int per = 0;
        const int S = pf_splits(w, Pp, &per);
        if ((size_t)S * Pp * w.tiles * TILE_ROWS > B.part_floats)
            return set_error(GH_ERR_INVALID, "internal: prefill partials too small");
        *S_out = S;
        const int ns = w.fmt == FMT_Q4 ? pf_ns(w, Pp) : 4;  // f32: 64-row groups
        PfGemm g{A(w.cols), w, per, B.part, w.tiles * TILE_ROWS, w.tiles * (8 / ns), Pp / 64, S};
        const dim3 grid(pf_grid(g.X, g.Y, g.S));
        if (w.fmt == FMT_Q4)
            return ns == 8 ? sink_launch(sink, name, pf_gemm_bytes(w, n), k_pf_gemm_q4<8>, grid, dim3(NT), 0, g)
                           : sink_launch(sink, name, pf_gemm_bytes(w, n), k_pf_gemm_q4<4>, grid, dim3(NT), 0, g);
        return sink_launch(sink, name, pf_gemm_bytes(w, n), k_pf_gemm_f32, grid, dim3(NT), 0, g);
    };
    auto rows = [&](const char* name, PfRows r, int n_rows) {
        return with_mg(H, [&](auto mg) {
            return sink_launch(sink, name, 0.0, k_pf_rows<decltype(mg)::value>, dim3(n_rows), dim3(NT), 0, r);
        });
    };
    int S = 0;
    for (int li = 0; li < c.n_layers; ++li) {
        const LayerDev& L = m->layers[li];
        const LayerDev* P = li > 0 ? &m->layers[li - 1] : nullptr;
        // residual (embedding at layer 0) + pre-attention norm
        {
            PfRows r{};
            r.tok = li == 0 ? B.tok : nullptr;
            r.embd = m->embd;
            r.escale = sqrtf((float)H);
            r.base = B.x1;
            r.part = B.part;
            r.S = S;
            r.ld = P ? P->down.tiles * TILE_ROWS : 0;
            r.Pp = Pp;
            r.w_post = P && (c.flags & GH_FLAG_POST_FFN_NORM) ? P->post_ffw : nullptr;
            r.w_norm = L.attn_norm;
            r.eps = eps;
            r.zc = zc;
            r.H = H;
            r.x_out = B.x;
            r.layer_out = li > 0 ? m->layer_out + (size_t)(li - 1) * H : nullptr;
            r.t_layer = n - 1;
            r.a = A(H);
            GH_CHECK(rows("pf_rows", r, n));
        }
        GH_CHECK(gemm("pf_qkv", L.qkv, &S));
        // QK-norm, RoPE, K/V append
        {
            PfQkv q{};
            q.part = B.part;
            q.S = S;
            q.ld = L.qkv.tiles * TILE_ROWS;
            q.Pp = Pp;
            q.q_off = 0;
            q.k_off = m->q_rows_pad;
            q.v_off = m->q_rows_pad + m->kv_rows_pad;
            q.q_norm = L.q_norm;
            q.k_norm = L.k_norm;
            q.use_qk_norm = (c.flags & GH_FLAG_QK_NORM) && L.q_norm && L.k_norm;
            q.zc = zc;
            q.eps = eps;
            const bool global_theta = c.mode == GH_MODE_REF ? true : L.global;
            q.rope = kv->rope + (global_theta ? (size_t)kv->max_seq * hd : 0);
            q.pos0 = pos0;
            q.nkv = nkv;
            q.q = B.q;
            q.kc = kv->k + li * kv_layer;
            q.vc = kv->v + li * kv_layer;
#define GH_PF_QKV(HD_, G_) \
    if (hd == HD_ && G == G_) GH_CHECK(sink_launch(sink, "pf_qkv_post", 0.0, k_pf_qkv<HD_, G_>, dim3(n * nkv * (G_ + 2)), dim3(64), 0, q)); else
            GH_PF_QKV(256, 1) GH_PF_QKV(256, 2) GH_PF_QKV(256, 4) GH_PF_QKV(256, 8)
            GH_PF_QKV(128, 1) GH_PF_QKV(128, 2) GH_PF_QKV(128, 4) GH_PF_QKV(128, 8)
            GH_PF_QKV(32, 1) GH_PF_QKV(32, 2) GH_PF_QKV(32, 4) GH_PF_QKV(32, 8)
            return set_error(GH_ERR_INVALID, "prefill: unsupported head_dim %d / group %d", hd, G);
#undef GH_PF_QKV
        }
        // causal attention per token, then o / l into operand A
        {
            AttnArgs a{};
            a.global = L.global;
            a.window = c.sliding_window;
            a.mode = c.mode;
            a.kc = kv->k + li * kv_layer;
            a.vc = kv->v + li * kv_layer;
            a.nkv = nkv;
            a.scale = 1.0f / sqrtf((float)hd);
            // chunks per token: one per 128 positions of the longest window
            a.nc = std::max(1, std::min(PF_ATTN_NC, (pos0 + n + 127) / 128));

            const PfA ao = A(c.n_heads * hd);
            // head_dim 256: the matrix-core kernel over prompt-wide key chunks
            // (multiples of 16 positions, at most PF_ATTN_NC of them), merged by
            // k_pf_attn_out: ~64 positions per chunk, shorter until the grid has
            // about 256 workgroups
            AttnArgs af = a;
            const int ptot = pos0 + n, fa_tiles = (n + 64 / G - 1) / (64 / G) * nkv;
            const int want = std::max((ptot + 63) / 64, (256 + fa_tiles - 1) / fa_tiles);
            int fa_ch = std::max(1, std::min(PF_ATTN_NC, want));
            fa_ch = ((ptot + fa_ch - 1) / fa_ch + FA_KB - 1) / FA_KB * FA_KB;
            af.nc = (ptot + fa_ch - 1) / fa_ch;  // <= PF_ATTN_NC
#define GH_PF_ATTN(HD_, G_)                                                                                      \
    if (hd == HD_ && G == G_) {                                                                                  \
        if constexpr (HD_ == 256) {                                                                              \
            GH_CHECK(sink_launch(sink, "pf_attn", 0.0, k_pf_fa<G_>,                                             \
                                 dim3((n + 64 / G_ - 1) / (64 / G_) * nkv * af.nc), dim3(NT), pf_fa_lds_bytes(), \
                                 af, (const float*)B.q, pos0, n, af.nc, fa_ch, B.st));                          \
            GH_CHECK(sink_launch(sink, "pf_attn_out", 0.0, k_pf_attn_out<HD_, G_>, dim3(n), dim3(NT),            \
                                 sizeof(float) * c.n_heads * hd, af, pos0, (const float*)B.st, ao, fa_ch));         \
        } else {                                                                                                 \
            GH_CHECK(sink_launch(sink, "pf_attn", 0.0, k_pf_attn<HD_, G_>, dim3(n * nkv * a.nc), dim3(NT), 0,    \
                                 a, (const float*)B.q, pos0, B.st));                                            \
            GH_CHECK(sink_launch(sink, "pf_attn_out", 0.0, k_pf_attn_out<HD_, G_>, dim3(n), dim3(NT),            \
                                 sizeof(float) * c.n_heads * hd, a, pos0, (const float*)B.st, ao, 0));          \
        }                                                                                                        \
    } else
            GH_PF_ATTN(256, 1) GH_PF_ATTN(256, 2) GH_PF_ATTN(256, 4) GH_PF_ATTN(256, 8)
            GH_PF_ATTN(128, 1) GH_PF_ATTN(128, 2) GH_PF_ATTN(128, 4) GH_PF_ATTN(128, 8)
            GH_PF_ATTN(32, 1) GH_PF_ATTN(32, 2) GH_PF_ATTN(32, 4) GH_PF_ATTN(32, 8)
            return set_error(GH_ERR_INVALID, "prefill: unsupported head_dim %d / group %d", hd, G);
#undef GH_PF_ATTN
        }
        GH_CHECK(gemm("pf_o", L.o, &S));
        // post-attention norm + residual + pre-FFN norm
        {
            PfRows r{};
            r.embd = m->embd;
            r.base = B.x;
            r.part = B.part;
            r.S = S;
            r.ld = L.o.tiles * TILE_ROWS;
            r.Pp = Pp;
            r.w_post = (c.flags & GH_FLAG_POST_ATTN_NORM) ? L.post_attn : nullptr;
            r.w_norm = L.ffn_norm ? L.ffn_norm : L.post_attn;
            r.eps = eps;
            r.zc = zc;
            r.H = H;
            r.x_out = B.x1;
            r.a = A(H);
            GH_CHECK(rows("pf_rows", r, n));
        }
        GH_CHECK(gemm("pf_gate_up", L.gu, &S));
        {
            auto geglu = [&](auto sc) {
                return sink_launch(sink, "pf_geglu", 0.0, k_pf_geglu<decltype(sc)::value>, dim3(n), dim3(NT),
                                   sizeof(float) * F, (const float*)B.part, L.gu.tiles * TILE_ROWS, Pp, F, m->f_pad,
                                   A(F));
            };
            switch (S) {
                case 1: GH_CHECK(geglu(std::integral_constant<int, 1>{})); break;
                case 2: GH_CHECK(geglu(std::integral_constant<int, 2>{})); break;
                case 3: GH_CHECK(geglu(std::integral_constant<int, 3>{})); break;
                case 4: GH_CHECK(geglu(std::integral_constant<int, 4>{})); break;
                case 5: GH_CHECK(geglu(std::integral_constant<int, 5>{})); break;
                case 6: GH_CHECK(geglu(std::integral_constant<int, 6>{})); break;
                case 7: GH_CHECK(geglu(std::integral_constant<int, 7>{})); break;
                case 8: GH_CHECK(geglu(std::integral_constant<int, 8>{})); break;
                default: return set_error(GH_ERR_INVALID, "prefill: %d gate/up splits (1..8)", S);
            }
        }
        GH_CHECK(gemm("pf_down", L.down, &S));
    }
    if (!head) {
        // the next chunk's layer 0 starts from the embedding; nothing carries over
        return GH_OK;
    }
    // last token: final residual + norm into the LM head's input, then the
    // decode step's LM head and next-token selection at its position
    {
        const LayerDev& P = m->layers[c.n_layers - 1];
        PfRows r{};
        r.embd = m->embd;
        r.base = B.x1;
        r.part = B.part;
        r.S = S;
        r.ld = P.down.tiles * TILE_ROWS;
        r.Pp = Pp;
        r.w_post = (c.flags & GH_FLAG_POST_FFN_NORM) ? P.post_ffw : nullptr;
        r.w_norm = m->out_norm;
        r.eps = eps;
        r.zc = zc;
        r.H = H;
        r.layer_out = m->layer_out + (size_t)(c.n_layers - 1) * H;
        r.t_layer = n - 1;
        r.a = A(H);
        r.xn_out = m->xn_final;
        r.t0 = n - 1;
        GH_CHECK(rows("pf_final_norm", r, 1));
    }
    return enqueue_head(m, kv, sink, pos0 + n - 1);
}
#endif  // GH_IN_TU(3)

#if GH_IN_TU(4)
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

__global__ void k_sum_partials(const float* part, int S, int ld, int rows, int softcap, float cap, float* y) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float a = 0.0f;
#pragma unroll 8
    for (int s = 0; s < S; ++s) a += part[(size_t)s * ld + r];
    y[r] = softcap ? cap * tanhf(a / cap) : a;
}

// The whole input vector (up to 256 * MG float4 groups) in registers, loaded
// in one round trip, for the row-group kernel (k_mq_rows).
template <int MG>
struct ProWide {
    const float* x;
    struct Regs {
        float4 v[MG];
    };
    __device__ void load(Regs& r, int c0, int n) const {
        const BufView X(x + c0, (size_t)n * 4);
#pragma unroll
        for (int k = 0; k < MG; ++k) r.v[k] = X.f4(16u * (threadIdx.x + k * NT));
    }
    template <int FMT>
    __device__ void finish(const MvLds& L, Regs& r, int, int n) const {
        const int ng = n >> 2;
#pragma unroll
        for (int k = 0; k < MG; ++k)
            if (k * NT < ng) emit_x4<FMT>(L, threadIdx.x + k * NT, ng, r.v[k]);
    }
};
constexpr int RG16_MG = 8;   // input columns up to 8192

int launch_matvec_plain(const DMat& w, const Plan& p, const float* x, float* part, float* y, int softcap, float cap,
                        hipStream_t s) {
    if (p.rg16) {
        const int R = p.rg16;
        if (w.fmt != FMT_Q4 || w.cols > 4 * NT * RG16_MG || (R != 4 && R != 8 && R != 16))
            return set_error(GH_ERR_INVALID, "row-group matvec: Q4_0 with at most %d columns, 4, 8 or 16 rows (%d)",
                             4 * NT * RG16_MG, R);
        DMat wk = w;
        wk.order_in = p.order_in;
        ProWide<RG16_MG> pro{x};
        EpiOut epi{y, w.rows, softcap, cap};
        const size_t lds = mv_lds_bytes(FMT_Q4M, w.nblk, 0);
        hipLaunchKernelGGL((k_mq_rows<ProWide<RG16_MG>, EpiOut>), dim3((w.rows + R - 1) / R), dim3(NT), lds, s, wk, R,
                           pro, epi);
        GH_HIP(hipGetLastError());
        return GH_OK;
    }
    ProPlain pro{x};
    Sink k;
    k.s = s;
    if (p.S == 1) {
        EpiOut epi{y, w.rows, softcap, cap};
        return launch_mv(k, "matvec", 0.0, w, p, pro, epi, 0);
    }
    EpiPartial epi{part, w.tiles * TILE_ROWS};
    GH_CHECK(launch_mv(k, "matvec", 0.0, w, p, pro, epi, 0));
    hipLaunchKernelGGL(k_sum_partials, dim3((w.rows + 255) / 256), dim3(256), 0, s, part, p.S, w.tiles * TILE_ROWS,
                       w.rows, softcap, cap, y);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

__global__ __launch_bounds__(NT) void k_rmsnorm(const float* x, const float* w, int n, float eps, int zc, float* y) {
    __shared__ float slot[4];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += NT) ss += x[i] * x[i];
    const float rms = sqrtf(block_sum(ss, slot) / (float)n + eps);
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

int launch_qk_norm(const float* x, const float* w, int n_heads, int hd, float eps, int zc, float* y, hipStream_t s) {
    const dim3 grid((n_heads + 3) / 4), block(NT);
    if (hd == 256) hipLaunchKernelGGL(k_qk_norm<256>, grid, block, 0, s, x, w, n_heads, eps, zc, y);
    else if (hd == 128) hipLaunchKernelGGL(k_qk_norm<128>, grid, block, 0, s, x, w, n_heads, eps, zc, y);
    else if (hd == 32) hipLaunchKernelGGL(k_qk_norm<32>, grid, block, 0, s, x, w, n_heads, eps, zc, y);
    else return set_error(GH_ERR_INVALID, "qk_norm: unsupported head_dim %d", hd);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

template <int HD>
__global__ void k_rope(float* x, int n_heads, const float2* cs) {
    const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (h >= n_heads) return;
    wave_head_rope<HD>(x + h * HD, cs);
}

int launch_rope(float* x, int n_heads, int hd, const float* cs_dev, hipStream_t s) {
    const dim3 grid((n_heads + 3) / 4), block(NT);
    const float2* cs = (const float2*)cs_dev;
    if (hd == 256) hipLaunchKernelGGL(k_rope<256>, grid, block, 0, s, x, n_heads, cs);
    else if (hd == 128) hipLaunchKernelGGL(k_rope<128>, grid, block, 0, s, x, n_heads, cs);
    else if (hd == 32) hipLaunchKernelGGL(k_rope<32>, grid, block, 0, s, x, n_heads, cs);
    else return set_error(GH_ERR_INVALID, "rope: unsupported head_dim %d", hd);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

int launch_attention(const float* q, const float* kc, const float* vc, int nq, int nkv, int hd, int p_begin, int p_end,
                     int n_splits, float* part, float* out, hipStream_t s) {
    AttnArgs a{};
    a.q = q;
    a.kc = const_cast<float*>(kc);
    a.vc = const_cast<float*>(vc);
    a.nkv = nkv;
    a.scale = 1.0f / sqrtf((float)hd);
    a.part = part;
    a.nc = n_splits;
    a.set_range(p_begin, p_end);
    Sink k;
    k.s = s;
    const int G = nq / nkv;
    // head_dim 256, chunks of 64 positions or more, or 64+ chunks: the step
    // kernel's streaming body (16 % faster than a separate wave-streaming
    // kernel at 8192 and 32768 positions on MI355X; at 8192 positions, 256
    // chunks of 32, it takes one round per wave and one HBM round trip:
    // 10.2 us against 11.6 with the sub-chunk kernel over cold caches);
    // fewer, shorter chunks: the 32-position sub-chunk kernel (0.3 us faster
    // on the last 512).  Eight waves per workgroup, to have every round of a
    // 128-position chunk in flight, need more than 256 VGPRs and spill.
    const bool g_ok = G == 1 || G == 2 || G == 4 || G == 8;
    const bool views_ok = (size_t)p_end * nkv * hd * 4 <= 0x7fffffffu;  // the body's buffer views
    // few chunks and 4+ q heads per kv head: one workgroup per (chunk, q
    // head), as in the step, while that keeps the grid within one per CU
    static const char* hs_env = std::getenv("GH_ATTN_HSPLIT");  // 0: one workgroup per chunk
    const bool hsplit = hd == 256 && views_ok && (G == 4 || G == 8) && nkv * a.n_used * G <= 256 &&
                        !(hs_env && *hs_env == '0');
    if (hsplit) {
        const char* xe = std::getenv("GH_ATTN_XCD");  // 0: workgroups in plain order
        a.xcd = xe && *xe == '0' ? 0 : 1;
        const dim3 grid(a.xcd ? 8 * G * ((nkv * a.nc + 7) / 8) : nkv * a.nc * G);
        if (G == 4) hipLaunchKernelGGL((k_attn_op<256, 4, 4>), grid, dim3(NT), 0, s, a);
        else hipLaunchKernelGGL((k_attn_op<256, 8, 8>), grid, dim3(NT), 0, s, a);
    } else if (hd == 256 && g_ok && views_ok && (a.ch >= 64 || a.n_used >= 64)) {
        const dim3 grid(nkv * a.nc);
        if (G == 1) hipLaunchKernelGGL((k_attn_op<256, 1>), grid, dim3(NT), 0, s, a);
        else if (G == 2) hipLaunchKernelGGL((k_attn_op<256, 2>), grid, dim3(NT), 0, s, a);
        else if (G == 4) hipLaunchKernelGGL((k_attn_op<256, 4>), grid, dim3(NT), 0, s, a);
        else hipLaunchKernelGGL((k_attn_op<256, 8>), grid, dim3(NT), 0, s, a);
    } else {
        GH_CHECK(launch_attn_t<false>(k, 0.0, hd, G, a, nkv));
    }
    const dim3 cgrid(nq * ((hd + COMB_DIMS - 1) / COMB_DIMS));
    if (G % 2 == 0) hipLaunchKernelGGL(k_attn_combine<true>, cgrid, dim3(NT), 0, s, part, n_splits, a.n_used, G, hd, out);
    else hipLaunchKernelGGL(k_attn_combine<false>, cgrid, dim3(NT), 0, s, part, n_splits, a.n_used, G, hd, out);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

// ------------------------------------------------------------------
// Scratch of the allocation-free attention entry point
// (gh_attention_decode_noalloc): the split-K chunk states live in this
// file-scope device array instead of the context's scratch, so the call
// makes no hipMalloc.  Each GPU holds its own copy, at its own address: the
// host takes that address once per device with hipGetSymbolAddress (the
// array's name is a host-side stand-in, not a device pointer) and passes it
// to the kernels.  Every chunk state the merge reads is written by the same
// call first, so nothing needs clearing; calls that overlap on one GPU
// share the array and race.
// ------------------------------------------------------------------
static __device__ __align__(256) float scratch[ATTN_NOALLOC_SCRATCH_FLOATS];

int attn_noalloc_scratch(float** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static float* ptr[kMaxDevices] = {};
    int dev = -1;
    GH_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return set_error(GH_ERR_INVALID, "device %d out of range", dev);
    std::lock_guard<std::mutex> g(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        GH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        ptr[dev] = (float*)p;
    }
    *out = ptr[dev];
    return GH_OK;
}

// Op-level sampling: per-64-row-block softmax statistics, then the draw.
__global__ __launch_bounds__(64) void k_sample_blocks(const float* logits, int n, float inv_t, float* bm, float* bs) {
    const int r = blockIdx.x * 64 + threadIdx.x;
    const bool in = r < n;
    const float y = in ? logits[r] : -INFINITY;
    const float m = wave_max(y);
    const float s = wave_sum(in ? expf((y - m) * inv_t) : 0.0f);
    if (threadIdx.x == 0) {
        bm[blockIdx.x] = m;
        bs[blockIdx.x] = s;
    }
}

__global__ __launch_bounds__(NT) void k_sample_select(const float* bm, const float* bs, int nb, const float* logits, int n,
                                                      float inv_t, uint64_t seed, uint64_t counter, int32_t* token) {
    const int t = sample_select(bm, bs, nb, 64, logits, n, inv_t, philox_uniform(seed, counter));
    if (threadIdx.x == 0) *token = t;
}

__global__ __launch_bounds__(NT) void k_sample_top_k(const float* bm, int nb, const float* logits, int n, int top_k,
                                                     float inv_t, uint64_t seed, uint64_t counter, int32_t* token) {
    const int t = sample_top_k(bm, nb, 64, logits, n, top_k, inv_t, philox_uniform(seed, counter));
    if (threadIdx.x == 0) *token = t;
}

int launch_sample_logits(const float* logits, int n, float inv_t, int top_k, uint64_t seed, uint64_t counter,
                         float* scratch, int32_t* token, hipStream_t s) {
    if (!(inv_t > 0.0f)) return set_error(GH_ERR_INVALID, "sampling needs a temperature > 0");
    if (top_k < 0 || top_k > GH_TOP_K_MAX) return set_error(GH_ERR_RANGE, "top_k %d outside [0, %d]", top_k, GH_TOP_K_MAX);
    const int nb = (n + 63) / 64;
    hipLaunchKernelGGL(k_sample_blocks, dim3(nb), dim3(64), 0, s, logits, n, inv_t, scratch, scratch + nb);
    if (top_k > 0)
        hipLaunchKernelGGL(k_sample_top_k, dim3(1), dim3(NT), 0, s, (const float*)scratch, nb, logits, n, top_k, inv_t,
                           seed, counter, token);
    else
        hipLaunchKernelGGL(k_sample_select, dim3(1), dim3(NT), 0, s, (const float*)scratch,
                           (const float*)(scratch + nb), nb, logits, n, inv_t, seed, counter, token);
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

// per-block argmax keys, then one block reduces them
__global__ __launch_bounds__(NT) void k_argmax_blocks(const float* v, int n, unsigned long long* cand) {
    __shared__ unsigned long long slot[4];
    unsigned long long best = 0ull;
    for (int i = blockIdx.x * NT + threadIdx.x; i < n; i += gridDim.x * NT) best = umax64(best, argmax_key(v[i], i));
    best = block_max_key(best, slot);
    if (threadIdx.x == 0) cand[blockIdx.x] = best;
}

__global__ __launch_bounds__(NT) void k_argmax_final(const unsigned long long* cand, int n, unsigned long long* key) {
    __shared__ unsigned long long slot[4];
    unsigned long long best = 0ull;
    for (int i = threadIdx.x; i < n; i += NT) best = umax64(best, cand[i]);
    best = block_max_key(best, slot);
    if (threadIdx.x == 0) *key = best;
}

int launch_argmax(const float* v, int n, unsigned long long* key, hipStream_t s) {
    const int blocks = std::max(1, std::min(1024, (n + NT - 1) / NT));
    // key points at a buffer of 1 + 1024 entries: [0] result, [1..] per-block keys
    hipLaunchKernelGGL(k_argmax_blocks, dim3(blocks), dim3(NT), 0, s, v, n, key + 1);
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(NT), 0, s, key + 1, blocks, key);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

// ------------------------------------------------------------------
// measured stream-read peak: every byte of a buffer read once with
// non-temporal 16-byte loads; workgroup b reads the contiguous chunk
// [b * chunk, (b + 1) * chunk) (the access shape of a matvec tile, and
// faster on HBM than a grid-stride walk), eight loads in flight per thread
// ------------------------------------------------------------------
constexpr int SR_GRID = 4096, SR_UNROLL = 8;

__global__ __launch_bounds__(NT) void k_stream_read(const void* p, uint32_t n4, uint32_t chunk4, float* sink) {
    const BufView B(p, (size_t)n4 * 16);  // the last chunk's tail reads zeros
    const uint32_t b = blockIdx.x * chunk4;
    float4 acc = f4z();
    for (uint32_t i = b + threadIdx.x; i < b + chunk4; i += SR_UNROLL * NT) {
        float4 v[SR_UNROLL];
#pragma unroll
        for (int u = 0; u < SR_UNROLL; ++u) v[u] = B.f4<CP_NT>(16u * (i + u * NT));
#pragma unroll
        for (int u = 0; u < SR_UNROLL; ++u) acc = acc + v[u];
    }
    const float t = (acc.x + acc.y) + (acc.z + acc.w);
    if (t == 1.5f) sink[blockIdx.x] = t;  // keeps the loads; the zero fill makes it never true
}

int launch_stream_read(const void* p, size_t bytes, float* sink, hipStream_t s) {
    if (bytes % 16 || bytes > (1u << 31) - 16u) return set_error(GH_ERR_INVALID, "stream read: %zu bytes", bytes);
    const uint32_t n4 = (uint32_t)(bytes / 16), step = SR_UNROLL * NT;
    const uint32_t chunk4 = ((n4 + SR_GRID - 1) / SR_GRID + step - 1) / step * step;
    hipLaunchKernelGGL(k_stream_read, dim3(SR_GRID), dim3(NT), 0, s, p, n4, chunk4, sink);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

// Exchange probe (gh_time_exchange): `rounds` all-to-all exchanges among the
// grid's workgroups through the persistent step's self-validating words.  In
// round r each workgroup publishes its word (epoch epoch0 + r) in buffer
// r % 2, then its first n_wg threads poll every workgroup's word of that
// buffer until it carries the round's epoch.  A workgroup starts round r + 1
// only after seeing every round-r word, so no one is two rounds ahead of a
// reader of the same buffer.  Workgroup 0 stamps s_memrealtime (100 MHz)
// before the first round and after the last.  Every wait is bounded: a
// timeout sets *err, after which all waits give up at once.
__global__ __launch_bounds__(NT) void k_xchg_probe(uint64_t* words, int n_wg, int rounds, uint32_t epoch0, int* err,
                                                   unsigned long long* stamps) {
    const int wg = blockIdx.x, tid = threadIdx.x;
    if (wg == 0 && tid == 0) stamps[0] = __builtin_amdgcn_s_memrealtime();
    for (int r = 0; r < rounds; ++r) {
        const uint32_t e = epoch0 + (uint32_t)r;
        uint64_t* buf = words + (size_t)(r & 1) * n_wg;
        if (tid == 0) st_word(buf + wg, e, (float)r);
        if (tid < n_wg) {
            uint64_t v = ld_word(buf + tid);
            for (int spin = 1; (uint32_t)(v >> 32) != e; ++spin) {
                if (spin >= XCHG_SPIN || ((spin & 63) == 0 &&
                                          __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
                    __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                v = ld_word(buf + tid);
            }
        }
        __syncthreads();
    }
    if (wg == 0 && tid == 0) stamps[1] = __builtin_amdgcn_s_memrealtime();
}

int launch_xchg_probe(uint64_t* words, int n_wg, int rounds, int* err, unsigned long long* stamps, hipStream_t s) {
    if (n_wg < 1 || n_wg > NT || rounds < 1) return set_error(GH_ERR_INVALID, "internal: exchange probe of %d workgroups", n_wg);
    hipLaunchKernelGGL(k_xchg_probe, dim3(n_wg), dim3(NT), 0, s, words, n_wg, rounds, 1u, err, stamps);
    GH_HIP(hipGetLastError());
    return GH_OK;
}

#endif  // GH_IN_TU(4)

}  // namespace gh
