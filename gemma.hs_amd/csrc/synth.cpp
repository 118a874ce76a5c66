// Seeded synthetic tensors: SplitMix64 streams + Box-Muller normals.
//
// The same seed and tensor name give the same bytes on every x86-64 host,
// so a GPU box regenerates a model bit-for-bit instead of shipping hundreds
// of MB of weights.  Streams are per (tensor, row) so large tensors are
// generated on several threads without changing the bytes.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "common.h"

namespace gh {

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct SplitMix {
    uint64_t s;
    explicit SplitMix(uint64_t seed) : s(seed) {}
    uint64_t next() {
        s += 0x9E3779B97F4A7C15ull;
        return mix64(s);
    }
    // N(0,1): Box-Muller in double, first output of the pair.
    double normal() {
        double u1 = (double)((next() >> 11) + 1) * 0x1.0p-53;  // (0, 1]
        double u2 = (double)(next() >> 11) * 0x1.0p-53;        // [0, 1)
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

static uint64_t fnv1a64(const char* s) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (; *s; ++s) {
        h ^= (uint8_t)*s;
        h *= 0x100000001B3ull;
    }
    return h;
}

static uint64_t stream_seed(uint64_t seed, const char* name, uint64_t row) {
    return mix64(mix64(seed ^ fnv1a64(name)) ^ (row * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull));
}

// IEEE binary32 -> binary16, round to nearest even, subnormals kept.
uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // >= 65520 -> inf
    if (ax < 0x33000000u) return (uint16_t)sign;                // < 2^-25 -> 0
    int e = (int)(ax >> 23);
    if (e < 113) {  // f16 subnormal range
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        int shift = 126 - e;  // 14..24
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t h = ((uint32_t)(e - 112) << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

static void parallel_rows(int64_t rows, const std::function<void(int64_t, int64_t)>& fn) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt > 16) nt = 16;
    if (nt < 1 || rows < 512) {
        fn(0, rows);
        return;
    }
    std::vector<std::thread> th;
    int64_t per = (rows + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        int64_t b = t * per, e = std::min<int64_t>(rows, b + per);
        if (b >= e) break;
        th.emplace_back(fn, b, e);
    }
    for (auto& t : th) t.join();
}

}  // namespace gh

using namespace gh;

extern "C" int gh_synth_f32(uint64_t seed, const char* name, float sigma, float* out, size_t n) {
    if (!name || (!out && n)) return set_error(GH_ERR_INVALID, "gh_synth_f32: null argument");
    SplitMix r(stream_seed(seed, name, 0));
    for (size_t i = 0; i < n; ++i) out[i] = (float)(r.normal() * (double)sigma);
    return GH_OK;
}

extern "C" int gh_synth_q4_0(uint64_t seed, const char* name, float scale_sigma, int64_t rows,
                             int64_t cols, uint8_t* out) {
    if (!name || !out || rows <= 0 || cols <= 0 || cols % 32)
        return set_error(GH_ERR_INVALID, "gh_synth_q4_0: bad arguments (cols %% 32 must be 0)");
    const int64_t nb = cols / 32;
    parallel_rows(rows, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r) {
            SplitMix g(stream_seed(seed, name, (uint64_t)r));
            uint8_t* row = out + r * nb * 18;
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t* blk = row + b * 18;
                float s = (float)(std::fabs(g.normal()) * (double)scale_sigma);
                uint16_t h = f32_to_f16_rne(s);
                blk[0] = (uint8_t)(h & 0xFF);
                blk[1] = (uint8_t)(h >> 8);
                uint64_t c0 = g.next(), c1 = g.next();
                std::memcpy(blk + 2, &c0, 8);
                std::memcpy(blk + 10, &c1, 8);
            }
        }
    });
    return GH_OK;
}

extern "C" int gh_synth_kv(uint64_t seed, int32_t layer, int32_t n_pos, int32_t width, float sigma, float* k_out,
                           float* v_out) {
    if (layer < 0 || n_pos < 0 || width <= 0 || (n_pos && (!k_out || !v_out)))
        return set_error(GH_ERR_INVALID, "gh_synth_kv: bad arguments");
    // one stream per (layer, K or V, position): rows of `width` values
    parallel_rows(n_pos, [&](int64_t p0, int64_t p1) {
        for (int64_t p = p0; p < p1; ++p) {
            const uint64_t row = ((uint64_t)(uint32_t)layer << 32) | (uint64_t)p;
            SplitMix gk(stream_seed(seed, "kv.k", row)), gv(stream_seed(seed, "kv.v", row));
            float* kr = k_out + p * (int64_t)width;
            float* vr = v_out + p * (int64_t)width;
            for (int32_t i = 0; i < width; ++i) kr[i] = (float)(gk.normal() * (double)sigma);
            for (int32_t i = 0; i < width; ++i) vr[i] = (float)(gv.normal() * (double)sigma);
        }
    });
    return GH_OK;
}

extern "C" int gh_synth_tokens(uint64_t seed, const char* name, int32_t n, int32_t vocab,
                               int32_t* out) {
    if (!name || !out || n < 0 || vocab <= 0)
        return set_error(GH_ERR_INVALID, "gh_synth_tokens: bad arguments");
    SplitMix r(stream_seed(seed, name, 0));
    for (int32_t i = 0; i < n; ++i)
        out[i] = (int32_t)(((r.next() >> 32) * (uint64_t)vocab) >> 32);
    return GH_OK;
}
