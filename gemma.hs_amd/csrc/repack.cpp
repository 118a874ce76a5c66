// Host-side layout conversion (GGUF Q4_0 rows / f32 rows -> device tiles),
// work-split planning, and the thread-local error slot of the C ABI.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "common.h"

namespace gh {

static thread_local std::string g_err;

int set_error(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

// IEEE binary16 -> binary32; subnormals flush to signed zero when ftz
// (src/Gemma/GGUF.hs:797-820 halfToFloat).
float f16_to_f32(uint16_t h, bool ftz) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF, bits;
    if (e == 0) {
        if (m == 0 || ftz) {
            bits = sign;
        } else {
            float f = (float)m * 5.9604644775390625e-08f;
            std::memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// GGUF Q4_0 (row-major, 18-byte blocks {f16 d, qs[16]}) -> device tiles.
// The code bytes are copied unchanged; a subnormal scale becomes a signed
// zero when ftz (the dequantised value then equals halfToFloat's), so the
// device never needs a denormal-mode-dependent conversion.
void repack_q4_0(const uint8_t* raw, int64_t rows, int64_t cols, bool ftz, uint8_t* codes,
                 uint16_t* scales, int64_t tiles) {
    const int64_t nb = cols / 32;
    std::memset(codes, 0, (size_t)tiles * nb * TILE_ROWS * 16);
    std::memset(scales, 0, (size_t)tiles * nb * TILE_ROWS * 2);
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t t = r / TILE_ROWS, lr = r % TILE_ROWS;
        const uint8_t* src = raw + r * nb * 18;
        for (int64_t b = 0; b < nb; ++b, src += 18) {
            const int64_t idx = (t * nb + b) * TILE_ROWS + lr;
            std::memcpy(codes + idx * 16, src + 2, 16);
            uint16_t h = (uint16_t)(src[0] | (src[1] << 8));
            if (ftz && ((h & 0x7C00) == 0)) h &= 0x8000;
            scales[idx] = h;
        }
    }
}

// f32 row-major -> tiles of 4-column blocks: dst[((t*nb4 + c/4)*128 + r%128)*4 + c%4].
void repack_f32(const float* src, int64_t rows, int64_t cols, float* dst, int64_t tiles) {
    const int64_t nb4 = cols / 4;
    std::memset(dst, 0, (size_t)tiles * nb4 * TILE_ROWS * 16);
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t t = r / TILE_ROWS, lr = r % TILE_ROWS;
        for (int64_t c = 0; c < cols; ++c)
            dst[((t * nb4 + c / 4) * TILE_ROWS + lr) * 4 + (c & 3)] = src[r * cols + c];
    }
}

// Pick S (column splits) so that tiles*S approaches target_wgs while each
// split keeps at least 4 column blocks, then the per-wave register batch.
int kbw_for(int fmt, int per_wave) {
    if (fmt != FMT_Q4) return 8;
    static const int kQ4[] = {1, 2, 3, 4, 6, 7, 9, 10};
    for (int k : kQ4)
        if (k >= per_wave) return k;
    return 10;
}

Plan choose_plan(int fmt, int tiles, int nblk, int target_wgs, int max_s) {
    Plan p;
    int cap = std::max(1, std::min(max_s, nblk / 4));
    int s = (target_wgs + tiles - 1) / tiles;
    p.S = std::max(1, std::min(s, cap));
    int per_wg = (nblk + p.S - 1) / p.S;
    p.kbw = kbw_for(fmt, (per_wg + 3) / 4);
    return p;
}

void rope_table(const float* inv_freq, int half, int pos0, int n_pos, float* out) {
    for (int p = 0; p < n_pos; ++p)
        for (int i = 0; i < half; ++i) {
            const float ang = (float)(pos0 + p) * inv_freq[i];
            out[((size_t)p * half + i) * 2] = cosf(ang);
            out[((size_t)p * half + i) * 2 + 1] = sinf(ang);
        }
}

}  // namespace gh

extern "C" const char* gh_last_error(void) { return gh::g_err.c_str(); }
extern "C" const char* gh_version(void) { return "gemma_hip 0.1 (gfx950)"; }
