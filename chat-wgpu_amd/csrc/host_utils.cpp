// Host-side helpers: the Q4_0 re-quantizer (q4.rs:37-61 with an f16 scale),
// GGUF block splitting, and the seeded synthetic data generators.
//
// Synthetic values are counter-based: element i of a tensor depends only on
// (key, i), so any thread count gives the same bytes.  Normals come from
// Box-Muller in f64 (glibc log/cos/sqrt), rounded once to the target type.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "cw_internal.hpp"

namespace {

inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t rnd(uint64_t key, uint64_t i) { return mix64(key ^ mix64(i)); }

inline double normal01(uint64_t key, uint64_t i) {
    const uint64_t h1 = rnd(key, 2 * i), h2 = rnd(key, 2 * i + 1);
    const double u1 = (double)((h1 >> 11) + 1) * 0x1p-53;  // (0, 1]
    const double u2 = (double)(h2 >> 11) * 0x1p-53;        // [0, 1)
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

// Rust f32::max (NaN operand ignored) and `f32 as i32` (saturating, NaN->0).
inline float rust_fmax(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}
inline int32_t rust_as_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return -2147483647 - 1;
    return (int32_t)v;
}

}  // namespace

extern "C" {

int cw_q4_quantize(const float *data, size_t out_f, size_t in_f, uint16_t *scales,
                   uint8_t *quants) {
    CW_CHECK_ARG(data && scales && quants, "cw_q4_quantize: null argument");
    CW_CHECK_ARG(in_f > 0 && in_f % 32 == 0, "cw_q4_quantize: in_f=%zu must be a multiple of 32",
                 in_f);
    const size_t nb = in_f / 32;
    cwi::parallel_for(out_f, [&](size_t lo, size_t hi) {
        for (size_t o = lo; o < hi; ++o) {
            for (size_t b = 0; b < nb; ++b) {
                const float *v = data + o * in_f + b * 32;
                float absmax = 0.0f;
                for (int j = 0; j < 32; ++j) absmax = rust_fmax(absmax, std::fabs(v[j]));
                const uint16_t h = cwi::f32_to_f16_bits(absmax / 8.0f);
                const float d = cwi::f16_bits_to_f32(h);
                const float inv = d != 0.0f ? 1.0f / d : 0.0f;
                scales[o * nb + b] = h;
                uint8_t *q = quants + (o * nb + b) * 16;
                for (int j = 0; j < 16; ++j) {
                    int32_t lo4 = rust_as_i32(std::round(v[j] * inv)) + 8;
                    int32_t hi4 = rust_as_i32(std::round(v[j + 16] * inv)) + 8;
                    lo4 = std::min(15, std::max(0, lo4));
                    hi4 = std::min(15, std::max(0, hi4));
                    q[j] = (uint8_t)(lo4 | (hi4 << 4));
                }
            }
        }
    });
    return CW_OK;
}

int cw_q4_split_blocks(const uint8_t *blocks, size_t nblocks, uint16_t *scales, uint8_t *quants) {
    CW_CHECK_ARG(blocks && scales && quants, "cw_q4_split_blocks: null argument");
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t *p = blocks + b * 18;
        scales[b] = (uint16_t)(p[0] | (p[1] << 8));
        std::memcpy(quants + b * 16, p + 2, 16);
    }
    return CW_OK;
}

uint64_t cw_synth_key(uint64_t seed, const char *name) {
    uint64_t h = 1469598103934665603ull;
    for (const unsigned char *p = (const unsigned char *)(name ? name : ""); *p; ++p)
        h = (h ^ (uint64_t)*p) * 1099511628211ull;
    return mix64(h ^ mix64(seed));
}

int cw_synth_q4(uint64_t key, size_t nblocks, float sigma, uint16_t *scales, uint8_t *quants) {
    CW_CHECK_ARG(scales && quants, "cw_synth_q4: null argument");
    const uint64_t kd = mix64(key ^ 0xD5ull), kq = mix64(key ^ 0x95ull);
    cwi::parallel_for(nblocks, [&](size_t lo, size_t hi) {
        for (size_t b = lo; b < hi; ++b) {
            const float d = (float)std::fabs((double)sigma * normal01(kd, b));
            scales[b] = cwi::f32_to_f16_bits(d);
            const uint64_t w0 = rnd(kq, 2 * b), w1 = rnd(kq, 2 * b + 1);
            std::memcpy(quants + b * 16, &w0, 8);
            std::memcpy(quants + b * 16 + 8, &w1, 8);
        }
    });
    return CW_OK;
}

int cw_synth_normal_f32(uint64_t key, size_t n, float mean, float std_, float *out) {
    CW_CHECK_ARG(out != nullptr, "cw_synth_normal_f32: null argument");
    cwi::parallel_for(n, [&](size_t lo, size_t hi) {
        for (size_t i = lo; i < hi; ++i)
            out[i] = (float)((double)mean + (double)std_ * normal01(key, i));
    });
    return CW_OK;
}

int cw_synth_normal_f16(uint64_t key, size_t n, float mean, float std_, uint16_t *out) {
    CW_CHECK_ARG(out != nullptr, "cw_synth_normal_f16: null argument");
    cwi::parallel_for(n, [&](size_t lo, size_t hi) {
        for (size_t i = lo; i < hi; ++i)
            out[i] = cwi::f32_to_f16_bits((float)((double)mean + (double)std_ * normal01(key, i)));
    });
    return CW_OK;
}

int cw_synth_tokens(uint64_t key, size_t n, uint32_t vocab, uint32_t *out) {
    CW_CHECK_ARG(out != nullptr && vocab > 0, "cw_synth_tokens: bad argument");
    for (size_t i = 0; i < n; ++i) out[i] = (uint32_t)(rnd(key, i) % vocab);
    return CW_OK;
}

}  // extern "C"
