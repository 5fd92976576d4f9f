/*
 * cw_oracle.c -- CPU restatement of chat-wgpu's decode token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the oracle the device results are
 * compared with: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (chat-wgpu_amd/) never links or
 * calls it.
 *
 * Every function restates one piece of the reference (Rust + WGSL), cited as
 * file:line relative to the reference repository root.  Arithmetic is plain
 * f32 in the order the reference states it, compiled with -ffp-contract=off
 * (Rust never contracts a*b+c into an FMA).  Where the reference leaves a
 * format undefined (f16 KV cache, f16 scale of the re-quantized tied LM head,
 * RoPE angles at large positions) the choice is stated at the function.
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   or_f16_to_f32          exhaustive vs numpy float16 + dequant.rs:137-142 KAT
 *   or_f32_to_f16          exhaustive round trip + numpy astype(float16)
 *   or_dequant_q4_0        dequant.rs:190-200 KAT + brute force over d x nibble
 *   or_dequant_f16         exhaustive over all 65,536 patterns (or_f16_to_f32)
 *   or_dequant_q8_0        dequant.rs:150-161 KAT; d = 1 -> the int8 bytes
 *   or_dequant_q4_1        dequant.rs:163-173 KAT; d = 1, m = 0 -> nibble map
 *   or_dequant_q6_k        dequant.rs:175-188 KAT; round trip through a
 *                          packer written from ggml's block_q6_K layout
 *   or_quantize_q4_0       q4.rs:37-61: exact-grid round trip, clamp, d==0 case
 *   or_q4_gemv / _refmt    main.rs:120-152 KAT shape, closed forms, f64 truth
 *   or_naive_matmul        closed form (ones -> k), f64 truth
 *   or_rmsnorm             main.rs:61-67 KAT, scale invariance, f64 truth
 *   or_rope_table/or_rope  main.rs:93-98 (pos 0 identity), norm preservation,
 *                          relative-position invariance, f32 literal formula,
 *                          rotation direction by one-hot inputs against
 *                          numpy's cos/sin in rope.wgsl:30-31's signs
 *   or_attention           main.rs:100-118 (seq=1 -> V), constant-K mean,
 *                          f64 two-pass softmax
 *   or_swiglu / or_add     main.rs:77-82 and main.rs:154-161 KATs
 *   or_argmax              argmax.wgsl:4-5,43 tie rule, brute force
 *   or_fill / or_fnv_seed  main.rs:253-266 ([-0.1, 0) range quirk)
 *   model forward          qwen3.rs:139-191: closed-form composition checks
 *   and generate           (tests/test_oracle_composition.py: attention and
 *                          FFN switched off, pos 0 -> V under the GQA map,
 *                          the K row written, zero query -> mean of V, the
 *                          FFN alone, P + N - 1 forwards) and the tiny-model
 *                          fixture; mod.rs:57-125
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_API __attribute__((visibility("default")))

/* Thread count of the OpenMP loops (rows of a GEMV, heads of attention).
 * Every row / head is summed by one thread in a fixed order, so results do
 * not depend on it. */
OR_API void or_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
OR_API int or_get_threads(void) { return omp_get_max_threads(); }

/* ------------------------------------------------------------------ */
/* f16 <-> f32                                                         */
/* ------------------------------------------------------------------ */

/* dequant.rs:9-21.  Computed exactly as the reference does: subnormal
 * mant*2^-24, normal (1+mant/1024)*2^(exp-15), exp==31 -> inf / NaN, then
 * the sign applied by negation (so a negative NaN stays negative). */
OR_API float or_f16_to_f32(uint16_t h) {
    int sign = (h >> 15) & 1;
    int e = (h >> 10) & 0x1f;
    float mant = (float)(h & 0x3ff);
    float mag;
    if (e == 0) {
        mag = mant * ldexpf(1.0f, -24);
    } else if (e == 0x1f) {
        mag = (mant == 0.0f) ? INFINITY : NAN;
    } else {
        mag = (1.0f + mant / 1024.0f) * ldexpf(1.0f, e - 15);
    }
    return sign ? -mag : mag;
}

/* IEEE 754 binary32 -> binary16, round to nearest even.  The reference has
 * no f32->f16 path; this is the textbook conversion, used for the f16 scale
 * of the re-quantized tied LM head and for the f16 KV cache. */
OR_API uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf or nan */
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) { /* below 2^-14: f16 subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 (2^-25 ties to even 0) */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e; /* value = m * 2^(e-150); want units of 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* ------------------------------------------------------------------ */
/* Q4_0 blocks                                                         */
/* ------------------------------------------------------------------ */

/* dequant.rs:60-78.  GGUF Q4_0: 18-byte blocks {f16 d, u8 qs[16]};
 * x[j] = d*((qs[j]&15)-8), x[j+16] = d*((qs[j]>>4)-8). */
OR_API void or_dequant_q4_0(const uint8_t *bytes, size_t n, float *out) {
    for (size_t blk = 0; blk < n / 32; ++blk) {
        const uint8_t *b = bytes + blk * 18;
        float d = or_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        for (int j = 0; j < 16; ++j) {
            uint8_t byte = b[2 + j];
            int lo = (int)(byte & 0x0f) - 8;
            int hi = (int)(byte >> 4) - 8;
            out[blk * 32 + j] = d * (float)lo;
            out[blk * 32 + j + 16] = d * (float)hi;
        }
    }
}

/* The same dequantization on the split (structure-of-arrays) image the GPU
 * streams: d[nblocks] f16 bits, qs[nblocks][16] bytes.  Identical values. */
OR_API void or_dequant_q4_0_soa(const uint16_t *d, const uint8_t *qs, size_t nblocks, float *out) {
    for (size_t blk = 0; blk < nblocks; ++blk) {
        float s = or_f16_to_f32(d[blk]);
        for (int j = 0; j < 16; ++j) {
            uint8_t byte = qs[blk * 16 + j];
            out[blk * 32 + j] = s * (float)((int)(byte & 0x0f) - 8);
            out[blk * 32 + j + 16] = s * (float)((int)(byte >> 4) - 8);
        }
    }
}

/* ------------------------------------------------------------------ */
/* The other ggml dtypes tensor_f32 decodes (gguf.rs:109-122)          */
/* ------------------------------------------------------------------ */

static uint16_t rd_u16(const uint8_t *b, size_t i) { return (uint16_t)(b[i] | (b[i + 1] << 8)); }

/* dequant.rs:37-39: n f16 values. */
OR_API void or_dequant_f16(const uint8_t *bytes, size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) out[i] = or_f16_to_f32(rd_u16(bytes, i * 2));
}

/* dequant.rs:44-56: Q8_0, 34-byte blocks {f16 d, i8 q[32]}, value d*q. */
OR_API void or_dequant_q8_0(const uint8_t *bytes, size_t n, float *out) {
    for (size_t blk = 0; blk < n / 32; ++blk) {
        size_t base = blk * 34;
        float d = or_f16_to_f32(rd_u16(bytes, base));
        for (int j = 0; j < 32; ++j) out[blk * 32 + j] = d * (float)(int8_t)bytes[base + 2 + j];
    }
}

/* dequant.rs:80-97: Q4_1, 20-byte blocks {f16 d, f16 m, u8 qs[16]};
 * x[j] = d*(qs[j]&15) + m, x[j+16] = d*(qs[j]>>4) + m. */
OR_API void or_dequant_q4_1(const uint8_t *bytes, size_t n, float *out) {
    for (size_t blk = 0; blk < n / 32; ++blk) {
        size_t base = blk * 20;
        float d = or_f16_to_f32(rd_u16(bytes, base));
        float m = or_f16_to_f32(rd_u16(bytes, base + 2));
        for (int j = 0; j < 16; ++j) {
            uint8_t byte = bytes[base + 4 + j];
            out[blk * 32 + j] = d * (float)(byte & 0x0f) + m;
            out[blk * 32 + j + 16] = d * (float)(byte >> 4) + m;
        }
    }
}

/* dequant.rs:99-131: Q6_K, 210-byte super-blocks of 256 {ql[128], qh[64],
 * i8 scales[16], f16 d}.  Per half (128 values): for l < 32, four 6-bit
 * values from ql[l], ql[l+32] (low then high nibbles) and the four 2-bit
 * fields of qh[l], each scaled by d*scale[is + 2k] with is = l/16. */
OR_API void or_dequant_q6_k(const uint8_t *bytes, size_t n, float *out) {
    for (size_t blk = 0; blk < n / 256; ++blk) {
        const uint8_t *b = bytes + blk * 210;
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *sc = (const int8_t *)(b + 192);
        float d = or_f16_to_f32(rd_u16(b, 208));
        float *y = out + blk * 256;
        for (int half = 0; half < 2; ++half) {
            int qlo = half * 64, qho = half * 32, sco = half * 8, yo = half * 128;
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                int q1 = ((ql[qlo + l] & 0x0f) | (((qh[qho + l] >> 0) & 3) << 4)) - 32;
                int q2 = ((ql[qlo + l + 32] & 0x0f) | (((qh[qho + l] >> 2) & 3) << 4)) - 32;
                int q3 = ((ql[qlo + l] >> 4) | (((qh[qho + l] >> 4) & 3) << 4)) - 32;
                int q4 = ((ql[qlo + l + 32] >> 4) | (((qh[qho + l] >> 6) & 3) << 4)) - 32;
                y[yo + l] = d * (float)sc[sco + is] * (float)q1;
                y[yo + l + 32] = d * (float)sc[sco + is + 2] * (float)q2;
                y[yo + l + 64] = d * (float)sc[sco + is + 4] * (float)q3;
                y[yo + l + 96] = d * (float)sc[sco + is + 6] * (float)q4;
            }
        }
    }
}

/* Rust `f32 as i32`: saturating, NaN -> 0. */
static int32_t rust_f32_as_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (-2147483647 - 1);
    return (int32_t)v;
}

/* Rust f32::max: returns the non-NaN operand when one is NaN. */
static float rust_fmax(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}

/* q4.rs:37-61, the reference's own re-quantizer: per 32-block d = absmax/8
 * (f32), inv = 1/d or 0, q = clamp(round(v*inv)+8, 0, 15) with Rust's
 * round-half-away-from-zero (C roundf); 8 nibbles per u32, nibble n of word w
 * is element b*32 + w*8 + n. */
OR_API void or_quantize_q4_0(const float *data, size_t out_f, size_t in_f, float *scales,
                             uint32_t *quants) {
    size_t nb = in_f / 32;
    for (size_t o = 0; o < out_f; ++o) {
        for (size_t b = 0; b < nb; ++b) {
            size_t base = o * in_f + b * 32;
            float absmax = 0.0f;
            for (int j = 0; j < 32; ++j) absmax = rust_fmax(absmax, fabsf(data[base + j]));
            float d = absmax / 8.0f;
            float inv = (d != 0.0f) ? 1.0f / d : 0.0f;
            scales[o * nb + b] = d;
            for (int w = 0; w < 4; ++w) {
                uint32_t word = 0;
                for (int n = 0; n < 8; ++n) {
                    float v = data[base + w * 8 + n];
                    int32_t q = rust_f32_as_i32(roundf(v * inv)) + 8;
                    if (q < 0) q = 0;
                    if (q > 15) q = 15;
                    word |= (uint32_t)q << (n * 4);
                }
                quants[o * (in_f / 8) + b * 4 + w] = word;
            }
        }
    }
}

/* The tied LM head (qwen3.rs:93-98 -> q4.rs:37-61) stored as GGUF Q4_0.
 * Same rule as or_quantize_q4_0 except that d is rounded to f16 first and the
 * quants are computed against that stored f16 value (d16 -> f32 -> inv), so the
 * block dequantizes by dequant.rs:60-78.  Nibbles are placed in GGUF order
 * (element j in the low nibble of byte j, element j+16 in its high nibble). */
OR_API void or_quantize_q4_0_gguf(const float *data, size_t out_f, size_t in_f, uint16_t *d16,
                                  uint8_t *qs) {
    size_t nb = in_f / 32;
    for (size_t o = 0; o < out_f; ++o) {
        for (size_t b = 0; b < nb; ++b) {
            size_t base = o * in_f + b * 32;
            float absmax = 0.0f;
            for (int j = 0; j < 32; ++j) absmax = rust_fmax(absmax, fabsf(data[base + j]));
            uint16_t h = or_f32_to_f16(absmax / 8.0f);
            float d = or_f16_to_f32(h);
            float inv = (d != 0.0f) ? 1.0f / d : 0.0f;
            d16[o * nb + b] = h;
            uint8_t *q = qs + (o * nb + b) * 16;
            for (int j = 0; j < 16; ++j) {
                int32_t lo = rust_f32_as_i32(roundf(data[base + j] * inv)) + 8;
                int32_t hi = rust_f32_as_i32(roundf(data[base + j + 16] * inv)) + 8;
                lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
                hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
                q[j] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* GEMV / matmul                                                       */
/* ------------------------------------------------------------------ */

/* main.rs:133-150: the reference's CPU q4 dot over its own layout (f32
 * scales, sequential nibbles): sum += d*(q-8)*x[k], blocks -> words ->
 * nibbles, evaluated left to right without FMA. */
OR_API void or_q4_gemv_refmt(const float *x, const float *scales, const uint32_t *quants,
                             int in_f, int out_f, float *y) {
    int nb = in_f / 32;
#pragma omp parallel for schedule(static)
    for (int o = 0; o < out_f; ++o) {
        float sum = 0.0f;
        for (int b = 0; b < nb; ++b) {
            float d = scales[(size_t)o * nb + b];
            for (int w = 0; w < 4; ++w) {
                uint32_t word = quants[(size_t)o * (in_f / 8) + b * 4 + w];
                for (int n = 0; n < 8; ++n) {
                    uint32_t q = (word >> (n * 4)) & 0xFu;
                    int k = b * 32 + w * 8 + n;
                    float t = d * ((float)q - 8.0f);
                    t = t * x[k];
                    sum = sum + t;
                }
            }
        }
        y[o] = sum;
    }
}

/* The GEMV on GGUF Q4_0 weights (SoA image): each weight dequantized by
 * dequant.rs:60-78 and dotted in ascending k like naive_matmul at m=1
 * (examples/bench/src/lib.rs:221-233): s += a[k]*b[k][j]. */
OR_API void or_q4_gemv(const float *x, const uint16_t *d16, const uint8_t *qs, int in_f, int out_f,
                       float *y) {
    int nb = in_f / 32;
#pragma omp parallel for schedule(static)
    for (int o = 0; o < out_f; ++o) {
        float s = 0.0f;
        for (int b = 0; b < nb; ++b) {
            size_t blk = (size_t)o * nb + b;
            float d = or_f16_to_f32(d16[blk]);
            const uint8_t *q = qs + blk * 16;
            float w[32];
            for (int j = 0; j < 16; ++j) {
                w[j] = d * (float)((int)(q[j] & 15) - 8);
                w[j + 16] = d * (float)((int)(q[j] >> 4) - 8);
            }
            for (int j = 0; j < 32; ++j) {
                float t = x[b * 32 + j] * w[j];
                s = s + t;
            }
        }
        y[o] = s;
    }
}

/* f64 truth of or_q4_gemv: the same dequantized weights, f64 accumulation.
 * Also returns sum_k |w*x| per row (the conditioning of each output). */
OR_API void or_q4_gemv_f64(const float *x, const uint16_t *d16, const uint8_t *qs, int in_f,
                           int out_f, double *y, double *absy) {
    int nb = in_f / 32;
#pragma omp parallel for schedule(static)
    for (int o = 0; o < out_f; ++o) {
        double s = 0.0, a = 0.0;
        for (int b = 0; b < nb; ++b) {
            size_t blk = (size_t)o * nb + b;
            double d = (double)or_f16_to_f32(d16[blk]);
            const uint8_t *q = qs + blk * 16;
            for (int j = 0; j < 16; ++j) {
                double t0 = d * (double)((int)(q[j] & 15) - 8) * (double)x[b * 32 + j];
                double t1 = d * (double)((int)(q[j] >> 4) - 8) * (double)x[b * 32 + j + 16];
                s += t0 + t1;
                a += fabs(t0) + fabs(t1);
            }
        }
        y[o] = s;
        if (absy) absy[o] = a;
    }
}

/* examples/bench/src/lib.rs:221-233, naive_matmul: C[m,n] = A[m,k] B[k,n]. */
OR_API void or_naive_matmul(const float *a, const float *b, int m, int k, int n, float *c) {
#pragma omp parallel for schedule(static)
    for (int j = 0; j < n; ++j) {
        for (int i = 0; i < m; ++i) {
            float s = 0.0f;
            for (int kk = 0; kk < k; ++kk) {
                float t = a[(size_t)i * k + kk] * b[(size_t)kk * n + j];
                s = s + t;
            }
            c[(size_t)i * n + j] = s;
        }
    }
}

/* ------------------------------------------------------------------ */
/* Elementwise / normalisation                                         */
/* ------------------------------------------------------------------ */

/* norm.wgsl:20-42 (rmsnorm): per row inv = inverseSqrt(sum(x^2)/dim + eps),
 * y = x * inv * w.  inverseSqrt is taken as the correctly rounded 1/sqrt. */
OR_API void or_rmsnorm(const float *x, const float *w, int rows, int dim, float eps, float *y) {
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * dim;
        float ss = 0.0f;
        for (int i = 0; i < dim; ++i) {
            float t = xr[i] * xr[i];
            ss = ss + t;
        }
        float inv = 1.0f / sqrtf(ss / (float)dim + eps);
        for (int i = 0; i < dim; ++i) {
            float t = xr[i] * inv;
            y[(size_t)r * dim + i] = t * w[i];
        }
    }
}

/* RoPE angle table.  rope.wgsl:18-35 defines freq_i = pos * theta^(-2i/hd)
 * and rotates with cos/sin(freq_i); the reference evaluates it in f32 with the
 * driver's pow/cos/sin, which WGSL leaves implementation-defined.  Here the
 * same formula is evaluated in f64 and rounded once to f32 (the value the f32
 * formula approximates).  Layout [pos][hd/2]. */
OR_API void or_rope_table(int max_pos, int head_dim, float theta, float *cos_t, float *sin_t) {
    int half = head_dim / 2;
    for (int p = 0; p < max_pos; ++p) {
        for (int i = 0; i < half; ++i) {
            double inv = pow((double)theta, -2.0 * (double)i / (double)head_dim);
            double f = (double)p * inv;
            cos_t[(size_t)p * half + i] = (float)cos(f);
            sin_t[(size_t)p * half + i] = (float)sin(f);
        }
    }
}

/* rope.wgsl:18-35 with the table: y[i] = x[i]c - x[i+h]s,
 * y[i+h] = x[i+h]c + x[i]s for every row (head) at one position. */
OR_API void or_rope(const float *x, int rows, int head_dim, int pos, const float *cos_t,
                    const float *sin_t, float *y) {
    int half = head_dim / 2;
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * head_dim;
        float *yr = y + (size_t)r * head_dim;
        for (int i = 0; i < half; ++i) {
            float c = cos_t[(size_t)pos * half + i];
            float s = sin_t[(size_t)pos * half + i];
            float lo = xr[i], hi = xr[i + half];
            float a = lo * c, b = hi * s;
            float e = hi * c, f = lo * s;
            yr[i] = a - b;
            yr[i + half] = e + f;
        }
    }
}

/* rope.wgsl:18-35 literally, in f32: exponent = -2i/hd, freq = pos *
 * pow(theta, exponent), cos/sin of the f32 freq.  Used only to bound the gap
 * between the f32 formula and the table. */
OR_API void or_rope_f32_literal(const float *x, int rows, int head_dim, int pos, float theta,
                                float *y) {
    int half = head_dim / 2;
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * head_dim;
        float *yr = y + (size_t)r * head_dim;
        for (int i = 0; i < half; ++i) {
            float exponent = -2.0f * (float)i / (float)head_dim;
            float freq = (float)pos * powf(theta, exponent);
            float c = cosf(freq), s = sinf(freq);
            float lo = xr[i], hi = xr[i + half];
            yr[i] = lo * c - hi * s;
            yr[i + half] = hi * c + lo * s;
        }
    }
}

/* glu.wgsl:15-26: silu(g)*u with silu(x) = x/(1+exp(-x)). */
OR_API void or_swiglu(const float *g, const float *u, int n, float *out) {
    for (int i = 0; i < n; ++i) {
        float s = g[i] / (1.0f + expf(-g[i]));
        out[i] = s * u[i];
    }
}

/* ewise.wgsl:9-13: C = A + B. */
OR_API void or_add(const float *a, const float *b, int n, float *c) {
    for (int i = 0; i < n; ++i) c[i] = a[i] + b[i];
}

/* argmax.wgsl:18-55: best starts at (-3.402823e38, 0); strict '>' keeps the
 * lowest index among equal maxima; NaN never wins. */
OR_API uint32_t or_argmax(const float *logits, int n) {
    float best = -3.402823e38f;
    uint32_t bi = 0;
    for (int i = 0; i < n; ++i) {
        if (logits[i] > best) {
            best = logits[i];
            bi = (uint32_t)i;
        }
    }
    return bi;
}

/* ------------------------------------------------------------------ */
/* Decode attention                                                    */
/* ------------------------------------------------------------------ */

static inline float kv_at(const void *p, int f16, size_t i) {
    return f16 ? or_f16_to_f32(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}

/* attention.wgsl:23-96.  For each query head h (kv head h/(n_heads/n_kv)):
 * 32 lanes, lane l scans keys j = l, l+32, ... with a private online softmax
 * (m, denom, acc[hd]); then m_all = max m, corr_l = exp(m_l - m_all),
 * inv = 1/sum(denom_l corr_l), o[t] = inv * sum_l acc_l[t] corr_l.  Lanes are
 * merged in ascending order.  K/V are [seq][n_kv*hd] (cache.rs:7-32); kv_f16
 * selects an f16 cache (the reference's cache is f32 only). */
OR_API void or_attention(const float *q, const void *k, const void *v, int kv_f16, int n_heads,
                         int n_kv, int seq, int hd, float *out) {
    const float NEG = -3.402823e38f;
    int hpk = n_heads / n_kv;
    size_t kvstride = (size_t)n_kv * hd;
    float scale = powf((float)hd, -0.5f);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; ++h) {
        int g = h / hpk;
        const float *qh = q + (size_t)h * hd;
        float m[32], den[32];
        float *acc = (float *)calloc((size_t)32 * hd, sizeof(float));
        for (int l = 0; l < 32; ++l) {
            m[l] = NEG;
            den[l] = 0.0f;
            for (int j = l; j < seq; j += 32) {
                size_t kb = (size_t)j * kvstride + (size_t)g * hd;
                float s = 0.0f;
                for (int t = 0; t < hd; ++t) {
                    float p = qh[t] * kv_at(k, kv_f16, kb + t);
                    s = s + p;
                }
                s = s * scale;
                float mn = m[l] > s ? m[l] : s;
                float corr = expf(m[l] - mn);
                float p = expf(s - mn);
                den[l] = den[l] * corr + p;
                for (int t = 0; t < hd; ++t) {
                    float a = acc[l * hd + t] * corr;
                    float b = kv_at(v, kv_f16, kb + t) * p;
                    acc[l * hd + t] = a + b;
                }
                m[l] = mn;
            }
        }
        float m_all = NEG;
        for (int l = 0; l < 32; ++l) m_all = m[l] > m_all ? m[l] : m_all;
        float corr[32], dsum = 0.0f;
        for (int l = 0; l < 32; ++l) {
            corr[l] = expf(m[l] - m_all);
            dsum = dsum + den[l] * corr[l];
        }
        float inv = 1.0f / dsum;
        for (int t = 0; t < hd; ++t) {
            float o = 0.0f;
            for (int l = 0; l < 32; ++l) o = o + acc[l * hd + t] * corr[l];
            out[(size_t)h * hd + t] = o * inv;
        }
        free(acc);
    }
}

/* f64 two-pass softmax attention (truth for or_attention). */
OR_API void or_attention_f64(const float *q, const void *k, const void *v, int kv_f16, int n_heads,
                             int n_kv, int seq, int hd, double *out) {
    int hpk = n_heads / n_kv;
    size_t kvstride = (size_t)n_kv * hd;
    double scale = 1.0 / sqrt((double)hd);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; ++h) {
        int g = h / hpk;
        double *s = (double *)malloc(sizeof(double) * (size_t)seq);
        double mx = -INFINITY;
        for (int j = 0; j < seq; ++j) {
            size_t kb = (size_t)j * kvstride + (size_t)g * hd;
            double a = 0.0;
            for (int t = 0; t < hd; ++t) a += (double)q[(size_t)h * hd + t] * kv_at(k, kv_f16, kb + t);
            s[j] = a * scale;
            if (s[j] > mx) mx = s[j];
        }
        double den = 0.0;
        for (int j = 0; j < seq; ++j) {
            s[j] = exp(s[j] - mx);
            den += s[j];
        }
        for (int t = 0; t < hd; ++t) {
            double o = 0.0;
            for (int j = 0; j < seq; ++j)
                o += s[j] * kv_at(v, kv_f16, (size_t)j * kvstride + (size_t)g * hd + t);
            out[(size_t)h * hd + t] = o / den;
        }
        free(s);
    }
}

/* ------------------------------------------------------------------ */
/* Seeded test data of the reference's `verify` harness                */
/* ------------------------------------------------------------------ */

/* main.rs:253-255: FNV-1a 64 over the tensor name. */
OR_API uint64_t or_fnv_seed(const char *name) {
    uint64_t h = 1469598103934665603ull;
    for (const unsigned char *p = (const unsigned char *)name; *p; ++p)
        h = (h ^ (uint64_t)*p) * 1099511628211ull;
    return h;
}

/* main.rs:257-266: s = seed|1; s = s*6364136223846793005 + 1442695040888963407;
 * value = ((s>>33) as f32 / u32::MAX as f32 - 0.5) * 0.2.  (s>>33) has 31 bits,
 * so every value lies in [-0.1, 0). */
OR_API void or_fill(uint64_t seed, size_t n, float *out) {
    uint64_t s = seed | 1ull;
    for (size_t i = 0; i < n; ++i) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        float v = (float)(s >> 33) / (float)4294967295u;
        v = v - 0.5f;
        out[i] = v * 0.2f;
    }
}

/* ------------------------------------------------------------------ */
/* Qwen3 forward (qwen3.rs:139-191) and the greedy loop (mod.rs:57-125) */
/* ------------------------------------------------------------------ */

enum {
    OR_T_ATTN_NORM = 0, OR_T_Q_NORM, OR_T_K_NORM, OR_T_FFN_NORM,
    OR_T_WQ, OR_T_WK, OR_T_WV, OR_T_WO, OR_T_GATE, OR_T_UP, OR_T_DOWN,
    OR_T_COUNT
};

typedef struct {
    const uint16_t *d;
    const uint8_t *qs;
} or_q4;

typedef struct {
    const float *norm[4];
    or_q4 w[7];
} or_layer;

typedef struct {
    int n_layers, dim, n_heads, n_kv, head_dim, hidden, vocab, max_seq, kv_f16;
    float eps, theta;
    or_layer *layers;
    const float *final_norm;
    const float *embed;
    or_q4 lm_head;
    void *kcache, *vcache; /* [n_layers][max_seq][kv_dim] f32 or f16 */
    float *cos_t, *sin_t;
} or_model;

/* spec = {n_layers, dim, n_heads, n_kv, head_dim, hidden, vocab, max_seq, kv_f16} */
OR_API or_model *or_model_new(const int *spec, float eps, float theta) {
    or_model *m = (or_model *)calloc(1, sizeof(or_model));
    m->n_layers = spec[0];
    m->dim = spec[1];
    m->n_heads = spec[2];
    m->n_kv = spec[3];
    m->head_dim = spec[4];
    m->hidden = spec[5];
    m->vocab = spec[6];
    m->max_seq = spec[7];
    m->kv_f16 = spec[8];
    m->eps = eps;
    m->theta = theta;
    m->layers = (or_layer *)calloc((size_t)m->n_layers, sizeof(or_layer));
    size_t kvn = (size_t)m->n_layers * m->max_seq * m->n_kv * m->head_dim;
    size_t es = m->kv_f16 ? 2 : 4;
    m->kcache = calloc(kvn, es);
    m->vcache = calloc(kvn, es);
    int half = m->head_dim / 2;
    m->cos_t = (float *)malloc(sizeof(float) * (size_t)m->max_seq * half);
    m->sin_t = (float *)malloc(sizeof(float) * (size_t)m->max_seq * half);
    or_rope_table(m->max_seq, m->head_dim, theta, m->cos_t, m->sin_t);
    return m;
}

OR_API void or_model_free(or_model *m) {
    if (!m) return;
    free(m->layers);
    free(m->kcache);
    free(m->vcache);
    free(m->cos_t);
    free(m->sin_t);
    free(m);
}

/* Norm gains (ids 0..3) take p0 = float*; projections (ids 4..10) take
 * p0 = f16 scales, p1 = GGUF quant bytes.  Arrays are borrowed, not copied. */
OR_API void or_model_set(or_model *m, int layer, int id, const void *p0, const void *p1) {
    or_layer *l = &m->layers[layer];
    if (id < OR_T_WQ) {
        l->norm[id] = (const float *)p0;
    } else {
        l->w[id - OR_T_WQ].d = (const uint16_t *)p0;
        l->w[id - OR_T_WQ].qs = (const uint8_t *)p1;
    }
}

OR_API void or_model_set_globals(or_model *m, const float *embed, const float *final_norm,
                                 const uint16_t *lm_d, const uint8_t *lm_qs) {
    m->embed = embed;
    m->final_norm = final_norm;
    m->lm_head.d = lm_d;
    m->lm_head.qs = lm_qs;
}

/* Fill positions [0, n_pos) of every layer's cache (layout [layer][pos][kv_dim],
 * in the cache dtype's element bytes). */
OR_API void or_model_prefill_kv(or_model *m, const void *k, const void *v, int n_pos) {
    size_t es = m->kv_f16 ? 2 : 4;
    size_t kv_dim = (size_t)m->n_kv * m->head_dim;
    for (int l = 0; l < m->n_layers; ++l) {
        size_t dst = (size_t)l * m->max_seq * kv_dim * es;
        size_t src = (size_t)l * n_pos * kv_dim * es;
        memcpy((char *)m->kcache + dst, (const char *)k + src, (size_t)n_pos * kv_dim * es);
        memcpy((char *)m->vcache + dst, (const char *)v + src, (size_t)n_pos * kv_dim * es);
    }
}

/* Read row `pos` of layer `layer`'s K and V caches back as f32 (f16 caches
 * widened exactly), kv_dim values each: lets tests see which rows a step
 * wrote (cache.rs:21-24 writes exactly one row per forward). */
OR_API void or_model_kv_row(const or_model *m, int layer, int pos, float *k_out, float *v_out) {
    size_t kv_dim = (size_t)m->n_kv * m->head_dim;
    size_t off = ((size_t)layer * m->max_seq + pos) * kv_dim;
    for (size_t j = 0; j < kv_dim; ++j) {
        if (m->kv_f16) {
            k_out[j] = or_f16_to_f32(((const uint16_t *)m->kcache)[off + j]);
            v_out[j] = or_f16_to_f32(((const uint16_t *)m->vcache)[off + j]);
        } else {
            k_out[j] = ((const float *)m->kcache)[off + j];
            v_out[j] = ((const float *)m->vcache)[off + j];
        }
    }
}

static void gemv(const or_q4 *w, const float *x, int in_f, int out_f, float *y) {
    or_q4_gemv(x, w->d, w->qs, in_f, out_f, y);
}

/* One token: embed (qwen3.rs:128-133), forward (qwen3.rs:139-191), logits
 * (qwen3.rs:135-137).  Writes logits[vocab]; optionally the final hidden
 * state and the per-layer hook taps: "q" after QK-norm and RoPE
 * (qwen3.rs:165), "post_attn" after the attention residual (qwen3.rs:180) and
 * "layer_out" (qwen3.rs:188), each [n_layers][len]. */
OR_API void or_model_step_taps(or_model *m, uint32_t tok, int pos, float *logits,
                               float *hidden_out, float *q_tap, float *post_attn,
                               float *layer_out) {
    int dim = m->dim, hd = m->head_dim, nh = m->n_heads, nkv = m->n_kv;
    int qd = nh * hd, kvd = nkv * hd, hid = m->hidden;
    float *hidden = (float *)malloc(sizeof(float) * dim);
    float *normed = (float *)malloc(sizeof(float) * dim);
    float *q = (float *)malloc(sizeof(float) * qd);
    float *k = (float *)malloc(sizeof(float) * kvd);
    float *v = (float *)malloc(sizeof(float) * kvd);
    float *t = (float *)malloc(sizeof(float) * (qd > kvd ? qd : kvd));
    float *attn = (float *)malloc(sizeof(float) * qd);
    float *tmp = (float *)malloc(sizeof(float) * dim);
    float *gate = (float *)malloc(sizeof(float) * hid);
    float *up = (float *)malloc(sizeof(float) * hid);
    float *act = (float *)malloc(sizeof(float) * hid);
    float *zero = (float *)calloc((size_t)dim, sizeof(float));

    /* clone_buf: x + 0 (qwen3.rs:194-197) */
    or_add(m->embed + (size_t)tok * dim, zero, dim, hidden);
    size_t es = m->kv_f16 ? 2 : 4;
    for (int i = 0; i < m->n_layers; ++i) {
        const or_layer *l = &m->layers[i];
        or_rmsnorm(hidden, l->norm[OR_T_ATTN_NORM], 1, dim, m->eps, normed);
        gemv(&l->w[OR_T_WQ - OR_T_WQ], normed, dim, qd, q);
        gemv(&l->w[OR_T_WK - OR_T_WQ], normed, dim, kvd, k);
        gemv(&l->w[OR_T_WV - OR_T_WQ], normed, dim, kvd, v);
        or_rmsnorm(q, l->norm[OR_T_Q_NORM], nh, hd, m->eps, t);
        or_rope(t, nh, hd, pos, m->cos_t, m->sin_t, q);
        or_rmsnorm(k, l->norm[OR_T_K_NORM], nkv, hd, m->eps, t);
        or_rope(t, nkv, hd, pos, m->cos_t, m->sin_t, k);
        if (q_tap) memcpy(q_tap + (size_t)i * qd, q, sizeof(float) * qd);
        /* cache.write (cache.rs:21-24) */
        size_t off = ((size_t)i * m->max_seq + pos) * kvd;
        if (m->kv_f16) {
            for (int j = 0; j < kvd; ++j) {
                ((uint16_t *)m->kcache)[off + j] = or_f32_to_f16(k[j]);
                ((uint16_t *)m->vcache)[off + j] = or_f32_to_f16(v[j]);
            }
        } else {
            memcpy((float *)m->kcache + off, k, sizeof(float) * kvd);
            memcpy((float *)m->vcache + off, v, sizeof(float) * kvd);
        }
        const char *kl = (const char *)m->kcache + (size_t)i * m->max_seq * kvd * es;
        const char *vl = (const char *)m->vcache + (size_t)i * m->max_seq * kvd * es;
        or_attention(q, kl, vl, m->kv_f16, nh, nkv, pos + 1, hd, attn);
        gemv(&l->w[OR_T_WO - OR_T_WQ], attn, qd, dim, tmp);
        or_add(hidden, tmp, dim, hidden);
        if (post_attn) memcpy(post_attn + (size_t)i * dim, hidden, sizeof(float) * dim);
        or_rmsnorm(hidden, l->norm[OR_T_FFN_NORM], 1, dim, m->eps, normed);
        gemv(&l->w[OR_T_GATE - OR_T_WQ], normed, dim, hid, gate);
        gemv(&l->w[OR_T_UP - OR_T_WQ], normed, dim, hid, up);
        or_swiglu(gate, up, hid, act);
        gemv(&l->w[OR_T_DOWN - OR_T_WQ], act, hid, dim, tmp);
        or_add(hidden, tmp, dim, hidden);
        if (layer_out) memcpy(layer_out + (size_t)i * dim, hidden, sizeof(float) * dim);
    }
    or_rmsnorm(hidden, m->final_norm, 1, dim, m->eps, normed);
    if (hidden_out) memcpy(hidden_out, normed, sizeof(float) * dim);
    if (logits) gemv(&m->lm_head, normed, dim, m->vocab, logits);
    free(hidden); free(normed); free(q); free(k); free(v); free(t); free(attn);
    free(tmp); free(gate); free(up); free(act); free(zero);
}

OR_API void or_model_step(or_model *m, uint32_t tok, int pos, float *logits, float *hidden_out,
                          float *layer_out) {
    or_model_step_taps(m, tok, pos, logits, hidden_out, NULL, NULL, layer_out);
}

/* mod.rs:57-125: greedy loop.  Position pos feeds prompt[pos] while inside
 * the prompt, then the previous argmax; every step computes logits and the
 * argmax (prompt logits are discarded); stops after max_new tokens, i.e.
 * after P+N-1 forwards.  start_pos lets the loop begin after a pre-filled
 * cache (the prompt's first token is fed at start_pos).  Returns the number
 * of produced tokens; margins[i] (optional) = top1 - top2 logit. */
OR_API int or_generate(or_model *m, const uint32_t *prompt, int n_prompt, int max_new,
                       int start_pos, uint32_t *out_tokens, float *margins) {
    float *logits = (float *)malloc(sizeof(float) * m->vocab);
    int produced = 0;
    uint32_t next = prompt[0];
    int total = n_prompt + max_new;
    for (int p = 0; p < total; ++p) {
        or_model_step(m, next, start_pos + p, logits, NULL, NULL);
        uint32_t tok = or_argmax(logits, m->vocab);
        if (p + 1 < n_prompt) {
            next = prompt[p + 1];
        } else {
            if (margins) {
                float b1 = -INFINITY, b2 = -INFINITY;
                for (int i = 0; i < m->vocab; ++i) {
                    float x = logits[i];
                    if (x > b1) { b2 = b1; b1 = x; } else if (x > b2) { b2 = x; }
                }
                margins[produced] = b1 - b2;
            }
            out_tokens[produced++] = tok;
            next = tok;
            if (produced >= max_new) break;
        }
    }
    free(logits);
    return produced;
}
