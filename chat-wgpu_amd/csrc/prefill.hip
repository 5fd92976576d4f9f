// Batched prefill for gfx950: M prompt positions through one layer at a time.
//
// The reference has no batched path: its prompt phase is the per-token loop
// (model::generate runs P forwards, src/model/mod.rs:57-125; each forward is
// Qwen3::forward, src/model/qwen3.rs:139-191).  This file computes the same
// forward for M positions at once, with the linear layers as Q4_0
// dequant-GEMMs on the matrix cores and causal attention as MFMA tiles.
//
// Precision.  The GEMM and attention must match the f32 per-token path, so no
// operand is rounded below what the reference computes with:
//  * Q4_0 weights enter the MFMA as the exact integers q-8 (bf16 holds them
//    exactly); the block scale d multiplies each 32-wide block's partial sum
//    in f32 (acc += d * (x . (q-8)), the shader's own order, q4.wgsl:25-82).
//  * f32 activations are split x = hi + lo with hi = bf16(x) and
//    lo = bf16(x - hi) (16 significant bits); each block is two MFMAs, hi
//    and lo, into the same f32 partial.
//  * Attention: K and V are f16 in the cache and enter f16 MFMAs exactly; q
//    and the softmax weights p are split into f16 hi + lo the same way.
//
// MFMA v_mfma_f32_16x16x32_{bf16,f16}: lane l holds A[l % 16][8 (l / 16) + j]
// and B[8 (l / 16) + j][l % 16] (j = 0..7) and receives D[4 (l / 16) + r][l % 16]
// (r = 0..3); any k order shared by A and B is valid.

#include <cmath>

#include "cw_internal.hpp"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kT = 256;  // threads per workgroup (4 waves)

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// f32 -> bf16 bits, round to nearest even (finite inputs)
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ float bf16_val(uint32_t h) { return __builtin_bit_cast(float, h << 16); }

// ---------------------------------------------------------------------------
// Rows -> bf16 hi/lo (optionally RMS-normalised first, norm.wgsl:20-42).
// One workgroup per row.
template <bool NORM>
__global__ __launch_bounds__(kT) void split_rows_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ w, float eps,
                                                        int K, uint16_t *__restrict__ hi,
                                                        uint16_t *__restrict__ lo) {
    __shared__ float red[kT / 64];
    const size_t base = (size_t)blockIdx.x * K;
    const int tid = threadIdx.x;
    float inv = 1.0f;
    if constexpr (NORM) {
        float ss = 0.0f;
        for (int i = tid; i < K; i += kT) {
            const float v = x[base + i];
            ss += v * v;
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        ss = (red[0] + red[1]) + (red[2] + red[3]);
        inv = 1.0f / sqrtf(ss / (float)K + eps);
    }
    for (int i = tid; i < K; i += kT) {
        float v = x[base + i];
        if constexpr (NORM) v = (v * inv) * w[i];
        const uint32_t h = bf16_bits(v);
        hi[base + i] = (uint16_t)h;
        lo[base + i] = (uint16_t)bf16_bits(v - bf16_val(h));
    }
}

// ---------------------------------------------------------------------------
// Q4_0 dequant-GEMM: y[M][N] = x[M][K] . W[N][K]^T (W split GGUF Q4_0).
//
// Workgroup tile 128 (rows of x) x 64 (rows of W), four waves of 64 x 32
// (4 x 2 MFMA tiles of 16 x 16).  Per 32-wide Q4 block the workgroup stages
// in LDS, double-buffered: the x tile as bf16 hi and lo, and the W tile
// dequantized once to bf16 (q - 8) with its f32 block scales.  While the
// waves run the block's MFMAs from one buffer, the next block's global loads
// are in flight into registers; they are written (and W dequantized) into the
// other buffer, then one barrier.  LDS rows are padded by 16 B so the 16 lanes
// of a fragment read hit 16 disjoint bank quads.
constexpr int kBM = 128, kBN = 64;
constexpr int kRowB = 64 + 16;  // bytes per LDS row: 32 bf16 + pad
constexpr int kStageA = kBM * kRowB;          // one of x hi / x lo
constexpr int kStageB = kBN * kRowB;          // W (q - 8)
constexpr int kStage = 2 * kStageA + kStageB; // + scales (f32) after

__device__ __forceinline__ float f16_bits_val(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// 8 nibbles (low or high halves of 8 quant bytes) -> bf16 (q - 8), exact
__device__ __forceinline__ uint4 dequant8(uint2 q, bool high) {
    uint32_t w0 = q.x, w1 = q.y;
    if (high) {
        w0 >>= 4;
        w1 >>= 4;
    }
    uint32_t p[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t w = h ? w1 : w0;
        const float f0 = (float)(int)(w & 15u) - 8.0f;
        const float f1 = (float)(int)((w >> 8) & 15u) - 8.0f;
        const float f2 = (float)(int)((w >> 16) & 15u) - 8.0f;
        const float f3 = (float)(int)((w >> 24) & 15u) - 8.0f;
        // small integers: the bf16 is the f32's high half, exactly
        p[2 * h] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1),
                                         __builtin_bit_cast(uint32_t, f0), 0x07060302u);
        p[2 * h + 1] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f3),
                                             __builtin_bit_cast(uint32_t, f2), 0x07060302u);
    }
    return make_uint4(p[0], p[1], p[2], p[3]);
}

// Global loads of one block into registers: thread t brings 4 x 16 B of x
// (hi rows t/2.., lo) and, for t < NM * 64, the 16 quant bytes and the scale
// of one W row.
template <int NM>
struct Stage {
    uint4 x[4];
    uint4 q;
    uint32_t d;
};

template <int NM>
__device__ __forceinline__ void stage_load(const cwi::GemmArgs &a, int nb, int b, int m0, int n0,
                                           int tid, Stage<NM> &st) {
    const int bc = b < nb ? b : nb - 1;
    // x: 128 rows x 64 B (hi) + 128 x 64 B (lo) = 1024 units of 16 B
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int f = tid + u * kT;             // 0..1023
        const int half = f >> 9;                // 0: hi, 1: lo
        const int row = (f >> 2) & (kBM - 1), c = f & 3;
        const int m = min(m0 + row, a.M - 1);
        const uint16_t *src = half ? a.xlo : a.xhi;
        st.x[u] = *reinterpret_cast<const uint4 *>(src + (size_t)m * a.K + (size_t)bc * 32 + c * 8);
    }
    if (tid < NM * kBN) {
        const int w = tid >> 6, col = tid & (kBN - 1);
        const int n = min(n0 + col, a.N - 1);
        const uint8_t *q = w ? a.qB : a.qA;
        const uint16_t *s = w ? a.sB : a.sA;
        const size_t blk = (size_t)n * nb + bc;
        st.q = *reinterpret_cast<const uint4 *>(q + blk * 16);
        st.d = s[blk];
    }
}

template <int NM>
__device__ __forceinline__ void stage_store(const Stage<NM> &st, unsigned char *buf, int tid) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int f = tid + u * kT;
        const int half = f >> 9;
        const int row = (f >> 2) & (kBM - 1), c = f & 3;
        *reinterpret_cast<uint4 *>(buf + half * kStageA + row * kRowB + c * 16) = st.x[u];
    }
    if (tid < NM * kBN) {
        const int w = tid >> 6, col = tid & (kBN - 1);
        unsigned char *wb = buf + 2 * kStageA + w * (kStageB + kBN * 4);
        // elements 0..15: low nibbles of bytes 0..15; 16..31: high nibbles
        const uint2 lo8 = make_uint2(st.q.x, st.q.y), hi8 = make_uint2(st.q.z, st.q.w);
        *reinterpret_cast<uint4 *>(wb + col * kRowB + 0) = dequant8(lo8, false);
        *reinterpret_cast<uint4 *>(wb + col * kRowB + 16) = dequant8(hi8, false);
        *reinterpret_cast<uint4 *>(wb + col * kRowB + 32) = dequant8(lo8, true);
        *reinterpret_cast<uint4 *>(wb + col * kRowB + 48) = dequant8(hi8, true);
        reinterpret_cast<float *>(wb + kStageB)[col] = f16_bits_val(st.d);
    }
}

template <int EPI>
__global__ __launch_bounds__(kT) void q4_gemm_kernel(cwi::GemmArgs a) {
    constexpr int NM = EPI == cwi::EPI_SWIGLU ? 2 : 1;  // weight matrices
    constexpr int kBuf = 2 * kStageA + NM * (kStageB + kBN * 4);
    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kBuf];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, lg = lane >> 4;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 32;  // wave tile within the block tile
    const int nb = a.K >> 5;

    f32x4 acc[NM][4][2];
#pragma unroll
    for (int w = 0; w < NM; ++w)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) acc[w][mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

    Stage<NM> st;
    stage_load<NM>(a, nb, 0, m0, n0, tid, st);
    stage_store<NM>(st, lds, tid);
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
        const unsigned char *cur = lds + (b & 1) * kBuf;
        stage_load<NM>(a, nb, b + 1, m0, n0, tid, st);  // past the end: a clamped re-load
        // fragments: A rows wr + 16 mi + li, k 8 lg..; B columns wc + 16 ni + li
        bf16x8 A[4][2];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            const int row = wr + 16 * mi + li;
            A[mi][0] = *reinterpret_cast<const bf16x8 *>(cur + row * kRowB + lg * 16);
            A[mi][1] = *reinterpret_cast<const bf16x8 *>(cur + kStageA + row * kRowB + lg * 16);
        }
#pragma unroll
        for (int w = 0; w < NM; ++w) {
            const unsigned char *wb = cur + 2 * kStageA + w * (kStageB + kBN * 4);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const int col = wc + 16 * ni + li;
                const bf16x8 B = *reinterpret_cast<const bf16x8 *>(wb + col * kRowB + lg * 16);
                const float d = reinterpret_cast<const float *>(wb + kStageB)[col];
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) {
                    f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
                    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mi][0], B, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mi][1], B, t, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[w][mi][ni][r] = __builtin_fmaf(d, t[r], acc[w][mi][ni][r]);
                }
            }
        }
        stage_store<NM>(st, lds + ((b + 1) & 1) * kBuf, tid);
        __syncthreads();
    }

    // lane holds rows 4 lg + r of each row tile, column li of each column tile
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int n = n0 + wc + ni * 16 + li;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wr + mi * 16 + 4 * lg + r;
                if (m < a.M && n < a.N) {
                    const size_t o = (size_t)m * a.N + n;
                    const float v = acc[0][mi][ni][r];
                    if constexpr (EPI == cwi::EPI_STORE) {
                        a.y[o] = v;
                    } else if constexpr (EPI == cwi::EPI_ADD) {
                        a.y[o] = a.resid[o] + v;
                    } else {
                        const float up = acc[NM - 1][mi][ni][r];
                        a.y[o] = v / (1.0f + expf(-v)) * up;
                    }
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Per position: per-head QK RMSNorm (qwen3.rs:154-155) and NeoX RoPE
// (rope.wgsl:18-35) on the raw q|k|v rows of the QKV GEMM, q out as f32
// [M][n_heads][hd], k and v written into the cache rows start..start+M-1
// (cache.rs:21-24).  One workgroup per position, one wave per head (looped).
template <typename KVT>
__global__ __launch_bounds__(kT) void qk_rope_kv_kernel(const float *__restrict__ qkv,
                                                        const float *__restrict__ qn,
                                                        const float *__restrict__ kn, float eps,
                                                        const float *__restrict__ cos_t,
                                                        const float *__restrict__ sin_t,
                                                        int n_heads, int n_kv, int start,
                                                        float *__restrict__ q_out,
                                                        KVT *__restrict__ kc,
                                                        KVT *__restrict__ vc) {
    constexpr int HD = 128, HALF = 64;
    const int i = blockIdx.x, pos = start + i;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q_dim = n_heads * HD, kv_dim = n_kv * HD;
    const float *row = qkv + (size_t)i * (q_dim + 2 * kv_dim);
    const float c = cos_t[(size_t)pos * HALF + lane], s = sin_t[(size_t)pos * HALF + lane];
    for (int h = wave; h < n_heads + n_kv; h += kT / 64) {
        const bool isq = h < n_heads;
        const float *src = isq ? row + (size_t)h * HD : row + q_dim + (size_t)(h - n_heads) * HD;
        const float *g = isq ? qn : kn;
        const float lo = src[lane], hi = src[lane + HALF];
        const float ss = wave_sum(lo * lo + hi * hi);
        const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
        const float l0 = (lo * inv) * g[lane], h0 = (hi * inv) * g[lane + HALF];
        const float r0 = l0 * c - h0 * s, r1 = h0 * c + l0 * s;
        if (isq) {
            float *dst = q_out + ((size_t)i * n_heads + h) * HD;
            dst[lane] = r0;
            dst[lane + HALF] = r1;
        } else {
            const int g2 = h - n_heads;
            KVT *kd = kc + (size_t)pos * kv_dim + (size_t)g2 * HD;
            kd[lane] = (KVT)r0;
            kd[lane + HALF] = (KVT)r1;
            const float *vs = row + q_dim + kv_dim + (size_t)g2 * HD;
            KVT *vd = vc + (size_t)pos * kv_dim + (size_t)g2 * HD;
            vd[lane] = (KVT)vs[lane];
            vd[lane + HALF] = (KVT)vs[lane + HALF];
        }
    }
}

// ---------------------------------------------------------------------------
// Causal attention (attention.wgsl:23-96 for each query position) on f16
// caches, flash style: workgroup = one query head x 64 positions, one wave
// per 16 positions.  Per 64-key tile: K rows and V^T staged in LDS;
// S = q K^T by MFMA (q split into f16 hi/lo), online max / sum per row,
// P (f16 hi/lo) through LDS into A layout, O += P V by MFMA.
constexpr int kAttQ = 64;   // positions per workgroup
constexpr int kAttK = 64;   // keys per tile
constexpr int kKRow = 128 + 8;  // K tile row stride (f16), padded
constexpr int kVRow = kAttK + 8; // V^T tile row stride (f16), padded

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)a);
    const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)b);
    return lo | (hi << 16);
}

__global__ __launch_bounds__(kT) void attn_prefill_kernel(const float *__restrict__ q,
                                                          const _Float16 *__restrict__ kc,
                                                          const _Float16 *__restrict__ vc,
                                                          int M, int n_heads, int n_kv, int start,
                                                          float scale, float *__restrict__ out) {
    constexpr int HD = 128;
    __shared__ _Float16 Ks[kAttK * kKRow];
    __shared__ _Float16 Vt[HD * kVRow];
    __shared__ float Ps[4][16 * kAttK];
    const int h = blockIdx.x, q0 = blockIdx.y * kAttQ;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, lg = lane >> 4;
    const int g = h / (n_heads / n_kv);
    const int kv_dim = n_kv * HD;
    const int wq = q0 + wave * 16;  // this wave's first position (row of q)

    // q operands: row li of the wave's 16, dims 8 lg + 32 ks .. +8, hi and lo
    f16x8 qa[4][2];
    {
        const int qi = min(wq + li, M - 1);
        const float *qr = q + ((size_t)qi * n_heads + h) * HD;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const float4 v0 = *reinterpret_cast<const float4 *>(qr + 32 * ks + 8 * lg);
            const float4 v1 = *reinterpret_cast<const float4 *>(qr + 32 * ks + 8 * lg + 4);
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            uint32_t ph[4], pl[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const _Float16 a0 = (_Float16)v[2 * j], a1 = (_Float16)v[2 * j + 1];
                ph[j] = (uint32_t)__builtin_bit_cast(uint16_t, a0) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, a1) << 16);
                pl[j] = pack_f16x2(v[2 * j] - (float)a0, v[2 * j + 1] - (float)a1);
            }
            qa[ks][0] = __builtin_bit_cast(f16x8, make_uint4(ph[0], ph[1], ph[2], ph[3]));
            qa[ks][1] = __builtin_bit_cast(f16x8, make_uint4(pl[0], pl[1], pl[2], pl[3]));
        }
    }

    // rows of this lane in the C layout: 4 lg + r of the wave's 16
    float mrow[4], lrow[4];
    f32x4 o[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        mrow[r] = -INFINITY;
        lrow[r] = 0.0f;
    }
#pragma unroll
    for (int ni = 0; ni < 8; ++ni) o[ni] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int last_pos = start + min(q0 + kAttQ, M) - 1;  // last key any row needs
    const int n_tiles = last_pos / kAttK + 1;
    for (int t = 0; t < n_tiles; ++t) {
        const int k0 = t * kAttK;
        __syncthreads();  // previous tile's LDS reads are done
        // stage K rows and V^T: 64 keys x 128 dims, 16 B per load (4 per thread)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int f = tid + u * kT;  // 0..1023
            const int key = f >> 4, c8 = (f & 15) * 8;
            const int p = min(k0 + key, last_pos);
            const uint4 kv = *reinterpret_cast<const uint4 *>(kc + (size_t)p * kv_dim + g * HD + c8);
            *reinterpret_cast<uint4 *>(&Ks[key * kKRow + c8]) = kv;
            const uint4 vv = *reinterpret_cast<const uint4 *>(vc + (size_t)p * kv_dim + g * HD + c8);
            const _Float16 *ve = reinterpret_cast<const _Float16 *>(&vv);
#pragma unroll
            for (int j = 0; j < 8; ++j) Vt[(c8 + j) * kVRow + key] = ve[j];
        }
        __syncthreads();

        // S (16 rows x 64 keys): 4 key tiles of 16, K = 128 dims in 4 steps
        f32x4 sc[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const f16x8 kb = *reinterpret_cast<const f16x8 *>(
                    &Ks[(ni * 16 + li) * kKRow + 32 * ks + 8 * lg]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[ks][0], kb, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[ks][1], kb, acc, 0, 0, 0);
            }
            sc[ni] = acc;
        }
        // mask (causal, and rows past M), scale, online softmax per row
        float pm[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row_pos = start + wq + 4 * lg + r;
            float mx = -INFINITY;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int key = k0 + ni * 16 + li;
                const float v = key <= row_pos ? sc[ni][r] * scale : -INFINITY;
                pm[ni][r] = v;
                mx = fmaxf(mx, v);
            }
            // max over the 16 lanes that share this row (same lg)
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
            const float mnew = fmaxf(mrow[r], mx);
            // a row with no key yet in this tile keeps mnew = -inf: guard the rescale
            const float alpha = mnew == -INFINITY ? 1.0f : expf(mrow[r] - mnew);
            float ls = 0.0f;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const float p = pm[ni][r] == -INFINITY ? 0.0f : expf(pm[ni][r] - mnew);
                pm[ni][r] = p;
                ls += p;
            }
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) ls += __shfl_xor(ls, off);
            lrow[r] = lrow[r] * alpha + ls;
            mrow[r] = mnew;
#pragma unroll
            for (int ni = 0; ni < 8; ++ni) o[ni][r] *= alpha;
        }
        // P to LDS (row-major 16 x 64), back in A layout as f16 hi/lo
        float *P = Ps[wave];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r) P[(4 * lg + r) * kAttK + ni * 16 + li] = pm[ni][r];
        // (a wave's LDS accesses complete in order: its reads below see these writes)
        f16x8 pa[2][2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const float *pr = P + li * kAttK + 32 * kk + 8 * lg;
            uint32_t ph[4], pl[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float v0 = pr[2 * j], v1 = pr[2 * j + 1];
                const _Float16 a0 = (_Float16)v0, a1 = (_Float16)v1;
                ph[j] = (uint32_t)__builtin_bit_cast(uint16_t, a0) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, a1) << 16);
                pl[j] = pack_f16x2(v0 - (float)a0, v1 - (float)a1);
            }
            pa[kk][0] = __builtin_bit_cast(f16x8, make_uint4(ph[0], ph[1], ph[2], ph[3]));
            pa[kk][1] = __builtin_bit_cast(f16x8, make_uint4(pl[0], pl[1], pl[2], pl[3]));
        }
        // O (16 rows x 128 dims) += P (16 x 64 keys) V (64 keys x 128 dims)
#pragma unroll
        for (int ni = 0; ni < 8; ++ni) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const f16x8 vb = *reinterpret_cast<const f16x8 *>(
                    &Vt[(ni * 16 + li) * kVRow + 32 * kk + 8 * lg]);
                o[ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[kk][0], vb, o[ni], 0, 0, 0);
                o[ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[kk][1], vb, o[ni], 0, 0, 0);
            }
        }
    }
    // normalise and store: lane holds rows 4 lg + r, dims ni * 16 + li
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int qi = wq + 4 * lg + r;
        if (qi < M) {
            const float inv = 1.0f / lrow[r];
            float *dst = out + (size_t)qi * n_heads * HD + (size_t)h * HD;
#pragma unroll
            for (int ni = 0; ni < 8; ++ni) dst[ni * 16 + li] = o[ni][r] * inv;
        }
    }
}

// Embedding rows of n tokens (Qwen3::embed, qwen3.rs:128-133): one workgroup
// per position.
__global__ __launch_bounds__(kT) void embed_rows_kernel(const float *__restrict__ table, int dim,
                                                        const uint32_t *__restrict__ tok,
                                                        float *__restrict__ out) {
    const size_t src = (size_t)tok[blockIdx.x] * dim, dst = (size_t)blockIdx.x * dim;
    for (int i = threadIdx.x; i < dim; i += kT) out[dst + i] = table[src + i];
}

}  // namespace

namespace cwi {

int launch_embed_rows(cw_ctx *ctx, const float *table, int dim, const uint32_t *tok_dev, int n,
                      float *out) {
    return launch(ctx, "prefill_embed", embed_rows_kernel, dim3(n), dim3(kT), 0, table, dim,
                  tok_dev, out);
}

int launch_split_rows(cw_ctx *ctx, const float *x, const float *norm_w, float eps, int rows, int K,
                      uint16_t *hi, uint16_t *lo) {
    if (norm_w)
        return launch(ctx, "prefill_split_rmsnorm", split_rows_kernel<true>, dim3(rows), dim3(kT),
                      0, x, norm_w, eps, K, hi, lo);
    return launch(ctx, "prefill_split", split_rows_kernel<false>, dim3(rows), dim3(kT), 0, x,
                  norm_w, eps, K, hi, lo);
}

int launch_q4_gemm(cw_ctx *ctx, Epi epi, const GemmArgs &a) {
    const dim3 grid((a.N + kBN - 1) / kBN, (a.M + kBM - 1) / kBM);
    switch (epi) {
        case EPI_STORE:
            return launch(ctx, "q4_gemm", q4_gemm_kernel<EPI_STORE>, grid, dim3(kT), 0, a);
        case EPI_ADD:
            return launch(ctx, "q4_gemm_add", q4_gemm_kernel<EPI_ADD>, grid, dim3(kT), 0, a);
        default:
            return launch(ctx, "q4_gemm_swiglu", q4_gemm_kernel<EPI_SWIGLU>, grid, dim3(kT), 0, a);
    }
}

int launch_qk_rope_kv(cw_ctx *ctx, const float *qkv, const float *qn, const float *kn, float eps,
                      const float *cos_t, const float *sin_t, int M, int n_heads, int n_kv,
                      int start, int kv_dtype, float *q_out, void *kc, void *vc) {
    if (kv_dtype == CW_F16)
        return launch(ctx, "prefill_qk_rope_kv", qk_rope_kv_kernel<_Float16>, dim3(M), dim3(kT), 0,
                      qkv, qn, kn, eps, cos_t, sin_t, n_heads, n_kv, start, q_out, (_Float16 *)kc,
                      (_Float16 *)vc);
    return launch(ctx, "prefill_qk_rope_kv", qk_rope_kv_kernel<float>, dim3(M), dim3(kT), 0, qkv,
                  qn, kn, eps, cos_t, sin_t, n_heads, n_kv, start, q_out, (float *)kc, (float *)vc);
}

int launch_attn_prefill(cw_ctx *ctx, const float *q, const void *kc, const void *vc, int M,
                        int n_heads, int n_kv, int start, float *out) {
    const float scale = 1.0f / sqrtf(128.0f);
    return launch(ctx, "prefill_attention", attn_prefill_kernel,
                  dim3(n_heads, (M + kAttQ - 1) / kAttQ), dim3(kT), 0, q,
                  (const _Float16 *)kc, (const _Float16 *)vc, M, n_heads, n_kv, start, scale, out);
}

}  // namespace cwi

using namespace cwi;

extern "C" int cw_q4_gemm(cw_ctx *ctx, const float *x, int m, const uint16_t *scales,
                          const uint8_t *quants, int in_f, int out_f, float *y) {
    CW_CHECK_ARG(ctx && x && scales && quants && y, "cw_q4_gemm: null argument");
    CW_CHECK_ARG(m > 0 && m <= 65536, "cw_q4_gemm: m=%d outside [1, 65536]", m);
    CW_CHECK_ARG(in_f > 0 && in_f % 32 == 0, "cw_q4_gemm: in_f=%d must be a positive multiple of 32",
                 in_f);
    CW_CHECK_ARG(out_f > 0, "cw_q4_gemm: out_f=%d must be positive", out_f);
    CW_CHECK_ARG(((uintptr_t)quants & 15) == 0 && ((uintptr_t)scales & 1) == 0,
                 "cw_q4_gemm: quants must be 16-byte and scales 2-byte aligned");
    void *scratch = nullptr;
    const size_t n = (size_t)m * in_f;
    CW_TRY(ctx_scratch(ctx, n * 4, &scratch));
    uint16_t *hi = (uint16_t *)scratch, *lo = hi + n;
    CW_TRY(launch_split_rows(ctx, x, nullptr, 0.0f, m, in_f, hi, lo));
    GemmArgs a{};
    a.xhi = hi;
    a.xlo = lo;
    a.sA = scales;
    a.qA = quants;
    a.y = y;
    a.M = m;
    a.N = out_f;
    a.K = in_f;
    return launch_q4_gemm(ctx, EPI_STORE, a);
}
