// Single-query GQA decode attention for gfx950.
//
// Replaces attention::attention (src/kernels/attention.rs:7-38,
// attention.wgsl:23-96).  Same mathematics: o_h = sum_j softmax_j(scale *
// q_h . k_j) v_j over j < seq, kv head = h / (n_heads / n_kv), scale =
// hd^-0.5, online (max-rescaled) softmax.
//
// Split over the sequence (flash-decoding): workgroup (chunk c, kv head g)
// covers 128 positions with 4 waves of 32.  Every kv head's K/V rows are
// read once for all its GQA query heads.  A wave reads 4 positions per step,
// 16 lanes per row (coalesced 16-byte loads of a position's head slice),
// reduces q.k within each 16-lane row with DPP, keeps a per-wave
// (max, sum, acc) and the 4 waves merge through LDS.  A second kernel merges
// the chunk partials.
//
// Fused prologue (decode step): the raw q/k/v come straight from the fused
// QKV projection; the kernel applies the per-head QK RMSNorm (norm.wgsl,
// qwen3.rs:154-155) and RoPE (rope.wgsl) and the workgroup whose chunk holds
// the new position writes k/v into the cache (cache.rs:21-24), substituting
// the new row from LDS for its own use.

#include <cmath>

#include "cw_internal.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 128;  // positions per workgroup
constexpr int kPerWave = 32;
constexpr int kSteps = kPerWave / 4;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float sum16(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

template <typename T>
__device__ __forceinline__ float kv_f(T v) {
    return (float)v;
}

template <typename T>
__device__ __forceinline__ T to_kv(float v) {
    return (T)v;  // f32 -> f16 rounds to nearest even
}

template <typename T, int N>
struct alignas((sizeof(T) * N) >= 16 ? 16 : (sizeof(T) * N)) Vec {
    T v[N];
};

template <typename T, int N>
__device__ __forceinline__ Vec<T, N> load_vec(const T *p) {
    return *reinterpret_cast<const Vec<T, N> *>(p);
}

template <typename KVT, int HD, int HPK>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(cwi::AttnArgs a, float scale,
                                                                int max_chunks) {
    constexpr int EPL = HD / 16;  // elements per lane
    constexpr int HALF = HD / 2;
    const int c = blockIdx.x, g = blockIdx.y;
    const int seq = a.pos_dev ? (*a.pos_dev + 1) : a.seq;
    const int c0 = c * kChunk;
    if (c0 >= seq) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int dg = lane & 15, pg = lane >> 4;
    const int kv_dim = a.n_kv * HD;
    const bool fused = a.qkv != nullptr;
    const int pos_new = seq - 1;
    const bool has_new = fused && pos_new >= c0 && pos_new < c0 + kChunk;
    KVT *kc = reinterpret_cast<KVT *>(a.k_cache);
    KVT *vc = reinterpret_cast<KVT *>(a.v_cache);

    __shared__ float q_s[HPK][HD];
    __shared__ float knew_s[HD], vnew_s[HD];
    __shared__ float w_o[4][HPK][HD];
    __shared__ float w_m[4][HPK], w_l[4][HPK];

    // ---- query heads (and the new k/v row) ----
    if (fused) {
        const int q_dim = a.n_heads * HD;
        for (int j = wave; j < HPK + 2; j += 4) {
            if (j >= HPK && !has_new) continue;
            if (j == HPK + 1) {  // v: plain copy, rounded to the cache type
                for (int i = lane; i < HD; i += 64)
                    vnew_s[i] = kv_f(to_kv<KVT>(a.qkv[q_dim + kv_dim + g * HD + i]));
                continue;
            }
            const float *src = j < HPK ? a.qkv + (size_t)(g * HPK + j) * HD : a.qkv + q_dim + g * HD;
            const float *nw = j < HPK ? a.q_norm_w : a.k_norm_w;
            float ss = 0.0f;
            for (int i = lane; i < HD; i += 64) ss += src[i] * src[i];
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
            for (int i = lane; i < HALF; i += 64) {
                const float lo = (src[i] * inv) * nw[i];
                const float hi = (src[i + HALF] * inv) * nw[i + HALF];
                const float cs = a.cos_t[(size_t)pos_new * HALF + i];
                const float sn = a.sin_t[(size_t)pos_new * HALF + i];
                const float y0 = lo * cs - hi * sn;
                const float y1 = hi * cs + lo * sn;
                if (j < HPK) {
                    q_s[j][i] = y0;
                    q_s[j][i + HALF] = y1;
                } else {
                    knew_s[i] = kv_f(to_kv<KVT>(y0));
                    knew_s[i + HALF] = kv_f(to_kv<KVT>(y1));
                }
            }
        }
    } else {
        for (int idx = tid; idx < HPK * HD; idx += kThreads)
            q_s[idx / HD][idx % HD] = a.q[(size_t)(g * HPK + idx / HD) * HD + idx % HD];
    }
    __syncthreads();
    if (has_new) {
        for (int i = tid; i < HD; i += kThreads) {
            kc[(size_t)pos_new * kv_dim + g * HD + i] = to_kv<KVT>(knew_s[i]);
            vc[(size_t)pos_new * kv_dim + g * HD + i] = to_kv<KVT>(vnew_s[i]);
        }
    }

    float qr[HPK][EPL];
#pragma unroll
    for (int j = 0; j < HPK; ++j)
#pragma unroll
        for (int e = 0; e < EPL; ++e) qr[j][e] = q_s[j][dg * EPL + e];

    // ---- stream this wave's 32 positions ----
    const int wbase = c0 + wave * kPerWave;
    Vec<KVT, EPL> kraw[kSteps], vraw[kSteps];
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        int p = wbase + st * 4 + pg;
        p = p < seq ? p : seq - 1;
        const size_t off = (size_t)p * kv_dim + g * HD + dg * EPL;
        kraw[st] = load_vec<KVT, EPL>(kc + off);
        vraw[st] = load_vec<KVT, EPL>(vc + off);
    }

    float s[kSteps][HPK];
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        const int p = wbase + st * 4 + pg;
        const bool is_new = has_new && p == pos_new;
        float kf[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) kf[e] = is_new ? knew_s[dg * EPL + e] : kv_f(kraw[st].v[e]);
#pragma unroll
        for (int j = 0; j < HPK; ++j) {
            float part = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) part = __builtin_fmaf(qr[j][e], kf[e], part);
            part = sum16(part);
            s[st][j] = p < seq ? part * scale : -INFINITY;
        }
    }

    float m[HPK], l[HPK];
#pragma unroll
    for (int j = 0; j < HPK; ++j) {
        float mx = s[0][j];
#pragma unroll
        for (int st = 1; st < kSteps; ++st) mx = fmaxf(mx, s[st][j]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        m[j] = mx;
        float ls = 0.0f;
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            const float pr = mx == -INFINITY ? 0.0f : expf(s[st][j] - mx);
            s[st][j] = pr;
            ls += pr;
        }
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        l[j] = ls;
    }

    float o[HPK][EPL];
#pragma unroll
    for (int j = 0; j < HPK; ++j)
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[j][e] = 0.0f;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        const int p = wbase + st * 4 + pg;
        const bool is_new = has_new && p == pos_new;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float vf = is_new ? vnew_s[dg * EPL + e] : kv_f(vraw[st].v[e]);
#pragma unroll
            for (int j = 0; j < HPK; ++j) o[j][e] = __builtin_fmaf(s[st][j], vf, o[j][e]);
        }
    }
#pragma unroll
    for (int j = 0; j < HPK; ++j)
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float v = o[j][e];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            o[j][e] = v;
        }
    if (pg == 0) {
#pragma unroll
        for (int j = 0; j < HPK; ++j)
#pragma unroll
            for (int e = 0; e < EPL; ++e) w_o[wave][j][dg * EPL + e] = o[j][e];
    }
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < HPK; ++j) {
            w_m[wave][j] = m[j];
            w_l[wave][j] = l[j];
        }
    }
    __syncthreads();

    // ---- merge the 4 waves, write the chunk partial ----
    float *po = a.part + ((size_t)g * max_chunks + c) * HPK * HD;
    float *pml = a.part + (size_t)a.n_kv * max_chunks * HPK * HD +
                 ((size_t)g * max_chunks + c) * HPK * 2;
    for (int idx = tid; idx < HPK * HD; idx += kThreads) {
        const int j = idx / HD, e = idx % HD;
        float M = w_m[0][j];
#pragma unroll
        for (int w = 1; w < 4; ++w) M = fmaxf(M, w_m[w][j]);
        float acc = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = w_m[w][j] == -INFINITY ? 0.0f : expf(w_m[w][j] - M);
            acc += f * w_o[w][j][e];
            L += f * w_l[w][j];
        }
        po[j * HD + e] = acc;
        if (e == 0) {
            pml[j * 2] = M;
            pml[j * 2 + 1] = L;
        }
    }
}

template <int HD>
__global__ __launch_bounds__(64) void attn_merge_kernel(const float *__restrict__ part, int n_kv,
                                                        int hpk, int max_chunks, int seq_host,
                                                        const int *__restrict__ pos_dev,
                                                        float *__restrict__ out) {
    const int h = blockIdx.x;
    const int g = h / hpk, j = h % hpk;
    const int seq = pos_dev ? (*pos_dev + 1) : seq_host;
    const int nc = (seq + kChunk - 1) / kChunk;
    const float *po = part + (size_t)g * max_chunks * hpk * HD;
    const float *pml = part + (size_t)n_kv * max_chunks * hpk * HD + (size_t)g * max_chunks * hpk * 2;
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, pml[(c * hpk + j) * 2]);
    float L = 0.0f;
    for (int c = 0; c < nc; ++c) L += expf(pml[(c * hpk + j) * 2] - M) * pml[(c * hpk + j) * 2 + 1];
    const float inv = 1.0f / L;
    for (int e = threadIdx.x; e < HD; e += 64) {
        float acc = 0.0f;
        for (int c = 0; c < nc; ++c)
            acc += expf(pml[(c * hpk + j) * 2] - M) * po[((size_t)c * hpk + j) * HD + e];
        out[(size_t)h * HD + e] = acc * inv;
    }
}

typedef void (*partial_fn)(cwi::AttnArgs, float, int);
typedef void (*merge_fn)(const float *, int, int, int, int, const int *, float *);

template <typename KVT, int HD>
partial_fn pick_hpk(int hpk) {
    switch (hpk) {
        case 1: return attn_partial_kernel<KVT, HD, 1>;
        case 2: return attn_partial_kernel<KVT, HD, 2>;
        case 4: return attn_partial_kernel<KVT, HD, 4>;
        case 8: return attn_partial_kernel<KVT, HD, 8>;
        default: return nullptr;
    }
}

template <typename KVT>
partial_fn pick_hd(int hd, int hpk) {
    switch (hd) {
        case 16: return pick_hpk<KVT, 16>(hpk);
        case 32: return pick_hpk<KVT, 32>(hpk);
        case 64: return pick_hpk<KVT, 64>(hpk);
        case 128: return pick_hpk<KVT, 128>(hpk);
        case 256: return pick_hpk<KVT, 256>(hpk);
        default: return nullptr;
    }
}

merge_fn pick_merge(int hd) {
    switch (hd) {
        case 16: return attn_merge_kernel<16>;
        case 32: return attn_merge_kernel<32>;
        case 64: return attn_merge_kernel<64>;
        case 128: return attn_merge_kernel<128>;
        case 256: return attn_merge_kernel<256>;
        default: return nullptr;
    }
}

}  // namespace

namespace cwi {

size_t attn_scratch_floats(int n_heads, int n_kv, int hd, int max_seq) {
    (void)n_kv;
    const size_t chunks = (size_t)(max_seq + kChunk - 1) / kChunk;
    return chunks * (size_t)n_heads * (hd + 2);
}

int launch_attention(cw_ctx *ctx, const AttnArgs &a) {
    const int hpk = a.n_heads / a.n_kv;
    partial_fn pf = a.kv_dtype == CW_F16 ? pick_hd<_Float16>(a.hd, hpk) : pick_hd<float>(a.hd, hpk);
    merge_fn mf = pick_merge(a.hd);
    if (!pf || !mf) {
        set_error("attention: unsupported head_dim=%d / heads per kv=%d", a.hd, hpk);
        return CW_ERR_ARG;
    }
    const int max_chunks = (a.max_seq + kChunk - 1) / kChunk;
    const float scale = powf((float)a.hd, -0.5f);
    prof_begin(ctx, "attention");
    hipLaunchKernelGGL(pf, dim3(max_chunks, a.n_kv), dim3(kThreads), 0, ctx->stream, a, scale,
                       max_chunks);
    prof_end(ctx);
    CW_TRY(launch_check("attention_partial"));
    prof_begin(ctx, "attention_merge");
    hipLaunchKernelGGL(mf, dim3(a.n_heads), dim3(64), 0, ctx->stream, a.part, a.n_kv, hpk,
                       max_chunks, a.seq, a.pos_dev, a.out);
    prof_end(ctx);
    return launch_check("attention_merge");
}

}  // namespace cwi

using namespace cwi;

extern "C" int cw_attention(cw_ctx *ctx, const float *q, const void *k, const void *v, int kv_dtype,
                            int n_heads, int n_kv_heads, int seq, int head_dim, float *out) {
    CW_CHECK_ARG(ctx && q && k && v && out, "cw_attention: null argument");
    CW_CHECK_ARG(kv_dtype == CW_F32 || kv_dtype == CW_F16, "cw_attention: kv_dtype=%d", kv_dtype);
    CW_CHECK_ARG(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                 "cw_attention: n_heads=%d n_kv_heads=%d", n_heads, n_kv_heads);
    CW_CHECK_ARG(seq > 0, "cw_attention: seq=%d must be positive", seq);
    const int hpk = n_heads / n_kv_heads;
    CW_CHECK_ARG(hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8,
                 "cw_attention: heads per kv head %d not in {1,2,4,8}", hpk);
    CW_CHECK_ARG(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 ||
                     head_dim == 256,
                 "cw_attention: head_dim=%d not in {16,32,64,128,256}", head_dim);
    void *scratch = nullptr;
    CW_TRY(ctx_scratch(ctx, attn_scratch_floats(n_heads, n_kv_heads, head_dim, seq) * sizeof(float),
                       &scratch));
    AttnArgs a{};
    a.q = q;
    a.k_cache = const_cast<void *>(k);
    a.v_cache = const_cast<void *>(v);
    a.kv_dtype = kv_dtype;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.hd = head_dim;
    a.seq = seq;
    a.max_seq = seq;
    a.out = out;
    a.part = (float *)scratch;
    return launch_attention(ctx, a);
}
