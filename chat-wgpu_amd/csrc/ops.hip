// Small decode-path kernels: RMSNorm, RoPE, residual add, SwiGLU, KV write,
// embedding gather and argmax (with the device-resident generate state).
//
// References: norm.wgsl:20-42, rope.wgsl:18-35, ewise.wgsl:9-13,
// glu.wgsl:22-26, cache.rs:21-24, qwen3.rs:128-133,194-197,
// argmax.wgsl:18-55, mod.rs:93-122.

#include "cw_internal.hpp"

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// norm.wgsl:20-42: y = x * inv * w, inv = 1/sqrt(sum(x^2)/dim + eps).
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ w, int dim,
                                                           float eps, float *__restrict__ y) {
    __shared__ float red[kThreads / 64];
    const size_t base = (size_t)blockIdx.x * dim;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < dim; i += kThreads) {
        float v = x[base + i];
        ss += v * v;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = threadIdx.x; i < dim; i += kThreads) y[base + i] = (x[base + i] * inv) * w[i];
}

// rope.wgsl:18-35 with angles from the table [pos][hd/2].
__global__ __launch_bounds__(kThreads) void rope_kernel(const float *__restrict__ x, int rows,
                                                        int hd, int pos,
                                                        const float *__restrict__ cos_t,
                                                        const float *__restrict__ sin_t,
                                                        float *__restrict__ y) {
    const int half = hd / 2;
    const int idx = blockIdx.x * kThreads + threadIdx.x;
    if (idx >= rows * half) return;
    const int r = idx / half, i = idx % half;
    const float c = cos_t[(size_t)pos * half + i], s = sin_t[(size_t)pos * half + i];
    const float lo = x[(size_t)r * hd + i], hi = x[(size_t)r * hd + i + half];
    y[(size_t)r * hd + i] = lo * c - hi * s;
    y[(size_t)r * hd + i + half] = hi * c + lo * s;
}

__global__ __launch_bounds__(kThreads) void add_kernel(const float *__restrict__ a,
                                                       const float *__restrict__ b, int n,
                                                       float *__restrict__ c) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n) c[i] = a[i] + b[i];
}

__global__ __launch_bounds__(kThreads) void swiglu_kernel(const float *__restrict__ g,
                                                          const float *__restrict__ u, int n,
                                                          float *__restrict__ out) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n) {
        const float x = g[i];
        out[i] = (x / (1.0f + expf(-x))) * u[i];
    }
}

template <typename T>
__device__ __forceinline__ T to_kv(float v);
template <>
__device__ __forceinline__ float to_kv<float>(float v) {
    return v;
}
template <>
__device__ __forceinline__ _Float16 to_kv<_Float16>(float v) {
    return (_Float16)v;  // round to nearest even
}

template <typename T>
__global__ __launch_bounds__(kThreads) void kv_write_kernel(T *__restrict__ kc, T *__restrict__ vc,
                                                            int pos, const int *__restrict__ pos_dev,
                                                            int kv_dim, const float *__restrict__ k,
                                                            const float *__restrict__ v) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= kv_dim) return;
    const int p = pos_dev ? *pos_dev : pos;
    kc[(size_t)p * kv_dim + i] = to_kv<T>(k[i]);
    vc[(size_t)p * kv_dim + i] = to_kv<T>(v[i]);
}

// qwen3.rs:128-133 (row gather) + clone_buf's "+ 0" (qwen3.rs:194-197).
__global__ __launch_bounds__(kThreads) void embed_kernel(const float *__restrict__ table, int vocab,
                                                         int dim, const uint32_t *__restrict__ tok,
                                                         float *__restrict__ out) {
    uint32_t t = *tok;
    t = t < (uint32_t)vocab ? t : (uint32_t)(vocab - 1);
    const size_t base = (size_t)t * dim;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < dim; i += gridDim.x * kThreads)
        out[i] = table[base + i] + 0.0f;
}

// ---- argmax (argmax.wgsl:18-55) ----
// Candidates need v > -3.402823e38 (strict, so NaN never wins); among equal
// values the lowest index wins; no candidate -> index 0.
struct Best {
    float v;
    uint32_t i;
};

__device__ __forceinline__ Best better(Best a, Best b) {
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}

__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        Best o{__shfl_xor(b.v, off), (uint32_t)__shfl_xor((int)b.i, off)};
        b = better(b, o);
    }
    return b;
}

constexpr float kNegInit = -3.402823e38f;
constexpr int kArgmaxBlocks = 256;

__device__ Best block_best(Best b) {
    __shared__ float sv[kThreads / 64];
    __shared__ uint32_t si[kThreads / 64];
    b = wave_best(b);
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = b.v;
        si[threadIdx.x >> 6] = b.i;
    }
    __syncthreads();
    Best r{sv[0], si[0]};
    for (int w = 1; w < kThreads / 64; ++w) r = better(r, Best{sv[w], si[w]});
    return r;
}

// stage 1: each block scans a contiguous slice
__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(const float *__restrict__ x,
                                                                  int n, int per_block,
                                                                  float *__restrict__ pv,
                                                                  uint32_t *__restrict__ pi) {
    const int lo = blockIdx.x * per_block;
    const int hi = min(n, lo + per_block);
    Best b{kNegInit, 0u};
    for (int i = lo + threadIdx.x; i < hi; i += kThreads) {
        const float v = x[i];
        if (v > b.v) {
            b.v = v;
            b.i = (uint32_t)i;
        }
    }
    b = block_best(b);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = b.v;
        pi[blockIdx.x] = b.i;
    }
}

// stage 2: merge partials; optionally advance the generate state
// (mod.rs:114-122: feed prompt[p+1] inside the prompt, else record the
// argmax and feed it back).
__global__ __launch_bounds__(kThreads) void argmax_final_kernel(const float *__restrict__ pv,
                                                                const uint32_t *__restrict__ pi,
                                                                int nparts, uint32_t *out,
                                                                cwi::GenState *st,
                                                                const uint32_t *__restrict__ prompt,
                                                                uint32_t *__restrict__ toks) {
    Best b{kNegInit, 0u};
    for (int i = threadIdx.x; i < nparts; i += kThreads) b = better(b, Best{pv[i], pi[i]});
    b = block_best(b);
    if (threadIdx.x == 0) {
        if (out) *out = b.i;
        if (st) {
            const int p = st->pos - st->start_pos;
            if (p + 1 < st->n_prompt) {
                st->token = prompt[p + 1];
            } else {
                if (st->produced < st->max_out) toks[st->produced] = b.i;
                st->produced += 1;
                st->token = b.i;
            }
            st->pos += 1;
        }
    }
}

// HBM read probe (the examples/q4probe.rs analogue): every thread streams
// 16-byte words over a grid-stride loop and folds them with XOR, so nothing
// but the reads costs time; one word per workgroup is written out.  The
// four loads in flight per thread are non-temporal: on MI355X that streams a
// 2 GiB buffer at 7.1-7.25 TB/s at two workgroups per CU, against
// 6.2-6.4 TB/s with plain loads.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4 *p) {
    return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p)));
}
__global__ __launch_bounds__(kThreads) void read_probe_kernel(const uint4 *__restrict__ p,
                                                              size_t n16, uint32_t *__restrict__ out) {
    uint4 acc = make_uint4(0, 0, 0, 0);
    const size_t stride = (size_t)gridDim.x * kThreads;
    size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = ld_stream(p + i), b = ld_stream(p + i + stride),
                    c = ld_stream(p + i + 2 * stride), d = ld_stream(p + i + 3 * stride);
        acc.x ^= a.x ^ b.x ^ c.x ^ d.x;
        acc.y ^= a.y ^ b.y ^ c.y ^ d.y;
        acc.z ^= a.z ^ b.z ^ c.z ^ d.z;
        acc.w ^= a.w ^ b.w ^ c.w ^ d.w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = ld_stream(p + i);
        acc.x ^= a.x;
        acc.y ^= a.y;
        acc.z ^= a.z;
        acc.w ^= a.w;
    }
    uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v ^= (uint32_t)__shfl_xor((int)v, off);
    __shared__ uint32_t red[kThreads / 64];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace

namespace cwi {

int launch_rmsnorm(cw_ctx *ctx, const float *x, const float *w, int rows, int dim, float eps,
                   float *y) {
    return launch(ctx, "rmsnorm", rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, x, w, dim, eps,
                  y);
}

int launch_rope(cw_ctx *ctx, const float *x, int rows, int hd, int pos, const float *cos_t,
                const float *sin_t, float *y) {
    const int n = rows * (hd / 2);
    return launch(ctx, "rope", rope_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0,
                  x, rows, hd, pos, cos_t, sin_t, y);
}

int launch_add(cw_ctx *ctx, const float *a, const float *b, int n, float *c) {
    return launch(ctx, "ewise_add", add_kernel, dim3((n + kThreads - 1) / kThreads),
                  dim3(kThreads), 0, a, b, n, c);
}

int launch_swiglu(cw_ctx *ctx, const float *g, const float *u, int n, float *out) {
    return launch(ctx, "swiglu", swiglu_kernel, dim3((n + kThreads - 1) / kThreads),
                  dim3(kThreads), 0, g, u, n, out);
}

int launch_kv_write(cw_ctx *ctx, void *kc, void *vc, int kv_dtype, int pos, const int *pos_dev,
                    int kv_dim, const float *k, const float *v) {
    dim3 grid((kv_dim + kThreads - 1) / kThreads);
    if (kv_dtype == CW_F16)
        return launch(ctx, "kv_write", kv_write_kernel<_Float16>, grid, dim3(kThreads), 0,
                      (_Float16 *)kc, (_Float16 *)vc, pos, pos_dev, kv_dim, k, v);
    return launch(ctx, "kv_write", kv_write_kernel<float>, grid, dim3(kThreads), 0, (float *)kc,
                  (float *)vc, pos, pos_dev, kv_dim, k, v);
}

int launch_embed(cw_ctx *ctx, const float *table, int vocab, int dim, const uint32_t *tok_dev,
                 float *out) {
    int blocks = (dim + kThreads - 1) / kThreads;
    return launch(ctx, "embed", embed_kernel, dim3(blocks), dim3(kThreads), 0, table, vocab, dim,
                  tok_dev, out);
}

size_t argmax_scratch_bytes(int n) {
    (void)n;
    return (size_t)kArgmaxBlocks * (sizeof(float) + sizeof(uint32_t));
}

int launch_argmax(cw_ctx *ctx, const float *logits, int n, uint32_t *out_dev, void *scratch,
                  GenState *state, const uint32_t *prompt_dev, uint32_t *tokens_out_dev) {
    int blocks = (n + 4095) / 4096;
    if (blocks > kArgmaxBlocks) blocks = kArgmaxBlocks;
    if (blocks < 1) blocks = 1;
    const int per_block = (n + blocks - 1) / blocks;
    float *pv = (float *)scratch;
    uint32_t *pi = (uint32_t *)(pv + kArgmaxBlocks);
    CW_TRY(launch(ctx, "argmax", argmax_partial_kernel, dim3(blocks), dim3(kThreads), 0, logits,
                  n, per_block, pv, pi));
    return launch(ctx, "argmax", argmax_final_kernel, dim3(1), dim3(kThreads), 0, pv, pi, blocks,
                  out_dev, state, prompt_dev, tokens_out_dev);
}

}  // namespace cwi

using namespace cwi;

extern "C" {

int cw_rmsnorm(cw_ctx *ctx, const float *x, const float *w, int rows, int dim, float eps,
               float *y) {
    CW_CHECK_ARG(ctx && x && w && y, "cw_rmsnorm: null argument");
    CW_CHECK_ARG(rows > 0 && dim > 0, "cw_rmsnorm: rows=%d dim=%d must be positive", rows, dim);
    return launch_rmsnorm(ctx, x, w, rows, dim, eps, y);
}

int cw_rope(cw_ctx *ctx, const float *x, int rows, int head_dim, int pos, float theta, float *y) {
    CW_CHECK_ARG(ctx && x && y, "cw_rope: null argument");
    CW_CHECK_ARG(rows > 0 && head_dim > 0 && head_dim % 2 == 0,
                 "cw_rope: rows=%d head_dim=%d (head_dim must be even)", rows, head_dim);
    CW_CHECK_ARG(pos >= 0 && pos < (1 << 20), "cw_rope: pos=%d out of range", pos);
    const cw_rope_tab *t = nullptr;
    CW_TRY(ctx_rope_table(ctx, theta, head_dim, pos + 1, &t));
    return launch_rope(ctx, x, rows, head_dim, pos, t->cos_t, t->sin_t, y);
}

int cw_add(cw_ctx *ctx, const float *a, const float *b, int n, float *c) {
    CW_CHECK_ARG(ctx && a && b && c, "cw_add: null argument");
    CW_CHECK_ARG(n > 0, "cw_add: n=%d must be positive", n);
    return launch_add(ctx, a, b, n, c);
}

int cw_swiglu(cw_ctx *ctx, const float *gate, const float *up, int n, float *out) {
    CW_CHECK_ARG(ctx && gate && up && out, "cw_swiglu: null argument");
    CW_CHECK_ARG(n > 0, "cw_swiglu: n=%d must be positive", n);
    return launch_swiglu(ctx, gate, up, n, out);
}

int cw_argmax(cw_ctx *ctx, const float *logits, int n, uint32_t *out_dev) {
    CW_CHECK_ARG(ctx && logits && out_dev, "cw_argmax: null argument");
    CW_CHECK_ARG(n > 0, "cw_argmax: n=%d must be positive", n);
    void *scratch = nullptr;
    CW_TRY(ctx_scratch(ctx, argmax_scratch_bytes(n), &scratch));
    return launch_argmax(ctx, logits, n, out_dev, scratch, nullptr, nullptr, nullptr);
}

int cw_kv_write(cw_ctx *ctx, void *k_cache, void *v_cache, int kv_dtype, int pos, int kv_dim,
                const float *k, const float *v) {
    CW_CHECK_ARG(ctx && k_cache && v_cache && k && v, "cw_kv_write: null argument");
    CW_CHECK_ARG(kv_dtype == CW_F32 || kv_dtype == CW_F16, "cw_kv_write: kv_dtype=%d", kv_dtype);
    CW_CHECK_ARG(pos >= 0 && kv_dim > 0, "cw_kv_write: pos=%d kv_dim=%d", pos, kv_dim);
    return launch_kv_write(ctx, k_cache, v_cache, kv_dtype, pos, nullptr, kv_dim, k, v);
}

int cw_embed(cw_ctx *ctx, const float *table, int vocab, int dim, const uint32_t *token_dev,
             float *out) {
    CW_CHECK_ARG(ctx && table && token_dev && out, "cw_embed: null argument");
    CW_CHECK_ARG(vocab > 0 && dim > 0, "cw_embed: vocab=%d dim=%d", vocab, dim);
    return launch_embed(ctx, table, vocab, dim, token_dev, out);
}

int cw_hbm_read_probe(cw_ctx *ctx, const void *buf, size_t bytes, int blocks, uint32_t *out_dev) {
    CW_CHECK_ARG(ctx && buf && out_dev, "cw_hbm_read_probe: null argument");
    CW_CHECK_ARG(((uintptr_t)buf & 15) == 0 && bytes >= 16,
                 "cw_hbm_read_probe: buf must be 16-byte aligned and bytes >= 16");
    CW_CHECK_ARG(blocks > 0 && blocks <= 65536, "cw_hbm_read_probe: blocks=%d", blocks);
    return launch(ctx, "hbm_read_probe", read_probe_kernel, dim3(blocks), dim3(kThreads), 0,
                  (const uint4 *)buf, bytes / 16, out_dev);
}

}  // extern "C"
