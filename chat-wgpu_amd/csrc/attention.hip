// Single-query GQA decode attention for gfx950.
//
// Replaces attention::attention (src/kernels/attention.rs:7-38,
// attention.wgsl:23-96).  Same mathematics: o_h = sum_j softmax_j(scale *
// q_h . k_j) v_j over j < seq, kv head = h / (n_heads / n_kv), scale =
// hd^-0.5, max-rescaled softmax.
//
// Split over the sequence (flash-decoding).  Workgroup (chunk c, kv head g)
// owns CP consecutive positions and one wave per query head of the GQA group:
//   1. the query, then the K rows, then the V rows of the chunk (this kv
//      head's slice) are loaded with coalesced 16-byte loads, all issued up
//      front in the order they are used, into LDS tiles with a 16-byte row
//      pad (conflict-free row reads);
//   2. wave j: lane = position, full q.k dot from the K tile against the
//      query broadcast from LDS (f16 keys feed v_fma_mix directly) while the
//      V rows are still arriving; wavefront max / sum give the chunk's
//      softmax partial;
//   3. wave j: lane = head dimension, P.V over the V tile's rows.
// No cross-lane reduction is needed per position.  A chunk partial
// (max, sum, unnormalised o) goes to HBM unless the sequence fits one chunk,
// in which case the normalised output is written directly; the merge kernel
// combines chunks with one round of independent loads.  (Scores on the matrix
// cores were tried for the 4-head groups of the 8B shape: with 4 of 16 MFMA
// rows used and q / p split into f16 pairs per lane, the kernel ran slower.)
//
// Fused prologue (decode step): the raw q/k/v come straight from the fused
// QKV projection; the kernel applies the per-head QK RMSNorm (norm.wgsl,
// qwen3.rs:154-155) and RoPE (rope.wgsl), and the workgroup whose chunk holds
// the new position writes k/v into the cache (cache.rs:21-24) and into its
// own tile.

#include <cmath>
#include <map>
#include <mutex>

#include "cw_internal.hpp"

namespace {

constexpr int kMaxChunkSpan = 32768;  // max_seq limit
// 512 threads: 4 chunk slices x 32 loads per thread cover the 68 chunks of a
// 4352-position cache in one pass (256 threads took two: 5.6 us against 4.3)
constexpr int kMergeThreads = 512;

template <typename KVT, int HD, int HPK>
struct Cfg {
    static constexpr int ES = (int)sizeof(KVT);
    static constexpr int THREADS = 64 * HPK;
    // 16-byte loads per thread for the K+V tile.  Chunks of <= 64 positions
    // keep the tile near 36 KB so several workgroups share a CU and every
    // chunk of a 4K-position cache is resident at once (8 kv heads x 68
    // chunks = 544 workgroups); small groups load more per thread.
    static constexpr int LB = THREADS <= 128 ? 32 : 8;
    static constexpr int CP0 = LB * THREADS * 16 / (2 * HD * ES);
    static constexpr int CP = CP0 > 64 ? 64 : CP0;  // positions per workgroup
    static constexpr int ROWB = HD * ES;              // bytes of one row slice
    static constexpr int ROWP = ROWB + 16;            // padded LDS row stride
    static constexpr int U4_ROW = ROWB / 16;          // 16-byte units per row
    static constexpr int NLOAD = (CP * U4_ROW + THREADS - 1) / THREADS;
    static constexpr int NT = (CP + 63) / 64;         // positions per lane
    static constexpr int DPL = HD >= 64 ? HD / 64 : 1;  // dims per lane in P.V
    static constexpr int EPU = 16 / ES;               // elements per 16 bytes
    // LDS: K tile, V tile, q [HPK][HD], p [HPK][CP]
    static constexpr int LDS = 2 * CP * ROWP + HPK * HD * 4 + HPK * CP * 4;
    static_assert(LDS <= 160 * 1024, "attention tile exceeds the CU's LDS");
    static_assert(CP >= 8 && CP % 8 == 0, "chunk must hold whole load groups");
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

template <typename T>
__device__ __forceinline__ T to_kv(float v) {
    return (T)v;  // f32 -> f16 rounds to nearest even
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// sum over the elements of one 16-byte unit of a K row times q (f32)
template <typename KVT>
__device__ __forceinline__ float dot16(uint4 k, const float *q, float acc);

template <>
__device__ __forceinline__ float dot16<_Float16>(uint4 k, const float *q, float acc) {
    const uint32_t w[4] = {k.x, k.y, k.z, k.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v h = __builtin_bit_cast(half2v, w[i]);
        acc = __builtin_fmaf((float)h.x, q[2 * i], acc);
        acc = __builtin_fmaf((float)h.y, q[2 * i + 1], acc);
    }
    return acc;
}

template <>
__device__ __forceinline__ float dot16<float>(uint4 k, const float *q, float acc) {
    acc = __builtin_fmaf(__builtin_bit_cast(float, k.x), q[0], acc);
    acc = __builtin_fmaf(__builtin_bit_cast(float, k.y), q[1], acc);
    acc = __builtin_fmaf(__builtin_bit_cast(float, k.z), q[2], acc);
    acc = __builtin_fmaf(__builtin_bit_cast(float, k.w), q[3], acc);
    return acc;
}

template <typename KVT, int HD, int HPK>
__global__ __launch_bounds__(64 * HPK) void attn_kernel(cwi::AttnArgs a, float scale,
                                                        int max_chunks) {
    using C = Cfg<KVT, HD, HPK>;
    constexpr int HALF = HD / 2;
    extern __shared__ uint4 lds_u4[];
    unsigned char *lds = reinterpret_cast<unsigned char *>(lds_u4);
    unsigned char *k_t = lds;                       // [CP][ROWP]
    unsigned char *v_t = lds + C::CP * C::ROWP;     // [CP][ROWP]
    float *q_s = reinterpret_cast<float *>(lds + 2 * C::CP * C::ROWP);  // [HPK][HD]
    float *p_s = q_s + HPK * HD;                                       // [HPK][CP]

    const int c = blockIdx.x, g = blockIdx.y;
    const int seq = a.pos_dev ? (*a.pos_dev + 1) : a.seq;
    const int c0 = c * C::CP;
    if (c0 >= seq) return;
    const int n_chunks = (seq + C::CP - 1) / C::CP;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kv_dim = a.n_kv * HD;
    const bool fused = a.qkv != nullptr;
    const int pos_new = seq - 1;
    const bool has_new = fused && pos_new >= c0 && pos_new < c0 + C::CP;
    const unsigned char *kc = reinterpret_cast<const unsigned char *>(a.k_cache);
    const unsigned char *vc = reinterpret_cast<const unsigned char *>(a.v_cache);
    const size_t row_bytes = (size_t)kv_dim * C::ES;

    // ---- 1. loads, in the order they are needed (they return in issue
    // order): this wave's query (and, in the workgroup holding the new
    // position, the new k and v), then the K rows, then the V rows, which
    // arrive while the scores are computed ----
    constexpr int QU = (HALF + 63) / 64, VU = (HD + 63) / 64;
    const int h = g * HPK + wave;
    float lo[QU], hi[QU], cs[QU], sn[QU], gl[QU], gh[QU];
    float klo[QU], khi[QU], kgl[QU], kgh[QU], vraw[VU], qp[VU];
    if (fused) {
        const float *src = a.qkv + (size_t)h * HD;
#pragma unroll
        for (int u = 0; u < QU; ++u) {
            const int i = min(lane + 64 * u, HALF - 1);
            lo[u] = src[i];
            hi[u] = src[i + HALF];
            cs[u] = a.cos_t[(size_t)pos_new * HALF + i];
            sn[u] = a.sin_t[(size_t)pos_new * HALF + i];
            gl[u] = a.q_norm_w[i];
            gh[u] = a.q_norm_w[i + HALF];
        }
        if (has_new && wave == 0) {
            const int q_dim = a.n_heads * HD;
            const float *ks = a.qkv + q_dim + g * HD;
            const float *vs = a.qkv + q_dim + kv_dim + g * HD;
#pragma unroll
            for (int u = 0; u < QU; ++u) {
                const int i = min(lane + 64 * u, HALF - 1);
                klo[u] = ks[i];
                khi[u] = ks[i + HALF];
                kgl[u] = a.k_norm_w[i];
                kgh[u] = a.k_norm_w[i + HALF];
            }
#pragma unroll
            for (int u = 0; u < VU; ++u) vraw[u] = vs[min(lane + 64 * u, HD - 1)];
        }
    } else {
#pragma unroll
        for (int u = 0; u < VU; ++u) qp[u] = a.q[(size_t)h * HD + min(lane + 64 * u, HD - 1)];
    }
    uint4 kr[C::NLOAD], vr[C::NLOAD];
#pragma unroll
    for (int i = 0; i < C::NLOAD; ++i) {
        const int f = tid + i * C::THREADS;
        const int row = f / C::U4_ROW, col = f % C::U4_ROW;
        int p = c0 + row;
        p = p < seq ? p : seq - 1;
        const size_t off = (size_t)p * row_bytes + (size_t)g * C::ROWB + (size_t)col * 16;
        if (f < C::CP * C::U4_ROW) kr[i] = *reinterpret_cast<const uint4 *>(kc + off);
    }
#pragma unroll
    for (int i = 0; i < C::NLOAD; ++i) {
        const int f = tid + i * C::THREADS;
        const int row = f / C::U4_ROW, col = f % C::U4_ROW;
        int p = c0 + row;
        p = p < seq ? p : seq - 1;
        const size_t off = (size_t)p * row_bytes + (size_t)g * C::ROWB + (size_t)col * 16;
        if (f < C::CP * C::U4_ROW) vr[i] = *reinterpret_cast<const uint4 *>(vc + off);
    }

    // ---- 2. query head of this wave (normalised + rotated when fused) ----
    float knew[QU][2], vnew[VU];
    if (fused) {
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < QU; ++u)
            if (lane + 64 * u < HALF) ss += lo[u] * lo[u] + hi[u] * hi[u];
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
        for (int u = 0; u < QU; ++u) {
            const int i = lane + 64 * u;
            if (i < HALF) {
                const float l0 = (lo[u] * inv) * gl[u];
                const float h0 = (hi[u] * inv) * gh[u];
                q_s[wave * HD + i] = l0 * cs[u] - h0 * sn[u];
                q_s[wave * HD + i + HALF] = h0 * cs[u] + l0 * sn[u];
            }
        }
        if (has_new && wave == 0) {  // the new k (normed + rotated) and v
            float kss = 0.0f;
#pragma unroll
            for (int u = 0; u < QU; ++u)
                if (lane + 64 * u < HALF) kss += klo[u] * klo[u] + khi[u] * khi[u];
            kss = wave_sum(kss);
            const float kinv = 1.0f / sqrtf(kss / (float)HD + a.eps);
#pragma unroll
            for (int u = 0; u < QU; ++u) {
                const float l0 = (klo[u] * kinv) * kgl[u];
                const float h0 = (khi[u] * kinv) * kgh[u];
                knew[u][0] = l0 * cs[u] - h0 * sn[u];
                knew[u][1] = h0 * cs[u] + l0 * sn[u];
            }
#pragma unroll
            for (int u = 0; u < VU; ++u) vnew[u] = vraw[u];
        }
    } else {
#pragma unroll
        for (int u = 0; u < VU; ++u)
            if (lane + 64 * u < HD) q_s[wave * HD + lane + 64 * u] = qp[u];
    }

    // ---- 3. K tile -> LDS (rows past the sequence as zeros); the new k and
    // v rows to the cache, the new k row also into the tile ----
#pragma unroll
    for (int i = 0; i < C::NLOAD; ++i) {
        const int f = tid + i * C::THREADS;
        if (f < C::CP * C::U4_ROW) {
            const int row = f / C::U4_ROW, col = f % C::U4_ROW;
            // select per component: a select of whole uint4 lvalues becomes a
            // pointer select that forces kr/vr into scratch memory
            uint4 kk = kr[i];
            if (c0 + row >= seq) kk = make_uint4(0, 0, 0, 0);
            *reinterpret_cast<uint4 *>(k_t + row * C::ROWP + col * 16) = kk;
        }
    }
    __syncthreads();
    if (has_new && wave == 0) {
        const int r = pos_new - c0;
        KVT *kt = reinterpret_cast<KVT *>(k_t + r * C::ROWP);
        KVT *kg = reinterpret_cast<KVT *>(const_cast<unsigned char *>(kc) +
                                          (size_t)pos_new * row_bytes + (size_t)g * C::ROWB);
        KVT *vg = reinterpret_cast<KVT *>(const_cast<unsigned char *>(vc) +
                                          (size_t)pos_new * row_bytes + (size_t)g * C::ROWB);
#pragma unroll
        for (int u = 0; u < QU; ++u) {
            const int i = lane + 64 * u;
            if (i < HALF) {
                const KVT k0 = to_kv<KVT>(knew[u][0]), k1 = to_kv<KVT>(knew[u][1]);
                kt[i] = k0;
                kt[i + HALF] = k1;
                kg[i] = k0;
                kg[i + HALF] = k1;
            }
        }
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int i = lane + 64 * u;
            if (i < HD) vg[i] = to_kv<KVT>(vnew[u]);
        }
    }
    if (has_new) __syncthreads();

    // ---- 4. scores: lane = position ----
    const float *qw = q_s + wave * HD;
    constexpr int NA = C::U4_ROW >= 4 ? 4 : C::U4_ROW;  // independent partial sums
    float s4[C::NT][NA];
#pragma unroll
    for (int t = 0; t < C::NT; ++t)
#pragma unroll
        for (int j = 0; j < NA; ++j) s4[t][j] = 0.0f;
#pragma unroll
    for (int u = 0; u < C::U4_ROW; ++u) {
        float qv[C::EPU];
#pragma unroll
        for (int e = 0; e < C::EPU; e += 4) {
            const float4 q4 = *reinterpret_cast<const float4 *>(qw + u * C::EPU + e);
            qv[e] = q4.x;
            qv[e + 1] = q4.y;
            qv[e + 2] = q4.z;
            qv[e + 3] = q4.w;
        }
#pragma unroll
        for (int t = 0; t < C::NT; ++t) {
            const int r = lane + 64 * t;
            if (r < C::CP) {
                const uint4 kk = *reinterpret_cast<const uint4 *>(k_t + r * C::ROWP + u * 16);
                s4[t][u % NA] = dot16<KVT>(kk, qv, s4[t][u % NA]);
            }
        }
    }
    float s[C::NT];
    float mloc = -INFINITY;
#pragma unroll
    for (int t = 0; t < C::NT; ++t) {
        float sv = s4[t][0];
#pragma unroll
        for (int j = 1; j < NA; ++j) sv += s4[t][j];
        const int r = lane + 64 * t;
        s[t] = (r < C::CP && c0 + r < seq) ? sv * scale : -INFINITY;
        mloc = fmaxf(mloc, s[t]);
    }
    const float m = wave_max(mloc);  // finite: row c0 < seq exists
    float lsum = 0.0f;
#pragma unroll
    for (int t = 0; t < C::NT; ++t) {
        const int r = lane + 64 * t;
        const float pr = s[t] == -INFINITY ? 0.0f : expf(s[t] - m);
        lsum += pr;
        if (r < C::CP) p_s[wave * C::CP + r] = pr;
    }
    const float l = wave_sum(lsum);

    // ---- V tile -> LDS (rows past the sequence as zeros), the new v row ----
#pragma unroll
    for (int i = 0; i < C::NLOAD; ++i) {
        const int f = tid + i * C::THREADS;
        if (f < C::CP * C::U4_ROW) {
            const int row = f / C::U4_ROW, col = f % C::U4_ROW;
            uint4 vv = vr[i];
            if (c0 + row >= seq) vv = make_uint4(0, 0, 0, 0);
            *reinterpret_cast<uint4 *>(v_t + row * C::ROWP + col * 16) = vv;
        }
    }
    __syncthreads();
    if (has_new) {
        if (wave == 0) {
            KVT *vt = reinterpret_cast<KVT *>(v_t + (pos_new - c0) * C::ROWP);
#pragma unroll
            for (int u = 0; u < VU; ++u) {
                const int i = lane + 64 * u;
                if (i < HD) vt[i] = to_kv<KVT>(vnew[u]);
            }
        }
        __syncthreads();
    }

    // ---- 5. P.V: lane = head dimension, every tile row (masked rows carry
    // p = 0 and a finite clamped V row), unrolled so LDS reads batch up ----
    float o[C::DPL];
    const int d0 = lane * C::DPL;
    {
        float o4[C::DPL][4];  // independent partial sums over rows
#pragma unroll
        for (int e = 0; e < C::DPL; ++e)
#pragma unroll
            for (int j = 0; j < 4; ++j) o4[e][j] = 0.0f;
        if (d0 < HD) {
            const float *pw = p_s + wave * C::CP;
#pragma unroll
            for (int r0 = 0; r0 < C::CP; r0 += 8) {
                const float4 pa = *reinterpret_cast<const float4 *>(pw + r0);
                const float4 pb = *reinterpret_cast<const float4 *>(pw + r0 + 4);
                const float pr[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const KVT *vrow = reinterpret_cast<const KVT *>(v_t + (r0 + i) * C::ROWP) + d0;
#pragma unroll
                    for (int e = 0; e < C::DPL; ++e)
                        o4[e][i & 3] = __builtin_fmaf(pr[i], (float)vrow[e], o4[e][i & 3]);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < C::DPL; ++e) o[e] = (o4[e][0] + o4[e][1]) + (o4[e][2] + o4[e][3]);
    }

    // ---- 6. output (one chunk) or chunk partial (h: this wave's head) ----
    if (n_chunks == 1) {
        const float inv = 1.0f / l;
        if (d0 < HD)
#pragma unroll
            for (int e = 0; e < C::DPL; ++e) a.out[(size_t)h * HD + d0 + e] = o[e] * inv;
        return;
    }
    float *po = a.part + ((size_t)h * max_chunks + c) * HD;
    if (d0 < HD)
#pragma unroll
        for (int e = 0; e < C::DPL; ++e) po[d0 + e] = o[e];
    if (lane == 0) {
        float *pml = a.part + (size_t)a.n_heads * max_chunks * HD + ((size_t)h * max_chunks + c) * 2;
        pml[0] = m;
        pml[1] = l;
    }
}

// Load of a chunk partial.  Partials are written by other workgroups of the
// previous kernel, on any XCD, at addresses every call reuses: an agent-scope
// load misses a line this XCD's L2 may still hold from an earlier call (the
// release at the end of the writing kernel has put the new data in memory).
__device__ __forceinline__ float part_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge of the chunk partials: one workgroup per query head; every partial
// load is independent and issued before the (max, sum) reduction.
template <int HD>
__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(const float *__restrict__ part,
                                                                   int n_heads, int cp,
                                                                   int max_chunks, int seq_host,
                                                                   const int *__restrict__ pos_dev,
                                                                   float *__restrict__ out) {
    constexpr int B = 32;  // chunk loads in flight per thread
    __shared__ float w[kMaxChunkSpan / 16];
    __shared__ float red[kMergeThreads / 64];
    const int h = blockIdx.x;
    const int seq = pos_dev ? (*pos_dev + 1) : seq_host;
    const int nc = (seq + cp - 1) / cp;
    if (nc == 1) return;  // the chunk kernel wrote the output itself
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *po = part + (size_t)h * max_chunks * HD;
    const float *pml = part + (size_t)n_heads * max_chunks * HD + (size_t)h * max_chunks * 2;
    // this thread's first (max, sum) pair, loaded ahead of the partials (one
    // round of loads in all; clamped so the load is unconditional)
    const int c0m = min(tid, nc - 1);
    const float2 ml0 = make_float2(part_load(pml + 2 * c0m), part_load(pml + 2 * c0m + 1));
    // first batch of partial elements (thread = element e, chunk slice)
    constexpr int EL = HD < kMergeThreads ? HD : kMergeThreads;
    constexpr int SL = kMergeThreads / EL;  // chunk slices
    const int e = tid % EL, sl = tid / EL;
    float v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
        const int cc = sl + SL * u;
        v[u] = cc < nc ? part_load(po + (size_t)cc * HD + e) : 0.0f;
    }
    // (max, sum) over chunks
    float mx = tid < nc ? ml0.x : -INFINITY;
    for (int cc = tid + kMergeThreads; cc < nc; cc += kMergeThreads)
        mx = fmaxf(mx, part_load(pml + cc * 2));
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int i = 1; i < kMergeThreads / 64; ++i) M = fmaxf(M, red[i]);
    __syncthreads();
    float ls = 0.0f;
    if (tid < nc) {
        const float f = expf(ml0.x - M);
        w[tid] = f;
        ls = f * ml0.y;
    }
    for (int cc = tid + kMergeThreads; cc < nc; cc += kMergeThreads) {
        const float f = expf(part_load(pml + cc * 2) - M);
        w[cc] = f;
        ls += f * part_load(pml + cc * 2 + 1);
    }
    ls = wave_sum(ls);
    if (lane == 0) red[wave] = ls;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (int i = 0; i < kMergeThreads / 64; ++i) L += red[i];
    const float inv = 1.0f / L;
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < B; ++u) {
        const int cc = sl + SL * u;
        if (cc < nc) acc += w[cc] * v[u];
    }
    for (int cc0 = SL * B; cc0 < nc; cc0 += SL * B) {  // more than SL*B chunks
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int cc = cc0 + sl + SL * u;
            v[u] = cc < nc ? part_load(po + (size_t)cc * HD + e) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int cc = cc0 + sl + SL * u;
            if (cc < nc) acc += w[cc] * v[u];
        }
    }
    if constexpr (SL > 1) {  // combine the chunk slices through LDS
        __shared__ float part_s[kMergeThreads];
        part_s[tid] = acc;
        __syncthreads();
        if (sl == 0) {
            for (int i = 1; i < SL; ++i) acc += part_s[e + i * EL];
            out[(size_t)h * HD + e] = acc * inv;
        }
    } else {
        out[(size_t)h * HD + e] = acc * inv;
    }
}

typedef void (*attn_fn)(cwi::AttnArgs, float, int);
typedef void (*merge_fn)(const float *, int, int, int, int, const int *, float *);

struct AttnPick {
    attn_fn fn;
    int threads, cp, lds;
};

template <typename KVT, int HD, int HPK>
AttnPick make_pick() {
    using C = Cfg<KVT, HD, HPK>;
    return {attn_kernel<KVT, HD, HPK>, C::THREADS, C::CP, C::LDS};
}

template <typename KVT, int HD>
AttnPick pick_hpk(int hpk) {
    switch (hpk) {
        case 1: return make_pick<KVT, HD, 1>();
        case 2: return make_pick<KVT, HD, 2>();
        case 4: return make_pick<KVT, HD, 4>();
        case 8: return make_pick<KVT, HD, 8>();
        default: return {nullptr, 0, 0, 0};
    }
}

template <typename KVT>
AttnPick pick_hd(int hd, int hpk) {
    switch (hd) {
        case 16: return pick_hpk<KVT, 16>(hpk);
        case 32: return pick_hpk<KVT, 32>(hpk);
        case 64: return pick_hpk<KVT, 64>(hpk);
        case 128: return pick_hpk<KVT, 128>(hpk);
        case 256: return pick_hpk<KVT, 256>(hpk);
        default: return {nullptr, 0, 0, 0};
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

std::mutex g_mu;
std::map<const void *, bool> g_lds_set;

int ensure_lds(attn_fn f, int lds) {
    std::lock_guard<std::mutex> lk(g_mu);
    const void *p = reinterpret_cast<const void *>(f);
    if (!g_lds_set[p]) {
        CW_HIP(hipFuncSetAttribute(p, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
        g_lds_set[p] = true;
    }
    return CW_OK;
}

AttnPick pick_attn(int kv_dtype, int hd, int hpk) {
    return kv_dtype == CW_F16 ? pick_hd<_Float16>(hd, hpk) : pick_hd<float>(hd, hpk);
}

}  // namespace

namespace cwi {

size_t attn_scratch_floats(int n_heads, int n_kv, int hd, int max_seq) {
    const AttnPick pk = pick_attn(CW_F32, hd, n_heads / n_kv);  // f32: smallest chunk
    const int cp = pk.cp > 0 ? pk.cp : 8;
    const size_t chunks = (size_t)(max_seq + cp - 1) / cp;
    return chunks * (size_t)n_heads * (hd + 2);
}

int launch_attention(cw_ctx *ctx, const AttnArgs &a) {
    const int hpk = a.n_heads / a.n_kv;
    const AttnPick pk = pick_attn(a.kv_dtype, a.hd, hpk);
    merge_fn mf = pick_merge(a.hd);
    if (!pk.fn || !mf) {
        set_error("attention: unsupported head_dim=%d / heads per kv=%d", a.hd, hpk);
        return CW_ERR_ARG;
    }
    if (a.max_seq > kMaxChunkSpan) {
        set_error("attention: max_seq=%d exceeds %d", a.max_seq, kMaxChunkSpan);
        return CW_ERR_ARG;
    }
    CW_TRY(ensure_lds(pk.fn, pk.lds));
    const int max_chunks = (a.max_seq + pk.cp - 1) / pk.cp;
    if (max_chunks > kMaxChunkSpan / 16) {  // the merge kernel's weight table
        set_error("attention: %d chunks of %d positions exceed %d", max_chunks, pk.cp,
                  kMaxChunkSpan / 16);
        return CW_ERR_ARG;
    }
    const float scale = powf((float)a.hd, -0.5f);
    prof_begin(ctx, "attention");
    hipLaunchKernelGGL(pk.fn, dim3(max_chunks, a.n_kv), dim3(pk.threads), pk.lds, ctx->stream, a,
                       scale, max_chunks);
    prof_end(ctx);
    CW_TRY(launch_check("attention"));
    if (max_chunks == 1) return CW_OK;
    prof_begin(ctx, "attention_merge");
    hipLaunchKernelGGL(mf, dim3(a.n_heads), dim3(kMergeThreads), 0, ctx->stream, a.part, a.n_heads,
                       pk.cp, max_chunks, a.seq, a.pos_dev, a.out);
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
    CW_CHECK_ARG(seq > 0 && seq <= kMaxChunkSpan, "cw_attention: seq=%d outside [1, %d]", seq,
                 kMaxChunkSpan);
    const int hpk = n_heads / n_kv_heads;
    CW_CHECK_ARG(hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8,
                 "cw_attention: heads per kv head %d not in {1,2,4,8}", hpk);
    CW_CHECK_ARG(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 ||
                     head_dim == 256,
                 "cw_attention: head_dim=%d not in {16,32,64,128,256}", head_dim);
    const size_t nfl = attn_scratch_floats(n_heads, n_kv_heads, head_dim, seq);
    void *scratch = nullptr;
    CW_TRY(ctx_scratch(ctx, nfl * sizeof(float), &scratch));
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
