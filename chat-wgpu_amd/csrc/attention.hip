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
//   3. wave j: lane = head dimension, P.V over its 1/HPK of the V tile's rows
//      for every head of the group (each V row leaves LDS once), the waves'
//      sums added through LDS.
// No cross-lane reduction is needed per position.  A chunk partial
// (max, sum, unnormalised o) goes to memory unless the sequence fits one
// chunk, in which case the normalised output is written directly.  The last
// workgroup of a kv head to finish (one agent-scope counter per kv head)
// merges that head group's partials in the same launch, so the merge costs
// no kernel boundary.  (Scores on the matrix cores were tried for the 4-head
// groups of the 8B shape: with 4 of 16 MFMA rows used and q / p split into
// f16 pairs per lane, the kernel ran slower.)
//
// Coherence across the 8 XCDs (one L2 each): partials are written with
// write-through (sc1) stores and read with sc1 loads, which miss any line an
// L2 still holds from an earlier call; a workgroup's stores are complete
// (s_waitcnt) before its counter increment, and the merging workgroup reads
// only after its own increment returned.  The merger resets the counter, so
// every launch, eager or replayed from a graph, starts from zero.
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
constexpr int kSc1 = 16;              // buffer-instruction cache policy bits: sc1 (agent scope)

template <typename KVT, int HD, int HPK>
struct Cfg {
    static constexpr int ES = (int)sizeof(KVT);
    static constexpr int THREADS = 64 * HPK;
    // 16-byte loads per thread for the K+V tile.  Chunks of <= 128
    // positions keep the tile near 70 KB, so two workgroups share a CU and
    // every chunk of a 4K-position cache is resident at once (8 kv heads x 34
    // chunks = 272 workgroups), while the merge reads few partials; small
    // groups load more per thread.
    static constexpr int LB = THREADS <= 128 ? 32 : 16;
    static constexpr int CP0 = LB * THREADS * 16 / (2 * HD * ES);
    static constexpr int CP = CP0 > 128 ? 128 : CP0;  // positions per workgroup
    static constexpr int ROWB = HD * ES;              // bytes of one row slice
    static constexpr int ROWP = ROWB + 16;            // padded LDS row stride
    static constexpr int U4_ROW = ROWB / 16;          // 16-byte units per row
    static constexpr int NLOAD = (CP * U4_ROW + THREADS - 1) / THREADS;
    static constexpr int NT = (CP + 63) / 64;         // positions per lane
    static constexpr int DPL = HD >= 64 ? HD / 64 : 1;  // dims per lane in P.V
    static constexpr int EPU = 16 / ES;               // elements per 16 bytes
    // LDS: K tile, V tile, q [HPK][HD], p [HPK][CP]; the merge reuses it
    // for the chunk weights [HPK][MAXC]
    static constexpr int MAXC = kMaxChunkSpan / CP;
    static constexpr int LDS_MAIN = 2 * CP * ROWP + HPK * HD * 4 + HPK * CP * 4;
    static constexpr int LDS = LDS_MAIN > HPK * MAXC * 4 ? LDS_MAIN : HPK * MAXC * 4;
    // merge: float4 columns per partial row, chunk slices per wave, partial
    // rows in flight per lane (one round covers MSL * MB chunks: 36 at
    // head_dim 128, at most 18 float4 registers)
    static constexpr int MU = HD / 4;
    static constexpr int MSL = 64 / MU;
    static constexpr int MB0 = 36 / MSL > 4 ? 36 / MSL : 4;
    static constexpr int MB = MB0 < 18 ? MB0 : 18;
    static_assert(LDS <= 160 * 1024, "attention tile exceeds the CU's LDS");
    static_assert(CP >= 8 && CP % 8 == 0, "chunk must hold whole load groups");
    static_assert((CP / HPK) % 4 == 0, "every wave's P.V rows come in fours");
    static_assert(HPK * HPK * HD * 4 <= CP * ROWP, "P.V sums must fit the K tile");
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

// A buffer resource over [p, p + bytes); both wave-uniform (readfirstlane
// keeps the descriptor in SGPRs).  Loads past `bytes` return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    void *u = reinterpret_cast<void *>(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, 0, __builtin_amdgcn_readfirstlane(bytes),
                                             0x00020000);
}

// write-through store of one partial value
__device__ __forceinline__ void st_part(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// (max, sum) pair of chunk c, read past this XCD's L2 (zeros past the range)
__device__ __forceinline__ float2 ld_pair(__amdgpu_buffer_rsrc_t r, int c) {
    return __builtin_bit_cast(float2,
                              __builtin_amdgcn_raw_buffer_load_b64(r, (uint32_t)c * 8, 0, kSc1));
}

// every memory operation this wave issued has completed
__device__ __forceinline__ void drain() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
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
                const float r0 = l0 * cs[u] - h0 * sn[u], r1 = h0 * cs[u] + l0 * sn[u];
                q_s[wave * HD + i] = r0;
                q_s[wave * HD + i + HALF] = r1;
                if (a.q_tap && c == 0) {  // the "q" tap (qwen3.rs:165)
                    a.q_tap[(size_t)h * HD + i] = r0;
                    a.q_tap[(size_t)h * HD + i + HALF] = r1;
                }
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

    // ---- 5. P.V: lane = head dimension.  One head: the wave runs over
    // every tile row.  A head group: wave w takes CP / HPK consecutive rows
    // for all HPK heads, so each V row is read from LDS once (not once per
    // head), and the per-wave sums meet in the K tile's space, which no wave
    // reads after the barrier above.  Masked rows carry p = 0 and a finite
    // clamped V row; loops are unrolled so LDS reads batch up ----
    float o[C::DPL];
    const int d0 = lane * C::DPL;
    if constexpr (HPK == 1) {
        float o4[C::DPL][4];  // independent partial sums over rows
#pragma unroll
        for (int e = 0; e < C::DPL; ++e)
#pragma unroll
            for (int j = 0; j < 4; ++j) o4[e][j] = 0.0f;
        if (d0 < HD) {
#pragma unroll
            for (int r0 = 0; r0 < C::CP; r0 += 8) {
                const float4 pa = *reinterpret_cast<const float4 *>(p_s + r0);
                const float4 pb = *reinterpret_cast<const float4 *>(p_s + r0 + 4);
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
    } else {
        constexpr int RPW = C::CP / HPK;                  // rows per wave
        constexpr int NS = HPK * C::DPL >= 8 ? 1 : 2;    // partial sums per output
        float acc[HPK][C::DPL][NS];
#pragma unroll
        for (int hh = 0; hh < HPK; ++hh)
#pragma unroll
            for (int e = 0; e < C::DPL; ++e)
#pragma unroll
                for (int j = 0; j < NS; ++j) acc[hh][e][j] = 0.0f;
        const int rbase = wave * RPW;
        if (d0 < HD) {
#pragma unroll
            for (int r0 = 0; r0 < RPW; r0 += 4) {
                float pr[HPK][4];
#pragma unroll
                for (int hh = 0; hh < HPK; ++hh) {
                    const float4 p4 =
                        *reinterpret_cast<const float4 *>(p_s + hh * C::CP + rbase + r0);
                    pr[hh][0] = p4.x;
                    pr[hh][1] = p4.y;
                    pr[hh][2] = p4.z;
                    pr[hh][3] = p4.w;
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const KVT *vrow =
                        reinterpret_cast<const KVT *>(v_t + (rbase + r0 + i) * C::ROWP) + d0;
                    float vv[C::DPL];
#pragma unroll
                    for (int e = 0; e < C::DPL; ++e) vv[e] = (float)vrow[e];
#pragma unroll
                    for (int hh = 0; hh < HPK; ++hh)
#pragma unroll
                        for (int e = 0; e < C::DPL; ++e)
                            acc[hh][e][i % NS] =
                                __builtin_fmaf(pr[hh][i], vv[e], acc[hh][e][i % NS]);
                }
            }
        }
        float *red = reinterpret_cast<float *>(k_t);  // [wave][head][HD]
        if (d0 < HD) {
#pragma unroll
            for (int hh = 0; hh < HPK; ++hh)
#pragma unroll
                for (int e = 0; e < C::DPL; ++e) {
                    float t = acc[hh][e][0];
#pragma unroll
                    for (int j = 1; j < NS; ++j) t += acc[hh][e][j];
                    red[(wave * HPK + hh) * HD + d0 + e] = t;
                }
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < C::DPL; ++e) o[e] = 0.0f;
        if (d0 < HD) {
#pragma unroll
            for (int w = 0; w < HPK; ++w)
#pragma unroll
                for (int e = 0; e < C::DPL; ++e) o[e] += red[(w * HPK + wave) * HD + d0 + e];
        }
    }

    // ---- 6. output (one chunk) or chunk partial (h: this wave's head) ----
    if (n_chunks == 1) {
        const float inv = 1.0f / l;
        if (d0 < HD)
#pragma unroll
            for (int e = 0; e < C::DPL; ++e) a.out[(size_t)h * HD + d0 + e] = o[e] * inv;
        return;
    }
    float *const part_ml = a.part + (size_t)a.n_heads * max_chunks * HD;
    {
        float *po = a.part + ((size_t)h * max_chunks + c) * HD;
        if (d0 < HD)
#pragma unroll
            for (int e = 0; e < C::DPL; ++e) st_part(po + d0 + e, o[e]);
        if (lane == 0) {
            float *pml = part_ml + ((size_t)h * max_chunks + c) * 2;
            st_part(pml, m);
            st_part(pml + 1, l);
        }
    }

    // ---- 7. arrival: the workgroup's partials are in memory, then one
    // increment of this kv head's counter; the last arriver merges ----
    __shared__ int last_s;
    drain();
    __syncthreads();
    if (tid == 0) {
        unsigned *cnt = a.cnt + 32 * g;
        const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old + 1 == (unsigned)n_chunks;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_s = last;
    }
    __syncthreads();
    if (!last_s) return;

    // ---- 8. merge of head h over the n_chunks partials (wave = head):
    // lane (slice sl, float4 column e4) takes chunks sl, sl + MSL, ...; the
    // (max, sum) pairs of chunks lane and lane + 64 and the first MB partial
    // rows are all requested before anything waits ----
    constexpr int MU = C::MU, MSL = C::MSL, MB = C::MB;
    const int e4 = lane % MU, sl = lane / MU;
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(a.part + (size_t)h * max_chunks * HD, (uint32_t)(n_chunks * HD * 4));
    const __amdgpu_buffer_rsrc_t rm =
        make_rsrc(part_ml + (size_t)h * max_chunks * 2, (uint32_t)(n_chunks * 8));
    // (the loads are read through bit casts to float vectors: element access
    // on the builtins' integer results does not give the loaded dwords)
    const float2 ml_a = ld_pair(rm, lane);
    const float2 ml_b = ld_pair(rm, lane + 64);
    // whole byte offsets in the vector offset, which the buffer range check
    // covers: rows past n_chunks read as zeros
    const uint32_t voff = (uint32_t)((sl * HD + 4 * e4) * 4);
    float4 v[MB];
#pragma unroll
    for (int u = 0; u < MB; ++u)
        v[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rp, voff + MSL * u * HD * 4, 0, kSc1));
    const float m_a = ml_a.x, l_a = ml_a.y, m_b = ml_b.x, l_b = ml_b.y;
    float mx = fmaxf(lane < n_chunks ? m_a : -INFINITY, lane + 64 < n_chunks ? m_b : -INFINITY);
    for (int cc = lane + 128; cc < n_chunks; cc += 64) {
        mx = fmaxf(mx, ld_pair(rm, cc).x);
    }
    const float M = wave_max(mx);
    float *wl = reinterpret_cast<float *>(lds) + wave * C::MAXC;  // tiles are no longer read
    float ls = 0.0f;
    if (lane < n_chunks) {
        const float f = expf(m_a - M);
        wl[lane] = f;
        ls = f * l_a;
    }
    if (lane + 64 < n_chunks) {
        const float f = expf(m_b - M);
        wl[lane + 64] = f;
        ls += f * l_b;
    }
    for (int cc = lane + 128; cc < n_chunks; cc += 64) {
        const float2 ml = ld_pair(rm, cc);
        const float f = expf(ml.x - M);
        wl[cc] = f;
        ls += f * ml.y;
    }
    const float L = wave_sum(ls);
    __syncthreads();  // the weights are in LDS
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto fold = [&](int cc, float4 x) {
        const float f = cc < n_chunks ? wl[cc] : 0.0f;
        acc.x = __builtin_fmaf(f, x.x, acc.x);
        acc.y = __builtin_fmaf(f, x.y, acc.y);
        acc.z = __builtin_fmaf(f, x.z, acc.z);
        acc.w = __builtin_fmaf(f, x.w, acc.w);
    };
#pragma unroll
    for (int u = 0; u < MB; ++u) fold(sl + MSL * u, v[u]);
    // chunks beyond the first round (long caches): rounds of 8 rows per lane
#pragma unroll 1
    for (int cc0 = MSL * MB; cc0 < n_chunks; cc0 += MSL * 8) {
        float4 t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            t[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rp, voff + (cc0 + MSL * u) * HD * 4, 0, kSc1));
#pragma unroll
        for (int u = 0; u < 8; ++u) fold(cc0 + sl + MSL * u, t[u]);
    }
    // combine the chunk slices (lanes e4 + MU * s) of each column
#pragma unroll
    for (int off = MU; off < 64; off <<= 1) {
        acc.x += __shfl_xor(acc.x, off);
        acc.y += __shfl_xor(acc.y, off);
        acc.z += __shfl_xor(acc.z, off);
        acc.w += __shfl_xor(acc.w, off);
    }
    if (sl == 0) {
        const float inv = 1.0f / L;
        *reinterpret_cast<float4 *>(a.out + (size_t)h * HD + 4 * e4) =
            make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    }
}

typedef void (*attn_fn)(cwi::AttnArgs, float, int);

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
    if (!pk.fn) {
        set_error("attention: unsupported head_dim=%d / heads per kv=%d", a.hd, hpk);
        return CW_ERR_ARG;
    }
    if (a.max_seq > kMaxChunkSpan) {
        set_error("attention: max_seq=%d exceeds %d", a.max_seq, kMaxChunkSpan);
        return CW_ERR_ARG;
    }
    if (a.n_kv > kMaxAttnKv) {
        set_error("attention: n_kv_heads=%d exceeds %d", a.n_kv, kMaxAttnKv);
        return CW_ERR_ARG;
    }
    CW_TRY(ensure_lds(pk.fn, pk.lds));
    const int max_chunks = (a.max_seq + pk.cp - 1) / pk.cp;
    AttnArgs b = a;
    b.cnt = ctx->attn_cnt;
    const float scale = powf((float)a.hd, -0.5f);
    prof_begin(ctx, "attention");
    hipLaunchKernelGGL(pk.fn, dim3(max_chunks, a.n_kv), dim3(pk.threads), pk.lds, ctx->stream, b,
                       scale, max_chunks);
    prof_end(ctx);
    return launch_check("attention");
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
