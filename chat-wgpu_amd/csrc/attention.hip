// Single-query GQA decode attention for gfx950.
//
// Replaces attention::attention (src/kernels/attention.rs:7-38,
// attention.wgsl:23-96).  Same mathematics: o_h = sum_j softmax_j(scale *
// q_h . k_j) v_j over j < seq, kv head = h / (n_heads / n_kv), scale =
// hd^-0.5, max-rescaled softmax.
//
// Split over the sequence (flash-decoding): a workgroup owns one kv head and a
// chunk of consecutive positions and writes one chunk partial (max, sum,
// unnormalised o per query head), unless the sequence fits one chunk, in
// which case it writes the normalised output.  The last workgroup of a kv head
// to finish (one agent-scope counter per kv head) merges that head group's
// partials in the same launch (merge_chunks), so the merge costs no kernel
// boundary.  Three kernels, by cache type and head size:
//   * attn_mfma_kernel (f16 cache, head_dim 128: the 8B decode workload):
//     waves of 16 positions with K and V in registers as loaded; scores and
//     P.V on the matrix cores with exact f16 operands (K, V as stored; q and
//     p split into f16 hi + lo), the W wave partials merged in LDS;
//   * attn_wave_kernel (f32 cache, head_dim 128): the same wave split with
//     scores and P.V on the vector ALUs;
//   * attn_kernel (other head sizes): K/V tiles in LDS, lane = position for
//     the scores, lane = dimension for P.V.
// Every kernel issues its global loads as straight-line code in the order
// they are used, and synchronises the workgroup on LDS data only while K/V
// rows are in flight: a __syncthreads fence, or a load under a branch,
// makes the compiler wait for every outstanding load first.
//
// Coherence across the 8 XCDs (one L2 each): partials are written with
// write-through (agent-scope, sc1) stores and read with sc1 loads, which miss
// any line an L2 still holds from an earlier call.  Every wave waits for its
// own partial stores to be acknowledged (s_waitcnt vmcnt(0): an acknowledged
// sc1 store has reached the memory side, where every XCD reads), then the
// workgroup barrier, then one agent-scope atomic increment; the merging
// workgroup's sc1 loads are issued only after its own increment returned the
// final count, so they observe every partial.  The merger resets the counter,
// so every launch, eager or replayed from a graph, starts from zero.
//
// Fused prologue (decode step): the raw q/k/v come straight from the fused
// QKV projection; the kernel applies the per-head QK RMSNorm (norm.wgsl,
// qwen3.rs:154-155) and RoPE (rope.wgsl), and the workgroup whose chunk holds
// the new position writes k/v into the cache (cache.rs:21-24) and uses them
// in place of what its loads read there.

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

// LDS written by some lanes of this wave is read by others: DS operations of
// one wave execute in order, so keeping the compiler from moving the accesses
// across this point (and waiting for the writes) is enough
__device__ __forceinline__ void wave_lds_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
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

// Merge of query head h over its n_chunks chunk partials (one wave): the
// (max, sum) pairs of chunks lane and lane + 64 and the first MB partial rows
// are all requested before anything waits; lane (slice sl, float4 column e4)
// takes chunks sl, sl + MSL, ...  Partials are read with sc1 loads (past any
// L2 line an earlier call left); wl is this wave's own LDS row of MAXC chunk
// weights, so only a wave-level fence orders its writes and reads.
template <int HD, int MAXC>
__device__ __forceinline__ void merge_chunks(const cwi::AttnArgs &a, int h, int n_chunks,
                                             int max_chunks, float *wl, int lane) {
    constexpr int MU = HD / 4;        // float4 columns per partial row
    constexpr int MSL = 64 / MU;      // chunk slices per wave
    // partial rows in flight per lane: one round covers MSL * MB chunks (36 at
    // head_dim 128), at most 18 float4 registers
    constexpr int MB0 = 36 / MSL > 4 ? 36 / MSL : 4;
    constexpr int MB = MB0 < 18 ? MB0 : 18;
    float *const part_ml = a.part + (size_t)a.n_heads * max_chunks * HD;
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
    for (int cc = lane + 128; cc < n_chunks; cc += 64) mx = fmaxf(mx, ld_pair(rm, cc).x);
    const float M = wave_max(mx);
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
    wave_lds_sync();  // the weights are in LDS
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
    // a device-resident position past the cache (the host bounds the
    // position it tracks; this covers a state it could not see): no KV
    // row is written and nothing past the cache is read
    if (seq < 1 || seq > a.max_seq) return;
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

    // ---- 8. merge of head h over the n_chunks partials (wave = head) ----
    merge_chunks<HD, C::MAXC>(a, h, n_chunks, max_chunks,
                              reinterpret_cast<float *>(lds) + wave * C::MAXC, lane);
}

// ---------------------------------------------------------------- head_dim 128

// Decode attention for head_dim 128 with the K/V rows kept in registers as
// they were loaded: workgroup (chunk c, kv head g) has W waves, wave w owns
// the PW positions c*CP + PW*w ... (PW = 16, or 8 for small caches).  A
// lane holds, for NR rows of its slice, one 16-byte unit of the row (EPU
// elements): the loads are plain coalesced row reads, and no LDS tile or
// workgroup barrier sits between a wave's data arriving and its compute, so
// each wave computes as soon as its own rows are in.
//   scores: per (row, head) a partial dot over the lane's EPU dims, summed
//     over the U4_ROW lanes of the row with DPP (every lane gets the sum);
//   softmax: per head over the wave's PW positions;
//   P.V: the lane's rows times their p, summed over the row groups;
// the W wave partials meet in LDS; the workgroup writes one chunk partial
// (or the output, for a single chunk) and the last workgroup of the kv head
// merges the chunks (merge_chunks).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// sum over aligned groups of G lanes (16 or 32); every lane gets its group's sum
template <int G>
__device__ __forceinline__ float row_group_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    if constexpr (G >= 32) v += __shfl_xor(v, 16);
    return v;
}

template <typename KVT, int HPK, int W, int PW_ = 16>
struct WaveCfg {
    static constexpr int HD = 128;
    static constexpr int HALF = HD / 2;             // = 64: one (lo, hi) pair per lane
    static constexpr int ES = (int)sizeof(KVT);
    static constexpr int EPU = 16 / ES;             // elements per 16-byte unit
    static constexpr int U4_ROW = HD / EPU;         // lanes per row: 16 (f16), 32 (f32)
    static constexpr int RPL = 64 / U4_ROW;         // rows per wave load
    static constexpr int PW = PW_;                  // positions per wave (16 or 8)
    static constexpr int NR = PW / RPL;             // rows per lane
    static constexpr int CP = PW * W;               // positions per workgroup
    static constexpr int THREADS = 64 * W;
    static constexpr int ROWB = HD * ES;
    static constexpr int MAXC = kMaxChunkSpan / CP;
    // LDS (floats): q [HPK][HD]; the new k and v [2][HD]; the wave partials
    // [W][HPK][HD + 2], whose space the chunk merge's weights [HPK][MAXC] reuse
    static constexpr int Q_F = HPK * HD;
    static constexpr int NEW_F = 2 * HD;
    static constexpr int WP_F = W * HPK * (HD + 2);
    static constexpr int CW_F = HPK * MAXC;
    static constexpr int LDS = (Q_F + NEW_F + (WP_F > CW_F ? WP_F : CW_F)) * 4;
    static_assert(W >= HPK, "the chunk merge takes one wave per query head");
    static_assert(LDS <= 64 * 1024, "attention LDS");
};

// EPU elements of a 16-byte unit as f32
template <typename KVT>
__device__ __forceinline__ void unpack16(uint4 w, float *out);
template <>
__device__ __forceinline__ void unpack16<_Float16>(uint4 w, float *out) {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v h = __builtin_bit_cast(half2v, d[i]);
        out[2 * i] = (float)h.x;
        out[2 * i + 1] = (float)h.y;
    }
}
template <>
__device__ __forceinline__ void unpack16<float>(uint4 w, float *out) {
    out[0] = __builtin_bit_cast(float, w.x);
    out[1] = __builtin_bit_cast(float, w.y);
    out[2] = __builtin_bit_cast(float, w.z);
    out[3] = __builtin_bit_cast(float, w.w);
}

// EPU f32 values (exactly representable in KVT) packed into a 16-byte unit
template <typename KVT>
__device__ __forceinline__ uint4 pack16(const float *v);
template <>
__device__ __forceinline__ uint4 pack16<_Float16>(const float *v) {
    uint32_t d[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        half2v h;
        h.x = (_Float16)v[2 * i];
        h.y = (_Float16)v[2 * i + 1];
        d[i] = __builtin_bit_cast(uint32_t, h);
    }
    return make_uint4(d[0], d[1], d[2], d[3]);
}
template <>
__device__ __forceinline__ uint4 pack16<float>(const float *v) {
    return make_uint4(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                      __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3]));
}

// workgroup barrier for LDS data only: the LDS writes are waited for, but not
// the global loads still in flight (a __syncthreads fence would wait for those
// too, so no wave could compute while its K/V rows arrive)
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <typename KVT, int HPK, int W, bool FUSED, int PW = 16>
__global__ __launch_bounds__(64 * W) void attn_wave_kernel(cwi::AttnArgs a, float scale,
                                                           int max_chunks) {
    using C = WaveCfg<KVT, HPK, W, PW>;
    constexpr int HD = C::HD, HALF = C::HALF, EPU = C::EPU, NR = C::NR;
    extern __shared__ float lds_f[];
    float *q_s = lds_f;              // [HPK][HD]
    float *new_s = q_s + C::Q_F;     // new k [HD], new v [HD]
    float *wp = new_s + C::NEW_F;    // [W][HPK][HD + 2]

    const int c = blockIdx.x, g = blockIdx.y;
    const int seq = a.pos_dev ? (*a.pos_dev + 1) : a.seq;
    // a device-resident position past the cache (the host bounds the
    // position it tracks; this covers a state it could not see): no KV
    // row is written and nothing past the cache is read
    if (seq < 1 || seq > a.max_seq) return;
    const int c0 = c * C::CP;
    if (c0 >= seq) return;
    const int n_chunks = (seq + C::CP - 1) / C::CP;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kv_dim = a.n_kv * HD;
    const int pos_new = seq - 1;
    const int w0 = c0 + wave * C::PW;  // this wave's first position
    const bool live = w0 < seq;        // (wave-uniform, like w_new)
    const bool w_new = FUSED && pos_new >= w0 && pos_new < w0 + C::PW;
    unsigned char *kc = reinterpret_cast<unsigned char *>(a.k_cache);
    unsigned char *vc = reinterpret_cast<unsigned char *>(a.v_cache);
    const size_t row_bytes = (size_t)kv_dim * C::ES;
    const int rg = lane / C::U4_ROW, u = lane % C::U4_ROW;  // row of a load, unit of the row

    // ---- 1. loads, all of them straight-line (a load under a branch makes
    // the compiler wait for every load at the join), in the order they are
    // used: a query head (head g*HPK + wave, clamped; only waves below HPK
    // use it), the new k and v and their RoPE row (used by the wave holding
    // pos_new), then this wave's K rows and V rows (rows past the sequence
    // clamped to its last row and masked later).  Issuing the rows before
    // the position is read, as the f16 kernel does, measured slower here
    // (Qwen3-0.6B-shape token loop, f32 cache of 160 positions: 1405-1419
    // against 1425-1437 tokens/s) ----
    const int h = g * HPK + (wave < HPK ? wave : HPK - 1);
    const bool q_wave = wave < HPK;
    // a wave that does not use a vector still issues its load, over a buffer
    // range of 0 bytes: no memory request, zeros back, straight-line code
    auto rs = [](const float *p, bool use) {
        return make_rsrc(p, use ? (uint32_t)(HD * sizeof(float)) : 0u);
    };
    auto ld2 = [&](__amdgpu_buffer_rsrc_t r, float &x0, float &x1) {
        x0 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, 0, 0));
        x1 = __builtin_bit_cast(float,
                                __builtin_amdgcn_raw_buffer_load_b32(r, (lane + HALF) * 4, 0, 0));
    };
    float lo, hi, gl = 0.f, gh = 0.f, cs = 0.f, sn = 0.f;
    float klo = 0.f, khi = 0.f, kgl = 0.f, kgh = 0.f, v0 = 0.f, v1 = 0.f;
    if constexpr (FUSED) {
        const int q_dim = a.n_heads * HD;
        const float *ks = a.qkv + q_dim + g * HD;
        ld2(rs(a.qkv + (size_t)h * HD, q_wave), lo, hi);
        ld2(rs(a.q_norm_w, q_wave), gl, gh);
        // the RoPE row of pos_new as [cos (64) | sin (64)] through two ranges
        const __amdgpu_buffer_rsrc_t rc =
            make_rsrc(a.cos_t + (size_t)pos_new * HALF, (q_wave || w_new) ? HALF * 4 : 0u);
        const __amdgpu_buffer_rsrc_t rsn =
            make_rsrc(a.sin_t + (size_t)pos_new * HALF, (q_wave || w_new) ? HALF * 4 : 0u);
        cs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rc, lane * 4, 0, 0));
        sn = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsn, lane * 4, 0, 0));
        ld2(rs(ks, w_new), klo, khi);
        ld2(rs(a.k_norm_w, w_new), kgl, kgh);
        ld2(rs(ks + kv_dim, w_new), v0, v1);
    } else {
        ld2(rs(a.q + (size_t)h * HD, q_wave), lo, hi);
    }
    // keep the issue order: the scheduler would otherwise sink the small
    // loads below the rows, and waiting for them would wait for the rows too
    __builtin_amdgcn_sched_barrier(0);
    uint4 kr[NR], vr[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        int p = w0 + i * C::RPL + rg;
        p = p < seq ? p : seq - 1;
        const size_t off = (size_t)p * row_bytes + (size_t)g * C::ROWB + (size_t)u * 16;
        kr[i] = *reinterpret_cast<const uint4 *>(kc + off);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        int p = w0 + i * C::RPL + rg;
        p = p < seq ? p : seq - 1;
        const size_t off = (size_t)p * row_bytes + (size_t)g * C::ROWB + (size_t)u * 16;
        vr[i] = *reinterpret_cast<const uint4 *>(vc + off);
    }

    // ---- 2. query head of waves below HPK (normalised + rotated when fused) ----
    if (wave < HPK) {
        float r0 = lo, r1 = hi;
        if constexpr (FUSED) {
            const float ss = wave_sum(lo * lo + hi * hi);
            const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
            const float l0 = (lo * inv) * gl;
            const float h0 = (hi * inv) * gh;
            r0 = l0 * cs - h0 * sn;
            r1 = h0 * cs + l0 * sn;
            if (a.q_tap && c == 0) {  // the "q" tap (qwen3.rs:165)
                a.q_tap[(size_t)h * HD + lane] = r0;
                a.q_tap[(size_t)h * HD + lane + HALF] = r1;
            }
        }
        q_s[wave * HD + lane] = r0;
        q_s[wave * HD + lane + HALF] = r1;
    }

    // ---- 3. the new position's k (normalised + rotated) and v: to the cache
    // (cache.rs:21-24) and to LDS, from where the lanes holding that row take
    // them in place of what their loads read ----
    if (w_new) {
        const float kss = wave_sum(klo * klo + khi * khi);
        const float kinv = 1.0f / sqrtf(kss / (float)HD + a.eps);
        const float l0 = (klo * kinv) * kgl;
        const float h0 = (khi * kinv) * kgh;
        const KVT k0 = to_kv<KVT>(l0 * cs - h0 * sn), k1 = to_kv<KVT>(h0 * cs + l0 * sn);
        const KVT vv0 = to_kv<KVT>(v0), vv1 = to_kv<KVT>(v1);
        KVT *kg = reinterpret_cast<KVT *>(kc + (size_t)pos_new * row_bytes + (size_t)g * C::ROWB);
        KVT *vg = reinterpret_cast<KVT *>(vc + (size_t)pos_new * row_bytes + (size_t)g * C::ROWB);
        kg[lane] = k0;
        kg[lane + HALF] = k1;
        vg[lane] = vv0;
        vg[lane + HALF] = vv1;
        new_s[lane] = (float)k0;
        new_s[lane + HALF] = (float)k1;
        new_s[HD + lane] = (float)vv0;
        new_s[HD + lane + HALF] = (float)vv1;
    }
    lds_barrier();  // q (and the new row) are in LDS
    if (w_new) {
        float kn[EPU], vn[EPU];
#pragma unroll
        for (int e = 0; e < EPU; ++e) {
            kn[e] = new_s[u * EPU + e];
            vn[e] = new_s[HD + u * EPU + e];
        }
        const uint4 kp = pack16<KVT>(kn), vp = pack16<KVT>(vn);
        const int r = pos_new - w0;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const bool mine = i * C::RPL + rg == r;
            kr[i].x = mine ? kp.x : kr[i].x;
            kr[i].y = mine ? kp.y : kr[i].y;
            kr[i].z = mine ? kp.z : kr[i].z;
            kr[i].w = mine ? kp.w : kr[i].w;
            vr[i].x = mine ? vp.x : vr[i].x;
            vr[i].y = mine ? vp.y : vr[i].y;
            vr[i].z = mine ? vp.z : vr[i].z;
            vr[i].w = mine ? vp.w : vr[i].w;
        }
    }

    float o[HPK][EPU], m[HPK], l[HPK];
    if (live) {
        // ---- 4. scores: partial dots over the lane's EPU dims, summed over
        // the U4_ROW lanes of each row ----
        float sc[NR][HPK];
#pragma unroll
        for (int hh = 0; hh < HPK; ++hh) {
            float qv[EPU];
#pragma unroll
            for (int e = 0; e < EPU; e += 4) {
                const float4 q4 = *reinterpret_cast<const float4 *>(q_s + hh * HD + u * EPU + e);
                qv[e] = q4.x;
                qv[e + 1] = q4.y;
                qv[e + 2] = q4.z;
                qv[e + 3] = q4.w;
            }
#pragma unroll
            for (int i = 0; i < NR; ++i) sc[i][hh] = dot16<KVT>(kr[i], qv, 0.0f);
        }
#pragma unroll
        for (int i = 0; i < NR; ++i)
#pragma unroll
            for (int hh = 0; hh < HPK; ++hh) sc[i][hh] = row_group_sum<C::U4_ROW>(sc[i][hh]);

        // ---- 5. softmax partial per head over the wave's positions ----
#pragma unroll
        for (int hh = 0; hh < HPK; ++hh) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const bool in = w0 + i * C::RPL + rg < seq;
                sc[i][hh] = in ? sc[i][hh] * scale : -INFINITY;
                mx = fmaxf(mx, sc[i][hh]);
            }
#pragma unroll
            for (int off = C::U4_ROW; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
            float ls = 0.0f;
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const float pr = sc[i][hh] == -INFINITY ? 0.0f : expf(sc[i][hh] - mx);
                sc[i][hh] = pr;
                ls += pr;
            }
#pragma unroll
            for (int off = C::U4_ROW; off < 64; off <<= 1) ls += __shfl_xor(ls, off);
            m[hh] = mx;
            l[hh] = ls;
        }

        // ---- 6. P.V over the lane's rows, summed over the row groups.  Rows
        // at or past the sequence were clamped to its last row, pos_new when
        // fused, whose loaded value is the cache's old one (this launch
        // writes the row): zero them, so their zero weights add exactly zero
        // whatever that was (0 * inf is not 0) ----
#pragma unroll
        for (int i = 0; i < NR; ++i)
            if (w0 + i * C::RPL + rg >= seq) vr[i] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int hh = 0; hh < HPK; ++hh)
#pragma unroll
            for (int e = 0; e < EPU; ++e) o[hh][e] = 0.0f;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            float vv[EPU];
            unpack16<KVT>(vr[i], vv);
#pragma unroll
            for (int hh = 0; hh < HPK; ++hh)
#pragma unroll
                for (int e = 0; e < EPU; ++e) o[hh][e] = __builtin_fmaf(sc[i][hh], vv[e], o[hh][e]);
        }
#pragma unroll
        for (int off = C::U4_ROW; off < 64; off <<= 1)
#pragma unroll
            for (int hh = 0; hh < HPK; ++hh)
#pragma unroll
                for (int e = 0; e < EPU; ++e) o[hh][e] += __shfl_xor(o[hh][e], off);
    } else {
#pragma unroll
        for (int hh = 0; hh < HPK; ++hh) {
            m[hh] = -INFINITY;
            l[hh] = 0.0f;
#pragma unroll
            for (int e = 0; e < EPU; ++e) o[hh][e] = 0.0f;
        }
    }

    // ---- 7. the wave's partial (o, m, l) per head into LDS ----
    if (rg == 0) {
#pragma unroll
        for (int hh = 0; hh < HPK; ++hh) {
            float *dst = wp + (wave * HPK + hh) * (HD + 2);
#pragma unroll
            for (int e = 0; e < EPU; ++e) dst[u * EPU + e] = o[hh][e];
            if (u == 0) {
                dst[HD] = m[hh];
                dst[HD + 1] = l[hh];
            }
        }
    }
    __syncthreads();

    // ---- 8. merge of the W wave partials: thread -> (head, dim); the chunk
    // partial goes to memory write-through, or the output when the sequence
    // is one chunk ----
    float *const part_ml = a.part + (size_t)a.n_heads * max_chunks * HD;
    for (int idx = tid; idx < HPK * HD; idx += C::THREADS) {
        const int hh = idx / HD, d = idx % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, wp[(w * HPK + hh) * (HD + 2) + HD]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float *src = wp + (w * HPK + hh) * (HD + 2);
            const float f = src[HD] == -INFINITY ? 0.0f : expf(src[HD] - M);
            L = __builtin_fmaf(f, src[HD + 1], L);
            O = __builtin_fmaf(f, src[d], O);
        }
        const int hg = g * HPK + hh;
        if (n_chunks == 1) {
            a.out[(size_t)hg * HD + d] = O / L;
        } else {
            st_part(a.part + ((size_t)hg * max_chunks + c) * HD + d, O);
            if (d == 0) {
                float *pml = part_ml + ((size_t)hg * max_chunks + c) * 2;
                st_part(pml, M);
                st_part(pml + 1, L);
            }
        }
    }
    if (n_chunks == 1) return;

    // ---- 9. arrival: every wave's partial stores are complete (s_waitcnt),
    // then one increment of this kv head's counter; the last arriver merges
    // the chunks, one wave per query head ----
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
    if (wave < HPK)
        merge_chunks<HD, C::MAXC>(a, g * HPK + wave, n_chunks, max_chunks, wp + wave * C::MAXC,
                                  lane);
}

// ---------------------------------------------------------------- f16 cache, head_dim 128: scores on MFMA

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Workgroup (chunk c, kv head g) with W waves (W = blockDim / 64, a launch
// choice), wave w owning the 16 positions c*16W + 16w ...  Per wave:
//   scores S^T[key][head] = K q^T on v_mfma_f32_16x16x32_f16: lane l holds
//     A[l % 16][8 (l / 16) + j] and B[8 (l / 16) + j][l % 16] and receives
//     D[4 (l / 16) + r][l % 16].  A is K row l % 16 (the wave's key), B is
//     q^T (column = query head, HPK of 16 used).  The k order only has to
//     agree between A and B, so in step t lane l takes dims 32 (l / 16) + 8t
//     .. + 8: its four steps read 64 contiguous bytes of its key row.  K is
//     f16 in the cache and enters exactly; q is split into f16 hi + lo (two
//     MFMAs per step), so the products are those of f32 q to ~22 bits, summed
//     in f32;
//   softmax per head over the 16 keys on the lanes holding that head's
//     column; p goes through a 16 x HPK LDS tile of the wave;
//   P.V on the vector ALUs: V rows in their natural layout (lane = 16-byte
//     unit of a row, row group = l / 16), summed over the row groups.
// The W wave partials merge in LDS, the chunk partial goes to memory (or
// the output for a single chunk), and the last workgroup of the kv head
// merges the chunks (merge_chunks).
template <int HPK>
struct MfmaCfg {
    static constexpr int HD = 128, HALF = 64;
    // waves per workgroup at most (8 for 8-head groups, whose accumulators
    // need the registers of 2 waves per SIMD)
    static constexpr int WMAX = HPK >= 8 ? 8 : 16;
    static constexpr int PW = 16;                   // positions per wave
    static constexpr int ROWB = HD * 2;             // f16 row slice of one kv head
    static constexpr int MAXC = kMaxChunkSpan / (PW * HPK);  // chunks at the smallest W = HPK
    // LDS (bytes): q hi/lo f16 [2][HPK][HD]; new k, v f32 [2][HD]; p per wave
    // f32 [WMAX][16][HPK]; wave partials f32 [WMAX][HPK][HD + 2], reused for
    // the chunk weights [HPK][MAXC]
    static constexpr int Q16_B = 2 * HPK * HD * 2;
    static constexpr int NEW_B = 2 * HD * 4;
    static constexpr int P_B = WMAX * PW * HPK * 4;
    static constexpr int WP_B0 = WMAX * HPK * (HD + 2) * 4;
    static constexpr int CW_B = HPK * MAXC * 4;
    static constexpr int WP_B = WP_B0 > CW_B ? WP_B0 : CW_B;
    static constexpr int LDS = Q16_B + NEW_B + P_B + WP_B;
    static_assert(LDS <= 160 * 1024, "attention LDS");
    static_assert(HPK <= 16, "query heads of a kv head fit the MFMA columns");
};

template <int HPK, bool FUSED>
__global__ __launch_bounds__(64 * MfmaCfg<HPK>::WMAX) void attn_mfma_kernel(cwi::AttnArgs a,
                                                                             float scale,
                                                                             int max_chunks) {
    using C = MfmaCfg<HPK>;
    constexpr int HD = C::HD, HALF = C::HALF;
    extern __shared__ float4 lds_mf[];
    unsigned char *lds = reinterpret_cast<unsigned char *>(lds_mf);
    _Float16 *q16 = reinterpret_cast<_Float16 *>(lds);              // [2][HPK][HD]
    float *new_s = reinterpret_cast<float *>(lds + C::Q16_B);       // [2][HD]
    float *p_all = reinterpret_cast<float *>(lds + C::Q16_B + C::NEW_B);  // [WMAX][16][HPK]
    float *wp = reinterpret_cast<float *>(lds + C::Q16_B + C::NEW_B + C::P_B);

    const int W = blockDim.x >> 6;
    const int CP = C::PW * W;
    const int c = blockIdx.x, g = blockIdx.y;
    const int c0 = c * CP;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kv_dim = a.n_kv * HD;
    const int w0 = c0 + wave * C::PW;  // this wave's first position
    unsigned char *kc = reinterpret_cast<unsigned char *>(a.k_cache);
    unsigned char *vc = reinterpret_cast<unsigned char *>(a.v_cache);
    const size_t row_bytes = (size_t)kv_dim * 2;
    const int lg = lane >> 4, li = lane & 15;  // lane group, lane in group

    // ---- 1. loads, straight-line (see attn_wave_kernel).  First the K rows
    // in the MFMA A layout (key li, bytes 64 lg + 16 t) and the V rows in
    // their natural layout (rows 4 i + lg, 16-byte unit li): their addresses
    // do not depend on the device-resident position, so they are in flight
    // while it is read (rows past the cache clamp to its last row; rows at
    // or past the sequence are masked once it is known).  Then the position,
    // and in the order they are used a query head (waves below HPK) and the
    // new k and v with their RoPE row (the wave holding pos_new) ----
    uint4 kr[4], vr[4];
    {
        int p = w0 + li;
        p = p < a.max_seq ? p : a.max_seq - 1;
        const unsigned char *src = kc + (size_t)p * row_bytes + (size_t)g * C::ROWB + lg * 64;
#pragma unroll
        for (int t = 0; t < 4; ++t) kr[t] = *reinterpret_cast<const uint4 *>(src + 16 * t);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int p = w0 + 4 * i + lg;
        p = p < a.max_seq ? p : a.max_seq - 1;
        vr[i] = *reinterpret_cast<const uint4 *>(vc + (size_t)p * row_bytes +
                                                (size_t)g * C::ROWB + (size_t)li * 16);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int seq = a.pos_dev ? (*a.pos_dev + 1) : a.seq;
    // a device-resident position past the cache (the host bounds the
    // position it tracks; this covers a state it could not see): no KV
    // row is written and nothing past the cache is read
    if (seq < 1 || seq > a.max_seq) return;
    if (c0 >= seq) return;
    const int n_chunks = (seq + CP - 1) / CP;
    const int pos_new = seq - 1;
    const bool live = w0 < seq;  // (wave-uniform, like w_new)
    const bool w_new = FUSED && pos_new >= w0 && pos_new < w0 + C::PW;
    const int h = g * HPK + (wave < HPK ? wave : HPK - 1);
    const bool q_wave = wave < HPK;
    auto rs = [](const float *p, bool use) {
        return make_rsrc(p, use ? (uint32_t)(HD * sizeof(float)) : 0u);
    };
    auto ld2 = [&](__amdgpu_buffer_rsrc_t r, float &x0, float &x1) {
        x0 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, 0, 0));
        x1 = __builtin_bit_cast(float,
                                __builtin_amdgcn_raw_buffer_load_b32(r, (lane + HALF) * 4, 0, 0));
    };
    float lo, hi, gl = 0.f, gh = 0.f, cs = 0.f, sn = 0.f;
    float klo = 0.f, khi = 0.f, kgl = 0.f, kgh = 0.f, v0 = 0.f, v1 = 0.f;
    if constexpr (FUSED) {
        const int q_dim = a.n_heads * HD;
        const float *ks = a.qkv + q_dim + g * HD;
        ld2(rs(a.qkv + (size_t)h * HD, q_wave), lo, hi);
        ld2(rs(a.q_norm_w, q_wave), gl, gh);
        const __amdgpu_buffer_rsrc_t rc =
            make_rsrc(a.cos_t + (size_t)pos_new * HALF, (q_wave || w_new) ? HALF * 4 : 0u);
        const __amdgpu_buffer_rsrc_t rsn =
            make_rsrc(a.sin_t + (size_t)pos_new * HALF, (q_wave || w_new) ? HALF * 4 : 0u);
        cs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rc, lane * 4, 0, 0));
        sn = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsn, lane * 4, 0, 0));
        ld2(rs(ks, w_new), klo, khi);
        ld2(rs(a.k_norm_w, w_new), kgl, kgh);
        ld2(rs(ks + kv_dim, w_new), v0, v1);
    } else {
        ld2(rs(a.q + (size_t)h * HD, q_wave), lo, hi);
    }
    // V rows at or past the sequence hold whatever the cache holds there
    // (zeros, or rows of an earlier sequence): zero them, so their zero
    // weights add exactly zero whatever those rows were (0 * inf is not 0).
    // Their scores are masked by position below.
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (w0 + 4 * i + lg >= seq) vr[i] = make_uint4(0u, 0u, 0u, 0u);

    // ---- 2. query head of waves below HPK (normalised + rotated when
    // fused), into LDS as f16 hi and lo parts ----
    if (q_wave) {
        float r0 = lo, r1 = hi;
        if constexpr (FUSED) {
            const float ss = wave_sum(lo * lo + hi * hi);
            const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
            const float l0 = (lo * inv) * gl;
            const float h0 = (hi * inv) * gh;
            r0 = l0 * cs - h0 * sn;
            r1 = h0 * cs + l0 * sn;
            if (a.q_tap && c == 0) {  // the "q" tap (qwen3.rs:165)
                a.q_tap[(size_t)h * HD + lane] = r0;
                a.q_tap[(size_t)h * HD + lane + HALF] = r1;
            }
        }
        const _Float16 a0 = (_Float16)r0, a1 = (_Float16)r1;
        q16[wave * HD + lane] = a0;
        q16[wave * HD + lane + HALF] = a1;
        q16[(HPK + wave) * HD + lane] = (_Float16)(r0 - (float)a0);
        q16[(HPK + wave) * HD + lane + HALF] = (_Float16)(r1 - (float)a1);
    }

    // ---- 3. the new position's k (normalised + rotated) and v: to the cache
    // and to LDS, from where the lanes holding that row take them ----
    if (w_new) {
        const float kss = wave_sum(klo * klo + khi * khi);
        const float kinv = 1.0f / sqrtf(kss / (float)HD + a.eps);
        const float l0 = (klo * kinv) * kgl;
        const float h0 = (khi * kinv) * kgh;
        const _Float16 k0 = (_Float16)(l0 * cs - h0 * sn), k1 = (_Float16)(h0 * cs + l0 * sn);
        const _Float16 vv0 = (_Float16)v0, vv1 = (_Float16)v1;
        _Float16 *kg = reinterpret_cast<_Float16 *>(kc + (size_t)pos_new * row_bytes + (size_t)g * C::ROWB);
        _Float16 *vg = reinterpret_cast<_Float16 *>(vc + (size_t)pos_new * row_bytes + (size_t)g * C::ROWB);
        kg[lane] = k0;
        kg[lane + HALF] = k1;
        vg[lane] = vv0;
        vg[lane + HALF] = vv1;
        new_s[lane] = (float)k0;
        new_s[lane + HALF] = (float)k1;
        new_s[HD + lane] = (float)vv0;
        new_s[HD + lane + HALF] = (float)vv1;
    }
    lds_barrier();  // q (and the new row) are in LDS
    if (w_new) {
        const int r = pos_new - w0;
        if (li == r) {  // K in the A layout: this lane holds key r, dims 32 lg + 8 t ..
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float kn[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) kn[e] = new_s[32 * lg + 8 * t + e];
                kr[t] = pack16<_Float16>(kn);
            }
        }
        float vn[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vn[e] = new_s[HD + li * 8 + e];
        const uint4 vp = pack16<_Float16>(vn);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool mine = 4 * i + lg == r;
            vr[i].x = mine ? vp.x : vr[i].x;
            vr[i].y = mine ? vp.y : vr[i].y;
            vr[i].z = mine ? vp.z : vr[i].z;
            vr[i].w = mine ? vp.w : vr[i].w;
        }
    }

    // od[t][r]: o of head 4 lg + r at dim 8 li + t (lane groups past the
    // heads hold zeros)
    f32x4 od[8];
    float m[HPK], l[HPK];
    if (live) {
        // ---- 4. scores S^T[key 4 lg + r][head li] ----
        f16x8 qb[4][2];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                f16x8 z = {};
                if (li < HPK)
                    z = *reinterpret_cast<const f16x8 *>(q16 + (part * HPK + li) * HD + 32 * lg + 8 * t);
                qb[t][part] = z;
            }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const f16x8 ka = __builtin_bit_cast(f16x8, kr[t]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[t][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[t][1], acc, 0, 0, 0);
        }

        // ---- 5. softmax partial per head (lanes li < HPK hold head li's
        // column: keys 4 lg + r) ----
        float sv[4], mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool in = w0 + 4 * lg + r < seq;
            sv[r] = in ? acc[r] * scale : -INFINITY;
            mx = fmaxf(mx, sv[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        float ls = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sv[r] = sv[r] == -INFINITY ? 0.0f : expf(sv[r] - mx);
            ls += sv[r];
        }
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        float *pw = p_all + wave * (C::PW * HPK);  // [key][head]
        if (li < HPK) {
#pragma unroll
            for (int r = 0; r < 4; ++r) pw[(4 * lg + r) * HPK + li] = sv[r];
        }
        // every lane needs (m, l) of every head: lane hh of group 0 holds head hh
#pragma unroll
        for (int hh = 0; hh < HPK; ++hh) {
            m[hh] = __shfl(mx, hh);
            l[hh] = __shfl(ls, hh);
        }
        wave_lds_sync();

        // ---- 6. P.V on v_mfma_f32_16x16x16_f16 (lane l holds A[l % 16][4 (l / 16)
        // + j], B[4 (l / 16) + j][l % 16], receives D[4 (l / 16) + r][l % 16]).
        // The key order of k slot 4 lg + j is key 4 j + lg, which is V row j of
        // this lane; output column li of MFMA t is dim 8 li + t, element t of
        // this lane's unit.  So B comes straight from the V registers, A is p
        // of head li (f16 hi + lo), and lanes 0..15 receive o[head r][dim
        // 8 li + t]: the sum over all 16 keys, with no cross-lane reduction ----
        f16x4 pa[2];
        {
            float pv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) pv[j] = li < HPK ? pw[(4 * j + lg) * HPK + li] : 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const _Float16 hi16 = (_Float16)pv[j];
                pa[0][j] = hi16;
                pa[1][j] = (_Float16)(pv[j] - (float)hi16);
            }
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            f16x4 vb;
#pragma unroll
            for (int j = 0; j < 4; ++j) vb[j] = __builtin_bit_cast(f16x8, vr[j])[t];
            f32x4 z = {0.f, 0.f, 0.f, 0.f};
            z = __builtin_amdgcn_mfma_f32_16x16x16f16(pa[0], vb, z, 0, 0, 0);
            od[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa[1], vb, z, 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int hh = 0; hh < HPK; ++hh) {
            m[hh] = -INFINITY;
            l[hh] = 0.0f;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) od[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // ---- 7. the wave's partial (o, m, l) per head into LDS: lane group lg
    // holds heads 4 lg .. 4 lg + 3 ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int hh = 4 * lg + r;
        if (hh < HPK) {
            float *dst = wp + (wave * HPK + hh) * (HD + 2);
#pragma unroll
            for (int t = 0; t < 8; ++t) dst[8 * li + t] = od[t][r];
        }
    }
    if (lane < HPK) {
        float *dst = wp + (wave * HPK + lane) * (HD + 2);
        float mm = m[0], ll = l[0];
#pragma unroll
        for (int hh = 1; hh < HPK; ++hh) {
            mm = lane == hh ? m[hh] : mm;
            ll = lane == hh ? l[hh] : ll;
        }
        dst[HD] = mm;
        dst[HD + 1] = ll;
    }
    __syncthreads();

    // ---- 8. merge of the W wave partials: the W x HPK weights exp(m_w - M)
    // once (one lane each, into the p tiles' space), then thread -> (head,
    // dim) sums; the chunk partial goes to memory write-through, or the
    // output for one chunk ----
    float *fac = p_all;             // [W][HPK] weights
    float *fl = p_all + W * HPK;    // [W][HPK] weight * l
    if (tid < W * HPK) {
        const int w = tid / HPK, hh = tid % HPK;
        float M = -INFINITY;
        for (int v = 0; v < W; ++v) M = fmaxf(M, wp[(v * HPK + hh) * (HD + 2) + HD]);
        const float *src = wp + (w * HPK + hh) * (HD + 2);
        const float f = src[HD] == -INFINITY ? 0.0f : expf(src[HD] - M);
        fac[tid] = f;
        fl[tid] = f * src[HD + 1];
    }
    __syncthreads();
    float *const part_ml = a.part + (size_t)a.n_heads * max_chunks * HD;
    for (int idx = tid; idx < HPK * HD; idx += (int)blockDim.x) {
        const int hh = idx / HD, d = idx % HD;
        float O = 0.0f;
        for (int w = 0; w < W; ++w)
            O = __builtin_fmaf(fac[w * HPK + hh], wp[(w * HPK + hh) * (HD + 2) + d], O);
        const int hg = g * HPK + hh;
        if (n_chunks == 1) {
            float L = 0.0f;
            for (int w = 0; w < W; ++w) L += fl[w * HPK + hh];
            a.out[(size_t)hg * HD + d] = O / L;
        } else {
            st_part(a.part + ((size_t)hg * max_chunks + c) * HD + d, O);
            if (d == 0) {
                float M = -INFINITY, L = 0.0f;
                for (int w = 0; w < W; ++w) {
                    M = fmaxf(M, wp[(w * HPK + hh) * (HD + 2) + HD]);
                    L += fl[w * HPK + hh];
                }
                float *pml = part_ml + ((size_t)hg * max_chunks + c) * 2;
                st_part(pml, M);
                st_part(pml + 1, L);
            }
        }
    }
    if (n_chunks == 1) return;

    // ---- 9. arrival, then the last arriver merges the chunks ----
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
    if (wave < HPK)
        merge_chunks<HD, C::MAXC>(a, g * HPK + wave, n_chunks, max_chunks, wp + wave * C::MAXC,
                                  lane);
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

// Kernels whose LDS limit was raised already: a fixed table (no heap
// allocation on the launch path, which cw_attention_noalloc relies on)
std::mutex g_mu;
constexpr int kLdsSlots = 128;
const void *g_lds_set[kLdsSlots];
int g_lds_n = 0;

int ensure_lds(attn_fn f, int lds) {
    std::lock_guard<std::mutex> lk(g_mu);
    const void *p = reinterpret_cast<const void *>(f);
    for (int i = 0; i < g_lds_n; ++i)
        if (g_lds_set[i] == p) return CW_OK;
    CW_HIP(hipFuncSetAttribute(p, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
    if (g_lds_n < kLdsSlots) g_lds_set[g_lds_n++] = p;
    return CW_OK;
}

// ---- the scratch of cw_attention_noalloc: chunk partials, then the
// per-kv-head arrival counters (one 128-byte line each).  One copy per GPU,
// shared by every call on that GPU; its address is taken once per device
// (attn_noalloc_setup, from cw_ctx_create).
constexpr size_t kNoAllocPartBytes = (size_t)8 << 20;
constexpr size_t kNoAllocCntBytes = (size_t)cwi::kMaxAttnKv * 128;
static __device__ __align__(256) unsigned char scratch[kNoAllocPartBytes + kNoAllocCntBytes];

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void *g_noalloc_ptr[kMaxDevices];

AttnPick pick_attn(int kv_dtype, int hd, int hpk) {
    return kv_dtype == CW_F16 ? pick_hd<_Float16>(hd, hpk) : pick_hd<float>(hd, hpk);
}

template <typename KVT, int HPK, int W, int PW = 16>
AttnPick make_wave_pick(bool fused) {
    using C = WaveCfg<KVT, HPK, W, PW>;
    return {fused ? attn_wave_kernel<KVT, HPK, W, true, PW>
                  : attn_wave_kernel<KVT, HPK, W, false, PW>,
            C::THREADS, C::CP, C::LDS};
}

// 8 waves of 8 positions: the small-cache f32 configuration
AttnPick pick_wave_small_f32(int hpk, bool f) {
    switch (hpk) {
        case 1: return make_wave_pick<float, 1, 8, 8>(f);
        case 2: return make_wave_pick<float, 2, 8, 8>(f);
        case 4: return make_wave_pick<float, 4, 8, 8>(f);
        case 8: return make_wave_pick<float, 8, 8, 8>(f);
        default: return {nullptr, 0, 0, 0};
    }
}

template <typename KVT>
AttnPick pick_wave_w(int hpk, int w, bool f) {
    switch (hpk) {
        case 1: return w == 8 ? make_wave_pick<KVT, 1, 8>(f)
                       : w == 4 ? make_wave_pick<KVT, 1, 4>(f) : make_wave_pick<KVT, 1, 2>(f);
        case 2: return w == 8 ? make_wave_pick<KVT, 2, 8>(f)
                       : w == 4 ? make_wave_pick<KVT, 2, 4>(f) : make_wave_pick<KVT, 2, 2>(f);
        case 4: return w == 8 ? make_wave_pick<KVT, 4, 8>(f) : make_wave_pick<KVT, 4, 4>(f);
        case 8: return make_wave_pick<KVT, 8, 8>(f);
        default: return {nullptr, 0, 0, 0};
    }
}

// head_dim 128: the register-resident kernel, with W waves (16 positions
// each) per workgroup: the largest W (at least the heads per kv head) whose
// grid for a full cache still gives every CU a workgroup.  When no W fills
// the chip (small caches), 64 positions per workgroup: sequences up to 64
// positions then need no cross-workgroup merge, which at these sizes is most
// of the kernel, and for f32 caches as 8 waves of 8 positions, which halves
// each wave's chain of dependent reductions (Qwen3-0.6B shape, 160-position
// f32 cache, per launch at 33 / 141 keys: 2 waves of 16, 7.5 / 7.6 us; 4 of
// 16, 5.3 / 7.3; 8 of 8, 5.7 / 7.7 on another box, with the token loop at
// 1498-1500 against 1485-1487 tokens/s for 4 of 16; 8 waves of 16 were
// slower past 128 positions, 9.6 us)
AttnPick pick_wave(const cw_ctx *ctx, int kv_dtype, int hpk, int n_kv, int max_seq, bool fused) {
    int w = 2;
    bool fills = false;
    for (int cand : {8, 4, 2}) {
        if (cand < hpk) continue;
        w = cand;
        const long wgs = (long)((max_seq + 16 * cand - 1) / (16 * cand)) * n_kv;
        if (wgs >= ctx->n_cu) {
            fills = true;
            break;
        }
    }
    if (!fills && kv_dtype == CW_F32) return pick_wave_small_f32(hpk, fused);
    if (!fills) w = 4;
    if (w < hpk) w = hpk;
    return kv_dtype == CW_F16 ? pick_wave_w<_Float16>(hpk, w, fused)
                              : pick_wave_w<float>(hpk, w, fused);
}

}  // namespace

namespace cwi {

size_t attn_scratch_floats(int n_heads, int n_kv, int hd, int max_seq) {
    // chunks of at least 16 positions (the head_dim-128 kernel's smallest;
    // the general kernel's are no smaller for these shapes)
    const AttnPick pk = pick_attn(CW_F32, hd, n_heads / n_kv);
    int cp = pk.cp > 0 ? pk.cp : 8;
    if (cp > 16) cp = 16;
    const size_t chunks = (size_t)(max_seq + cp - 1) / cp;
    return chunks * (size_t)n_heads * (hd + 2);
}

// f16 cache, head_dim 128: the MFMA kernel with W waves (16 positions each)
// per workgroup, the fewest that keep a full cache's grid within one
// workgroup per CU (at least HPK waves, at most 16)
template <int HPK>
int launch_mfma_hpk(cw_ctx *ctx, const AttnArgs &b, float scale, bool prof) {
    using C = MfmaCfg<HPK>;
    const long per_cu = ((long)b.max_seq * b.n_kv + ctx->n_cu - 1) / ctx->n_cu;
    int w = (int)((per_cu + C::PW - 1) / C::PW);
    w = w < HPK ? HPK : w > C::WMAX ? C::WMAX : w;
    const int max_chunks = (b.max_seq + C::PW * w - 1) / (C::PW * w);
    auto fn = b.qkv ? attn_mfma_kernel<HPK, true> : attn_mfma_kernel<HPK, false>;
    CW_TRY(ensure_lds(fn, C::LDS));
    if (!prof) {
        hipLaunchKernelGGL(fn, dim3(max_chunks, b.n_kv), dim3(64 * w), C::LDS, ctx->stream, b,
                           scale, max_chunks);
        return launch_check("attention");
    }
    return launch(ctx, "attention", fn, dim3(max_chunks, b.n_kv), dim3(64 * w), C::LDS, b, scale,
                  max_chunks);
}

// Enqueue attention; a.cnt (the arrival counters) defaults to the context's.
// Without `prof` no profiling events are taken (their creation allocates).
int launch_attention_impl(cw_ctx *ctx, const AttnArgs &a, bool prof);

int launch_attention(cw_ctx *ctx, const AttnArgs &a) { return launch_attention_impl(ctx, a, true); }

int launch_attention_impl(cw_ctx *ctx, const AttnArgs &a, bool prof) {
    const int hpk = a.n_heads / a.n_kv;
    if (a.hd == 128 && a.kv_dtype == CW_F16) {
        if (a.max_seq > kMaxChunkSpan) {
            set_error("attention: max_seq=%d exceeds %d", a.max_seq, kMaxChunkSpan);
            return CW_ERR_ARG;
        }
        if (a.n_kv > kMaxAttnKv) {
            set_error("attention: n_kv_heads=%d exceeds %d", a.n_kv, kMaxAttnKv);
            return CW_ERR_ARG;
        }
        AttnArgs b = a;
        b.cnt = a.cnt ? a.cnt : ctx->attn_cnt;
        const float scale = powf((float)a.hd, -0.5f);
        switch (hpk) {
            case 1: return launch_mfma_hpk<1>(ctx, b, scale, prof);
            case 2: return launch_mfma_hpk<2>(ctx, b, scale, prof);
            case 4: return launch_mfma_hpk<4>(ctx, b, scale, prof);
            case 8: return launch_mfma_hpk<8>(ctx, b, scale, prof);
            default: break;
        }
    }
    const AttnPick pk = a.hd == 128 ? pick_wave(ctx, a.kv_dtype, hpk, a.n_kv, a.max_seq, a.qkv != nullptr)
                                    : pick_attn(a.kv_dtype, a.hd, hpk);
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
    b.cnt = a.cnt ? a.cnt : ctx->attn_cnt;
    const float scale = powf((float)a.hd, -0.5f);
    if (!prof) {
        hipLaunchKernelGGL(pk.fn, dim3(max_chunks, a.n_kv), dim3(pk.threads), pk.lds, ctx->stream,
                           b, scale, max_chunks);
        return launch_check("attention");
    }
    return launch(ctx, "attention", pk.fn, dim3(max_chunks, a.n_kv), dim3(pk.threads), pk.lds, b,
                  scale, max_chunks);
}

int attn_noalloc_setup(cw_ctx *ctx) {
    CW_CHECK_ARG(ctx->device >= 0 && ctx->device < kMaxDevices,
                 "attention scratch: device %d beyond %d", ctx->device, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[ctx->device]) {
        // this device's copy of the array (the caller made the device current);
        // the counters must start at zero, every launch leaves them at zero
        void *ptr = nullptr;
        CW_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        CW_HIP(hipMemsetAsync(static_cast<unsigned char *>(ptr) + kNoAllocPartBytes, 0,
                              kNoAllocCntBytes, ctx->stream));
        CW_HIP(hipStreamSynchronize(ctx->stream));
        g_noalloc_ptr[ctx->device] = ptr;
    }
    ctx->noalloc_scratch = g_noalloc_ptr[ctx->device];
    return CW_OK;
}

}  // namespace cwi

using namespace cwi;

static int check_attention_args(const char *what, const float *q, const void *k, const void *v,
                                int kv_dtype, int n_heads, int n_kv_heads, int seq, int head_dim,
                                const float *out) {
    CW_CHECK_ARG(q && k && v && out, "%s: null argument", what);
    CW_CHECK_ARG(kv_dtype == CW_F32 || kv_dtype == CW_F16, "%s: kv_dtype=%d", what, kv_dtype);
    CW_CHECK_ARG(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                 "%s: n_heads=%d n_kv_heads=%d", what, n_heads, n_kv_heads);
    CW_CHECK_ARG(seq > 0 && seq <= kMaxChunkSpan, "%s: seq=%d outside [1, %d]", what, seq,
                 kMaxChunkSpan);
    const int hpk = n_heads / n_kv_heads;
    CW_CHECK_ARG(hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8,
                 "%s: heads per kv head %d not in {1,2,4,8}", what, hpk);
    CW_CHECK_ARG(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 ||
                     head_dim == 256,
                 "%s: head_dim=%d not in {16,32,64,128,256}", what, head_dim);
    return CW_OK;
}

extern "C" int cw_attention_noalloc(cw_ctx *ctx, const float *q, const void *k, const void *v,
                                    int kv_dtype, int n_heads, int n_kv_heads, int seq,
                                    int head_dim, float *out) {
    CW_CHECK_ARG(ctx != nullptr, "cw_attention_noalloc: null ctx");
    CW_TRY(check_attention_args("cw_attention_noalloc", q, k, v, kv_dtype, n_heads, n_kv_heads,
                                seq, head_dim, out));
    CW_CHECK_ARG(n_kv_heads <= kMaxAttnKv, "cw_attention_noalloc: n_kv_heads=%d exceeds %d",
                 n_kv_heads, kMaxAttnKv);
    const size_t need = attn_scratch_floats(n_heads, n_kv_heads, head_dim, seq) * sizeof(float);
    CW_CHECK_ARG(need <= kNoAllocPartBytes,
                 "cw_attention_noalloc: the chunk partials need %zu bytes, the static scratch "
                 "holds %zu (n_heads * ceil(seq / 16) * (head_dim + 2) floats)",
                 need, kNoAllocPartBytes);
    if (!ctx->noalloc_scratch) {
        set_error("cw_attention_noalloc: the context has no static scratch address");
        return CW_ERR_STATE;
    }
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
    unsigned char *base = static_cast<unsigned char *>(ctx->noalloc_scratch);
    a.part = reinterpret_cast<float *>(base);
    a.cnt = reinterpret_cast<unsigned *>(base + kNoAllocPartBytes);
    return launch_attention_impl(ctx, a, false);
}

extern "C" int cw_attention(cw_ctx *ctx, const float *q, const void *k, const void *v, int kv_dtype,
                            int n_heads, int n_kv_heads, int seq, int head_dim, float *out) {
    CW_CHECK_ARG(ctx != nullptr, "cw_attention: null argument");
    CW_TRY(check_attention_args("cw_attention", q, k, v, kv_dtype, n_heads, n_kv_heads, seq,
                                head_dim, out));
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
