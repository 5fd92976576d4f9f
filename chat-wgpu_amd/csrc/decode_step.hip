// One Qwen3 decode step as one persistent, cooperatively launched kernel.
//
// Replaces the per-token op sequence of Qwen3::forward + logits + argmax
// (src/model/qwen3.rs:128-191, src/model/mod.rs:93-103): the reference
// records ~560 small dispatches per token; here one launch of one workgroup
// per CU walks the whole step, phase by phase, with a grid barrier between
// phases that depend on each other:
//
//   per layer l:
//     A  RMSNorm(h_l) -> fused QKV Q4 GEMV                     -> qkv[l]
//     B  QK-norm + RoPE + KV write + split-sequence attention,
//        merged by the last workgroup to finish each kv head   -> attn[l]
//     C  O Q4 GEMV + residual                                  -> hb[l]
//     D  RMSNorm(hb) -> gate/up Q4 GEMV pair + SwiGLU          -> act[l]
//     E  down Q4 GEMV + residual                               -> h_{l+1}
//   LM head: final RMSNorm -> Q4 GEMV -> logits, per-workgroup argmax,
//   merged by the last workgroup, which also advances the generate state.
//
// Weights never depend on activations, so each workgroup issues the loads of
// its share of the next phase between arriving at a barrier and waiting on
// it: HBM keeps streaming while the grid synchronises.  Every phase output is
// written once per launch into its own per-layer buffer.
//
// Coherence across the 8 XCDs (one L2 each): activations shared between
// workgroups are written with agent-scope (sc1, write-through) stores and
// read with agent-scope (sc1) loads, so no L2 writeback/invalidate is needed;
// a barrier arrival waits for the workgroup's own stores (s_waitcnt) before
// its atomic.  Weights and the KV cache are read with ordinary loads.
//
// Grid barrier: a two-level counter tree (kTreeG groups of workgroups, the
// last arriver of a group bumps the root), polled by one thread per
// workgroup with a bounded spin: a barrier that does not complete within
// `timeout` wall-clock ticks sets the error word and every workgroup leaves
// the kernel, so a fault in the protocol ends the launch instead of hanging
// the device.

#include <map>
#include <mutex>

#include "cw_internal.hpp"

// Hooks for a CPU execution of the kernel (tests/step_emu): compiler barriers
// that pin a value in a scalar / vector register, and the workgroup's LDS.
#ifndef CW_STEP_HOOKS
#define CW_OPAQUE_S(v) asm volatile("" : "+s"(v))
#define CW_OPAQUE_V(v) asm volatile("" : "+v"(v))
#define CW_WG_SHARED(T, name) __shared__ T name
#define CW_WG_DYNAMIC(T, name) extern __shared__ T name[]
#endif

namespace {

using cwi::StepArgs;
using cwi::StepLayer;

constexpr int kT = 512;         // threads per workgroup (one workgroup per CU, 2 waves per SIMD)
constexpr int kW = kT / 64;     // waves per workgroup
constexpr int kQ = 16;          // 16-byte weight loads in flight per lane (the ring)
constexpr int kPF = 8;          // of which issued before a grid barrier: what arrives
                                // while the barrier completes (~64 KB per CU)
constexpr int kHD = 128;        // head_dim of the fused path
constexpr int kMaxK = 16384;    // largest GEMV input width (8 float4 per thread)

// sync word layout (unsigned), one 128-byte line per counter
constexpr int kTreeG = 8;
constexpr int kSyncRoot = kTreeG * 32;
constexpr int kSyncArgmax = kSyncRoot + 32;
constexpr int kSyncAttn = kSyncArgmax + 32;  // + 32 * kv head
constexpr int kSyncErr = kSyncAttn + 32 * cwi::kStepMaxKv;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- memory helpers

// A buffer resource over [p, p + bytes).  Both are wave-uniform by
// construction; readfirstlane makes that visible to the compiler, so the
// descriptor lives in SGPRs (a descriptor it cannot prove uniform turns every
// load into a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    void *u = reinterpret_cast<void *>(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, 0, __builtin_amdgcn_readfirstlane(bytes),
                                             0x00020000);
}
// 16-byte load through L2 of an activation buffer (see the coherence note
// at the top: every such buffer is written once per launch, before any read)
__device__ __forceinline__ float4 ld_act4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float ld_coh(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_cnt(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned add_cnt(unsigned *p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_cnt(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// every memory operation this wave issued has completed
__device__ __forceinline__ void drain() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// A value the optimiser cannot see through: shapes pass through it at each
// phase entry so that their derived offsets and predicates are recomputed in
// the phase rather than hoisted out of the layer loop and kept live across it.
__device__ __forceinline__ int opaque(int v) {
    v = __builtin_amdgcn_readfirstlane(v);
    CW_OPAQUE_S(v);
    return v;
}
// the thread index, re-read per phase for the same reason
__device__ __forceinline__ int tid_() {
    int v = (int)threadIdx.x;
    CW_OPAQUE_V(v);
    return v;
}

// ---------------------------------------------------------------- reductions

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum8(float v) {  // aligned groups of 8 lanes
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    return v;
}
// all-reduce over aligned groups of g lanes (g a power of two, runtime)
__device__ __forceinline__ float group_sum(float v, int g) {
    for (int off = 1; off < g; off <<= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

struct Best {
    float v;
    uint32_t i;
};
__device__ __forceinline__ Best better(Best a, Best b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}
__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        b = better(b, Best{__shfl_xor(b.v, off), (uint32_t)__shfl_xor((int)b.i, off)});
    return b;
}
constexpr float kNegInit = -3.402823e38f;  // argmax candidates must exceed this

// ---------------------------------------------------------------- grid barrier

struct Ctl {
    unsigned *sync;
    long long timeout;
    unsigned epoch;
    long long *trace;  // optional: workgroup 0 stamps [2e] arrive, [2e+1] released
};

// Arrive: this workgroup's stores are complete, then one atomic per
// workgroup on its group counter; the group's last arriver bumps the root.
__device__ __forceinline__ void bar_arrive(Ctl &c) {
    ++c.epoch;
    drain();
    __syncthreads();
    if (threadIdx.x == 0) {
        if (c.trace && blockIdx.x == 0) c.trace[2 * c.epoch] = wall_clock64();
        const unsigned g = blockIdx.x % kTreeG;
        const unsigned per = (gridDim.x - g + kTreeG - 1) / kTreeG;
        const unsigned old = add_cnt(c.sync + g * 32, 1u);
        if (old + 1 == c.epoch * per) add_cnt(c.sync + kSyncRoot, 1u);
    }
}

// Wait for every workgroup's arrival (bounded); false = timed out.
__device__ __forceinline__ bool bar_wait(Ctl &c, int *ok_s) {
    if (threadIdx.x == 0) {
        int ok = 1;
        const unsigned groups = gridDim.x < kTreeG ? gridDim.x : kTreeG;
        const unsigned target = c.epoch * groups;
        if (ld_cnt(c.sync + kSyncRoot) < target) {
            const long long t0 = wall_clock64();
            while (ld_cnt(c.sync + kSyncRoot) < target) {
                if (wall_clock64() - t0 > c.timeout) {
                    ok = 0;
                    st_cnt(c.sync + kSyncErr, 1u);
                    break;
                }
            }
        }
        *ok_s = ok;
        if (c.trace && blockIdx.x == 0) c.trace[2 * c.epoch + 1] = wall_clock64();
    }
    __syncthreads();
    return *ok_s != 0;
}

// ---------------------------------------------------------------- activation staging

// x (K floats) -> LDS as [8][K/32] float4, element quarter i of block b at
// lds4[i*nb + b], quarters 0-3 scaled by 2^24 and 4-7 by 2^20 (see
// dot_word), plus sx[b] = sum of the block's 32 values.  Modes:
//   X_PLAIN   x = src
//   X_NORM    x = src * (1/sqrt(mean(src^2) + eps)) * w      (norm.wgsl:20-42)
//   X_SWIGLU  x = silu(src[i]) * src[K + i], silu(g) = g/(1+e^-g) (glu.wgsl:22-26)
// src is an activation buffer (or the embedding row).  mid() runs after the
// source loads are issued and before their first use: loads it issues do not
// delay them (vmcnt retires in issue order).
enum { X_PLAIN = 0, X_NORM = 1, X_SWIGLU = 2 };

template <class Mid>
__device__ __forceinline__ void stage_x(int mode, const float *src, const float *w, int K,
                                        float eps, float4 *lds4, float *sx, float *red,
                                        float *copy_out, Mid mid) {
    constexpr int J = kMaxK / 4 / kT;
    const int tid = tid_(), lane = tid & 63, wave = tid >> 6;
    K = opaque(K);
    mode = opaque(mode);
    const int K4 = K >> 2, nb = K >> 5;
    const bool glu = mode == X_SWIGLU;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src, (uint32_t)K * (glu ? 8 : 4));
    float4 v[J], u[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int idx = tid + j * kT;
        const bool in = idx < K4;
        v[j] = in ? ld_act4(r, (uint32_t)idx * 16) : make_float4(0.f, 0.f, 0.f, 0.f);
        u[j] = (in && glu) ? ld_act4(r, (uint32_t)(K4 + idx) * 16) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __builtin_amdgcn_sched_barrier(0);
    mid();
    __builtin_amdgcn_sched_barrier(0);
    float inv = 1.0f;
    if (mode == X_NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j)
            ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        ss = 0.0f;
#pragma unroll
        for (int i = 0; i < kW; ++i) ss += red[i];
        inv = 1.0f / sqrtf(ss / (float)K + eps);
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int idx = tid + j * kT;
        if (j * kT < K4) {  // wave-uniform for K4 a multiple of 8
            float4 x = v[j];
            if (idx < K4) {
                if (mode == X_NORM) {
                    const float4 g = reinterpret_cast<const float4 *>(w)[idx];
                    x.x = (x.x * inv) * g.x;
                    x.y = (x.y * inv) * g.y;
                    x.z = (x.z * inv) * g.z;
                    x.w = (x.w * inv) * g.w;
                    if (copy_out) reinterpret_cast<float4 *>(copy_out)[idx] = x;
                } else if (glu) {
                    const float4 gg = x;
                    x.x = (gg.x / (1.0f + expf(-gg.x))) * u[j].x;
                    x.y = (gg.y / (1.0f + expf(-gg.y))) * u[j].y;
                    x.z = (gg.z / (1.0f + expf(-gg.z))) * u[j].z;
                    x.w = (gg.w / (1.0f + expf(-gg.w))) * u[j].w;
                }
                const int blk = idx >> 3, i = idx & 7;
                const float sc = i < 4 ? 0x1p24f : 0x1p20f;
                lds4[i * nb + blk] = make_float4(x.x * sc, x.y * sc, x.z * sc, x.w * sc);
            }
            float part = (x.x + x.y) + (x.z + x.w);
            part = sum8(part);
            if (idx < K4 && (idx & 7) == 0) sx[idx >> 3] = part;
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------- Q4 GEMV phase

__device__ __forceinline__ float f16lo(uint32_t v) {
    return (float)__builtin_bit_cast(half2v, v).x;
}
__device__ __forceinline__ float f16hi(uint32_t v) {
    return (float)__builtin_bit_cast(half2v, v).y;
}
// sum_j q_j x_j over one quant dword: masking leaves f16 subnormals q*2^-24
// (low nibbles) and q*2^-20 (high nibbles); the LDS copy of x carries the
// matching 2^24 / 2^20 factors, so each product is q*x exactly.
__device__ __forceinline__ float dot_word(uint32_t dw, float4 xl, float4 xh, float s) {
    const uint32_t a = dw & 0x000F000Fu;
    const uint32_t b = dw & 0x00F000F0u;
    const uint32_t d8 = dw >> 8;
    const uint32_t c = d8 & 0x000F000Fu;
    const uint32_t e = d8 & 0x00F000F0u;
    s = __builtin_fmaf(f16lo(a), xl.x, s);
    s = __builtin_fmaf(f16lo(c), xl.y, s);
    s = __builtin_fmaf(f16hi(a), xl.z, s);
    s = __builtin_fmaf(f16hi(c), xl.w, s);
    s = __builtin_fmaf(f16lo(b), xh.x, s);
    s = __builtin_fmaf(f16lo(e), xh.y, s);
    s = __builtin_fmaf(f16hi(b), xh.z, s);
    s = __builtin_fmaf(f16hi(e), xh.w, s);
    return s;
}

// One wave's share of a Q4 GEMV: whole row groups (RPS rows of G lanes each,
// S steps of G blocks per row), listed as groups (row group, step).  Weights
// are read through buffer resources (buffer_load: vmcnt only, range-checked).
struct Gemv {
    const uint8_t *q;
    const uint16_t *sc;
    uint32_t nblk;
    int N, nb, G, lgG, S, RPS;
    int rg0, nrg;
};

__device__ __forceinline__ Gemv gemv_setup(const uint8_t *q, const uint16_t *sc, int N, int K,
                                           int gw, int nw) {
    Gemv p;
    N = opaque(N);
    K = opaque(K);
    p.N = N;
    p.nb = K >> 5;
    p.nblk = (uint32_t)N * (uint32_t)p.nb;
    p.q = q;
    p.sc = sc;
    int g = 64;
    while (g > 1 && (p.nb & (g - 1))) g >>= 1;
    p.G = g;
    p.lgG = 31 - __builtin_clz(g);
    p.S = p.nb / g;
    p.RPS = 64 / g;
    const int nrg_all = (N + p.RPS - 1) / p.RPS;
    const int r0 = (int)((long long)gw * nrg_all / nw);
    const int r1 = (int)((long long)(gw + 1) * nrg_all / nw);
    p.rg0 = r0;
    p.nrg = r1 - r0;
    return p;
}

// Position of the next group to load (row group rgl of the wave, step s).
struct Cursor {
    int rgl, s;
    __device__ __forceinline__ void next(int S) {
        if (++s == S) {
            s = 0;
            ++rgl;
        }
    }
};

__device__ __forceinline__ void gemv_load(const Gemv &p, Cursor c, int lane, uint4 &q, uint32_t &d) {
    int row = (p.rg0 + c.rgl) * p.RPS + (lane >> p.lgG);
    row = row < p.N ? row : p.N - 1;
    const uint32_t idx = (uint32_t)row * (uint32_t)p.nb + (uint32_t)(c.s * p.G + (lane & (p.G - 1)));
    q = __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(p.q, p.nblk * 16), idx * 16, 0, 0));
    d = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(p.sc, p.nblk * 2), idx * 2, 0, 0);
}

// Issue ring slots [u0, u1) (groups u0 .. u1-1 of the wave's list).
template <int U0, int U1>
__device__ __forceinline__ void gemv_issue(const Gemv &p, uint4 (&rq)[kQ], uint32_t (&rd)[kQ]) {
    const int lane = tid_() & 63;
    const int T = p.nrg * p.S;
    Cursor c{U0 / p.S, U0 % p.S};
#pragma unroll
    for (int u = U0; u < U1; ++u) {
        if (u < T) gemv_load(p, c, lane, rq[u], rd[u]);
        c.next(p.S);
    }
}
// the prefetch before a barrier, and the rest of the ring after staging
__device__ __forceinline__ void gemv_prefetch(const Gemv &p, uint4 (&rq)[kQ], uint32_t (&rd)[kQ]) {
    gemv_issue<0, kPF>(p, rq, rd);
}
__device__ __forceinline__ void gemv_fill(const Gemv &p, uint4 (&rq)[kQ], uint32_t (&rd)[kQ]) {
    gemv_issue<kPF, kQ>(p, rq, rd);
}

enum { E_STORE = 0, E_RESID = 1, E_LOGITS = 2 };

struct Epi {
    int kind;
    float *out;          // E_STORE / E_RESID: agent-coherent stores; E_LOGITS: plain
    const float *resid;  // E_RESID: an activation buffer (or the embedding row)
};

// Consume the ring (its first kQ groups were issued), refilling each slot
// with the group kQ ahead; reduce and write each finished row group.
__device__ __forceinline__ void gemv_run(const Gemv &p, uint4 (&rq)[kQ], uint32_t (&rd)[kQ],
                                         const float4 *lds4, const float *sx, const Epi &e,
                                         Best &best) {
    const int lane = tid_() & 63;
    const int T = p.nrg * p.S;
    const int sl = lane & (p.G - 1);
    int lg = T < kQ ? T : kQ;
    Cursor lc{kQ / p.S, kQ % p.S};  // position of group kQ
    int cs = 0, crg = 0;
    float acc = 0.0f, rv = 0.0f;
    for (int base = 0; base < T; base += kQ) {
#pragma unroll
        for (int u = 0; u < kQ; ++u) {
            if (base + u < T) {
                if (e.kind == E_RESID && cs == 0) {  // the row's residual, as its group starts
                    int row = (p.rg0 + crg) * p.RPS + (lane >> p.lgG);
                    row = row < p.N ? row : p.N - 1;
                    rv = e.resid[row];
                }
                const int b = cs * p.G + sl;
                const uint4 q = rq[u];
                const float s0 = dot_word(q.x, lds4[0 * p.nb + b], lds4[4 * p.nb + b], 0.0f);
                const float s1 = dot_word(q.y, lds4[1 * p.nb + b], lds4[5 * p.nb + b], 0.0f);
                const float s2 = dot_word(q.z, lds4[2 * p.nb + b], lds4[6 * p.nb + b], 0.0f);
                const float s3 = dot_word(q.w, lds4[3 * p.nb + b], lds4[7 * p.nb + b], 0.0f);
                const float t = __builtin_fmaf(-8.0f, sx[b], (s0 + s1) + (s2 + s3));
                const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)rd[u]);
                acc = __builtin_fmaf((float)d, t, acc);
                if (lg < T) {
                    gemv_load(p, lc, lane, rq[u], rd[u]);
                    ++lg;
                    lc.next(p.S);
                }
                if (++cs == p.S) {
                    cs = 0;
                    acc = group_sum(acc, p.G);
                    const int row = (p.rg0 + crg) * p.RPS + (lane >> p.lgG);
                    if (sl == 0 && row < p.N) {
                        if (e.kind == E_LOGITS) {
                            e.out[row] = acc;
                            if (acc > best.v) best = Best{acc, (uint32_t)row};
                        } else {
                            st_coh(e.out + row, e.kind == E_RESID ? rv + acc : acc);
                        }
                    }
                    acc = 0.0f;
                    ++crg;
                }
            }
        }
    }
}

// ---------------------------------------------------------------- attention phase

template <typename KVT, int HPK>
struct At {
    static constexpr int ES = (int)sizeof(KVT);
    static constexpr int HALF = kHD / 2;
    static constexpr int GT = 64 * HPK;           // threads per item
    static constexpr int IPW = kW / HPK;          // items per workgroup
    static constexpr int ROWB = kHD * ES;         // bytes of one K/V row slice
    static constexpr int ROWP = ROWB + 16;        // padded LDS row stride
    static constexpr int U4_ROW = ROWB / 16;
    // positions per item: the K and V loads fit half the register ring each,
    // the tiles of IPW items fit 148 KB of LDS, at most 128 (two per lane)
    static constexpr int REG_CP = (kQ / 2) * GT / U4_ROW;
    static constexpr int ITEM_LDS(int cp) { return 2 * cp * ROWP + HPK * kHD * 4 + HPK * cp * 4; }
    static constexpr int pick_cp() {
        int cp = REG_CP < 128 ? REG_CP : 128;
        cp &= ~7;
        while (cp > 8 && IPW * ITEM_LDS(cp) > 148 * 1024) cp -= 8;
        return cp;
    }
    static constexpr int CPMAX = pick_cp();
    static constexpr int NT = (CPMAX + 63) / 64;  // positions per lane in the scores
    static constexpr int NLOAD = (CPMAX * U4_ROW + GT - 1) / GT;  // 16-byte loads per thread (K or V)
    static constexpr int ILDS = ITEM_LDS(CPMAX);
    static_assert(CPMAX >= 8 && 2 * NLOAD <= kQ, "attention tile does not fit");
};

struct AttnGeo {
    int seq, pos, cp, n_chunks, n_items, slots, rounds;
};

template <typename KVT>
__device__ __forceinline__ KVT to_kv(float v) {
    return (KVT)v;  // f16: round to nearest even
}

// Issue the K/V tile loads of this thread's item in the first pass.
template <typename KVT, int HPK>
__device__ __forceinline__ void attn_load(const StepArgs &a, const StepLayer &L, const AttnGeo &g,
                                          int item, uint4 (&rq)[kQ]) {
    using C = At<KVT, HPK>;
    const int t = tid_() % C::GT;
    if (item >= g.n_items) return;
    const int kvh = item / g.n_chunks, c = item - kvh * g.n_chunks;
    const int c0 = c * g.cp;
    const uint32_t row_bytes = (uint32_t)a.n_kv * C::ROWB;
    const uint32_t span = (uint32_t)a.max_seq * row_bytes;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(L.kc, span), vr = make_rsrc(L.vc, span);
#pragma unroll
    for (int i = 0; i < C::NLOAD; ++i) {
        const int f = t + i * C::GT;
        if (f < g.cp * C::U4_ROW) {
            const int row = f / C::U4_ROW, col = f % C::U4_ROW;
            int p = c0 + row;
            p = p < g.seq ? p : g.seq - 1;
            const uint32_t off = (uint32_t)p * row_bytes + (uint32_t)kvh * C::ROWB + (uint32_t)col * 16;
            rq[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0));
            rq[C::NLOAD + i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0));
        }
    }
}

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

// One round of items: per item (kv head, chunk) the HPK waves of its group
// normalise and rotate their query heads (and, for the chunk holding the new
// position, the new key; the value is copied), write the tile to LDS, score
// (lane = position), softmax-partial and P.V (lane = dims), and store the
// chunk partial (o[128], m, l).  Uniform barrier sequence for every group.
template <typename KVT, int HPK>
__device__ __forceinline__ void attn_round(const StepArgs &a, const StepLayer &L, int l,
                                           const AttnGeo &g, int item, uint4 (&rq)[kQ],
                                           unsigned char *lds) {
    using C = At<KVT, HPK>;
    constexpr int HALF = C::HALF;
    const int tid = tid_(), lane = tid & 63, wave = tid >> 6;
    const int grp = wave / HPK, wq = wave % HPK;
    const int t = tid % C::GT;
    unsigned char *base = lds + grp * C::ILDS;
    unsigned char *k_t = base;
    unsigned char *v_t = base + C::CPMAX * C::ROWP;
    float *q_s = reinterpret_cast<float *>(base + 2 * C::CPMAX * C::ROWP);  // [HPK][HD]
    float *p_s = q_s + HPK * kHD;                                           // [HPK][CPMAX]
    const bool live = item < g.n_items;
    const int kvh = live ? item / g.n_chunks : 0;
    const int c = live ? item - kvh * g.n_chunks : 0;
    const int c0 = c * g.cp;
    const int q_dim = a.n_heads * kHD, kv_dim = a.n_kv * kHD;
    const bool has_new = live && g.pos >= c0 && g.pos < c0 + g.cp;
    const float *qkv = a.qkv + (size_t)l * (q_dim + 2 * kv_dim);
    const float *cs_t = a.cos_t + (size_t)g.pos * HALF;
    const float *sn_t = a.sin_t + (size_t)g.pos * HALF;

    // ---- query (and new key / value) of this wave
    float knew0 = 0.f, knew1 = 0.f, vnew0 = 0.f, vnew1 = 0.f;
    if (live) {
        const int h = kvh * HPK + wq;
        const float lo = qkv[(size_t)h * kHD + lane];
        const float hi = qkv[(size_t)h * kHD + lane + HALF];
        const float cs = cs_t[lane], sn = sn_t[lane];
        float ss = wave_sum(lo * lo + hi * hi);
        float inv = 1.0f / sqrtf(ss / (float)kHD + a.eps);
        const float l0 = (lo * inv) * L.q_norm[lane];
        const float h0 = (hi * inv) * L.q_norm[lane + HALF];
        q_s[wq * kHD + lane] = l0 * cs - h0 * sn;
        q_s[wq * kHD + lane + HALF] = h0 * cs + l0 * sn;
        if (has_new && wq == 0) {
            const float *ks = qkv + q_dim + (size_t)kvh * kHD;
            const float *vs = qkv + q_dim + kv_dim + (size_t)kvh * kHD;
            const float klo = ks[lane], khi = ks[lane + HALF];
            vnew0 = vs[lane];
            vnew1 = vs[lane + HALF];
            ss = wave_sum(klo * klo + khi * khi);
            inv = 1.0f / sqrtf(ss / (float)kHD + a.eps);
            const float kl = (klo * inv) * L.k_norm[lane];
            const float kh = (khi * inv) * L.k_norm[lane + HALF];
            knew0 = kl * cs - kh * sn;
            knew1 = kh * cs + kl * sn;
        }
    }

    // ---- tile -> LDS (rows past the sequence as zeros)
    if (live) {
#pragma unroll
        for (int i = 0; i < C::NLOAD; ++i) {
            const int f = t + i * C::GT;
            if (f < g.cp * C::U4_ROW) {
                const int row = f / C::U4_ROW, col = f % C::U4_ROW;
                uint4 kv = rq[i], vv = rq[C::NLOAD + i];
                if (c0 + row >= g.seq) {  // rows past the sequence read as zeros
                    kv = make_uint4(0u, 0u, 0u, 0u);
                    vv = kv;
                }
                *reinterpret_cast<uint4 *>(k_t + row * C::ROWP + col * 16) = kv;
                *reinterpret_cast<uint4 *>(v_t + row * C::ROWP + col * 16) = vv;
            }
        }
    }
    __syncthreads();
    if (has_new && wq == 0) {  // the new row: into the tile and the cache (cache.rs:21-24)
        const int r = g.pos - c0;
        KVT *kt = reinterpret_cast<KVT *>(k_t + r * C::ROWP);
        KVT *vt = reinterpret_cast<KVT *>(v_t + r * C::ROWP);
        const size_t row_bytes = (size_t)kv_dim * C::ES;
        KVT *kg = reinterpret_cast<KVT *>(reinterpret_cast<unsigned char *>(L.kc) +
                                          (size_t)g.pos * row_bytes + (size_t)kvh * C::ROWB);
        KVT *vg = reinterpret_cast<KVT *>(reinterpret_cast<unsigned char *>(L.vc) +
                                          (size_t)g.pos * row_bytes + (size_t)kvh * C::ROWB);
        const KVT k0 = to_kv<KVT>(knew0), k1 = to_kv<KVT>(knew1);
        const KVT v0 = to_kv<KVT>(vnew0), v1 = to_kv<KVT>(vnew1);
        kt[lane] = k0;
        kt[lane + HALF] = k1;
        vt[lane] = v0;
        vt[lane + HALF] = v1;
        kg[lane] = k0;
        kg[lane + HALF] = k1;
        vg[lane] = v0;
        vg[lane + HALF] = v1;
    }
    __syncthreads();

    // ---- scores: lane = position (NT positions per lane)
    float m = -INFINITY, lsum = 0.0f;
    if (live) {
        const float *qw = q_s + wq * kHD;
        constexpr int EPU = 16 / C::ES;
        float s4[C::NT][4];
#pragma unroll
        for (int t2 = 0; t2 < C::NT; ++t2)
#pragma unroll
            for (int j = 0; j < 4; ++j) s4[t2][j] = 0.0f;
#pragma unroll
        for (int u = 0; u < C::U4_ROW; ++u) {
            float qv[EPU];
#pragma unroll
            for (int e = 0; e < EPU; e += 4) {
                const float4 q4 = *reinterpret_cast<const float4 *>(qw + u * EPU + e);
                qv[e] = q4.x;
                qv[e + 1] = q4.y;
                qv[e + 2] = q4.z;
                qv[e + 3] = q4.w;
            }
#pragma unroll
            for (int t2 = 0; t2 < C::NT; ++t2) {
                int r = lane + 64 * t2;
                r = r < g.cp ? r : 0;
                const uint4 kk = *reinterpret_cast<const uint4 *>(k_t + r * C::ROWP + u * 16);
                s4[t2][u & 3] = dot16<KVT>(kk, qv, s4[t2][u & 3]);
            }
            if ((u & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
        float sv[C::NT];
        float mloc = -INFINITY;
#pragma unroll
        for (int t2 = 0; t2 < C::NT; ++t2) {
            const int r = lane + 64 * t2;
            const bool valid = r < g.cp && c0 + r < g.seq;
            sv[t2] = valid ? ((s4[t2][0] + s4[t2][1]) + (s4[t2][2] + s4[t2][3])) * a.scale
                           : -INFINITY;
            mloc = fmaxf(mloc, sv[t2]);
        }
        m = wave_max(mloc);  // finite: position c0 < seq is valid
        float ploc = 0.0f;
#pragma unroll
        for (int t2 = 0; t2 < C::NT; ++t2) {
            const int r = lane + 64 * t2;
            const float pr = sv[t2] == -INFINITY ? 0.0f : expf(sv[t2] - m);
            ploc += pr;
            if (r < C::CPMAX) p_s[wq * C::CPMAX + r] = pr;
        }
        lsum = wave_sum(ploc);
    }
    __syncthreads();

    // ---- P.V: lane = dims (lane, lane + 64); write the chunk partial
    if (live) {
        const float *pw = p_s + wq * C::CPMAX;
        float o0[4] = {0.f, 0.f, 0.f, 0.f}, o1[4] = {0.f, 0.f, 0.f, 0.f};
        for (int r0 = 0; r0 < g.cp; r0 += 8) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float pr = pw[r0 + i];
                const KVT *vrow = reinterpret_cast<const KVT *>(v_t + (r0 + i) * C::ROWP);
                o0[i & 3] = __builtin_fmaf(pr, (float)vrow[lane], o0[i & 3]);
                o1[i & 3] = __builtin_fmaf(pr, (float)vrow[lane + HALF], o1[i & 3]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        const int h = kvh * HPK + wq;
        float *po = a.part + ((size_t)h * a.max_chunks + c) * (kHD + 2);
        st_coh(po + lane, (o0[0] + o0[1]) + (o0[2] + o0[3]));
        st_coh(po + lane + HALF, (o1[0] + o1[1]) + (o1[2] + o1[3]));
        if (lane == 0) {
            st_coh(po + kHD, m);
            st_coh(po + kHD + 1, lsum);
        }
    }
    __syncthreads();  // the tile LDS is reused by the next round
}

// Merge every chunk partial of kv head kvh (this workgroup arrived last).
// Thread = (query head, dim); a wave covers half a head, so per-head (m, l)
// sit one chunk per lane.  Chunks go in batches of 64: all loads of a batch
// are issued before any is used (one round trip per batch), and the batches
// combine with the usual running-max rescale.  (64-chunk batches spill.)
template <int HPK>
__device__ __forceinline__ void attn_merge(const StepArgs &a, int l, int kvh, int n_chunks) {
    const int tid = tid_(), lane = tid & 63;
    constexpr int B = 32;
    const int q_dim = a.n_heads * kHD;
    for (int o = tid; o < HPK * kHD; o += kT) {
        const int hl = o / kHD, d = o - hl * kHD;  // hl is uniform per wave
        const float *ph = a.part + (size_t)(kvh * HPK + hl) * a.max_chunks * (kHD + 2);
        float M = -INFINITY, L = 0.0f, acc = 0.0f;
        for (int c0 = 0; c0 < n_chunks; c0 += B) {
            const int nc = n_chunks - c0 < B ? n_chunks - c0 : B;
            float v[B];
#pragma unroll
            for (int i = 0; i < B; ++i)
                v[i] = i < nc ? ld_coh(ph + (size_t)(c0 + i) * (kHD + 2) + d) : 0.0f;
            const bool mine = lane < nc;
            const float mc = mine ? ld_coh(ph + (size_t)(c0 + lane) * (kHD + 2) + kHD) : -INFINITY;
            const float lc = mine ? ld_coh(ph + (size_t)(c0 + lane) * (kHD + 2) + kHD + 1) : 0.0f;
            const float mb = wave_max(mc);  // finite: chunk c0 exists
            const float Mn = fmaxf(M, mb);
            const float wc = mine ? expf(mc - Mn) : 0.0f;
            const float r = expf(M - Mn);   // 0 on the first batch
            L = L * r + wave_sum(wc * lc);
            acc *= r;
#pragma unroll
            for (int i = 0; i < B; ++i)
                if (i < nc) acc = __builtin_fmaf(__shfl(wc, i), v[i], acc);
            M = Mn;
        }
        st_coh(a.attn + (size_t)l * q_dim + (size_t)(kvh * HPK + hl) * kHD + d, acc / L);
    }
}

template <typename KVT, int HPK>
__device__ __forceinline__ AttnGeo attn_geo(const StepArgs &a, int pos) {
    using C = At<KVT, HPK>;
    AttnGeo g;
    g.pos = pos;
    g.seq = pos + 1;
    g.slots = (int)gridDim.x * C::IPW;
    int cp = (g.seq * a.n_kv + g.slots - 1) / g.slots;
    cp = (cp + 7) & ~7;
    cp = cp < 8 ? 8 : cp > C::CPMAX ? C::CPMAX : cp;
    g.cp = cp;
    g.n_chunks = (g.seq + cp - 1) / cp;
    g.n_items = a.n_kv * g.n_chunks;
    g.rounds = (g.n_items + g.slots - 1) / g.slots;
    return g;
}

__device__ __forceinline__ AttnGeo opaque_geo(const AttnGeo &g0) {
    AttnGeo g;
    g.seq = opaque(g0.seq);
    g.pos = opaque(g0.pos);
    g.cp = opaque(g0.cp);
    g.n_chunks = opaque(g0.n_chunks);
    g.n_items = opaque(g0.n_items);
    g.slots = opaque(g0.slots);
    g.rounds = opaque(g0.rounds);
    return g;
}

template <typename KVT, int HPK>
__device__ __forceinline__ void attn_prefetch(const StepArgs &a, const StepLayer &L,
                                              const AttnGeo &g0, uint4 (&rq)[kQ]) {
    using C = At<KVT, HPK>;
    const AttnGeo g = opaque_geo(g0);
    const int grp = (tid_() >> 6) / HPK;
    attn_load<KVT, HPK>(a, L, g, blockIdx.x * C::IPW + grp, rq);
}

template <typename KVT, int HPK>
__device__ __forceinline__ void attn_phase(const StepArgs &a, const StepLayer &L, int l,
                                           const AttnGeo &g0, uint4 (&rq)[kQ], unsigned char *lds,
                                           int *merge_s) {
    using C = At<KVT, HPK>;
    const AttnGeo g = opaque_geo(g0);
    const int grp = (threadIdx.x >> 6) / HPK;
    for (int r = 0; r < g.rounds; ++r) {
        const int item = r * g.slots + blockIdx.x * C::IPW + grp;
        if (r > 0) attn_load<KVT, HPK>(a, L, g, item, rq);
        attn_round<KVT, HPK>(a, L, l, g, item, rq, lds);
    }
    // arrival per kv head: partials complete, then one atomic per (workgroup,
    // kv head) with the number of chunks this workgroup produced
    drain();
    __syncthreads();
    if (threadIdx.x == 0) {
        int n_merge = 0;
        int cur = -1, cnt = 0;
        for (int r = 0; r <= g.rounds; ++r) {
            for (int k = 0; k < C::IPW; ++k) {
                const int item = r * g.slots + blockIdx.x * C::IPW + k;
                const bool end = r == g.rounds;
                const int kvh = (!end && item < g.n_items) ? item / g.n_chunks : -1;
                if (kvh != cur || end) {
                    if (cur >= 0 && cnt > 0) {
                        const unsigned old = add_cnt(a.sync + kSyncAttn + 32 * cur, (unsigned)cnt);
                        if (old + cnt == (unsigned)g.n_chunks) merge_s[1 + n_merge++] = cur;
                    }
                    cur = kvh;
                    cnt = 0;
                }
                if (kvh >= 0) ++cnt;
                if (end) break;
            }
        }
        merge_s[0] = n_merge;
    }
    __syncthreads();
    const int n_merge = merge_s[0];
    for (int i = 0; i < n_merge; ++i) {
        const int kvh = merge_s[1 + i];
        attn_merge<HPK>(a, l, kvh, g.n_chunks);
        if (threadIdx.x == 0) st_cnt(a.sync + kSyncAttn + 32 * kvh, 0u);
    }
}

// ---------------------------------------------------------------- the step kernel

// The argument block is read through a pointer the optimiser cannot see
// through, re-derived at every phase: its ~30 pointers are loaded where they
// are used instead of being held in registers across the whole step.
__device__ __forceinline__ const StepArgs *fresh(const StepArgs *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    CW_OPAQUE_S(lo);
    CW_OPAQUE_S(hi);
    return reinterpret_cast<const StepArgs *>(((uint64_t)hi << 32) | lo);
}

// The phases of one step, in order: per layer QKV, ATTN, O, GU, DOWN; then LM.
enum { P_QKV = 0, P_ATTN = 1, P_O = 2, P_GU = 3, P_DOWN = 4, P_LM = 5 };

// The kernel's static LDS (one struct, so the host check sizes it exactly).
struct StepShared {
    float red[kW];                       // RMSNorm partial sums per wave
    int ok_s;                            // grid barrier completed
    int merge_s[1 + cwi::kStepMaxKv];    // kv heads this workgroup merges
    float best_v[kW];                    // argmax per wave
    uint32_t best_i[kW];
    int last_s;                          // last workgroup of the argmax merge
};

// The end (bytes) of the dynamic LDS a GEMV phase of input width K touches:
// x as [8][K/32] float4 from offset 0, the block sums from the fixed offset
// 8 * (kMaxK / 32) float4.
__host__ __device__ inline size_t gemv_lds_end(int K) {
    return (size_t)8 * (kMaxK / 32) * 16 + (size_t)(K / 32) * 4;
}
// ... and of an attention phase: IPW item tiles of ILDS bytes each.
template <typename KVT, int HPK>
__host__ __device__ inline size_t attn_lds_end() {
    return (size_t)At<KVT, HPK>::IPW * At<KVT, HPK>::ILDS;
}

// What a GEMV phase reads and writes, from (layer, kind).
struct PhaseSpec {
    const uint8_t *q;
    const uint16_t *sc;
    int N, K;
    int xmode;
    const float *src, *normw;
    float *copy_out;
    int epi;
    float *out;
    const float *resid;
};

// (host and device: the host-side range check walks the same table)
__host__ __device__ inline PhaseSpec phase_spec(const StepArgs &a, int l, int kind, uint32_t token,
                                              bool first_wg) {
    const int q_dim = a.n_heads * kHD, qkv_n = q_dim + 2 * a.n_kv * kHD;
    const float *h_in = l == 0 ? a.embed + (size_t)token * a.dim : a.h_a + (size_t)l * a.dim;
    PhaseSpec f{};
    if (kind == P_LM) {  // final RMSNorm, tied / output head (qwen3.rs:135-137, 190)
        f.q = a.lm_q;
        f.sc = a.lm_s;
        f.N = a.vocab;
        f.K = a.dim;
        f.xmode = X_NORM;
        f.src = a.h_a + (size_t)a.n_layers * a.dim;
        f.normw = a.final_norm;
        f.copy_out = first_wg ? a.hidden_out : nullptr;
        f.epi = E_LOGITS;
        f.out = a.logits;
        return f;
    }
    const StepLayer &L = a.layers[l];
    if (kind == P_QKV) {  // RMSNorm + fused q|k|v projection (qwen3.rs:150-153)
        f.q = L.qkv_q;
        f.sc = L.qkv_s;
        f.N = qkv_n;
        f.K = a.dim;
        f.xmode = X_NORM;
        f.src = h_in;
        f.normw = L.attn_norm;
        f.epi = E_STORE;
        f.out = a.qkv + (size_t)l * qkv_n;
    } else if (kind == P_O) {  // O projection + residual (qwen3.rs:178-179)
        f.q = L.o_q;
        f.sc = L.o_s;
        f.N = a.dim;
        f.K = q_dim;
        f.xmode = X_PLAIN;
        f.src = a.attn + (size_t)l * q_dim;
        f.epi = E_RESID;
        f.out = a.h_b + (size_t)l * a.dim;
        f.resid = h_in;
    } else if (kind == P_GU) {  // RMSNorm + gate|up projection (qwen3.rs:182-184)
        f.q = L.gu_q;
        f.sc = L.gu_s;
        f.N = 2 * a.hidden;
        f.K = a.dim;
        f.xmode = X_NORM;
        f.src = a.h_b + (size_t)l * a.dim;
        f.normw = L.ffn_norm;
        f.epi = E_STORE;
        f.out = a.act + (size_t)l * 2 * a.hidden;
    } else {  // SwiGLU + down projection + residual (qwen3.rs:185-187)
        f.q = L.down_q;
        f.sc = L.down_s;
        f.N = a.dim;
        f.K = a.hidden;
        f.xmode = X_SWIGLU;
        f.src = a.act + (size_t)l * 2 * a.hidden;
        f.epi = E_RESID;
        f.out = a.h_a + (size_t)(l + 1) * a.dim;
        f.resid = a.h_b + (size_t)l * a.dim;
    }
    return f;
}

// ---------------------------------------------------------------- host-side range check

template <typename KVT>
int attn_lds_of(int hpk);

struct RangeCheck {
    const std::vector<cwi::Extent> &ext;
    std::string *why;
    bool ok = true;
    // [p, p + bytes) must lie inside one extent
    void need(const void *p, size_t bytes, const char *what, int layer) {
        if (!ok) return;
        const uintptr_t lo = reinterpret_cast<uintptr_t>(p), hi = lo + bytes;
        for (const auto &e : ext) {
            const uintptr_t b = reinterpret_cast<uintptr_t>(e.p);
            if (lo >= b && hi <= b + e.bytes) return;
        }
        ok = false;
        char buf[224];
        size_t best = 0;
        uintptr_t bb = 0;
        for (const auto &e : ext) {  // the extent the range starts in, if any
            const uintptr_t b = reinterpret_cast<uintptr_t>(e.p);
            if (lo >= b && lo < b + e.bytes) {
                bb = b;
                best = e.bytes;
            }
        }
        if (best)
            snprintf(buf, sizeof buf,
                     "layer %d %s reads/writes %zu bytes at offset %zu of a %zu-byte allocation "
                     "(%zu bytes past its end)",
                     layer, what, bytes, (size_t)(lo - bb), best, (size_t)(hi - (bb + best)));
        else
            snprintf(buf, sizeof buf, "layer %d %s: %zu bytes outside every allocation", layer,
                     what, bytes);
        *why = buf;
    }
};

const char *kPhaseName[6] = {"QKV", "ATTN", "O", "GATE|UP", "DOWN", "LM head"};

}  // namespace

namespace cwi {

bool step_check_ranges(const StepArgs &a, const void *args_dev, const void *layers_dev,
                       int kv_dtype, int head_dim, int n_cu, const std::vector<Extent> &ext,
                       std::string *why) {
    RangeCheck rc{ext, why};
    // the argument block every phase re-reads (`fresh`) and the layer table
    rc.need(args_dev, sizeof(StepArgs), "step argument block", 0);
    rc.need(layers_dev, (size_t)a.n_layers * sizeof(StepLayer), "layer table", 0);
    // LDS: the dynamic size the launch passes must cover every phase's
    // extent, and with the static block fit the CU's 160 KiB
    const int hpk = a.n_heads / a.n_kv;
    const size_t dyn = (size_t)step_lds_bytes(kv_dtype, hpk, a.max_seq);
    const size_t at_end = kv_dtype == CW_F16 ? attn_lds_of<_Float16>(hpk) : attn_lds_of<float>(hpk);
    const int q_dim_i = a.n_heads * head_dim;
    for (int K : {a.dim, q_dim_i, a.hidden}) {
        if (rc.ok && gemv_lds_end(K) > dyn) {
            rc.ok = false;
            *why = "a GEMV phase of input width " + std::to_string(K) + " touches " +
                   std::to_string(gemv_lds_end(K)) + " bytes of LDS, the launch passes " +
                   std::to_string(dyn);
        }
    }
    if (rc.ok && at_end > dyn) {
        rc.ok = false;
        *why = "the attention phase touches " + std::to_string(at_end) +
               " bytes of LDS, the launch passes " + std::to_string(dyn);
    }
    if (rc.ok && dyn + sizeof(StepShared) > (size_t)160 * 1024) {
        rc.ok = false;
        *why = "dynamic + static LDS (" + std::to_string(dyn + sizeof(StepShared)) +
               " bytes) exceed 160 KiB";
    }
    const size_t es = kv_dtype == CW_F16 ? 2 : 4;
    const size_t q_dim = (size_t)a.n_heads * head_dim, kv_dim = (size_t)a.n_kv * head_dim;
    const size_t qkv_n = q_dim + 2 * kv_dim;
    char what[64];
    // GEMV phases: the phase table the kernel uses, for the first and the
    // last token id (layer 0 reads the token's embedding row)
    for (uint32_t token : {0u, (uint32_t)(a.vocab - 1)}) {
        for (int l = 0; l <= a.n_layers; ++l) {
            for (int kind = 0; kind < 5; ++kind) {
                const bool lm = l == a.n_layers;
                if (lm && kind != 0) break;
                const int k = lm ? P_LM : kind;
                if (k == P_ATTN) continue;
                const PhaseSpec f = phase_spec(a, lm ? 0 : l, k, token, true);
                const size_t nblk = (size_t)f.N * (f.K / 32);
                snprintf(what, sizeof what, "%s quants", kPhaseName[k]);
                rc.need(f.q, nblk * 16, what, l);
                snprintf(what, sizeof what, "%s scales", kPhaseName[k]);
                rc.need(f.sc, nblk * 2, what, l);
                snprintf(what, sizeof what, "%s input", kPhaseName[k]);
                rc.need(f.src, (size_t)f.K * 4 * (f.xmode == X_SWIGLU ? 2 : 1), what, l);
                if (f.xmode == X_NORM) {
                    snprintf(what, sizeof what, "%s norm gain", kPhaseName[k]);
                    rc.need(f.normw, (size_t)f.K * 4, what, l);
                }
                if (f.copy_out) {
                    snprintf(what, sizeof what, "%s normed copy", kPhaseName[k]);
                    rc.need(f.copy_out, (size_t)f.K * 4, what, l);
                }
                snprintf(what, sizeof what, "%s output", kPhaseName[k]);
                rc.need(f.out, (size_t)f.N * 4, what, l);
                if (f.epi == E_RESID) {
                    snprintf(what, sizeof what, "%s residual", kPhaseName[k]);
                    rc.need(f.resid, (size_t)f.N * 4, what, l);
                }
            }
        }
    }
    // attention phases: raw q|k|v row, QK-norm gains, RoPE rows of every
    // position, the whole cache of the layer, the chunk partials, the output
    const size_t half = (size_t)head_dim / 2;
    for (int l = 0; l < a.n_layers; ++l) {
        const StepLayer &L = a.layers[l];
        rc.need(a.qkv + (size_t)l * qkv_n, qkv_n * 4, "ATTN q|k|v", l);
        rc.need(L.q_norm, (size_t)head_dim * 4, "ATTN q norm gain", l);
        rc.need(L.k_norm, (size_t)head_dim * 4, "ATTN k norm gain", l);
        rc.need(a.cos_t, (size_t)a.max_seq * half * 4, "ATTN RoPE cos", l);
        rc.need(a.sin_t, (size_t)a.max_seq * half * 4, "ATTN RoPE sin", l);
        rc.need(L.kc, (size_t)a.max_seq * kv_dim * es, "ATTN K cache", l);
        rc.need(L.vc, (size_t)a.max_seq * kv_dim * es, "ATTN V cache", l);
        rc.need(a.part, (size_t)a.n_heads * a.max_chunks * (head_dim + 2) * 4, "ATTN partials", l);
        rc.need(a.attn + (size_t)l * q_dim, q_dim * 4, "ATTN output", l);
    }
    // at most (max_seq + 7) / 8 chunks (8-position minimum) fit the partials
    if (rc.ok && (a.max_seq + 7) / 8 > a.max_chunks) {
        rc.ok = false;
        *why = "attention partials hold fewer chunks than the cache can need";
    }
    // the argmax merge (one slot per workgroup: the grid is one workgroup
    // per CU), the counters and the decode state
    rc.need(a.am_v, (size_t)n_cu * 4, "LM head argmax values", a.n_layers);
    rc.need(a.am_i, (size_t)n_cu * 4, "LM head argmax ids", a.n_layers);
    rc.need(a.sync, step_sync_words() * 4, "grid counters", a.n_layers);
    rc.need(a.hidden_out, (size_t)a.dim * 4, "final hidden state", a.n_layers);
    rc.need(a.state, sizeof(GenState), "decode state", a.n_layers);
    rc.need(a.prompt, (size_t)a.max_seq * 4, "prompt ids", a.n_layers);
    rc.need(a.tokens, (size_t)a.max_seq * 4, "produced ids", a.n_layers);
    rc.need(a.argmax_out, 4, "argmax output", a.n_layers);
    // the phase stamps, when on: [2e], [2e + 1] per barrier e <= 5L, the
    // end at [10L + 2], two per phase from [10L + 4]
    if (a.trace)
        rc.need(a.trace, step_trace_words(a.n_layers) * 8, "phase stamps", a.n_layers);
    return rc.ok;
}

size_t step_trace_words(int n_layers) { return (size_t)20 * n_layers + 8; }

}  // namespace cwi

namespace {

// The step is a loop over its phase list, so each kind of work exists once in
// the code: the loop body stays small enough for the instruction cache.
template <typename KVT, int HPK>
__global__ __launch_bounds__(kT) void decode_step_kernel(const StepArgs *__restrict__ ap) {
    CW_WG_DYNAMIC(float4, lds4);
    CW_WG_SHARED(StepShared, sh);
    float *red = sh.red;
    int &ok_s = sh.ok_s;
    int *merge_s = sh.merge_s;
    float *best_v = sh.best_v;
    uint32_t *best_i = sh.best_i;
    int &last_s = sh.last_s;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gw = blockIdx.x * kW + wave, nw = gridDim.x * kW;
    float *sx = reinterpret_cast<float *>(lds4 + 8 * (kMaxK / 32));
    unsigned char *lds = reinterpret_cast<unsigned char *>(lds4);

    int pos, n_layers;
    uint32_t token;
    {
        const StepArgs &a = *fresh(ap);
        pos = a.state->pos;
        if (pos < 0 || pos >= a.max_seq) {  // no room for the new KV row: report, touch nothing
            if (tid == 0 && blockIdx.x == 0) st_cnt(a.sync + kSyncErr, 2u);
            return;
        }
        token = a.state->token;
        token = token < (uint32_t)a.vocab ? token : (uint32_t)(a.vocab - 1);
        n_layers = a.n_layers;
        if (a.trace && blockIdx.x == 0 && tid == 0) a.trace[0] = wall_clock64();
    }
    Ctl ctl{nullptr, 0, 0u, nullptr};
    uint4 rq[kQ];
    uint32_t rd[kQ];
    Best best{kNegInit, 0u};
    AttnGeo geo;
    Gemv p;
    {
        const StepArgs &a = *fresh(ap);
        geo = attn_geo<KVT, HPK>(a, pos);
        const PhaseSpec f = phase_spec(a, 0, P_QKV, token, blockIdx.x == 0);
        p = gemv_setup(f.q, f.sc, f.N, f.K, gw, nw);
        gemv_prefetch(p, rq, rd);
    }
    // sub-phase stamps (workgroup 0): k = 0 after staging, k = 1 after compute
    auto mark = [&](const StepArgs &a, int ph, int k) {
        if (a.trace && blockIdx.x == 0 && tid == 0)
            a.trace[10 * n_layers + 4 + ph * 2 + k] = wall_clock64();
    };
    const int nph = 5 * n_layers + 1;
    for (int ph = 0; ph < nph; ++ph) {
        const int l = ph / 5, kind = ph == nph - 1 ? P_LM : ph % 5;
        {
            const StepArgs &a = *fresh(ap);
            if (kind == P_ATTN) {  // QK-norm, RoPE, KV write, attention (qwen3.rs:154-177)
                attn_phase<KVT, HPK>(a, a.layers[l], l, geo, rq, lds, merge_s);
            } else {
                const PhaseSpec f = phase_spec(a, l, kind, token, blockIdx.x == 0);
                stage_x(f.xmode, f.src, f.normw, f.K, a.eps, lds4, sx, red, f.copy_out,
                        [&] { gemv_fill(p, rq, rd); });
                mark(a, ph, 0);
                gemv_run(p, rq, rd, lds4, sx, Epi{f.epi, f.out, f.resid}, best);
            }
            mark(a, ph, 1);
        }
        if (ph + 1 == nph) break;
        {  // barrier; the next phase's first loads go out while it completes
            const StepArgs &a = *fresh(ap);
            ctl.sync = a.sync;
            ctl.timeout = a.timeout;
            ctl.trace = a.trace;
            bar_arrive(ctl);
            const int nl = (ph + 1) / 5, nk = ph + 2 == nph ? P_LM : (ph + 1) % 5;
            if (nk == P_ATTN) {
                attn_prefetch<KVT, HPK>(a, a.layers[nl], geo, rq);
            } else {
                const PhaseSpec f = phase_spec(a, nl, nk, token, blockIdx.x == 0);
                p = gemv_setup(f.q, f.sc, f.N, f.K, gw, nw);
                gemv_prefetch(p, rq, rd);
            }
            if (!bar_wait(ctl, &ok_s)) return;
        }
    }
    const StepArgs &a = *fresh(ap);
    if (a.trace && blockIdx.x == 0 && tid == 0) a.trace[10 * n_layers + 2] = wall_clock64();
    best = wave_best(best);
    if (lane == 0) {
        best_v[wave] = best.v;
        best_i[wave] = best.i;
    }
    __syncthreads();
    if (tid == 0) {
        Best b{best_v[0], best_i[0]};
        for (int w = 1; w < kW; ++w) b = better(b, Best{best_v[w], best_i[w]});
        st_coh(a.am_v + blockIdx.x, b.v);
        st_coh(reinterpret_cast<float *>(a.am_i) + blockIdx.x, __builtin_bit_cast(float, b.i));
        drain();
        const unsigned old = add_cnt(a.sync + kSyncArgmax, 1u);
        last_s = old + 1 == gridDim.x;
    }
    __syncthreads();
    if (!last_s) return;
    // the last workgroup: merge, advance the generate state (mod.rs:114-122),
    // reset the counters for the next launch
    Best b{kNegInit, 0u};
    for (int i = tid; i < (int)gridDim.x; i += kT)
        b = better(b, Best{ld_coh(a.am_v + i),
                           __builtin_bit_cast(uint32_t, ld_coh(reinterpret_cast<float *>(a.am_i) + i))});
    b = wave_best(b);
    if (lane == 0) {
        best_v[wave] = b.v;
        best_i[wave] = b.i;
    }
    __syncthreads();
    if (tid == 0) {
        Best r{best_v[0], best_i[0]};
        for (int w = 1; w < kW; ++w) r = better(r, Best{best_v[w], best_i[w]});
        if (a.argmax_out) *a.argmax_out = r.i;
        cwi::GenState *st = a.state;
        const int pr = st->pos - st->start_pos;
        if (pr + 1 < st->n_prompt) {
            st->token = a.prompt[pr + 1];
        } else {
            if (st->produced < st->max_out) a.tokens[st->produced] = r.i;
            st->produced += 1;
            st->token = r.i;
        }
        st->pos += 1;
        for (int g = 0; g < kTreeG; ++g) st_cnt(a.sync + g * 32, 0u);
        st_cnt(a.sync + kSyncRoot, 0u);
        st_cnt(a.sync + kSyncArgmax, 0u);
    }
}

typedef void (*step_fn)(const StepArgs *);

template <typename KVT>
step_fn pick_hpk(int hpk) {
    switch (hpk) {
        case 1: return decode_step_kernel<KVT, 1>;
        case 2: return decode_step_kernel<KVT, 2>;
        case 4: return decode_step_kernel<KVT, 4>;
        case 8: return decode_step_kernel<KVT, 8>;
        default: return nullptr;
    }
}

template <typename KVT>
int cpmax_of(int hpk) {
    switch (hpk) {
        case 1: return At<KVT, 1>::CPMAX;
        case 2: return At<KVT, 2>::CPMAX;
        case 4: return At<KVT, 4>::CPMAX;
        case 8: return At<KVT, 8>::CPMAX;
        default: return 0;
    }
}

template <typename KVT>
int attn_lds_of(int hpk) {
    switch (hpk) {
        case 1: return At<KVT, 1>::IPW * At<KVT, 1>::ILDS;
        case 2: return At<KVT, 2>::IPW * At<KVT, 2>::ILDS;
        case 4: return At<KVT, 4>::IPW * At<KVT, 4>::ILDS;
        case 8: return At<KVT, 8>::IPW * At<KVT, 8>::ILDS;
        default: return 0;
    }
}

std::mutex g_mu;
std::map<const void *, bool> g_attr;

}  // namespace

namespace cwi {

size_t step_sync_words() { return (size_t)kSyncErr + 32; }
int step_sync_err_index() { return kSyncErr; }

int step_cpmax(int kv_dtype, int hpk) {
    return kv_dtype == CW_F16 ? cpmax_of<_Float16>(hpk) : cpmax_of<float>(hpk);
}

int step_lds_bytes(int kv_dtype, int hpk, int max_seq) {
    const int x_bytes = 8 * (kMaxK / 32) * 16 + (kMaxK / 32) * 4;
    const int at = kv_dtype == CW_F16 ? attn_lds_of<_Float16>(hpk) : attn_lds_of<float>(hpk);
    (void)max_seq;
    return x_bytes > at ? x_bytes : at;
}

const char *step_unsupported(int head_dim, int hpk, int n_kv, int dim, int q_dim, int hidden,
                             int max_seq) {
    if (head_dim != kHD) return "head_dim must be 128";
    if (hpk != 1 && hpk != 2 && hpk != 4 && hpk != 8) return "heads per kv head not in {1,2,4,8}";
    if (n_kv > kStepMaxKv) return "too many kv heads";
    if (dim > kMaxK || q_dim > kMaxK || hidden > kMaxK) return "GEMV width above 16384";
    if (dim % 256 || q_dim % 256 || hidden % 256) return "widths must be multiples of 256";
    (void)max_seq;
    return nullptr;
}

int launch_decode_step(cw_ctx *ctx, const StepArgs *a_dev, int kv_dtype, int hpk, int max_seq) {
    step_fn fn = kv_dtype == CW_F16 ? pick_hpk<_Float16>(hpk) : pick_hpk<float>(hpk);
    if (!fn) {
        set_error("decode step: unsupported heads per kv head %d", hpk);
        return CW_ERR_ARG;
    }
    const int lds = step_lds_bytes(kv_dtype, hpk, max_seq);
    {
        std::lock_guard<std::mutex> lk(g_mu);
        const void *f = reinterpret_cast<const void *>(fn);
        if (!g_attr[f]) {
            CW_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
            int occ = 0;
            CW_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kT, (size_t)lds));
            if (occ < 1) {
                set_error("decode step: kernel does not fit one workgroup per CU (lds %d)", lds);
                return CW_ERR_ARG;
            }
            g_attr[f] = true;
        }
    }
    const StepArgs *args = a_dev;
    void *kargs[] = {&args};
    prof_begin(ctx, "decode_step");
    hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void *>(fn), dim3(ctx->n_cu),
                                              dim3(kT), kargs, (unsigned)lds, ctx->stream);
    prof_end(ctx);
    if (e != hipSuccess) return hip_fail(e, "hipLaunchCooperativeKernel(decode_step)", __FILE__, __LINE__);
    return CW_OK;
}

}  // namespace cwi
