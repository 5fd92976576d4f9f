// Q4_0 dequant-fused GEMV for gfx950 (decode, one token).
//
// Replaces q4::gemv (src/kernels/q4.rs:9-30) and its shader q4.wgsl:25-82.
// Same arithmetic identity as the shader, y[o] = sum_b d[o,b] *
// (sum_j q_j x_j - 8 * sum_j x_j), over GGUF Q4_0 blocks kept packed in HBM.
//
// Layout in HBM (split GGUF Q4_0): quants [N][K/32][16] bytes (one 128-bit
// load per block), scales [N][K/32] f16.  Byte j of a block holds element j
// in its low nibble and element j+16 in its high nibble.
//
// Work split: a wave64 covers 64 blocks per step.  G = lanes per row (the
// largest power of two <= 64 dividing K/32); 64/G rows share a wave step.
// A wave tile is R row slots x all K; waves walk wave tiles over a
// persistent grid of 1024-thread workgroups (two per CU, all resident ones
// for the LM head; launches with fewer tiles one per CU, only some of whose
// waves take tiles), so the activation is staged into LDS once per
// workgroup: [8][K/32] float4 (conflict-free: lane b reads float4 i of block
// b) plus the per-block sums sum_j x_j.
//
// Latency: every wave issues the loads of its first (tile, step) group before
// the activation is staged, and each iteration issues the next group's loads
// (crossing tile boundaries) before computing the current one.  Latency is
// hidden by occupancy (32 waves per CU within 64 VGPRs) rather than by a deep
// per-wave register ring, which measured slower.
//
// Nibble decode costs 5 VALU ops per 8 weights: AND-ing a quant dword with
// 0x000F000F / 0x00F000F0 (and the same after one >>8) leaves two f16
// *subnormals* whose values are q*2^-24 and q*2^-20 exactly.  v_fma_mix_f32
// widens either f16 half to f32 inside the FMA, so with the LDS copy of x
// pre-scaled by 2^24 (elements 0..15 of a block) and 2^20 (elements 16..31)
// each weight costs one fma_mix: q*x accumulated in f32 with no rounding
// beyond the reference's own multiply-add.  8 fma_mix + 5 bit ops per 8
// weights keeps the VALU below the HBM rate on 256 CUs.
//
// Optional prologue: RMSNorm of the raw hidden state (norm.wgsl:20-42) in the
// same single pass that stages x: x*w is staged and 1/rms(x), a scalar of the
// row, scales each output sum (the same value up to f32 rounding order).
// Optional epilogues: residual add (ewise.wgsl:9-13) and SwiGLU of a gate/up
// row pair (glu.wgsl:22-26).

#include <algorithm>
#include <map>
#include <mutex>

#include "cw_internal.hpp"

namespace {

using cwi::GemvArgs;

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// All-reduce sum within aligned groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (G >= 4) v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (G >= 8) v += dpp<0x141>(v);  // row_half_mirror
    if constexpr (G >= 16) v += dpp<0x140>(v); // row_mirror
    if constexpr (G >= 32) v += __shfl_xor(v, 16);
    if constexpr (G >= 64) v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ float f16lo(uint32_t v) {
    return (float)__builtin_bit_cast(half2v, v).x;
}
__device__ __forceinline__ float f16hi(uint32_t v) {
    return (float)__builtin_bit_cast(half2v, v).y;
}

// sum_j q_j * x_j over one quant dword; xl = 2^24 * x[4w..4w+3],
// xh = 2^20 * x[16+4w..16+4w+3].
__device__ __forceinline__ float dot_word(uint32_t dw, float4 xl, float4 xh, float s) {
    const uint32_t a = dw & 0x000F000Fu;          // elements 4w+0, 4w+2     (q * 2^-24)
    const uint32_t b = dw & 0x00F000F0u;          // elements 16+4w+0, +2    (q * 2^-20)
    const uint32_t d8 = dw >> 8;
    const uint32_t c = d8 & 0x000F000Fu;          // elements 4w+1, 4w+3
    const uint32_t e = d8 & 0x00F000F0u;          // elements 16+4w+1, +3
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

// ---- argmax over the launch (argmax.wgsl:18-55): candidates need v above
// kNegInit (strict, so NaN never wins), the lowest index among equal values
struct Best {
    float v;
    uint32_t i;
};
constexpr float kNegInit = -3.402823e38f;

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

// The workgroup's best goes to memory write-through (am_v/am_i[block]); its
// stores are complete before one agent-scope increment of the counter; the
// last workgroup to arrive reads every best with agent-scope loads, writes
// the argmax and advances the generate state (mod.rs:114-122: feed
// prompt[p+1] inside the prompt, else record the argmax and feed it back),
// and resets the counter for the next launch.
__device__ __forceinline__ void argmax_tail(const GemvArgs &a, Best best, int tid, int lane,
                                          int wave) {
    __shared__ float bv[kWaves];
    __shared__ uint32_t bi[kWaves];
    __shared__ int last_s;
    best = wave_best(best);
    if (lane == 0) {
        bv[wave] = best.v;
        bi[wave] = best.i;
    }
    __syncthreads();
    if (tid == 0) {
        Best r{bv[0], bi[0]};
        for (int w = 1; w < kWaves; ++w) r = better(r, Best{bv[w], bi[w]});
        __hip_atomic_store(a.am_v + blockIdx.x, r.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.am_i + blockIdx.x, r.i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        const unsigned old = __hip_atomic_fetch_add(a.am_cnt, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old + 1 == gridDim.x;
        if (last) __hip_atomic_store(a.am_cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_s = last;
    }
    __syncthreads();
    if (!last_s) return;
    Best b{kNegInit, 0u};
    for (int i = tid; i < (int)gridDim.x; i += kThreads)
        b = better(b, Best{__hip_atomic_load(a.am_v + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                           __hip_atomic_load(a.am_i + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)});
    b = wave_best(b);
    __syncthreads();  // every wave is done with bv / bi above
    if (lane == 0) {
        bv[wave] = b.v;
        bi[wave] = b.i;
    }
    __syncthreads();
    if (tid == 0) {
        Best r{bv[0], bi[0]};
        for (int w = 1; w < kWaves; ++w) r = better(r, Best{bv[w], bi[w]});
        if (a.am_out) *a.am_out = r.i;
        cwi::GenState *st = a.state;
        if (st) {
            const int p = st->pos - st->start_pos;
            if (p + 1 < st->n_prompt) {
                st->token = a.prompt[p + 1];
            } else {
                if (st->produced < st->max_out) a.tokens[st->produced] = r.i;
                st->produced += 1;
                st->token = r.i;
            }
            st->pos += 1;
        }
    }
}

template <int G, int R, int EPI>
struct Tile {
    static constexpr int RPS = 64 / G;                         // rows per wave step
    static constexpr int NR = (EPI == cwi::EPI_SWIGLU) ? R / 2 : R;  // distinct rows
    static constexpr int ROWS = NR * RPS;                      // rows per wave tile
};

// Issue the loads of one (tile, block) group: R quant blocks + R scales.
template <int G, int R, int EPI>
__device__ __forceinline__ void load_group(const GemvArgs &a, int nb, int wt, int b, int rl,
                                           uint4 (&qv)[R], uint32_t (&dv)[R]) {
    using T = Tile<G, R, EPI>;
    const int row0 = wt * T::ROWS;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int row = row0 + (r % T::NR) * T::RPS + rl;
        row = row < a.N ? row : a.N - 1;
        const bool second = (EPI == cwi::EPI_SWIGLU) && r >= T::NR;
        const uint8_t *qb = second ? a.qB : a.qA;
        const uint16_t *sb = second ? a.sB : a.sA;
        qv[r] = reinterpret_cast<const uint4 *>(qb)[(size_t)row * nb + b];
        dv[r] = sb[(size_t)row * nb + b];
    }
}

// Occupancy over prefetch depth: at most 64 VGPRs (8 waves per SIMD, two or
// more workgroups per CU) with PD = 1 or 2 groups in flight per wave streams
// faster than one workgroup per CU with a deep register ring (measured on
// MI355X: 13-26 % less time on the 4096- and 12288-wide layers).
template <int G, int R, int XS, int EPI, int PD>
__global__ __launch_bounds__(kThreads, 8) void q4_gemv_kernel(GemvArgs a, int n_wave_tiles) {
    using T = Tile<G, R, EPI>;
    extern __shared__ float4 lds4[];
    __shared__ float red[kWaves];
    const int K = a.K;
    const int nb = K >> 5;
    const int K4 = K >> 2;
    const int S = nb / G;  // steps per tile
    float *sx = reinterpret_cast<float *>(lds4 + 8 * nb);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform: keeps tile/row/address arithmetic in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int s = lane & (G - 1);
    const int rl = lane / G;

    // this wave's tiles: wv, wv + stride, ... (the first tile_waves waves of
    // each workgroup take tiles; the others only stage the activation, and
    // their unused first loads re-read this workgroup's own last tile, in
    // cache, not the next workgroup's)
    const int tw = a.tile_waves ? a.tile_waves : kWaves;
    const int wv = blockIdx.x * tw + (wave < tw ? wave : tw - 1);
    const int stride = gridDim.x * tw;
    const int n_my = (wave < tw && wv < n_wave_tiles) ? (n_wave_tiles - 1 - wv) / stride + 1 : 0;
    const int total = n_my * S;

    // a ring of PD (tile, block) groups in flight per wave, issued before the
    // activation is staged; slot u always holds group it with it % PD == u
    // the activation gates the first compute, so its loads go out ahead of
    // the weights (loads return in issue order); K <= 12288 stays in
    // registers across the weight issue (K <= 4096 with a norm gain)
    constexpr int kXR = XS == cwi::XS_RMSNORM ? 1 : 3;
    const float *xsrc = a.x;
    if (a.x_tok) {  // the embedding row of the device-resident token
        uint32_t t = *a.x_tok;
        t = t < (uint32_t)a.tok_rows ? t : (uint32_t)(a.tok_rows - 1);
        xsrc = a.x + (size_t)t * K;
    }
    const float4 *x4 = reinterpret_cast<const float4 *>(xsrc);
    const float4 *w4 = reinterpret_cast<const float4 *>(a.norm_w);
    float4 xv[kXR], wn[kXR];
#pragma unroll
    for (int j = 0; j < kXR; ++j) {
        const int idx = tid + j * kThreads;
        const int ci = idx < K4 ? idx : K4 - 1;
        xv[j] = x4[ci];
        if constexpr (XS == cwi::XS_RMSNORM) wn[j] = w4[ci];
    }

    // The activation lands before the first weight groups are requested:
    // issued together, its loads queue behind the whole chip's weight
    // requests (2.4 us to staging, against about 1.1 us alone; QKV 0.6 us and
    // O 0.35 us faster per launch, the long launches unchanged).  The first
    // PD groups are then issued on every path (a wave with fewer groups
    // re-reads an in-range one, unused), so the compiler's wait counts stay
    // exact; the scheduling barriers keep this order.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    uint4 qv[PD][R];
    uint32_t dv[PD][R];
    int lk = 0, lstep = 0;  // next group to load
#pragma unroll
    for (int u = 0; u < PD; ++u) {
        const bool have = u < total;
        load_group<G, R, EPI>(a, nb, wv + lk * stride, s + (have ? lstep : 0) * G, rl, qv[u],
                              dv[u]);
        if (have && ++lstep == S) {
            lstep = 0;
            ++lk;
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- stage the activation in one pass: x (times the norm gain) into
    // LDS pre-scaled, with its block sums; the RMS factor 1/rms(x) is a
    // scalar of the whole row, so it multiplies the row sums in the
    // epilogue instead of every element here ----
    float ss = 0.0f;
    auto stage = [&](int idx, float4 v, float4 w) {
        if constexpr (XS == cwi::XS_RMSNORM) {
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            v.x *= w.x;
            v.y *= w.y;
            v.z *= w.z;
            v.w *= w.w;
        }
        const int blk = idx >> 3, i = idx & 7;
        const float sc = i < 4 ? 0x1p24f : 0x1p20f;
        lds4[i * nb + blk] = make_float4(v.x * sc, v.y * sc, v.z * sc, v.w * sc);
        // the 8 float4 of a block sit in 8 consecutive lanes (K4 is a
        // multiple of 8, so they are active together)
        float part = (v.x + v.y) + (v.z + v.w);
        part = group_sum<8>(part);
        if (i == 0) sx[blk] = part;
    };
#pragma unroll
    for (int j = 0; j < kXR; ++j) {
        const int idx = tid + j * kThreads;
        if (idx < K4) stage(idx, xv[j], wn[j]);
    }
    for (int idx = tid + kXR * kThreads; idx < K4; idx += kThreads)
        stage(idx, x4[idx], XS == cwi::XS_RMSNORM ? w4[idx] : make_float4(0, 0, 0, 0));
    if constexpr (XS == cwi::XS_RMSNORM) {
        ss = group_sum<64>(ss);
        if (lane == 0) red[wave] = ss;
    }
    // LDS-only barrier: a __syncthreads fence would also wait for the weight
    // groups in flight, which staging does not read
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    float inv = 1.0f;
    if constexpr (XS == cwi::XS_RMSNORM) {
        ss = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) ss += red[w];
        inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    }

    // ---- stream the weights ----
    const float *rsrc = a.resid;
    if constexpr (EPI == cwi::EPI_ADD) {
        if (a.resid_tok) {  // the residual is the embedding row (first layer)
            uint32_t t = *a.resid_tok;
            t = t < (uint32_t)a.tok_rows ? t : (uint32_t)(a.tok_rows - 1);
            rsrc = a.resid + (size_t)t * a.N;
        }
    }
    Best best{kNegInit, 0u};  // EPI_ARGMAX: this lane's best row so far
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    int k = 0, step = 0;  // group being computed
    for (int base = 0; base < total; base += PD) {
#pragma unroll
        for (int u = 0; u < PD; ++u) {
            if (base + u < total) {
                const int b = s + step * G;
                const float sxb = sx[b];
                // one accumulator per (row, quant dword): independent fma_mix
                // chains interleave without dependency stalls; x is read per
                // dword (2 float4) to keep the register budget
                float sum[R][4];
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const float4 xl = lds4[w * nb + b], xh = lds4[(4 + w) * nb + b];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint4 q = qv[u][r];
                        const uint32_t dw = w == 0 ? q.x : w == 1 ? q.y : w == 2 ? q.z : q.w;
                        sum[r][w] = dot_word(dw, xl, xh, 0.0f);
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float sr = (sum[r][0] + sum[r][1]) + (sum[r][2] + sum[r][3]);
                    const float t = __builtin_fmaf(-8.0f, sxb, sr);
                    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)dv[u][r]);
                    acc[r] = __builtin_fmaf((float)d, t, acc[r]);
                }
                // refill this slot with the group PD ahead; past the wave's
                // last group re-load that group (a cache hit) so the refill
                // needs no branch
                {
                    const bool past = lk >= n_my;
                    load_group<G, R, EPI>(a, nb, wv + (past ? n_my - 1 : lk) * stride,
                                          s + (past ? S - 1 : lstep) * G, rl, qv[u], dv[u]);
                    if (!past && ++lstep == S) {
                        lstep = 0;
                        ++lk;
                    }
                }
                if (step == S - 1) {  // tile done: reduce over the G lanes of each row, write
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        acc[r] = group_sum<G>(acc[r]);
                        if constexpr (XS == cwi::XS_RMSNORM) acc[r] *= inv;
                    }
                    if (s == 0) {
                        const int row0 = (wv + k * stride) * T::ROWS;
#pragma unroll
                        for (int rr = 0; rr < T::NR; ++rr) {
                            const int row = row0 + rr * T::RPS + rl;
                            if (row < a.N) {
                                if constexpr (EPI == cwi::EPI_STORE) {
                                    a.y[row] = acc[rr];
                                } else if constexpr (EPI == cwi::EPI_ARGMAX) {
                                    a.y[row] = acc[rr];
                                    best = better(best, Best{acc[rr], (uint32_t)row});
                                } else if constexpr (EPI == cwi::EPI_ADD) {
                                    a.y[row] = rsrc[row] + acc[rr];
                                } else {
                                    const float g = acc[rr], up = acc[rr + T::NR];
                                    const float sg = g / (1.0f + expf(-g));
                                    a.y[row] = sg * up;
                                }
                            }
                        }
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
                }
                if (++step == S) {
                    step = 0;
                    ++k;
                }
            }
        }
    }
    if constexpr (EPI == cwi::EPI_ARGMAX) argmax_tail(a, best, tid, lane, wave);
}

typedef void (*gemv_fn)(GemvArgs, int);

template <int G, int R, int XS, int PD>
gemv_fn pick_epi(int epi) {
    switch (epi) {
        case cwi::EPI_STORE: return q4_gemv_kernel<G, R, XS, cwi::EPI_STORE, PD>;
        case cwi::EPI_ADD: return q4_gemv_kernel<G, R, XS, cwi::EPI_ADD, PD>;
        case cwi::EPI_ARGMAX:
            if constexpr (XS == cwi::XS_RMSNORM) return q4_gemv_kernel<G, R, XS, cwi::EPI_ARGMAX, PD>;
            return nullptr;
        default:
            if constexpr (R % 2 == 0) return q4_gemv_kernel<G, R, XS, cwi::EPI_SWIGLU, PD>;
            return nullptr;
    }
}

template <int G, int R, int PD>
gemv_fn pick_xs(int xs, int epi) {
    return xs == cwi::XS_RMSNORM ? pick_epi<G, R, cwi::XS_RMSNORM, PD>(epi)
                                 : pick_epi<G, R, cwi::XS_PLAIN, PD>(epi);
}

// PD: one group in flight per wave, two for single-row tiles of long rows
// (steps per tile S >= 3), where it measured faster (3072 x 1024: 4.8-4.9
// against 5.2 us; at S = 2, 4096 x 4096, one group is faster).
template <int G>
gemv_fn pick_r(int r, int xs, int epi, bool deep) {
    if (r == 2) return pick_xs<G, 2, 1>(xs, epi);
    return deep ? pick_xs<G, 1, 2>(xs, epi) : pick_xs<G, 1, 1>(xs, epi);
}

gemv_fn pick(int g, int r, int xs, int epi, bool deep) {
    switch (g) {
        case 64: return pick_r<64>(r, xs, epi, deep);
        case 32: return pick_r<32>(r, xs, epi, deep);
        case 16: return pick_r<16>(r, xs, epi, deep);
        case 8: return pick_r<8>(r, xs, epi, deep);
        case 4: return pick_r<4>(r, xs, epi, deep);
        case 2: return pick_r<2>(r, xs, epi, deep);
        default: return pick_r<1>(r, xs, epi, deep);
    }
}

struct OccKey {
    const void *fn;
    int lds;
    bool operator<(const OccKey &o) const { return fn != o.fn ? fn < o.fn : lds < o.lds; }
};

std::mutex g_occ_mu;
std::map<OccKey, int> g_occ;
std::map<const void *, bool> g_attr_set;

int occupancy(gemv_fn fn, int lds, int *blocks) {
    std::lock_guard<std::mutex> lk(g_occ_mu);
    const void *f = reinterpret_cast<const void *>(fn);
    if (!g_attr_set[f]) {
        // static + dynamic LDS of a workgroup must fit the CU's 160 KB
        hipFuncAttributes attr{};
        CW_HIP(hipFuncGetAttributes(&attr, f));
        const int max_dyn = 160 * 1024 - (int)attr.sharedSizeBytes;
        CW_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, max_dyn));
        g_attr_set[f] = true;
    }
    OccKey k{f, lds};
    auto it = g_occ.find(k);
    if (it != g_occ.end()) {
        *blocks = it->second;
        return CW_OK;
    }
    int nb = 0;
    CW_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, kThreads, (size_t)lds));
    if (nb < 1) nb = 1;
    g_occ[k] = nb;
    *blocks = nb;
    return CW_OK;
}

const char *label_of(int xs, int epi) {
    static const char *names[2][4] = {
        {"q4_gemv", "q4_gemv_add", "q4_gemv_swiglu", "q4_gemv_argmax"},
        {"q4_gemv_rmsnorm", "q4_gemv_rmsnorm_add", "q4_gemv_rmsnorm_swiglu",
         "q4_gemv_rmsnorm_argmax"}};
    return names[xs][epi];
}

}  // namespace

namespace cwi {

int launch_q4_gemv(cw_ctx *ctx, XSrc xs, Epi epi, const GemvArgs &a) {
    const int nb = a.K / 32;
    int g = 64;
    while (g > 1 && nb % g) g >>= 1;
    const int rps = 64 / g;
    auto tiles_for = [&](int r) {
        const int nr = epi == EPI_SWIGLU ? r / 2 : r;
        const int rows = nr * rps;
        return (a.N + rows - 1) / rows;
    };
    // R (row slots per wave tile) and the grid, as measured fastest on MI355X
    // over the Qwen3 shapes: two-row tiles (gate/up pairs for SwiGLU) unless
    // that leaves more than a quarter of the CUs without a workgroup, in which
    // case single rows (e.g. 4096 x 4096: 4.8 us against 5.8); grids of two
    // workgroups per CU, four for long streams (>= 8 tiles per wave of two
    // workgroups per CU, e.g. the LM head: 62 us against 66).
    const int r = (epi == EPI_SWIGLU ||
                   4 * ((tiles_for(2) + kWaves - 1) / kWaves) >= 3 * ctx->n_cu)
                      ? 2
                      : 1;
    const int n_tiles = tiles_for(r);
    gemv_fn fn = pick(g, r, xs, epi, nb / g >= 3);
    const int lds = nb * 132;
    int occ = 1;
    CW_TRY(occupancy(fn, lds, &occ));  // raises the kernel's LDS limit
    (void)occ;
    const bool long_stream = n_tiles >= 16 * ctx->n_cu * kWaves;
    int grid = (n_tiles + kWaves - 1) / kWaves;
    const int cap = (long_stream ? 4 : 2) * ctx->n_cu;
    if (grid > cap) grid = cap;
    // Too few tiles for a workgroup on every CU: spread them over one
    // workgroup per CU with fewer waves taking tiles each, so every CU's
    // memory pipeline carries part of the stream (Qwen3-0.6B shape, token
    // loop 1491-1494 against 1427-1461 tokens/s; 8B QKV 6144 x 4096 at 12
    // waves on 256 CUs, 5.75-5.82 against 6.06-6.11 us)
    GemvArgs spread = a;
    if (grid < ctx->n_cu) {
        spread.tile_waves = (n_tiles + ctx->n_cu - 1) / ctx->n_cu;
        grid = (n_tiles + spread.tile_waves - 1) / spread.tile_waves;
    }
    return launch(ctx, label_of(xs, epi), fn, dim3(grid), dim3(kThreads), lds, spread, n_tiles);
}

size_t lm_argmax_scratch_bytes(const cw_ctx *ctx) {
    // bests for up to four workgroups per CU (launch_q4_gemv's largest grid),
    // then the counter on its own 128-byte line
    return (size_t)4 * ctx->n_cu * 8 + 256;
}

int launch_lm_head_argmax(cw_ctx *ctx, GemvArgs g, void *scratch, uint32_t *out_dev,
                          GenState *state, const uint32_t *prompt_dev, uint32_t *tokens_out_dev) {
    const size_t cap = (size_t)4 * ctx->n_cu;
    unsigned char *base = static_cast<unsigned char *>(scratch);
    g.am_v = reinterpret_cast<float *>(base);
    g.am_i = reinterpret_cast<uint32_t *>(base + cap * 4);
    g.am_cnt = reinterpret_cast<unsigned *>(base + ((cap * 8 + 127) & ~(size_t)127));
    g.am_out = out_dev;
    g.state = state;
    g.prompt = prompt_dev;
    g.tokens = tokens_out_dev;
    return launch_q4_gemv(ctx, XS_RMSNORM, EPI_ARGMAX, g);
}

}  // namespace cwi

using namespace cwi;

static int check_q4_shape(const char *what, int in_f, int out_f) {
    CW_CHECK_ARG(in_f > 0 && in_f % 32 == 0, "%s: in_f=%d must be a positive multiple of 32", what,
                 in_f);
    CW_CHECK_ARG(in_f <= 32768, "%s: in_f=%d exceeds 32768", what, in_f);
    CW_CHECK_ARG(out_f > 0, "%s: out_f=%d must be positive", what, out_f);
    return CW_OK;
}

// x and quants are read with 128-bit loads, scales with 16-bit loads.
static int check_q4_align(const char *what, const float *x, const uint16_t *s, const uint8_t *q) {
    CW_CHECK_ARG(((uintptr_t)x & 15) == 0, "%s: x must be 16-byte aligned", what);
    CW_CHECK_ARG(((uintptr_t)q & 15) == 0, "%s: quants must be 16-byte aligned", what);
    CW_CHECK_ARG(((uintptr_t)s & 1) == 0, "%s: scales must be 2-byte aligned", what);
    return CW_OK;
}

extern "C" {

int cw_q4_gemv(cw_ctx *ctx, const float *x, const uint16_t *scales, const uint8_t *quants,
               int in_f, int out_f, float *y) {
    CW_CHECK_ARG(ctx && x && scales && quants && y, "cw_q4_gemv: null argument");
    CW_TRY(check_q4_shape("cw_q4_gemv", in_f, out_f));
    CW_TRY(check_q4_align("cw_q4_gemv", x, scales, quants));
    GemvArgs a{};
    a.x = x;
    a.sA = scales;
    a.qA = quants;
    a.y = y;
    a.K = in_f;
    a.N = out_f;
    return launch_q4_gemv(ctx, XS_PLAIN, EPI_STORE, a);
}

int cw_q4_gemv_add(cw_ctx *ctx, const float *x, const uint16_t *scales, const uint8_t *quants,
                   int in_f, int out_f, const float *residual, float *y) {
    CW_CHECK_ARG(ctx && x && scales && quants && residual && y, "cw_q4_gemv_add: null argument");
    CW_TRY(check_q4_shape("cw_q4_gemv_add", in_f, out_f));
    CW_TRY(check_q4_align("cw_q4_gemv_add", x, scales, quants));
    GemvArgs a{};
    a.x = x;
    a.sA = scales;
    a.qA = quants;
    a.resid = residual;
    a.y = y;
    a.K = in_f;
    a.N = out_f;
    return launch_q4_gemv(ctx, XS_PLAIN, EPI_ADD, a);
}

int cw_q4_gemv_swiglu(cw_ctx *ctx, const float *x, const uint16_t *gate_scales,
                      const uint8_t *gate_quants, const uint16_t *up_scales,
                      const uint8_t *up_quants, int in_f, int out_f, float *y) {
    CW_CHECK_ARG(ctx && x && gate_scales && gate_quants && up_scales && up_quants && y,
                 "cw_q4_gemv_swiglu: null argument");
    CW_TRY(check_q4_shape("cw_q4_gemv_swiglu", in_f, out_f));
    CW_TRY(check_q4_align("cw_q4_gemv_swiglu", x, gate_scales, gate_quants));
    CW_TRY(check_q4_align("cw_q4_gemv_swiglu", x, up_scales, up_quants));
    GemvArgs a{};
    a.x = x;
    a.sA = gate_scales;
    a.qA = gate_quants;
    a.sB = up_scales;
    a.qB = up_quants;
    a.y = y;
    a.K = in_f;
    a.N = out_f;
    return launch_q4_gemv(ctx, XS_PLAIN, EPI_SWIGLU, a);
}

}  // extern "C"
