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
//  * GEMM: every Q4_0 weight (q - 8) d enters the f16 MFMAs exactly, as two
//    f16 parts; each f32 activation row is split into f16 hi + lo (22
//    significant bits) after an exact power-of-two row scaling (details at
//    the kernel).  The MFMAs accumulate in f32.
//  * Attention: K and V are f16 in the cache and enter f16 MFMAs exactly; q
//    and the softmax weights p are split into f16 hi + lo the same way.
//
// MFMA v_mfma_f32_16x16x32_f16: lane l holds A[l % 16][8 (l / 16) + j]
// and B[8 (l / 16) + j][l % 16] (j = 0..7) and receives D[4 (l / 16) + r][l % 16]
// (r = 0..3); any k order shared by A and B is valid.

#include <cmath>

#include "cw_internal.hpp"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kT = 256;  // threads per workgroup (4 waves)

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}


// ---------------------------------------------------------------------------
// Rows -> f16 hi/lo for the GEMM (optionally RMS-normalised first,
// norm.wgsl:20-42).  Per row a power of two 2^e brings max|x| into
// [2^8, 2^9): x 2^-e = hi + lo with hi = f16(.), lo = f16(remainder), and
// rowscale[row] = 2^e restores the scale in the GEMM epilogue (exactly).
// One workgroup per row.
template <bool NORM>
__global__ __launch_bounds__(kT) void split_rows_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ w, float eps,
                                                        int K, uint16_t *__restrict__ hi,
                                                        uint16_t *__restrict__ lo,
                                                        float *__restrict__ rowscale) {
    constexpr int R = 4;  // float4 per thread held in registers (K <= 4096)
    __shared__ float red[2][kT / 64];
    const size_t base = (size_t)blockIdx.x * K;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K4 = K >> 2;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + base);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    // one pass for the sum of squares and max|x w| (1/rms > 0 is a common
    // factor, so max|(x/rms) w| = max|x w| / rms)
    float4 xr[R], wr[R];
    float ss = 0.0f, mx = 0.0f;
    auto scan = [&](float4 v, float4 g) {
        if constexpr (NORM) {
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            v.x *= g.x;
            v.y *= g.y;
            v.z *= g.z;
            v.w *= g.w;
        }
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    };
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int i = min(tid + j * kT, K4 - 1);
        xr[j] = x4[i];
        if constexpr (NORM) wr[j] = w4[i];
    }
#pragma unroll
    for (int j = 0; j < R; ++j)
        if (tid + j * kT < K4) scan(xr[j], NORM ? wr[j] : xr[j]);
    for (int i = tid + R * kT; i < K4; i += kT) scan(x4[i], NORM ? w4[i] : x4[i]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        ss += __shfl_xor(ss, off);
        mx = fmaxf(mx, __shfl_xor(mx, off));
    }
    if (lane == 0) {
        red[0][wave] = ss;
        red[1][wave] = mx;
    }
    __syncthreads();
    ss = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    mx = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    const float inv = NORM ? 1.0f / sqrtf(ss / (float)K + eps) : 1.0f;
    mx *= inv;
    const int e = mx > 0.0f ? max(ilogbf(mx) - 8, -100) : 0;
    const float sc = ldexpf(1.0f, -e);
    if (tid == 0) rowscale[blockIdx.x] = ldexpf(1.0f, e);
    auto emit = [&](int i, float4 v, float4 g) {
        if constexpr (NORM) {
            v.x = (v.x * inv) * g.x;
            v.y = (v.y * inv) * g.y;
            v.z = (v.z * inv) * g.z;
            v.w = (v.w * inv) * g.w;
        }
        const float t[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};  // exact: a power of two
        uint16_t hb[4], lb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const _Float16 h = (_Float16)t[k];
            hb[k] = __builtin_bit_cast(uint16_t, h);
            lb[k] = __builtin_bit_cast(uint16_t, (_Float16)(t[k] - (float)h));
        }
        *reinterpret_cast<uint2 *>(hi + base + 4 * (size_t)i) =
            make_uint2(hb[0] | (uint32_t)hb[1] << 16, hb[2] | (uint32_t)hb[3] << 16);
        *reinterpret_cast<uint2 *>(lo + base + 4 * (size_t)i) =
            make_uint2(lb[0] | (uint32_t)lb[1] << 16, lb[2] | (uint32_t)lb[3] << 16);
    };
#pragma unroll
    for (int j = 0; j < R; ++j)
        if (tid + j * kT < K4) emit(tid + j * kT, xr[j], NORM ? wr[j] : xr[j]);
    for (int i = tid + R * kT; i < K4; i += kT) emit(i, x4[i], NORM ? w4[i] : x4[i]);
}

// ---------------------------------------------------------------------------
// Q4_0 dequant-GEMM: y[M][N] = x[M][K] . W[N][K]^T (W split GGUF Q4_0).
//
// Operands, all exact or split exactly into two f16 parts:
//  * x: per row m a power of two 2^e_m brings max|x| into [2^8, 2^9) (the
//    split kernel), then x 2^-e_m = x_hi + x_lo with x_hi = f16(.) and x_lo
//    = f16(remainder): 22 significant bits, no overflow;
//  * W: the block scale d (f16, 11 bits) = d_hi + d_lo with d_hi rounded to
//    8 bits and d_lo the 3-bit remainder, and each weight (q - 8) d =
//    (q - 8) d_hi + (q - 8) d_lo, both parts exact in f16 (at most 11 and 6
//    significant bits) for |d| < 8192.
// y = 2^e_m (x_hi W_hi + x_hi W_lo + x_lo W_hi): three f16 MFMAs per
// 32-wide block accumulate straight into the f32 accumulators, so there is
// no per-block scaling on the vector ALUs; the dropped x_lo W_lo term is
// below 2^-19 of each product.
//
// Tiling: workgroup tile 128 (rows of x) x 128 (rows of W), four waves in
// 2 x 2 of 64 x 64 (4 x 4 MFMA tiles of 16 x 16).  K runs one Q4 block per
// stage, double-buffered in LDS (the x tile hi/lo and the W tile hi/lo, 64 B
// rows with XOR-swizzled 16-byte chunks against bank conflicts); the global
// loads run two stages ahead in registers while the waves run 48 MFMAs per
// stage from LDS.  64 KB of LDS and at most 256 registers per lane let two
// workgroups share a CU, so one workgroup's barrier and load waits overlap
// the other's MFMAs.
//
// SwiGLU: the W tile is 64 gate rows + the same 64 up rows; each wave holds
// 32 gate and the matching 32 up columns, so silu(g) * u is formed in
// registers.
//
// Work split: tiles are numbered so that the workgroups one XCD receives
// (consecutive ids go round-robin over the 8 XCDs) share their x rows, which
// then stay in that XCD's L2 across its N tiles.  When M x N has too few
// tiles to fill every CU twice, K is split over S workgroups that write f32
// partials; a second kernel adds them in a fixed order (deterministic) with
// the epilogue.
constexpr int kGM = 128, kGN = 128;           // workgroup tile
constexpr int kGRow = 64;                     // LDS row bytes: 32 f16
constexpr int kPre = 2;                       // stages of global loads in flight

// Byte offset of 16-byte chunk c (0..3) in LDS row `row`: the chunk index is
// XOR-swizzled by (row / 2) % 4, so the 4 lanes per row of a staging store
// and the 16 rows of a fragment read both spread over distinct bank groups.
__device__ __forceinline__ int swz(int row, int c) { return (c ^ ((row >> 1) & 3)) << 4; }
constexpr int kGA = kGM * kGRow;              // one of x hi / x lo
constexpr int kGB = kGN * kGRow;              // one of W hi / W lo
constexpr int kGBuf = 2 * kGA + 2 * kGB;      // 40 KB per stage
constexpr int kMaxSplit = 8;

__device__ __forceinline__ float f16_bits_val(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Nibbles of a quant dword w at bits 4h + {0, 8, 16, 24} (h = 0: the low
// nibbles, elements 4i..4i+3 of the dword's bytes; h = 1: the high ones)
// -> the f16 pairs (q - 8) of elements (0, 1) and (2, 3), exactly: 0x6400 | q
// is the f16 1024 + q.
__device__ __forceinline__ void nib_pairs(uint32_t w, int h, f16x2 &p01, f16x2 &p23) {
    const uint32_t s = w >> (4 * h);
    const uint32_t a = (s & 0x000F000Fu) | 0x64006400u;         // bytes 0, 2
    const uint32_t b = ((s >> 8) & 0x000F000Fu) | 0x64006400u;  // bytes 1, 3
    const f16x2 off = {(_Float16)1032.0f, (_Float16)1032.0f};
    p01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(b, a, 0x05040100u)) - off;
    p23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(b, a, 0x07060302u)) - off;
}

// One stage in registers: 4 x 16 B of x per thread (128 rows x 64 B, hi
// then lo) and the 16 quant bytes and the f16 scale of one W row's block
// (thread pairs share a row: the even thread dequantizes its low nibbles,
// the odd one its high nibbles).  Native vector registers: an array of
// HIP's uint4 class is copied with memcpy and stays in scratch memory.
template <bool SWI>
__device__ __forceinline__ void w_row(const cwi::GemmArgs &a, int n0, int vc, int *n,
                                      const uint8_t **q, const uint16_t **s) {
    if constexpr (SWI) {
        const bool up = vc >= kGN / 2;
        *n = n0 + (vc & (kGN / 2 - 1));
        *q = up ? a.qB : a.qA;
        *s = up ? a.sB : a.sA;
    } else {
        *n = n0 + vc;
        *q = a.qA;
        *s = a.sA;
    }
}

// Block kb of the tile; at or past kb_end the scale is 0 (loads clamped in
// range, so every operand stays finite and the block adds exact zeros).
template <bool SWI>
__device__ __forceinline__ void gstage_load(const cwi::GemmArgs &a, int nb, int kb, int kb_end,
                                            int m0, int n0, int tid, u32x4 (&sx)[4], u32x4 &sq,
                                            uint32_t &sd) {
    const int blk = min(kb, nb - 1);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int f = tid + u * kT;              // 0..1023
        const int half = f >> 9;                 // 0: hi, 1: lo
        const int row = (f >> 2) & (kGM - 1), c = f & 3;
        const int m = min(m0 + row, a.M - 1);
        const uint16_t *src = half ? a.xlo : a.xhi;
        sx[u] = *reinterpret_cast<const u32x4 *>(src + (size_t)m * a.K + (size_t)blk * 32 + c * 8);
    }
    int n;
    const uint8_t *q;
    const uint16_t *s;
    w_row<SWI>(a, n0, tid >> 1, &n, &q, &s);
    const size_t o = (size_t)min(n, a.N - 1) * nb + blk;
    sq = *reinterpret_cast<const u32x4 *>(q + o * 16);
    const uint32_t dd = s[o];  // loaded unconditionally, then selected
    sd = kb < kb_end ? dd : 0u;
}

__device__ __forceinline__ void gstage_store(const u32x4 (&sx)[4], u32x4 sq, uint32_t sd,
                                             unsigned char *buf, int tid) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int f = tid + u * kT;
        const int half = f >> 9;
        const int row = (f >> 2) & (kGM - 1), c = f & 3;
        *reinterpret_cast<u32x4 *>(buf + half * kGA + row * kGRow + swz(row, c)) = sx[u];
    }
    // d = d_hi + d_lo: d_hi the f32 d rounded to 8 significant bits
    const float d = f16_bits_val(sd);
    uint32_t u = __builtin_bit_cast(uint32_t, d);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    const float dh = __builtin_bit_cast(float, u);
    const _Float16 h16 = (_Float16)dh, l16 = (_Float16)(d - dh);  // both exact
    const f16x2 dh2 = {h16, h16}, dl2 = {l16, l16};
    // elements 16 h .. 16 h + 15 of the block: nibble half h of bytes 0..15
    const int vc = tid >> 1, h = tid & 1;
    u32x4 ph[2], pl[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f16x2 p01, p23;
        nib_pairs(sq[i], h, p01, p23);
        const int k = 4 * i;  // elements k..k+3 of this half
        const f16x2 h01 = p01 * dh2, h23 = p23 * dh2, l01 = p01 * dl2, l23 = p23 * dl2;
        ph[k >> 3][(k & 7) >> 1] = __builtin_bit_cast(uint32_t, h01);
        ph[k >> 3][((k & 7) >> 1) + 1] = __builtin_bit_cast(uint32_t, h23);
        pl[k >> 3][(k & 7) >> 1] = __builtin_bit_cast(uint32_t, l01);
        pl[k >> 3][((k & 7) >> 1) + 1] = __builtin_bit_cast(uint32_t, l23);
    }
    unsigned char *wh = buf + 2 * kGA + vc * kGRow;
    unsigned char *wl = wh + kGB;
    const int o0 = swz(vc, 2 * h), o1 = swz(vc, 2 * h + 1);
    *reinterpret_cast<u32x4 *>(wh + o0) = ph[0];
    *reinterpret_cast<u32x4 *>(wh + o1) = ph[1];
    *reinterpret_cast<u32x4 *>(wl + o0) = pl[0];
    *reinterpret_cast<u32x4 *>(wl + o1) = pl[1];
}

// Tile t of MT x NT x S -> (m tile, n tile, split), XCD-grouped when the
// count divides evenly over the 8 XCDs.
__device__ __forceinline__ void tile_of(int w, int total, int NT, int MT, int *mt, int *nt,
                                        int *sp) {
    int t = w;
    if ((total & 7) == 0) t = (w & 7) * (total >> 3) + (w >> 3);
    *nt = t % NT;
    const int r = t / NT;
    *mt = r % MT;
    *sp = r / MT;
}

// OUT: 0 = the epilogue EPI into y, 1 = f32 partial of split sp into part
template <int EPI, int OUT>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(2, 2))) void q4_gemm_kernel(
    cwi::GemmArgs a, int MT, int NT, int S) {
    constexpr bool SWI = EPI == cwi::EPI_SWIGLU;
    extern __shared__ __attribute__((aligned(16))) unsigned char glds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, lg = lane >> 4;
    int mt, nt, sp;
    tile_of(blockIdx.x, MT * NT * S, NT, MT, &mt, &nt, &sp);
    const int m0 = mt * kGM, n0 = nt * (SWI ? kGN / 2 : kGN);
    const int wm = wave >> 1, wn = wave & 1;
    const int nb = a.K >> 5;
    // this split's blocks [kb0, kb1), one per stage
    const int per = (nb + S - 1) / S;
    const int kb0 = sp * per, kb1 = min(nb, kb0 + per);
    const int n_st = kb1 - kb0;

    // column tile j of this wave -> virtual column (LDS W row) of its lane
    int vcol[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        vcol[j] = SWI ? (j < 2 ? wn * 32 + j * 16 : kGN / 2 + wn * 32 + (j - 2) * 16) + li
                      : wn * 64 + j * 16 + li;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // a ring of kPre register stages: the loads of stage s + 1 + kPre go out
    // right after stage s + 1 is written to LDS, kPre stages ahead of use;
    // every load is unconditional (past the end a stage re-loads the last
    // block, unused), which keeps the registers out of scratch and the loads
    // where they are issued
    u32x4 sx[kPre][4], sq[kPre];
    uint32_t sd[kPre];
    if (n_st > 0) {
        gstage_load<SWI>(a, nb, kb0, kb1, m0, n0, tid, sx[0], sq[0], sd[0]);
        gstage_store(sx[0], sq[0], sd[0], glds, tid);
    }
#pragma unroll
    for (int u = 0; u < kPre; ++u)
        gstage_load<SWI>(a, nb, kb0 + min(1 + u, max(n_st - 1, 0)), kb1, m0, n0, tid, sx[u], sq[u],
                         sd[u]);
    __syncthreads();
    for (int s0 = 0; s0 < n_st; s0 += kPre) {
#pragma unroll
        for (int u = 0; u < kPre; ++u) {
            const int s = s0 + u;
            if (s < n_st) {
                const unsigned char *cur = glds + (s & 1) * kGBuf;
                f16x8 A[4][2], B[4][2];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = wm * 64 + 16 * i + li;
                    A[i][0] = *reinterpret_cast<const f16x8 *>(cur + row * kGRow + swz(row, lg));
                    A[i][1] = *reinterpret_cast<const f16x8 *>(cur + kGA + row * kGRow + swz(row, lg));
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int o = vcol[j] * kGRow + swz(vcol[j], lg);
                    B[j][0] = *reinterpret_cast<const f16x8 *>(cur + 2 * kGA + o);
                    B[j][1] = *reinterpret_cast<const f16x8 *>(cur + 2 * kGA + kGB + o);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i][0], B[j][0], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i][0], B[j][1], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i][1], B[j][0], acc[i][j], 0, 0, 0);
                    }
                // (after the last stage this fills the idle buffer, not read)
                gstage_store(sx[u], sq[u], sd[u], glds + ((s + 1) & 1) * kGBuf, tid);
                gstage_load<SWI>(a, nb, kb0 + min(s + 1 + kPre, n_st - 1), kb1, m0, n0, tid, sx[u],
                                 sq[u], sd[u]);
                __builtin_amdgcn_sched_barrier(0);
                __syncthreads();
            }
        }
    }

    // lane holds rows 4 lg + r of each row tile, column li of each column tile
    constexpr int JN = SWI ? 2 : 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * 64 + i * 16 + 4 * lg + r;
            const float rs = a.rowscale[min(m, a.M - 1)];
#pragma unroll
            for (int j = 0; j < JN; ++j) {
                const int n = n0 + (SWI ? wn * 32 + j * 16 : wn * 64 + j * 16) + li;
                if (m < a.M && n < a.N) {
                    const size_t o = (size_t)m * a.N + n;
                    const float v = acc[i][j][r] * rs;
                    if constexpr (OUT == 1) {
                        a.part[(size_t)sp * a.M * a.N + o] = v;
                    } else if constexpr (EPI == cwi::EPI_STORE) {
                        a.y[o] = v;
                    } else if constexpr (EPI == cwi::EPI_ADD) {
                        a.y[o] = a.resid[o] + v;
                    } else {
                        const float up = acc[i][j + 2][r] * rs;
                        a.y[o] = v / (1.0f + expf(-v)) * up;
                    }
                }
            }
        }
}

// y = [resid +] sum over s of part[s], s in order (one float4 per thread).
template <int EPI>
__global__ __launch_bounds__(kT) void gemm_reduce_kernel(const float *__restrict__ part, int S,
                                                         size_t n, const float *resid,
                                                         float *y) {
    const size_t i = ((size_t)blockIdx.x * kT + threadIdx.x) * 4;
    if (i >= n) return;
    const bool vec = ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(resid)) & 15) == 0;
    if (vec && i + 4 <= n) {
        float4 v = *reinterpret_cast<const float4 *>(part + i);
        for (int s = 1; s < S; ++s) {
            const float4 p = *reinterpret_cast<const float4 *>(part + (size_t)s * n + i);
            v.x += p.x;
            v.y += p.y;
            v.z += p.z;
            v.w += p.w;
        }
        if constexpr (EPI == cwi::EPI_ADD) {
            const float4 r = *reinterpret_cast<const float4 *>(resid + i);
            v.x = r.x + v.x;
            v.y = r.y + v.y;
            v.z = r.z + v.z;
            v.w = r.w + v.w;
        }
        *reinterpret_cast<float4 *>(y + i) = v;
        return;
    }
    for (size_t e = i; e < n && e < i + 4; ++e) {
        float v = part[e];
        for (int s = 1; s < S; ++s) v += part[(size_t)s * n + e];
        if constexpr (EPI == cwi::EPI_ADD) v = resid[e] + v;
        y[e] = v;
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
    // K and V rows of key tile t, 64 keys x 128 dims, 16 B per load (4 each
    // per thread); the next tile's loads are in flight during this tile's
    // MFMAs (past the last tile a clamped re-load, unused)
    u32x4 kn[4], vn[4];
    auto tile_load = [&](int t) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int f = tid + u * kT;  // 0..1023
            const int key = f >> 4, c8 = (f & 15) * 8;
            const int p = min(t * kAttK + key, last_pos);
            kn[u] = *reinterpret_cast<const u32x4 *>(kc + (size_t)p * kv_dim + g * HD + c8);
            vn[u] = *reinterpret_cast<const u32x4 *>(vc + (size_t)p * kv_dim + g * HD + c8);
        }
    };
    tile_load(0);
    for (int t = 0; t < n_tiles; ++t) {
        const int k0 = t * kAttK;
        __syncthreads();  // previous tile's LDS reads are done
        // stage K rows and V^T
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int f = tid + u * kT;
            const int key = f >> 4, c8 = (f & 15) * 8;
            *reinterpret_cast<u32x4 *>(&Ks[key * kKRow + c8]) = kn[u];
            const f16x8 ve = __builtin_bit_cast(f16x8, vn[u]);
#pragma unroll
            for (int j = 0; j < 8; ++j) Vt[(c8 + j) * kVRow + key] = ve[j];
        }
        tile_load(min(t + 1, n_tiles - 1));
        __builtin_amdgcn_sched_barrier(0);
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
                      uint16_t *hi, uint16_t *lo, float *rowscale) {
    if (norm_w)
        return launch(ctx, "prefill_split_rmsnorm", split_rows_kernel<true>, dim3(rows), dim3(kT),
                      0, x, norm_w, eps, K, hi, lo, rowscale);
    return launch(ctx, "prefill_split", split_rows_kernel<false>, dim3(rows), dim3(kT), 0, x,
                  norm_w, eps, K, hi, lo, rowscale);
}

int gemm_splits(const cw_ctx *ctx, Epi epi, int M, int N, int K) {
    if (epi == EPI_SWIGLU) return 1;
    const int tiles = ((M + kGM - 1) / kGM) * ((N + kGN - 1) / kGN);
    int s = 1;
    // split K while the workgroups fill less than two per CU and each split
    // keeps at least 16 blocks
    while (s < kMaxSplit && s * tiles < 2 * ctx->n_cu && (K / 32) / (2 * s) >= 16) s *= 2;
    return s;
}

template <int EPI, int OUT>
int launch_gemm_tiles(cw_ctx *ctx, const char *label, const GemmArgs &a, int MT, int NT, int S) {
    auto fn = q4_gemm_kernel<EPI, OUT>;
    static bool attr = false;  // per instantiation
    if (!attr) {
        CW_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 2 * kGBuf));
        attr = true;
    }
    return launch(ctx, label, fn, dim3(MT * NT * S), dim3(kT), 2 * kGBuf, a, MT, NT, S);
}

int launch_q4_gemm(cw_ctx *ctx, Epi epi, const GemmArgs &a) {
    const int MT = (a.M + kGM - 1) / kGM;
    if (epi == EPI_SWIGLU)
        return launch_gemm_tiles<EPI_SWIGLU, 0>(ctx, "q4_gemm_swiglu", a, MT,
                                                (a.N + kGN / 2 - 1) / (kGN / 2), 1);
    const int NT = (a.N + kGN - 1) / kGN;
    const int S = a.part ? gemm_splits(ctx, epi, a.M, a.N, a.K) : 1;
    if (S > 1 && a.part_floats < (size_t)S * a.M * a.N) {
        set_error("q4 gemm: split-K workspace of %zu floats, %zu needed", a.part_floats,
                  (size_t)S * a.M * a.N);
        return CW_ERR_ARG;
    }
    if (S == 1)
        return epi == EPI_ADD ? launch_gemm_tiles<EPI_ADD, 0>(ctx, "q4_gemm_add", a, MT, NT, 1)
                              : launch_gemm_tiles<EPI_STORE, 0>(ctx, "q4_gemm", a, MT, NT, 1);
    const int rc = epi == EPI_ADD
                       ? launch_gemm_tiles<EPI_ADD, 1>(ctx, "q4_gemm_add_splitk", a, MT, NT, S)
                       : launch_gemm_tiles<EPI_STORE, 1>(ctx, "q4_gemm_splitk", a, MT, NT, S);
    if (rc != CW_OK) return rc;
    const size_t n = (size_t)a.M * a.N;
    const unsigned blocks = (unsigned)((n + 4 * kT - 1) / (4 * kT));
    if (epi == EPI_ADD)
        return launch(ctx, "q4_gemm_reduce", gemm_reduce_kernel<EPI_ADD>, dim3(blocks), dim3(kT),
                      0, (const float *)a.part, S, n, a.resid, a.y);
    return launch(ctx, "q4_gemm_reduce", gemm_reduce_kernel<EPI_STORE>, dim3(blocks), dim3(kT), 0,
                  (const float *)a.part, S, n, (const float *)nullptr, a.y);
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
    const size_t n = (size_t)m * in_f;
    const int S = gemm_splits(ctx, EPI_STORE, m, out_f, in_f);
    const size_t part = S > 1 ? (size_t)S * m * out_f : 0;
    void *scratch = nullptr;
    // hi, lo (2 B each per element), row scales, partials (16-byte aligned)
    const size_t rs_off = (n * 4 + 15) & ~size_t(15);
    const size_t part_off = (rs_off + (size_t)m * 4 + 15) & ~size_t(15);
    CW_TRY(ctx_scratch(ctx, part_off + part * 4, &scratch));
    uint16_t *hi = (uint16_t *)scratch, *lo = hi + n;
    float *rs = reinterpret_cast<float *>((char *)scratch + rs_off);
    CW_TRY(launch_split_rows(ctx, x, nullptr, 0.0f, m, in_f, hi, lo, rs));
    GemmArgs a{};
    a.xhi = hi;
    a.xlo = lo;
    a.rowscale = rs;
    a.sA = scales;
    a.qA = quants;
    a.y = y;
    a.M = m;
    a.N = out_f;
    a.K = in_f;
    if (part) {
        a.part = reinterpret_cast<float *>((char *)scratch + part_off);
        a.part_floats = part;
    }
    return launch_q4_gemm(ctx, EPI_STORE, a);
}
