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
//  * GEMM: every Q4_0 quant (q - 8) enters the f16 MFMAs exactly and the
//    block scale multiplies each block's f32 sum; each f32 activation row is
//    split into f16 hi + lo (22 significant bits) after an exact power-of-two
//    row scaling (details at the kernel).  The MFMAs accumulate in f32.
//  * Attention: K and V are f16 in the cache and enter f16 MFMAs exactly; q
//    and the softmax weights p are split into f16 hi + lo the same way.
//
// MFMA v_mfma_f32_16x16x32_f16 (attention): lane l holds A[l % 16][8 (l / 16)
// + j] and B[8 (l / 16) + j][l % 16] (j = 0..7) and receives
// D[4 (l / 16) + r][l % 16] (r = 0..3); any k order shared by A and B is
// valid.

#include <cmath>

#include "cw_internal.hpp"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

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
// The split of one row given the first R float4 per thread in registers
// (xr[j], gains wr[j], element tid + j kT) and, for rows longer than R kT
// float4, the rest read from x4 (row) and w4.
template <bool NORM>
__device__ __forceinline__ void split_row(const float4 (&xr)[4], const float4 (&wr)[4],
                                          const float4 *x4, const float4 *w4, int K, float eps,
                                          size_t base, uint16_t *__restrict__ hi,
                                          uint16_t *__restrict__ lo, float *__restrict__ rowscale) {
    constexpr int R = 4;
    __shared__ float red[2][kT / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K4 = K >> 2;
    // one pass for the sum of squares and max|x w| (1/rms > 0 is a common
    // factor, so max|(x/rms) w| = max|x w| / rms)
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

template <bool NORM>
__global__ __launch_bounds__(kT) void split_rows_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ w, float eps,
                                                        int K, uint16_t *__restrict__ hi,
                                                        uint16_t *__restrict__ lo,
                                                        float *__restrict__ rowscale) {
    constexpr int R = 4;  // float4 per thread held in registers (K <= 4096)
    const size_t base = (size_t)blockIdx.x * K;
    const int tid = threadIdx.x;
    const int K4 = K >> 2;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + base);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 xr[R], wr[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int i = min(tid + j * kT, K4 - 1);
        xr[j] = x4[i];
        if constexpr (NORM) wr[j] = w4[i];
    }
    split_row<NORM>(xr, wr, x4, w4, K, eps, base, hi, lo, rowscale);
}

// The split-K reduction of one row (y = [resid +] the partials summed in
// order, as gemm_reduce_kernel) and, in the same pass, the row's split for
// the next GEMM (split_rows_kernel's arithmetic on y).  One workgroup per
// row of N <= 4 kT float4.
template <bool NORM, int EPI>
__global__ __launch_bounds__(kT) void reduce_split_kernel(const float *__restrict__ part, int S,
                                                          int N, size_t MN,
                                                          const float *__restrict__ resid,
                                                          float *__restrict__ y,
                                                          const float *__restrict__ w, float eps,
                                                          uint16_t *__restrict__ hi,
                                                          uint16_t *__restrict__ lo,
                                                          float *__restrict__ rowscale) {
    constexpr int R = 4;
    const size_t base = (size_t)blockIdx.x * N;
    const int tid = threadIdx.x;
    const int K4 = N >> 2;
    const float4 *p4 = reinterpret_cast<const float4 *>(part + base);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 xr[R], wr[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int i = min(tid + j * kT, K4 - 1);
        float4 v = p4[i];
        for (int s = 1; s < S; ++s) {
            const float4 p = reinterpret_cast<const float4 *>(part + (size_t)s * MN + base)[i];
            v.x += p.x;
            v.y += p.y;
            v.z += p.z;
            v.w += p.w;
        }
        if constexpr (EPI == cwi::EPI_ADD) {
            const float4 r = reinterpret_cast<const float4 *>(resid + base)[i];
            v.x = r.x + v.x;
            v.y = r.y + v.y;
            v.z = r.z + v.z;
            v.w = r.w + v.w;
        }
        xr[j] = v;
        if (tid + j * kT < K4) reinterpret_cast<float4 *>(y + base)[tid + j * kT] = v;
        if constexpr (NORM) wr[j] = w4[i];
    }
    split_row<NORM>(xr, wr, reinterpret_cast<const float4 *>(y + base), w4, N, eps, base, hi, lo,
                    rowscale);
}

// ---------------------------------------------------------------------------
// Q4_0 dequant-GEMM: y[M][N] = x[M][K] . W[N][K]^T (W split GGUF Q4_0).
//
// Operands, all exact or split exactly into two f16 parts:
//  * x: per row m a power of two 2^e_m brings max|x| into [2^8, 2^9) (the
//    split kernel), then x 2^-e_m = x_hi + x_lo with x_hi = f16(.) and x_lo
//    = f16(remainder): 22 significant bits, no overflow;
//  * W: the quants as q - 8 (small integers, exact in f16); the block scale
//    d is applied to the block's f32 sum, not to the operand.
// Per block b: t = sum over its 32 k of (x_hi + x_lo) (q - 8), two f16 MFMAs
// per 16-wide k slice (every product exact, the sum in f32); then
// acc += d_b t, one f32 FMA per output element and block.  y = 2^e_m acc.
// This is the reference's sum of d (q - 8) x over the blocks with the
// rounding of an f32 computation (q4.wgsl:25-82 forms d (q - 8) per weight;
// here d multiplies each block's partial sum).
//
// Matrix cores: v_mfma_f32_32x32x16_f16 (lane l holds A[l % 32][8 (l / 32)
// + j] and B[8 (l / 32) + j][l % 32], j = 0..7, and receives
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32], r = 0..15).  A Q4 block is two
// k slices: the low nibbles of its bytes 0..15 (elements 0..15) and the high
// nibbles (elements 16..31); the lanes of half g of the wave take bytes
// 8g..8g+7, i.e. elements 8g + j of the low slice and 16 + 8g + j of the
// high one, so one 8-byte read gives a lane both slices of B.
//
// Tiling: workgroup tile 128 (rows of x) x 128 (rows of W), four waves in
// 2 x 2 of 64 x 64 (2 x 2 MFMA tiles of 32 x 32).  A K stage is two Q4
// blocks.  Its x tile (hi and lo, 128 rows x 64 k) and the raw quants of its
// W tile go from global memory straight into LDS (global_load_lds, 16 bytes
// per lane, no registers), double-buffered: stage s + 1 is in flight while
// the waves compute stage s, with one barrier per stage.  The DMA writes LDS
// in lane order, so the x rows' XOR swizzle (16-byte chunk c of row r at
// slot c ^ ((r / 2) % 8): conflict-free fragment reads) is made by choosing
// which global chunk each lane loads.  The block scales come through
// registers and are stored as f32.  Each wave dequantizes its own B
// fragments from the nibbles (perm into the f16 1024 + q, minus 1032: exact).
// Within a block a wave issues all its LDS reads first, then interleaves the
// previous block's scale FMAs with this block's first MFMAs, tile by tile, so
// the vector ALU works while the matrix core runs.
// 74 KB of LDS (two stage buffers) and at most 256 registers per lane let
// two workgroups share a CU.
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
constexpr int kGM = 128;               // workgroup tile rows (of x)
constexpr int kSB = 2;                 // Q4 blocks per K stage
constexpr int kXRow = kSB * 32 * 2;    // LDS bytes of one x row (one half) per stage
constexpr int kXHalf = kGM * kXRow;    // x hi (then x lo): 16 KB
constexpr int kMaxSplit = 8;
static_assert(kXRow == 128, "the x swizzle assumes 8 chunks of 16 bytes per row");

// Tile geometry for WN waves along N (2 x WN waves): BN rows of W (LDS
// columns) per tile, one W unit (column, block) per thread per stage.
template <int WN>
struct GT {
    static constexpr int WAVES = 2 * WN, THREADS = 64 * WAVES;
    static constexpr int BN = 64 * WN;
    static constexpr int WQ = 2 * kXHalf;          // quants [block][col] x 16 B
    static constexpr int WD = WQ + kSB * BN * 16;  // d as f32 [block][col]
    static constexpr int BUF = WD + kSB * BN * 4;  // one stage: 37 KB (WN 2), 39.5 KB (WN 3)
    static_assert(kSB * BN == THREADS, "one W unit per thread per stage");
    static_assert(2 * BUF * 2 <= 160 * 1024, "two workgroups per CU");
};

typedef __attribute__((address_space(3))) unsigned char lds_u8;

// One 16-byte-per-lane global -> LDS DMA: lane i's 16 bytes land at LDS byte
// lds_off + 16 i (lds_off wave-uniform, passed in M0 through the operand
// constraint, so the compiler sets M0 itself).  Written as asm so the
// compiler's wait-count pass does not track it: its own waits (for register
// loads) stay correct, being only stricter with loads it does not count, and
// it adds none before LDS reads; the kernel orders the DMA itself with
// counted vmcnt waits and a barrier.
__device__ __forceinline__ void dma16(const void *src, unsigned char *lds_dst) {
    const uint32_t off =
        __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8 *)lds_dst);
    asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(off) : "memory");
}

__device__ __forceinline__ float f16_bits_val(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// LDS byte offset of 16-byte chunk c (0..7) of x row `row` within one half
__device__ __forceinline__ int xoff(int row, int c) {
    return row * kXRow + ((c ^ ((row >> 1) & 7)) << 4);
}

// W tile column -> weight row and its matrix (SwiGLU: BN / 2 gate rows, then
// the same up rows)
template <bool SWI, int BN>
__device__ __forceinline__ void w_col(const cwi::GemmArgs &a, int n0, int col, int *n,
                                      const uint8_t **q, const uint16_t **s) {
    if constexpr (SWI) {
        const bool up = col >= BN / 2;
        *n = n0 + (up ? col - BN / 2 : col);
        *q = up ? a.qB : a.qA;
        *s = up ? a.sB : a.sA;
    } else {
        *n = n0 + col;
        *q = a.qA;
        *s = a.sA;
    }
}

// The x DMAs of one workgroup stage: 2 halves x 16 groups of 8 rows, one
// 1 KB DMA each, wave w taking groups t = w, w + WAVES, ...  Lane i of a
// group fills slot i % 8 of row 8 grp + i / 8 with the chunk the swizzle puts
// there: chunk c = (i % 8) ^ ((row / 2) % 8), which for a given lane only
// depends on the parity of grp.  xl[p] is the lane's element offset for
// parity p (row and chunk within the stage); the stage adds 32 kbs.
template <int WN>
__device__ __forceinline__ void stage_x(const cwi::GemmArgs &a, const size_t (&xl)[2], int kbs,
                                        int wave, unsigned char *buf) {
    constexpr int WAVES = GT<WN>::WAVES;
#pragma unroll
    for (int u = 0; u < (32 + WAVES - 1) / WAVES; ++u) {
        const int t = wave + u * WAVES;  // wave-uniform
        if (u < 32 / WAVES || t < 32) {  // (only the last round can fall short)
            const int half = t >> 4, grp = t & 15;
            const uint16_t *base = half ? a.xlo : a.xhi;
            dma16(base + xl[grp & 1] + ((size_t)grp * 8 * a.K + (size_t)kbs * 32),
                  buf + half * kXHalf + grp * 1024);
        }
    }
}

// W of one stage, unit t = block * BN + column: its 16 quant bytes and its
// scale, as loaded (two loads; past kb_end the last block's, never used:
// that block's MFMAs are skipped)
struct WUnit {
    uint4 q;
    uint32_t d;
};
template <bool SWI, int BN>
__device__ __forceinline__ WUnit stage_w(const cwi::GemmArgs &a, int nb, int kb, int kb_end,
                                         int n0, int tid) {
    int n;
    const uint8_t *q;
    const uint16_t *s;
    w_col<SWI, BN>(a, n0, tid % BN, &n, &q, &s);
    const size_t o = (size_t)min(n, a.N - 1) * nb + min(kb + tid / BN, kb_end - 1);
    return WUnit{*reinterpret_cast<const uint4 *>(q + o * 16), s[o]};
}

// Workgroup barrier on LDS data only: __syncthreads would also wait for
// every global load in flight (the W loads two stages ahead)
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Nibbles (4 bits at byte offsets 0..3 of t) -> f16 pairs (q - 8) of bytes
// (0, 1) and (2, 3): 0x64 over a nibble is the f16 1024 + q
__device__ __forceinline__ void nib4(uint32_t t, f16x2 &p01, f16x2 &p23) {
    const f16x2 off = {(_Float16)1032.0f, (_Float16)1032.0f};
    p01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, t, 0x04010400u)) - off;
    p23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, t, 0x04030402u)) - off;
}

// 8 quant bytes -> the B fragment (q - 8, exact in f16) of the low slice
// (ks 0: low nibbles) or the high slice (ks 1: high nibbles)
__device__ __forceinline__ f16x8 dequant_slice(uint2 q, int ks) {
    const uint32_t t0 = (q.x >> (4 * ks)) & 0x0F0F0F0Fu, t1 = (q.y >> (4 * ks)) & 0x0F0F0F0Fu;
    f16x2 p[4];
    nib4(t0, p[0], p[1]);
    nib4(t1, p[2], p[3]);
    return __builtin_bit_cast(f16x8, (u32x4){__builtin_bit_cast(uint32_t, p[0]),
                                             __builtin_bit_cast(uint32_t, p[1]),
                                             __builtin_bit_cast(uint32_t, p[2]),
                                             __builtin_bit_cast(uint32_t, p[3])});
}

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
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

// OUT: 0 = the epilogue EPI into y, 1 = f32 partial of split sp into part.
// x hi / lo hold ceil(M / 128) * 128 rows plus 32 elements (the DMA reads
// whole row tiles and, for an odd final block, one block past the split).
template <int EPI, int OUT, int WN>
__global__ __launch_bounds__(GT<WN>::THREADS) __attribute__((amdgpu_waves_per_eu(WN, WN)))
void q4_gemm_kernel(cwi::GemmArgs a, int MT, int NT, int S) {
    constexpr bool SWI = EPI == cwi::EPI_SWIGLU;
    using G = GT<WN>;
    constexpr int BN = G::BN;
    // the two stage buffers are separate LDS objects, and the stage loop
    // below is unrolled by two so each access names one of them
    __shared__ __attribute__((aligned(16))) unsigned char lds_a[G::BUF];
    __shared__ __attribute__((aligned(16))) unsigned char lds_b[G::BUF];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, lg = lane >> 5;
    int mt, nt, sp;
    tile_of(blockIdx.x, MT * NT * S, NT, MT, &mt, &nt, &sp);
    const int m0 = mt * kGM, n0 = nt * (SWI ? BN / 2 : BN);
    const int wm = wave / WN, wn = wave % WN;
    const int nb = a.K >> 5;
    // this split's blocks [kb0, kb1), two per stage
    const int per = (((nb + S - 1) / S) + kSB - 1) / kSB * kSB;
    const int kb0 = min(nb, sp * per), kb1 = min(nb, kb0 + per);
    const int n_st = (kb1 - kb0 + kSB - 1) / kSB;

    // LDS column of this lane in column tile j
    int col[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
        col[j] = (SWI ? j * (BN / 2) + wn * 32 : wn * 64 + j * 32) + li;
    // this lane's x DMA element offsets (row and chunk) for even / odd groups
    size_t xl[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int row = p * 8 + (lane >> 3);
        const int c = (lane & 7) ^ ((row >> 1) & 7);
        xl[p] = (size_t)(m0 + (lane >> 3)) * a.K + (c >> 2) * 32 + (c & 3) * 8;
    }

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Pipeline: the x tile of stage st + 1 (L2-resident) is one stage ahead
    // by DMA; W (streamed from HBM) two stages ahead in a register ring
    // w[2], stored to LDS one stage ahead.  Loads complete in issue order,
    // and every stage issues its x DMAs, then its two W loads, so "all but
    // the last two loads done" means the x tile has landed.  Every stage
    // issues the same loads (past the split's end they re-read its last
    // block, in range and unused) and the stage count is padded to even, so
    // the loop is straight-line code whose wait counts are exact.
    // t: the current block's sums; dp: its scales.  A block's scale FMAs are
    // issued in the next block, beside that block's first MFMAs (and after
    // the loop for the last one); t = 0, dp = 0 make the first ones no-ops.
    f32x16 t[2][2];
    float dp[2] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) t[i][j][r] = 0.0f;
    if (n_st > 0) {
        WUnit w[2];
        auto store_w = [&](unsigned char *buf, const WUnit &u) {
            *reinterpret_cast<uint4 *>(buf + G::WQ + tid * 16) = u.q;
            *reinterpret_cast<float *>(buf + G::WD + tid * 4) = f16_bits_val(u.d);
        };
        // the loads in flight at the loop head come in the loop's own order:
        // W of stage 1, x of stage 0, W of stage 2
        w[0] = stage_w<SWI, BN>(a, nb, kb0, kb1, n0, tid);
        w[1] = stage_w<SWI, BN>(a, nb, kb0 + kSB, kb1, n0, tid);
        __builtin_amdgcn_sched_barrier(0);
        stage_x<WN>(a, xl, kb0, wave, lds_a);
        __builtin_amdgcn_sched_barrier(0);
        store_w(lds_a, w[0]);
        __builtin_amdgcn_sched_barrier(0);
        w[0] = stage_w<SWI, BN>(a, nb, kb0 + 2 * kSB, kb1, n0, tid);
        // stage st from cur while stage st + 1 goes into nxt; wn holds W of
        // stage st + 1 and is reloaded with stage st + 3
        auto step = [&](unsigned char *cur, unsigned char *nxt, WUnit &wnx, int st) {
            const int kb = kb0 + st * kSB;
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(0x0F72);  // vmcnt(2): x of st landed, W of st + 2 may fly
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();  // stage st published; stage st - 1 retired from nxt
            store_w(nxt, wnx);
            stage_x<WN>(a, xl, min(kb + kSB, kb1 - 1), wave, nxt);
            __builtin_amdgcn_sched_barrier(0);
            wnx = stage_w<SWI, BN>(a, nb, kb + 3 * kSB, kb1, n0, tid);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int bi = 0; bi < kSB; ++bi) {
                if (kb + bi < kb1) {  // wave-uniform
                    // every LDS read of the block first: the quants and scales
                    // of both column tiles, x hi / lo of both k slices
                    uint2 q[2];
                    float d[2];
                    f16x8 ah[2][2], al[2][2];  // [k slice][row tile]
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        q[j] = *reinterpret_cast<const uint2 *>(cur + G::WQ + (bi * BN + col[j]) * 16 + 8 * lg);
                        d[j] = *reinterpret_cast<const float *>(cur + G::WD + (bi * BN + col[j]) * 4);
                    }
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                        for (int i = 0; i < 2; ++i) {
                            const int o = xoff(wm * 64 + i * 32 + li, bi * 4 + 2 * ks + lg);
                            ah[ks][i] = *reinterpret_cast<const f16x8 *>(cur + o);
                            al[ks][i] = *reinterpret_cast<const f16x8 *>(cur + kXHalf + o);
                        }
                    __builtin_amdgcn_sched_barrier(0);
                    // The previous block's scale FMAs go one tile at a time,
                    // each right before that tile's first MFMA of this block
                    // (which overwrites the tile's sums), so they issue while
                    // the matrix core runs the MFMA before.  The barriers pin
                    // that order.
                    auto scale_tile = [&](int i, int j) {
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[i][j][r] = __builtin_fmaf(dp[j], t[i][j][r], acc[i][j][r]);
                    };
                    f16x8 bq[2][2];  // [column tile][k slice]
                    scale_tile(0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    bq[0][0] = dequant_slice(q[0], 0);
                    bq[1][0] = dequant_slice(q[1], 0);
                    __builtin_amdgcn_sched_barrier(0);
                    t[0][0] = mfma32(ah[0][0], bq[0][0], (f32x16){});
                    __builtin_amdgcn_sched_barrier(0);
                    scale_tile(0, 1);
                    __builtin_amdgcn_sched_barrier(0);
                    t[0][1] = mfma32(ah[0][0], bq[1][0], (f32x16){});
                    __builtin_amdgcn_sched_barrier(0);
                    scale_tile(1, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    t[1][0] = mfma32(ah[0][1], bq[0][0], (f32x16){});
                    __builtin_amdgcn_sched_barrier(0);
                    scale_tile(1, 1);
                    __builtin_amdgcn_sched_barrier(0);
                    t[1][1] = mfma32(ah[0][1], bq[1][0], (f32x16){});
                    __builtin_amdgcn_sched_barrier(0);
                    // the high-nibble slice beside slice 0's x_lo MFMAs
                    bq[0][1] = dequant_slice(q[0], 1);
                    bq[1][1] = dequant_slice(q[1], 1);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j) t[i][j] = mfma32(al[0][i], bq[j][0], t[i][j]);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j) t[i][j] = mfma32(ah[1][i], bq[j][1], t[i][j]);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j) t[i][j] = mfma32(al[1][i], bq[j][1], t[i][j]);
                    dp[0] = d[0];
                    dp[1] = d[1];
                }
            }
        };
        for (int st = 0; st < n_st; st += 2) {
            step(lds_a, lds_b, w[1], st);
            step(lds_b, lds_a, w[0], st + 1);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(dp[j], t[i][j][r], acc[i][j][r]);

    // lane holds rows 8 (r / 4) + 4 lg + r % 4 of each row tile, column li
    // of each column tile
    constexpr int JN = SWI ? 1 : 2;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
            const float rs = a.rowscale[min(m, a.M - 1)];
#pragma unroll
            for (int j = 0; j < JN; ++j) {
                const int n = n0 + (SWI ? wn * 32 : wn * 64 + j * 32) + li;
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
                        const float up = acc[i][1][r] * rs;
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
// (cache.rs:21-24).  Workgroup (position, y) takes four heads of the
// position, one per wave.
// With S > 0 the rows are the QKV GEMM's S split-K partials, summed here in
// order (gemm_reduce_kernel's sum) instead of read from qkv.
template <typename KVT>
__global__ __launch_bounds__(kT) void qk_rope_kv_kernel(const float *__restrict__ qkv,
                                                        const float *__restrict__ qn,
                                                        const float *__restrict__ kn, float eps,
                                                        const float *__restrict__ cos_t,
                                                        const float *__restrict__ sin_t,
                                                        int n_heads, int n_kv, int start,
                                                        float *__restrict__ q_out,
                                                        KVT *__restrict__ kc,
                                                        KVT *__restrict__ vc,
                                                        const float *__restrict__ part, int S,
                                                        size_t MN) {
    constexpr int HD = 128, HALF = 64;
    const int i = blockIdx.x, pos = start + i;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q_dim = n_heads * HD, kv_dim = n_kv * HD;
    const size_t row_off = (size_t)i * (q_dim + 2 * kv_dim);
    const float *row = (S > 0 ? part : qkv) + row_off;
    auto val = [&](const float *p) {  // p: an element of row (of partial 0)
        float v = *p;
        for (int s2 = 1; s2 < S; ++s2) v += p[(size_t)s2 * MN];
        return v;
    };
    const float c = cos_t[(size_t)pos * HALF + lane], s = sin_t[(size_t)pos * HALF + lane];
    // one head per wave: workgroup y takes heads 4 y .. 4 y + 3 of the row
    for (int h = blockIdx.y * (kT / 64) + wave; h < n_heads + n_kv; h += gridDim.y * (kT / 64)) {
        const bool isq = h < n_heads;
        const float *src = isq ? row + (size_t)h * HD : row + q_dim + (size_t)(h - n_heads) * HD;
        const float *g = isq ? qn : kn;
        const float lo = val(src + lane), hi = val(src + lane + HALF);
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
            vd[lane] = (KVT)val(vs + lane);
            vd[lane + HALF] = (KVT)val(vs + lane + HALF);
        }
    }
}

// ---------------------------------------------------------------------------
// Causal attention (attention.wgsl:23-96 for each query position) on f16
// caches, flash style: workgroup = one query head x 64 positions, in two
// groups of four waves (one wave per 16 positions) that take alternate
// 64-key tiles, so the longest workgroup runs half as many tile steps.  Per
// tile: K and V rows staged in LDS as they are stored (16-byte writes);
// S = q K^T by MFMA (q split into f16 hi/lo), online max / sum per row,
// P (f16 hi/lo) through LDS into A layout, O += P V by MFMA with the V
// operand read by LDS transpose loads.  At the end the second group's
// (max, sum, o) per row merges into the first's through LDS.
constexpr int kAttQ = 64;   // positions per workgroup
constexpr int kAttK = 64;   // keys per tile
constexpr int kKRow = 128 + 8;  // K and V tile row stride (f16), padded

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// B operand of v_mfma_f32_16x16x32_f16 (lane l: B[8 (l / 16) + j][l % 16],
// j = 0..7) from a row-major LDS tile, B[k][n] = tile[k0 + k][n0 + n].
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// i % 4 of the 8 bytes addressed by lane 4 j + i / 4, for j = 0..3.  So lane
// m of group g addresses row k0 + 8 g + m / 4 (+ 4 for the second read),
// columns n0 + 4 (m % 4) .. + 3, and lane i gets column n0 + i of rows
// k0 + 8 g + j.
__device__ __forceinline__ f16x8 lds_b_tr(const _Float16 *tile, int row_stride, int k0, int n0,
                                          int lane) {
    const int g = lane >> 4, m = lane & 15;
    const _Float16 *p = tile + (size_t)(k0 + 8 * g + (m >> 2)) * row_stride + n0 + 4 * (m & 3);
    const s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)p);
    const s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p + 4 * row_stride));
    const uint2 a = __builtin_bit_cast(uint2, r0), b = __builtin_bit_cast(uint2, r1);
    return __builtin_bit_cast(f16x8, make_uint4(a.x, a.y, b.x, b.y));
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)a);
    const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)b);
    return lo | (hi << 16);
}

constexpr int kAttThreads = 2 * kT;  // two groups of four waves

__global__ __launch_bounds__(kAttThreads) void attn_prefill_kernel(
    const float *__restrict__ q, const _Float16 *__restrict__ kc, const _Float16 *__restrict__ vc,
    int M, int n_heads, int n_kv, int start, float scale, float *__restrict__ out) {
    constexpr int HD = 128;
    constexpr int TILE = kAttK * kKRow;  // f16 elements of one K (or V) tile
    // [group][K | V]; after the loop, group 1's (o, m, l) for the merge
    __shared__ __attribute__((aligned(16))) _Float16 KV[2][2][TILE];
    __shared__ float Ps[8][16 * kAttK];
    const int h = blockIdx.x, q0 = blockIdx.y * kAttQ;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2, gw = wave & 3, gtid = tid & (kT - 1);
    const int li = lane & 15, lg = lane >> 4;
    const int g = h / (n_heads / n_kv);
    const int kv_dim = n_kv * HD;
    const int wq = q0 + gw * 16;  // this wave's first position (row of q)
    _Float16 *Ks = KV[grp][0], *Vs = KV[grp][1];

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
    const int n_steps = (n_tiles + 1) / 2;  // group grp takes tiles grp, grp + 2, ...
    // K and V rows of key tile t, 64 keys x 128 dims, 16 B per load (4 each
    // per thread of the group); the group's next tile's loads are in flight
    // during this tile's MFMAs (past the last tile a clamped re-load, unused)
    u32x4 kn[4], vn[4];
    auto tile_load = [&](int t) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int f = gtid + u * kT;  // 0..1023
            const int key = f >> 4, c8 = (f & 15) * 8;
            const int p = min(t * kAttK + key, last_pos);
            kn[u] = *reinterpret_cast<const u32x4 *>(kc + (size_t)p * kv_dim + g * HD + c8);
            vn[u] = *reinterpret_cast<const u32x4 *>(vc + (size_t)p * kv_dim + g * HD + c8);
        }
    };
    tile_load(min(grp, n_tiles - 1));
    for (int st = 0; st < n_steps; ++st) {
        const int t = 2 * st + grp;
        const bool active = t < n_tiles;  // (uniform over the group)
        const int k0 = t * kAttK;
        __syncthreads();  // previous step's LDS reads are done
        // stage K and V rows
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int f = gtid + u * kT;
            const int key = f >> 4, c8 = (f & 15) * 8;
            *reinterpret_cast<u32x4 *>(&Ks[key * kKRow + c8]) = kn[u];
            *reinterpret_cast<u32x4 *>(&Vs[key * kKRow + c8]) = vn[u];
        }
        tile_load(min(t + 2, n_tiles - 1));
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        if (!active) continue;

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
            // a row with no key yet keeps mnew = -inf: guard the rescale
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
                const f16x8 vb = lds_b_tr(Vs, kKRow, 32 * kk, ni * 16, lane);
                o[ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[kk][0], vb, o[ni], 0, 0, 0);
                o[ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[kk][1], vb, o[ni], 0, 0, 0);
            }
        }
    }

    // merge: group 1's (o, m, l) of each row through LDS into group 0's
    // (rescaled to the common max), then normalise and store.  Lane holds
    // rows 4 lg + r, dims ni * 16 + li.
    __syncthreads();  // every group is done with its K / V tile
    float *mo = reinterpret_cast<float *>(&KV[0][0][0]);  // [4 waves][16 rows][128]
    float *mml = mo + 4 * 16 * HD;                        // [4 waves][16 rows][2]
    if (grp == 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * lg + r;
#pragma unroll
            for (int ni = 0; ni < 8; ++ni) mo[(gw * 16 + row) * HD + ni * 16 + li] = o[ni][r];
            if (li == 0) {
                mml[(gw * 16 + row) * 2] = mrow[r];
                mml[(gw * 16 + row) * 2 + 1] = lrow[r];
            }
        }
    }
    __syncthreads();
    if (grp == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * lg + r;
            const int qi = wq + row;
            const float m1 = mml[(gw * 16 + row) * 2], l1 = mml[(gw * 16 + row) * 2 + 1];
            const float mm = fmaxf(mrow[r], m1);
            const float f0 = mrow[r] == -INFINITY ? 0.0f : expf(mrow[r] - mm);
            const float f1 = m1 == -INFINITY ? 0.0f : expf(m1 - mm);
            const float inv = 1.0f / (lrow[r] * f0 + l1 * f1);
            if (qi < M) {
                float *dst = out + (size_t)qi * n_heads * HD + (size_t)h * HD;
#pragma unroll
                for (int ni = 0; ni < 8; ++ni)
                    dst[ni * 16 + li] =
                        (o[ni][r] * f0 + mo[(gw * 16 + row) * HD + ni * 16 + li] * f1) * inv;
            }
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

// Tile shape (WN waves along N) and K splits for one GEMM.  A round is one
// workgroup per slot (two per CU); the cost of a plan is its rounds times the
// stages each workgroup runs times WN (the MFMA work of a stage grows with
// WN), plus, for split K, the partials' round trip through memory (S M N
// floats written and read back, about 0.6 us of stage time per 4 MB).  Plans
// that leave the last round part empty pay for the whole round, which is
// what the shape choice avoids: Qwen3-8B at 512 positions runs every GEMM
// as one full round (QKV 3 x 4 splits, O and down 2 x 4, gate/up 3 x 1).
struct GemmPlan {
    int wn, S, MT, NT;
};

GemmPlan gemm_plan(const cw_ctx *ctx, Epi epi, int M, int N, int K) {
    const int MT = (M + kGM - 1) / kGM, nb = K / 32, slots = 2 * ctx->n_cu;
    GemmPlan best{2, 1, MT, 0};
    double best_cost = 1e30;
    for (int wn = 2; wn <= 2; ++wn) {  // (a 2 x 3 wave tile measured slower at every shape)
        const int bn = (epi == EPI_SWIGLU ? 32 : 64) * wn;
        const int NT = (N + bn - 1) / bn;
        for (int S = 1; S <= (epi == EPI_SWIGLU ? 1 : kMaxSplit); S *= 2) {
            if (S > 1 && (nb + S - 1) / S < 16) break;  // at least 16 blocks per split
            const long T = (long)MT * NT * S;
            const long rounds = (T + slots - 1) / slots;
            const int stages = ((nb + S - 1) / S + kSB - 1) / kSB;
            const double split = S > 1 ? (double)S * M * N * 4 / (4 << 20) : 0.0;
            const double cost = (double)rounds * stages * wn + split;
            if (cost < best_cost - 1e-9) {
                best_cost = cost;
                best = GemmPlan{wn, S, MT, NT};
            }
        }
    }
    return best;
}

int gemm_splits(const cw_ctx *ctx, Epi epi, int M, int N, int K) {
    return gemm_plan(ctx, epi, M, N, K).S;
}

size_t gemm_x_elems(int M, int K) {
    return (size_t)((M + kGM - 1) / kGM) * kGM * K + 32;
}

template <int EPI, int OUT, int WN>
int launch_gemm_tiles(cw_ctx *ctx, const char *label, const GemmArgs &a, const GemmPlan &p) {
    return launch(ctx, label, q4_gemm_kernel<EPI, OUT, WN>, dim3(p.MT * p.NT * p.S),
                  dim3(GT<WN>::THREADS), 0, a, p.MT, p.NT, p.S);
}

template <int EPI, int OUT>
int launch_gemm_wn(cw_ctx *ctx, const char *label, const GemmArgs &a, const GemmPlan &p) {
    return launch_gemm_tiles<EPI, OUT, 2>(ctx, label, a, p);
}

// y split for the next GEMM after the GEMM wrote it
int split_next(cw_ctx *ctx, const GemmArgs &a) {
    if (!a.split_next) return CW_OK;
    return launch_split_rows(ctx, a.y, a.next_norm, a.next_eps, a.M, a.N, a.next_hi, a.next_lo,
                             a.next_rowscale);
}

template <int EPI>
int launch_reduce_split(cw_ctx *ctx, const GemmArgs &a, int S) {
    const size_t mn = (size_t)a.M * a.N;
    if (a.next_norm)
        return launch(ctx, "q4_gemm_reduce_split", reduce_split_kernel<true, EPI>, dim3(a.M),
                      dim3(kT), 0, (const float *)a.part, S, a.N, mn, a.resid, a.y, a.next_norm,
                      a.next_eps, a.next_hi, a.next_lo, a.next_rowscale);
    return launch(ctx, "q4_gemm_reduce_split", reduce_split_kernel<false, EPI>, dim3(a.M), dim3(kT),
                  0, (const float *)a.part, S, a.N, mn, a.resid, a.y, a.next_norm, a.next_eps,
                  a.next_hi, a.next_lo, a.next_rowscale);
}

int launch_q4_gemm(cw_ctx *ctx, Epi epi, const GemmArgs &a, int *kept_splits) {
    if (kept_splits) *kept_splits = 0;
    const GemmPlan p0 = gemm_plan(ctx, epi, a.M, a.N, a.K);
    GemmPlan p = p0;
    if (epi == EPI_SWIGLU) {
        const int rc = launch_gemm_wn<EPI_SWIGLU, 0>(ctx, "q4_gemm_swiglu", a, p);
        if (rc != CW_OK) return rc;
        return split_next(ctx, a);
    }
    if (p.S > 1 && !a.part) {  // no workspace: the best unsplit plan
        p.S = 1;
        p.wn = 2;
        p.NT = (a.N + 127) / 128;
    }
    if (p.S > 1 && a.part_floats < (size_t)p.S * a.M * a.N) {
        set_error("q4 gemm: split-K workspace of %zu floats, %zu needed", a.part_floats,
                  (size_t)p.S * a.M * a.N);
        return CW_ERR_ARG;
    }
    if (p.S == 1) {
        const int rc = epi == EPI_ADD ? launch_gemm_wn<EPI_ADD, 0>(ctx, "q4_gemm_add", a, p)
                                      : launch_gemm_wn<EPI_STORE, 0>(ctx, "q4_gemm", a, p);
        if (rc != CW_OK) return rc;
        return split_next(ctx, a);
    }
    const int rc = epi == EPI_ADD ? launch_gemm_wn<EPI_ADD, 1>(ctx, "q4_gemm_add_splitk", a, p)
                                  : launch_gemm_wn<EPI_STORE, 1>(ctx, "q4_gemm_splitk", a, p);
    if (rc != CW_OK) return rc;
    if (kept_splits) {  // the caller reduces the partials itself
        *kept_splits = p.S;
        return CW_OK;
    }
    // the reduction and the next split in one pass when a row fits one
    // workgroup's registers (float4 rows, 16-byte aligned)
    const bool aligned = ((reinterpret_cast<uintptr_t>(a.y) | reinterpret_cast<uintptr_t>(a.resid) |
                           reinterpret_cast<uintptr_t>(a.part)) & 15) == 0;
    if (a.split_next && a.N % 4 == 0 && a.N / 4 <= 4 * kT && aligned)
        return epi == EPI_ADD ? launch_reduce_split<EPI_ADD>(ctx, a, p.S)
                              : launch_reduce_split<EPI_STORE>(ctx, a, p.S);
    const size_t n = (size_t)a.M * a.N;
    const unsigned blocks = (unsigned)((n + 4 * kT - 1) / (4 * kT));
    const int rr =
        epi == EPI_ADD
            ? launch(ctx, "q4_gemm_reduce", gemm_reduce_kernel<EPI_ADD>, dim3(blocks), dim3(kT), 0,
                     (const float *)a.part, p.S, n, a.resid, a.y)
            : launch(ctx, "q4_gemm_reduce", gemm_reduce_kernel<EPI_STORE>, dim3(blocks), dim3(kT),
                     0, (const float *)a.part, p.S, n, (const float *)nullptr, a.y);
    if (rr != CW_OK) return rr;
    return split_next(ctx, a);
}

int launch_qk_rope_kv(cw_ctx *ctx, const float *qkv, const float *qn, const float *kn, float eps,
                      const float *cos_t, const float *sin_t, int M, int n_heads, int n_kv,
                      int start, int kv_dtype, float *q_out, void *kc, void *vc, const float *part,
                      int splits) {
    const size_t mn = (size_t)M * (n_heads + 2 * n_kv) * 128;
    const int S = part ? splits : 0;
    const dim3 grid(M, (n_heads + n_kv + kT / 64 - 1) / (kT / 64));
    if (kv_dtype == CW_F16)
        return launch(ctx, "prefill_qk_rope_kv", qk_rope_kv_kernel<_Float16>, grid, dim3(kT), 0,
                      qkv, qn, kn, eps, cos_t, sin_t, n_heads, n_kv, start, q_out, (_Float16 *)kc,
                      (_Float16 *)vc, part, S, mn);
    return launch(ctx, "prefill_qk_rope_kv", qk_rope_kv_kernel<float>, grid, dim3(kT), 0, qkv,
                  qn, kn, eps, cos_t, sin_t, n_heads, n_kv, start, q_out, (float *)kc, (float *)vc,
                  part, S, mn);
}

int launch_attn_prefill(cw_ctx *ctx, const float *q, const void *kc, const void *vc, int M,
                        int n_heads, int n_kv, int start, float *out) {
    const float scale = 1.0f / sqrtf(128.0f);
    return launch(ctx, "prefill_attention", attn_prefill_kernel,
                  dim3(n_heads, (M + kAttQ - 1) / kAttQ), dim3(kAttThreads), 0, q,
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
    const size_t n = gemm_x_elems(m, in_f);
    const int S = gemm_splits(ctx, EPI_STORE, m, out_f, in_f);
    const size_t part = S > 1 ? (size_t)S * m * out_f : 0;
    void *scratch = nullptr;
    // hi, lo (2 B each per element, whole row tiles), row scales, partials
    // (16-byte aligned)
    const size_t lo_off = (n * 2 + 15) & ~size_t(15);
    const size_t rs_off = lo_off + ((n * 2 + 15) & ~size_t(15));
    const size_t part_off = (rs_off + (size_t)m * 4 + 15) & ~size_t(15);
    CW_TRY(ctx_scratch(ctx, part_off + part * 4, &scratch));
    uint16_t *hi = (uint16_t *)scratch, *lo = (uint16_t *)((char *)scratch + lo_off);
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
