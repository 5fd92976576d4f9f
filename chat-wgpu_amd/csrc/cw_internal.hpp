// Internal declarations shared by the HIP translation units of libchatwgpu.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <deque>
#include <string>
#include <thread>
#include <vector>

#include "chat_wgpu.h"

namespace cwi {

void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int hip_fail(hipError_t e, const char *what, const char *file, int line);

// Run f(lo, hi) over [0, n) split across up to 16 host threads (one thread
// below 64 Ki items).  Each item's result depends only on the item, so the
// split never changes the output.
template <class F>
void parallel_for(size_t n, F f) {
    unsigned hw = std::thread::hardware_concurrency();
    if (hw == 0) hw = 1;
    const size_t nt = std::min<size_t>(std::min<size_t>(hw, 16), n / 65536 + 1);
    if (nt <= 1) {
        f((size_t)0, n);
        return;
    }
    std::vector<std::thread> ts;
    const size_t step = (n + nt - 1) / nt;
    for (size_t t = 0; t < nt; ++t) {
        const size_t lo = t * step, hi = std::min(n, lo + step);
        if (lo >= hi) break;
        ts.emplace_back([=] { f(lo, hi); });
    }
    for (auto &t : ts) t.join();
}

}  // namespace cwi

#define CW_HIP(call)                                                         \
    do {                                                                     \
        hipError_t cw_e_ = (call);                                           \
        if (cw_e_ != hipSuccess) return cwi::hip_fail(cw_e_, #call, __FILE__, __LINE__); \
    } while (0)

#define CW_CHECK_ARG(cond, ...)          \
    do {                                 \
        if (!(cond)) {                   \
            cwi::set_error(__VA_ARGS__); \
            return CW_ERR_ARG;           \
        }                                \
    } while (0)

#define CW_TRY(expr)                   \
    do {                               \
        int cw_rc_ = (expr);           \
        if (cw_rc_ != CW_OK) return cw_rc_; \
    } while (0)

// One profiled launch: events bracketing it and its label.
struct cw_prof_rec {
    hipEvent_t start, stop;
    const char *label;
};

// A RoPE angle table resident on the device: cos/sin [max_pos][hd/2] f32.
struct cw_rope_tab {
    float theta;
    int head_dim;
    int max_pos;
    float *cos_t;
    float *sin_t;
};

struct cw_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int n_cu = 0;
    size_t hbm_bytes = 0;
    std::string arch;

    // persistent allocations (freed at destroy)
    std::vector<void *> allocs;

    // per-frame arena: chunks handed out in call order, rewound by reset
    struct Chunk {
        char *base;
        size_t size;
    };
    std::vector<Chunk> chunks;
    size_t chunk_idx = 0, chunk_off = 0;

    // attention arrival counters, one 128-byte line per kv head, zero
    // between launches (each launch's merging workgroup resets its own)
    unsigned *attn_cnt = nullptr;

    // kernel scratch (attention partials, argmax partials, counters) for the
    // standalone kernel entry points; grows on demand between launches, at
    // least doubling each time
    void *scratch = nullptr;
    size_t scratch_size = 0;
    // a recording (cw_graph_begin) was opened while `scratch` was current, so
    // a recorded launch sequence may name it
    bool scratch_recorded = false;
    // smaller scratch buffers a larger request replaced while a recording
    // could name them: they live until cw_ctx_destroy (at most the sum of a
    // doubling sequence, i.e. less than the current buffer)
    std::vector<void *> scratch_retired;

    // this device's static scratch of cw_attention_noalloc (set at create)
    void *noalloc_scratch = nullptr;

    // RoPE tables; a deque, so a table's address stays valid as others are added
    std::deque<cw_rope_tab> ropes;

    // a cw_graph_begin .. cw_graph_end recording is open on the stream
    bool capturing = false;

    // profiling
    bool profiling = false;
    std::vector<cw_prof_rec> prof;
    std::vector<hipEvent_t> event_pool;
    size_t event_next = 0;
};

namespace cwi {

// Scratch of at least `bytes` for the standalone kernels (synchronises the
// stream before it replaces a smaller buffer).
int ctx_scratch(cw_ctx *ctx, size_t bytes, void **out);
// Device RoPE table covering positions [0, min_pos) for (theta, head_dim).
int ctx_rope_table(cw_ctx *ctx, float theta, int head_dim, int min_pos, const cw_rope_tab **out);
// Build the host table (f64 angles rounded to f32), layout [pos][hd/2].
void rope_table_host(int max_pos, int head_dim, float theta, float *cos_t, float *sin_t);

// Profiling hooks around a launch (no-ops unless profiling): marker events
// before and after it, so the interval also holds the dispatch overhead.
void prof_begin(cw_ctx *ctx, const char *label);
void prof_end(cw_ctx *ctx);
// A profile record for the next launch and its two events (profiling only).
void prof_events(cw_ctx *ctx, const char *label, hipEvent_t *start, hipEvent_t *stop);
// Check the launch that was just enqueued.
int launch_check(const char *what);

template <typename T>
struct same_type {
    using type = T;
};

// Enqueue fn on ctx->stream.  While profiling, the dispatch itself stamps a
// pair of events at the kernel's start and end (hipExtLaunchKernel), so the
// profile holds kernel execution time, as a kernel trace does, with no
// marker packets between launches.
template <typename... KA>
int launch(cw_ctx *ctx, const char *label, void (*fn)(KA...), dim3 grid, dim3 block,
           unsigned lds, typename same_type<KA>::type... args) {
    if (ctx->profiling) {
        hipEvent_t e0 = nullptr, e1 = nullptr;
        prof_events(ctx, label, &e0, &e1);
        hipExtLaunchKernelGGL(fn, grid, block, lds, ctx->stream, e0, e1, 0, args...);
    } else {
        hipLaunchKernelGGL(fn, grid, block, lds, ctx->stream, args...);
    }
    return launch_check(label);
}

// f16 helpers on the host (IEEE binary16, round to nearest even).
uint16_t f32_to_f16_bits(float f);
float f16_bits_to_f32(uint16_t h);

// ---- kernel launchers (all enqueue on ctx->stream) ----

enum XSrc { XS_PLAIN = 0, XS_RMSNORM = 1 };
// EPI_ARGMAX: store, and the argmax of y over the whole launch (the last
// workgroup to finish merges the workgroups' bests and advances the decode
// state, like launch_argmax)
enum Epi { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

struct GenState;

struct GemvArgs {
    const float *x;         // activation [K] (raw hidden for XS_RMSNORM)
    const float *norm_w;    // XS_RMSNORM gain [K]
    float eps;
    const uint16_t *sA;     // scales of matrix A [N][K/32]
    const uint8_t *qA;      // quants of matrix A [N][K/32][16]
    const uint16_t *sB;     // EPI_SWIGLU: the up matrix
    const uint8_t *qB;
    const float *resid;     // EPI_ADD
    float *y;               // [N]
    int K, N;
    // x (resid) as row x_tok[0] (resid_tok[0]) of a table of tok_rows rows
    // at that pointer, when set: the embedding row of the device-resident
    // token (Qwen3::embed, qwen3.rs:128-133), read by the first layer
    const uint32_t *x_tok;
    const uint32_t *resid_tok;
    int tok_rows;
    // EPI_ARGMAX: per-workgroup bests [grid], the arrival counter (zero
    // between launches), the argmax output and the generate state to advance
    float *am_v;
    uint32_t *am_i;
    unsigned *am_cnt;
    uint32_t *am_out;
    GenState *state;
    const uint32_t *prompt;
    uint32_t *tokens;
    // waves of a workgroup that take wave tiles (0: all of them); set by
    // launch_q4_gemv for launches too small to give every CU a workgroup
    int tile_waves;
};

int launch_q4_gemv(cw_ctx *ctx, XSrc xs, Epi epi, const GemvArgs &a);

// Attention: fused q/k-norm + RoPE + KV write + split-sequence partial
// softmax + merge.
struct AttnArgs {
    const float *q;        // [n_heads*hd] (already normed/rotated) if qkv == null
    const float *qkv;      // fused path: raw [q | k | v] GEMV output
    const float *q_norm_w; // fused path gains [hd]
    const float *k_norm_w;
    float eps;
    const float *cos_t, *sin_t;  // fused path RoPE table [max_pos][hd/2]
    void *k_cache, *v_cache;     // [max_seq][n_kv*hd]
    int kv_dtype;
    int n_heads, n_kv, hd;
    int seq;                // used when pos_dev == null
    const int *pos_dev;     // device position; seq = pos+1 (fused path writes KV at pos)
    int max_seq;            // grid sizing (positions the cache can hold)
    float *out;             // [n_heads*hd]
    float *part;            // chunk partials, attn_scratch_floats() floats
    unsigned *cnt;          // set by launch_attention: the context's per-kv-head counters
    float *q_tap;           // fused path, optional: the normalised, rotated q [n_heads*hd]
};

// kv heads the attention counters cover (cw_ctx::attn_cnt)
constexpr int kMaxAttnKv = 1024;

size_t attn_scratch_floats(int n_heads, int n_kv, int hd, int max_seq);
// Take this device's address of cw_attention_noalloc's static scratch (once
// per device; the device must be current) and clear its counters.
int attn_noalloc_setup(cw_ctx *ctx);
int launch_attention(cw_ctx *ctx, const AttnArgs &a);

int launch_rmsnorm(cw_ctx *ctx, const float *x, const float *w, int rows, int dim, float eps,
                   float *y);
int launch_rope(cw_ctx *ctx, const float *x, int rows, int hd, int pos, const float *cos_t,
                const float *sin_t, float *y);
int launch_add(cw_ctx *ctx, const float *a, const float *b, int n, float *c);
int launch_swiglu(cw_ctx *ctx, const float *g, const float *u, int n, float *out);
int launch_kv_write(cw_ctx *ctx, void *kc, void *vc, int kv_dtype, int pos, const int *pos_dev,
                    int kv_dim, const float *k, const float *v);
int launch_embed(cw_ctx *ctx, const float *table, int vocab, int dim, const uint32_t *tok_dev,
                 float *out);

// Argmax: stage 1 over blocks, stage 2 merge.  When `state` is non-null the
// merge also advances the device-resident generate state.
struct GenState {
    int pos;          // position of the next forward
    uint32_t token;   // token fed at pos
    int start_pos;    // position of the first forward of this generate call
    int n_prompt;
    int produced;
    int max_out;
};
size_t argmax_scratch_bytes(int n);
// Scratch of the LM head's fused argmax (EPI_ARGMAX): per-workgroup bests
// for any grid launch_q4_gemv picks, then the arrival counter line.
size_t lm_argmax_scratch_bytes(const cw_ctx *ctx);
// The LM head with the fused argmax over its own scratch (zeroed once).
int launch_lm_head_argmax(cw_ctx *ctx, GemvArgs g, void *scratch, uint32_t *out_dev,
                          GenState *state, const uint32_t *prompt_dev, uint32_t *tokens_out_dev);
int launch_argmax(cw_ctx *ctx, const float *logits, int n, uint32_t *out_dev, void *scratch,
                  GenState *state, const uint32_t *prompt_dev, uint32_t *tokens_out_dev);

// ---- batched prefill (M positions per launch)

// y[M][N] = x[M][K] . W[N][K]^T with x given as bf16 hi/lo rows and W split
// GGUF Q4_0; EPI_SWIGLU reads a second matrix (B) and stores silu(A x) * (B x).
struct GemmArgs {
    const uint16_t *xhi, *xlo;  // [M][K] f16 bits, row m scaled by 1 / rowscale[m]
                                // (allocated for gemm_x_elems(M, K))
    const float *rowscale;      // [M] powers of two
    const uint16_t *sA;
    const uint8_t *qA;
    const uint16_t *sB;
    const uint8_t *qB;
    const float *resid;  // EPI_ADD: [M][N]
    float *y;            // [M][N]
    int M, N, K;
    float *part;         // split-K partials (null: no split)
    size_t part_floats;  // capacity of part
    // optional: y also split for the next GEMM, exactly as launch_split_rows
    // (x = y, norm_w = next_norm) would; with split K it is done by the
    // reduction of the partials, in the same pass
    bool split_next;
    const float *next_norm;
    float next_eps;
    uint16_t *next_hi, *next_lo;
    float *next_rowscale;
};
// K splits the GEMM uses for this shape (the partial workspace holds
// splits * M * N floats)
int gemm_splits(const cw_ctx *ctx, Epi epi, int M, int N, int K);
// Elements each of GemmArgs::xhi / xlo must hold for M rows of K: whole
// 128-row tiles plus one block (the GEMM's DMA reads them; rows past M are
// never stored to y, so they need no values)
size_t gemm_x_elems(int M, int K);
// token ids on the device (validated < vocab by the caller)
int launch_embed_rows(cw_ctx *ctx, const float *table, int dim, const uint32_t *tok_dev, int n,
                      float *out);
int launch_split_rows(cw_ctx *ctx, const float *x, const float *norm_w, float eps, int rows, int K,
                      uint16_t *hi, uint16_t *lo, float *rowscale);
// kept_splits (optional): with split K, leave the partials in a.part
// unreduced and set *kept_splits = K splits (0 when y was written)
int launch_q4_gemm(cw_ctx *ctx, Epi epi, const GemmArgs &a, int *kept_splits = nullptr);
// qkv: [M][q | k | v] rows, or (splits > 0) the sum in order of `splits`
// partials part[s][M][q | k | v] (gemm_reduce_kernel's sum)
int launch_qk_rope_kv(cw_ctx *ctx, const float *qkv, const float *qn, const float *kn, float eps,
                      const float *cos_t, const float *sin_t, int M, int n_heads, int n_kv,
                      int start, int kv_dtype, float *q_out, void *kc, void *vc,
                      const float *part = nullptr, int splits = 0);
// causal attention of positions start..start+M-1 over an f16 cache, head_dim 128
int launch_attn_prefill(cw_ctx *ctx, const float *q, const void *kc, const void *vc, int M,
                        int n_heads, int n_kv, int start, float *out);

// ---- the fused decode step (one persistent cooperative kernel per token)

constexpr int kStepMaxKv = 32;

struct StepLayer {
    const float *attn_norm, *q_norm, *k_norm, *ffn_norm;
    const uint8_t *qkv_q;
    const uint16_t *qkv_s;
    const uint8_t *o_q;
    const uint16_t *o_s;
    const uint8_t *gu_q;      // gate rows then up rows: [2*hidden][dim]
    const uint16_t *gu_s;
    const uint8_t *down_q;
    const uint16_t *down_s;
    void *kc, *vc;  // this layer's [max_seq][n_kv*128] caches
};

struct StepArgs {
    const StepLayer *layers;  // device array [n_layers]
    int n_layers, dim, n_heads, n_kv, hidden, vocab;
    int max_chunks;           // attention partial slots per head
    int max_seq;              // KV cache capacity (positions)
    float eps, scale;
    const float *embed, *final_norm;
    const uint8_t *lm_q;
    const uint16_t *lm_s;
    const float *cos_t, *sin_t;
    // per-launch activations, each written once: h_a [L+1][dim], h_b [L][dim],
    // qkv [L][q+2kv], attn [L][q], act [L][2*hidden] (gate then up outputs)
    float *h_a, *h_b, *qkv, *attn, *act;
    float *part;              // [n_heads][max_chunks][130]
    float *logits, *hidden_out;
    float *am_v;              // per-workgroup argmax [n_cu]
    uint32_t *am_i;
    unsigned *sync;           // step_sync_words() counters, zero between launches
    GenState *state;
    const uint32_t *prompt;
    uint32_t *tokens, *argmax_out;
    long long timeout;        // barrier spin limit in wall-clock ticks
    long long *trace;         // optional phase stamps (workgroup 0), else null
};

// A device allocation [p, p + bytes) the fused step may touch.
struct Extent {
    const void *p;
    size_t bytes;
};
// Host-side check of the fused step's buffer layout: every range that any
// phase of the step reads or writes (weights, activations, caches, partials,
// counters), computed from the same phase table the kernel uses, must lie
// inside one of `ext`.  `a.layers` must point at the host copy of the layer
// table.  Returns false with the first offending range in *why.
// The check also covers the device argument block `args_dev` and layer
// table `layers_dev` (sizeof(StepArgs), n_layers StepLayer), the dynamic and
// static LDS of every phase, and the phase stamps when `a.trace` is set.
bool step_check_ranges(const StepArgs &a, const void *args_dev, const void *layers_dev,
                       int kv_dtype, int head_dim, int n_cu, const std::vector<Extent> &ext,
                       std::string *why);
// int64 phase stamps one launch writes when tracing
size_t step_trace_words(int n_layers);

size_t step_sync_words();
int step_sync_err_index();
int step_cpmax(int kv_dtype, int hpk);
int step_lds_bytes(int kv_dtype, int hpk, int max_seq);
// nullptr if the fused step supports the shape, else the reason
const char *step_unsupported(int head_dim, int hpk, int n_kv, int dim, int q_dim, int hidden,
                             int max_seq);
// a_dev: the argument block in device memory
int launch_decode_step(cw_ctx *ctx, const StepArgs *a_dev, int kv_dtype, int hpk, int max_seq);

}  // namespace cwi
