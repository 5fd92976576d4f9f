// Qwen3 decode model and the greedy token loop.
//
// Replaces Qwen3::load/forward/logits (src/model/qwen3.rs:44-191), KvCache
// (src/model/cache.rs), Q4Linear/Proj/RmsNorm (src/model/layers.rs:74-191)
// and model::generate (src/model/mod.rs:57-125).
//
// One decode step is 2 + 6 * n_layers launches on one stream:
//   embed (token read on the device)
//   per layer: RMSNorm+QKV GEMV | QK-norm+RoPE+KV write+attention partials |
//              attention merge | O GEMV + residual | RMSNorm+gate/up GEMV+SwiGLU |
//              down GEMV + residual
//   final RMSNorm + LM head GEMV | argmax (advances the device generate state)
// Position and token live in device memory, so the same launch sequence is
// valid for every token and is captured once as a HIP graph and replayed
// (the reference keeps "the same op sequence every token", mod.rs:78-81).

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "cw_internal.hpp"

using namespace cwi;

namespace {

struct Q4W {
    uint16_t *s = nullptr;
    uint8_t *q = nullptr;
    int out_f = 0, in_f = 0;
};

struct Layer {
    float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *ffn_norm = nullptr;
    // q|k|v rows in one matrix; gate then up rows in one matrix `gu`
    // [2*hidden][dim], with `gate` and `up` its two halves
    Q4W qkv, wo, gu, gate, up, down;
};

// tensor ids within a layer
enum { T_ATTN_NORM, T_Q_NORM, T_K_NORM, T_FFN_NORM, T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN, T_N };
const char *kLayerNames[T_N] = {"attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm", "attn_q",
                                "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                                "ffn_down"};

}  // namespace

struct cw_model {
    cw_ctx *ctx = nullptr;
    cw_model_config cfg{};
    int q_dim = 0, kv_dim = 0;
    std::vector<Layer> layers;
    std::vector<std::vector<bool>> have;  // [layer][T_N]
    bool have_embed = false, have_final = false, have_output = false;
    float *embed = nullptr, *final_norm = nullptr;
    Q4W lm_head;
    void *kcache = nullptr, *vcache = nullptr;  // [L][max_seq][kv_dim]
    size_t kv_layer_bytes = 0;
    const float *cos_t = nullptr, *sin_t = nullptr;
    float *hidden = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
    float *hidden_out = nullptr;
    // hook taps of the last decode step (cw_model_set_taps): "q" [L][q_dim],
    // "post_attn" and "layer_out" [L][dim]; with taps on, the layers' hidden
    // states are written straight into them
    bool taps = false;
    float *tap_q = nullptr, *tap_post = nullptr, *tap_out = nullptr;
    float *part = nullptr;
    void *argmax_scratch = nullptr;
    void *lm_scratch = nullptr;  // the LM head's fused argmax (counter zero between launches)
    int host_pos = 0;            // the device state's pos, mirrored (every step advances it by 1)
    GenState *state = nullptr;
    uint32_t *prompt_dev = nullptr, *tokens_dev = nullptr, *argmax_out = nullptr;
    bool finalized = false;
    // every device allocation of the model, for the fused step's range check
    std::vector<Extent> extents;
    // dry plan: addresses are handed out from an unmapped range and nothing
    // touches a device (cw_step_layout_check); `dry_split_gu` lays gate and up
    // out as two allocations, the layout the step's range check refuses
    bool dry = false;
    bool dry_split_gu = false;
    int dry_n_cu = 0;
    uintptr_t dry_next = 0;
    char fused_why[256] = {0};
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    std::vector<void *> allocs;

    // batched prefill buffers, sized for pf_cap positions (grown on demand)
    int pf_cap = 0;
    float *pf_hidden = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_attn = nullptr,
          *pf_act = nullptr;
    uint16_t *pf_hi = nullptr, *pf_lo = nullptr;
    float *pf_rowscale = nullptr;  // per-row powers of two of the GEMM operand split
    float *pf_part = nullptr;  // split-K partials of the prefill GEMMs
    size_t pf_part_floats = 0;
    std::vector<void *> pf_allocs;

    // fused decode step (one persistent kernel per token)
    const char *fused_unsupported = nullptr;
    StepArgs step{};
    StepArgs *step_dev = nullptr;  // `step` in device memory (the kernel reads it there)
    StepLayer *step_layers = nullptr;
    unsigned *step_sync = nullptr;
};

namespace {

// The persistent decode-step kernel is switched off: it raised an illegal
// memory access on the GPU, and again after its gate|up layout was fixed (the
// layout the host-side range check now enforces), so a second cause remains
// unfound.  Every entry point that would launch it returns CW_ERR_STATE.
constexpr bool kFusedStepDisabled = true;

// Model calls synchronise, allocate or clear memory, none of which may be
// recorded into a caller's launch sequence (cw_graph_begin .. cw_graph_end).
int refuse_recording(const cw_model *m, const char *what) {
    if (!m->ctx->capturing) return CW_OK;
    set_error("%s: not allowed while a graph is being recorded (end it with cw_graph_end)", what);
    return CW_ERR_STATE;
}

int dalloc(cw_model *m, size_t bytes, void **out) {
    void *p = nullptr;
    if (m->dry) {
        // page-aligned, one unmapped page between allocations, so a range
        // that runs past its buffer never lands inside the next one
        m->dry_next = (m->dry_next + 4095) & ~(uintptr_t)4095;
        p = reinterpret_cast<void *>(m->dry_next);
        m->dry_next += bytes + 4096;
    } else {
        CW_HIP(hipMalloc(&p, bytes));
        m->allocs.push_back(p);
    }
    m->extents.push_back(Extent{p, bytes});
    *out = p;
    return CW_OK;
}

int alloc_q4(cw_model *m, Q4W &w, int out_f, int in_f) {
    w.out_f = out_f;
    w.in_f = in_f;
    const size_t nblk = (size_t)out_f * (in_f / 32);
    CW_TRY(dalloc(m, nblk * 2, (void **)&w.s));
    CW_TRY(dalloc(m, nblk * 16, (void **)&w.q));
    return CW_OK;
}

// rows [row0, row0 + rows) of w as a matrix of its own (no allocation)
Q4W q4_rows(const Q4W &w, int row0, int rows) {
    const size_t nb = w.in_f / 32;
    Q4W v;
    v.s = w.s + (size_t)row0 * nb;
    v.q = w.q + (size_t)row0 * nb * 16;
    v.out_f = rows;
    v.in_f = w.in_f;
    return v;
}

int upload_rows(cw_model *m, Q4W &w, int row0, int rows, const uint16_t *s, const uint8_t *q) {
    const size_t nb = w.in_f / 32;
    CW_TRY(cw_upload(m->ctx, w.s + (size_t)row0 * nb, s, (size_t)rows * nb * 2));
    CW_TRY(cw_upload(m->ctx, w.q + (size_t)row0 * nb * 16, q, (size_t)rows * nb * 16));
    return CW_OK;
}

// Parse "blk.<i>.<name>.weight" -> (layer, tensor id); -1 when not a layer tensor.
int parse_layer_name(const char *name, int n_layers, int *layer, int *id) {
    int li = -1, consumed = 0;
    if (sscanf(name, "blk.%d.%n", &li, &consumed) != 1 || consumed == 0) return -1;
    if (li < 0 || li >= n_layers) return -2;
    const char *rest = name + consumed;
    for (int t = 0; t < T_N; ++t) {
        std::string want = std::string(kLayerNames[t]) + ".weight";
        if (want == rest) {
            *layer = li;
            *id = t;
            return 0;
        }
    }
    return -2;
}

// The shape (out_f, in_f) of a projection.
void proj_shape(const cw_model *m, int id, int *out_f, int *in_f) {
    const auto &c = m->cfg;
    switch (id) {
        case T_Q: *out_f = m->q_dim; *in_f = c.dim; break;
        case T_K:
        case T_V: *out_f = m->kv_dim; *in_f = c.dim; break;
        case T_O: *out_f = c.dim; *in_f = m->q_dim; break;
        case T_GATE:
        case T_UP: *out_f = c.hidden; *in_f = c.dim; break;
        default: *out_f = c.dim; *in_f = c.hidden; break;  // T_DOWN
    }
}

// The hidden state after the last layer of a decode step.
float *last_hidden(cw_model *m) {
    return m->taps ? m->tap_out + (size_t)(m->cfg.n_layers - 1) * m->cfg.dim : m->hidden;
}

int enqueue_step(cw_model *m) {
    cw_ctx *ctx = m->ctx;
    const auto &c = m->cfg;
    // the first layer reads the token's embedding row itself (its QKV input
    // and its attention residual): no separate gather launch
    const float *h_in = m->hidden;  // this layer's input; updated in place unless taps are on
    for (int i = 0; i < c.n_layers; ++i) {
        Layer &L = m->layers[i];
        float *h_post = m->taps ? m->tap_post + (size_t)i * c.dim : m->hidden;
        float *h_out = m->taps ? m->tap_out + (size_t)i * c.dim : h_post;
        const bool first = i == 0;
        GemvArgs g{};
        g.x = first ? m->embed : h_in;
        g.x_tok = first ? &m->state->token : nullptr;
        g.tok_rows = c.vocab;
        g.norm_w = L.attn_norm;
        g.eps = c.eps;
        g.sA = L.qkv.s;
        g.qA = L.qkv.q;
        g.y = m->qkv;
        g.K = c.dim;
        g.N = L.qkv.out_f;
        CW_TRY(launch_q4_gemv(ctx, XS_RMSNORM, EPI_STORE, g));

        AttnArgs a{};
        a.qkv = m->qkv;
        a.q_norm_w = L.q_norm;
        a.k_norm_w = L.k_norm;
        a.eps = c.eps;
        a.cos_t = m->cos_t;
        a.sin_t = m->sin_t;
        a.k_cache = (char *)m->kcache + (size_t)i * m->kv_layer_bytes;
        a.v_cache = (char *)m->vcache + (size_t)i * m->kv_layer_bytes;
        a.kv_dtype = c.kv_dtype;
        a.n_heads = c.n_heads;
        a.n_kv = c.n_kv_heads;
        a.hd = c.head_dim;
        a.pos_dev = &m->state->pos;
        a.max_seq = c.max_seq;
        a.out = m->attn;
        a.part = m->part;
        a.q_tap = m->taps ? m->tap_q + (size_t)i * m->q_dim : nullptr;
        CW_TRY(launch_attention(ctx, a));

        g = GemvArgs{};
        g.x = m->attn;
        g.sA = L.wo.s;
        g.qA = L.wo.q;
        g.resid = first ? m->embed : h_in;
        g.resid_tok = first ? &m->state->token : nullptr;
        g.tok_rows = c.vocab;
        g.y = h_post;
        g.K = m->q_dim;
        g.N = c.dim;
        CW_TRY(launch_q4_gemv(ctx, XS_PLAIN, EPI_ADD, g));

        g = GemvArgs{};
        g.x = h_post;
        g.norm_w = L.ffn_norm;
        g.eps = c.eps;
        g.sA = L.gate.s;
        g.qA = L.gate.q;
        g.sB = L.up.s;
        g.qB = L.up.q;
        g.y = m->act;
        g.K = c.dim;
        g.N = c.hidden;
        CW_TRY(launch_q4_gemv(ctx, XS_RMSNORM, EPI_SWIGLU, g));

        g = GemvArgs{};
        g.x = m->act;
        g.sA = L.down.s;
        g.qA = L.down.q;
        g.resid = h_post;
        g.y = h_out;
        g.K = c.hidden;
        g.N = c.dim;
        CW_TRY(launch_q4_gemv(ctx, XS_PLAIN, EPI_ADD, g));
        h_in = h_out;
    }
    GemvArgs g{};
    g.x = h_in;
    g.norm_w = m->final_norm;
    g.eps = c.eps;
    g.sA = m->lm_head.s;
    g.qA = m->lm_head.q;
    g.y = m->logits;
    g.K = c.dim;
    g.N = c.vocab;
    // logits, their argmax and the generate state's advance in one launch
    return launch_lm_head_argmax(ctx, g, m->lm_scratch, m->argmax_out, m->state, m->prompt_dev,
                                 m->tokens_dev);
}

int ensure_graph(cw_model *m) {
    if (m->graph_exec) return CW_OK;
    cw_ctx *ctx = m->ctx;
    const bool prof = ctx->profiling;
    ctx->profiling = false;
    CW_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
    ctx->scratch_recorded = true;  // (the step uses the model's own buffers)
    int rc = enqueue_step(m);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    ctx->profiling = prof;
    if (rc != CW_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
    }
    m->graph = graph;
    m->graph_exec = exec;
    return CW_OK;
}

// The fused step's counters after a launch sequence: a set error word means
// a grid barrier timed out; the counters are cleared for the next launch.
int check_fused(cw_model *m) {
    if (!m->step_sync) return CW_OK;
    unsigned err = 0;
    CW_HIP(hipMemcpyAsync(&err, m->step_sync + step_sync_err_index(), 4, hipMemcpyDeviceToHost,
                          m->ctx->stream));
    CW_HIP(hipStreamSynchronize(m->ctx->stream));
    if (err) {
        CW_HIP(hipMemsetAsync(m->step_sync, 0, step_sync_words() * 4, m->ctx->stream));
        set_error(err == 2 ? "decode step: position outside the KV cache (launch skipped)"
                           : "decode step: a grid barrier timed out (launch abandoned)");
        return CW_ERR_HIP;
    }
    return CW_OK;
}

int run_steps(cw_model *m, int n, int mode) {
    if (mode == CW_STEP_FUSED) {
        if (kFusedStepDisabled) {
            set_error("fused decode step disabled: it raised an illegal memory access on the "
                      "GPU whose cause is not yet found (use CW_STEP_GRAPH)");
            return CW_ERR_STATE;
        }
        if (m->fused_unsupported) {
            set_error("fused decode step unavailable for this model: %s", m->fused_unsupported);
            return CW_ERR_ARG;
        }
        const auto &c = m->cfg;
        for (int i = 0; i < n; ++i) {
            CW_TRY(launch_decode_step(m->ctx, m->step_dev, c.kv_dtype, c.n_heads / c.n_kv_heads,
                                      c.max_seq));
            ++m->host_pos;
        }
    } else if (mode == CW_STEP_GRAPH) {
        CW_TRY(ensure_graph(m));
        for (int i = 0; i < n; ++i) {
            CW_HIP(hipGraphLaunch(m->graph_exec, m->ctx->stream));
            ++m->host_pos;
        }
    } else if (mode == CW_STEP_EAGER) {
        // a step advances the device position in its last launch (the LM
        // head's epilogue): a step whose launches failed part-way never does
        for (int i = 0; i < n; ++i) {
            CW_TRY(enqueue_step(m));
            ++m->host_pos;
        }
    } else {
        set_error("unknown step mode %d", mode);
        return CW_ERR_ARG;
    }
    return CW_OK;
}

// The fused step's layer table (host copy) and argument block, with the
// buffers it owns; nothing is uploaded or launched (so the dry plan runs it).
int build_step(cw_model *m, std::vector<StepLayer> &host) {
    const auto &c = m->cfg;
    const int L = c.n_layers;
    host.assign(L, StepLayer{});
    for (int i = 0; i < L; ++i) {
        const Layer &y = m->layers[i];
        StepLayer &s = host[i];
        s.attn_norm = y.attn_norm;
        s.q_norm = y.q_norm;
        s.k_norm = y.k_norm;
        s.ffn_norm = y.ffn_norm;
        s.qkv_q = y.qkv.q;
        s.qkv_s = y.qkv.s;
        s.o_q = y.wo.q;
        s.o_s = y.wo.s;
        // the step reads gate|up as one [2*hidden][dim] matrix: `gu`, of
        // which gate and up are the halves (a split plan hands it the gate
        // matrix alone, the layout the range check below refuses)
        const Q4W &gu = m->dry_split_gu ? y.gate : y.gu;
        s.gu_q = gu.q;
        s.gu_s = gu.s;
        s.down_q = y.down.q;
        s.down_s = y.down.s;
        s.kc = (char *)m->kcache + (size_t)i * m->kv_layer_bytes;
        s.vc = (char *)m->vcache + (size_t)i * m->kv_layer_bytes;
    }
    StepArgs &a = m->step;
    CW_TRY(dalloc(m, sizeof(StepLayer) * L, (void **)&m->step_layers));
    const int max_chunks = (c.max_seq + 7) / 8;
    const int n_cu = m->dry ? m->dry_n_cu : m->ctx->n_cu;
    CW_TRY(dalloc(m, (size_t)(L + 1) * c.dim * 4, (void **)&a.h_a));
    CW_TRY(dalloc(m, (size_t)L * c.dim * 4, (void **)&a.h_b));
    CW_TRY(dalloc(m, (size_t)L * (m->q_dim + 2 * m->kv_dim) * 4, (void **)&a.qkv));
    CW_TRY(dalloc(m, (size_t)L * m->q_dim * 4, (void **)&a.attn));
    CW_TRY(dalloc(m, (size_t)L * 2 * c.hidden * 4, (void **)&a.act));
    CW_TRY(dalloc(m, (size_t)c.n_heads * max_chunks * (c.head_dim + 2) * 4, (void **)&a.part));
    CW_TRY(dalloc(m, (size_t)n_cu * 4, (void **)&a.am_v));
    CW_TRY(dalloc(m, (size_t)n_cu * 4, (void **)&a.am_i));
    CW_TRY(dalloc(m, step_sync_words() * 4, (void **)&m->step_sync));
    a.layers = m->step_layers;
    a.n_layers = L;
    a.dim = c.dim;
    a.n_heads = c.n_heads;
    a.n_kv = c.n_kv_heads;
    a.hidden = c.hidden;
    a.vocab = c.vocab;
    a.max_chunks = max_chunks;
    a.max_seq = c.max_seq;
    a.eps = c.eps;
    a.scale = powf((float)c.head_dim, -0.5f);
    a.embed = m->embed;
    a.final_norm = m->final_norm;
    a.lm_q = m->lm_head.q;
    a.lm_s = m->lm_head.s;
    a.cos_t = m->cos_t;
    a.sin_t = m->sin_t;
    a.logits = m->logits;
    a.hidden_out = m->hidden_out;
    a.sync = m->step_sync;
    a.state = m->state;
    a.prompt = m->prompt_dev;
    a.tokens = m->tokens_dev;
    a.argmax_out = m->argmax_out;
    a.trace = nullptr;
    CW_TRY(dalloc(m, sizeof(StepArgs), (void **)&m->step_dev));
    return CW_OK;
}

// The step's range check over the model's allocations: false (with the
// reason in m->fused_why) when some phase would touch memory outside them.
bool check_step(cw_model *m, const std::vector<StepLayer> &host) {
    StepArgs a = m->step;
    a.layers = host.data();
    std::string why;
    const int n_cu = m->dry ? m->dry_n_cu : m->ctx->n_cu;
    if (step_check_ranges(a, m->step_dev, m->step_layers, m->cfg.kv_dtype, m->cfg.head_dim, n_cu,
                          m->extents, &why))
        return true;
    snprintf(m->fused_why, sizeof m->fused_why, "buffer layout check failed: %s", why.c_str());
    return false;
}

// Buffers and the layer table of the fused step (after every weight exists).
int setup_fused(cw_model *m) {
    const auto &c = m->cfg;
    m->fused_unsupported = step_unsupported(c.head_dim, c.n_heads / c.n_kv_heads, c.n_kv_heads,
                                            c.dim, m->q_dim, c.hidden, c.max_seq);
    if (m->fused_unsupported) return CW_OK;
    std::vector<StepLayer> host;
    CW_TRY(build_step(m, host));
    if (!check_step(m, host)) {
        m->fused_unsupported = m->fused_why;
        return CW_OK;
    }
    if (m->dry) return CW_OK;
    CW_TRY(cw_upload(m->ctx, m->step_layers, host.data(), sizeof(StepLayer) * host.size()));
    CW_HIP(hipMemsetAsync(m->step_sync, 0, step_sync_words() * 4, m->ctx->stream));
    int rate_khz = 0;
    CW_HIP(hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, m->ctx->device));
    if (rate_khz <= 0) rate_khz = 100000;
    m->step.timeout = (long long)rate_khz * 1000 * 2;  // 2 s
    CW_TRY(cw_upload(m->ctx, m->step_dev, &m->step, sizeof(StepArgs)));
    return CW_OK;
}

// Batched prefill buffers for n positions.
int ensure_prefill(cw_model *m, int n) {
    if (n <= m->pf_cap) return CW_OK;
    CW_HIP(hipStreamSynchronize(m->ctx->stream));
    for (void *p : m->pf_allocs) CW_HIP(hipFree(p));
    m->pf_allocs.clear();
    m->pf_cap = 0;
    const auto &c = m->cfg;
    const size_t wide = std::max({(size_t)c.dim, (size_t)m->q_dim, (size_t)c.hidden});
    auto al = [&](size_t bytes, void **out) -> int {
        CW_HIP(hipMalloc(out, bytes));
        m->pf_allocs.push_back(*out);
        return CW_OK;
    };
    CW_TRY(al((size_t)n * c.dim * 4, (void **)&m->pf_hidden));
    CW_TRY(al((size_t)n * (m->q_dim + 2 * m->kv_dim) * 4, (void **)&m->pf_qkv));
    CW_TRY(al((size_t)n * m->q_dim * 4, (void **)&m->pf_q));
    CW_TRY(al((size_t)n * m->q_dim * 4, (void **)&m->pf_attn));
    CW_TRY(al((size_t)n * c.hidden * 4, (void **)&m->pf_act));
    CW_TRY(al(gemm_x_elems(n, (int)wide) * 2, (void **)&m->pf_hi));
    CW_TRY(al(gemm_x_elems(n, (int)wide) * 2, (void **)&m->pf_lo));
    CW_TRY(al((size_t)n * 4, (void **)&m->pf_rowscale));
    // split-K workspace: the largest splits x M x N of the unfused GEMMs
    size_t part = 0;
    const int qkv_n = m->q_dim + 2 * m->kv_dim;
    const int shapes[3][2] = {{qkv_n, c.dim}, {c.dim, m->q_dim}, {c.dim, c.hidden}};  // N, K
    for (const auto &sh : shapes) {
        const int S = gemm_splits(m->ctx, EPI_ADD, n, sh[0], sh[1]);
        if (S > 1) part = std::max(part, (size_t)S * n * sh[0]);
    }
    if (part > 0) {
        CW_TRY(al(part * 4, (void **)&m->pf_part));
        m->pf_part_floats = part;
    }
    m->pf_cap = n;
    return CW_OK;
}

// One linear layer of the batched forward: rows of x (optionally
// RMS-normalised) through a Q4_0 matrix pair or single matrix.
// y[n][out] = [resid +] (RMSNorm?) x . W^T on the batched GEMM.  x_split:
// pf_hi / pf_lo / pf_rowscale already hold x's split (the previous GEMM left
// it); next_split: leave y's split there for the next GEMM, RMS-normalised
// with next_norm when set.
int pf_linear(cw_model *m, const float *x, const float *norm_w, int n, int K, Epi epi,
              const Q4W &w, const Q4W *w2, const float *resid, float *y, bool x_split = false,
              bool next_split = false, const float *next_norm = nullptr,
              int *kept_splits = nullptr) {
    if (!x_split)
        CW_TRY(launch_split_rows(m->ctx, x, norm_w, m->cfg.eps, n, K, m->pf_hi, m->pf_lo,
                                 m->pf_rowscale));
    GemmArgs a{};
    a.split_next = next_split;
    a.next_norm = next_norm;
    a.next_eps = m->cfg.eps;
    a.next_hi = m->pf_hi;
    a.next_lo = m->pf_lo;
    a.next_rowscale = m->pf_rowscale;
    a.xhi = m->pf_hi;
    a.xlo = m->pf_lo;
    a.rowscale = m->pf_rowscale;
    a.sA = w.s;
    a.qA = w.q;
    if (w2) {
        a.sB = w2->s;
        a.qB = w2->q;
    }
    a.resid = resid;
    a.y = y;
    a.M = n;
    a.N = w.out_f;
    a.K = K;
    a.part = m->pf_part;
    a.part_floats = m->pf_part_floats;
    return launch_q4_gemm(m->ctx, epi, a, kept_splits);
}

// With taps on: row `row` of a batched [n][floats] buffer into a tap.
int tap_row(cw_model *m, float *dst, const float *src, int row, int floats) {
    if (!m->taps) return CW_OK;
    CW_HIP(hipMemcpyAsync(dst, src + (size_t)row * floats, (size_t)floats * 4,
                          hipMemcpyDeviceToDevice, m->ctx->stream));
    return CW_OK;
}

// Forward of n positions start..start+n-1 (tokens in m->prompt_dev) through
// every layer with the batched kernels; leaves the hidden rows in pf_hidden.
// With taps on, the taps are those of the last position's forward.
int enqueue_prefill(cw_model *m, int n, int start) {
    cw_ctx *ctx = m->ctx;
    const auto &c = m->cfg;
    CW_TRY(launch_embed_rows(ctx, m->embed, c.dim, m->prompt_dev, n, m->pf_hidden));
    for (int i = 0; i < c.n_layers; ++i) {
        Layer &L = m->layers[i];
        void *kc = (char *)m->kcache + (size_t)i * m->kv_layer_bytes;
        void *vc = (char *)m->vcache + (size_t)i * m->kv_layer_bytes;
        // the split of the layer's input: the previous layer's down GEMM left
        // it; with split K the partials go straight to the QK-norm + RoPE pass
        int qkv_splits = 0;
        CW_TRY(pf_linear(m, m->pf_hidden, L.attn_norm, n, c.dim, EPI_STORE, L.qkv, nullptr,
                         nullptr, m->pf_qkv, i > 0, false, nullptr, &qkv_splits));
        CW_TRY(launch_qk_rope_kv(ctx, m->pf_qkv, L.q_norm, L.k_norm, c.eps, m->cos_t, m->sin_t, n,
                                 c.n_heads, c.n_kv_heads, start, c.kv_dtype, m->pf_q, kc, vc,
                                 qkv_splits ? m->pf_part : nullptr, qkv_splits));
        CW_TRY(tap_row(m, m->tap_q + (size_t)i * m->q_dim, m->pf_q, n - 1, m->q_dim));
        CW_TRY(launch_attn_prefill(ctx, m->pf_q, kc, vc, n, c.n_heads, c.n_kv_heads, start,
                                   m->pf_attn));
        CW_TRY(pf_linear(m, m->pf_attn, nullptr, n, m->q_dim, EPI_ADD, L.wo, nullptr,
                         m->pf_hidden, m->pf_hidden, false, true, L.ffn_norm));
        CW_TRY(tap_row(m, m->tap_post + (size_t)i * c.dim, m->pf_hidden, n - 1, c.dim));
        CW_TRY(pf_linear(m, m->pf_hidden, L.ffn_norm, n, c.dim, EPI_SWIGLU, L.gate, &L.up,
                         nullptr, m->pf_act, true));
        const bool more = i + 1 < c.n_layers;
        CW_TRY(pf_linear(m, m->pf_act, nullptr, n, c.hidden, EPI_ADD, L.down, nullptr,
                         m->pf_hidden, m->pf_hidden, false, more,
                         more ? m->layers[i + 1].attn_norm : nullptr));
        CW_TRY(tap_row(m, m->tap_out + (size_t)i * c.dim, m->pf_hidden, n - 1, c.dim));
    }
    return CW_OK;
}

int set_state(cw_model *m, const GenState &s) {
    CW_HIP(hipMemcpyAsync(m->state, &s, sizeof s, hipMemcpyHostToDevice, m->ctx->stream));
    CW_HIP(hipStreamSynchronize(m->ctx->stream));
    m->host_pos = s.pos;
    return CW_OK;
}

int require_final(cw_model *m, const char *what) {
    if (!m->finalized) {
        set_error("%s: model not finalized (call cw_model_finalize)", what);
        return CW_ERR_STATE;
    }
    return CW_OK;
}

// The configuration checks of cw_model_create.
int check_config(const cw_model_config &cfg, const char *what) {
    const auto &c = cfg;
    CW_CHECK_ARG(c.family.norm_unit_gain == 0 && c.family.act == 0 && c.family.qk_norm == 1 &&
                     c.family.qkv_bias == 0,
                 "%s: only the qwen3 family spec is built (plain norm, SwiGLU, "
                 "qk_norm, no qkv bias)", what);
    CW_CHECK_ARG(c.n_layers > 0 && c.dim > 0 && c.n_heads > 0 && c.n_kv_heads > 0 &&
                     c.hidden > 0 && c.vocab > 0 && c.max_seq > 0,
                 "%s: every dimension must be positive", what);
    CW_CHECK_ARG(c.max_seq <= 32768, "%s: max_seq=%d exceeds 32768", what, c.max_seq);
    CW_CHECK_ARG(c.n_heads % c.n_kv_heads == 0, "%s: n_heads %% n_kv_heads != 0", what);
    const int hpk = c.n_heads / c.n_kv_heads;
    CW_CHECK_ARG(hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8,
                 "%s: heads per kv head %d not in {1,2,4,8}", what, hpk);
    CW_CHECK_ARG(c.head_dim == 16 || c.head_dim == 32 || c.head_dim == 64 || c.head_dim == 128 ||
                     c.head_dim == 256,
                 "%s: head_dim=%d not in {16,32,64,128,256}", what, c.head_dim);
    const int q_dim = c.n_heads * c.head_dim;
    CW_CHECK_ARG(c.dim % 32 == 0 && c.hidden % 32 == 0 && q_dim % 32 == 0,
                 "%s: dim, hidden and n_heads*head_dim must be multiples of 32", what);
    CW_CHECK_ARG(c.dim <= 32768 && c.hidden <= 32768 && q_dim <= 32768,
                 "%s: GEMV input width above 32768", what);
    CW_CHECK_ARG(c.kv_dtype == CW_F32 || c.kv_dtype == CW_F16, "%s: kv_dtype=%d", what,
                 c.kv_dtype);
    return CW_OK;
}

// Every device buffer of the model (weights, cache, activations, decode
// state) for config c, in a fixed order; in a dry plan nothing touches a
// device.
int model_alloc(cw_model *m, const cw_model_config &c) {
    const int q_dim = c.n_heads * c.head_dim, kv_dim = c.n_kv_heads * c.head_dim;
    m->cfg = c;
    m->q_dim = q_dim;
    m->kv_dim = kv_dim;
    m->layers.resize(c.n_layers);
    m->have.assign(c.n_layers, std::vector<bool>(T_N, false));
    for (auto &L : m->layers) {
        CW_TRY(dalloc(m, c.dim * 4, (void **)&L.attn_norm));
        CW_TRY(dalloc(m, c.head_dim * 4, (void **)&L.q_norm));
        CW_TRY(dalloc(m, c.head_dim * 4, (void **)&L.k_norm));
        CW_TRY(dalloc(m, c.dim * 4, (void **)&L.ffn_norm));
        CW_TRY(alloc_q4(m, L.qkv, q_dim + 2 * kv_dim, c.dim));
        CW_TRY(alloc_q4(m, L.wo, c.dim, q_dim));
        if (m->dry_split_gu) {
            CW_TRY(alloc_q4(m, L.gate, c.hidden, c.dim));
            CW_TRY(alloc_q4(m, L.up, c.hidden, c.dim));
        } else {
            CW_TRY(alloc_q4(m, L.gu, 2 * c.hidden, c.dim));
            L.gate = q4_rows(L.gu, 0, c.hidden);
            L.up = q4_rows(L.gu, c.hidden, c.hidden);
        }
        CW_TRY(alloc_q4(m, L.down, c.dim, c.hidden));
    }
    const size_t es = c.kv_dtype == CW_F16 ? 2 : 4;
    m->kv_layer_bytes = (size_t)c.max_seq * kv_dim * es;
    const size_t part_floats = attn_scratch_floats(c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq);
    CW_TRY(dalloc(m, (size_t)c.vocab * c.dim * 4, (void **)&m->embed));
    CW_TRY(dalloc(m, c.dim * 4, (void **)&m->final_norm));
    CW_TRY(alloc_q4(m, m->lm_head, c.vocab, c.dim));
    CW_TRY(dalloc(m, m->kv_layer_bytes * c.n_layers, &m->kcache));
    CW_TRY(dalloc(m, m->kv_layer_bytes * c.n_layers, &m->vcache));
    CW_TRY(dalloc(m, c.dim * 4, (void **)&m->hidden));
    CW_TRY(dalloc(m, c.dim * 4, (void **)&m->hidden_out));
    CW_TRY(dalloc(m, (size_t)(q_dim + 2 * kv_dim) * 4, (void **)&m->qkv));
    CW_TRY(dalloc(m, (size_t)q_dim * 4, (void **)&m->attn));
    CW_TRY(dalloc(m, (size_t)c.hidden * 4, (void **)&m->act));
    CW_TRY(dalloc(m, (size_t)c.vocab * 4, (void **)&m->logits));
    CW_TRY(dalloc(m, part_floats * 4, (void **)&m->part));
    CW_TRY(dalloc(m, argmax_scratch_bytes(c.vocab), &m->argmax_scratch));
    CW_TRY(dalloc(m, m->dry ? (size_t)4 * m->dry_n_cu * 8 + 256 : lm_argmax_scratch_bytes(m->ctx),
                  &m->lm_scratch));
    CW_TRY(dalloc(m, sizeof(GenState), (void **)&m->state));
    CW_TRY(dalloc(m, (size_t)c.max_seq * 4, (void **)&m->prompt_dev));
    CW_TRY(dalloc(m, (size_t)c.max_seq * 4, (void **)&m->tokens_dev));
    CW_TRY(dalloc(m, 4, (void **)&m->argmax_out));
    // the RoPE table [max_pos][hd/2] (shared through the context); in a dry
    // plan, a table of the context's size for this max_seq
    int max_pos = 1024;
    while (max_pos < c.max_seq) max_pos *= 2;
    const size_t tab = (size_t)max_pos * (c.head_dim / 2) * 4;
    if (m->dry) {
        CW_TRY(dalloc(m, tab, (void **)&m->cos_t));
        CW_TRY(dalloc(m, tab, (void **)&m->sin_t));
    } else {
        const cw_rope_tab *t = nullptr;
        CW_TRY(ctx_rope_table(m->ctx, c.rope_theta, c.head_dim, c.max_seq, &t));
        m->cos_t = t->cos_t;
        m->sin_t = t->sin_t;
        const size_t n = (size_t)t->max_pos * (c.head_dim / 2) * 4;
        m->extents.push_back(Extent{t->cos_t, n});
        m->extents.push_back(Extent{t->sin_t, n});
    }
    return CW_OK;
}

}  // namespace

extern "C" {

int cw_model_create(cw_ctx *ctx, const cw_model_config *cfg, cw_model **out) {
    CW_CHECK_ARG(ctx && cfg && out, "cw_model_create: null argument");
    *out = nullptr;
    if (ctx->capturing) {
        set_error("cw_model_create: not allowed while a graph is being recorded (end it with "
                  "cw_graph_end)");
        return CW_ERR_STATE;
    }
    CW_TRY(check_config(*cfg, "cw_model_create"));
    const auto &c = *cfg;
    cw_model *m = new cw_model();
    m->ctx = ctx;
    int rc = model_alloc(m, c);
    if (rc != CW_OK) {
        cw_model_destroy(m);
        return rc;
    }
    // zero the caches so positions never written read as 0, not garbage
    // cleared on the context stream, so every later copy and launch is ordered after
    if (hipMemsetAsync(m->kcache, 0, m->kv_layer_bytes * c.n_layers, ctx->stream) != hipSuccess ||
        hipMemsetAsync(m->vcache, 0, m->kv_layer_bytes * c.n_layers, ctx->stream) != hipSuccess ||
        hipMemsetAsync(m->lm_scratch, 0, lm_argmax_scratch_bytes(ctx), ctx->stream) != hipSuccess) {
        set_error("cw_model_create: clearing the KV cache failed");
        cw_model_destroy(m);
        return CW_ERR_HIP;
    }
    *out = m;
    return CW_OK;
}

int cw_step_layout_check(const cw_model_config *cfg, int n_cu, int split_gate_up, char *why,
                         size_t why_len) {
    CW_CHECK_ARG(cfg && n_cu > 0, "cw_step_layout_check: bad argument");
    CW_TRY(check_config(*cfg, "cw_step_layout_check"));
    cw_model m;
    m.dry = true;
    m.dry_split_gu = split_gate_up != 0;
    m.dry_n_cu = n_cu;
    m.dry_next = (uintptr_t)1 << 44;
    CW_TRY(model_alloc(&m, *cfg));
    CW_TRY(setup_fused(&m));
    const char *msg = m.fused_unsupported ? m.fused_unsupported : "";
    if (why && why_len) snprintf(why, why_len, "%s", msg);
    if (m.fused_unsupported == m.fused_why) {
        set_error("cw_step_layout_check: %s", m.fused_why);
        return CW_ERR_STATE;
    }
    CW_CHECK_ARG(m.fused_unsupported == nullptr,
                 "cw_step_layout_check: the fused step does not cover this config: %s",
                 m.fused_unsupported);
    return CW_OK;
}

int cw_step_dry_plan(const cw_model_config *cfg, int n_cu, int split_gate_up, void *args_out,
                     size_t args_len, void *layers_out, size_t layers_len, void **ext_ptr,
                     size_t *ext_bytes, int max_ext, int *n_ext) {
    CW_CHECK_ARG(cfg && n_cu > 0 && args_out && layers_out && ext_ptr && ext_bytes && n_ext,
                 "cw_step_dry_plan: bad argument");
    CW_TRY(check_config(*cfg, "cw_step_dry_plan"));
    cw_model m;
    m.dry = true;
    m.dry_split_gu = split_gate_up != 0;
    m.dry_n_cu = n_cu;
    m.dry_next = (uintptr_t)1 << 44;
    CW_TRY(model_alloc(&m, *cfg));
    m.fused_unsupported = step_unsupported(cfg->head_dim, cfg->n_heads / cfg->n_kv_heads,
                                           cfg->n_kv_heads, cfg->dim, m.q_dim, cfg->hidden,
                                           cfg->max_seq);
    CW_CHECK_ARG(m.fused_unsupported == nullptr,
                 "cw_step_dry_plan: the fused step does not cover this config: %s",
                 m.fused_unsupported);
    std::vector<StepLayer> host;
    CW_TRY(build_step(&m, host));
    CW_CHECK_ARG(args_len >= sizeof(StepArgs), "cw_step_dry_plan: args_len %zu < %zu", args_len,
                 sizeof(StepArgs));
    CW_CHECK_ARG(layers_len >= host.size() * sizeof(StepLayer),
                 "cw_step_dry_plan: layers_len %zu < %zu", layers_len,
                 host.size() * sizeof(StepLayer));
    CW_CHECK_ARG((int)m.extents.size() <= max_ext, "cw_step_dry_plan: %zu allocations > %d",
                 m.extents.size(), max_ext);
    memcpy(args_out, &m.step, sizeof(StepArgs));
    memcpy(layers_out, host.data(), host.size() * sizeof(StepLayer));
    for (size_t i = 0; i < m.extents.size(); ++i) {
        ext_ptr[i] = const_cast<void *>(m.extents[i].p);
        ext_bytes[i] = m.extents[i].bytes;
    }
    *n_ext = (int)m.extents.size();
    return CW_OK;
}

int cw_model_destroy(cw_model *m) {
    if (!m) return CW_OK;
    CW_TRY(refuse_recording(m, "cw_model_destroy"));
    (void)hipStreamSynchronize(m->ctx->stream);
    if (m->graph_exec) (void)hipGraphExecDestroy(m->graph_exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    for (void *p : m->allocs) (void)hipFree(p);
    for (void *p : m->pf_allocs) (void)hipFree(p);
    delete m;
    return CW_OK;
}

int cw_model_set_q4(cw_model *m, const char *name, const uint16_t *scales, const uint8_t *quants) {
    CW_CHECK_ARG(m && name && scales && quants, "cw_model_set_q4: null argument");
    CW_TRY(refuse_recording(m, "cw_model_set_q4"));
    if (strcmp(name, "output.weight") == 0) {
        CW_TRY(upload_rows(m, m->lm_head, 0, m->cfg.vocab, scales, quants));
        m->have_output = true;
        return CW_OK;
    }
    int li = 0, id = 0;
    const int pr = parse_layer_name(name, m->cfg.n_layers, &li, &id);
    CW_CHECK_ARG(pr == 0 && id >= T_Q, "cw_model_set_q4: unknown projection \"%s\"", name);
    Layer &L = m->layers[li];
    int out_f = 0, in_f = 0;
    proj_shape(m, id, &out_f, &in_f);
    // NaN and infinite block scales are refused: the batched prefill
    // multiplies each block's f32 sum by d, where the per-token path forms
    // d (q - 8) per weight, and the two agree for every finite d only
    const size_t nblk = (size_t)out_f * (in_f / 32);
    for (size_t b = 0; b < nblk; ++b)
        CW_CHECK_ARG((scales[b] & 0x7C00u) != 0x7C00u,
                     "cw_model_set_q4: %s block %zu has scale bits 0x%04x (not finite)", name, b,
                     (unsigned)scales[b]);
    switch (id) {
        case T_Q: CW_TRY(upload_rows(m, L.qkv, 0, out_f, scales, quants)); break;
        case T_K: CW_TRY(upload_rows(m, L.qkv, m->q_dim, out_f, scales, quants)); break;
        case T_V: CW_TRY(upload_rows(m, L.qkv, m->q_dim + m->kv_dim, out_f, scales, quants)); break;
        case T_O: CW_TRY(upload_rows(m, L.wo, 0, out_f, scales, quants)); break;
        case T_GATE: CW_TRY(upload_rows(m, L.gate, 0, out_f, scales, quants)); break;
        case T_UP: CW_TRY(upload_rows(m, L.up, 0, out_f, scales, quants)); break;
        default: CW_TRY(upload_rows(m, L.down, 0, out_f, scales, quants)); break;
    }
    m->have[li][id] = true;
    return CW_OK;
}

int cw_model_set_f32(cw_model *m, const char *name, const float *data) {
    CW_CHECK_ARG(m && name && data, "cw_model_set_f32: null argument");
    CW_TRY(refuse_recording(m, "cw_model_set_f32"));
    const auto &c = m->cfg;
    if (strcmp(name, "token_embd.weight") == 0) {
        CW_TRY(cw_upload(m->ctx, m->embed, data, (size_t)c.vocab * c.dim * 4));
        m->have_embed = true;
        return CW_OK;
    }
    if (strcmp(name, "output_norm.weight") == 0) {
        CW_TRY(cw_upload(m->ctx, m->final_norm, data, (size_t)c.dim * 4));
        m->have_final = true;
        return CW_OK;
    }
    int li = 0, id = 0;
    const int pr = parse_layer_name(name, c.n_layers, &li, &id);
    CW_CHECK_ARG(pr == 0 && id < T_Q, "cw_model_set_f32: unknown vector \"%s\"", name);
    Layer &L = m->layers[li];
    float *dst = id == T_ATTN_NORM ? L.attn_norm
                 : id == T_Q_NORM  ? L.q_norm
                 : id == T_K_NORM  ? L.k_norm
                                   : L.ffn_norm;
    const size_t n = (id == T_Q_NORM || id == T_K_NORM) ? c.head_dim : c.dim;
    CW_TRY(cw_upload(m->ctx, dst, data, n * 4));
    m->have[li][id] = true;
    return CW_OK;
}

int cw_model_load_synthetic(cw_model *m, uint64_t seed) {
    CW_CHECK_ARG(m != nullptr, "cw_model_load_synthetic: null model");
    CW_TRY(refuse_recording(m, "cw_model_load_synthetic"));
    const auto &c = m->cfg;
    std::vector<uint16_t> s;
    std::vector<uint8_t> q;
    std::vector<float> f;
    char name[96];
    for (int i = 0; i < c.n_layers; ++i) {
        for (int id = 0; id < T_N; ++id) {
            snprintf(name, sizeof name, "blk.%d.%s.weight", i, kLayerNames[id]);
            const uint64_t key = cw_synth_key(seed, name);
            if (id < T_Q) {
                const size_t n = (id == T_Q_NORM || id == T_K_NORM) ? c.head_dim : c.dim;
                f.resize(n);
                CW_TRY(cw_synth_normal_f32(key, n, 1.0f, 0.02f, f.data()));
                CW_TRY(cw_model_set_f32(m, name, f.data()));
            } else {
                int out_f = 0, in_f = 0;
                proj_shape(m, id, &out_f, &in_f);
                const size_t nblk = (size_t)out_f * (in_f / 32);
                s.resize(nblk);
                q.resize(nblk * 16);
                CW_TRY(cw_synth_q4(key, nblk, 0.02f, s.data(), q.data()));
                CW_TRY(cw_model_set_q4(m, name, s.data(), q.data()));
            }
        }
    }
    f.resize(c.dim);
    CW_TRY(cw_synth_normal_f32(cw_synth_key(seed, "output_norm.weight"), c.dim, 1.0f, 0.02f,
                               f.data()));
    CW_TRY(cw_model_set_f32(m, "output_norm.weight", f.data()));
    f.resize((size_t)c.vocab * c.dim);
    CW_TRY(cw_synth_normal_f32(cw_synth_key(seed, "token_embd.weight"), f.size(), 0.0f, 0.02f,
                               f.data()));
    CW_TRY(cw_model_set_f32(m, "token_embd.weight", f.data()));
    return CW_OK;
}

int cw_model_load_gguf(cw_model *m, const cw_gguf *g) {
    CW_CHECK_ARG(m && g, "cw_model_load_gguf: null argument");
    CW_TRY(refuse_recording(m, "cw_model_load_gguf"));
    const auto &c = m->cfg;
    std::vector<uint16_t> s;
    std::vector<uint8_t> q;
    std::vector<float> f;
    char name[96];
    for (int i = 0; i < c.n_layers; ++i) {
        for (int id = 0; id < T_N; ++id) {
            snprintf(name, sizeof name, "blk.%d.%s.weight", i, kLayerNames[id]);
            if (id < T_Q) {
                f.resize((id == T_Q_NORM || id == T_K_NORM) ? c.head_dim : c.dim);
                CW_TRY(cw_gguf_tensor_f32(g, name, f.data(), f.size()));
                CW_TRY(cw_model_set_f32(m, name, f.data()));
            } else {
                int out_f = 0, in_f = 0;
                proj_shape(m, id, &out_f, &in_f);
                const size_t nblk = (size_t)out_f * (in_f / 32);
                s.resize(nblk);
                q.resize(nblk * 16);
                CW_TRY(cw_gguf_tensor_q4(g, name, out_f, in_f, s.data(), q.data()));
                CW_TRY(cw_model_set_q4(m, name, s.data(), q.data()));
            }
        }
    }
    f.resize(c.dim);
    CW_TRY(cw_gguf_tensor_f32(g, "output_norm.weight", f.data(), f.size()));
    CW_TRY(cw_model_set_f32(m, "output_norm.weight", f.data()));
    f.resize((size_t)c.vocab * c.dim);
    CW_TRY(cw_gguf_tensor_f32(g, "token_embd.weight", f.data(), f.size()));
    CW_TRY(cw_model_set_f32(m, "token_embd.weight", f.data()));
    if (cw_gguf_has(g, "output.weight")) {
        const size_t nblk = (size_t)c.vocab * (c.dim / 32);
        s.resize(nblk);
        q.resize(nblk * 16);
        CW_TRY(cw_gguf_tensor_q4(g, "output.weight", c.vocab, c.dim, s.data(), q.data()));
        CW_TRY(cw_model_set_q4(m, "output.weight", s.data(), q.data()));
    }
    return CW_OK;
}

int cw_model_finalize(cw_model *m) {
    CW_CHECK_ARG(m != nullptr, "cw_model_finalize: null model");
    CW_TRY(refuse_recording(m, "cw_model_finalize"));
    const auto &c = m->cfg;
    for (int i = 0; i < c.n_layers; ++i)
        for (int id = 0; id < T_N; ++id)
            if (!m->have[i][id]) {
                set_error("missing tensor blk.%d.%s.weight", i, kLayerNames[id]);
                return CW_ERR_STATE;
            }
    if (!m->have_embed) {
        set_error("missing tensor token_embd.weight");
        return CW_ERR_STATE;
    }
    if (!m->have_final) {
        set_error("missing tensor output_norm.weight");
        return CW_ERR_STATE;
    }
    if (!m->have_output) {
        // tied LM head (qwen3.rs:93-98): re-quantize the f32 embedding
        std::vector<float> e((size_t)c.vocab * c.dim);
        CW_TRY(cw_download(m->ctx, e.data(), m->embed, e.size() * 4));
        const size_t nblk = (size_t)c.vocab * (c.dim / 32);
        std::vector<uint16_t> s(nblk);
        std::vector<uint8_t> q(nblk * 16);
        CW_TRY(cw_q4_quantize(e.data(), c.vocab, c.dim, s.data(), q.data()));
        CW_TRY(upload_rows(m, m->lm_head, 0, c.vocab, s.data(), q.data()));
    }
    if (!m->step_layers) CW_TRY(setup_fused(m));
    m->finalized = true;
    return CW_OK;
}

int cw_model_prefill_kv(cw_model *m, const void *k, const void *v, int n_pos) {
    CW_CHECK_ARG(m && k && v, "cw_model_prefill_kv: null argument");
    CW_TRY(refuse_recording(m, "cw_model_prefill_kv"));
    CW_CHECK_ARG(n_pos > 0 && n_pos <= m->cfg.max_seq, "cw_model_prefill_kv: n_pos=%d (max_seq %d)",
                 n_pos, m->cfg.max_seq);
    const size_t es = m->cfg.kv_dtype == CW_F16 ? 2 : 4;
    const size_t row = (size_t)n_pos * m->kv_dim * es;
    for (int l = 0; l < m->cfg.n_layers; ++l) {
        CW_TRY(cw_upload(m->ctx, (char *)m->kcache + l * m->kv_layer_bytes,
                         (const char *)k + l * row, row));
        CW_TRY(cw_upload(m->ctx, (char *)m->vcache + l * m->kv_layer_bytes,
                         (const char *)v + l * row, row));
    }
    return CW_OK;
}

int cw_model_step(cw_model *m, uint32_t token, int pos, uint32_t *argmax_out) {
    CW_CHECK_ARG(m != nullptr, "cw_model_step: null model");
    CW_TRY(refuse_recording(m, "cw_model_step"));
    CW_TRY(require_final(m, "cw_model_step"));
    CW_CHECK_ARG(token < (uint32_t)m->cfg.vocab, "cw_model_step: token %u >= vocab %d", token,
                 m->cfg.vocab);
    CW_CHECK_ARG(pos >= 0 && pos < m->cfg.max_seq, "cw_model_step: pos=%d outside [0, %d)", pos,
                 m->cfg.max_seq);
    GenState s{pos, token, pos, 0, 0, 0};
    CW_TRY(set_state(m, s));
    CW_TRY(enqueue_step(m));
    m->host_pos = pos + 1;
    CW_TRY(launch_rmsnorm(m->ctx, last_hidden(m), m->final_norm, 1, m->cfg.dim, m->cfg.eps,
                          m->hidden_out));
    uint32_t r = 0;
    CW_HIP(hipMemcpyAsync(&r, m->argmax_out, 4, hipMemcpyDeviceToHost, m->ctx->stream));
    CW_HIP(hipStreamSynchronize(m->ctx->stream));
    if (argmax_out) *argmax_out = r;
    return CW_OK;
}

int cw_model_logits(cw_model *m, float *host_out) {
    CW_CHECK_ARG(m && host_out, "cw_model_logits: null argument");
    return cw_download(m->ctx, host_out, m->logits, (size_t)m->cfg.vocab * 4);
}

int cw_model_hidden(cw_model *m, float *host_out) {
    CW_CHECK_ARG(m && host_out, "cw_model_hidden: null argument");
    return cw_download(m->ctx, host_out, m->hidden_out, (size_t)m->cfg.dim * 4);
}

int cw_model_set_taps(cw_model *m, int enable) {
    CW_CHECK_ARG(m != nullptr, "cw_model_set_taps: null model");
    CW_TRY(refuse_recording(m, "cw_model_set_taps"));
    const auto &c = m->cfg;
    if (enable) {
        // each buffer is made (and cleared) once; a failed allocation leaves
        // the taps off and the next call retries the missing ones
        float **bufs[3] = {&m->tap_q, &m->tap_post, &m->tap_out};
        const size_t floats[3] = {(size_t)c.n_layers * m->q_dim, (size_t)c.n_layers * c.dim,
                                  (size_t)c.n_layers * c.dim};
        for (int i = 0; i < 3; ++i) {
            if (*bufs[i]) continue;
            void *p = nullptr;
            CW_TRY(dalloc(m, floats[i] * 4, &p));
            CW_HIP(hipMemsetAsync(p, 0, floats[i] * 4, m->ctx->stream));
            *bufs[i] = static_cast<float *>(p);
        }
    }
    if ((enable != 0) != m->taps) {
        // the captured step holds the other buffer addresses: capture again
        CW_HIP(hipStreamSynchronize(m->ctx->stream));
        if (m->graph_exec) CW_HIP(hipGraphExecDestroy(m->graph_exec));
        if (m->graph) CW_HIP(hipGraphDestroy(m->graph));
        m->graph_exec = nullptr;
        m->graph = nullptr;
        m->taps = enable != 0;
    }
    return CW_OK;
}

int cw_model_tap(cw_model *m, const char *name, int layer, float *host_out, int len) {
    CW_CHECK_ARG(m && name && host_out, "cw_model_tap: null argument");
    const auto &c = m->cfg;
    if (!m->taps) {
        set_error("cw_model_tap: taps are off (cw_model_set_taps)");
        return CW_ERR_STATE;
    }
    CW_CHECK_ARG(layer >= 0 && layer < c.n_layers, "cw_model_tap: layer %d outside [0, %d)",
                 layer, c.n_layers);
    const float *src = nullptr;
    int n = 0;
    if (!strcmp(name, "q")) {
        src = m->tap_q + (size_t)layer * m->q_dim;
        n = m->q_dim;
    } else if (!strcmp(name, "post_attn")) {
        src = m->tap_post + (size_t)layer * c.dim;
        n = c.dim;
    } else if (!strcmp(name, "layer_out")) {
        src = m->tap_out + (size_t)layer * c.dim;
        n = c.dim;
    } else {
        set_error("cw_model_tap: unknown tap '%s' (q, post_attn, layer_out)", name);
        return CW_ERR_ARG;
    }
    CW_CHECK_ARG(len == n, "cw_model_tap: tap '%s' holds %d floats, len=%d", name, n, len);
    return cw_download(m->ctx, host_out, src, (size_t)n * 4);
}

int cw_generate(cw_model *m, const uint32_t *prompt, int n_prompt, int max_new, int start_pos,
                int mode, uint32_t *out_tokens) {
    CW_CHECK_ARG(m && prompt && out_tokens, "cw_generate: null argument");
    CW_TRY(refuse_recording(m, "cw_generate"));
    CW_TRY(require_final(m, "cw_generate"));
    CW_CHECK_ARG(n_prompt >= 1 && max_new >= 1, "cw_generate: n_prompt=%d max_new=%d", n_prompt,
                 max_new);
    const long total = (long)n_prompt + max_new - 1;
    CW_CHECK_ARG(start_pos >= 0 && start_pos + total <= m->cfg.max_seq,
                 "cw_generate: positions [%d, %ld) exceed max_seq %d", start_pos,
                 start_pos + total, m->cfg.max_seq);
    for (int i = 0; i < n_prompt; ++i)
        CW_CHECK_ARG(prompt[i] < (uint32_t)m->cfg.vocab, "cw_generate: prompt[%d]=%u >= vocab", i,
                     prompt[i]);
    CW_TRY(cw_upload(m->ctx, m->prompt_dev, prompt, (size_t)n_prompt * 4));
    GenState s{start_pos, prompt[0], start_pos, n_prompt, 0, max_new};
    CW_TRY(set_state(m, s));
    CW_TRY(run_steps(m, (int)total, mode));
    CW_HIP(hipMemcpyAsync(out_tokens, m->tokens_dev, (size_t)max_new * 4, hipMemcpyDeviceToHost,
                          m->ctx->stream));
    CW_HIP(hipStreamSynchronize(m->ctx->stream));
    return check_fused(m);
}

int cw_model_prefill(cw_model *m, const uint32_t *tokens, int n, int start_pos,
                     uint32_t *next_token) {
    CW_CHECK_ARG(m && tokens, "cw_model_prefill: null argument");
    CW_TRY(refuse_recording(m, "cw_model_prefill"));
    CW_TRY(require_final(m, "cw_model_prefill"));
    const auto &c = m->cfg;
    CW_CHECK_ARG(n >= 1 && start_pos >= 0 && (long)start_pos + n <= c.max_seq,
                 "cw_model_prefill: positions [%d, %ld) outside max_seq %d", start_pos,
                 (long)start_pos + n, c.max_seq);
    for (int i = 0; i < n; ++i)
        CW_CHECK_ARG(tokens[i] < (uint32_t)c.vocab, "cw_model_prefill: tokens[%d]=%u >= vocab", i,
                     tokens[i]);
    CW_TRY(cw_upload(m->ctx, m->prompt_dev, tokens, (size_t)n * 4));
    const bool batched = c.kv_dtype == CW_F16 && c.head_dim == 128;
    if (batched) {
        CW_TRY(ensure_prefill(m, n));
        CW_TRY(enqueue_prefill(m, n, start_pos));
        // the last position's logits (the prompt phase discards the others,
        // mod.rs:93-103) and the final-normed hidden state
        const float *last = m->pf_hidden + (size_t)(n - 1) * c.dim;
        GemvArgs g{};
        g.x = last;
        g.norm_w = m->final_norm;
        g.eps = c.eps;
        g.sA = m->lm_head.s;
        g.qA = m->lm_head.q;
        g.y = m->logits;
        g.K = c.dim;
        g.N = c.vocab;
        CW_TRY(launch_lm_head_argmax(m->ctx, g, m->lm_scratch, m->argmax_out, nullptr, nullptr,
                                     nullptr));
        CW_TRY(launch_rmsnorm(m->ctx, last, m->final_norm, 1, c.dim, c.eps, m->hidden_out));
    } else {
        // head_dim other than 128 or an f32 cache: the per-token step, n times
        GenState s{start_pos, tokens[0], start_pos, n, 0, 0};
        CW_TRY(set_state(m, s));
        CW_TRY(run_steps(m, n, CW_STEP_EAGER));
        CW_TRY(launch_rmsnorm(m->ctx, last_hidden(m), m->final_norm, 1, c.dim, c.eps,
                              m->hidden_out));
    }
    uint32_t r = 0;
    CW_HIP(hipMemcpyAsync(&r, m->argmax_out, 4, hipMemcpyDeviceToHost, m->ctx->stream));
    CW_HIP(hipStreamSynchronize(m->ctx->stream));
    if (next_token) *next_token = r;
    // decoding continues at start_pos + n with the predicted token
    GenState s{start_pos + n, r, start_pos + n, 1, 0, c.max_seq};
    return set_state(m, s);
}

int cw_model_reset_state(cw_model *m, uint32_t token, int pos) {
    CW_CHECK_ARG(m != nullptr, "cw_model_reset_state: null model");
    CW_TRY(refuse_recording(m, "cw_model_reset_state"));
    CW_CHECK_ARG(token < (uint32_t)m->cfg.vocab && pos >= 0 && pos < m->cfg.max_seq,
                 "cw_model_reset_state: token=%u pos=%d", token, pos);
    GenState s{pos, token, pos, 1, 0, m->cfg.max_seq};
    return set_state(m, s);
}

int cw_model_decode_async(cw_model *m, int n_steps, int mode) {
    CW_CHECK_ARG(m != nullptr && n_steps >= 0, "cw_model_decode_async: bad argument");
    CW_TRY(refuse_recording(m, "cw_model_decode_async"));
    CW_TRY(require_final(m, "cw_model_decode_async"));
    CW_CHECK_ARG(m->host_pos + n_steps <= m->cfg.max_seq,
                 "cw_model_decode_async: %d steps from pos %d exceed max_seq %d", n_steps,
                 m->host_pos, m->cfg.max_seq);
    return run_steps(m, n_steps, mode);
}

int cw_model_decode_next(cw_model *m, uint32_t *next_out) {
    CW_CHECK_ARG(m && next_out, "cw_model_decode_next: null argument");
    CW_TRY(refuse_recording(m, "cw_model_decode_next"));
    CW_TRY(require_final(m, "cw_model_decode_next"));
    CW_CHECK_ARG(m->host_pos < m->cfg.max_seq, "cw_model_decode_next: pos %d at max_seq %d",
                 m->host_pos, m->cfg.max_seq);
    CW_TRY(run_steps(m, 1, CW_STEP_GRAPH));
    // the step's LM head leaves its argmax here: one 4-byte read per token
    uint32_t r = 0;
    CW_HIP(hipMemcpyAsync(&r, m->argmax_out, 4, hipMemcpyDeviceToHost, m->ctx->stream));
    CW_HIP(hipStreamSynchronize(m->ctx->stream));
    *next_out = r;
    return CW_OK;
}

int cw_model_profile_step(cw_model *m, int64_t *ticks, int max_n, int *n_out, double *tick_hz) {
    CW_CHECK_ARG(m && ticks && n_out && tick_hz, "cw_model_profile_step: null argument");
    CW_TRY(refuse_recording(m, "cw_model_profile_step"));
    CW_TRY(require_final(m, "cw_model_profile_step"));
    if (kFusedStepDisabled) {
        set_error("fused decode step disabled (see CW_STEP_FUSED)");
        return CW_ERR_STATE;
    }
    if (m->fused_unsupported) {
        set_error("fused decode step unavailable for this model: %s", m->fused_unsupported);
        return CW_ERR_ARG;
    }
    GenState s{};
    CW_HIP(hipMemcpyAsync(&s, m->state, sizeof s, hipMemcpyDeviceToHost, m->ctx->stream));
    CW_HIP(hipStreamSynchronize(m->ctx->stream));
    CW_CHECK_ARG(s.pos < m->cfg.max_seq, "cw_model_profile_step: pos %d at max_seq", s.pos);
    const int n = (int)step_trace_words(m->cfg.n_layers);  // stamps written by one launch
    long long *dev = nullptr;
    StepArgs *args_dev = nullptr;
    CW_HIP(hipMalloc(&dev, (size_t)n * 8 + sizeof(StepArgs)));
    args_dev = reinterpret_cast<StepArgs *>(dev + n);
    StepArgs a = m->step;
    a.trace = dev;
    hipError_t e = hipMemsetAsync(dev, 0, (size_t)n * 8, m->ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(args_dev, &a, sizeof a, hipMemcpyHostToDevice, m->ctx->stream);
    const auto &c = m->cfg;
    int rc = e == hipSuccess ? CW_OK : hip_fail(e, "trace setup", __FILE__, __LINE__);
    if (rc == CW_OK)
        rc = launch_decode_step(m->ctx, args_dev, c.kv_dtype, c.n_heads / c.n_kv_heads, c.max_seq);
    std::vector<long long> host(n);
    if (rc == CW_OK) {
        e = hipMemcpyAsync(host.data(), dev, (size_t)n * 8, hipMemcpyDeviceToHost, m->ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(m->ctx->stream);
        if (e != hipSuccess) rc = hip_fail(e, "trace download", __FILE__, __LINE__);
    }
    (void)hipFree(dev);
    CW_TRY(rc);
    CW_TRY(check_fused(m));
    const int k = n < max_n ? n : max_n;
    for (int i = 0; i < k; ++i) ticks[i] = host[i];
    *n_out = k;
    int rate_khz = 0;
    CW_HIP(hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, m->ctx->device));
    *tick_hz = (double)rate_khz * 1000.0;
    return CW_OK;
}

int cw_model_tokens(cw_model *m, uint32_t *host_out, int max_n, int *n_out) {
    CW_CHECK_ARG(m && host_out && n_out, "cw_model_tokens: null argument");
    CW_TRY(refuse_recording(m, "cw_model_tokens"));
    CW_TRY(check_fused(m));
    GenState s{};
    CW_HIP(hipMemcpyAsync(&s, m->state, sizeof s, hipMemcpyDeviceToHost, m->ctx->stream));
    CW_HIP(hipStreamSynchronize(m->ctx->stream));
    int n = s.produced < s.max_out ? s.produced : s.max_out;
    if (n > max_n) n = max_n;
    if (n > 0) CW_TRY(cw_download(m->ctx, host_out, m->tokens_dev, (size_t)n * 4));
    *n_out = n;
    return CW_OK;
}

}  // extern "C"
