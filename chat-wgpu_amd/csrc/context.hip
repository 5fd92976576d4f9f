// Context, memory, errors and profiling: the HIP counterpart of the
// reference's GpuContext (src/context.rs) and Profiler (src/profile.rs).
// One stream per context; a deterministic per-frame arena; events for the
// per-kernel profile.

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>

#include "cw_internal.hpp"

namespace {
thread_local std::string g_last_error;
}

namespace cwi {

void set_error(const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

int hip_fail(hipError_t e, const char *what, const char *file, int line) {
    set_error("HIP error %d (%s) in %s at %s:%d", (int)e, hipGetErrorString(e), what, file, line);
    if (e == hipErrorOutOfMemory) return CW_ERR_OOM;
    return CW_ERR_HIP;
}

int launch_check(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("launch of %s failed: %s", what, hipGetErrorString(e));
        return CW_ERR_HIP;
    }
    return CW_OK;
}

uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {  // subnormal: normalise
            int sh = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                ++sh;
            }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 + 1 - sh) << 23) | (m << 13);
        }
    } else if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0u);
    } else {
        bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// What would allocate or synchronise cannot run while a graph is being
// recorded: the first use at a size must come before cw_graph_begin.
static int refuse_while_capturing(const cw_ctx *ctx, const char *what) {
    if (!ctx->capturing) return CW_OK;
    set_error("%s while a graph is being recorded: run the sequence once before cw_graph_begin",
              what);
    return CW_ERR_STATE;
}

int ctx_scratch(cw_ctx *ctx, size_t bytes, void **out) {
    if (bytes > ctx->scratch_size) {
        CW_TRY(refuse_while_capturing(ctx, "kernel scratch must grow"));
        // geometric growth: a caller whose size creeps up (attention over a
        // growing sequence) reallocates O(log n) times, not every few steps
        size_t sz = std::max(bytes, std::max((size_t)1 << 20, 2 * ctx->scratch_size));
        void *p = nullptr;
        CW_HIP(hipMalloc(&p, sz));
        if (ctx->scratch) {
            if (ctx->scratch_recorded) {
                // a launch sequence recorded earlier (cw_graph_*) may name the
                // old buffer; replaying it must not write freed memory, so it
                // is retired, not freed, until the context is destroyed
                ctx->scratch_retired.push_back(ctx->scratch);
            } else {
                // only queued launches use it: free it once they are done
                hipError_t e = hipStreamSynchronize(ctx->stream);
                if (e == hipSuccess) e = hipFree(ctx->scratch);
                if (e != hipSuccess) {
                    (void)hipFree(p);
                    return hip_fail(e, "ctx_scratch: releasing the old scratch", __FILE__, __LINE__);
                }
            }
        }
        ctx->scratch = p;
        ctx->scratch_recorded = false;
        // counters inside scratch must start at zero (cleared in stream order)
        CW_HIP(hipMemsetAsync(ctx->scratch, 0, sz, ctx->stream));
        ctx->scratch_size = sz;
    }
    *out = ctx->scratch;
    return CW_OK;
}

void rope_table_host(int max_pos, int head_dim, float theta, float *cos_t, float *sin_t) {
    int half = head_dim / 2;
    for (int p = 0; p < max_pos; ++p) {
        for (int i = 0; i < half; ++i) {
            double inv = std::pow((double)theta, -2.0 * (double)i / (double)head_dim);
            double f = (double)p * inv;
            cos_t[(size_t)p * half + i] = (float)std::cos(f);
            sin_t[(size_t)p * half + i] = (float)std::sin(f);
        }
    }
}

int ctx_rope_table(cw_ctx *ctx, float theta, int head_dim, int min_pos, const cw_rope_tab **out) {
    for (auto &t : ctx->ropes) {
        if (t.theta == theta && t.head_dim == head_dim && t.max_pos >= min_pos) {
            *out = &t;
            return CW_OK;
        }
    }
    CW_TRY(refuse_while_capturing(ctx, "a RoPE table must be built"));
    int max_pos = 1024;
    while (max_pos < min_pos) max_pos *= 2;
    size_t n = (size_t)max_pos * (head_dim / 2);
    std::vector<float> c(n), s(n);
    rope_table_host(max_pos, head_dim, theta, c.data(), s.data());
    cw_rope_tab t{theta, head_dim, max_pos, nullptr, nullptr};
    CW_HIP(hipMalloc(&t.cos_t, n * sizeof(float)));
    CW_HIP(hipMalloc(&t.sin_t, n * sizeof(float)));
    CW_HIP(hipMemcpy(t.cos_t, c.data(), n * sizeof(float), hipMemcpyHostToDevice));
    CW_HIP(hipMemcpy(t.sin_t, s.data(), n * sizeof(float), hipMemcpyHostToDevice));
    // an older, shorter table for the same key may still be referenced by
    // queued work: keep it alive until the context is destroyed
    ctx->ropes.push_back(t);
    *out = &ctx->ropes.back();
    return CW_OK;
}

static hipEvent_t next_event(cw_ctx *ctx) {
    if (ctx->event_next == ctx->event_pool.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        ctx->event_pool.push_back(e);
    }
    return ctx->event_pool[ctx->event_next++];
}

void prof_begin(cw_ctx *ctx, const char *label) {
    if (!ctx->profiling) return;
    cw_prof_rec r{next_event(ctx), nullptr, label};
    if (r.start) (void)hipEventRecord(r.start, ctx->stream);
    ctx->prof.push_back(r);
}

void prof_end(cw_ctx *ctx) {
    if (!ctx->profiling || ctx->prof.empty()) return;
    cw_prof_rec &r = ctx->prof.back();
    r.stop = next_event(ctx);
    if (r.stop) (void)hipEventRecord(r.stop, ctx->stream);
}

void prof_events(cw_ctx *ctx, const char *label, hipEvent_t *start, hipEvent_t *stop) {
    cw_prof_rec r{next_event(ctx), next_event(ctx), label};
    ctx->prof.push_back(r);
    *start = r.start;
    *stop = r.stop;
}

}  // namespace cwi

using namespace cwi;

extern "C" {

const char *cw_last_error(void) { return g_last_error.c_str(); }

const char *cw_version(void) { return "chat-wgpu-amd 0.1 (gfx950)"; }

int cw_ctx_create(int device, cw_ctx **out) {
    CW_CHECK_ARG(out != nullptr, "cw_ctx_create: out is null");
    *out = nullptr;
    int n = 0;
    CW_HIP(hipGetDeviceCount(&n));
    CW_CHECK_ARG(device >= 0 && device < n, "cw_ctx_create: device %d of %d", device, n);
    CW_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    CW_HIP(hipGetDeviceProperties(&prop, device));
    cw_ctx *ctx = new cw_ctx();
    ctx->device = device;
    ctx->n_cu = prop.multiProcessorCount;
    ctx->hbm_bytes = prop.totalGlobalMem;
    ctx->arch = prop.gcnArchName;
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return hip_fail(e, "hipStreamCreateWithFlags", __FILE__, __LINE__);
    }
    const size_t cnt_bytes = (size_t)cwi::kMaxAttnKv * 128;
    e = hipMalloc(&ctx->attn_cnt, cnt_bytes);
    if (e == hipSuccess) e = hipMemsetAsync(ctx->attn_cnt, 0, cnt_bytes, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        if (ctx->attn_cnt) (void)hipFree(ctx->attn_cnt);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_fail(e, "attention counters", __FILE__, __LINE__);
    }
    const int rc = cwi::attn_noalloc_setup(ctx);
    if (rc != CW_OK) {
        cw_ctx_destroy(ctx);
        return rc;
    }
    *out = ctx;
    return CW_OK;
}

int cw_ctx_destroy(cw_ctx *ctx) {
    if (!ctx) return CW_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (void *p : ctx->allocs) (void)hipFree(p);
    for (auto &c : ctx->chunks) (void)hipFree(c.base);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    for (void *p : ctx->scratch_retired) (void)hipFree(p);
    if (ctx->attn_cnt) (void)hipFree(ctx->attn_cnt);
    for (auto &t : ctx->ropes) {
        (void)hipFree(t.cos_t);
        (void)hipFree(t.sin_t);
    }
    for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return CW_OK;
}

int cw_device_info(cw_ctx *ctx, int *n_cu, size_t *hbm_bytes, char *arch, size_t arch_len) {
    CW_CHECK_ARG(ctx != nullptr, "cw_device_info: null ctx");
    if (n_cu) *n_cu = ctx->n_cu;
    if (hbm_bytes) *hbm_bytes = ctx->hbm_bytes;
    if (arch && arch_len) {
        snprintf(arch, arch_len, "%s", ctx->arch.c_str());
    }
    return CW_OK;
}

int cw_alloc(cw_ctx *ctx, size_t bytes, void **out) {
    CW_CHECK_ARG(ctx && out, "cw_alloc: null argument");
    CW_CHECK_ARG(bytes > 0, "cw_alloc: zero-length request");
    void *p = nullptr;
    CW_HIP(hipMalloc(&p, bytes));
    ctx->allocs.push_back(p);
    *out = p;
    return CW_OK;
}

int cw_free(cw_ctx *ctx, void *ptr) {
    CW_CHECK_ARG(ctx != nullptr, "cw_free: null ctx");
    if (!ptr) return CW_OK;
    for (size_t i = 0; i < ctx->allocs.size(); ++i) {
        if (ctx->allocs[i] == ptr) {
            CW_HIP(hipStreamSynchronize(ctx->stream));
            CW_HIP(hipFree(ptr));
            ctx->allocs.erase(ctx->allocs.begin() + (long)i);
            return CW_OK;
        }
    }
    set_error("cw_free: %p was not allocated by this context", ptr);
    return CW_ERR_ARG;
}

int cw_frame_alloc(cw_ctx *ctx, size_t bytes, void **out) {
    CW_CHECK_ARG(ctx && out, "cw_frame_alloc: null argument");
    CW_CHECK_ARG(bytes > 0, "cw_frame_alloc: zero-length request");
    size_t need = (bytes + 255) & ~(size_t)255;
    while (ctx->chunk_idx < ctx->chunks.size()) {
        auto &c = ctx->chunks[ctx->chunk_idx];
        if (ctx->chunk_off + need <= c.size) {
            *out = c.base + ctx->chunk_off;
            ctx->chunk_off += need;
            return CW_OK;
        }
        ctx->chunk_idx++;
        ctx->chunk_off = 0;
    }
    CW_TRY(refuse_while_capturing(ctx, "the frame arena must grow"));
    size_t sz = need < (64u << 20) ? (64u << 20) : need;
    cw_ctx::Chunk c{nullptr, sz};
    CW_HIP(hipMalloc((void **)&c.base, sz));
    ctx->chunks.push_back(c);
    ctx->chunk_idx = ctx->chunks.size() - 1;
    ctx->chunk_off = need;
    *out = c.base;
    return CW_OK;
}

int cw_frame_reset(cw_ctx *ctx) {
    CW_CHECK_ARG(ctx != nullptr, "cw_frame_reset: null ctx");
    ctx->chunk_idx = 0;
    ctx->chunk_off = 0;
    return CW_OK;
}

int cw_upload(cw_ctx *ctx, void *dst, const void *src, size_t bytes) {
    CW_CHECK_ARG(ctx && dst && src, "cw_upload: null argument");
    CW_TRY(refuse_while_capturing(ctx, "cw_upload"));
    if (!bytes) return CW_OK;
    CW_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    // the source is pageable host memory owned by the caller: finish before
    // returning so the caller may reuse it
    CW_HIP(hipStreamSynchronize(ctx->stream));
    return CW_OK;
}

int cw_download(cw_ctx *ctx, void *dst, const void *src, size_t bytes) {
    CW_CHECK_ARG(ctx && dst && src, "cw_download: null argument");
    CW_TRY(refuse_while_capturing(ctx, "cw_download"));
    if (!bytes) return CW_OK;
    CW_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    CW_HIP(hipStreamSynchronize(ctx->stream));
    return CW_OK;
}

int cw_copy(cw_ctx *ctx, void *dst, const void *src, size_t bytes) {
    CW_CHECK_ARG(ctx && dst && src, "cw_copy: null argument");
    if (!bytes) return CW_OK;
    CW_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return CW_OK;
}

int cw_flush(cw_ctx *ctx) {
    CW_CHECK_ARG(ctx != nullptr, "cw_flush: null ctx");
    CW_TRY(refuse_while_capturing(ctx, "cw_flush"));
    CW_HIP(hipStreamSynchronize(ctx->stream));
    return CW_OK;
}

int cw_profile_begin(cw_ctx *ctx) {
    CW_CHECK_ARG(ctx != nullptr, "cw_profile_begin: null ctx");
    CW_TRY(refuse_while_capturing(ctx, "cw_profile_begin"));
    ctx->profiling = true;
    ctx->prof.clear();
    ctx->event_next = 0;
    return CW_OK;
}

int cw_profile_report(cw_ctx *ctx, char *buf, size_t buf_len) {
    CW_CHECK_ARG(ctx && buf && buf_len, "cw_profile_report: null argument");
    CW_HIP(hipStreamSynchronize(ctx->stream));
    struct Agg {
        int count = 0;
        double ms = 0.0;
    };
    std::map<std::string, Agg> agg;
    std::vector<std::string> order;
    for (auto &r : ctx->prof) {
        if (!r.start || !r.stop) continue;
        float ms = 0.f;
        CW_HIP(hipEventElapsedTime(&ms, r.start, r.stop));
        auto it = agg.find(r.label);
        if (it == agg.end()) order.push_back(r.label);
        Agg &a = agg[r.label];
        a.count++;
        a.ms += ms;
    }
    ctx->profiling = false;
    ctx->prof.clear();
    ctx->event_next = 0;
    std::string out;
    char line[256];
    for (auto &name : order) {
        snprintf(line, sizeof line, "%s %d %.6f\n", name.c_str(), agg[name].count, agg[name].ms);
        out += line;
    }
    snprintf(buf, buf_len, "%s", out.c_str());
    return CW_OK;
}

struct cw_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

int cw_graph_begin(cw_ctx *ctx) {
    CW_CHECK_ARG(ctx != nullptr, "cw_graph_begin: null ctx");
    if (ctx->capturing || ctx->profiling) {
        set_error("cw_graph_begin: %s", ctx->capturing ? "a recording is already open"
                                                       : "profiling is on (cw_profile_report first)");
        return CW_ERR_STATE;
    }
    CW_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
    ctx->capturing = true;
    // the recording may name the current scratch: keep it alive when it grows
    ctx->scratch_recorded = true;
    return CW_OK;
}

int cw_graph_end(cw_ctx *ctx, cw_graph **out) {
    CW_CHECK_ARG(ctx && out, "cw_graph_end: null argument");
    *out = nullptr;
    if (!ctx->capturing) {
        set_error("cw_graph_end: no recording is open (cw_graph_begin)");
        return CW_ERR_STATE;
    }
    ctx->capturing = false;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
    }
    cw_graph *g = new cw_graph();
    g->graph = graph;
    g->exec = exec;
    *out = g;
    return CW_OK;
}

int cw_graph_launch(cw_ctx *ctx, const cw_graph *g) {
    CW_CHECK_ARG(ctx && g, "cw_graph_launch: null argument");
    CW_TRY(refuse_while_capturing(ctx, "cw_graph_launch"));
    CW_HIP(hipGraphLaunch(g->exec, ctx->stream));
    return CW_OK;
}

int cw_graph_destroy(cw_graph *g) {
    if (!g) return CW_OK;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return CW_OK;
}

}  // extern "C"
