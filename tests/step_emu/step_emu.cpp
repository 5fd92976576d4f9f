// CPU execution of the fused decode-step kernel (decode_step.hip) under
// AddressSanitizer.  Test infrastructure only.
//
// The kernel source is compiled for the host with hip/hip_runtime.h beside
// this file standing in for HIP.  Every thread of the grid (n_cu workgroups
// of 512 threads, the launch the library makes) runs as a fiber of one OS
// thread; a fiber runs until it waits in a collective (shuffle, DPP move,
// workgroup barrier) or polls an atomic, then the next one runs.
//
// The buffers are the library's own plan (cw_step_dry_plan, written to a
// file by tests/test_step_emu.py): every planned allocation becomes one host
// allocation of exactly its size, every pointer of the argument block and
// layer table is moved into its allocation, and the kernel reads the argument
// block from its allocation, as on the device.  Each workgroup's LDS is two
// host allocations of exactly the static and dynamic bytes of the launch.
//
// usage: step_emu PLAN_FILE KV_DTYPE(0 f32 / 1 f16) N_CU STEPS PROMPT_LEN
// Exit 0 when every step completes; AddressSanitizer aborts on the first
// access outside an allocation; a deadlock (no fiber can progress) exits 3.
#include <sanitizer/common_interface_defs.h>
#include <sys/mman.h>

#include <vector>

#include "hip/hip_runtime.h"

// ---- the pieces of context.hip the step's host code names
#include "cw_internal.hpp"
namespace cwi {
void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    fputc('\n', stderr);
}
int hip_fail(hipError_t e, const char *what, const char *file, int line) {
    set_error("HIP error %d in %s at %s:%d", (int)e, what, file, line);
    return CW_ERR_HIP;
}
void prof_begin(cw_ctx *, const char *) {}
void prof_end(cw_ctx *) {}
}  // namespace cwi

#include "decode_step.hip"

// ---------------------------------------------------------------- fibers

extern "C" void emu_switch(void **save_sp, void *load_sp);
asm(R"(
.text
.globl emu_switch
.type emu_switch,@function
emu_switch:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
)");

namespace emu {

constexpr size_t kStack = 256 << 10;

struct Wave {
    int arrived = 0;
    unsigned gen = 0;
    int kind[64], param[64];
    uint32_t in[64], out[64];
};
struct Group {
    int arrived = 0;
    unsigned gen = 0;
    std::vector<Wave> waves;
    void *lds_static = nullptr;
    size_t lds_static_bytes = 0;
    void *lds_dynamic = nullptr;
};
struct Fiber {
    void *sp = nullptr;
    unsigned char *stack = nullptr;
    Idx tid, bid;
    int group = 0, wave = 0, lane = 0;
    bool done = false;
};

struct Launch {
    void (*kernel)(const cwi::StepArgs *) = nullptr;
    const cwi::StepArgs *args = nullptr;
    Idx bdim, gdim;
    size_t lds_dynamic = 0;
    std::vector<Fiber> fibers;
    std::vector<Group> groups;
};

Launch *g_launch = nullptr;
Fiber *g_cur = nullptr;
void *g_sched_sp = nullptr;
unsigned long long g_progress = 0, g_clock = 0;
const void *g_sched_stack_bottom = nullptr;
size_t g_sched_stack_size = 0;

Fiber *cur() { return g_cur; }
const Idx &thread_idx() { return g_cur->tid; }
const Idx &block_idx() { return g_cur->bid; }
const Idx &block_dim() { return g_launch->bdim; }
const Idx &grid_dim() { return g_launch->gdim; }
void progress() { ++g_progress; }
unsigned long long clock() { return ++g_clock; }

void *wg_static(size_t bytes) {
    Group &g = g_launch->groups[g_cur->group];
    if (!g.lds_static) {
        g.lds_static = calloc(1, bytes);
        g.lds_static_bytes = bytes;
    }
    if (bytes != g.lds_static_bytes) {
        fprintf(stderr, "static LDS requested with two sizes\n");
        abort();
    }
    return g.lds_static;
}
void *wg_dynamic() { return g_launch->groups[g_cur->group].lds_dynamic; }

void yield() {
    Fiber *f = g_cur;
    void *fake = nullptr;
    __sanitizer_start_switch_fiber(&fake, g_sched_stack_bottom, g_sched_stack_size);
    emu_switch(&f->sp, g_sched_sp);
    __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
}

static uint32_t dpp(const Wave &w, int lane, int ctrl) {
    int src = lane;
    if (ctrl < 0x100) {  // quad_perm
        src = (lane & ~3) | ((ctrl >> (2 * (lane & 3))) & 3);
    } else if (ctrl == 0x141) {  // row_half_mirror
        src = (lane & ~7) | (7 - (lane & 7));
    } else if (ctrl == 0x140) {  // row_mirror
        src = (lane & ~15) | (15 - (lane & 15));
    } else {
        fprintf(stderr, "DPP control 0x%x not emulated\n", ctrl);
        abort();
    }
    return w.in[src];
}

uint32_t wave_op(uint32_t v, int kind, int param) {
    Fiber *f = g_cur;
    Wave &w = g_launch->groups[f->group].waves[f->wave];
    w.in[f->lane] = v;
    w.kind[f->lane] = kind;
    w.param[f->lane] = param;
    const unsigned gen = w.gen;
    if (++w.arrived == 64) {
        for (int l = 0; l < 64; ++l) {
            if (w.kind[l] != w.kind[0]) {
                fprintf(stderr, "wave %d of workgroup %d: lanes reached different collectives\n",
                        f->wave, f->group);
                abort();
            }
            const int p = w.param[l];
            if (kind == OP_FIRST && w.in[l] != w.in[0]) {
                fprintf(stderr, "wave %d of workgroup %d: readfirstlane of a value that is not "
                                "uniform (lane %d holds 0x%x, lane 0 0x%x)\n",
                        f->wave, f->group, l, w.in[l], w.in[0]);
                abort();
            }
            if (kind == OP_FIRST) w.out[l] = w.in[0];
            else if (kind == OP_SHFL) w.out[l] = w.in[((p % 64) + 64) % 64];
            else if (kind == OP_SHFL_XOR) w.out[l] = w.in[(l ^ p) & 63];
            else w.out[l] = dpp(w, l, p);
        }
        w.arrived = 0;
        ++w.gen;
        progress();
    } else {
        while (w.gen == gen) yield();
    }
    return w.out[f->lane];
}

void sync_threads() {
    Group &g = g_launch->groups[g_cur->group];
    const unsigned gen = g.gen;
    const int n = (int)(g_launch->bdim.x * g_launch->bdim.y * g_launch->bdim.z);
    if (++g.arrived == n) {
        g.arrived = 0;
        ++g.gen;
        progress();
    } else {
        while (g.gen == gen) yield();
    }
}

extern "C" void emu_fiber_main() {
    // (first entry: learn the scheduler's stack bounds)
    __sanitizer_finish_switch_fiber(nullptr, &g_sched_stack_bottom, &g_sched_stack_size);
    g_launch->kernel(g_launch->args);
    g_cur->done = true;
    progress();
    __sanitizer_start_switch_fiber(nullptr, g_sched_stack_bottom, g_sched_stack_size);  // ends
    void *dead = nullptr;
    emu_switch(&dead, g_sched_sp);
    abort();  // never resumed
}

// Run one launch to completion; false on a deadlock.
bool run(Launch &L) {
    g_launch = &L;
    const unsigned nthr = L.bdim.x, ngrp = L.gdim.x;
    L.groups.assign(ngrp, Group{});
    for (auto &g : L.groups) {
        g.waves.assign((nthr + 63) / 64, Wave{});
        g.lds_dynamic = L.lds_dynamic ? calloc(1, L.lds_dynamic) : nullptr;
    }
    L.fibers.assign((size_t)ngrp * nthr, Fiber{});
    for (unsigned b = 0; b < ngrp; ++b)
        for (unsigned t = 0; t < nthr; ++t) {
            Fiber &f = L.fibers[(size_t)b * nthr + t];
            f.tid = Idx{t, 0, 0};
            f.bid = Idx{b, 0, 0};
            f.group = (int)b;
            f.wave = (int)(t / 64);
            f.lane = (int)(t % 64);
            f.stack = static_cast<unsigned char *>(mmap(nullptr, kStack, PROT_READ | PROT_WRITE,
                                                        MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE,
                                                        -1, 0));
            if (f.stack == MAP_FAILED) {
                perror("mmap");
                exit(4);
            }
            // entry frame: six callee-saved registers, then the entry address
            uintptr_t top = (uintptr_t)(f.stack + kStack) & ~(uintptr_t)15;
            uint64_t *sp = reinterpret_cast<uint64_t *>(top - 8);
            *sp = 0;                                           // no return address
            *--sp = (uint64_t)(uintptr_t)&emu_fiber_main;
            for (int r = 0; r < 6; ++r) *--sp = 0;
            f.sp = sp;
        }
    size_t live = L.fibers.size();
    int idle_passes = 0;
    while (live) {
        const unsigned long long p0 = g_progress;
        for (auto &f : L.fibers) {
            if (f.done) continue;
            g_cur = &f;
            void *fake = nullptr;
            __sanitizer_start_switch_fiber(&fake, f.stack, kStack);
            emu_switch(&g_sched_sp, f.sp);
            __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
            if (f.done) {
                --live;
                munmap(f.stack, kStack);
                f.stack = nullptr;
            }
        }
        if (g_progress == p0) {
            if (++idle_passes > 4) {
                size_t waiting = 0;
                for (auto &f : L.fibers) waiting += !f.done;
                fprintf(stderr, "deadlock: %zu fibers wait and none can progress\n", waiting);
                return false;
            }
        } else {
            idle_passes = 0;
        }
    }
    for (auto &g : L.groups) {
        free(g.lds_static);
        free(g.lds_dynamic);
    }
    L.fibers.clear();
    L.groups.clear();
    return true;
}

}  // namespace emu

// ---------------------------------------------------------------- the plan

struct Plan {
    std::vector<unsigned char> args, layers;
    std::vector<uint64_t> ext_ptr, ext_bytes;
};

static bool read_plan(const char *path, Plan &p) {
    FILE *f = fopen(path, "rb");
    if (!f) return false;
    uint64_t hdr[4];  // sizeof(StepArgs), layer table bytes, n extents, sizeof(StepLayer)
    bool ok = fread(hdr, 8, 4, f) == 4;
    if (ok && (hdr[0] != sizeof(cwi::StepArgs) || hdr[3] != sizeof(cwi::StepLayer))) {
        fprintf(stderr, "plan written for another layout of StepArgs / StepLayer\n");
        ok = false;
    }
    if (ok) {
        p.args.resize(hdr[0]);
        p.layers.resize(hdr[1]);
        p.ext_ptr.resize(hdr[2]);
        p.ext_bytes.resize(hdr[2]);
        ok = fread(p.args.data(), 1, hdr[0], f) == hdr[0] &&
             fread(p.layers.data(), 1, hdr[1], f) == hdr[1] &&
             fread(p.ext_ptr.data(), 8, hdr[2], f) == hdr[2] &&
             fread(p.ext_bytes.data(), 8, hdr[2], f) == hdr[2];
    }
    fclose(f);
    return ok;
}

struct Memory {
    std::vector<uint64_t> dry, bytes;
    std::vector<unsigned char *> host;
    // the host address of dry address d; null stays null; a pointer outside
    // every planned allocation is a finding
    template <class T>
    T *map(T *d, const char *what) {
        if (!d) return nullptr;
        const uint64_t a = (uint64_t)(uintptr_t)d;
        for (size_t i = 0; i < dry.size(); ++i)
            if (a >= dry[i] && a < dry[i] + bytes[i])
                return reinterpret_cast<T *>(host[i] + (a - dry[i]));
        fprintf(stderr, "%s points outside every planned allocation\n", what);
        exit(5);
    }
    // the rest of the host allocation holding p, from p on
    size_t tail(const void *p) const {
        const unsigned char *c = static_cast<const unsigned char *>(p);
        for (size_t i = 0; i < host.size(); ++i)
            if (c >= host[i] && c < host[i] + bytes[i]) return (size_t)(host[i] + bytes[i] - c);
        return 0;
    }
};

// deterministic data: quants random, f16 scales 0.01, gains 1, the embedding
// and the RoPE table small random values, so tokens and softmax weights vary
static uint32_t g_rng = 12345u;
static uint32_t rnd() {
    g_rng = g_rng * 1664525u + 1013904223u;
    return g_rng;
}
static void fill_bytes(const Memory &m, const void *p) {
    unsigned char *c = (unsigned char *)p;
    for (size_t i = 0, n = m.tail(p); i < n; ++i) c[i] = (unsigned char)(rnd() >> 24);
}
static void fill_f16(const Memory &m, const void *p, uint16_t bits) {
    uint16_t *h = (uint16_t *)p;
    for (size_t i = 0, n = m.tail(p) / 2; i < n; ++i) h[i] = bits;
}
static void fill_f32(const Memory &m, const void *p, float v, float noise) {
    float *f = (float *)p;
    for (size_t i = 0, n = m.tail(p) / 4; i < n; ++i)
        f[i] = v + noise * ((float)(rnd() >> 8) / 16777216.0f - 0.5f);
}

int main(int argc, char **argv) {
    if (argc < 6) {
        fprintf(stderr, "usage: %s PLAN KV_DTYPE N_CU STEPS PROMPT_LEN\n", argv[0]);
        return 2;
    }
    Plan plan;
    if (!read_plan(argv[1], plan)) {
        fprintf(stderr, "cannot read the plan %s\n", argv[1]);
        return 2;
    }
    const int kv_dtype = atoi(argv[2]), n_cu = atoi(argv[3]), steps = atoi(argv[4]),
              n_prompt = atoi(argv[5]);
    Memory mem;
    for (size_t i = 0; i < plan.ext_ptr.size(); ++i) {
        mem.dry.push_back(plan.ext_ptr[i]);
        mem.bytes.push_back(plan.ext_bytes[i]);
        mem.host.push_back(static_cast<unsigned char *>(calloc(1, plan.ext_bytes[i])));
    }
    cwi::StepArgs a;
    memcpy(&a, plan.args.data(), sizeof a);
    const int L = a.n_layers;
    std::vector<cwi::StepLayer> layers(L);
    memcpy(layers.data(), plan.layers.data(), sizeof(cwi::StepLayer) * L);
    for (int l = 0; l < L; ++l) {
        cwi::StepLayer &y = layers[l];
        y.attn_norm = mem.map(y.attn_norm, "attn_norm");
        y.q_norm = mem.map(y.q_norm, "q_norm");
        y.k_norm = mem.map(y.k_norm, "k_norm");
        y.ffn_norm = mem.map(y.ffn_norm, "ffn_norm");
        y.qkv_q = mem.map(y.qkv_q, "qkv quants");
        y.qkv_s = mem.map(y.qkv_s, "qkv scales");
        y.o_q = mem.map(y.o_q, "o quants");
        y.o_s = mem.map(y.o_s, "o scales");
        y.gu_q = mem.map(y.gu_q, "gate|up quants");
        y.gu_s = mem.map(y.gu_s, "gate|up scales");
        y.down_q = mem.map(y.down_q, "down quants");
        y.down_s = mem.map(y.down_s, "down scales");
        y.kc = mem.map(y.kc, "K cache");
        y.vc = mem.map(y.vc, "V cache");
    }
    // the layer table lives in its planned allocation, read by the kernel
    cwi::StepLayer *layers_host = const_cast<cwi::StepLayer *>(mem.map(a.layers, "layer table"));
    memcpy(layers_host, layers.data(), sizeof(cwi::StepLayer) * L);
    a.layers = layers_host;
    a.embed = mem.map(a.embed, "embedding");
    a.final_norm = mem.map(a.final_norm, "final norm");
    a.lm_q = mem.map(a.lm_q, "LM head quants");
    a.lm_s = mem.map(a.lm_s, "LM head scales");
    a.cos_t = mem.map(a.cos_t, "RoPE cos");
    a.sin_t = mem.map(a.sin_t, "RoPE sin");
    a.h_a = mem.map(a.h_a, "h_a");
    a.h_b = mem.map(a.h_b, "h_b");
    a.qkv = mem.map(a.qkv, "qkv");
    a.attn = mem.map(a.attn, "attn");
    a.act = mem.map(a.act, "act");
    a.part = mem.map(a.part, "partials");
    a.logits = mem.map(a.logits, "logits");
    a.hidden_out = mem.map(a.hidden_out, "hidden_out");
    a.am_v = mem.map(a.am_v, "argmax values");
    a.am_i = mem.map(a.am_i, "argmax ids");
    a.sync = mem.map(a.sync, "grid counters");
    a.state = mem.map(a.state, "decode state");
    a.prompt = mem.map(a.prompt, "prompt");
    a.tokens = mem.map(a.tokens, "tokens");
    a.argmax_out = mem.map(a.argmax_out, "argmax output");
    a.trace = nullptr;
    a.timeout = (long long)1 << 50;
    // the argument block the kernel reads: the plan's last allocation (the
    // fused step allocates it after every other buffer)
    cwi::StepArgs *args_host = nullptr;
    if (!mem.bytes.empty() && mem.bytes.back() == sizeof(cwi::StepArgs))
        args_host = reinterpret_cast<cwi::StepArgs *>(mem.host.back());
    if (!args_host) {
        fprintf(stderr, "no planned allocation holds the argument block\n");
        return 5;
    }
    const uint16_t d16 = 0x211F;  // f16 0.01
    for (int l = 0; l < L; ++l) {
        const cwi::StepLayer &y = layers[l];
        for (const void *g : {(const void *)y.attn_norm, (const void *)y.ffn_norm,
                              (const void *)y.q_norm, (const void *)y.k_norm})
            fill_f32(mem, g, 1.0f, 0.0f);
        for (const void *q : {(const void *)y.qkv_q, (const void *)y.o_q, (const void *)y.gu_q,
                              (const void *)y.down_q})
            fill_bytes(mem, q);
        for (const void *sc : {(const void *)y.qkv_s, (const void *)y.o_s, (const void *)y.gu_s,
                               (const void *)y.down_s})
            fill_f16(mem, sc, d16);
    }
    fill_f32(mem, a.embed, 0.0f, 0.2f);
    fill_f32(mem, a.final_norm, 1.0f, 0.0f);
    fill_bytes(mem, a.lm_q);
    fill_f16(mem, a.lm_s, d16);
    fill_f32(mem, a.cos_t, 0.0f, 2.0f);
    fill_f32(mem, a.sin_t, 0.0f, 2.0f);
    // decode state and prompt (cw_generate: prompt ids, state at position 0)
    cwi::GenState st{};
    st.pos = 0;
    st.token = 1;
    st.start_pos = 0;
    st.n_prompt = n_prompt;
    st.produced = 0;
    st.max_out = steps;
    memcpy(a.state, &st, sizeof st);
    for (int i = 0; i < n_prompt; ++i) const_cast<uint32_t *>(a.prompt)[i] = 1 + i;
    memcpy(args_host, &a, sizeof a);

    const int hpk = a.n_heads / a.n_kv;
    emu::Launch launch;
    launch.kernel = kv_dtype == CW_F16 ? pick_hpk<_Float16>(hpk) : pick_hpk<float>(hpk);
    if (!launch.kernel) {
        fprintf(stderr, "no kernel for %d heads per kv head\n", hpk);
        return 2;
    }
    launch.args = args_host;
    launch.bdim = emu::Idx{(unsigned)kT, 1, 1};
    launch.gdim = emu::Idx{(unsigned)n_cu, 1, 1};
    launch.lds_dynamic = (size_t)cwi::step_lds_bytes(kv_dtype, hpk, a.max_seq);
    for (int s = 0; s < steps; ++s) {
        if (!emu::run(launch)) return 3;
        cwi::GenState now;
        memcpy(&now, a.state, sizeof now);
        const unsigned err = a.sync[cwi::step_sync_err_index()];
        printf("step %d: pos %d -> %d, token %u, argmax %u, produced %d, error word %u\n", s,
               st.pos + s, now.pos, now.token, *a.argmax_out, now.produced, err);
        fflush(stdout);
        if (err) return 6;
    }
    for (auto *h : mem.host) free(h);
    return 0;
}
