/*
 * chat_wgpu.h -- C ABI of the MI355X-native chat-wgpu decode path.
 *
 * Plain C: opaque handles, raw pointers and sizes, int status codes.  Device
 * pointers are HIP device addresses (from cw_alloc / cw_frame_alloc); host
 * pointers are ordinary memory.  Every entry point returns CW_OK (0) or a
 * negative CW_ERR_*; cw_last_error() then holds a message (thread-local).
 * Kernel entry points validate their arguments on the host before anything
 * is launched and enqueue asynchronously on the context's single HIP stream;
 * only cw_download, cw_flush, cw_profile_report and the cw_model_* calls that
 * return host data synchronise.  A context is not thread-safe (the reference's
 * GpuContext is !Sync, src/context.rs:9,29-56).
 *
 * Each declaration names the reference interface it replaces (file:line in
 * EggerMarc/chat-wgpu).
 */
#ifndef CHAT_WGPU_H
#define CHAT_WGPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CW_OK 0
#define CW_ERR_ARG (-1)     /* invalid argument (shape, null pointer, range) */
#define CW_ERR_HIP (-2)     /* a HIP runtime call failed */
#define CW_ERR_OOM (-3)     /* device or host allocation failed */
#define CW_ERR_STATE (-4)   /* call not valid in the current state */
#define CW_ERR_FORMAT (-5)  /* malformed or unsupported file contents (GGUF) */
#define CW_ERR_IO (-6)      /* a file could not be opened, read or mapped */

/* element types of a KV cache */
#define CW_F32 0
#define CW_F16 1

typedef struct cw_ctx cw_ctx;
typedef struct cw_model cw_model;
typedef struct cw_gguf cw_gguf;
typedef struct cw_graph cw_graph;

/* ---------------------------------------------------------------- */
/* Context: device, stream, arena (src/context.rs)                   */
/* ---------------------------------------------------------------- */

/* GpuContext::new (src/context.rs:60-104): open `device`, create the stream. */
int cw_ctx_create(int device, cw_ctx **out);
/* Drop for GpuContext: waits for the stream, frees every allocation. */
int cw_ctx_destroy(cw_ctx *ctx);
/* Text of the last error on this thread ("" if none). */
const char *cw_last_error(void);
/* Library version string. */
const char *cw_version(void);
/* Device facts: compute units, HBM bytes, gfx arch name. */
int cw_device_info(cw_ctx *ctx, int *n_cu, size_t *hbm_bytes, char *arch, size_t arch_len);

/* GpuContext::empty_persistent / storage (src/context.rs:177-227): a
 * persistent device allocation, 256-byte aligned. */
int cw_alloc(cw_ctx *ctx, size_t bytes, void **out);
int cw_free(cw_ctx *ctx, void *ptr);
/* GpuContext::empty (src/context.rs:210-227): per-frame scratch.  Valid until
 * cw_frame_reset; the same call sequence after a reset returns the same
 * addresses (the arena is deterministic, like the reference's). */
int cw_frame_alloc(cw_ctx *ctx, size_t bytes, void **out);
/* GpuContext::reset_frame (src/context.rs:237-240). */
int cw_frame_reset(cw_ctx *ctx);
/* GpuContext::storage's upload (create_buffer_init, src/context.rs:177-194):
 * host -> device, ordered on the stream. */
int cw_upload(cw_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes);
/* GpuContext::read (src/context.rs:361-389): flush, then device -> host;
 * returns after the data is on the host. */
int cw_download(cw_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes);
/* GpuContext::copy (src/context.rs:255-269): device -> device on the stream. */
int cw_copy(cw_ctx *ctx, void *dst_dev, const void *src_dev, size_t bytes);
/* GpuContext::flush (src/context.rs:141-151): wait until the stream drains. */
int cw_flush(cw_ctx *ctx);

/* Recorded launch sequences: the counterpart of the reference's per-frame
 * command-buffer replay, whose bind-group cache needs the same op sequence
 * every frame (src/context.rs:141-151, 330-334).  cw_graph_begin starts
 * recording the context's kernel launches instead of running them;
 * cw_graph_end closes the recording into an executable graph; cw_graph_launch
 * replays it on the stream (the buffers, shapes and scalars recorded stay
 * fixed; device-resident values, such as a position read by a kernel, may
 * change between replays); cw_graph_destroy frees it.  While recording, calls
 * that would allocate or synchronise fail with CW_ERR_STATE (uploads,
 * downloads, flush, profiling, a first frame-arena chunk, kernel scratch or
 * RoPE table at a new size): run the sequence once before recording.  The
 * cw_model_* and cw_generate calls keep their own graph and are not
 * recordable: while recording they return CW_ERR_STATE and change nothing. */
int cw_graph_begin(cw_ctx *ctx);
int cw_graph_end(cw_ctx *ctx, cw_graph **out);
int cw_graph_launch(cw_ctx *ctx, const cw_graph *g);
int cw_graph_destroy(cw_graph *g);

/* ---------------------------------------------------------------- */
/* Kernels (src/kernels/NAME.rs).  Q4 weights are GGUF Q4_0 split into   */
/* two arrays: scales = f16 bits [out_f][in_f/32], quants = the 16     */
/* packed bytes of every block [out_f][in_f/32][16] (low nibble of byte */
/* j -> element j, high nibble -> element j+16; value d*(q-8)).        */
/* ---------------------------------------------------------------- */

/* q4::gemv (src/kernels/q4.rs:9-30, q4.wgsl:25-82): y[out_f] = W x[in_f].
 * in_f must be a positive multiple of 32 and at most 32768. */
int cw_q4_gemv(cw_ctx *ctx, const float *x, const uint16_t *scales, const uint8_t *quants,
               int in_f, int out_f, float *y);
/* q4::gemv followed by attention::add (src/model/qwen3.rs:178-179,186-187):
 * y = residual + W x.  y may alias residual. */
int cw_q4_gemv_add(cw_ctx *ctx, const float *x, const uint16_t *scales, const uint8_t *quants,
                   int in_f, int out_f, const float *residual, float *y);
/* gate/up q4::gemv then activation::swiglu (src/model/qwen3.rs:183-185):
 * y = silu(Wg x) * (Wu x), both matrices [out_f][in_f]. */
int cw_q4_gemv_swiglu(cw_ctx *ctx, const float *x, const uint16_t *gate_scales,
                      const uint8_t *gate_quants, const uint16_t *up_scales,
                      const uint8_t *up_quants, int in_f, int out_f, float *y);
/* norm::rmsnorm (src/kernels/norm.rs:26-29, norm.wgsl:20-42): per row
 * y = x * inverseSqrt(sum(x^2)/dim + eps) * w. */
int cw_rmsnorm(cw_ctx *ctx, const float *x, const float *w, int rows, int dim, float eps, float *y);
/* rope::rope (src/kernels/rope.rs:8-27, rope.wgsl:18-35): NeoX rotate-half of
 * rows x head_dim at position pos.  Angles pos*theta^(-2i/hd) come from a
 * table evaluated in f64 and rounded to f32. */
int cw_rope(cw_ctx *ctx, const float *x, int rows, int head_dim, int pos, float theta, float *y);
/* attention::attention (src/kernels/attention.rs:7-38, attention.wgsl:23-96):
 * single-query GQA attention over seq positions of a [seq][n_kv*hd] cache of
 * element type kv_dtype (CW_F32 or CW_F16).  head_dim in {16,32,64,128,256}. */
int cw_attention(cw_ctx *ctx, const float *q, const void *k, const void *v, int kv_dtype,
                 int n_heads, int n_kv_heads, int seq, int head_dim, float *out);
/* No counterpart in the reference: cw_attention for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as cw_attention, but the
 * chunk partials and arrival counters live in a static device array of
 * 8 MiB + 128 KiB that each GPU holds from the first cw_ctx_create on it
 * until the process ends; the call allocates nothing (no device memory, no
 * profiling events).  Limit: n_heads * ceil(seq / 16) * (head_dim + 2) * 4
 * bytes of partials must fit 8 MiB (32 heads of 128 dims: seq <= 8064), else
 * CW_ERR_ARG.  Every call on a GPU shares that GPU's array, so calls that
 * overlap on one GPU (other streams, other contexts) race. */
int cw_attention_noalloc(cw_ctx *ctx, const float *q, const void *k, const void *v,
                         int kv_dtype, int n_heads, int n_kv_heads, int seq, int head_dim,
                         float *out);
/* attention::add (src/kernels/attention.rs:40-51, ewise.wgsl:9-13): c = a + b. */
int cw_add(cw_ctx *ctx, const float *a, const float *b, int n, float *c);
/* activation::swiglu (src/kernels/activation.rs:42-44, glu.wgsl:22-26). */
int cw_swiglu(cw_ctx *ctx, const float *gate, const float *up, int n, float *out);
/* argmax::argmax (src/kernels/argmax.rs:11-18, argmax.wgsl:18-55): index of
 * the maximum, lowest index among equals, written to out_dev[0]. */
int cw_argmax(cw_ctx *ctx, const float *logits, int n, uint32_t *out_dev);
/* KvCache::write (src/model/cache.rs:21-24): k,v [kv_dim] f32 -> row pos of
 * the caches (converted to f16, round to nearest even, for CW_F16). */
int cw_kv_write(cw_ctx *ctx, void *k_cache, void *v_cache, int kv_dtype, int pos, int kv_dim,
                const float *k, const float *v);
/* Qwen3::embed (src/model/qwen3.rs:128-133) plus clone_buf (qwen3.rs:194-197):
 * out = table[token_dev[0]] + 0, token read on the device (< vocab). */
int cw_embed(cw_ctx *ctx, const float *table, int vocab, int dim, const uint32_t *token_dev,
             float *out);

/* examples/q4probe.rs (raw read-bandwidth sweep): stream `bytes` of buf with
 * 128-bit loads over `blocks` workgroups of 256 threads, XOR-fold, write one
 * word per workgroup to out_dev.  Time it with the profiler or events. */
int cw_hbm_read_probe(cw_ctx *ctx, const void *buf, size_t bytes, int blocks, uint32_t *out_dev);

/* Batched form of q4::gemv (src/kernels/q4.rs:9-30): y[m][out_f] = x[m][in_f]
 * . W^T for m rows at once, on the matrix cores (the reference has no batched
 * path; every row equals cw_q4_gemv of that row to within 1e-4 relative).
 * x and y device f32, row-major; quants 16-byte aligned; block scales must be
 * finite (each block's f32 sum is multiplied by its scale). */
int cw_q4_gemm(cw_ctx *ctx, const float *x, int m, const uint16_t *scales, const uint8_t *quants,
               int in_f, int out_f, float *y);

/* ---------------------------------------------------------------- */
/* Host-side Q4 helpers                                              */
/* ---------------------------------------------------------------- */

/* q4::quantize_q4_0 (src/kernels/q4.rs:37-61) producing GGUF Q4_0: d =
 * absmax/8 rounded to f16, q = clamp(round(v/d)+8, 0, 15) against the stored
 * f16 d.  data is [out_f][in_f] row-major; in_f % 32 == 0. */
int cw_q4_quantize(const float *data, size_t out_f, size_t in_f, uint16_t *scales,
                   uint8_t *quants);
/* GGUF Q4_0 18-byte blocks (dequant.rs:60-78 layout) -> split image. */
int cw_q4_split_blocks(const uint8_t *blocks, size_t nblocks, uint16_t *scales, uint8_t *quants);

/* ---------------------------------------------------------------- */
/* Seeded synthetic data (counter-based, independent of thread count) */
/* ---------------------------------------------------------------- */

/* Stream key of a named tensor: FNV-1a 64 of the name mixed with seed. */
uint64_t cw_synth_key(uint64_t seed, const char *name);
/* Q4_0 blocks: d = f16(|N(0, sigma)|), 16 uniform random bytes per block. */
int cw_synth_q4(uint64_t key, size_t nblocks, float sigma, uint16_t *scales, uint8_t *quants);
/* n f32 values ~ N(mean, std). */
int cw_synth_normal_f32(uint64_t key, size_t n, float mean, float std, float *out);
/* n f16 values ~ N(mean, std), rounded to nearest even. */
int cw_synth_normal_f16(uint64_t key, size_t n, float mean, float std, uint16_t *out);
/* n token ids uniform in [0, vocab). */
int cw_synth_tokens(uint64_t key, size_t n, uint32_t vocab, uint32_t *out);

/* ---------------------------------------------------------------- */
/* Model: Qwen3 forward + greedy loop (src/model/NAME.rs)              */
/* ---------------------------------------------------------------- */

/* The per-family composition switches the reference pins for qwen3
 * (README.md:47-63): plain RMSNorm gain, SwiGLU, per-head QK-norm, no QKV
 * bias, LM head tied to the embedding unless "output.weight" is given. */
typedef struct cw_family_spec {
    int norm_unit_gain;  /* 0: y = x/rms * w (the only form built) */
    int act;             /* 0: SwiGLU (the only form built) */
    int qk_norm;         /* 1: per-head RMSNorm on q and k */
    int qkv_bias;        /* 0: no bias (the only form built) */
} cw_family_spec;

/* The metadata Qwen3::load reads (src/model/qwen3.rs:45-53). */
typedef struct cw_model_config {
    cw_family_spec family;
    int n_layers, dim, n_heads, n_kv_heads, head_dim, hidden, vocab;
    float eps, rope_theta;
    int max_seq;   /* KV capacity (Model::new_cache's max_seq, mod.rs:65) */
    int kv_dtype;  /* CW_F32 or CW_F16 */
} cw_model_config;

/* Qwen3 (src/model/qwen3.rs:44-113): allocate device storage for every
 * tensor and the KV cache.  Weights are then supplied by name. */
int cw_model_create(cw_ctx *ctx, const cw_model_config *cfg, cw_model **out);
int cw_model_destroy(cw_model *m);
/* Weights::matrix_raw + Q4Linear (src/model/mod.rs:130-153, layers.rs:74-95),
 * by GGUF name ("blk.3.attn_q.weight", "output.weight", ...).  Layer
 * projections need finite block scales: CW_ERR_ARG otherwise. */
int cw_model_set_q4(cw_model *m, const char *name, const uint16_t *scales_host,
                    const uint8_t *quants_host);
/* Weights::vector (norm gains "blk.3.attn_norm.weight", "output_norm.weight";
 * the embedding "token_embd.weight" [vocab][dim]). */
int cw_model_set_f32(cw_model *m, const char *name, const float *data_host);
/* Every tensor of the config's distributions generated from seed by the
 * cw_synth_* functions under its GGUF name (host side, then uploaded). */
int cw_model_load_synthetic(cw_model *m, uint64_t seed);
/* Checks every tensor is present; builds the tied LM head (qwen3.rs:93-98)
 * when "output.weight" was not given. */
int cw_model_finalize(cw_model *m);
/* Fill KV positions [0, n_pos) of every layer from host arrays laid out
 * [layer][pos][kv_dim] in the cache's element type. */
int cw_model_prefill_kv(cw_model *m, const void *k_host, const void *v_host, int n_pos);
/* One forward at pos for token (embed -> forward -> logits -> argmax), the
 * body of generate's loop (src/model/mod.rs:93-103).  Returns the argmax. */
int cw_model_step(cw_model *m, uint32_t token, int pos, uint32_t *argmax_out);
/* Download the logits [vocab] of the last step. */
int cw_model_logits(cw_model *m, float *host_out);
/* Download the final hidden state [dim] (post final norm) of the last step. */
int cw_model_hidden(cw_model *m, float *host_out);
/* Hook (src/model/mod.rs:158-165) in the shape of main.rs's Capture hook
 * (main.rs:193-207): with taps on, every decode step (eager or graph) keeps
 * the forward's taps of each layer: "q" after QK-norm and RoPE
 * (qwen3.rs:165, n_heads*head_dim floats), "post_attn" after the attention
 * residual (qwen3.rs:180, dim floats) and "layer_out" (qwen3.rs:188, dim
 * floats).  Toggling re-captures the graph step; the batched prompt phase
 * (cw_model_prefill) records the taps of its last position. */
int cw_model_set_taps(cw_model *m, int enable);
/* Copy the tap `name` of `layer` from the last decode step to host (len
 * floats; synchronises).  CW_ERR_STATE while taps are off. */
int cw_model_tap(cw_model *m, const char *name, int layer, float *host_out, int len);
/* How a decode step is executed (cw_generate, cw_model_decode_async). */
#define CW_STEP_EAGER 0  /* 1 + 5*n_layers kernel launches per token */
#define CW_STEP_GRAPH 1  /* the same launches captured once as a HIP graph and replayed */
#define CW_STEP_FUSED 2  /* one persistent cooperative kernel per token (head_dim 128) */

/* model::generate (src/model/mod.rs:57-125): greedy loop over the prompt then
 * max_new produced tokens (P+N-1 forwards), the whole step device-resident
 * (position and token live on the device), executed as `mode` (CW_STEP_*).
 * The first prompt token is fed at start_pos (0 = empty cache).  Writes
 * max_new ids to out_tokens.  CW_STEP_FUSED returns CW_ERR_ARG for shapes it
 * does not cover and CW_ERR_HIP if a grid barrier timed out. */
int cw_generate(cw_model *m, const uint32_t *prompt, int n_prompt, int max_new, int start_pos,
                int mode, uint32_t *out_tokens);
/* Launch n_steps more decode steps of the current generate state without
 * synchronising (for timing); cw_flush waits. */
int cw_model_decode_async(cw_model *m, int n_steps, int mode);
/* One token of the chat decode loop (src/wasm.rs:95-114: embed the last id,
 * forward, logits, argmax): replays one CW_STEP_GRAPH step of the current
 * decode state and returns the new argmax in *next_out with a single 4-byte
 * read.  CW_ERR_ARG once the state's position reaches max_seq. */
int cw_model_decode_next(cw_model *m, uint32_t *next_out);
/* Per-phase timeline of one fused decode step (profile.rs:17-118 reports per
 * kernel; the fused step is one kernel, so it reports per phase): runs one
 * CW_STEP_FUSED step of the current generate state and writes the wall-clock
 * stamps workgroup 0 took: [0] start, then per grid barrier e = 1..5L
 * [2e] arrive and [2e+1] release, [10L+2] the end of the LM head, and from
 * [10L+4] per phase (5 per layer, then the LM head) two stamps: after
 * staging, after compute (20L+8 stamps in all); *tick_hz is the clock rate. */
int cw_model_profile_step(cw_model *m, int64_t *ticks, int max_n, int *n_out, double *tick_hz);
/* No counterpart in the reference: a host-only check, for tests and for
 * callers that plan memory before creating a model, of the buffer layout the
 * CW_STEP_FUSED kernel would use for cfg on a device of n_cu compute units.
 * It lays out every buffer cw_model_create and the fused step allocate, at
 * addresses that are never mapped (no device is touched), then walks the
 * step's own phase table and checks that every range each phase reads or
 * writes lies inside one allocation.  split_gate_up = 1 lays the gate and up
 * projections out as two allocations while the step reads them as one
 * [2*hidden][dim] matrix (a layout the check must refuse); 0 is the layout
 * cw_model_create uses.  CW_OK when the layout holds; CW_ERR_STATE with the
 * first offending range in why (and cw_last_error) when it does not;
 * CW_ERR_ARG for configs the fused step does not cover. */
int cw_step_layout_check(const cw_model_config *cfg, int n_cu, int split_gate_up, char *why,
                         size_t why_len);
/* No counterpart in the reference: for a CPU execution of the CW_STEP_FUSED
 * kernel (tests/step_emu).  The same unmapped buffer plan as
 * cw_step_layout_check, without its range check: copies the step's argument
 * block (args_len bytes of the library's internal StepArgs) and its layer
 * table (layers_len bytes, n_layers internal StepLayer records) and lists
 * every planned allocation as (ext_ptr[i], ext_bytes[i]), i < *n_ext <=
 * max_ext, so a caller can back each one with real memory of exactly that
 * size and relocate the pointers.  CW_ERR_ARG when a length is too small or
 * the fused step does not cover cfg. */
int cw_step_dry_plan(const cw_model_config *cfg, int n_cu, int split_gate_up, void *args_out,
                     size_t args_len, void *layers_out, size_t layers_len, void **ext_ptr,
                     size_t *ext_bytes, int max_ext, int *n_ext);
/* The prompt phase of model::generate (src/model/mod.rs:57-125: P forwards,
 * the logits of all but the last discarded) for n tokens at positions
 * start_pos..start_pos+n-1, batched: each layer runs as Q4_0 GEMMs on the
 * matrix cores and causal attention over the cache (f16 cache and head_dim
 * 128; other configurations run the per-token step n times).  Writes the KV
 * rows, leaves the last position's logits (cw_model_logits) and final-normed
 * hidden state (cw_model_hidden), returns its argmax in *next_token, and sets
 * the decode state to (next_token, start_pos + n). */
int cw_model_prefill(cw_model *m, const uint32_t *tokens, int n, int start_pos,
                     uint32_t *next_token);
/* Reset the decode state to (token, pos) without touching the cache. */
int cw_model_reset_state(cw_model *m, uint32_t token, int pos);
/* Download the tokens produced so far by the device-resident loop. */
int cw_model_tokens(cw_model *m, uint32_t *host_out, int max_n, int *n_out);

/* ---------------------------------------------------------------- */
/* GGUF container (src/loader/gguf.rs, src/loader/dequant.rs)         */
/* ---------------------------------------------------------------- */

/* ggml tensor dtypes tensor_f32 decodes (gguf.rs:109-122). */
#define CW_GGML_F32 0
#define CW_GGML_F16 1
#define CW_GGML_Q4_0 2
#define CW_GGML_Q4_1 3
#define CW_GGML_Q8_0 8
#define CW_GGML_Q6_K 14

/* GgufWeights::parse (gguf.rs:68-106) of a file, memory-mapped read-only (the
 * file is not copied; tensors are decoded from the mapping on request).
 * Magic "GGUF", version, tensor and metadata counts, the metadata key/values
 * (kinds 0-12, arrays skipped), the tensor table, then the data section at
 * the next multiple of general.alignment (default 32).  A repeated key or
 * tensor name keeps its last entry.  Errors: CW_ERR_IO (open/map),
 * CW_ERR_FORMAT ("not a GGUF file", truncated header, unknown metadata kind,
 * data section past the end). */
int cw_gguf_open(const char *path, cw_gguf **out);
/* The same over bytes in memory (GgufWeights::parse(bytes)); the bytes are
 * copied, the caller keeps its buffer. */
int cw_gguf_parse(const void *bytes, size_t len, cw_gguf **out);
int cw_gguf_close(cw_gguf *g);
/* Header facts: version, tensor and metadata counts (distinct names), and the
 * byte offset of the data section.  Any pointer may be NULL. */
int cw_gguf_info(const cw_gguf *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_meta,
                 uint64_t *data_offset);
/* Weights::meta_u32 (gguf.rs:165-179): integers truncated to 32 bits, floats
 * converted like Rust's `as u32` (saturating, NaN -> 0), a missing key 0
 * except "*vocab_size", which falls back to token_embd.weight's largest dim. */
int cw_gguf_meta_u32(const cw_gguf *g, const char *key, uint32_t *out);
/* Weights::meta_f32 (gguf.rs:180-186): floats and integers as f32, missing 0. */
int cw_gguf_meta_f32(const cw_gguf *g, const char *key, float *out);
/* A string metadata value (the reference keeps them as Meta::Str without an
 * accessor): copied NUL-terminated into buf (truncated to buf_len-1 bytes),
 * its full length in *len_out.  CW_ERR_FORMAT when absent or not a string. */
int cw_gguf_meta_str(const cw_gguf *g, const char *key, char *buf, size_t buf_len,
                     size_t *len_out);
/* Weights::has (gguf.rs:187-189): 1 when the tensor exists, else 0. */
int cw_gguf_has(const cw_gguf *g, const char *name);
/* Name of tensor `index` in file order (0 <= index < n_tensors). */
int cw_gguf_tensor_name(const cw_gguf *g, uint64_t index, char *buf, size_t buf_len);
/* The tensor table entry: dtype, dims (ne[0] fastest; up to max_dims written),
 * element count, byte offset inside the data section.  Pointers may be NULL. */
int cw_gguf_tensor_info(const cw_gguf *g, const char *name, uint32_t *dtype, int *n_dims,
                        uint64_t *dims, int max_dims, uint64_t *n_elems, uint64_t *offset);
/* tensor_f32 / matrix_raw / vector_data (gguf.rs:109-122, 201-208): decode a
 * tensor to f32 in its stored order ([out][in] for a matrix, no transpose),
 * bit-identical to dequant.rs for F32, F16, Q4_0, Q4_1, Q8_0 and Q6_K.  n must
 * equal the element count.  Unknown dtype: "tensor NAME: ggml dtype D not
 * supported yet"; absent: "missing tensor NAME" (both CW_ERR_FORMAT). */
int cw_gguf_tensor_f32(const cw_gguf *g, const char *name, float *out, size_t n);
/* A projection [out_f][in_f] (ne0 = in_f) as the split Q4_0 image the GEMV
 * reads: scales f16 [out_f][in_f/32], quants [out_f][in_f/32][16].  A Q4_0
 * tensor is repacked block for block (its bytes unchanged); any other dtype is
 * decoded (cw_gguf_tensor_f32) and quantized by cw_q4_quantize, the
 * Proj::load + Q4Linear::from_f32 route (layers.rs:103-116). */
int cw_gguf_tensor_q4(const cw_gguf *g, const char *name, size_t out_f, size_t in_f,
                      uint16_t *scales, uint8_t *quants);
/* The model config from the metadata Qwen3::load reads (qwen3.rs:44-53):
 * qwen3.block_count, .embedding_length, .attention.head_count(_kv),
 * .attention.key_length, .feed_forward_length, .vocab_size (with the
 * meta_u32 fallback), .attention.layer_norm_rms_epsilon, .rope.freq_base;
 * the qwen3 family switches; max_seq and kv_dtype from the caller.  A zero
 * size, or general.architecture naming another family, is CW_ERR_FORMAT. */
int cw_gguf_model_config(const cw_gguf *g, int max_seq, int kv_dtype, cw_model_config *cfg);
/* Qwen3::load's tensor walk (qwen3.rs:56-100) from a GGUF: every layer's
 * projections through cw_gguf_tensor_q4 and norm gains through
 * cw_gguf_tensor_f32, output_norm.weight, token_embd.weight decoded to f32,
 * and output.weight when the file has it (otherwise cw_model_finalize ties
 * the head to the embedding).  Element counts must match the model's config.
 * Call cw_model_finalize afterwards. */
int cw_model_load_gguf(cw_model *m, const cw_gguf *g);

/* ---------------------------------------------------------------- */
/* Profiling (src/profile.rs, GpuContext::begin_profile/report_profile) */
/* ---------------------------------------------------------------- */

/* Start recording a HIP event pair around every launch, labelled by kernel. */
int cw_profile_begin(cw_ctx *ctx);
/* Synchronise, stop recording and write a table "label count total_ms" (one
 * label per line, like profile.rs:121-134) into buf. */
int cw_profile_report(cw_ctx *ctx, char *buf, size_t buf_len);

#ifdef __cplusplus
}
#endif

#endif /* CHAT_WGPU_H */
