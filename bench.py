"""Decode throughput of the Qwen3-8B-shape Q4_0 token loop on one MI355X.

Workload (one step = one greedy decode token): Qwen3-8B shape (hidden 4096,
36 layers, 32/8 heads x 128, intermediate 12288, vocab 151936), Q4_0 linear
weights of seeded synthetic values, tied Q4 LM head, f16 KV cache pre-filled
with 4096 positions of N(0,1), batch 1.  Timed: K decode steps from position
4096 (HIP-graph replay of the device-resident step), inputs resident in HBM.

Prints one JSON line.  Extra fields: the roofline of the dominant kernel
family, the Q4 GEMV (kernel start/end timestamps that the dispatch itself
writes into HIP events, hipExtLaunchKernel, for every launch of 8 eager steps
of the same workload on the library stream), its HBM traffic per launch from
the committed rocprofv3 counter summary, the whole-token byte roofline, the
CPU oracle baseline on a bounded sample, and the Qwen3-0.6B-shape token loop.

  python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
import argparse
import contextlib
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "chat-wgpu_amd"))
import cw  # noqa: E402

HBM_PEAK_GBS = 8000.0
PRE = 4096
DECODE = 256  # the 8B workload: 256 greedy steps from a 4096-position cache


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4_bytes(out_f, in_f):
    return out_f * (in_f // 32) * 18


def cpu_info():
    model = platform.processor() or ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except OSError:
        pass
    return model, os.cpu_count()


def gemv_bytes_per_token(cfg):
    """Algorithmic HBM bytes of one token's Q4 GEMV launches: each weight once
    (18 B per 32), the activation read (K f32) and the output write (N f32),
    plus the residual read of the O and down launches."""
    q, kv, d, h, v = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.dim, \
        cfg.hidden, cfg.vocab
    per_layer = [  # (rows, K, output floats, residual floats)
        (q + 2 * kv, d, q + 2 * kv, 0),  # RMSNorm + q|k|v
        (d, q, d, d),                    # O + residual
        (2 * h, d, h, 0),                # gate|up + SwiGLU
        (d, h, d, d),                    # down + residual
    ]
    total = sum(q4_bytes(n, k) + 4 * k + 4 * o + 4 * r for n, k, o, r in per_layer)
    total = total * cfg.n_layers + q4_bytes(v, d) + 4 * d + 4 * v
    return total


def step_bytes(cfg, seq, es):
    """Algorithmic HBM bytes of one decode step at sequence length seq: every
    Q4 weight once (18 B per 32), the K and V rows of seq positions read and
    one row of each written, the embedding row, the norm gains, the logits."""
    q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    d, h, v, L = cfg.dim, cfg.hidden, cfg.vocab, cfg.n_layers
    w = L * (q4_bytes(q + 2 * kv, d) + q4_bytes(d, q) + q4_bytes(2 * h, d) + q4_bytes(d, h))
    w += q4_bytes(v, d)
    kv_rw = L * (seq + 1) * kv * 2 * es
    small = 4 * d + 4 * (L * (2 * d + 2 * cfg.head_dim) + d) + 4 * v
    return w + kv_rw + small, w


@contextlib.contextmanager
def pinned_core():
    """Run the calling thread (the one-thread oracle runs on it) on one core,
    the lowest this process may use (core 0 when allowed), as `taskset -c 0`
    would; yields that core and restores the previous affinity."""
    old = os.sched_getaffinity(0)
    core = 0 if 0 in old else min(old)
    os.sched_setaffinity(0, {core})
    try:
        yield core
    finally:
        os.sched_setaffinity(0, old)


def cpu_baseline_8b(cfg, weights, k, v, start_tok, budget_s):
    """The CPU oracle (C restatement of the reference forward, single thread
    pinned to one core) on decode tokens from position 4096 until budget_s
    has elapsed.  Returns (tokens/s, tokens, seconds, core)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    orc.set_threads(1)
    o = orc.OracleModel(cfg, weights)
    o.prefill_kv(k, v, PRE)
    with pinned_core() as core:
        tok, n, t0 = int(start_tok), 0, time.perf_counter()
        while True:
            logits, _ = o.step(tok, PRE + n)
            tok = int(np.argmax(logits))
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s or n >= 8:
                break
    o.close()
    return n / el, n, el, core


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 matrix peak


def bench_prefill_8b(ctx, m, cfg, P=512, reps=3):
    """Batched prefill of a P-token prompt (uniform ids) on the 8B model:
    wall time of cw_model_prefill (synchronous), the linear-layer flops
    (2 P sum(N K) over the 36 layers; the LM head runs for the last position
    only) and the causal attention flops, and a per-kernel profile of one
    prefill."""
    prompt = cw.synth_tokens(cw.synth_key(8008, "prefill"), P, cfg.vocab)
    m.prefill(prompt)  # allocates the batched buffers
    ctx.flush()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        m.prefill(prompt)
        ts.append(time.perf_counter() - t0)
    el = min(ts)
    ctx.profile_begin()
    m.prefill(prompt)
    prof = {}
    for name, c, ms in ctx.profile_report():
        prof[name] = prof.get(name, 0.0) + ms
    q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    d, h = cfg.dim, cfg.hidden
    lin = 2.0 * P * cfg.n_layers * ((q + 2 * kv) * d + d * q + 2 * h * d + d * h)
    att = 2.0 * 2.0 * cfg.n_heads * cfg.head_dim * (P * (P + 1) / 2) * cfg.n_layers
    gemm_ms = sum(v for k, v in prof.items() if k.startswith("q4_gemm"))
    return {
        "workload": f"qwen3-8b-shape batched prefill, {P}-token uniform prompt from position 0, "
                    "f16 KV, logits of the last position",
        "tok_s": round(P / el, 1), "ms": round(el * 1e3, 3),
        "linear_tflop": round(lin / 1e12, 3), "attention_gflop": round(att / 1e9, 2),
        "gemm_ms": round(gemm_ms, 3),
        "mfma_util": round(lin / (gemm_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
        "mfma_util_note": "useful linear flops / GEMM kernel time (incl. split-K reduce) / "
                          "2.5 PFLOP/s dense fp16; each 16-wide k slice issues two f16 "
                          "MFMAs (x_hi and x_lo against the exact q - 8, for f32-level "
                          "parity; the block scale goes on each block's f32 sum), so the "
                          "matrix pipes run 2x the useful flops",
        "kernel_ms": {k: round(v, 3) for k, v in prof.items()},
    }


def gemv_profile(prof, n_steps):
    """(ms per token, launches per token) of the q4_gemv labels of a profile."""
    g = [(c, ms) for name, c, ms in prof if name.startswith("q4_gemv")]
    return sum(ms for _, ms in g) / n_steps, sum(c for c, _ in g) / n_steps


def bench_06b(ctx, warm=True):
    """Qwen3-0.6B-shape token loop (32 prompt + 128 greedy, f32 KV, graph
    replay), and the same model's Q4 GEMV launches of one decode token timed
    by kernel timestamps over 8 eager steps (the GEMVs of one 0.6B step)."""
    P, N = 32, 128
    cfg = cw.make_config(28, 1024, 16, 8, 128, 3072, 151936, P + N, cw.CW_F32, 1e-6, 1e6)
    m = cw.Model(ctx, cfg)
    m.load_synthetic(2024)
    m.finalize()
    prompt = cw.synth_tokens(cw.synth_key(2024, "prompt"), P, cfg.vocab)
    if warm:
        m.generate(prompt, N, mode=cw.STEP_GRAPH)
    t0 = time.perf_counter()
    m.generate(prompt, N, mode=cw.STEP_GRAPH)
    el = time.perf_counter() - t0
    NP = 8
    m.reset_state(int(prompt[-1]), P)
    ctx.flush()
    ctx.profile_begin()
    m.decode_async(NP, mode=cw.STEP_EAGER)
    gms, gl = gemv_profile(ctx.profile_report(), NP)
    m.close()
    return (P + N - 1) / el, el, gemv_bytes_per_token(cfg), gms, gl


def bench_single_gemv(ctx, out_f=3072, in_f=1024, pool_bytes=600 << 20, passes=3):
    """One Q4_0 GEMV y[out_f] = W x[in_f] (x ~ N(0,1), d = f16(|N(0,0.02)|),
    uniform nibbles) over a rotating pool of weight copies larger than the
    256 MB last-level cache, so every launch streams its weights from HBM.
    Kernel time from the dispatch's own start/end timestamps; returns
    (us per launch, algorithmic bytes per launch, copies in the pool)."""
    s, q = cw.synth_q4(cw.synth_key(7, "c0.w"), out_f, in_f)
    x = cw.synth_normal_f32(cw.synth_key(7, "c0.x"), in_f)
    wb = s.nbytes + q.nbytes
    n = max(2, pool_bytes // wb)
    sd0, qd0 = ctx.storage(s), ctx.storage(q)
    pool = []
    for _ in range(n):
        sd, qd = ctx.empty(s.shape, np.uint16), ctx.empty(q.shape, np.uint8)
        cw.check(cw.lib().cw_copy(ctx.h, sd.ptr, sd0.ptr, s.nbytes))
        cw.check(cw.lib().cw_copy(ctx.h, qd.ptr, qd0.ptr, q.nbytes))
        pool.append((sd, qd))
    xd, yd = ctx.storage(x), ctx.empty(out_f, np.float32)
    for sd, qd in pool:  # warm
        ctx.q4_gemv(xd, sd, qd, in_f, out_f, y=yd)
    ctx.flush()
    ctx.profile_begin()
    for _ in range(passes):
        for sd, qd in pool:
            ctx.q4_gemv(xd, sd, qd, in_f, out_f, y=yd)
    _, cnt, ms = ctx.profile_report()[0]
    for sd, qd in pool:
        ctx.free(sd)
        ctx.free(qd)
    for d in (sd0, qd0, xd, yd):
        ctx.free(d)
    return ms * 1e3 / cnt, q4_bytes(out_f, in_f) + 4 * in_f + 4 * out_f, n


def small_probe(ctx, passes=3):
    """The small configurations' kernels, for a kernel trace: the 0.6B-shape
    model's 32-token prompt and 8 greedy steps (graph-replayed), 8 eager
    decode steps from the end of the prompt, then `passes` passes of the
    3072x1024 GEMV over the rotating pool of bench_single_gemv (no library
    profiling, so the trace's own timestamps are the only ones taken)."""
    P = 32
    cfg = cw.make_config(28, 1024, 16, 8, 128, 3072, 151936, P + 128, cw.CW_F32, 1e-6, 1e6)
    m = cw.Model(ctx, cfg)
    m.load_synthetic(2024)
    m.finalize()
    prompt = cw.synth_tokens(cw.synth_key(2024, "prompt"), P, cfg.vocab)
    m.generate(prompt, 8, mode=cw.STEP_GRAPH)
    m.reset_state(int(prompt[-1]), P)
    m.decode_async(8, mode=cw.STEP_EAGER)
    ctx.flush()
    m.close()
    log("0.6B steps done")
    out_f, in_f = 3072, 1024
    s, q = cw.synth_q4(cw.synth_key(7, "c0.w"), out_f, in_f)
    x = cw.synth_normal_f32(cw.synth_key(7, "c0.x"), in_f)
    n = max(2, (600 << 20) // (s.nbytes + q.nbytes))
    pool = [(ctx.storage(s), ctx.storage(q)) for _ in range(n)]
    xd, yd = ctx.storage(x), ctx.empty(out_f, np.float32)
    for _ in range(1 + passes):  # the first pass warms
        for sd, qd in pool:
            ctx.q4_gemv(xd, sd, qd, in_f, out_f, y=yd)
    ctx.flush()
    log(f"3072x1024 GEMV: {1 + passes} passes over {n} weight copies done")
    for sd, qd in pool:
        ctx.free(sd)
        ctx.free(qd)
    ctx.free(xd)
    ctx.free(yd)


def bench_read_probe(ctx, nbytes=2 << 30, passes=4):
    """Achievable HBM read bandwidth: the read probe (cw_hbm_read_probe, the
    examples/q4probe.rs analogue) streams one 2 GiB buffer (8x the 256 MB
    last-level cache) with non-temporal 16-byte loads, XOR-folded, at 1 to 16
    workgroups per CU; kernel timestamps.  Returns {workgroups per CU: GB/s}."""
    buf = ctx.empty(nbytes // 4, np.uint32)
    n_cu = ctx.info()["n_cu"]
    out = ctx.empty(16 * n_cu, np.uint32)
    res = {}
    for per_cu in (1, 2, 4, 8, 16):
        blocks = per_cu * n_cu
        ctx.hbm_read_probe(buf, nbytes, blocks, out)  # warm
        ctx.flush()
        ctx.profile_begin()
        for _ in range(passes):
            ctx.hbm_read_probe(buf, nbytes, blocks, out)
        _, cnt, ms = ctx.profile_report()[0]
        res[per_cu] = nbytes / (ms * 1e-3 / cnt) / 1e9
    ctx.free(buf)
    ctx.free(out)
    return res


def cpu_single_gemv(out_f=3072, in_f=1024, budget_s=1.0):
    """The reference's CPU GEMV paths restated in the oracle, one thread: the
    sequential Q4 dequant-dot (src/main.rs:133-150) and naive_matmul at m=1
    on the dequantized f32 weights (examples/bench/src/lib.rs:221-233).
    Returns (us per q4 dot GEMV, us per naive_matmul GEMV)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    orc.set_threads(1)
    s, q = cw.synth_q4(cw.synth_key(7, "c0.w"), out_f, in_f)
    x = cw.synth_normal_f32(cw.synth_key(7, "c0.x"), in_f)
    wt = np.ascontiguousarray(orc.dequant_q4_0_soa(s, q).reshape(out_f, in_f).T)  # B [k, n]

    def timed(fn):
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                return el / n * 1e6
    with pinned_core():
        t_q4 = timed(lambda: orc.q4_gemv(x, s, q, in_f, out_f))
        t_nm = timed(lambda: orc.naive_matmul(x, wt, 1, in_f, out_f))
    return t_q4, t_nm


TRAFFIC_MD = os.path.join(ROOT, "profiles", "q4_gemv_qwen3-8b-decode_hbm-traffic.md")


def committed_gemv_traffic():
    """HBM bytes per Q4 GEMV launch (FETCH_SIZE and WRITE_SIZE, calibrated,
    averaged over one token's launches) from the committed rocprofv3 counter
    summary, or (None, reason) when there is none."""
    try:
        with open(TRAFFIC_MD) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip().replace(",", "")), \
                        "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, " + os.path.relpath(TRAFFIC_MD, ROOT)
    except OSError:
        pass
    return None, "no committed counter summary"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--probe", action="store_true",
                    help="for rocprofv3 --pmc runs: one 256 MiB device-to-device copy (the "
                         "counter calibration), then 4 eager decode steps of the workload; "
                         "prints no JSON")
    ap.add_argument("--graph-probe", type=int, default=0, metavar="N",
                    help="for rocprofv3 kernel traces of the replayed step: 8 + N decode steps "
                         "of the workload, each one graph launch followed by the next (the chat "
                         "loop's pattern); prints no JSON")
    ap.add_argument("--small-probe", action="store_true",
                    help="for rocprofv3 kernel traces of the small configurations: 8 eager decode "
                         "steps of the Qwen3-0.6B-shape model after its 32-token prompt, then "
                         "3 passes of the 3072x1024 GEMV over its rotating weight pool; prints "
                         "no JSON")
    ap.add_argument("--prefill-only", action="store_true",
                    help="for rocprofv3 traces of the batched prefill: build the 8B model and "
                         "print only the 512-token prefill figures (one JSON line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this library runs on one GPU; --gpus must be 1 "
                          "(no multi-GPU path is built)"}))
        sys.exit(2)
    K, W = args.steps, args.warmup

    ctx = cw.Context(0)
    info = ctx.info()
    log(f"device {info}")
    if args.small_probe:
        small_probe(ctx)
        ctx.close()
        return
    cfg = cw.make_config(36, 4096, 32, 8, 128, 12288, 151936, PRE + max(DECODE, K, W, 8) + 1,
                         cw.CW_F16, 1e-6, 1e6)
    t = time.perf_counter()
    weights = cw.synthetic_weights(cfg, 8008)
    log(f"synthetic weights generated in {time.perf_counter() - t:.1f}s")
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    kv_n = cfg.n_layers * PRE * cfg.n_kv_heads * cfg.head_dim
    k = cw.synth_normal_f16(cw.synth_key(8008, "kv.k"), kv_n)
    v = cw.synth_normal_f16(cw.synth_key(8008, "kv.v"), kv_n)
    m.prefill_kv(k, v, PRE)
    start = int(cw.synth_tokens(cw.synth_key(8008, "start"), 1, cfg.vocab)[0])
    log(f"model ready in {time.perf_counter() - t:.1f}s")

    if args.prefill_only:
        print(json.dumps(bench_prefill_8b(ctx, m, cfg)), flush=True)
        m.close()
        ctx.close()
        return

    if args.probe:
        n = 256 << 20
        src, dst = ctx.empty(n, np.uint8), ctx.empty(n, np.uint8)
        cw.check(cw.lib().cw_copy(ctx.h, dst.ptr, src.ptr, n))
        ctx.flush()
        m.reset_state(start, PRE)
        m.decode_async(4, mode=cw.STEP_EAGER)
        ctx.flush()
        log("probe done")
        m.close()
        ctx.close()
        return

    if args.graph_probe:
        m.reset_state(start, PRE)
        for _ in range(8 + args.graph_probe):
            m.decode_async(1, mode=cw.STEP_GRAPH)
        ctx.flush()
        log("graph probe done")
        m.close()
        ctx.close()
        return

    m.reset_state(start, PRE)
    m.decode_async(W, mode=cw.STEP_GRAPH)
    ctx.flush()
    log("warmup done")

    # timed: K decode steps of the 256-step workload, the step replayed as a
    # HIP graph.  Fewer than 256 timed steps sit at the middle of the
    # workload (the steps before them run untimed first), so the timed
    # window's mean cache length is the workload's own.
    skip = max(0, (DECODE - K) // 2)
    t0pos = PRE + skip
    m.reset_state(start, PRE)
    if skip:
        m.decode_async(skip, mode=cw.STEP_GRAPH)
    ctx.flush()
    t0 = time.perf_counter()
    m.decode_async(K, mode=cw.STEP_GRAPH)
    ctx.flush()
    el = time.perf_counter() - t0
    toks = m.tokens(K)
    tok_s = K / el
    log(f"timed {K} steps in {el * 1e3:.2f} ms -> {tok_s:.1f} tok/s; first tokens {toks[:8]}")

    # roofline of the dominant kernel family (the Q4 GEMVs): every launch of NP
    # eager steps of the same workload carries a start/stop event pair that
    # its dispatch stamps with the kernel's own start and end times
    NP = 8
    m.reset_state(start, PRE)
    ctx.flush()
    ctx.profile_begin()
    m.decode_async(NP, mode=cw.STEP_EAGER)
    prof = {name: (count / NP, ms / NP) for name, count, ms in ctx.profile_report()}
    gemv = {n: v for n, v in prof.items() if n.startswith("q4_gemv")}
    gemv_ms = sum(ms for _, ms in gemv.values())
    gemv_launches = sum(c for c, _ in gemv.values())
    gbytes = gemv_bytes_per_token(cfg)
    achieved = gbytes / (gemv_ms * 1e-3) / 1e9
    kernel_ms = sum(ms for _, ms in prof.values())
    log("per-token kernel ms (eager, kernel timestamps): " +
        ", ".join(f"{n}={ms:.3f}" for n, (_, ms) in prof.items()))
    traffic, traffic_src = committed_gemv_traffic()
    bytes_avg = sum(step_bytes(cfg, t0pos + i + 1, 2)[0] for i in range(K)) / K

    result = {
        "metric": "decode tokens/s (Qwen3-0.6B/8B Q4_0, 1 GPU); Q4 GEMV HBM GB/s vs peak",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(el * 1e3 / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q4_0 weights, N(0,1) f16 KV pre-fill)",
        "config": {"workload": f"qwen3-8b-shape q4_0 greedy decode, batch 1, f16 KV prefilled "
                               f"to {PRE}, {DECODE}-step decode; timed steps {skip}..{skip + K - 1} "
                               f"(KV {t0pos + 1}->{t0pos + K}), step replayed as a HIP graph",
                   "weights": "q4_0", "hidden": 4096, "layers": 36, "heads": "32/8x128",
                   "intermediate": 12288, "vocab": 151936, "kv_prefill": PRE,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": "q4_gemv_kernel (all 4 fused variants; 4 launches per layer "
                               "+ the LM head)",
                     "algorithmic_bytes_per_token": gbytes,
                     "avg_bytes_per_launch": round(gbytes / gemv_launches),
                     "avg_launch_us": round(gemv_ms * 1e3 / gemv_launches, 2),
                     "launches_per_token": gemv_launches},
        "kernel_us_per_launch": {n: round(ms * 1e3 / c, 2) for n, (c, ms) in prof.items()},
        "token_roofline": {"algorithmic_bytes_per_token": round(bytes_avg),
                           "ideal_ms_at_peak": round(bytes_avg / (HBM_PEAK_GBS * 1e6), 4),
                           "kernel_ms_per_token_eager": round(kernel_ms, 4),
                           "frac_of_peak": round(bytes_avg / (el / K) / 1e9 / HBM_PEAK_GBS, 4)},
        "extras": {},
    }

    if not args.no_cpu_baseline:
        log("cpu baseline (oracle, 1 thread) ...")
        tps, n, cel, core = cpu_baseline_8b(cfg, weights, k, v, start, args.cpu_budget)
        model_name, ncpu = cpu_info()
        result["cpu_baseline"] = {"value": round(tps, 5), "unit": "tokens/s", "cores": 1,
                                  "kind": "port",
                                  "sample": f"{n} decode tokens of the same 8B workload from "
                                            f"position 4096 on the C oracle ({cel:.1f}s), one "
                                            f"thread pinned to cpu {core}; host {model_name}, "
                                            f"{ncpu} cpus"}
    del weights
    if not args.no_extras:
        log("prefill (512 tokens, batched) ...")
        result["extras"]["qwen3_8b_prefill_512"] = bench_prefill_8b(ctx, m, cfg)
    m.close()

    if not args.no_extras:
        tps06, el06, gb06, gms06, gl06 = bench_06b(ctx)
        ex = result["extras"]
        ex["qwen3_0.6b_token_loop_tok_s"] = round(tps06, 1)
        ex["qwen3_0.6b_token_loop"] = ("32 prompt + 128 greedy, f32 KV, 159 forwards incl. "
                                       "prompt, HIP graph")
        ex["qwen3_0.6b_step_gemvs"] = {
            "workload": "one Qwen3-0.6B-shape decode step's Q4_0 GEMVs (28 layers x "
                        "QKV, O, gate/up, down + LM head 1024->151936), kernel timestamps "
                        "over 8 eager steps",
            "algorithmic_bytes": gb06, "launches": gl06, "us": round(gms06 * 1e3, 2),
            "GB_s": round(gb06 / (gms06 * 1e-3) / 1e9, 1),
            "frac_of_peak": round(gb06 / (gms06 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        rp = bench_read_probe(ctx)
        best = max(rp.values())
        ex["hbm_read_probe"] = {
            "workload": "XOR-fold of a 2 GiB device buffer with non-temporal 16-byte loads (the reference's "
                        "q4probe read sweep), kernel timestamps; GB/s by workgroups per CU",
            "GB_s_by_wg_per_cu": {str(k): round(v, 1) for k, v in rp.items()},
            "best_GB_s": round(best, 1), "best_frac_of_peak": round(best / HBM_PEAK_GBS, 4),
            "q4_gemv_frac_of_achievable": round(achieved / best, 4)}
        us1, b1, n1 = bench_single_gemv(ctx)
        ex["single_q4_gemv_3072x1024"] = {
            "workload": f"y[3072] = W x[1024], Q4_0, rotating pool of {n1} weight copies "
                        "(> the 256 MB last-level cache), kernel timestamps",
            "algorithmic_bytes": b1, "us_per_launch": round(us1, 3),
            "GB_s": round(b1 / (us1 * 1e-6) / 1e9, 1),
            "frac_of_peak": round(b1 / (us1 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if not args.no_cpu_baseline:
            t_q4, t_nm = cpu_single_gemv()
            ex["single_q4_gemv_3072x1024"]["cpu_baseline"] = {
                "q4_dot_us": round(t_q4, 1), "naive_matmul_us": round(t_nm, 1), "cores": 1,
                "kind": "port",
                "sample": "the reference's sequential Q4 dequant-dot (main.rs:133-150) and "
                          "naive_matmul at m=1 on the dequantized weights "
                          "(examples/bench/src/lib.rs:221-233), C restatement, 1 thread "
                          "pinned to one core, repeated for 1 s each"}
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
