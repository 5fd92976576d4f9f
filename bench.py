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


def cpu_baseline_8b(cfg, weights, k, v, start_tok, budget_s):
    """The CPU oracle (C restatement of the reference forward, single thread)
    on decode tokens from position 4096 until budget_s has elapsed."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    orc.set_threads(1)
    o = orc.OracleModel(cfg, weights)
    o.prefill_kv(k, v, PRE)
    tok, n, t0 = int(start_tok), 0, time.perf_counter()
    while True:
        logits, _ = o.step(tok, PRE + n)
        tok = int(np.argmax(logits))
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 8:
            break
    o.close()
    return n / el, n, el


def bench_06b(ctx, warm=True):
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
    m.close()
    return (P + N - 1) / el, el


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
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                          "(no multi-GPU path is built)"}))
        sys.exit(2)
    K, W = args.steps, args.warmup

    ctx = cw.Context(0)
    info = ctx.info()
    log(f"device {info}")
    cfg = cw.make_config(36, 4096, 32, 8, 128, 12288, 151936, PRE + max(K, W, 8) + 1, cw.CW_F16,
                         1e-6, 1e6)
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

    m.reset_state(start, PRE)
    m.decode_async(W, mode=cw.STEP_GRAPH)
    ctx.flush()
    log("warmup done")

    # timed: K decode steps from position PRE, the step replayed as a HIP graph
    m.reset_state(start, PRE)
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
    bytes_avg = sum(step_bytes(cfg, PRE + i + 1, 2)[0] for i in range(K)) / K

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
        "config": {"workload": "qwen3-8b-shape q4_0 greedy decode, batch 1, KV 4096->"
                               f"{PRE + K} f16, {K} steps, step replayed as a HIP graph",
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
        tps, n, cel = cpu_baseline_8b(cfg, weights, k, v, start, args.cpu_budget)
        model_name, ncpu = cpu_info()
        result["cpu_baseline"] = {"value": round(tps, 5), "unit": "tokens/s", "cores": 1,
                                  "kind": "port",
                                  "sample": f"{n} decode tokens of the same 8B workload from "
                                            f"position 4096 on the C oracle ({cel:.1f}s); "
                                            f"host {model_name}, {ncpu} cpus"}
    del weights
    m.close()

    if not args.no_extras:
        tps06, el06 = bench_06b(ctx)
        result["extras"]["qwen3_0.6b_token_loop_tok_s"] = round(tps06, 1)
        result["extras"]["qwen3_0.6b_token_loop"] = ("32 prompt + 128 greedy, f32 KV, 159 "
                                                     "forwards incl. prompt, HIP graph")
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
