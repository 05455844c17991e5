"""Benchmark of the speculative verify step on one MI355X.

Workload (the configuration the metric is quoted on): Qwen2.5-0.5B shape (24 layers, hidden 896,
14 heads / 2 KV heads, FFN 4864, vocab 151936, tied), random-init N(0, 0.02) weights (seed 1)
quantized to int8 with groups of 64 and clip search by the engine's restatement of quant.rs;
a prompt of 512 uniform random ids is prefilled, then speculative decoding with k=8 chain
drafts from a scripted drafter that proposes the target's greedy token with probability 0.6.
A step is one fused verify pass (forward over k+1 rows, argmax, acceptance, rollback). W warmup
steps, then exactly K timed steps. value = verified tokens (m+1 per step) / wall time.

Usage: python bench.py [--gpus 1] [--steps 96] [--warmup 4] [--cpu-steps 24] [--no-cpu]
       python bench.py --calibrate-copy MIB   (one device-to-device copy of MIB MiB, repeated: the
                                               known-size kernel that scales HBM counter readings)
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "verified tok/s & verify-step latency at 1 GPU; % HBM roofline"
HBM_PEAK_GBS = 8000.0
GREEDY_REF = 400  # tokens of the target's greedy continuation that script the drafter
ROOF_STEPS = 24  # verify steps timed per launch for the roofline figure


def hip_sync():
    h = C.CDLL("libamdhip64.so")
    if h.hipDeviceSynchronize() != 0:
        raise RuntimeError("hipDeviceSynchronize failed")


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "k_mm_qwen05b_int8_verify_hbm_traffic.md")


def measured_traffic():
    """HBM bytes per matrix launch from the committed rocprofv3 --pmc summary (FETCH_SIZE and
    WRITE_SIZE runs of this workload, scaled by a copy of known size), or None."""
    import re

    try:
        with open(TRAFFIC_PROFILE) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read(), re.M)
        return int(m.group(1)) if m else None
    except OSError:
        return None


def calibrate_copy(mib, reps=8):
    """Plain device-to-device copies of a known size, for scaling FETCH_SIZE / WRITE_SIZE."""
    h = C.CDLL("libamdhip64.so")
    n = mib << 20
    a, b = C.c_void_p(), C.c_void_p()
    if h.hipMalloc(C.byref(a), C.c_size_t(n)) or h.hipMalloc(C.byref(b), C.c_size_t(n)):
        raise RuntimeError("hipMalloc failed")
    h.hipMemset(a, 1, C.c_size_t(n))
    for _ in range(reps):
        if h.hipMemcpy(b, a, C.c_size_t(n), 3):  # hipMemcpyDeviceToDevice
            raise RuntimeError("hipMemcpy failed")
    hip_sync()
    h.hipFree(a)
    h.hipFree(b)
    print(json.dumps({"calibration": "device-to-device copy", "bytes_read": n, "bytes_written": n, "reps": reps}), flush=True)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def step_bytes(cfg, layer_bytes, row_bytes, ctx, t):
    """Algorithmic HBM bytes of one verify step: every layer block, the whole tied head, t
    embedding rows, and the f32 K/V cache read once plus the t new rows written."""
    L, kv = cfg["layers"], cfg["kv_heads"] * cfg["head_dim"]
    return L * layer_bytes + cfg["vocab"] * row_bytes + t * row_bytes + 2 * L * kv * 4 * (ctx + t)


def build_workload(seed=1, fmt=(8, 64), threads=0):
    import layerstream_amd as LS

    text = LS.qwen2_config_text(**LS.QWEN2_05B)
    t0 = time.time()
    m = LS.synth_bf16_model(text, seed, threads=threads)
    img = LS.quantize_model(text, m["layers"], m["embed"], m["norm"], fmt, clip=True, threads=threads)
    log(f"workload: synth + quantize {time.time() - t0:.1f}s, image {img.nbytes / 2**20:.1f} MiB")
    return text, img


def cpu_baseline(img, cfg, qtext, prompt, drafter_g, p_accept, seed, k, n_steps, gpu_m):
    """The oracle (C restatement of the reference CPU path) on the host's cores: the same prompt
    prefilled, then n_steps verify passes with the same drafts. Returns the JSON object."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_py as O
    import tinymodels as T
    import layerstream_amd as LS

    parts = T.split_lsq(img.tobytes(), {"layers": cfg["layers"]})
    ocfg = {kk: cfg[kk] for kk in ("format", "embed_format", "hidden", "inter", "layers", "heads", "kv_heads", "head_dim", "vocab", "eps", "rope_theta")}
    cores = len(os.sched_getaffinity(0))
    om = O.OracleModel(ocfg, parts["layers"], parts["embed"], parts["norm"], threads=cores, max_ctx=len(prompt) + 16 * (n_steps + 2))
    d = LS.ScriptedDrafter(drafter_g, p_accept, seed, cfg["vocab"])
    t0 = time.time()
    a = int(np.argmax(om.forward(prompt)))
    t_prefill = time.time() - t0
    n_out, toks, ms_list, ms_acc = 1, 0, [], []
    for _ in range(n_steps):
        drafts = [d.token(n_out + i) for i in range(k)]
        block = [a] + drafts
        p = om.pos()
        t1 = time.perf_counter()
        logits = om.forward_multi(block, k + 1)
        am = logits.argmax(1)
        m = 0
        while m < k and am[m] == drafts[m]:
            m += 1
        om.truncate(p + m + 1)
        ms_list.append(time.perf_counter() - t1)
        ms_acc.append(m)
        a = int(am[m])
        n_out += m + 1
        toks += m + 1
    d.close()
    om.close()
    secs = sum(ms_list)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except Exception:
        pass
    return {
        "value": toks / secs,
        "unit": "verified tok/s",
        "cores": cores,
        "kind": "port",
        "sample": f"prefill {len(prompt)} tokens (untimed, {t_prefill:.1f}s), then {n_steps} verify steps of k={k} with the same drafts; "
        f"C restatement of the reference CPU path (Rust toolchain unavailable), -O3 -ffp-contract=off, {cores} threads; {cpu_model}",
        "verify_ms_p50": float(np.median(ms_list) * 1e3),
        "accepted_match_gpu": ms_acc == list(gpu_m[: len(ms_acc)]),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=96)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--k", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=512)
    ap.add_argument("--p-accept", type=float, default=0.6)
    ap.add_argument("--cpu-steps", type=int, default=24)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--mode", choices=["resident", "stream"], default="resident")
    ap.add_argument("--no-graphs", action="store_true", help="launch each kernel of a verify step separately (for tracers)")
    ap.add_argument("--greedy-ref", type=int, default=GREEDY_REF, help="tokens of greedy continuation scripting the drafter")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}, WORLD_SIZE {world}).", file=sys.stderr)
        sys.exit(2)

    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return

    import layerstream_amd as LS

    qfmt = (8, 64)
    text, img = build_workload(fmt=qfmt)
    src = LS.Source.from_lsq_image(img)
    if args.mode == "stream":
        src = src.pinned_copy()
    cfg = src.config()
    qtext = LS.inject_quant(text, *qfmt)
    _, layer_bytes = LS.layer_layout(qtext)
    row_bytes = LS.row_bytes(cfg["embed_format"], cfg["hidden"])
    k, W, K = args.k, args.warmup, args.steps
    max_new = 9 * (W + K + ROOF_STEPS) + 2
    max_ctx = args.ctx + max(max_new, args.greedy_ref) + k + 8
    rng = np.random.default_rng(512)
    prompt = rng.integers(0, cfg["vocab"], args.ctx).tolist()

    t0 = time.time()
    model = LS.Model(src, LS.MODE_STREAM if args.mode == "stream" else LS.MODE_RESIDENT, 2, max_ctx)
    log(f"model load {time.time() - t0:.1f}s")
    if args.no_graphs:
        model.use_graphs(False)
    # The drafter's script: the target's own greedy continuation.
    t0 = time.time()
    g = LS.greedy_generate(model, prompt, args.greedy_ref) if args.greedy_ref > 0 else []
    model.reset()
    log(f"greedy reference {len(g)} tokens in {time.time() - t0:.1f}s")
    seed = 2024
    drafter = LS.ScriptedDrafter(g, args.p_accept, seed, cfg["vocab"])
    run = LS.SpecRun(model, drafter, prompt, max_new, k)
    run.step(W)
    hip_sync()
    t0 = time.perf_counter()
    run.step(K)
    hip_sync()
    wall = time.perf_counter() - t0
    # Per-launch timing of the matrix kernels: HIP events on the compute stream around every
    # launch, over ROOF_STEPS further verify steps of the same run (kept out of the timed steps,
    # whose launches they would space out).
    model.profile(True)
    run.step(ROOF_STEPS)
    hip_sync()
    prof = model.profile_read()
    model.profile(False)
    ms, m = run.step_log()
    tm, tms = m[W : W + K], ms[W : W + K]
    toks = int(np.sum(tm + 1))
    value = toks / wall
    out_tokens = run.tokens()
    n_cmp = min(len(out_tokens), len(g))
    match = out_tokens[:n_cmp] == g[:n_cmp]
    ctx0 = args.ctx + 1 + int(np.sum(m[:W] + 1))
    ctx_mean = ctx0 + float(np.mean(np.cumsum(tm + 1) - (tm + 1)))
    sb = step_bytes(cfg, layer_bytes, row_bytes, ctx_mean, k + 1)
    step_ms_p50 = float(np.median(tms))

    avg_ms = prof["ms"] / max(prof["launches"], 1)
    avg_bytes = prof["bytes"] / max(prof["launches"], 1)
    achieved = avg_bytes / (avg_ms * 1e-3) / 1e9 if avg_ms > 0 else 0.0
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": measured_traffic(),
        "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT),
        "kernel": "k_mm (fused MFMA weight-streaming matmul: q|k|v, o, gate|up, down, head; int8, t=9)",
        "measured_over": f"{ROOF_STEPS} verify steps after the timed ones, start/stop events recorded by each dispatch (hipExtLaunchKernel)",
        "launches": int(prof["launches"]),
        "avg_launch_us": round(avg_ms * 1e3, 3),
        "avg_bytes_per_launch": round(avg_bytes),
    }
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "verified tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall / K * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Qwen2.5-0.5B-shape int8-g64 (clip search), random-init N(0,0.02) seed 1; prompt 512 random ids; k=8 chain drafts, scripted 60% per-token acceptance; greedy verify",
            "mode": args.mode,
            "k": k,
            "ctx_start": ctx0,
            "ctx_mean": round(ctx_mean, 1),
            "graphs": not args.no_graphs,
        },
        "verify_ms_p50": round(step_ms_p50, 4),
        "verify_ms_p90": round(float(np.percentile(tms, 90)), 4),
        "tokens_per_step": round(toks / K, 3),
        "acceptance": round(float(np.sum(tm)) / (K * k), 4),
        "step_algorithmic_bytes": int(sb),
        "step_hbm_frac": round(sb / (step_ms_p50 * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
        "tokens_match_greedy": bool(match),
        "roofline": roofline,
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        t0 = time.time()
        res["cpu_baseline"] = cpu_baseline(img, cfg, qtext, prompt, g, args.p_accept, seed, k, args.cpu_steps, list(m))
        log(f"cpu baseline {time.time() - t0:.1f}s")
    run.close()
    drafter.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
