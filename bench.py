#!/usr/bin/env python3
"""Decode benchmark of the MI355X pocketinfer backend (one GPU).

Workload: greedy decode of the synthetic MiniCPM-2B-shaped Q4_K_M model
(40 layers, hidden 2304, 36x64 MHA, FFN 5760, vocab 122753; Q4_K with a Q6_K
head, Q6_K attn_v and Q8_0 ffn_down in even layers, Q4_0 ffn_down in odd
ones; f32 KV), prompt of 128 random ids, 256 greedy tokens at batch 1.
A step is one decode forward (embedding, 40 layers, head, argmax).

metric: decode tok/s = gen_tokens / gen_ms as the reference defines it
(model.rs:1297-1350, PerfLog.kt:43): n tokens take n-1 forwards.

Also measured here:
  roofline  -- the Q4_K GEMV kernel at 5760x2304 (one launch = 7 497 216
               algorithmic bytes: weights + f32 x + f32 y), timed with HIP events
               on its stream while rotating 70 weight copies (522 MB, twice the
               256 MB Infinity Cache) so the reads come from HBM;
  q6k_head  -- the Q6_K head GEMV at 122753x2304 (232 503 398 B per launch);
  cpu_baseline -- the CPU oracle's decode tok/s on a bounded sample (32-id
               prompt, 9 greedy tokens) with every host thread.

  prefill  -- the 2048-token prompt of the same model on the batched int8-MFMA
               prefill kernels (64 chunks of 32), then the prompt extended by
               512 tokens reusing the 2048 cached positions;
  long_context -- decode at 4096 and 16384 positions of N(0,1) KV
               (737 280 KV bytes per position on top of the weights).

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
       python bench.py --profile-gemv   (GEMV launches and a 256 MiB device
                                         copy only, for counter runs)
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path[:0] = [str(REPO), str(REPO / "pocket-workbench-android_amd")]

import pocketinfer_hip as pih  # noqa: E402

HBM_PEAK_GBS = 8000.0
Q4K_ROWS, Q4K_K = 5760, 2304
Q4K_LAUNCH_BYTES = Q4K_ROWS * (Q4K_K // 256) * 144 + Q4K_K * 4 + Q4K_ROWS * 4     # 7 497 216
Q6K_ROWS, Q6K_K = 122753, 2304
Q6K_LAUNCH_BYTES = Q6K_ROWS * (Q6K_K // 256) * 210 + Q6K_K * 4 + Q6K_ROWS * 4     # 232 503 398
MODEL_SEED, PROMPT_SEED, N_PROMPT = 1234, 77, 128
# HBM bytes per Q4_K GEMV launch from rocprofv3 FETCH_SIZE / WRITE_SIZE, each
# scaled by what the counter reads for a 256 MiB copy (read x1.9997, write x1.0):
# profiles/gemv_q4k_5760x2304_traffic.md
Q4K_TRAFFIC_BYTES = round((3714.5 * 1.9997 + 25.7 * 1.0) * 1024)


def splitmix_ids(seed: int, n: int, vocab: int) -> list:
    out, s = [], (seed + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        z ^= z >> 31
        out.append(z % vocab)
    return out


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_gemv(b, t, rows, k, gen, copies, iters):
    w = gen(1, rows, k)
    ws = [b.upload(t, w, rows, k) for _ in range(copies)]
    x = pih.synth_normal(2, k)
    xd, yd = b.to_device(x), b.alloc(rows * 4)
    qd, dd, sd = b.alloc(k), b.alloc(k // 32 * 4), b.alloc(k // 32 * 4)
    b.q8_quantize_dev(xd.ptr, k, 1, qd.ptr, dd.ptr, sd.ptr)
    b.time_gemv(ws, qd.ptr, dd.ptr, sd.ptr, yd.ptr, max(copies, 8))          # warm
    us = b.time_gemv(ws, qd.ptr, dd.ptr, sd.ptr, yd.ptr, iters)
    for wt in ws:
        wt.free()
    return us


def bench_prefill(b, model, spec):
    """2048-token prompt, then +512 tokens with prefix reuse (model.rs:1258-1268)."""
    ids = splitmix_ids(91, 2048 + 512, spec.n_vocab)
    eng = pih.HipEngine(b, model, n_ctx=2048 + 512 + 16)
    eng.generate(ids[:96], 1)                       # first launches of every prefill kernel
    eng.forward([ids[0]], [0], want_logits=False)   # a manual forward drops the reusable prefix
    _, sa = eng.generate(ids[:2048], 1)
    _, sb = eng.generate(ids, 1)
    return {"prompt_tokens": 2048, "prefill_ms": round(sa["prefill_ms"], 2),
            "tok_s": round(2048 / (sa["prefill_ms"] / 1000.0), 1), "chunk_tokens": 32,
            "extension": {"new_tokens": sb["prefill_tokens"], "reused_tokens": sb["prefill_cached_tokens"],
                          "prefill_ms": round(sb["prefill_ms"], 2),
                          "tok_s": round(sb["prefill_tokens"] / (sb["prefill_ms"] / 1000.0), 1)}}


def bench_long_context(b, model, n_fill, steps, wbytes):
    """Decode after N(0,1) K/V for positions 0..n_fill-1 (seed 4242)."""
    eng = pih.HipEngine(b, model, n_ctx=n_fill + steps + 16)
    eng.kv_fill_normal(n_fill, 4242)
    eng.kv_set_tokens([0] * n_fill)
    _, st = eng.generate([0] * n_fill + [17], steps + 1)   # reuses n_fill, evaluates token 17, then decodes
    tps = st["gen_tokens"] / (st["gen_ms"] / 1000.0)
    kv_bytes = 737280 * (n_fill + steps // 2)
    per_tok = wbytes + kv_bytes
    return {"context": n_fill, "tok_s": round(tps, 2), "gen_tokens": st["gen_tokens"],
            "device_us_per_forward": round(eng.last_decode_us(), 1), "reused": st["prefill_cached_tokens"],
            "bytes_per_token": per_tok, "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / per_tok, 1),
            "frac": round(tps * per_tok / (HBM_PEAK_GBS * 1e9), 4)}


def profile_gemv(b):
    """Q4_K GEMV launches over 70 weight copies and one 256 MiB device copy:
    a short program for rocprofv3 counter runs (FETCH_SIZE / WRITE_SIZE)."""
    us = time_gemv(b, pih.Q4_K, Q4K_ROWS, Q4K_K, pih.synth_q4k_random, 70, 210)
    n = 256 << 20
    src, dst = b.alloc(n), b.alloc(n)
    b.copy_d2d(dst, src, n)
    b.synchronize()
    print(json.dumps({"profile": "gemv", "q4k_us_per_launch": round(us, 3), "copy_bytes": n}), flush=True)


def cpu_baseline(model, prompt):
    from oracle import oracle
    threads = min(os.cpu_count() or 1, 16)
    eng = oracle.OracleEngine(model, n_ctx=64, threads=threads)
    ids, st = eng.generate(prompt[:32], 9)
    eng.close()
    tps = st["gen_tokens"] / (st["gen_ms"] / 1000.0)
    return {"value": round(tps, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"oracle greedy decode of the same model: 32-id prompt, {st['gen_tokens']} tokens "
                      f"({st['gen_tokens'] - 1} forwards, {st['gen_ms']:.0f} ms); prefill {st['prefill_ms']:.0f} ms"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=255, help="timed decode forwards (tokens = steps + 1)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graphs", action="store_true", help="launch kernels one by one (for profilers)")
    ap.add_argument("--no-extra", action="store_true", help="skip the prefill and long-context sections")
    ap.add_argument("--profile-gemv", action="store_true", help="GEMV launches and a device copy only")
    ap.add_argument("--no-gemv", action="store_true", help="skip the standalone GEMV measurements")
    ap.add_argument("--skip", default="", help="comma list of sections to leave out: gemv,decode,prefill,long,cpu")
    args = ap.parse_args()
    skip = set(x for x in args.skip.split(",") if x)
    args.no_gemv |= "gemv" in skip
    args.no_cpu_baseline |= "cpu" in skip
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on one MI355X only: multi-GPU runs are not part of this build "
              "(the sharding plan is described in DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    t_start = time.time()
    b = pih.HipBackend(0)
    b.use_graphs(not args.no_graphs)
    log(f"device: {b.name()}")
    if args.profile_gemv:
        profile_gemv(b)
        return

    # -- roofline: dominant kernel, config-1 shape, HBM-cold -----------------
    q4k_us = q6k_us = float("nan")
    if not args.no_gemv:
        q4k_us = time_gemv(b, pih.Q4_K, Q4K_ROWS, Q4K_K, pih.synth_q4k_random, 70, 700)
        q6k_us = time_gemv(b, pih.Q6_K, Q6K_ROWS, Q6K_K, pih.synth_q6k_random, 3, 30)
    q4k_gbs = Q4K_LAUNCH_BYTES / (q4k_us * 1e-6) / 1e9
    log(f"Q4_K GEMV {Q4K_ROWS}x{Q4K_K}: {q4k_us:.2f} us/launch, {q4k_gbs:.0f} GB/s")
    q6k_gbs = Q6K_LAUNCH_BYTES / (q6k_us * 1e-6) / 1e9
    log(f"Q6_K GEMV {Q6K_ROWS}x{Q6K_K}: {q6k_us:.2f} us/launch, {q6k_gbs:.0f} GB/s")

    # -- decode ------------------------------------------------------------
    spec = pih.minicpm2b_spec()
    t0 = time.time()
    model = pih.synth_model(spec, MODEL_SEED)
    log(f"model synthesized in {time.time() - t0:.1f}s; {model.weight_bytes_per_token()} weight bytes/token")
    prompt = splitmix_ids(PROMPT_SEED, N_PROMPT, spec.n_vocab)
    n_tokens = args.steps + 1
    if "decode" in skip:
        ids, st = [], {"gen_tokens": 1, "gen_ms": float("nan"), "stop": "skipped", "prefill_ms": 0.0,
                       "prefill_cached_tokens": 0}
        eng = None
    else:
        eng = pih.HipEngine(b, model, n_ctx=N_PROMPT + max(n_tokens, args.warmup + 1) + 8)
        eng.generate(prompt, args.warmup + 1)
        b.synchronize()
        ids, st = eng.generate(prompt, n_tokens)
        b.synchronize()
    fwd = max(st["gen_tokens"] - 1, 1)
    tps = st["gen_tokens"] / (st["gen_ms"] / 1000.0)
    dev_us = eng.last_decode_us() if eng else float("nan")
    wbytes = model.weight_bytes_per_token()
    log(f"decode: {st['gen_tokens']} tokens in {st['gen_ms']:.1f} ms ({tps:.1f} tok/s), "
        f"device {dev_us:.1f} us/forward, stop={st['stop']}, prefill {st['prefill_ms']:.1f} ms "
        f"({st['prefill_cached_tokens']} reused)")
    golden = REPO / "tests" / "golden" / "minicpm2b_greedy.json"
    match = None
    if golden.exists():
        g = json.loads(golden.read_text())
        if g["prompt"] == prompt and g["model_seed"] == MODEL_SEED and len(ids) >= g["n_gen"]:
            match = ids[: g["n_gen"]] == g["gen_ids"]

    prefill = long_ctx = None
    if not args.no_extra and "prefill" not in skip:
        prefill = bench_prefill(b, model, spec)
        log(f"prefill: {prefill}")
    if not args.no_extra and "long" not in skip:
        long_ctx = [bench_long_context(b, model, n, 16, wbytes) for n in (4096, 16384)]
        log(f"long context: {long_ctx}")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(model, prompt)
        log(f"cpu baseline: {cpu}")

    out = {
        "metric": "decode tok/s, 2B Q4_K_M synthetic",
        "value": round(tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": fwd,
        "warmup": args.warmup,
        "ms_per_step": round(st["gen_ms"] / fwd, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot / f32",
        "data": "synthetic (seeded random weights N(0,0.02) quantized Q4_K_M-style, random prompt ids)",
        "config": {"workload": "greedy decode, MiniCPM-2B-shaped Q4_K_M synthetic model: 40 layers, "
                               "hidden 2304, 36x64 MHA, FFN 5760, vocab 122753, f32 KV",
                   "prompt_tokens": N_PROMPT, "gen_tokens": st["gen_tokens"], "batch": 1},
        "roofline": {"bound": "hbm", "achieved": round(q4k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(q4k_gbs / HBM_PEAK_GBS, 4), "traffic": Q4K_TRAFFIC_BYTES,
                     "kernel": "Q4_K GEMV 5760x2304 (k_gemv<12,1,0>)", "us_per_launch": round(q4k_us, 3),
                     "bytes_per_launch": Q4K_LAUNCH_BYTES},
        "q6k_head_gemv": {"achieved": round(q6k_gbs, 1), "unit": "GB/s", "frac": round(q6k_gbs / HBM_PEAK_GBS, 4),
                          "us_per_launch": round(q6k_us, 3), "bytes_per_launch": Q6K_LAUNCH_BYTES},
        "decode_weight_roofline": {"weight_bytes_per_token": wbytes,
                                   "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / wbytes, 1),
                                   "frac": round(tps * wbytes / (HBM_PEAK_GBS * 1e9), 4),
                                   "device_us_per_forward": round(dev_us, 2)},
        "greedy_first_64_match_oracle": match,
        "prefill": prefill,
        "long_context": long_ctx,
        "cpu_baseline": cpu,
        "wall_s": round(time.time() - t_start, 1),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
