#!/usr/bin/env python3
"""Decode benchmark of the MI355X pocketinfer backend (one GPU).

Workload (one step): the full greedy decode of the synthetic MiniCPM-2B-shaped
Q4_K_M model (40 layers, hidden 2304, 36x64 MHA, FFN 5760, vocab 122753; Q4_K
with a Q6_K head, Q6_K attn_v and Q8_0 ffn_down in even layers, Q4_0 ffn_down
in odd ones; f32 KV): a prompt of 128 random ids, then 256 greedy tokens at
batch 1 (255 decode forwards).  `--steps K` times K such decodes, `--warmup W`
runs W untimed ones first; the decode length never changes.

metric: decode tok/s = gen_tokens / gen_ms as the reference defines it
(model.rs:1297-1350, PerfLog.kt:43): n tokens take n-1 forwards.

Also measured here:
  roofline   -- the persistent decode kernel k_mega (one launch = one decode
                forward): algorithmic bytes per launch = every weight byte of a
                token (1 766 384 226 B) + the KV rows attention reads and
                writes (737 280 B per position, positions 0..p for the
                forward at position p; mean over the 255 forwards) + one
                embedding row, over the mean device time of a launch, timed
                with an event pair around every launch of the timed decodes;
  gemv_q4k / gemv_q6k -- the standalone GEMVs of configs 1 and 2 with their
                Q8 pass (the whole pi_hip_gemv_dev job) and without it,
                rotating weight copies (twice the 256 MB Infinity Cache) so
                the reads come from HBM; gemv_q5k_f32_path -- the same
                5760 x 2304 shape in Q5_K on the reference's f32 path;
  prefill    -- the 2048-token prompt on the batched int8-MFMA prefill
                kernels (64 chunks of 32), then the prompt extended by 512
                tokens reusing the 2048 cached positions; int8_mfma gives
                the projections' useful int8 operations over the prefill time;
  long_context -- 64 greedy tokens after 4096 and 16384 positions of N(0,1) KV;
  cpu_baseline -- the CPU oracle's int8 decode (the reference's aarch64 CPU
                path restated) of the same model on a bounded sample, at 4
                threads (the reference default) and at every available core
                (at most 16, the host share of one GPU), plus the restated f32
                path the reference runs on x86 (quant.rs:377-476).

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--skip SECTIONS]
       python bench.py --profile-gemv     (GEMV launches and a 256 MiB copy, for counter runs)
       python bench.py --profile-decode   (one config-3 decode and a 256 MiB copy, for counter runs)
       python bench.py --profile-prefill  (the prefill workload and a 256 MiB copy, for counter runs)
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

METRIC = "decode tok/s, 2B Q4_K_M synthetic; Q4_K/Q6_K GEMV HBM GB/s (% of peak)"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0   # dense int8 MFMA, MI355X
Q4K_ROWS, Q4K_K = 5760, 2304
Q4K_LAUNCH_BYTES = Q4K_ROWS * (Q4K_K // 256) * 144 + Q4K_K * 4 + Q4K_ROWS * 4     # 7 497 216
Q6K_ROWS, Q6K_K = 122753, 2304
Q6K_LAUNCH_BYTES = Q6K_ROWS * (Q6K_K // 256) * 210 + Q6K_K * 4 + Q6K_ROWS * 4     # 232 503 398
MODEL_SEED, PROMPT_SEED, N_PROMPT, N_GEN = 1234, 77, 128, 256
KV_BYTES_PER_POS = 2 * 40 * 36 * 64 * 4                                          # 737 280
EMBD_ROW_BYTES = Q4K_K // 256 * 144                                               # 1 296
# HBM bytes per k_mega launch from rocprofv3 FETCH_SIZE / WRITE_SIZE, each
# scaled by what the counter reads for a 256 MiB copy, over one decode of
# this workload (profiles/decode_minicpm2b_k_mega_traffic.md).
K_MEGA_TRAFFIC_BYTES = round((1056837.97 * 1.99974 + 9539.16 * 1.0) * 1024)      # 2 173 887 ...
# Same for the Q4_K GEMV launch (profiles/gemv_q4k_5760x2304_traffic.md).
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
    """(us of the whole job: Q8 of x + GEMV, us of the GEMV alone)."""
    w = gen(1, rows, k)
    ws = [b.upload(t, w, rows, k) for _ in range(copies)]
    x = pih.synth_normal(2, k)
    xd, yd = b.to_device(x), b.alloc(rows * 4)
    qd, dd, sd = b.alloc(k), b.alloc(k // 32 * 4), b.alloc(k // 32 * 4)
    b.q8_quantize_dev(xd.ptr, k, 1, qd.ptr, dd.ptr, sd.ptr)
    b.time_gemv_x(ws, xd.ptr, yd.ptr, max(copies, 8))                       # warm
    whole = b.time_gemv_x(ws, xd.ptr, yd.ptr, iters)
    alone = b.time_gemv(ws, qd.ptr, dd.ptr, sd.ptr, yd.ptr, iters)
    for wt in ws:
        wt.free()
    for buf in (xd, yd, qd, dd, sd):
        buf.free()
    return whole, alone


def q5k_rows(rows, k, seed=3):
    """Random Q5_K blocks with finite f16 scales (GGUF row layout)."""
    rng = np.random.default_rng(seed)
    nb = rows * (k // 256)
    blk = rng.integers(0, 256, size=(nb, 176), dtype=np.uint8)
    for off in (0, 2):
        blk[:, off:off + 2] = (rng.standard_normal(nb) * 0.02).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1).copy()


def time_gemv_row(b, t, rows, k, w, copies, iters):
    """us per launch of the f32-path GEMV (whole job: x f32 in HBM)."""
    ws = [b.upload(t, w, rows, k) for _ in range(copies)]
    x = pih.synth_normal(2, k)
    xd, yd = b.to_device(x), b.alloc(rows * 4)
    b.time_gemv_x(ws, xd.ptr, yd.ptr, max(copies, 8))                       # warm
    us = b.time_gemv_x(ws, xd.ptr, yd.ptr, iters)
    for wt in ws:
        wt.free()
    for buf in (xd, yd):
        buf.free()
    return us


def gemv_entry(whole_us, alone_us, nbytes, kernel):
    g = nbytes / (whole_us * 1e-6) / 1e9
    ga = nbytes / (alone_us * 1e-6) / 1e9
    return {"kernel": kernel, "bytes_per_launch": nbytes,
            "us_with_q8": round(whole_us, 3), "achieved_gbs": round(g, 1), "frac": round(g / HBM_PEAK_GBS, 4),
            "us_gemv_alone": round(alone_us, 3), "achieved_gbs_gemv_alone": round(ga, 1),
            "frac_gemv_alone": round(ga / HBM_PEAK_GBS, 4)}


def bench_prefill(b, model, spec):
    """2048-token prompt, then +512 tokens with prefix reuse (model.rs:1258-1268)."""
    ids = splitmix_ids(91, 2048 + 512, spec.n_vocab)
    eng = pih.HipEngine(b, model, n_ctx=2048 + 512 + 16)
    eng.generate(ids[:96], 1)                       # first launches of every prefill kernel
    eng.forward([ids[0]], [0], want_logits=False)   # a manual forward drops the reusable prefix
    _, sa = eng.generate(ids[:2048], 1)
    _, sb = eng.generate(ids, 1)
    # The projections' useful int8 work: one multiply-add per layer weight per
    # token (the int8 MFMA forms every weight x activation product once; Q6_K's
    # half-masked operands and padded tokens are not counted).
    qdim, kvdim = spec.n_head * spec.head_dim, spec.n_head_kv * spec.head_dim
    macs_tok = spec.n_layer * (spec.n_embd * (qdim + 2 * kvdim) + qdim * spec.n_embd + 3 * spec.n_embd * spec.n_ff)
    ops = 2 * macs_tok * 2048
    tops = ops / (sa["prefill_ms"] / 1000.0) / 1e12
    return {"prompt_tokens": 2048, "prefill_ms": round(sa["prefill_ms"], 2),
            "tok_s": round(2048 / (sa["prefill_ms"] / 1000.0), 1), "chunk_tokens": 32, "pass_tokens": b.prefill_pass_tokens(),
            "extension": {"new_tokens": sb["prefill_tokens"], "reused_tokens": sb["prefill_cached_tokens"],
                          "prefill_ms": round(sb["prefill_ms"], 2),
                          "tok_s": round(sb["prefill_tokens"] / (sb["prefill_ms"] / 1000.0), 1)},
            "int8_mfma": {"ops_per_prompt": ops, "tops_over_prefill": round(tops, 1), "peak_tops": INT8_PEAK_TOPS,
                          "frac": round(tops / INT8_PEAK_TOPS, 4),
                          "note": "useful int8 multiply-adds of the projections over the whole prefill time; "
                                  "the exact float epilogue of each term, not the int8 dot products, bounds the GEMMs"}}


def bench_long_context(b, model, n_fill, n_gen, wbytes):
    """n_gen greedy tokens after N(0,1) K/V at positions 0..n_fill-1 (seed 4242)."""
    eng = pih.HipEngine(b, model, n_ctx=n_fill + n_gen + 16)
    eng.kv_fill_normal(n_fill, 4242)
    eng.kv_set_tokens([0] * n_fill)
    b.time_kernels(True)
    _, st = eng.generate([0] * n_fill + [17], n_gen)   # reuses n_fill, evaluates token 17, then decodes
    kern_us, kern_n = eng.last_kernel_us()
    b.time_kernels(False)
    tps = st["gen_tokens"] / (st["gen_ms"] / 1000.0)
    trace = stage_breakdown(b, eng, 17, n_fill + n_gen, spec_heads(model), spec_kv(model))
    # forward j (1..n_gen-1) sits at position n_fill + j and reads positions 0..n_fill + j
    kv_bytes = KV_BYTES_PER_POS * (n_fill + 1 + n_gen / 2)
    per_tok = wbytes + kv_bytes
    return {"context": n_fill, "tok_s": round(tps, 2), "gen_tokens": st["gen_tokens"],
            "forwards": kern_n, "kernel_us_per_forward": round(kern_us, 1),
            "reused": st["prefill_cached_tokens"], "bytes_per_forward": round(per_tok),
            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / per_tok, 1),
            "frac": round(tps * per_tok / (HBM_PEAK_GBS * 1e9), 4),
            "kernel_gbs": round(per_tok / (kern_us * 1e-6) / 1e9, 1) if kern_us else None,
            "attention_us_per_layer": trace["us_per_layer"]["attention"],
            "attention_gbs": trace["attention_gbs"], "attention_frac": trace["attention_frac"],
            "stage_trace": trace}


def spec_heads(model):
    return model.spec.n_head


def spec_kv(model):
    return model.spec.n_head_kv


STAGES = ("qkv", "attention", "attn_output", "ffn_gate_up", "ffn_down")


def stage_breakdown(b, eng, tok, pos, n_head=36, n_kv=36, dh=64):
    """One traced forward of `tok` at `pos` on the persistent kernel: every
    workgroup records the device clock (100 MHz) at the end of each stage.
    A stage of layer l ends when its slowest workgroup ends it; its time runs
    from the end of the previous stage.  Attention reads (and writes) the K
    and V rows of positions 0..pos of every KV head: 2 * n_kv * (pos+1) * dh
    * 4 bytes per layer."""
    b.stage_trace(True)
    eng.forward([tok], [pos], want_logits=True)
    tr = b.stage_trace_read().astype("int64")
    b.stage_trace(False)
    n_layer = (tr.shape[1] - 4 - 32) // 5
    end = tr.max(axis=0)                                  # slowest workgroup per slot
    per = {k: [] for k in STAGES}
    for l in range(n_layer):
        prev = end[1] if l == 0 else end[6 + 5 * (l - 1)]
        for i, k in enumerate(STAGES):
            cur = end[2 + 5 * l + i]
            per[k].append((cur - prev) / 100.0)           # us
            prev = cur
    mean = {k: round(float(sum(v) / len(v)), 2) for k, v in per.items()}
    kv_layer = 2 * n_kv * (pos + 1) * dh * 4
    total = (end[2 + 5 * n_layer] - end[0]) / 100.0
    return {"position": pos, "us_per_layer": mean, "layers": n_layer, "forward_us": round(float(total), 1),
            "attention_kv_bytes_per_layer": kv_layer,
            "attention_gbs": round(kv_layer / (mean["attention"] * 1e-6) / 1e9, 1),
            "attention_frac": round(kv_layer / (mean["attention"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def profile_gemv(b):
    """Q4_K GEMV launches over 70 weight copies and one 256 MiB device copy:
    a short program for rocprofv3 counter runs (FETCH_SIZE / WRITE_SIZE)."""
    us, alone = time_gemv(b, pih.Q4_K, Q4K_ROWS, Q4K_K, pih.synth_q4k_random, 70, 210)
    n = 256 << 20
    src, dst = b.alloc(n), b.alloc(n)
    b.copy_d2d(dst, src, n)
    b.synchronize()
    print(json.dumps({"profile": "gemv", "q4k_us_with_q8": round(us, 3), "q4k_us_alone": round(alone, 3),
                      "copy_bytes": n}), flush=True)


def profile_prefill(b, model, spec):
    """The prefill workload (96-token warm-up, 2048-token prompt, 512-token
    extension) on the per-stage kernels, then one 256 MiB device copy: a short
    program for rocprofv3 counter runs on the prefill kernels."""
    b.use_persistent(False)
    st = bench_prefill(b, model, spec)
    n = 256 << 20
    src, dst = b.alloc(n), b.alloc(n)
    b.copy_d2d(dst, src, n)
    b.synchronize()
    print(json.dumps({"profile": "prefill", "prefill_ms": st["prefill_ms"], "copy_bytes": n}), flush=True)


def profile_decode(b, model, prompt):
    """One config-3 decode (128-id prompt, 256 tokens: k_mega at positions
    128..382) and one 256 MiB device copy: a short program for rocprofv3
    counter runs on k_mega."""
    eng = pih.HipEngine(b, model, n_ctx=N_PROMPT + N_GEN + 8)
    ids, st = eng.generate(prompt, N_GEN)
    n = 256 << 20
    src, dst = b.alloc(n), b.alloc(n)
    b.copy_d2d(dst, src, n)
    b.synchronize()
    print(json.dumps({"profile": "decode", "gen_tokens": st["gen_tokens"], "gen_ms": round(st["gen_ms"], 2),
                      "copy_bytes": n}), flush=True)


def cpu_baseline(model, prompt):
    """The oracle (the reference's CPU path restated) on the host's cores."""
    from oracle import oracle
    nproc = os.cpu_count() or 1
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    all_threads = max(1, min(avail, 16))

    def run(threads, n_prompt, n_tok, int8=True):
        eng = oracle.OracleEngine(model, n_ctx=64, threads=threads)
        eng.set_int8(int8)
        _, st = eng.generate(prompt[:n_prompt], n_tok)
        eng.close()
        return {"threads": threads, "tok_s": round(st["gen_tokens"] / (st["gen_ms"] / 1000.0), 3),
                "gen_tokens": st["gen_tokens"], "gen_ms": round(st["gen_ms"], 1),
                "prefill_tokens": n_prompt, "prefill_ms": round(st["prefill_ms"], 1)}

    t4 = run(4, 32, 12)
    ta = run(all_threads, 32, 16)
    f32 = run(all_threads, 8, 4, int8=False)
    return {"value": ta["tok_s"], "unit": "tok/s", "cores": all_threads, "kind": "port",
            "nproc": nproc, "available_cores": avail,
            "sample": f"oracle int8 greedy decode of the same model (the reference's aarch64 CPU path restated): "
                      f"32-id prompt, {ta['gen_tokens']} tokens ({ta['gen_tokens'] - 1} forwards) at "
                      f"{all_threads} threads; 12 tokens at 4 threads; f32 path (quant.rs:377-476): 8-id prompt, "
                      f"4 tokens",
            "threads_4": t4, "threads_all": ta, "f32_path_threads_all": f32}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3, help="timed full decodes (128-id prompt + 256 tokens each)")
    ap.add_argument("--warmup", type=int, default=2, help="untimed full decodes first")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graphs", action="store_true", help="launch kernels one by one (for profilers)")
    ap.add_argument("--per-stage", action="store_true",
                    help="engine tokens on the per-stage kernels, no cooperative launch (for profilers)")
    ap.add_argument("--no-extra", action="store_true", help="skip the prefill and long-context sections")
    ap.add_argument("--profile-gemv", action="store_true", help="GEMV launches and a device copy only")
    ap.add_argument("--profile-decode", action="store_true",
                    help="one config-3 decode (128-id prompt, 256 tokens) and a device copy only")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="the prefill workload on the per-stage kernels and a device copy only")
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
    steps, warmup = max(1, args.steps), max(0, args.warmup)
    t_start = time.time()
    b = pih.HipBackend(0)
    try:
        run(args, skip, steps, warmup, b, t_start)
    finally:
        b.close()


def run(args, skip, steps, warmup, b, t_start):
    b.use_graphs(not args.no_graphs)
    if args.per_stage:
        b.use_persistent(False)
    log(f"device: {b.name()}")
    if args.profile_gemv:
        profile_gemv(b)
        return

    # -- standalone GEMVs of configs 1 and 2, HBM-cold ----------------------
    g4 = g6 = g5 = None
    if not args.no_gemv:
        w4, a4 = time_gemv(b, pih.Q4_K, Q4K_ROWS, Q4K_K, pih.synth_q4k_random, 70, 700)
        w6, a6 = time_gemv(b, pih.Q6_K, Q6K_ROWS, Q6K_K, pih.synth_q6k_random, 3, 30)
        g4 = gemv_entry(w4, a4, Q4K_LAUNCH_BYTES,
                        "Q4_K GEMV 5760x2304: k_gemv_x<12,1> (Q8 of x in its prologue); alone: k_gemv<12,1,0>")
        g4["traffic_gemv_alone"] = Q4K_TRAFFIC_BYTES
        g6 = gemv_entry(w6, a6, Q6K_LAUNCH_BYTES,
                        "Q6_K head GEMV 122753x2304: k_gemv_x<14,1> (Q8 of x in its prologue); alone: k_gemv<14,1,0>")
        q5w = q5k_rows(Q4K_ROWS, Q4K_K)
        u5 = time_gemv_row(b, pih.Q5_K, Q4K_ROWS, Q4K_K, q5w, 20, 100)
        q5_bytes = q5w.nbytes + Q4K_K * 4 + Q4K_ROWS * 4
        g5 = {"kernel": "Q5_K GEMV 5760x2304, the reference's f32 path (dot_row_scalar order): k_gemv_row<13>",
              "bytes_per_launch": q5_bytes, "us": round(u5, 2),
              "achieved_gbs": round(q5_bytes / (u5 * 1e-6) / 1e9, 1),
              "frac": round(q5_bytes / (u5 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
              "bound": "the row's dependent adds in element order (one chain lane per row; ~7.5 cycles per add), not HBM"}
        log(f"gemv q5_k (f32 path): {g5}")
        log(f"gemv q4k: {g4}")
        log(f"gemv q6k: {g6}")

    # -- decode (config 3) ----------------------------------------------------
    spec = pih.minicpm2b_spec()
    t0 = time.time()
    model = pih.synth_model(spec, MODEL_SEED)
    wbytes = model.weight_bytes_per_token()
    log(f"model synthesized in {time.time() - t0:.1f}s; {wbytes} weight bytes/token")
    prompt = splitmix_ids(PROMPT_SEED, N_PROMPT, spec.n_vocab)
    if args.profile_decode:
        profile_decode(b, model, prompt)
        return
    if args.profile_prefill:
        profile_prefill(b, model, spec)
        return
    runs, match, kern = [], None, []
    eng = None
    if "decode" not in skip:
        eng = pih.HipEngine(b, model, n_ctx=N_PROMPT + N_GEN + 8)
        for _ in range(warmup):
            eng.generate(prompt, N_GEN)
        b.synchronize()
        b.time_kernels(True)
        for i in range(steps):
            ids, st = eng.generate(prompt, N_GEN)
            runs.append(st)
            kern.append(eng.last_kernel_us())
            log(f"decode {i}: {st['gen_tokens']} tokens in {st['gen_ms']:.1f} ms "
                f"({st['gen_tokens'] / st['gen_ms'] * 1000:.1f} tok/s), k_mega {kern[-1][0]:.1f} us/launch, "
                f"stop={st['stop']}, prefill {st['prefill_ms']:.1f} ms ({st['prefill_cached_tokens']} reused)")
            if i == 0:
                golden = REPO / "tests" / "golden" / "minicpm2b_greedy.json"
                if golden.exists():
                    g = json.loads(golden.read_text())
                    if g["prompt"] == prompt and g["model_seed"] == MODEL_SEED and len(ids) >= g["n_gen"]:
                        match = ids[: g["n_gen"]] == g["gen_ids"]
        b.time_kernels(False)
    trace = stage_breakdown(b, eng, 17, N_PROMPT + N_GEN - 1) if eng is not None else None
    if trace:
        log(f"stage trace: {trace}")
    gen_tokens = sum(st["gen_tokens"] for st in runs)
    gen_ms = sum(st["gen_ms"] for st in runs)
    fwd = sum(max(st["gen_tokens"] - 1, 0) for st in runs)
    tps = gen_tokens / (gen_ms / 1000.0) if runs else float("nan")
    kern_n = sum(n for _, n in kern)
    kern_us = sum(u * n for u, n in kern) / kern_n if kern_n else float("nan")
    # forward j (1..255) evaluates position 127 + j and reads the KV of
    # positions 0..127 + j: 128 + j rows, mean 256
    n_fwd = N_GEN - 1
    kv_mean = KV_BYTES_PER_POS * sum(N_PROMPT + j for j in range(1, n_fwd + 1)) / n_fwd
    launch_bytes = wbytes + kv_mean + EMBD_ROW_BYTES
    mega_gbs = launch_bytes / (kern_us * 1e-6) / 1e9

    prefill = long_ctx = None
    if not args.no_extra and "prefill" not in skip:
        prefill = bench_prefill(b, model, spec)
        log(f"prefill: {prefill}")
    if not args.no_extra and "long" not in skip:
        long_ctx = [bench_long_context(b, model, n, 64, wbytes) for n in (4096, 16384)]
        log(f"long context: {long_ctx}")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(model, prompt)
        log(f"cpu baseline: {cpu}")

    out = {
        "metric": METRIC,
        "value": round(tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": len(runs),
        "warmup": warmup,
        "ms_per_step": round(gen_ms / max(len(runs), 1), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot / f32",
        "data": "synthetic (seeded random weights N(0,0.02) quantized Q4_K_M-style, random prompt ids)",
        "config": {"workload": "greedy decode, MiniCPM-2B-shaped Q4_K_M synthetic model: 40 layers, "
                               "hidden 2304, 36x64 MHA, FFN 5760, vocab 122753, f32 KV; one step = 128-id "
                               "prompt then 256 greedy tokens (255 forwards) at batch 1",
                   "prompt_tokens": N_PROMPT, "gen_tokens": runs[0]["gen_tokens"] if runs else 0, "batch": 1,
                   "forwards_timed": fwd, "ms_per_forward": round(gen_ms / fwd, 4) if fwd else None},
        "roofline": {"bound": "hbm", "achieved": round(mega_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(mega_gbs / HBM_PEAK_GBS, 4), "traffic": K_MEGA_TRAFFIC_BYTES,
                     "kernel": "k_mega (persistent decode kernel, one launch per decode forward)",
                     "us_per_launch": round(kern_us, 2), "launches_timed": kern_n,
                     "bytes_per_launch": round(launch_bytes), "weight_bytes": wbytes,
                     "kv_bytes_mean": round(kv_mean),
                     "gemv_q4k": g4, "gemv_q6k": g6, "gemv_q5k_f32_path": g5},
        "decode_weight_roofline": {"weight_bytes_per_token": wbytes,
                                   "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / wbytes, 1),
                                   "frac": round(tps * wbytes / (HBM_PEAK_GBS * 1e9), 4)},
        "decode_stage_trace": trace,
        "greedy_first_64_match_oracle": match,
        "prefill": prefill,
        "long_context": long_ctx,
        "cpu_baseline": cpu,
        "wall_s": round(time.time() - t_start, 1),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
