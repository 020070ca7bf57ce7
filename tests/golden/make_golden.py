"""Writes tests/golden/minicpm2b_greedy.json: the CPU oracle's first greedy
ids for the synthetic MiniCPM-2B-shaped Q4_K_M model.

Workload: model seed 1234 (pocketinfer_hip.synth_model), prompt = 128 ids
drawn from SplitMix64 seed 77 (u64 % n_vocab), greedy decode of 64 tokens.
The file also records SHA-256 digests of a few synthetic tensors, so a test
can check that the generator reproduces the same bytes on another machine,
and the top-1 / top-2 logit margin of every step (how close each greedy
choice is to a tie).

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(REPO), str(REPO / "pocket-workbench-android_amd")]

import pocketinfer_hip as pih  # noqa: E402
from oracle import oracle  # noqa: E402

MODEL_SEED, PROMPT_SEED, N_PROMPT, N_GEN = 1234, 77, 128, 64


def splitmix_ids(seed: int, n: int, vocab: int) -> list[int]:
    """SplitMix64 (sampler.rs:1-19) draws, u64 % vocab."""
    out, s = [], (seed + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        z ^= z >> 31
        out.append(z % vocab)
    return out


def digests(model) -> dict:
    names = ["token_embd.weight", "blk.0.attn_q.weight", "blk.0.attn_v.weight", "blk.0.ffn_down.weight",
             "blk.1.ffn_down.weight", "blk.39.attn_norm.weight", "output.weight"]
    return {n: hashlib.sha256(model.tensors[n][3].tobytes()).hexdigest() for n in names}


def main():
    threads = min(16, os.cpu_count() or 1)
    t0 = time.time()
    spec = pih.minicpm2b_spec()
    model = pih.synth_model(spec, MODEL_SEED, threads)
    print(f"model synthesized in {time.time() - t0:.1f}s", flush=True)
    prompt = splitmix_ids(PROMPT_SEED, N_PROMPT, spec.n_vocab)
    eng = oracle.OracleEngine(model, n_ctx=N_PROMPT + N_GEN + 8, threads=threads)
    # prefill in 32-token chunks, then greedy steps, keeping per-step margins
    t1 = time.time()
    for off in range(0, N_PROMPT, 32):
        ids = prompt[off:off + 32]
        eng.forward(ids, list(range(off, off + len(ids))), want_logits=off + 32 >= N_PROMPT)
    print(f"prefill {time.time() - t1:.1f}s", flush=True)
    gen, margins = [], []
    pos = N_PROMPT
    for i in range(N_GEN):
        lg = eng.logits()
        top2 = np.argsort(lg)[-2:]
        tok = int(np.argmax(lg))
        margins.append(float(lg[top2[1]] - lg[top2[0]]))
        gen.append(tok)
        if i + 1 == N_GEN:
            break
        eng.forward([tok], [pos], want_logits=True)
        pos += 1
        if i % 8 == 0:
            print(f"step {i} tok {tok} margin {margins[-1]:.4g} ({time.time() - t1:.0f}s)", flush=True)
    # cross-check with the generate loop (model.rs:1235-1352) on a fresh engine
    eng2 = oracle.OracleEngine(model, n_ctx=N_PROMPT + N_GEN + 8, threads=threads)
    ids2, stats = eng2.generate(prompt, N_GEN)
    assert ids2 == gen, "generate() and the forward loop disagree"
    out = {
        "workload": "synthetic MiniCPM-2B-shaped Q4_K_M model, greedy decode",
        "model_seed": MODEL_SEED, "prompt_seed": PROMPT_SEED, "prompt": prompt,
        "n_gen": N_GEN, "gen_ids": gen, "top1_top2_margin": margins,
        "eos_ids": list(spec.eos_ids), "stop": stats["stop"],
        "tensor_sha256": digests(model),
        "weight_bytes_per_token": model.weight_bytes_per_token(),
    }
    path = Path(__file__).with_name("minicpm2b_greedy.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path} in {time.time() - t0:.0f}s; min margin {min(margins):.4g}")


if __name__ == "__main__":
    main()
