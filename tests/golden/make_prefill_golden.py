"""Writes tests/golden/minicpm2b_prefill.json: the CPU oracle's results for
the long-prompt prefill workload with prefix reuse.

Workload: the synthetic MiniCPM-2B-shaped Q4_K_M model (seed 1234,
pocketinfer_hip.synth_model); prompt A = 2048 ids drawn from SplitMix64
seed 91 (u64 % n_vocab); prompt B = A followed by 512 more ids of the same
stream.  generate(A, 2) and then generate(B, 4) on one engine, so the second
call reuses the cached prefix by the rule of model.rs:1258-1268
(min(common, cached, len-1) // 32 * 32 = 2048).  Recorded per call: greedy
ids, reused tokens, SHA-256 of the final logits' bytes and the top-8 logits
(index, value bits).

Run from the repository root:  python tests/golden/make_prefill_golden.py
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

MODEL_SEED, PROMPT_SEED, N_A, N_EXT = 1234, 91, 2048, 512


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


def summary(logits: np.ndarray) -> dict:
    lg = np.ascontiguousarray(logits, np.float32)
    top = np.argsort(-lg, kind="stable")[:8]
    return {"sha256": hashlib.sha256(lg.tobytes()).hexdigest(),
            "top8": [[int(i), int(lg[i:i + 1].view(np.uint32)[0])] for i in top]}


def main():
    threads = min(16, os.cpu_count() or 1)
    t0 = time.time()
    spec = pih.minicpm2b_spec()
    model = pih.synth_model(spec, MODEL_SEED, threads)
    ids = splitmix_ids(PROMPT_SEED, N_A + N_EXT, spec.n_vocab)
    a, b = ids[:N_A], ids
    n_ctx = N_A + N_EXT + 16
    eng = oracle.OracleEngine(model, n_ctx=n_ctx, threads=threads)
    ga, sa = eng.generate(a, 2)
    la = summary(eng.logits())
    print(f"prompt A: ids {ga} {sa} ({time.time() - t0:.0f}s)", flush=True)
    gb, sb = eng.generate(b, 4)
    lb = summary(eng.logits())
    print(f"prompt B: ids {gb} {sb} ({time.time() - t0:.0f}s)", flush=True)
    assert sb["prefill_cached_tokens"] == 2048, sb
    out = {
        "workload": "synthetic MiniCPM-2B-shaped Q4_K_M model, 2048-token prompt then a 512-token extension",
        "model_seed": MODEL_SEED, "prompt_seed": PROMPT_SEED, "n_a": N_A, "n_ext": N_EXT, "n_ctx": n_ctx,
        "a": {"gen_ids": ga, "prefill_cached_tokens": sa["prefill_cached_tokens"], "logits": la},
        "b": {"gen_ids": gb, "prefill_cached_tokens": sb["prefill_cached_tokens"], "logits": lb},
    }
    path = Path(__file__).with_name("minicpm2b_prefill.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path} in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
