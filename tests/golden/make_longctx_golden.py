"""Writes tests/golden/minicpm2b_longctx.json: the CPU oracle's first greedy
ids for long-context decode on the synthetic MiniCPM-2B-shaped model.

Workload, for each context length N in (4096, 16384): the f32 K/V caches of
every layer and head hold N(0,1) values for positions 0..N-1 (the values of
pocketinfer_hip.synth_kv_normal, seed 4242, the same bits the device fill
writes), written straight into the engine's caches as the reference's pub
KvCache allows (model.rs:352-359).  Then 64 forwards at positions N..N+63:
the first evaluates token 17; each next one the greedy id (first index of
the maximum logit, sampler.rs:26-36) of the previous.  Recorded: the 64
greedy ids and each step's top-1 / top-2 logit margin.

Run from the repository root:  python tests/golden/make_longctx_golden.py
(about 12 GiB of host memory for the 16384 case).
"""
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

MODEL_SEED, KV_SEED, FIRST_TOKEN, N_GEN = 1234, 4242, 17, 64
CONTEXTS = (4096, 16384)


def run(model, n_fill: int, threads: int) -> dict:
    s = model.spec
    t0 = time.time()
    eng = oracle.OracleEngine(model, n_ctx=n_fill + N_GEN + 8, threads=threads)
    K, V = eng.kv()
    for layer in range(s.n_layer):
        for h in range(s.n_head_kv):
            k, v = pih.synth_kv_normal(KV_SEED, layer * s.n_head_kv + h, 0, n_fill, s.head_dim)
            K[layer, h, :n_fill] = k
            V[layer, h, :n_fill] = v
    print(f"N={n_fill}: KV filled in {time.time() - t0:.0f}s", flush=True)
    tok, ids, margins = FIRST_TOKEN, [], []
    for i in range(N_GEN):
        eng.forward([tok], [n_fill + i], want_logits=True)
        lg = eng.logits()
        tok = int(np.argmax(lg))
        top2 = np.sort(lg)[-2:]
        ids.append(tok)
        margins.append(float(top2[1] - top2[0]))
        if i % 8 == 0:
            print(f"N={n_fill} step {i}: {tok} margin {margins[-1]:.4g} ({time.time() - t0:.0f}s)", flush=True)
    eng.close()
    return {"n_fill": n_fill, "gen_ids": ids, "top1_top2_margin": margins}


def main():
    threads = min(16, os.cpu_count() or 1)
    t0 = time.time()
    model = pih.synth_model(pih.minicpm2b_spec(), MODEL_SEED, threads)
    out = {"workload": "synthetic MiniCPM-2B-shaped Q4_K_M model, N(0,1) KV prefilled to N positions, "
                       "64 greedy forwards from token 17 at batch 1",
           "model_seed": MODEL_SEED, "kv_seed": KV_SEED, "first_token": FIRST_TOKEN, "n_gen": N_GEN,
           "runs": [run(model, n, threads) for n in CONTEXTS]}
    path = Path(__file__).with_name("minicpm2b_longctx.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path} in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
