"""GPU parity of the long-prompt and long-context workloads on the full-size
synthetic MiniCPM-2B-shaped model, against committed oracle fixtures:

* prefill: a 2048-token prompt in 64 batched chunks, then the prompt
  extended by 512 tokens reusing the cached prefix (model.rs:1258-1268);
  greedy ids, reused-token count and the final logits bit for bit (SHA-256
  of their bytes), and the reused run equal to a fresh one
  (tests/prefix_cache.rs:27-63);
* long context: N(0,1) K/V prefilled to 4096 and to 16384 positions, then
  64 greedy forwards at batch 1; the first 64 greedy ids.
"""
import hashlib
import json
import time
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).parent / "golden"


def _sha(logits):
    return hashlib.sha256(np.ascontiguousarray(logits, np.float32).tobytes()).hexdigest()


def _splitmix_ids(seed, n, vocab):
    out, s = [], (seed + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        z ^= z >> 31
        out.append(z % vocab)
    return out


@pytest.fixture(scope="module")
def model2b(pih):
    return pih.synth_model(pih.minicpm2b_spec(), 1234)


def test_kv_fill_matches_host_generator(pih, backend):
    """The device fill and pi_synth_kv_normal give the same bits."""
    m = pih.synth_model(pih.tiny_spec(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_vocab=1000), seed=3)
    eng = pih.HipEngine(backend, m, n_ctx=96)
    eng.kv_fill_normal(90, 4242)
    for layer in range(2):
        for h in (0, 3):
            k, v = eng.kv_read(layer, h, 0, 90)
            hk, hv = pih.synth_kv_normal(4242, layer * 4 + h, 0, 90)
            assert np.array_equal(k.ravel().view(np.uint32), hk.ravel().view(np.uint32)) and \
                np.array_equal(v.ravel().view(np.uint32), hv.ravel().view(np.uint32)), (layer, h)


def test_minicpm2b_prefill_2048_then_reuse(pih, backend, model2b):
    g = json.loads((GOLDEN / "minicpm2b_prefill.json").read_text())
    ids = _splitmix_ids(g["prompt_seed"], g["n_a"] + g["n_ext"], model2b.spec.n_vocab)
    a, b = ids[:g["n_a"]], ids
    eng = pih.HipEngine(backend, model2b, n_ctx=g["n_ctx"])
    t0 = time.time()
    ga, sa = eng.generate(a, 2)
    print(f"prefill {len(a)} tokens: {sa['prefill_ms']:.1f} ms "
          f"({len(a) / sa['prefill_ms'] * 1000:.0f} tok/s), wall {time.time() - t0:.1f}s", flush=True)
    assert ga == g["a"]["gen_ids"] and sa["prefill_cached_tokens"] == 0
    assert _sha(eng.logits()) == g["a"]["logits"]["sha256"]
    gb, sb = eng.generate(b, 4)
    print(f"extension: {sb['prefill_tokens']} new tokens, {sb['prefill_cached_tokens']} reused, "
          f"{sb['prefill_ms']:.1f} ms", flush=True)
    assert sb["prefill_cached_tokens"] == g["b"]["prefill_cached_tokens"] == 2048
    assert gb == g["b"]["gen_ids"]
    reused_logits = eng.logits()
    assert _sha(reused_logits) == g["b"]["logits"]["sha256"]
    fresh = pih.HipEngine(backend, model2b, n_ctx=g["n_ctx"])
    gf, sf = fresh.generate(b, 4)
    assert sf["prefill_cached_tokens"] == 0 and gf == gb
    assert np.array_equal(fresh.logits().view(np.uint32), reused_logits.view(np.uint32))


@pytest.mark.parametrize("run", [0, 1], ids=["4096", "16384"])
def test_minicpm2b_long_context_greedy(pih, backend, model2b, run):
    g = json.loads((GOLDEN / "minicpm2b_longctx.json").read_text())
    r = g["runs"][run]
    n_fill = r["n_fill"]
    eng = pih.HipEngine(backend, model2b, n_ctx=n_fill + g["n_gen"] + 8)
    eng.kv_fill_normal(n_fill, g["kv_seed"])
    tok, got = g["first_token"], []
    t0 = time.time()
    for i in range(g["n_gen"]):
        eng.forward([tok], [n_fill + i], want_logits=True)
        tok = eng.argmax()
        got.append(tok)
    dt = time.time() - t0
    print(f"context {n_fill}: {g['n_gen']} forwards in {dt * 1000:.0f} ms ({g['n_gen'] / dt:.1f} tok/s)", flush=True)
    assert got == r["gen_ids"], f"first mismatch at {next(i for i, (x, y) in enumerate(zip(got, r['gen_ids'])) if x != y)}"
