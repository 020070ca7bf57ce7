"""GPU parity of the whole-forward engine against the CPU oracle.

Tiny models check logits (1e-3 relative + 1e-4 absolute, the contract's
tolerance) and greedy ids against the oracle run in the same process; the
full-size synthetic MiniCPM-2B model checks the first 64 greedy ids against
the committed oracle fixture tests/golden/minicpm2b_greedy.json.
"""
import json
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).parent / "golden" / "minicpm2b_greedy.json"


@pytest.fixture(params=["persistent", "per_stage", "token_prefill"], autouse=True)
def engine_mode(request, backend):
    """Every engine test runs on the persistent kernel (one cooperative
    launch per token) and on the per-stage kernels, with multi-token chunks
    on the batched MFMA prefill kernels; and once more with every prompt
    token evaluated on its own."""
    backend.use_persistent(request.param != "per_stage")
    backend.use_batch_prefill(request.param != "token_prefill")
    yield "per_stage" if request.param == "per_stage" else "persistent"
    backend.use_persistent(True)
    backend.use_batch_prefill(True)


@pytest.fixture(scope="module")
def tiny(pih):
    return pih.synth_model(pih.tiny_spec(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_vocab=1000), seed=7)


@pytest.fixture(scope="module")
def gqa(pih):
    """8 query heads over 2 KV heads (kh = h / group, model.rs:995) with RoPE
    on the first 32 of 64 dimensions (model.rs:930, 953-979)."""
    return pih.synth_model(pih.tiny_spec(n_layer=2, n_embd=512, n_ff=1024, n_head=8, n_vocab=1000, n_head_kv=2,
                                         n_rot=32), seed=13)


def _with_eos(pih, model, eos):
    """The same weights with another end-of-generation id."""
    import dataclasses
    return pih.SynthModel(dataclasses.replace(model.spec, eos_ids=(eos,)), model.tensors)


def _close(got, want, rtol=1e-3, atol=1e-4):
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    return float(err.max())


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_tiny_forward_logits(pih, backend, oracle, tiny, engine_mode):
    """Batch-1 forwards: logits within the contract's tolerance, and in fact
    bit-identical since every float op keeps the reference order."""
    eng = pih.HipEngine(backend, tiny, n_ctx=128)
    assert backend.persistent_active() == (engine_mode == "persistent")
    ref = oracle.OracleEngine(tiny, n_ctx=128, threads=4)
    ids = [5, 17, 999, 0, 123, 456, 7, 8] + [(i * 131 + 3) % 1000 for i in range(70)]
    for pos, tok in enumerate(ids):
        eng.forward([tok], [pos], want_logits=True)
        ref.forward([tok], [pos], want_logits=True)
        got, want = eng.logits(), ref.logits()
        assert _close(got, want) <= 0.0, f"pos {pos}: max excess {_close(got, want)}"
        assert _bits_equal(got, want), f"pos {pos}"


def test_tiny_batched_forward_matches_oracle(pih, backend, oracle, tiny):
    """A batch of more than one token takes the reference's scalar order
    (model.rs:812-822, 1028-1038); a batch of one the NEON order."""
    for b in (10, 1):
        eng = pih.HipEngine(backend, tiny, n_ctx=64)
        ref = oracle.OracleEngine(tiny, n_ctx=64, threads=4)
        ids = list(range(3, 13))
        for off in range(0, 10, b):
            eng.forward(ids[off:off + b], list(range(off, off + b)), want_logits=True)
            ref.forward(ids[off:off + b], list(range(off, off + b)), want_logits=True)
        assert _bits_equal(eng.logits(), ref.logits()), f"b={b}"


def test_tiny_kv_rows_match_oracle(pih, backend, oracle, tiny):
    eng = pih.HipEngine(backend, tiny, n_ctx=32)
    ref = oracle.OracleEngine(tiny, n_ctx=32, threads=4)
    ids = [3, 1, 4, 1, 5]
    eng.forward(ids, list(range(5)), want_logits=False)
    ref.forward(ids, list(range(5)), want_logits=False)
    kr, vr = ref.kv()
    for layer in range(tiny.spec.n_layer):
        for h in range(tiny.spec.n_head_kv):
            k, v = eng.kv_read(layer, h, 0, 5)
            assert _bits_equal(k, kr[layer, h, :5]) and _bits_equal(v, vr[layer, h, :5]), (layer, h)


@pytest.mark.parametrize("n_prompt", [45, 33, 64, 1])
def test_tiny_generate_matches_oracle(pih, backend, oracle, tiny, n_prompt):
    """Prefill chunks of 32 (the last one partial, or a single token), then
    greedy decode; ids and final logits equal the oracle's generate."""
    eng = pih.HipEngine(backend, tiny, n_ctx=256)
    ref = oracle.OracleEngine(tiny, n_ctx=256, threads=4)
    prompt = [(i * 37 + 11) % 1000 for i in range(n_prompt)]
    got, st = eng.generate(prompt, 40)
    want, st_ref = ref.generate(prompt, 40)
    assert got == want
    assert st["stop"] == st_ref["stop"]
    assert st["prefill_tokens"] == n_prompt and st["prefill_cached_tokens"] == 0
    assert _bits_equal(eng.logits(), ref.logits())


@pytest.mark.parametrize("n_prompt", [1100, 1057, 1025])
def test_tiny_generate_passes_span_chunks(pih, backend, oracle, tiny, n_prompt):
    """Prompts longer than one 1024-token device pass: the passes group the
    reference's 32-token chunks (1100: passes of 1024 + 76; 1057: 1024 + 32,
    then the single-token last chunk; 1025: 1024, then the single token); ids
    and final logits equal the oracle's."""
    eng = pih.HipEngine(backend, tiny, n_ctx=1200)
    assert backend.prefill_pass_tokens() == 1024
    ref = oracle.OracleEngine(tiny, n_ctx=1200, threads=4)
    prompt = [(i * 29 + 3) % 1000 for i in range(n_prompt)]
    got, st = eng.generate(prompt, 8)
    want, _ = ref.generate(prompt, 8)
    assert got == want and st["prefill_tokens"] == n_prompt
    assert _bits_equal(eng.logits(), ref.logits())


_WIDE_REF = {}


def test_pass_shrinks_at_long_context(pih, backend, oracle):
    """With 36 heads at n_ctx 8192 a 1024-token pass would need 1.2 GB of
    attention scores (1024 x 36 x 8192 floats), over the 1 GiB budget: the
    pass halves to 512, and a 540-token prompt (passes of 512 + 28) still
    equals the oracle."""
    model = pih.synth_model(pih.tiny_spec(n_layer=2, n_embd=2304, n_ff=512, n_head=36, n_vocab=1000), seed=29)
    eng = pih.HipEngine(backend, model, n_ctx=8192)
    assert backend.prefill_pass_tokens() == 512
    prompt = [(i * 31 + 7) % 1000 for i in range(540)]
    got, _ = eng.generate(prompt, 2)
    if not _WIDE_REF:   # the oracle's result does not depend on the engine mode
        ref = oracle.OracleEngine(model, n_ctx=8192, threads=8)
        _WIDE_REF["ids"], _ = ref.generate(prompt, 2)
        _WIDE_REF["logits"] = ref.logits().copy()
    assert got == _WIDE_REF["ids"] and _bits_equal(eng.logits(), _WIDE_REF["logits"])


def test_tiny_attention_skips_zero_weights(pih, backend, oracle, tiny):
    """model.rs:1048-1069 adds e_p * v_p only where e_p != 0.  The cache rows
    of positions 0..63 are set so that one position takes every weight: K is
    zero except +-1e6 * u at positions 10 and 37, so one of them holds a score
    of order 1e5 and every other e_p is exp(-1e5) == 0; the V rows of the
    other positions hold inf, -inf and NaN.  Skipping them leaves finite
    outputs (adding 0 * inf would not).  Logits of a batched forward and of
    the next single token equal the oracle's bit for bit."""
    s = tiny.spec
    eng = pih.HipEngine(backend, tiny, n_ctx=128)
    ref = oracle.OracleEngine(tiny, n_ctx=128, threads=4)
    rk, rv = ref.kv()
    rng = np.random.default_rng(5)
    npos = 64
    u = rng.standard_normal(s.head_dim).astype(np.float32)
    for layer in range(s.n_layer):
        for h in range(s.n_head_kv):
            k = np.zeros((npos, s.head_dim), np.float32)
            k[10], k[37] = 1e6 * u, -1e6 * u
            v = rng.standard_normal((npos, s.head_dim)).astype(np.float32)
            for i, p in enumerate(p for p in range(npos) if p not in (10, 37) and p % 3 == 0):
                v[p, (7 * i) % s.head_dim] = (np.inf, -np.inf, np.nan)[i % 3]
            eng.kv_write(layer, h, 0, k, v)
            rk[layer, h, :npos], rv[layer, h, :npos] = k, v
    ids = list(range(100, 108))
    eng.forward(ids, list(range(npos, npos + 8)), want_logits=True)
    ref.forward(ids, list(range(npos, npos + 8)), want_logits=True)
    want = ref.logits()
    assert np.isfinite(want).all()
    assert _bits_equal(eng.logits(), want)
    eng.forward([7], [npos + 8], want_logits=True)
    ref.forward([7], [npos + 8], want_logits=True)
    assert _bits_equal(eng.logits(), ref.logits())


def test_tiny_prefix_reuse(pih, backend, oracle, tiny):
    """tests/prefix_cache.rs:27-63 invariants on the device engine.  A context
    holds one engine, so the fresh run comes first."""
    base = [(i * 13 + 5) % 997 for i in range(70)]
    ext = base + [(i * 7 + 1) % 991 for i in range(40)]
    fresh = pih.HipEngine(backend, tiny, n_ctx=256)
    ids2, st2 = fresh.generate(ext, 4)
    assert st2["prefill_cached_tokens"] == 0
    fresh_logits = fresh.logits()
    eng = pih.HipEngine(backend, tiny, n_ctx=256)
    with pytest.raises(RuntimeError):
        fresh.generate(ext, 4)                        # replaced by the bind above
    eng.generate(base, 2)
    ids, st = eng.generate(ext, 4)
    assert st["prefill_cached_tokens"] == 64          # min(common 70, cached 70, 109) // 32 * 32
    assert st["prefill_cached_tokens"] + st["prefill_tokens"] == len(ext)
    assert ids == ids2 and _bits_equal(eng.logits(), fresh_logits)
    ref_ids, _ = oracle.OracleEngine(tiny, n_ctx=256, threads=4).generate(ext, 4)
    assert ids == ref_ids
    # a manual forward invalidates reuse (model.rs:825-831)
    eng.forward([ext[0]], [0], want_logits=False)
    ids3, st3 = eng.generate(ext, 4)
    assert st3["prefill_cached_tokens"] == 0 and ids3 == ids
    # stop request -> user_stop, then a clean retry
    eng.request_stop()
    _, st4 = eng.generate(ext, 4)
    assert st4["stop"] == "user_stop"
    eng.clear_stop()
    ids5, st5 = eng.generate(ext, 4)
    assert st5["prefill_cached_tokens"] == 0 and ids5 == ids


def test_tiny_context_full_and_eog(pih, backend, oracle, tiny):
    eng = pih.HipEngine(backend, tiny, n_ctx=50)
    ref = oracle.OracleEngine(tiny, n_ctx=50, threads=4)
    prompt = list(range(40))
    got, st = eng.generate(prompt, 30)
    want, st_ref = ref.generate(prompt, 30)
    assert got == want and st["stop"] == st_ref["stop"] == "context_full"
    with pytest.raises(pih.PiError):
        eng.forward([1], [50])


@pytest.mark.parametrize("at", [0, 5, 20])
def test_tiny_eog_matches_oracle(pih, backend, oracle, tiny, at):
    """generate stops at an end-of-generation id the oracle actually samples
    (model.rs:1305-1306): the same ids and stop reason, and the logits left
    behind are those that produced the EOG, as in Engine::generate, although
    the device may have launched later forwards before it read that id."""
    prompt = [(i * 29 + 3) % 1000 for i in range(37)]
    free, _ = oracle.OracleEngine(tiny, n_ctx=256, threads=4).generate(prompt, 40)
    # an id at index `at` that does not occur earlier
    idx = next(i for i in range(at, len(free)) if free[i] not in free[:i])
    m = _with_eos(pih, tiny, free[idx])
    eng = pih.HipEngine(backend, m, n_ctx=256)
    ref = oracle.OracleEngine(m, n_ctx=256, threads=4)
    got, st = eng.generate(prompt, 40)
    want, st_ref = ref.generate(prompt, 40)
    assert got == want == free[:idx]
    assert st["stop"] == st_ref["stop"] == "eog"
    assert _bits_equal(eng.logits(), ref.logits())
    assert eng.argmax() == free[idx]
    # the engine continues cleanly after an EOG stop
    got2, _ = eng.generate(prompt + want, 3)
    want2, _ = ref.generate(prompt + want, 3)
    assert got2 == want2


@pytest.mark.parametrize("temp,top_p,n_prompt", [(0.7, 0.95, 37), (1.0, 1.0, 1), (0.4, 0.5, 64)])
def test_tiny_sampled_generate_matches_oracle(pih, backend, oracle, tiny, temp, top_p, n_prompt):
    """Temperature / top-p generate (the app's temp 0.7, top_p 0.95 and seed
    0xC0FFEE, jni.rs:459-466): the same ids and stop as the oracle's generate,
    and the same weights left in the logits (sampler.rs:21-92)."""
    eng = pih.HipEngine(backend, tiny, n_ctx=256)
    ref = oracle.OracleEngine(tiny, n_ctx=256, threads=4)
    prompt = [(i * 41 + 7) % 1000 for i in range(n_prompt)]
    got, st = eng.generate(prompt, 40, temp=temp, top_p=top_p, seed=0xC0FFEE)
    want, st_ref = ref.generate(prompt, 40, temp=temp, top_p=top_p, seed=0xC0FFEE)
    assert got == want and st["stop"] == st_ref["stop"]
    assert _bits_equal(eng.logits(), ref.logits())
    # greedy afterwards is unaffected by the sampled run
    g1, _ = eng.generate(prompt, 8)
    g2, _ = ref.generate(prompt, 8)
    assert g1 == g2


def test_gqa_forward_logits(pih, backend, oracle, gqa, engine_mode):
    """Grouped-query attention and partial RoPE, batch-1 forwards: logits bit
    for bit at every position."""
    eng = pih.HipEngine(backend, gqa, n_ctx=128)
    assert backend.persistent_active() == (engine_mode == "persistent")
    ref = oracle.OracleEngine(gqa, n_ctx=128, threads=4)
    ids = [(i * 53 + 9) % 1000 for i in range(70)]
    for pos, tok in enumerate(ids):
        eng.forward([tok], [pos], want_logits=True)
        ref.forward([tok], [pos], want_logits=True)
        assert _bits_equal(eng.logits(), ref.logits()), f"pos {pos}"


def test_gqa_kv_rows_and_generate(pih, backend, oracle, gqa):
    """KV rows of every (layer, kv head) after a batched chunk, then greedy
    generate with a partial last chunk, against the oracle."""
    eng = pih.HipEngine(backend, gqa, n_ctx=160)
    ref = oracle.OracleEngine(gqa, n_ctx=160, threads=4)
    ids = [(i * 7 + 2) % 1000 for i in range(40)]
    eng.forward(ids, list(range(40)), want_logits=True)
    ref.forward(ids, list(range(40)), want_logits=True)
    assert _bits_equal(eng.logits(), ref.logits())
    kr, vr = ref.kv()
    for layer in range(gqa.spec.n_layer):
        for h in range(gqa.spec.n_head_kv):
            k, v = eng.kv_read(layer, h, 0, 40)
            assert _bits_equal(k, kr[layer, h, :40]) and _bits_equal(v, vr[layer, h, :40]), (layer, h)
    prompt = [(i * 31 + 4) % 1000 for i in range(45)]
    got, st = eng.generate(prompt, 40)
    want, st_ref = ref.generate(prompt, 40)
    assert got == want and st["stop"] == st_ref["stop"]
    assert _bits_equal(eng.logits(), ref.logits())


def test_minicpm2b_first_64_greedy_ids(pih, backend, engine_mode):
    """Full-size synthetic model; ids from the committed oracle fixture."""
    g = json.loads(GOLDEN.read_text())
    spec = pih.minicpm2b_spec()
    model = pih.synth_model(spec, g["model_seed"])
    import hashlib
    for name, h in g["tensor_sha256"].items():
        assert hashlib.sha256(model.tensors[name][3].tobytes()).hexdigest() == h, name
    eng = pih.HipEngine(backend, model, n_ctx=len(g["prompt"]) + g["n_gen"] + 8)
    assert backend.persistent_active() == (engine_mode == "persistent")
    ids, st = eng.generate(g["prompt"], g["n_gen"])
    assert ids == g["gen_ids"], f"first mismatch at {next(i for i, (a, b) in enumerate(zip(ids, g['gen_ids'])) if a != b)}"
