"""The device engine bound from a GGUF file (Engine::load, model.rs:487-601
and 678-760): the file is mapped, its tensors are uploaded from the mapping,
and the engine computes what the same weights bound from host arrays
compute, bit for bit, through prefill, decode and prefix reuse
(tests/prefix_cache.rs:27-63).
"""
import numpy as np
import pytest

from gguf_writer import synth_model_gguf

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gqa(pih):
    return pih.synth_model(pih.tiny_spec(n_layer=2, n_embd=512, n_ff=1024, n_head=8, n_vocab=1000, n_head_kv=2,
                                         n_rot=32), seed=23)


@pytest.fixture(scope="module")
def gguf_path(gqa, tmp_path_factory):
    p = tmp_path_factory.mktemp("gguf") / "gqa.gguf"
    p.write_bytes(synth_model_gguf(gqa))
    return p


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_gguf_engine_equals_host_engine(pih, backend, oracle, gqa, gguf_path):
    ids = [(i * 53 + 9) % 1000 for i in range(40)]
    host = pih.HipEngine(backend, gqa, n_ctx=128)
    want = []
    for pos, tok in enumerate(ids):
        host.forward([tok], [pos], want_logits=True)
        want.append(host.logits())
    g = pih.Gguf(gguf_path)
    eng = pih.HipEngine(backend, g, n_ctx=128)
    assert eng.model.spec.n_head_kv == 2 and eng.model.spec.n_rot == 32 and eng.model.spec.eos_ids == (999,)
    for pos, tok in enumerate(ids):
        eng.forward([tok], [pos], want_logits=True)
        assert np.array_equal(_bits(eng.logits()), _bits(want[pos])), pos
    # a batched chunk and greedy generate against the oracle on the host tensors
    ref = oracle.OracleEngine(gqa, n_ctx=128, threads=4)
    prompt = [(i * 31 + 4) % 1000 for i in range(45)]
    got, st = eng.generate(prompt, 30)
    exp, st_ref = ref.generate(prompt, 30)
    assert got == exp and st["stop"] == st_ref["stop"]
    assert np.array_equal(_bits(eng.logits()), _bits(ref.logits()))


def test_gguf_engine_prefix_reuse(pih, backend, oracle, gqa, gguf_path):
    """prefix_cache.rs:27-63 on the file-bound engine: a 64-token aligned
    prefix is reused and the ids and logits equal a fresh run's."""
    base = [(i * 13 + 5) % 997 for i in range(70)]
    ext = base + [(i * 7 + 1) % 991 for i in range(40)]
    ref = oracle.OracleEngine(gqa, n_ctx=256, threads=4)
    want, _ = ref.generate(ext, 4)
    eng = pih.HipEngine(backend, pih.Gguf(gguf_path), n_ctx=256)
    eng.generate(base, 2)
    ids, st = eng.generate(ext, 4)
    assert st["prefill_cached_tokens"] == 64 and st["prefill_tokens"] == len(ext) - 64
    assert ids == want and np.array_equal(_bits(eng.logits()), _bits(ref.logits()))


def test_gguf_tied_output(pih, backend, oracle, gqa):
    """No output.weight: the head is token_embd (model.rs:526-530)."""
    tied = pih.SynthModel(gqa.spec, dict(gqa.tensors))
    tied.tensors["output.weight"] = tied.tensors["token_embd.weight"]
    eng = pih.HipEngine(backend, pih.Gguf(data=synth_model_gguf(gqa, tie_output=True)), n_ctx=64)
    ref = oracle.OracleEngine(tied, n_ctx=64, threads=4)
    prompt = [(i * 17 + 2) % 1000 for i in range(33)]
    got, _ = eng.generate(prompt, 12)
    exp, _ = ref.generate(prompt, 12)
    assert got == exp and np.array_equal(_bits(eng.logits()), _bits(ref.logits()))
