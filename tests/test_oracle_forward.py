"""Pins the oracle's forward pass and integer block sums against independent
float64 / integer numpy restatements of the textbook forms (CPU only).

* Forward: embedding (model.rs:857-869), RMSNorm (777-823), adjacent-pair
  RoPE with inv_i = theta^(-2i/n_rot) (413-417, 953-979), KV write (984-992),
  causal softmax attention with scale 1/sqrt(dh) (993-1087), residuals
  (1095-1097, 1123-1125), SwiGLU (1111-1115), output norm + head
  (1131-1170).  The oracle runs its f32-activation path (int8 off), so the
  only differences from the float64 model are f32 rounding: 1e-4 relative to
  the largest logit.  Planted mistakes in a copy of the numpy model (NeoX
  pair order, a dropped residual, a missing 1/sqrt(dh), the norm weight
  left out) must each exceed that tolerance, which shows the check can
  catch them.
* Block sums: integer weights unpacked straight from the GGML byte layouts
  (quant.rs:129-322) and dotted with the Q8 quants in int64.
* Greedy sample: first index of the maximum (sampler.rs:26-36).
"""
import numpy as np
import pytest

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14


@pytest.fixture(scope="module")
def tiny(pih):
    return pih.synth_model(pih.tiny_spec(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_vocab=1000), seed=11)


@pytest.fixture(scope="module")
def gqa(pih):
    """Grouped-query attention (8 query heads over 2 KV heads, model.rs:995
    kh = h / group) with RoPE on the first 32 of 64 dimensions (n_rot,
    model.rs:930, 953-979)."""
    return pih.synth_model(pih.tiny_spec(n_layer=2, n_embd=512, n_ff=1024, n_head=8, n_vocab=1000, n_head_kv=2,
                                         n_rot=32), seed=13)


def _deq(oracle, entry):
    t, ne0, ne1, buf = entry
    if t == 0:
        return np.asarray(buf, np.float64).reshape(ne1, ne0)
    raw = buf.view(np.uint8)
    rb = raw.size // ne1
    return np.stack([oracle.dequant_row(t, raw[r * rb:(r + 1) * rb], ne0) for r in range(ne1)]).astype(np.float64)


class NumpyModel:
    """Float64 decoder over dequantized weights; `mutate` plants one mistake."""

    def __init__(self, oracle, model, mutate=None):
        s = model.spec
        self.s, self.mutate = s, mutate
        T = model.tensors
        self.embd = _deq(oracle, T["token_embd.weight"])
        self.out = _deq(oracle, T["output.weight"])
        self.out_norm = _deq(oracle, T["output_norm.weight"])[0]
        self.layers = []
        for l in range(s.n_layer):
            g = lambda n: _deq(oracle, T[f"blk.{l}.{n}.weight"])  # noqa: E731
            self.layers.append({n: g(n) for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate",
                                                    "ffn_up", "ffn_down")})
            self.layers[-1]["attn_norm"] = g("attn_norm")[0]
            self.layers[-1]["ffn_norm"] = g("ffn_norm")[0]
        self.kc = [[] for _ in range(s.n_layer)]
        self.vc = [[] for _ in range(s.n_layer)]

    def _norm(self, x, w):
        y = x / np.sqrt(np.mean(x * x) + self.s.rms_eps)
        return y if self.mutate == "no_norm_weight" else y * w

    def _rope(self, v, pos):
        s = self.s
        dh, half = s.head_dim, s.n_rot // 2
        v = v.reshape(-1, dh).copy()
        inv = s.rope_theta ** (-2.0 * np.arange(half) / s.n_rot)
        c, sn = np.cos(pos * inv), np.sin(pos * inv)
        if self.mutate == "rope_all_dims":
            half = dh // 2
            inv = s.rope_theta ** (-2.0 * np.arange(half) / dh)
            c, sn = np.cos(pos * inv), np.sin(pos * inv)
        if self.mutate == "neox_pairs":
            i0, i1 = np.arange(half), np.arange(half) + half
        else:
            i0, i1 = 2 * np.arange(half), 2 * np.arange(half) + 1
        x0, x1 = v[:, i0].copy(), v[:, i1].copy()
        v[:, i0] = x0 * c - x1 * sn
        v[:, i1] = x0 * sn + x1 * c
        return v.reshape(-1)

    def step(self, tok, pos):
        s = self.s
        dh = s.head_dim
        x = self.embd[tok].copy()
        for l, L in enumerate(self.layers):
            xn = self._norm(x, L["attn_norm"])
            q = self._rope(L["attn_q"] @ xn, pos).reshape(s.n_head, dh)
            k = self._rope(L["attn_k"] @ xn, pos).reshape(s.n_head_kv, dh)
            v = (L["attn_v"] @ xn).reshape(s.n_head_kv, dh)
            self.kc[l].append(k)
            self.vc[l].append(v)
            K, V = np.stack(self.kc[l], 1), np.stack(self.vc[l], 1)      # [kv][pos][dh]
            group = s.n_head // s.n_head_kv
            scale = 1.0 if self.mutate == "no_scale" else 1.0 / np.sqrt(dh)
            o = np.empty((s.n_head, dh))
            for h in range(s.n_head):
                kh = h % s.n_head_kv if self.mutate == "kv_head_mod" else h // group
                sc = K[kh] @ q[h] * scale
                e = np.exp(sc - sc.max())
                o[h] = (e / e.sum()) @ V[kh]
            proj = L["attn_output"] @ o.reshape(-1)
            x = proj if self.mutate == "no_residual" else x + proj
            xn = self._norm(x, L["ffn_norm"])
            g, u = L["ffn_gate"] @ xn, L["ffn_up"] @ xn
            x = x + L["ffn_down"] @ (g / (1.0 + np.exp(-g)) * u)
        return self.out @ self._norm(x, self.out_norm)


def _oracle_logits(oracle, model, ids):
    eng = oracle.OracleEngine(model, n_ctx=64, threads=2)
    eng.set_int8(False)
    out = []
    for pos, tok in enumerate(ids):
        eng.forward([tok], [pos], want_logits=True)
        out.append(eng.logits().astype(np.float64))
    eng.close()
    return out


IDS = [5, 999, 17, 0, 321, 17, 64, 800]


def _max_rel(got, want):
    return max(float(np.max(np.abs(g - w)) / np.max(np.abs(w))) for g, w in zip(got, want))


def test_forward_matches_float64_model(oracle, tiny):
    got = _oracle_logits(oracle, tiny, IDS)
    m = NumpyModel(oracle, tiny)
    want = [m.step(t, p) for p, t in enumerate(IDS)]
    assert _max_rel(got, want) < 1e-4


@pytest.mark.parametrize("mutate", ["neox_pairs", "no_residual", "no_scale", "no_norm_weight"])
def test_planted_mistakes_are_caught(oracle, tiny, mutate):
    got = _oracle_logits(oracle, tiny, IDS)
    m = NumpyModel(oracle, tiny, mutate)
    want = [m.step(t, p) for p, t in enumerate(IDS)]
    assert _max_rel(got, want) > 1e-3, mutate


def test_gqa_partial_rope_forward_matches_float64_model(oracle, gqa):
    got = _oracle_logits(oracle, gqa, IDS)
    m = NumpyModel(oracle, gqa)
    want = [m.step(t, p) for p, t in enumerate(IDS)]
    assert _max_rel(got, want) < 1e-4


@pytest.mark.parametrize("mutate", ["kv_head_mod", "rope_all_dims", "neox_pairs"])
def test_gqa_planted_mistakes_are_caught(oracle, gqa, mutate):
    """Query head h must read KV head h / group (not h mod n_kv), and only
    the first n_rot dimensions rotate."""
    got = _oracle_logits(oracle, gqa, IDS)
    m = NumpyModel(oracle, gqa, mutate)
    want = [m.step(t, p) for p, t in enumerate(IDS)]
    assert _max_rel(got, want) > 1e-3, mutate


def _int_weights(t, row, k):
    """Integer weights of one row straight from the GGML byte layout."""
    b = row.view(np.uint8)
    if t == Q8_0:
        blk = b.reshape(-1, 34)
        return blk[:, 2:].view(np.int8).astype(np.int64).reshape(-1)
    if t == Q4_0:
        blk = b.reshape(-1, 18)[:, 2:]
        return np.concatenate([blk & 0xF, blk >> 4], 1).astype(np.int64).reshape(-1)
    if t == Q4_K:
        qs = b.reshape(-1, 144)[:, 16:].reshape(-1, 4, 32)                 # 4 groups of 32 bytes
        return np.stack([qs & 0xF, qs >> 4], 2).astype(np.int64).reshape(-1)   # lo -> 2g, hi -> 2g+1
    if t == Q6_K:
        blk = b.reshape(-1, 210)
        out = np.empty((blk.shape[0], 256), np.int64)
        for hf in range(2):
            ql = blk[:, hf * 64:hf * 64 + 64].astype(np.int64)
            qh = blk[:, 128 + hf * 32:128 + hf * 32 + 32].astype(np.int64)
            for s4 in range(4):
                lo = (ql[:, (s4 & 1) * 32:(s4 & 1) * 32 + 32] >> (4 * (s4 >> 1))) & 0xF
                hi = (qh >> (2 * s4)) & 3
                out[:, hf * 128 + s4 * 32:hf * 128 + s4 * 32 + 32] = (lo | (hi << 4)) - 32
        return out.reshape(-1)
    raise ValueError(t)


@pytest.mark.parametrize("t,k", [(Q8_0, 256), (Q4_0, 512), (Q4_K, 512), (Q6_K, 768)])
def test_block_sums_brute_force(pih, oracle, t, k):
    row = pih.synth_tensor(5, t, 1, k, 0.0, 0.02) if t in (Q8_0, Q4_0) else \
        (pih.synth_q4k_random(5, 1, k) if t == Q4_K else pih.synth_q6k_random(5, 1, k))
    x = np.random.default_rng(t).standard_normal(k).astype(np.float32)
    act = oracle.Act(x, k, 1)
    got = oracle.block_sums(t, row, k, act)
    prod = _int_weights(t, row, k) * act.q.astype(np.int64)
    if t == Q6_K:
        # 16-element sums in the q6_k_lanes visiting order: half, g, s
        p = prod.reshape(-1, 2, 4, 2, 16)                                # blk, half, s, g, 16
        want = p.sum(-1).transpose(0, 1, 3, 2).reshape(-1)
    else:
        want = prod.reshape(-1, 32).sum(1)
    assert np.array_equal(got.astype(np.int64), want)


def test_greedy_sample_first_max(oracle):
    v = np.array([0.1, 3.0, -1.0, 3.0, 2.9], np.float32)
    assert oracle.sample(v, 0.0, 1.0, 1) == 1
    v = np.full(1000, -5.0, np.float32)
    v[[700, 123, 999]] = 7.25
    assert oracle.sample(v, 0.0, 1.0, 1) == 123
