"""The GGUF reader (gguf.rs:113-336) and the model description built from it
(Config::from_gguf model.rs:31-97, Model::load / finish 487-601, the
tokenizer's vocabulary and end-of-generation ids tokenizer.rs:41-109).  CPU
only.

* A file assembled byte by byte here (independent of the test writer) with
  one metadata entry of every value type, a nested array, a 64-byte
  alignment and two tensors: every getter returns the written value and the
  tensor data start at the aligned data offset plus the tensor offset.
* Malformed files fail with the reference's errors, never read out of
  bounds: every truncation of a valid file, a bad magic, versions 1 and 4,
  implausible counts, an unknown value type, five dimensions, data past the
  end, a truncated tensor and a row length not divisible by the block.
* A synthetic model written by tests/gguf_writer.py gives back its own
  configuration, types, shapes, tensor bytes and end-of-generation ids, and
  the oracle bound to the file's tensors computes the same logits bit for
  bit as bound to the model.
"""
import struct

import numpy as np
import pytest

from gguf_writer import ARR, F32, GgufWriter, I32, STR, U32, synth_model_gguf

KV_TYPES = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8, "arr": 9,
            "u64": 10, "i64": 11, "f64": 12}


def s_(x: bytes) -> bytes:
    return struct.pack("<Q", len(x)) + x


def handmade() -> tuple:
    """(bytes, expected data offset) of a small v3 file."""
    kv = [
        (b"a.u8", 0, struct.pack("<B", 200)),
        (b"a.i8", 1, struct.pack("<b", -5)),
        (b"a.u16", 2, struct.pack("<H", 65535)),
        (b"a.i16", 3, struct.pack("<h", -300)),
        (b"a.u32", 4, struct.pack("<I", 4000000000)),
        (b"a.i32", 5, struct.pack("<i", -7)),
        (b"a.f32", 6, struct.pack("<f", 0.25)),
        (b"a.bool", 7, struct.pack("<B", 1)),
        (b"a.str", 8, s_("héllo".encode())),
        (b"a.strs", 9, struct.pack("<IQ", 8, 3) + s_(b"x") + s_(b"") + s_(b"yz")),
        (b"a.i32s", 9, struct.pack("<IQ", 5, 3) + struct.pack("<iii", 1, -2, 3)),
        (b"a.f32s", 9, struct.pack("<IQ", 6, 2) + struct.pack("<ff", 1.5, -0.5)),
        (b"a.nested", 9, struct.pack("<IQ", 9, 2) + struct.pack("<IQ", 4, 2) + struct.pack("<II", 1, 2) +
         struct.pack("<IQ", 8, 1) + s_(b"q")),
        (b"a.u64", 10, struct.pack("<Q", 2 ** 40 + 3)),
        (b"a.i64", 11, struct.pack("<q", -2 ** 40)),
        (b"a.f64", 12, struct.pack("<d", 1.0 / 3.0)),
        (b"general.alignment", 4, struct.pack("<I", 64)),
    ]
    tensors = [(b"w0", [64, 2], 8, 0), (b"w1", [3], 0, 192)]    # Q8_0 2x64 (136 B), F32 [3]
    out = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kv))
    for k, t, v in kv:
        out += s_(k) + struct.pack("<I", t) + v
    for name, ne, t, off in tensors:
        out += s_(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", t, off)
    data_off = (len(out) + 63) // 64 * 64
    out += b"\0" * (data_off - len(out))
    out += bytes(range(136)) + b"\0" * (192 - 136) + struct.pack("<fff", 1.0, 2.0, 3.0)
    return out, data_off


def test_handmade_known_answers(pih):
    data, data_off = handmade()
    g = pih.Gguf(data=data)
    assert g.version == 3 and g.data_offset == data_off and data_off % 64 == 0
    assert g.keys()[0] == "a.u8" and g.keys()[-1] == "general.alignment" and len(g.keys()) == 17
    assert g.get_u64("a.u8") == 200
    assert g.get_u64("a.i8") == (-5) % 2 ** 64                    # `as u64` sign-extends (gguf.rs:210-218)
    assert g.get_u64("a.u16") == 65535 and g.get_u64("a.i16") == (-300) % 2 ** 64
    assert g.get_u64("a.u32") == 4000000000 and g.get_u64("a.i32") == (-7) % 2 ** 64
    assert g.get_u64("a.u64") == 2 ** 40 + 3 and g.get_u64("a.i64") == (-2 ** 40) % 2 ** 64
    assert g.get_u64("a.f32") is None and g.get_u64("a.str") is None
    assert g.get_f32("a.f32") == 0.25 and abs(g.get_f32("a.f64") - 1.0 / 3.0) < 1e-7
    assert g.get_f32("a.u32") == 4000000000.0                    # integers convert (gguf.rs:229-235)
    assert g.get_bool("a.bool") is True and g.get_bool("a.u8") is True and g.get_bool("a.i32") is None
    assert g.get_str("a.str") == "héllo".encode() and g.get_str("a.u8") is None
    assert g.array_info("a.strs") == (8, 3) and g.array_strings("a.strs") == [b"x", b"", b"yz"]
    assert g.array_i32("a.i32s").tolist() == [1, -2, 3]
    assert g.array_f32("a.f32s").tolist() == [1.5, -0.5]
    assert g.array_info("a.nested") == (9, 2)
    assert g.kv_type("a.f64") == KV_TYPES["f64"] and g.kv_type("missing") is None
    assert g.n_tensors() == 2 and g.find("w1") == 1 and g.find("w2") == -1
    assert g.tensor_info(0) == {"name": "w0", "type": 8, "ne": [64, 2], "offset": 0}
    assert g.tensor_info(1) == {"name": "w1", "type": 0, "ne": [3], "offset": 192}
    assert g.tensor_data(0).tobytes() == bytes(range(136))       # tensor_nbytes: 2 rows x 2 blocks x 34
    assert np.frombuffer(g.tensor_data(1).tobytes(), np.float32).tolist() == [1.0, 2.0, 3.0]
    g.close()


def test_every_truncation_fails_cleanly(pih):
    data, data_off = handmade()
    for n in range(0, data_off):
        with pytest.raises(pih.PiError):
            pih.Gguf(data=data[:n])
    # header intact, tensor data cut: opening works, the tensor read fails
    g = pih.Gguf(data=data[: data_off + 100])
    with pytest.raises(pih.PiError, match="truncated"):
        g.tensor_data(0)


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b"GGUX" + b[4:], "not a GGUF file"),
    (lambda b: b[:4] + struct.pack("<I", 1) + b[8:], "unsupported GGUF version 1"),
    (lambda b: b[:4] + struct.pack("<I", 4) + b[8:], "unsupported GGUF version 4"),
    (lambda b: b[:8] + struct.pack("<Q", 2_000_000) + b[16:], "implausible"),
])
def test_bad_headers(pih, mutate, msg):
    data, _ = handmade()
    with pytest.raises(pih.PiError, match=msg):
        pih.Gguf(data=mutate(data))


def test_bad_metadata_and_tensors(pih):
    with pytest.raises(pih.PiError, match="unknown gguf metadata type 13"):
        pih.Gguf(data=struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + s_(b"k") + struct.pack("<I", 13))
    five = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + s_(b"t") + struct.pack("<I", 5) + b"\1\0\0\0\0\0\0\0" * 5
    with pytest.raises(pih.PiError, match="5 dims"):
        pih.Gguf(data=five + struct.pack("<IQ", 0, 0))
    w = GgufWriter()
    w.add_tensor("odd", 8, [48, 1], b"\0" * 34)          # 48 is not a multiple of the 32-element block
    g = pih.Gguf(data=w.to_bytes())
    with pytest.raises(pih.PiError, match="not divisible by block 32"):
        g.tensor_data(0)
    w = GgufWriter()
    w.add_tensor("far", 0, [4], b"\0" * 16)
    raw = bytearray(w.to_bytes())
    off_pos = raw.index(b"far") + 3 + 4 + 8 + 4           # name, n_dims, dim, type -> offset field
    raw[off_pos:off_pos + 8] = struct.pack("<Q", 10 ** 9)
    g = pih.Gguf(data=bytes(raw))
    with pytest.raises(pih.PiError, match="outside file"):
        g.tensor_data(0)


@pytest.fixture(scope="module")
def tiny_gqa(pih):
    spec = pih.tiny_spec(n_layer=2, n_embd=512, n_ff=1024, n_head=8, n_vocab=1000, n_head_kv=2, n_rot=32)
    return pih.synth_model(spec, seed=21)


def test_model_desc_round_trip(pih, tiny_gqa, tmp_path):
    path = tmp_path / "tiny.gguf"
    path.write_bytes(synth_model_gguf(tiny_gqa))
    g = pih.Gguf(path)
    d, _ = g.model_desc()
    s = tiny_gqa.spec
    assert (d.n_layer, d.n_embd, d.n_ff, d.n_head, d.n_head_kv, d.head_dim, d.n_rot, d.n_vocab) == \
        (s.n_layer, s.n_embd, s.n_ff, s.n_head, s.n_head_kv, s.head_dim, s.n_rot, s.n_vocab)
    assert d.rope_theta == np.float32(s.rope_theta) and d.rms_eps == np.float32(s.rms_eps)
    # eos_token_id and the control token "<|im_end|>" (the last id), sorted
    assert [d.eos_ids[i] for i in range(d.n_eos)] == sorted({s.eos_ids[0], s.n_vocab - 1})
    import ctypes
    names = {"attn_o": "attn_output"}
    for l in range(s.n_layer):
        for f in ("attn_q", "attn_k", "attn_v", "attn_o", "attn_norm", "ffn_gate", "ffn_up", "ffn_down", "ffn_norm"):
            td = getattr(d.layers[l], f)
            t, ne0, ne1, buf = tiny_gqa.tensors[f"blk.{l}.{names.get(f, f)}.weight"]
            assert (td.type, td.ne0, td.ne1) == (t, ne0, ne1), (l, f)
            assert ctypes.string_at(td.data, buf.nbytes) == buf.tobytes(), (l, f)
    g.close()


def test_tied_output_and_missing_tensors(pih, tiny_gqa):
    g = pih.Gguf(data=synth_model_gguf(tiny_gqa, tie_output=True))
    d, _ = g.model_desc()
    assert d.output.data == d.token_embd.data and d.output.type == d.token_embd.type   # model.rs:526-530
    w = GgufWriter()
    w.add("general.architecture", STR, "llama")
    with pytest.raises(pih.PiError, match="missing metadata llama.block_count"):
        pih.Gguf(data=w.to_bytes()).model_desc()
    raw = synth_model_gguf(tiny_gqa).replace(b"blk.1.ffn_up.weight", b"blk.1.ffn_UP.weight")
    with pytest.raises(pih.PiError, match="missing tensor blk.1.ffn_up.weight"):
        pih.Gguf(data=raw).model_desc()


def test_config_checks(pih, tiny_gqa):
    def with_meta(key, t, v):
        w = GgufWriter()
        for k, tt, vv in (("general.architecture", STR, "llama"), ("llama.block_count", U32, 2),
                          ("llama.embedding_length", U32, 512), ("llama.feed_forward_length", U32, 1024),
                          ("llama.attention.head_count", U32, 8), ("tokenizer.ggml.tokens", ARR, (STR, ["a"]))):
            if k != key:
                w.add(k, tt, vv)
        w.add(key, t, v)
        return pih.Gguf(data=w.to_bytes())
    with pytest.raises(pih.PiError, match="invalid GQA configuration"):
        with_meta("llama.attention.head_count_kv", U32, 3).model_desc()
    with pytest.raises(pih.PiError, match="invalid RoPE"):
        with_meta("llama.rope.dimension_count", U32, 65).model_desc()
    with pytest.raises(pih.PiError, match="invalid RoPE"):
        with_meta("llama.attention.layer_norm_rms_epsilon", F32, -1.0).model_desc()
    with pytest.raises(pih.PiError, match="value head dimension"):
        with_meta("llama.attention.value_length", U32, 32).model_desc()
    with pytest.raises(pih.PiError, match="zero layer"):
        with_meta("llama.block_count", U32, 0).model_desc()


def _synth_from_gguf(pih, g):
    """A SynthModel whose tensors are views of the file's mapping."""
    d, keep = g.model_desc()
    m = pih.SynthModel(g.spec())
    for i in range(g.n_tensors()):
        info = g.tensor_info(i)
        ne1 = info["ne"][1] if len(info["ne"]) > 1 else 1
        buf = g.tensor_data(i)
        m.tensors[info["name"]] = (info["type"], info["ne"][0], ne1, buf.view(np.float32) if info["type"] == 0 else buf)
    return m


def test_oracle_on_file_tensors_matches_model(pih, oracle, tiny_gqa):
    g = pih.Gguf(data=synth_model_gguf(tiny_gqa))
    m = _synth_from_gguf(pih, g)
    a = oracle.OracleEngine(tiny_gqa, n_ctx=64, threads=2)
    b = oracle.OracleEngine(m, n_ctx=64, threads=2)
    for pos, tok in enumerate([3, 999, 17, 400]):
        a.forward([tok], [pos], want_logits=True)
        b.forward([tok], [pos], want_logits=True)
        assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32)), pos
