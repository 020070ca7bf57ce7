"""Minimal GGUF v3 writer (test infrastructure).

Written from the GGUF file format: little-endian header (magic "GGUF",
version, tensor count, metadata count), metadata entries (u64-length
string key, u32 value type, value; strings are u64 length + bytes, arrays
u32 element type + u64 count + elements), tensor infos (name, u32 dim
count, u64 dims, u32 type, u64 offset from the data start), zero padding to
`general.alignment` (32 by default), then the tensor data, each tensor at an
aligned offset.  It writes the synthetic models the tests bind, in the
tensor names and metadata keys Model::load and Config::from_gguf read
(model.rs:31-97, 487-569), with a byte-string vocabulary for the tokenizer
fields (tokenizer.rs:41-109).
"""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v) -> bytes:
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_FMT[t], v)


class GgufWriter:
    def __init__(self, alignment: int = 32, version: int = 3):
        self.alignment, self.version = alignment, version
        self.kv, self.tensors = [], []
        if alignment != 32:
            self.kv.append(("general.alignment", U32, alignment))

    def add(self, key: str, t: int, value) -> None:
        self.kv.append((key, t, value))

    def add_tensor(self, name: str, ttype: int, ne, data) -> None:
        self.tensors.append((name, ttype, list(ne), bytes(data)))

    def to_bytes(self) -> bytes:
        out = struct.pack("<IIQQ", 0x46554747, self.version, len(self.tensors), len(self.kv))
        for key, t, v in self.kv:
            out += _str(key) + struct.pack("<I", t) + _value(t, v)
        offs, pos = [], 0
        for _, _, _, data in self.tensors:
            offs.append(pos)
            pos = (pos + len(data) + self.alignment - 1) // self.alignment * self.alignment
        for (name, ttype, ne, _), off in zip(self.tensors, offs):
            out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
            out += struct.pack("<IQ", ttype, off)
        out += b"\0" * (-len(out) % self.alignment)
        base = len(out)
        for (_, _, _, data), off in zip(self.tensors, offs):
            assert len(out) - base == off
            out += data + b"\0" * (-len(data) % self.alignment)
        return out


def synth_model_gguf(model, arch: str = "llama", specials=("<|im_end|>",), tie_output: bool = False) -> bytes:
    """GGUF bytes of a pocketinfer_hip.SynthModel: the model's tensors under
    their GGUF names, Config keys of `arch`, and a vocabulary of byte-string
    tokens whose last len(specials) entries are control tokens (type 3) named
    by `specials`; tokenizer.ggml.eos_token_id is the spec's first eos id."""
    s = model.spec
    w = GgufWriter()
    w.add("general.architecture", STR, arch)
    w.add("general.name", STR, "synthetic")
    p = arch + "."
    w.add(p + "block_count", U32, s.n_layer)
    w.add(p + "embedding_length", U32, s.n_embd)
    w.add(p + "feed_forward_length", U32, s.n_ff)
    w.add(p + "attention.head_count", U32, s.n_head)
    w.add(p + "attention.head_count_kv", U32, s.n_head_kv)
    w.add(p + "rope.dimension_count", U32, s.n_rot)
    w.add(p + "rope.freq_base", F32, s.rope_theta)
    w.add(p + "attention.layer_norm_rms_epsilon", F32, s.rms_eps)
    w.add(p + "context_length", U32, 4096)
    toks = [f"t{i}" for i in range(s.n_vocab - len(specials))] + list(specials)
    types = [1] * (s.n_vocab - len(specials)) + [3] * len(specials)
    w.add("tokenizer.ggml.model", STR, "gpt2")
    w.add("tokenizer.ggml.tokens", ARR, (STR, toks))
    w.add("tokenizer.ggml.token_type", ARR, (I32, types))
    if s.eos_ids:
        w.add("tokenizer.ggml.eos_token_id", U32, s.eos_ids[0])
    for name, (t, ne0, ne1, buf) in model.tensors.items():
        if tie_output and name == "output.weight":
            continue
        ne = [ne0] if ne1 == 1 and name.endswith("norm.weight") else [ne0, ne1]
        w.add_tensor(name, t, ne, buf.tobytes())
    return w.to_bytes()
