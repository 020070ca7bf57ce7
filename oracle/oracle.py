"""ctypes binding of the CPU oracle (oracle/libpi_oracle.so).

TEST INFRASTRUCTURE, NOT PRODUCT CODE: only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg load this module.  It restates the reference
engine's CPU path (see pi_oracle.h for the file:line of each function).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libpi_oracle.so"

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 0, 1, 2, 3, 6, 7, 8, 9
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, BF16 = 10, 11, 12, 13, 14, 15, 30

_lib = None


def build() -> None:
    subprocess.run(["make", "-C", str(HERE)], check=True, stdout=subprocess.DEVNULL)


class Q8Act(C.Structure):
    _fields_ = [("q", C.c_void_p), ("d", C.c_void_p), ("sum", C.c_void_p),
                ("k", C.c_size_t), ("b", C.c_size_t), ("nb", C.c_size_t)]


class PoTensor(C.Structure):
    _fields_ = [("type", C.c_uint32), ("ne0", C.c_size_t), ("ne1", C.c_size_t), ("data", C.c_void_p)]


class PoLayer(C.Structure):
    _fields_ = [(n, PoTensor) for n in ("attn_q", "attn_k", "attn_v", "attn_o", "attn_norm",
                                        "ffn_gate", "ffn_up", "ffn_down", "ffn_norm")]


class PoModel(C.Structure):
    _fields_ = [("n_layer", C.c_size_t), ("n_embd", C.c_size_t), ("n_ff", C.c_size_t), ("n_head", C.c_size_t),
                ("n_head_kv", C.c_size_t), ("head_dim", C.c_size_t), ("n_rot", C.c_size_t),
                ("n_vocab", C.c_size_t), ("rope_theta", C.c_float), ("rms_eps", C.c_float),
                ("eos_ids", C.POINTER(C.c_uint32)), ("n_eos", C.c_size_t),
                ("token_embd", PoTensor), ("output", PoTensor), ("output_norm", PoTensor),
                ("layers", C.POINTER(PoLayer))]


class PoGenOpts(C.Structure):
    _fields_ = [("max_tokens", C.c_size_t), ("temp", C.c_float), ("top_p", C.c_float), ("seed", C.c_uint64)]


class PoGenStats(C.Structure):
    _fields_ = [("prefill_tokens", C.c_size_t), ("prefill_cached_tokens", C.c_size_t), ("gen_tokens", C.c_size_t),
                ("prefill_ms", C.c_double), ("gen_ms", C.c_double), ("stop", C.c_char * 32)]


class PoRng(C.Structure):
    _fields_ = [("s", C.c_uint64)]


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        vp, sz = C.c_void_p, C.c_size_t
        L.po_f16_to_f32.restype, L.po_f16_to_f32.argtypes = C.c_float, [C.c_uint16]
        L.po_f32_to_f16.restype, L.po_f32_to_f16.argtypes = C.c_uint16, [C.c_float]
        L.po_q8_prepare.restype, L.po_q8_prepare.argtypes = None, [vp, sz, sz, vp, vp, vp]
        L.po_dot_row_q8.restype, L.po_dot_row_q8.argtypes = C.c_float, [C.c_uint32, vp, sz, C.POINTER(Q8Act), sz]
        L.po_dot_row_q8_lanes.restype = None
        L.po_dot_row_q8_lanes.argtypes = [C.c_uint32, vp, sz, C.POINTER(Q8Act), vp, sz]
        L.po_block_sums.restype = C.c_long
        L.po_block_sums.argtypes = [C.c_uint32, vp, sz, C.POINTER(Q8Act), sz, vp]
        L.po_dequant_row.restype, L.po_dequant_row.argtypes = None, [C.c_uint32, vp, sz, vp]
        L.po_dot_row_scalar.restype, L.po_dot_row_scalar.argtypes = C.c_float, [C.c_uint32, vp, sz, vp]
        L.po_row_dot_multi.restype, L.po_row_dot_multi.argtypes = None, [C.c_uint32, vp, sz, vp, sz, vp]
        L.po_pool_new.restype, L.po_pool_new.argtypes = vp, [C.c_int]
        L.po_pool_free.restype, L.po_pool_free.argtypes = None, [vp]
        L.po_pool_matmul.restype = None
        L.po_pool_matmul.argtypes = [vp, C.c_uint32, vp, sz, sz, vp, sz, vp, sz, C.POINTER(Q8Act)]
        L.po_rng_init.restype, L.po_rng_init.argtypes = None, [C.POINTER(PoRng), C.c_uint64]
        L.po_rng_next_u64.restype, L.po_rng_next_u64.argtypes = C.c_uint64, [C.POINTER(PoRng)]
        L.po_rng_next_f32.restype, L.po_rng_next_f32.argtypes = C.c_float, [C.POINTER(PoRng)]
        L.po_sample.restype = C.c_uint32
        L.po_sample.argtypes = [vp, sz, C.c_float, C.c_float, C.POINTER(PoRng)]
        L.po_engine_create.restype = vp
        L.po_engine_create.argtypes = [C.POINTER(PoModel), sz, C.c_int, C.c_char_p, sz]
        L.po_engine_destroy.restype, L.po_engine_destroy.argtypes = None, [vp]
        L.po_engine_set_int8.restype, L.po_engine_set_int8.argtypes = None, [vp, C.c_int]
        L.po_forward.restype, L.po_forward.argtypes = C.c_int, [vp, vp, vp, sz, C.c_int]
        L.po_logits.restype, L.po_logits.argtypes = C.POINTER(C.c_float), [vp]
        L.po_n_logits.restype, L.po_n_logits.argtypes = sz, [vp]
        L.po_kv_k.restype, L.po_kv_k.argtypes = C.POINTER(C.c_float), [vp]
        L.po_kv_v.restype, L.po_kv_v.argtypes = C.POINTER(C.c_float), [vp]
        L.po_kv_index.restype, L.po_kv_index.argtypes = sz, [vp, sz, sz, sz, sz]
        L.po_last_error.restype, L.po_last_error.argtypes = C.c_char_p, [vp]
        L.po_generate.restype = C.c_int
        L.po_generate.argtypes = [vp, vp, sz, C.POINTER(PoGenOpts), C.POINTER(PoGenStats), vp]
        for fn in ("po_det_expf", "po_det_cosf", "po_det_sinf"):
            getattr(L, fn).restype, getattr(L, fn).argtypes = C.c_float, [C.c_float]
        L.po_det_powf.restype, L.po_det_powf.argtypes = C.c_float, [C.c_float, C.c_float]
        L.po_request_stop.restype, L.po_request_stop.argtypes = None, []
        L.po_clear_stop.restype, L.po_clear_stop.argtypes = None, []
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# -- scalar helpers -----------------------------------------------------------
def f16_to_f32(h: int) -> float:
    return lib().po_f16_to_f32(h)


def f32_to_f16(v: float) -> int:
    return lib().po_f32_to_f16(v)


class Act:
    """Q8Act (quant_int.rs:3-62) owning its arrays."""

    def __init__(self, x: np.ndarray, k: int, b: int):
        x = np.ascontiguousarray(x, np.float32)
        assert x.size == k * b
        self.k, self.b, self.nb = k, b, k // 32
        self.q = np.empty(k * b, np.int8)
        self.d = np.empty(self.nb * b, np.float32)
        self.sum = np.empty(self.nb * b, np.int32)
        lib().po_q8_prepare(_p(x), k, b, _p(self.q), _p(self.d), _p(self.sum))
        self.s = Q8Act(_p(self.q), _p(self.d), _p(self.sum), k, b, self.nb)

    @classmethod
    def from_arrays(cls, q, d, s, k, b):
        a = cls.__new__(cls)
        a.k, a.b, a.nb = k, b, k // 32
        a.q, a.d, a.sum = (np.ascontiguousarray(v) for v in (q, d, s))
        a.s = Q8Act(_p(a.q), _p(a.d), _p(a.sum), k, b, a.nb)
        return a


def dot_row_q8(t: int, row: np.ndarray, k: int, act: Act, lane: int = 0) -> float:
    return lib().po_dot_row_q8(t, _p(row), k, C.byref(act.s), lane)


def dot_row_q8_lanes(t: int, row: np.ndarray, k: int, act: Act) -> np.ndarray:
    out = np.zeros(act.b, np.float32)
    lib().po_dot_row_q8_lanes(t, _p(row), k, C.byref(act.s), _p(out), act.b)
    return out


def block_sums(t: int, row: np.ndarray, k: int, act: Act, lane: int = 0) -> np.ndarray:
    out = np.empty(k // 16, np.int32)
    n = lib().po_block_sums(t, _p(row), k, C.byref(act.s), lane, _p(out))
    assert n >= 0
    return out[:n].copy()


def dequant_row(t: int, data: np.ndarray, k: int) -> np.ndarray:
    out = np.empty(k, np.float32)
    lib().po_dequant_row(t, _p(data), k, _p(out))
    return out


def dot_row(t: int, data: np.ndarray, k: int, x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, np.float32)
    return lib().po_dot_row_scalar(t, _p(data), k, _p(x))


def row_dot_multi(t: int, row: np.ndarray, k: int, xt: np.ndarray, b: int) -> np.ndarray:
    xt = np.ascontiguousarray(xt, np.float32)
    out = np.zeros(b, np.float32)
    lib().po_row_dot_multi(t, _p(row), k, _p(xt), b, _p(out))
    return out


class Pool:
    def __init__(self, threads: int):
        self.h = lib().po_pool_new(threads)

    def matmul(self, t, w: np.ndarray, row_bytes: int, k: int, x: np.ndarray, b: int, rows: int,
               act: Act | None) -> np.ndarray:
        out = np.empty(rows * b, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        lib().po_pool_matmul(self.h, t, _p(w), row_bytes, k, _p(x), b, _p(out), rows,
                             C.byref(act.s) if act is not None else None)
        return out

    def close(self):
        if self.h:
            lib().po_pool_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sample(logits: np.ndarray, temp: float, top_p: float, seed: int) -> int:
    v = np.array(logits, np.float32)
    r = PoRng()
    lib().po_rng_init(C.byref(r), seed)
    return lib().po_sample(_p(v), v.size, temp, top_p, C.byref(r))


class OracleEngine:
    """Engine (model.rs:678-1352) restated on the CPU, over the same host
    tensors a HipEngine is bound to (a pocketinfer_hip.SynthModel)."""

    def __init__(self, model, n_ctx: int, threads: int = 8):
        s = model.spec
        T = model.tensors
        self.model = model

        def td(name):
            t, ne0, ne1, buf = T[name]
            return PoTensor(t, ne0, ne1, buf.ctypes.data)

        self._layers = (PoLayer * s.n_layer)()
        names = {"attn_o": "attn_output"}
        for l in range(s.n_layer):
            for f in PoLayer._fields_:
                fn = f[0]
                setattr(self._layers[l], fn, td(f"blk.{l}.{names.get(fn, fn)}.weight"))
        self._eos = (C.c_uint32 * max(1, len(s.eos_ids)))(*s.eos_ids)
        self._m = PoModel(s.n_layer, s.n_embd, s.n_ff, s.n_head, s.n_head_kv, s.head_dim, s.n_rot, s.n_vocab,
                          s.rope_theta, s.rms_eps, self._eos, len(s.eos_ids), td("token_embd.weight"),
                          td("output.weight"), td("output_norm.weight"), self._layers)
        err = C.create_string_buffer(256)
        self.h = lib().po_engine_create(C.byref(self._m), n_ctx, threads, err, 256)
        if not self.h:
            raise RuntimeError(err.value.decode())
        self.n_ctx = n_ctx

    def forward(self, ids, positions, want_logits=True) -> None:
        ids = np.ascontiguousarray(ids, np.uint32)
        pos = np.ascontiguousarray(positions, np.uint64)
        rc = lib().po_forward(self.h, _p(ids), _p(pos), ids.size, int(want_logits))
        if rc:
            raise RuntimeError(lib().po_last_error(self.h).decode())

    def set_int8(self, enabled: bool) -> None:
        """Engine int8 toggle (model.rs:689-694): False selects the f32 path."""
        lib().po_engine_set_int8(self.h, int(enabled))

    def logits(self) -> np.ndarray:
        n = self.model.spec.n_vocab
        return np.ctypeslib.as_array(lib().po_logits(self.h), (n,)).copy()

    def generate(self, prompt, max_tokens: int, temp=0.0, top_p=1.0, seed=1):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        ids = np.zeros(max(1, max_tokens), np.uint32)
        st = PoGenStats()
        rc = lib().po_generate(self.h, _p(prompt), prompt.size, C.byref(PoGenOpts(max_tokens, temp, top_p, seed)),
                               C.byref(st), _p(ids))
        if rc:
            raise RuntimeError(lib().po_last_error(self.h).decode())
        stats = {"prefill_tokens": st.prefill_tokens, "prefill_cached_tokens": st.prefill_cached_tokens,
                 "gen_tokens": st.gen_tokens, "prefill_ms": st.prefill_ms, "gen_ms": st.gen_ms,
                 "stop": st.stop.decode()}
        return ids[: st.gen_tokens].tolist(), stats

    def kv(self):
        s = self.model.spec
        n = s.n_layer * s.n_head_kv * self.n_ctx * s.head_dim
        k = np.ctypeslib.as_array(lib().po_kv_k(self.h), (n,))
        v = np.ctypeslib.as_array(lib().po_kv_v(self.h), (n,))
        shape = (s.n_layer, s.n_head_kv, self.n_ctx, s.head_dim)
        return k.reshape(shape), v.reshape(shape)

    def close(self):
        if self.h:
            lib().po_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def request_stop() -> None:
    lib().po_request_stop()


def clear_stop() -> None:
    lib().po_clear_stop()
