"""Python binding of libpocketinfer_hip.so (the MI355X decode backend).

A thin ctypes layer over the C ABI in include/pocketinfer_hip.h.  It mirrors
the reference engine's backend interface so callers read like the reference:

* ``HipBackend`` -- the OpenClBackend twin (rust/pocketinfer/src/backend/
  opencl.rs:79-516): ``probe``, ``new``, ``name``, ``supports``, ``selftest``,
  ``matvec``; plus explicit upload, device-pointer GEMV and test hooks.
* ``HipEngine`` -- the device-resident Engine (model.rs:678-1352):
  ``forward``, ``logits``, ``argmax``, ``generate``, KV access.
* ``synth_*`` -- seeded synthetic weights, including the MiniCPM-2B-shaped
  Q4_K_M model (40 layers, hidden 2304, 36x64 MHA, FFN 5760, vocab 122753).

There is no CPU fallback here: a missing library or device raises.
"""
from __future__ import annotations

import ctypes as C
import os
import sys
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libpocketinfer_hip.so"

# GGML type ids (quant.rs:3-17)
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K, Q8_K, BF16 = 3, 6, 7, 9, 10, 11, 13, 15, 30   # f32-path types
BLOCK = {F32: (1, 4), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}

PI_OK = 0
PI_NOALLOC_MAX_K, PI_NOALLOC_MAX_ROWS = 16384, 262144   # pi_hip_matvec_noalloc limits (pocketinfer_hip.h)
ERRORS = {-1: "PI_E_INVALID", -2: "PI_E_UNSUPPORTED", -3: "PI_E_HIP", -4: "PI_E_SELFTEST",
          -5: "PI_E_NOMEM", -6: "PI_E_INJECTED", -7: "PI_E_STOPPED", -8: "PI_E_CONTEXT_FULL",
          -9: "PI_E_NOMODEL"}

# Every exported symbol of include/pocketinfer_hip.h.
EXPORTS = [
    "pi_hip_probe", "pi_hip_create", "pi_hip_destroy", "pi_hip_name", "pi_last_error",
    "pi_hip_supports", "pi_hip_selftest", "pi_hip_matvec", "pi_hip_clear_weight_cache", "pi_hip_matvec_noalloc",
    "pi_hip_upload", "pi_hip_tensor_free", "pi_hip_tensor_bytes", "pi_hip_gemv_dev",
    "pi_hip_gemv_q8_dev", "pi_hip_time_gemv", "pi_hip_q8_quantize_dev", "pi_hip_dev_alloc",
    "pi_hip_dev_free", "pi_hip_copy_h2d", "pi_hip_copy_d2h", "pi_hip_copy_d2d", "pi_hip_set_stream", "pi_hip_synchronize",
    "pi_hip_q8_quantize", "pi_hip_block_sums", "pi_hip_fail_next",
    "pi_hip_model_bind", "pi_hip_forward", "pi_hip_logits", "pi_hip_argmax", "pi_hip_generate",
    "pi_hip_kv_write", "pi_hip_kv_read", "pi_hip_kv_fill_normal", "pi_hip_kv_set_tokens",
    "pi_hip_request_stop", "pi_hip_clear_stop", "pi_hip_use_graphs", "pi_hip_last_decode_us",
    "pi_hip_time_kernels", "pi_hip_last_kernel_us", "pi_hip_time_gemv_x",
    "pi_hip_use_persistent", "pi_hip_persistent_active", "pi_hip_use_batch_prefill", "pi_hip_prefill_pass_tokens", "pi_hip_stage_trace", "pi_hip_stage_trace_read",
    "pi_synth_q4k_random", "pi_synth_q6k_random", "pi_synth_normal", "pi_synth_tensor", "pi_synth_kv_normal",
    "pi_quantize_row", "pi_rng_new", "pi_rng_next_u64", "pi_sample",
    "pi_gguf_open", "pi_gguf_parse", "pi_gguf_close", "pi_gguf_version", "pi_gguf_data_offset", "pi_gguf_n_kv",
    "pi_gguf_key", "pi_gguf_kv_type", "pi_gguf_get_u64", "pi_gguf_get_f32", "pi_gguf_get_bool", "pi_gguf_get_str",
    "pi_gguf_array_info", "pi_gguf_array_str", "pi_gguf_array_i32", "pi_gguf_array_f32", "pi_gguf_n_tensors",
    "pi_gguf_find_tensor", "pi_gguf_tensor_info", "pi_gguf_tensor_data", "pi_gguf_model_desc",
]


class PiError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code


class TensorDesc(C.Structure):
    _fields_ = [("type", C.c_uint32), ("ne0", C.c_uint64), ("ne1", C.c_uint64), ("data", C.c_void_p)]


class LayerDesc(C.Structure):
    _fields_ = [(n, TensorDesc) for n in ("attn_q", "attn_k", "attn_v", "attn_o", "attn_norm",
                                          "ffn_gate", "ffn_up", "ffn_down", "ffn_norm")]


class ModelDesc(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_embd", C.c_uint32), ("n_ff", C.c_uint32),
                ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32), ("head_dim", C.c_uint32),
                ("n_rot", C.c_uint32), ("n_vocab", C.c_uint32), ("rope_theta", C.c_float),
                ("rms_eps", C.c_float), ("eos_ids", C.POINTER(C.c_uint32)), ("n_eos", C.c_uint32),
                ("token_embd", TensorDesc), ("output", TensorDesc), ("output_norm", TensorDesc),
                ("layers", C.POINTER(LayerDesc))]


class GenOpts(C.Structure):
    _fields_ = [("max_tokens", C.c_uint32), ("temp", C.c_float), ("top_p", C.c_float), ("seed", C.c_uint64)]


class GenStats(C.Structure):
    _fields_ = [("prefill_tokens", C.c_uint32), ("prefill_cached_tokens", C.c_uint32),
                ("gen_tokens", C.c_uint32), ("prefill_ms", C.c_double), ("gen_ms", C.c_double),
                ("stop", C.c_char * 32)]


_lib = None


def load_library(path: Path | str | None = None) -> C.CDLL:
    """Loads the in-tree HIP library; raises when it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} is missing: build it with `make -C {p.parent}` (or __graft_entry__.build())")
    lib = C.CDLL(str(p))
    vp, sz, u32, u64, i32, f32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint64, C.c_int, C.c_float
    sig = {
        "pi_hip_probe": (i32, [C.c_char_p, sz]),
        "pi_hip_create": (i32, [C.POINTER(vp), i32]),
        "pi_hip_destroy": (None, [vp]),
        "pi_hip_name": (C.c_char_p, [vp]),
        "pi_last_error": (C.c_char_p, [vp]),
        "pi_hip_supports": (i32, [vp, u32]),
        "pi_hip_selftest": (i32, [vp]),
        "pi_hip_matvec": (i32, [vp, u32, vp, sz, sz, vp, vp, sz]),
        "pi_hip_clear_weight_cache": (None, [vp]),
        "pi_hip_matvec_noalloc": (i32, [vp, vp, vp, vp]),
        "pi_hip_upload": (i32, [vp, u32, vp, sz, sz, C.POINTER(vp)]),
        "pi_hip_tensor_free": (None, [vp, vp]),
        "pi_hip_tensor_bytes": (sz, [vp]),
        "pi_hip_gemv_dev": (i32, [vp, vp, vp, vp]),
        "pi_hip_gemv_q8_dev": (i32, [vp, vp, vp, vp, vp, vp]),
        "pi_hip_time_gemv": (i32, [vp, C.POINTER(vp), i32, vp, vp, vp, vp, i32, C.POINTER(C.c_double)]),
        "pi_hip_q8_quantize_dev": (i32, [vp, vp, sz, i32, vp, vp, vp]),
        "pi_hip_dev_alloc": (i32, [vp, sz, C.POINTER(vp)]),
        "pi_hip_dev_free": (None, [vp, vp]),
        "pi_hip_copy_h2d": (i32, [vp, vp, vp, sz]),
        "pi_hip_copy_d2h": (i32, [vp, vp, vp, sz]),
        "pi_hip_copy_d2d": (i32, [vp, vp, vp, sz]),
        "pi_hip_set_stream": (i32, [vp, vp]),
        "pi_hip_synchronize": (i32, [vp]),
        "pi_hip_q8_quantize": (i32, [vp, vp, sz, i32, vp, vp, vp]),
        "pi_hip_block_sums": (i32, [vp, vp, vp, vp, vp, vp]),
        "pi_hip_fail_next": (i32, [vp]),
        "pi_hip_model_bind": (i32, [vp, C.POINTER(ModelDesc), u32]),
        "pi_hip_forward": (i32, [vp, vp, vp, i32, i32]),
        "pi_hip_logits": (i32, [vp, vp, sz]),
        "pi_hip_argmax": (i32, [vp, C.POINTER(u32)]),
        "pi_hip_generate": (i32, [vp, vp, sz, C.POINTER(GenOpts), C.POINTER(GenStats), vp]),
        "pi_hip_kv_write": (i32, [vp, u32, u32, u32, u32, vp, vp]),
        "pi_hip_kv_read": (i32, [vp, u32, u32, u32, u32, vp, vp]),
        "pi_hip_kv_fill_normal": (i32, [vp, u32, u64]),
        "pi_hip_kv_set_tokens": (i32, [vp, vp, u32]),
        "pi_hip_request_stop": (None, [vp]),
        "pi_hip_clear_stop": (None, [vp]),
        "pi_hip_use_graphs": (i32, [vp, i32]),
        "pi_hip_use_persistent": (i32, [vp, i32]),
        "pi_hip_persistent_active": (i32, [vp]),
        "pi_hip_prefill_pass_tokens": (i32, [vp]),
        "pi_hip_use_batch_prefill": (i32, [vp, i32]),
        "pi_hip_stage_trace": (i32, [vp, i32]),
        "pi_hip_stage_trace_read": (i32, [vp, vp, C.c_size_t, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
        "pi_hip_last_decode_us": (i32, [vp, C.POINTER(C.c_double)]),
        "pi_hip_time_kernels": (i32, [vp, i32]),
        "pi_hip_last_kernel_us": (i32, [vp, C.POINTER(C.c_double), C.POINTER(u32)]),
        "pi_hip_time_gemv_x": (i32, [vp, C.POINTER(vp), i32, vp, vp, i32, C.POINTER(C.c_double)]),
        "pi_synth_q4k_random": (i32, [u64, sz, sz, f32, f32, vp]),
        "pi_synth_q6k_random": (i32, [u64, sz, sz, f32, f32, vp]),
        "pi_synth_normal": (i32, [u64, sz, f32, f32, vp]),
        "pi_synth_kv_normal": (i32, [u64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp]),
        "pi_synth_tensor": (i32, [u64, u32, sz, sz, f32, f32, vp, i32]),
        "pi_quantize_row": (i32, [u32, vp, sz, vp]),
        "pi_gguf_open": (i32, [C.c_char_p, C.POINTER(vp), C.c_char_p, sz]),
        "pi_gguf_parse": (i32, [vp, sz, C.POINTER(vp), C.c_char_p, sz]),
        "pi_gguf_close": (None, [vp]),
        "pi_gguf_version": (u32, [vp]),
        "pi_gguf_data_offset": (u64, [vp]),
        "pi_gguf_n_kv": (sz, [vp]),
        "pi_gguf_key": (C.c_char_p, [vp, sz]),
        "pi_gguf_kv_type": (i32, [vp, C.c_char_p, C.POINTER(u32)]),
        "pi_gguf_get_u64": (i32, [vp, C.c_char_p, C.POINTER(u64)]),
        "pi_gguf_get_f32": (i32, [vp, C.c_char_p, C.POINTER(f32)]),
        "pi_gguf_get_bool": (i32, [vp, C.c_char_p, C.POINTER(i32)]),
        "pi_gguf_get_str": (i32, [vp, C.c_char_p, C.POINTER(vp), C.POINTER(sz)]),
        "pi_gguf_array_info": (i32, [vp, C.c_char_p, C.POINTER(u32), C.POINTER(u64)]),
        "pi_gguf_array_str": (i32, [vp, C.c_char_p, u64, C.POINTER(vp), C.POINTER(sz)]),
        "pi_gguf_array_i32": (i32, [vp, C.c_char_p, vp, sz]),
        "pi_gguf_array_f32": (i32, [vp, C.c_char_p, vp, sz]),
        "pi_gguf_n_tensors": (sz, [vp]),
        "pi_gguf_find_tensor": (C.c_int64, [vp, C.c_char_p]),
        "pi_gguf_tensor_info": (i32, [vp, sz, C.POINTER(C.c_char_p), C.POINTER(u32), C.POINTER(u32),
                                      C.POINTER(u64), C.POINTER(u64)]),
        "pi_gguf_tensor_data": (i32, [vp, sz, C.POINTER(vp), C.POINTER(sz), C.c_char_p, sz]),
        "pi_gguf_model_desc": (i32, [vp, C.POINTER(ModelDesc), vp, u32, vp, u32, C.c_char_p, sz]),
        "pi_rng_new": (u64, [u64]),
        "pi_rng_next_u64": (u64, [C.POINTER(u64)]),
        "pi_sample": (u32, [vp, sz, f32, f32, C.POINTER(u64)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def row_bytes(t: int, k: int) -> int:
    be, bb = BLOCK[t]
    if k % be:
        raise ValueError(f"row length {k} not divisible by block {be}")
    return k // be * bb


def probe() -> str | None:
    """probe() (opencl.rs:235-258): description of a visible gfx950, else None."""
    buf = C.create_string_buffer(256)
    rc = load_library().pi_hip_probe(buf, 256)
    return buf.value.decode() if rc == PI_OK else None


# ---------------------------------------------------------------------------
# synthetic data (host, deterministic)
# ---------------------------------------------------------------------------
def synth_q4k_random(seed: int, rows: int, k: int, dlo=1e-3, dhi=2e-2) -> np.ndarray:
    out = np.empty(rows * row_bytes(Q4_K, k), np.uint8)
    _check(load_library().pi_synth_q4k_random(seed, rows, k, dlo, dhi, _ptr(out)), None)
    return out


def synth_q6k_random(seed: int, rows: int, k: int, dlo=1e-4, dhi=5e-3) -> np.ndarray:
    out = np.empty(rows * row_bytes(Q6_K, k), np.uint8)
    _check(load_library().pi_synth_q6k_random(seed, rows, k, dlo, dhi, _ptr(out)), None)
    return out


def synth_normal(seed: int, n: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    _check(load_library().pi_synth_normal(seed, n, mean, std, _ptr(out)), None)
    return out


def synth_kv_normal(seed: int, lh: int, p0: int, n: int, dh: int = 64):
    """Host copy of what HipEngine.kv_fill_normal writes: (k, v), [n][dh] each,
    for positions p0..p0+n-1 of layer-major kv head lh."""
    k = np.empty((n, dh), np.float32)
    v = np.empty((n, dh), np.float32)
    _check(load_library().pi_synth_kv_normal(seed, lh, p0, n, dh, _ptr(k), _ptr(v)), None)
    return k, v


def synth_tensor(seed: int, t: int, rows: int, k: int, mean=0.0, std=0.02, threads: int | None = None) -> np.ndarray:
    out = np.empty(rows * row_bytes(t, k), np.uint8)
    th = threads or min(16, os.cpu_count() or 1)
    _check(load_library().pi_synth_tensor(seed, t, rows, k, mean, std, _ptr(out), th), None)
    return out


def quantize_row(t: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(row_bytes(t, x.size), np.uint8)
    _check(load_library().pi_quantize_row(t, _ptr(x), x.size, _ptr(out)), None)
    return out


class Rng:
    """sampler.rs:1-20 (SplitMix64) over the library's host sampler."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(load_library().pi_rng_new(seed))

    def next_u64(self) -> int:
        return load_library().pi_rng_next_u64(C.byref(self.state))


def sample(logits: np.ndarray, temp: float, top_p: float, rng: Rng) -> int:
    """sample() (sampler.rs:21-92) on a float32 array, overwritten like the
    reference's &mut [f32]."""
    assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
    return load_library().pi_sample(_ptr(logits), logits.size, temp, top_p, C.byref(rng.state))


def _check(rc: int, ctx) -> None:
    if rc != PI_OK:
        msg = load_library().pi_last_error(ctx).decode() if ctx else ""
        raise PiError(rc, msg)


# ---------------------------------------------------------------------------
# backend
# ---------------------------------------------------------------------------
class Tensor:
    """Weights resident in HBM (tiled layout; GGUF rows for the f32-path types)."""

    def __init__(self, backend: "HipBackend", handle: int, t: int, rows: int, k: int):
        self._b, self.handle, self.type, self.rows, self.k = backend, handle, t, rows, k

    @property
    def nbytes(self) -> int:
        return load_library().pi_hip_tensor_bytes(self.handle)

    def free(self) -> None:
        if self.handle:
            load_library().pi_hip_tensor_free(self._b.ctx, self.handle)
            self.handle = 0

    def __del__(self):
        # At interpreter shutdown the HIP runtime (and any profiler attached to
        # it) may already be finalized: leave the memory to process exit.
        if sys.is_finalizing():
            return
        try:
            if self._b.ctx:
                self.free()
        except Exception:
            pass


class DevBuf:
    """Device allocation owned by a backend context."""

    def __init__(self, backend: "HipBackend", ptr: int, nbytes: int):
        self._b, self.ptr, self.nbytes = backend, ptr, nbytes

    def to_host(self, dtype, count: int | None = None) -> np.ndarray:
        n = count if count is not None else self.nbytes // np.dtype(dtype).itemsize
        out = np.empty(n, dtype)
        self._b.check(self._b.lib.pi_hip_copy_d2h(self._b.ctx, _ptr(out), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            self._b.lib.pi_hip_dev_free(self._b.ctx, self.ptr)
            self.ptr = 0

    def __del__(self):
        # At interpreter shutdown the HIP runtime (and any profiler attached to
        # it) may already be finalized: leave the memory to process exit.
        if sys.is_finalizing():
            return
        try:
            if self._b.ctx:
                self.free()
        except Exception:
            pass


class HipBackend:
    """OpenClBackend twin (backend/opencl.rs:79-516) over the C ABI."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = C.c_void_p()
        rc = self.lib.pi_hip_create(C.byref(h), device)
        if rc != PI_OK:
            raise PiError(rc, f"no gfx950 device {device}")
        self.ctx = h.value
        self._keep: list = []
        self.bind_gen = 0   # bumped by every model bind: a context holds one engine

    # -- OpenClBackend surface --------------------------------------------
    def name(self) -> str:
        return self.lib.pi_hip_name(self.ctx).decode()

    def supports(self, ggml_type: int) -> bool:
        return bool(self.lib.pi_hip_supports(self.ctx, ggml_type))

    def selftest(self) -> None:
        self.check(self.lib.pi_hip_selftest(self.ctx))

    def matvec(self, ggml_type: int, w: np.ndarray, k: int, x: np.ndarray, rows: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(rows, np.float32)
        self._keep.append(w)  # the upload cache is keyed by the host pointer (opencl.rs:439)
        self.check(self.lib.pi_hip_matvec(self.ctx, ggml_type, _ptr(w), w.nbytes, k, _ptr(x), _ptr(out), rows))
        return out

    def matvec_noalloc(self, w: "Tensor", x: np.ndarray) -> np.ndarray:
        """W x for an uploaded tensor, staged through the library's static
        device array (no device allocation; see pi_hip_matvec_noalloc)."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(w.rows, np.float32)
        self.check(self.lib.pi_hip_matvec_noalloc(self.ctx, w.handle, _ptr(x), _ptr(out)))
        return out

    def clear_weight_cache(self) -> None:
        self.lib.pi_hip_clear_weight_cache(self.ctx)
        self._keep.clear()

    # -- explicit upload / device GEMV ------------------------------------
    def upload(self, ggml_type: int, w: np.ndarray, rows: int, k: int) -> Tensor:
        h = C.c_void_p()
        self.check(self.lib.pi_hip_upload(self.ctx, ggml_type, _ptr(w), rows, k, C.byref(h)))
        return Tensor(self, h.value, ggml_type, rows, k)

    def gemv_dev(self, w: Tensor, x_ptr: int, y_ptr: int) -> None:
        self.check(self.lib.pi_hip_gemv_dev(self.ctx, w.handle, x_ptr, y_ptr))

    def gemv_q8_dev(self, w: Tensor, q_ptr: int, d_ptr: int, s_ptr: int, y_ptr: int) -> None:
        self.check(self.lib.pi_hip_gemv_q8_dev(self.ctx, w.handle, q_ptr, d_ptr, s_ptr, y_ptr))

    def time_gemv(self, ws: list[Tensor], q_ptr: int, d_ptr: int, s_ptr: int, y_ptr: int, iters: int) -> float:
        arr = (C.c_void_p * len(ws))(*[w.handle for w in ws])
        us = C.c_double()
        self.check(self.lib.pi_hip_time_gemv(self.ctx, arr, len(ws), q_ptr, d_ptr, s_ptr, y_ptr, iters, C.byref(us)))
        return us.value

    def time_gemv_x(self, ws: list[Tensor], x_ptr: int, y_ptr: int, iters: int) -> float:
        """Mean microseconds of the whole gemv_dev job (Q8 of x, then the GEMV)."""
        arr = (C.c_void_p * len(ws))(*[w.handle for w in ws])
        us = C.c_double()
        self.check(self.lib.pi_hip_time_gemv_x(self.ctx, arr, len(ws), x_ptr, y_ptr, iters, C.byref(us)))
        return us.value

    def time_kernels(self, enable: bool) -> None:
        """Event pair around every decode forward of generate (see last_kernel_us)."""
        self.check(self.lib.pi_hip_time_kernels(self.ctx, int(enable)))

    def q8_quantize_dev(self, x_ptr: int, k: int, b: int, q_ptr: int, d_ptr: int, s_ptr: int) -> None:
        self.check(self.lib.pi_hip_q8_quantize_dev(self.ctx, x_ptr, k, b, q_ptr, d_ptr, s_ptr))

    def alloc(self, nbytes: int) -> "DevBuf":
        p = C.c_void_p()
        self.check(self.lib.pi_hip_dev_alloc(self.ctx, nbytes, C.byref(p)))
        return DevBuf(self, p.value, nbytes)

    def to_device(self, a: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(a)
        buf = self.alloc(a.nbytes)
        self.check(self.lib.pi_hip_copy_h2d(self.ctx, buf.ptr, _ptr(a), a.nbytes))
        return buf

    def copy_d2d(self, dst: "DevBuf", src: "DevBuf", nbytes: int) -> None:
        assert nbytes <= dst.nbytes and nbytes <= src.nbytes
        self.check(self.lib.pi_hip_copy_d2d(self.ctx, dst.ptr, src.ptr, nbytes))

    def set_stream(self, stream_ptr: int | None) -> None:
        self.check(self.lib.pi_hip_set_stream(self.ctx, stream_ptr or None))

    def use_graphs(self, enable: bool) -> None:
        self.check(self.lib.pi_hip_use_graphs(self.ctx, int(enable)))

    def use_persistent(self, enable: bool) -> None:
        """Engine tokens on the persistent kernel (default) or per-stage kernels."""
        self.check(self.lib.pi_hip_use_persistent(self.ctx, int(enable)))

    def use_batch_prefill(self, enable: bool) -> None:
        """Prompt chunks on the batched MFMA prefill kernels (default) or token by token."""
        self.check(self.lib.pi_hip_use_batch_prefill(self.ctx, int(enable)))

    def persistent_active(self) -> bool:
        return self.lib.pi_hip_persistent_active(self.ctx) == 1

    def prefill_pass_tokens(self) -> int:
        """Tokens per batched prefill pass of the bound model (0: none)."""
        return self.lib.pi_hip_prefill_pass_tokens(self.ctx)

    def stage_trace(self, enable: bool) -> None:
        self.check(self.lib.pi_hip_stage_trace(self.ctx, int(enable)))

    def stage_trace_read(self) -> np.ndarray:
        """[workgroup][slot] device clock (100 MHz) of the last persistent launch."""
        nb, ns = C.c_uint32(), C.c_uint32()
        self.check(self.lib.pi_hip_stage_trace_read(self.ctx, None, 0, C.byref(nb), C.byref(ns)))
        out = np.zeros((nb.value, ns.value), np.uint64)
        self.check(self.lib.pi_hip_stage_trace_read(self.ctx, _ptr(out), out.size, C.byref(nb), C.byref(ns)))
        return out

    def synchronize(self) -> None:
        self.check(self.lib.pi_hip_synchronize(self.ctx))

    # -- test hooks -----------------------------------------------------------
    def q8_quantize(self, x: np.ndarray, k: int, b: int):
        x = np.ascontiguousarray(x, np.float32)
        assert x.size == k * b
        q = np.empty(k * b, np.int8)
        d = np.empty(k // 32 * b, np.float32)
        s = np.empty(k // 32 * b, np.int32)
        self.check(self.lib.pi_hip_q8_quantize(self.ctx, _ptr(x), k, b, _ptr(q), _ptr(d), _ptr(s)))
        return q, d, s

    def block_sums(self, w: Tensor, q: np.ndarray, d: np.ndarray, s: np.ndarray) -> np.ndarray:
        per_row = w.k // 16 if w.type == Q6_K else w.k // 32
        out = np.empty(w.rows * per_row, np.int32)
        q, d, s = (np.ascontiguousarray(a) for a in (q, d, s))
        self.check(self.lib.pi_hip_block_sums(self.ctx, w.handle, _ptr(q), _ptr(d), _ptr(s), _ptr(out)))
        return out.reshape(w.rows, per_row)

    def fail_next(self) -> None:
        self.check(self.lib.pi_hip_fail_next(self.ctx))

    def check(self, rc: int) -> None:
        if rc != PI_OK:
            raise PiError(rc, self.lib.pi_last_error(self.ctx).decode())

    def close(self) -> None:
        if self.ctx:
            self.lib.pi_hip_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        # At interpreter shutdown the HIP runtime (and any profiler attached to
        # it) may already be finalized: leave the memory to process exit.
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# models
# ---------------------------------------------------------------------------
@dataclass
class ModelSpec:
    """Config (model.rs:14-29) plus per-tensor types."""
    n_layer: int
    n_embd: int
    n_ff: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_vocab: int
    n_rot: int = 0
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    eos_ids: tuple = ()
    embd_type: int = Q4_K
    out_type: int = Q6_K
    default_type: int = Q4_K
    attn_v_types: tuple = ()     # per layer
    ffn_down_types: tuple = ()   # per layer

    def __post_init__(self):
        if not self.n_rot:
            self.n_rot = self.head_dim


def minicpm2b_spec() -> ModelSpec:
    """MiniCPM-2B-shaped Q4_K_M model: Q4_K by default, Q6_K head, Q6_K attn_v
    in even layers; ffn_down (row length 5760, not a multiple of 256) is Q8_0
    in even layers and Q4_0 in odd ones."""
    n = 40
    return ModelSpec(n_layer=n, n_embd=2304, n_ff=5760, n_head=36, n_head_kv=36, head_dim=64,
                     n_vocab=122753, eos_ids=(2,),
                     attn_v_types=tuple(Q6_K if l % 2 == 0 else Q4_K for l in range(n)),
                     ffn_down_types=tuple(Q8_0 if l % 2 == 0 else Q4_0 for l in range(n)))


def tiny_spec(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_vocab=1000, n_head_kv=None, n_rot=0) -> ModelSpec:
    """Small model of the same families (k multiple of 256 for K-quants).
    n_head_kv < n_head gives grouped-query attention and n_rot < 64 partial
    RoPE (Config::from_gguf, model.rs:46-64)."""
    return ModelSpec(n_layer=n_layer, n_embd=n_embd, n_ff=n_ff, n_head=n_head,
                     n_head_kv=n_head_kv or n_head, head_dim=64, n_rot=n_rot,
                     n_vocab=n_vocab, eos_ids=(n_vocab - 1,),
                     attn_v_types=tuple(Q6_K if l % 2 == 0 else Q4_K for l in range(n_layer)),
                     ffn_down_types=tuple(Q8_0 if l % 2 == 0 else Q4_0 for l in range(n_layer)),
                     default_type=Q4_K)


LAYER_TENSORS = ("attn_q", "attn_k", "attn_v", "attn_o", "attn_norm", "ffn_gate", "ffn_up", "ffn_down", "ffn_norm")


@dataclass
class SynthModel:
    """Host tensors (as mmap'd GGUF tensors would be): name -> (type, ne0, ne1, bytes)."""
    spec: ModelSpec
    tensors: dict = field(default_factory=dict)

    def weight_bytes_per_token(self) -> int:
        """Bytes of every layer tensor (norms included), the head and
        output_norm: what one decoded token streams (one embedding row aside)."""
        return sum(buf.nbytes for name, (t, ne0, ne1, buf) in self.tensors.items() if name != "token_embd.weight")


def synth_model(spec: ModelSpec, seed: int = 1234, threads: int | None = None) -> SynthModel:
    """Weights N(0, 0.02) quantized per spec; norm weights 1 + N(0, 0.02) f32.
    Tensor i (in the order below) draws from seed*1000003 + i."""
    m = SynthModel(spec)
    qdim, kdim = spec.n_head * spec.head_dim, spec.n_head_kv * spec.head_dim
    idx = [0]

    def add(name, t, ne0, ne1, mean=0.0, std=0.02):
        s = seed * 1000003 + idx[0]
        idx[0] += 1
        buf = synth_tensor(s, t, ne1, ne0, mean, std, threads)
        if t == F32:
            buf = buf.view(np.float32)
        m.tensors[name] = (t, ne0, ne1, buf)

    add("token_embd.weight", spec.embd_type, spec.n_embd, spec.n_vocab)
    for l in range(spec.n_layer):
        p = f"blk.{l}."
        add(p + "attn_norm.weight", F32, spec.n_embd, 1, 1.0, 0.02)
        add(p + "attn_q.weight", spec.default_type, spec.n_embd, qdim)
        add(p + "attn_k.weight", spec.default_type, spec.n_embd, kdim)
        add(p + "attn_v.weight", spec.attn_v_types[l] if spec.attn_v_types else spec.default_type, spec.n_embd, kdim)
        add(p + "attn_output.weight", spec.default_type, qdim, spec.n_embd)
        add(p + "ffn_norm.weight", F32, spec.n_embd, 1, 1.0, 0.02)
        add(p + "ffn_gate.weight", spec.default_type, spec.n_embd, spec.n_ff)
        add(p + "ffn_up.weight", spec.default_type, spec.n_embd, spec.n_ff)
        add(p + "ffn_down.weight", spec.ffn_down_types[l] if spec.ffn_down_types else Q8_0, spec.n_ff, spec.n_embd)
    add("output_norm.weight", F32, spec.n_embd, 1, 1.0, 0.02)
    add("output.weight", spec.out_type, spec.n_embd, spec.n_vocab)
    return m


class Gguf:
    """Gguf (gguf.rs:31-336) over the library's reader: the file stays mapped
    read-only until close(); tensor data are numpy views of the mapping."""

    def __init__(self, path: str | None = None, data: bytes | None = None):
        L = load_library()
        h, err = C.c_void_p(), C.create_string_buffer(512)
        if data is not None:
            self._buf = C.create_string_buffer(bytes(data), len(data))   # kept alive: no copy in the library
            rc = L.pi_gguf_parse(self._buf, len(data), C.byref(h), err, 512)
        else:
            rc = L.pi_gguf_open(str(path).encode(), C.byref(h), err, 512)
        if rc != PI_OK:
            raise PiError(rc, err.value.decode())
        self.h = h.value

    # -- header and metadata -------------------------------------------------
    @property
    def version(self) -> int:
        return load_library().pi_gguf_version(self.h)

    @property
    def data_offset(self) -> int:
        return load_library().pi_gguf_data_offset(self.h)

    def keys(self) -> list:
        L = load_library()
        return [L.pi_gguf_key(self.h, i).decode() for i in range(L.pi_gguf_n_kv(self.h))]

    def kv_type(self, key: str) -> int | None:
        t = C.c_uint32()
        return t.value if load_library().pi_gguf_kv_type(self.h, key.encode(), C.byref(t)) == PI_OK else None

    def get_u64(self, key: str) -> int | None:
        v = C.c_uint64()
        return v.value if load_library().pi_gguf_get_u64(self.h, key.encode(), C.byref(v)) == PI_OK else None

    def get_f32(self, key: str) -> float | None:
        v = C.c_float()
        return v.value if load_library().pi_gguf_get_f32(self.h, key.encode(), C.byref(v)) == PI_OK else None

    def get_bool(self, key: str) -> bool | None:
        v = C.c_int()
        return bool(v.value) if load_library().pi_gguf_get_bool(self.h, key.encode(), C.byref(v)) == PI_OK else None

    def get_str(self, key: str) -> bytes | None:
        p, n = C.c_void_p(), C.c_size_t()
        if load_library().pi_gguf_get_str(self.h, key.encode(), C.byref(p), C.byref(n)) != PI_OK:
            return None
        return C.string_at(p.value, n.value) if n.value else b""

    def array_info(self, key: str):
        et, n = C.c_uint32(), C.c_uint64()
        if load_library().pi_gguf_array_info(self.h, key.encode(), C.byref(et), C.byref(n)) != PI_OK:
            return None
        return et.value, n.value

    def array_strings(self, key: str) -> list:
        info = self.array_info(key)
        if info is None:
            raise KeyError(key)
        out = []
        for i in range(info[1]):
            p, n = C.c_void_p(), C.c_size_t()
            _check(load_library().pi_gguf_array_str(self.h, key.encode(), i, C.byref(p), C.byref(n)), None)
            out.append(C.string_at(p.value, n.value) if n.value else b"")
        return out

    def array_i32(self, key: str) -> np.ndarray:
        info = self.array_info(key)
        out = np.empty(info[1] if info else 0, np.int32)
        _check(load_library().pi_gguf_array_i32(self.h, key.encode(), _ptr(out) if out.size else None, out.size), None)
        return out

    def array_f32(self, key: str) -> np.ndarray:
        info = self.array_info(key)
        out = np.empty(info[1] if info else 0, np.float32)
        _check(load_library().pi_gguf_array_f32(self.h, key.encode(), _ptr(out) if out.size else None, out.size), None)
        return out

    # -- tensors -----------------------------------------------------------------
    def n_tensors(self) -> int:
        return load_library().pi_gguf_n_tensors(self.h)

    def tensor_info(self, i: int) -> dict:
        name, t, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
        ne, off = (C.c_uint64 * 4)(), C.c_uint64()
        _check(load_library().pi_gguf_tensor_info(self.h, i, C.byref(name), C.byref(t), C.byref(nd), ne, C.byref(off)),
               None)
        return {"name": name.value.decode(), "type": t.value, "ne": list(ne)[: nd.value], "offset": off.value}

    def find(self, name: str) -> int:
        return load_library().pi_gguf_find_tensor(self.h, name.encode())

    def tensor_data(self, i: int) -> np.ndarray:
        p, n, err = C.c_void_p(), C.c_size_t(), C.create_string_buffer(256)
        rc = load_library().pi_gguf_tensor_data(self.h, i, C.byref(p), C.byref(n), err, 256)
        if rc != PI_OK:
            raise PiError(rc, err.value.decode())
        return np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p.value)) if n.value else np.empty(0, np.uint8)

    # -- the model ---------------------------------------------------------------
    def model_desc(self, max_layers: int = 512, max_eos: int = 64):
        """(ModelDesc, keepalive) for pi_hip_model_bind: Config::from_gguf and
        Model::load's tensor binding (model.rs:31-97, 487-601)."""
        desc = ModelDesc()
        layers = (LayerDesc * max_layers)()
        eos = (C.c_uint32 * max_eos)()
        err = C.create_string_buffer(512)
        rc = load_library().pi_gguf_model_desc(self.h, C.byref(desc), layers, max_layers, eos, max_eos, err, 512)
        if rc != PI_OK:
            raise PiError(rc, err.value.decode())
        return desc, (layers, eos)

    def spec(self) -> "ModelSpec":
        d, _ = self.model_desc()
        return ModelSpec(n_layer=d.n_layer, n_embd=d.n_embd, n_ff=d.n_ff, n_head=d.n_head, n_head_kv=d.n_head_kv,
                         head_dim=d.head_dim, n_vocab=d.n_vocab, n_rot=d.n_rot, rope_theta=d.rope_theta,
                         rms_eps=d.rms_eps, eos_ids=tuple(d.eos_ids[i] for i in range(d.n_eos)))

    def close(self) -> None:
        if self.h:
            load_library().pi_gguf_close(self.h)
            self.h = None

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


def _tdesc(entry) -> TensorDesc:
    t, ne0, ne1, buf = entry
    return TensorDesc(t, ne0, ne1, buf.ctypes.data)


class HipEngine:
    """Device-resident Engine (model.rs:678-1352) on a HipBackend context."""

    def __init__(self, backend: HipBackend, model, n_ctx: int):
        """model: a SynthModel (host tensors) or a Gguf (tensors in the file's
        mapping, bound as Engine::load binds them)."""
        self.b, self.n_ctx = backend, n_ctx
        if isinstance(model, Gguf):
            desc, self._keep = model.model_desc()
            self.model = SynthModel(model.spec())
            self._gguf = model
        else:
            self.model = model
            s = model.spec
            T = model.tensors
            self._layers = (LayerDesc * s.n_layer)()
            names = {"attn_o": "attn_output"}
            for l in range(s.n_layer):
                for f in LAYER_TENSORS:
                    setattr(self._layers[l], f, _tdesc(T[f"blk.{l}.{names.get(f, f)}.weight"]))
            self._eos = (C.c_uint32 * max(1, len(s.eos_ids)))(*s.eos_ids)
            desc = ModelDesc(s.n_layer, s.n_embd, s.n_ff, s.n_head, s.n_head_kv, s.head_dim, s.n_rot, s.n_vocab,
                             s.rope_theta, s.rms_eps, self._eos, len(s.eos_ids), _tdesc(T["token_embd.weight"]),
                             _tdesc(T["output.weight"]), _tdesc(T["output_norm.weight"]), self._layers)
        backend.bind_gen += 1
        self._gen = backend.bind_gen
        backend.check(backend.lib.pi_hip_model_bind(backend.ctx, C.byref(desc), n_ctx))

    def _live(self) -> None:
        """A context holds one engine: binding another model frees this one."""
        if self._gen != self.b.bind_gen:
            raise RuntimeError("this HipEngine was replaced by a later model bind on the same HipBackend")

    def forward(self, ids, positions, want_logits=True) -> None:
        self._live()
        ids = np.ascontiguousarray(ids, np.uint32)
        pos = np.ascontiguousarray(positions, np.int32)
        self.b.check(self.b.lib.pi_hip_forward(self.b.ctx, _ptr(ids), _ptr(pos), len(ids), int(want_logits)))

    def logits(self, n: int | None = None) -> np.ndarray:
        self._live()
        n = n or self.model.spec.n_vocab
        out = np.empty(n, np.float32)
        self.b.check(self.b.lib.pi_hip_logits(self.b.ctx, _ptr(out), n))
        return out

    def argmax(self) -> int:
        self._live()
        v = C.c_uint32()
        self.b.check(self.b.lib.pi_hip_argmax(self.b.ctx, C.byref(v)))
        return v.value

    def generate(self, prompt, max_tokens: int, temp: float = 0.0, top_p: float = 1.0, seed: int = 1):
        self._live()
        prompt = np.ascontiguousarray(prompt, np.uint32)
        ids = np.zeros(max(1, max_tokens), np.uint32)
        opts = GenOpts(max_tokens, temp, top_p, seed)
        st = GenStats()
        self.b.check(self.b.lib.pi_hip_generate(self.b.ctx, _ptr(prompt), len(prompt), C.byref(opts), C.byref(st),
                                                _ptr(ids)))
        stats = {"prefill_tokens": st.prefill_tokens, "prefill_cached_tokens": st.prefill_cached_tokens,
                 "gen_tokens": st.gen_tokens, "prefill_ms": st.prefill_ms, "gen_ms": st.gen_ms,
                 "stop": st.stop.decode()}
        return ids[: st.gen_tokens].tolist(), stats

    def last_decode_us(self) -> float:
        self._live()
        v = C.c_double()
        self.b.check(self.b.lib.pi_hip_last_decode_us(self.b.ctx, C.byref(v)))
        return v.value

    def last_kernel_us(self) -> tuple[float, int]:
        """(mean device microseconds of one decode forward's kernels, forwards
        timed) of the last generate call; (0, 0) unless kernel timing is on."""
        self._live()
        v, n = C.c_double(), C.c_uint32()
        self.b.check(self.b.lib.pi_hip_last_kernel_us(self.b.ctx, C.byref(v), C.byref(n)))
        return v.value, n.value

    def kv_write(self, layer, head, pos0, k: np.ndarray, v: np.ndarray) -> None:
        self._live()
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        n = k.size // self.model.spec.head_dim
        self.b.check(self.b.lib.pi_hip_kv_write(self.b.ctx, layer, head, pos0, n, _ptr(k), _ptr(v)))

    def kv_read(self, layer, head, pos0, n):
        self._live()
        dh = self.model.spec.head_dim
        k = np.empty(n * dh, np.float32)
        v = np.empty(n * dh, np.float32)
        self.b.check(self.b.lib.pi_hip_kv_read(self.b.ctx, layer, head, pos0, n, _ptr(k), _ptr(v)))
        return k.reshape(n, dh), v.reshape(n, dh)

    def kv_fill_normal(self, n: int, seed: int) -> None:
        self._live()
        self.b.check(self.b.lib.pi_hip_kv_fill_normal(self.b.ctx, n, seed))

    def kv_set_tokens(self, ids) -> None:
        self._live()
        ids = np.ascontiguousarray(ids, np.uint32)
        self.b.check(self.b.lib.pi_hip_kv_set_tokens(self.b.ctx, _ptr(ids) if ids.size else None, ids.size))

    def request_stop(self) -> None:
        self.b.lib.pi_hip_request_stop(self.b.ctx)

    def clear_stop(self) -> None:
        self.b.lib.pi_hip_clear_stop(self.b.ctx)
