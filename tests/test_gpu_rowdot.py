"""GPU parity of the f32-path GEMV (the GGUF types without an int8 path:
Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K, Q8_K, BF16) against the oracle's
single-token dot (`dot_row_scalar`, quant.rs:377-441): every row bit for bit,
through the OpenClBackend twin (`pi_hip_matvec`), the device-pointer GEMV and
the no-allocation entry point.  The oracle's decoders of these types are
pinned in tests/test_oracle_quant_types.py.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K, Q8_K, BF16 = 3, 6, 7, 9, 10, 11, 13, 15, 30
BLOCK = {Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q8_1: (32, 36), Q2_K: (256, 84), Q3_K: (256, 110),
         Q5_K: (256, 176), Q8_K: (256, 292), BF16: (1, 2)}
# byte offsets of f16 fields in a block (set to finite values); Q8_K's f32 d is at 0
F16_FIELDS = {Q4_1: (0, 2), Q5_0: (0,), Q5_1: (0, 2), Q8_1: (0, 2), Q2_K: (80, 82), Q3_K: (108,), Q5_K: (0, 2)}


def random_rows(t, rows, k, seed):
    """Random block bytes with finite scales (GGUF row layout)."""
    rng = np.random.default_rng(seed)
    if t == BF16:
        v = (rng.standard_normal(rows * k) * 0.05).astype(np.float32)
        return (v.view(np.uint32) >> 16).astype("<u2").view(np.uint8).copy()
    be, bb = BLOCK[t]
    nb = rows * (k // be)
    blk = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if t == Q8_K:
        blk[:, 0:4] = (rng.standard_normal(nb).astype(np.float32) * 1e-3).view(np.uint8).reshape(nb, 4)
    for off in F16_FIELDS.get(t, ()):
        h = (rng.standard_normal(nb) * 0.02).astype(np.float16)
        h[::17] = np.float16(6.0e-6)                       # some subnormal scales
        blk[:, off:off + 2] = h.view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1).copy()


def oracle_rows(oracle, t, w, rows, k, x):
    rb = w.size // rows
    return np.array([oracle.dot_row(t, w[r * rb:(r + 1) * rb], k, x) for r in range(rows)], np.float32)


TYPES = [Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K, Q8_K, BF16]


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("rows,k", [(37, 256), (300, 2304), (65, 4096)])
def test_matvec_matches_oracle(pih, backend, oracle, t, rows, k):
    w = random_rows(t, rows, k, 1000 * t + rows)
    x = np.random.default_rng(k + t).standard_normal(k).astype(np.float32)
    got = backend.matvec(t, w, k, x, rows)
    want = oracle_rows(oracle, t, w, rows, k, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (t, rows, k)


@pytest.mark.parametrize("t", [Q4_1, Q5_0, Q5_1, Q8_1, BF16])
def test_row_types_at_ffn_down_length(pih, backend, oracle, t):
    """k = 5760 (a multiple of 32, not of 256), 96 rows."""
    rows, k = 96, 5760
    w = random_rows(t, rows, k, 77 + t)
    x = np.random.default_rng(t).standard_normal(k).astype(np.float32)
    want = oracle_rows(oracle, t, w, rows, k, x)
    assert np.array_equal(backend.matvec(t, w, k, x, rows).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", [Q5_K, Q5_0])
def test_gemv_dev_and_noalloc_equal_matvec(pih, backend, oracle, t):
    rows, k = 200, 2304
    w = random_rows(t, rows, k, 5 + t)
    x = np.random.default_rng(9).standard_normal(k).astype(np.float32)
    ref = backend.matvec(t, w, k, x, rows)
    dev = backend.upload(t, w, rows, k)
    assert dev.nbytes == w.size                        # GGUF rows, not repacked
    xd, yd = backend.to_device(x), backend.alloc(rows * 4)
    backend.gemv_dev(dev, xd.ptr, yd.ptr)
    backend.synchronize()
    assert np.array_equal(yd.to_host(np.float32).view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(backend.matvec_noalloc(dev, x).view(np.uint32), ref.view(np.uint32))
    # the pre-quantized entry point is for the int8 path only
    with pytest.raises(pih.PiError):
        backend.gemv_q8_dev(dev, xd.ptr, xd.ptr, xd.ptr, yd.ptr)


def test_bad_shapes_rejected(pih, backend):
    w = random_rows(Q5_K, 2, 256, 1)
    with pytest.raises(pih.PiError):
        backend.matvec(Q5_K, w, 128, np.zeros(128, np.float32), 4)       # k not a multiple of 256
    with pytest.raises(pih.PiError):
        backend.matvec(Q5_K, w[:-1], 256, np.zeros(256, np.float32), 2)  # byte count
