"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI.

Contract: Q8 activation quants and per-block integer
sums bit-exact; GEMV outputs within 1e-3 relative + 1e-4 absolute.  The GEMV
kernels keep the reference's float order, so outputs are also checked bitwise.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
RTOL, ATOL = 1e-3, 1e-4


def _rows(pih, t, rows, k, seed):
    if t == Q4_K:
        return pih.synth_q4k_random(seed, rows, k)
    if t == Q6_K:
        return pih.synth_q6k_random(seed, rows, k)
    return pih.synth_tensor(seed, t, rows, k, 0.0, 0.02)


def test_probe_name_supports_selftest(pih, backend):
    assert pih.probe() is not None and "gfx950" in pih.probe()
    assert "gfx950" in backend.name()
    for t in (Q4_0, Q8_0, Q4_K, Q6_K):               # int8 path
        assert backend.supports(t)
    for t in (3, 6, 7, 9, 10, 11, 13, 15, 30):       # f32 path (tests/test_gpu_rowdot.py)
        assert backend.supports(t)
    for t in (0, 1, 4, 5, 16, 31):                   # F32 / F16 matrices, unknown ids
        assert not backend.supports(t)
    backend.selftest()


@pytest.mark.parametrize("k,b", [(2304, 1), (5760, 1), (2304, 32), (256, 7), (32, 1)])
def test_q8_quantize_bit_exact(pih, backend, oracle, k, b):
    rng = np.random.default_rng(k * 100 + b)
    x = rng.standard_normal(k * b).astype(np.float32)
    x[: min(k * b, 64)] *= 1e-3            # small blocks
    if k * b >= 256:
        x[64:96] = 0.0                     # all-zero block -> d = 0, q = 0
        x[96:128] = np.float32(0.5)         # halfway values
        x[128:160] = np.linspace(-127, 127, 32, dtype=np.float32)
    q, d, s = backend.q8_quantize(x, k, b)
    ref = oracle.Act(x, k, b)
    assert np.array_equal(q, ref.q)
    assert np.array_equal(d.view(np.uint32), ref.d.view(np.uint32))
    assert np.array_equal(s, ref.sum)


def test_q8_quantize_halfway_vector(pih, backend, oracle):
    """simd_q8.rs:58-80 input on the device."""
    k = 512
    x = ((np.arange(k) % 73).astype(np.float32) - np.float32(36.0)) * np.float32(0.0625)
    x[0], x[1], x[2] = 127.0, 0.5, -0.5
    q, d, s = backend.q8_quantize(x, k, 1)
    ref = oracle.Act(x, k, 1)
    assert q[0] == 127 and q[1] == 1 and q[2] == -1 and d[0] == 1.0
    assert np.array_equal(q, ref.q) and np.array_equal(d.view(np.uint32), ref.d.view(np.uint32))
    assert np.array_equal(s, ref.sum)


def test_q8_quantize_every_tie(pih, backend, oracle):
    """Every exact tie k + 0.5 in (-127, 127) and both float neighbours of each
    tie: blocks whose maximum is 127, so d = 1 and inv = 1 (quant_int.rs:41-49)."""
    ties = np.arange(-127, 127, dtype=np.float32) + np.float32(0.5)
    vals = np.concatenate([ties, np.nextafter(ties, np.float32(-np.inf)), np.nextafter(ties, np.float32(np.inf))])
    per = 31
    nb = -(-vals.size // per)
    x = np.zeros((nb, 32), np.float32)
    x[:, 0] = 127.0
    flat = np.zeros(nb * per, np.float32)
    flat[: vals.size] = vals
    x[:, 1:] = flat.reshape(nb, per)
    k = 32 * nb
    x = x.reshape(-1)
    q, d, s = backend.q8_quantize(x, k, 1)
    ref = oracle.Act(x, k, 1)
    assert np.all(d == 1.0)
    assert np.array_equal(q, ref.q)
    assert np.array_equal(s, ref.sum)
    tie_q = q.reshape(nb, 32)[:, 1:].reshape(-1)[: ties.size]
    assert np.array_equal(tie_q, np.where(ties > 0, np.ceil(ties), np.floor(ties)).astype(np.int8))


CASES = [
    (Q4_K, 5760, 2304),     # config 1 shape
    (Q4_K, 2304, 2304),     # attn_q/k/o
    (Q6_K, 2304, 2304),     # attn_v (Q6_K half)
    (Q4_0, 2304, 5760),     # ffn_down (Q4_0 half)
    (Q8_0, 2304, 5760),     # ffn_down (Q8_0 half)
    (Q4_K, 13, 256),        # ragged tiles, one block per row
    (Q6_K, 29, 512),
    (Q4_0, 11, 2304),
    (Q8_0, 5, 64),
    (Q4_K, 1, 4096),
    (Q4_0, 9, 288),         # row lengths that end in a partial 256-element
    (Q8_0, 7, 480),         # row of the LDS activation (q8 chunk permutation)
]


@pytest.mark.parametrize("t,rows,k", CASES)
def test_block_sums_bit_exact(pih, backend, oracle, t, rows, k):
    w = _rows(pih, t, rows, k, 100 + t)
    x = np.random.default_rng(rows + k).standard_normal(k).astype(np.float32)
    act = oracle.Act(x, k, 1)
    dev = backend.upload(t, w, rows, k)
    got = backend.block_sums(dev, act.q, act.d, act.sum)
    rb = pih.row_bytes(t, k)
    for r in sorted({0, rows // 2, rows - 1}):
        want = oracle.block_sums(t, w[r * rb:(r + 1) * rb], k, act)
        assert np.array_equal(got[r], want), f"row {r}"
    dev.free()


@pytest.mark.parametrize("t,rows,k", CASES)
def test_gemv_matches_oracle(pih, backend, oracle, t, rows, k):
    w = _rows(pih, t, rows, k, 200 + t)
    x = np.random.default_rng(rows * 7 + k).standard_normal(k).astype(np.float32)
    got = backend.matvec(t, w, k, x, rows)
    act = oracle.Act(x, k, 1)
    want = oracle.Pool(8).matmul(t, w, pih.row_bytes(t, k), k, x, 1, rows, act)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    # same Q8 input and the reference's float order: bitwise equal
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    backend.clear_weight_cache()


# f16 scale patterns: subnormals (smallest, largest, negative), signed zeros,
# infinities, a quiet and a signalling NaN
SPECIAL_F16 = [0x0001, 0x03FF, 0x8200, 0x0000, 0x8000, 0x7C00, 0xFC00, 0x7E00, 0x7C01]
# (block bytes, offsets of the f16 scale fields in a block)
SCALE_FIELDS = {Q4_K: (144, (0, 2)), Q6_K: (210, (208,)), Q4_0: (18, (0,)), Q8_0: (34, (0,))}


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q4_0, Q8_0])
def test_gemv_special_scales(pih, backend, oracle, t):
    """Rows whose block scales (d, and dmin for Q4_K) are f16 subnormals, zeros,
    infinities and NaNs: finite outputs bitwise equal to the oracle's, NaN
    outputs in the same rows (quant_int.rs decodes scales with the f16 crate)."""
    bb, offs = SCALE_FIELDS[t]
    k = 512
    rows = 2 + len(SPECIAL_F16) * len(offs)
    w = _rows(pih, t, rows, k, 300 + t).copy()
    rb = pih.row_bytes(t, k)
    r = 2
    for off in offs:
        for v in SPECIAL_F16:
            row = w[r * rb:(r + 1) * rb].reshape(-1, bb)
            row[:, off] = v & 0xFF
            row[:, off + 1] = v >> 8
            r += 1
    x = np.random.default_rng(7).standard_normal(k).astype(np.float32)
    got = backend.matvec(t, w, k, x, rows)
    want = oracle.Pool(4).matmul(t, w, rb, k, x, 1, rows, oracle.Act(x, k, 1))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    backend.clear_weight_cache()


@pytest.mark.parametrize("t,rows,k", [(Q4_K, 5760, 2304), (Q6_K, 29, 512), (Q4_0, 2304, 5760), (Q8_0, 7, 480)])
def test_gemv_dev_one_launch_equals_q8_pass(pih, backend, oracle, t, rows, k):
    """gemv_dev (Q8 of x in every workgroup's LDS, one launch) equals the
    GEMV on the separately quantized activation and the oracle, bit for bit."""
    w = _rows(pih, t, rows, k, 400 + t)
    x = np.random.default_rng(rows + 3 * k).standard_normal(k).astype(np.float32)
    dev = backend.upload(t, w, rows, k)
    xd, y1, y2 = backend.to_device(x), backend.alloc(rows * 4), backend.alloc(rows * 4)
    qd, dd, sd = backend.alloc(k), backend.alloc(k // 32 * 4), backend.alloc(k // 32 * 4)
    backend.gemv_dev(dev, xd.ptr, y1.ptr)
    backend.q8_quantize_dev(xd.ptr, k, 1, qd.ptr, dd.ptr, sd.ptr)
    backend.gemv_q8_dev(dev, qd.ptr, dd.ptr, sd.ptr, y2.ptr)
    backend.synchronize()
    a, b = y1.to_host(np.float32), y2.to_host(np.float32)
    want = oracle.Pool(8).matmul(t, w, pih.row_bytes(t, k), k, x, 1, rows, oracle.Act(x, k, 1))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(a.view(np.uint32), want.view(np.uint32))


def test_gemv_config2_head(pih, backend, oracle):
    """Q6_K output head, 122753 x 2304; x ~ N(0,1), RMS-normalised."""
    rows, k = 122753, 2304
    w = pih.synth_q6k_random(2, rows, k)
    x = pih.synth_normal(22, k)
    x = (x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)).astype(np.float32)
    dev = backend.upload(Q6_K, w, rows, k)
    xd = backend.to_device(x)
    yd = backend.alloc(rows * 4)
    backend.gemv_dev(dev, xd.ptr, yd.ptr)
    backend.synchronize()
    got = yd.to_host(np.float32)
    want = oracle.Pool(16).matmul(Q6_K, w, pih.row_bytes(Q6_K, k), k, x, 1, rows, oracle.Act(x, k, 1))
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_selftest_vectors_values(pih, backend):
    """The OpenCL self-test blocks (opencl.rs:391-430): closed forms -0.6, 5.2."""
    x = ((np.arange(256) % 7).astype(np.float32) * np.float32(0.1) - np.float32(0.3)).astype(np.float32)
    w4 = np.zeros(144, np.uint8)
    w4[0:2] = (0x00, 0x3C)
    w4[4] = 1
    w4[16:] = 0x21
    w6 = np.zeros(210, np.uint8)
    w6[:128], w6[128:192], w6[192:208] = 0x95, 0x1B, 2
    w6[208:210] = (0x00, 0x3C)
    assert abs(backend.matvec(Q4_K, w4, 256, x, 1)[0] - (-0.6)) <= 0.6 * 0.02 + 0.01
    assert abs(backend.matvec(Q6_K, w6, 256, x, 1)[0] - 5.2) <= 5.2 * 0.02 + 0.01
    backend.clear_weight_cache()


def test_fail_next_is_reported_then_clears(pih, backend):
    w = pih.synth_q4k_random(9, 4, 256)
    x = np.ones(256, np.float32)
    backend.fail_next()
    with pytest.raises(pih.PiError) as e:
        backend.matvec(Q4_K, w, 256, x, 4)
    assert e.value.code == -6
    backend.matvec(Q4_K, w, 256, x, 4)
    backend.clear_weight_cache()


def test_matvec_rejects_bad_shapes(pih, backend):
    w = pih.synth_q4k_random(9, 4, 256)
    with pytest.raises(pih.PiError):
        backend.matvec(Q4_K, w, 512, np.ones(512, np.float32), 4)
    with pytest.raises(pih.PiError):
        backend.matvec(0, w, 256, np.ones(256, np.float32), 4)


@pytest.mark.parametrize("n", [1 << 20, 4096 * 16 + 5, 7])
def test_copy_d2d(pih, backend, n):
    """Copy kernel for the 16-byte bulk plus a runtime copy of the tail."""
    src = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8)
    s, d = backend.to_device(src), backend.alloc(n)
    backend.copy_d2d(d, s, n)
    backend.synchronize()
    assert np.array_equal(d.to_host(np.uint8), src)
