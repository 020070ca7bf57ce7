"""The reference's own known-answer tests, restated against the CPU oracle.

Each test cites the reference test it follows (paths relative to
rust/pocketinfer/).  These pin the oracle before it is trusted as the checker
of the HIP library.
"""
from fractions import Fraction

import numpy as np
import pytest

from conftest import lcg

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
ONE_F16 = (0x00, 0x3C)


def test_q6k_block_layout(oracle):
    """tests/quant_layout.rs:3-24"""
    block = np.zeros(210, np.uint8)
    block[0], block[128], block[192], block[194], block[196], block[198] = 0x19, 0x55, 1, 2, 3, 4
    block[208:210] = ONE_F16
    out = oracle.dequant_row(Q6_K, block, 256)
    assert out[0] == -7.0 and out[32] == -32.0 and out[64] == -45.0 and out[96] == -64.0 and out[1] == -32.0


def test_q4k_block_layout(oracle):
    """tests/quant_layout.rs:26-39"""
    block = np.zeros(144, np.uint8)
    block[0:2] = ONE_F16
    block[2:4] = ONE_F16
    block[4], block[8], block[16] = 1, 0, 0x21
    out = oracle.dequant_row(Q4_K, block, 256)
    assert out[0] == 1.0 and out[1] == 0.0 and out[32] == 0.0


@pytest.mark.parametrize("v", [0.0, 1.0, -1.0, 0.5, 0.1, 65504.0, 6.1e-5, -0.333])
def test_f16_roundtrip(oracle, v):
    """tests/quant_layout.rs:41-48"""
    back = oracle.f16_to_f32(oracle.f32_to_f16(v))
    assert abs(back - v) <= abs(v) * 1e-3 + 1e-6


def test_f16_exhaustive_against_numpy(oracle):
    """f16 -> f32 is exact for every half (util.rs:76-100) and f32 -> f16 is
    round-to-nearest-even (util.rs:102-138); numpy implements IEEE binary16
    independently."""
    lib = oracle.lib()
    halves = np.arange(65536, dtype=np.uint32)
    got = np.array([lib.po_f16_to_f32(int(h)) for h in halves], np.float32)
    want = halves.astype(np.uint16).view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    rng = np.random.default_rng(5)
    xs = np.concatenate([(rng.standard_normal(20000) * 10.0 ** rng.integers(-8, 5, 20000)).astype(np.float32),
                         np.array([65504, 65519.99, 65520, 6.0e-8, 2.98e-8, 1e-9, -0.0], np.float32)])
    got16 = np.array([lib.po_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got16, xs.astype(np.float16).view(np.uint16))


def test_int8_q8_0_matches(oracle):
    """tests/quant_layout.rs:50-66: want 496 +- 0.5"""
    w = np.zeros(34, np.uint8)
    w[0:2] = ONE_F16
    w[2:] = np.arange(32, dtype=np.uint8)
    act = oracle.Act(np.ones(32, np.float32), 32, 1)
    assert abs(oracle.dot_row_q8(Q8_0, w, 32, act) - 496.0) < 0.5


def test_int8_q4_0_matches(oracle):
    """tests/quant_layout.rs:68-84: want 32 +- 0.5"""
    w = np.zeros(18, np.uint8)
    w[0:2] = ONE_F16
    w[2:] = 0x99
    act = oracle.Act(np.ones(32, np.float32), 32, 1)
    assert abs(oracle.dot_row_q8(Q4_0, w, 32, act) - 32.0) < 0.5


def test_int8_q4k_matches_scalar(oracle):
    """tests/quant_layout.rs:86-108"""
    w = np.zeros(144, np.uint8)
    w[0:2] = ONE_F16
    w[2:4] = ONE_F16
    w[4], w[8] = 1, 2
    w[16:] = 0x21
    x = (0.25 + (np.arange(256) % 7).astype(np.float32) * np.float32(0.01)).astype(np.float32)
    got = oracle.dot_row_q8(Q4_K, w, 256, oracle.Act(x, 256, 1))
    want = oracle.dot_row(Q4_K, w, 256, x)
    assert abs(got - want) <= abs(want) * 0.02 + 1.0


def test_int8_q6k_matches_scalar(oracle):
    """tests/quant_layout.rs:110-135"""
    w = np.zeros(210, np.uint8)
    w[:128], w[128:192], w[192:208] = 0x95, 0x1B, 2
    w[208:210] = ONE_F16
    x = (0.5 + (np.arange(256) % 5).astype(np.float32) * np.float32(0.02)).astype(np.float32)
    got = oracle.dot_row_q8(Q6_K, w, 256, oracle.Act(x, 256, 1))
    want = oracle.dot_row(Q6_K, w, 256, x)
    assert abs(got - want) <= abs(want) * 0.02 + 1.0


def _lcg_bytes(st, n):
    out = np.empty(n, np.uint8)
    for i in range(n):
        st, v = lcg(st)
        out[i] = v & 0xFF
    return st, out


def _lcg_x(st, n):
    out = np.empty(n, np.float32)
    for i in range(n):
        st, v = lcg(st)
        out[i] = np.float32(v % 2000) / np.float32(1000.0) - np.float32(1.0)
    return st, out


def test_int8_q4k_random_block(oracle):
    """tests/quant_layout.rs:142-168 (LCG seed 12345, k=2048, 2% + 0.01)"""
    st = 12345
    w = np.zeros(288 * 8, np.uint8)
    w[0:2] = (0x00, 0x32)
    w[2:4] = (0x00, 0x2C)
    st, w[4:] = _lcg_bytes(st, 288 * 8 - 4)
    for blk in range(8):
        w[blk * 144:blk * 144 + 2] = (0x00, 0x30)
        w[blk * 144 + 2:blk * 144 + 4] = (0x00, 0x28)
    st, x = _lcg_x(st, 2048)
    got = oracle.dot_row_q8(Q4_K, w, 2048, oracle.Act(x, 2048, 1))
    want = oracle.dot_row(Q4_K, w, 2048, x)
    assert abs(got - want) <= abs(want) * 0.02 + 0.01


def test_int8_q6k_random_block(oracle):
    """tests/quant_layout.rs:170-192 (LCG seed 999, k=512)"""
    st, w = _lcg_bytes(999, 420)
    w[208:210] = (0x00, 0x34)
    w[418:420] = (0x00, 0x34)
    st, x = _lcg_x(st, 512)
    got = oracle.dot_row_q8(Q6_K, w, 512, oracle.Act(x, 512, 1))
    want = oracle.dot_row(Q6_K, w, 512, x)
    assert abs(got - want) <= abs(want) * 0.02 + 0.01


def test_row_dot_multi_matches_dot_row(oracle):
    """tests/quant_layout.rs:194-224 (seed 777, b=5, k=1024, 1e-4)"""
    st, w = _lcg_bytes(777, 144 * 4)
    for blk in range(4):
        w[blk * 144:blk * 144 + 2] = (0x00, 0x30)
        w[blk * 144 + 2:blk * 144 + 4] = (0x00, 0x28)
    k, b = 1024, 5
    st, xt = _lcg_x(st, k * b)
    multi = oracle.row_dot_multi(Q4_K, w, k, xt, b)
    for bi in range(b):
        single = oracle.dot_row(Q4_K, w, k, xt.reshape(k, b)[:, bi].copy())
        assert abs(multi[bi] - single) <= abs(single) * 1e-4 + 1e-4


def _random_row(st, t, k):
    be, bb = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}[t]
    nblk = k // be
    st, row = _lcg_bytes(st, bb * nblk)
    for blk in range(nblk):
        base = blk * bb
        row[base:base + 2] = (0x00, 0x32)
        if t == Q4_K:
            row[base + 2:base + 4] = (0x00, 0x2C)
        elif t == Q6_K:
            row[base + 208:base + 210] = (0x00, 0x32)
    return st, row


def test_int8_multi_matches_single(oracle):
    """tests/quant_layout.rs:242-286 (seed 4242, b=32, k=1024)"""
    st, b, k = 4242, 32, 1024
    for t in (Q4_0, Q8_0, Q4_K, Q6_K):
        st, row = _random_row(st, t, k)
        st, x = _lcg_x(st, k * b)
        act = oracle.Act(x, k, b)
        multi = oracle.dot_row_q8_lanes(t, row, k, act)
        for lane in range(b):
            single = oracle.dot_row_q8(t, row, k, act, lane)
            assert abs(multi[lane] - single) <= abs(single) * 1e-5 + 1e-4


def test_int8_multi_exact_bitwise(oracle):
    """tests/quant_layout.rs:327-357 (seed 99, b=32, k=512): to_bits equality"""
    st, b, k = 99, 32, 512
    for t in (Q4_K, Q6_K):
        st, row = _random_row(st, t, k)
        st, x = _lcg_x(st, k * b)
        act = oracle.Act(x, k, b)
        multi = oracle.dot_row_q8_lanes(t, row, k, act)
        single = np.array([oracle.dot_row_q8(t, row, k, act, lane) for lane in range(b)], np.float32)
        assert np.array_equal(multi.view(np.uint32), single.view(np.uint32))


def test_q8_halfway_values(oracle):
    """simd_q8.rs:58-80: k=512, x_i = (i mod 73 - 36)/16, x0 = 127, x1 = 0.5,
    x2 = -0.5.  Block 0 has amax 127, so d = 1 and the halfway values round
    away from zero to +1 and -1; the rest follow the rule restated with
    float64 rounding (exact for float32 products)."""
    k = 512
    x = ((np.arange(k) % 73).astype(np.float32) - np.float32(36.0)) * np.float32(0.0625)
    x[0], x[1], x[2] = 127.0, 0.5, -0.5
    act = oracle.Act(x, k, 1)
    assert act.d[0] == 1.0 and act.q[0] == 127 and act.q[1] == 1 and act.q[2] == -1
    for blk in range(k // 32):
        xb = x[blk * 32:(blk + 1) * 32]
        amax = np.float32(np.max(np.abs(xb)))
        d = np.float32(amax / np.float32(127.0))
        inv = np.float32(np.float32(1.0) / d) if d > 0 else np.float32(0.0)
        prod = (xb * inv).astype(np.float64)
        q = np.clip(np.sign(prod) * np.floor(np.abs(prod) + 0.5), -127, 127).astype(np.int32)
        assert np.array_equal(act.q[blk * 32:(blk + 1) * 32].astype(np.int32), q), blk
        assert act.d[blk].view(np.uint32) == d.view(np.uint32)
        assert act.sum[blk] == q.sum()


def _selftest_x():
    return [Fraction(j % 7, 10) - Fraction(3, 10) for j in range(256)]


def test_opencl_selftest_vectors_closed_form(oracle):
    """backend/opencl.rs:391-430.  Q4_K block: only sub-block 0 has a scale
    (1) and every low nibble is 1, so the dot is sum_{j<32} x_j = -0.6.  Q6_K
    block: ql=0x95, qh=0x1B give q = (21, 5, -7, -23) for the four 32-element
    quarters of each half, every scale 2, so the dot is
    2 * sum_quarters q_s * sum(x over the quarter)."""
    xs = _selftest_x()
    x = np.array([float(v) for v in xs], np.float32)
    w4 = np.zeros(144, np.uint8)
    w4[0:2] = ONE_F16
    w4[4] = 1
    w4[16:] = 0x21
    want4 = float(sum(xs[:32]))
    assert want4 == pytest.approx(-0.6)
    assert oracle.dot_row(Q4_K, w4, 256, x) == pytest.approx(want4, abs=1e-5)
    w6 = np.zeros(210, np.uint8)
    w6[:128], w6[128:192], w6[192:208] = 0x95, 0x1B, 2
    w6[208:210] = ONE_F16
    qs = (21, 5, -7, -23)
    want6 = float(sum(2 * qs[s] * sum(xs[h * 128 + 32 * s:h * 128 + 32 * s + 32]) for h in range(2) for s in range(4)))
    assert want6 == pytest.approx(5.2)
    assert oracle.dot_row(Q6_K, w6, 256, x) == pytest.approx(want6, abs=1e-4)
    # and the int8 path passes the reference's self-test tolerance
    act = oracle.Act(x, 256, 1)
    for t, w, want in ((Q4_K, w4, want4), (Q6_K, w6, want6)):
        got = oracle.dot_row_q8(t, w, 256, act)
        assert abs(got - want) <= abs(want) * 0.02 + 0.01
