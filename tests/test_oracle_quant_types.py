"""The oracle's dequantization of the GGUF types the int8 path does not cover
(quant.rs:102-359): Q4_1, Q5_0, Q5_1, Q8_1, Q8_K, Q2_K, Q3_K, Q5_K, F16 and
BF16, and the single-token f32 dot over them (`dot_row_scalar`,
quant.rs:377-441).

Each block is assembled here from chosen integer fields by an encoder written
from the GGUF block layouts (which byte and bit holds which element), not from
the oracle's decoder.  With power-of-two scales every dequantized value is an
exact small number, so the expected values follow from integer arithmetic:
a wrong nibble, bit, byte or scale index, or a dropped minimum, changes them.

The reference's own Q2_K, Q3_K and Q5_K decoders advance their quant / mask
index past the end of the slice they index (quant.rs:211, 254, 295-314) and
panic on every block; the oracle follows the GGUF layout for those three
types (the test below shows the layout is the format's: every element reaches
a distinct quant bit position).
"""
import numpy as np
import pytest

F32, F16, Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K, Q8_K, BF16 = 0, 1, 3, 6, 7, 9, 10, 11, 13, 15, 30
F16_BITS = {0.25: 0x3400, 0.5: 0x3800, 1.0: 0x3C00, 2.0: 0x4000, -1.0: 0xBC00}


def h(v):
    return F16_BITS[v].to_bytes(2, "little")


def enc_q4_1(d, m, q):                       # q[32] in 0..15
    qs = bytes((q[j] & 15) | ((q[j + 16] & 15) << 4) for j in range(16))
    return h(d) + h(m) + qs, [qi * d + m for qi in q]


def enc_q5(q):                               # q[32] in 0..31 -> qh, qs
    qh = 0
    for j in range(32):
        qh |= ((q[j] >> 4) & 1) << j
    qs = bytes((q[j] & 15) | ((q[j + 16] & 15) << 4) for j in range(16))
    return qh.to_bytes(4, "little"), qs


def enc_q5_0(d, q):
    qh, qs = enc_q5(q)
    return h(d) + qh + qs, [(qi - 16) * d for qi in q]


def enc_q5_1(d, m, q):
    qh, qs = enc_q5(q)
    return h(d) + h(m) + qh + qs, [qi * d + m for qi in q]


def enc_q8_1(d, q):                          # q[32] int8; s is not read
    return h(d) + h(1.0) + bytes(v & 255 for v in q), [v * d for v in q]


def enc_q8_k(d, q):                          # q[256] int8, d f32, bsums not read
    return np.float32(d).tobytes() + bytes(v & 255 for v in q) + bytes(32), [v * d for v in q]


def enc_q2_k(d, dmin, sc, mn, q):            # sc, mn[16] in 0..15; q[256] in 0..3
    scales = bytes((sc[i] & 15) | ((mn[i] & 15) << 4) for i in range(16))
    qs = bytearray(64)
    vals = []
    for i in range(256):
        hh, r = divmod(i, 128)
        j, l = divmod(r, 32)
        qs[32 * hh + l] |= (q[i] & 3) << (2 * j)
        g = 8 * hh + 2 * j + (l >= 16)
        vals.append(d * sc[g] * q[i] - dmin * mn[g])
    return scales + bytes(qs) + h(d) + h(dmin), vals


def enc_q3_k(d, sc, q):                      # sc[16] in 0..63 (value - 32 is the scale); q[256] in -4..3
    hm, qs, sb = bytearray(32), bytearray(64), bytearray(12)
    for g in range(16):
        if g < 8:
            sb[g] |= sc[g] & 15
        else:
            sb[g - 8] |= (sc[g] & 15) << 4
        sb[8 + g % 4] |= ((sc[g] >> 4) & 3) << (2 * (g // 4))
    vals = []
    for i in range(256):
        hh, r = divmod(i, 128)
        j, l = divmod(r, 32)
        v = q[i] + 4 if q[i] < 0 else q[i]            # low 2 bits; the high bit set means "no -4"
        qs[32 * hh + l] |= (v & 3) << (2 * j)
        if q[i] >= 0:
            hm[l] |= 1 << (4 * hh + j)
        g = 8 * hh + 2 * j + (l >= 16)
        vals.append(d * (sc[g] - 32) * q[i])
    return bytes(hm) + bytes(qs) + bytes(sb) + h(d), vals


def enc_scale_min_k4(sc, mn):                 # 8 six-bit (scale, min) pairs -> 12 bytes
    b = bytearray(12)
    for j in range(8):
        if j < 4:
            b[j] |= sc[j] & 63
            b[j + 4] |= mn[j] & 63
        else:
            b[j + 4] |= (sc[j] & 15) | ((mn[j] & 15) << 4)
            b[j - 4] |= (sc[j] >> 4) << 6
            b[j] |= (mn[j] >> 4) << 6
    return bytes(b)


def enc_q5_k(d, dmin, sc, mn, q):            # sc, mn[8] in 0..63; q[256] in 0..31
    qh, qs = bytearray(32), bytearray(128)
    vals = []
    for i in range(256):
        p, r = divmod(i, 64)
        hi, l = divmod(r, 32)
        qs[32 * p + l] |= (q[i] & 15) << (4 * hi)
        qh[l] |= ((q[i] >> 4) & 1) << (2 * p + hi)
        g = 2 * p + hi
        vals.append(d * sc[g] * q[i] - dmin * mn[g])
    return h(d) + h(dmin) + enc_scale_min_k4(sc, mn) + bytes(qh) + bytes(qs), vals


def _dq(oracle, t, blk, k):
    return oracle.dequant_row(t, np.frombuffer(blk, np.uint8).copy(), k)


@pytest.mark.parametrize("seed", range(6))
def test_legacy_blocks(oracle, seed):
    rng = np.random.default_rng(seed)
    for d in (1.0, 0.5, 2.0):
        q = [int(v) for v in rng.integers(0, 16, 32)]
        blk, want = enc_q4_1(d, -1.0, q)
        assert len(blk) == 20 and _dq(oracle, Q4_1, blk, 32).tolist() == want
        q = [int(v) for v in rng.integers(0, 32, 32)]
        blk, want = enc_q5_0(d, q)
        assert len(blk) == 22 and _dq(oracle, Q5_0, blk, 32).tolist() == want
        blk, want = enc_q5_1(d, 0.25, q)
        assert len(blk) == 24 and _dq(oracle, Q5_1, blk, 32).tolist() == want
        q = [int(v) for v in rng.integers(-128, 128, 32)]
        blk, want = enc_q8_1(d, q)
        assert len(blk) == 36 and _dq(oracle, Q8_1, blk, 32).tolist() == want
        q = [int(v) for v in rng.integers(-128, 128, 256)]
        blk, want = enc_q8_k(d, q)
        assert len(blk) == 292 and _dq(oracle, Q8_K, blk, 256).tolist() == want


@pytest.mark.parametrize("seed", range(6))
def test_k_blocks(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    for d, dmin in ((1.0, 1.0), (0.5, 2.0), (2.0, 0.25)):
        sc, mn = [int(v) for v in rng.integers(0, 16, 16)], [int(v) for v in rng.integers(0, 16, 16)]
        q = [int(v) for v in rng.integers(0, 4, 256)]
        blk, want = enc_q2_k(d, dmin, sc, mn, q)
        assert len(blk) == 84 and _dq(oracle, Q2_K, blk, 256).tolist() == want
        sc3 = [int(v) for v in rng.integers(0, 64, 16)]
        q3 = [int(v) for v in rng.integers(-4, 4, 256)]
        blk, want = enc_q3_k(d, sc3, q3)
        assert len(blk) == 110 and _dq(oracle, Q3_K, blk, 256).tolist() == want
        sc5, mn5 = [int(v) for v in rng.integers(0, 64, 8)], [int(v) for v in rng.integers(0, 64, 8)]
        q5 = [int(v) for v in rng.integers(0, 32, 256)]
        blk, want = enc_q5_k(d, dmin, sc5, mn5, q5)
        assert len(blk) == 176 and _dq(oracle, Q5_K, blk, 256).tolist() == want


def test_every_k_element_has_its_own_bits(oracle):
    """One quant set at a time (every other field fixed): exactly that element
    moves, for each of the 256 positions of Q2_K, Q3_K and Q5_K."""
    sc, mn = [1] * 16, [0] * 16
    base2, _ = enc_q2_k(1.0, 1.0, sc, mn, [0] * 256)
    base3, _ = enc_q3_k(1.0, [33] * 16, [0] * 256)
    base5, _ = enc_q5_k(1.0, 1.0, [1] * 8, [0] * 8, [0] * 256)
    z2, z3, z5 = _dq(oracle, Q2_K, base2, 256), _dq(oracle, Q3_K, base3, 256), _dq(oracle, Q5_K, base5, 256)
    for i in range(0, 256, 7):
        q = [0] * 256
        q[i] = 3
        d2 = _dq(oracle, Q2_K, enc_q2_k(1.0, 1.0, sc, mn, q)[0], 256) - z2
        assert np.flatnonzero(d2).tolist() == [i] and d2[i] == 3.0
        d3 = _dq(oracle, Q3_K, enc_q3_k(1.0, [33] * 16, q)[0], 256) - z3
        assert np.flatnonzero(d3).tolist() == [i] and d3[i] == 3.0
        q[i] = 17                                   # the high bit of Q5_K as well
        d5 = _dq(oracle, Q5_K, enc_q5_k(1.0, 1.0, [1] * 8, [0] * 8, q)[0], 256) - z5
        assert np.flatnonzero(d5).tolist() == [i] and d5[i] == 17.0


def test_half_and_bfloat_rows(oracle):
    vals = np.array([1.0, -2.5, 0.0, 65504.0, 3.0e-5], np.float32)
    f16 = vals.astype(np.float16).view(np.uint16)
    got = _dq(oracle, F16, f16.astype("<u2").tobytes(), vals.size)
    assert np.array_equal(got, vals.astype(np.float16).astype(np.float32))
    bf = (vals.view(np.uint32) >> 16).astype("<u2")
    got = _dq(oracle, BF16, bf.tobytes(), vals.size)
    assert np.array_equal(got.view(np.uint32), (vals.view(np.uint32) >> 16) << 16)


def test_f32_dot_order(oracle):
    """dot_row_scalar's generic form: 0 + w_0 x_0 + w_1 x_1 + ... with each
    product rounded (quant.rs:428-440).  One-hot x picks one weight exactly;
    x of ones sums exact integers; and 1 + 2^-24 + ... shows the order: the
    ordered sum of (1, 2^-24, 2^-24) rounds both small terms away, the
    reversed one would keep them."""
    rng = np.random.default_rng(7)
    q = [int(v) for v in rng.integers(0, 32, 256)]
    blk, want = enc_q5_k(1.0, 1.0, [int(v) for v in rng.integers(0, 64, 8)], [int(v) for v in rng.integers(0, 64, 8)], q)
    row = np.frombuffer(blk, np.uint8).copy()
    for i in (0, 37, 255):
        x = np.zeros(256, np.float32)
        x[i] = 1.0
        assert oracle.dot_row(Q5_K, row, 256, x) == np.float32(want[i])
    assert oracle.dot_row(Q5_K, row, 256, np.ones(256, np.float32)) == float(sum(want))
    # Q8_K weights 1, then 2^-24 twice: the order 1 + a + b keeps 1.0
    q8 = [0] * 256
    q8[0], q8[1], q8[2] = 1, 1, 1
    blk, _ = enc_q8_k(1.0, q8)
    row = np.frombuffer(blk, np.uint8).copy()
    x = np.zeros(256, np.float32)
    x[0], x[1], x[2] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert oracle.dot_row(Q8_K, row, 256, x) == 1.0
    x[0], x[1], x[2] = 2.0 ** -24, 2.0 ** -24, 1.0
    assert oracle.dot_row(Q8_K, row, 256, x) == np.float32(1.0 + 2.0 ** -23)
