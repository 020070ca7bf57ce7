"""The oracle's exp / cos / sin / pow (po_detmath.h) against numpy's float64
libm rounded to float32: they must be the correctly rounded float result on
all but a vanishing fraction of inputs, and never more than 1 ulp away."""
import numpy as np
import pytest


def _ulps(a, b):
    ai = a.view(np.int32).astype(np.int64)
    bi = b.view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, np.int64(-2**31) - ai, ai)
    bi = np.where(bi < 0, np.int64(-2**31) - bi, bi)
    return np.abs(ai - bi)


def _check(fn, xs, ref):
    got = np.array([fn(float(x)) for x in xs], np.float32)
    want = ref(xs.astype(np.float64)).astype(np.float32)
    u = _ulps(got, want)
    assert u.max() <= 1, (xs[np.argmax(u)], got[np.argmax(u)], want[np.argmax(u)])
    assert (u > 0).mean() < 1e-3


def test_expf(oracle):
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.uniform(-104, 88, 20000), rng.uniform(-1, 1, 20000), rng.standard_normal(20000) * 5,
                         np.array([0.0, -0.0, 1.0, -1.0, 88.7, -87.3, -103.9, -100.0])]).astype(np.float32)
    _check(oracle.lib().po_det_expf, xs, np.exp)
    lib = oracle.lib()
    assert lib.po_det_expf(0.0) == 1.0 and lib.po_det_expf(-200.0) == 0.0 and np.isinf(lib.po_det_expf(200.0))


@pytest.mark.parametrize("name,ref", [("po_det_cosf", np.cos), ("po_det_sinf", np.sin)])
def test_sincos(oracle, name, ref):
    rng = np.random.default_rng(2)
    # RoPE angles pos * theta^(-2i/d): up to n_ctx radians
    xs = np.concatenate([rng.uniform(0, 20000, 20000), rng.uniform(-4, 4, 20000), np.arange(0, 2048, 0.5)]).astype(np.float32)
    _check(getattr(oracle.lib(), name), xs, ref)


def test_powf(oracle):
    lib = oracle.lib()
    for theta in (10000.0, 500000.0, 1e6):
        ys = (np.arange(64) * 2.0 / 128.0).astype(np.float32)
        got = np.array([lib.po_det_powf(theta, float(y)) for y in ys], np.float32)
        want = np.power(np.float64(theta), ys.astype(np.float64)).astype(np.float32)
        assert _ulps(got, want).max() <= 1
