"""pi_hip_matvec_noalloc (no device allocation; x and y staged in the
library's static device array) against pi_hip_matvec, through the C ABI."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14


def _rows(pih, t, rows, k, seed):
    if t == Q4_K:
        return pih.synth_q4k_random(seed, rows, k)
    if t == Q6_K:
        return pih.synth_q6k_random(seed, rows, k)
    return pih.synth_tensor(seed, t, rows, k, 0.0, 0.02)


def test_matvec_noalloc_equals_matvec_twice(pih, backend):
    """Two calls in a row, the second on a smaller tensor: each output equals
    pi_hip_matvec's bit for bit (the same kernel on the same Q8 input)."""
    for t, rows, k, seed in [(Q4_K, 5760, 2304, 1), (Q6_K, 29, 512, 2)]:
        w = _rows(pih, t, rows, k, 500 + seed)
        x = np.random.default_rng(seed).standard_normal(k).astype(np.float32)
        want = backend.matvec(t, w, k, x, rows)
        dev = backend.upload(t, w, rows, k)
        got = backend.matvec_noalloc(dev, x)
        assert got.shape == want.shape
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (t, rows, k)
        dev.free()
    backend.clear_weight_cache()


def test_matvec_noalloc_rejects_oversize(pih, backend):
    # rows longer than PI_NOALLOC_MAX_K cannot be uploaded at all (at most 64
    # units of at most 8 blocks per row), so only the row limit is reachable
    k = pih.PI_NOALLOC_MAX_K + 256
    with pytest.raises(pih.PiError):
        backend.upload(Q8_0, _rows(pih, Q8_0, 2, k, 3), 2, k)
    rows = pih.PI_NOALLOC_MAX_ROWS + 1
    w = _rows(pih, Q8_0, rows, 32, 4)
    dev = backend.upload(Q8_0, w, rows, 32)
    with pytest.raises(pih.PiError) as e:
        backend.matvec_noalloc(dev, np.ones(32, np.float32))
    assert e.value.code == -1
    dev.free()
