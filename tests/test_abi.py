"""The C ABI library loads and exports every function include/*.h declares;
host-only helpers (synthetic data, quantizers) work without a GPU."""
import ctypes
import hashlib
import json
import re
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
HEADERS = sorted((REPO / "include").glob("*.h"))
Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14


def declared_functions():
    names = []
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:[A-Za-z_][\w\s\*]*?[\s\*])(pi_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_functions():
    names = declared_functions()
    assert "pi_hip_matvec" in names and "pi_hip_selftest" in names and len(names) >= 40


def test_library_exports_every_declared_symbol(pih):
    lib = ctypes.CDLL(str(pih.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(pih.EXPORTS) == declared_functions()


def test_probe_without_device_reports_error(pih):
    # on a machine without a GPU the probe says so instead of crashing
    import os
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present")
    assert pih.probe() is None


def test_synth_is_deterministic_and_thread_independent(pih):
    a = pih.synth_tensor(5, Q4_K, 64, 512, 0.0, 0.02, threads=1)
    b = pih.synth_tensor(5, Q4_K, 64, 512, 0.0, 0.02, threads=7)
    assert np.array_equal(a, b)
    c = pih.synth_tensor(6, Q4_K, 64, 512, 0.0, 0.02, threads=3)
    assert not np.array_equal(a, c)


def test_synth_normal_moments(pih):
    x = pih.synth_normal(11, 200_000, 0.0, 1.0).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert abs((x ** 3).mean()) < 0.03 and abs((x ** 4).mean() - 3.0) < 0.06


@pytest.mark.parametrize("t,k,tol", [(Q8_0, 256, 0.01), (Q4_0, 256, 0.15), (Q4_K, 512, 0.12), (Q6_K, 512, 0.04)])
def test_quantize_row_roundtrip(pih, oracle, t, k, tol):
    """The encoders produce blocks that the reference layout decodes back to
    the input (relative RMS error bounded by the format's resolution)."""
    x = pih.synth_normal(3, k, 0.0, 0.02)
    blocks = pih.quantize_row(t, x)
    y = oracle.dequant_row(t, blocks, k)
    rel = np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert rel < tol


def test_random_block_generators_ranges(pih, oracle):
    w = pih.synth_q4k_random(1, 8, 512)
    d = np.array([oracle.f16_to_f32(int(w[i]) | (int(w[i + 1]) << 8)) for i in range(0, w.size, 144)])
    dm = np.array([oracle.f16_to_f32(int(w[i + 2]) | (int(w[i + 3]) << 8)) for i in range(0, w.size, 144)])
    assert d.min() >= 9.9e-4 and d.max() <= 2.001e-2 and dm.min() >= 9.9e-4 and dm.max() <= 2.001e-2
    w6 = pih.synth_q6k_random(1, 8, 512).reshape(-1, 210)
    sc = w6[:, 192:208].view(np.int8)
    assert sc.min() >= -64 and sc.max() <= 63
    d6 = np.array([oracle.f16_to_f32(int(r[208]) | (int(r[209]) << 8)) for r in w6])
    assert d6.min() >= 9.9e-5 and d6.max() <= 5.001e-3


def test_golden_fixture_tensors_reproduce(pih):
    """The synthetic generator gives the same bytes here as when the fixture
    was written (checked on a few tensors of the 2B model)."""
    g = json.loads((REPO / "tests/golden/minicpm2b_greedy.json").read_text())
    spec = pih.minicpm2b_spec()
    assert g["weight_bytes_per_token"] == 1766384226
    names = ["blk.39.attn_norm.weight"]
    idx = {"blk.39.attn_norm.weight": 1 + 39 * 9}
    for n in names:
        t = pih.synth_tensor(g["model_seed"] * 1000003 + idx[n], 0, 1, spec.n_embd, 1.0, 0.02)
        assert hashlib.sha256(t.tobytes()).hexdigest() == g["tensor_sha256"][n]
