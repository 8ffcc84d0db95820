"""Sessions that alternate between the HIP backend and a host backend. The HIP build ships no CPU
backend; oracle/test_cpu_backend.cpp (libvknn_testcpu.so, test infrastructure) registers a minimal
one, which a session uses only with the option cpu_fallback=1 — the reference's CPU fallback
(src/core/session.cpp partitioning, src/backend/cpu) exercised through the same Session code.

  * host only (no device): a session whose every node the host backend runs, checked against numpy
  * the alternating network of tests/onnx_writer.py (mixed_model) splits into seven segments,
    HIP -> CPU -> HIP -> CPU -> HIP -> CPU -> HIP, with the boundary tensors the graph implies, and
    its output matches tests/golden/onnx_mixed.npz (the reference importer + CPU backend on the same
    model); bar max|d|/max|ref| <= 2e-2, cosine >= 0.9999 (fp16 storage on the HIP segments)
  * without cpu_fallback=1 the same model is refused (no silent host fallback)
"""
import ctypes
import hashlib
import os

import numpy as np
import pytest

import vknn_amd as V
from tests import onnx_writer as W
from tests.golden.make_onnx_golden import MIXED_IN, MIXED_OUT
from tests.oracle_lib import parity

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "libvknn_testcpu.so")
GOLDEN = os.path.join(ROOT, "tests", "golden", "onnx_mixed.npz")


@pytest.fixture(scope="module")
def host_backend():
    V.vknn()  # the product library first: the test backend registers into its registry
    if not os.path.exists(LIB):
        pytest.skip("oracle/libvknn_testcpu.so not built")
    lib = ctypes.CDLL(LIB, mode=ctypes.RTLD_GLOBAL)
    assert lib.vknn_test_cpu_backend_register() == 0
    return lib


def _session(path, options):
    h = ctypes.c_void_p()
    if V.vknn().vknn_session_create_onnx(str(path).encode(), options.encode(), ctypes.byref(h)):
        raise V.VkhipError(V.vknn().vknn_last_error().decode(errors='replace'))
    s = V.Session.__new__(V.Session)
    s.h = h.value
    return s


def _run(s, x, n):
    y = np.zeros(n, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    if V.vknn().vknn_session_run_host(s.h, x.ctypes.data, x.size, y.ctypes.data, y.size):
        raise V.VkhipError(V.vknn().vknn_last_error().decode(errors='replace'))
    return y


def test_host_only_session(host_backend, tmp_path):
    if V.vkhip().vkhip_available() == 1:
        pytest.skip("a device is present: the HIP backend would take the pooling node")
    p = W.host_only_model(str(tmp_path / "h.onnx"))
    s = _session(p, "cpu_fallback=1")
    assert [(b, n) for b, n, _, _ in s.segments()] == [("CPU(test)", 5)]
    x = np.random.default_rng(1).standard_normal((2, 3, 4, 5)).astype(np.float32)
    l = np.where(x >= 0, x, 0.2 * x)
    t = np.tanh(l) + x
    e = np.where(t >= 0, t, np.expm1(t))
    np.testing.assert_allclose(_run(s, x, 6), e.mean((2, 3)).ravel(), rtol=1e-5, atol=1e-6)


def test_mixed_fixture_is_pinned(tmp_path):
    """The committed outputs belong to this model and agree with a plain fp32 torch restatement."""
    import torch
    import torch.nn.functional as F
    z = np.load(GOLDEN)
    blob = open(W.mixed_model(str(tmp_path / "m.onnx")), "rb").read()
    assert hashlib.sha256(blob).digest() == z["model_sha256"].tobytes(), "mixed model bytes changed: rerun make_onnx_golden.py"
    r = np.random.default_rng(5)
    wa = torch.tensor((r.standard_normal((12, 8, 3, 3)) * 0.2).astype(np.float32))
    ba = torch.tensor((r.standard_normal(12) * 0.1).astype(np.float32))
    wb = torch.tensor((r.standard_normal((12, 12, 1, 1)) * 0.3).astype(np.float32))
    bb = torch.tensor((r.standard_normal(12) * 0.1).astype(np.float32))
    wc = torch.tensor((r.standard_normal((8, 12, 1, 1)) * 0.3).astype(np.float32))
    x = torch.tensor(z["x"])
    a = F.conv2d(x, wa, ba, padding=1)
    s = torch.tanh(F.conv2d(F.leaky_relu(a, 0.1), wb, bb)) + a
    y = F.conv2d(F.elu(s, 0.7), wc).mean((2, 3))
    np.testing.assert_allclose(z["y"], y.numpy().ravel(), rtol=1e-4, atol=1e-5)


@pytest.mark.gpu
def test_hip_cpu_alternating_segments(gpu, host_backend, tmp_path):
    p = W.mixed_model(str(tmp_path / "m.onnx"))
    with pytest.raises(V.VkhipError, match="no backend supports"):
        _session(p, "")
    s = _session(p, "cpu_fallback=1")
    segs = s.segments()
    print(segs, flush=True)
    assert [b for b, _, _, _ in segs] == ["HIP", "CPU(test)", "HIP", "CPU(test)", "HIP", "CPU(test)", "HIP"]
    assert segs[0][3] == ["a"] and segs[2][2] == ["l"] and sorted(segs[4][2]) == ["a", "t"]
    z = np.load(GOLDEN)
    assert list(z["x"].shape) == MIXED_IN
    got = _run(s, z["x"], sum(MIXED_OUT))
    rel, cos = parity(got, z["y"])
    print(f"mixed: max_rel={rel:.2e} cos={cos:.7f}", flush=True)
    assert rel <= 2e-2 and cos >= 0.9999, (rel, cos)
    assert np.array_equal(_run(s, z["x"], sum(MIXED_OUT)), got)
