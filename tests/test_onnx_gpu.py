"""ONNX models on the HIP backend (vknn_session_create_onnx): the imported network runs exactly as
the directly built one does, and the edge-case network matches what the reference computed for it.

  * each benchmark network written as ONNX (tests/onnx_writer.py zoo_to_onnx) and imported gives
    bit-identical outputs to the session over the zoo graph it was written from, with the same
    options and heuristic (untimed) plans so both sessions pick the same kernels
  * the edge-case network (symbolic batch, fp16/double weights, Constant-node parameters, Split
    sizes as an input, ReduceMean pool, ...) against tests/golden/onnx_edge.npz, the output of the
    reference's importer and CPU backend; bar max|d|/max|ref| <= 2e-2, cosine >= 0.9999
"""
import numpy as np
import pytest

import vknn_amd as V
from tests import onnx_writer as W
from tests.golden.make_onnx_golden import EDGE_IN, EDGE_OUT
from tests.oracle_lib import parity
from tests.test_onnx import GOLDEN, zoo_onnx

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("model,batch,opts", [
    ("mnv2_block", 2, "tuning=off"),
    ("resnet50", 2, "tuning=off"),
    ("mobilenetv3_large", 2, "tuning=off;fuse_se=1;fuse_dwpw=1"),
    ("yolov8n", 1, "tuning=off"),
])
def test_onnx_session_equals_zoo_session(gpu, tmp_path, model, batch, opts):
    print(f"onnx vs zoo: {model} N={batch} [{opts}]", flush=True)
    p = zoo_onnx(tmp_path, model, batch)
    zoo = V.Session(model, batch, seed=7, options=opts)
    onx = V.Session.from_onnx(p, zoo.in_shape, zoo.out_elems, options=opts)
    x = np.random.default_rng(9).standard_normal(zoo.in_shape).astype(np.float32)
    a, b = zoo.run(x), onx.run(x)
    assert np.array_equal(a, b), float(np.abs(a - b).max())
    assert onx.describe() == zoo.describe()


def test_edge_model_matches_reference_fixture(gpu, tmp_path):
    z = np.load(GOLDEN)
    p = W.edge_model(str(tmp_path / "edge.onnx"))
    s = V.Session.from_onnx(p, EDGE_IN, EDGE_OUT)
    got = s.run(z["x"])
    rel, cos = parity(got, z["y"])
    print(f"edge: max_rel={rel:.2e} cos={cos:.7f}", flush=True)
    assert rel <= 2e-2 and cos >= 0.9999, (rel, cos)
    assert np.array_equal(s.run(z["x"]), got)
