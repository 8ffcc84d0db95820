"""The ONNX importer (vknn_amd/csrc/host/onnx_import.cpp) against the reference's own importer
(src/import/onnx/*, compiled into oracle/_ref/libvknn_ref.so) on models written by the hand-made
encoder in tests/onnx_writer.py. Host only: no device is needed.

  * every benchmark network, exported from the zoo graph: the imported graph equals the reference's
    import tensor for tensor and node for node, and after the standard passes equals the zoo graph
    after the same passes; the reference runs the ONNX model bit-identically to the zoo graph
  * weight storage variants (float_data, external data file) and ReduceMean pools import alike
  * one small graph per import rule (SSA names, unary defaults, unnamed/unknown nodes, dtypes,
    Constant tensors, value_info hints) equals the reference's import
  * element types the reference reads as zeros are checked against their values instead
  * malformed files are rejected with an error, never read past their end
  * the committed edge-model fixture is what the reference computes, and what a plain fp32 torch
    restatement of that network computes

The reference imports run only where oracle/_ref exists (this container); the rest runs anywhere.
Node ORDER is not compared: the reference's topological sort is FIFO over hash-set predecessor
lists, this build's takes the lowest ready index; both are valid orders of the same nodes.
"""
import ctypes
import hashlib
import os
import struct

import numpy as np
import pytest

import vknn_amd as V
from tests import onnx_writer as W
from tests import oracle_lib as O
from tests.golden.make_onnx_golden import EDGE_IN, EDGE_OUT

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "onnx_edge.npz")
MODELS = ["conv3x3_bn_relu", "mnv2_block", "resnet50", "mobilenetv3_large", "yolov8n"]
need_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (reference build) not available")


def ref_describe(path):
    buf = ctypes.create_string_buffer(1 << 24)
    assert O.ref().ref_onnx_describe(str(path).encode(), buf, len(buf)) == 0, O.ref().ref_last_error()
    return buf.value.decode()


def same_graph(a, b):
    """Equal up to the order of node lines (tensor ids, names, hashes, attributes all compared)."""
    la, lb = sorted(a.splitlines()), sorted(b.splitlines())
    if la != lb:
        diff = [(x, y) for x, y in zip(la, lb) if x != y][:3]
        pytest.fail("imported graphs differ:\n" + "\n".join(f"  ours: {x}\n  ref:  {y}" for x, y in diff))


def zoo_onnx(tmp_path, model, batch=1, **kw):
    vxm = tmp_path / f"{model}.vxm"
    rc = V.vknn().vknn_model_save_vxm(model.encode(), batch, 7, b"passes=0", str(vxm).encode())
    assert rc == 0, V.vknn().vknn_last_error()
    return W.zoo_to_onnx(str(vxm), str(tmp_path / f"{model}.onnx"), **kw)


@need_ref
@pytest.mark.parametrize("model", MODELS)
def test_zoo_model_import_matches_reference(tmp_path, model):
    p = zoo_onnx(tmp_path, model)
    same_graph(V.onnx_describe(p), ref_describe(p))


@pytest.mark.parametrize("model", MODELS)
def test_zoo_model_after_passes_equals_zoo_graph(tmp_path, model):
    p = zoo_onnx(tmp_path, model)
    for opts in ("", "fuse_se=1;fuse_dwpw=1"):
        assert V.onnx_after_passes(p, opts) == V.graph_after_passes(model, 1, opts)


@need_ref
@pytest.mark.parametrize("model", ["conv3x3_bn_relu", "mnv2_block", "mobilenetv3_large", "yolov8n"])
def test_reference_runs_onnx_like_zoo_graph(tmp_path, model):
    p = zoo_onnx(tmp_path, model)
    in_shape, outs = O.model_io(model, 1)
    x = np.random.default_rng(4).standard_normal(in_shape).astype(np.float32)
    y = np.zeros(sum(outs), np.float32)
    assert O.ref().ref_onnx_run(p.encode(), x.ctypes.data, x.size, y.ctypes.data, y.size) == 0, O.ref().ref_last_error()
    assert np.array_equal(y, O.ref_model_run(model, 1, 7, x))


@pytest.mark.parametrize("variant", ["typed", "external", "reduce_mean"])
def test_storage_variants_import_alike(tmp_path, variant):
    base = V.onnx_describe(zoo_onnx(tmp_path, "mnv2_block"))
    d = tmp_path / variant
    d.mkdir()
    kw = dict(weights="typed") if variant == "typed" else dict(weights="external", external_file="weights.bin") \
        if variant == "external" else dict(reduce_mean_gap=True)
    p = zoo_onnx(d, "mnv2_block", **kw)
    got = V.onnx_describe(p)
    if O.ref_available():
        same_graph(got, ref_describe(p))
    if variant != "reduce_mean":
        assert got == base
    else:  # a ReduceMean pool imports as a global average pool with the ReduceMean attributes
        assert V.onnx_after_passes(p) == V.graph_after_passes("mnv2_block", 1)


@need_ref
@pytest.mark.parametrize("case", W.IMPORT_CASES + ["edge"])
def test_import_rules_match_reference(tmp_path, case):
    p = str(tmp_path / f"{case}.onnx")
    W.edge_model(p) if case == "edge" else W.import_case(p, case)
    same_graph(V.onnx_describe(p), ref_describe(p))


def test_import_rules_spot_checks(tmp_path):
    """What the rules must produce, stated directly (holds without the reference too)."""
    p = W.import_case(str(tmp_path / "ssa.onnx"), "ssa")
    d = V.onnx_describe(p)
    outs = [ln for ln in d.splitlines() if ln.startswith("output ")]
    nodes = {ln.split("'")[1]: ln for ln in d.splitlines() if ln.startswith("node ")}
    # the declared output "y" is the LAST producer's tensor (s2), which reads r2's "y"
    out_id = outs[0].split()[1]
    assert ("out=" + out_id + ";") in nodes["s2"]
    r2_out = nodes["r2"].split("out=")[1].split(";")[0]
    assert r2_out != out_id and ("in=" + r2_out + ";") in nodes["s2"]
    p = W.import_case(str(tmp_path / "defaults.onnx"), "defaults")
    lines = [ln for ln in V.onnx_describe(p).splitlines() if ln.startswith("node Unary")]
    hexf = lambda f: struct.pack(">f", f).hex()
    want = [(0.01, 0.0), (1.0, 0.0), (0.2, 0.5), (0.25, 0.0), (0.5, 0.0), (0.125, 0.25)]
    assert len(lines) == 6
    for ln, (lo, hi) in zip(lines, want):
        assert f"lo={hexf(lo)} hi={hexf(hi)}" in ln, ln
    p = W.import_case(str(tmp_path / "unnamed.onnx"), "unnamed")
    names = [ln.split("'")[1] for ln in V.onnx_describe(p).splitlines() if ln.startswith("node ")]
    assert sorted(names) == sorted(["Relu_0", "Unknown_1", "Unary_2", "Reduce_3", "Binary_4"])


def _fnv(b):
    h = 1469598103934665603
    for c in b:
        h = ((h ^ c) * 1099511628211) & (2 ** 64 - 1)
    return "%016x" % h


def test_extra_element_types_decode_to_their_values(tmp_path):
    p = W.import_case(str(tmp_path / "x.onnx"), "dtypes_extra")
    inits = {ln.split()[1].split(":")[1]: ln for ln in V.onnx_describe(p).splitlines() if ln.startswith("init ")}
    for name, vals, dt, _ in W.DTYPES_EXTRA:
        want = np.asarray(vals).astype(W._NP[dt]).astype(np.float32).tobytes()
        assert f"bytes={len(want)} fnv={_fnv(want)}" in inits[name], (name, inits[name])


def test_malformed_files_are_rejected(tmp_path):
    good = open(W.import_case(str(tmp_path / "g.onnx"), "inputs_inits"), "rb").read()
    cases = {
        "truncated": good[:len(good) - 7],
        "no_graph": W.f_varint(1, 8),
        "bad_wire_type": W.key(7, 3) + b"\x00",
        "overlong_varint": W.key(1, 0) + b"\xff" * 11,
        "length_past_end": W.key(7, 2) + W.varint(1 << 20) + b"\x00" * 8,
    }
    w = np.zeros((6, 4, 1, 1), np.float32)
    bad_raw = W.f_packed_varints(1, [6, 4, 1, 1]) + W.f_varint(2, W.FLOAT) + W.f_bytes(8, "w") + W.f_bytes(9, w.tobytes()[:-4])
    cases["short_raw"] = W.model(W.graph([W.node("Conv", ["x", "w"], ["y"], name="c")], [W.value_info("x", [1, 4, 5, 5])],
                                         [W.value_info("y")], [bad_raw]))
    ext = W.tensor("w", w, store="external", external=("missing.bin", 0, w.nbytes))
    cases["missing_external"] = W.model(W.graph([W.node("Conv", ["x", "w"], ["y"], name="c")], [W.value_info("x", [1, 4, 5, 5])],
                                                [W.value_info("y")], [ext]))
    (tmp_path / "small.bin").write_bytes(b"\0" * 16)
    ext = W.tensor("w", w, store="external", external=("small.bin", 8, w.nbytes))
    cases["external_out_of_range"] = W.model(W.graph([W.node("Conv", ["x", "w"], ["y"], name="c")], [W.value_info("x", [1, 4, 5, 5])],
                                                     [W.value_info("y")], [ext]))
    # an offset near INT64_MAX: offset + length would wrap negative if the check added them
    ext = W.tensor("w", w, store="external", external=("small.bin", 9223372036854775807, w.nbytes))
    cases["external_offset_overflow"] = W.model(W.graph([W.node("Conv", ["x", "w"], ["y"], name="c")], [W.value_info("x", [1, 4, 5, 5])],
                                                        [W.value_info("y")], [ext]))
    # dims whose product wraps to 2 elements (3 x 6148914691236517206 = 2 mod 2^64), with 8 raw bytes
    huge = W.f_packed_varints(1, [3, 6148914691236517206]) + W.f_varint(2, W.FLOAT) + W.f_bytes(8, "w") + W.f_bytes(9, b"\0" * 8)
    cases["dims_overflow"] = W.model(W.graph([W.node("Conv", ["x", "w"], ["y"], name="c")], [W.value_info("x", [1, 4, 5, 5])],
                                             [W.value_info("y")], [huge]))
    for name, blob in cases.items():
        p = tmp_path / f"{name}.onnx"
        p.write_bytes(blob)
        with pytest.raises(V.VkhipError) as e:
            V.onnx_describe(p)
        msg = str(e.value)
        assert ("InvalidArgument" in msg or "IoError" in msg), (name, msg)
    with pytest.raises(V.VkhipError, match="IoError"):
        V.onnx_describe(tmp_path / "does_not_exist.onnx")


def _torch_edge(x):
    """The edge network restated in plain fp32 torch (tests/onnx_writer.py edge_model)."""
    import torch
    import torch.nn.functional as F
    r = np.random.default_rng(3)
    w1 = torch.tensor((r.standard_normal((12, 8, 3, 3)) * 0.2).astype(np.float16).astype(np.float32))
    b1 = torch.tensor((r.standard_normal(12) * 0.1).astype(np.float32))
    w2 = torch.tensor((r.standard_normal((4, 8, 1, 1)) * 0.3).astype(np.float32))
    wf = torch.tensor((r.standard_normal((10, 8)) * 0.3).astype(np.float32))
    bf = torch.tensor((r.standard_normal(10) * 0.1).astype(np.float32))
    x = torch.tensor(x)
    t = F.conv2d(x, w1, b1, padding=1).clamp(0.0, 6.0)
    a, b = t[:, :4], t[:, 4:]
    a2 = (0.2 * a + 0.5).clamp(0.0, 1.0)
    b3 = F.relu(F.conv2d(b, w2))
    c = torch.cat([a2, b3], 1)
    d = c.repeat_interleave(2, 2).repeat_interleave(2, 3)
    f = F.max_pool2d(d, 2, 2) + x
    s = torch.sigmoid(f.mean((2, 3), keepdim=True))
    h = (f * s).mean((2, 3))
    return (h @ wf.T + bf).numpy().ravel()


def test_edge_fixture_is_pinned(tmp_path):
    z = np.load(GOLDEN)
    blob = open(W.edge_model(str(tmp_path / "edge.onnx")), "rb").read()
    assert hashlib.sha256(blob).digest() == z["model_sha256"].tobytes(), "edge model bytes changed: rerun make_onnx_golden.py"
    assert list(z["x"].shape) == EDGE_IN and z["y"].size == sum(EDGE_OUT)
    np.testing.assert_allclose(z["y"], _torch_edge(z["x"]), rtol=1e-4, atol=1e-5)
    if O.ref_available():
        from tests.golden.make_onnx_golden import ref_onnx_run
        assert np.array_equal(ref_onnx_run(tmp_path / "edge.onnx", z["x"], z["y"].size), z["y"])


def test_corrupted_files_never_crash(tmp_path):
    """Seeded truncations, byte flips and spliced bytes of valid models either import or raise
    the library's error — the reader checks every length against its buffer, so nothing reads past
    the end or crashes the process."""
    rng = np.random.default_rng(123)
    blobs = [open(W.import_case(str(tmp_path / f"{c}.onnx"), c), "rb").read() for c in ("const_attrs", "dtypes", "ssa")]
    blobs.append(open(W.edge_model(str(tmp_path / "edge.onnx")), "rb").read())
    outcomes = {"ok": 0, "error": 0}
    p = tmp_path / "fuzz.onnx"
    for i in range(300):
        b = bytearray(blobs[i % len(blobs)])
        kind = i % 3
        if kind == 0:
            b = b[:int(rng.integers(0, len(b)))]
        elif kind == 1:
            for _ in range(int(rng.integers(1, 6))):
                b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
        else:
            at = int(rng.integers(0, len(b)))
            b[at:at] = bytes(rng.integers(0, 256, int(rng.integers(1, 12)), dtype=np.uint8))
        p.write_bytes(bytes(b))
        try:
            V.onnx_describe(p)
            outcomes["ok"] += 1
        except V.VkhipError as e:
            assert "InvalidArgument" in str(e) or "IoError" in str(e), str(e)
            outcomes["error"] += 1
    assert outcomes["error"] > 50, outcomes
