"""Writes tests/golden/onnx_edge.npz and onnx_mixed.npz: the ONNX edge-case network and the
HIP/host alternating network of tests/onnx_writer.py (edge_model, mixed_model) run by the REFERENCE — its own importer (src/import/onnx/onnx_parser.cpp) and its CPU
Session (src/core/session.cpp) — on a seeded input. The GPU test imports the same model bytes with
this build's importer, runs them on the HIP backend and compares with these outputs, so the
import path is checked end to end where the reference is absent.

Run in the build container only (it needs oracle/_ref/libvknn_ref.so):
    python tests/golden/make_onnx_golden.py
"""
import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests import oracle_lib as O  # noqa: E402
from tests import onnx_writer as W  # noqa: E402

EDGE_IN, EDGE_OUT = [1, 8, 12, 12], [10]
MIXED_IN, MIXED_OUT = [2, 8, 10, 10], [16]


def mixed_input():
    return np.random.default_rng(22).standard_normal(MIXED_IN).astype(np.float32)


def edge_input():
    return np.random.default_rng(21).standard_normal(EDGE_IN).astype(np.float32)


def ref_onnx_run(path, x, n_out):
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.zeros(n_out, np.float32)
    rc = O.ref().ref_onnx_run(str(path).encode(), x.ctypes.data, x.size, y.ctypes.data, y.size)
    assert rc == 0, O.ref().ref_last_error()
    return y


def main():
    with tempfile.TemporaryDirectory() as d:
        p = W.edge_model(os.path.join(d, "edge.onnx"))
        blob = open(p, "rb").read()
        x = edge_input()
        y = ref_onnx_run(p, x, sum(EDGE_OUT))
    np.savez_compressed(os.path.join(HERE, "onnx_edge.npz"), x=x, y=y,
                        model_sha256=np.frombuffer(hashlib.sha256(blob).digest(), np.uint8))
    print("onnx_edge.npz: y", y[:4], "...")
    with tempfile.TemporaryDirectory() as d:
        p = W.mixed_model(os.path.join(d, "mixed.onnx"))
        blob = open(p, "rb").read()
        x = mixed_input()
        y = ref_onnx_run(p, x, sum(MIXED_OUT))
    np.savez_compressed(os.path.join(HERE, "onnx_mixed.npz"), x=x, y=y,
                        model_sha256=np.frombuffer(hashlib.sha256(blob).digest(), np.uint8))
    print("onnx_mixed.npz: y", y[:4], "...")


if __name__ == "__main__":
    main()
