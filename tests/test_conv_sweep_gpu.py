"""Seeded sweep over conv geometries against the CPU oracle (through the vkhip C ABI).

Each case draws batch, channels, spatial size, kernel size, stride, asymmetric padding, dilation,
depthwise grouping, activation and residual from a fixed seed, then checks the plan the library
picks by itself and a sample of the explicit tile / split-K / Winograd plans that accept the shape
(every plan is validated by vkhip_conv_plan_make before it launches). Bar: max|d|/max|ref| <= 2e-2
and cosine >= 0.9999, as for every conv test."""
import ctypes

import numpy as np
import pytest

import vknn_amd as V
from tests.gpu_helpers import conv_desc, gpu_conv, round_half
from tests.oracle_lib import oracle_conv, parity

pytestmark = pytest.mark.gpu

REL_TOL, COS_TOL = 2e-2, 0.9999
NUM_CASES = 160


def draw_case(seed):
    r = np.random.default_rng(1000 + seed)
    dw = r.random() < 0.2
    K = int(r.choice([1, 3, 3, 5, 7]))
    S = int(r.choice([1, 1, 2]))
    D = int(r.choice([1, 1, 2])) if K == 3 else 1
    C = int(r.choice([3, 8, 16, 24, 32, 48, 64, 128, 256])) if not dw else int(r.integers(4, 140))
    Co = C if dw else int(r.integers(1, 300 if C <= 64 else 130))
    N = int(r.integers(1, 4))
    hi = 40 if r.random() < 0.3 else 20
    H, W = int(r.integers(max(1, D * (K - 1) - 1), hi)), int(r.integers(max(1, D * (K - 1) - 1), hi))
    pads = tuple(int(r.integers(0, K // 2 + 1)) for _ in range(4)) if K > 1 else (0, 0, 0, 0)
    act = int(r.integers(0, 6))
    res = bool(r.random() < 0.3)
    return dict(N=N, C=C, Co=Co, H=H, W=W, K=K, S=S, D=D, pads=pads, group=C if dw else 1, act=act, res=res)


def plans_for(case, d):
    """(algo, tile, ksplit) triples to run: auto, up to three accepting GEMM tiles, one split-K
    and Winograd when accepted."""
    lib = V.vkhip()
    r = np.random.default_rng(7 + case["C"] * 131 + case["H"])
    out = [(V.CONV_AUTO, -1, 0)]
    if case["group"] > 1:
        return out
    ok = []
    for t in range(lib.vkhip_conv_tile_count()):
        p = V.ConvPlan()
        if lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, t, 0, ctypes.byref(p)) == 0:
            ok.append(t)
    for t in r.permutation(ok)[:3]:
        out.append((V.CONV_GEMM, int(t), 0))
    for t in r.permutation(ok):
        p = V.ConvPlan()
        if lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_SPLITK, int(t), 2, ctypes.byref(p)) == 0:
            out.append((V.CONV_SPLITK, int(t), 2))
            break
    p = V.ConvPlan()
    if lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_WINOGRAD, -1, 0, ctypes.byref(p)) == 0:
        out.append((V.CONV_WINOGRAD, -1, 0))
    return out


@pytest.mark.parametrize("seed", range(NUM_CASES))
def test_conv_sweep(gpu, seed):
    c = draw_case(seed)
    if (c["H"] + c["pads"][0] + c["pads"][2] - c["D"] * (c["K"] - 1) - 1) < 0 or (c["W"] + c["pads"][1] + c["pads"][3] - c["D"] * (c["K"] - 1) - 1) < 0:
        pytest.skip("empty output")
    r = np.random.default_rng(seed)
    x = round_half(r.standard_normal((c["N"], c["C"], c["H"], c["W"])))
    w = (r.standard_normal((c["Co"], c["C"] // c["group"], c["K"], c["K"])) / np.sqrt(c["C"] // c["group"] * c["K"] ** 2)).astype(np.float32)
    b = (r.standard_normal(c["Co"]) * 0.1).astype(np.float32)
    d, yshape = conv_desc(x.shape, w.shape, (c["S"], c["S"]), c["pads"], (c["D"], c["D"]), c["group"], c["act"], 0.0, 6.0, int(c["res"]))
    res = round_half(r.standard_normal(yshape)) if c["res"] else None
    ref = oracle_conv(x, w, b, (c["S"], c["S"]), c["pads"], (c["D"], c["D"]), c["group"], res, c["act"], 0.0, 6.0)
    for algo, tile, ks in plans_for(c, d):
        print(f"case {seed}: {c} algo={algo} tile={tile} ks={ks}", flush=True)
        got, plan, _ = gpu_conv(x, w, b, (c["S"], c["S"]), c["pads"], (c["D"], c["D"]), c["group"], c["act"], 0.0, 6.0, res, algo, tile, ks)
        rel, cos = parity(got, ref)
        assert rel <= REL_TOL and cos >= COS_TOL, (seed, c, algo, tile, ks, rel, cos)
