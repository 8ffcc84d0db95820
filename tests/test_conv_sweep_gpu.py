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


def draw_dwpw(seed):
    r = np.random.default_rng(5000 + seed)
    k = int(r.choice([3, 5]))
    s = int(r.choice([1, 2]))
    return dict(N=int(r.integers(1, 4)), E=int(r.integers(4, 200)), H=int(r.integers(2, 30)), W=int(r.integers(2, 30)), k=k, s=s,
                pads=tuple(int(r.integers(0, k // 2 + 1)) for _ in range(4)), Cout=int(r.integers(1, 120)),
                dw_act=int(r.choice([0, 1, 2])), act=int(r.integers(0, 6)), res=bool(r.random() < 0.4))


@pytest.mark.parametrize("kernel", ["ring", "strip"])
@pytest.mark.parametrize("seed", range(40))
def test_fused_dwpw_sweep(gpu, monkeypatch, kernel, seed):
    """The fused dw+pw kernel over seeded geometries (ragged channel counts, odd sizes,
    asymmetric pads, stride 2, every activation pair, residual) against the oracle."""
    from tests.gpu_helpers import DeviceBuffer, check, from_device_nc4, to_device_nc4
    from tests.oracle_lib import oracle_dwpw
    monkeypatch.setenv("VKHIP_DWPW_RING", "1" if kernel == "ring" else "0")
    lib = V.vkhip()
    c = draw_dwpw(seed)
    N, E, H, W, k, s, pads, Cout = c["N"], c["E"], c["H"], c["W"], c["k"], c["s"], c["pads"], c["Cout"]
    OH, OW = (H + pads[0] + pads[2] - k) // s + 1, (W + pads[1] + pads[3] - k) // s + 1
    if OH < 1 or OW < 1:
        pytest.skip("empty output")
    r = np.random.default_rng(seed)
    x = round_half(r.standard_normal((N, E, H, W)))
    dw_w = (r.standard_normal((E, 1, k, k)) * 0.3).astype(np.float32)
    dw_b = (r.standard_normal(E) * 0.1).astype(np.float32)
    pw_w = (r.standard_normal((Cout, E)) * np.sqrt(1.0 / E)).astype(np.float32)
    pw_b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    resid = round_half(r.standard_normal((N, Cout, OH, OW))) if c["res"] else None
    lo, hi = (-0.3, 0.4) if c["act"] == 3 else (0.0, 6.0)
    dwd, _ = conv_desc(x.shape, (E, 1, k, k), (s, s), pads, group=E, act=c["dw_act"], lo=0.0, hi=6.0)
    d = V.DwPwDesc(dw=dwd, Cout=Cout, act=c["act"], act_lo=lo, act_hi=hi, has_res=int(c["res"]))
    print(f"dwpw case {seed}: {c}", flush=True)
    if lib.vkhip_dwpw_supported(ctypes.byref(d)) != 1:
        pytest.skip("shape outside the fused kernel")
    blob = np.zeros(lib.vkhip_dwpw_weight_bytes(ctypes.byref(d)), np.uint8)
    check(lib.vkhip_dwpw_pack_weights(ctypes.byref(d), dw_w.ctypes.data, dw_b.ctypes.data, pw_w.ctypes.data, pw_b.ctypes.data,
                                      blob.ctypes.data))
    dblob = DeviceBuffer.from_array(blob)
    dx = to_device_nc4(x)
    dres = to_device_nc4(resid) if resid is not None else None
    dy = DeviceBuffer(V.nc4_elems(N, Cout, OH, OW) * 2)
    check(lib.vkhip_dwpw_forward(ctypes.byref(d), dx.ptr, dblob.ptr, dres.ptr if dres else None, dy.ptr, None))
    check(lib.vkhip_stream_sync(None))
    got = from_device_nc4(dy, (N, Cout, OH, OW))
    ref = oracle_dwpw(x, dw_w, dw_b, pw_w, pw_b, (s, s), pads, dw_act=c["dw_act"], res=resid, act=c["act"], lo=lo, hi=hi)
    rel, cos = parity(got, ref)
    assert rel <= REL_TOL and cos >= COS_TOL, (seed, c, rel, cos)


@pytest.mark.parametrize("seed", range(40))
def test_pool_fc_sweep(gpu, seed):
    """Max pool (the generic and the 3x3/s2 pixel-pair kernels), global average pool (lane counts
    8..64 by plane size) and the skinny-GEMM FC over seeded shapes against the oracle: pools
    bit-exact (a max of fp16 values is exact; the mean within the conv tolerance), FC within it."""
    from tests.gpu_helpers import DeviceBuffer, check, from_device_nc4, to_device_nc4
    from tests.oracle_lib import oracle
    lib, o = V.vkhip(), oracle()
    r = np.random.default_rng(9000 + seed)
    N, C = int(r.integers(1, 5)), int(r.integers(1, 80))
    H, W = int(r.integers(1, 40)), int(r.integers(1, 40))
    if seed % 2 == 0:  # the stem-pool shape family: 3x3 s2, pad 1 left/top, even W
        k, s, pt, pl = 3, 2, 1, 1
        W += W % 2
    else:
        k, s = int(r.choice([1, 2, 3, 5])), int(r.choice([1, 2, 3]))
        pt, pl = int(r.integers(0, k // 2 + 1)), int(r.integers(0, k // 2 + 1))
    pb, pr = int(r.integers(0, k // 2 + 1)), int(r.integers(0, k // 2 + 1))
    OH, OW = (H + pt + pb - k) // s + 1, (W + pl + pr - k) // s + 1
    x = round_half(r.standard_normal((N, C, H, W)) * 2)
    dx = to_device_nc4(x)
    print(f"pool/fc case {seed}: N={N} C={C} H={H} W={W} k={k} s={s} pads={pt, pl, pb, pr}", flush=True)
    if OH >= 1 and OW >= 1 and pt < k and pl < k:
        d = V.PoolDesc(N=N, C=C, H=H, W=W, OH=OH, OW=OW, KH=k, KW=k, SH=s, SW=s, PT=pt, PL=pl)
        dy = DeviceBuffer(V.nc4_elems(N, C, OH, OW) * 2)
        check(lib.vkhip_maxpool(ctypes.byref(d), dx.ptr, dy.ptr, None))
        ref = np.zeros((N, C, OH, OW), np.float32)
        o.oracle_maxpool(x.ctypes.data, ref.ctypes.data, N, C, H, W, k, k, s, s, pt, pl, OH, OW)
        assert np.array_equal(from_device_nc4(dy, (N, C, OH, OW)), ref), ("maxpool", seed)
    davg = DeviceBuffer(V.nc4_elems(N, C, 1, 1) * 2)
    check(lib.vkhip_global_avg_pool(dx.ptr, davg.ptr, N, C, H, W, None))
    avg_ref = np.zeros((N, C), np.float32)
    o.oracle_global_avg_pool(x.ctypes.data, avg_ref.ctypes.data, N, C, H * W)
    avg = from_device_nc4(davg, (N, C, 1, 1)).reshape(N, C)
    rel, cos = parity(avg, avg_ref)
    assert rel <= REL_TOL and cos >= COS_TOL, ("gap", seed, rel, cos)
    M, act = int(r.integers(1, 300)), int(r.integers(0, 3))
    w = (r.standard_normal((M, C)) / np.sqrt(C)).astype(np.float32)
    b = (r.standard_normal(M) * 0.1).astype(np.float32)
    blob = np.zeros(lib.vkhip_fc_weight_bytes(C, M), np.uint8)
    check(lib.vkhip_fc_pack_weights(C, M, w.ctypes.data, 1, b.ctypes.data, 1.0, 1.0, blob.ctypes.data))
    dblob = DeviceBuffer.from_array(blob)
    a16 = round_half(avg)
    dfc = DeviceBuffer(V.nc4_elems(N, M, 1, 1) * 2)
    check(lib.vkhip_fc(davg.ptr, dblob.ptr, dfc.ptr, N, C, M, act, 0.0, 6.0, None))
    check(lib.vkhip_stream_sync(None))
    fc_ref = np.zeros((N, M), np.float32)
    o.oracle_gemm(a16.ctypes.data, w.ctypes.data, b.ctypes.data, fc_ref.ctypes.data, N, C, M, 1, 1.0, 1.0, act, 0.0, 6.0)
    rel, cos = parity(from_device_nc4(dfc, (N, M, 1, 1)).reshape(N, M), fc_ref)
    assert rel <= REL_TOL and cos >= COS_TOL, ("fc", seed, rel, cos)
