"""CPU tests that pin the oracle (oracle/oracle.c) before it is trusted as the parity checker.

Each oracle function is checked three ways:
  * against the golden fixtures under tests/golden/ (outputs of the reference's own CPU backend,
    src/backend/cpu/*, compiled from source; see tests/golden/make_golden.py) — bit-exact;
  * against oracle/_ref (the same reference build) on fresh inputs, where that library is built;
  * against closed forms and independent textbook routines (numpy float16, torch conv2d in float64,
    brute force on tiny inputs), chosen so a dropped term, a transposed operand or a wrong index fails.
"""
import ctypes
import os

import numpy as np
import pytest

from tests import oracle_lib as O
from tests.golden import make_golden as G

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with np.load(os.path.join(GOLD, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


OPS = _load("ops.npz")
lib = O.oracle()
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference sources absent)")


def f2h(x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    h = np.zeros(x.size, np.uint16)
    lib.oracle_float_to_half_n(x.ctypes.data, h.ctypes.data, x.size)
    return h


def h2f(h):
    h = np.ascontiguousarray(h, np.uint16).ravel()
    f = np.zeros(h.size, np.float32)
    lib.oracle_half_to_float_n(h.ctypes.data, f.ctypes.data, h.size)
    return f


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


# ---------------------------------------------------------------- codec (include/vknn/dtype.h:60-157)
def test_codec_matches_golden():
    g = _load("codec.npz")
    assert np.array_equal(f2h(g["f32_bits"].view(np.float32)), g["f16"])
    assert np.array_equal(h2f(np.arange(65536, dtype=np.uint16)).view(np.uint32), g["all_h2f_bits"])


def test_half_to_float_is_exact():
    """halfToFloat is exact: equals IEEE widening for every non-NaN half (numpy float16)."""
    h = np.arange(65536, dtype=np.uint16)
    got = h2f(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert bits_equal(got[~nan], want[~nan])
    assert np.isnan(got[nan]).all()


def test_float_to_half_closed_form():
    """floatToHalf rounds half AWAY from zero on the 13 dropped bits; IEEE RNE (numpy) rounds ties
    to even. So the two agree everywhere except exact ties whose kept LSB is even, where the
    reference result is one ulp larger in magnitude. Checked over every fp32 exponent in and near
    the fp16 range and every value of the dropped bits that matters."""
    hi = np.arange(1 << 19, dtype=np.uint32) << 13
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF], np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    f = bits.view(np.float32)
    got = f2h(f)
    with np.errstate(over="ignore"):
        rne = f.astype(np.float16).view(np.uint16)
    exp = (bits >> 23) & 0xFF
    normal = (exp >= 113) & (exp <= 142)          # fp16 normal range, below the overflow edge
    tie = (bits & 0x1FFF) == 0x1000
    even = ((bits >> 13) & 1) == 0
    expect_diff = normal & tie & even
    same = normal & ~expect_diff
    assert np.array_equal(got[same], rne[same])
    assert np.array_equal(got[expect_diff], rne[expect_diff] + 1)
    # NaN -> sign | 0x7E00, inf stays inf, beyond 65520 -> inf, tiny -> signed zero
    sp = np.array([np.nan, -np.nan, np.inf, -np.inf, 70000.0, -1e30, 1e-12, -1e-12], np.float32)
    assert list(f2h(sp)) == [0x7E00, 0xFE00, 0x7C00, 0xFC00, 0x7C00, 0xFC00, 0x0000, 0x8000]


def test_reference_half_roundtrip():
    """tests/test_core.cpp:15-23 (DType.HalfRoundTrip)."""
    for v in (0.0, 1.0, -1.0, 0.5, 6.0, 3.14159, -2.71828, 65504.0):
        r = h2f(f2h(np.float32(v)))[0]
        assert abs(r - v) <= abs(v) * 0.01 + 1e-3


@needs_ref
def test_codec_vs_ref_exhaustive_boundaries():
    hi = np.arange(1 << 19, dtype=np.uint32) << 13
    bits = (hi[:, None] | np.array([0, 0x0FFF, 0x1000, 0x1001, 0x1FFF, 0x0800], np.uint32)[None, :]).ravel()
    f = bits.view(np.float32)
    want = np.zeros(f.size, np.uint16)
    O.ref().ref_float_to_half_n(f.ctypes.data, want.ctypes.data, f.size)
    assert np.array_equal(f2h(f), want)


# ---------------------------------------------------------------- pack / unpack (vk_backend.cpp:558-696)
@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (1, 3, 5, 7), (2, 5, 3, 3), (2, 6, 4, 9), (1, 7, 2, 2), (1, 8, 3, 3)])
def test_pack_index_map_brute_force(shape):
    """NC4HW4 element (n,c,h,w) at (((n*Cb + c/4)*H + h)*W + w)*4 + c%4 (include/vknn/nchw.h:50-58),
    lanes c >= C are +0; values go through the codec."""
    x = np.random.default_rng(3).standard_normal(shape).astype(np.float32)
    N, C, H, W = shape
    Cb = (C + 3) // 4
    got = O.oracle_pack(x)
    want = np.zeros(N * Cb * H * W * 4, np.uint16)
    codes = f2h(x).reshape(shape)
    for n in range(N):
        for c in range(C):
            for h in range(H):
                for w in range(W):
                    want[(((n * Cb + c // 4) * H + h) * W + w) * 4 + c % 4] = codes[n, c, h, w]
    assert np.array_equal(got, want)
    back = O.oracle_unpack(got, shape)
    assert bits_equal(back, h2f(codes.ravel()).reshape(shape))


# ---------------------------------------------------------------- conv (src/backend/cpu/ops/conv.cpp:9-92)
def _conv_case(case):
    d = {k.split("/")[-1]: v for k, v in OPS.items() if k.startswith(f"conv/{case[0]}/")}
    _, N, C, H, W, Cout, KH, KW, st, pd, dl, g, act, lo, hi, hb, hr = case
    y = O.oracle_conv(d["x"], d["w"], d.get("b"), st, pd, dl, g, d.get("res"), act, lo, hi)
    return d, y


@pytest.mark.parametrize("case", G.CONV_CASES, ids=[c[0] for c in G.CONV_CASES])
def test_conv_matches_golden(case):
    d, y = _conv_case(case)
    assert y.shape == d["y"].shape
    assert bits_equal(y, d["y"]), np.abs(y - d["y"]).max()


def test_reference_conv1x1_relu_values():
    """tests/test_ops.cpp:204-273 (Conv1x1Relu: {0, 10}) and tests/test_core.cpp:83-140 ({-1, 10})."""
    x = np.array([1, 5], np.float32).reshape(1, 2, 1, 1)
    w = np.array([2, 0, 0, 2], np.float32).reshape(2, 2, 1, 1)
    b = np.array([-3, 0], np.float32)
    assert O.oracle_conv(x, w, b, act=1).ravel().tolist() == [0.0, 10.0]
    assert O.oracle_conv(x, w, b).ravel().tolist() == [-1.0, 10.0]
    assert OPS["conv/ref_conv1x1_relu/y"].ravel().tolist() == [0.0, 10.0]


def _act_np(y, act, lo, hi):
    if act == 1:
        return np.maximum(y, 0)
    if act == 2:
        return np.clip(y, 0, 6)
    if act == 3:
        return np.clip(y, lo, hi)
    if act == 4:
        return y * np.clip(y + 3, 0, 6) / 6
    if act == 5:
        return y / (1 + np.exp(-y))
    return y


@pytest.mark.parametrize("case", G.CONV_CASES, ids=[c[0] for c in G.CONV_CASES])
def test_conv_vs_torch_float64(case):
    """Independent textbook cross-check: torch conv2d in float64 (explicit asymmetric padding)."""
    torch = pytest.importorskip("torch")
    import torch.nn.functional as F
    d, y = _conv_case(case)
    _, N, C, H, W, Cout, KH, KW, st, pd, dl, g, act, lo, hi, hb, hr = case
    x = torch.from_numpy(d["x"].astype(np.float64))
    x = F.pad(x, (pd[1], pd[3], pd[0], pd[2]))
    b = torch.from_numpy(d["b"].astype(np.float64)) if "b" in d else None
    ref = F.conv2d(x, torch.from_numpy(d["w"].astype(np.float64)), b, stride=st, dilation=dl, groups=g).numpy()
    if "res" in d:
        ref = ref + d["res"]
    ref = _act_np(ref, act, lo, hi)
    assert ref.shape == y.shape
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_conv_brute_force_tiny():
    """Direct six-loop definition on a tiny input with stride, asymmetric pad, dilation and groups."""
    r = np.random.default_rng(9)
    N, C, H, W, Cout, KH, KW, g = 1, 4, 5, 6, 6, 2, 3, 2
    st, pd, dl = (2, 1), (1, 0, 0, 2), (1, 2)
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    w = r.standard_normal((Cout, C // g, KH, KW)).astype(np.float32)
    b = r.standard_normal(Cout).astype(np.float32)
    y = O.oracle_conv(x, w, b, st, pd, dl, g)
    OH = (H + pd[0] + pd[2] - (dl[0] * (KH - 1) + 1)) // st[0] + 1
    OW = (W + pd[1] + pd[3] - (dl[1] * (KW - 1) + 1)) // st[1] + 1
    ref = np.zeros((N, Cout, OH, OW))
    cg, og = C // g, Cout // g
    for oc in range(Cout):
        gi = oc // og
        for oy in range(OH):
            for ox in range(OW):
                s = float(b[oc])
                for ic in range(cg):
                    for ky in range(KH):
                        for kx in range(KW):
                            iy, ix = oy * st[0] - pd[0] + ky * dl[0], ox * st[1] - pd[1] + kx * dl[1]
                            if 0 <= iy < H and 0 <= ix < W:
                                s += float(x[0, gi * cg + ic, iy, ix]) * float(w[oc, ic, ky, kx])
                ref[0, oc, oy, ox] = s
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


@needs_ref
def test_conv_vs_ref_random_shapes():
    """Fresh random shapes through the reference CPU Session: bit-exact."""
    r = np.random.default_rng(21)
    for t in range(6):
        C, Cout, H, W = (int(v) for v in r.integers(1, 10, 4))
        K = int(r.choice([1, 3, 5]))
        s = int(r.choice([1, 2]))
        p = K // 2
        act = int(r.integers(0, 6))
        case = (f"rand{t}", 1, C, H + 4, W + 4, Cout, K, K, (s, s), (p, p, p, p), (1, 1), 1, act, -0.5, 0.5, True, False)
        x, w, b, _ = G.conv_inputs(case, 900 + t)
        want, ys = O.ref_single_node("Conv", [x, w, b], G.conv_attrs(case), fused_act=act, lo=-0.5, hi=0.5)
        got = O.oracle_conv(x, w, b, (s, s), (p, p, p, p), (1, 1), 1, None, act, -0.5, 0.5)
        assert got.shape == ys
        assert bits_equal(got.ravel(), want[:got.size])


# ---------------------------------------------------------------- fused dw+pw (fused_dwpw.cpp:10-87)
@pytest.mark.parametrize("case", G.DWPW_CASES, ids=[c[0] for c in G.DWPW_CASES])
def test_dwpw_matches_golden_and_composition(case):
    _, N, E, H, W, Cout, K, s, p, dwa, act, lo, hi, hr = case
    d = {k.split("/")[-1]: v for k, v in OPS.items() if k.startswith(f"dwpw/{case[0]}/")}
    y = O.oracle_dwpw(d["x"], d["dw_w"], d["dw_b"], d["pw_w"], d["pw_b"], (s, s), (p, p, p, p), (1, 1), dwa,
                      d.get("res"), act, lo, hi)
    assert bits_equal(y, d["y"])
    # composition identity: dw conv (+dw act, Clip bounds fixed 0/6) then 1x1 conv (+res, act)
    t = O.oracle_conv(d["x"], d["dw_w"], d["dw_b"], (s, s), (p, p, p, p), (1, 1), E, None, dwa, 0.0, 6.0)
    y2 = O.oracle_conv(t, d["pw_w"], d["pw_b"], res=d.get("res"), act=act, lo=lo, hi=hi)
    np.testing.assert_allclose(y, y2, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- fused SE (fused_se.cpp:9-47)
@pytest.mark.parametrize("case", G.SE_CASES, ids=[c[0] for c in G.SE_CASES])
def test_se_matches_golden_and_closed_form(case):
    _, N, C, Cr, a, b = case
    d = {k.split("/")[-1]: v for k, v in OPS.items() if k.startswith(f"se/{case[0]}/")}
    y = np.zeros((N, C), np.float32)
    lib.oracle_fused_se(d["avg"].ctypes.data, N, C, d["w1"].ctypes.data, Cr, d["b1"].ctypes.data, d["w2"].ctypes.data,
                        d["b2"].ctypes.data, a, b, y.ctypes.data)
    assert bits_equal(y.ravel(), d["y"].ravel())
    avg = d["avg"].reshape(N, C).astype(np.float64)
    h = np.maximum(avg @ d["w1"].reshape(Cr, C).T.astype(np.float64) + d["b1"], 0).astype(np.float32)
    z = h.astype(np.float64) @ d["w2"].reshape(C, Cr).T.astype(np.float64) + d["b2"]
    np.testing.assert_allclose(y, np.clip(a * z + b, 0, 1), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- element-wise / pooling / FC
def _call(fn, *args):
    fn(*args)


def test_add_mul_unary_gap_maxpool_gemm_match_golden():
    a, b = OPS["add/none/a"], OPS["add/none/b"]
    for nm, act, lo, hi in (("none", 0, 0, 0), ("relu", 1, 0, 0), ("clip", 3, -0.3, 0.4)):
        y = np.zeros_like(a)
        lib.oracle_add(a.ctypes.data, b.ctypes.data, y.ctypes.data, a.size, act, lo, hi)
        assert bits_equal(y, OPS[f"add/{nm}/y"])
        np.testing.assert_array_equal(y, _act_np(a + b, act, lo, hi))
    s = OPS["mul_channel/bcast/s"]
    y = np.zeros_like(a)
    lib.oracle_mul_channel(a.ctypes.data, s.ctypes.data, y.ctypes.data, 2, 6, 25)
    assert bits_equal(y, OPS["mul_channel/bcast/y"])
    np.testing.assert_array_equal(y, a * s)
    xu = OPS["unary/sigmoid/x"]
    for nm, code, p0, p1 in (("sigmoid", 0, 0, 0), ("hardswish", 2, 0, 0), ("hardsigmoid", 3, 1 / 6, 0.5),
                             ("silu", 14, 0, 0)):
        y = np.zeros_like(xu)
        lib.oracle_unary(xu.ctypes.data, y.ctypes.data, xu.size, code, p0, p1)
        assert bits_equal(y, OPS[f"unary/{nm}/y"]), nm
    x64 = xu.astype(np.float64)
    closed = {"sigmoid": 1 / (1 + np.exp(-x64)), "hardswish": x64 * np.clip(x64 + 3, 0, 6) / 6,
              "hardsigmoid": np.clip(x64 / 6 + 0.5, 0, 1), "silu": x64 / (1 + np.exp(-x64))}
    for nm, v in closed.items():
        np.testing.assert_allclose(OPS[f"unary/{nm}/y"], v, rtol=1e-5, atol=1e-6)
    y = np.zeros((1, 5), np.float32)
    lib.oracle_global_avg_pool(xu.ctypes.data, y.ctypes.data, 1, 5, 42)
    assert bits_equal(y.ravel(), OPS["gap/basic/y"].ravel())
    np.testing.assert_allclose(y.ravel(), xu.reshape(5, -1).mean(1), rtol=1e-6)
    y = np.zeros((1, 5, 3, 4), np.float32)
    lib.oracle_maxpool(xu.ctypes.data, y.ctypes.data, 1, 5, 6, 7, 3, 3, 2, 2, 1, 1, 3, 4)
    assert bits_equal(y, OPS["maxpool/k3s2p1/y"])
    pad = np.pad(xu, ((0, 0), (0, 0), (1, 1), (1, 1)), constant_values=-np.inf)
    mp = np.array([[[[pad[0, c, 2 * i:2 * i + 3, 2 * j:2 * j + 3].max() for j in range(4)] for i in range(3)]
                    for c in range(5)]])
    np.testing.assert_array_equal(y, mp)
    ga, gb, gc = OPS["gemm/transB/a"], OPS["gemm/transB/b"], OPS["gemm/transB/c"]
    y = np.zeros((3, 7), np.float32)
    lib.oracle_gemm(ga.ctypes.data, gb.ctypes.data, gc.ctypes.data, y.ctypes.data, 3, 20, 7, 1, 1.0, 1.0, 0, 0.0, 0.0)
    assert bits_equal(y, OPS["gemm/transB/y"])
    np.testing.assert_allclose(y, ga.astype(np.float64) @ gb.T + gc, rtol=1e-5, atol=1e-5)


def test_bn_fold_closed_form():
    """fold_batchnorm.cpp:57-78: w*a, (b-mean)*a+beta with a = gamma/sqrt(var+eps); folding then
    convolving equals convolving then applying BN (float64 check)."""
    r = np.random.default_rng(5)
    Cout, Cin = 6, 4
    w = r.standard_normal((Cout, Cin, 3, 3)).astype(np.float32)
    b = r.standard_normal(Cout).astype(np.float32)
    g, be, m = (r.uniform(0.5, 1.5, Cout).astype(np.float32), r.normal(0, 0.1, Cout).astype(np.float32),
                r.normal(0, 0.1, Cout).astype(np.float32))
    v = r.uniform(0.5, 1.5, Cout).astype(np.float32)
    wf, bf = w.copy(), b.copy()
    lib.oracle_fold_bn(wf.ctypes.data, bf.ctypes.data, Cout, Cin * 9, g.ctypes.data, be.ctypes.data, m.ctypes.data,
                       v.ctypes.data, 1e-5)
    a = g / np.sqrt(v + np.float32(1e-5))
    np.testing.assert_allclose(wf, w * a[:, None, None, None], rtol=1e-6)
    np.testing.assert_allclose(bf, (b - m) * a + be, rtol=1e-6, atol=1e-7)
    x = r.standard_normal((1, Cin, 5, 5)).astype(np.float32)
    y1 = O.oracle_conv(x, wf, bf, pads=(1, 1, 1, 1))
    y0 = O.oracle_conv(x, w, b, pads=(1, 1, 1, 1)).astype(np.float64)
    y0 = (y0 - m[None, :, None, None]) * a[None, :, None, None] + be[None, :, None, None]
    np.testing.assert_allclose(y1, y0, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- whole graphs (passes + CPU backend)
MODELS = _load("models.npz")


@pytest.mark.parametrize("name,batch", G.MODELS, ids=[f"{m}_b{b}" for m, b in G.MODELS])
def test_model_graph_matches_golden(name, batch):
    """The oracle graph runner (the same zoo graph, this build's passes, the restated CPU ops)
    equals the reference Session's output bit for bit."""
    x = MODELS[f"{name}/b{batch}/x"]
    y = O.oracle_model_run(name, batch, G.MODEL_SEED, x)
    want = MODELS[f"{name}/b{batch}/y"]
    assert y.shape == want.shape
    assert bits_equal(y, want), np.abs(y - want).max()


@needs_ref
def test_config0_vs_ref():
    """Config 0 (3x3 64->64 @56 + folded BN + ReLU) at full size against the reference Session."""
    in_shape, _ = O.model_io("conv3x3_bn_relu", 1)
    x = np.random.default_rng(0).uniform(-1, 1, in_shape).astype(np.float32)
    assert bits_equal(O.oracle_model_run("conv3x3_bn_relu", 1, 7, x), O.ref_model_run("conv3x3_bn_relu", 1, 7, x))


@needs_ref
@pytest.mark.parametrize("name", ["mnv2_block", "resnet50", "mobilenetv3_large", "yolov8n"])
def test_full_config_vs_ref(name):
    """Configs 1-4 at N=1 and full size: the oracle graph runner equals the reference Session (the
    reference CPU backend compiled from its sources) bit for bit on the same seeded graph."""
    in_shape, _ = O.model_io(name, 1)
    x = np.random.default_rng(1).standard_normal(in_shape).astype(np.float32)
    assert bits_equal(O.oracle_model_run(name, 1, 7, x), O.ref_model_run(name, 1, 7, x))
