"""Writes the golden fixtures of the fused fp16 conv path from the REFERENCE's own CPU backend.

Run in the build container only (it needs oracle/_ref/libvknn_ref.so, which oracle/Makefile compiles
from the reference sources under /root/reference):  python tests/golden/make_golden.py

Every fixture is data: seeded inputs and the outputs the reference CPU Session
(src/core/session.cpp:649-814 -> src/backend/cpu/cpu_backend.cpp:84-149) computed for them. The
tests replay the inputs through the oracle restatement (oracle/oracle.c) and require bit-exact
equality, so the oracle is pinned to the reference without the reference being present.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests import oracle_lib as O  # noqa: E402

# ---------------------------------------------------------------- cases (shared with the tests)
# (name, N, C, H, W, Cout, KH, KW, strides, pads[t,l,b,r], dil, group, act, lo, hi, bias, residual)
CONV_CASES = [
    ("ref_conv1x1_relu", 1, 2, 1, 1, 2, 1, 1, (1, 1), (0, 0, 0, 0), (1, 1), 1, 1, 0.0, 0.0, True, False),
    ("c3x3_s1_relu_c5", 1, 5, 7, 6, 6, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 1, 1, 0.0, 0.0, True, False),
    ("c3x3_s2_relu6_n2", 2, 6, 9, 8, 7, 3, 3, (2, 2), (1, 1, 1, 1), (1, 1), 1, 2, 0.0, 6.0, True, False),
    ("c7x7_s2_stem", 1, 3, 11, 11, 8, 7, 7, (2, 2), (3, 3, 3, 3), (1, 1), 1, 0, 0.0, 0.0, True, False),
    ("c1x1_res_relu", 1, 7, 5, 5, 9, 1, 1, (1, 1), (0, 0, 0, 0), (1, 1), 1, 1, 0.0, 0.0, True, True),
    ("c1x1_res_none_c24", 2, 24, 4, 3, 24, 1, 1, (1, 1), (0, 0, 0, 0), (1, 1), 1, 0, 0.0, 0.0, True, True),
    ("c1x1_s2_hswish", 1, 8, 6, 6, 4, 1, 1, (2, 2), (0, 0, 0, 0), (1, 1), 1, 4, 0.0, 0.0, True, False),
    ("dw3x3_silu", 1, 12, 7, 7, 12, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 12, 5, 0.0, 0.0, True, False),
    ("dw5x5_s2_clip", 1, 10, 9, 9, 10, 5, 5, (2, 2), (2, 2, 2, 2), (1, 1), 10, 3, -0.5, 0.7, True, False),
    ("c3x3_dil2", 1, 4, 6, 6, 5, 3, 3, (1, 1), (2, 2, 2, 2), (2, 2), 1, 1, 0.0, 0.0, True, False),
    ("c3x3_nobias_asympad", 1, 3, 5, 8, 4, 3, 3, (1, 2), (0, 1, 1, 0), (1, 1), 1, 0, 0.0, 0.0, False, False),
    ("c3x3_s1_c32", 1, 32, 6, 6, 32, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 1, 1, 0.0, 0.0, True, False),
]

# (name, N, E, H, W, Cout, K, stride, pad, dw_act, act, lo, hi, residual)
DWPW_CASES = [
    ("dwpw_relu6_res", 1, 16, 6, 6, 8, 3, 1, 1, 2, 0, 0.0, 0.0, True),
    ("dwpw_5x5_s2_relu", 2, 12, 9, 7, 6, 5, 2, 2, 1, 1, 0.0, 0.0, False),
    ("dwpw_none_hswish", 1, 9, 5, 5, 5, 3, 1, 1, 0, 4, 0.0, 0.0, False),
]

# (name, N, C, Cr, alpha, beta)
SE_CASES = [("se_c16_r8", 2, 16, 8, 1.0 / 6.0, 0.5), ("se_c40_r16", 1, 40, 16, 0.2, 0.5)]

MODELS = [("conv_tiny", 1), ("conv_tiny", 2), ("mnv2_tiny", 1), ("resnet_tiny", 1), ("mnv3_tiny", 1), ("yolo_tiny", 1)]
MODEL_SEED = 7


def conv_inputs(case, seed):
    _, N, C, H, W, Cout, KH, KW, st, pd, dl, g, act, lo, hi, has_b, has_r = case
    r = np.random.default_rng(seed)
    if case[0] == "ref_conv1x1_relu":  # tests/test_ops.cpp:204-273: w = 2*I, b = {-3, 0}, x = {1, 5}
        x = np.array([1, 5], np.float32).reshape(1, 2, 1, 1)
        w = np.array([2, 0, 0, 2], np.float32).reshape(2, 2, 1, 1)
        return x, w, np.array([-3, 0], np.float32), None
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    w = (r.standard_normal((Cout, C // g, KH, KW)) * np.sqrt(2.0 / (C // g * KH * KW))).astype(np.float32)
    b = r.standard_normal(Cout).astype(np.float32) * 0.1 if has_b else None
    OH = (H + pd[0] + pd[2] - (dl[0] * (KH - 1) + 1)) // st[0] + 1
    OW = (W + pd[1] + pd[3] - (dl[1] * (KW - 1) + 1)) // st[1] + 1
    res = r.standard_normal((N, Cout, OH, OW)).astype(np.float32) if has_r else None
    return x, w, b, res


def conv_attrs(case):
    _, N, C, H, W, Cout, KH, KW, st, pd, dl, g = case[:12]
    return (f"l:strides={st[0]},{st[1]};l:pads={','.join(map(str, pd))};l:dilations={dl[0]},{dl[1]};"
            f"i:group={g};l:kernel_shape={KH},{KW}")


def dwpw_inputs(case, seed):
    _, N, E, H, W, Cout, K, s, p, dwa, act, lo, hi, has_r = case
    r = np.random.default_rng(seed)
    x = r.standard_normal((N, E, H, W)).astype(np.float32)
    dw_w = (r.standard_normal((E, 1, K, K)) * np.sqrt(2.0 / (K * K))).astype(np.float32)
    dw_b = (r.standard_normal(E) * 0.1).astype(np.float32)
    pw_w = (r.standard_normal((Cout, E, 1, 1)) * np.sqrt(2.0 / E)).astype(np.float32)
    pw_b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    OH = (H + 2 * p - K) // s + 1
    OW = (W + 2 * p - K) // s + 1
    res = r.standard_normal((N, Cout, OH, OW)).astype(np.float32) if has_r else None
    return x, dw_w, dw_b, pw_w, pw_b, res


def se_inputs(case, seed):
    _, N, C, Cr, a, b = case
    r = np.random.default_rng(seed)
    avg = r.standard_normal((N, C, 1, 1)).astype(np.float32)
    w1 = (r.standard_normal((Cr, C, 1, 1)) * np.sqrt(2.0 / C)).astype(np.float32)
    b1 = (r.standard_normal(Cr) * 0.1).astype(np.float32)
    w2 = (r.standard_normal((C, Cr, 1, 1)) * np.sqrt(2.0 / Cr)).astype(np.float32)
    b2 = (r.standard_normal(C) * 0.1).astype(np.float32)
    return avg, w1, b1, w2, b2


def codec_inputs():
    """fp32 bit patterns around every kind of fp16 rounding edge: exact halves, ties of the 13
    dropped bits, the subnormal range, the overflow edge, NaN/inf, plus random patterns."""
    r = np.random.default_rng(11)
    hi = r.integers(0, 1 << 19, 8192, dtype=np.uint32) << 13
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF], np.uint32)
    edge = (hi[:, None] | lows[None, :]).ravel()
    named = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e9, np.inf, -np.inf, np.nan,
                      6.1035156e-05, 6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-10, -3e-8,
                      1.00048828125, 1.0009765625, 1.00146484375, 2049.0, 2051.0, 0.1, 1.0 / 3.0], np.float32)
    # every exponent in and below the fp16 subnormal range, with tie mantissas
    sub = np.array([(e << 23) | m for e in range(96, 114) for m in (0, 0x1000, 0x2000, 0x3000, 0x7FF000, 0x7FFFFF)],
                   np.uint32)
    rand = r.integers(0, 1 << 32, 4096, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([named.view(np.uint32), edge, sub, rand, sub | 0x80000000])


def main():
    assert O.ref_available(), "build oracle/_ref first (make -C oracle ref)"
    R = O.ref()
    out = {}

    # codec: floatToHalf on edge patterns; halfToFloat on all 65536 halves
    bits = codec_inputs()
    f = bits.view(np.float32)
    h = np.zeros(f.size, np.uint16)
    R.ref_float_to_half_n(f.ctypes.data, h.ctypes.data, f.size)
    allh = np.arange(65536, dtype=np.uint16)
    back = np.zeros(65536, np.float32)
    R.ref_half_to_float_n(allh.ctypes.data, back.ctypes.data, 65536)
    np.savez_compressed(os.path.join(HERE, "codec.npz"), f32_bits=bits, f16=h, all_h2f_bits=back.view(np.uint32))

    # single-node conv graphs (Conv with fused act / residual as the passes leave them)
    for k, case in enumerate(CONV_CASES):
        x, w, b, res = conv_inputs(case, 100 + k)
        inputs = [x, w, b]
        fused_res = -1
        if res is not None:
            inputs.append(res)
            fused_res = 3
        y, ys = O.ref_single_node("Conv", inputs, conv_attrs(case), fused_act=case[12], lo=case[13], hi=case[14],
                                  fused_res=fused_res)
        n = int(np.prod(ys))
        out["conv/" + case[0]] = dict(x=x, w=w, b=b, res=res, y=y[:n].reshape(ys))

    for k, case in enumerate(DWPW_CASES):
        x, dw_w, dw_b, pw_w, pw_b, res = dwpw_inputs(case, 200 + k)
        _, N, E, H, W, Cout, K, s, p, dwa, act, lo, hi, has_r = case
        inputs = [x, dw_w, dw_b, pw_w, pw_b] + ([res] if has_r else [])
        attrs = f"l:strides={s},{s};l:pads={p},{p},{p},{p};l:dilations=1,1"
        y, ys = O.ref_single_node("FusedDwPw", inputs, attrs, sub_op=dwa, fused_act=act, lo=lo, hi=hi,
                                  fused_res=5 if has_r else -1)
        out["dwpw/" + case[0]] = dict(x=x, dw_w=dw_w, dw_b=dw_b, pw_w=pw_w, pw_b=pw_b, res=res,
                                      y=y[:int(np.prod(ys))].reshape(ys))

    for k, case in enumerate(SE_CASES):
        avg, w1, b1, w2, b2 = se_inputs(case, 300 + k)
        y, ys = O.ref_single_node("FusedSE", [avg, w1, b1, w2, b2], "", lo=case[4], hi=case[5])
        out["se/" + case[0]] = dict(avg=avg, w1=w1, b1=b1, w2=w2, b2=b2, y=y[:int(np.prod(ys))].reshape(ys))

    r = np.random.default_rng(400)
    a = r.standard_normal((2, 6, 5, 5)).astype(np.float32)
    b = r.standard_normal((2, 6, 5, 5)).astype(np.float32)
    for act, lo, hi, nm in ((0, 0, 0, "none"), (1, 0, 0, "relu"), (3, -0.3, 0.4, "clip")):
        y, ys = O.ref_single_node("Add", [a, b], "", fused_act=act, lo=lo, hi=hi)
        out[f"add/{nm}"] = dict(a=a, b=b, y=y[:a.size].reshape(a.shape))
    s = r.uniform(0, 1, (2, 6, 1, 1)).astype(np.float32)
    y, ys = O.ref_single_node("Binary", [a, s], "", sub_op=0)
    out["mul_channel/bcast"] = dict(a=a, s=s, y=y[:a.size].reshape(a.shape))
    xu = (r.standard_normal((1, 5, 6, 7)) * 4).astype(np.float32)
    for code, p0, p1, nm in ((0, 0, 0, "sigmoid"), (2, 0, 0, "hardswish"), (3, 1.0 / 6.0, 0.5, "hardsigmoid"),
                             (14, 0, 0, "silu")):
        y, ys = O.ref_single_node("Unary", [xu], "", sub_op=code, lo=p0, hi=p1)
        out[f"unary/{nm}"] = dict(x=xu, y=y[:xu.size].reshape(xu.shape))
    y, ys = O.ref_single_node("GlobalAvgPool", [xu], "")
    out["gap/basic"] = dict(x=xu, y=y[:int(np.prod(ys))].reshape(ys))
    y, ys = O.ref_single_node("MaxPool", [xu], "l:kernel_shape=3,3;l:strides=2,2;l:pads=1,1,1,1")
    out["maxpool/k3s2p1"] = dict(x=xu, y=y[:int(np.prod(ys))].reshape(ys))
    ga = r.standard_normal((3, 20)).astype(np.float32)
    gb = r.standard_normal((7, 20)).astype(np.float32)
    gc = r.standard_normal(7).astype(np.float32)
    y, ys = O.ref_single_node("Gemm", [ga, gb, gc], "i:transB=1;f:alpha=1.0;f:beta=1.0")
    out["gemm/transB"] = dict(a=ga, b=gb, c=gc, y=y[:21].reshape(3, 7))

    flat = {}
    for key, d in out.items():
        for k2, v in d.items():
            if v is not None:
                flat[f"{key}/{k2}"] = v
    np.savez_compressed(os.path.join(HERE, "ops.npz"), **flat)

    # whole graphs from the shared zoo source, passes + CPU backend of the reference
    mflat = {}
    for name, batch in MODELS:
        in_shape, _ = O.model_io(name, batch)
        x = np.random.default_rng(500 + batch).standard_normal(in_shape).astype(np.float32)
        y = O.ref_model_run(name, batch, MODEL_SEED, x)
        mflat[f"{name}/b{batch}/x"] = x
        mflat[f"{name}/b{batch}/y"] = y
    np.savez_compressed(os.path.join(HERE, "models.npz"), **mflat)
    for fn in ("codec.npz", "ops.npz", "models.npz"):
        print(fn, os.path.getsize(os.path.join(HERE, fn)), "bytes")


if __name__ == "__main__":
    main()
