"""ctypes access to the CPU oracle (oracle/liboracle.so) and, where built, the reference CPU backend
(oracle/_ref/libvknn_ref.so). Test infrastructure: the checker, never the thing measured."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_PATH = os.path.join(ROOT, "oracle", "_ref", "libvknn_ref.so")

c_i32, c_i64, c_u64, c_f, c_vp, c_char_p = (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float,
                                            ctypes.c_void_p, ctypes.c_char_p)
P = ctypes.POINTER

ORACLE_API = {
    "oracle_float_to_half_n": (None, [c_vp, c_vp, c_i64]),
    "oracle_half_to_float_n": (None, [c_vp, c_vp, c_i64]),
    "oracle_pack_nc4hw4": (None, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64]),
    "oracle_unpack_nc4hw4": (None, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64]),
    "oracle_apply_act": (None, [c_vp, c_i64, ctypes.c_int, c_f, c_f]),
    "oracle_conv2d": (None, [c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64,
                             c_vp, ctypes.c_int, c_f, c_f, c_vp]),
    "oracle_conv_out_hw": (None, [c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, P(c_i64), P(c_i64)]),
    "oracle_fused_dwpw": (None, [c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp,
                                 c_vp, c_vp, ctypes.c_int, c_vp, ctypes.c_int, c_f, c_f, c_vp]),
    "oracle_fused_se": (None, [c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_f, c_f, c_vp]),
    "oracle_add": (None, [c_vp, c_vp, c_vp, c_i64, ctypes.c_int, c_f, c_f]),
    "oracle_mul_channel": (None, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64]),
    "oracle_binary": (None, [c_vp, c_vp, c_vp, c_i64, ctypes.c_int]),
    "oracle_unary": (None, [c_vp, c_vp, c_i64, ctypes.c_int, c_f, c_f]),
    "oracle_global_avg_pool": (None, [c_vp, c_vp, c_i64, c_i64, c_i64]),
    "oracle_maxpool": (None, [c_vp, c_vp] + [c_i64] * 12),
    "oracle_gemm": (None, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, ctypes.c_int, c_f, c_f, ctypes.c_int, c_f, c_f]),
    "oracle_concat_channels": (None, [P(c_vp), P(c_i64), ctypes.c_int, c_vp, c_i64, c_i64]),
    "oracle_slice_channels": (None, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64]),
    "oracle_resize_nearest": (None, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int]),
    "oracle_fold_bn": (None, [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_f]),
    "oracle_float_to_half_rne": (ctypes.c_uint16, [c_f]),
    "oracle_boundary_convert": (None, [c_vp, ctypes.c_int, ctypes.c_int, c_vp, ctypes.c_int, ctypes.c_int, c_i64, c_i64, c_i64, c_i64]),
    "oracle_last_error": (c_char_p, []),
    "oracle_model_run": (ctypes.c_int, [c_char_p, c_i64, c_u64, c_vp, c_i64, c_vp, c_i64]),
    "oracle_model_io": (ctypes.c_int, [c_char_p, c_i64, P(c_i64), P(c_i64), P(c_i32), c_i32]),
    "oracle_model_flops": (ctypes.c_double, [c_char_p]),
}

REF_API = {
    "ref_last_error": (c_char_p, []),
    "ref_float_to_half_n": (None, [c_vp, c_vp, c_i64]),
    "ref_half_to_float_n": (None, [c_vp, c_vp, c_i64]),
    "ref_model_run": (ctypes.c_int, [c_char_p, c_i64, c_u64, c_vp, c_i64, c_vp, c_i64]),
    "ref_onnx_describe": (ctypes.c_int, [c_char_p, c_char_p, c_i64]),
    "ref_onnx_run": (ctypes.c_int, [c_char_p, c_vp, c_i64, c_vp, c_i64]),
    "ref_single_node": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, c_f, c_f, c_char_p, ctypes.c_int, P(c_vp),
                                       P(c_i64), P(c_i32), ctypes.c_int, ctypes.c_int, c_vp, c_i64, P(c_i64)]),
}

_libs = {}


def _bind(lib, api):
    for name, (res, args) in api.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def oracle():
    if "o" not in _libs:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError("oracle/liboracle.so missing: run __graft_entry__.build()")
        _libs["o"] = _bind(ctypes.CDLL(ORACLE_PATH), ORACLE_API)
    return _libs["o"]


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    if "r" not in _libs:
        _libs["r"] = _bind(ctypes.CDLL(REF_PATH), REF_API)
    return _libs["r"]


def f32p(a):
    return a.ctypes.data if a is not None else None


def i64arr(v):
    return np.asarray(v, dtype=np.int64)


def parity(got, ref_):
    """(max |got-ref| / max |ref|, cosine) — the north-star parity metrics."""
    got = np.asarray(got, np.float64).ravel()
    ref_ = np.asarray(ref_, np.float64).ravel()
    denom = max(np.abs(ref_).max(), 1e-30)
    rel = float(np.abs(got - ref_).max() / denom)
    n1, n2 = np.linalg.norm(got), np.linalg.norm(ref_)
    cos = float(got @ ref_ / (n1 * n2)) if n1 > 0 and n2 > 0 else (1.0 if n1 == n2 else 0.0)
    return rel, cos


def model_io(name, batch):
    in4 = (c_i64 * 4)()
    outs = (c_i64 * 16)()
    n = c_i32()
    assert oracle().oracle_model_io(name.encode(), batch, in4, outs, ctypes.byref(n), 16) == 0
    return list(in4), list(outs)[:n.value]


def oracle_model_run(name, batch, seed, x):
    _, outs = model_io(name, batch)
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.zeros(sum(outs), np.float32)
    rc = oracle().oracle_model_run(name.encode(), batch, seed, x.ctypes.data, x.size, y.ctypes.data, y.size)
    assert rc == 0, oracle().oracle_last_error()
    return y


def ref_model_run(name, batch, seed, x):
    _, outs = model_io(name, batch)
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.zeros(sum(outs), np.float32)
    rc = ref().ref_model_run(name.encode(), batch, seed, x.ctypes.data, x.size, y.ctypes.data, y.size)
    assert rc == 0, ref().ref_last_error()
    return y


def oracle_conv(x, w, b=None, stride=(1, 1), pads=(0, 0, 0, 0), dil=(1, 1), group=1, res=None, act=0, lo=0.0, hi=0.0):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    N, C, H, W = x.shape
    Cout, _, KH, KW = w.shape
    st, pd, dl = i64arr(stride), i64arr(pads), i64arr(dil)
    OH, OW = c_i64(), c_i64()
    oracle().oracle_conv_out_hw(H, W, KH, KW, st.ctypes.data, pd.ctypes.data, dl.ctypes.data, ctypes.byref(OH),
                                ctypes.byref(OW))
    y = np.zeros((N, Cout, OH.value, OW.value), np.float32)
    b = None if b is None else np.ascontiguousarray(b, np.float32)
    res = None if res is None else np.ascontiguousarray(res, np.float32)
    oracle().oracle_conv2d(x.ctypes.data, N, C, H, W, w.ctypes.data, Cout, KH, KW, f32p(b), st.ctypes.data,
                           pd.ctypes.data, dl.ctypes.data, group, f32p(res), act, lo, hi, y.ctypes.data)
    return y


def oracle_dwpw(x, dw_w, dw_b, pw_w, pw_b, stride=(1, 1), pads=(1, 1, 1, 1), dil=(1, 1), dw_act=0, res=None, act=0,
                lo=0.0, hi=0.0):
    x = np.ascontiguousarray(x, np.float32)
    N, E, H, W = x.shape
    KH, KW = dw_w.shape[2], dw_w.shape[3]
    Cout = pw_w.shape[0]
    st, pd, dl = i64arr(stride), i64arr(pads), i64arr(dil)
    OH = (H + pads[0] + pads[2] - (dil[0] * (KH - 1) + 1)) // stride[0] + 1
    OW = (W + pads[1] + pads[3] - (dil[1] * (KW - 1) + 1)) // stride[1] + 1
    y = np.zeros((N, Cout, OH, OW), np.float32)
    arrs = [np.ascontiguousarray(a, np.float32) if a is not None else None for a in (dw_w, dw_b, pw_w, pw_b, res)]
    oracle().oracle_fused_dwpw(x.ctypes.data, N, E, H, W, f32p(arrs[0]), KH, KW, f32p(arrs[1]), f32p(arrs[2]), Cout,
                               f32p(arrs[3]), st.ctypes.data, pd.ctypes.data, dl.ctypes.data, dw_act, f32p(arrs[4]),
                               act, lo, hi, y.ctypes.data)
    return y


def oracle_pack(x):
    x = np.ascontiguousarray(x, np.float32)
    N, C, H, W = x.shape
    out = np.zeros(N * ((C + 3) // 4) * 4 * H * W, np.uint16)
    oracle().oracle_pack_nc4hw4(x.ctypes.data, out.ctypes.data, N, C, H, W)
    return out


def oracle_unpack(h, shape):
    N, C, H, W = shape
    h = np.ascontiguousarray(h, np.uint16)
    out = np.zeros((N, C, H, W), np.float32)
    oracle().oracle_unpack_nc4hw4(h.ctypes.data, out.ctypes.data, N, C, H, W)
    return out


# OpType codes shared by the reference and this build (include/vknn/op_type.h order)
OP = {"Conv": 1, "Clip": 3, "Relu": 4, "Add": 5, "GlobalAvgPool": 6, "MaxPool": 8, "Gemm": 9, "Concat": 20,
      "Unary": 27, "Binary": 28, "Resize": 30, "Split": 37, "FusedSE": 45, "FusedDwPw": 46}


def ref_single_node(op, inputs, attrs="", sub_op=0, fused_act=0, lo=0.0, hi=0.0, fused_res=-1, n_out=1, out_size=None):
    """Run one node through the reference CPU Session. inputs: list of arrays (or None); input 0
    (and the fused residual) are graph inputs, the rest constants."""
    n = len(inputs)
    arrs = [None if a is None else np.ascontiguousarray(a, np.float32) for a in inputs]
    data = (c_vp * n)(*[a.ctypes.data if a is not None else None for a in arrs])
    shapes = np.zeros(4 * n, np.int64)
    ranks = np.zeros(n, np.int32)
    for k, a in enumerate(arrs):
        if a is not None:
            ranks[k] = a.ndim
            shapes[4 * k:4 * k + a.ndim] = a.shape
    size = out_size or max(int(a.size) for a in arrs if a is not None) * 8
    y = np.zeros(size, np.float32)
    ys = np.zeros(4, np.int64)
    rc = ref().ref_single_node(OP[op], sub_op, fused_act, lo, hi, attrs.encode(), n, data,
                               shapes.ctypes.data_as(P(c_i64)), ranks.ctypes.data_as(P(c_i32)), fused_res, n_out,
                               y.ctypes.data, y.size, ys.ctypes.data_as(P(c_i64)))
    assert rc == 0, ref().ref_last_error()
    return y, tuple(int(v) for v in ys)
