"""Helpers that drive the HIP kernels through the vkhip C ABI on numpy data (GPU tests only)."""
import ctypes

import numpy as np

import vknn_amd as V
from vknn_amd import DeviceBuffer, check


def to_device_nc4(x):
    """NCHW fp32 numpy -> NC4HW4 fp16 device buffer via the GPU pack kernel."""
    x = np.ascontiguousarray(x, np.float32)
    N, C, H, W = x.shape
    src = DeviceBuffer.from_array(x)
    dst = DeviceBuffer(V.nc4_elems(N, C, H, W) * 2)
    check(V.vkhip().vkhip_pack_nchw_f32(src.ptr, dst.ptr, N, C, H, W, None), "pack")
    check(V.vkhip().vkhip_stream_sync(None), "sync")
    return dst


def from_device_nc4(buf, shape):
    N, C, H, W = shape
    out = DeviceBuffer(N * C * H * W * 4)
    check(V.vkhip().vkhip_unpack_nchw_f32(buf.ptr, out.ptr, N, C, H, W, None), "unpack")
    check(V.vkhip().vkhip_stream_sync(None), "sync")
    return out.download(np.float32, N * C * H * W).reshape(shape)


def raw_nc4(buf, shape):
    N, C, H, W = shape
    return buf.download(np.uint16, V.nc4_elems(N, C, H, W))


def round_half(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def conv_desc(x_shape, w_shape, stride=(1, 1), pads=(0, 0, 0, 0), dil=(1, 1), group=1, act=0, lo=0.0, hi=0.0,
              has_res=0):
    N, C, H, W = x_shape
    Cout, _, KH, KW = w_shape
    OH = (H + pads[0] + pads[2] - (dil[0] * (KH - 1) + 1)) // stride[0] + 1
    OW = (W + pads[1] + pads[3] - (dil[1] * (KW - 1) + 1)) // stride[1] + 1
    d = V.ConvDesc(N=N, Cin=C, H=H, W=W, Cout=Cout, OH=OH, OW=OW, KH=KH, KW=KW, SH=stride[0], SW=stride[1],
                   PT=pads[0], PL=pads[1], DH=dil[0], DW=dil[1], group=group, act=act, act_lo=lo, act_hi=hi,
                   has_res=has_res)
    return d, (N, Cout, OH, OW)


def gpu_conv(x, w, b=None, stride=(1, 1), pads=(0, 0, 0, 0), dil=(1, 1), group=1, act=0, lo=0.0, hi=0.0, res=None,
             algo=V.CONV_AUTO, tile=-1, ksplit=0, res_post=False):
    """res_post: the residual is added after the activation (has_res 2) instead of before it."""
    lib = V.vkhip()
    d, yshape = conv_desc(x.shape, w.shape, stride, pads, dil, group, act, lo, hi, (2 if res_post else 1) if res is not None else 0)
    plan = V.ConvPlan()
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), algo, tile, ksplit, ctypes.byref(plan)), "plan")
    blob = np.zeros(plan.weight_bytes, np.uint8)
    w = np.ascontiguousarray(w, np.float32)
    bb = None if b is None else np.ascontiguousarray(b, np.float32)
    check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data,
                                      bb.ctypes.data if bb is not None else None, blob.ctypes.data), "pack weights")
    dblob = DeviceBuffer.from_array(blob)
    dx = to_device_nc4(x)
    dres = to_device_nc4(res) if res is not None else None
    dy = DeviceBuffer(V.nc4_elems(*yshape) * 2)
    dy.zero()
    ws = DeviceBuffer(plan.workspace_bytes) if plan.workspace_bytes else None
    if ws:
        ws.zero()  # SPLITK_LAST keeps arrival counters in it that start at zero
    check(lib.vkhip_conv_forward(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr,
                                 dres.ptr if dres else None, dy.ptr, ws.ptr if ws else None, None), "conv_forward")
    check(lib.vkhip_stream_sync(None), "sync")
    return from_device_nc4(dy, yshape), plan, dy
