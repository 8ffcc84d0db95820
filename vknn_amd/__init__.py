"""vknn_amd — Python bindings (ctypes) for the MI355X HIP backend of vknn's fused fp16 conv path.

Two native libraries, both built in-tree by ``__graft_entry__.build()``:

* ``libvkhip.so`` — the gfx950 kernels behind the ``vkhip`` C ABI (``include/vkhip.h``).
* ``libvknn.so``  — the vknn C++ host library (graph, passes, Session, HIP backend) and its
  C ABI (``include/vknn_c.h``).

Nothing here computes on the host: every op goes to the HIP kernels, and loading fails loudly when
the libraries are missing.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
VKHIP_PATH = os.path.join(_HERE, "libvkhip.so")
VKNN_PATH = os.path.join(_HERE, "libvknn.so")

c_int, c_i32, c_i64, c_u64, c_f, c_vp, c_sz, c_char_p = (
    ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p,
    ctypes.c_size_t, ctypes.c_char_p)
c_dbl = ctypes.c_double

ACT = {"none": 0, "relu": 1, "relu6": 2, "clip": 3, "hardswish": 4, "silu": 5}
CONV_AUTO, CONV_GEMM, CONV_SPLITK, CONV_WINOGRAD, CONV_DEPTHWISE, CONV_SPLITK_LAST = 0, 1, 2, 3, 4, 5


class ConvDesc(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("N", "Cin", "H", "W", "Cout", "OH", "OW", "KH", "KW", "SH", "SW", "PT",
                                     "PL", "DH", "DW", "group", "act")] + \
               [("act_lo", c_f), ("act_hi", c_f), ("has_res", c_i32), ("in_scale", c_i32)]


class ConvPlan(ctypes.Structure):
    _fields_ = [("algo", c_i32), ("tile", c_i32), ("ksplit", c_i32), ("reserved", c_i32),
                ("weight_bytes", c_sz), ("workspace_bytes", c_sz)]


class DwPwDesc(ctypes.Structure):
    _fields_ = [("dw", ConvDesc), ("Cout", c_i32), ("act", c_i32), ("act_lo", c_f), ("act_hi", c_f),
                ("has_res", c_i32)]


class ConvPwDesc(ctypes.Structure):
    _fields_ = [("conv", ConvDesc), ("Cout", c_i32), ("act", c_i32), ("act_lo", c_f), ("act_hi", c_f),
                ("has_res", c_i32)]


class ConvPw2Desc(ctypes.Structure):
    _fields_ = [("pw", ConvPwDesc), ("Cout3", c_i32), ("act3", c_i32), ("act3_lo", c_f), ("act3_hi", c_f)]


class PoolDesc(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("N", "C", "H", "W", "OH", "OW", "KH", "KW", "SH", "SW", "PT", "PL")]


P = ctypes.POINTER
# name -> (restype, argtypes); every symbol declared in include/vkhip.h
VKHIP_API = {
    "vkhip_init": (c_int, []),
    "vkhip_available": (c_int, []),
    "vkhip_device_info": (c_int, [c_char_p, c_int, P(c_int), P(c_int), P(c_sz)]),
    "vkhip_last_error": (c_char_p, []),
    "vkhip_build_info": (c_char_p, []),
    "vkhip_malloc": (c_int, [P(c_vp), c_sz]),
    "vkhip_free": (c_int, [c_vp]),
    "vkhip_dispatch_marker": (c_int, [c_i32, c_vp]),
    "vkhip_conv_maxpool_supported": (c_int, [c_vp, c_vp, c_vp]),
    "vkhip_conv_maxpool_forward": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_conv_plan_kernel": (c_char_p, [c_vp]),
    "vkhip_dmabuf_import": (c_int, [c_int, c_sz, P(c_vp), P(c_vp)]),
    "vkhip_dmabuf_release": (c_int, [c_vp]),
    "vkhip_dmabuf_export": (c_int, [c_vp, c_sz, P(c_int)]),
    "vkhip_memcpy_h2d": (c_int, [c_vp, c_vp, c_sz, c_vp]),
    "vkhip_memcpy_d2h": (c_int, [c_vp, c_vp, c_sz, c_vp]),
    "vkhip_memcpy_d2d": (c_int, [c_vp, c_vp, c_sz, c_vp]),
    "vkhip_fill_zero": (c_int, [c_vp, c_sz, c_vp]),
    "vkhip_gpu_sleep": (c_int, [c_i32, c_vp]),
    "vkhip_stream_create": (c_int, [P(c_vp)]),
    "vkhip_stream_destroy": (c_int, [c_vp]),
    "vkhip_stream_sync": (c_int, [c_vp]),
    "vkhip_device_sync": (c_int, []),
    "vkhip_event_create": (c_int, [P(c_vp)]),
    "vkhip_event_destroy": (c_int, [c_vp]),
    "vkhip_event_record": (c_int, [c_vp, c_vp]),
    "vkhip_stream_wait_event": (c_int, [c_vp, c_vp]),
    "vkhip_event_sync": (c_int, [c_vp]),
    "vkhip_event_elapsed_ms": (c_int, [c_vp, c_vp, P(c_f)]),
    "vkhip_graph_begin": (c_int, [c_vp]),
    "vkhip_graph_end": (c_int, [c_vp, P(c_vp)]),
    "vkhip_graph_launch": (c_int, [c_vp, c_vp]),
    "vkhip_graph_destroy": (c_int, [c_vp]),
    "vkhip_pack_nchw_f32": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "vkhip_unpack_nchw_f32": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "vkhip_unpack_nchw_f32_multi": (c_int, [P(c_vp), P(c_vp), P(c_i64), c_i32, c_vp]),
    "vkhip_convert_layout": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_vp]),
    "vkhip_boundary_convert": (c_int, [c_vp, c_i32, c_i32, c_vp, c_i32, c_i32, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "vkhip_pack_flat_f32": (c_int, [c_vp, c_vp, c_i64, c_vp]),
    "vkhip_unpack_flat_f32": (c_int, [c_vp, c_vp, c_i64, c_vp]),
    "vkhip_conv_plan_make": (c_int, [P(ConvDesc), c_i32, c_i32, c_i32, P(ConvPlan)]),
    "vkhip_conv_tile_count": (c_int, []),
    "vkhip_conv_pack_weights": (c_int, [P(ConvDesc), P(ConvPlan), c_vp, c_vp, c_vp]),
    "vkhip_conv_forward": (c_int, [P(ConvDesc), P(ConvPlan), c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_conv_forward_noalloc": (c_int, [P(ConvDesc), P(ConvPlan), c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_convpw_plan": (c_int, [P(ConvPwDesc), P(ConvPlan)]),
    "vkhip_convpw_pack_weights": (c_int, [P(ConvPwDesc), P(ConvPlan), c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_convpw_forward": (c_int, [P(ConvPwDesc), P(ConvPlan), c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_convpw2_plan": (c_int, [P(ConvPw2Desc), P(ConvPlan)]),
    "vkhip_convpw2_pack_weights": (c_int, [P(ConvPw2Desc), P(ConvPlan), c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_convpw2_forward": (c_int, [P(ConvPw2Desc), P(ConvPlan), c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_conv_forward_stages": (c_int, [P(ConvDesc), P(ConvPlan), c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_vp]),
    "vkhip_conv_forward_scaled": (c_int, [P(ConvDesc), P(ConvPlan), c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_conv_pool_parts": (c_int, [P(ConvDesc), P(ConvPlan)]),
    "vkhip_conv_forward_view": (c_int, [P(ConvDesc), P(ConvPlan), c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp]),
    "vkhip_conv_forward_view_res": (c_int, [P(ConvDesc), P(ConvPlan), c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp]),
    "vkhip_conv3x3_pair_plan": (c_int, [P(ConvDesc), P(ConvDesc), P(ConvPlan), P(ConvPlan)]),
    "vkhip_conv3x3_pair_forward": (c_int, [P(ConvDesc), P(ConvDesc), c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp]),
    "vkhip_conv3x3s2_pair_plan": (c_int, [P(ConvDesc), P(ConvDesc), P(ConvDesc), P(ConvPlan), P(ConvPlan), P(ConvPlan)]),
    "vkhip_conv3x3s2_pair_forward": (c_int, [P(ConvDesc), P(ConvDesc), P(ConvDesc), c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp]),
    "vkhip_stem_dwpw_plan": (c_int, [P(ConvDesc), P(ConvDesc), P(ConvDesc), P(ConvPlan), P(ConvPlan), P(ConvPlan)]),
    "vkhip_stem_dwpw_forward": (c_int, [P(ConvDesc), P(ConvDesc), P(ConvDesc), c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp]),
    "vkhip_add_view": (c_int, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_i64, c_i32, c_f, c_f, c_vp]),
    "vkhip_maxpool_view": (c_int, [P(PoolDesc), c_vp, c_i64, c_vp, c_i64, c_vp]),
    "vkhip_maxpool_chain": (c_int, [P(PoolDesc), c_vp, c_i64, P(c_vp), P(c_i64), c_i32, c_vp]),
    "vkhip_resize_nearest_view": (c_int, [c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "vkhip_conv_forward_pooled": (c_int, [P(ConvDesc), P(ConvPlan), c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_dwpw_supported": (c_int, [P(DwPwDesc)]),
    "vkhip_dwpw_weight_bytes": (c_sz, [P(DwPwDesc)]),
    "vkhip_dwpw_pack_weights": (c_int, [P(DwPwDesc), c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_dwpw_forward": (c_int, [P(DwPwDesc), c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_global_avg_pool": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "vkhip_se_weight_bytes": (c_sz, [c_i64, c_i64]),
    "vkhip_se_pack_weights": (c_int, [c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "vkhip_se_workspace_bytes": (c_sz, [c_i64, c_i64]),
    "vkhip_fused_se": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_f, c_f, c_vp, c_vp]),
    "vkhip_fused_se_pooled": (c_int, [c_vp, c_i32, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_f, c_f, c_vp, c_vp]),
    "vkhip_channel_scale": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp]),
    "vkhip_add": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i32, c_f, c_f, c_vp]),
    "vkhip_unary": (c_int, [c_vp, c_vp, c_i64, c_i32, c_f, c_f, c_vp]),
    "vkhip_binary": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i32, c_vp]),
    "vkhip_maxpool": (c_int, [P(PoolDesc), c_vp, c_vp, c_vp]),
    "vkhip_fc_weight_bytes": (c_sz, [c_i64, c_i64]),
    "vkhip_fc_pack_weights": (c_int, [c_i64, c_i64, c_vp, c_i32, c_vp, c_f, c_f, c_vp]),
    "vkhip_fc": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i32, c_f, c_f, c_vp]),
    "vkhip_fc_pooled": (c_int, [c_vp, c_i32, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_i32, c_f, c_f, c_vp]),
    "vkhip_concat_channels": (c_int, [P(c_vp), P(c_i64), c_i32, c_vp, c_i64, c_i64, c_vp]),
    "vkhip_slice_channels": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "vkhip_resize_nearest": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp]),
}

VKNN_API = {
    "vknn_last_error": (c_char_p, []),
    "vknn_model_io": (c_int, [c_char_p, c_i64, P(c_i64), P(c_i64), P(c_i32), c_i32]),
    "vknn_model_flops": (c_dbl, [c_char_p]),
    "vknn_session_create_model": (c_int, [c_char_p, c_i64, c_u64, c_char_p, P(c_vp)]),
    "vknn_session_destroy": (c_int, [c_vp]),
    "vknn_session_run_host": (c_int, [c_vp, c_vp, c_i64, c_vp, c_i64]),
    "vknn_session_bind_device_input": (c_int, [c_vp, c_vp]),
    "vknn_session_bind_device_input_as": (c_int, [c_vp, c_vp, c_i32, c_i32]),
    "vknn_session_run_device": (c_int, [c_vp]),
    "vknn_session_sync": (c_int, [c_vp]),
    "vknn_session_device_output": (c_vp, [c_vp, c_i32]),
    "vknn_session_read_outputs": (c_int, [c_vp, c_vp, c_i64]),
    "vknn_session_stream": (c_vp, [c_vp]),
    "vknn_session_profile_json": (c_int, [c_vp, c_char_p, c_i64]),
    "vknn_session_describe": (c_int, [c_vp, c_char_p, c_i64]),
    "vknn_session_count_ops": (c_int, [c_vp, c_char_p]),
    "vknn_session_segments": (c_int, [c_vp, c_char_p, c_i64]),
    "vknn_session_run_dmabuf": (c_int, [c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64]),
    "vknn_graph_after_passes": (c_int, [c_char_p, c_i64, c_char_p, c_char_p, c_i64]),
    "vknn_model_save_vxm": (c_int, [c_char_p, c_i64, c_u64, c_char_p, c_char_p]),
    "vknn_vxm_describe": (c_int, [c_char_p, c_char_p, c_i64]),
    "vknn_session_create_vxm": (c_int, [c_char_p, c_char_p, P(c_vp)]),
    "vknn_session_save_optimized": (c_int, [c_vp, c_char_p]),
    "vknn_onnx_describe": (c_int, [c_char_p, c_char_p, c_i64]),
    "vknn_onnx_after_passes": (c_int, [c_char_p, c_char_p, c_char_p, c_i64]),
    "vknn_session_create_onnx": (c_int, [c_char_p, c_char_p, P(c_vp)]),
    "vknn_tune_cache_load": (c_int, [c_char_p]),
    "vknn_tune_cache_save": (c_int, [c_char_p]),
    "vknn_tune_cache_put": (c_int, [c_char_p, c_i32]),
    "vknn_tune_cache_get": (c_int, [c_char_p, P(c_i32)]),
    "vknn_tune_cache_clear": (c_int, []),
    "vknn_tune_cache_stats": (c_int, [P(c_i64), P(c_i64), P(c_i64)]),
    "vknn_weight_cache_stats": (c_int, [P(c_i64), P(c_i64), P(c_i64)]),
    "vknn_tune_cache_gpu_tag": (c_int, [c_char_p, c_i64]),
}

_libs = {}


def _load(path, api):
    if not os.path.exists(path):
        raise RuntimeError(f"native library {path} is missing: run __graft_entry__.build() first "
                           "(the HIP path has no fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in api.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def vkhip():
    """The kernel library (include/vkhip.h)."""
    if "vkhip" not in _libs:
        _libs["vkhip"] = _load(VKHIP_PATH, VKHIP_API)
    return _libs["vkhip"]


def vknn():
    """The host library (include/vknn_c.h); loads libvkhip.so first (its dependency)."""
    if "vknn" not in _libs:
        vkhip()
        _libs["vknn"] = _load(VKNN_PATH, VKNN_API)
    return _libs["vknn"]


class VkhipError(RuntimeError):
    pass


def check(rc, what="vkhip"):
    if rc != 0:
        raise VkhipError(f"{what} failed ({rc}): {vkhip().vkhip_last_error().decode(errors='replace')}")


def require_gpu():
    lib = vkhip()
    if lib.vkhip_available() != 1:
        raise VkhipError("no gfx950 device: " + lib.vkhip_last_error().decode(errors='replace'))
    return lib


class DeviceBuffer:
    """A device allocation made through vkhip_malloc (freed on close / garbage collection)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = c_vp()
        check(vkhip().vkhip_malloc(ctypes.byref(p), max(self.nbytes, 256)), "vkhip_malloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(vkhip().vkhip_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, None), "h2d")

    def download(self, dtype, count):
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(vkhip().vkhip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, None), "d2h")
        return out

    def zero(self):
        check(vkhip().vkhip_fill_zero(self.ptr, self.nbytes, None), "fill_zero")

    def close(self):
        if getattr(self, "ptr", None):
            vkhip().vkhip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def nc4_elems(n, c, h, w):
    return n * ((c + 3) // 4) * 4 * h * w


class Session:
    """A vknn Session on the HIP backend over a zoo model (include/vknn_c.h)."""

    def __init__(self, model, batch, seed=7, options=""):
        lib = vknn()
        require_gpu()
        self.model, self.batch = model, batch
        h = c_vp()
        rc = lib.vknn_session_create_model(model.encode(), batch, seed, options.encode(), ctypes.byref(h))
        if rc:
            raise VkhipError("session create: " + lib.vknn_last_error().decode(errors='replace'))
        self.h = h.value
        self.in_shape, self.out_elems = model_io(model, batch)

    @classmethod
    def from_vxm(cls, path, model, batch, options=""):
        """A session planned from a .vxm file; `model`/`batch` name the zoo model it was saved
        from, which fixes the input and output sizes."""
        lib = vknn()
        require_gpu()
        self = cls.__new__(cls)
        self.model, self.batch = model, batch
        h = c_vp()
        if lib.vknn_session_create_vxm(str(path).encode(), options.encode(), ctypes.byref(h)):
            raise VkhipError("session create: " + lib.vknn_last_error().decode(errors='replace'))
        self.h = h.value
        self.in_shape, self.out_elems = model_io(model, batch)
        return self

    @classmethod
    def from_onnx(cls, path, in_shape, out_elems, options=""):
        """A session imported from an ONNX file with one input of `in_shape` and outputs of
        `out_elems` elements each."""
        lib = vknn()
        require_gpu()
        self = cls.__new__(cls)
        self.model, self.batch = str(path), in_shape[0]
        h = c_vp()
        if lib.vknn_session_create_onnx(str(path).encode(), options.encode(), ctypes.byref(h)):
            raise VkhipError("session create: " + lib.vknn_last_error().decode(errors='replace'))
        self.h = h.value
        self.in_shape, self.out_elems = list(in_shape), list(out_elems)
        return self

    def save_optimized(self, path):
        if vknn().vknn_session_save_optimized(self.h, str(path).encode()):
            raise VkhipError(vknn().vknn_last_error().decode(errors='replace'))

    def run(self, x):
        lib = vknn()
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.empty(sum(self.out_elems), np.float32)
        if lib.vknn_session_run_host(self.h, x.ctypes.data, x.size, y.ctypes.data, y.size):
            raise VkhipError("run: " + lib.vknn_last_error().decode(errors='replace'))
        return y

    def bind_device_input(self, ptr):
        if vknn().vknn_session_bind_device_input(self.h, ptr):
            raise VkhipError(vknn().vknn_last_error().decode(errors='replace'))

    def bind_device_input_as(self, ptr, fmt, f16):
        """Device input in a declared layout (0 NCHW, 1 NHWC, 2 NC4HW4) and type (fp16 if f16)."""
        if vknn().vknn_session_bind_device_input_as(self.h, ptr, fmt, int(f16)):
            raise VkhipError(vknn().vknn_last_error().decode(errors='replace'))

    def run_device(self):
        if vknn().vknn_session_run_device(self.h):
            raise VkhipError(vknn().vknn_last_error().decode(errors='replace'))

    def sync(self):
        if vknn().vknn_session_sync(self.h):
            raise VkhipError(vknn().vknn_last_error().decode(errors='replace'))

    def read_outputs(self):
        y = np.empty(sum(self.out_elems), np.float32)
        if vknn().vknn_session_read_outputs(self.h, y.ctypes.data, y.size):
            raise VkhipError(vknn().vknn_last_error().decode(errors='replace'))
        return y

    @property
    def stream(self):
        return vknn().vknn_session_stream(self.h)

    def profile(self):
        import json
        buf = ctypes.create_string_buffer(1 << 22)
        vknn().vknn_session_profile_json(self.h, buf, len(buf))
        return json.loads(buf.value.decode() or "[]")

    def describe(self):
        buf = ctypes.create_string_buffer(1 << 20)
        vknn().vknn_session_describe(self.h, buf, len(buf))
        return buf.value.decode()

    def segments(self):
        """[(backend, nodes, inputs, outputs)] per segment, in run order."""
        out = []
        for ln in _text(vknn().vknn_session_segments, self.h).splitlines():
            be, rest = ln.split(" nodes=")
            n, rest = rest.split(" in=")
            ins, outs = rest.split(" out=")
            out.append((be, int(n), [t for t in ins.split(",") if t], [t for t in outs.split(",") if t]))
        return out

    def count_ops(self, op):
        return vknn().vknn_session_count_ops(self.h, op.encode())

    def close(self):
        if getattr(self, "h", None):
            vknn().vknn_session_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def model_io(model, batch):
    in4 = (c_i64 * 4)()
    outs = (c_i64 * 16)()
    n = c_i32()
    if vknn().vknn_model_io(model.encode(), batch, in4, outs, ctypes.byref(n), 16):
        raise VkhipError(vknn().vknn_last_error().decode(errors='replace'))
    return list(in4), list(outs)[:n.value]


def _text(fn, *args, cap=1 << 24):
    buf = ctypes.create_string_buffer(cap)
    if fn(*args, buf, len(buf)):
        raise VkhipError(vknn().vknn_last_error().decode(errors='replace'))
    out = buf.value.decode(errors='replace')  # names come from the model file and need not be UTF-8
    if len(buf.value) >= cap - 1:
        raise VkhipError("text output larger than %d bytes" % cap)
    return out


def onnx_describe(path):
    """The graph an ONNX file imports to, before any pass, in full text form (host only)."""
    return _text(vknn().vknn_onnx_describe, str(path).encode())


def onnx_after_passes(path, options=""):
    """Node list of an imported ONNX model after the standard passes (host only)."""
    return _text(vknn().vknn_onnx_after_passes, str(path).encode(), options.encode())


def graph_after_passes(model, batch=1, options=""):
    """Node list of a zoo model after the standard passes (host only, no device needed)."""
    buf = ctypes.create_string_buffer(1 << 20)
    if vknn().vknn_graph_after_passes(model.encode(), batch, options.encode(), buf, len(buf)):
        raise VkhipError(vknn().vknn_last_error().decode(errors='replace'))
    return buf.value.decode()
