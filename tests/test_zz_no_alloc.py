"""vkhip_conv_forward_noalloc (the allocation-free variant of vkhip_conv_forward) against
vkhip_conv_forward with a caller-allocated workspace, through the C ABI: identical plans run the
same kernels, so the outputs must agree bit for bit. Two calls in a row on each plan family, the
second on a smaller input, so the shared scratch is reused with stale contents from the first
(split-K with the in-kernel reduction keeps its arrival counters apart from the scratch)."""
import ctypes

import numpy as np
import pytest

import vknn_amd as V
from vknn_amd import DeviceBuffer, check
from tests.gpu_helpers import conv_desc, round_half, to_device_nc4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return V.require_gpu()


def _run_both(lib, x, w, b, algo, ksplit=0, pads=(0, 0, 0, 0), res=None):
    d, yshape = conv_desc(x.shape, w.shape, pads=pads, act=1,
                          has_res=int(res is not None))
    plan = V.ConvPlan()
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), algo, -1, ksplit, ctypes.byref(plan)), "plan")
    assert plan.algo == algo and plan.workspace_bytes > 0
    blob = np.zeros(plan.weight_bytes, np.uint8)
    check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, b.ctypes.data, blob.ctypes.data), "pack")
    dblob = DeviceBuffer.from_array(blob)
    dx = to_device_nc4(x)
    dres = to_device_nc4(res) if res is not None else None
    nbytes = V.nc4_elems(*yshape) * 2
    y_ref, y_new = DeviceBuffer(nbytes), DeviceBuffer(nbytes)
    y_ref.zero()
    y_new.zero()
    ws = DeviceBuffer(plan.workspace_bytes)
    ws.zero()  # SPLITK_LAST keeps arrival counters in it that start at zero
    check(lib.vkhip_conv_forward(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr, dres.ptr if dres else None, y_ref.ptr,
                                 ws.ptr, None), "conv_forward")
    check(lib.vkhip_conv_forward_noalloc(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr, dres.ptr if dres else None,
                                         y_new.ptr, None), "conv_forward_noalloc")
    check(lib.vkhip_stream_sync(None), "sync")
    a = y_ref.download(np.uint16, nbytes // 2)
    n = y_new.download(np.uint16, nbytes // 2)
    return a, n, plan


@pytest.mark.parametrize("algo", [V.CONV_SPLITK, V.CONV_SPLITK_LAST])
@pytest.mark.parametrize("shapes", [[(4, 512, 7, 7, 256), (2, 256, 7, 7, 128)], [(1, 2048, 7, 7, 512), (1, 1024, 5, 5, 96)]])
def test_noalloc_splitk_matches_workspace_path(lib, shapes, algo):
    for i, (N, C, H, W, Co) in enumerate(shapes):
        r = np.random.default_rng(300 + i + C)
        x = round_half(r.standard_normal((N, C, H, W)))
        w = (r.standard_normal((Co, C, 1, 1)) * 0.05).astype(np.float32)
        b = (r.standard_normal(Co) * 0.1).astype(np.float32)
        res = round_half(r.standard_normal((N, Co, H, W)))
        a, n, plan = _run_both(lib, x, w, b, algo, ksplit=4, res=res)
        print(f"split-K (algo {algo}) call {i} {(N, C, H, W, Co)} ksplit={plan.ksplit} workspace={plan.workspace_bytes}", flush=True)
        assert np.array_equal(a, n), f"call {i}: {np.count_nonzero(a != n)} of {a.size} fp16 values differ"


@pytest.mark.parametrize("shapes", [[(2, 128, 14, 14, 128), (1, 64, 9, 11, 72)]])
def test_noalloc_winograd_matches_workspace_path(lib, shapes):
    for i, (N, C, H, W, Co) in enumerate(shapes):
        r = np.random.default_rng(400 + i + C)
        x = round_half(r.standard_normal((N, C, H, W)))
        w = (r.standard_normal((Co, C, 3, 3)) * 0.05).astype(np.float32)
        b = (r.standard_normal(Co) * 0.1).astype(np.float32)
        a, n, plan = _run_both(lib, x, w, b, V.CONV_WINOGRAD, pads=(1, 1, 1, 1))
        print(f"winograd call {i} {(N, C, H, W, Co)} workspace={plan.workspace_bytes}", flush=True)
        assert np.array_equal(a, n), f"call {i}: {np.count_nonzero(a != n)} of {a.size} fp16 values differ"


def test_noalloc_rejects_oversized_workspace(lib):
    """A plan whose workspace exceeds the scratch is refused before anything runs."""
    d, _ = conv_desc((64, 64, 56, 56), (64, 64, 3, 3), pads=(1, 1, 1, 1))
    plan = V.ConvPlan()
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_WINOGRAD, -1, 0, ctypes.byref(plan)), "plan")
    assert plan.workspace_bytes > (64 << 20)
    rc = lib.vkhip_conv_forward_noalloc(ctypes.byref(d), ctypes.byref(plan), None, None, None, None, None)
    assert rc == 1 and b"scratch" in lib.vkhip_last_error()
