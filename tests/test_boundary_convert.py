"""Layout + dtype conversion at the boundary (row A4): NC4HW4 <-> flat (reference
shaders/convert_layout.comp, ops/convert_layout.cpp) and the declared-format converter
(shaders/boundary_convert.comp, ops/boundary_convert.cpp; fp32 -> fp16 rounds to nearest even
there, unlike the host codec).

CPU tests pin the oracle: its RNE conversion against numpy's IEEE float16 cast (exhaustive over
the rounding boundaries), its layouts against numpy reshape/transpose constructions. GPU tests
compare vkhip_boundary_convert / vkhip_convert_layout with the oracle bit for bit."""
import ctypes

import numpy as np
import pytest

import vknn_amd as V
from tests.oracle_lib import oracle

FMTS = {0: "NCHW", 1: "NHWC", 2: "NC4HW4"}
SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -np.inf, np.inf, 6.1035156e-05, 6.0975552e-05,
                    5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1.00048828125, 1.00146484375, 2049.0, 2051.0, 0.1], np.float32)


def rne_oracle(x):
    o = oracle()
    return np.array([o.oracle_float_to_half_rne(float(v)) for v in x.ravel()], np.uint16)


def test_rne_matches_ieee_float16_on_rounding_boundaries():
    """Every sign/exponent/high-mantissa pattern with low 13 bits on a rounding boundary
    (2^19 * 6 inputs, NaN patterns excluded): oracle == numpy float16 cast bit for bit."""
    hi = np.arange(1 << 19, dtype=np.uint32) << 13
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF], np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    x = bits.view(np.float32)
    keep = ~np.isnan(x)
    x = np.ascontiguousarray(x[keep])
    lib = oracle()
    # vectorised through the boundary converter (fp32 NCHW -> fp16 NCHW is the element-wise cast)
    got = np.zeros(x.size, np.uint16)
    lib.oracle_boundary_convert(x.ctypes.data, 0, 0, got.ctypes.data, 0, 1, 1, 1, 1, x.size)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(x.view(np.uint32)[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]


def test_rne_nan_stays_nan():
    for bits in (0x7FC00000, 0xFFC00001, 0x7F800001, 0x7FBFFFFF):
        v = np.array([bits], np.uint32).view(np.float32)[0]
        h = np.array([oracle().oracle_float_to_half_rne(float(v))], np.uint16).view(np.float16)[0]
        assert np.isnan(h)


def to_fmt(x, fmt):
    """numpy construction of a layout from logical NCHW (NC4HW4: pad C to 4, split c = 4cb + l)."""
    N, C, H, W = x.shape
    if fmt == 0:
        return x.copy()
    if fmt == 1:
        return np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    Cp = (C + 3) // 4 * 4
    xp = np.zeros((N, Cp, H, W), x.dtype)
    xp[:, :C] = x
    return np.ascontiguousarray(xp.reshape(N, Cp // 4, 4, H, W).transpose(0, 1, 3, 4, 2))


@pytest.mark.parametrize("sf", [0, 1, 2])
@pytest.mark.parametrize("df", [0, 1, 2])
@pytest.mark.parametrize("s16,d16", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_oracle_layouts_match_numpy(sf, df, s16, d16):
    N, C, H, W = 2, 5, 3, 4
    x = np.random.default_rng(sf * 9 + df).standard_normal((N, C, H, W)).astype(np.float32) * 100
    x16 = x.astype(np.float16)
    src = to_fmt(x16.view(np.uint16) if s16 else x, sf)
    dst = np.zeros(to_fmt(x, df).size, np.uint16 if d16 else np.float32)
    oracle().oracle_boundary_convert(src.ctypes.data, sf, s16, dst.ctypes.data, df, d16, N, C, H, W)
    logical = x16.astype(np.float32) if s16 else x
    want = to_fmt(logical.astype(np.float16).view(np.uint16) if d16 else logical, df).ravel()
    assert np.array_equal(dst.view(np.uint16 if d16 else np.uint32), want.view(np.uint16 if d16 else np.uint32))


def dev(a):
    return V.DeviceBuffer.from_array(np.ascontiguousarray(a))


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(2, 5, 3, 4), (1, 3, 7, 9), (3, 8, 2, 2), (1, 67, 5, 6)])
@pytest.mark.parametrize("s16,d16", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_boundary_convert_matches_oracle(gpu, shape, s16, d16):
    lib = V.vkhip()
    N, C, H, W = shape
    rng = np.random.default_rng(C * 7 + W)
    x = (rng.standard_normal(shape) * 300).astype(np.float32)
    flat = x.ravel()
    flat[:min(flat.size, SPECIAL.size)] = SPECIAL[:min(flat.size, SPECIAL.size)]
    for sf in FMTS:
        for df in FMTS:
            with np.errstate(over="ignore"):
                src = to_fmt(x.astype(np.float16).view(np.uint16) if s16 else x, sf)
            n_out = to_fmt(x, df).size
            want = np.zeros(n_out, np.uint16 if d16 else np.float32)
            oracle().oracle_boundary_convert(src.ctypes.data, sf, s16, want.ctypes.data, df, d16, N, C, H, W)
            ds = dev(src)
            dd = V.DeviceBuffer(n_out * (2 if d16 else 4))
            V.check(lib.vkhip_boundary_convert(ds.ptr, sf, s16, dd.ptr, df, d16, N, C, H, W, None))
            V.check(lib.vkhip_stream_sync(None))
            got = dd.download(np.uint16 if d16 else np.float32, n_out)
            assert np.array_equal(got.view(np.uint16 if d16 else np.uint32), want.view(np.uint16 if d16 else np.uint32)), (FMTS[sf], FMTS[df])


@pytest.mark.gpu
@pytest.mark.parametrize("elem", [2, 4])
def test_convert_layout_roundtrip(gpu, elem):
    """NC4HW4 -> flat -> NC4HW4 is the identity (padding lanes zero) and flat matches numpy."""
    lib = V.vkhip()
    N, C, H, W = 2, 6, 5, 3
    x = np.random.default_rng(5).standard_normal((N, C, H, W)).astype(np.float32)
    xs = x.astype(np.float16).view(np.uint16) if elem == 2 else x
    nc4 = to_fmt(xs, 2)
    d0 = dev(nc4)
    d1 = V.DeviceBuffer(xs.size * elem)
    d2 = V.DeviceBuffer(nc4.size * elem)
    V.check(lib.vkhip_convert_layout(d0.ptr, d1.ptr, N, C, H, W, 0, elem, None))
    V.check(lib.vkhip_convert_layout(d1.ptr, d2.ptr, N, C, H, W, 1, elem, None))
    V.check(lib.vkhip_stream_sync(None))
    dt = np.uint16 if elem == 2 else np.uint32
    assert np.array_equal(d1.download(dt, xs.size), xs.view(dt).ravel())
    assert np.array_equal(d2.download(dt, nc4.size), nc4.view(dt).ravel())
    assert lib.vkhip_convert_layout(d0.ptr, d1.ptr, N, C, H, W, 2, elem, None) != 0
