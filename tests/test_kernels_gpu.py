"""Kernel-level parity of the HIP path against the CPU oracle, through the vkhip C ABI.

Bar (north star): pack/unpack/layout bit-exact; fp16 conv outputs max|d|/max|ref| <= 2e-2 and
cosine >= 0.9999 against the oracle on the same seeded inputs (the oracle sees the fp16-rounded
input the kernel sees; weights stay fp32 in the oracle, fp16 on the device).
"""
import ctypes

import numpy as np
import pytest

import vknn_amd as V
from tests.gpu_helpers import (DeviceBuffer, check, conv_desc, from_device_nc4, gpu_conv, raw_nc4, round_half,
                               to_device_nc4)
from tests.oracle_lib import (oracle, oracle_conv, oracle_dwpw, oracle_pack, oracle_unpack, parity)

pytestmark = pytest.mark.gpu

REL_TOL, COS_TOL = 2e-2, 0.9999


def assert_parity(got, ref, what=""):
    rel, cos = parity(got, ref)
    print(f"{what}: max_rel={rel:.2e} cos={cos:.7f}", flush=True)
    assert rel <= REL_TOL and cos >= COS_TOL, (what, rel, cos)


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- pack / unpack (bit-exact)
EDGE = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e9, -1e9, np.inf, -np.inf, np.nan,
                 6.1035156e-05, 6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-10, -3e-8,
                 1.00048828125, 1.0009765625, 1.00146484375, 2049.0, 2051.0, 0.1, 1.0 / 3.0], np.float32)


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (1, 3, 5, 7), (2, 5, 3, 3), (2, 6, 4, 9), (1, 7, 11, 2),
                                   (3, 64, 14, 14), (1, 3, 224, 224), (2, 5, 2, 2), (3, 1, 8, 6), (4, 8, 1, 1),
                                   (3, 10, 1, 1), (2, 1000, 1, 1)])
def test_pack_bitexact(gpu, shape):
    x = rng(1).standard_normal(shape).astype(np.float32) * 300
    flat = x.ravel()
    flat[:min(flat.size, EDGE.size)] = EDGE[:min(flat.size, EDGE.size)]
    buf = to_device_nc4(x)
    got = raw_nc4(buf, shape)
    want = oracle_pack(x)
    nan = np.isnan(x).any()
    assert np.array_equal(got, want), f"pack mismatch at {np.nonzero(got != want)[0][:10]} (nan={nan})"
    back = from_device_nc4(buf, shape)
    assert np.array_equal(back.view(np.uint32), oracle_unpack(want, shape).view(np.uint32))


def test_pack_exhaustive_rounding_boundaries(gpu):
    """Every fp32 bit pattern whose low 13 bits sit on a rounding boundary, for all sign/exponent/
    high-mantissa values (2^19 * 6 inputs): device pack == oracle codec bit for bit."""
    hi = np.arange(1 << 19, dtype=np.uint32) << 13
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF], np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    x = bits.view(np.float32).reshape(1, 1, 1, -1)
    x4 = np.zeros((1, 4, 1, x.shape[-1]), np.float32)
    x4[0, 0] = x[0, 0]
    buf = to_device_nc4(x4)
    got = raw_nc4(buf, x4.shape).reshape(-1, 4)[:, 0]
    want = np.zeros(bits.size, np.uint16)
    oracle().oracle_float_to_half_n(x.ctypes.data, want.ctypes.data, bits.size)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(bits[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]


def test_unpack_multi(gpu):
    """Several tensors unpacked by one vkhip_unpack_nchw_f32_multi call: the same bits as one
    vkhip_unpack_nchw_f32 per tensor, for quad-path tensors (grouped, more than 8 of them) and for
    one whose H*W is not a multiple of 4 (handled on its own)."""
    lib = V.vkhip()
    r = rng(1900)
    shapes = [(2, 144, 8, 8), (2, 144, 4, 4), (2, 144, 2, 2), (1, 7, 6, 6), (3, 5, 3, 3)] + [(1, 12, 4, 4)] * 6
    xs = [round_half(r.standard_normal(sh)) for sh in shapes]
    dxs = [to_device_nc4(x) for x in xs]
    outs = [DeviceBuffer(int(np.prod(sh)) * 4) for sh in shapes]
    srcs = (ctypes.c_void_p * len(shapes))(*[d.ptr for d in dxs])
    dsts = (ctypes.c_void_p * len(shapes))(*[o.ptr for o in outs])
    sh = (ctypes.c_int64 * (4 * len(shapes)))(*[v for s_ in shapes for v in s_])
    check(lib.vkhip_unpack_nchw_f32_multi(srcs, dsts, sh, len(shapes), None), "unpack multi")
    check(lib.vkhip_stream_sync(None), "sync")
    for x, sh_, o in zip(xs, shapes, outs):
        assert np.array_equal(o.download(np.float32, int(np.prod(sh_))).reshape(sh_), x)


def test_flat_pack_unpack(gpu):
    x = rng(2).standard_normal(1003).astype(np.float32) * 1000
    src = DeviceBuffer.from_array(x)
    dst = DeviceBuffer(x.size * 2)
    check(V.vkhip().vkhip_pack_flat_f32(src.ptr, dst.ptr, x.size, None))
    check(V.vkhip().vkhip_stream_sync(None))
    got = dst.download(np.uint16, x.size)
    want = np.zeros(x.size, np.uint16)
    oracle().oracle_float_to_half_n(x.ctypes.data, want.ctypes.data, x.size)
    assert np.array_equal(got, want)
    back = DeviceBuffer(x.size * 4)
    check(V.vkhip().vkhip_unpack_flat_f32(dst.ptr, back.ptr, x.size, None))
    check(V.vkhip().vkhip_stream_sync(None))
    ref = np.zeros(x.size, np.float32)
    oracle().oracle_half_to_float_n(want.ctypes.data, ref.ctypes.data, x.size)
    assert np.array_equal(back.download(np.float32, x.size), ref)


# ---------------------------------------------------------------- dense conv (implicit GEMM on MFMA)
# (N, Cin, H, W, Cout, K, stride, pad, act, residual)
CONV_CASES = [
    (1, 64, 56, 56, 64, 3, 1, 1, 1, False),     # config 0 shape
    (1, 24, 56, 56, 144, 1, 1, 0, 2, False),    # MNv2 expand
    (2, 144, 14, 14, 24, 1, 1, 0, 0, True),     # MNv2 project + residual
    (2, 64, 28, 28, 256, 1, 1, 0, 1, True),     # ResNet 1x1 + residual + relu
    (2, 256, 14, 14, 512, 1, 2, 0, 0, False),   # ResNet downsample 1x1 s2
    (2, 128, 28, 28, 128, 3, 2, 1, 1, False),   # ResNet v1.5 3x3 s2
    (1, 3, 64, 64, 64, 7, 2, 3, 1, False),      # stem 7x7 s2 (Cin=3)
    (1, 3, 32, 32, 16, 3, 2, 1, 4, False),      # MNv3 stem, HardSwish
    (2, 16, 20, 20, 32, 3, 1, 1, 5, False),     # YOLO 3x3 SiLU
    (1, 40, 9, 9, 20, 3, 1, 1, 3, False),       # clip act, ragged channels
    (1, 5, 7, 7, 7, 3, 1, 1, 0, False),         # odd everything
    (1, 512, 7, 7, 2048, 1, 1, 0, 1, True),     # deep 1x1 at 7x7
]


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: "x".join(map(str, c[:6])) + f"s{c[6]}a{c[8]}r{int(c[9])}")
def test_conv_auto(gpu, case):
    N, C, H, W, Cout, K, s, p, act, has_res = case
    r = rng(hash(case) & 0xFFFF)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, K, K)) * np.sqrt(2.0 / (C * K * K))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    OH = (H + 2 * p - K) // s + 1
    res = round_half(r.standard_normal((N, Cout, OH, OH))) if has_res else None
    lo, hi = (-0.5, 0.7) if act == 3 else (0.0, 0.0)
    got, plan, _ = gpu_conv(x, w, b, (s, s), (p, p, p, p), act=act, lo=lo, hi=hi, res=res)
    ref = oracle_conv(x, w, b, (s, s), (p, p, p, p), res=res, act=act, lo=lo, hi=hi)
    assert_parity(got, ref, f"conv {case} algo={plan.algo} tile={plan.tile}")


NUM_TILES = V.vkhip().vkhip_conv_tile_count()
BD_TILES = [8, 9, 10]            # conv_bd_kernel tiles (A via LDS DMA, B gathered into registers)
PERS_TILES = [36, 37, 38, 39, 40, 41, 42]  # conv_dma_persist_kernel tiles (conv_dma_kernel's tiles, one workgroup walks many)
LE_TILES = [46, 47, 48, 49]                # conv_dma_kernel with the LDS-staged epilogue (even pixel count per image)
DMA_TILES = [11, 12, 13, 14, 15, 16, 24, 25, 28, 29, 30, 31] + PERS_TILES  # dense-B tiles (A and B via LDS DMA)
HALO_TILES = [17, 18, 19, 20, 26, 27, 32, 33, 34, 35]      # conv_halo_kernel tiles (3x3 s1 p1: input band staged once for all taps)
STEM_TILES = [21, 22, 23]                 # conv_stem_kernel tiles (3x3/7x7 over at most 4 input channels)
THIN_TILES = [43, 44, 45]                 # conv_thin_kernel tiles (<= 32 input, 16/32/64 output channels)
GATHER_TILES = [t for t in range(NUM_TILES) if t not in DMA_TILES + HALO_TILES + STEM_TILES + THIN_TILES + LE_TILES]


@pytest.mark.parametrize("tile", GATHER_TILES)
def test_conv_every_tile(gpu, tile):
    r = rng(10 + tile)
    x = round_half(r.standard_normal((2, 48, 17, 19)))
    w = (r.standard_normal((72, 48, 3, 3)) * 0.1).astype(np.float32)
    b = (r.standard_normal(72) * 0.1).astype(np.float32)
    got, _, _ = gpu_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1, algo=V.CONV_GEMM, tile=tile)
    ref = oracle_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1)
    assert_parity(got, ref, f"tile {tile}")


@pytest.mark.parametrize("tile", [0, 3, 6] + BD_TILES)
def test_conv_every_tile_1x1_aligned(gpu, tile):
    r = rng(20 + tile)
    x = round_half(r.standard_normal((3, 64, 9, 9)))
    w = (r.standard_normal((96, 64, 1, 1)) * 0.1).astype(np.float32)
    got, _, _ = gpu_conv(x, w, None, act=0, algo=V.CONV_GEMM, tile=tile)
    assert_parity(got, oracle_conv(x, w), f"1x1 tile {tile}")


@pytest.mark.parametrize("tile", BD_TILES)
def test_conv_bd_general_gather_residual(gpu, tile):
    """Channel counts that are not a multiple of 16 (per-slot tap decode), stride 2, a K tail,
    ragged output channels and pixels, residual + ReLU6 epilogue."""
    r = rng(40 + tile)
    x = round_half(r.standard_normal((3, 22, 13, 11)))
    w = (r.standard_normal((70, 22, 3, 3)) * 0.1).astype(np.float32)
    b = (r.standard_normal(70) * 0.1).astype(np.float32)
    res = round_half(r.standard_normal((3, 70, 7, 6)))
    got, plan, _ = gpu_conv(x, w, b, (2, 2), (1, 1, 1, 1), act=2, res=res, algo=V.CONV_GEMM, tile=tile)
    ref = oracle_conv(x, w, b, (2, 2), (1, 1, 1, 1), res=res, act=2)
    assert_parity(got, ref, f"bd general tile {tile}")


@pytest.mark.parametrize("tile", DMA_TILES)
@pytest.mark.parametrize("shape", [(3, 72, 6, 10, 70), (2, 256, 14, 14, 300), (1, 24, 8, 8, 8), (3, 72, 7, 7, 70),
                                   (5, 64, 5, 9, 40)])
def test_conv_dma_1x1(gpu, tile, shape):
    """Dense-B kernel: K tail (Cin not a multiple of 64), ragged output channels, pixel tiles
    crossing image boundaries and the end of the batch, odd pixel counts per image (one padding
    column per image), residual + ReLU epilogue."""
    N, C, H, W, Cout = shape
    r = rng(80 + tile + C)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, 1, 1)) * 0.1).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    res = round_half(r.standard_normal((N, Cout, H, W)))
    got, plan, _ = gpu_conv(x, w, b, act=1, res=res, algo=V.CONV_GEMM, tile=tile)
    assert plan.tile == tile
    assert_parity(got, oracle_conv(x, w, b, res=res, act=1), f"dma 1x1 tile {tile} {shape}")


@pytest.mark.parametrize("shape", [(2, 16, 20, 24, 16, 3, 1), (2, 16, 20, 24, 32, 3, 2), (1, 3, 32, 34, 16, 3, 2), (2, 32, 18, 18, 32, 3, 1),
                                   (2, 32, 16, 16, 64, 1, 1), (3, 24, 10, 14, 24, 3, 1), (2, 16, 30, 150, 16, 3, 1), (2, 5, 16, 16, 40, 3, 2),
                                   (1, 8, 9, 130, 12, 3, 2), (2, 12, 7, 6, 64, 3, 1), (1, 32, 12, 12, 20, 3, 2),
                                   (2, 3, 224, 224, 64, 7, 2), (1, 3, 30, 34, 40, 7, 2), (3, 4, 18, 20, 16, 7, 2), (1, 1, 9, 136, 64, 7, 2)])
@pytest.mark.parametrize("act", [1, 5])
def test_conv_thin(gpu, shape, act):
    """Thin-channel kernel (16x16x32 MFMA, weights in registers, double-buffered input bands):
    every tile that takes the shape, against the oracle. Ragged channel counts (Cin 3, 5, 12, 24:
    zero slots of the rounded reduction), column blocks cut by the image edge, bands above and
    below the image, stride 2, 1x1, the 7x7 stride-2 stem over 1-4 channels, ReLU and SiLU
    epilogues."""
    N, C, H, W, Cout, K, S = shape
    r = rng(900 + C + H + Cout + K * S)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, K, K)) * np.sqrt(2.0 / (K * K * C))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    p = K // 2
    ref = oracle_conv(x, w, b, (S, S), (p, p, p, p), act=act)
    ran = 0
    lib = V.vkhip()
    for tile in THIN_TILES:
        d, _ = conv_desc(x.shape, w.shape, (S, S), (p, p, p, p), act=act)
        if lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, tile, 0, ctypes.byref(V.ConvPlan())) != 0:
            assert Cout > {43: 16, 44: 32, 45: 64}[tile] or (C > 16 and tile == 45), (tile, shape)  # not instantiated: weights over budget
            continue
        got, plan, _ = gpu_conv(x, w, b, (S, S), (p, p, p, p), act=act, algo=V.CONV_GEMM, tile=tile)
        assert plan.tile == tile
        assert_parity(got, ref, f"thin tile {tile} {shape} act {act}")
        ran += 1
    assert ran > 0


def test_conv_thin_refuses_other_shapes(gpu):
    """Thin tiles refuse residuals except on 3x3 stride 1, odd input widths, 5x5, dilation, grouped convs, too many
    channels and split-K / Winograd plans."""
    lib = V.vkhip()
    plan = V.ConvPlan()
    bad = [dict(x=(1, 16, 8, 8), w=(16, 16, 1, 1), pads=(0, 0, 0, 0), has_res=1), dict(x=(1, 16, 8, 9), w=(16, 16, 3, 3), pads=(1, 1, 1, 1)),
           dict(x=(1, 16, 8, 8), w=(16, 16, 5, 5), pads=(2, 2, 2, 2)), dict(x=(1, 16, 8, 8), w=(16, 16, 3, 3), pads=(2, 2, 2, 2), dil=(2, 2)),
           dict(x=(1, 40, 8, 8), w=(16, 40, 3, 3), pads=(1, 1, 1, 1)), dict(x=(1, 16, 8, 8), w=(80, 16, 3, 3), pads=(1, 1, 1, 1))]
    for c in bad:
        d, _ = conv_desc(c["x"], c["w"], pads=c["pads"], dil=c.get("dil", (1, 1)), has_res=c.get("has_res", 0))
        for t in THIN_TILES:
            assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, t, 0, ctypes.byref(plan)) != 0, (c, t)
    d, _ = conv_desc((1, 16, 8, 8), (16, 16, 3, 3), pads=(1, 1, 1, 1))
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, 43, 0, ctypes.byref(plan)) == 0
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_SPLITK, 43, 2, ctypes.byref(plan)) != 0
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_WINOGRAD, 43, 0, ctypes.byref(plan)) != 0


# (algo, tile, ksplit, kernel size): one or two tiles of every kernel family that takes a residual
RES_POST_CASES = [(V.CONV_GEMM, t, 0, 3) for t in (0, 3, 8, 10, 26, 33, 43, 44, 45)] + \
                 [(V.CONV_GEMM, t, 0, 1) for t in (14, 24, 38, 47)] + \
                 [(V.CONV_SPLITK, 3, 2, 3), (V.CONV_SPLITK_LAST, 26, 2, 3)]


@pytest.mark.parametrize("has_res", [1, 2])
@pytest.mark.parametrize("case", RES_POST_CASES)
def test_conv_residual_after_activation(gpu, case, has_res):
    """has_res 2: y = act(conv + bias) + res (a conv followed by a standalone Add, the YOLOv8
    bottleneck shortcut), against the oracle conv then the oracle's fp16 add; has_res 1 (residual
    before the activation) on the same tiles, which covers the thin kernel's residual path. Ragged
    output channels, column blocks cut by the image edge."""
    algo, tile, ks, k = case
    r = rng(1300 + tile * 3 + k + has_res)
    N, C, H, W, Cout = (2, 32, 11, 36, 40) if k == 3 else (3, 64, 10, 12, 70)
    if tile in THIN_TILES:
        Cout = {43: 16, 44: 28, 45: 60}[tile]
        C = 16 if tile == 45 else C  # 64 outputs over 32 inputs exceed the weight register budget
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, k, k)) * np.sqrt(2.0 / (k * k * C))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    p = k // 2
    res = round_half(r.standard_normal((N, Cout, H, W)))
    d, _ = conv_desc(x.shape, w.shape, (1, 1), (p,) * 4, act=5, has_res=has_res)
    plan = V.ConvPlan()
    check(V.vkhip().vkhip_conv_plan_make(ctypes.byref(d), algo, tile, ks, ctypes.byref(plan)), f"plan {case}")
    if has_res == 2:
        ref = round_half(oracle_conv(x, w, b, (1, 1), (p,) * 4, act=5)) + res
        got, plan, _ = gpu_conv(x, w, b, (1, 1), (p,) * 4, act=5, res=res, algo=algo, tile=tile, ksplit=ks, res_post=True)
    else:
        ref = oracle_conv(x, w, b, (1, 1), (p,) * 4, res=res, act=5)
        got, plan, _ = gpu_conv(x, w, b, (1, 1), (p,) * 4, act=5, res=res, algo=algo, tile=tile, ksplit=ks)
    assert plan.algo == algo and plan.tile == tile
    assert_parity(got, ref, f"residual mode {has_res} algo {algo} tile {tile}")


def test_conv_residual_after_activation_refusals(gpu):
    """Winograd, depthwise and stem plans have no residual-after-activation epilogue; has_res
    outside 0..2 is an error."""
    lib = V.vkhip()
    plan = V.ConvPlan()
    d, _ = conv_desc((1, 64, 14, 14), (64, 64, 3, 3), pads=(1, 1, 1, 1), act=5, has_res=2)
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_WINOGRAD, -1, 0, ctypes.byref(plan)) != 0
    d, _ = conv_desc((1, 16, 14, 14), (16, 1, 3, 3), pads=(1, 1, 1, 1), group=16, act=5, has_res=2)
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_DEPTHWISE, -1, 0, ctypes.byref(plan)) != 0
    d, _ = conv_desc((1, 3, 32, 32), (16, 3, 3, 3), pads=(1, 1, 1, 1), act=5, has_res=2)
    for t in STEM_TILES:
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, t, 0, ctypes.byref(plan)) != 0
    d, _ = conv_desc((1, 16, 8, 8), (16, 16, 3, 3), pads=(1, 1, 1, 1), has_res=3)
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, 43, 0, ctypes.byref(plan)) != 0


@pytest.mark.parametrize("tile", [43, 33, 3])
def test_conv_view_residual(gpu, tile):
    """vkhip_conv_forward_view_res as in a YOLOv8 C2f block: the residual is one channel slice of a
    wide tensor and the output another slice of the same tensor (both at its plane stride), the
    input a third slice; y = SiLU(conv(x)) + res. The other slices stay untouched."""
    lib = V.vkhip()
    r = rng(1400 + tile)
    N, H, W, C = 2, 12, 40, 16
    wide = round_half(r.standard_normal((N, 4 * C, H, W)))  # slices: [x | res | y | spare]
    x, res = wide[:, 0:C], wide[:, C:2 * C]
    w = (r.standard_normal((C, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b = (r.standard_normal(C) * 0.1).astype(np.float32)
    d, _ = conv_desc(x.shape, w.shape, (1, 1), (1, 1, 1, 1), act=5, has_res=2)
    plan = V.ConvPlan()
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, tile, 0, ctypes.byref(plan)), "plan")
    blob = np.zeros(plan.weight_bytes, np.uint8)
    check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, b.ctypes.data, blob.ctypes.data), "pack")
    dblob, dwide = DeviceBuffer.from_array(blob), to_device_nc4(wide)
    ws = DeviceBuffer(plan.workspace_bytes) if plan.workspace_bytes else None
    plane = H * W * 8  # bytes of one 4-channel plane
    cb, ps = C // 4, 4 * C // 4
    check(lib.vkhip_conv_forward_view_res(ctypes.byref(d), ctypes.byref(plan), dwide.ptr, ps, dblob.ptr, dwide.ptr + cb * plane,
                                          dwide.ptr + 2 * cb * plane, ps, ws.ptr if ws else None, None), "forward_view_res")
    check(lib.vkhip_stream_sync(None), "sync")
    out = from_device_nc4(dwide, wide.shape)
    ref = round_half(oracle_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=5)) + res
    assert_parity(out[:, 2 * C:3 * C], ref, f"view residual tile {tile}")
    for sl in (slice(0, C), slice(C, 2 * C), slice(3 * C, 4 * C)):
        assert np.array_equal(out[:, sl], wide[:, sl])
    # the plain view entry refuses a residual descriptor
    assert lib.vkhip_conv_forward_view(ctypes.byref(d), ctypes.byref(plan), dwide.ptr, ps, dblob.ptr, dwide.ptr, ps, None, None) != 0


def gpu_conv_pair(x, w1, b1, w2, b2, act, res, wide=None):
    """vkhip_conv3x3_pair_forward on x (or, with wide = (Cw, in_off, out_off), on a channel slice of a
    wider tensor holding x at channel in_off, the output written at channel out_off)."""
    lib = V.vkhip()
    N, C, H, W = x.shape
    d1, _ = conv_desc(x.shape, w1.shape, (1, 1), (1, 1, 1, 1), act=act)
    d2, yshape = conv_desc(x.shape, w2.shape, (1, 1), (1, 1, 1, 1), act=act, has_res=2 if res else 0)
    p1, p2 = V.ConvPlan(), V.ConvPlan()
    check(lib.vkhip_conv3x3_pair_plan(ctypes.byref(d1), ctypes.byref(d2), ctypes.byref(p1), ctypes.byref(p2)), "pair plan")
    blobs = []
    for d, p, w, b in ((d1, p1, w1, b1), (d2, p2, w2, b2)):
        blob = np.zeros(p.weight_bytes, np.uint8)
        check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(p), w.ctypes.data, b.ctypes.data, blob.ctypes.data), "pack")
        blobs.append(DeviceBuffer.from_array(blob))
    if wide is None:
        dx = to_device_nc4(x)
        dy = DeviceBuffer(V.nc4_elems(*yshape) * 2)
        dy.zero()
        check(lib.vkhip_conv3x3_pair_forward(ctypes.byref(d1), ctypes.byref(d2), dx.ptr, 0, blobs[0].ptr, blobs[1].ptr, dy.ptr, 0, None), "pair")
        return from_device_nc4(dy, yshape)
    Cw, cin, cout = wide
    r = rng(77)
    full = round_half(r.standard_normal((N, Cw, H, W)))
    full[:, cin:cin + C] = x
    dw = to_device_nc4(full)
    plane = H * W * 8
    check(lib.vkhip_conv3x3_pair_forward(ctypes.byref(d1), ctypes.byref(d2), dw.ptr + cin // 4 * plane, Cw // 4, blobs[0].ptr, blobs[1].ptr,
                                         dw.ptr + cout // 4 * plane, Cw // 4, None), "pair view")
    out = from_device_nc4(dw, full.shape)
    keep = [c for c in range(Cw) if not cout <= c < cout + C]
    assert np.array_equal(out[:, keep], full[:, keep])  # nothing outside the output slice changes
    return out[:, cout:cout + C]


def oracle_pair(x, w1, b1, w2, b2, act, res):
    t = round_half(oracle_conv(x, w1, b1, (1, 1), (1, 1, 1, 1), act=act))
    y = oracle_conv(t, w2, b2, (1, 1), (1, 1, 1, 1), act=act)
    return round_half(y) + x if res else y


PAIR_CASES = [(2, 16, 20, 36, 5, True), (3, 32, 13, 70, 5, True), (2, 24, 9, 18, 1, False), (1, 12, 5, 130, 5, True),
              (2, 32, 33, 66, 0, False), (1, 16, 4, 64, 2, True)]


@pytest.mark.parametrize("case", PAIR_CASES)
def test_conv3x3_pair(gpu, case):
    """Two 3x3 convs in one kernel (the intermediate kept in LDS, rounded to fp16 like the separate
    conv's store), with and without the bottleneck shortcut, against the oracle's two convs (+ its
    add): 16 and 32 channels and ragged counts (12, 24: zero slots), item rows and columns cut by
    the image edge, several column blocks, ReLU / ReLU6 / SiLU / no activation."""
    N, C, H, W, act, res = case
    r = rng(1500 + C + H + W)
    x = round_half(r.standard_normal((N, C, H, W)))
    w1 = (r.standard_normal((C, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    w2 = (r.standard_normal((C, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b1 = (r.standard_normal(C) * 0.1).astype(np.float32)
    b2 = (r.standard_normal(C) * 0.1).astype(np.float32)
    got = gpu_conv_pair(x, w1, b1, w2, b2, act, res)
    assert_parity(got, oracle_pair(x, w1, b1, w2, b2, act, res), f"pair {case}")


@pytest.mark.parametrize("C", [16, 32])
def test_conv3x3_pair_views(gpu, C):
    """The pair reading a channel slice of a wide tensor and writing another slice of the same
    tensor (the C2f split half in, the concat slice out), other slices untouched."""
    r = rng(1600 + C)
    x = round_half(r.standard_normal((2, C, 10, 40)))
    w1 = (r.standard_normal((C, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    w2 = (r.standard_normal((C, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b1 = (r.standard_normal(C) * 0.1).astype(np.float32)
    b2 = (r.standard_normal(C) * 0.1).astype(np.float32)
    got = gpu_conv_pair(x, w1, b1, w2, b2, 5, True, wide=(4 * C, C, 2 * C))
    assert_parity(got, oracle_pair(x, w1, b1, w2, b2, 5, True), f"pair views C={C}")


def test_conv3x3_pair_refusals(gpu):
    """Channel counts outside 9-32 or unequal, odd widths, stride 2, 1x1, a residual before the
    activation are refused."""
    lib = V.vkhip()
    p1, p2 = V.ConvPlan(), V.ConvPlan()
    def ok(x, c1w, c2w, st=(1, 1), pads=(1, 1, 1, 1), res=0):
        d1, ys = conv_desc(x, c1w, st, pads, act=5)
        d2, _ = conv_desc(ys, c2w, (1, 1), (1, 1, 1, 1), act=5, has_res=res)
        return lib.vkhip_conv3x3_pair_plan(ctypes.byref(d1), ctypes.byref(d2), ctypes.byref(p1), ctypes.byref(p2)) == 0
    assert ok((1, 16, 8, 8), (16, 16, 3, 3), (16, 16, 3, 3), res=2)
    assert not ok((1, 40, 8, 8), (40, 40, 3, 3), (40, 40, 3, 3))
    assert not ok((1, 8, 8, 8), (8, 8, 3, 3), (8, 8, 3, 3))
    assert not ok((1, 16, 8, 8), (32, 16, 3, 3), (32, 32, 3, 3))
    assert not ok((1, 16, 8, 9), (16, 16, 3, 3), (16, 16, 3, 3))
    assert not ok((1, 16, 8, 8), (16, 16, 3, 3), (16, 16, 3, 3), st=(2, 2))
    assert not ok((1, 16, 8, 8), (16, 16, 1, 1), (16, 16, 3, 3), pads=(0, 0, 0, 0))
    assert not ok((1, 16, 8, 8), (16, 16, 3, 3), (16, 16, 3, 3), res=1)


def gpu_stem2(x, w1, b1, act1, w2, b2, act2, y_wide=None, tail=None):
    """vkhip_conv3x3s2_pair_forward; with y_wide = (Cw, off) the output goes to channel `off` of a
    wider zero-filled tensor, which is returned whole; tail = (w3, b3, act3) adds the 1x1 tail."""
    lib = V.vkhip()
    d1, ys1 = conv_desc(x.shape, w1.shape, (2, 2), (1, 1, 1, 1), act=act1)
    d2, ys2 = conv_desc(ys1, w2.shape, (2, 2), (1, 1, 1, 1), act=act2)
    d3, ys3 = conv_desc(ys2, tail[0].shape, act=tail[2]) if tail else (None, ys2)
    p1, p2, p3 = V.ConvPlan(), V.ConvPlan(), V.ConvPlan()
    r3 = ctypes.byref(d3) if tail else None
    check(lib.vkhip_conv3x3s2_pair_plan(ctypes.byref(d1), ctypes.byref(d2), r3, ctypes.byref(p1), ctypes.byref(p2), ctypes.byref(p3)), "stem2 plan")
    blobs = []
    for d, p, w, b in ((d1, p1, w1, b1), (d2, p2, w2, b2)) + (((d3, p3, tail[0], tail[1]),) if tail else ()):
        blob = np.zeros(p.weight_bytes, np.uint8)
        check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(p), w.ctypes.data, b.ctypes.data, blob.ctypes.data), "pack")
        blobs.append(DeviceBuffer.from_array(blob))
    dx = to_device_nc4(x)
    N, C2, H2, W2 = ys3
    shape = ys3 if y_wide is None else (N, y_wide[0], H2, W2)
    dy = DeviceBuffer(V.nc4_elems(*shape) * 2)
    dy.zero()
    off = 0 if y_wide is None else y_wide[1] // 4 * H2 * W2 * 8
    check(lib.vkhip_conv3x3s2_pair_forward(ctypes.byref(d1), ctypes.byref(d2), r3, dx.ptr, blobs[0].ptr, blobs[1].ptr,
                                           blobs[2].ptr if tail else None, dy.ptr + off, 0 if y_wide is None else y_wide[0] // 4, None), "stem2")
    check(lib.vkhip_stream_sync(None), "sync")
    return from_device_nc4(dy, shape)


STEM2_CASES = [(2, 3, 64, 96, 16, 32, 5), (1, 3, 50, 130, 16, 32, 5), (3, 4, 22, 18, 12, 24, 1), (2, 1, 30, 262, 16, 16, 4),
               (1, 3, 9, 8, 10, 7, 2), (2, 3, 640, 640, 16, 32, 5)]


@pytest.mark.parametrize("tail", [None, 32, 20])
@pytest.mark.parametrize("case", STEM2_CASES)
def test_conv3x3s2_pair(gpu, case, tail):
    """The two stride-2 stem convs in one kernel (the intermediate in LDS, rounded to fp16 like
    the separate conv's store) against the oracle's two convs, and with the 1x1 tail conv over
    the second conv's output (its output in LDS too; 32 or 20 channels out): the YOLOv8n stem at
    full size, odd intermediate and output sizes, items cut by the image edge, ragged channel
    counts (1, 4 in; 10, 12 between; 7, 24 out), SiLU / ReLU / ReLU6 / hard-swish."""
    N, C, H, W, C1, C2, act = case
    r = rng(1700 + C + H + W + C1 + C2)
    x = round_half(r.standard_normal((N, C, H, W)))
    w1 = (r.standard_normal((C1, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    w2 = (r.standard_normal((C2, C1, 3, 3)) * np.sqrt(2.0 / (9 * C1))).astype(np.float32)
    b1 = (r.standard_normal(C1) * 0.1).astype(np.float32)
    b2 = (r.standard_normal(C2) * 0.1).astype(np.float32)
    t = round_half(oracle_conv(x, w1, b1, (2, 2), (1, 1, 1, 1), act=act))
    ref = oracle_conv(t, w2, b2, (2, 2), (1, 1, 1, 1), act=act)
    if tail:
        w3 = (r.standard_normal((tail, C2, 1, 1)) * np.sqrt(2.0 / C2)).astype(np.float32)
        b3 = (r.standard_normal(tail) * 0.1).astype(np.float32)
        got = gpu_stem2(x, w1, b1, act, w2, b2, act, tail=(w3, b3, act))
        ref = oracle_conv(round_half(ref), w3, b3, act=act)
    else:
        got = gpu_stem2(x, w1, b1, act, w2, b2, act)
    assert_parity(got, ref, f"stem2 {case} tail {tail}")


def test_conv3x3s2_pair_view_and_refusals(gpu):
    """The output written into a channel slice of a wider tensor (other slices stay zero), with and
    without the tail; shapes outside the kernel's range are refused."""
    r = rng(1800)
    x = round_half(r.standard_normal((2, 3, 40, 64)))
    w1 = (r.standard_normal((16, 3, 3, 3)) * 0.3).astype(np.float32)
    w2 = (r.standard_normal((32, 16, 3, 3)) * 0.1).astype(np.float32)
    w3 = (r.standard_normal((32, 32, 1, 1)) * 0.2).astype(np.float32)
    b1, b2, b3 = np.zeros(16, np.float32), np.zeros(32, np.float32), np.zeros(32, np.float32)
    t = round_half(oracle_conv(x, w1, b1, (2, 2), (1, 1, 1, 1), act=5))
    ref = oracle_conv(t, w2, b2, (2, 2), (1, 1, 1, 1), act=5)
    for tail, want in ((None, ref), ((w3, b3, 5), oracle_conv(round_half(ref), w3, b3, act=5))):
        got = gpu_stem2(x, w1, b1, 5, w2, b2, 5, y_wide=(64, 16), tail=tail)
        assert_parity(got[:, 16:48], want, f"stem2 view tail {tail is not None}")
        assert not got[:, :16].any() and not got[:, 48:].any()
    lib = V.vkhip()
    p1, p2, p3 = V.ConvPlan(), V.ConvPlan(), V.ConvPlan()
    def ok(xs, c1, c2, s1=2, s2=2, c3=None, k3=1):
        d1, ys = conv_desc(xs, (c1, xs[1], 3, 3), (s1, s1), (1, 1, 1, 1))
        d2, ys2 = conv_desc(ys, (c2, c1, 3, 3), (s2, s2), (1, 1, 1, 1))
        d3 = conv_desc(ys2, (c3, c2, k3, k3), pads=(k3 // 2,) * 4)[0] if c3 else None
        return lib.vkhip_conv3x3s2_pair_plan(ctypes.byref(d1), ctypes.byref(d2), ctypes.byref(d3) if d3 else None, ctypes.byref(p1),
                                             ctypes.byref(p2), ctypes.byref(p3)) == 0
    assert ok((1, 3, 32, 32), 16, 32) and ok((1, 3, 32, 32), 16, 32, c3=32)
    assert not ok((1, 8, 32, 32), 16, 32)      # more than 4 input channels
    assert not ok((1, 3, 32, 32), 32, 32)      # more than 16 between
    assert not ok((1, 3, 32, 32), 16, 64)      # more than 32 out
    assert not ok((1, 3, 32, 33), 16, 32)      # odd input width
    assert not ok((1, 3, 32, 32), 16, 32, s2=1)
    assert not ok((1, 3, 32, 32), 16, 32, c3=64)       # tail wider than 32
    assert not ok((1, 3, 32, 32), 16, 32, c3=32, k3=3)  # tail not 1x1


def gpu_stem_dwpw(x, ws, bs, acts, wd, bd, actd, wp, bp, actp, res=True, y_wide=None):
    """vkhip_stem_dwpw_forward; with y_wide = (Cw, off) the output goes to channel `off` of a
    wider zero-filled tensor, which is returned whole."""
    lib = V.vkhip()
    C1 = ws.shape[0]
    ds, ys1 = conv_desc(x.shape, ws.shape, (2, 2), (1, 1, 1, 1), act=acts)
    dd, _ = conv_desc(ys1, wd.shape, (1, 1), (1, 1, 1, 1), group=C1, act=actd, lo=0.0, hi=6.0)
    dp, ys = conv_desc(ys1, wp.shape, act=actp, has_res=1 if res else 0)
    ps, pd, pp = V.ConvPlan(), V.ConvPlan(), V.ConvPlan()
    check(lib.vkhip_stem_dwpw_plan(ctypes.byref(ds), ctypes.byref(dd), ctypes.byref(dp), ctypes.byref(ps), ctypes.byref(pd),
                                   ctypes.byref(pp)), "stem_dwpw plan")
    blobs = []
    for d, p, w, b in ((ds, ps, ws, bs), (dd, pd, wd, bd), (dp, pp, wp, bp)):
        blob = np.zeros(p.weight_bytes, np.uint8)
        check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(p), w.ctypes.data, b.ctypes.data, blob.ctypes.data), "pack")
        blobs.append(DeviceBuffer.from_array(blob))
    dx = to_device_nc4(x)
    N, C2, H2, W2 = ys
    shape = ys if y_wide is None else (N, y_wide[0], H2, W2)
    dy = DeviceBuffer(V.nc4_elems(*shape) * 2)
    dy.zero()
    off = 0 if y_wide is None else y_wide[1] // 4 * H2 * W2 * 8
    check(lib.vkhip_stem_dwpw_forward(ctypes.byref(ds), ctypes.byref(dd), ctypes.byref(dp), dx.ptr, blobs[0].ptr, blobs[1].ptr,
                                      blobs[2].ptr, dy.ptr + off, 0 if y_wide is None else y_wide[0] // 4, None), "stem_dwpw")
    check(lib.vkhip_stream_sync(None), "sync")
    return from_device_nc4(dy, shape)


def stem_dwpw_case(r, N, C, H, W, C1, C2):
    x = round_half(r.standard_normal((N, C, H, W)))
    ws = (r.standard_normal((C1, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    wd = (r.standard_normal((C1, 1, 3, 3)) * np.sqrt(2.0 / 9)).astype(np.float32)
    wp = (r.standard_normal((C2, C1, 1, 1)) * np.sqrt(1.0 / C1)).astype(np.float32)
    bs, bd, bp = ((r.standard_normal(c) * 0.1).astype(np.float32) for c in (C1, C1, C2))
    return x, ws, bs, wd, bd, wp, bp


def oracle_stem_dwpw(x, ws, bs, acts, wd, bd, actd, wp, bp, actp, res=True):
    t = round_half(oracle_conv(x, ws, bs, (2, 2), (1, 1, 1, 1), act=acts))
    return oracle_dwpw(t, wd, bd, wp.reshape(wp.shape[0], -1), bp, dw_act=actd, res=t if res else None, act=actp)


# N, C, H, W, stem channels, out channels, (stem act, dw act, projection act), residual
STEM_DWPW_CASES = [(2, 3, 224, 224, 16, 16, (4, 1, 0), True), (1, 3, 98, 130, 16, 16, (4, 1, 0), True),
                   (3, 4, 22, 18, 12, 12, (1, 2, 5), True), (2, 1, 30, 262, 16, 8, (5, 0, 1), False),
                   (1, 3, 10, 8, 10, 7, (2, 1, 0), False), (1, 2, 6, 4, 9, 9, (4, 4, 4), True)]


@pytest.mark.parametrize("case", STEM_DWPW_CASES)
def test_stem_dwpw(gpu, case):
    """The MobileNetV3 stem and first block in one kernel (stem output and depthwise output in LDS,
    each rounded to fp16 like the separate kernels' stores) against the oracle's conv and fused
    depthwise + projection, with the stem's output as the residual: MobileNetV3-Large's first block
    at full size, odd stem outputs, items cut by the image edge, 1-4 input channels, 9-16 between,
    7-16 out, with and without the residual, and the activation combinations the planner can meet."""
    N, C, H, W, C1, C2, (acts, actd, actp), res = case
    r = rng(1900 + C + H + W + C1 + C2)
    x, ws, bs, wd, bd, wp, bp = stem_dwpw_case(r, N, C, H, W, C1, C2)
    got = gpu_stem_dwpw(x, ws, bs, acts, wd, bd, actd, wp, bp, actp, res=res)
    assert_parity(got, oracle_stem_dwpw(x, ws, bs, acts, wd, bd, actd, wp, bp, actp, res=res), f"stem_dwpw {case}")


def test_stem_dwpw_view_and_refusals(gpu):
    """The output written into a channel slice of a wider tensor (other slices stay zero); shapes
    outside the kernel's range are refused."""
    r = rng(1950)
    x, ws, bs, wd, bd, wp, bp = stem_dwpw_case(r, 2, 3, 40, 64, 16, 16)
    got = gpu_stem_dwpw(x, ws, bs, 4, wd, bd, 1, wp, bp, 0, y_wide=(48, 16))
    assert_parity(got[:, 16:32], oracle_stem_dwpw(x, ws, bs, 4, wd, bd, 1, wp, bp, 0), "stem_dwpw view")
    assert not got[:, :16].any() and not got[:, 32:].any()
    lib = V.vkhip()
    ps, pd, pp = V.ConvPlan(), V.ConvPlan(), V.ConvPlan()
    def ok(xs, c1, c2, sd=1, kp=1, res=1, cd=None):
        ds, ys = conv_desc(xs, (c1, xs[1], 3, 3), (2, 2), (1, 1, 1, 1))
        cd = cd or c1
        dd = conv_desc(ys, (cd, 1, 3, 3), (sd, sd), (1, 1, 1, 1), group=cd)[0]
        dp = conv_desc(ys, (c2, c1, kp, kp), pads=(kp // 2,) * 4, has_res=res)[0]
        return lib.vkhip_stem_dwpw_plan(ctypes.byref(ds), ctypes.byref(dd), ctypes.byref(dp), ctypes.byref(ps), ctypes.byref(pd),
                                        ctypes.byref(pp)) == 0
    assert ok((1, 3, 32, 32), 16, 16) and ok((1, 3, 32, 32), 16, 8, res=0)
    assert not ok((1, 8, 32, 32), 16, 16)           # more than 4 input channels
    assert not ok((1, 3, 32, 32), 32, 32)           # more than 16 between
    assert not ok((1, 3, 32, 32), 16, 32, res=0)    # more than 16 out
    assert not ok((1, 3, 32, 33), 16, 16)           # odd input width
    assert not ok((1, 3, 32, 32), 16, 16, sd=2)     # strided depthwise conv
    assert not ok((1, 3, 32, 32), 16, 16, kp=3)     # projection not 1x1
    assert not ok((1, 3, 32, 32), 16, 8)            # residual with a channel count other than the stem's
    assert not ok((1, 3, 32, 32), 16, 16, res=2)    # residual after the activation


@pytest.mark.parametrize("tile", PERS_TILES)
@pytest.mark.parametrize("shape", [(32, 64, 28, 28, 512), (17, 200, 7, 7, 256), (9, 96, 15, 15, 200)])
def test_conv_dma_persist_many_tiles(gpu, tile, shape):
    """Persistent tiles on shapes with more tiles than resident workgroups (every workgroup walks
    several tiles and its ring crosses tile boundaries), K tails, odd images, ragged channels,
    residual + ReLU6 epilogue; then the same shape without a residual."""
    N, C, H, W, Cout = shape
    r = rng(700 + tile + C)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, 1, 1)) * 0.1).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    res = round_half(r.standard_normal((N, Cout, H, W)))
    got, plan, _ = gpu_conv(x, w, b, act=2, res=res, algo=V.CONV_GEMM, tile=tile)
    assert plan.tile == tile
    assert_parity(got, oracle_conv(x, w, b, res=res, act=2), f"persistent 1x1 tile {tile} {shape}")
    got, plan, _ = gpu_conv(x, w, b, act=1, algo=V.CONV_GEMM, tile=tile)
    assert_parity(got, oracle_conv(x, w, b, act=1), f"persistent 1x1 no residual tile {tile} {shape}")


@pytest.mark.parametrize("tile", LE_TILES)
@pytest.mark.parametrize("shape,stride,act", [((3, 72, 6, 10, 70), 1, 1), ((2, 256, 14, 14, 300), 1, 4), ((1, 24, 8, 8, 8), 1, 2),
                                              ((5, 64, 6, 9, 40), 1, 5), ((1, 256, 28, 28, 512), 2, 1), ((2, 48, 12, 12, 130), 2, 0)])
def test_conv_dma_lds_epilogue(gpu, tile, shape, stride, act):
    """LDS-staged epilogue (residual copied into LDS as kilobyte rows, outputs finished in place,
    16-byte row stores): pixel tiles crossing images and the end of the batch, ragged channels,
    stride 2, every activation family, with and without a residual."""
    N, C, H, W, Cout = shape
    r = rng(470 + tile + C + H)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, 1, 1)) * 0.1).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    OH, OW = (H - 1) // stride + 1, (W - 1) // stride + 1
    res = round_half(r.standard_normal((N, Cout, OH, OW)))
    for rr in (res, None):
        got, plan, _ = gpu_conv(x, w, b, (stride, stride), act=act, res=rr, algo=V.CONV_GEMM, tile=tile)
        assert plan.tile == tile
        assert_parity(got, oracle_conv(x, w, b, (stride, stride), res=rr, act=act), f"lds epilogue tile {tile} {shape} s{stride}")


def test_conv_dma_lds_epilogue_refuses_odd_images(gpu):
    lib = V.vkhip()
    plan = V.ConvPlan()
    d, _ = conv_desc((2, 64, 7, 7), (64, 64, 1, 1))
    for t in LE_TILES:
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, t, 0, ctypes.byref(plan)) != 0


def test_conv_persist_tiles_refuse_other_algorithms(gpu):
    """Persistent tiles run plain GEMM plans only: split-K and Winograd plans are refused."""
    lib = V.vkhip()
    plan = V.ConvPlan()
    d, _ = conv_desc((2, 64, 8, 8), (64, 64, 1, 1))
    d3, _ = conv_desc((2, 64, 8, 8), (64, 64, 3, 3), pads=(1, 1, 1, 1))
    for t in PERS_TILES:
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_SPLITK, t, 2, ctypes.byref(plan)) != 0
        assert lib.vkhip_conv_plan_make(ctypes.byref(d3), V.CONV_WINOGRAD, t, 0, ctypes.byref(plan)) != 0


@pytest.mark.parametrize("tile", [14, 15, 24, 25, 36, 38, 40, 41])
@pytest.mark.parametrize("shape", [(2, 64, 14, 14, 128), (3, 72, 9, 11, 70), (1, 256, 28, 28, 512)])
def test_conv_dma_1x1_stride2(gpu, tile, shape):
    """Stride-2 1x1 (ResNet downsample) on the dense-B kernel: one pixel per copy lane with its
    unused right neighbour, odd input sizes (the last column's neighbour is the next row's first
    pixel), residual + ReLU."""
    N, C, H, W, Cout = shape
    r = rng(160 + tile + C + H)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, 1, 1)) * 0.1).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    OH, OW = (H - 1) // 2 + 1, (W - 1) // 2 + 1
    res = round_half(r.standard_normal((N, Cout, OH, OW)))
    got, plan, _ = gpu_conv(x, w, b, (2, 2), act=1, res=res, algo=V.CONV_GEMM, tile=tile)
    assert plan.tile == tile
    assert_parity(got, oracle_conv(x, w, b, (2, 2), res=res, act=1), f"dma 1x1 s2 tile {tile} {shape}")


@pytest.mark.parametrize("tile", [11, 14])
def test_conv_dma_winograd_and_splitk(gpu, tile):
    r = rng(90 + tile)
    x = round_half(r.standard_normal((2, 128, 14, 14)))
    w = (r.standard_normal((96, 128, 3, 3)) * 0.05).astype(np.float32)
    b = (r.standard_normal(96) * 0.1).astype(np.float32)
    ref = oracle_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1)
    got, plan, _ = gpu_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1, algo=V.CONV_WINOGRAD, tile=tile)
    assert_parity(got, ref, f"dma winograd tile {tile}")
    xo = round_half(r.standard_normal((1, 32, 6, 6)))   # 9 Winograd tiles: odd column count
    wo = (r.standard_normal((40, 32, 3, 3)) * 0.1).astype(np.float32)
    got, plan, _ = gpu_conv(xo, wo, None, (1, 1), (1, 1, 1, 1), act=0, algo=V.CONV_WINOGRAD, tile=tile)
    assert_parity(got, oracle_conv(xo, wo, None, (1, 1), (1, 1, 1, 1)), f"dma winograd odd tiles {tile}")
    x1 = round_half(r.standard_normal((1, 512, 8, 8)))
    w1 = (r.standard_normal((256, 512, 1, 1)) * 0.05).astype(np.float32)
    got, plan, _ = gpu_conv(x1, w1, None, act=0, algo=V.CONV_SPLITK, tile=tile, ksplit=4)
    assert plan.ksplit == 4
    assert_parity(got, oracle_conv(x1, w1), f"dma split-K tile {tile}")


def test_conv_dma_rejects_gather_shapes(gpu):
    """The dense-B tiles refuse shapes whose B operand is a gather (3x3, stride 2, padded 1x1)."""
    lib = V.vkhip()
    plan = V.ConvPlan()
    for xs, ws, st, pd in [((1, 8, 8, 8), (8, 8, 3, 3), (1, 1), (1, 1, 1, 1)), ((1, 8, 8, 8), (8, 8, 1, 1), (2, 2), (0, 0, 0, 0)),
                           ((1, 8, 7, 7), (8, 8, 1, 1), (1, 1), (1, 1, 1, 1))]:
        d, _ = conv_desc(xs, ws, st, pd)
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, 11, 0, ctypes.byref(plan)) != 0


@pytest.mark.parametrize("tile", HALO_TILES)
@pytest.mark.parametrize("shape", [(2, 64, 14, 14, 72), (1, 32, 8, 10, 40), (3, 128, 6, 6, 128), (1, 64, 56, 56, 64),
                                   (2, 96, 28, 28, 100), (2, 64, 7, 7, 64), (3, 32, 9, 11, 40)])
def test_conv_halo_3x3(gpu, tile, shape):
    """Band-staged 3x3 kernel: pixel tiles crossing one or several image boundaries (zero rows
    between images), the end of the batch, ragged output channels, residual + ReLU epilogue."""
    N, C, H, W, Cout = shape
    r = rng(120 + tile + C + H)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    res = round_half(r.standard_normal((N, Cout, H, W)))
    got, plan, _ = gpu_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1, res=res, algo=V.CONV_GEMM, tile=tile)
    assert plan.tile == tile
    ref = oracle_conv(x, w, b, (1, 1), (1, 1, 1, 1), res=res, act=1)
    assert_parity(got, ref, f"halo tile {tile} {shape}")


@pytest.mark.parametrize("tile", HALO_TILES)
@pytest.mark.parametrize("shape", [(2, 64, 56, 56, 64), (3, 32, 14, 14, 40), (2, 128, 28, 28, 100), (5, 64, 14, 10, 64),
                                   (2, 48, 7, 8, 32), (2, 32, 9, 9, 32), (1, 64, 15, 13, 48)])
def test_conv_halo_3x3_stride2(gpu, tile, shape):
    """Stride-2 band: two input rows per output row, output rows from odd input heights (the last
    centre row's lower neighbour is the zero row), odd output widths, several images per tile."""
    N, C, H, W, Cout = shape
    r = rng(140 + tile + C + H + W)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    OH, OW = (H - 1) // 2 + 1, (W - 1) // 2 + 1
    res = round_half(r.standard_normal((N, Cout, OH, OW)))
    lib = V.vkhip()
    plan = V.ConvPlan()
    d, _ = conv_desc((N, C, H, W), (Cout, C, 3, 3), (2, 2), (1, 1, 1, 1))
    if lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, tile, 0, ctypes.byref(plan)) != 0:
        pytest.skip("band does not fit this tile's LDS budget")
    got, plan, _ = gpu_conv(x, w, b, (2, 2), (1, 1, 1, 1), act=1, res=res, algo=V.CONV_GEMM, tile=tile)
    assert plan.tile == tile
    ref = oracle_conv(x, w, b, (2, 2), (1, 1, 1, 1), res=res, act=1)
    assert_parity(got, ref, f"halo s2 tile {tile} {shape}")


@pytest.mark.parametrize("tile", STEM_TILES)
@pytest.mark.parametrize("case", [(2, 3, 224, 224, 64, 7, 2), (3, 3, 32, 30, 16, 3, 2), (2, 4, 20, 18, 40, 3, 1),
                                  (1, 3, 40, 38, 24, 7, 1), (2, 1, 16, 16, 8, 7, 2), (5, 2, 9, 10, 70, 3, 2)])
def test_conv_stem(gpu, tile, case):
    """Stem kernel: 3 or fewer channels padded to one slot, 7x7 and 3x3 taps packed four to an
    MFMA step, stride 1/2, odd heights, ragged output channels, tiles across images, residual."""
    N, C, H, W, Cout, K, S = case
    r = rng(150 + tile + H + K)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, K, K)) * np.sqrt(2.0 / (K * K * C))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    p = K // 2
    OH, OW = (H + 2 * p - K) // S + 1, (W + 2 * p - K) // S + 1
    res = round_half(r.standard_normal((N, Cout, OH, OW)))
    got, plan, _ = gpu_conv(x, w, b, (S, S), (p, p, p, p), act=1, res=res, algo=V.CONV_GEMM, tile=tile)
    assert plan.tile == tile
    ref = oracle_conv(x, w, b, (S, S), (p, p, p, p), res=res, act=1)
    assert_parity(got, ref, f"stem tile {tile} {case}")


STEM_POOL_CASES = [(2, 3, 224, 224, 64, 7, 2, 1), (1, 3, 33, 40, 64, 7, 2, 0), (3, 4, 30, 46, 48, 3, 2, 2), (2, 1, 17, 18, 20, 7, 1, 1),
                   (1, 3, 9, 250, 64, 7, 2, 1)]
# the thin-tile kernel: 7x7 stride 2 over an even width only
THIN_POOL_CASES = [(2, 3, 224, 224, 64, 7, 2, 1), (1, 3, 33, 40, 64, 7, 2, 0), (1, 3, 9, 250, 64, 7, 2, 1), (3, 4, 30, 46, 48, 7, 2, 2),
                   (2, 1, 17, 18, 20, 7, 2, 1), (1, 2, 6, 4, 9, 7, 2, 0)]


@pytest.mark.parametrize("tile,case", [(t, c) for t in (21, 22) for c in STEM_POOL_CASES] + [(45, c) for c in THIN_POOL_CASES])
def test_conv_maxpool_fused(gpu, tile, case):
    """Stem conv + 3x3/s2/p1 max pool in one kernel: bit-identical to the conv kernel followed by
    the max-pool kernel (odd heights, ragged output channels, stride 1 and 2, wide rows with one
    pooled row per workgroup; on the stem tiles 21/22 and on the thin tile 45, whose kernel splits
    the pooled width into items of at most 28 columns: 28, 20, 21, 12, 5 and 1 here), and the pool
    of the oracle conv within the fp16 tolerance."""
    lib = V.vkhip()
    N, C, H, W, Cout, K, S, act = case
    r = rng(170 + tile + H + K)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, K, K)) * np.sqrt(2.0 / (K * K * C))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    p = K // 2
    lo, hi = (0.0, 6.0) if act == 2 else (0.0, 0.0)
    d, (_, _, OH, OW) = conv_desc(x.shape, w.shape, (S, S), (p, p, p, p), act=act, lo=lo, hi=hi)
    POH, POW = (OH - 1) // 2 + 1, (OW - 1) // 2 + 1
    pd = V.PoolDesc(N=N, C=Cout, H=OH, W=OW, OH=POH, OW=POW, KH=3, KW=3, SH=2, SW=2, PT=1, PL=1)
    plan = V.ConvPlan()
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, tile, 0, ctypes.byref(plan)), "plan")
    assert lib.vkhip_conv_maxpool_supported(ctypes.byref(d), ctypes.byref(plan), ctypes.byref(pd)) == 1
    blob = np.zeros(plan.weight_bytes, np.uint8)
    check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, b.ctypes.data, blob.ctypes.data))
    dblob = DeviceBuffer.from_array(blob)
    dx = to_device_nc4(x)
    dconv = DeviceBuffer(V.nc4_elems(N, Cout, OH, OW) * 2)
    dpool = DeviceBuffer(V.nc4_elems(N, Cout, POH, POW) * 2)
    dfused = DeviceBuffer(V.nc4_elems(N, Cout, POH, POW) * 2)
    print(f"conv+maxpool tile {tile} case {case}", flush=True)
    check(lib.vkhip_conv_forward(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr, None, dconv.ptr, None, None))
    check(lib.vkhip_maxpool(ctypes.byref(pd), dconv.ptr, dpool.ptr, None))
    check(lib.vkhip_conv_maxpool_forward(ctypes.byref(d), ctypes.byref(plan), ctypes.byref(pd), dx.ptr, dblob.ptr, dfused.ptr, None))
    check(lib.vkhip_stream_sync(None))
    assert np.array_equal(raw_nc4(dfused, (N, Cout, POH, POW)), raw_nc4(dpool, (N, Cout, POH, POW)))
    conv_ref = oracle_conv(x, w, b, (S, S), (p, p, p, p), act=act, lo=lo, hi=hi)
    ref = np.zeros((N, Cout, POH, POW), np.float32)
    oracle().oracle_maxpool(np.ascontiguousarray(conv_ref).ctypes.data, ref.ctypes.data, N, Cout, OH, OW, 3, 3, 2, 2, 1, 1, POH, POW)
    assert_parity(from_device_nc4(dfused, (N, Cout, POH, POW)), ref, f"conv+maxpool {case}")


def test_conv_maxpool_rejects_other_shapes(gpu):
    lib = V.vkhip()
    plan = V.ConvPlan()
    d, (_, _, OH, OW) = conv_desc((1, 3, 32, 32), (64, 3, 7, 7), (2, 2), (3, 3, 3, 3), act=1)
    ok = V.PoolDesc(N=1, C=64, H=OH, W=OW, OH=(OH - 1) // 2 + 1, OW=(OW - 1) // 2 + 1, KH=3, KW=3, SH=2, SW=2, PT=1, PL=1)
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, 21, 0, ctypes.byref(plan)))
    assert lib.vkhip_conv_maxpool_supported(ctypes.byref(d), ctypes.byref(plan), ctypes.byref(ok)) == 1
    for field, val in [("KH", 2), ("SH", 1), ("PT", 0), ("OH", ok.OH + 1), ("C", 32)]:
        bad = V.PoolDesc(**{f: getattr(ok, f) for f, _ in V.PoolDesc._fields_})
        setattr(bad, field, val)
        assert lib.vkhip_conv_maxpool_supported(ctypes.byref(d), ctypes.byref(plan), ctypes.byref(bad)) == 0, field
    wide, _ = conv_desc((1, 3, 32, 32), (96, 3, 7, 7), (2, 2), (3, 3, 3, 3))
    assert lib.vkhip_conv_plan_make(ctypes.byref(wide), V.CONV_GEMM, 21, 0, ctypes.byref(plan)) != 0 or \
        lib.vkhip_conv_maxpool_supported(ctypes.byref(wide), ctypes.byref(plan), ctypes.byref(ok)) == 0
    # the thin tile: 7x7 stride 2 pad 3 over an even width only
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, 45, 0, ctypes.byref(plan)))
    assert lib.vkhip_conv_maxpool_supported(ctypes.byref(d), ctypes.byref(plan), ctypes.byref(ok)) == 1
    for shape, wshape, st, pads in [((1, 3, 32, 31), (64, 3, 7, 7), 2, 3), ((1, 3, 32, 32), (64, 3, 3, 3), 2, 1), ((1, 3, 32, 32), (64, 3, 7, 7), 1, 3)]:
        o, (_, _, oh, ow) = conv_desc(shape, wshape, (st, st), (pads,) * 4)
        op = V.PoolDesc(N=1, C=64, H=oh, W=ow, OH=(oh - 1) // 2 + 1, OW=(ow - 1) // 2 + 1, KH=3, KW=3, SH=2, SW=2, PT=1, PL=1)
        assert lib.vkhip_conv_plan_make(ctypes.byref(o), V.CONV_GEMM, 45, 0, ctypes.byref(plan)) != 0 or \
            lib.vkhip_conv_maxpool_supported(ctypes.byref(o), ctypes.byref(plan), ctypes.byref(op)) == 0, (shape, wshape, st)
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, 0, 0, ctypes.byref(plan)))
    assert lib.vkhip_conv_maxpool_supported(ctypes.byref(d), ctypes.byref(plan), ctypes.byref(ok)) == 0


def test_conv_stem_rejects_other_shapes(gpu):
    lib = V.vkhip()
    plan = V.ConvPlan()
    for xs, ws, st, pd in [((1, 5, 8, 8), (8, 5, 3, 3), (1, 1), (1, 1, 1, 1)), ((1, 3, 8, 8), (8, 3, 5, 5), (1, 1), (2, 2, 2, 2)),
                           ((1, 3, 9, 9), (8, 3, 3, 3), (2, 2), (1, 1, 1, 1)), ((1, 3, 8, 8), (8, 3, 3, 3), (1, 1), (0, 0, 0, 0))]:
        d, _ = conv_desc(xs, ws, st, pd)
        for t in STEM_TILES:
            assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, t, 0, ctypes.byref(plan)) != 0


@pytest.mark.parametrize("tile", [17, 18, 20, 26])
def test_conv_halo_splitk(gpu, tile):
    r = rng(130 + tile)
    x = round_half(r.standard_normal((2, 256, 14, 14)))
    w = (r.standard_normal((128, 256, 3, 3)) * 0.03).astype(np.float32)
    b = (r.standard_normal(128) * 0.1).astype(np.float32)
    got, plan, _ = gpu_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1, algo=V.CONV_SPLITK, tile=tile, ksplit=4)
    assert plan.ksplit == 4 and plan.tile == tile
    assert_parity(got, oracle_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1), f"halo split-K tile {tile}")


def test_conv_halo_rejects_other_shapes(gpu):
    """The halo tiles refuse stride 3, dilation 2, 1x1, Cin not a multiple of 16 and Winograd."""
    lib = V.vkhip()
    plan = V.ConvPlan()
    d, _ = conv_desc((1, 16, 9, 9), (8, 16, 3, 3), (1, 1), (2, 2, 2, 2), dil=(2, 2))
    for t in HALO_TILES:
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, t, 0, ctypes.byref(plan)) != 0
    for xs, ws, st, pd in [((1, 16, 9, 9), (8, 16, 3, 3), (3, 3), (1, 1, 1, 1)),
                           ((1, 16, 8, 8), (8, 16, 1, 1), (1, 1), (0, 0, 0, 0)), ((1, 24, 8, 8), (8, 24, 3, 3), (1, 1), (1, 1, 1, 1))]:
        d, _ = conv_desc(xs, ws, st, pd)
        for t in HALO_TILES:
            assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, t, 0, ctypes.byref(plan)) != 0
    d, _ = conv_desc((1, 16, 8, 8), (8, 16, 3, 3), (1, 1), (1, 1, 1, 1))
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_WINOGRAD, 17, 0, ctypes.byref(plan)) != 0
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, 17, 0, ctypes.byref(plan)) == 0


@pytest.mark.parametrize("tile", [8, 10])
def test_conv_bd_splitk_and_winograd(gpu, tile):
    r = rng(60 + tile)
    x = round_half(r.standard_normal((1, 256, 7, 7)))
    w = (r.standard_normal((128, 256, 3, 3)) * 0.05).astype(np.float32)
    b = (r.standard_normal(128) * 0.1).astype(np.float32)
    ref = oracle_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1)
    got, plan, _ = gpu_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1, algo=V.CONV_SPLITK, tile=tile, ksplit=6)
    assert plan.ksplit == 6
    assert_parity(got, ref, f"bd split-K tile {tile}")
    got, plan, _ = gpu_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1, algo=V.CONV_WINOGRAD, tile=tile)
    assert_parity(got, ref, f"bd winograd tile {tile}")


@pytest.mark.parametrize("ksplit", [2, 3, 8, 16])
def test_conv_splitk(gpu, ksplit):
    r = rng(30 + ksplit)
    x = round_half(r.standard_normal((1, 512, 7, 7)))
    w = (r.standard_normal((128, 512, 1, 1)) * 0.05).astype(np.float32)
    b = (r.standard_normal(128) * 0.1).astype(np.float32)
    res = round_half(r.standard_normal((1, 128, 7, 7)))
    got, plan, _ = gpu_conv(x, w, b, act=1, res=res, algo=V.CONV_SPLITK, tile=3, ksplit=ksplit)
    assert plan.algo == V.CONV_SPLITK
    assert_parity(got, oracle_conv(x, w, b, res=res, act=1), f"splitk {ksplit}")


# (tile, ksplit, x shape, Cout, kernel size, residual): gather (3, 6, 1), B-direct (8, 10), LDS-DMA
# (14, 16) and halo (17, 18, 20, 26) tiles, up to 16 splits and tiles with several workgroups
SPLITK_LAST_CASES = [(3, 2, (1, 512, 7, 7), 128, 1, True), (3, 16, (1, 1024, 7, 7), 256, 1, True), (6, 4, (1, 256, 7, 7), 32, 3, False),
                     (1, 3, (2, 256, 14, 14), 64, 1, True), (8, 6, (1, 256, 7, 7), 128, 3, False), (10, 4, (1, 256, 7, 7), 128, 3, False),
                     (14, 4, (2, 512, 14, 14), 256, 1, True), (16, 2, (2, 512, 14, 14), 128, 1, False),
                     (17, 4, (2, 256, 14, 14), 128, 3, False), (18, 4, (2, 256, 14, 14), 128, 3, False),
                     (20, 8, (1, 512, 7, 7), 512, 3, False), (26, 2, (4, 512, 7, 7), 512, 3, True)]


@pytest.mark.parametrize("case", SPLITK_LAST_CASES, ids=lambda c: f"t{c[0]}k{c[1]}")
def test_conv_splitk_last(gpu, case):
    """Split-K with the reduction in the conv kernel (the last workgroup of each tile sums the
    partials in split order): oracle parity, the same bits on a second call over the same workspace
    (the sum does not depend on which workgroup arrives last), and every arrival counter back at
    zero after each call."""
    tile, ks, xs, Cout, k, has_res = case
    lib = V.vkhip()
    r = rng(700 + tile * 17 + ks)
    x = round_half(r.standard_normal(xs))
    w = (r.standard_normal((Cout, xs[1], k, k)) * (0.6 / np.sqrt(xs[1] * k * k))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    pad = k // 2
    d, yshape = conv_desc(x.shape, w.shape, (1, 1), (pad,) * 4, act=1, has_res=int(has_res))
    res = round_half(r.standard_normal(yshape)) if has_res else None
    plan = V.ConvPlan()
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_SPLITK_LAST, tile, ks, ctypes.byref(plan)), "plan")
    assert plan.algo == V.CONV_SPLITK_LAST and plan.tile == tile and plan.ksplit == ks
    blob = np.zeros(plan.weight_bytes, np.uint8)
    check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, b.ctypes.data, blob.ctypes.data), "pack")
    dblob, dx = DeviceBuffer.from_array(blob), to_device_nc4(x)
    dres = to_device_nc4(res) if has_res else None
    ws = DeviceBuffer(plan.workspace_bytes)
    ws.zero()
    coutb, P = (Cout + 3) // 4, xs[0] * xs[2] * xs[3]
    cnt_off = -(-(ks * coutb * P * 16) // 256) * 256
    ntiles = (plan.workspace_bytes - cnt_off) // 4
    assert ntiles >= 1
    outs = []
    for call in range(2):
        dy = DeviceBuffer(V.nc4_elems(*yshape) * 2)
        dy.zero()
        check(lib.vkhip_conv_forward(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr, dres.ptr if dres else None, dy.ptr,
                                     ws.ptr, None), "conv_forward")
        check(lib.vkhip_stream_sync(None), "sync")
        cnt = ws.download(np.int32, plan.workspace_bytes // 4)[cnt_off // 4:]
        assert not cnt.any(), f"call {call}: {np.count_nonzero(cnt)} of {ntiles} arrival counters left nonzero"
        outs.append(raw_nc4(dy, yshape))
        if call == 0:
            ref = oracle_conv(x, w, b, (1, 1), (pad,) * 4, res=res, act=1)
            assert_parity(from_device_nc4(dy, yshape), ref, f"split-K in-kernel reduction tile {tile} ksplit {ks}")
    assert np.array_equal(outs[0], outs[1]), "a second call gave other bits"


def test_conv_splitk_last_refuses_other_tiles(gpu):
    """Stem, thin, persistent and LDS-staged-epilogue tiles have no in-kernel split-K reduction."""
    lib = V.vkhip()
    plan = V.ConvPlan()
    d, _ = conv_desc((2, 64, 14, 14), (64, 64, 1, 1))
    for t in (36, 37, 46):
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_SPLITK_LAST, t, 2, ctypes.byref(plan)) != 0
    d, _ = conv_desc((1, 3, 32, 32), (16, 3, 3, 3), (1, 1), (1, 1, 1, 1))
    for t in (21, 43):
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_SPLITK_LAST, t, 2, ctypes.byref(plan)) != 0
    d, _ = conv_desc((1, 64, 8, 8), (64, 64, 1, 1))
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), 6, 3, 2, ctypes.byref(plan)) != 0


@pytest.mark.parametrize("shape", [(1, 64, 56, 56, 64), (2, 32, 13, 15, 40), (1, 256, 14, 14, 256), (2, 512, 7, 7, 512)])
def test_conv_winograd(gpu, shape):
    N, C, H, W, Cout = shape
    r = rng(sum(shape))
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    got, plan, _ = gpu_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1, algo=V.CONV_WINOGRAD)
    assert plan.algo == V.CONV_WINOGRAD
    assert_parity(got, oracle_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1), f"winograd {shape}")


@pytest.mark.parametrize("shape", [(1, 128, 15, 7, 31), (2, 64, 14, 14, 64)])
def test_conv_winograd_residual(gpu, shape):
    """Winograd with a fused residual: added after the bias and before the activation in the
    output transform (a regression: the output transform once dropped it)."""
    N, C, H, W, Cout = shape
    r = rng(sum(shape) + 1)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    res = round_half(r.standard_normal((N, Cout, H, W)))
    got, plan, _ = gpu_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=5, res=res, algo=V.CONV_WINOGRAD)
    assert plan.algo == V.CONV_WINOGRAD
    assert_parity(got, oracle_conv(x, w, b, (1, 1), (1, 1, 1, 1), res=res, act=5), f"winograd+res {shape}")


def test_conv_winograd_stages(gpu):
    """The three Winograd stages run one call each (vkhip_conv_forward_stages, masks 1, 2, 4) leave
    the same bits as the whole conv; a non-Winograd plan refuses a partial mask."""
    N, C, H, W, Cout = 2, 64, 14, 14, 64
    r = rng(77)
    x = round_half(r.standard_normal((N, C, H, W)))
    w = (r.standard_normal((Cout, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    res = round_half(r.standard_normal((N, Cout, H, W)))
    whole, plan, _ = gpu_conv(x, w, b, (1, 1), (1, 1, 1, 1), act=1, res=res, algo=V.CONV_WINOGRAD)
    assert plan.algo == V.CONV_WINOGRAD
    lib = V.vkhip()
    d, yshape = conv_desc(x.shape, w.shape, (1, 1), (1, 1, 1, 1), act=1, has_res=1)
    blob = np.zeros(plan.weight_bytes, np.uint8)
    check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, b.ctypes.data, blob.ctypes.data), "pack")
    dblob, dx, dres = DeviceBuffer.from_array(blob), to_device_nc4(x), to_device_nc4(res)
    dy, ws = DeviceBuffer(V.nc4_elems(*yshape) * 2), DeviceBuffer(plan.workspace_bytes)
    dy.zero()
    for m in (1, 2, 4):
        check(lib.vkhip_conv_forward_stages(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr, dres.ptr, dy.ptr, ws.ptr, m, None), f"stage {m}")
    check(lib.vkhip_stream_sync(None), "sync")
    assert np.array_equal(from_device_nc4(dy, yshape), whole)
    gplan = V.ConvPlan()
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, -1, 0, ctypes.byref(gplan)), "gemm plan")
    assert lib.vkhip_conv_forward_stages(ctypes.byref(d), ctypes.byref(gplan), dx.ptr, dblob.ptr, dres.ptr, dy.ptr, ws.ptr, 1, None) != 0


def gpu_convpw(x, w3, b3, stride, act3, w1, b1, act1, res=None):
    """The fused 3x3 -> 1x1 kernel through the C ABI (vkhip_convpw_*)."""
    lib = V.vkhip()
    d3, mshape = conv_desc(x.shape, w3.shape, stride, (1, 1, 1, 1), act=act3)
    d = V.ConvPwDesc(conv=d3, Cout=w1.shape[0], act=act1, act_lo=0.0, act_hi=6.0, has_res=int(res is not None))
    plan = V.ConvPlan()
    check(lib.vkhip_convpw_plan(ctypes.byref(d), ctypes.byref(plan)), "convpw plan")
    blob = np.zeros(plan.weight_bytes, np.uint8)
    w3 = np.ascontiguousarray(w3, np.float32)
    w1 = np.ascontiguousarray(w1.reshape(w1.shape[0], -1), np.float32)
    check(lib.vkhip_convpw_pack_weights(ctypes.byref(d), ctypes.byref(plan), w3.ctypes.data, b3.ctypes.data, w1.ctypes.data,
                                        b1.ctypes.data, blob.ctypes.data), "convpw pack")
    dblob, dx = DeviceBuffer.from_array(blob), to_device_nc4(x)
    dres = to_device_nc4(res) if res is not None else None
    yshape = (x.shape[0], w1.shape[0], mshape[2], mshape[3])
    dy = DeviceBuffer(V.nc4_elems(*yshape) * 2)
    dy.zero()
    check(lib.vkhip_convpw_forward(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr, dres.ptr if dres else None, dy.ptr, None), "convpw")
    check(lib.vkhip_stream_sync(None), "sync")
    return from_device_nc4(dy, yshape), dy, yshape


@pytest.mark.parametrize("N,Cin,H,W,Cmid,Cout,S,act3,act1,res", [
    (2, 64, 14, 14, 64, 256, 1, 1, 1, True),     # layer-1 bottleneck shape, small map
    (1, 32, 9, 10, 64, 40, 1, 2, 2, False),      # ragged: odd H, Cout not a multiple of 32
    (2, 256, 16, 16, 64, 256, 2, 1, 1, True),    # stride 2
    (3, 128, 12, 8, 64, 100, 1, 5, 0, False),    # SiLU mid, no 1x1 activation, 3 images across workgroups
])
def test_convpw(gpu, N, Cin, H, W, Cmid, Cout, S, act3, act1, res):
    """3x3 (+bias, act, fp16 rounding) then 1x1 (+bias, residual, act) in one kernel against the
    oracle running the two convs with the intermediate rounded to fp16 between them."""
    r = rng(N * 1000 + Cin + H + Cout)
    x = round_half(r.standard_normal((N, Cin, H, W)))
    w3 = (r.standard_normal((Cmid, Cin, 3, 3)) * np.sqrt(2.0 / (9 * Cin))).astype(np.float32)
    b3 = (r.standard_normal(Cmid) * 0.1).astype(np.float32)
    w1 = (r.standard_normal((Cout, Cmid, 1, 1)) * np.sqrt(2.0 / Cmid)).astype(np.float32)
    b1 = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    OH, OW = (H - 1) // S + 1, (W - 1) // S + 1
    rs = round_half(r.standard_normal((N, Cout, OH, OW))) if res else None
    got, dy, yshape = gpu_convpw(x, w3, b3, (S, S), act3, w1, b1, act1, rs)
    mid = round_half(oracle_conv(x, w3, b3, (S, S), (1, 1, 1, 1), act=act3))
    ref = oracle_conv(mid, w1, b1, (1, 1), (0, 0, 0, 0), res=rs, act=act1, lo=0.0, hi=6.0)
    assert_parity(got, ref, f"convpw N{N} C{Cin} {H}x{W} s{S} mid{Cmid} out{Cout}")
    if Cout % 4:  # channel lanes past Cout stay +0
        raw = raw_nc4(dy, yshape).reshape(N, -1, OH, OW, 4)
        assert np.all(raw[:, -1, :, :, Cout % 4:] == 0)


@pytest.mark.parametrize("N,Cin,H,W,Cout,Cout3,res", [
    (2, 64, 14, 14, 256, 64, True),   # layer-1 bottleneck then the next block's reduction
    (1, 32, 9, 10, 72, 40, False),    # ragged: Cout and Cout3 not multiples of 32, odd H
    (3, 64, 8, 8, 128, 24, True),     # one chained fragment (Cout3 <= 32)
])
def test_convpw2_chain(gpu, N, Cin, H, W, Cout, Cout3, res):
    """3x3 -> 1x1 (+residual) -> 1x1 in one kernel: y against the oracle and bit-equal to the pair
    kernel; y2 against the oracle's 1x1 over y rounded to fp16 (what the chained 1x1 reads)."""
    lib = V.vkhip()
    r = rng(N * 100 + Cin + Cout + Cout3)
    x = round_half(r.standard_normal((N, Cin, H, W)))
    w3 = (r.standard_normal((64, Cin, 3, 3)) * np.sqrt(2.0 / (9 * Cin))).astype(np.float32)
    b3 = (r.standard_normal(64) * 0.1).astype(np.float32)
    w1 = (r.standard_normal((Cout, 64)) * np.sqrt(2.0 / 64)).astype(np.float32)
    b1 = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    w2 = (r.standard_normal((Cout3, Cout)) * np.sqrt(2.0 / Cout)).astype(np.float32)
    b2 = (r.standard_normal(Cout3) * 0.1).astype(np.float32)
    rs = round_half(r.standard_normal((N, Cout, H, W))) if res else None
    d3, _ = conv_desc(x.shape, w3.shape, (1, 1), (1, 1, 1, 1), act=1)
    pw = V.ConvPwDesc(conv=d3, Cout=Cout, act=1, act_lo=0.0, act_hi=0.0, has_res=int(res))
    d = V.ConvPw2Desc(pw=pw, Cout3=Cout3, act3=1, act3_lo=0.0, act3_hi=0.0)
    plan = V.ConvPlan()
    check(lib.vkhip_convpw2_plan(ctypes.byref(d), ctypes.byref(plan)), "convpw2 plan")
    blob = np.zeros(plan.weight_bytes, np.uint8)
    check(lib.vkhip_convpw2_pack_weights(ctypes.byref(d), ctypes.byref(plan), w3.ctypes.data, b3.ctypes.data, w1.ctypes.data,
                                         b1.ctypes.data, w2.ctypes.data, b2.ctypes.data, blob.ctypes.data), "convpw2 pack")
    dblob, dx = DeviceBuffer.from_array(blob), to_device_nc4(x)
    dres = to_device_nc4(rs) if res else None
    yshape, y2shape = (N, Cout, H, W), (N, Cout3, H, W)
    dy, dy2 = DeviceBuffer(V.nc4_elems(*yshape) * 2), DeviceBuffer(V.nc4_elems(*y2shape) * 2)
    dy.zero()
    dy2.zero()
    check(lib.vkhip_convpw2_forward(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr, dres.ptr if dres else None, dy.ptr, dy2.ptr,
                                    None), "convpw2")
    check(lib.vkhip_stream_sync(None), "sync")
    y, y2 = from_device_nc4(dy, yshape), from_device_nc4(dy2, y2shape)
    pair, _, _ = gpu_convpw(x, w3, b3, (1, 1), 1, w1.reshape(Cout, 64, 1, 1), b1, 1, rs)
    assert np.array_equal(y, pair)
    mid = round_half(oracle_conv(x, w3, b3, (1, 1), (1, 1, 1, 1), act=1))
    yref = oracle_conv(mid, w1.reshape(Cout, 64, 1, 1), b1, res=rs, act=1)
    assert_parity(y, yref, f"convpw2 y N{N} {H}x{W} {Cout}")
    y2ref = oracle_conv(round_half(yref), w2.reshape(Cout3, Cout, 1, 1), b2, act=1)
    assert_parity(y2, y2ref, f"convpw2 y2 N{N} {H}x{W} {Cout}->{Cout3}")
    if Cout3 % 4:
        raw = raw_nc4(dy2, y2shape).reshape(N, -1, H, W, 4)
        assert np.all(raw[:, -1, :, :, Cout3 % 4:] == 0)


def test_convpw_rejects_unsupported(gpu):
    """Mid widths other than 64, 1x1 or padded-wrong convs and a 3x3 with a residual have no
    fused kernel: the plan call says so and launches nothing."""
    lib = V.vkhip()
    for shape, w, kw in [((1, 64, 8, 8), (96, 64, 3, 3), {}), ((1, 64, 8, 8), (128, 64, 3, 3), {}), ((1, 64, 8, 8), (64, 64, 1, 1), {}),
                         ((1, 64, 8, 8), (64, 64, 3, 3), {"has_res": 1})]:
        d3, _ = conv_desc(shape, w, (1, 1), (1, 1, 1, 1) if w[2] == 3 else (0, 0, 0, 0), **kw)
        d = V.ConvPwDesc(conv=d3, Cout=256, act=1, act_lo=0.0, act_hi=0.0, has_res=0)
        plan = V.ConvPlan()
        assert lib.vkhip_convpw_plan(ctypes.byref(d), ctypes.byref(plan)) != 0


def test_conv_dilation(gpu):
    r = rng(40)
    x = round_half(r.standard_normal((1, 16, 15, 15)))
    w = (r.standard_normal((16, 16, 3, 3)) * 0.2).astype(np.float32)
    got, _, _ = gpu_conv(x, w, None, (1, 1), (2, 2, 2, 2), dil=(2, 2))
    assert_parity(got, oracle_conv(x, w, None, (1, 1), (2, 2, 2, 2), (2, 2)), "dilated")


def test_conv_padding_lanes_zero(gpu):
    """Channel lanes past Cout stay +0 even with an activation that maps 0 to a nonzero value."""
    r = rng(41)
    x = round_half(r.standard_normal((1, 8, 6, 6)))
    w = (r.standard_normal((6, 8, 1, 1))).astype(np.float32)
    _, _, dy = gpu_conv(x, w, None, act=3, lo=0.5, hi=2.0)
    raw = raw_nc4(dy, (1, 6, 6, 6)).reshape(1, 2, 6, 6, 4)
    assert np.all(raw[:, 1, :, :, 2:] == 0)


# ---------------------------------------------------------------- depthwise
@pytest.mark.parametrize("k,s,C,act", [(3, 1, 144, 2), (3, 2, 72, 1), (5, 1, 120, 4), (5, 2, 40, 0), (3, 1, 6, 2)])
def test_depthwise(gpu, k, s, C, act):
    r = rng(50 + k * 10 + s + C)
    x = round_half(r.standard_normal((2, C, 23, 21)))
    w = (r.standard_normal((C, 1, k, k)) * 0.3).astype(np.float32)
    b = (r.standard_normal(C) * 0.1).astype(np.float32)
    p = k // 2
    got, plan, _ = gpu_conv(x, w, b, (s, s), (p, p, p, p), group=C, act=act)
    assert plan.algo == V.CONV_DEPTHWISE
    assert_parity(got, oracle_conv(x, w, b, (s, s), (p, p, p, p), group=C, act=act), f"dw k{k} s{s}")


@pytest.mark.parametrize("shape,k,s,act,res", [((3, 20, 28, 28), 3, 1, 4, True), ((2, 24, 56, 56), 5, 2, 1, False),
                                               ((4, 160, 7, 7), 5, 1, 2, True), ((1, 16, 112, 112), 3, 2, 3, False),
                                               ((2, 6, 14, 13), 3, 1, 5, True)])
@pytest.mark.parametrize("rt", [4, 7, 14, 204, 207, 404, 407])
def test_depthwise_tiled_shapes(gpu, shape, k, s, act, res, rt):
    """Even/odd widths (16- and 8-byte row copies), several planes per workgroup, row tiles with
    halos (4, 7 or 14 output rows per strip, the plan's tile), 2 or 4 strips per workgroup with
    the next strip's input prefetched (tile 2xx / 4xx; odd widths fall back to one strip),
    residual epilogue, ragged channel count."""
    N, C, H, W = shape
    r = rng(70 + k + s + C)
    x = round_half(r.standard_normal(shape))
    w = (r.standard_normal((C, 1, k, k)) * 0.3).astype(np.float32)
    b = (r.standard_normal(C) * 0.1).astype(np.float32)
    p = k // 2
    OH, OW = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    rr = round_half(r.standard_normal((N, C, OH, OW))) if res else None
    lo, hi = (-0.5, 0.7) if act == 3 else (0.0, 0.0)
    got, plan, _ = gpu_conv(x, w, b, (s, s), (p, p, p, p), group=C, act=act, lo=lo, hi=hi, res=rr, algo=V.CONV_DEPTHWISE, tile=rt)
    assert plan.tile == rt
    ref = oracle_conv(x, w, b, (s, s), (p, p, p, p), group=C, res=rr, act=act, lo=lo, hi=hi)
    assert_parity(got, ref, f"dw {shape} k{k} s{s} rows/strip {rt}")


@pytest.mark.parametrize("shape,k,s,act,res,rt", [((128, 960, 7, 7), 5, 1, 4, False, 907), ((128, 480, 14, 14), 3, 1, 1, True, 914),
                                                  ((32, 88, 8, 8), 3, 2, 2, False, 904), ((9, 22, 7, 7), 3, 1, 5, True, 907),
                                                  ((128, 200, 14, 14), 5, 1, 4, False, 914)])
def test_depthwise_persistent_groups(gpu, shape, k, s, act, res, rt):
    """Persistent plane groups (tile 9xx): more groups than resident workgroups (each walks
    several, its channel blocks fixed by the grid size), the tile halo kept across groups, a last
    group with fewer planes, ragged channels, residual."""
    N, C, H, W = shape
    r = rng(310 + k + s + C)
    x = round_half(r.standard_normal(shape))
    w = (r.standard_normal((C, 1, k, k)) * 0.3).astype(np.float32)
    b = (r.standard_normal(C) * 0.1).astype(np.float32)
    p = k // 2
    OH, OW = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    rr = round_half(r.standard_normal((N, C, OH, OW))) if res else None
    got, plan, _ = gpu_conv(x, w, b, (s, s), (p, p, p, p), group=C, act=act, res=rr, algo=V.CONV_DEPTHWISE, tile=rt)
    assert plan.tile == rt
    ref = oracle_conv(x, w, b, (s, s), (p, p, p, p), group=C, res=rr, act=act)
    assert_parity(got, ref, f"dw persistent {shape} k{k} s{s} tile {rt}")


def test_depthwise_persistent_refuses_large_groups(gpu):
    """Tile 9xx needs one strip per plane and at most 4096 input pixels per plane group."""
    lib = V.vkhip()
    plan = V.ConvPlan()
    for xs, k, s, rt in [((2, 64, 28, 28), 3, 1, 907), ((2, 64, 14, 14), 3, 1, 907), ((2, 64, 56, 56), 3, 1, 914)]:
        d, _ = conv_desc(xs, (xs[1], 1, k, k), (s, s), (k // 2,) * 4, group=xs[1])
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_DEPTHWISE, rt, 0, ctypes.byref(plan)) != 0, (xs, k, s, rt)


def test_depthwise_dilated_generic(gpu):
    r = rng(55)
    x = round_half(r.standard_normal((1, 12, 16, 16)))
    w = (r.standard_normal((12, 1, 3, 3)) * 0.3).astype(np.float32)
    got, _, _ = gpu_conv(x, w, None, (1, 1), (2, 2, 2, 2), dil=(2, 2), group=12)
    assert_parity(got, oracle_conv(x, w, None, (1, 1), (2, 2, 2, 2), (2, 2), group=12), "dw dilated")


# ---------------------------------------------------------------- fused dw + pw
@pytest.mark.parametrize("N,E,H,k,s,Cout,dw_act,act,res", [(2, 144, 14, 3, 1, 24, 2, 0, True),
                                                           (1, 960, 7, 5, 1, 160, 1, 0, False),
                                                           (3, 72, 11, 3, 2, 40, 0, 1, False),
                                                           (1, 22, 9, 3, 1, 10, 2, 3, True),
                                                           (2, 144, 56, 3, 1, 24, 2, 0, True),
                                                           (1, 96, 40, 5, 2, 64, 1, 0, True),
                                                           (1, 40, 130, 3, 2, 24, 2, 0, False)])
@pytest.mark.parametrize("kernel", ["ring", "strip", "untiled"])
def test_fused_dwpw(gpu, monkeypatch, kernel, N, E, H, k, s, Cout, dw_act, act, res):
    """Each fused kernel (the launcher takes the first that fits: ring-staged for even input
    widths, strip-tiled, untiled; the environment switches the first two off) against the oracle."""
    monkeypatch.setenv("VKHIP_DWPW_RING", "1" if kernel == "ring" else "0")
    monkeypatch.setenv("VKHIP_DWPW_STRIP", "0" if kernel == "untiled" else "1")
    lib = V.vkhip()
    r = rng(E + Cout + H)
    x = round_half(r.standard_normal((N, E, H, H)))
    dw_w = (r.standard_normal((E, 1, k, k)) * 0.3).astype(np.float32)
    dw_b = (r.standard_normal(E) * 0.1).astype(np.float32)
    pw_w = (r.standard_normal((Cout, E)) * np.sqrt(1.0 / E)).astype(np.float32)
    pw_b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    p = k // 2
    OH = (H + 2 * p - k) // s + 1
    resid = round_half(r.standard_normal((N, Cout, OH, OH))) if res else None
    lo, hi = (-0.3, 0.4) if act == 3 else (0.0, 0.0)
    dwd, _ = conv_desc(x.shape, (E, 1, k, k), (s, s), (p, p, p, p), group=E, act=dw_act, lo=0.0, hi=6.0)
    d = V.DwPwDesc(dw=dwd, Cout=Cout, act=act, act_lo=lo, act_hi=hi, has_res=int(res))
    assert lib.vkhip_dwpw_supported(ctypes.byref(d)) == 1
    blob = np.zeros(lib.vkhip_dwpw_weight_bytes(ctypes.byref(d)), np.uint8)
    check(lib.vkhip_dwpw_pack_weights(ctypes.byref(d), dw_w.ctypes.data, dw_b.ctypes.data, pw_w.ctypes.data,
                                      pw_b.ctypes.data, blob.ctypes.data))
    dblob = DeviceBuffer.from_array(blob)
    dx = to_device_nc4(x)
    dres = to_device_nc4(resid) if res else None
    yshape = (N, Cout, OH, OH)
    dy = DeviceBuffer(V.nc4_elems(*yshape) * 2)
    check(lib.vkhip_dwpw_forward(ctypes.byref(d), dx.ptr, dblob.ptr, dres.ptr if dres else None, dy.ptr, None))
    check(lib.vkhip_stream_sync(None))
    got = from_device_nc4(dy, yshape)
    ref = oracle_dwpw(x, dw_w, dw_b, pw_w, pw_b, (s, s), (p, p, p, p), dw_act=dw_act, res=resid, act=act, lo=lo, hi=hi)
    assert_parity(got, ref, f"dwpw E{E} k{k} s{s}")


# ---------------------------------------------------------------- SE + pooling + element-wise
@pytest.mark.parametrize("N,C,H,Cr", [(3, 120, 14, 32), (128, 960, 7, 240), (5, 72, 9, 24)])
def test_gap_se_scale(gpu, N, C, H, Cr):
    lib = V.vkhip()
    o = oracle()
    r = rng(60)
    x = round_half(r.standard_normal((N, C, H, H)))
    dx = to_device_nc4(x)
    davg = DeviceBuffer(V.nc4_elems(N, C, 1, 1) * 2)
    check(lib.vkhip_global_avg_pool(dx.ptr, davg.ptr, N, C, H, H, None))
    avg_ref = np.zeros((N, C), np.float32)
    o.oracle_global_avg_pool(x.ctypes.data, avg_ref.ctypes.data, N, C, H * H)
    avg = from_device_nc4(davg, (N, C, 1, 1)).reshape(N, C)
    assert_parity(avg, avg_ref, "gap")
    w1 = (r.standard_normal((Cr, C)) * 0.2).astype(np.float32)
    b1 = (r.standard_normal(Cr) * 0.1).astype(np.float32)
    w2 = (r.standard_normal((C, Cr)) * 0.2).astype(np.float32)
    b2 = (r.standard_normal(C) * 0.1).astype(np.float32)
    blob = np.zeros(lib.vkhip_se_weight_bytes(C, Cr), np.uint8)
    check(lib.vkhip_se_pack_weights(C, Cr, w1.ctypes.data, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data, blob.ctypes.data))
    dblob = DeviceBuffer.from_array(blob)
    ds = DeviceBuffer(V.nc4_elems(N, C, 1, 1) * 2)
    dws = DeviceBuffer(lib.vkhip_se_workspace_bytes(N, Cr))
    check(lib.vkhip_fused_se(davg.ptr, dblob.ptr, ds.ptr, N, C, Cr, 1.0 / 6.0, 0.5, dws.ptr, None))
    avg16 = round_half(avg)
    s_ref = np.zeros((N, C), np.float32)
    o.oracle_fused_se(avg16.ctypes.data, N, C, w1.ctypes.data, Cr, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data,
                      1.0 / 6.0, 0.5, s_ref.ctypes.data)
    s = from_device_nc4(ds, (N, C, 1, 1)).reshape(N, C)
    assert_parity(s, s_ref, "fused_se")
    dy = DeviceBuffer(V.nc4_elems(N, C, H, H) * 2)
    check(lib.vkhip_channel_scale(dx.ptr, ds.ptr, dy.ptr, N, C, H * H, None))
    y = from_device_nc4(dy, (N, C, H, H))
    y_ref = np.zeros_like(x)
    s16 = round_half(s)
    o.oracle_mul_channel(x.ctypes.data, s16.ctypes.data, y_ref.ctypes.data, N, C, H * H)
    assert_parity(y, y_ref, "channel scale")


@pytest.mark.parametrize("act", [0, 1, 2, 3, 4, 5])
def test_add_act(gpu, act):
    lib = V.vkhip()
    r = rng(70 + act)
    shape = (2, 13, 9, 7)
    a = round_half(r.standard_normal(shape) * 4)
    b = round_half(r.standard_normal(shape) * 4)
    da, db = to_device_nc4(a), to_device_nc4(b)
    dy = DeviceBuffer(V.nc4_elems(*shape) * 2)
    check(lib.vkhip_add(da.ptr, db.ptr, dy.ptr, V.nc4_elems(*shape), act, -1.0, 2.0, None))
    ref = np.zeros(a.size, np.float32)
    oracle().oracle_add(a.ctypes.data, b.ctypes.data, ref.ctypes.data, a.size, act, -1.0, 2.0)
    assert_parity(from_device_nc4(dy, shape), ref, f"add act{act}")


@pytest.mark.parametrize("op,p0,p1", [(0, 0, 0), (2, 0, 0), (3, 1.0 / 6, 0.5), (13, 0, 0), (14, 0, 0), (-1, -0.5, 1.5)])
def test_unary(gpu, op, p0, p1):
    lib = V.vkhip()
    shape = (1, 10, 5, 5)
    x = round_half(rng(80).standard_normal(shape) * 4)
    dx = to_device_nc4(x)
    dy = DeviceBuffer(V.nc4_elems(*shape) * 2)
    check(lib.vkhip_unary(dx.ptr, dy.ptr, V.nc4_elems(*shape), op, p0, p1, None))
    ref = np.zeros(x.size, np.float32)
    oracle().oracle_unary(x.ctypes.data, ref.ctypes.data, x.size, op, p0, p1)
    assert_parity(from_device_nc4(dy, shape), ref, f"unary {op}")


def test_maxpool(gpu):
    lib = V.vkhip()
    shape = (2, 9, 17, 17)
    x = round_half(rng(90).standard_normal(shape))
    for k, s, p in [(3, 2, 1), (5, 1, 2)]:
        OH = (17 + 2 * p - k) // s + 1
        d = V.PoolDesc(N=2, C=9, H=17, W=17, OH=OH, OW=OH, KH=k, KW=k, SH=s, SW=s, PT=p, PL=p)
        dx = to_device_nc4(x)
        dy = DeviceBuffer(V.nc4_elems(2, 9, OH, OH) * 2)
        check(lib.vkhip_maxpool(ctypes.byref(d), dx.ptr, dy.ptr, None))
        ref = np.zeros((2, 9, OH, OH), np.float32)
        oracle().oracle_maxpool(x.ctypes.data, ref.ctypes.data, 2, 9, 17, 17, k, k, s, s, p, p, OH, OH)
        got = from_device_nc4(dy, (2, 9, OH, OH))
        assert np.array_equal(got, ref), f"maxpool k{k}"  # max of fp16 values is exact


@pytest.mark.parametrize("shape,k", [((16, 128, 20, 20), 5), ((2, 9, 17, 23), 3), ((1, 6, 1, 30), 5), ((3, 4, 40, 56), 5), ((1, 8, 10, 62), 3),
                                     ((1, 4, 8, 70), 5), ((2, 12, 3, 3), 5)])
def test_maxpool_same(gpu, shape, k):
    """"Same" max pools (KxK, stride 1, pad K/2; the SPPF pools) on the LDS plane kernel: exact
    against the oracle, widths above 64 columns, windows larger than the image; then written into
    a channel slice of a wider tensor through vkhip_maxpool_view (the in-place concat of SPPF)."""
    lib = V.vkhip()
    N, C, H, W = shape
    x = round_half(rng(95 + H + W + k).standard_normal(shape) * 3)
    p = k // 2
    d = V.PoolDesc(N=N, C=C, H=H, W=W, OH=H, OW=W, KH=k, KW=k, SH=1, SW=1, PT=p, PL=p)
    dx = to_device_nc4(x)
    dy = DeviceBuffer(V.nc4_elems(N, C, H, W) * 2)
    check(lib.vkhip_maxpool(ctypes.byref(d), dx.ptr, dy.ptr, None))
    ref = np.zeros((N, C, H, W), np.float32)
    oracle().oracle_maxpool(x.ctypes.data, ref.ctypes.data, N, C, H, W, k, k, 1, 1, p, p, H, W)
    assert np.array_equal(from_device_nc4(dy, (N, C, H, W)), ref)
    if C % 4 == 0:
        Ct = 2 * C
        dw = DeviceBuffer(V.nc4_elems(N, Ct, H, W) * 2)
        dw.zero()
        check(lib.vkhip_maxpool_view(ctypes.byref(d), dx.ptr, 0, dw.ptr + (C // 4) * H * W * 8, Ct // 4, None))
        wide = from_device_nc4(dw, (N, Ct, H, W))
        assert np.array_equal(wide[:, C:], ref) and not wide[:, :C].any()


@pytest.mark.parametrize("count,k", [(3, 5), (2, 3), (4, 5), (1, 5)])
def test_maxpool_chain(gpu, count, k):
    """vkhip_maxpool_chain (the SPPF pools in one launch): every output bit-identical to the oracle
    pool applied 1..count times, the outputs written into channel slices of one wide tensor (the
    in-place concat) with the input in another; the other slices untouched."""
    lib = V.vkhip()
    N, C, H, W = 2, 8, 20, 20
    x = round_half(rng(97 + count + k).standard_normal((N, C, H, W)) * 3)
    p = k // 2
    d = V.PoolDesc(N=N, C=C, H=H, W=W, OH=H, OW=W, KH=k, KW=k, SH=1, SW=1, PT=p, PL=p)
    Ct = C * (count + 1)
    wide = np.zeros((N, Ct, H, W), np.float32)
    wide[:, :C] = x
    dw = to_device_nc4(wide)
    plane = H * W * 8
    ys = (ctypes.c_void_p * 4)(*[dw.ptr + (c + 1) * (C // 4) * plane for c in range(count)] + [None] * (4 - count))
    ps = (ctypes.c_int64 * 4)(*([Ct // 4] * 4))
    check(lib.vkhip_maxpool_chain(ctypes.byref(d), dw.ptr, Ct // 4, ys, ps, count, None), "maxpool chain")
    got = from_device_nc4(dw, wide.shape)
    assert np.array_equal(got[:, :C], x)
    cur = x
    for c in range(count):
        ref = np.zeros_like(cur)
        oracle().oracle_maxpool(np.ascontiguousarray(cur).ctypes.data, ref.ctypes.data, N, C, H, W, k, k, 1, 1, p, p, H, W)
        assert np.array_equal(got[:, (c + 1) * C:(c + 2) * C], ref), c
        cur = ref
    bad = (ctypes.c_void_p * 4)(dw.ptr, None, None, None)
    assert lib.vkhip_maxpool_chain(ctypes.byref(d), dw.ptr, 0, bad, ps, 5, None) != 0


@pytest.mark.parametrize("shape,pb", [((2, 9, 18, 18), 1), ((1, 8, 16, 20), 1), ((3, 5, 15, 20), 0), ((2, 4, 15, 12), 1),
                                      ((1, 64, 112, 112), 1), ((2, 7, 2, 2), 1), ((1, 4, 1, 6), 1)])
def test_maxpool_3x3_s2_pairs(gpu, shape, pb):
    """The stem-pool kernel (3x3 s2, pad 1 left/top, even W): odd and even output widths and
    heights, bottom/right pad 0 or 1, a single-row input. Exact against the oracle, including the
    -inf-free edges (every output has at least one in-image tap)."""
    lib = V.vkhip()
    N, C, H, W = shape
    x = round_half(rng(91 + H + W).standard_normal(shape) * 3)
    OH, OW = (H + 1 + pb - 3) // 2 + 1, (W + 1 + pb - 3) // 2 + 1
    d = V.PoolDesc(N=N, C=C, H=H, W=W, OH=OH, OW=OW, KH=3, KW=3, SH=2, SW=2, PT=1, PL=1)
    dx = to_device_nc4(x)
    dy = DeviceBuffer(V.nc4_elems(N, C, OH, OW) * 2)
    check(lib.vkhip_maxpool(ctypes.byref(d), dx.ptr, dy.ptr, None))
    ref = np.zeros((N, C, OH, OW), np.float32)
    oracle().oracle_maxpool(x.ctypes.data, ref.ctypes.data, N, C, H, W, 3, 3, 2, 2, 1, 1, OH, OW)
    got = from_device_nc4(dy, (N, C, OH, OW))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("N,K,M,act", [(5, 2048, 1000, 0), (64, 2048, 1000, 0), (33, 1000, 37, 1), (1, 7, 3, 2), (130, 1280, 1000, 0)])
def test_fc(gpu, N, K, M, act):
    """Skinny GEMM kernel: partial n tiles (N % 32), K not a multiple of 16 or 4, M not a
    multiple of 16 or 4, fused ReLU / ReLU6."""
    lib = V.vkhip()
    r = rng(100 + N + K)
    x = round_half(r.standard_normal((N, K)))
    w = (r.standard_normal((M, K)) * 0.02).astype(np.float32)
    b = (r.standard_normal(M) * 0.1).astype(np.float32)
    blob = np.zeros(lib.vkhip_fc_weight_bytes(K, M), np.uint8)
    check(lib.vkhip_fc_pack_weights(K, M, w.ctypes.data, 1, b.ctypes.data, 1.0, 1.0, blob.ctypes.data))
    dblob = DeviceBuffer.from_array(blob)
    dx = to_device_nc4(x.reshape(N, K, 1, 1))
    dy = DeviceBuffer(V.nc4_elems(N, M, 1, 1) * 2)
    check(lib.vkhip_fc(dx.ptr, dblob.ptr, dy.ptr, N, K, M, act, 0.0, 6.0, None))
    ref = np.zeros((N, M), np.float32)
    oracle().oracle_gemm(x.ctypes.data, w.ctypes.data, b.ctypes.data, ref.ctypes.data, N, K, M, 1, 1.0, 1.0, act, 0.0, 6.0)
    assert_parity(from_device_nc4(dy, (N, M, 1, 1)).reshape(N, M), ref, "fc")
    # the padding lanes of the last channel block are zero
    if M % 4:
        check(lib.vkhip_stream_sync(None))
        raw = dy.download(np.uint16, V.nc4_elems(N, M, 1, 1)).reshape(N, -1)
        assert not raw[:, M:].any()


@pytest.mark.parametrize("shape", [(2, 13, 5, 7, 10, 14), (1, 8, 4, 6, 12, 6), (3, 4, 6, 5, 6, 15), (16, 256, 20, 20, 40, 40),
                                   (1, 4, 3, 300, 6, 600), (2, 6, 5, 5, 7, 9), (2, 64, 1, 1, 3, 2)])
def test_resize_nearest_factors(gpu, shape):
    """Nearest resize: integer factors (2x2 with odd and even widths, 3x1, 1x3, the detector-neck
    2x at 20x20, a 1x1 image) on the division-free kernel, a width above 256 and a non-integer
    factor on the generic one. Integer factors: bit-equal to the oracle's nearest under half_pixel
    coordinates (and under asymmetric ones at 2x); every shape: bit-equal to floor indexing."""
    lib, o = V.vkhip(), oracle()
    N, C, H, W, OH, OW = shape
    x = round_half(rng(120 + H + W).standard_normal((N, C, H, W)))
    dx = to_device_nc4(x)
    dy = DeviceBuffer(V.nc4_elems(N, C, OH, OW) * 2)
    check(lib.vkhip_resize_nearest(dx.ptr, dy.ptr, N, C, H, W, OH, OW, None))
    got = from_device_nc4(dy, (N, C, OH, OW))
    iy, ix = (np.arange(OH) * H) // OH, (np.arange(OW) * W) // OW
    assert np.array_equal(got, x[:, :, iy][:, :, :, ix])
    if OH % H == 0 and OW % W == 0:
        modes = [0] + ([2] if max(OH // H, OW // W) <= 2 else [])
        for mode in modes:
            want = np.zeros((N, C, OH, OW), np.float32)
            o.oracle_resize_nearest(np.ascontiguousarray(x).ctypes.data, want.ctypes.data, N * C, H, W, OH, OW, mode)
            assert np.array_equal(got, want), mode


def test_concat_slice_resize(gpu):
    lib = V.vkhip()
    o = oracle()
    r = rng(110)
    N, H = 2, 6
    parts = [round_half(r.standard_normal((N, c, H, H))) for c in (8, 6, 5, 4)]
    dparts = [to_device_nc4(p) for p in parts]
    cs = np.array([p.shape[1] for p in parts], np.int64)
    Ct = int(cs.sum())
    dy = DeviceBuffer(V.nc4_elems(N, Ct, H, H) * 2)
    ptrs = (ctypes.c_void_p * 4)(*[d.ptr for d in dparts])
    check(lib.vkhip_concat_channels(ptrs, cs.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), 4, dy.ptr, N, H * H, None))
    got = from_device_nc4(dy, (N, Ct, H, H))
    ref = np.concatenate(parts, axis=1)
    assert np.array_equal(got, ref)
    raw = raw_nc4(dy, (N, Ct, H, H)).reshape(N, -1, H, H, 4)
    assert np.all(raw[:, -1, :, :, Ct % 4:] == 0)  # padding lanes stay zero
    for c0, c in [(0, 8), (8, 6), (14, 9), (3, 5)]:
        ds = DeviceBuffer(V.nc4_elems(N, c, H, H) * 2)
        check(lib.vkhip_slice_channels(dy.ptr, ds.ptr, N, Ct, c0, c, H * H, None))
        assert np.array_equal(from_device_nc4(ds, (N, c, H, H)), ref[:, c0:c0 + c])
    dr = DeviceBuffer(V.nc4_elems(N, Ct, 2 * H, 2 * H) * 2)
    check(lib.vkhip_resize_nearest(dy.ptr, dr.ptr, N, Ct, H, H, 2 * H, 2 * H, None))
    want = np.zeros((N, Ct, 2 * H, 2 * H), np.float32)
    o.oracle_resize_nearest(ref.ctypes.data, want.ctypes.data, N * Ct, H, H, 2 * H, 2 * H, 2)
    assert np.array_equal(from_device_nc4(dr, (N, Ct, 2 * H, 2 * H)), want)


def test_binary_same_shape(gpu):
    lib = V.vkhip()
    r = rng(120)
    shape = (1, 9, 4, 4)
    a = round_half(r.standard_normal(shape))
    b = round_half(r.standard_normal(shape) + 3)
    for op in (0, 1, 2, 3, 4, 6):
        da, db = to_device_nc4(a), to_device_nc4(b)
        dy = DeviceBuffer(V.nc4_elems(*shape) * 2)
        check(lib.vkhip_binary(da.ptr, db.ptr, dy.ptr, V.nc4_elems(*shape), op, None))
        ref = np.zeros(a.size, np.float32)
        oracle().oracle_binary(a.ctypes.data, b.ctypes.data, ref.ctypes.data, a.size, op)
        assert_parity(from_device_nc4(dy, shape), ref, f"binary {op}")


def test_graph_capture_replay(gpu):
    """A conv captured into a HIP graph replays to the eager result, several times, with eager work
    and synchronisation between replays."""
    lib = V.vkhip()
    r = rng(130)
    x = round_half(r.standard_normal((2, 64, 14, 14)))
    w = (r.standard_normal((64, 64, 3, 3)) * 0.05).astype(np.float32)
    eager, plan, _ = gpu_conv(x, w, None, (1, 1), (1, 1, 1, 1), act=1, algo=V.CONV_GEMM, tile=3)
    d, yshape = conv_desc(x.shape, w.shape, (1, 1), (1, 1, 1, 1), act=1)
    blob = np.zeros(plan.weight_bytes, np.uint8)
    check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, None, blob.ctypes.data))
    dblob = DeviceBuffer.from_array(blob)
    dx = to_device_nc4(x)
    dy = DeviceBuffer(V.nc4_elems(*yshape) * 2)
    s = ctypes.c_void_p()
    check(lib.vkhip_stream_create(ctypes.byref(s)))
    g = ctypes.c_void_p()
    check(lib.vkhip_graph_begin(s))
    check(lib.vkhip_conv_forward(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr, None, dy.ptr, None, s))
    check(lib.vkhip_graph_end(s, ctypes.byref(g)))
    for _ in range(3):
        dy.zero()
        check(lib.vkhip_stream_sync(None))
        check(lib.vkhip_graph_launch(g, s))
        check(lib.vkhip_stream_sync(s))
        assert np.array_equal(from_device_nc4(dy, yshape), eager)
    check(lib.vkhip_graph_destroy(g))
    check(lib.vkhip_stream_destroy(s))


def test_invalid_arguments_rejected(gpu):
    lib = V.vkhip()
    d, _ = conv_desc((1, 8, 5, 5), (8, 8, 3, 3), (1, 1), (1, 1, 1, 1))
    plan = V.ConvPlan()
    d.group = 2  # grouped but not depthwise
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_AUTO, -1, 0, ctypes.byref(plan)) == 2
    d.group = 1
    d.KH = 0
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_AUTO, -1, 0, ctypes.byref(plan)) == 1
    d2, _ = conv_desc((1, 8, 5, 5), (8, 8, 3, 3), (2, 2), (1, 1, 1, 1))
    assert lib.vkhip_conv_plan_make(ctypes.byref(d2), V.CONV_WINOGRAD, -1, 0, ctypes.byref(plan)) == 1


XS_TILES = [14, 16, 24, 25]  # conv_dma_kernel tiles with the input-scale (squeeze-excite) variant


@pytest.mark.parametrize("tile", XS_TILES)
@pytest.mark.parametrize("shape", [(3, 72, 14, 14, 40), (5, 960, 7, 7, 160), (2, 120, 28, 28, 40), (7, 36, 5, 9, 24)])
def test_conv_input_scale(gpu, tile, shape):
    """1x1 conv on x * s with s of shape [N,C,1,1] (a squeeze-excite scale folded into the conv):
    equals the separate channel-broadcast Mul (fp16 store) followed by the same conv plan, bit for
    bit, and the oracle conv of the fp16-rounded product within the tolerance. Shapes cover odd
    pixel counts per image (padding columns), several images per tile, K tails, residual."""
    lib = V.vkhip()
    N, C, H, W, Co = shape
    r = rng(700 + tile + C)
    x = round_half(r.standard_normal((N, C, H, W)))
    s = round_half(r.uniform(0.0, 1.0, (N, C, 1, 1)))
    w = (r.standard_normal((Co, C, 1, 1)) * 0.1).astype(np.float32)
    b = (r.standard_normal(Co) * 0.1).astype(np.float32)
    res = round_half(r.standard_normal((N, Co, H, W)))
    d, yshape = conv_desc(x.shape, w.shape, act=1, has_res=1)
    d.in_scale = 1
    plan = V.ConvPlan()
    rc = lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_GEMM, tile, 0, ctypes.byref(plan))
    if rc:
        pytest.skip(f"tile {tile} takes no input scale at {shape}: {lib.vkhip_last_error().decode(errors='replace')}")
    blob = np.zeros(plan.weight_bytes, np.uint8)
    check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, b.ctypes.data, blob.ctypes.data))
    dblob = DeviceBuffer.from_array(blob)
    dx, ds, dres = to_device_nc4(x), to_device_nc4(s), to_device_nc4(res)
    nbytes = V.nc4_elems(*yshape) * 2
    dy = DeviceBuffer(nbytes)
    check(lib.vkhip_conv_forward_scaled(ctypes.byref(d), ctypes.byref(plan), dx.ptr, ds.ptr, dblob.ptr, dres.ptr, dy.ptr, None, None))
    # the unfused pair: channel-broadcast Mul into an fp16 tensor, then the same plan without scale
    dt = DeviceBuffer(V.nc4_elems(N, C, H, W) * 2)
    check(lib.vkhip_channel_scale(dx.ptr, ds.ptr, dt.ptr, N, C, H * W, None))
    d0, _ = conv_desc(x.shape, w.shape, act=1, has_res=1)
    dy0 = DeviceBuffer(nbytes)
    check(lib.vkhip_conv_forward(ctypes.byref(d0), ctypes.byref(plan), dt.ptr, dblob.ptr, dres.ptr, dy0.ptr, None, None))
    check(lib.vkhip_stream_sync(None))
    a, u = dy.download(np.uint16, nbytes // 2), dy0.download(np.uint16, nbytes // 2)
    assert np.array_equal(a, u), f"{np.count_nonzero(a != u)} of {a.size} fp16 values differ from Mul + conv"
    got = from_device_nc4(dy, yshape)
    assert_parity(got, oracle_conv(round_half(x * s), w, b, res=res, act=1), f"input-scale conv tile {tile} {shape}")


def test_conv_input_scale_rejects_other_shapes(gpu):
    lib = V.vkhip()
    for wshape, stride in [((8, 16, 3, 3), (1, 1)), ((8, 16, 1, 1), (2, 2))]:
        d, _ = conv_desc((2, 16, 8, 8), wshape, stride=stride, pads=(1, 1, 1, 1) if wshape[2] == 3 else (0, 0, 0, 0))
        d.in_scale = 1
        plan = V.ConvPlan()
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_AUTO, -1, 0, ctypes.byref(plan)) == 2


@pytest.mark.parametrize("N,C,Cr,R,HW", [(20, 960, 240, 1, 49), (3, 72, 24, 4, 784), (33, 120, 32, 2, 784), (16, 672, 168, 1, 196)])
def test_se_pooled(gpu, N, C, Cr, R, HW):
    """vkhip_fused_se_pooled (pooled partial sums -> FC1 -> FC2 -> hard-sigmoid; image counts
    that are not a multiple of the kernels' image groups) against a float64 restatement: x = fp16(sum of the partials / HW),
    h = fp16(relu(W1 x + b1)), y = clamp(alpha (W2 h + b2) + beta, 0, 1), weights rounded to fp16."""
    lib = V.vkhip()
    r = rng(500 + C + N)
    Cb = (C + 3) // 4
    part = (r.standard_normal((N, Cb, R, 4)) * HW * 0.3).astype(np.float32)
    w1 = (r.standard_normal((Cr, C)) * 0.1).astype(np.float32)
    b1 = (r.standard_normal(Cr) * 0.1).astype(np.float32)
    w2 = (r.standard_normal((C, Cr)) * 0.2).astype(np.float32)
    b2 = (r.standard_normal(C) * 0.1).astype(np.float32)
    blob = np.zeros(lib.vkhip_se_weight_bytes(C, Cr), np.uint8)
    check(lib.vkhip_se_pack_weights(C, Cr, w1.ctypes.data, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data, blob.ctypes.data))
    dblob, dpart = DeviceBuffer.from_array(blob), DeviceBuffer.from_array(part)
    ws = DeviceBuffer(lib.vkhip_se_workspace_bytes(N, Cr))
    out = DeviceBuffer(V.nc4_elems(N, C, 1, 1) * 2)
    check(lib.vkhip_fused_se_pooled(dpart.ptr, R, HW, dblob.ptr, out.ptr, N, C, Cr, 1.0 / 6, 0.5, ws.ptr, None))
    check(lib.vkhip_stream_sync(None))
    got = from_device_nc4(out, (N, C, 1, 1)).reshape(N, C)
    f16 = lambda a: np.asarray(a, np.float64).astype(np.float16).astype(np.float64)
    x = f16(part.astype(np.float64).sum(2).reshape(N, Cb * 4)[:, :C].astype(np.float32) / np.float32(HW))
    h = f16(np.maximum(x @ f16(w1).T + b1, 0.0))
    ref = np.clip((h @ f16(w2).T + b2) / 6 + 0.5, 0.0, 1.0)
    assert_parity(got, ref, f"se pooled N{N} C{C} Cr{Cr}")


@pytest.mark.parametrize("pooled", [False, True])
@pytest.mark.parametrize("N,C,Cr", [(128, 960, 240), (128, 72, 24), (128, 120, 32), (128, 480, 120), (128, 672, 168), (1, 960, 240),
                                    (37, 240, 64), (200, 96, 24)])
def test_se_matches_two_fc_launches(gpu, N, C, Cr, pooled):
    """vkhip_fused_se / vkhip_fused_se_pooled against vkhip_fc (or vkhip_fc_pooled) for FC1 and
    vkhip_fc for FC2 on the same blob (the SE blob is the two fc blobs, W2's at the next 256-byte
    boundary): the same bits, on two calls in a row over one workspace."""
    lib = V.vkhip()
    r = rng(900 + C + N + pooled)
    Cb, R, HW = (C + 3) // 4, 2, 49
    w1 = (r.standard_normal((Cr, C)) * 0.1).astype(np.float32)
    b1 = (r.standard_normal(Cr) * 0.1).astype(np.float32)
    w2 = (r.standard_normal((C, Cr)) * 0.2).astype(np.float32)
    b2 = (r.standard_normal(C) * 0.1).astype(np.float32)
    blob = np.zeros(lib.vkhip_se_weight_bytes(C, Cr), np.uint8)
    check(lib.vkhip_se_pack_weights(C, Cr, w1.ctypes.data, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data, blob.ctypes.data))
    w1_bytes = lib.vkhip_fc_weight_bytes(C, Cr)
    w2_off = (w1_bytes + 255) // 256 * 256
    dblob = DeviceBuffer.from_array(blob)
    if pooled:
        src = DeviceBuffer.from_array((r.standard_normal((N, Cb, R, 4)) * HW * 0.3).astype(np.float32))
    else:
        src = to_device_nc4(round_half(r.standard_normal((N, C, 1, 1))))
    nbytes = V.nc4_elems(N, C, 1, 1) * 2
    ws_bytes = lib.vkhip_se_workspace_bytes(N, Cr)
    ws = DeviceBuffer(ws_bytes)
    ws.zero()
    hid, ref = DeviceBuffer(V.nc4_elems(N, Cr, 1, 1) * 2), DeviceBuffer(nbytes)
    if pooled:
        check(lib.vkhip_fc_pooled(src.ptr, R, HW, dblob.ptr, hid.ptr, N, C, Cr, 1, 0.0, 0.0, None))
    else:
        check(lib.vkhip_fc(src.ptr, dblob.ptr, hid.ptr, N, C, Cr, 1, 0.0, 0.0, None))
    check(lib.vkhip_fc(hid.ptr, dblob.ptr + w2_off, ref.ptr, N, Cr, C, 6, 1.0 / 6, 0.5, None))
    want = None
    for call in range(2):
        out = DeviceBuffer(nbytes)
        out.zero()
        if pooled:
            check(lib.vkhip_fused_se_pooled(src.ptr, R, HW, dblob.ptr, out.ptr, N, C, Cr, 1.0 / 6, 0.5, ws.ptr, None))
        else:
            check(lib.vkhip_fused_se(src.ptr, dblob.ptr, out.ptr, N, C, Cr, 1.0 / 6, 0.5, ws.ptr, None))
        check(lib.vkhip_stream_sync(None))
        want = ref.download(np.uint16, nbytes // 2) if want is None else want
        got = out.download(np.uint16, nbytes // 2)
        assert np.array_equal(got, want), f"call {call}: {np.count_nonzero(got != want)} of {got.size} fp16 values differ"


# ---------------------------------------------------------------- depthwise + squeeze-excite pool sums
@pytest.mark.parametrize("shape,k,s,rt", [((3, 72, 28, 28), 3, 2, 7), ((2, 120, 28, 28), 5, 1, 4), ((4, 960, 7, 7), 5, 1, 7),
                                          ((2, 22, 14, 14), 3, 1, 14), ((5, 40, 56, 56), 5, 2, 4),
                                          ((3, 120, 28, 28), 5, 1, 207), ((4, 72, 56, 56), 3, 1, 404), ((128, 960, 7, 7), 5, 1, 907),
                                          ((96, 120, 14, 14), 3, 1, 914)])
def test_depthwise_pool_sums(gpu, shape, k, s, rt):
    """vkhip_conv_forward_pooled writes exactly the depthwise output of vkhip_conv_forward and the
    per-(plane, row tile) sums of it; a squeeze-excite fed from those sums (vkhip_fused_se_pooled)
    matches the one fed by vkhip_global_avg_pool on the stored output (the fp32 sums are formed in
    another order, so the fp16 averages may differ by one rounding step)."""
    lib = V.vkhip()
    N, C, H, W = shape
    r = rng(90 + C + k)
    x = round_half(r.standard_normal(shape))
    w = (r.standard_normal((C, 1, k, k)) * 0.3).astype(np.float32)
    b = (r.standard_normal(C) * 0.1).astype(np.float32)
    p = k // 2
    ref, plan, dref = gpu_conv(x, w, b, (s, s), (p, p, p, p), group=C, act=4, algo=V.CONV_DEPTHWISE, tile=rt)
    d, yshape = conv_desc(x.shape, w.shape, (s, s), (p, p, p, p), (1, 1), C, 4, 0.0, 0.0, 0)
    R = lib.vkhip_conv_pool_parts(ctypes.byref(d), ctypes.byref(plan))
    OH = yshape[2]
    assert R == -(-OH // (rt % 100))
    blob = np.zeros(plan.weight_bytes, np.uint8)
    check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, b.ctypes.data, blob.ctypes.data))
    dblob = DeviceBuffer.from_array(blob)
    dx = to_device_nc4(x)
    dy = DeviceBuffer(V.nc4_elems(*yshape) * 2)
    Cb = (C + 3) // 4
    dpart = DeviceBuffer(N * Cb * R * 16)
    check(lib.vkhip_conv_forward_pooled(ctypes.byref(d), ctypes.byref(plan), dx.ptr, dblob.ptr, None, dy.ptr, dpart.ptr, None))
    check(lib.vkhip_stream_sync(None))
    assert np.array_equal(raw_nc4(dy, yshape), raw_nc4(dref, yshape))
    part = dpart.download(np.float32, N * Cb * R * 4).reshape(N, Cb, R, 4)
    y = from_device_nc4(dy, yshape).astype(np.float64)
    sums = y.reshape(N, C, -1).sum(-1)
    got = part.sum(2).reshape(N, Cb * 4)[:, :C]
    np.testing.assert_allclose(got, sums, rtol=1e-5, atol=1e-3)
    # squeeze-excite from the sums vs from the pooled tensor
    Cr = max(8, C // 4)
    w1 = (r.standard_normal((Cr, C)) * 0.2).astype(np.float32)
    b1 = (r.standard_normal(Cr) * 0.1).astype(np.float32)
    w2 = (r.standard_normal((C, Cr)) * 0.2).astype(np.float32)
    b2 = (r.standard_normal(C) * 0.1).astype(np.float32)
    sblob = np.zeros(lib.vkhip_se_weight_bytes(C, Cr), np.uint8)
    check(lib.vkhip_se_pack_weights(C, Cr, w1.ctypes.data, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data, sblob.ctypes.data))
    dsb = DeviceBuffer.from_array(sblob)
    davg = DeviceBuffer(V.nc4_elems(N, C, 1, 1) * 2)
    check(lib.vkhip_global_avg_pool(dy.ptr, davg.ptr, N, C, OH, yshape[3], None))
    ws = DeviceBuffer(lib.vkhip_se_workspace_bytes(N, Cr))
    o1, o2 = DeviceBuffer(V.nc4_elems(N, C, 1, 1) * 2), DeviceBuffer(V.nc4_elems(N, C, 1, 1) * 2)
    check(lib.vkhip_fused_se(davg.ptr, dsb.ptr, o1.ptr, N, C, Cr, 1.0 / 6, 0.5, ws.ptr, None))
    check(lib.vkhip_fused_se_pooled(dpart.ptr, R, OH * yshape[3], dsb.ptr, o2.ptr, N, C, Cr, 1.0 / 6, 0.5, ws.ptr, None))
    check(lib.vkhip_stream_sync(None))
    a1 = from_device_nc4(o1, (N, C, 1, 1))
    a2 = from_device_nc4(o2, (N, C, 1, 1))
    np.testing.assert_allclose(a2, a1, atol=4e-3)
    assert parity(a2, a1)[1] >= 0.99999


def test_pool_sums_reject_untiled_plan(gpu):
    lib = V.vkhip()
    d, _ = conv_desc((1, 12, 16, 16), (12, 1, 3, 3), (1, 1), (2, 2, 2, 2), (2, 2), 12, 0, 0.0, 0.0, 0)
    plan = V.ConvPlan()
    check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_DEPTHWISE, -1, 0, ctypes.byref(plan)))
    assert lib.vkhip_conv_pool_parts(ctypes.byref(d), ctypes.byref(plan)) == 0
