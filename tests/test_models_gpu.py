"""Network-level parity: the vknn Session on the HIP backend (through include/vknn_c.h) against the
CPU oracle on the same seeded graphs and inputs. Bar: max|d|/max|ref| <= 2e-2, cosine >= 0.9999
per output tensor. The input is fp32 NCHW on both sides (the HIP path packs it to fp16 itself)."""
import numpy as np
import pytest

import vknn_amd as V
from tests.oracle_lib import oracle_model_run, parity

pytestmark = pytest.mark.gpu

REL_TOL, COS_TOL = 2e-2, 0.9999


def check_outputs(got, ref, outs, what):
    off = 0
    for k, n in enumerate(outs):
        rel, cos = parity(got[off:off + n], ref[off:off + n])
        print(f"{what} out{k}: max_rel={rel:.2e} cos={cos:.7f}", flush=True)
        assert rel <= REL_TOL and cos >= COS_TOL, (what, k, rel, cos)
        off += n


def make_input(shape, seed, uniform=False):
    r = np.random.default_rng(seed)
    if uniform:
        return r.uniform(-1, 1, size=shape).astype(np.float32)
    return r.standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("model,batch,opts", [
    ("conv_tiny", 2, ""),
    ("mnv2_tiny", 2, ""),
    ("mnv2_tiny", 2, "fuse_dwpw=1"),
    ("resnet_tiny", 3, ""),
    ("resnet_tiny", 2, "winograd=on"),
    ("mnv3_tiny", 2, ""),
    ("mnv3_tiny", 2, "fuse_se=1;fuse_dwpw=1"),
    ("yolo_tiny", 2, ""),
    ("resnet_tiny", 2, "tuning=off;graphs=0"),
    ("resnet_tiny", 3, "VKNN_HIP_REFINE=0"),
    ("yolo_tiny", 2, "VKNN_HIP_REFINE=0"),
    ("mnv3_tiny", 2, "VKNN_HIP_FOLD_ACT=0"),
    ("yolo_tiny", 2, "VKNN_HIP_FOLD_ADD=0"),
    ("mnv3_tiny", 2, "VKNN_HIP_AUTO_SE=0"),
    ("mnv3_tiny", 2, "hip_auto_se=0"),
    ("mnv2_tiny", 2, "hip_auto_dwpw=0"),
    ("mnv3_tiny", 2, "hip_auto_se=0;hip_auto_dwpw=0"),
])
def test_tiny_models(gpu, monkeypatch, model, batch, opts):
    if opts.startswith("VKNN_"):  # an environment switch of the backend, not a session option
        monkeypatch.setenv(*opts.split("="))
        opts = ""
    sess = V.Session(model, batch, seed=11, options=opts)
    x = make_input(sess.in_shape, 5)
    got = sess.run(x)
    ref = oracle_model_run(model, batch, 11, x)
    check_outputs(got, ref, sess.out_elems, f"{model}[{opts}]")
    # a second and third run replay the captured graph and must give the same bits
    assert np.array_equal(sess.run(x), got)
    assert np.array_equal(sess.run(x), got)


def test_config0_conv3x3_bn_relu(gpu):
    sess = V.Session("conv3x3_bn_relu", 1, seed=7)
    x = make_input(sess.in_shape, 0, uniform=True)
    check_outputs(sess.run(x), oracle_model_run("conv3x3_bn_relu", 1, 7, x), sess.out_elems, "config0")


@pytest.mark.parametrize("opts", ["", "fuse_dwpw=1"])
def test_config1_mnv2_block(gpu, opts):
    sess = V.Session("mnv2_block", 1, seed=7, options=opts)
    x = make_input(sess.in_shape, 1)
    check_outputs(sess.run(x), oracle_model_run("mnv2_block", 1, 7, x), sess.out_elems, f"config1[{opts}]")


def test_config2_resnet50_b1(gpu):
    sess = V.Session("resnet50", 1, seed=7)
    x = make_input(sess.in_shape, 2)
    check_outputs(sess.run(x), oracle_model_run("resnet50", 1, 7, x), sess.out_elems, "resnet50 b1")


def test_device_input_path_matches_host_path(gpu):
    """Binding a device-resident fp32 input gives the same bits as the host upload path."""
    sess = V.Session("resnet_tiny", 2, seed=3)
    x = make_input(sess.in_shape, 9)
    host = sess.run(x)
    dx = V.DeviceBuffer.from_array(x)
    sess.bind_device_input(dx.ptr)
    for _ in range(3):
        sess.run_device()
        sess.sync()
        assert np.array_equal(sess.read_outputs(), host)


@pytest.mark.parametrize("fmt", [0, 1, 2])
@pytest.mark.parametrize("f16", [False, True])
def test_declared_format_device_input(gpu, fmt, f16):
    """A device input declared as NCHW/NHWC/NC4HW4 in fp32 or fp16 gives the host path's bits when
    the values are fp16-representable (then the boundary converter's round-to-nearest-even and the
    host codec agree)."""
    from tests.test_boundary_convert import to_fmt
    sess = V.Session("resnet_tiny", 2, seed=3)
    x16 = make_input(sess.in_shape, 11).astype(np.float16)
    host = sess.run(x16.astype(np.float32))
    src = x16.view(np.uint16) if f16 else x16.astype(np.float32)
    dx = V.DeviceBuffer.from_array(to_fmt(src.reshape(sess.in_shape), fmt))
    sess.bind_device_input_as(dx.ptr, fmt, f16)
    for _ in range(2):
        sess.run_device()
        sess.sync()
        assert np.array_equal(sess.read_outputs(), host)
    with pytest.raises(V.VkhipError, match="declared input layout"):
        sess.bind_device_input_as(dx.ptr, 3, f16)


def test_batch_items_independent(gpu):
    """Item k of a batched run equals a batch-1 run on image k (convs are per-image)."""
    sb = V.Session("resnet_tiny", 4, seed=3)
    s1 = V.Session("resnet_tiny", 1, seed=3)
    x = make_input(sb.in_shape, 4)
    yb = sb.run(x).reshape(4, -1)
    for k in (0, 3):
        y1 = s1.run(x[k:k + 1])
        rel, cos = parity(yb[k], y1)
        assert rel <= 5e-3 and cos >= 0.99999, (k, rel, cos)


def check_batch_items(model, batch, items, seed, opts=""):
    """Batched session on the HIP path; selected items against the oracle run at batch 1 on the
    same images (the conv path is independent across the batch)."""
    sess = V.Session(model, batch, seed=seed, options=opts)
    x = make_input(sess.in_shape, 100 + batch)
    got = sess.run(x)
    per_item = [n // batch for n in sess.out_elems]
    for k in items:
        ref = oracle_model_run(model, 1, seed, x[k:k + 1])
        g = np.concatenate([got[sum(sess.out_elems[:o]):sum(sess.out_elems[:o + 1])].reshape(batch, -1)[k]
                            for o in range(len(per_item))])
        check_outputs(g, ref, per_item, f"{model} b{batch}[{opts}] item {k}")


@pytest.mark.parametrize("opts", ["", "fuse_dwpw=1"])
def test_config1_mnv2_block_b32(gpu, opts):
    check_batch_items("mnv2_block", 32, (0, 31), 7, opts)


def test_config2_resnet50_b64_items(gpu):
    check_batch_items("resnet50", 64, (0, 63), 7)


@pytest.mark.parametrize("opts", ["", "fuse_se=1;fuse_dwpw=1"])
def test_config3_mobilenetv3_large(gpu, opts):
    sess = V.Session("mobilenetv3_large", 1, seed=7, options=opts)
    x = make_input(sess.in_shape, 3)
    check_outputs(sess.run(x), oracle_model_run("mobilenetv3_large", 1, 7, x), sess.out_elems, f"config3[{opts}]")


@pytest.mark.parametrize("opts", ["", "fuse_se=1"])
def test_se_scale_folded_into_projection(gpu, opts, monkeypatch):
    """The squeeze-excite channel scale of every MobileNetV3 block is folded into its projection
    conv (no separate Mul launch) and the result matches both the oracle and the unfolded session."""
    sess = V.Session("mobilenetv3_large", 2, seed=7, options=opts)
    plan = sess.describe()
    assert plan.count("+input scale") == 8 and plan.count("scale folded into") == 8, plan
    x = make_input(sess.in_shape, 4)
    got = sess.run(x)
    check_outputs(got, oracle_model_run("mobilenetv3_large", 2, 7, x), sess.out_elems, f"config3 b2 folded[{opts}]")
    monkeypatch.setenv("VKNN_HIP_FOLD_SCALE", "0")
    plain = V.Session("mobilenetv3_large", 2, seed=7, options=opts)
    assert "+input scale" not in plain.describe()
    check_outputs(got, plain.run(x), sess.out_elems, f"config3 b2 folded vs unfolded[{opts}]")


def test_squeeze_excite_fused_by_default(gpu, monkeypatch):
    """Default options: the HIP backend still fuses every MobileNetV3 squeeze-excite (its pool then
    folds into the depthwise conv), and the result matches the oracle's unfused graph and the
    session without the automatic fusion."""
    sess = V.Session("mobilenetv3_large", 2, seed=7)
    plan = sess.describe()
    assert plan.count("pool folded into the depthwise conv") == 8, plan
    x = make_input(sess.in_shape, 8)
    got = sess.run(x)
    check_outputs(got, oracle_model_run("mobilenetv3_large", 2, 7, x), sess.out_elems, "config3 b2 auto SE")
    plain = V.Session("mobilenetv3_large", 2, seed=7, options="hip_auto_se=0")
    assert "pool folded into the depthwise conv" not in plain.describe()
    check_outputs(got, plain.run(x), sess.out_elems, "config3 b2 auto SE vs unfused")


def test_stem_convs_and_pool_chain_fused(gpu, monkeypatch):
    """YOLOv8n's two stride-2 stem convs (3 -> 16 -> 32) and the 1x1 after them run as one kernel
    with both intermediates in LDS, the three SPPF pools as one launch, and the 16-channel bottleneck's two
    3x3 convs and shortcut as one kernel; the result matches the oracle and the session with none
    of them."""
    sess = V.Session("yolov8n", 1, seed=7)
    plan = sess.describe()
    assert plan.count("runs with the stride-2 conv that reads it") == 1 and "conv_stem2_kernel" in plan, plan
    assert plan.count("runs as the tail of the stride-2 pair") == 1, plan
    assert plan.count("+2 chained pools in one launch") == 1 and plan.count("computed in the launch of the chain's first pool") == 2, plan
    assert plan.count("kernel=conv_pair_kernel") == 1 and plan.count("runs with the 3x3 conv that reads it") == 1, plan
    x = make_input(sess.in_shape, 7)
    got = sess.run(x)
    check_outputs(got, oracle_model_run("yolov8n", 1, 7, x), sess.out_elems, "config4 b1 stem fused")
    monkeypatch.setenv("VKNN_HIP_FUSE_STEM2", "0")
    monkeypatch.setenv("VKNN_HIP_POOL_CHAIN", "0")
    monkeypatch.setenv("VKNN_HIP_FUSE_PAIR", "0")
    plain = V.Session("yolov8n", 1, seed=7)
    assert "conv_stem2_kernel" not in plain.describe() and "chained pools" not in plain.describe() and "conv_pair_kernel" not in plain.describe()
    check_outputs(got, plain.run(x), sess.out_elems, "config4 b1 stem fused vs two launches")


def test_stem_and_first_block_fused(gpu, monkeypatch):
    """MobileNetV3's stem conv (3 -> 16, hard-swish) and its first block (depthwise 3x3 + ReLU, 1x1
    16 -> 16 + the stem's output) run as one kernel with both 16-channel tensors in LDS; the result
    matches the oracle and the session with the two ops apart."""
    sess = V.Session("mobilenetv3_large", 2, seed=7)
    plan = sess.describe()
    assert plan.count("kernel=conv_stem_dwpw_kernel") == 1 and plan.count("runs with the depthwise block that reads it") == 1, plan
    x = make_input(sess.in_shape, 9)
    got = sess.run(x)
    check_outputs(got, oracle_model_run("mobilenetv3_large", 2, 7, x), sess.out_elems, "config3 b2 stem block fused")
    monkeypatch.setenv("VKNN_HIP_FUSE_STEM_BLOCK", "0")
    plain = V.Session("mobilenetv3_large", 2, seed=7)
    assert "conv_stem_dwpw_kernel" not in plain.describe()
    check_outputs(got, plain.run(x), sess.out_elems, "config3 b2 stem block fused vs apart")


def test_bottleneck_add_folded_into_conv(gpu, monkeypatch):
    """The six YOLOv8n bottleneck shortcuts (an Add after an activated 3x3 conv, writing a slice of
    the C2f concat) run inside that conv's epilogue as a residual after the activation: no add
    launch, the same result as the oracle and as the unfolded session."""
    sess = V.Session("yolov8n", 1, seed=7)
    plan = sess.describe()
    assert plan.count("add (a residual after the activation) folded into") == 6, plan
    x = make_input(sess.in_shape, 6)
    got = sess.run(x)
    check_outputs(got, oracle_model_run("yolov8n", 1, 7, x), sess.out_elems, "config4 b1 add folded")
    monkeypatch.setenv("VKNN_HIP_FOLD_ADD", "0")
    plain = V.Session("yolov8n", 1, seed=7)
    assert "residual after the activation" not in plain.describe()
    check_outputs(got, plain.run(x), sess.out_elems, "config4 b1 add folded vs unfolded")


@pytest.mark.parametrize("opts", ["", "fuse_se=1;fuse_dwpw=1"])
def test_config3_mobilenetv3_large_b128_items(gpu, opts):
    check_batch_items("mobilenetv3_large", 128, (0, 127), 7, opts)


def test_config4_yolov8n(gpu):
    sess = V.Session("yolov8n", 1, seed=7)
    x = make_input(sess.in_shape, 4)
    check_outputs(sess.run(x), oracle_model_run("yolov8n", 1, 7, x), sess.out_elems, "config4")


def test_config4_yolov8n_b16_items(gpu):
    check_batch_items("yolov8n", 16, (0, 15), 7)


@pytest.mark.parametrize("model,batch,opts,side", [("resnet_tiny", 2, "", False), ("yolo_tiny", 1, "", False),
                                                   ("resnet50", 1, "", False), ("resnet50", 64, "", True),
                                                   ("yolov8n", 16, "", False)])
@pytest.mark.parametrize("graphs", ["1", "0"])
def test_side_stream_branches_match_single_stream(gpu, model, batch, opts, graphs, side):
    """Independent branches on a second stream (projection shortcuts, YOLO concat inputs) give
    bit-identical outputs to one in-order stream: same plans (the in-process tune table is
    shared), same kernels, only the overlap differs. Only ops estimated at 4 us or more leave the
    main stream, so the small graphs stay on one stream and the full-size ones use both. Several
    runs cover the eager first run and the captured graph's replays."""
    base = f"{opts};graphs={graphs}"
    s1 = V.Session(model, batch, seed=9, options=base + ";branches=0")
    s2 = V.Session(model, batch, seed=9, options=base + ";branches=1")
    d2 = s2.describe()
    assert ("(side stream)" in d2) == side
    assert s1.describe() == d2.replace(" (side stream)", "")
    rng = np.random.default_rng(4)
    for _ in range(3):
        x = rng.standard_normal(int(np.prod(s1.in_shape))).astype(np.float32)
        np.testing.assert_array_equal(s2.run(x), s1.run(x))


@pytest.mark.parametrize("model,batch,env", [("resnet_tiny", 3, "1"), ("resnet50", 2, "1"), ("resnet50", 3, None)])
def test_stem_maxpool_fused(gpu, model, batch, env, monkeypatch):
    """By default the ResNet-50 stem conv (7x7/s2) and its 3x3/s2 max pool run as one thin-tile
    kernel (the pool node folded into the conv); VKNN_HIP_FUSE_POOL=1 also allows the stem tiles
    (resnet_tiny's 3x3 stem). Outputs within the tolerance of the session that runs them apart
    (VKNN_HIP_FUSE_POOL=0), and of the oracle."""
    if env:
        monkeypatch.setenv("VKNN_HIP_FUSE_POOL", env)
    else:
        monkeypatch.delenv("VKNN_HIP_FUSE_POOL", raising=False)
    sess = V.Session(model, batch, seed=7)
    plan = sess.describe()
    assert plan.count("+max pool") == 1 and plan.count("max pool folded into") == 1, plan
    if model == "resnet50":
        assert "kernel=conv_thin_pool_kernel" in plan, plan
    x = make_input(sess.in_shape, 6)
    got = sess.run(x)
    monkeypatch.setenv("VKNN_HIP_FUSE_POOL", "0")
    plain = V.Session(model, batch, seed=7)
    assert "+max pool" not in plain.describe()
    ref = plain.run(x)
    # the two sessions may pick different tiles for the other convs, so compare at the tolerance
    check_outputs(got, ref, sess.out_elems, f"{model} fused stem pool vs apart")
    check_outputs(got, oracle_model_run(model, batch, 7, x), sess.out_elems, f"{model} fused stem pool vs oracle")


@pytest.mark.parametrize("model,batch", [("yolo_tiny", 2), ("yolov8n", 2)])
def test_inplace_concat_split(gpu, model, batch, monkeypatch):
    """Channel concats and splits done in place (producers write straight into their slice of the
    concat's buffer, split outputs are views of the split input, views read and written with plane
    strides by the conv, add, max pool and resize kernels): bit-identical to the session that copies
    (same plans: tuning and Winograd off), across the eager run and graph replays, and within the
    tolerance of the oracle."""
    opts = "tuning=off;winograd=off;branches=0"
    sess = V.Session(model, batch, seed=7, options=opts)
    plan = sess.describe()
    assert "concat in place" in plan and "split in place" in plan, plan
    monkeypatch.setenv("VKNN_HIP_VIEWS", "0")
    plain = V.Session(model, batch, seed=7, options=opts)
    assert "in place" not in plain.describe()
    rng = np.random.default_rng(8)
    for k in range(3):
        x = rng.standard_normal(int(np.prod(sess.in_shape))).astype(np.float32)
        got = sess.run(x)
        np.testing.assert_array_equal(got, plain.run(x))
        if k == 0:
            check_outputs(got, oracle_model_run(model, batch, 7, x), sess.out_elems, f"{model} in-place concat")
