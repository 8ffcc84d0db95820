"""CPU tests of the host side: the C-ABI libraries load and export every declared entry point,
and the host graph passes produce the fused-node contract the kernels rely on (no device needed)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import vknn_amd as V

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    """Function names declared in a C header (prototypes ending in ';' at file scope)."""
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = set()
    for m in re.finditer(r"\b(vk\w+|vknn_\w+)\s*\(", text):
        names.add(m.group(1))
    return {n for n in names if not n.endswith("_t") and not n.endswith("_s")}


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.mark.parametrize("header,lib", [("vkhip.h", V.VKHIP_PATH), ("vknn_c.h", V.VKNN_PATH)])
def test_library_exports_every_declared_symbol(header, lib):
    names = declared(header)
    assert len(names) > 10
    missing = names - exported(lib)
    assert not missing, missing


def test_python_bindings_cover_headers():
    assert declared("vkhip.h") == set(V.VKHIP_API)
    assert declared("vknn_c.h") == set(V.VKNN_API)


def test_libraries_load_without_gpu():
    lib = V.vknn()
    assert V.vkhip().vkhip_build_info()
    assert lib.vknn_model_flops(b"resnet50") > 0


def test_no_device_reports_unavailable():
    """Without a device the product path refuses to run (no CPU fallback)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert V.vkhip().vkhip_available() == 0
    with pytest.raises(V.VkhipError):
        V.require_gpu()


def nodes(model, batch=1, options=""):
    out = []
    for line in V.graph_after_passes(model, batch, options).strip().splitlines():
        parts = line.split()
        kv = dict(p.split("=", 1) for p in parts[2:])
        out.append((parts[0], parts[1], int(kv["act"]), int(kv["res"]), kv["out"]))
    return out


def test_config0_passes_fold_bn_and_relu():
    """BN folds into the conv and the ReLU fuses into it (fold_batchnorm.cpp:57-78, fuse_activations.cpp)."""
    ns = nodes("conv3x3_bn_relu")
    assert [(n[0], n[2], n[3], n[4]) for n in ns] == [("Conv", 1, 0, "[1,64,56,56]")]


def test_config1_mnv2_block_contract():
    """ReLU6 (Clip 0..6) fuses as act=2; the residual Add fuses into the 1x1 project (fuse_residual_add.cpp:20-32)."""
    ns = nodes("mnv2_block", 32)
    assert [(n[0], n[2], n[3]) for n in ns] == [("Conv", 2, 0), ("Conv", 2, 0), ("Conv", 0, 1)]
    assert ns[-1][4] == "[32,24,56,56]"
    fused = nodes("mnv2_block", 1, "fuse_dwpw=1")
    assert [n[0] for n in fused] == ["Conv", "FusedDwPw"]


def test_config2_resnet50_structure():
    ns = nodes("resnet50", 64)
    convs = [n for n in ns if n[0] == "Conv"]
    assert len(convs) == 53
    assert sum(n[3] for n in convs) == 16           # one fused residual per bottleneck (1x1 expand)
    assert all(n[2] == 1 for n in convs if n[3] == 1)  # ReLU moved onto the conv with the residual
    assert [n[0] for n in ns if n[0] != "Conv"] == ["MaxPool", "GlobalAveragePool", "Flatten", "Gemm"]
    assert ns[-1][4] == "[64,1000]"


def test_config3_mnv3_se_and_swish():
    ns = nodes("mobilenetv3_large", 1, "fuse_se=1")
    types = [n[0] for n in ns]
    assert types.count("FusedSE") == 8
    assert any(n[2] == 4 for n in ns if n[0] == "Conv")  # HardSwish fused (fuse_swish.cpp:5-99)


def test_config4_yolo_silu():
    ns = nodes("yolov8n", 1)
    convs = [n for n in ns if n[0] == "Conv"]
    assert len(convs) >= 40
    assert all(n[2] == 5 for n in convs if n[4] != ns[-1][4])  # SiLU fused into every backbone/neck conv
    assert "Concat" in {n[0] for n in ns} and "Resize" in {n[0] for n in ns}


def _desc(N, Cin, H, W, Cout, K, S, P, group=1):
    OH = (H + 2 * P - K) // S + 1
    OW = (W + 2 * P - K) // S + 1
    return V.ConvDesc(N=N, Cin=Cin, H=H, W=W, Cout=Cout, OH=OH, OW=OW, KH=K, KW=K, SH=S, SW=S, PT=P, PL=P, DH=1, DW=1,
                      group=group, act=1, act_lo=0.0, act_hi=0.0, has_res=0)


def test_conv_planner_selection_on_host():
    """Kernel selection is host-only: depthwise for group == C, Winograd for 3x3 s1 p1 when forced,
    GEMM otherwise; invalid descriptors are rejected."""
    lib = V.vkhip()
    plan = V.ConvPlan()
    d = _desc(1, 32, 14, 14, 32, 3, 1, 1, group=32)
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_AUTO, -1, 0, ctypes.byref(plan)) == 0
    assert plan.algo == V.CONV_DEPTHWISE
    d = _desc(64, 64, 56, 56, 64, 3, 1, 1)
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_WINOGRAD, -1, 0, ctypes.byref(plan)) == 0
    assert plan.algo == V.CONV_WINOGRAD and plan.weight_bytes > 0 and plan.workspace_bytes > 0
    d = _desc(1, 64, 56, 56, 256, 1, 1, 0)
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_AUTO, -1, 0, ctypes.byref(plan)) == 0
    assert plan.algo in (V.CONV_GEMM, V.CONV_SPLITK)
    assert plan.weight_bytes >= 64 * 256 * 2
    d = _desc(1, 64, 56, 56, 64, 3, 2, 1)
    assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_WINOGRAD, -1, 0, ctypes.byref(plan)) != 0
    bad = _desc(1, 0, 56, 56, 64, 3, 1, 1)
    assert lib.vkhip_conv_plan_make(ctypes.byref(bad), V.CONV_AUTO, -1, 0, ctypes.byref(plan)) != 0


def test_model_flops_match_survey_arithmetic():
    """Algorithmic conv+FC FLOPs per image: ResNet-50 v1.5 ~8.17 GFLOP conv-only (+ 4.1 MFLOP FC)."""
    f = V.vknn().vknn_model_flops(b"resnet50")
    assert abs(f - 8.17e9) / 8.17e9 < 0.01
    assert abs(V.vknn().vknn_model_flops(b"conv3x3_bn_relu") - 231.2e6) / 231.2e6 < 0.001


def test_weights_pack_with_the_reference_codec_rounding():
    """Packed conv weights carry the reference GPU path's fp16 weights: its codec rounds half away
    from zero (include/vknn/dtype.h:121-157), where a plain fp16 cast rounds ties to even. Ties
    placed in the weights of a 1x1 conv (GEMM and depthwise packers, host code, no GPU needed)
    come out as the away-from-zero neighbour, the non-tie as the nearest value."""
    lib = V.vkhip()
    ties = np.array([1 + 2.0 ** -11, -(1 + 2.0 ** -11), 2 + 2.0 ** -10, 0.1], np.float32)
    away = np.array([1 + 2.0 ** -10, -(1 + 2.0 ** -10), 2 + 2.0 ** -9, np.float16(0.1)], np.float32)
    assert (np.float16(ties[:3]).astype(np.float32) != away[:3]).all()  # a plain cast would differ
    C = len(ties)
    for group in (1, C):
        w = np.ascontiguousarray((np.diag(ties) if group == 1 else ties.reshape(C, 1))[:, :, None, None], np.float32)
        d = V.ConvDesc(N=1, Cin=C, H=4, W=4, Cout=C, OH=4, OW=4, KH=1, KW=1, SH=1, SW=1, PT=0, PL=0, DH=1, DW=1, group=group)
        plan = V.ConvPlan()
        assert lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_DEPTHWISE if group > 1 else V.CONV_GEMM, -1, 0, ctypes.byref(plan)) == 0
        blob = np.zeros(plan.weight_bytes, np.uint8)
        assert lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, None, blob.ctypes.data) == 0
        halves = blob.view(np.float16).astype(np.float32)
        assert sorted(halves[halves != 0]) == sorted(away), group


def test_noalloc_refuses_plan_for_another_shape():
    """The allocation-free conv sizes its fixed scratch from the descriptor: a split-K plan made for
    a larger batch (a bigger workspace than this descriptor needs) or an edited workspace size is
    refused before any device call, so no kernel can write past the scratch array."""
    from tests.gpu_helpers import conv_desc
    lib = V.vkhip()
    big, _ = conv_desc((8, 256, 14, 14), (256, 256, 1, 1))
    small, _ = conv_desc((1, 256, 14, 14), (256, 256, 1, 1))
    plan = V.ConvPlan()
    V.check(lib.vkhip_conv_plan_make(ctypes.byref(big), V.CONV_SPLITK, -1, 4, ctypes.byref(plan)), "plan")
    assert plan.workspace_bytes > 0
    rc = lib.vkhip_conv_forward_noalloc(ctypes.byref(small), ctypes.byref(plan), None, None, None, None, None)
    assert rc == 1 and b"differ" in lib.vkhip_last_error()
    V.check(lib.vkhip_conv_plan_make(ctypes.byref(small), V.CONV_SPLITK, -1, 4, ctypes.byref(plan)), "plan")
    plan.workspace_bytes -= 256
    rc = lib.vkhip_conv_forward_noalloc(ctypes.byref(small), ctypes.byref(plan), None, None, None, None, None)
    assert rc == 1 and b"differ" in lib.vkhip_last_error()
