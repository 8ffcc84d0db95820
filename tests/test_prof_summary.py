"""The per-layer roofline join of vknn_amd/prof_summary.py on a synthetic kernel trace: dispatches
cut at the marker kernels, assigned to the plan's operators in order, boundary packs excluded,
times averaged over the timed steps, each operator placed under its MFMA or HBM roof, and the
measured counter bytes attributed per operator."""
import csv
import subprocess
import sys

import pytest

import bench

PLAN = ("conv_0 [conv] gemm tile=14 ksplit=0 kernel=conv_dma_kernel {flops=2e+09 bytes=1000000}\n"
        "pool_1 [maxpool]  {flops=0 bytes=4000000}\n"
        "conv_2 [conv] splitk tile=26 ksplit=2 kernel=conv_halo_kernel {flops=5e+09 bytes=8000000}\n"
        "flat_3 [alias]  {flops=0 bytes=0}\n")
K = "void vkhip::{}(vkhip::GemmArgs)"


def _rows(steps):
    rows, t, did = [], 1000, 0
    def add(name, dur):
        nonlocal t, did
        did += 1
        rows.append({"Kernel_Name": K.format(name), "Start_Timestamp": str(t), "End_Timestamp": str(t + dur), "Dispatch_Id": str(did)})
        t += dur + 100
    add("conv_dma_kernel<2,2>", 999)  # an untimed warm-up dispatch before the first pack
    for _ in range(steps):
        add("pack_kernel<int>", 500)
        for k, kern in enumerate([["conv_dma_kernel<2,2>"], ["maxpool3s2_kernel<int>"], ["conv_halo_kernel<2,1>", "splitk_reduce_kernel"], []]):
            add("dispatch_marker_kernel", 10)
            for j, name in enumerate(kern):
                add(name, [4000, 1000, 2500, 500][k] if j == 0 else 300)
        add("unpack_kernel", 200)
        add("unpack_quad_kernel", 160)  # a second boundary unpack after the last operator (not conv_2's or flat_3's)
    return rows


def _write(path, rows, counter=None, value=0.0):
    with open(path, "w", newline="") as f:
        cols = ["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Dispatch_Id"] + (["Counter_Name", "Counter_Value"] if counter else [])
        w = csv.DictWriter(f, fieldnames=cols)
        w.writeheader()
        for r in rows:
            w.writerow(dict(r, Counter_Name=counter, Counter_Value=value) if counter else r)


def test_layers_join(tmp_path):
    rows = _rows(3)
    _write(tmp_path / "t.csv", rows)
    _write(tmp_path / "f.csv", rows, "FETCH_SIZE", 1000.0)  # KiB per dispatch
    _write(tmp_path / "w.csv", rows, "WRITE_SIZE", 500.0)
    (tmp_path / "plan.txt").write_text(PLAN)
    out = subprocess.run([sys.executable, "-m", "vknn_amd.prof_summary", "layers", str(tmp_path / "t.csv"), str(tmp_path / "plan.txt"),
                          "--steps", "3", "--fetch", str(tmp_path / "f.csv"), "--write", str(tmp_path / "w.csv"),
                          "--fetch-scale", "2", "--write-scale", "1"], capture_output=True, text=True, check=True).stdout
    lines = {ln.split("|")[2].strip(): [c.strip() for c in ln.split("|")] for ln in out.splitlines() if ln.startswith("| ") and ln.split("|")[1].strip().isdigit()}
    assert set(lines) == {"conv_0", "pool_1", "conv_2", "flat_3"}
    c0, p1, c2, f3 = lines["conv_0"], lines["pool_1"], lines["conv_2"], lines["flat_3"]
    assert c0[6] == "4.00" and p1[6] == "1.00" and c2[6] == "2.80" and f3[6] == "0.00"  # us: 2500 + 300 reduce for conv_2
    assert "splitk_reduce_kernel" in c2[5] and "conv_halo_kernel" in c2[5] and f3[5] == "-"
    # conv_0: 2 GFLOP over 1 MB = 2000 flop/B > ridge -> MFMA: 2e9 / 4e-6 = 500 TFLOP/s -> 0.2 of 2500
    assert c0[11] == "mfma" and c0[9] == "500.0" and c0[12] == "0.200"
    # pool_1: 4 MB in 1 us = 4000 GB/s -> 0.5 of HBM
    assert p1[11] == "hbm" and p1[10] == "4000" and p1[12] == "0.500"
    # measured bytes: one dispatch 1000 KiB x2 + 500 KiB x1; conv_2 has two dispatches
    assert float(c0[13]) == pytest.approx(2.56) and float(c2[13]) == pytest.approx(5.12)
    assert f3[13] == "0.00"
    # the boundary conversions (500 + 200 + 160 ns per step) are reported apart from the operators
    assert "7.8 us of operator kernels, and 0.9 us of the segment's boundary conversions" in out


def test_layers_rejects_unmarked_trace(tmp_path):
    rows = [r for r in _rows(2) if "dispatch_marker" not in r["Kernel_Name"]]
    _write(tmp_path / "t.csv", rows)
    (tmp_path / "plan.txt").write_text(PLAN)
    r = subprocess.run([sys.executable, "-m", "vknn_amd.prof_summary", "layers", str(tmp_path / "t.csv"), str(tmp_path / "plan.txt"),
                        "--steps", "2"], capture_output=True, text=True)
    assert r.returncode != 0 and "VKNN_HIP_OP_MARKERS" in (r.stdout + r.stderr)


def test_bench_plan_info():
    info = bench.plan_info(PLAN)
    assert info == {"conv_0": "conv_dma_kernel tile=14", "pool_1": "maxpool", "conv_2": "conv_halo_kernel tile=26", "flat_3": "alias"}
