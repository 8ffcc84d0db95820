"""Benchmark of the fused fp16 conv path on one MI355X: ResNet-50 v1.5 forward (config 2) through
the vknn Session on the HIP backend.

A step = one forward pass of one batch (default 64) with the fp32 NCHW input already resident in
HBM: device pack to NC4HW4 fp16, 53 convs (+ fused BN/ReLU/residual epilogues), max pool, global
average pool, FC, device unpack of the logits. Prints one JSON line (see the end of main()).

Also reported: batch-1 latency/throughput, the conv layers' MFMA fraction and the bandwidth of the
1x1 convs (per-op HIP events on the segment stream), and the reference CPU backend timed on this
host on a bounded sample (cpu_baseline).
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA (published)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E (published)
RIDGE = PEAK_FP16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)  # 312.5 flop/byte


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_steps(sess, steps, warmup):
    """Warm up, then time exactly `steps` forward passes on the session stream: host wall clock
    bracketed by a device sync on both sides, and HIP events on the stream."""
    import vknn_amd as V
    lib = V.vkhip()
    for _ in range(warmup):
        sess.run_device()
    sess.sync()
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    V.check(lib.vkhip_event_create(ctypes.byref(e0)))
    V.check(lib.vkhip_event_create(ctypes.byref(e1)))
    stream = sess.stream
    V.check(lib.vkhip_device_sync())
    t0 = time.perf_counter()
    V.check(lib.vkhip_event_record(e0, stream))
    for _ in range(steps):
        sess.run_device()
    V.check(lib.vkhip_event_record(e1, stream))
    sess.sync()
    V.check(lib.vkhip_device_sync())
    wall = time.perf_counter() - t0
    ms = ctypes.c_float()
    V.check(lib.vkhip_event_elapsed_ms(e0, e1, ctypes.byref(ms)))
    lib.vkhip_event_destroy(e0)
    lib.vkhip_event_destroy(e1)
    return wall, ms.value / 1e3


def profile_ops(model, batch, x_dev, options="", reps=3, launches=5):
    # (options carry the plan file, so the profiled session runs the timed session's plans)
    """Per-op device times: HIP events on the segment stream around `launches` back-to-back
    launches of each op (their average; one launch per event pair would add the event overhead,
    several microseconds, to every short kernel)."""
    import vknn_amd as V
    sess = V.Session(model, batch, seed=7, options=(options + f";profile=1;profile_reps={launches}").lstrip(";"))
    sess.bind_device_input(x_dev.ptr)
    sess.run_device()
    sess.sync()
    sess.profile()
    acc = {}
    for _ in range(reps):
        sess.run_device()
        sess.sync()
        for r in sess.profile():
            a = acc.setdefault(r["name"], dict(r, gpu_ms=0.0))
            a["gpu_ms"] += r["gpu_ms"] / reps
    plan = sess.describe()
    sess.close()
    return list(acc.values()), plan


def plan_info(plan):
    """op name -> kernel family ("conv_dma_kernel tile=14", or the op kind) from a session plan."""
    import re
    out = {}
    for ln in plan.splitlines():
        m = re.match(r"(\S+) \[(\w+)\] ?(.*?) ?\{", ln)
        if not m:
            continue
        k = re.search(r"kernel=(\S+)", m.group(3))
        t = re.search(r"tile=(\d+)", m.group(3))
        out[m.group(1)] = f"{k.group(1)} tile={t.group(1)}" if k and t else m.group(2)
    return out


PLANS = os.path.join(ROOT, "profiles", "bench_plans.vkc")


def layer_rows(stem):
    """Rows of a committed per-layer rocprofv3 summary (profiles/<stem>_layers.md, written by
    `python -m vknn_amd.prof_summary layers`): op, kind, plan, kernels, us, GFLOP, alg. MB, HBM MB."""
    path = os.path.join(ROOT, "profiles", f"{stem}_layers.md")
    if not os.path.exists(path):
        return []
    rows = []
    for ln in open(path):
        c = [x.strip() for x in ln.split("|")]
        if len(c) < 16 or not c[1].isdigit():
            continue
        try:
            rows.append({"op": c[2], "kind": c[3], "plan": c[4], "kernels": c[5], "us": float(c[6]), "gflop": float(c[7]),
                         "alg_mb": float(c[8]), "hbm_mb": float(c[13])})
        except ValueError:
            continue
    return rows


def profiled_traffic(stem, names):
    """Measured HBM bytes per launch (FETCH_SIZE x2 + WRITE_SIZE x1) over the same operators as
    `names`, from the committed per-layer summary of this workload; None when it does not list
    every one of them (then it was taken on another plan)."""
    rows = {r["op"]: r for r in layer_rows(stem)}
    if not names or any(n not in rows for n in names):
        return None
    hbm = sum(rows[n]["hbm_mb"] for n in names) * 1e6
    alg = sum(rows[n]["alg_mb"] for n in names) * 1e6
    us = sum(rows[n]["us"] for n in names)
    return {"traffic": round(hbm / len(names)), "profile_algorithmic_bytes_per_launch": round(alg / len(names)),
            "profile_launch_us": round(us / len(names), 3), "traffic_over_algorithmic": round(hbm / max(alg, 1), 3)}


def profiled_kind(stem, kind):
    """In-graph figures of one operator kind from the committed per-layer summary: the kernels'
    device time inside the profiled forward passes (no repeated launches), their algorithmic and
    measured HBM bytes."""
    rows = [r for r in layer_rows(stem) if r["kind"] == kind and r["us"] > 0]
    if not rows:
        return None
    us = sum(r["us"] for r in rows)
    alg = sum(r["alg_mb"] for r in rows) * 1e6
    hbm = sum(r["hbm_mb"] for r in rows) * 1e6
    return {"source": f"profiles/{stem}_layers.md", "ops": len(rows), "device_us_per_step": round(us, 2),
            "achieved_GBs": round(alg / us / 1e3, 1), "frac": round(alg / us / 1e3 / PEAK_HBM_GBS, 4),
            "hbm_over_algorithmic": round(hbm / max(alg, 1), 3)}


PROFILED = [("conv3x3_bn_relu_b1", "config 0"), ("mnv2_block_b32", "config 1"), ("mnv2_block_b128", "config 1, fuse_dwpw=1"),
            ("resnet50_b1", "config 2"), ("resnet50_b64", "config 2"), ("mobilenetv3_large_b128", "config 3"), ("yolov8n_b16", "config 4")]


def profiled_roofline(stem):
    """Every operator of one profiled forward pass against its own roofline, from the committed
    per-layer summary: attainable time = sum over operators of max(FLOPs / MFMA peak, algorithmic
    bytes / HBM peak) over the measured kernel time, plus the MFMA- and HBM-bound operators' own
    fractions."""
    rows = [r for r in layer_rows(stem) if r["us"] > 0]
    if not rows:
        return None
    us = sum(r["us"] for r in rows)
    att = sum(max(r["gflop"] * 1e3 / PEAK_FP16_TFLOPS, r["alg_mb"] / PEAK_HBM_GBS * 1e3) for r in rows)
    mf = [r for r in rows if r["alg_mb"] > 0 and r["gflop"] * 1e3 / r["alg_mb"] > RIDGE]
    hb = [r for r in rows if r not in mf]
    out = {"source": f"profiles/{stem}_layers.md", "kernel_us_per_step": round(us, 1), "attainable_us": round(att, 1),
           "frac": round(att / us, 4)}
    if mf:
        mu = sum(r["us"] for r in mf)
        out["mfma_bound_ops"] = {"n": len(mf), "TFLOPs": round(sum(r["gflop"] for r in mf) / mu * 1e3, 1),
                                 "frac": round(sum(r["gflop"] for r in mf) / mu * 1e3 / PEAK_FP16_TFLOPS, 4)}
    if hb:
        hu = sum(r["us"] for r in hb)
        out["hbm_bound_ops"] = {"n": len(hb), "GBs": round(sum(r["alg_mb"] for r in hb) / hu * 1e3, 1),
                                "frac": round(sum(r["alg_mb"] for r in hb) / hu * 1e3 / PEAK_HBM_GBS, 4)}
    return out


CPU_CONFIGS = [("conv3x3_bn_relu", "config 0"), ("mnv2_block", "config 1"), ("resnet50", "config 2"),
               ("mobilenetv3_large", "config 3"), ("yolov8n", "config 4")]


def winograd_stages(batch, launches=20):
    """The three Winograd F(2x2,3x3) stages of ResNet-50's four 3x3 stride-1 conv shapes at this
    batch, each timed on its own (vkhip_conv_forward_stages) with HIP events around `launches`
    back-to-back launches. The transforms are HBM-bound: input transform reads x and writes the
    16 V planes, output transform reads the 16 M planes (and the residual) and writes y, all fp16.
    The GEMM stage does 16 batched Cout x Cin x tiles GEMMs."""
    import vknn_amd as V
    lib = V.vkhip()
    rng = np.random.default_rng(11)
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    V.check(lib.vkhip_event_create(ctypes.byref(e0)))
    V.check(lib.vkhip_event_create(ctypes.byref(e1)))
    rows, tot = [], {"in": [0.0, 0], "out": [0.0, 0], "gemm": [0.0, 0]}
    for C, H in ((64, 56), (128, 28), (256, 14), (512, 7)):
        d = V.ConvDesc(N=batch, Cin=C, H=H, W=H, Cout=C, OH=H, OW=H, KH=3, KW=3, SH=1, SW=1, PT=1, PL=1, DH=1, DW=1,
                       group=1, act=1, act_lo=0.0, act_hi=0.0, has_res=1)
        plan = V.ConvPlan()
        V.check(lib.vkhip_conv_plan_make(ctypes.byref(d), V.CONV_WINOGRAD, -1, 0, ctypes.byref(plan)), "winograd plan")
        w = (rng.standard_normal((C, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
        b = (rng.standard_normal(C) * 0.1).astype(np.float32)
        blob = np.zeros(plan.weight_bytes, np.uint8)
        V.check(lib.vkhip_conv_pack_weights(ctypes.byref(d), ctypes.byref(plan), w.ctypes.data, b.ctypes.data, blob.ctypes.data))
        act_bytes = V.nc4_elems(batch, C, H, H) * 2
        xb = V.DeviceBuffer.from_array(rng.standard_normal(act_bytes // 2).astype(np.float16))
        rb = V.DeviceBuffer.from_array(rng.standard_normal(act_bytes // 2).astype(np.float16))
        yb = V.DeviceBuffer(act_bytes)
        wb = V.DeviceBuffer.from_array(blob)
        ws = V.DeviceBuffer(plan.workspace_bytes)
        nT = batch * ((H + 1) // 2) ** 2
        planes = 16 * ((C + 3) // 4) * nT * 8  # the 16 V (or M) planes, fp16 x 4 channels
        row = {"shape": f"{C}->{C} 3x3 at {H}x{H}, b{batch}", "tiles": nT}
        for name, mask, nbytes, flops in (("in", 1, act_bytes + planes, 0), ("gemm", 2, 0, 2 * 16 * C * C * nT),
                                          ("out", 4, planes + 2 * act_bytes, 0)):
            args = (ctypes.byref(d), ctypes.byref(plan), xb.ptr, wb.ptr, rb.ptr, yb.ptr, ws.ptr)
            for _ in range(3):
                V.check(lib.vkhip_conv_forward_stages(*args, 7, None))
            V.check(lib.vkhip_event_record(e0, None))
            for _ in range(launches):
                V.check(lib.vkhip_conv_forward_stages(*args, mask, None))
            V.check(lib.vkhip_event_record(e1, None))
            V.check(lib.vkhip_stream_sync(None))
            ms = ctypes.c_float()
            V.check(lib.vkhip_event_elapsed_ms(e0, e1, ctypes.byref(ms)))
            us = ms.value * 1e3 / launches
            row[name + "_us"] = round(us, 2)
            if nbytes:
                row[name + "_GBs"] = round(nbytes / us / 1e3, 1)
                tot[name][0] += us; tot[name][1] += nbytes
            else:
                row["gemm_TFLOPs"] = round(flops / us / 1e6, 1)
                tot[name][0] += us; tot[name][1] += flops
        rows.append(row)
        for buf in (xb, rb, yb, wb, ws):
            buf.close()
    lib.vkhip_event_destroy(e0)
    lib.vkhip_event_destroy(e1)
    tb = tot["in"][1] + tot["out"][1]
    tu = tot["in"][0] + tot["out"][0]
    return {"workload": f"ResNet-50 3x3 stride-1 shapes at b{batch}, forced winograd, {launches} launches per stage",
            "transforms_achieved_GBs": round(tb / tu / 1e3, 1), "peak_GBs": PEAK_HBM_GBS,
            "transforms_frac": round(tb / tu / 1e3 / PEAK_HBM_GBS, 4),
            "input_frac": round(tot["in"][1] / tot["in"][0] / 1e3 / PEAK_HBM_GBS, 4),
            "output_frac": round(tot["out"][1] / tot["out"][0] / 1e3 / PEAK_HBM_GBS, 4),
            "gemm_TFLOPs": round(tot["gemm"][1] / tot["gemm"][0] / 1e6, 1), "shapes": rows}


def _cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(model, reps=3):
    """The reference CPU backend (oracle/_ref, compiled from the reference sources) or, where that
    library is absent, the oracle restatement: one thread pinned to one core (sched_setaffinity on
    this thread, restored afterwards), batch 1, the median of `reps` whole forward passes of every
    config; the headline model's median is the reported value."""
    from tests import oracle_lib as O
    kind = "reference" if O.ref_available() else "port"
    run = O.ref_model_run if kind == "reference" else O.oracle_model_run
    allowed = sorted(os.sched_getaffinity(0))
    core = allowed[-1]
    os.sched_setaffinity(0, {core})
    per = {}
    try:
        for name, label in CPU_CONFIGS:
            in_shape, _ = O.model_io(name, 1)
            x = np.random.default_rng(0).standard_normal(in_shape).astype(np.float32)
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                run(name, 1, 7, x)
                ts.append(time.perf_counter() - t0)
            med = float(np.median(ts))
            per[name] = {"config": label, "ms_per_img": round(med * 1e3, 2), "img_per_s": round(1.0 / med, 4),
                         "runs_s": [round(t, 3) for t in ts]}
    finally:
        os.sched_setaffinity(0, set(allowed))
    head = per[model]
    return {"value": head["img_per_s"], "unit": "img/s", "cores": 1, "kind": kind,
            "sample": f"{model} at batch 1, full forward, median of {reps} runs on one pinned core (core {core})",
            "cpu_model": _cpu_model(), "nproc": os.cpu_count(), "threads": 1, "per_config": per}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--model", default="resnet50")
    ap.add_argument("--options", default="")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config throughput section")
    ap.add_argument("--b1-steps", type=int, default=100)
    ap.add_argument("--dw-batch", type=int, default=128, help="batch of the MobileNetV3-Large depthwise measurement (0 = skip)")
    ap.add_argument("--plan-out", default="", help="write the timed session's plan (one line per op with its flops and "
                                                   "bytes) to this file, for vknn_amd.prof_summary layers")
    ap.add_argument("--plans", default=PLANS if os.path.exists(PLANS) else "",
                    help="tune-table file every session of this run reads its plans from (and writes new ones to): the "
                         "committed profiles/bench_plans.vkc by default, so the bench line and the committed rocprofv3 "
                         "summaries run the same plans; 'none' tunes every session afresh")
    ap.add_argument("--traffic-probe", type=int, default=0, metavar="MELEMS",
                    help="only run the flat fp32->fp16 convert over MELEMS million elements 5 times (known HBM "
                         "traffic: 6 bytes per element), to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    plan_opts = f"cache_mode=tune;cache_file={args.plans}" if args.plans and args.plans != "none" else ""

    def opts(*extra):
        return ";".join(o for o in (args.options, plan_opts) + extra if o)

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (--gpus {args.gpus} refused). "
              "The conv path shards by batch with no exchange; run one process per GPU.", file=sys.stderr)
        sys.exit(2)

    import vknn_amd as V
    V.require_gpu()
    if args.traffic_probe:
        n = args.traffic_probe * 1000000
        src, dst = V.DeviceBuffer(4 * n), V.DeviceBuffer(2 * n)
        src.zero()
        for _ in range(5):
            V.check(V.vkhip().vkhip_pack_flat_f32(src.ptr, dst.ptr, n, None))
        V.check(V.vkhip().vkhip_device_sync())
        print(json.dumps({"traffic_probe": "pack_flat_kernel", "read_bytes": 4 * n, "write_bytes": 2 * n, "launches": 5}))
        return
    flops_img = V.vknn().vknn_model_flops(args.model.encode())

    # ---- batch-B throughput (the headline)
    t = time.perf_counter()
    sess = V.Session(args.model, args.batch, seed=7, options=opts())
    log(f"session create (plan + autotune) {time.perf_counter() - t:.1f}s")
    x = np.random.default_rng(0).standard_normal(sess.in_shape).astype(np.float32)
    x_dev = V.DeviceBuffer.from_array(x)
    sess.bind_device_input(x_dev.ptr)
    wall, ev = time_steps(sess, args.steps, args.warmup)
    ms_step = wall / args.steps * 1e3
    img_s = args.batch * args.steps / wall
    log(f"b{args.batch}: {ms_step:.3f} ms/step wall, {ev / args.steps * 1e3:.3f} ms/step events, {img_s:.1f} img/s")
    if args.plan_out:
        with open(args.plan_out, "w") as f:
            f.write(sess.describe())

    # ---- batch-1 latency (skipped with --b1-steps 0, e.g. under a profiler)
    b1_ms = None
    if args.b1_steps > 0:
        s1 = V.Session(args.model, 1, seed=7, options=opts())
        x1 = V.DeviceBuffer.from_array(x[:1])
        s1.bind_device_input(x1.ptr)
        wall1, _ = time_steps(s1, args.b1_steps, 10)
        b1_ms = wall1 / args.b1_steps * 1e3
        s1.close()
        log(f"b1: {b1_ms:.3f} ms/img")

    # ---- per-op roofline (separate profiled session, same graph and tuned plans)
    extra = {}
    roof = None
    if not args.no_profile:
        ops, plan = profile_ops(args.model, args.batch, x_dev, opts())
        # Per-op times come from back-to-back replays of each op (warmer caches, no gaps); scale
        # them so they add up to the measured graph step, i.e. every op's share of the real pass.
        scale = ms_step / sum(o["gpu_ms"] for o in ops)
        for o in ops:
            o["replay_ms"] = o["gpu_ms"]
            o["gpu_ms"] = o["gpu_ms"] * scale
        conv = [o for o in ops if o["type"] in ("Conv", "Gemm", "FusedDwPw") and o["flops"] > 0]
        conv_ms = sum(o["gpu_ms"] for o in conv)
        conv_fl = sum(o["flops"] for o in conv)
        all_ms = sum(o["gpu_ms"] for o in ops)
        # the kernel family (kernel + tile) with the most device time in the step is the "dominant
        # kernel"; its roofline is MFMA or HBM by its arithmetic intensity against the ridge point
        info = plan_info(plan)
        fams = {}
        for o in ops:
            fam = info.get(o["name"])
            if fam and o["gpu_ms"] > 0:
                e = fams.setdefault(fam, dict(n=0, ms=0.0, flops=0.0, bytes=0, names=[]))
                e["n"] += 1
                e["ms"] += o["gpu_ms"]
                e["flops"] += o["flops"]
                e["bytes"] += o["bytes"]
                e["names"].append(o["name"])
        dom = max(fams, key=lambda k: fams[k]["ms"])
        d = fams[dom]
        hbm = d["bytes"] > 0 and d["flops"] / d["bytes"] <= RIDGE
        launch_s = d["ms"] / d["n"] * 1e-3
        if hbm:
            ach, peak, unit = d["bytes"] / d["n"] / launch_s / 1e9, PEAK_HBM_GBS, "GB/s"
        else:
            ach, peak, unit = d["flops"] / d["n"] / launch_s / 1e12, PEAK_FP16_TFLOPS, "TFLOP/s"
        tr = profiled_traffic(f"{args.model}_b{args.batch}", d["names"])
        roof = {"bound": "hbm" if hbm else "mfma", "achieved": round(ach, 2), "peak": peak, "unit": unit,
                "frac": round(ach / peak, 4),
                "traffic": tr["traffic"] if tr else None,
                "traffic_unit": "HBM bytes per launch (FETCH_SIZE x2 + WRITE_SIZE x1) over the same operators, from "
                                "profiles/<model>_b<batch>_layers.md (taken on the same plan file); null if that summary lacks any of them",
                "traffic_detail": tr,
                "kernel": f"{dom}: {d['n']} launches per step ({', '.join(d['names'])})",
                "launch_us": round(launch_s * 1e6, 3),
                "algorithmic_bytes_per_launch": round(d["bytes"] / d["n"]), "flops_per_launch": round(d["flops"] / d["n"]),
                "intensity_flop_per_byte": round(d["flops"] / max(d["bytes"], 1), 1), "ridge_flop_per_byte": RIDGE}
        # every op against its own roofline: the step's attainable time (sum over ops of
        # max(flops / MFMA peak, algorithmic bytes / HBM peak)) over the measured op time
        lb_ms = sum(max(o["flops"] / (PEAK_FP16_TFLOPS * 1e12), o["bytes"] / (PEAK_HBM_GBS * 1e9)) * 1e3 for o in ops)
        extra["step_roofline"] = {"attainable_ms": round(lb_ms, 4), "op_ms": round(all_ms, 4), "frac": round(lb_ms / all_ms, 4),
                                  "mfma_bound_ops": sum(1 for o in ops if o["bytes"] and o["flops"] / o["bytes"] > RIDGE),
                                  "hbm_bound_ops": sum(1 for o in ops if o["bytes"] and o["flops"] / o["bytes"] <= RIDGE)}
        achieved = conv_fl / (conv_ms * 1e-3) / 1e12
        extra["conv_mfma"] = {"achieved_TFLOPs": round(achieved, 2), "peak_TFLOPs": PEAK_FP16_TFLOPS,
                              "frac": round(achieved / PEAK_FP16_TFLOPS, 4), "conv_ms": round(conv_ms, 4), "flops_per_step": conv_fl,
                              "note": "all conv/FC flops over all conv/FC time against the MFMA peak, including the layers whose "
                                      "intensity puts them under the HBM roof"}
        pw = [o for o in conv if "conv" in o["name"] and o["bytes"] > 0]
        one = [o for o in pw if o["flops"] / max(o["bytes"], 1) <= RIDGE]  # layers below the ridge
        if one:
            b_ms = sum(o["gpu_ms"] for o in one)
            b_bytes = sum(o["bytes"] for o in one)
            extra["hbm_bound_convs"] = {"count": len(one), "achieved_GBs": round(b_bytes / (b_ms * 1e-3) / 1e9, 1),
                                        "peak_GBs": PEAK_HBM_GBS, "frac": round(b_bytes / (b_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        extra["op_time_share"] = {"conv_ms": round(conv_ms, 4), "all_ops_ms": round(all_ms, 4),
                                  "replay_to_step_scale": round(scale, 4)}
        with open(os.path.join(ROOT, "gpurun_out", "bench_ops.json") if os.path.isdir(os.path.join(ROOT, "gpurun_out")) else os.devnull, "w") as f:
            json.dump({"ops": ops, "plan": plan}, f, indent=1)

    # ---- bandwidth-bound kernels: depthwise convs of MobileNetV3-Large (config 3) at batch 128
    if not args.no_profile and args.dw_batch > 0:
        xs, _ = V.model_io("mobilenetv3_large", args.dw_batch)
        xd = V.DeviceBuffer.from_array(np.random.default_rng(1).standard_normal(xs).astype(np.float32))
        dops, dplan = profile_ops("mobilenetv3_large", args.dw_batch, xd, plan_opts)
        ds = V.Session("mobilenetv3_large", args.dw_batch, seed=7, options=plan_opts)
        ds.bind_device_input(xd.ptr)
        dwall, _ = time_steps(ds, 10, 3)
        ds.close()
        dscale = dwall / 10 * 1e3 / sum(o["gpu_ms"] for o in dops)
        for o in dops:
            o["replay_ms"] = o["gpu_ms"]
            o["gpu_ms"] = o["gpu_ms"] * dscale
        kinds = {ln.split()[0]: ln.split()[1] for ln in dplan.splitlines() if len(ln.split()) > 1}
        dw = [o for o in dops if kinds.get(o["name"]) == "[dwconv]" and o["bytes"] > 0]
        with open(os.path.join(ROOT, "gpurun_out", "bench_dw_ops.json") if os.path.isdir(os.path.join(ROOT, "gpurun_out")) else os.devnull, "w") as f:
            json.dump({"ops": dops, "plan": dplan}, f, indent=1)
        if dw:
            # frac: algorithmic bytes over the kernels' own launch time (HIP events around the
            # launches); frac_of_step_time charges them their share of the whole step instead
            b_ms = sum(o["replay_ms"] for o in dw)
            b_bytes = sum(o["bytes"] for o in dw)
            extra["depthwise"] = {"workload": f"mobilenetv3_large b{args.dw_batch}, {len(dw)} depthwise 3x3/5x5 convs",
                                  "achieved_GBs": round(b_bytes / (b_ms * 1e-3) / 1e9, 1), "peak_GBs": PEAK_HBM_GBS,
                                  "frac": round(b_bytes / (b_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                  "launch_ms": round(b_ms, 4), "bytes_per_step": b_bytes,
                                  "replay_to_step_scale": round(dscale, 4),
                                  "frac_of_step_time": round(b_bytes / (b_ms * dscale * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                  "in_graph": profiled_kind(f"mobilenetv3_large_b{args.dw_batch}", "dwconv")}
        xd.close()

    # ---- fused dw+pw (config 1: the MobileNetV2 block with the dw+pw fusion pass) at batch 128
    if not args.no_profile and args.dw_batch > 0:
        xs, _ = V.model_io("mnv2_block", args.dw_batch)
        xd = V.DeviceBuffer.from_array(np.random.default_rng(2).standard_normal(xs).astype(np.float32))
        fops, fplan = profile_ops("mnv2_block", args.dw_batch, xd, ";".join(o for o in ("fuse_dwpw=1", plan_opts) if o))
        fs = V.Session("mnv2_block", args.dw_batch, seed=7, options=";".join(o for o in ("fuse_dwpw=1", plan_opts) if o))
        fs.bind_device_input(xd.ptr)
        fwall, _ = time_steps(fs, 10, 3)
        fs.close()
        fscale = fwall / 10 * 1e3 / sum(o["gpu_ms"] for o in fops)
        fused = [o for o in fops if o["type"] == "FusedDwPw" and o["bytes"] > 0]
        if fused:
            f_ms = sum(o["gpu_ms"] for o in fused)
            f_bytes = sum(o["bytes"] for o in fused)
            extra["fused_dwpw"] = {"workload": f"config-1 MobileNetV2 block (24-144-24 @56x56) b{args.dw_batch} (fuse_dwpw=1), {len(fused)} fused dw+pw op(s)",
                                   "achieved_GBs": round(f_bytes / (f_ms * 1e-3) / 1e9, 1), "peak_GBs": PEAK_HBM_GBS,
                                   "frac": round(f_bytes / (f_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                   "launch_ms": round(f_ms, 4), "bytes_per_step": f_bytes, "replay_to_step_scale": round(fscale, 4),
                                   "frac_of_step_time": round(f_bytes / (f_ms * fscale * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                   "execution": [ln for ln in fplan.splitlines() if "[dwpw]" in ln],
                                   "in_graph": profiled_kind(f"mnv2_block_b{args.dw_batch}", "dwpw")}
        xd.close()

    # ---- Winograd transforms (the tuner rarely picks Winograd on these shapes; forced here)
    if not args.no_profile:
        extra["winograd"] = winograd_stages(args.batch)

    # ---- every config at its two batch sizes (img/s and TFLOP/s of whole forward passes, the
    # default session options; the headline config is the line's value)
    if not args.no_configs:
        per = {}
        for name, batches, copts in (("conv3x3_bn_relu", (1,), ""), ("mnv2_block", (1, 32), ""), ("mnv2_block", (32,), "fuse_dwpw=1"),
                                     ("mobilenetv3_large", (1, 128), ""), ("mobilenetv3_large", (128,), "fuse_se=1"),
                                     ("yolov8n", (1, 16), "")):
            fl = V.vknn().vknn_model_flops(name.encode())
            for b in batches:
                cs = V.Session(name, b, seed=7, options=";".join(o for o in (copts, plan_opts) if o))
                cx = V.DeviceBuffer.from_array(np.random.default_rng(3).standard_normal(cs.in_shape).astype(np.float32))
                cs.bind_device_input(cx.ptr)
                n = 50 if b == 1 else 20
                cw, _ = time_steps(cs, n, 5)
                cs.close()
                cx.close()
                key = name + (f" ({copts})" if copts else "")
                per.setdefault(key, {})[f"b{b}"] = {"ms_per_step": round(cw / n * 1e3, 4), "img_per_s": round(b * n / cw, 1),
                                                      "tflops": round(fl * b * n / cw / 1e12, 2)}
                log(f"{key} b{b}: {cw / n * 1e3:.3f} ms/step")
        extra["per_config"] = per

    pr = {f"{stem} ({label})": profiled_roofline(stem) for stem, label in PROFILED}
    extra["profiled_rooflines"] = {k: v for k, v in pr.items() if v}

    cpu = None if args.no_cpu_baseline else cpu_baseline(args.model)

    out = {
        "metric": "ResNet-50 fp16 img/s at b=1/64; conv % of MFMA peak; dw/1x1 HBM GB/s",
        "value": round(img_s, 2),
        "unit": "img/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 storage, fp32 accumulation (MFMA f32_32x32x16_f16)",
        "data": "synthetic N(0,1) input, random He-init weights with folded random BN (seeded; BN gamma U[0.5,1.5], except the last BN of each residual branch, gamma U[0.1,0.3], which keeps fp16 activations finite through 16 residual adds)",
        "config": {"workload": f"{args.model} v1.5 forward, config 2" if args.model == "resnet50" else args.model,
                   "batch": args.batch, "input": "x".join(map(str, sess.in_shape[1:])),
                   "layout": "NC4HW4 fp16", "options": args.options or "default",
                   "plans": os.path.relpath(args.plans, ROOT) if plan_opts else "tuned in this run",
                   "tflops_per_step": round(flops_img * args.batch / 1e12, 4)},
        "b1_ms_per_img": round(b1_ms, 4) if b1_ms else None,
        "b1_img_per_s": round(1000.0 / b1_ms, 1) if b1_ms else None,
        "tflops": round(flops_img * img_s / 1e12, 2),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    out.update(extra)
    sess.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
