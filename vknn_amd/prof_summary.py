"""Summarise a rocprofv3 kernel trace of `bench.py` into a short text table.

Usage: python -m vknn_amd.prof_summary <run_kernel_trace.csv> --steps K [--title T] [--command C]

The timed region of bench.py is K forward passes, each starting with one NCHW->NC4HW4 pack
dispatch; the last K pack dispatches therefore delimit the timed steps (session creation,
autotuning and warm-up come before them). Per kernel family the table gives dispatches per
step, the mean duration and the per-step total, so the conv kernels' time per step can be set
against the per-op HIP-event figure bench.py reports (roofline.launch_ms).
"""
import argparse
import csv
import re
from collections import OrderedDict


def family(name):
    m = re.search(r"vkhip::(\w+)(<[^>(]*>)?\(", name)
    if m:
        return m.group(1) + (m.group(2) or "").replace(" ", "")
    m = re.search(r"_ZN5vkhip\d+(\w+?)E", name)
    return m.group(1) if m else name[:40]


def summarise(path, steps):
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    packs = [i for i, r in enumerate(rows) if family(r["Kernel_Name"]).startswith("pack_kernel")]
    if len(packs) < steps:
        raise SystemExit(f"found {len(packs)} pack dispatches, need {steps}")
    first = packs[-steps]
    timed = rows[first:]
    span_ns = int(timed[-1]["End_Timestamp"]) - int(timed[0]["Start_Timestamp"])
    fam = OrderedDict()
    for r in timed:
        f = family(r["Kernel_Name"])
        d = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        e = fam.setdefault(f, [0, 0])
        e[0] += 1
        e[1] += d
    return fam, span_ns, len(timed)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--steps", type=int, required=True)
    ap.add_argument("--title", default="kernel time per forward pass")
    ap.add_argument("--command", default="")
    a = ap.parse_args()
    fam, span_ns, n = summarise(a.trace, a.steps)
    total = sum(v[1] for v in fam.values())
    conv = sum(v[1] for k, v in fam.items() if k.startswith(("conv_gemm", "splitk_reduce", "wino_", "dwconv", "dwpw")))
    gemm = sum(v[1] for k, v in fam.items() if k.startswith("conv_gemm"))
    print(f"# {a.title}\n")
    if a.command:
        print(f"Command: `{a.command}`\n")
    print(f"Timed steps: {a.steps}; dispatches in them: {n}; first-to-last dispatch span {span_ns / a.steps / 1e3:.1f} us/step\n")
    print("| kernel | dispatches/step | mean us | us/step | share |")
    print("|---|---:|---:|---:|---:|")
    for k, (c, d) in sorted(fam.items(), key=lambda kv: -kv[1][1]):
        print(f"| `{k}` | {c / a.steps:.1f} | {d / c / 1e3:.2f} | {d / a.steps / 1e3:.1f} | {100 * d / total:.1f}% |")
    print(f"\nSum of kernel time per step: {total / a.steps / 1e3:.1f} us; conv kernels (gemm, split-K reduce, "
          f"Winograd transforms, depthwise): {conv / a.steps / 1e3:.1f} us; conv_gemm_kernel alone: {gemm / a.steps / 1e3:.1f} us")


if __name__ == "__main__":
    main()
