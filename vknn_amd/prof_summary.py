"""Summarise rocprofv3 output of `bench.py` into short text tables.

Kernel time:   python -m vknn_amd.prof_summary trace <run_kernel_trace.csv> --steps K
HBM traffic:   python -m vknn_amd.prof_summary traffic <fetch counter csv> <write counter csv> --steps K
                   --fetch-scale F --write-scale W

The timed region of bench.py is K forward passes, each starting with one NCHW->NC4HW4 pack
dispatch; the last K pack dispatches therefore delimit the timed steps (session creation,
autotuning and warm-up come before them). Per kernel family the tables give dispatches per step,
mean duration / per-step time, or per-step HBM bytes read and written. FETCH_SIZE and WRITE_SIZE
(KiB per dispatch) are multiplied by the calibration factors measured on a kernel of known traffic
(`bench.py --traffic-probe`), so the totals are bytes that crossed the HBM interface.
"""
import argparse
import csv
import re
from collections import OrderedDict

CONV_PREFIX = ("conv_gemm", "conv_bd", "conv_dma", "conv_halo", "conv_stem", "splitk_reduce", "wino_", "dwconv", "dwpw", "fc_kernel")


def family(name):
    m = re.search(r"vkhip::(\w+)(<[^>(]*>)?\(", name)
    if m:
        return m.group(1) + (m.group(2) or "").replace(" ", "")
    # mangled (the tool could not demangle it): _ZN5vkhip<len><name>[I<args>E]...; integer and bool
    # template arguments are Li<n>E / Lb<0|1>E
    m = re.match(r"_ZN5vkhip(\d+)", name)
    if m:
        n = int(m.group(1))
        base = name[m.end():m.end() + n]
        rest = name[m.end() + n:]
        if rest.startswith("I"):
            args = []
            for am in re.finditer(r"L([ib])(\d+)E", rest[1:rest.find("EE") + 1] if "EE" in rest else ""):
                args.append(am.group(2) if am.group(1) == "i" else ("true" if am.group(2) == "1" else "false"))
            if args:
                return base + "<" + ",".join(args) + ">"
        return base
    return name[:40]


def timed_rows(rows, steps):
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    packs = [i for i, r in enumerate(rows) if family(r["Kernel_Name"]).startswith(("pack_kernel", "pack4_kernel"))]
    if len(packs) < steps:
        raise SystemExit(f"found {len(packs)} pack dispatches, need {steps}")
    return rows[packs[-steps]:]


def summarise(path, steps):
    timed = timed_rows(list(csv.DictReader(open(path))), steps)
    span_ns = int(timed[-1]["End_Timestamp"]) - int(timed[0]["Start_Timestamp"])
    fam = OrderedDict()
    for r in timed:
        f = family(r["Kernel_Name"])
        d = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        e = fam.setdefault(f, [0, 0])
        e[0] += 1
        e[1] += d
    return fam, span_ns, len(timed)


def counter_per_family(path, steps, counter):
    rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
    byid = {}
    for r in rows:  # one row per dispatch (values already summed over instances)
        byid.setdefault(r["Dispatch_Id"], r)
    timed = timed_rows(list(byid.values()), steps)
    fam = OrderedDict()
    for r in timed:
        f = family(r["Kernel_Name"])
        e = fam.setdefault(f, [0, 0.0])
        e[0] += 1
        e[1] += float(r["Counter_Value"]) * 1024.0
    return fam


def cmd_trace(a):
    fam, span_ns, n = summarise(a.trace, a.steps)
    total = sum(v[1] for v in fam.values())
    conv = sum(v[1] for k, v in fam.items() if k.startswith(CONV_PREFIX))
    gemm = sum(v[1] for k, v in fam.items() if k.startswith(("conv_gemm", "conv_bd", "conv_dma", "conv_halo", "conv_stem")))
    print(f"# {a.title}\n")
    if a.command:
        print(f"Command: `{a.command}`\n")
    print(f"Timed steps: {a.steps}; dispatches in them: {n}; first-to-last dispatch span {span_ns / a.steps / 1e3:.1f} us/step\n")
    print("| kernel | dispatches/step | mean us | us/step | share |")
    print("|---|---:|---:|---:|---:|")
    for k, (c, d) in sorted(fam.items(), key=lambda kv: -kv[1][1]):
        print(f"| `{k}` | {c / a.steps:.1f} | {d / c / 1e3:.2f} | {d / a.steps / 1e3:.1f} | {100 * d / total:.1f}% |")
    print(f"\nSum of kernel time per step: {total / a.steps / 1e3:.1f} us; conv kernels (gemm, split-K reduce, "
          f"Winograd transforms, depthwise, FC): {conv / a.steps / 1e3:.1f} us; implicit-GEMM kernels (conv_gemm, conv_bd, conv_dma, conv_halo, conv_stem) alone: {gemm / a.steps / 1e3:.1f} us")


def cmd_traffic(a):
    fr = counter_per_family(a.fetch, a.steps, "FETCH_SIZE")
    wr = counter_per_family(a.write, a.steps, "WRITE_SIZE")
    print(f"# {a.title}\n")
    if a.command:
        print(f"Command: `{a.command}`\n")
    print(f"Calibration: FETCH_SIZE x {a.fetch_scale}, WRITE_SIZE x {a.write_scale} (bench.py --traffic-probe)\n")
    print("| kernel | dispatches/step | read MB/step | written MB/step |")
    print("|---|---:|---:|---:|")
    tot_r = tot_w = conv_r = conv_w = 0.0
    for k in sorted(fr, key=lambda k: -fr[k][1]):
        r = fr[k][1] * a.fetch_scale / a.steps
        w = wr.get(k, [0, 0.0])[1] * a.write_scale / a.steps
        tot_r += r
        tot_w += w
        if k.startswith(CONV_PREFIX):
            conv_r += r
            conv_w += w
        print(f"| `{k}` | {fr[k][0] / a.steps:.1f} | {r / 1e6:.1f} | {w / 1e6:.1f} |")
    print(f"\nPer step: all kernels read {tot_r / 1e6:.1f} MB and wrote {tot_w / 1e6:.1f} MB; conv kernels read "
          f"{conv_r / 1e6:.1f} MB and wrote {conv_w / 1e6:.1f} MB (total {(conv_r + conv_w) / 1e6:.1f} MB)")


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("trace")
    c = sub.add_parser("traffic")
    c.add_argument("fetch")
    c.add_argument("write")
    c.add_argument("--fetch-scale", type=float, default=1.0)
    c.add_argument("--write-scale", type=float, default=1.0)
    for p in (t, c):
        p.add_argument("--steps", type=int, required=True)
        p.add_argument("--title", default="kernel time per forward pass")
        p.add_argument("--command", default="")
    a = ap.parse_args()
    cmd_trace(a) if a.cmd == "trace" else cmd_traffic(a)


if __name__ == "__main__":
    main()
