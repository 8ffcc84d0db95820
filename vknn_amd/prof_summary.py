"""Summarise rocprofv3 output of `bench.py` into short text tables.

Kernel time:   python -m vknn_amd.prof_summary trace <run_kernel_trace.csv> --steps K
HBM traffic:   python -m vknn_amd.prof_summary traffic <fetch counter csv> <write counter csv> --steps K
                   --fetch-scale F --write-scale W
Per layer:     python -m vknn_amd.prof_summary layers <run_kernel_trace.csv> <plan.txt> --steps K
                   [--fetch <csv> --write <csv> --fetch-scale F --write-scale W]
Wave states:   python -m vknn_amd.prof_summary stalls <counter csv> [<counter csv> ...] --steps K
                   (runs with SQ_WAVE_CYCLES in every --pmc pass, e.g. SQ_WAIT_ANY, SQ_WAIT_INST_ANY,
                   SQ_ACTIVE_INST_VALU/_VMEM/_LDS, SQ_VALU_MFMA_BUSY_CYCLES)

The timed region of bench.py is K forward passes, each starting with one NCHW->NC4HW4 pack
dispatch; the last K pack dispatches therefore delimit the timed steps (session creation,
autotuning and warm-up come before them). Per kernel family the tables give dispatches per step,
mean duration / per-step time, or per-step HBM bytes read and written. FETCH_SIZE and WRITE_SIZE
(KiB per dispatch) are multiplied by the calibration factors measured on a kernel of known traffic
(`bench.py --traffic-probe`), so the totals are bytes that crossed the HBM interface.

The per-layer table needs a run with VKNN_HIP_OP_MARKERS=1 (the session then enqueues an empty
dispatch_marker_kernel before each operator, all operators on one stream) and the plan that
`bench.py --plan-out` writes: one line per operator, in launch order, ending in
"{flops=F bytes=B}" (the operator's algorithmic work). Each step's dispatches are cut at the
markers, the i-th group belongs to the i-th plan line, and every operator gets its kernels, mean
device time per step, achieved TFLOP/s and GB/s, and the fraction of the roofline that bounds it:
MFMA fp16 (2500 TFLOP/s dense) above the ridge of 2.5e15 / 8e12 = 312.5 flop/byte, HBM (8 TB/s)
below it. With the PMC runs of the same command, each operator's measured HBM bytes are added.
"""
import argparse
import csv
import re
from collections import OrderedDict

CONV_PREFIX = ("conv_gemm", "conv_bd", "conv_dma", "conv_halo", "conv_stem", "conv_thin", "splitk_reduce", "wino_", "dwconv", "dwpw", "fc_kernel")


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
    packs = [i for i, r in enumerate(rows) if family(r["Kernel_Name"]).startswith(("pack_kernel", "pack2_kernel", "pack4_kernel"))]
    if len(packs) < steps:
        raise SystemExit(f"found {len(packs)} pack dispatches, need {steps}")
    return rows[packs[-steps]:]


MARKER = "dispatch_marker_kernel"  # the empty per-operator separators of VKNN_HIP_OP_MARKERS=1


def busy_and_gaps(timed):
    """Device time covered by at least one kernel (overlapping dispatches of two streams counted
    once) and the idle gaps between consecutive covered intervals, in ns."""
    iv = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in timed)
    busy, gaps, cur_s, cur_e = 0, [], iv[0][0], iv[0][1]
    for s0, e0 in iv[1:]:
        if s0 > cur_e:
            busy += cur_e - cur_s
            gaps.append(s0 - cur_e)
            cur_s, cur_e = s0, e0
        else:
            cur_e = max(cur_e, e0)
    busy += cur_e - cur_s
    return busy, gaps


def summarise(path, steps):
    timed = [r for r in timed_rows(list(csv.DictReader(open(path))), steps) if not family(r["Kernel_Name"]).startswith(MARKER)]
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
        if f.startswith(MARKER):
            continue
        e = fam.setdefault(f, [0, 0.0])
        e[0] += 1
        e[1] += float(r["Counter_Value"]) * 1024.0
    return fam


def cmd_stalls(a):
    """Per kernel family over the timed steps: each SQ counter summed over its dispatches as a
    fraction of SQ_WAVE_CYCLES from the same pass (the share of resident-wave time spent waiting on
    a dependency counter, waiting to issue, or issuing each instruction type), and the MFMA busy
    share, SQ_VALU_MFMA_BUSY_CYCLES over the dispatches' duration x clock x 4 SIMDs x CUs."""
    cols, fams = [], OrderedDict()
    for path in a.csv:
        rows = list(csv.DictReader(open(path)))
        names = sorted({r["Counter_Name"] for r in rows})
        byid = OrderedDict()
        for r in rows:
            e = byid.setdefault(r["Dispatch_Id"], dict(r))
            e[r["Counter_Name"]] = float(r["Counter_Value"])
        timed = timed_rows(list(byid.values()), a.steps)
        for r in timed:
            f = fams.setdefault(family(r["Kernel_Name"]), {})
            for n in names:
                f.setdefault(n, [0.0, 0])
                f[n][0] += r.get(n, 0.0)
                f[n][1] += 1
            dus = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            f.setdefault("#us", {})[path] = f.get("#us", {}).get(path, 0.0) + dus
            if "SQ_VALU_MFMA_BUSY_CYCLES" in names:
                f["#mf_us"] = f.get("#mf_us", 0.0) + dus
        cols += [n for n in names if n not in ("SQ_WAVE_CYCLES", "SQ_WAVES") and not n.startswith("GRBM_") and n not in cols]
    print(f"# {a.title}\n")
    if a.command:
        print(f"Command: `{a.command}`\n")
    print("Shares of SQ_WAVE_CYCLES (resident-wave time) per kernel family over the timed steps; "
          f"mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (dispatch time x {a.clock_ghz} GHz x 4 x {a.cus} CUs); "
          "insts_valu = SQ_INSTS_VALU per wave (SQ_WAVES of the same pass).\n")
    hdr = [c.replace("SQ_", "").lower() for c in cols if c != "SQ_VALU_MFMA_BUSY_CYCLES"]
    mf = "SQ_VALU_MFMA_BUSY_CYCLES" in cols
    print("| kernel | us/step | " + " | ".join(hdr) + (" | mfma_busy |" if mf else " |"))
    print("|---|---:|" + "---:|" * (len(hdr) + (1 if mf else 0)))
    def us(f):
        return min(f["#us"].values()) / a.steps
    for k, f in sorted(fams.items(), key=lambda kv: -us(kv[1])):
        if us(f) < a.min_us:
            continue
        cells = []
        for c in cols:
            if c == "SQ_VALU_MFMA_BUSY_CYCLES":
                continue
            wc = f.get("SQ_WAVE_CYCLES", [0.0, 0])[0]
            if c == "SQ_INSTS_VALU":
                nw = f.get("SQ_WAVES", [0.0, 0])[0]
                cells.append(f"{f[c][0] / nw:.0f}" if c in f and nw > 0 else "-")
                continue
            cells.append(f"{f[c][0] / wc:.3f}" if c in f and wc > 0 else "-")
        if mf:
            p = f.get("#mf_us")
            cells.append(f"{f['SQ_VALU_MFMA_BUSY_CYCLES'][0] / (p * 1e3 * a.clock_ghz * 4 * a.cus):.3f}" if p and "SQ_VALU_MFMA_BUSY_CYCLES" in f else "-")
        print(f"| `{k}` | {us(f):.1f} | " + " | ".join(cells) + " |")


def cmd_trace(a):
    fam, span_ns, n = summarise(a.trace, a.steps)
    total = sum(v[1] for v in fam.values())
    conv = sum(v[1] for k, v in fam.items() if k.startswith(CONV_PREFIX))
    gemm = sum(v[1] for k, v in fam.items() if k.startswith(("conv_gemm", "conv_bd", "conv_dma", "conv_halo", "conv_stem")))
    print(f"# {a.title}\n")
    if a.command:
        print(f"Command: `{a.command}`\n")
    print(f"Timed steps: {a.steps}; dispatches in them: {n}; first-to-last dispatch span {span_ns / a.steps / 1e3:.1f} us/step\n")
    timed = [r for r in timed_rows(list(csv.DictReader(open(a.trace))), a.steps) if not family(r["Kernel_Name"]).startswith(MARKER)]
    busy, gaps = busy_and_gaps(timed)
    if gaps:
        gs = sorted(gaps)
        print(f"Device busy (at least one kernel running) {busy / a.steps / 1e3:.1f} us/step = {100 * busy / span_ns:.1f}% of the span; "
              f"{len(gaps) / a.steps:.1f} idle gaps per step between dispatches, {sum(gaps) / a.steps / 1e3:.1f} us/step in total, "
              f"median {gs[len(gs) // 2] / 1e3:.2f} us, 90th percentile {gs[int(len(gs) * 0.9)] / 1e3:.2f} us\n")
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


PEAK_TFLOPS, PEAK_GBS = 2500.0, 8000.0
RIDGE = PEAK_TFLOPS * 1e12 / (PEAK_GBS * 1e9)
# the segment's boundary conversions (fp32 NCHW <-> NC4HW4 fp16), which belong to no operator
BOUNDARY = ("pack_kernel", "pack2_kernel", "pack4_kernel", "unpack", "boundary_convert")


def read_plan(path):
    ops = []
    for ln in open(path):
        m = re.match(r"(\S+) \[(\w+)\] ?(.*?) ?\{flops=([0-9.eE+-]+) bytes=(\d+)\}\s*$", ln.rstrip("\n"))
        if m:
            ops.append(dict(name=m.group(1), kind=m.group(2), plan=m.group(3), flops=float(m.group(4)), bytes=int(m.group(5))))
    return ops


def marker_groups(rows, steps, n_ops, boundary=None):
    """Per timed step, the dispatch rows of each operator (cut at the markers); the boundary
    conversions of each step go to `boundary` (a list) if given."""
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    starts = [i for i, r in enumerate(rows) if family(r["Kernel_Name"]).startswith(("pack_kernel", "pack2_kernel", "pack4_kernel"))]
    if len(starts) < steps:
        raise SystemExit(f"found {len(starts)} pack dispatches, need {steps}")
    out = []
    for s_i, beg in enumerate(starts[-steps:]):
        end = starts[starts.index(beg) + 1] if starts.index(beg) + 1 < len(starts) else len(rows)
        groups = []
        for r in rows[beg:end]:
            f = family(r["Kernel_Name"])
            if f.startswith("dispatch_marker"):
                groups.append([])
            elif f.startswith(BOUNDARY):
                if boundary is not None:
                    boundary.append(r)
            elif groups:
                groups[-1].append(r)
        if len(groups) != n_ops:
            raise SystemExit(f"step {s_i}: {len(groups)} marker groups for {n_ops} plan lines (run with VKNN_HIP_OP_MARKERS=1)")
        out.append(groups)
    return out


def counters_by_dispatch(path, counter):
    vals, rows = {}, {}
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        vals[r["Dispatch_Id"]] = vals.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"]) * 1024.0
        rows.setdefault(r["Dispatch_Id"], r)
    return vals, list(rows.values())


def cmd_layers(a):
    ops = read_plan(a.plan)
    bnd = []
    steps = marker_groups(list(csv.DictReader(open(a.trace))), a.steps, len(ops), bnd)
    measured = None
    if a.fetch and a.write:
        fv, frows = counters_by_dispatch(a.fetch, "FETCH_SIZE")
        wv, wrows = counters_by_dispatch(a.write, "WRITE_SIZE")
        fsteps = marker_groups(frows, a.steps, len(ops))
        wsteps = marker_groups(wrows, a.steps, len(ops))
        measured = []
        for k in range(len(ops)):
            rd = sum(fv[r["Dispatch_Id"]] for st in fsteps for r in st[k]) * a.fetch_scale / a.steps
            wr = sum(wv[r["Dispatch_Id"]] for st in wsteps for r in st[k]) * a.write_scale / a.steps
            measured.append((rd, wr))
    print(f"# {a.title}\n")
    if a.command:
        print(f"Command: `{a.command}`\n")
    print(f"Timed steps: {a.steps}. Roofline: MFMA fp16 {PEAK_TFLOPS:.0f} TFLOP/s above {RIDGE:.1f} flop/B, HBM {PEAK_GBS:.0f} GB/s below."
          + (f" Measured HBM bytes: FETCH_SIZE x {a.fetch_scale} + WRITE_SIZE x {a.write_scale}." if measured else "") + "\n")
    head = "| # | op | kind | plan | kernels | us | GFLOP | alg. MB | TFLOP/s | GB/s | bound | frac |"
    sep = "|---:|---|---|---|---|---:|---:|---:|---:|---:|---|---:|"
    if measured:
        head += " HBM MB | HBM/alg |"
        sep += "---:|---:|"
    print(head)
    print(sep)
    tot = dict(mfma=[0.0, 0.0], hbm=[0.0, 0.0])
    all_us = 0.0
    for k, op in enumerate(ops):
        rows = [r for st in steps for r in st[k]]
        us = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rows) / a.steps / 1e3
        all_us += us
        fams = OrderedDict()
        for r in steps[-1][k]:
            f = family(r["Kernel_Name"])
            fams[f] = fams.get(f, 0) + 1
        kern = ", ".join(f"`{f}`" + (f" x{c}" if c > 1 else "") for f, c in fams.items()) or "-"
        line = f"| {k} | {op['name']} | {op['kind']} | {op['plan']} | {kern} | {us:.2f} |"
        if us > 0 and (op["flops"] > 0 or op["bytes"] > 0):
            tf = op["flops"] / (us * 1e-6) / 1e12
            gbs = op["bytes"] / (us * 1e-6) / 1e9
            bound = "mfma" if op["bytes"] == 0 or op["flops"] / op["bytes"] > RIDGE else "hbm"
            frac = tf / PEAK_TFLOPS if bound == "mfma" else gbs / PEAK_GBS
            tot[bound][0] += op["flops"] if bound == "mfma" else op["bytes"]
            tot[bound][1] += us
            line += f" {op['flops'] / 1e9:.2f} | {op['bytes'] / 1e6:.2f} | {tf:.1f} | {gbs:.0f} | {bound} | {frac:.3f} |"
        else:
            line += f" {op['flops'] / 1e9:.2f} | {op['bytes'] / 1e6:.2f} | - | - | - | - |"
        if measured:
            rd, wr = measured[k]
            line += f" {(rd + wr) / 1e6:.2f} | " + (f"{(rd + wr) / op['bytes']:.2f} |" if op["bytes"] else "- |")
        print(line)
    mf, hb = tot["mfma"], tot["hbm"]
    bnd_us = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in bnd) / a.steps / 1e3
    print(f"\nPer step: {all_us:.1f} us of operator kernels, and {bnd_us:.1f} us of the segment's boundary conversions "
          f"(input pack, output unpack; in no operator row).")
    if mf[1]:
        print(f"MFMA-bound operators: {mf[0] / 1e9:.1f} GFLOP in {mf[1]:.1f} us = {mf[0] / (mf[1] * 1e-6) / 1e12:.1f} TFLOP/s, "
              f"{mf[0] / (mf[1] * 1e-6) / 1e12 / PEAK_TFLOPS:.3f} of peak.")
    if hb[1]:
        print(f"HBM-bound operators: {hb[0] / 1e6:.1f} MB in {hb[1]:.1f} us = {hb[0] / (hb[1] * 1e-6) / 1e9:.0f} GB/s, "
              f"{hb[0] / (hb[1] * 1e-6) / 1e9 / PEAK_GBS:.3f} of peak.")


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
    lay = sub.add_parser("layers")
    lay.add_argument("trace")
    lay.add_argument("plan")
    lay.add_argument("--fetch", default="")
    lay.add_argument("--write", default="")
    lay.add_argument("--fetch-scale", type=float, default=1.0)
    lay.add_argument("--write-scale", type=float, default=1.0)
    st = sub.add_parser("stalls")
    st.add_argument("csv", nargs="+")
    st.add_argument("--cus", type=int, default=256)
    st.add_argument("--min-us", type=float, default=2.0)
    st.add_argument("--clock-ghz", type=float, default=2.4)
    for p in (t, c, lay, st):
        p.add_argument("--steps", type=int, required=True)
        p.add_argument("--title", default="kernel time per forward pass")
        p.add_argument("--command", default="")
    a = ap.parse_args()
    {"trace": cmd_trace, "traffic": cmd_traffic, "layers": cmd_layers, "stalls": cmd_stalls}[a.cmd](a)


if __name__ == "__main__":
    main()
