"""Summaries of rocprofv3 output, as the tables under profiles/ are made.

    python3 -m nert_amd.profsum trace KERNEL_TRACE_CSV --anchor NAME --blocks N [--conv-gflop G]
    python3 -m nert_amd.profsum traffic FETCH_CSV WRITE_CSV --anchor NAME [--trace CSV --blocks N]
                                [--conv-json OUT]
    python3 -m nert_amd.profsum mfma COUNTER_CSV --anchor NAME
    python3 -m nert_amd.profsum ops KERNEL_TRACE_CSV OPS_JSONL [--fetch CSV --write CSV
                                --fetch-scale F --write-scale W]

A "block" is one pass over a program: the dispatches from one launch of the
anchor kernel (the program's first kernel, e.g. StemQuadKernel for ResNet-18)
up to the next. `trace` averages the last N blocks of the run of identical
blocks that holds the most dispatches (the timed graph replays). `traffic` and `mfma` read the
last block of a `--pmc` run of `python3 -m nert_amd.replay W --eager
--copy-probe` and scale FETCH_SIZE/WRITE_SIZE by what the copy probe (the
final elementwise kernel: 256 MiB read, 256 MiB written) reads for them.
`ops` splits a trace of `bench.py --ops` into its cases: each case's timed
row is one graph of 20 back-to-back launches replayed 3 times, the only
stretch of the trace where one dispatch sequence repeats 60 times.

MFMA utilisation per dispatch = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE /
8 XCDs x 1024 SIMDs): GRBM_GUI_ACTIVE is summed over the eight XCDs, the
busy counter over all SIMDs of the chip.
"""

from __future__ import annotations

import argparse
import collections
import csv
import json
import re
import sys

PROBE_BYTES = 256 * 1024 * 1024
CONV_PATTERN = re.compile(r"(Conv|Stem|Halo|Patch|ResidualRelu)")
XCDS, SIMDS = 8, 1024


def short(name: str) -> str:
    name = re.sub(r"^void ", "", name)
    name = re.sub(r"nert_hip::(\(anonymous namespace\)::)?", "", name)
    return re.sub(r"\(.*$", "", name)


def read_trace(path: str) -> list[dict]:
    rows = list(csv.DictReader(open(path, newline="")))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    for r in rows:
        r["short"] = short(r["Kernel_Name"])
        r["us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    return rows


def read_counters(path: str) -> list[dict]:
    """One dict per dispatch: short name, grid, and every counter of the file."""
    by: dict[int, dict] = {}
    for r in csv.DictReader(open(path, newline="")):
        d = by.setdefault(int(r["Dispatch_Id"]), {"short": short(r["Kernel_Name"]), "grid": r.get("Grid_Size", "")})
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [by[k] for k in sorted(by)]


def blocks(names: list[str], anchor: str) -> list[tuple[int, int]]:
    starts = [i for i, n in enumerate(names) if n.startswith(anchor)]
    if not starts:
        raise SystemExit(f"anchor {anchor!r} not found")
    return [(a, b) for a, b in zip(starts, starts[1:] + [len(names)])]


def cmd_trace(a) -> None:
    rows = read_trace(a.csv)
    names = [r["short"] for r in rows]
    bl = blocks(names, a.anchor)[:-1]  # the last block runs to the end of the trace
    sig = [tuple(names[s:e]) for s, e in bl]
    best, i = None, 0
    while i < len(bl):
        j = i
        while j + 1 < len(bl) and sig[j + 1] == sig[i]:
            j += 1
        if j > i and (best is None or (j - i + 1) * len(sig[i]) > (best[1] - best[0] + 1) * len(sig[best[0]])):
            best = (i, j)
        i = j + 1
    i, j = best
    use = bl[max(i, j - a.blocks + 1): j + 1]
    n = len(use)
    print(f"{j - i + 1} identical blocks of {bl[i][1] - bl[i][0]} dispatches in a row; averaged over the last {n}")
    per: dict[str, list[float]] = collections.OrderedDict()
    for s, e in use:
        for r in rows[s:e]:
            per.setdefault(r["short"], []).append(r["us"])
    total = sum(sum(v) for v in per.values()) / n
    span = (int(rows[use[-1][1] - 1]["End_Timestamp"]) - int(rows[use[0][0]]["Start_Timestamp"])) / 1e3 / n
    print(f"kernel time per block {total:.1f} us; first start to last end {span:.1f} us per block")
    print()
    print("| kernel | calls/block | avg µs | µs/block | % of kernel time |")
    print("|---|---:|---:|---:|---:|")
    conv = 0.0
    for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        s = sum(v) / n
        if CONV_PATTERN.search(k):
            conv += s
        print(f"| `{k}` | {len(v) // n} | {sum(v) / len(v):.2f} | {s:.1f} | {100 * s / total:.1f} |")
    if a.conv_gflop:
        tf = a.conv_gflop * 1e9 / (conv * 1e-6) / 1e12
        print()
        print(f"Conv-row kernels (conv, stem, split/tail reduce) per block: {conv:.1f} us -> "
              f"{tf:.2f} TFLOP/s = {tf / 157.3:.4f} of the 157.3 TFLOP/s fp32 MFMA peak")


def probe_scale(disp: list[dict], counter: str) -> tuple[float, float]:
    probe = [d for d in disp if d["short"].startswith("UnaryF32Kernel")][-1]
    kib = probe[counter]
    return PROBE_BYTES / (kib * 1024), kib


def last_block(disp: list[dict], anchor: str) -> list[dict]:
    body = disp[:-1] if disp[-1]["short"].startswith("UnaryF32Kernel") else disp
    s, e = blocks([d["short"] for d in body], anchor)[-1]
    return [d for d in body[s:e] if not d["short"].startswith("__amd_rocclr")]


def cmd_traffic(a) -> None:
    out = {}
    for counter, path in (("FETCH_SIZE", a.fetch), ("WRITE_SIZE", a.write)):
        disp = read_counters(path)
        scale, kib = probe_scale(disp, counter)
        out[counter] = (last_block(disp, a.anchor), scale, kib)
    fetch, write = out["FETCH_SIZE"][0], out["WRITE_SIZE"][0]
    if [d["short"] for d in fetch] != [d["short"] for d in write]:
        raise SystemExit("the FETCH_SIZE and WRITE_SIZE runs dispatched different kernels")
    dur: dict[str, list[float]] = collections.defaultdict(list)
    if a.trace:
        rows = read_trace(a.trace)
        names = [r["short"] for r in rows]
        for s, e in blocks(names, a.anchor)[:-1][-a.blocks:]:
            for r in rows[s:e]:
                dur[r["short"]].append(r["us"])
    print(f"copy probe: FETCH_SIZE {out['FETCH_SIZE'][2]:.1f} KiB -> scale {out['FETCH_SIZE'][1]:.4f}; "
          f"WRITE_SIZE {out['WRITE_SIZE'][2]:.1f} KiB -> scale {out['WRITE_SIZE'][1]:.4f}; "
          f"{len(fetch)} dispatches in the last block")
    print()
    print("| kernel | calls | fetch MB/call | write MB/call | HBM MB/call | avg µs | TB/s |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    agg: dict[str, list[tuple[float, float]]] = collections.OrderedDict()
    for f, w in zip(fetch, write):
        agg.setdefault(f["short"], []).append((f["FETCH_SIZE"] * 1024 * out["FETCH_SIZE"][1],
                                               w["WRITE_SIZE"] * 1024 * out["WRITE_SIZE"][1]))
    for k, v in sorted(agg.items(), key=lambda kv: -sum(dur.get(kv[0], [0.0]))):
        fb = sum(x for x, _ in v) / len(v)
        wb = sum(y for _, y in v) / len(v)
        d = dur.get(k)
        avg = sum(d) / len(d) if d else float("nan")
        print(f"| `{k}` | {len(v)} | {fb / 1e6:.2f} | {wb / 1e6:.2f} | {(fb + wb) / 1e6:.2f} | {avg:.2f} | "
              f"{(fb + wb) / avg / 1e6:.2f} |")
    if a.conv_json:
        conv = [(f, w) for f, w in zip(fetch, write) if CONV_PATTERN.search(f["short"])]
        rows_per_block = sum(1 for f, _ in conv if not re.search(r"Reduce|ResidualRelu", f["short"]))
        fb = sum(f["FETCH_SIZE"] for f, _ in conv) * 1024 * out["FETCH_SIZE"][1] / rows_per_block
        wb = sum(w["WRITE_SIZE"] for _, w in conv) * 1024 * out["WRITE_SIZE"][1] / rows_per_block
        res = {"bytes_per_conv_row": int(round(fb + wb)), "fetch_bytes_per_conv_row": int(round(fb)),
               "write_bytes_per_conv_row": int(round(wb)), "conv_rows": rows_per_block,
               "fetch_scale": round(out["FETCH_SIZE"][1], 4), "write_scale": round(out["WRITE_SIZE"][1], 4)}
        with open(a.conv_json, "w") as fh:
            json.dump(res, fh, indent=1)
            fh.write("\n")
        print()
        print(f"Conv rows: {rows_per_block} per block; per row fetch {fb / 2**20:.1f} MiB + write "
              f"{wb / 2**20:.1f} MiB = {(fb + wb) / 2**20:.1f} MiB -> {a.conv_json}")


def cmd_mfma(a) -> None:
    disp = last_block(read_counters(a.csv), a.anchor)
    print("| # | kernel | grid | MFMA ops (G, counter x 512) | MFMA busy % |")
    print("|---:|---|---:|---:|---:|")
    for i, d in enumerate(disp):
        mops = d.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0)
        if mops <= 0:
            continue
        busy = d["SQ_VALU_MFMA_BUSY_CYCLES"] / (d["GRBM_GUI_ACTIVE"] / XCDS * SIMDS) * 100
        print(f"| {i} | `{d['short']}` | {d['grid']} | {mops * 512 / 1e9:.3f} | {busy:.1f} |")


def _periodic_runs(sig: list[tuple], min_reps: int) -> list[tuple[int, int, int]]:
    """(start, period, reps) of every stretch where one dispatch sequence of
    period <= 8 repeats at least min_reps times back to back."""
    found, i = [], 0
    while i < len(sig):
        hit = None
        for p in range(1, 9):
            reps = 1
            while i + (reps + 1) * p <= len(sig) and sig[i + reps * p: i + (reps + 1) * p] == sig[i: i + p]:
                reps += 1
            if reps >= min_reps:
                hit = (i, p, reps)
                break
        if hit:
            found.append(hit)
            i += hit[1] * hit[2]
        else:
            i += 1
    return found


def _case_bytes(path: str, counter: str, scale: float, n_cases: int) -> list[float]:
    """Per case: the counter (KiB per dispatch, scaled) summed over one launch
    of the row, averaged over the last 20 of its 60 timed launches."""
    disp = read_counters(path)
    sig = [(d["short"], d["grid"]) for d in disp]
    runs = _periodic_runs(sig, 60)
    if len(runs) != n_cases:
        raise SystemExit(f"{path}: {len(runs)} timed stretches for {n_cases} cases")
    out = []
    for s, p, reps in runs:
        last = disp[s + (reps - 20) * p: s + reps * p]
        out.append(sum(d[counter] for d in last) * 1024 * scale / 20)
    return out


def cmd_ops(a) -> None:
    rows = read_trace(a.csv)
    sig = [(r["short"], r["Grid_Size_X"], r["Grid_Size_Y"], r["Grid_Size_Z"]) for r in rows]
    runs = _periodic_runs(sig, 60)
    cases = [json.loads(line) for line in open(a.jsonl) if line.startswith("{")]
    if len(runs) != len(cases):
        raise SystemExit(f"{len(runs)} timed stretches in the trace for {len(cases)} cases")
    traffic = None
    if a.fetch and a.write:
        traffic = list(zip(_case_bytes(a.fetch, "FETCH_SIZE", a.fetch_scale, len(cases)),
                           _case_bytes(a.write, "WRITE_SIZE", a.write_scale, len(cases))))
    head = ("| case | reference fixture | kernels per launch | kernel-only µs (rocprof) | achieved | % of peak |"
            + (" HBM MB per launch (counters) | algorithmic MB |" if traffic else "")
            + " MI300X reference HIP µs | speed-up | reference CPU row ms (1 core) | parity |")
    print(head)
    print("|---|---|---|---:|---:|---:|" + ("---:|---:|" if traffic else "") + "---:|---:|---:|---|")
    for k, ((s, p, reps), c) in enumerate(zip(runs, cases)):
        last = rows[s + (reps - 20) * p: s + reps * p]
        us = sum(r["us"] for r in last) / 20
        kern = " + ".join(dict.fromkeys(r["short"].split("<")[0] for r in rows[s: s + p]))
        if c["bound"] == "mfma":
            ach = f"{c['work'] / (us * 1e-6) / 1e12:.1f} TFLOP/s"
            frac = c["work"] / (us * 1e-6) / 1e12 / 157.3
        else:
            ach = f"{c['work'] / (us * 1e-6) / 1e9:.0f} GB/s"
            frac = c["work"] / (us * 1e-6) / 1e9 / 8000.0
        ref = c.get("mi300x_ref_hip_ms")
        line = f"| {c['case']} | {c['source']} | {kern} | {us:.2f} | {ach} | {100 * frac:.1f} |"
        if traffic:
            fb, wb = traffic[k]
            alg = c.get("algorithmic_bytes", c["work"] if c["bound"] == "hbm" else None)
            line += f" {(fb + wb) / 1e6:.2f} | {'' if alg is None else f'{alg / 1e6:.2f}'} |"
        line += (f" {'' if ref is None else f'{ref * 1e3:.0f}'} |"
                 f" {'' if ref is None else f'{ref * 1e3 / us:.0f}x'} |")
        cpu = c.get("cpu_baseline")
        if cpu:
            exact = "bit-exact" if cpu["float_max_ratio_to_1e-4_bar"] == 0 else \
                f"{cpu['float_max_ratio_to_1e-4_bar']:.2f} of the 1e-4 bar"
            line += f" {cpu['ms']:.3f} | {'ok' if cpu['parity_ok'] else 'FAIL'} ({exact}) |"
        else:
            line += " | |"
        print(line)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python3 -m nert_amd.profsum")
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("csv")
    t.add_argument("--anchor", required=True)
    t.add_argument("--blocks", type=int, default=20)
    t.add_argument("--conv-gflop", type=float)
    f = sub.add_parser("traffic")
    f.add_argument("fetch")
    f.add_argument("write")
    f.add_argument("--anchor", required=True)
    f.add_argument("--trace")
    f.add_argument("--blocks", type=int, default=10)
    f.add_argument("--conv-json")
    m = sub.add_parser("mfma")
    m.add_argument("csv")
    m.add_argument("--anchor", required=True)
    o = sub.add_parser("ops")
    o.add_argument("csv")
    o.add_argument("jsonl")
    o.add_argument("--fetch", help="counter CSV of a FETCH_SIZE run of the same command")
    o.add_argument("--write", help="counter CSV of a WRITE_SIZE run of the same command")
    o.add_argument("--fetch-scale", type=float, default=1.0)
    o.add_argument("--write-scale", type=float, default=1.0)
    a = ap.parse_args(argv)
    {"trace": cmd_trace, "traffic": cmd_traffic, "mfma": cmd_mfma, "ops": cmd_ops}[a.cmd](a)
    return 0


if __name__ == "__main__":
    sys.exit(main())
