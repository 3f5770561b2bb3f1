"""Summaries of rocprofv3 output for the SpartonHead kernels.

Two subcommands, each reading rocprofv3 CSV output (``--output-format csv``):

  stats    --kernel-trace --stats:  per-kernel calls and mean/min/max duration.
  mfma     one --pmc pass of SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_MFMA and GRBM_GUI_ACTIVE:
           per kernel, the medians per dispatch and the matrix pipes' busy fraction,
           busy / (GPU cycles x 1024 SIMDs), GPU cycles = GRBM_GUI_ACTIVE / 8 XCDs.
  traffic  two --pmc passes (FETCH_SIZE, then WRITE_SIZE):  HBM bytes per dispatch
           of every SpartonHead kernel, scaled by what the same counters read for a
           plain device copy of known size (bench.py --copy-probe-mib N launches one
           torch copy of N MiB, i.e. N MiB read and N MiB written).

Example (FETCH pass and WRITE pass already collected under out/fetch and out/write):
    python -m sparton_amd.profiling traffic out/fetch out/write --copy-mib 1024 \\
        --json profiles/hbm_traffic_cfg2.json
"""
import argparse
import collections
import csv
import glob
import json
import os
import re
import sys

KIB = 1024


def _csvs(path, suffix):
    if os.path.isfile(path):
        return [path]
    return sorted(glob.glob(os.path.join(path, "**", f"*{suffix}"), recursive=True))


def short_name(name):
    """Readable kernel name: 'sparton::fwd::sparton_fwd_kernel<bf16>' style when mangled."""
    m = re.match(r"_ZN7sparton(\d)(\w+?)(\d+)(\w+?)I(DF16b|DF16_|f)", name)
    if m:
        ns_len = int(m.group(1))
        rest = m.group(2) + m.group(3) + m.group(4)
        ns, rest = rest[:ns_len], rest[ns_len:]
        klen = re.match(r"(\d+)", rest)
        kname = rest[len(klen.group(1)):len(klen.group(1)) + int(klen.group(1))] if klen else rest
        t = {"DF16b": "bf16", "DF16_": "f16", "f": "f32"}[m.group(5)]
        return f"sparton::{ns}::{kname}<{t}>"
    # rocprof's demangled names of kernels with int/bool template arguments: keep short
    # argument lists ('sparton::fwd::fwd_small_kernel<float, 2, true>'), elide long ones
    m = re.match(r"(?:void )?(sparton::\w+::\w+)<([^()]*)>\(", name)
    if m and len(m.group(2)) <= 40 and "_Accum" not in name:
        return f"{m.group(1)}<{m.group(2)}>"
    m = re.match(r"(?:void )?(sparton::\w+::\w+)<", name)
    if m and ("_Accum" in name or len(name) >= 90):
        return m.group(1) + "<...>"
    return name if len(name) < 90 else name[:87] + "..."


def kernel_stats(path):
    rows = []
    for p in _csvs(path, "kernel_stats.csv"):
        for r in csv.DictReader(open(p)):
            rows.append({"kernel": short_name(r["Name"]), "calls": int(r["Calls"]),
                         "mean_us": float(r["AverageNs"]) / 1e3, "min_us": float(r["MinNs"]) / 1e3,
                         "max_us": float(r["MaxNs"]) / 1e3, "pct": float(r["Percentage"])})
    return rows


def counter_values(path, counter):
    """Counter value of every dispatch, by kernel name."""
    acc = collections.defaultdict(list)
    for p in _csvs(path, "counter_collection.csv"):
        for r in csv.DictReader(open(p)):
            if r["Counter_Name"] == counter:
                acc[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return acc


def mfma(path, simds=1024, xcds=8):
    """{kernel: dict} of median MFMA counters per dispatch and the busy fraction."""
    import statistics
    busy = counter_values(path, "SQ_VALU_MFMA_BUSY_CYCLES")
    insts = counter_values(path, "SQ_INSTS_MFMA")
    grbm = counter_values(path, "GRBM_GUI_ACTIVE")
    out = {}
    for k, v in busy.items():
        if k not in grbm or k not in insts:
            continue
        b, n, g = statistics.median(v), statistics.median(insts[k]), statistics.median(grbm[k])
        if n <= 0:
            continue
        cyc = g / xcds
        out[short_name(k)] = {"dispatches": len(v), "gpu_cycles": cyc, "mfma_busy_cycles": b,
                              "mfma_insts": n, "busy_cycles_per_mfma": b / n,
                              "mfma_busy_frac": b / (cyc * simds)}
    return out


def _probe(values):
    """(value, kernel) of the largest single copy dispatch: the copy probe."""
    return max(((max(v), k) for k, v in values.items() if "copy" in k.lower() and "sparton" not in k),
               default=None)


def traffic(fetch_dir, write_dir, copy_mib):
    fvals = counter_values(fetch_dir, "FETCH_SIZE")
    wvals = counter_values(write_dir, "WRITE_SIZE")
    fetch = {k: (sum(v) / len(v), len(v)) for k, v in fvals.items()}
    write = {k: (sum(v) / len(v), len(v)) for k, v in wvals.items()}
    copy_bytes = copy_mib * KIB * KIB
    cf, cw = _probe(fvals), _probe(wvals)
    if cf is None or cw is None:
        raise SystemExit("no copy kernel found in the PMC output (run bench.py with --copy-probe-mib)")
    f_scale = copy_bytes / (cf[0] * KIB)
    w_scale = copy_bytes / (cw[0] * KIB)
    kernels = {}
    for k in sorted(set(fetch) | set(write)):
        if "sparton" not in k:
            continue
        fk = fetch.get(k, (0.0, 0))
        wk = write.get(k, (0.0, 0))
        kernels[short_name(k)] = {
            "fetch_kib_raw": round(fk[0], 1), "write_kib_raw": round(wk[0], 1),
            "dispatches": [fk[1], wk[1]],
            "hbm_read_bytes": round(fk[0] * KIB * f_scale),
            "hbm_write_bytes": round(wk[0] * KIB * w_scale),
            "traffic_bytes": round(fk[0] * KIB * f_scale + wk[0] * KIB * w_scale),
        }
    return {"copy_probe_bytes": copy_bytes, "copy_kernel": short_name(cf[1]),
            "copy_fetch_kib_raw": round(cf[0], 1), "copy_write_kib_raw": round(cw[0], 1),
            "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4), "kernels": kernels}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("path")
    m = sub.add_parser("mfma")
    m.add_argument("path")
    t = sub.add_parser("traffic")
    t.add_argument("fetch_dir")
    t.add_argument("write_dir")
    t.add_argument("--copy-mib", type=int, required=True)
    t.add_argument("--json", help="also write the result as JSON here")
    a = ap.parse_args(argv)
    if a.cmd == "stats":
        print(f"{'kernel':<60} {'calls':>6} {'mean us':>9} {'min us':>9} {'max us':>9} {'%':>6}")
        for r in kernel_stats(a.path):
            print(f"{r['kernel']:<60} {r['calls']:>6} {r['mean_us']:>9.1f} {r['min_us']:>9.1f} "
                  f"{r['max_us']:>9.1f} {r['pct']:>6.2f}")
    elif a.cmd == "mfma":
        for k, r in mfma(a.path).items():
            print(f"{k}: {r['dispatches']} dispatches, {r['gpu_cycles'] / 1e3:.1f} K GPU cycles, "
                  f"{r['mfma_insts'] / 1e6:.3f} M MFMA, {r['busy_cycles_per_mfma']:.1f} busy cycles "
                  f"per MFMA, matrix pipes busy {100 * r['mfma_busy_frac']:.1f}%")
    else:
        res = traffic(a.fetch_dir, a.write_dir, a.copy_mib)
        print(json.dumps(res, indent=1))
        if a.json:
            with open(a.json, "w") as f:
                json.dump(res, f, indent=1)
                f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
