"""rocprofv3 counter pipeline: per-dispatch HBM bytes and durations per workload.

The MI355X counterpart of the reference's NCU tooling
(validation/analysis/parse_ncu.py:26-148 finds the rounds of a profiled run and
reduces per-kernel DRAM bytes and durations; validation/scripts/ncu_collect.sh:31
lists the metrics).  Here the profiled program is ``bench.py --profile-pass``,
which writes a manifest of what it launched, in order:

  1. ``copy_calls`` device-to-device copies of ``copy_bytes`` bytes (the
     calibration kernel: it reads and writes exactly ``copy_bytes``);
  2. for each workload, ``calls`` fused calls of ``kernels_per_call`` HIP
     kernels of this library each, over cache-defeating replicas.

Three rocprofv3 runs of that program feed :func:`summarize`: ``--kernel-trace``
(durations), ``--pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE`` (KiB per dispatch,
one counter per run).  Both counters are scaled by what they read for the
calibration copy, so ``traffic`` is in bytes of the copy's scale:
``scale = copy_bytes / (median counter KiB of the copies * 1024)``.

    python -m decodebench_amd.rocprof --manifest M.json --trace T.csv \\
        --fetch F.csv --write W.csv --md out.md --json out.json

Workload dispatches are matched in launch order: the library's kernels (names
containing ``dbk::``) are taken ``calls * kernels_per_call`` at a time, so the
profiled program must launch nothing else from this library.  The first
``warmup`` calls of a workload are dropped before taking medians.
"""

from __future__ import annotations

import argparse
import csv
import json
import statistics
from dataclasses import dataclass, field
from pathlib import Path

LIB_TAG = "dbk::"
COPY_TAG = "copyBuffer"


@dataclass
class Dispatch:
    dispatch_id: int
    name: str
    grid: int
    workgroup: int
    duration_ns: int = 0
    counters: dict = field(default_factory=dict)


def _int(v) -> int:
    return int(float(v))


def short_name(name: str) -> str:
    """Kernel name without its trailing parameter list."""
    if not name.endswith(")"):
        return name
    depth = 0
    for i in range(len(name) - 1, -1, -1):
        if name[i] == ")":
            depth += 1
        elif name[i] == "(":
            depth -= 1
            if depth == 0:
                return name[:i]
    return name


def read_trace(path) -> list[Dispatch]:
    """Dispatches of a ``--kernel-trace`` CSV, in dispatch order."""
    out = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            out.append(Dispatch(
                dispatch_id=_int(r["Dispatch_Id"]), name=r["Kernel_Name"],
                grid=_int(r.get("Grid_Size_X") or r.get("Grid_Size") or 0),
                workgroup=_int(r.get("Workgroup_Size_X") or r.get("Workgroup_Size") or 0),
                duration_ns=_int(r["End_Timestamp"]) - _int(r["Start_Timestamp"])))
    out.sort(key=lambda d: d.dispatch_id)
    return out


def read_counters(path) -> list[Dispatch]:
    """Dispatches of a ``--pmc`` counter-collection CSV (one row per counter)."""
    by_id: dict[int, Dispatch] = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            did = _int(r["Dispatch_Id"])
            d = by_id.get(did)
            if d is None:
                d = by_id[did] = Dispatch(
                    dispatch_id=did, name=r["Kernel_Name"], grid=_int(r.get("Grid_Size", 0)),
                    workgroup=_int(r.get("Workgroup_Size", 0)))
            d.counters[r["Counter_Name"]] = d.counters.get(r["Counter_Name"], 0.0) + float(
                r["Counter_Value"])
    return [by_id[k] for k in sorted(by_id)]


def split_workloads(dispatches: list[Dispatch], manifest: dict) -> dict[str, list[list[Dispatch]]]:
    """Assign the library's dispatches to the manifest's workloads, in order.

    Returns ``{label: [[dispatches of call 0], [call 1], ...]}``."""
    ours = [d for d in dispatches if LIB_TAG in d.name]
    need = sum(w["calls"] * w["kernels_per_call"] for w in manifest["workloads"])
    if len(ours) != need:
        raise ValueError(f"profile has {len(ours)} library dispatches, manifest expects {need}")
    out, i = {}, 0
    for w in manifest["workloads"]:
        k = w["kernels_per_call"]
        calls = []
        for _ in range(w["calls"]):
            calls.append(ours[i:i + k])
            i += k
        out[w["label"]] = calls
    return out


def copy_scale(dispatches: list[Dispatch], manifest: dict, counter: str) -> float:
    """Bytes per counter unit, from the calibration copies (the first copies)."""
    copies = [d for d in dispatches if COPY_TAG in d.name][: manifest["copy_calls"]]
    if len(copies) < manifest["copy_calls"]:
        raise ValueError(f"{counter}: calibration copies missing from the profile")
    kib = statistics.median(d.counters[counter] for d in copies)
    if kib <= 0:
        raise ValueError(f"{counter}: calibration copy reads {kib} KiB")
    return manifest["copy_bytes"] / (kib * 1024.0)


def summarize(manifest: dict, trace=None, fetch=None, write=None) -> dict:
    """Per-workload median kernel duration and scaled HBM traffic per call."""
    res: dict = {"copy_bytes": manifest["copy_bytes"], "workloads": {}}
    per: dict[str, dict] = {w["label"]: {"algorithmic_bytes": w["algorithmic_bytes"]}
                            for w in manifest["workloads"]}
    warm = {w["label"]: w.get("warmup", 0) for w in manifest["workloads"]}
    if trace is not None:
        tw = split_workloads(trace, manifest)
        for label, calls in tw.items():
            calls = calls[warm[label]:]
            kern = {}
            for j, d in enumerate(calls[0]):
                durs = [c[j].duration_ns for c in calls]
                kern[short_name(d.name)] = statistics.median(durs) / 1e3
            total = statistics.median(sum(d.duration_ns for d in c) for c in calls) / 1e3
            per[label].update({"kernel_us": kern, "call_us": total,
                               "GB/s": per[label]["algorithmic_bytes"] / (total * 1e3)})
    for counter, disp, key in (("FETCH_SIZE", fetch, "fetch_bytes"),
                               ("WRITE_SIZE", write, "write_bytes")):
        if disp is None:
            continue
        scale = copy_scale(disp, manifest, counter)
        res[f"{counter}_scale"] = scale
        cw = split_workloads(disp, manifest)
        for label, calls in cw.items():
            calls = calls[warm[label]:]
            per[label][key] = statistics.median(
                sum(d.counters[counter] for d in c) * 1024.0 * scale for c in calls)
    for label, p in per.items():
        if "fetch_bytes" in p and "write_bytes" in p:
            p["traffic_bytes"] = p["fetch_bytes"] + p["write_bytes"]
            p["traffic_over_algorithmic"] = p["traffic_bytes"] / p["algorithmic_bytes"]
    res["workloads"] = per
    return res


def to_markdown(res: dict, command: str) -> str:
    lines = ["# Fused decode kernels on MI355X: duration and HBM traffic per call", "",
             "Commands (repo root, one MI355X):", "", "```", command.strip(), "```", ""]
    if "FETCH_SIZE_scale" in res:
        lines.append(f"Calibration: a {res['copy_bytes'] / 2**20:.0f} MiB device copy reads "
                     f"FETCH_SIZE x {res['FETCH_SIZE_scale']:.3f} and WRITE_SIZE x "
                     f"{res.get('WRITE_SIZE_scale', float('nan')):.3f} bytes per KiB-unit "
                     "(factors applied below).")
        lines.append("")
    lines += ["| Workload | Kernel us (median) | Call us | Algorithmic B | GB/s | % of 8 TB/s | "
              "Fetch B | Write B | Traffic / algorithmic |",
              "|---|---|---|---|---|---|---|---|---|"]
    for label, p in res["workloads"].items():
        ku = "; ".join(f"{k.split('::')[-1]} {v:.2f}" for k, v in p.get("kernel_us", {}).items())
        call = p.get("call_us")
        gbs = p.get("GB/s")
        lines.append(
            f"| {label} | {ku} | {call:.2f} | {p['algorithmic_bytes']:,} | {gbs:.0f} | "
            f"{gbs / 80:.1f} | {p.get('fetch_bytes', float('nan')):,.0f} | "
            f"{p.get('write_bytes', float('nan')):,.0f} | "
            f"{p.get('traffic_over_algorithmic', float('nan')):.3f} |"
            if call is not None else f"| {label} | | | {p['algorithmic_bytes']:,} | | | | | |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="summarise rocprofv3 runs of bench.py --profile-pass")
    ap.add_argument("--manifest", required=True)
    ap.add_argument("--trace")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--md")
    ap.add_argument("--json")
    ap.add_argument("--command", default="", help="command line recorded in the markdown")
    args = ap.parse_args(argv)
    manifest = json.loads(Path(args.manifest).read_text())
    res = summarize(manifest,
                    trace=read_trace(args.trace) if args.trace else None,
                    fetch=read_counters(args.fetch) if args.fetch else None,
                    write=read_counters(args.write) if args.write else None)
    if args.json:
        Path(args.json).write_text(json.dumps(res, indent=1, sort_keys=True) + "\n")
    text = to_markdown(res, args.command)
    if args.md:
        Path(args.md).write_text(text)
    print(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
