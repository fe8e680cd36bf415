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

Workloads are of two kinds.  *Fused* workloads are calls of this library's
kernels; *unfused* workloads are calls of the reference's torch stage chain
(an unknown number of torch kernels per call) on the same inputs, whose
per-round kernel time τ_u and HBM bytes feed the decomposition checks of
``decodebench_amd.validate``.  The profiled program brackets every
workload's calls between two launches of the library's empty kernel
(``db_null_kernel``, the ``delimiter`` the manifest names), so a workload is
the dispatches between its two delimiters, whatever launched them; warm-up
calls made between workloads fall outside every segment.  Within a segment
the calls are the rounds: the dispatch count must be a whole number of
calls, and the kernel-name sequence must be periodic with a period that
divides a call (:func:`find_round_size`, the reference's round detection,
parse_ncu.py:26-48) -- a profiler-injected or stray kernel makes the
profile fail instead of silently shifting rounds.  Manifests without a
``delimiter`` (older profiles) match the library's dispatches in launch
order instead.

Three rocprofv3 runs of that program feed :func:`summarize`: ``--kernel-trace``
(durations), ``--pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE`` (KiB per dispatch,
one counter per run).  Both counters are scaled by what they read for the
calibration copy, so ``traffic`` is in bytes of the copy's scale:
``scale = copy_bytes / (median counter KiB of the copies * 1024)``.  The
read-only streaming probe (``read_calls`` launches over ``read_bytes``) is a
second calibration with the kernels' own load pattern; FETCH_SIZE must give
the same scale for both.  A fourth, optional run of the raw read-request
counters (:data:`RAW_READ_COUNTERS`) shows why the FETCH_SIZE scale is not 1
(:func:`request_bytes`).

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
READ_TAG = "stream_read_kernel"
DELIM_TAG = "null_kernel"
# The copy and the read-only probe must give one bytes-per-unit scale for a
# counter to within this fraction, or the profile is rejected.
SCALE_AGREEMENT = 0.05
# Raw L2->memory read-request counters (one rocprofv3 --pmc run): requests of
# any size, of 32 bytes, counted as 128-byte by the FETCH_SIZE formula
# (TCC_BUBBLE), and of 128 bytes as gfx950 reports them.
RAW_READ_COUNTERS = ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_BUBBLE_sum",
                     "TCC_EA0_RDREQ_128B_sum")


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


def find_round_size(names: list[str]) -> int:
    """Smallest period of a kernel-name sequence (the reference's round
    detection, validation/analysis/parse_ncu.py:26-48): [a, b, a, b] -> 2,
    [a, a, a] -> 1.  A sequence with no period raises ValueError."""
    n = len(names)
    for period in range(1, n // 2 + 1):
        if all(names[i] == names[i % period] for i in range(n)):
            return period
    if n >= 1 and len(set(names)) == 1:
        return 1
    raise ValueError(
        "kernel sequence is not periodic; cannot group rounds reliably. "
        f"Distinct kernels: {sorted(set(names))[:8]}. First 12: {names[:12]}")


def split_segments(dispatches: list[Dispatch],
                   manifest: dict) -> dict[str, list[list[Dispatch]]]:
    """Workloads as the dispatches between their begin and end delimiters.

    Returns ``{label: [[dispatches of call 0], [call 1], ...]}``; raises
    ValueError when the delimiters, the call count or the round structure do
    not match the manifest."""
    tag = manifest["delimiter"]
    marks = [i for i, d in enumerate(dispatches) if tag in d.name]
    work = manifest["workloads"]
    if len(marks) != 2 * len(work):
        raise ValueError(f"profile has {len(marks)} '{tag}' delimiters, manifest expects "
                         f"{2 * len(work)} (two per workload)")
    out = {}
    for j, w in enumerate(work):
        label, calls = w["label"], w["calls"]
        seg = dispatches[marks[2 * j] + 1:marks[2 * j + 1]]
        if w.get("kind", "fused") == "fused":
            # a fused call is the library's launches; a graph replay also runs
            # the fill kernel that zeroed its capture's F4 workspace (once per
            # replay, not per call), which is not part of any call
            seg = [d for d in seg if LIB_TAG in d.name]
        if not seg or len(seg) % calls:
            raise ValueError(f"{label}: {len(seg)} dispatches are not {calls} whole calls")
        per = len(seg) // calls
        k = w.get("kernels_per_call")
        if k is not None and per != k:
            raise ValueError(f"{label}: {per} kernels per call, manifest expects {k}")
        period = find_round_size([d.name for d in seg])
        if per % period:
            raise ValueError(f"{label}: kernel sequence period {period} does not divide the "
                             f"{per} kernels of a call")
        out[label] = [seg[i * per:(i + 1) * per] for i in range(calls)]
    return out


def split_workloads(dispatches: list[Dispatch], manifest: dict) -> dict[str, list[list[Dispatch]]]:
    """Assign the dispatches to the manifest's workloads.

    With a ``delimiter`` in the manifest, see :func:`split_segments`;
    otherwise the library's dispatches (less the read-probe calibration) are
    taken in launch order.
    Returns ``{label: [[dispatches of call 0], [call 1], ...]}``."""
    if manifest.get("delimiter"):
        return split_segments(dispatches, manifest)
    ours = [d for d in dispatches if LIB_TAG in d.name and READ_TAG not in d.name]
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


def read_scale(dispatches: list[Dispatch], manifest: dict, counter: str) -> float:
    """Bytes per counter unit, from the read-only probe's calibration launches."""
    reads = [d for d in dispatches if READ_TAG in d.name][: manifest["read_calls"]]
    if len(reads) < manifest["read_calls"]:
        raise ValueError(f"{counter}: read-probe calibration launches missing from the profile")
    kib = statistics.median(d.counters[counter] for d in reads)
    if kib <= 0:
        raise ValueError(f"{counter}: read-probe calibration reads {kib} units")
    return manifest["read_bytes"] / (kib * 1024.0)


def request_bytes(c: dict) -> dict:
    """Bytes read from memory per request size from the raw counters of one
    dispatch (or a sum of them): 128-byte requests as gfx950 counts them
    (TCC_EA0_RDREQ_128B), 32-byte ones, and the rest of TCC_EA0_RDREQ as
    64-byte; plus what the FETCH_SIZE formula makes of the same counters
    (it takes 128-byte requests from TCC_BUBBLE)."""
    rd, r32 = c["TCC_EA0_RDREQ_sum"], c["TCC_EA0_RDREQ_32B_sum"]
    bub, r128 = c["TCC_BUBBLE_sum"], c["TCC_EA0_RDREQ_128B_sum"]
    return {"requests": rd, "req_32B": r32, "req_128B": r128, "bubble": bub,
            "bytes_by_size": 128 * r128 + 64 * (rd - r128 - r32) + 32 * r32,
            "fetch_size_formula_bytes": 128 * bub + 64 * (rd - bub - r32) + 32 * r32}


def summarize(manifest: dict, trace=None, fetch=None, write=None, raw=None) -> dict:
    """Per-workload median kernel duration and scaled HBM traffic per call.

    With ``raw`` (a run of :data:`RAW_READ_COUNTERS`), the read requests of
    the calibration kernels and of every workload are broken down by size
    (:func:`request_bytes`)."""
    res: dict = {"copy_bytes": manifest["copy_bytes"], "mode": manifest.get("mode", "eager"),
                 "workloads": {}}
    per: dict[str, dict] = {w["label"]: {"algorithmic_bytes": w["algorithmic_bytes"]}
                            for w in manifest["workloads"]}
    warm = {w["label"]: w.get("warmup", 0) for w in manifest["workloads"]}
    kind = {w["label"]: w.get("kind", "fused") for w in manifest["workloads"]}
    for w in manifest["workloads"]:
        per[w["label"]]["kind"] = kind[w["label"]]
    if trace is not None:
        tw = split_workloads(trace, manifest)
        for label, calls in tw.items():
            calls = calls[warm[label]:]
            if not calls:
                raise ValueError(f"{label}: no calls left after {warm[label]} warm-up calls")
            total = statistics.median(sum(d.duration_ns for d in c) for c in calls) / 1e3
            per[label].update({"call_us": total, "kernels_per_call": len(calls[0]),
                               "GB/s": per[label]["algorithmic_bytes"] / (total * 1e3)})
            if kind[label] == "fused":
                kern = {}
                for j, d in enumerate(calls[0]):
                    durs = [c[j].duration_ns for c in calls]
                    kern[short_name(d.name)] = statistics.median(durs) / 1e3
                per[label]["kernel_us"] = kern
    for counter, disp, key in (("FETCH_SIZE", fetch, "fetch_bytes"),
                               ("WRITE_SIZE", write, "write_bytes")):
        if disp is None:
            continue
        scale = copy_scale(disp, manifest, counter)
        res[f"{counter}_scale"] = scale
        if manifest.get("read_calls") and counter == "FETCH_SIZE":
            rscale = read_scale(disp, manifest, counter)
            res[f"{counter}_read_scale"] = rscale
            if abs(rscale / scale - 1.0) > SCALE_AGREEMENT:
                raise ValueError(f"{counter}: the copy gives {scale:.3f} bytes per unit but the "
                                 f"read-only probe {rscale:.3f}; the counter's unit depends on "
                                 "the access pattern, so its traffic figures cannot be trusted")
        cw = split_workloads(disp, manifest)
        for label, calls in cw.items():
            calls = calls[warm[label]:]
            if not calls:
                raise ValueError(f"{label}: no calls left after {warm[label]} warm-up calls")
            per[label][key] = statistics.median(
                sum(d.counters[counter] for d in c) * 1024.0 * scale for c in calls)
    if raw is not None:
        def per_call(calls):
            tot = {k: statistics.median(sum(d.counters.get(k, 0.0) for d in c) for c in calls)
                   for k in RAW_READ_COUNTERS}
            return request_bytes(tot)

        calib = {}
        copies = [d for d in raw if COPY_TAG in d.name][: manifest["copy_calls"]]
        if copies:
            calib["copy"] = per_call([[d] for d in copies])
            calib["copy"]["bytes_read"] = manifest["copy_bytes"]
        if manifest.get("read_calls"):
            reads = [d for d in raw if READ_TAG in d.name][: manifest["read_calls"]]
            if reads:
                calib["read_probe"] = per_call([[d] for d in reads])
                calib["read_probe"]["bytes_read"] = manifest["read_bytes"]
        res["raw_read_requests"] = calib
        for label, calls in split_workloads(raw, manifest).items():
            calls = calls[warm[label]:]
            if calls:
                per[label]["read_requests"] = per_call(calls)
    # Traffic = reads + writes.  Reads come from the read requests counted by
    # size when that run exists: the FETCH_SIZE factor is calibrated on
    # 128-byte requests and doubles the 64-byte ones (kernel arguments, code,
    # small records), which matters for calls of a few MB.
    for label, p in per.items():
        if "write_bytes" not in p:
            continue
        if "fetch_bytes" in p:
            p["traffic_fetch_scaled_bytes"] = p["fetch_bytes"] + p["write_bytes"]
        if "read_requests" in p:
            p["traffic_bytes"] = p["read_requests"]["bytes_by_size"] + p["write_bytes"]
            p["traffic_source"] = "read requests by size + WRITE_SIZE"
        elif "fetch_bytes" in p:
            p["traffic_bytes"] = p["traffic_fetch_scaled_bytes"]
            p["traffic_source"] = "FETCH_SIZE x calibration + WRITE_SIZE"
        if "traffic_bytes" in p:
            p["traffic_over_algorithmic"] = p["traffic_bytes"] / p["algorithmic_bytes"]
    res["workloads"] = per
    return res


TRAFFIC_KEYS = ("fetch_bytes", "write_bytes", "read_requests", "traffic_bytes",
                "traffic_fetch_scaled_bytes", "traffic_over_algorithmic", "traffic_source")


def merge_traffic(res: dict, traffic: dict) -> dict:
    """Add the per-workload byte figures of a counter summary (``traffic``,
    this module's JSON of the FETCH_SIZE / WRITE_SIZE / raw-request runs) to
    a kernel-trace summary ``res``, matching workloads by label; workloads the
    counter runs did not cover keep empty byte columns."""
    tw = traffic.get("workloads", {})
    for label, p in res["workloads"].items():
        t = tw.get(label)
        if not t:
            continue
        if t.get("algorithmic_bytes") != p.get("algorithmic_bytes"):
            raise ValueError(f"{label}: algorithmic bytes {p.get('algorithmic_bytes')} in the "
                             f"trace but {t.get('algorithmic_bytes')} in the traffic summary")
        for k in TRAFFIC_KEYS:
            if k in t:
                p[k] = t[k]
    return res


def to_markdown(res: dict, command: str,
                title: str = "Fused decode kernels on MI355X: duration and HBM traffic per call",
                note: str = "") -> str:
    lines = [f"# {title}", "", "Commands (repo root, one MI355X):", "", "```", command.strip(),
             "```", ""]
    if note:
        lines += [note.strip(), ""]
    if "FETCH_SIZE_scale" in res:
        lines.append(f"Calibration: a {res['copy_bytes'] / 2**20:.0f} MiB device copy reads "
                     f"FETCH_SIZE x {res['FETCH_SIZE_scale']:.3f} and WRITE_SIZE x "
                     f"{res.get('WRITE_SIZE_scale', float('nan')):.3f} bytes per KiB-unit "
                     "(factors applied below).")
        if "FETCH_SIZE_read_scale" in res:
            lines.append(f"The read-only streaming probe (`db_stream_read`, 16-byte non-temporal "
                         f"loads) gives FETCH_SIZE x {res['FETCH_SIZE_read_scale']:.3f}; the "
                         f"pipeline rejects a profile where the two differ by more than "
                         f"{SCALE_AGREEMENT:.0%}.")
        lines.append("")
    if res.get("raw_read_requests"):
        lines += ["Read requests from L2 to memory by size (raw counters, one run; per "
                  "calibration kernel or per call):", "",
                  "| Kernel / workload | requests | 32 B | 128 B (TCC_EA0_RDREQ_128B) | "
                  "TCC_BUBBLE | bytes by size | FETCH_SIZE formula bytes | bytes read |",
                  "|---|---|---|---|---|---|---|---|"]
        rows = list(res["raw_read_requests"].items()) + [
            (k, p["read_requests"]) for k, p in res["workloads"].items() if "read_requests" in p]
        for label, r in rows:
            lines.append(f"| {label} | {r['requests']:,.0f} | {r['req_32B']:,.0f} | "
                         f"{r['req_128B']:,.0f} | {r['bubble']:,.0f} | "
                         f"{r['bytes_by_size']:,.0f} | {r['fetch_size_formula_bytes']:,.0f} | "
                         + (f"{r['bytes_read']:,}" if "bytes_read" in r else "") + " |")
        lines.append("")
    if any(p.get("kind") == "unfused" for p in res["workloads"].values()):
        lines.append("Rows ending in `_unfused` are the torch stage chain of the same config "
                     "(kernel time summed over a call); their 'Algorithmic B' is the byte "
                     "model's total (`bytes_model.total_bytes` of the stage traces).")
        lines.append("")
    by_size = any("read_requests" in p for p in res["workloads"].values())
    if by_size:
        lines.append("Traffic / algorithmic = (read bytes by request size + WRITE_SIZE) / "
                     "algorithmic bytes. 'Fetch B' is FETCH_SIZE times the calibration factor, "
                     "which is right for 128-byte requests and counts each 64-byte request "
                     "(kernel arguments, code, small records) twice.")
        lines.append("")
    lines += ["| Workload | Kernel us (median) | Call us | Algorithmic B | GB/s | % of 8 TB/s | "
              "Fetch B | " + ("Read B by size | " if by_size else "") +
              "Write B | Traffic / algorithmic |",
              "|---|---|---|---|---|---|---|---|---|" + ("---|" if by_size else "")]
    for label, p in res["workloads"].items():
        if p.get("kind") == "unfused":
            ku = f"{p.get('kernels_per_call', '?')} torch kernels (unfused stages)"
        else:
            ku = "; ".join(f"{k.split('::')[-1]} {v:.2f}"
                           for k, v in p.get("kernel_us", {}).items())
        call = p.get("call_us")
        gbs = p.get("GB/s")

        def num(key, fmt):
            return format(p[key], fmt) if key in p else ""

        timing = (f"{ku} | {call:.2f} | {p['algorithmic_bytes']:,} | {gbs:.0f} | "
                  f"{gbs / 80:.1f}" if call is not None
                  else f" | | {p['algorithmic_bytes']:,} | | ")
        rb = ""
        if by_size:
            rb = (f"{p['read_requests']['bytes_by_size']:,.0f}" if "read_requests" in p else "")
            rb += " | "
        lines.append(f"| {label} | {timing} | {num('fetch_bytes', ',.0f')} | {rb}"
                     f"{num('write_bytes', ',.0f')} | {num('traffic_over_algorithmic', '.3f')} |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="summarise rocprofv3 runs of bench.py --profile-pass")
    ap.add_argument("--manifest", required=True)
    ap.add_argument("--trace")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--raw", help="counter CSV of a run of the raw read-request counters")
    ap.add_argument("--traffic", help="JSON of a counter summary (--json of a FETCH_SIZE / "
                    "WRITE_SIZE run) whose byte columns are added to this summary's workloads")
    ap.add_argument("--md")
    ap.add_argument("--json")
    ap.add_argument("--command", default="", help="command line recorded in the markdown")
    ap.add_argument("--title", default=None, help="markdown title")
    ap.add_argument("--note", default="", help="paragraph recorded under the commands")
    args = ap.parse_args(argv)
    manifest = json.loads(Path(args.manifest).read_text())
    res = summarize(manifest,
                    trace=read_trace(args.trace) if args.trace else None,
                    fetch=read_counters(args.fetch) if args.fetch else None,
                    write=read_counters(args.write) if args.write else None,
                    raw=read_counters(args.raw) if args.raw else None)
    if args.traffic:
        merge_traffic(res, json.loads(Path(args.traffic).read_text()))
    if args.json:
        Path(args.json).write_text(json.dumps(res, indent=1, sort_keys=True) + "\n")
    text = (to_markdown(res, args.command, args.title, args.note) if args.title
            else to_markdown(res, args.command, note=args.note))
    if args.md:
        Path(args.md).write_text(text)
    print(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
