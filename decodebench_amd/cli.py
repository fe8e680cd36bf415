"""``decodebench`` command line: demo, profile, sweep, calibrate.

The ``demo``, ``profile`` and ``sweep`` commands keep the reference's CLI
(src/decodebench/cli.py:16-170): the same arguments, defaults, dry-run lines,
error messages and exit codes, and the same sweep CSV header, so scripts
written against the reference run unchanged:

    python -m decodebench_amd.cli demo f1 --dim 4096 --batch 1
    python -m decodebench_amd.cli profile my_chain.py:build --trials 30
    python -m decodebench_amd.cli sweep f4 --batch 1,2,4 --csv sweep.csv

Two additions for this build:

* ``demo --fused`` (and ``sweep --fused``) also times this library's HIP
  kernel for the demo (F1, F2 or F4) as the ``fused=`` variant of
  ``Sequence.profile``, so the report adds the fused time and its residual;
* ``calibrate --null | --gate-g2`` is the calibration harness
  (validation/src/bench/calibrate.cu:42-230, see
  ``decodebench_amd.calibrate``); ``calibrate --vendor-f4`` adds F4 against
  torch's scaled_dot_product_attention.

The GPU is only touched after argument validation and dry runs.
"""

from __future__ import annotations

import argparse
import csv
import os
import runpy
import sys

from decodebench_amd.verdict import DEFAULT_BYTE_THRESHOLD


def _int_list(text: str) -> list[int]:
    """``"1,2,4"`` -> ``[1, 2, 4]``; anything else is an argparse error."""
    items = [part.strip() for part in text.split(",")]
    if not items or not all(part.lstrip("-").isdigit() for part in items if part):
        raise argparse.ArgumentTypeError(f"expected integers separated by commas, got {text!r}")
    return [int(part) for part in items if part]


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(
        prog="decodebench",
        description=("Split a decode-chain fusion gain into launch overhead (stream vs graph "
                     "replay) and an analytic estimate of the intermediate bytes it removes."))
    sub = parser.add_subparsers(dest="command", required=True)

    def timing_opts(p, threshold=True):
        p.add_argument("--trials", type=int, default=30, help="timed trials per variant")
        if threshold:
            p.add_argument("--byte-threshold", type=float, default=DEFAULT_BYTE_THRESHOLD,
                           help="eliminable/total byte ratio above which bytes are material")
        p.add_argument("--dry-run", action="store_true",
                       help="print what would run, touch no GPU")

    demo_p = sub.add_parser("demo", help="profile one of the Llama-shaped decode demos")
    demo_p.add_argument("name", choices=["f1", "f2", "f4"],
                        help="f1 RMSNorm->GEMV, f2 gate/up+SwiGLU, f4 attention")
    demo_p.add_argument("--dim", type=int, choices=[2048, 4096], default=4096,
                        help="model width")
    demo_p.add_argument("--batch", type=int, default=1, help="decode batch rows")
    timing_opts(demo_p)
    demo_p.add_argument("--csv", type=str, help="write every trial to this CSV file")
    demo_p.add_argument("--fused", action="store_true",
                        help="add this library's HIP kernel as the fused variant")

    prof_p = sub.add_parser("profile", help="profile a Sequence built by your own script")
    prof_p.add_argument("target", help="FILE.py:FUNCTION returning (sequence, inputs)")
    timing_opts(prof_p)
    prof_p.add_argument("--csv", type=str, help="write every trial to this CSV file")

    sweep_p = sub.add_parser("sweep", help="profile a demo over several batch sizes")
    sweep_p.add_argument("name", choices=["f1", "f2", "f4"],
                         help="f1 RMSNorm->GEMV, f2 gate/up+SwiGLU, f4 attention")
    sweep_p.add_argument("--batch", type=_int_list, default=[1, 2, 4, 8],
                         help="batch sizes, e.g. 1,2,4,8")
    sweep_p.add_argument("--dim", type=int, choices=[2048, 4096], default=4096,
                         help="model width")
    timing_opts(sweep_p, threshold=False)
    sweep_p.add_argument("--csv", type=str, help="write one summary row per batch to this CSV")
    sweep_p.add_argument("--fused", action="store_true",
                         help="add this library's HIP kernel as the fused variant")

    cal_p = sub.add_parser("calibrate", help="launch-cost and bandwidth calibration")
    cal_p.add_argument("--null", action="store_true",
                       help="cost of an empty launch, eager and replayed from a graph")
    cal_p.add_argument("--gate-g2", action="store_true",
                       help="fp16 GEMV bandwidth against the vendor BLAS (G2 gate)")
    cal_p.add_argument("--stream-floor", action="store_true",
                       help="single-launch streaming floor: bytes read by one launch vs time")
    cal_p.add_argument("--iters", type=int, default=None,
                       help="launches per measurement (default: 500 empty, 200 GEMV)")
    cal_p.add_argument("--no-rotate", action="store_true",
                       help="G2 on a single weight copy (it then stays in the caches)")
    cal_p.add_argument("--vendor-f4", action="store_true",
                       help="F4 against torch scaled_dot_product_attention")
    cal_p.add_argument("--kv-len", type=int, default=8192, help="KV length for --vendor-f4")
    cal_p.add_argument("--kv-batch", type=int, default=1, help="batch for --vendor-f4")
    cal_p.add_argument("--dry-run", action="store_true",
                       help="print what would run, touch no GPU")
    return parser


def _gpu_or_error() -> bool:
    import torch

    if not torch.cuda.is_available():
        print("Error: GPU/CUDA is not available.", file=sys.stderr)
        return False
    return True


def _print_report(report, csv_path) -> int:
    try:
        print(report.render())
    except RuntimeError as e:
        print(f"Error: {e}", file=sys.stderr)
        return 1
    if csv_path:
        report.to_csv(csv_path)
        print(f"Saved trials to {csv_path}")
    return 0


def _demo(args) -> int:
    if args.dry_run:
        print(f"[dry-run] demo {args.name} with dim={args.dim}, batch={args.batch}, "
              f"trials={args.trials}, threshold={args.byte_threshold}"
              + (", fused=hip" if args.fused else ""))
        return 0
    if not _gpu_or_error():
        return 1
    from decodebench_amd.demos.llama_decode import build_demo, demo_fused

    seq, inputs, replicas = build_demo(args.name, dim=args.dim, batch=args.batch)
    fused = demo_fused(args.name) if args.fused else None
    report = seq.profile(inputs, trials=args.trials, byte_threshold=args.byte_threshold,
                         input_replicas=replicas, fused=fused)
    return _print_report(report, args.csv)


def _load_target(path: str, name: str):
    """Execute the user's file as a script module and return its ``name``."""
    namespace = runpy.run_path(path, run_name="decodebench_target")
    fn = namespace.get(name)
    if not callable(fn):
        raise AttributeError(f"{path} defines no function {name!r}")
    return fn


def _profile(args) -> int:
    if ":" not in args.target:
        print("Error: Target must be in the format 'path/to/module.py:build_fn'", file=sys.stderr)
        return 2
    module_path, build_fn_name = args.target.split(":", 1)
    if args.dry_run:
        print(f"[dry-run] profile target {module_path}:{build_fn_name} with trials={args.trials}, "
              f"threshold={args.byte_threshold}")
        return 0
    if not os.path.exists(module_path):
        print(f"Error: Module path '{module_path}' does not exist.", file=sys.stderr)
        return 1
    try:
        build_fn = _load_target(module_path, build_fn_name)
    except Exception as e:  # report any failure of the user's file, then stop
        print(f"Error loading target: {e}", file=sys.stderr)
        return 1
    if not _gpu_or_error():
        return 1
    seq, inputs = build_fn()
    report = seq.profile(inputs, trials=args.trials, byte_threshold=args.byte_threshold)
    return _print_report(report, args.csv)


SWEEP_HEADER = ["demo", "dim", "batch", "trials", "t_stream_us", "t_graph_us", "delta_launch_us",
                "b_bytes_est_us", "bound", "total_bytes", "eliminable_bytes", "ci_lo", "ci_hi"]


def _sweep(args) -> int:
    if args.dry_run:
        print(f"[dry-run] sweep demo {args.name} with batch={args.batch}, dim={args.dim}, "
              f"trials={args.trials}" + (", fused=hip" if args.fused else ""))
        return 0
    if not _gpu_or_error():
        return 1
    from decodebench_amd.demos.llama_decode import build_demo, demo_fused

    rows = []
    for b in args.batch:
        print(f"Sweeping {args.name} dim={args.dim} batch={b}...")
        seq, inputs, replicas = build_demo(args.name, dim=args.dim, batch=b)
        fused = demo_fused(args.name) if args.fused else None
        report = seq.profile(inputs, trials=args.trials, input_replicas=replicas, fused=fused)
        try:
            v = report.verdict()
        except RuntimeError as e:
            print(f"  WARN: {e}", file=sys.stderr)
            continue
        ci_lo = v.delta_launch_ci[0] if v.delta_launch_ci else 0.0
        ci_hi = v.delta_launch_ci[1] if v.delta_launch_ci else 0.0
        line = f"  Stream: {v.t_stream:.2f} us | Graph: {v.t_graph:.2f} us | Bound: {v.bound}"
        if v.t_fused is not None:
            line += f" | Fused: {v.t_fused:.2f} us"
        print(line)
        rows.append([args.name, args.dim, b, args.trials, f"{v.t_stream:.2f}",
                     f"{v.t_graph:.2f}", f"{v.delta_launch:.2f}", f"{v.b_bytes_est:.2f}",
                     v.bound, v.total_bytes, v.eliminable_bytes, f"{ci_lo:.2f}", f"{ci_hi:.2f}"])
    if args.csv:
        with open(args.csv, "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(SWEEP_HEADER)
            w.writerows(rows)
        print(f"Saved sweep results to {args.csv}")
    return 0


def _calibrate(args) -> int:
    if not (args.null or args.gate_g2 or args.vendor_f4 or args.stream_floor):
        print("Error: calibrate needs --null, --gate-g2, --stream-floor and/or --vendor-f4",
              file=sys.stderr)
        return 2
    if args.iters is not None and args.iters < 1:
        print("Error: --iters must be >= 1", file=sys.stderr)
        return 2
    if args.kv_len < 1 or args.kv_batch < 1:
        print("Error: --kv-len and --kv-batch must be >= 1", file=sys.stderr)
        return 2
    if args.dry_run:
        what = [w for w, on in (("null", args.null), ("gate-g2", args.gate_g2),
                                ("stream-floor", args.stream_floor),
                                ("vendor-f4", args.vendor_f4)) if on]
        print(f"[dry-run] calibrate {' '.join(what)} with iters={args.iters or 'default'}, "
              f"rotate={not args.no_rotate}"
              + (f", kv_len={args.kv_len}, kv_batch={args.kv_batch}" if args.vendor_f4 else ""))
        return 0
    if not _gpu_or_error():
        return 1
    from decodebench_amd import calibrate

    rc = 0
    if args.null:
        print(calibrate.null_launch(iters=args.iters or 500).render())
    if args.gate_g2:
        g2 = calibrate.gate_g2(iters=args.iters or 200, rotate=not args.no_rotate)
        print(g2.render())
        if g2.max_abs_diff > 5e-2:
            print(f"Error: GEMV output differs from the vendor BLAS by {g2.max_abs_diff:.3e}",
                  file=sys.stderr)
            rc = 1
    if args.stream_floor:
        print(calibrate.stream_floor().render())
    if args.vendor_f4:
        v = calibrate.vendor_f4(L=args.kv_len, B=args.kv_batch)
        print(v.render())
        if v.max_abs_diff > 5e-3:
            print(f"Error: F4 output differs from torch SDPA by {v.max_abs_diff:.3e}",
                  file=sys.stderr)
            rc = 1
    return rc


def main(argv: list[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    return {"demo": _demo, "profile": _profile, "sweep": _sweep,
            "calibrate": _calibrate}[args.command](args)


if __name__ == "__main__":
    sys.exit(main())
