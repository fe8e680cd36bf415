"""Write tests/golden/stats_vectors.json from the reference's stats module.

The exact endpoints of bootstrap_diff_ci depend on the order in which the
reference draws from numpy's generator (src/decodebench/stats.py:43-54); the
reference's own tests only check orderings, so the only way to pin them is to
run the reference function.  This script imports that one file (numpy only)
from /root/reference by path and records inputs and outputs; the committed
JSON is what the tests read, so /root/reference is not needed at test time.

    python tests/golden/gen_stats_vectors.py
"""

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

REF = Path("/root/reference/src/decodebench/stats.py")
OUT = Path(__file__).resolve().parent / "stats_vectors.json"


def main() -> None:
    spec = importlib.util.spec_from_file_location("ref_stats", REF)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ref_stats"] = mod  # dataclasses look their module up
    spec.loader.exec_module(mod)
    rng = np.random.default_rng(7)
    cases = []
    for n_a, n_b, n_res, seed, ci in [(30, 30, 10000, 42, 0.95), (10, 17, 1000, 3, 0.9),
                                      (200, 200, 1000, 42, 0.95), (5, 3, 257, 11, 0.5)]:
        a = np.round(rng.normal(20.0, 1.5, n_a), 6).tolist()
        b = np.round(rng.normal(16.0, 1.0, n_b), 6).tolist()
        lo, hi, point = mod.bootstrap_diff_ci(a, b, n_resamples=n_res, ci=ci, seed=seed)
        s = mod.summarize(a)
        cases.append({"a": a, "b": b, "n_resamples": n_res, "seed": seed, "ci": ci,
                      "lo": lo, "hi": hi, "point": point,
                      "summary_a": [s.median, s.p25, s.p75, s.n]})
    OUT.write_text(json.dumps({"source": "src/decodebench/stats.py:17-57", "cases": cases},
                              indent=1))
    print(f"wrote {OUT} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
