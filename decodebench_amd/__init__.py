"""decodebench_amd: DecodeBench's fused decode hot path, MI355X-native.

The host API mirrors the reference package ``decodebench``
(src/decodebench/__init__.py:8-26): ``Sequence`` stages, ``profile`` with
stream / graph / fused timing, ``Report`` and ``Verdict`` with Delta_launch and
B, the byte model and the statistics.  The fused kernels (F1 RMSNorm->GEMV,
F2 gate/up GEMV + SwiGLU, F4 split-KV GQA FlashDecode) are hand-written HIP
for gfx950 in ``csrc/``, reached through the C ABI of
``include/decodebench_hip.h`` by ``decodebench_amd.ops``.

torch is imported lazily: the byte model, verdict, report and statistics work
without it, as in the reference.
"""

__version__ = "0.1.0"

from decodebench_amd.bytes_model import StageTrace, eliminable_bytes, total_bytes
from decodebench_amd.report import Report
from decodebench_amd.sequence import Sequence
from decodebench_amd.stats import Summary, bootstrap_diff_ci, summarize
from decodebench_amd.verdict import Verdict, compute_verdict

__all__ = [
    "__version__",
    "StageTrace",
    "eliminable_bytes",
    "total_bytes",
    "Verdict",
    "compute_verdict",
    "Report",
    "Summary",
    "bootstrap_diff_ci",
    "summarize",
    "Sequence",
]
