"""OCP fp8 e4m3 weight quantisation with one fp32 scale per output row.

The fp8 GEMV entry points take ``W`` as ``torch.float8_e4m3fn`` [N, K] (one
byte per weight) plus ``scale`` fp32 [N] and compute
``y[n] = fp16(scale[n] * sum_k e4m3(W[n, k]) * x[k])`` in fp32.  This module
produces such a pair from an fp16/fp32 matrix: per-row absmax scaling onto
the e4m3 range (max finite 448), round-to-nearest-even, saturating.

This is data preparation, run once per weight matrix (on the GPU or the
CPU); no kernel path calls it.
"""

from __future__ import annotations

E4M3_MAX = 448.0


def quantize_e4m3_rows(W):
    """Return ``(Wq, scale)``: Wq float8_e4m3fn [N, K], scale float32 [N].

    ``scale[n] = max_k |W[n, k]| / 448`` (1 for an all-zero row), and
    ``Wq[n] = e4m3(clamp(W[n] / scale[n], -448, 448))``."""
    import torch

    if W.dim() != 2:
        raise ValueError(f"expected a [N, K] matrix, got shape {tuple(W.shape)}")
    Wf = W.float()
    amax = Wf.abs().amax(dim=1)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = (Wf / scale[:, None]).clamp_(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q.contiguous(), scale.contiguous()


def dequantize_e4m3_rows(Wq, scale):
    """fp32 [N, K] matrix ``scale[n] * e4m3(Wq[n, k])`` (exact in fp32)."""
    return Wq.float() * scale.float()[:, None]
