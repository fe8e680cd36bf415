"""The reference's PyTorch stage definitions, restated for CPU tensors.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  These are the functions
the north-star parity criterion names: the fused HIP kernels must match them
on the same seeded inputs within rtol 1e-2 / atol 1e-2.

Each stage restates a stage body of src/decodebench/demos/llama_decode.py
with the benchmark's settings where the reference leaves them open:
  * rmsnorm eps 1e-6 (llama_decode.py:39 already uses 1e-6);
  * attention scale 1/sqrt(D) applied to the fp32 scores (the reference demo
    has no scale, llama_decode.py:125; its CUDA kernels and harness oracle do,
    f4.cu:195 and bench_variant.cu:189);
  * grouped-query attention: query head h reads KV head h // G, G = Hq / Hkv
    (the reference demo is MHA, llama_decode.py:110-116).
The tensors stay fp16 wherever the reference keeps them fp16, so rounding
happens at the same points.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def rmsnorm(x: torch.Tensor, g: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """llama_decode.py:36-39 -- fp32 statistic, fp16 normalised output."""
    var = x.float().pow(2).mean(dim=-1, keepdim=True)
    return (x.float() * torch.rsqrt(var + eps)).half() * g


def gemv(xh: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
    """llama_decode.py:41-43 -- xh . W^T, fp16 in/out."""
    return F.linear(xh, W)


def gate(xh: torch.Tensor, Wg: torch.Tensor) -> torch.Tensor:
    """llama_decode.py:77-79."""
    return F.linear(xh, Wg)


def up(xh: torch.Tensor, Wu: torch.Tensor) -> torch.Tensor:
    """llama_decode.py:81-83."""
    return F.linear(xh, Wu)


def swiglu(up_out: torch.Tensor, gate_out: torch.Tensor) -> torch.Tensor:
    """llama_decode.py:85-87 -- silu(gate) * up on fp16 tensors."""
    return F.silu(gate_out) * up_out


def scores(q: torch.Tensor, K: torch.Tensor, scale: float) -> torch.Tensor:
    """llama_decode.py:120-125 with GQA and the scale: fp16 q.K, fp32 out.

    q [B,Hq,D], K [B,Hkv,L,D] -> [B,Hq,L] fp32."""
    B, Hq, D = q.shape
    Hkv, L = K.shape[1], K.shape[2]
    qg = q.reshape(B, Hkv, Hq // Hkv, D)
    s = torch.matmul(qg, K.transpose(-1, -2).contiguous())  # fp16 [B,Hkv,G,L]
    return s.float().mul(scale).reshape(B, Hq, L)


def softmax(s: torch.Tensor) -> torch.Tensor:
    """llama_decode.py:127-129 -- fp32 softmax over L."""
    return torch.softmax(s, dim=-1)


def weighted_v(p: torch.Tensor, V: torch.Tensor) -> torch.Tensor:
    """llama_decode.py:131-134 -- p rounded to fp16, then p . V in fp16."""
    B, Hq, L = p.shape
    Hkv, D = V.shape[1], V.shape[3]
    pg = p.half().reshape(B, Hkv, Hq // Hkv, L)
    return torch.matmul(pg, V).reshape(B, Hq, D)


# ------------------------------------------------------------ whole chains
def f1(x, g, W, eps: float = 1e-6) -> torch.Tensor:
    return gemv(rmsnorm(x, g, eps), W)


def f2(x, Wg, Wu) -> torch.Tensor:
    return swiglu(up(x, Wu), gate(x, Wg))


def f4(q, K, V, scale: float | None = None) -> torch.Tensor:
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    return weighted_v(softmax(scores(q, K, scale)), V)


# ------------------------------------------------ fp8 e4m3 weight stages
def gemv_fp8(xh: torch.Tensor, Wq: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """gemv with OCP e4m3 weights and one fp32 scale per output row:
    fp16(scale * (xh . e4m3(Wq)^T)), dequantised exactly and accumulated in
    fp32 (the reference has no fp8 stage; this is the definition the fp8
    entry points follow: dequantise-then-GEMV equals GEMV-then-scale)."""
    return (F.linear(xh.float(), Wq.float()) * scale.float()).half()


def f1_fp8(x, g, Wq, s, eps: float = 1e-6) -> torch.Tensor:
    return gemv_fp8(rmsnorm(x, g, eps), Wq, s)


def f2_fp8(x, Wgq, sg, Wuq, su) -> torch.Tensor:
    return swiglu(gemv_fp8(x, Wuq, su), gemv_fp8(x, Wgq, sg))


def f2_rmsnorm(x, g, Wg, Wu, eps: float = 1e-6) -> torch.Tensor:
    """rmsnorm followed by the F2 stages (the chain's post-attention half)."""
    return f2(rmsnorm(x, g, eps), Wg, Wu)


def decode_layer(x, g1, Wqkv, K, V, Wo, g2, Wg, Wu, Wd, n_q_heads: int,
                 eps: float = 1e-6, scales: dict | None = None) -> torch.Tensor:
    """Config-5 chain: RMSNorm -> QKV -> attention -> O -> RMSNorm -> SwiGLU -> down.

    x [B,d]; Wqkv [(Hq+2Hkv)*D, d]; K/V cache [B,Hkv,L,D] (the new token's k, v
    are not appended: the chain measures the decode read path); Wo [d, Hq*D];
    Wg/Wu [F, d]; Wd [d, F].  With ``scales`` (keys "qkv", "o", "gate", "up",
    "down") the weights are e4m3 and every projection is gemv_fp8."""
    B = x.shape[0]
    D = K.shape[3]

    def proj(a, W, key):
        return gemv(a, W) if scales is None else gemv_fp8(a, W, scales[key])

    qkv = proj(rmsnorm(x, g1, eps), Wqkv, "qkv")
    q = qkv[:, : n_q_heads * D].reshape(B, n_q_heads, D).contiguous()
    attn = f4(q, K, V).reshape(B, n_q_heads * D)
    h = proj(attn, Wo, "o")
    hn = rmsnorm(h, g2, eps)
    ff = swiglu(proj(hn, Wu, "up"), proj(hn, Wg, "gate"))
    return proj(ff, Wd, "down")
