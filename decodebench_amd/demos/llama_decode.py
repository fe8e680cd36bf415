"""Llama decode-chain demos: F1 (RMSNorm+GEMV), F2 (gate/up+SwiGLU), F4 (attention).

Two builders:

* ``build_demo(name, dim=4096, batch=1)`` keeps the reference's demo API
  (src/decodebench/demos/llama_decode.py:155-161): it returns
  ``(seq, inputs, replicas)`` for the reference's shapes -- F1 with a square
  ``W[dim, dim]``, F2 with the reference's FFN width (11008 at dim 4096), F4
  as multi-head attention with ``dim/128`` heads, L = 1024 and no score scale
  -- so existing callers switch over unchanged.
* ``build_config(name, batch=1, ...)`` builds the MI355X benchmark
  configurations: F1 ``W[4096,4096]`` (config 1), F1-QKV ``W[6144,4096]``
  (config 3), F2 ``[14336,4096]`` (config 2), F4 with 32 query / 8 KV heads
  and scale 1/sqrt(128) (config 4).  It returns a :class:`Case` that also
  carries the fused HIP callable, the algorithmic bytes and a replica list
  sized to defeat the whole cache hierarchy (8 L2s + the 256 MB MALL).

Inputs are generated on the CPU from ``torch.Generator().manual_seed(seed)``
in fp32, cast to fp16 and copied to the device, so they are identical on every
machine (the reference demos draw unseeded GPU randoms).

The unfused stages are the reference's stage bodies
(llama_decode.py:36-43, 77-87, 120-134) in torch; attention gains grouped
query heads and the optional scale.  Products keep contiguous right operands.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable

from decodebench_amd.sequence import Sequence
from decodebench_amd.timing import cache_defeat_replicas, n_weight_replicas

DEMO_NAMES = ("f1", "f2", "f4")
CONFIG_NAMES = ("f1", "f1_qkv", "f2", "f4")
_FFN = {2048: 8192, 4096: 11008}
_L = 1024
_HEAD_DIM = 128


# ----------------------------------------------------------- random inputs
def _randn(gen, shape, std: float = 1.0, mean: float = 0.0, device="cuda"):
    """Seeded normal fp16 tensor on ``device``.  Drawn on the generator's own
    device: a CPU generator gives values identical on every machine, a GPU
    generator is fast for the large KV caches of benchmark sweeps."""
    import torch

    t = torch.randn(*shape, generator=gen, dtype=torch.float32, device=gen.device)
    if std != 1.0:
        t.mul_(std)
    if mean != 0.0:
        t.add_(mean)
    return t.half().to(device)


# -------------------------------------------------------------- the stages
def f1_sequence(eps: float = 1e-6) -> Sequence:
    import torch

    seq = Sequence("f1")

    @seq.stage
    def rmsnorm(x, g):
        var = x.float().pow(2).mean(dim=-1, keepdim=True)
        return (x.float() * torch.rsqrt(var + eps)).half() * g

    @seq.stage
    def gemv(xh, W):
        return torch.nn.functional.linear(xh, W)

    return seq


def f2_sequence() -> Sequence:
    import torch

    seq = Sequence("f2")

    @seq.stage
    def gate(xh, Wg):
        return torch.nn.functional.linear(xh, Wg)

    @seq.stage
    def up(xh, Wu):
        return torch.nn.functional.linear(xh, Wu)

    @seq.stage
    def swiglu(up, gate):
        return torch.nn.functional.silu(gate) * up

    return seq


def f4_sequence(scale: float = 1.0) -> Sequence:
    """scores -> softmax -> weighted_v with grouped query heads.

    q [B,Hq,D], K/V [B,Hkv,L,D]; query head h reads KV head h // (Hq/Hkv)."""
    import torch

    seq = Sequence("f4")

    @seq.stage
    def scores(q, K):
        B, Hq, D = q.shape
        Hkv = K.shape[1]
        qt = q.reshape(B, Hkv, Hq // Hkv, D).transpose(-1, -2).contiguous()
        s = torch.matmul(K, qt)                        # fp16 [B,Hkv,L,G]
        return s.transpose(-1, -2).float().mul(scale).reshape(B, Hq, K.shape[2])

    @seq.stage
    def softmax(s):
        return torch.softmax(s, dim=-1)

    @seq.stage
    def weighted_v(p, V):
        B, Hq, L = p.shape
        Hkv = V.shape[1]
        pg = p.half().reshape(B, Hkv, Hq // Hkv, L)
        return torch.matmul(pg, V).reshape(B, Hq, V.shape[3])

    return seq


# --------------------------------------------------- reference-shaped demos
def _build_f1(dim: int, batch: int, seed: int):
    import torch

    gen = torch.Generator().manual_seed(seed)
    x = _randn(gen, (batch, dim))
    g = _randn(gen, (dim,))
    W = _randn(gen, (dim, dim))
    inputs = {"x": x, "g": g, "W": W}
    reps = [{"x": x, "g": g, "W": W.clone()} for _ in range(n_weight_replicas(W.nbytes))]
    return f1_sequence(), inputs, reps


def _build_f2(dim: int, batch: int, seed: int):
    import torch

    ff = _FFN[dim]
    gen = torch.Generator().manual_seed(seed)
    xh = _randn(gen, (batch, dim))
    Wg = _randn(gen, (ff, dim))
    Wu = _randn(gen, (ff, dim))
    inputs = {"xh": xh, "Wg": Wg, "Wu": Wu}
    n = n_weight_replicas(Wg.nbytes + Wu.nbytes)
    reps = [{"xh": xh, "Wg": Wg.clone(), "Wu": Wu.clone()} for _ in range(n)]
    return f2_sequence(), inputs, reps


def _build_f4(dim: int, batch: int, seed: int):
    import torch

    H = dim // _HEAD_DIM
    gen = torch.Generator().manual_seed(seed)
    q = _randn(gen, (batch, H, _HEAD_DIM))
    K = _randn(gen, (batch, H, _L, _HEAD_DIM))
    V = _randn(gen, (batch, H, _L, _HEAD_DIM))
    inputs = {"q": q, "K": K, "V": V}
    n = n_weight_replicas(K.nbytes + V.nbytes)
    reps = [{"q": q, "K": K.clone(), "V": V.clone()} for _ in range(n)]
    return f4_sequence(scale=1.0), inputs, reps


_BUILDERS = {"f1": _build_f1, "f2": _build_f2, "f4": _build_f4}


def build_demo(name: str, dim: int = 4096, batch: int = 1, seed: int = 42):
    """Build a named fusion demo. Returns ``(seq, inputs, input_replicas)``."""
    if name not in _BUILDERS:
        raise ValueError(f"unknown demo '{name}'; choose from {list(_BUILDERS)}")
    return _BUILDERS[name](dim, batch, seed)


def demo_fused(name: str) -> Callable[[dict], object]:
    """The HIP fused callable matching ``build_demo(name)``'s inputs."""
    from decodebench_amd import ops

    if name == "f1":
        return lambda inp: ops.f1_rmsnorm_gemv(inp["x"], inp["g"], inp["W"], 1e-6)
    if name == "f2":
        return lambda inp: ops.f2_gateup_swiglu(inp["xh"], inp["Wg"], inp["Wu"])
    if name == "f4":
        return lambda inp: ops.f4_flashdecode(inp["q"], inp["K"], inp["V"], scale=1.0)
    raise ValueError(f"unknown demo '{name}'; choose from {list(_BUILDERS)}")


# ------------------------------------------------------ benchmark configs
@dataclass
class Case:
    name: str
    seq: Sequence
    inputs: dict
    fused: Callable[[dict], object]
    big: tuple[str, ...]          # keys of the streamed operands
    algorithmic_bytes: int        # bytes a perfect fused kernel moves
    flops: int
    shape: dict = field(default_factory=dict)
    replicas: list[dict] = field(default_factory=list)


def _replicate(inputs: dict, big: tuple[str, ...], n: int) -> list[dict]:
    reps = [inputs]
    for _ in range(n - 1):
        reps.append({k: (v.clone() if k in big else v) for k, v in inputs.items()})
    return reps


def build_config(name: str, batch: int = 1, L: int = 8192, n_splits: int | None = None,
                 seed: int = 42, device="cuda", replicas: int | None = None,
                 K: int = 4096, gen_device: str = "cpu") -> Case:
    """BASELINE-shaped case; ``replicas=None`` sizes a cache-defeating rotation.

    ``gen_device="cpu"`` draws the inputs on the CPU (device-independent
    values, what the parity tests use); ``"cuda"`` draws them on the GPU."""
    import torch

    from decodebench_amd import ops

    gen = torch.Generator(device=gen_device).manual_seed(seed)
    B = batch
    if name in ("f1", "f1_qkv"):
        N = 4096 if name == "f1" else 6144
        w_std = 1.0 / 64.0 if name == "f1" else 0.02
        x = _randn(gen, (B, K), device=device)
        g = _randn(gen, (K,), std=0.1, mean=1.0, device=device)
        W = _randn(gen, (N, K), std=w_std, device=device)
        inputs = {"x": x, "g": g, "W": W}
        seq = f1_sequence(1e-6)
        fused = lambda inp: ops.f1_rmsnorm_gemv(inp["x"], inp["g"], inp["W"], 1e-6)  # noqa: E731
        big = ("W",)
        nbytes = N * K * 2 + K * 2 + B * (K + N) * 2
        flops = 2 * B * N * K
        shape = {"B": B, "K": K, "N": N}
    elif name == "f2":
        N = 14336
        x = _randn(gen, (B, K), device=device)
        Wg = _randn(gen, (N, K), std=0.02, device=device)
        Wu = _randn(gen, (N, K), std=0.02, device=device)
        inputs = {"xh": x, "Wg": Wg, "Wu": Wu}
        seq = f2_sequence()
        fused = lambda inp: ops.f2_gateup_swiglu(inp["xh"], inp["Wg"], inp["Wu"])  # noqa: E731
        big = ("Wg", "Wu")
        nbytes = 2 * N * K * 2 + B * (K + N) * 2
        flops = 4 * B * N * K
        shape = {"B": B, "K": K, "N": N}
    elif name == "f4":
        Hq, Hkv, D = 32, 8, _HEAD_DIM
        q = _randn(gen, (B, Hq, D), device=device)
        Kc = _randn(gen, (B, Hkv, L, D), device=device)
        Vc = _randn(gen, (B, Hkv, L, D), device=device)
        inputs = {"q": q, "K": Kc, "V": Vc}
        scale = 1.0 / math.sqrt(D)
        seq = f4_sequence(scale)
        fused = lambda inp: ops.f4_flashdecode(inp["q"], inp["K"], inp["V"], scale=scale,  # noqa: E731
                                               n_splits=n_splits)
        big = ("K", "V")
        nbytes = 2 * B * Hkv * L * D * 2 + 2 * B * Hq * D * 2
        flops = 4 * B * Hq * L * D
        shape = {"B": B, "Hq": Hq, "Hkv": Hkv, "L": L, "D": D, "S": n_splits}
    else:
        raise ValueError(f"unknown config '{name}'; choose from {list(CONFIG_NAMES)}")
    big_bytes = sum(inputs[k].nbytes for k in big)
    n = cache_defeat_replicas(big_bytes) if replicas is None else max(1, replicas)
    return Case(name, seq, inputs, fused, big, nbytes, flops, shape,
                _replicate(inputs, big, n))
