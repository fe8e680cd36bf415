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
  and scale 1/sqrt(128) (config 4), and the Llama-3-8B-shaped decode layer
  (config 5: RMSNorm -> QKV -> attention -> O -> RMSNorm -> gate/up SwiGLU ->
  down).  ``dtype="fp8"`` stores the projection weights as OCP e4m3 with
  one fp32 scale per output row.  It returns a :class:`Case` that also
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
CONFIG_NAMES = ("f1", "f1_qkv", "f2", "f4", "layer")
DTYPES = ("f16", "fp8")
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


def _qk(q, K):
    """fp16 q.K^T per KV head: [B,Hkv,L,G] (the right operand, q, is the
    small contiguous one)."""
    import torch

    B, Hq, D = q.shape
    Hkv = K.shape[1]
    qt = q.reshape(B, Hkv, Hq // Hkv, D).transpose(-1, -2).contiguous()
    return torch.matmul(K, qt)


def _scores_f32(qk, scale: float):
    """[B,Hkv,L,G] fp16 -> scaled fp32 scores [B,Hq,L], contiguous, made by
    one conversion kernel (plus an in-place scale)."""
    import torch

    B, Hkv, L, G = qk.shape
    if G == 1:
        out = qk.reshape(B, Hkv, L).float()
    else:
        out = qk.transpose(-1, -2).to(torch.float32, memory_format=torch.contiguous_format)
    if scale != 1.0:
        out.mul_(scale)
    return out.view(B, Hkv * G, L)


def _weighted_v(p16, V):
    import torch

    B, Hq, L = p16.shape
    Hkv = V.shape[1]
    return torch.matmul(p16.view(B, Hkv, Hq // Hkv, L), V).view(B, Hq, V.shape[3])


def f4_sequence(scale: float = 1.0, split_stages: bool = False) -> Sequence:
    """scores -> softmax -> weighted_v with grouped query heads.

    q [B,Hq,D], K/V [B,Hkv,L,D]; query head h reads KV head h // (Hq/Hkv).
    With ``split_stages`` every intermediate is a declared stage output, so
    the byte model sees all of them and no stage allocates a temporary:
    qk (fp16 q.K^T) -> scores (fp32, scaled) -> softmax -> probs16 (the fp16
    probabilities P.V reads) -> weighted_v.  Without it the three stages
    keep the reference demo's shape (llama_decode.py:120-134)."""
    import torch

    seq = Sequence("f4")

    if split_stages:
        @seq.stage
        def qk(q, K):
            return _qk(q, K)

        @seq.stage
        def scores(qk):
            return _scores_f32(qk, scale)
    else:
        @seq.stage
        def scores(q, K):
            return _scores_f32(_qk(q, K), scale)

    @seq.stage
    def softmax(scores):
        return torch.softmax(scores, dim=-1)

    if split_stages:
        @seq.stage
        def probs16(softmax):
            return softmax.half()

        @seq.stage
        def weighted_v(probs16, V):
            return _weighted_v(probs16, V)
    else:
        @seq.stage
        def weighted_v(softmax, V):
            return _weighted_v(softmax.half(), V)

    return seq


def _linear_fp8(a, W, s):
    """The unfused e4m3 projection stage: the library's plain GEMV
    (``db_gemv``, one launch) on e4m3 weights with per-row scales, fp32
    accumulation, the row scale applied before the fp16 rounding -- the
    counterpart of the reference's unfused gemv kernel
    (validation/src/kernels/unfused/gemv.cu:15-48).  Its bytes are the
    weights and scales it reads: nothing is dequantised into memory."""
    from decodebench_amd import ops

    return ops.gemv(a, W, w_scale=s)


def f1_fp8_sequence(eps: float = 1e-6) -> Sequence:
    import torch

    seq = Sequence("f1_fp8")

    @seq.stage
    def rmsnorm(x, g):
        var = x.float().pow(2).mean(dim=-1, keepdim=True)
        return (x.float() * torch.rsqrt(var + eps)).half() * g

    @seq.stage
    def gemv(xh, W, s):
        return _linear_fp8(xh, W, s)

    return seq


def f2_fp8_sequence() -> Sequence:
    import torch

    seq = Sequence("f2_fp8")

    @seq.stage
    def gate(xh, Wg, sg):
        return _linear_fp8(xh, Wg, sg)

    @seq.stage
    def up(xh, Wu, su):
        return _linear_fp8(xh, Wu, su)

    @seq.stage
    def swiglu(up, gate):
        return torch.nn.functional.silu(gate) * up

    return seq


def layer_sequence(n_q_heads: int, scale: float, eps: float = 1e-6,
                   fp8: bool = False) -> Sequence:
    """The decode-layer chain as single-op stages: rmsnorm, QKV, the query
    heads of QKV (copied: a stage returns a tensor of its own), q.K^T, fp32
    scores, softmax, fp16 probabilities, weighted V, O projection, rmsnorm,
    gate, up, SwiGLU, down.  Torch ops, except that the e4m3 projections run
    on the library's plain GEMV (see :func:`_linear_fp8`).

    The new token's k and v columns of QKV are not appended to the cache:
    the chain measures the decode read path over a given KV cache."""
    import torch

    F = torch.nn.functional
    seq = Sequence("layer_fp8" if fp8 else "layer")

    def norm(x, g):
        var = x.float().pow(2).mean(dim=-1, keepdim=True)
        return (x.float() * torch.rsqrt(var + eps)).half() * g

    @seq.stage
    def rmsnorm1(x, g1):
        return norm(x, g1)

    if fp8:
        @seq.stage
        def qkv(rmsnorm1, Wqkv, s_qkv):
            return _linear_fp8(rmsnorm1, Wqkv, s_qkv)
    else:
        @seq.stage
        def qkv(rmsnorm1, Wqkv):
            return F.linear(rmsnorm1, Wqkv)

    @seq.stage
    def q_heads(qkv):
        B = qkv.shape[0]
        return qkv[:, : n_q_heads * _HEAD_DIM].reshape(B, n_q_heads, _HEAD_DIM).clone()

    @seq.stage
    def qk(q_heads, K):
        return _qk(q_heads, K)

    @seq.stage
    def scores(qk):
        return _scores_f32(qk, scale)

    @seq.stage
    def softmax(scores):
        return torch.softmax(scores, dim=-1)

    @seq.stage
    def probs16(softmax):
        return softmax.half()

    @seq.stage
    def weighted_v(probs16, V):
        B = probs16.shape[0]
        return _weighted_v(probs16, V).view(B, -1)

    if fp8:
        @seq.stage
        def o_proj(weighted_v, Wo, s_o):
            return _linear_fp8(weighted_v, Wo, s_o)
    else:
        @seq.stage
        def o_proj(weighted_v, Wo):
            return F.linear(weighted_v, Wo)

    @seq.stage
    def rmsnorm2(o_proj, g2):
        return norm(o_proj, g2)

    if fp8:
        @seq.stage
        def gate(rmsnorm2, Wg, s_gate):
            return _linear_fp8(rmsnorm2, Wg, s_gate)

        @seq.stage
        def up(rmsnorm2, Wu, s_up):
            return _linear_fp8(rmsnorm2, Wu, s_up)
    else:
        @seq.stage
        def gate(rmsnorm2, Wg):
            return F.linear(rmsnorm2, Wg)

        @seq.stage
        def up(rmsnorm2, Wu):
            return F.linear(rmsnorm2, Wu)

    @seq.stage
    def swiglu(up, gate):
        return F.silu(gate) * up

    if fp8:
        @seq.stage
        def down(swiglu, Wd, s_down):
            return _linear_fp8(swiglu, Wd, s_down)
    else:
        @seq.stage
        def down(swiglu, Wd):
            return F.linear(swiglu, Wd)

    return seq


def layer_fused(n_q_heads: int, scale: float, eps: float = 1e-6,
                n_splits: int | None = None) -> Callable[[dict], object]:
    """The decode layer on the HIP kernels: F1 (RMSNorm -> QKV), F4 (two
    launches), the O projection, RMSNorm -> gate/up SwiGLU in one kernel, and
    the down projection.  fp16 or e4m3 weights, as the inputs hold them."""
    from decodebench_amd import ops

    def run(inp):
        import torch

        fp8 = inp["Wqkv"].dtype != torch.float16
        sc = (lambda k: inp[k]) if fp8 else (lambda k: None)
        x = inp["x"]
        B = x.shape[0]
        qkv = ops.f1_rmsnorm_gemv(x, inp["g1"], inp["Wqkv"], eps, w_scale=sc("s_qkv"))
        q = qkv[:, : n_q_heads * _HEAD_DIM]
        q = (q if B == 1 else q.contiguous()).view(B, n_q_heads, _HEAD_DIM)
        attn = ops.f4_flashdecode(q, inp["K"], inp["V"], scale=scale, n_splits=n_splits)
        h = ops.gemv(attn.view(B, n_q_heads * _HEAD_DIM), inp["Wo"], w_scale=sc("s_o"))
        ff = ops.f2_rmsnorm_gateup_swiglu(h, inp["g2"], inp["Wg"], inp["Wu"], eps,
                                          sg=sc("s_gate"), su=sc("s_up"))
        return ops.gemv(ff, inp["Wd"], w_scale=sc("s_down"))

    return run


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


# Llama-3-8B layer shape of the decode chain.
LAYER = {"d": 4096, "Hq": 32, "Hkv": 8, "D": _HEAD_DIM, "F": 14336}


def _weight(gen, shape, std, device, fp8: bool):
    """An fp16 weight matrix, or its e4m3 quantisation and row scales."""
    W = _randn(gen, shape, std=std, device=device)
    if not fp8:
        return W, None
    from decodebench_amd.quant import quantize_e4m3_rows

    return quantize_e4m3_rows(W)


def build_config(name: str, batch: int = 1, L: int = 8192, n_splits: int | None = None,
                 seed: int = 42, device="cuda", replicas: int | None = None,
                 K: int = 4096, gen_device: str = "cpu", dtype: str = "f16") -> Case:
    """A case at the benchmark's shapes (configs 1-5); ``replicas=None`` sizes a cache-defeating rotation.

    ``gen_device="cpu"`` draws the inputs on the CPU (device-independent
    values, what the parity tests use); ``"cuda"`` draws them on the GPU.
    ``dtype="fp8"`` (F1, F1-QKV, F2 and the layer) quantises the projection
    weights to e4m3 with per-row scales; algorithmic bytes then count one
    byte per weight plus four per row scale."""
    import torch

    from decodebench_amd import ops

    if dtype not in DTYPES:
        raise ValueError(f"unknown dtype '{dtype}'; choose from {list(DTYPES)}")
    fp8 = dtype == "fp8"
    if fp8 and name == "f4":
        raise ValueError("f4 has no weights; dtype='fp8' applies to f1, f1_qkv, f2, layer")
    wb = 1 if fp8 else 2            # bytes per weight
    sb = 4 if fp8 else 0            # bytes of row scale per output row
    gen = torch.Generator(device=gen_device).manual_seed(seed)
    B = batch
    if name in ("f1", "f1_qkv"):
        N = 4096 if name == "f1" else 6144
        w_std = 1.0 / 64.0 if name == "f1" else 0.02
        x = _randn(gen, (B, K), device=device)
        g = _randn(gen, (K,), std=0.1, mean=1.0, device=device)
        W, s = _weight(gen, (N, K), w_std, device, fp8)
        if fp8:
            inputs = {"x": x, "g": g, "W": W, "s": s}
            seq = f1_fp8_sequence(1e-6)
            fused = lambda inp: ops.f1_rmsnorm_gemv(inp["x"], inp["g"], inp["W"], 1e-6,  # noqa: E731
                                                    w_scale=inp["s"])
        else:
            inputs = {"x": x, "g": g, "W": W}
            seq = f1_sequence(1e-6)
            fused = lambda inp: ops.f1_rmsnorm_gemv(inp["x"], inp["g"], inp["W"], 1e-6)  # noqa: E731
        big = ("W",)
        nbytes = N * K * wb + N * sb + K * 2 + B * (K + N) * 2
        flops = 2 * B * N * K
        shape = {"B": B, "K": K, "N": N, "dtype": dtype}
    elif name == "f2":
        N = 14336
        x = _randn(gen, (B, K), device=device)
        Wg, sg = _weight(gen, (N, K), 0.02, device, fp8)
        Wu, su = _weight(gen, (N, K), 0.02, device, fp8)
        if fp8:
            inputs = {"xh": x, "Wg": Wg, "Wu": Wu, "sg": sg, "su": su}
            seq = f2_fp8_sequence()
            fused = lambda inp: ops.f2_gateup_swiglu(inp["xh"], inp["Wg"], inp["Wu"],  # noqa: E731
                                                     inp["sg"], inp["su"])
        else:
            inputs = {"xh": x, "Wg": Wg, "Wu": Wu}
            seq = f2_sequence()
            fused = lambda inp: ops.f2_gateup_swiglu(inp["xh"], inp["Wg"], inp["Wu"])  # noqa: E731
        big = ("Wg", "Wu")
        nbytes = 2 * N * K * wb + 2 * N * sb + B * (K + N) * 2
        flops = 4 * B * N * K
        shape = {"B": B, "K": K, "N": N, "dtype": dtype}
    elif name == "layer":
        d, Hq, Hkv, D, F = (LAYER[k] for k in ("d", "Hq", "Hkv", "D", "F"))
        Nqkv = (Hq + 2 * Hkv) * D
        x = _randn(gen, (B, d), device=device)
        g1 = _randn(gen, (d,), std=0.1, mean=1.0, device=device)
        g2 = _randn(gen, (d,), std=0.1, mean=1.0, device=device)
        Wqkv, s_qkv = _weight(gen, (Nqkv, d), 0.02, device, fp8)
        Kc = _randn(gen, (B, Hkv, L, D), device=device)
        Vc = _randn(gen, (B, Hkv, L, D), device=device)
        Wo, s_o = _weight(gen, (d, Hq * D), 0.02, device, fp8)
        Wg, s_gate = _weight(gen, (F, d), 0.02, device, fp8)
        Wu, s_up = _weight(gen, (F, d), 0.02, device, fp8)
        Wd, s_down = _weight(gen, (d, F), 0.02, device, fp8)
        inputs = {"x": x, "g1": g1, "Wqkv": Wqkv, "K": Kc, "V": Vc, "Wo": Wo, "g2": g2,
                  "Wg": Wg, "Wu": Wu, "Wd": Wd, "s_qkv": s_qkv, "s_o": s_o,
                  "s_gate": s_gate, "s_up": s_up, "s_down": s_down}
        if not fp8:  # the fp16 stages take no scales
            inputs = {k: v for k, v in inputs.items() if not k.startswith("s_")}
        scale = 1.0 / math.sqrt(D)
        seq = layer_sequence(Hq, scale, 1e-6, fp8)
        fused = layer_fused(Hq, scale, 1e-6, n_splits)
        big = ("Wqkv", "K", "V", "Wo", "Wg", "Wu", "Wd")
        rows = Nqkv + d + 2 * F + d
        wbytes = (Nqkv * d + d * Hq * D + 2 * F * d + d * F) * wb + rows * sb
        nbytes = wbytes + 2 * B * Hkv * L * D * 2 + 2 * d * 2 + 2 * B * d * 2
        flops = 2 * B * (Nqkv * d + d * Hq * D + 2 * F * d + d * F) + 4 * B * Hq * L * D
        shape = {"B": B, "d": d, "Hq": Hq, "Hkv": Hkv, "L": L, "D": D, "F": F,
                 "S": n_splits, "dtype": dtype}
    elif name == "f4":
        Hq, Hkv, D = 32, 8, _HEAD_DIM
        q = _randn(gen, (B, Hq, D), device=device)
        Kc = _randn(gen, (B, Hkv, L, D), device=device)
        Vc = _randn(gen, (B, Hkv, L, D), device=device)
        inputs = {"q": q, "K": Kc, "V": Vc}
        scale = 1.0 / math.sqrt(D)
        seq = f4_sequence(scale, split_stages=True)
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
