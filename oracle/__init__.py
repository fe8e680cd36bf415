"""CPU oracle for the fused decode hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the CPU implementation being timed).  The product path
(``decodebench_amd``) never imports, links or calls anything here; it fails
loudly when its HIP library is missing instead of falling back to the CPU.

Contents
  stages.py  the reference's PyTorch stage definitions restated for CPU
             tensors (src/decodebench/demos/llama_decode.py:36-43, 77-87,
             120-134) with the benchmark's settings: eps 1e-6, scale 1/sqrt(D),
             grouped-query attention; plus the decode-layer chain.
  cref.c     plain-C restatement with double accumulation and explicit fp16
             rounding points; cref.py is its ctypes/numpy wrapper.
  Makefile   builds liboracle.so and, when /root/reference is present, the
             reference's own CPU reference into oracle/_ref/.

How each function is pinned (see tests/test_oracle_*.py):
  fp16 conversions     every fp16 value and every midpoint vs numpy.float16.
  orc_*_f32            known answers of validation/src/tests/test_reference.cpp
                       and the reference's compiled cpu_reference.cpp
                       (oracle/_ref) on random inputs.
  rmsnorm / gemv       closed forms, integer-exact small cases, fp64 numpy,
                       scale invariance; torch-stage restatement cross-checked.
  swiglu               closed form, silu(0)=0, silu(1), silu(2) known answers.
  attention (GQA)      test_reference.cpp known answer (unscaled MHA case),
                       GQA == MHA with K/V repeated per group, uniform scores
                       -> mean of V, L=1 -> the V row, softmax shift invariance,
                       split-KV with any S equal to S=1.
  fp8 e4m3             all 256 codes vs torch.float8_e4m3fn; dequantise-then-
                       GEMV equals GEMV-then-scale.
No oracle function is left "parity unpinned".
"""
