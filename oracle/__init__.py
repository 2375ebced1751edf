"""CPU oracle for the int4 decode hot path — TEST INFRASTRUCTURE ONLY.

A plain numpy restatement of the reference's algorithms (each function cites the reference file:line it follows).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only as the checker or as
the timed CPU baseline; the product path (rumik-fast_amd/) never imports or calls anything here.

Modules:
  int4   pack/unpack, quantize (exporter maths), dequantize, int4 GEMV, int8 per-row GEMV, int4 prefill matmul
  glue   Cohere LayerNorm, interleaved RoPE, GQA decode attention, flash-decoding split/combine, SiLU*up,
         and one whole decode step

How each function is pinned (checked by tests/test_oracle.py against closed forms, brute force and invariants,
never against a retyped copy of itself) is listed in that test file's docstring. Parity status: every function
here is pinned; the reference holds no golden vectors for this path (its checks recompute references on the fly
from CUDA RNG inputs), so the pins are the closed-form known-answer tests.
"""
