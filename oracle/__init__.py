"""CPU oracle for one GPT-OSS-120B-shaped (and DeepSeek-V3-shaped) MoE pipeline-stage step.

TEST INFRASTRUCTURE ONLY.  This package is the test oracle, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  Nothing under ``flyai_amd/`` imports it, and the product path has no CPU fallback.

It restates, on the CPU, the arithmetic the reference's stage step performs.  The GPT-OSS math
lives in the third-party ``transformers`` package that the reference pins
(``phase0/requirements_vmoe.txt:178``: transformers 5.12.1; this container has 5.15.0) and in the
HF-hub ``triton_kernels`` package (not installed, never fetched).  Every function cites the file
and line it follows.  Integer/index work (packing, top-k indices, histogram, permutation) is
restated with numpy and is bit-exact by definition; floating-point work is fp32 torch on the CPU.

Modules
  numerics   bf16 rounding helpers
  mxfp4      E2M1/E8M0 block format (row a5)
  packing    ragged batch packing (row a1)
  routing    router top-k, grouped sigmoid, histogram/permute, combine (rows a2-a4)
  experts    GPT-OSS SwiGLU experts on MXFP4, DeepSeek FP8 block-scaled experts (rows a6, a7)
  attention  ragged GQA attention with sinks and sliding window (row a8)
  layer      RMSNorm, linear, yarn RoPE, decoder layer and stage step (rows a9, a10)

Parity status of each function (how it is pinned) is listed in the module docstrings and in the
tests under tests/test_oracle_*.py.
"""
