"""CPU oracle for the quantized-GEMM path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with numpy (bit-level format work) and
fp32/fp64 matmuls, what the reference computes on its quantized GEMM path:

* formats.py -- E4M3 / E2M1 / E8M0 encode and decode, bf16 rounding.
* quant.py   -- the quantize/pack contract (per-tensor, block-wise FP8,
                MXFP4, NVFP4) that the HIP kernels must match bit for bit.
* gemm.py    -- dequantize -> fp32 matmul references, the reference's tiled
                CPU path restated, the grouped (MoE) reference, and the
                exact-sum bf16 GEMM reference.
* fused.py   -- the bf16 values the fused quantize producers encode
                (RMSNorm, SwiGLU).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
timed CPU baseline.  The product path (``dsl_tool_amd``) never imports it and
fails loudly when its HIP library is missing.

Pinning (each function's docstring names its pins; the tests under
``tests/test_oracle.py`` enforce them):

* E4M3 encode  -- torch's ``Tensor.to(float8_e4m3fn)`` (an independent
  library routine) over every bf16 bit pattern and a dense fp32 sweep, plus
  the OCP 8-bit FP spec's special values.
* E2M1 encode  -- exhaustive brute force over all 65 536 bf16 patterns
  against a nearest-value search with the OCP tie rule, and a committed
  golden table (``tests/golden/e2m1_bf16.npy``).
* E8M0 encode  -- ``math.frexp`` over every positive finite bf16 value.
* quantizers   -- closed forms (power-of-two invariance, amax element maps to
  +-448 / +-6, zero blocks), brute-force loops on tiny inputs.
* GEMMs        -- float64 brute-force triple loops on tiny shapes, and the
  identity ``sum_g s_a s_b sum_{k in g} a b == (a*s_a) @ (b*s_b)``.
"""
