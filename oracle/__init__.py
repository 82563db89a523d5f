"""CPU oracle of the quantized-weight GEMM hot path — TEST INFRASTRUCTURE ONLY.

This package is a plain numpy restatement of the reference's arithmetic for the
path (rdna2-ops/rdna2_ops/int8_gemm.py, comfy_int8.py, fp8_weight_gemm_v06.py,
int4_weight_gemm_v07.py; each function cites the lines it follows). It is used
only by ``tests/``, by ``__graft_entry__.smoke()`` as the checker and by
``bench.py``'s ``cpu_baseline`` leg. The product path (rdna2_ops,
librdna2_qgemm.so) never imports, calls or falls back to it.

How each function is pinned (see tests/test_oracle_*.py):
  int8.int8_matmul       brute-force int64 loops on tiny inputs, torch._int_mm,
                         closed forms (identity, all -128 rows, K=131071 bound).
  int8.epilogue_*        hand-computed values, torch CPU fp32 ops in the
                         reference's order, FMA emulation checked against
                         exact rational arithmetic.
  int8.quant_rows        exact ties (x/step = k + 1/2) for both rounding rules,
                         torch CPU division + round, zero rows, clamp.
  int8.gelu_tanh         torch CPU F.gelu(approximate="tanh") to <= 1 fp32 ulp class.
  convrot.*              Sylvester recursion and scipy.linalg.hadamard, H H^T = g I,
                         Parseval / involution / e_0 closed forms, the exact float64
                         rotation within the fp32 error bound, exact small-integer
                         cases, planted wrong variants, torch CPU fp32 in Kitchen's
                         order for the residual epilogue.
  int4.*, fp8.*          see their module headers.
"""
