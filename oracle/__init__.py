"""CPU oracle for the MXFP4 mixture-of-experts step (test infrastructure only).

This package restates, on the CPU, the reference's MoE block of the Kimi K3
decode oracle (megabench/tasks/kimi.py:307-324), its MXFP4 decode
(megabench/tasks/quantization.py:40-51), the softmax-top-k / SiLU variant
(megabench/tasks/distributed.py:174-186) and the band grader
(megabench/tasks/kimi.py:413-429). It is the checker: only tests, the smoke
entry and the benchmark's CPU-baseline leg may import it. The product path
(the k3moe package) never imports, links or runs anything here.

Modules
  moe_ref   torch-CPU restatement of the op chain (BF16 oracle and FP32 truth)
  grading   band check, route validity, no-mutation snapshot
  cdecode   ctypes binding of mxfp4_ref.c, an independent C restatement of
            the E2M1/E8M0 decode, top-k selection and token grouping
"""
