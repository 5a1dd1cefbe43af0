"""CPU oracle for the FP8 MoE forward -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import
this package, and only as the checker or as the timed CPU baseline; the
product path (the package's ops/moe_layer) never calls it.

Modules
  numerics      e4m3/bf16 codecs from the OCP / IEEE definitions, the sigmoid
                evaluation shared with the GPU router.
  routing       no-aux-loss routing (reference/moe_ref.py:81-107), numpy.
  pack          the packed-weight permutation restated with reshape/transpose.
  moe_cpu       reference-semantics forward (moe_ref.py:5-136, fp32, torch CPU)
                and the kernel-semantics model (block-scaled fp32 accumulation,
                FP8 requant of the SwiGLU output as in kernels/moe.cu:468-541,
                652-685).

Pinning (what checks each part; see tests/):
  numerics  exhaustive against torch's CPU float8_e4m3fn / bfloat16 casts.
  routing   golden top-8 sets computed with the reference's own torch op
            sequence at all five configs; brute force over C(8,4) group
            choices on small T; constructed known-answer cases; weight-sum
            invariant.
  pack      byte-exact against the GPU pack and its inverse.
  moe_cpu   reference model: golden bf16 output of the real reference at
            config 0 (tests/golden, written by importing moe_ref.run here);
            one-hot block tests that fix every scale index; float64 closed
            forms.  Kernel model: agrees with the reference model to the
            FP8-requant error and reduces to it when C is exactly
            representable.
"""
