"""CPU oracle for the FP8 SwiGLU MLP path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg
of ``bench.py`` use it, and only to check results (or as the timed CPU baseline),
never as the thing being measured on the GPU.

``fp8_mlp`` restates the reference recipe (spark-gpt ``train.py:911-1253``) in
plain torch-CPU fp32 arithmetic with the reference's rounding points.
``fp8_bits`` is an independent closed-form (integer, numpy) restatement of the
OCP e4m3fn / e5m2 round-to-nearest-even casts and of the power-of-two scale
rule, used to pin the torch casts the oracle relies on.
"""
