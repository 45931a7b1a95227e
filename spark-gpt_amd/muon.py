"""Drop-in momentum stage of spark-gpt's Muon optimizer -- the consumer of the
MLP's fp32 weight gradients -- on a gfx950 kernel.

Mirrors the reference's interface (N8python/spark-gpt train.py):

* ``_momentum_stage_supported(g, v, u, momentum)``   -- train.py:2820-2826
* ``_momentum_stage(g, v, u, momentum)``             -- train.py:2829-2839

v <- lerp(v, g, 1 - momentum) in place and u <- lerp(g, v, momentum) stored
in u's dtype (bf16: the Newton-Schulz staging stack), one HBM pass, bit for
bit the two-pass torch update the reference falls back to
(train.py:2990-2996).  The predicate adds what the kernel needs beyond the
reference's: a bf16 u and a length divisible by 4 (else the caller's torch
path runs, as for the reference's own unsupported cases).

``ops.wgrad_momentum`` fuses this stage into the FP8 weight gradient's split
reduction: the gradient goes from the registers into v and the staging
matrix without being written and read back.  It needs the optimizer state
at backward time and no gradient reduction or accumulation in between, so it
is an entry point for hosts that run backward and step together, not part of
the autograd Function.
"""
from __future__ import annotations

import torch

from . import ops


def _momentum_stage_supported(g, v, u, momentum: float) -> bool:
    """The reference's predicate plus what the kernel needs: a bf16 u, a
    length divisible by 4, one device, g and v 16-byte and u 8-byte aligned,
    and -0.5 < 1 - momentum (the kernel's fp32 weights).  Anything else takes
    the caller's torch path."""
    import numpy as np

    return (g.is_cuda and v.is_cuda and u.is_cuda and v.device == g.device and u.device == g.device
            and g.is_contiguous() and v.is_contiguous() and u.is_contiguous()
            and g.dtype == torch.float32 and v.dtype == torch.float32 and u.dtype == torch.bfloat16
            and g.numel() == v.numel() == u.numel() and g.numel() % 4 == 0
            and g.data_ptr() % 16 == 0 and v.data_ptr() % 16 == 0 and u.data_ptr() % 8 == 0
            and bool(-0.5 < np.float32(1.0 - momentum) < 0.5 <= np.float32(momentum)))


def _momentum_stage(g, v, u, momentum: float) -> None:
    """One fused pass: momentum buffer update + Nesterov update staged as bf16."""
    ops.momentum_stage(g.view(-1), v.view(-1), u.view(-1), momentum)
