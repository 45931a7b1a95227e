"""Drop-in bf16 SwiGLU MLP path of spark-gpt (its default, non-FP8 path), on
hand-written gfx950 kernels.

Mirrors the reference's interface for this path (N8python/spark-gpt train.py):

* ``FUSED_SWIGLU``, ``FUSED_NORM_MLP``                    -- train.py:1618, 2093
* ``_use_fused_swiglu(x)``                                 -- train.py:1621-1622
* ``_use_fused_norm_mlp(block, h)``                        -- train.py:2096-2098
  (``make_fused_swiglu_guard`` / ``make_fused_norm_mlp_guard`` build them over
  a trainer's own flags)
* ``_FusedSwiGLU.apply(x, weight, offs) -> h``             -- train.py:2067-2090
* ``_NormSwiGLU.apply(h, norm_w, w_gu, eps) -> out``       -- train.py:2101-2131

Same numerics and rounding points as the reference: gate/up accumulated in
fp32, rounded to bf16 (after the row scale rstd with the folded norm), SwiGLU
in fp32 from the rounded values, bf16 out; the backward's d_gate / d_up
rounded to bf16 before both GEMMs, the dgrad and the weight gradient rounded
to bf16.  The SwiGLU gradient is computed once, by one row kernel, where the
reference recomputes it in the prologue of each of its two GEMMs.  Grouped
rows (``offs`` with several experts) are laid out per expert from 256-row
boundaries on the device (no host sync), as for the FP8 experts.

Shapes: D % 64 == 0 and I % 64 == 0 (the reference's Triton kernels mask any
shape; every spark-gpt width qualifies).  The guards check D; I is checked
when the operator runs.
"""
from __future__ import annotations

import torch

from . import torch_ops  # noqa: F401  (registers the sparkfp8:: bf16 operators)

FUSED_SWIGLU = True  # --no-fused-swiglu (train.py:1618)
FUSED_NORM_MLP = True  # --no-fused-norm-mlp (train.py:2093)


def make_fused_swiglu_guard(flag):
    """The guard of train.py:1621-1622 over a flag read at call time: fused
    when the flag is set and x is a 2-D CUDA bf16 tensor whose width is a
    multiple of 64 (the Triton clause becomes "the HIP library is built")."""

    def _use_fused_swiglu(x: torch.Tensor) -> bool:
        return bool(flag()) and x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.shape[-1] % 64 == 0

    return _use_fused_swiglu


def make_fused_norm_mlp_guard(flag, use_fused_swiglu):
    """The guard of train.py:2096-2098: the norm-folded path for a dense block
    (sparse blocks are checked first: their mlp has no gate_up_proj)."""

    def _use_fused_norm_mlp(block, h: torch.Tensor) -> bool:
        if not (flag() and not block.is_sparse and use_fused_swiglu(h) and h.dim() == 2):
            return False
        return block.mlp.gate_up_proj.weight.shape[0] % 128 == 0

    return _use_fused_norm_mlp


# the package's own switches
_use_fused_swiglu = make_fused_swiglu_guard(lambda: FUSED_SWIGLU)
_use_fused_norm_mlp = make_fused_norm_mlp_guard(lambda: FUSED_NORM_MLP, _use_fused_swiglu)


class _FusedSwiGLU(torch.autograd.Function):
    """h = silu(x W_gate^T) * (x W_up^T) per group of rows (train.py:2067-2090).

    x [R, D] bf16 with rows sorted by group; weight [E, 2I, D] bf16 (gate rows
    first); offs [E] int32 inclusive row-count prefix sums.  Forward: the
    grouped gate/up GEMM with the SwiGLU epilogue (saves gu [R, 2I]).
    Backward: the bf16 SwiGLU gradient of the rows, then dx = G' W (bf16) and
    dW = G'^T x (bf16 [E, 2I, D]).  Both halves are the custom operators
    ``sparkfp8::swiglu_fwd`` / ``swiglu_bwd``."""

    @staticmethod
    def forward(ctx, x, weight, offs):
        h, gu, plan = torch.ops.sparkfp8.swiglu_fwd(x, weight, offs)
        ctx.save_for_backward(x, weight, gu, plan)
        return h

    @staticmethod
    def backward(ctx, dh):
        x, weight, gu, plan = ctx.saved_tensors
        dx, dw = torch.ops.sparkfp8.swiglu_bwd(dh, x, weight, gu, plan)
        return dx, dw, None


class _NormSwiGLU(torch.autograd.Function):
    """SwiGLU(gate_up(rmsnorm(h))) of a dense MLP (train.py:2101-2131), the
    norm weight folded into the gate/up weight (W' = bf16(w_gu * norm_w)) and
    the rows normalised in the GEMM epilogue (rstd from a row pass; the weight
    gradient reads h and G' through transposing LDS reads).

    Returns out [T, I] bf16 (the down projection and the residual stay the
    caller's, train.py:2366-2369).  Backward: (dh bf16, dnorm_w fp32 [D],
    dw_gu fp32 [2I, D], None), the norm backward a row kernel.  Both halves
    are the custom operators ``sparkfp8::norm_swiglu_fwd`` / ``_bwd``."""

    @staticmethod
    def forward(ctx, h, norm_w, w_gu, eps):
        out, wt, gu, rstd = torch.ops.sparkfp8.norm_swiglu_fwd(h, norm_w, w_gu, float(eps))
        ctx.save_for_backward(h, norm_w, w_gu, wt, gu, rstd)
        return out

    @staticmethod
    def backward(ctx, dout):
        h, norm_w, w_gu, wt, gu, rstd = ctx.saved_tensors
        dh, dnw, dw = torch.ops.sparkfp8.norm_swiglu_bwd(dout, h, norm_w, w_gu, wt, gu, rstd)
        return dh, dnw, dw, None
