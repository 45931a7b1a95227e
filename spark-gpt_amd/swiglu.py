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

Shapes: the kernels take D % 64 == 0 and I % 64 == 0 (every spark-gpt width
qualifies).  The reference's Triton kernels mask any shape, so other shapes
are not refused: the guards send them to the reference's unfused torch path
(MLP.forward's gate_up_proj -> F.silu(gate) * up, train.py:260-261), and
``_FusedSwiGLU`` / ``_NormSwiGLU`` called directly with such a shape run that
same torch path (with the reference's RMSNorm for ``_NormSwiGLU``,
train.py:166-168), with torch's autograd for the backward.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import torch_ops  # the sparkfp8:: bf16 operators and their implementations

FUSED_SWIGLU = True  # --no-fused-swiglu (train.py:1618)
FUSED_NORM_MLP = True  # --no-fused-norm-mlp (train.py:2093)


def _kernel_shape(D: int, I: int) -> bool:
    """Widths the HIP kernels take: D and I multiples of 64."""
    return D % 64 == 0 and I % 64 == 0


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
        w = block.mlp.gate_up_proj.weight
        return w.shape[0] % 2 == 0 and _kernel_shape(h.shape[-1], w.shape[0] // 2)

    return _use_fused_norm_mlp


# the package's own switches
_use_fused_swiglu = make_fused_swiglu_guard(lambda: FUSED_SWIGLU)
_use_fused_norm_mlp = make_fused_norm_mlp_guard(lambda: FUSED_NORM_MLP, _use_fused_swiglu)


def _unfused_swiglu(x, weight, offs):
    """The reference's unfused grouped SwiGLU (train.py:2313-2317 with the
    eager branch of _grouped_linear, 2181-2190): per group F.linear of its
    rows, chunk into gate and up, F.silu(gate) * up; rows past the last group
    are zero."""
    I = weight.shape[1] // 2
    parts, start = [], 0
    for e, end in enumerate(int(v) for v in offs.tolist()):
        if end > start:
            gate, up = F.linear(x[start:end], weight[e]).chunk(2, dim=-1)
            parts.append(F.silu(gate) * up)
            start = end
    if start < x.shape[0]:
        parts.append(x.new_zeros(x.shape[0] - start, I))
    return torch.cat(parts) if parts else x.new_zeros(0, I)


def _rmsnorm(x, weight, eps):
    """spark-gpt's RMSNorm (train.py:166-168): fp32 statistics, output in x's dtype."""
    out = x.float() * torch.rsqrt(x.float().pow(2).mean(dim=-1, keepdim=True) + eps)
    return out.to(dtype=x.dtype) * weight.to(dtype=x.dtype)


def _unfused_norm_swiglu(h, norm_w, w_gu, eps):
    """The reference's unfused dense path for the same sub-block: its RMSNorm
    module, then MLP.forward's torch branch (train.py:260-261)."""
    gate, up = F.linear(_rmsnorm(h, norm_w, eps), w_gu.to(h.dtype)).chunk(2, dim=-1)
    return F.silu(gate) * up


def _torch_forward(ctx, fn, *args):
    """Run `fn` (a torch path) on detached leaves with autograd on, keep its
    graph for the backward, return the detached output."""
    with torch.enable_grad():
        leaves = [a.detach().requires_grad_(a.is_floating_point()) if isinstance(a, torch.Tensor) else a
                  for a in args]
        out = fn(*leaves)
    ctx.torch_graph = (out, leaves)
    return out.detach()


def _torch_backward(ctx, dout, n_grads):
    out, leaves = ctx.torch_graph
    ctx.torch_graph = None
    wrt = [t for t in leaves[:n_grads]]
    grads = torch.autograd.grad(out, wrt, dout, allow_unused=True)
    return tuple(grads)


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
        ctx.torch_graph = None
        if not _kernel_shape(x.shape[-1], weight.shape[1] // 2) or weight.shape[1] % 2:
            return _torch_forward(ctx, _unfused_swiglu, x, weight, offs)
        h, gu, plan = torch_ops.op("swiglu_fwd")(x, weight, offs)
        ctx.save_for_backward(x, weight, gu, plan)
        return h

    @staticmethod
    def backward(ctx, dh):
        if ctx.torch_graph is not None:
            return _torch_backward(ctx, dh, 2) + (None,)
        x, weight, gu, plan = ctx.saved_tensors
        dx, dw = torch_ops.op("swiglu_bwd")(dh, x, weight, gu, plan)
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
        ctx.torch_graph = None
        if not _kernel_shape(h.shape[-1], w_gu.shape[0] // 2) or w_gu.shape[0] % 2:
            return _torch_forward(ctx, _unfused_norm_swiglu, h, norm_w, w_gu, eps)
        out, wt, gu, rstd = torch_ops.op("norm_swiglu_fwd")(h, norm_w, w_gu, float(eps))
        ctx.save_for_backward(h, norm_w, w_gu, wt, gu, rstd)
        return out

    @staticmethod
    def backward(ctx, dout):
        if ctx.torch_graph is not None:
            return _torch_backward(ctx, dout, 3) + (None,)
        h, norm_w, w_gu, wt, gu, rstd = ctx.saved_tensors
        dh, dnw, dw = torch_ops.op("norm_swiglu_bwd")(dout, h, norm_w, w_gu, wt, gu, rstd)
        return dh, dnw, dw, None
