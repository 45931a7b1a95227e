"""Drop-in FP8 MoE experts for spark-gpt, on the same gfx950 kernels as the block.

Mirrors the reference's interface for this path (N8python/spark-gpt train.py):

* ``_use_fp8_moe(experts, x)``                              -- train.py:1258-1263
  (``make_fp8_moe_guard(flag)`` builds it over a trainer's own flag)
* ``_FP8Experts.apply(x, w_gu, w_d, token_index, inverse_permutation, offsets,
  top_k, scale, amax)``                                     -- train.py:1543-1605

The grouped twin of ``_FP8MLPBlock``: the expert-order gather of x is fused
with its e4m3 quantization, gu and h are stored e4m3 and d_gu e5m2, the expert
weights get per-expert pow2 e4m3 copies (fp32 masters and grads), and the
result is the unweighted bf16 rows in expert order (the router-weighted top-k
combine stays the caller's).  Rows are laid out per expert from 256-row
boundaries on the device (no host sync); the weight gradients are
deterministic (split partials summed in order, where the reference uses fp32
atomics, train.py:1527).
"""
from __future__ import annotations

import torch

from . import mlp as _mlp
from . import torch_ops  # the sparkfp8::moe_fwd / moe_bwd operators and their implementations


def make_fp8_moe_guard(flag):
    """The guard of train.py:1258-1263 over a flag read at call time (see
    ``make_fp8_mlp_guard``)."""

    def _use_fp8_moe(experts, x: torch.Tensor) -> bool:
        if not (flag() and experts.training and x.is_cuda and x.dtype == torch.bfloat16):
            return False
        d, inter = experts.hidden_dim, experts.intermediate_dim
        return d % 128 == 0 and d & (d - 1) == 0 and inter % 128 == 0

    return _use_fp8_moe


# the package's own switch (spark_gpt_amd.set_fp8_mlp)
_use_fp8_moe = make_fp8_moe_guard(lambda: _mlp.FP8_MLP)


class _FP8Experts(torch.autograd.Function):
    """Grouped expert SwiGLU MLP with fp8 storage (train.py:1543-1605).

    Forward: gather + e4m3 quantization of x -> grouped gate/up FP8 GEMM with
    the SwiGLU epilogue -> grouped down FP8 GEMM; returns [R, D] bf16 rows in
    expert order.  Backward: e5m2 copy of the upstream gradient -> grouped
    bf16 down dgrad with the SwiGLU backward epilogue -> grouped gate/up FP8
    dgrad -> the two grouped FP8 weight gradients -> the sum over each token's
    top_k rows.  Both halves are the custom operators ``sparkfp8::moe_fwd`` /
    ``sparkfp8::moe_bwd`` (opaque nodes under torch.compile)."""

    @staticmethod
    def forward(ctx, x, w_gu, w_d, token_index, inverse_permutation, offsets, top_k, scale, amax):
        out, plan, x8, gu8, h8 = torch_ops.op("moe_fwd")(x, w_gu, w_d, token_index, offsets, scale, amax)
        ctx.save_for_backward(w_gu, w_d, plan, x8, gu8, h8, inverse_permutation, scale, amax)
        ctx.shape = (x.shape[0], int(top_k))
        return out

    @staticmethod
    def backward(ctx, dout):
        w_gu, w_d, plan, x8, gu8, h8, inverse_permutation, scale, amax = ctx.saved_tensors
        T, top_k = ctx.shape
        dxn, dw_gu, dw_d = torch_ops.op("moe_bwd")(dout, w_gu, w_d, plan, x8, gu8, h8, inverse_permutation, T,
                                                      top_k, scale, amax)
        return dxn, dw_gu, dw_d, None, None, None, None, None, None
