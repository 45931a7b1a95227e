"""Drop-in FP8 SwiGLU MLP sub-block for spark-gpt, on hand-written gfx950 kernels.

Mirrors the reference's interface for this path (N8python/spark-gpt train.py):

* ``FP8_MLP``, ``FP8_SITE_MAX``, ``FP8_HEADROOM_BINADES`` -- train.py:914-924
* ``_use_fp8_mlp(block, h)``                            -- train.py:927-934
* ``fp8_update_scales(model)``                          -- train.py:937-946
* ``MLP(dim, hidden_dim)`` (same parameter/buffer names) -- train.py:247-262
* ``_FP8MLPBlock.apply(h, norm_w, w_gu, w_down, scale, amax, eps)``
                                                        -- train.py:1193-1252

y = h + down(SwiGLU(gate_up(rmsnorm(h)))) with x, gu, h stored e4m3 and d_gu
(and the in-register dy of the down wgrad) e5m2, delayed per-tensor pow2
scales, fp32 master weights quantized just in time, fp32 weight/norm grads,
bf16 dh.  There is no CPU or eager-torch fallback: without the HIP library the
block raises.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from . import torch_ops  # noqa: F401  (registers the sparkfp8:: operators)

FP8_MLP = False  # set True to route dense MLP sub-blocks through _FP8MLPBlock while training

# slot map: 0 = x (normed MLP input, e4m3), 1 = gu (gate/up pre-activation, e4m3),
# 2 = h (SwiGLU output, e4m3), 3 = d_gu (its gradient, e5m2), 4 = dy (e5m2)
FP8_SITE_MAX = (448.0, 448.0, 448.0, 57344.0, 57344.0)
FP8_HEADROOM_BINADES = 1
MAX_HIDDEN = 4096  # largest hidden size the norm kernels tile (a whole row per wave)


def _use_fp8_mlp(block, h: torch.Tensor) -> bool:
    """Same predicate as the reference guard (train.py:927-934), with the
    Triton clause replaced by the HIP build and the norm kernels' hidden-size
    cap (128 <= D <= 4096)."""
    if not (FP8_MLP and block.training and not getattr(block, "is_sparse", False)
            and h.is_cuda and h.dtype == torch.bfloat16):
        return False  # checked first: sparse blocks' mlp has no down_proj
    d, inter = h.shape[1], block.mlp.down_proj.weight.shape[1]
    return d % 128 == 0 and d & (d - 1) == 0 and d <= MAX_HIDDEN and inter % 128 == 0


@torch.no_grad()
def fp8_update_scales(model: nn.Module) -> None:
    """Roll every fp8 block's recorded amax into next step's scales (device-side,
    no host sync).  Applies to every module carrying ``fp8_scale``/``fp8_amax``
    5-slot buffers (this module's ``MLP`` and the reference's MLP/Experts)."""
    for m in model.modules():
        scale = getattr(m, "fp8_scale", None)
        amax = getattr(m, "fp8_amax", None)
        if isinstance(scale, torch.Tensor) and isinstance(amax, torch.Tensor) and scale.numel() == 5:
            ops.update_scales(scale, amax)


class MLP(nn.Module):
    """Same parameters and buffers as the reference MLP (train.py:247-262)."""

    def __init__(self, dim: int, hidden_dim: int):
        super().__init__()
        self.gate_up_proj = nn.Linear(dim, 2 * hidden_dim, bias=False)
        self.down_proj = nn.Linear(hidden_dim, dim, bias=False)
        # fp8 state: per-rank, not checkpointed (train.py:251-254)
        self.register_buffer("fp8_scale", torch.ones(5), persistent=False)
        self.register_buffer("fp8_amax", torch.zeros(5), persistent=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * up)


class _FP8MLPBlock(torch.autograd.Function):
    """y = h + down(SwiGLU(gate_up(rmsnorm(h)))) with fp8 activations.

    Forward: norm_quant -> weight_quant x2 -> gate/up FP8 GEMM with SwiGLU
    epilogue -> down FP8 GEMM with residual epilogue.
    Backward: bf16 down dgrad with SwiGLU-backward epilogue (d_gu e5m2) ->
    gate/up FP8 dgrad -> RMSNorm backward (+ e5m2 dy^T) -> the two FP8 weight
    gradients reduced over tokens.

    The two halves run as the custom operators ``sparkfp8::block_fwd`` and
    ``sparkfp8::block_bwd`` (torch_ops.py), so a ``torch.compile``d model
    (train.py:3787) traces them as two opaque nodes."""

    @staticmethod
    def forward(ctx, h, norm_w, w_gu, w_down, scale, amax, eps):
        y, wdt, x8t, rstd, w8t, wscale, gu8, h8t = torch.ops.sparkfp8.block_fwd(
            h, norm_w, w_gu, w_down, scale, amax, eps)
        # backward needs the token-contiguous x8t / h8t (weight grads), gu8
        # (SwiGLU backward), W8^T (gate/up dgrad) and bf16 Wd^T (down dgrad)
        ctx.save_for_backward(h, norm_w, wdt, x8t, rstd, w8t, wscale, gu8, h8t, scale, amax)
        return y

    @staticmethod
    def backward(ctx, dy):
        h, norm_w, wdt, x8t, rstd, w8t, wscale, gu8, h8t, scale, amax = ctx.saved_tensors
        dh, dnw, dwgu, dwd = torch.ops.sparkfp8.block_bwd(dy, h, norm_w, wdt, x8t, rstd, w8t, wscale, gu8, h8t,
                                                          scale, amax)
        return dh, dnw, dwgu, dwd, None, None, None


def fp8_mlp_block(h: torch.Tensor, norm: nn.Module, mlp: MLP) -> torch.Tensor:
    """h + mlp(norm(h)) through _FP8MLPBlock, as Block.forward calls it
    (train.py:2359-2365)."""
    return _FP8MLPBlock.apply(h, norm.weight, mlp.gate_up_proj.weight, mlp.down_proj.weight,
                              mlp.fp8_scale, mlp.fp8_amax, norm.eps)
