"""Drop-in FP8 SwiGLU MLP sub-block for spark-gpt, on hand-written gfx950 kernels.

Mirrors the reference's interface for this path (N8python/spark-gpt train.py):

* ``FP8_MLP``, ``FP8_SITE_MAX``, ``FP8_HEADROOM_BINADES`` -- train.py:914-924
* ``_use_fp8_mlp(block, h)``                            -- train.py:927-934
  (``make_fp8_mlp_guard(flag)`` builds the same guard over a trainer's own
  flag, ``set_fp8_mlp(flag)`` sets this module's)
* ``fp8_update_scales(model)``                          -- train.py:937-946
* ``MLP(dim, hidden_dim)`` (same parameter/buffer names) -- train.py:247-262
* ``_FP8MLPBlock.apply(h, norm_w, w_gu, w_down, scale, amax, eps)``
                                                        -- train.py:1193-1252

y = h + down(SwiGLU(gate_up(rmsnorm(h)))) with x, gu, h stored e4m3 and d_gu
(and the in-register dy of the down wgrad) e5m2, delayed per-tensor pow2
scales, fp32 master weights quantized just in time, fp32 weight/norm grads,
bf16 dh.  There is no CPU or eager-torch fallback: without the HIP library the
block raises.

Weight quantization is cached per optimizer step: the e4m3 copies of the two
fp32 masters are made once and reused by every forward until the weights
change, instead of in every forward as train.py:1211-1212 does.  The copy is
refreshed by ``fp8_update_scales`` (which the trainer calls right after
``optimizer.step()``, train.py:4049-4050) and whenever a master's version
counter moves; the bytes are those a per-forward quantization gives.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from . import swiglu as _swiglu
from . import torch_ops  # registers the sparkfp8:: operators; holds the weight cache

FP8_MLP = False  # set True to route dense MLP sub-blocks through _FP8MLPBlock while training

# slot map: 0 = x (normed MLP input, e4m3), 1 = gu (gate/up pre-activation, e4m3),
# 2 = h (SwiGLU output, e4m3), 3 = d_gu (its gradient, e5m2), 4 = dy (e5m2)
FP8_SITE_MAX = (448.0, 448.0, 448.0, 57344.0, 57344.0)
FP8_HEADROOM_BINADES = 1

def set_fp8_mlp(flag: bool) -> None:
    """Sets ``FP8_MLP``, the switch ``_use_fp8_mlp`` reads (``--fp8-mlp``)."""
    global FP8_MLP
    FP8_MLP = bool(flag)


def make_fp8_mlp_guard(flag):
    """The guard of train.py:927-934 over a flag read at call time: ``flag``
    is a zero-argument callable returning the trainer's switch (spark-gpt's
    ``main()`` rebinds its module global ``FP8_MLP``, train.py:3642, so the
    guard must read that global, not a copy taken at import).  The Triton
    clause of the reference becomes "the HIP build", which importing this
    package already requires; the shape predicate is the reference's."""

    def _use_fp8_mlp(block, h: torch.Tensor) -> bool:
        if not (flag() and block.training and not getattr(block, "is_sparse", False)
                and h.is_cuda and h.dtype == torch.bfloat16):
            return False  # checked first: sparse blocks' mlp has no down_proj
        d, inter = h.shape[1], block.mlp.down_proj.weight.shape[1]
        return d % 128 == 0 and d & (d - 1) == 0 and inter % 128 == 0

    return _use_fp8_mlp


# this module's own switch
_use_fp8_mlp = make_fp8_mlp_guard(lambda: FP8_MLP)


@torch.no_grad()
def fp8_update_scales(model: nn.Module) -> None:
    """Roll every fp8 block's recorded amax into next step's scales (device-side,
    no host sync).  Applies to every module carrying ``fp8_scale``/``fp8_amax``
    5-slot buffers (this module's ``MLP`` and the reference's MLP/Experts).

    The trainer calls this right after ``optimizer.step()``, so it is also where
    the cached e4m3 weight copies of each dense MLP are re-quantized from the
    updated fp32 masters (the optimizer may write them through raw pointers,
    train.py:2955, which no version counter sees)."""
    for m in model.modules():
        scale = getattr(m, "fp8_scale", None)
        amax = getattr(m, "fp8_amax", None)
        if isinstance(scale, torch.Tensor) and isinstance(amax, torch.Tensor) and scale.numel() == 5:
            w_gu, w_down = _dense_weights(m)
            # a dense block's re-quantization rolls the scales in its own launches
            rolled = w_gu is not None and torch_ops.refresh_weight_cache(w_gu, w_down, scale, amax)
            if not rolled:
                ops.update_scales(scale, amax)


def _dense_weights(m: nn.Module):
    """(gate_up, down) fp32 master weights of an fp8 module: a dense MLP's two
    Linear weights (2-D), or the packed expert Parameters of the reference's
    Experts (3-D [E, 2I, D], [E, D, I], train.py:2252-2257); else (None, None)."""
    gu, dn = getattr(m, "gate_up_proj", None), getattr(m, "down_proj", None)
    if isinstance(gu, torch.Tensor) and isinstance(dn, torch.Tensor) and gu.dim() == 3 and dn.dim() == 3:
        return gu, dn
    w_gu, w_down = getattr(gu, "weight", None), getattr(dn, "weight", None)
    if isinstance(w_gu, torch.Tensor) and isinstance(w_down, torch.Tensor) and w_gu.dim() == 2 \
            and w_down.dim() == 2:
        return w_gu, w_down
    return None, None


class MLP(nn.Module):
    """Same parameters, buffers and forward as the reference MLP
    (train.py:247-262): the fused bf16 SwiGLU (``_FusedSwiGLU``) when
    ``_use_fused_swiglu(x)``, else gate/up -> silu * up -> down in torch."""

    def __init__(self, dim: int, hidden_dim: int):
        super().__init__()
        self.gate_up_proj = nn.Linear(dim, 2 * hidden_dim, bias=False)
        self.down_proj = nn.Linear(hidden_dim, dim, bias=False)
        # fp8 state: per-rank, not checkpointed (train.py:251-254)
        self.register_buffer("fp8_scale", torch.ones(5), persistent=False)
        self.register_buffer("fp8_amax", torch.zeros(5), persistent=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _swiglu._use_fused_swiglu(x):
            weight = self.gate_up_proj.weight.to(dtype=x.dtype).unsqueeze(0)
            offs = torch.full((1,), x.shape[0], device=x.device, dtype=torch.int32)
            return self.down_proj(_swiglu._FusedSwiGLU.apply(x, weight, offs))
        gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * up)


class _FP8MLPBlock(torch.autograd.Function):
    """y = h + down(SwiGLU(gate_up(rmsnorm(h)))) with fp8 activations.

    Forward: norm_quant -> weight_quant x2 -> gate/up FP8 GEMM with SwiGLU
    epilogue -> down FP8 GEMM with residual epilogue.
    Backward: bf16 down dgrad with SwiGLU-backward epilogue (d_gu e5m2) ->
    gate/up FP8 dgrad -> RMSNorm backward (+ e5m2 dy^T) -> the two FP8 weight
    gradients reduced over tokens.

    The two halves are the custom operators ``sparkfp8::block_fwd`` and
    ``sparkfp8::block_bwd`` (torch_ops.py), so a ``torch.compile``d model
    (train.py:3787) traces them as two opaque nodes; eager calls run their
    implementations directly (``torch_ops.op``)."""

    @staticmethod
    def forward(ctx, h, norm_w, w_gu, w_down, scale, amax, eps):
        y, x8, rstd, gu8, h8 = torch_ops.op("block_fwd")(h, norm_w, w_gu, w_down, scale, amax, eps)
        # backward needs x8 and h8 (weight grads), gu8 (SwiGLU backward)
        # and the masters, whose quantized copies (W8^T for
        # the gate/up dgrad, bf16 Wd^T for the down dgrad) it finds cached
        ctx.save_for_backward(h, norm_w, w_gu, w_down, x8, rstd, gu8, h8, scale, amax)
        return y

    @staticmethod
    def backward(ctx, dy):
        h, norm_w, w_gu, w_down, x8, rstd, gu8, h8, scale, amax = ctx.saved_tensors
        dh, dnw, dwgu, dwd = torch_ops.op("block_bwd")(dy, h, norm_w, w_gu, w_down, x8, rstd, gu8, h8,
                                                          scale, amax)
        return dh, dnw, dwgu, dwd, None, None, None


def fp8_mlp_block(h: torch.Tensor, norm: nn.Module, mlp: MLP) -> torch.Tensor:
    """h + mlp(norm(h)) through _FP8MLPBlock, as Block.forward calls it
    (train.py:2359-2365)."""
    return _FP8MLPBlock.apply(h, norm.weight, mlp.gate_up_proj.weight, mlp.down_proj.weight,
                              mlp.fp8_scale, mlp.fp8_amax, norm.eps)
