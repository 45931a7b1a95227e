"""The block's forward and backward as ``torch.library`` custom operators.

spark-gpt compiles the whole model with ``torch.compile(model, mode="default",
dynamic=False)`` (train.py:3787).  The kernels here are reached through
ctypes, which TorchDynamo cannot trace; as custom operators with fake
(shape-only) implementations they become two opaque nodes of the compiled
graph instead of graph breaks.  Both mutate the module's 5-slot ``amax``
buffer in place (``mutates_args``), as the reference's kernels do with their
atomic max (train.py:1015-1016, 1094).

* ``sparkfp8::block_fwd(h, norm_w, w_gu, w_down, scale, amax, eps)`` returns
  y and the tensors the backward needs (train.py:1200-1226).
* ``sparkfp8::block_bwd(dy, h, norm_w, wdt, x8t, rstd, w8t, wscale, gu8, h8t,
  scale, amax)`` returns (dh, d_norm_w, dW_gate_up, dW_down)
  (train.py:1228-1252).
* ``sparkfp8::update_scales(scale, amax)`` is the delayed-scale roll
  (train.py:937-946).
"""
from __future__ import annotations

from typing import Tuple

import torch
from torch import Tensor

from . import ops

E4M3 = ops.E4M3
E5M2 = ops.E5M2


def _master(w: Tensor) -> Tensor:
    w = w.detach()
    if w.dtype != torch.float32:
        w = w.float()
    return w.contiguous()


@torch.library.custom_op("sparkfp8::block_fwd", mutates_args={"amax"})
def block_fwd(h: Tensor, norm_w: Tensor, w_gu: Tensor, w_down: Tensor, scale: Tensor, amax: Tensor,
              eps: float) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """y, then for the backward: wdt (bf16 K-slab of W_down^T), x8t, rstd,
    w8t (K-slab of W8^T), wscale [q_gu, q_d], gu8 (K-slab of [T, 2I]), h8t."""
    I = w_down.shape[1]
    h = h.contiguous()
    x8, x8t, rstd = ops.norm_quant(h, _master(norm_w), scale, amax, eps)
    wscale = torch.empty(2, dtype=torch.float32, device=h.device)
    w8, w8t, _ = ops.weight_quant(_master(w_gu), wscale[0:1], w8=True, w8t=True)
    wd8, _, wdt = ops.weight_quant(_master(w_down), wscale[1:2], w8=True, bf16t=True)
    gu8, h8, h8t = ops.gateup_swiglu_fwd(x8, w8, scale, wscale, amax, h.shape[0], I)
    y = ops.down_fwd(h8, wd8, h, scale, wscale)
    return y, wdt, x8t, rstd, w8t, wscale, gu8, h8t


@block_fwd.register_fake
def _block_fwd_fake(h, norm_w, w_gu, w_down, scale, amax, eps):
    T, D = h.shape
    I = w_down.shape[1]
    ldt = ops.ldt_of(T)
    sr = ops.slab_rows
    return (h.new_empty((T, D), dtype=torch.bfloat16),
            h.new_empty((D // 32, sr(I), 32), dtype=torch.bfloat16),
            h.new_empty((ldt // 64, sr(D), 64), dtype=E4M3),
            h.new_empty((T,), dtype=torch.float32),
            h.new_empty((2 * I // 64, sr(D), 64), dtype=E4M3),
            h.new_empty((2,), dtype=torch.float32),
            h.new_empty((2 * I // 64, ldt, 64), dtype=E4M3),
            h.new_empty((ldt // 64, sr(I), 64), dtype=E4M3))


@torch.library.custom_op("sparkfp8::block_bwd", mutates_args={"amax"})
def block_bwd(dy: Tensor, h: Tensor, norm_w: Tensor, wdt: Tensor, x8t: Tensor, rstd: Tensor, w8t: Tensor,
              wscale: Tensor, gu8: Tensor, h8t: Tensor, scale: Tensor,
              amax: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dh bf16, d_norm_w fp32, dW_gate_up fp32, dW_down fp32)."""
    dy = dy.contiguous()
    if dy.dtype != torch.bfloat16:
        dy = dy.to(torch.bfloat16)
    h = h.contiguous()
    T, D = h.shape
    I = gu8.shape[0] * ops.SLAB // 2
    dgu8, dgu8t = ops.down_dgrad_swiglu(dy, wdt, gu8, scale, amax)
    dxn = ops.gateup_dgrad(dgu8, w8t, scale, wscale, T, D)
    del dgu8
    dh, dnw, dy8t = ops.norm_bwd(h, rstd, dxn, dy, _master(norm_w), scale, amax)
    del dxn
    dwd = ops.wgrad(dy8t, h8t, D, I, scale[4:5], scale[2:3])
    dwgu = ops.wgrad(dgu8t, x8t, 2 * I, D, scale[3:4], scale[0:1])
    return dh, dnw, dwgu, dwd


@block_bwd.register_fake
def _block_bwd_fake(dy, h, norm_w, wdt, x8t, rstd, w8t, wscale, gu8, h8t, scale, amax):
    T, D = h.shape
    I = gu8.shape[0] * ops.SLAB // 2
    return (h.new_empty((T, D), dtype=torch.bfloat16),
            h.new_empty((D,), dtype=torch.float32),
            h.new_empty((2 * I, D), dtype=torch.float32),
            h.new_empty((D, I), dtype=torch.float32))


@torch.library.custom_op("sparkfp8::update_scales", mutates_args={"scale", "amax"})
def update_scales(scale: Tensor, amax: Tensor) -> None:
    ops.update_scales(scale, amax)


@update_scales.register_fake
def _update_scales_fake(scale, amax):
    return None
