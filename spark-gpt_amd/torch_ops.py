"""The block's forward and backward as ``torch.library`` custom operators.

spark-gpt compiles the whole model with ``torch.compile(model, mode="default",
dynamic=False)`` (train.py:3787).  The kernels here are reached through
ctypes, which TorchDynamo cannot trace; as custom operators with fake
(shape-only) implementations they become two opaque nodes of the compiled
graph instead of graph breaks.  Both mutate the module's 5-slot ``amax``
buffer in place (``mutates_args``), as the reference's kernels do with their
atomic max (train.py:1015-1016, 1094).

* ``sparkfp8::block_fwd(h, norm_w, w_gu, w_down, scale, amax, eps)`` returns
  y and the activations the backward needs (train.py:1200-1226).
* ``sparkfp8::block_bwd(dy, h, norm_w, w_gu, w_down, x8, rstd, gu8, h8,
  scale, amax)`` returns (dh, d_norm_w, dW_gate_up, dW_down)
  (train.py:1228-1252).
* ``sparkfp8::update_scales(scale, amax)`` is the delayed-scale roll
  (train.py:937-946).

Each operator's Python implementation is ``<name>_impl``; ``op(name)`` hands
the autograd Functions the operator while torch.compile traces and the
implementation itself in eager mode.

The forward's e4m3 weight copies come from a cache keyed on the fp32
masters (``cached_weights``), so the two just-in-time quantizations of
train.py:1211-1212 run once per optimizer step rather than once per forward.
"""
from __future__ import annotations

import threading
import weakref
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


# ------------------------------------------------------------ weight cache
FP8_WEIGHT_CACHE = True  # False: quantize the masters in every forward, as train.py:1211-1212

# id(w_gu) -> (weakref(w_gu), weakref(w_down), key, (w8, w8t, wd8, wdt, wscale)).
# Entries hold device memory only while their gate/up master is alive.
_WCACHE: dict = {}
_WLOCK = threading.Lock()


def _wkey(w_gu: Tensor, w_down: Tensor):
    return (w_gu._version, w_gu.data_ptr(), tuple(w_gu.shape), w_down._version, w_down.data_ptr(),
            tuple(w_down.shape))


def quantize_weights(w_gu: Tensor, w_down: Tensor, scale=None, amax=None):
    """(w8, w8t, wd8, wdt, wscale): e4m3 K-slabs of W_gu and its transpose,
    of W_down, the bf16 K-slab of W_down^T and the pow2 weight scales.
    Dense masters (2-D): wscale = [q_gu, q_d] (train.py:949-952, 1211-1213,
    1224-1225), both in two launches, which also roll the block's 5 scale
    slots when scale and amax are given (the post-step hook's update_scales).
    Expert masters (3-D, [E, 2I, D] and [E, D, I]): every copy stacked per
    expert and wscale [2, E] (train.py:1536-1540, 1561-1562, 1572-1573);
    scale and amax must not be given for them."""
    if w_gu.dim() == 3:
        assert scale is None and amax is None
        wscale = torch.empty(2, w_gu.shape[0], dtype=torch.float32, device=w_gu.device)
        w8, w8t, _ = ops.weight_quant_experts(_master(w_gu), wscale[0], w8=True, w8t=True)
        wd8, _, wdt = ops.weight_quant_experts(_master(w_down), wscale[1], w8=True, bf16t=True)
        return w8, w8t, wd8, wdt, wscale
    return ops.block_weight_quant(_master(w_gu), _master(w_down), scale, amax)


def _drop_entry(i: int, ref) -> None:
    with _WLOCK:
        ent = _WCACHE.get(i)
        if ent is not None and ent[0] is ref:
            del _WCACHE[i]


def _store(w_gu: Tensor, w_down: Tensor, q) -> None:
    i = id(w_gu)
    ref = weakref.ref(w_gu, lambda r, i=i: _drop_entry(i, r))
    with _WLOCK:
        _WCACHE[i] = (ref, weakref.ref(w_down), _wkey(w_gu, w_down), q)


def cached_weights(w_gu: Tensor, w_down: Tensor):
    """The forward's quantized weights: the cached copies while the same two
    masters are unchanged since they were quantized (same objects, storage
    and version counters), else a fresh quantization, which is cached.
    Cached tensors are never written again: a refresh allocates new ones, so
    a pending backward keeps the copies its forward used."""
    if not FP8_WEIGHT_CACHE:
        return quantize_weights(w_gu, w_down)
    with _WLOCK:
        ent = _WCACHE.get(id(w_gu))
    if ent is not None and ent[0]() is w_gu and ent[1]() is w_down and ent[2] == _wkey(w_gu, w_down):
        return ent[3]
    q = quantize_weights(w_gu, w_down)
    _store(w_gu, w_down, q)
    return q


def op(name: str):
    """The callable the autograd Functions run for operator ``name``: under
    torch.compile the registered ``sparkfp8::`` operator (one opaque node of
    the compiled graph); in eager mode its Python implementation itself,
    which does the same launches without the dispatcher's custom-operator
    layer (tens of microseconds per call, felt by small steps)."""
    if torch.compiler.is_compiling():
        return getattr(torch.ops.sparkfp8, name)
    return globals()[name + "_impl"]


@torch.no_grad()
def refresh_weight_cache(w_gu: Tensor, w_down: Tensor, scale=None, amax=None) -> bool:
    """Re-quantize the cached copies of (w_gu, w_down), if there are any:
    called after the optimizer has written the masters (which it may do
    without moving their version counters).  With the block's 5-slot scale
    and amax (dense masters only), the same launches also roll them; returns
    whether they did (when nothing was re-quantized, the caller rolls)."""
    with _WLOCK:
        ent = _WCACHE.get(id(w_gu))
    if ent is None or ent[0]() is not w_gu:
        return False
    if not FP8_WEIGHT_CACHE or not w_gu.is_cuda:
        _drop_entry(id(w_gu), ent[0])
        return False
    roll = scale is not None and w_gu.dim() == 2
    _store(w_gu, w_down, quantize_weights(w_gu, w_down, scale if roll else None, amax if roll else None))
    return roll


def clear_weight_cache() -> None:
    with _WLOCK:
        _WCACHE.clear()


def block_fwd_impl(h: Tensor, norm_w: Tensor, w_gu: Tensor, w_down: Tensor, scale: Tensor, amax: Tensor,
              eps: float) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """y, then for the backward: x8 (K-slab of [T, D]), rstd, gu8 (K-slab of
    [T, 2I]) and h8 (K-slab of [T, I]).  The weight gradients read x8 and h8
    through transposing LDS reads, so no token-contiguous copy is written.
    The quantized weights stay in the weight cache: they are never an output
    (a compiled graph may recycle the memory of the tensors it saves for
    backward), and the backward looks them up from the same masters."""
    I = w_down.shape[1]
    h = h.contiguous()
    x8, _, rstd = ops.norm_quant(h, _master(norm_w), scale, amax, eps, copy=False)
    w8, _w8t, wd8, _wdt, wscale = cached_weights(w_gu, w_down)
    gu8, h8, _ = ops.gateup_swiglu_fwd(x8, w8, scale, wscale, amax, h.shape[0], I, copy=False)
    y = ops.down_fwd(h8, wd8, h, scale, wscale)
    return y, x8, rstd, gu8, h8


block_fwd = torch.library.custom_op("sparkfp8::block_fwd", block_fwd_impl, mutates_args={"amax"})


@block_fwd.register_fake
def _block_fwd_fake(h, norm_w, w_gu, w_down, scale, amax, eps):
    T, D = h.shape
    I = w_down.shape[1]
    ldt = ops.ldt_of(T)
    sr = ops.slab_rows
    return (h.new_empty((T, D), dtype=torch.bfloat16),
            h.new_empty((D // 64, ldt, 64), dtype=E4M3),
            h.new_empty((T,), dtype=torch.float32),
            h.new_empty((2 * I // 64, ldt, 64), dtype=E4M3),
            h.new_empty((I // 64, ldt, 64), dtype=E4M3))


def block_bwd_impl(dy: Tensor, h: Tensor, norm_w: Tensor, w_gu: Tensor, w_down: Tensor, x8: Tensor, rstd: Tensor,
              gu8: Tensor, h8: Tensor, scale: Tensor, amax: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dh bf16, d_norm_w fp32, dW_gate_up fp32, dW_down fp32).  W8^T, the
    bf16 W_down^T and the weight scales are the forward's (the cache entry of
    the same, unchanged masters; train.py:1224-1225 saves them instead)."""
    dy = dy.contiguous()
    if dy.dtype != torch.bfloat16:
        dy = dy.to(torch.bfloat16)
    h = h.contiguous()
    T, D = h.shape
    I = gu8.shape[0] * ops.SLAB // 2
    _w8, w8t, _wd8, wdt, wscale = cached_weights(w_gu, w_down)
    dgu8, _ = ops.down_dgrad_swiglu(dy, wdt, gu8, scale, amax, copy=False)
    dxn = ops.gateup_dgrad(dgu8, w8t, scale, wscale, T, D)
    # x8, h8 and dgu8 are read as the token-major K-slabs their producers
    # wrote (transposing LDS reads); dy8t is the norm backward's
    # token-contiguous copy (a gradient with both operands transposed on
    # read is 2-3 % slower, the norm backward no faster for the row K-slab).
    # The gate/up weight gradient runs right after the other reader of
    # d_gu8, while part of it is still in the last-level cache (the launch
    # order of train.py:1249-1251 is a9, a10, a11, a12, a13; the results
    # do not depend on it): about 1 % off the backward.
    dwgu = ops.wgrad_rows(dgu8, x8, 2 * I, D, scale[3:4], scale[0:1])
    del dgu8
    dh, dnw, dy8t = ops.norm_bwd(h, rstd, dxn, dy, _master(norm_w), scale, amax)
    del dxn
    dwd = ops.wgrad_rows(dy8t, h8, D, I, scale[4:5], scale[2:3], a_rows=False)
    return dh, dnw, dwgu, dwd


block_bwd = torch.library.custom_op("sparkfp8::block_bwd", block_bwd_impl, mutates_args={"amax"})


@block_bwd.register_fake
def _block_bwd_fake(dy, h, norm_w, w_gu, w_down, x8, rstd, gu8, h8, scale, amax):
    T, D = h.shape
    I = gu8.shape[0] * ops.SLAB // 2
    return (h.new_empty((T, D), dtype=torch.bfloat16),
            h.new_empty((D,), dtype=torch.float32),
            h.new_empty((2 * I, D), dtype=torch.float32),
            h.new_empty((D, I), dtype=torch.float32))


# ------------------------------------------------------------ MoE experts
def moe_fwd_impl(x: Tensor, w_gu: Tensor, w_d: Tensor, token_index: Tensor, offsets: Tensor, scale: Tensor,
            amax: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """_FP8Experts.forward (train.py:1552-1587): out [R, D] bf16 expert-order
    rows (unweighted), then for the backward the plan, x8, gu8 and h8 (K-slabs
    over padded expert order; the weight gradients read x8 and h8 through
    transposing LDS reads).  Quantized expert weights stay in the weight
    cache."""
    x = x.contiguous()
    R = token_index.numel()
    E, I2, D = w_gu.shape
    plan = ops.moe_plan(offsets, R)
    ldp = ops.moe_padded_rows(R, E)
    x8, _ = ops.moe_rows_quant(x, token_index, plan, ldp, scale, 0, amax, 0, ops.FMT_E4M3, True, False)
    w8, _w8t, wd8, _wdt, wscale = cached_weights(w_gu, w_d)
    gu8, h8, _ = ops.moe_gateup_swiglu_fwd(x8, w8, plan, scale, wscale[0], amax, I2 // 2, copy=False)
    out = ops.moe_down_fwd(h8, wd8, plan, scale, wscale[1], R, D)
    return out, plan, x8, gu8, h8


moe_fwd = torch.library.custom_op("sparkfp8::moe_fwd", moe_fwd_impl, mutates_args={"amax"})


@moe_fwd.register_fake
def _moe_fwd_fake(x, w_gu, w_d, token_index, offsets, scale, amax):
    R = token_index.numel()
    E, I2, D = w_gu.shape
    ldp = 256 * ((R + 255) // 256 + E)
    return (x.new_empty((R, D), dtype=torch.bfloat16),
            x.new_empty((8 + 2 * E + 3 * (ldp // 256),), dtype=torch.int32),
            x.new_empty(ops.kslab_shape(ldp, D, E4M3), dtype=E4M3),
            x.new_empty(ops.kslab_shape(ldp, I2, E4M3), dtype=E4M3),
            x.new_empty(ops.kslab_shape(ldp, I2 // 2, E4M3), dtype=E4M3))


def moe_bwd_impl(dout: Tensor, w_gu: Tensor, w_d: Tensor, plan: Tensor, x8: Tensor, gu8: Tensor, h8: Tensor,
            inverse_permutation: Tensor, T: int, top_k: int, scale: Tensor,
            amax: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """_FP8Experts.backward (train.py:1589-1605): (dx [T, D] bf16 summed over
    each token's top_k rows, dW_gate_up fp32 [E, 2I, D], dW_down fp32 [E, D, I])."""
    dout = dout.contiguous()
    if dout.dtype != torch.bfloat16:
        dout = dout.to(torch.bfloat16)
    R, D = dout.shape
    E, I2, _ = w_gu.shape
    ldp = gu8.shape[1]
    _w8, w8t, _wd8, wdt, wscale = cached_weights(w_gu, w_d)
    # e5m2 dout over padded expert order (the down wgrad's operand) and amax[4]
    _, dout8t = ops.moe_rows_quant(dout, None, plan, ldp, scale, 4, amax, 4, ops.FMT_E5M2, False)
    dgu8, _ = ops.moe_down_dgrad_swiglu(dout, wdt, gu8, plan, scale, amax, copy=False)
    dx = ops.moe_gateup_dgrad(dgu8, w8t, plan, scale, wscale[0], R, D)
    # d_gu8, x8 and h8 read as their K-slabs (transposing LDS reads), dout8t
    # token-contiguous, as in the dense block
    dw_gu = ops.moe_wgrad_rows(dgu8, x8, I2, D, E, plan, scale[3:4], scale[0:1])
    dw_d = ops.moe_wgrad_rows(dout8t, h8, D, I2 // 2, E, plan, scale[4:5], scale[2:3], a_rows=False)
    dxn = ops.moe_topk_sum(dx, inverse_permutation, T, top_k)
    return dxn, dw_gu, dw_d


moe_bwd = torch.library.custom_op("sparkfp8::moe_bwd", moe_bwd_impl, mutates_args={"amax"})


@moe_bwd.register_fake
def _moe_bwd_fake(dout, w_gu, w_d, plan, x8, gu8, h8, inverse_permutation, T, top_k, scale, amax):
    E, I2, D = w_gu.shape
    return (dout.new_empty((T, D), dtype=torch.bfloat16),
            dout.new_empty((E, I2, D), dtype=torch.float32),
            dout.new_empty((E, D, I2 // 2), dtype=torch.float32))


def update_scales_impl(scale: Tensor, amax: Tensor) -> None:
    ops.update_scales(scale, amax)


update_scales = torch.library.custom_op("sparkfp8::update_scales", update_scales_impl, mutates_args={"scale", "amax"})


@update_scales.register_fake
def _update_scales_fake(scale, amax):
    return None


# ----------------------------------------------------- bf16 SwiGLU path
BF16 = torch.bfloat16


def norm_swiglu_fwd_impl(h: Tensor, norm_w: Tensor, w_gu: Tensor, eps: float) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """_NormSwiGLU.forward (train.py:2111-2121): out = SwiGLU(gate_up(rmsnorm(h)))
    [T, I] bf16, the norm weight folded into the gate/up weight (W' =
    bf16(w_gu * norm_w)); then, for the backward, the bf16 K-slab of W'^T, gu
    [T, 2I] and rstd [T] (the weight gradient reads h itself, through
    transposing LDS reads)."""
    h = h.contiguous()
    T, D = h.shape
    I = w_gu.shape[0] // 2
    ws, wt = ops.bf16_weight_slabs(w_gu.detach().contiguous().unsqueeze(0), norm_w.detach().contiguous())
    # rstd, and the row K-slab of h that the GEMM reads (whole 128-byte
    # lines per K stage; the weight gradient reads h itself)
    rstd, _, hs = ops.bf16_rows_prep(h, None, ops.ldt_of(T), float(eps), copy=False, rows=True)
    gu, out = ops.bf16_swiglu_fwd(h, ws, I, rstd=rstd, xs=hs)
    return out, wt, gu, rstd


norm_swiglu_fwd = torch.library.custom_op("sparkfp8::norm_swiglu_fwd", norm_swiglu_fwd_impl, mutates_args=())


@norm_swiglu_fwd.register_fake
def _norm_swiglu_fwd_fake(h, norm_w, w_gu, eps):
    T, D = h.shape
    I2 = w_gu.shape[0]
    return (h.new_empty((T, I2 // 2), dtype=BF16), h.new_empty((1,) + ops.kslab_shape(D, I2, BF16), dtype=BF16),
            h.new_empty((T, I2), dtype=BF16), h.new_empty((T,), dtype=torch.float32))


def norm_swiglu_bwd_impl(dout: Tensor, h: Tensor, norm_w: Tensor, w_gu: Tensor, wt: Tensor, gu: Tensor,
                    rstd: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """_NormSwiGLU.backward (train.py:2123-2131): (dh bf16 [T, D], dnorm_w fp32
    [D], dw_gu fp32 [2I, D]).  G' = rstd * d_gu (bf16) once for both GEMMs:
    p = bf16(G' W'), dh = bf16(p - rstd^2 sum(h p) / D h), dW' = bf16(G'^T h),
    dw_gu = dW' * norm_w, dnorm_w = sum_rows(dW' * w_gu)."""
    dout = dout.contiguous()
    if dout.dtype != BF16:
        dout = dout.to(BF16)
    h = h.contiguous()
    T, D = h.shape
    I2 = gu.shape[1]
    gs, _ = ops.bf16_swiglu_bwd(gu, dout, rstd, None, ops.ldt_of(T), copy=False)
    p = ops.bf16_gemm(gs, wt, T, D, I2)
    dh = ops.bf16_norm_dh(p, h, rstd)
    del p
    # G' and h both read through transposing LDS reads (no copies)
    dwp = ops.bf16_wgrad_rows(gs, h, I2, D)
    dw, dnw = ops.bf16_fold_grads(dwp, w_gu.detach().contiguous(), norm_w.detach().contiguous())
    return dh, dnw, dw


norm_swiglu_bwd = torch.library.custom_op("sparkfp8::norm_swiglu_bwd", norm_swiglu_bwd_impl, mutates_args=())


@norm_swiglu_bwd.register_fake
def _norm_swiglu_bwd_fake(dout, h, norm_w, w_gu, wt, gu, rstd):
    T, D = h.shape
    return (h.new_empty((T, D), dtype=BF16), h.new_empty((D,), dtype=torch.float32),
            h.new_empty(tuple(w_gu.shape), dtype=torch.float32))


def _plan_ints(R: int, E: int) -> int:
    return 8 + 2 * E + 3 * ((R + 255) // 256 + E)


def swiglu_fwd_impl(x: Tensor, weight: Tensor, offs: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """_FusedSwiGLU.forward (train.py:2077-2081): h = SwiGLU(x W_e^T) [R, I]
    bf16 for the rows of each group e (offs: inclusive int32 row-count prefix
    sums), then gu [R, 2I] and the device-built row plan for the backward."""
    x = x.contiguous()
    weight = weight.contiguous()
    R, D = x.shape
    E, I2, _ = weight.shape
    plan = ops.moe_plan(offs, R)
    ldp = ops.moe_padded_rows(R, E)
    ws, _ = ops.bf16_weight_slabs(weight, rows=True, transposed=False)
    gu, h = ops.bf16_swiglu_fwd(x, ws, I2 // 2, plan=plan, ldp=ldp)
    return h, gu, plan


swiglu_fwd = torch.library.custom_op("sparkfp8::swiglu_fwd", swiglu_fwd_impl, mutates_args=())


@swiglu_fwd.register_fake
def _swiglu_fwd_fake(x, weight, offs):
    R, D = x.shape
    E, I2, _ = weight.shape
    return (x.new_empty((R, I2 // 2), dtype=BF16), x.new_empty((R, I2), dtype=BF16),
            x.new_empty((_plan_ints(R, E),), dtype=torch.int32))


def swiglu_bwd_impl(dh: Tensor, x: Tensor, weight: Tensor, gu: Tensor, plan: Tensor) -> Tuple[Tensor, Tensor]:
    """_FusedSwiGLU.backward (train.py:2083-2090): (dx [R, D] bf16, dW [E, 2I, D]
    bf16), the SwiGLU gradient G' (bf16) computed once for both GEMMs."""
    dh = dh.contiguous()
    if dh.dtype != BF16:
        dh = dh.to(BF16)
    x = x.contiguous()
    weight = weight.contiguous()
    R, D = x.shape
    E, I2, _ = weight.shape
    ldp = ops.moe_padded_rows(R, E)
    _, wt = ops.bf16_weight_slabs(weight, rows=False, transposed=True)
    _, xt, _ = ops.bf16_rows_prep(x, plan, ldp)
    gs, _ = ops.bf16_swiglu_bwd(gu, dh, None, plan, ldp, copy=False)
    dx = ops.bf16_gemm(gs, wt, R, D, I2, plan=plan)
    # G' read through transposing LDS reads, x as its token-contiguous copy
    dw = ops.bf16_wgrad_rows(gs, xt, I2, D, plan=plan, E=E)
    return dx, dw


swiglu_bwd = torch.library.custom_op("sparkfp8::swiglu_bwd", swiglu_bwd_impl, mutates_args=())


@swiglu_bwd.register_fake
def _swiglu_bwd_fake(dh, x, weight, gu, plan):
    return x.new_empty(tuple(x.shape), dtype=BF16), x.new_empty(tuple(weight.shape), dtype=BF16)
