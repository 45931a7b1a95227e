"""Torch-CPU restatement of spark-gpt's bf16 SwiGLU MLP path (its default,
non-FP8 path).  TEST INFRASTRUCTURE ONLY (results are checked against it;
never shipped).

Follows ``train.py`` of N8python/spark-gpt: ``_swiglu_gemm_kernel``
(train.py:1625-1716), ``_swiglu_tiles`` / ``_swiglu_dgrad_kernel`` /
``_swiglu_wgrad_kernel`` (train.py:1899-2063), ``_FusedSwiGLU``
(train.py:2067-2090) and ``_NormSwiGLU`` (train.py:2101-2131).  Arithmetic is
fp32 with the reference's bf16 rounding points:

* gate/up accumulated in fp32 (bf16 products are exact in fp32), scaled by
  rstd with the folded norm, rounded to bf16 (train.py:1696-1707);
* h = g * sigmoid(g) * u in fp32 from the rounded g, u, rounded to bf16
  (train.py:1709-1715);
* d_gate, d_up rounded to bf16 before both GEMMs (train.py:1900-1905);
* the dgrad output and the weight gradient rounded to bf16 (train.py:1980,
  2024-2026); the norm backward and the fold of the weight gradient in fp32
  torch ops (train.py:2125-2131).

The norm statistic follows the FP8 oracle's fixed spec (``fp8_mlp.norm_stats``):
the sum of squares exact, rstd = fl32(1 / sqrt(fl64(v))).
"""
from __future__ import annotations

import torch

from .fp8_mlp import bf, f, norm_stats


def fold_weight(w_gu: torch.Tensor, norm_w: torch.Tensor) -> torch.Tensor:
    """W' = bf16(w_gu * norm_w) (train.py:2112), as fp32 values."""
    return bf(w_gu.float() * norm_w.float())


def swiglu_rows(acc_g: torch.Tensor, acc_u: torch.Tensor):
    """(g, u, h) from fp32 gate/up accumulators (already row-scaled):
    g, u = bf16(acc), h = bf16(g * sigmoid(g) * u) (train.py:1703-1715)."""
    g, u = bf(acc_g), bf(acc_u)
    return g, u, bf(g * torch.sigmoid(g) * u)


def swiglu_grad(g: torch.Tensor, u: torch.Tensor, dh: torch.Tensor):
    """(d_gate, d_up) = bf16 of dh * u * (sig * (1 + g * (1 - sig))) and
    dh * g * sig, sig = sigmoid(g) (_swiglu_tiles, train.py:1900-1905)."""
    sig = torch.sigmoid(g)
    return bf(dh * u * (sig * (1.0 + g * (1.0 - sig)))), bf(dh * g * sig)


def norm_swiglu_forward(h: torch.Tensor, norm_w: torch.Tensor, w_gu: torch.Tensor, eps: float):
    """_NormSwiGLU.forward (train.py:2111-2121): (out [T, I] bf16, saved)."""
    I = w_gu.shape[0] // 2
    hf = f(h)
    wp = fold_weight(w_gu, norm_w)
    rstd = norm_stats(h, eps)
    acc = hf @ wp.t()
    g, u, out = swiglu_rows(acc[:, :I] * rstd[:, None], acc[:, I:] * rstd[:, None])
    gu = torch.cat([g, u], dim=1)
    return out.to(torch.bfloat16), dict(h=h, norm_w=norm_w, w_gu=w_gu, wp=wp, gu=gu, rstd=rstd)


def norm_swiglu_backward(dout: torch.Tensor, saved: dict):
    """_NormSwiGLU.backward (train.py:2123-2131): (dh bf16, dnorm_w fp32,
    dw_gu fp32)."""
    gu, rstd, wp, h = saved["gu"], saved["rstd"], saved["wp"], saved["h"]
    I = gu.shape[1] // 2
    d_gate, d_up = swiglu_grad(gu[:, :I], gu[:, I:], f(dout) * rstd[:, None])
    gp = torch.cat([d_gate, d_up], dim=1)  # rstd * d_gu, bf16 values
    p = bf(gp @ wp)  # _swiglu_dgrad stores bf16 (train.py:1980), .float() at 2124
    hf = f(h)
    coef = rstd * rstd * (hf * p).sum(-1) / h.shape[1]
    dh = (p - coef[:, None] * hf).to(torch.bfloat16)
    dwp = bf(gp.t() @ hf)  # _swiglu_wgrad stores bf16 (train.py:2024-2026)
    return dh, (dwp * saved["w_gu"].float()).sum(0), dwp * saved["norm_w"].float()


def group_ranges(offs: torch.Tensor):
    """[(start, end)] of each group from its inclusive prefix sums."""
    ends = [int(v) for v in offs.tolist()]
    return [(ends[e - 1] if e else 0, ends[e]) for e in range(len(ends))]


def fused_swiglu_forward(x: torch.Tensor, w: torch.Tensor, offs: torch.Tensor):
    """_FusedSwiGLU.forward (train.py:2077-2081): (h [R, I] bf16, gu [R, 2I] as
    fp32 values); rows past the last group stay zero here (the reference
    leaves them unwritten)."""
    R = x.shape[0]
    I = w.shape[1] // 2
    h = torch.zeros(R, I)
    gu = torch.zeros(R, 2 * I)
    for e, (r0, r1) in enumerate(group_ranges(offs)):
        if r1 <= r0:
            continue
        acc = f(x[r0:r1]) @ f(w[e]).t()
        g, u, hh = swiglu_rows(acc[:, :I], acc[:, I:])
        h[r0:r1], gu[r0:r1] = hh, torch.cat([g, u], dim=1)
    return h.to(torch.bfloat16), gu


def fused_swiglu_backward(dh: torch.Tensor, x: torch.Tensor, w: torch.Tensor, gu: torch.Tensor, offs: torch.Tensor):
    """_FusedSwiGLU.backward (train.py:2083-2090): (dx [R, D] bf16, dw [E, 2I, D]
    bf16); groups without rows get a zero gradient."""
    R, D = x.shape
    E, I2, _ = w.shape
    I = I2 // 2
    dx = torch.zeros(R, D)
    dw = torch.zeros(E, I2, D)
    for e, (r0, r1) in enumerate(group_ranges(offs)):
        if r1 <= r0:
            continue
        d_gate, d_up = swiglu_grad(gu[r0:r1, :I], gu[r0:r1, I:], f(dh[r0:r1]))
        gp = torch.cat([d_gate, d_up], dim=1)
        dx[r0:r1] = gp @ f(w[e])
        dw[e] = gp.t() @ f(x[r0:r1])
    return dx.to(torch.bfloat16), dw.to(torch.bfloat16)


def fp32_norm_swiglu(h, norm_w, w_gu, eps, probe):
    """The fp32 function _NormSwiGLU computes, with autograd (as spark-gpt
    tests/test_moe.py:484-487): (out, dh, dnorm_w, dw_gu) for upstream
    gradient ``probe``."""
    h32 = h.float().clone().requires_grad_(True)
    nw = norm_w.detach().float().clone().requires_grad_(True)
    wgu = w_gu.detach().float().clone().requires_grad_(True)
    xn = h32 * torch.rsqrt(h32.pow(2).mean(-1, keepdim=True) + eps) * nw
    gate, up = (xn @ wgu.t()).chunk(2, dim=-1)
    out = torch.nn.functional.silu(gate) * up
    grads = torch.autograd.grad((out * probe).sum(), [h32, nw, wgu])
    return (out.detach(),) + tuple(g.detach() for g in grads)


def fp32_fused_swiglu(x, w, offs, probe):
    """The fp32 grouped SwiGLU with autograd (spark-gpt tests/test_moe.py:394-407):
    (h, dx, dw)."""
    x32 = x.float().clone().requires_grad_(True)
    w32 = w.detach().float().clone().requires_grad_(True)
    parts = []
    for e, (r0, r1) in enumerate(group_ranges(offs)):
        gate, up = (x32[r0:r1] @ w32[e].t()).chunk(2, dim=-1)
        parts.append(torch.nn.functional.silu(gate) * up)
    h = torch.cat(parts)
    gx, gw = torch.autograd.grad((h * probe.float()).sum(), (x32, w32))
    return h.detach(), gx, gw
