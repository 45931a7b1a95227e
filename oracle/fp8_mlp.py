"""Torch-CPU restatement of spark-gpt's FP8 SwiGLU MLP block.  TEST
INFRASTRUCTURE ONLY (results are checked against it, and it is the timed CPU
baseline; never shipped).

Every function follows one piece of the reference (``train.py`` in
N8python/spark-gpt) and cites it.  Arithmetic is fp32 with the reference's
rounding points; FP8 values are exact in fp32, so every GEMM is an fp32 matmul
of dequantized operands (products exact, sums rounded in torch's order).

Two places where the reference is not bit-specified get a fixed spec here, which
the HIP kernels implement identically:

* norm statistics (``train.py:964``: ``tl.rsqrt(tl.sum(h*h, 1) / D + EPS)``):
  the sum of squares is accumulated in fp64 (exact for bf16 inputs unless the
  row spans more than 37 binades) and rounded once to fp32; rstd is
  ``fl32(1 / sqrt(fl64(v)))`` with IEEE double sqrt and divide.
* the power-of-two scale (``train.py:944, 951``) uses the correctly rounded
  fp32 log2 (torch CPU agrees with it on every band value; see
  ``oracle/fp8_bits.py``).
"""
from __future__ import annotations

import torch

# train.py:916-924 -- slot map 0=x, 1=gu, 2=h (e4m3), 3=d_gu, 4=dy (e5m2)
FP8_SITE_MAX = (448.0, 448.0, 448.0, 57344.0, 57344.0)
FP8_HEADROOM_BINADES = 1
E4M3_MAX = 448.0
E5M2_MAX = 57344.0


def e4m3(x: torch.Tensor) -> torch.Tensor:
    """clamp(x, +-448).to(e4m3fn) -- train.py:952, 968, 1013-1014."""
    return x.float().clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)


def e5m2(x: torch.Tensor) -> torch.Tensor:
    """clamp(x, +-57344).to(e5m2) -- train.py:1091-1092, 1172."""
    return x.float().clamp(-E5M2_MAX, E5M2_MAX).to(torch.float8_e5m2)


def bf(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> bf16 (RNE) -> fp32, the reference's bf16 rounding points."""
    return x.to(torch.bfloat16).float()


def f(x: torch.Tensor) -> torch.Tensor:
    return x.float()


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def amax_of(x: torch.Tensor) -> torch.Tensor:
    return x.float().abs().amax() if x.numel() else torch.zeros((), dtype=torch.float32)


# ----------------------------------------------------------------- a3 / a4
def update_scales(scale: torch.Tensor, amax: torch.Tensor,
                  site_max=FP8_SITE_MAX, headroom=FP8_HEADROOM_BINADES) -> None:
    """In-place scale roll, train.py:937-946 (same torch expression)."""
    fmax = scale.new_tensor(site_max)
    new = torch.exp2(torch.floor(torch.log2(fmax / amax.clamp(min=1e-30))) - headroom)
    scale.copy_(torch.where(amax > 0, new, scale))
    amax.zero_()


def quantize_weight(w: torch.Tensor):
    """Just-in-time per-tensor pow2 e4m3 copy, train.py:949-952."""
    q = torch.exp2(torch.floor(torch.log2(448.0 / w.detach().float().abs().amax().clamp(min=1e-30))))
    return (w.detach().float() * q).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), q


# ----------------------------------------------------------------- a5
def norm_stats(h: torch.Tensor, eps: float) -> torch.Tensor:
    """rstd per row (spec for train.py:964, see module docstring)."""
    D = h.shape[1]
    ss = (h.double() ** 2).sum(1).float()
    v = ss / D + torch.tensor(eps, dtype=torch.float32)
    return (1.0 / v.double().sqrt()).float()


def norm_quant(h: torch.Tensor, norm_w: torch.Tensor, s0: torch.Tensor, eps: float):
    """x8 = e4m3(rmsnorm(h)*w*s0) row-major and transposed, rstd, amax0 --
    train.py:955-972 (``n = h * rstd * w`` evaluated left to right)."""
    hf = f(h)
    r = norm_stats(h, eps)
    n = (hf * r[:, None]) * norm_w.float()[None, :]
    x8 = e4m3(n * s0)
    return x8, x8.t().contiguous(), r, amax_of(n)


def quant_rowcol(x: torch.Tensor, s: torch.Tensor):
    """Standalone quantizer: the norm-free core of train.py:966-972."""
    x8 = e4m3(f(x) * s)
    return x8, x8.t().contiguous(), amax_of(x)


# ----------------------------------------------------------------- a6 / a7
def swiglu_fwd(x8, w8, s, wscale, I: int):
    """gate/up FP8 GEMM + SwiGLU epilogue, train.py:975-1016."""
    xf, wf = f(x8), f(w8)
    deq = 1.0 / (s[0] * wscale[0])
    g = bf((xf @ wf[:I].t()) * deq)
    u = bf((xf @ wf[I:].t()) * deq)
    h = g * torch.sigmoid(g) * u
    gu8 = torch.cat([e4m3(g * s[1]), e4m3(u * s[1])], dim=1)
    h8 = e4m3(h * s[2])
    a1 = torch.maximum(amax_of(g), amax_of(u))
    return gu8, h8, a1, amax_of(h)


def down_fwd(h8, wd8, res, s, wscale):
    """down FP8 GEMM + residual, train.py:1019-1046."""
    out = bf((f(h8) @ f(wd8).t()) / (s[2] * wscale[1]))
    return (f(res) + out).to(torch.bfloat16)


# ----------------------------------------------------------------- a9 / a10
def down_dgrad_swiglu(dy, wd_bf16, gu8, s, I: int):
    """bf16 dy @ Wd + SwiGLU backward epilogue, d_gu in e5m2, train.py:1049-1094."""
    dh = bf(f(dy) @ f(wd_bf16))
    s_gu = 1.0 / s[1]
    g = f(gu8[:, :I]) * s_gu
    u = f(gu8[:, I:]) * s_gu
    sig = torch.sigmoid(g)
    d_gate = dh * u * (sig * (1.0 + g * (1.0 - sig)))
    d_up = dh * g * sig
    dgu8 = torch.cat([e5m2(d_gate * s[3]), e5m2(d_up * s[3])], dim=1)
    a3 = torch.maximum(amax_of(d_gate), amax_of(d_up))
    return dgu8, a3, amax_of(dy)


def gateup_dgrad(dgu8, w8, s, wscale):
    """dxn = (d_gu8 @ W8) / (s3 * q_gu) in bf16, train.py:1239-1241."""
    return ((f(dgu8) @ f(w8)) * (1.0 / s[3]) * (1.0 / wscale[0])).to(torch.bfloat16)


# ----------------------------------------------------------------- a11
def norm_bwd(h, rstd, dxn, dy, norm_w):
    """RMSNorm backward + residual grad, train.py:1130-1147 and the dnw sum at
    train.py:1252."""
    D = h.shape[1]
    hf, g, r = f(h), f(dxn), rstd.float()
    gw = g * norm_w.float()[None, :]
    S = (gw * hf).sum(1)
    dh = gw * r[:, None] - hf * (S * r * r * r * (1.0 / D))[:, None]
    dh = dh + f(dy)
    dnw = (g * (hf * r[:, None])).sum(0)
    return dh.to(torch.bfloat16), dnw


# ----------------------------------------------------------------- a12 / a13
def down_wgrad(dy, h8, s, splits: int = 2, block_r: int = 32):
    """dWd = sum_t e5m2(dy*s4)^T h8 / (s4*s2), split over tokens, train.py:1150-1187
    (called with BLOCK_R=32 at train.py:1247)."""
    T = dy.shape[0]
    dq = f(e5m2(f(dy) * s[4]))
    hf = f(h8)
    rows = _cdiv(_cdiv(T, splits), block_r) * block_r
    out = torch.zeros(dy.shape[1], h8.shape[1])
    for sp in range(splits):
        a, b = sp * rows, min((sp + 1) * rows, T)
        if a < b:
            out = out + (dq[a:b].t() @ hf[a:b]) / (s[4] * s[2])
    return out


def gateup_wgrad(dgu8, x8, s):
    """dWgu = d_gu8^T x8 / (s3*s0), train.py:1097-1127 called at train.py:1249-1251."""
    return (f(dgu8).t() @ f(x8)) * (1.0 / (s[3] * s[0]))


# ----------------------------------------------------------------- a8 / a14
def block_forward(h, norm_w, w_gu, w_down, scale, amax, eps):
    """_FP8MLPBlock.forward (train.py:1200-1226).  Mutates ``amax`` (max-accumulate
    slots 0-2) and returns (y, saved) where ``saved`` holds what backward needs."""
    T, D = h.shape
    I = w_down.shape[1]
    s = scale.float()
    x8, x8t, rstd, a0 = norm_quant(h, norm_w, s[0], eps)
    w8, q_gu = quantize_weight(w_gu)
    wd8, q_d = quantize_weight(w_down)
    wscale = torch.stack((q_gu, q_d)).float()
    gu8, h8, a1, a2 = swiglu_fwd(x8, w8, s, wscale, I)
    y = down_fwd(h8, wd8, h, s, wscale)
    amax[0] = torch.maximum(amax[0], a0)
    amax[1] = torch.maximum(amax[1], a1)
    amax[2] = torch.maximum(amax[2], a2)
    saved = dict(h=h, norm_w=norm_w, wd=w_down.detach().to(torch.bfloat16), x8=x8, x8t=x8t,
                 rstd=rstd, w8=w8, wd8=wd8, wscale=wscale, gu8=gu8, h8=h8, I=I)
    return y, saved


def block_backward(dy, saved, scale, amax):
    """_FP8MLPBlock.backward (train.py:1228-1252).  Mutates ``amax`` slots 3-4 and
    returns (dh bf16, dnw fp32[D], dWgu fp32[2I,D], dWd fp32[D,I]) plus the
    intermediates (for kernel-level parity)."""
    s = scale.float()
    I = saved["I"]
    dgu8, a3, a4 = down_dgrad_swiglu(dy, saved["wd"], saved["gu8"], s, I)
    dxn = gateup_dgrad(dgu8, saved["w8"], s, saved["wscale"])
    dh, dnw = norm_bwd(saved["h"], saved["rstd"], dxn, dy, saved["norm_w"])
    dwd = down_wgrad(dy, saved["h8"], s)
    dwgu = gateup_wgrad(dgu8, saved["x8"], s)
    amax[3] = torch.maximum(amax[3], a3)
    amax[4] = torch.maximum(amax[4], a4)
    inter = dict(dgu8=dgu8, dxn=dxn)
    return (dh, dnw, dwgu, dwd), inter


def fp32_reference(h, norm_w, w_gu, w_down, probe, eps=1e-6):
    """fp32 autograd MLP, as in spark-gpt tests/test_fp8_mlp.py:42-47.  Returns
    (y, dh, dnorm_w, dW_gate_up, dW_down) for upstream gradient ``probe``."""
    x32 = h.float().clone().requires_grad_(True)
    p32 = [p.detach().float().clone().requires_grad_(True) for p in (norm_w, w_gu, w_down)]
    n = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps) * p32[0]
    g, u = (n @ p32[1].t()).chunk(2, dim=-1)
    y32 = x32 + (torch.nn.functional.silu(g) * u) @ p32[2].t()
    grads = torch.autograd.grad((y32 * probe).sum(), [x32] + p32)
    return (y32.detach(),) + tuple(g_.detach() for g_ in grads)


def rel_l2(a: torch.Tensor, r: torch.Tensor) -> float:
    a, r = a.detach().double(), r.detach().double()
    return float((a - r).norm() / r.norm().clamp(min=1e-300))
