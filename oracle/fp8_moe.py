"""Torch-CPU restatement of spark-gpt's FP8 MoE experts (``_FP8Experts``).
TEST INFRASTRUCTURE ONLY (results are checked against it; never shipped).

Follows ``train.py`` of N8python/spark-gpt, lines 1255-1606, per expert with
the dense block's pieces (``oracle/fp8_mlp.py``): the expert-order gather and
e4m3 quantization of x (train.py:1300-1314), per-expert pow2 weight scales
(train.py:1536-1540), the grouped SwiGLU forward (1316-1353), down forward
(1356-1378), down dgrad + SwiGLU backward (1381-1423), gate/up dgrad
(1425-1448), the two weight gradients (1450-1533) and the top-k row sum
(2213-2217).  Expert e owns expert-order rows offsets[e-1] .. offsets[e]-1.
"""
from __future__ import annotations

import torch

from .fp8_mlp import amax_of, down_dgrad_swiglu, e4m3, e5m2, f, swiglu_fwd


def quantize_experts(w: torch.Tensor):
    """Per-expert e4m3 copies of (E, out, in) fp32 masters, train.py:1536-1540."""
    amax = w.detach().float().abs().amax(dim=(1, 2)).clamp(min=1e-30)
    q = torch.exp2(torch.floor(torch.log2(448.0 / amax)))
    return (w.detach().float() * q[:, None, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), q


def expert_ranges(offsets: torch.Tensor):
    """[(start, end)] per expert from the inclusive prefix sums (train.py:2284-2290)."""
    ends = [int(v) for v in offsets.tolist()]
    return [(ends[e - 1] if e else 0, ends[e]) for e in range(len(ends))]


def moe_forward(x, w_gu, w_d, token_index, offsets, scale, amax):
    """_FP8Experts.forward (train.py:1552-1587).  Mutates ``amax`` slots 0-2;
    returns (out [R, D] bf16 expert-order rows, saved)."""
    s = scale.float()
    E, I2, D = w_gu.shape
    I = I2 // 2
    R = token_index.numel()
    xg = x[token_index]
    x8 = e4m3(f(xg) * s[0])  # train.py:1311-1313: e4m3(x[tok] * s0), amax of |x|
    w8, q_gu = quantize_experts(w_gu)
    wd8, q_d = quantize_experts(w_d)
    gu8 = torch.zeros(R, I2, dtype=torch.float8_e4m3fn)
    h8 = torch.zeros(R, I, dtype=torch.float8_e4m3fn)
    out = torch.zeros(R, D, dtype=torch.bfloat16)
    a1 = a2 = torch.zeros(())
    for e, (r0, r1) in enumerate(expert_ranges(offsets)):
        if r1 <= r0:
            continue
        ws = torch.stack((q_gu[e], q_d[e])).float()
        g8, hh8, ea1, ea2 = swiglu_fwd(x8[r0:r1], w8[e], s, ws, I)
        gu8[r0:r1], h8[r0:r1] = g8, hh8
        a1, a2 = torch.maximum(a1, ea1), torch.maximum(a2, ea2)
        # train.py:1374-1377: acc / (s2 * q_d[e]) stored as bf16 (no residual)
        out[r0:r1] = ((f(hh8) @ f(wd8[e]).t()) / (s[2] * q_d[e])).to(torch.bfloat16)
    amax[0] = torch.maximum(amax[0], amax_of(xg))
    amax[1] = torch.maximum(amax[1], a1)
    amax[2] = torch.maximum(amax[2], a2)
    saved = dict(x8=x8, w8=w8, q_gu=q_gu, wd=w_d.detach().to(torch.bfloat16), gu8=gu8, h8=h8, offsets=offsets,
                 I=I)
    return out, saved


def sum_topk_rows(rows, inverse_permutation, top_k):
    """out[t] = sum over the top_k slots of rows[inverse_permutation[t, s]] (train.py:2213-2217)."""
    return rows[inverse_permutation].view(-1, top_k, rows.shape[-1]).sum(dim=1)


def moe_backward(dout, saved, scale, amax, inverse_permutation, top_k):
    """_FP8Experts.backward (train.py:1589-1605).  Mutates ``amax`` slots 3-4;
    returns (dx [T, D] bf16, dW_gate_up fp32 [E, 2I, D], dW_down fp32 [E, D, I])."""
    s = scale.float()
    I = saved["I"]
    E, D, _ = saved["wd"].shape
    R = dout.shape[0]
    dgu8 = torch.zeros(R, 2 * I, dtype=torch.float8_e5m2)
    dx = torch.zeros(R, D, dtype=torch.bfloat16)
    dw_gu = torch.zeros(E, 2 * I, D)
    dw_d = torch.zeros(E, D, I)
    a3 = a4 = torch.zeros(())
    x8, h8 = saved["x8"], saved["h8"]
    for e, (r0, r1) in enumerate(expert_ranges(saved["offsets"])):
        if r1 <= r0:
            continue
        d8, ea3, ea4 = down_dgrad_swiglu(dout[r0:r1], saved["wd"][e], saved["gu8"][r0:r1], s, I)
        dgu8[r0:r1] = d8
        a3, a4 = torch.maximum(a3, ea3), torch.maximum(a4, ea4)
        # train.py:1437-1443: acc / (s3 * q_gu[e]) as bf16
        dx[r0:r1] = ((f(d8) @ f(saved["w8"][e])) / (s[3] * saved["q_gu"][e])).to(torch.bfloat16)
        # train.py:1469-1477: d_gu8^T x8 / (s3 * s0)
        dw_gu[e] = (f(d8).t() @ f(x8[r0:r1])) / (s[3] * s[0])
        # train.py:1519-1529: e5m2(dout * s4)^T h8 / (s4 * s2)
        dq = f(e5m2(f(dout[r0:r1]) * s[4]))
        dw_d[e] = (dq.t() @ f(h8[r0:r1])) / (s[4] * s[2])
    amax[3] = torch.maximum(amax[3], a3)
    amax[4] = torch.maximum(amax[4], a4)
    return (sum_topk_rows(dx, inverse_permutation, top_k), dw_gu, dw_d), dict(dgu8=dgu8, dx=dx)


def route(selected: torch.Tensor, num_experts: int):
    """The expert-order bookkeeping of Experts.forward (train.py:2268-2290):
    (token_index, inverse_permutation, offsets int32, permutation)."""
    top_k = selected.shape[-1]
    flat = selected.reshape(-1)
    sorted_experts, permutation = torch.sort(flat)
    token_index = permutation // top_k
    inverse_permutation = torch.empty_like(permutation)
    inverse_permutation[permutation] = torch.arange(permutation.numel(), device=permutation.device)
    counts = torch.bincount(sorted_experts, minlength=num_experts)
    offsets = torch.cumsum(counts, dim=0).to(torch.int32)
    return token_index, inverse_permutation, offsets, permutation


def combine_topk(rows, sorted_weights, inverse_permutation, top_k):
    """_CombineTopK.forward (train.py:2229-2233): out[t] = sum over the top_k
    slots of w * rows, in the rows' dtype."""
    return sum_topk_rows(rows * sorted_weights.unsqueeze(-1), inverse_permutation, top_k)


def combine_topk_backward(grad_out, sorted_weights, token_index):
    """_CombineTopK.backward's row gradient (train.py:2236-2239)."""
    return grad_out[token_index] * sorted_weights.unsqueeze(-1)


def fp32_experts_reference(x, selected, weights, w_gu, w_d, probe):
    """fp32 autograd of the routed expert MLPs, as in spark-gpt
    tests/test_fp8_mlp.py:90-98: (y, dx, dW_gate_up, dW_down) for upstream
    gradient ``probe``."""
    x32 = x.float().clone().requires_grad_(True)
    wgu = w_gu.detach().float().clone().requires_grad_(True)
    wd = w_d.detach().float().clone().requires_grad_(True)
    y32 = torch.zeros(x.shape[0], w_d.shape[1])
    for s_ in range(selected.shape[1]):
        e = selected[:, s_]
        g, u = torch.einsum("td,tod->to", x32, wgu[e]).chunk(2, dim=-1)
        y32 = y32 + weights[:, s_, None].float() * torch.einsum("ti,tdi->td", torch.nn.functional.silu(g) * u, wd[e])
    grads = torch.autograd.grad((y32 * probe).sum(), [x32, wgu, wd])
    return (y32.detach(),) + tuple(g_.detach() for g_ in grads)
