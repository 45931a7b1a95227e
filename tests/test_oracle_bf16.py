"""CPU pins of the bf16 SwiGLU oracle (oracle/bf16_swiglu.py).

Each path is checked against an fp32 autograd of the function it computes
(the mathematics fixes the gradient): _NormSwiGLU with the reference test's
shapes and protocol (spark-gpt tests/test_moe.py:468-517) and _FusedSwiGLU
dense and grouped with an empty group (tests/test_moe.py:385-423, its bound
0.05 * scale + 1e-3).  Planted mistakes -- a dropped term of the norm
backward, gate and up swapped in the SwiGLU gradient, the norm weight left
out of the weight fold, a group's gradient given to another -- must fail
the same bounds."""
import pytest
import torch

from oracle import bf16_swiglu as B
from oracle import fp8_mlp as O


def _norm_case(hidden, rows=1000, inter=768, seed=0):
    g = torch.Generator().manual_seed(seed)
    norm_w = torch.rand(hidden, generator=g) + 0.5  # uniform(0.5, 1.5), tests/test_moe.py:474
    w_gu = torch.randn(2 * inter, hidden, generator=g) * hidden ** -0.5
    h = (torch.randn(rows, hidden, generator=g) * 3.0).to(torch.bfloat16)
    probe = torch.randn(rows, inter, generator=g)
    return h, norm_w, w_gu, probe


def _norm_oracle(h, norm_w, w_gu, probe, eps=1e-6, planted=None):
    out, saved = B.norm_swiglu_forward(h, norm_w, w_gu, eps)
    if planted == "no_fold":
        saved["wp"] = B.bf(w_gu.float())
    dh, dnw, dw = B.norm_swiglu_backward(probe.to(torch.bfloat16), saved)
    if planted == "no_coef":
        gu, rstd = saved["gu"], saved["rstd"]
        I = gu.shape[1] // 2
        dg, du = B.swiglu_grad(gu[:, :I], gu[:, I:], probe * rstd[:, None])
        dh = B.bf(torch.cat([dg, du], 1) @ saved["wp"]).to(torch.bfloat16)
    return out.float(), dh.float(), dnw, dw


@pytest.mark.parametrize("hidden", [512, 1024])
def test_norm_swiglu_oracle_tracks_fp32(hidden):
    h, norm_w, w_gu, probe = _norm_case(hidden)
    ref = B.fp32_norm_swiglu(h, norm_w, w_gu, 1e-6, probe)
    got = _norm_oracle(h, norm_w, w_gu, probe)
    for name, a, r in zip(("out", "dh", "dnorm_w", "dw_gu"), got, ref):
        err = O.rel_l2(a, r)
        assert err < 2e-2, (hidden, name, err)


@pytest.mark.parametrize("planted", ["no_fold", "no_coef"])
def test_norm_swiglu_oracle_planted_mistakes_fail(planted):
    h, norm_w, w_gu, probe = _norm_case(512)
    ref = B.fp32_norm_swiglu(h, norm_w, w_gu, 1e-6, probe)
    got = _norm_oracle(h, norm_w, w_gu, probe, planted=planted)
    assert max(O.rel_l2(a, r) for a, r in zip(got, ref)) > 5e-2


def test_swiglu_grad_is_the_derivative():
    """d_gate, d_up of _swiglu_tiles against fp64 autograd of silu(g) * u."""
    g = torch.Generator().manual_seed(1)
    gate = torch.randn(4096, generator=g, dtype=torch.float64) * 4
    up = torch.randn(4096, generator=g, dtype=torch.float64)
    dh = torch.randn(4096, generator=g, dtype=torch.float64)
    gg, uu = gate.clone().requires_grad_(True), up.clone().requires_grad_(True)
    dg_ref, du_ref = torch.autograd.grad((torch.nn.functional.silu(gg) * uu * dh).sum(), [gg, uu])
    dg, du = B.swiglu_grad(gate.float(), up.float(), dh.float())
    # bf16 rounding: half an ulp (2^-9 relative) plus fp32 noise
    assert torch.all((dg.double() - dg_ref).abs() <= 2.0 ** -8 * dg_ref.abs() + 1e-30)
    assert torch.all((du.double() - du_ref).abs() <= 2.0 ** -8 * du_ref.abs() + 1e-30)
    swapped = B.swiglu_grad(up.float(), gate.float(), dh.float())[0]
    assert not torch.all((swapped.double() - dg_ref).abs() <= 2.0 ** -8 * dg_ref.abs() + 1e-30)


def _fused_case(counts, rows=1000, dim=128, inter=192, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, dim, generator=g).to(torch.bfloat16)
    probe = torch.randn(rows, inter, generator=g).to(torch.bfloat16)
    w = (torch.randn(len(counts), 2 * inter, dim, generator=g) * 0.05).to(torch.bfloat16)
    offs = torch.cumsum(torch.tensor(counts), 0).to(torch.int32)
    return x, w, offs, probe


@pytest.mark.parametrize("counts", [[1000], [300, 0, 700]])
def test_fused_swiglu_oracle_tracks_fp32(counts):
    x, w, offs, probe = _fused_case(counts)
    h, gu = B.fused_swiglu_forward(x, w, offs)
    dx, dw = B.fused_swiglu_backward(probe, x, w, gu, offs)
    rh, rx, rw = B.fp32_fused_swiglu(x, w, offs, probe)
    for name, a, r in (("h", h, rh), ("dx", dx, rx), ("dw", dw, rw)):
        err = (a.float() - r).abs().max().item()
        assert err < 0.05 * r.abs().max().item() + 1e-3, (name, err)
    if len(counts) > 1:
        assert torch.all(dw[1] == 0)


def test_fused_swiglu_oracle_planted_group_swap_fails():
    x, w, offs, probe = _fused_case([300, 0, 700])
    h, gu = B.fused_swiglu_forward(x, w, offs)
    dx, dw = B.fused_swiglu_backward(probe, x, w, gu, offs)
    rh, rx, rw = B.fp32_fused_swiglu(x, w, offs, probe)
    bad = dw.flip(0)
    assert (bad.float() - rw).abs().max().item() > 0.05 * rw.abs().max().item() + 1e-3
