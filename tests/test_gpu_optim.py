"""GPU parity of the consumer of the MLP's weight gradients: the Muon
momentum stage (spark-gpt train.py:2805-2839) bit for bit against the
reference's two-pass torch update (train.py:2990-2996), and the FP8 weight
gradient fused with it (ops.wgrad_momentum) bit for bit against the weight
gradient followed by the stage."""
import pytest
import torch

import spark_gpt_amd as sg

pytestmark = pytest.mark.gpu


def _torch_stage(g, v, momentum):
    """The reference's torch path (train.py:2991-2994): v.lerp_(g, 1 - m),
    torch.lerp(g, v, m, out=staged) into a bf16 staging matrix."""
    v = v.clone()
    u = torch.empty(g.shape, dtype=torch.bfloat16, device=g.device)
    v.lerp_(g, 1 - momentum)
    torch.lerp(g, v, momentum, out=u)
    return v, u


@pytest.mark.parametrize("momentum", [0.95, 0.9, 0.6, 0.999])
@pytest.mark.parametrize("n", [4, 1 << 20, 6144 * 1024 + 4])
def test_momentum_stage_matches_torch(dev, momentum, n):
    g0 = torch.Generator(device=dev).manual_seed(n % 97)
    g = torch.randn(n, device=dev, generator=g0) * torch.exp2(torch.randint(-20, 20, (n,), device=dev, generator=g0))
    v = torch.randn(n, device=dev, generator=g0) * 1e-3
    rv, ru = _torch_stage(g, v, momentum)
    u = torch.empty(n, dtype=torch.bfloat16, device=dev)
    assert sg._momentum_stage_supported(g, v, u, momentum)
    sg._momentum_stage(g, v, u, momentum)
    assert torch.equal(v, rv)
    assert torch.equal(u, ru)


def test_momentum_stage_predicate(dev):
    g = torch.zeros(8, device=dev)
    u = torch.zeros(8, dtype=torch.bfloat16, device=dev)
    assert sg._momentum_stage_supported(g, g.clone(), u, 0.95)
    assert not sg._momentum_stage_supported(g, g.clone(), u, 0.4)  # 1 - m >= 0.5
    assert not sg._momentum_stage_supported(g, g.clone(), u.float(), 0.95)  # u not bf16
    assert not sg._momentum_stage_supported(g[:6], g[:6].clone(), u[:6], 0.95)  # length % 4
    assert not sg._momentum_stage_supported(g.cpu(), g.cpu(), u.cpu(), 0.95)
    # what the kernel refuses takes the torch path instead of raising:
    # 1 - momentum <= -0.5, and storage offsets that break the alignment
    assert not sg._momentum_stage_supported(g, g.clone(), u, 1.6)
    g12 = torch.zeros(12, device=dev)
    u12 = torch.zeros(12, dtype=torch.bfloat16, device=dev)
    assert not sg._momentum_stage_supported(g12[2:10], g12[:8].clone(), u12[:8], 0.95)  # g at 8 bytes
    assert not sg._momentum_stage_supported(g12[:8], g12[2:10], u12[:8], 0.95)  # v at 8 bytes
    assert not sg._momentum_stage_supported(g12[:8], g12[:8].clone(), u12[2:10], 0.95)  # u at 4 bytes
    assert not sg._momentum_stage_supported(g, g.clone(), u.to("cpu"), 0.95)


def test_momentum_wrappers_reject_bad_state(dev):
    """ops.momentum_stage and ops.wgrad_momentum refuse, with ValueError and
    before any launch, every state tensor of the wrong dtype, size, device or
    alignment (the kernels write fp32 v / grad and packed bf16 u through raw
    pointers)."""
    ops = sg.ops
    M, N, T = 256, 128, 512
    at, bt, sa, sb = _wgrad_operands(dev, M, N, T, 5)
    v0 = torch.zeros(M, N, device=dev)
    u0 = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
    bad_v = (v0.to(torch.bfloat16), v0[:-1], v0.cpu(), torch.zeros(M * N + 4, device=dev)[1:M * N + 1])
    bad_u = (u0.float(), u0[:-1], u0.cpu(), torch.zeros(M * N + 4, dtype=torch.bfloat16, device=dev)[1:M * N + 1])
    sentinel = torch.full((M, N), 7.0, device=dev)
    for v in bad_v:
        with pytest.raises(ValueError):
            ops.wgrad_momentum(at, bt, M, N, sa, sb, v, u0, 0.95)
    for u in bad_u:
        with pytest.raises(ValueError):
            ops.wgrad_momentum(at, bt, M, N, sa, sb, v0, u, 0.95)
    for grad in (torch.zeros(M, N, dtype=torch.bfloat16, device=dev), torch.zeros(M * N // 2, device=dev),
                 torch.zeros(M, N)):
        with pytest.raises(ValueError):
            ops.wgrad_momentum(at, bt, M, N, sa, sb, v0, u0, 0.95, grad=grad)
    for scale in (sa.cpu(), sa.double(), torch.empty(0, device=dev)):
        with pytest.raises(ValueError):
            ops.wgrad_momentum(at, bt, M, N, scale, sb, v0, u0, 0.95)
    with pytest.raises(ValueError):
        ops.wgrad_momentum(at, bt, M, N, sa, sb, v0, u0, 1.6)
    g = sentinel.view(-1)
    for v, u in ((bad_v[0].view(-1), u0.view(-1)), (v0.view(-1)[:-4], u0.view(-1)), (v0.view(-1), bad_u[0].view(-1)),
                 (v0.view(-1).cpu(), u0.view(-1)), (v0.view(-1), bad_u[3])):
        with pytest.raises(ValueError):
            ops.momentum_stage(g, v, u, 0.95)
    torch.cuda.synchronize()
    assert bool((v0 == 0).all()) and bool((u0 == 0).all()) and bool((sentinel == 7.0).all())


def _wgrad_operands(dev, M, N, T, seed):
    ops = sg.ops
    g = torch.Generator(device=dev).manual_seed(seed)
    a = (torch.randn(M, T, device=dev, generator=g) * 4).to(ops.E5M2)
    b = (torch.randn(N, T, device=dev, generator=g) * 4).to(ops.E4M3)
    ldt = ops.ldt_of(T)
    at = torch.zeros(ldt // 64, ops.slab_rows(M), 64, dtype=ops.E5M2, device=dev)
    bt = torch.zeros(ldt // 64, ops.slab_rows(N), 64, dtype=ops.E4M3, device=dev)
    at.view(torch.uint8)[:, :M].copy_(torch.nn.functional.pad(a.view(torch.uint8), (0, ldt - T))
                                      .view(M, ldt // 64, 64).permute(1, 0, 2))
    bt.view(torch.uint8)[:, :N].copy_(torch.nn.functional.pad(b.view(torch.uint8), (0, ldt - T))
                                      .view(N, ldt // 64, 64).permute(1, 0, 2))
    sa = torch.tensor([2.0 ** 6], device=dev)
    sb = torch.tensor([2.0 ** -3], device=dev)
    return at, bt, sa, sb


@pytest.mark.parametrize("M,N,T", [(256, 256, 16384), (768, 320, 1000), (6144, 1024, 4096)])
def test_wgrad_momentum_matches_wgrad_then_stage(dev, M, N, T):
    """Fused == ops.wgrad followed by the momentum stage, bytes equal, with
    and without the gradient output; one split and several."""
    ops = sg.ops
    at, bt, sa, sb = _wgrad_operands(dev, M, N, T, M + T)
    dw = ops.wgrad(at, bt, M, N, sa, sb)
    v0 = torch.randn(M, N, device=dev) * 1e-2
    rv, ru = v0.clone(), torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    ops.momentum_stage(dw.view(-1), rv.view(-1), ru.view(-1), 0.95)
    v, u = v0.clone(), torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    grad = torch.empty(M, N, device=dev)
    ops.wgrad_momentum(at, bt, M, N, sa, sb, v, u, 0.95, grad=grad)
    assert torch.equal(grad, dw)
    assert torch.equal(v, rv) and torch.equal(u, ru)
    v2, u2 = v0.clone(), torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    ops.wgrad_momentum(at, bt, M, N, sa, sb, v2, u2, 0.95)
    assert torch.equal(v2, rv) and torch.equal(u2, ru)
    # the same operands as row K-slabs ([rows/64, ldt, 64], read through
    # transposing LDS reads), in each layout pair the backward can hand over
    a_rows = ops.to_slab(ops.unslab(at, M).t().contiguous())
    b_rows = ops.to_slab(ops.unslab(bt, N).t().contiguous())
    for a8, b8, ar, br in ((a_rows, bt, True, False), (at, b_rows, False, True), (a_rows, b_rows, True, True)):
        v3, u3 = v0.clone(), torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        grad3 = torch.empty(M, N, device=dev)
        ops.wgrad_momentum(a8, b8, M, N, sa, sb, v3, u3, 0.95, grad=grad3, a_rows=ar, b_rows=br)
        assert torch.equal(grad3, dw), (ar, br)
        assert torch.equal(v3, rv) and torch.equal(u3, ru), (ar, br)


def test_wgrad_momentum_zero_tokens(dev):
    """No tokens: the gradient is zero and the stage still runs on it."""
    ops = sg.ops
    M, N = 256, 128
    at = torch.empty(0, ops.slab_rows(M), 64, dtype=ops.E5M2, device=dev)
    bt = torch.empty(0, ops.slab_rows(N), 64, dtype=ops.E4M3, device=dev)
    one = torch.ones(1, device=dev)
    v0 = torch.randn(M, N, device=dev)
    rv, ru = _torch_stage(torch.zeros(M, N, device=dev), v0, 0.9)
    v, u = v0.clone(), torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    ops.wgrad_momentum(at, bt, M, N, one, one, v, u, 0.9)
    assert torch.equal(v, rv) and torch.equal(u, ru)
