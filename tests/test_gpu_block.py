"""GPU parity of the whole FP8 MLP block (the reference's own test, mirrored,
plus the oracle comparison, amax lifecycle and determinism)."""
import pytest
import torch
import torch.nn as nn

import spark_gpt_amd as sg
from oracle import fp8_mlp as O

pytestmark = pytest.mark.gpu


class _Norm(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = 1e-6


def _setup(dev, T, D, I, seed, wstd=None, norm_uniform=True):
    torch.manual_seed(seed)
    norm = _Norm(D)
    mlp = sg.MLP(D, I)
    with torch.no_grad():
        if norm_uniform:
            norm.weight.uniform_(0.5, 1.5)
        if wstd is None:
            mlp.gate_up_proj.weight.normal_(0, D ** -0.5)
            mlp.down_proj.weight.normal_(0, I ** -0.5)
        else:
            mlp.gate_up_proj.weight.normal_(0, wstd)
            mlp.down_proj.weight.normal_(0, wstd)
    norm, mlp = norm.to(dev).train(), mlp.to(dev).train()
    return norm, mlp


def _step(h, probe, norm, mlp):
    params = [norm.weight, mlp.gate_up_proj.weight, mlp.down_proj.weight]
    x = h.clone().requires_grad_(True)
    y = sg._FP8MLPBlock.apply(x, *params, mlp.fp8_scale, mlp.fp8_amax, norm.eps)
    return (y,) + torch.autograd.grad((y.float() * probe).sum(), [x] + params)


def test_fp8_mlp_block_tracks_fp32_reference(dev):
    """Mirror of spark-gpt tests/test_fp8_mlp.py:10-53 (same shapes, init,
    protocol and bound)."""
    torch.manual_seed(0)
    D, I, rows = 256, 768, 1000
    norm, mlp = _setup(dev, rows, D, I, 0, wstd=0.05)
    h = torch.randn(rows, D, device=dev).to(torch.bfloat16)
    probe = torch.randn(rows, D, device=dev)
    _step(h, probe, norm, mlp)  # prewarm: records amax under the initial scales
    assert bool((mlp.fp8_amax > 0).all()), mlp.fp8_amax
    sg.fp8_update_scales(mlp)
    assert bool((mlp.fp8_amax == 0).all())
    out = _step(h, probe, norm, mlp)
    params = [norm.weight, mlp.gate_up_proj.weight, mlp.down_proj.weight]
    ref = O.fp32_reference(h, *params, probe)
    for name, a, r in zip(("mlp out", "dh", "dnorm_w", "dW_gate_up", "dW_down"), out, ref):
        if name == "mlp out":
            a, r = a.float() - h.float(), r - h.float()
        err = O.rel_l2(a.float(), r)
        assert torch.isfinite(a).all(), name
        assert err < 0.12, f"{name}: rel err {err:.3e}"


@pytest.mark.parametrize("T,D,I", [(1000, 256, 768), (257, 128, 384), (2048, 1024, 3072), (8192, 256, 1024),
                                   (300, 8192, 512)])
def test_block_matches_oracle(dev, T, D, I):
    """Same inputs, same delayed scales: every output and grad within rel-L2
    1e-2 of the CPU emulation of the recipe; bit-exact amax slots 0 and 4."""
    norm, mlp = _setup(dev, T, D, I, T + D)
    g = torch.Generator().manual_seed(T)
    h = torch.randn(T, D, generator=g).to(torch.bfloat16)
    dy = (torch.randn(T, D, generator=g) * 1e-3).to(torch.bfloat16)
    params = [norm.weight, mlp.gate_up_proj.weight, mlp.down_proj.weight]

    def gpu():
        x = h.to(dev).requires_grad_(True)
        y = sg._FP8MLPBlock.apply(x, *params, mlp.fp8_scale, mlp.fp8_amax, norm.eps)
        return [y] + list(torch.autograd.grad(y, [x] + params, dy.to(dev)))

    gpu()
    sg.fp8_update_scales(mlp)
    s = mlp.fp8_scale.cpu().clone()
    out = [t.detach().cpu() for t in gpu()]
    a_gpu = mlp.fp8_amax.cpu()
    a_ref = torch.zeros(5)
    cpu_params = [p.detach().cpu() for p in params]
    y, saved = O.block_forward(h, *cpu_params, s.clone(), a_ref, 1e-6)
    grads, _ = O.block_backward(dy, saved, s.clone(), a_ref)
    ref = [y] + list(grads)
    for name, a, r in zip(("y", "dh", "dnorm_w", "dW_gate_up", "dW_down"), out, ref):
        if name == "y":
            a, r = a.float() - h.float(), r.float() - h.float()
        err = O.rel_l2(a.float(), r.float())
        assert torch.isfinite(a.float()).all(), name
        assert err < 1e-2, f"{name}: rel-L2 vs oracle {err:.3e}"
    assert a_gpu[0] == a_ref[0] and a_gpu[4] == a_ref[4]
    torch.testing.assert_close(a_gpu, a_ref, rtol=2e-2, atol=0)
    # every scale a power of two
    m, e = torch.frexp(mlp.fp8_scale.cpu())
    assert torch.all(m == 0.5)


def test_block_zero_tokens(dev):
    """No tokens: empty y and dh, zero weight and norm gradients, amax
    untouched (the reference's sums over zero rows)."""
    D, I = 256, 384
    norm, mlp = _setup(dev, 0, D, I, 3)
    mlp.fp8_amax.fill_(0.5)
    h = torch.empty(0, D, dtype=torch.bfloat16, device=dev)
    probe = torch.empty(0, D, device=dev)
    y, dh, dnw, dwgu, dwd = _step(h, probe, norm, mlp)
    assert y.shape == (0, D) and y.dtype == torch.bfloat16
    assert dh.shape == (0, D) and dh.dtype == torch.bfloat16
    for g, shape in ((dnw, (D,)), (dwgu, (2 * I, D)), (dwd, (D, I))):
        assert g.shape == shape and g.dtype == torch.float32
        assert bool((g == 0).all())
    assert bool((mlp.fp8_amax == 0.5).all())


def test_block_deterministic(dev):
    T, D, I = 1000, 256, 768
    norm, mlp = _setup(dev, T, D, I, 5)
    h = torch.randn(T, D, device=dev).to(torch.bfloat16)
    probe = torch.randn(T, D, device=dev)
    _step(h, probe, norm, mlp)
    sg.fp8_update_scales(mlp)
    s0 = mlp.fp8_scale.clone()
    a = _step(h, probe, norm, mlp)
    amax_a = mlp.fp8_amax.clone()
    mlp.fp8_amax.zero_()
    mlp.fp8_scale.copy_(s0)
    b = _step(h, probe, norm, mlp)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert torch.equal(amax_a, mlp.fp8_amax)


def test_custom_ops_opcheck(dev):
    """Fake implementations of the two operators against real runs (shapes,
    dtypes, strides).  opcheck's schema test perturbs tensors arithmetically,
    which torch does not implement for float8 device tensors, so it is not
    run; the mutation of amax is covered by the compile test below."""
    T, D, I = 300, 256, 384
    norm, mlp = _setup(dev, T, D, I, 21)
    h = torch.randn(T, D, device=dev).to(torch.bfloat16)
    dy = (torch.randn(T, D, device=dev) * 1e-3).to(torch.bfloat16)
    args = (h, norm.weight.detach(), mlp.gate_up_proj.weight.detach(), mlp.down_proj.weight.detach(),
            mlp.fp8_scale, mlp.fp8_amax, norm.eps)
    utils = ("test_faketensor",)
    torch.library.opcheck(torch.ops.sparkfp8.block_fwd.default, args, test_utils=utils)
    out = torch.ops.sparkfp8.block_fwd(*args)
    bargs = (dy, h, norm.weight.detach(), args[2], args[3]) + tuple(out[1:]) + (mlp.fp8_scale, mlp.fp8_amax)
    torch.library.opcheck(torch.ops.sparkfp8.block_bwd.default, bargs, test_utils=utils)


class _Block(nn.Module):
    def __init__(self, norm, mlp):
        super().__init__()
        self.norm, self.mlp = norm, mlp

    def forward(self, h):
        return sg.fp8_mlp_block(h, self.norm, self.mlp)


@pytest.mark.parametrize("backend", ["inductor", "aot_eager"])
def test_compiled_block_matches_eager(dev, backend):
    """torch.compile (train.py:3787, mode="default": the inductor backend)
    traces the block as the two custom operators: no graph break, and the
    same bytes as eager for y, every gradient and the amax slots."""
    T, D, I = 300, 256, 384
    norm, mlp = _setup(dev, T, D, I, 22)
    blk = _Block(norm, mlp)
    h = torch.randn(T, D, device=dev).to(torch.bfloat16)
    dy = (torch.randn(T, D, device=dev) * 1e-3).to(torch.bfloat16)
    mlp.fp8_scale.copy_(torch.tensor([16.0, 2.0 ** -6, 64.0, 2.0 ** 10, 2.0 ** 15], device=dev))

    def run(m):
        mlp.fp8_amax.zero_()
        for p in blk.parameters():
            p.grad = None
        x = h.clone().requires_grad_(True)
        y = m(x)
        y.backward(dy)
        return [y.detach(), x.grad] + [p.grad.clone() for p in blk.parameters()] + [mlp.fp8_amax.clone()]

    ref = run(blk)
    explain = torch._dynamo.explain(blk)(h.clone().requires_grad_(True))
    assert explain.graph_break_count == 0, explain.break_reasons
    torch._dynamo.reset()
    cblk = torch.compile(blk, backend=backend, mode="default" if backend == "inductor" else None, dynamic=False)
    for _ in range(2):  # the second call runs the cached compiled graphs
        got = run(cblk)
        for a, b in zip(got, ref):
            assert torch.equal(a, b)
    torch._dynamo.reset()


def _count_weight_quant(monkeypatch):
    """Counts weight quantizations: one per weight_quant call, two per
    block_weight_quant call (both masters of a block)."""
    calls = []
    real = sg.ops.weight_quant
    real_pair = sg.ops.block_weight_quant

    def counted(*a, **k):
        calls.append(a[0].shape)
        return real(*a, **k)

    def counted_pair(*a, **k):
        calls.extend([a[0].shape, a[1].shape])
        return real_pair(*a, **k)

    monkeypatch.setattr(sg.ops, "weight_quant", counted)
    monkeypatch.setattr(sg.ops, "block_weight_quant", counted_pair)
    return calls


def test_weight_cache_reuses_quantization(dev, monkeypatch):
    """Forwards after the first launch no weight quantization while the
    masters are unchanged; the block's outputs and gradients are the bytes of
    the per-forward quantization (the reference's behaviour, cache off); an
    optimizer write that moves no version counter is picked up by
    fp8_update_scales, one that does by the next forward."""
    from spark_gpt_amd import torch_ops as TO

    T, D, I = 1000, 256, 768
    norm, mlp = _setup(dev, T, D, I, 31)
    h = torch.randn(T, D, device=dev).to(torch.bfloat16)
    probe = torch.randn(T, D, device=dev)
    TO.clear_weight_cache()
    calls = _count_weight_quant(monkeypatch)
    _step(h, probe, norm, mlp)
    assert len(calls) == 2
    sg.fp8_update_scales(mlp)  # re-quantizes the cached masters (2 launches)
    assert len(calls) == 4
    s0 = mlp.fp8_scale.clone()

    def fresh_run(cache):
        mlp.fp8_amax.zero_()
        mlp.fp8_scale.copy_(s0)
        monkeypatch.setattr(TO, "FP8_WEIGHT_CACHE", cache)
        out = _step(h, probe, norm, mlp)
        return out, mlp.fp8_amax.clone()

    n = len(calls)
    cached, a1 = fresh_run(True)
    cached2, _ = fresh_run(True)
    assert len(calls) == n  # neither forward nor backward quantized
    per_fwd, a2 = fresh_run(False)
    assert len(calls) == n + 4  # forward 2, backward 2
    for x, y, z in zip(cached, cached2, per_fwd):
        assert torch.equal(x, y) and torch.equal(x, z)
    assert torch.equal(a1, a2)
    monkeypatch.setattr(TO, "FP8_WEIGHT_CACHE", True)
    # an in-place update moves the version counter: the next forward re-quantizes
    w = mlp.gate_up_proj.weight
    with torch.no_grad():
        w.mul_(0.5)
    n = len(calls)
    halved, _ = fresh_run(True)
    assert len(calls) == n + 2
    assert not torch.equal(halved[0], cached[0])
    # a write that bypasses the version counter (as an optimizer writing
    # through raw pointers): fp8_update_scales re-quantizes
    w.data.mul_(2.0)
    sg.fp8_update_scales(mlp)
    back, a3 = fresh_run(True)
    for x, y in zip(back, cached):
        assert torch.equal(x, y)
    assert torch.equal(a3, a1)
    TO.clear_weight_cache()


def _rmsnorm_ref(x, weight, eps):
    """spark-gpt's RMSNorm (train.py:166-168): fp32 statistics, output in x's dtype."""
    out = x.float() * torch.rsqrt(x.float().pow(2).mean(dim=-1, keepdim=True) + eps)
    return out.to(dtype=x.dtype) * weight.to(dtype=x.dtype)


@pytest.mark.parametrize("T,D,I", [(4096, 1024, 3072)])
def test_block_vs_bf16_mlp(dev, T, D, I, capsys):
    """The FP8 block against an independent bf16 MLP for the same sub-block
    (train.py:2370-2374: RMSNorm, then the MLP under bf16 autocast, plus the
    residual), same weights and upstream gradient.  The comparator is the
    reference's unfused torch branch of MLP.forward (train.py:260-261:
    gate_up_proj, chunk, F.silu(gate) * up, down_proj) on torch's own
    matmuls and autograd, so no kernel of this library is on its path.  The
    FP8 recipe differs from bf16 by its e4m3/e5m2 roundings: the reference
    measured 5-8 % per element (CHANGES.md:372-373); rel-L2 here stays under
    the reference test's 0.12 bound, and each number is printed for the
    record."""
    norm, mlp = _setup(dev, T, D, I, 41)
    g = torch.Generator(device=dev).manual_seed(42)
    h = torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16)
    dy = (torch.randn(T, D, generator=g, device=dev) * 1e-3).to(torch.bfloat16)
    params = [norm.weight, mlp.gate_up_proj.weight, mlp.down_proj.weight]

    def fp8():
        x = h.clone().requires_grad_(True)
        y = sg._FP8MLPBlock.apply(x, *params, mlp.fp8_scale, mlp.fp8_amax, norm.eps)
        return [y] + list(torch.autograd.grad(y, [x] + params, dy))

    fp8()
    sg.fp8_update_scales(mlp)
    got = fp8()
    x = h.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        gate, up = mlp.gate_up_proj(_rmsnorm_ref(x, norm.weight, norm.eps)).chunk(2, dim=-1)
        y = x + mlp.down_proj(torch.nn.functional.silu(gate) * up)
    ref = [y] + list(torch.autograd.grad(y, [x] + params, dy))
    errs = {}
    for name, a, r in zip(("y - h", "dh", "dnorm_w", "dW_gate_up", "dW_down"), got, ref):
        a, r = a.float(), r.float()
        if name == "y - h":
            a, r = a - h.float(), r - h.float()
        errs[name] = O.rel_l2(a, r)
    with capsys.disabled():
        print("\nrel-L2 of the FP8 block vs the bf16 MLP:", {k: round(v, 4) for k, v in errs.items()})
    for name, e in errs.items():
        assert e < 0.12, (name, e)
