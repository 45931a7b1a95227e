"""GPU parity of the FP8 MoE experts (_FP8Experts, train.py:1543-1605): the
device-built plan, the gather + e4m3 quantization (bit-exact), the grouped
layer against the oracle (oracle/fp8_moe.py) on the same scales, the mirror of
the reference's own test (tests/test_fp8_mlp.py:57-109: vs an fp32 autograd of
the routed experts, an expert without tokens gets exactly zero gradients),
determinism and the expert weight cache."""
import pytest
import torch
import torch.nn as nn

import spark_gpt_amd as sg
from oracle import fp8_mlp as O
from oracle import fp8_moe as M

pytestmark = pytest.mark.gpu
E4 = torch.float8_e4m3fn


class _Experts(nn.Module):
    """The reference's packed experts (train.py:2244-2260): parameters and fp8
    buffers, and the FP8 branch of its forward (train.py:2268-2299)."""

    def __init__(self, E, D, I):
        super().__init__()
        self.num_experts, self.hidden_dim, self.intermediate_dim = E, D, I
        self.gate_up_proj = nn.Parameter(torch.empty(E, 2 * I, D))
        self.down_proj = nn.Parameter(torch.empty(E, D, I))
        self.register_buffer("fp8_scale", torch.ones(5), persistent=False)
        self.register_buffer("fp8_amax", torch.zeros(5), persistent=False)

    def forward(self, x, selected, weights):
        T, k = x.shape[0], selected.shape[-1]
        tok, inv, offsets, perm = M.route(selected, self.num_experts)
        sw = weights.reshape(-1)[perm]
        rows = sg._FP8Experts.apply(x, self.gate_up_proj, self.down_proj, tok, inv, offsets, k, self.fp8_scale,
                                    self.fp8_amax)
        return M.combine_topk(rows, sw, inv, k)


def _u8(t):
    return t.contiguous().view(torch.uint8).cpu()


def _padded_rows(offsets, ldp):
    """expert-order row of each padded row (-1: padding), as the plan lays them out."""
    out = torch.full((ldp,), -1, dtype=torch.int64)
    p = 0
    for e, (r0, r1) in enumerate(M.expert_ranges(offsets.cpu())):
        n = r1 - r0
        out[p:p + n] = torch.arange(r0, r1)
        p += -(-n // 256) * 256
    return out


def test_plan_matches_routing(dev):
    E, R = 6, 1000
    counts = torch.tensor([300, 0, 513, 1, 0, 186])
    offsets = torch.cumsum(counts, 0).to(torch.int32)
    plan = sg.ops.moe_plan(offsets.to(dev), R).cpu()
    tiles = []
    ps = 0
    for e, c in enumerate(counts.tolist()):
        assert plan[8 + e] == ps and plan[8 + E + e] == -(-c // 256) * 256
        u0 = int(offsets[e]) - c
        for j in range(-(-c // 256)):
            tiles.append((e, u0 + 256 * j, min(256, c - 256 * j)))
        ps += -(-c // 256) * 256
    assert int(plan[0]) == len(tiles) and int(plan[1]) == E
    got = plan[8 + 2 * E: 8 + 2 * E + 3 * len(tiles)].view(-1, 3)
    assert got.tolist() == [list(t) for t in tiles]


@pytest.mark.parametrize("D", [1024, 384, 640, 2560])
def test_gather_quant_bit_exact(dev, D):
    """x gathered and quantized: one column chunk (384), whole chunks (1024,
    2560) and a ragged last chunk (640)."""
    T, E, k = 700, 5, 2
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(T, D, generator=g) * 3).to(torch.bfloat16)
    x[7, 5] = float("nan")
    selected = torch.stack([torch.randint(0, E, (T,), generator=g), torch.randint(0, E, (T,), generator=g)], 1)
    tok, inv, offsets, _ = M.route(selected, E)
    R = tok.numel()
    plan = sg.ops.moe_plan(offsets.to(dev), R)
    ldp = sg.ops.moe_padded_rows(R, E)
    scale = torch.tensor([16.0, 1, 1, 1, 1], device=dev)
    amax = torch.zeros(5, device=dev)
    x8, x8t = sg.ops.moe_rows_quant(x.to(dev), tok.to(dev), plan, ldp, scale, 0, amax, 0, sg.ops.FMT_E4M3, True)
    ref = _u8(O.e4m3(x[tok].float() * 16.0))
    rows = _padded_rows(offsets, ldp)
    got = _u8(sg.ops.unslab(x8, ldp))
    gt = _u8(sg.ops.unslab(x8t, D))
    valid = rows >= 0
    assert torch.equal(got[valid], ref[rows[valid]])
    assert torch.all(got[~valid] == 0) and torch.all(gt[:, ~valid] == 0)
    assert torch.equal(gt.t(), got)
    finite = x[tok].float().abs()
    assert amax[0].item() == finite[~torch.isnan(finite)].max().item()
    # the row K-slab alone (no token-contiguous copy): the same bytes and amax
    amax2 = torch.zeros(5, device=dev)
    x8b, none = sg.ops.moe_rows_quant(x.to(dev), tok.to(dev), plan, ldp, scale, 0, amax2, 0, sg.ops.FMT_E4M3, True,
                                      False)
    assert none is None and torch.equal(_u8(x8b), _u8(x8)) and torch.equal(amax2, amax)


def test_dout_quant_e5m2_bit_exact(dev):
    """The e5m2 form (no gather, no row copy): dout rows of the caller's expert
    order to the token-contiguous K-slab over padded expert order, amax of
    |dout| in slot 4, saturating values clamped to +-57344."""
    E, D = 3, 512
    counts = torch.tensor([300, 0, 77])
    offsets = torch.cumsum(counts, 0).to(torch.int32)
    R = int(counts.sum())
    g = torch.Generator().manual_seed(4)
    dout = (torch.randn(R, D, generator=g) * 1e-3).to(torch.bfloat16)
    dout[5, :3] = torch.tensor([1.0, -1.0, 0.25]).to(torch.bfloat16)  # x scale 2^16: clamps
    plan = sg.ops.moe_plan(offsets.to(dev), R)
    ldp = sg.ops.moe_padded_rows(R, E)
    scale = torch.tensor([1, 1, 1, 1, 2.0 ** 16], device=dev)
    amax = torch.zeros(5, device=dev)
    xs, xt = sg.ops.moe_rows_quant(dout.to(dev), None, plan, ldp, scale, 4, amax, 4, sg.ops.FMT_E5M2, False)
    assert xs is None
    ref = _u8(O.e5m2(dout.float() * 2.0 ** 16))
    rows = _padded_rows(offsets, ldp)
    gt = _u8(sg.ops.unslab(xt, D))
    valid = rows >= 0
    assert torch.equal(gt.t()[valid], ref[rows[valid]])
    assert torch.all(gt[:, ~valid] == 0)
    assert amax[4].item() == dout.float().abs().max().item() and amax[:4].sum().item() == 0


@pytest.mark.parametrize("M_,N_,counts", [(1536, 1024, [300, 0, 513, 1, 0, 186]), (1024, 768, [4000, 2600, 0, 900]),
                                           (256, 320, [70])])
def test_moe_wgrad_rows_equals_token_contiguous(dev, M_, N_, counts):
    """The grouped weight gradient with row K-slab operands (transposing LDS
    reads) gives the bytes of the one on token-contiguous copies, in every
    layout pair; experts without rows get zeros."""
    ops = sg.ops
    counts = torch.tensor(counts)
    E = counts.numel()
    offsets = torch.cumsum(counts, 0).to(torch.int32)
    R = int(counts.sum())
    plan = ops.moe_plan(offsets.to(dev), R)
    ldp = ops.moe_padded_rows(R, E)
    rows = _padded_rows(offsets, ldp).to(dev)
    g = torch.Generator(device=dev).manual_seed(M_ + N_ + R)
    a = (torch.randn(ldp, M_, device=dev, generator=g) * 8).to(ops.E5M2)
    b = (torch.randn(ldp, N_, device=dev, generator=g) * 8).to(ops.E4M3)
    a.view(torch.uint8)[rows < 0] = 0  # padding rows are zeros, as the producers write them
    b.view(torch.uint8)[rows < 0] = 0
    a_rows, b_rows = ops.to_slab(a), ops.to_slab(b)                                # [cols/64, ldp, 64]
    a_t, b_t = ops.to_slab(a.t().contiguous()), ops.to_slab(b.t().contiguous())    # [ldp/64, cols, 64]
    sa = torch.tensor([2.0 ** 4], device=dev)
    sb = torch.tensor([2.0 ** -2], device=dev)
    ref = ops.moe_wgrad(a_t, b_t, M_, N_, E, plan, sa, sb)
    assert torch.equal(ops.moe_wgrad_rows(a_rows, b_rows, M_, N_, E, plan, sa, sb), ref)
    assert torch.equal(ops.moe_wgrad_rows(a_rows, b_t, M_, N_, E, plan, sa, sb, b_rows=False), ref)
    assert torch.equal(ops.moe_wgrad_rows(a_t, b_rows, M_, N_, E, plan, sa, sb, a_rows=False), ref)
    for e in range(E):
        if int(counts[e]) == 0:
            assert torch.all(ref[e] == 0)


@pytest.mark.parametrize("I,counts", [(256, [700, 0, 1500, 1, 2049]), (1536, [3000, 257, 0, 5000]),
                                      (1536, [16476, 16579, 16396, 16215, 16245, 16370, 16368, 16423])])
def test_moe_swiglu_pipe_equals_dense_per_expert(dev, I, counts):
    """At D = 1024 the grouped gate/up forward runs the persistent SwiGLU
    pipe over the plan's tiles, changing expert (weights and scale) from
    tile to tile: each expert's gu8 and h8 rows are the bytes the dense
    forward gives for that expert's rows alone, padding rows stay zero, and
    amax slots 1, 2 are the maxima of the per-expert amax.  The last case is
    the MoE workload's full size (131 072 routed rows over 8 experts: about
    49 tiles per work-group of the persistent kernel)."""
    ops = sg.ops
    D = 1024
    counts = torch.tensor(counts)
    E = counts.numel()
    offsets = torch.cumsum(counts, 0).to(torch.int32)
    R = int(counts.sum())
    plan = ops.moe_plan(offsets.to(dev), R)
    ldp = ops.moe_padded_rows(R, E)
    g = torch.Generator(device=dev).manual_seed(I + R)
    x = (torch.randn(R, D, device=dev, generator=g) * 2).to(torch.bfloat16)
    w = torch.randn(E, 2 * I, D, device=dev, generator=g) * 0.03
    w[1] *= 4.0  # experts with different weight scales
    scale = torch.tensor([4.0, 2.0 ** -3, 2.0 ** -2, 1.0, 1.0], device=dev)
    amax = torch.zeros(5, device=dev)
    xs, _ = ops.moe_rows_quant(x, None, plan, ldp, scale, 0, amax, 0, ops.FMT_E4M3, True, with_copy=False)
    q = torch.empty(E, device=dev)
    w8, _, _ = ops.weight_quant_experts(w, q)
    gu8, h8, _ = ops.moe_gateup_swiglu_fwd(xs, w8, plan, scale, q, amax, I, copy=False)
    torch.cuda.synchronize()
    gu_rows, h_rows = ops.unslab(gu8, ldp), ops.unslab(h8, ldp)  # [ldp, 2I], [ldp, I] (padded order)
    a1 = a2 = 0.0
    p = 0
    for e in range(E):
        n = int(counts[e])
        if n == 0:
            continue
        npad = -(-n // 256) * 256
        x8e = xs[:, p:p + npad, :].contiguous()  # the expert's K-slab over its padded rows
        ae = torch.zeros(5, device=dev)
        gue, he, _ = ops.gateup_swiglu_fwd(x8e, w8[e], scale, q[e:e + 1], ae, n, I, copy=False)
        torch.cuda.synchronize()
        assert torch.equal(gu_rows[p:p + n].view(torch.uint8), ops.unslab(gue, n).view(torch.uint8)), e
        assert torch.equal(h_rows[p:p + n].view(torch.uint8), ops.unslab(he, n).view(torch.uint8)), e
        assert torch.all(gu_rows[p + n:p + npad].view(torch.uint8) == 0), e
        a1, a2 = max(a1, float(ae[1])), max(a2, float(ae[2]))
        p += npad
    assert float(amax[1]) == a1 and float(amax[2]) == a2


def _make(dev, E, D, I, seed, std=None):
    ex = _Experts(E, D, I)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        ex.gate_up_proj.copy_(torch.randn(E, 2 * I, D, generator=g) * (std or D ** -0.5))
        ex.down_proj.copy_(torch.randn(E, D, I, generator=g) * (std or I ** -0.5))
    return ex.to(dev).train()


def _gpu_step(ex, x, selected, weights, probe):
    xx = x.clone().requires_grad_(True)
    out = ex(xx, selected, weights)
    grads = torch.autograd.grad((out.float() * probe).sum(), [xx, ex.gate_up_proj, ex.down_proj])
    return [out.detach()] + list(grads)


def test_fp8_experts_track_fp32_reference(dev):
    """Mirror of spark-gpt tests/test_fp8_mlp.py:57-109 (same shapes, init,
    routing, protocol and bound), plus exactly-zero gradients of the expert
    that gets no tokens."""
    torch.manual_seed(0)
    E, D, I, T, k = 4, 256, 128, 500, 2
    ex = _make(dev, E, D, I, 0, std=0.05)
    x = torch.randn(T, D, device=dev).to(torch.bfloat16)
    choices = torch.tensor([[0, 1], [1, 3], [0, 3]], device=dev)  # expert 2 gets no tokens
    selected = choices[torch.randint(0, 3, (T,), device=dev)]
    weights = torch.softmax(torch.randn(T, k, device=dev), -1).to(torch.bfloat16)
    probe = torch.randn(T, D, device=dev)
    _gpu_step(ex, x, selected, weights, probe)
    assert bool((ex.fp8_amax > 0).all()), ex.fp8_amax
    sg.fp8_update_scales(ex)
    assert bool((ex.fp8_amax == 0).all())
    out = _gpu_step(ex, x, selected, weights, probe)
    ref = M.fp32_experts_reference(x.cpu(), selected.cpu(), weights.cpu(), ex.gate_up_proj.cpu(),
                                   ex.down_proj.cpu(), probe.cpu())
    for name, a, r in zip(("out", "dx", "dW_gate_up", "dW_down"), out, ref):
        a = a.float().cpu()
        assert torch.isfinite(a).all(), name
        assert O.rel_l2(a, r) < 0.12, name
    assert bool((out[2][2] == 0).all()) and bool((out[3][2] == 0).all())  # unused expert


@pytest.mark.parametrize("T,D,I,E,k,skew", [(500, 256, 128, 4, 2, False), (4096, 1024, 256, 8, 2, True),
                                            (300, 128, 384, 3, 1, False), (65536, 1024, 1536, 8, 2, False)])
def test_moe_matches_oracle(dev, T, D, I, E, k, skew):
    """Same inputs and scales: every output and gradient within rel-L2 1e-2 of
    the oracle; amax slots 0 and 4 bit-exact.  `skew` routes half of the
    tokens' first slot to expert 0 (the imbalance spark-gpt sees in
    practice).  The last case is the MoE workload's full size (65536 tokens
    top-2 of 8 experts, D=1024, I=1536: about 16.4k rows per expert), forward
    and backward."""
    ex = _make(dev, E, D, I, T + E)
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, D, generator=g).to(torch.bfloat16)
    sel = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    if skew:
        sel[: T // 2, 0] = 0
        sel[: T // 2, 1] = torch.randint(1, E, (T // 2,), generator=g)
    weights = torch.softmax(torch.randn(T, k, generator=g), -1).to(torch.bfloat16)
    probe = torch.randn(T, D, generator=g) * 1e-2
    args = (x.to(dev), sel.to(dev), weights.to(dev), probe.to(dev))
    _gpu_step(ex, *args)
    sg.fp8_update_scales(ex)
    s = ex.fp8_scale.cpu().clone()
    out = [t.cpu() for t in _gpu_step(ex, *args)]
    a_gpu = ex.fp8_amax.cpu()
    a_ref = torch.zeros(5)
    tok, inv, offsets, perm = M.route(sel, E)
    sw = weights.reshape(-1)[perm]
    rows, saved = M.moe_forward(x, ex.gate_up_proj.detach().cpu(), ex.down_proj.detach().cpu(), tok, offsets,
                                s.clone(), a_ref)
    y = M.combine_topk(rows, sw, inv, k)
    d_rows = M.combine_topk_backward(probe.to(torch.bfloat16), sw, tok)
    (dx, dwgu, dwd), _ = M.moe_backward(d_rows, saved, s.clone(), a_ref, inv, k)
    for name, a, r in zip(("out", "dx", "dW_gate_up", "dW_down"), out, (y, dx, dwgu, dwd)):
        assert torch.isfinite(a.float()).all(), name
        assert O.rel_l2(a.float(), r.float()) < 1e-2, name
    assert a_gpu[0] == a_ref[0] and a_gpu[4] == a_ref[4]
    torch.testing.assert_close(a_gpu, a_ref, rtol=2e-2, atol=0)


def test_moe_deterministic(dev):
    E, D, I, T, k = 4, 512, 256, 1000, 2
    ex = _make(dev, E, D, I, 9)
    x = torch.randn(T, D, device=dev).to(torch.bfloat16)
    sel = torch.stack([torch.randperm(E)[:k] for _ in range(T)]).to(dev)
    weights = torch.softmax(torch.randn(T, k, device=dev), -1).to(torch.bfloat16)
    probe = torch.randn(T, D, device=dev)
    _gpu_step(ex, x, sel, weights, probe)
    sg.fp8_update_scales(ex)
    s0 = ex.fp8_scale.clone()
    a = _gpu_step(ex, x, sel, weights, probe)
    am = ex.fp8_amax.clone()
    ex.fp8_amax.zero_()
    ex.fp8_scale.copy_(s0)
    b = _gpu_step(ex, x, sel, weights, probe)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    assert torch.equal(am, ex.fp8_amax)


def test_moe_weight_cache_refresh(dev, monkeypatch):
    """The expert copies are quantized once per optimizer step: forwards after
    the first launch no weight quantization, fp8_update_scales re-quantizes
    (an optimizer may write the masters through raw pointers), and the bytes
    equal a per-forward quantization."""
    from spark_gpt_amd import torch_ops as TO

    E, D, I, T, k = 4, 256, 128, 300, 2
    ex = _make(dev, E, D, I, 12)
    x = torch.randn(T, D, device=dev).to(torch.bfloat16)
    sel = torch.stack([torch.randperm(E)[:k] for _ in range(T)]).to(dev)
    weights = torch.softmax(torch.randn(T, k, device=dev), -1).to(torch.bfloat16)
    probe = torch.randn(T, D, device=dev)
    calls = []
    real = sg.ops.weight_quant_experts
    monkeypatch.setattr(sg.ops, "weight_quant_experts", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    TO.clear_weight_cache()
    _gpu_step(ex, x, sel, weights, probe)
    assert len(calls) == 2
    sg.fp8_update_scales(ex)
    assert len(calls) == 4
    s0 = ex.fp8_scale.clone()

    def run(cache):
        ex.fp8_amax.zero_()
        ex.fp8_scale.copy_(s0)
        monkeypatch.setattr(TO, "FP8_WEIGHT_CACHE", cache)
        return _gpu_step(ex, x, sel, weights, probe)

    n = len(calls)
    cached = run(True)
    assert len(calls) == n
    fresh = run(False)
    for u, v in zip(cached, fresh):
        assert torch.equal(u, v)
    monkeypatch.setattr(TO, "FP8_WEIGHT_CACHE", True)
    ex.gate_up_proj.data.mul_(0.5)  # bypasses the version counter
    sg.fp8_update_scales(ex)
    halved = run(True)
    assert not torch.equal(halved[0], cached[0])
    TO.clear_weight_cache()
