"""GPU parity: norm-fused quantizer (bit-exact) and norm backward."""
import pytest
import torch

import spark_gpt_amd as sg
from oracle import fp8_mlp as O

pytestmark = pytest.mark.gpu


def u8(t):
    return t.contiguous().view(torch.uint8).cpu()


CASES = [(1, 128), (257, 256), (1000, 256), (333, 512), (1000, 1024), (4099, 1024), (300, 2048),
         (200, 4096), (300, 8192), (1, 8192), (129, 16384)]


@pytest.mark.parametrize("T,D", CASES)
def test_norm_quant_bit_exact(dev, T, D):
    g = torch.Generator().manual_seed(T + D)
    h = (torch.randn(T, D, generator=g) * 3).to(torch.bfloat16)
    nw = torch.empty(D).uniform_(0.5, 1.5, generator=g)
    s0 = 16.0
    scale = torch.tensor([s0, 1, 1, 1, 1], device=dev)
    amax = torch.zeros(5, device=dev)
    x8, x8t, rstd = sg.ops.norm_quant(h.to(dev), nw.to(dev), scale, amax, 1e-6)
    r8, r8t, rr, ra = O.norm_quant(h, nw, torch.tensor(s0), 1e-6)
    assert torch.equal(rstd.cpu(), rr)
    ldt = sg.ops.ldt_of(T)
    assert x8.shape == (D // 64, ldt, 64)
    assert torch.equal(u8(sg.ops.unslab(x8, T)), u8(r8))
    assert torch.all(u8(sg.ops.unslab(x8, ldt))[T:] == 0)
    assert x8t.shape == (ldt // 64, sg.ops.slab_rows(D), 64)
    xt = u8(sg.ops.unslab(x8t, D))
    assert torch.equal(xt[:, :T], u8(r8t))
    assert torch.all(xt[:, T:] == 0)
    assert amax[0].item() == ra.item()
    # without the token-contiguous copy: the same x8 (padding included), rstd and amax
    amax2 = torch.zeros(5, device=dev)
    x8b, none, rstd2 = sg.ops.norm_quant(h.to(dev), nw.to(dev), scale, amax2, 1e-6, copy=False)
    assert none is None
    assert torch.equal(u8(x8b), u8(x8)) and torch.equal(rstd2, rstd) and torch.equal(amax2, amax)


def test_norm_quant_heavy_tails(dev):
    """Student-t(3) activations: saturation at +-448 and tiny values."""
    T, D = 2048, 2048
    g = torch.Generator().manual_seed(11)
    z = torch.randn(T, D, generator=g)
    chi = (torch.randn(T, D, 3, generator=g) ** 2).sum(-1)  # chi-square, 3 dof
    h = (z / torch.sqrt(chi / 3)).to(torch.bfloat16)
    nw = torch.ones(D)
    scale = torch.tensor([64.0, 1, 1, 1, 1], device=dev)
    amax = torch.zeros(5, device=dev)
    x8, x8t, rstd = sg.ops.norm_quant(h.to(dev), nw.to(dev), scale, amax, 1e-6)
    r8, r8t, rr, ra = O.norm_quant(h, nw, torch.tensor(64.0), 1e-6)
    assert torch.equal(rstd.cpu(), rr)
    assert torch.equal(u8(sg.ops.unslab(x8, T)), u8(r8))
    assert amax[0].item() == ra.item()
    assert (u8(r8) & 0x7F).eq(0x7E).any()  # some saturate


@pytest.mark.parametrize("T,D", [(1000, 256), (257, 1024), (4099, 1024), (300, 4096), (300, 8192),
                                 (65, 16384)])
def test_norm_bwd(dev, T, D):
    g = torch.Generator().manual_seed(T * D)
    h = torch.randn(T, D, generator=g).to(torch.bfloat16)
    nw = torch.empty(D).uniform_(0.5, 1.5, generator=g)
    dxn = torch.randn(T, D, generator=g).to(torch.bfloat16)
    dy = (torch.randn(T, D, generator=g) * 1e-3).to(torch.bfloat16)
    rstd = O.norm_stats(h, 1e-6)
    scale = torch.tensor([1, 1, 1, 1, 2.0 ** 15], device=dev)
    amax = torch.zeros(5, device=dev)
    dh, dnw, dy8t = sg.ops.norm_bwd(h.to(dev), rstd.to(dev), dxn.to(dev), dy.to(dev), nw.to(dev), scale, amax)
    rdh, rdnw = O.norm_bwd(h, rstd, dxn, dy, nw)
    # sums over D/T in a different order: dh within one bf16 ulp, dnw to fp32 rounding
    torch.testing.assert_close(dh.cpu().float(), rdh.float(), rtol=8e-3, atol=1e-6)
    assert O.rel_l2(dh.cpu().float(), rdh.float()) < 1e-3
    torch.testing.assert_close(dnw.cpu(), rdnw, rtol=1e-4, atol=1e-4)
    ref8 = O.e5m2(dy.float() * 2.0 ** 15)
    yt = u8(sg.ops.unslab(dy8t, D))
    assert torch.equal(yt[:, :T], u8(ref8).t())
    assert torch.all(yt[:, T:] == 0)
    assert amax[4].item() == dy.float().abs().max().item()
    # dy8 as the K-slab of [T, D] instead: the same dh, dnw and amax
    amax2 = torch.zeros(5, device=dev)
    dh2, dnw2, dy8 = sg.ops.norm_bwd(h.to(dev), rstd.to(dev), dxn.to(dev), dy.to(dev), nw.to(dev), scale, amax2,
                                     rows=True)
    assert torch.equal(dh2, dh) and torch.equal(dnw2, dnw) and torch.equal(amax2, amax)
    ldt = sg.ops.ldt_of(T)
    assert dy8.shape == (D // 64, ldt, 64)
    y8 = u8(sg.ops.unslab(dy8, ldt))
    assert torch.equal(y8[:T], u8(ref8))
    assert torch.all(y8[T:] == 0)
