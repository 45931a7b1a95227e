"""GPU parity: standalone quantizer, scale roll, weight quantization (bit-exact)."""
import numpy as np
import pytest
import torch

import spark_gpt_amd as sg
from oracle import fp8_bits, fp8_mlp as O

pytestmark = pytest.mark.gpu

E4 = torch.float8_e4m3fn
E5 = torch.float8_e5m2


def u8(t):
    return t.contiguous().view(torch.uint8).cpu()


def all_bf16(nan: bool = True, cols: int = 128) -> torch.Tensor:
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    if not nan:
        f = bits.float()
        bits = bits[~torch.isnan(f)]
        bits = bits[: (bits.numel() // cols) * cols]
    return bits.reshape(-1, cols).contiguous()


@pytest.mark.parametrize("cols", [128, 256])
@pytest.mark.parametrize("log2s", [-12, -3, 0, 1, 5, 12])
def test_e4m3_cast_exhaustive(dev, log2s, cols):
    """Every bf16 bit pattern x scale: bytes equal torch's clamp+cast (NaN
    incl.), through the 128 x 128 tile (128 columns) and the 64 x 256 tile."""
    x = all_bf16(cols=cols)
    s = torch.tensor([2.0 ** log2s, 1, 1, 1, 1])
    x8, x8t = sg.ops.quant_e4m3_rowcol(x.to(dev), s.to(dev), torch.zeros(5, device=dev))
    ref = O.e4m3(x.float() * s[0])
    assert torch.equal(u8(x8), u8(ref))
    assert torch.equal(u8(sg.ops.unslab(x8t, x.shape[1])), u8(ref).t())


def test_e5m2_cast_exhaustive_via_norm_bwd(dev):
    """dy8t = e5m2(dy * s4)^T from the norm backward, over every bf16 pattern."""
    dy = all_bf16()
    T, D = dy.shape
    for log2s in (-8, 0, 7):
        scale = torch.tensor([1, 1, 1, 1, 2.0 ** log2s], device=dev)
        amax = torch.zeros(5, device=dev)
        z = torch.zeros(T, D, dtype=torch.bfloat16, device=dev)
        _, _, dy8t = sg.ops.norm_bwd(z, torch.ones(T, device=dev), z, dy.to(dev), torch.ones(D, device=dev),
                                     scale, amax)
        ref = O.e5m2(dy.float() * 2.0 ** log2s)
        yt = u8(sg.ops.unslab(dy8t, D))
        assert torch.equal(yt[:, :T], u8(ref).t())
        assert torch.all(yt[:, T:] == 0)


def test_cast_matches_closed_form_table(dev):
    """The GPU bytes also equal the independent closed-form RNE (finite inputs)."""
    x = all_bf16(nan=False)
    xf = x.float().clamp(-448, 448)
    x8, _ = sg.ops.quant_e4m3_rowcol(xf.to(torch.bfloat16).to(dev), torch.ones(5, device=dev),
                                     torch.zeros(5, device=dev))
    assert np.array_equal(u8(x8).numpy(), fp8_bits.cast_e4m3(xf.to(torch.bfloat16).float().numpy()))


@pytest.mark.parametrize("R,C", [(1, 128), (257, 256), (1000, 384), (4099, 1024)])
def test_quant_rowcol_ragged(dev, R, C):
    g = torch.Generator().manual_seed(R * 7 + C)
    x = torch.randn(R, C, generator=g)
    x[:, 3] *= 50.0  # outlier channel
    x = x.to(torch.bfloat16)
    s = torch.tensor([8.0, 1, 1, 1, 1])
    amax = torch.zeros(5, device=dev)
    x8, x8t = sg.ops.quant_e4m3_rowcol(x.to(dev), s.to(dev), amax)
    r8, r8t, ra = O.quant_rowcol(x, s[0])
    assert torch.equal(u8(x8), u8(r8))
    xt = u8(sg.ops.unslab(x8t, C))
    assert torch.equal(xt[:, :R], u8(r8t))
    assert torch.all(xt[:, R:] == 0)
    assert torch.all(u8(x8t)[:, C:, :] == 0)  # slab padding rows
    assert amax[0].item() == ra.item()
    assert torch.all(amax[1:].cpu() == 0)


@pytest.mark.parametrize("R,C,ldt", [(100, 256, 128), (100, 384, 320), (257, 128, 1024), (1, 256, 64),
                                     (64, 512, 64)])
def test_quant_rowcol_ldt_padding(dev, R, C, ldt):
    """Through the C ABI with ldt > rows: x8t tokens rows..ldt-1 and the slab's
    padding rows are written as zeros over a buffer prefilled with 0x55."""
    from spark_gpt_amd import _lib
    g = torch.Generator().manual_seed(R + ldt)
    x = torch.randn(R, C, generator=g).to(torch.bfloat16)
    s = torch.tensor([4.0, 1, 1, 1, 1])
    amax = torch.zeros(5, device=dev)
    x8 = torch.empty(R, C, dtype=torch.uint8, device=dev)
    x8t = torch.full((ldt // 64, sg.ops.slab_rows(C), 64), 0x55, dtype=torch.uint8, device=dev)
    xd, sd = x.to(dev), s.to(dev)
    _lib.call("sfp8_quant_e4m3_rowcol", xd.data_ptr(), R, C, sd.data_ptr(), amax.data_ptr(), x8.data_ptr(),
              x8t.data_ptr(), ldt, _lib.stream_of(xd))
    r8, r8t, ra = O.quant_rowcol(x, s[0])
    assert torch.equal(x8.cpu(), u8(r8))
    xt = sg.ops.unslab(x8t, C).cpu()
    assert torch.equal(xt[:, :R], u8(r8t))
    assert torch.all(xt[:, R:] == 0)
    assert torch.all(x8t[:, C:, :] == 0)
    assert amax[0].item() == ra.item()


@pytest.mark.parametrize("C", [128, 256])
def test_quant_rowcol_amax_ignores_nan(dev, C):
    """NaN elements get torch's NaN codes; amax is the maximum over the finite
    magnitudes (a NaN activation does not poison the next delayed scale)."""
    g = torch.Generator().manual_seed(11 + C)
    x = torch.randn(300, C, generator=g)
    x[7, 5] = float("nan")
    x[250, C - 1] = float("nan")
    x[100, 3] = -37.5  # the largest finite magnitude
    x = x.to(torch.bfloat16)
    s = torch.tensor([2.0, 1, 1, 1, 1])
    amax = torch.zeros(5, device=dev)
    x8, x8t = sg.ops.quant_e4m3_rowcol(x.to(dev), s.to(dev), amax)
    ref = O.e4m3(x.float() * s[0])
    assert torch.equal(u8(x8), u8(ref))
    assert torch.equal(u8(sg.ops.unslab(x8t, C))[:, :300], u8(ref).t())
    assert amax[0].item() == 37.5


def test_quant_rowcol_full_size(dev):
    """65536 x 4096 bf16 with 0.1% outlier columns x50, delayed scale from a
    prewarm pass; bytes, transpose, amax and next scale bit-exact."""
    g = torch.Generator().manual_seed(3)
    R, C = 65536, 4096
    x = torch.randn(R, C, generator=g)
    cols = torch.randperm(C, generator=g)[: C // 1000]
    x[:, cols] *= 50.0
    x = x.to(torch.bfloat16)
    xd = x.to(dev)
    scale = torch.ones(5, device=dev)
    amax = torch.zeros(5, device=dev)
    sg.ops.quant_e4m3_rowcol(xd, scale, amax)  # prewarm: records amax under scale 1
    sg.ops.update_scales(scale, amax)
    s_ref = torch.ones(5)
    a_ref = torch.zeros(5)
    a_ref[0] = x.float().abs().max()
    O.update_scales(s_ref, a_ref)
    assert torch.equal(scale.cpu(), s_ref)
    x8, x8t = sg.ops.quant_e4m3_rowcol(xd, scale, amax)
    r8 = O.e4m3(x.float() * s_ref[0])
    assert torch.equal(u8(x8), u8(r8))
    assert torch.equal(sg.ops.unslab(x8t, C).view(torch.uint8)[:, :R], x8.view(torch.uint8).t())
    assert amax[0].item() == x.float().abs().max().item()


def _band_amax(fmax: float) -> list[float]:
    """amax values whose quotient fmax/amax lands within a few ulps below a
    power of two (where the rounded log2 decides the binade)."""
    out = []
    for K in (-20, -7, -3, 2, 3, 5, 8, 9, 17, 40):
        base = int(np.float32(2.0 ** K).view(np.uint32))
        for n in range(0, 50, 3):
            r = np.array([base - n], dtype=np.uint32).view(np.float32)[0]
            a = int(np.float32(np.float32(fmax) / r).view(np.uint32))
            for da in range(-2, 3):
                cand = np.array([a + da], dtype=np.uint32).view(np.float32)[0]
                out.append(float(cand))
    return out


def test_update_scales_bit_exact(dev):
    g = np.random.default_rng(0)
    vals = list(np.exp(g.uniform(-60, 60, 2000)).astype(np.float32))
    vals += _band_amax(448.0) + _band_amax(57344.0)
    vals += [0.0, 1e-38, 1e-30, 1e-29, 448.0, 57344.0, 3.4e38, float("inf"), float("nan")]
    n = (len(vals) // 5 + 1) * 5
    vals = (vals + [1.0] * n)[:n]
    amax = torch.tensor(vals, dtype=torch.float32)
    scale0 = torch.exp2(torch.randint(-10, 10, (n,)).float())
    s_ref, a_ref = scale0.clone(), amax.clone()
    for i in range(0, n, 5):
        O.update_scales(s_ref[i:i + 5], a_ref[i:i + 5])
    s_gpu, a_gpu = scale0.to(dev), amax.to(dev)
    sg.ops.update_scales(s_gpu, a_gpu)
    got = s_gpu.cpu()
    same = (got == s_ref) | (torch.isnan(got) & torch.isnan(s_ref))
    assert bool(same.all()), (amax[~same], got[~same], s_ref[~same])
    assert torch.all(a_gpu.cpu() == 0)


@pytest.mark.parametrize("R,C,std", [(768, 256, 0.05), (6144, 1024, 1 / 32), (1024, 3072, 1e-4),
                                     (192, 320, 3.0)])
def test_weight_quant_bit_exact(dev, R, C, std):
    """The three K-slab copies (W8, W8^T, bf16 W^T) against the reference
    recipe, padding rows (to multiples of 256) zero."""
    g = torch.Generator().manual_seed(R + C)
    w = torch.randn(R, C, generator=g) * std
    q = torch.empty(1, device=dev)
    w8, w8t, wbt = sg.ops.weight_quant(w.to(dev), q, w8=True, w8t=True, bf16t=True)
    r8, rq = O.quantize_weight(w)
    assert q.item() == rq.item()
    assert w8.shape == (C // 64, sg.ops.slab_rows(R), 64)
    assert torch.equal(u8(sg.ops.unslab(w8, R)), u8(r8))
    assert torch.equal(u8(sg.ops.unslab(w8t, C)), u8(r8).t())
    assert torch.equal(sg.ops.unslab(wbt, C).cpu(), w.to(torch.bfloat16).t())
    for t in (w8, w8t, wbt):
        rows = R if t is w8 else C
        assert torch.all(t.view(torch.uint8)[:, rows:].cpu() == 0)


def test_weight_quant_ragged_rows(dev):
    """130 rows (not a multiple of 64): W8 only, padding rows 130..255 zero."""
    g = torch.Generator().manual_seed(5)
    w = torch.randn(130, 128, generator=g)
    q = torch.empty(1, device=dev)
    w8, _, _ = sg.ops.weight_quant(w.to(dev), q, w8=True)
    r8, rq = O.quantize_weight(w)
    assert q.item() == rq.item()
    assert torch.equal(u8(sg.ops.unslab(w8, 130)), u8(r8))
    assert torch.all(w8.view(torch.uint8)[:, 130:].cpu() == 0)


def test_weight_scale_band(dev):
    """Weights whose amax puts 448/amax in the log2 rounding band."""
    amaxes = [a for a in _band_amax(448.0) if np.isfinite(a) and a > 0][:200]
    for a in amaxes[::7]:
        w = torch.zeros(1, 64)
        w[0, :3] = torch.tensor([a, -a / 3, 0.1 * a], dtype=torch.float32)
        q = torch.empty(1, device=dev)
        sg.ops.weight_quant(w.to(dev), q, w8=True)
        _, rq = O.quantize_weight(w)
        assert q.item() == rq.item(), a


@pytest.mark.parametrize("D,I", [(1024, 3072), (256, 1024), (192, 128)])
def test_block_weight_quant_equals_two_calls(dev, D, I):
    """The post-step hook's two-launch form (scale roll + both weight
    quantizations) writes the same bytes as update_scales and the two
    weight_quant calls, and every output against the reference recipe."""
    g = torch.Generator().manual_seed(D + I)
    w_gu = (torch.randn(2 * I, D, generator=g) * D ** -0.5).to(dev)
    w_d = (torch.randn(D, I, generator=g) * I ** -0.5).to(dev)
    amax = torch.tensor([3.0, 0.0, 1e-3, 70000.0, float("nan")])
    scale0 = torch.tensor([1.0, 2.0, 4.0, 8.0, 16.0])
    s1, a1 = scale0.to(dev), amax.to(dev)
    s2, a2 = scale0.to(dev), amax.to(dev)
    w8, w8t, wd8, wdt, ws = sg.ops.block_weight_quant(w_gu, w_d, s1, a1)
    sg.ops.update_scales(s2, a2)
    q = torch.empty(2, device=dev)
    r8, r8t, _ = sg.ops.weight_quant(w_gu, q[0:1], w8=True, w8t=True)
    rd8, _, rdt = sg.ops.weight_quant(w_d, q[1:2], w8=True, bf16t=True)
    torch.cuda.synchronize()
    for a, b in ((w8, r8), (w8t, r8t), (wd8, rd8), (wdt, rdt), (ws, q)):
        assert torch.equal(a.view(torch.uint8).cpu(), b.view(torch.uint8).cpu())
    same = (s1.cpu() == s2.cpu()) | (torch.isnan(s1.cpu()) & torch.isnan(s2.cpu()))
    assert bool(same.all()) and torch.all(a1.cpu() == 0) and torch.all(a2.cpu() == 0)
    q_ref_gu = O.quantize_weight(w_gu.cpu())[1]
    q_ref_d = O.quantize_weight(w_d.cpu())[1]
    assert ws[0].item() == q_ref_gu.item() and ws[1].item() == q_ref_d.item()
    # without scale and amax nothing is rolled
    s3, a3 = scale0.to(dev), amax.to(dev)
    sg.ops.block_weight_quant(w_gu, w_d)
    torch.cuda.synchronize()
    assert torch.equal(s3.cpu(), scale0) and torch.equal(a3.cpu().nan_to_num(-1), amax.nan_to_num(-1))
