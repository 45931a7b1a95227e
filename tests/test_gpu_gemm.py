"""GPU parity of each GEMM kernel against the oracle on identical inputs.

* exact-integer operands (every partial sum exact in fp32, so accumulation
  order cannot matter): outputs bit-exact wherever no transcendental is
  involved, fp8 epilogue outputs after a sigmoid within one code;
* random operands: outputs within tolerance.  The gfx950 FP8 MFMA does not
  accumulate exactly in fp32: products are summed in groups aligned to the
  group's largest product, so a product about 2^17 times smaller than the
  largest one in its group is dropped.  Accumulators that cancel to small
  values can therefore move by a couple of fp8 codes; the bf16 MFMA is exact.
"""
import pytest
import torch

import spark_gpt_amd as sg
from oracle import fp8_mlp as O

pytestmark = pytest.mark.gpu

E4 = torch.float8_e4m3fn
E5 = torch.float8_e5m2


def u8(t):
    return t.contiguous().view(torch.uint8).cpu()


def code_dist(a, b):
    """Distance in fp8 codes (sign-magnitude ordinal) between two byte tensors."""
    def ordinal(x):
        x = x.to(torch.int32)
        return torch.where(x >= 128, -(x - 128), x)
    return (ordinal(u8(a)) - ordinal(u8(b))).abs()


def slab(x, dev):
    """K-slab device copy of a plain [R, K] operand (zero padding rows)."""
    return sg.ops.to_slab(x.contiguous()).to(dev)


def int_fp8(shape, dtype, g, lo=-8, hi=8):
    return torch.randint(lo, hi + 1, shape, generator=g).float().to(dtype)


SHAPES = [(1000, 256, 768), (257, 128, 384), (512, 512, 256), (1, 256, 128)]
# D = 1024 runs the persistent SwiGLU kernel whose epilogue of one tile is
# overlapped with the next tile's K loop: fewer tiles than CUs (one each),
# slightly more (some work-groups take two), several per work-group; ragged T.
SHAPES_PIPE = [(1000, 1024, 768), (2049, 1024, 1920), (4099, 1024, 3072), (1, 1024, 128)]


@pytest.mark.parametrize("T,D,I", SHAPES + SHAPES_PIPE)
def test_swiglu_fwd_integer_operands(dev, T, D, I):
    g = torch.Generator().manual_seed(T + D + I)
    x8 = int_fp8((T, D), E4, g)
    w8 = int_fp8((2 * I, D), E4, g)
    s = torch.tensor([0.5, 2.0 ** -6, 4.0, 1, 1])
    ws = torch.tensor([2.0 ** -3, 1.0])
    amax = torch.zeros(5, device=dev)
    gu8s, h8s, h8t = sg.ops.gateup_swiglu_fwd(slab(x8, dev), slab(w8, dev), s.to(dev), ws.to(dev), amax, T, I)
    rgu8, rh8, ra1, ra2 = O.swiglu_fwd(x8, w8, s, ws, I)
    ldt = sg.ops.ldt_of(T)
    assert gu8s.shape == (2 * I // 64, ldt, 64)
    assert torch.equal(u8(sg.ops.unslab(gu8s, T)), u8(rgu8))
    assert torch.all(u8(sg.ops.unslab(gu8s, ldt))[T:] == 0)
    assert h8s.shape == (I // 64, ldt, 64)
    h8 = sg.ops.unslab(h8s, T)
    assert torch.all(u8(sg.ops.unslab(h8s, ldt))[T:] == 0)
    assert int(code_dist(h8, rh8).max()) <= 1
    assert float((code_dist(h8, rh8) > 0).float().mean()) < 0.01
    assert h8t.shape == (ldt // 64, sg.ops.slab_rows(I), 64)
    ht = u8(sg.ops.unslab(h8t, I))
    assert torch.equal(ht[:, :T], u8(h8).t())
    assert torch.all(ht[:, T:] == 0)
    assert amax[1].item() == ra1.item()
    torch.testing.assert_close(amax[2].cpu(), ra2, rtol=1e-5, atol=0)
    # without the token-contiguous copy: the same rows and amax
    amax2 = torch.zeros(5, device=dev)
    gu8b, h8b, none = sg.ops.gateup_swiglu_fwd(slab(x8, dev), slab(w8, dev), s.to(dev), ws.to(dev), amax2, T, I,
                                               copy=False)
    assert none is None
    assert torch.equal(u8(gu8b), u8(gu8s)) and torch.equal(u8(h8b), u8(h8s))
    assert torch.equal(amax2, amax)


@pytest.mark.parametrize("T,D,I", [(300, 256, 256), (300, 1024, 256)])
def test_swiglu_fwd_nan_rows(dev, T, D, I):
    """A NaN code in a token's x8 row makes that token's gate, up and h all
    NaN: they must carry NaN codes, the other rows must be unaffected, and
    NaN values do not enter the amax slots."""
    g = torch.Generator().manual_seed(21 + D)
    x8 = int_fp8((T, D), E4, g)
    w8 = int_fp8((2 * I, D), E4, g)
    bad = torch.tensor([0, 77, T - 1])
    xb = x8.view(torch.uint8).clone()
    xb[bad, 5] = 0x7F
    x8n = xb.view(E4)
    s = torch.tensor([1.0, 2.0 ** -8, 2.0 ** -12, 1, 1])
    ws = torch.tensor([1.0, 1.0])
    amax = torch.zeros(5, device=dev)
    gu8s, h8s, _ = sg.ops.gateup_swiglu_fwd(slab(x8n, dev), slab(w8, dev), s.to(dev), ws.to(dev), amax, T, I)
    h8 = u8(sg.ops.unslab(h8s, T))
    gu = u8(sg.ops.unslab(gu8s, T))
    assert torch.all((gu[bad] & 0x7F) == 0x7F) and torch.all((h8[bad] & 0x7F) == 0x7F)
    keep = torch.ones(T, dtype=torch.bool)
    keep[bad] = False
    rgu8, rh8, ra1, ra2 = O.swiglu_fwd(x8[keep], w8, s, ws, I)
    assert torch.equal(gu[keep], u8(rgu8))
    assert int(code_dist(h8[keep].view(E4), rh8).max()) <= 1
    assert amax[1].item() == ra1.item()
    torch.testing.assert_close(amax[2].cpu(), ra2, rtol=1e-5, atol=0)


@pytest.mark.parametrize("T,D,I", SHAPES[:3])
def test_swiglu_fwd_random(dev, T, D, I):
    g = torch.Generator().manual_seed(1 + T + D + I)
    h = torch.randn(T, D, generator=g).to(torch.bfloat16)
    nw = torch.ones(D)
    s = torch.tensor([32.0, 64.0, 128.0, 1, 1])
    x8, _, _, _ = O.norm_quant(h, nw, s[0], 1e-6)
    w8, q = O.quantize_weight(torch.randn(2 * I, D, generator=g) * D ** -0.5)
    ws = torch.stack([q, torch.tensor(1.0)])
    amax = torch.zeros(5, device=dev)
    gu8s, h8s, _ = sg.ops.gateup_swiglu_fwd(slab(x8, dev), slab(w8, dev), s.to(dev), ws.to(dev), amax, T, I)
    gu8, h8 = sg.ops.unslab(gu8s, T), sg.ops.unslab(h8s, T)
    rgu8, rh8, ra1, ra2 = O.swiglu_fwd(x8, w8, s, ws, I)
    for got, ref in ((gu8, rgu8), (h8, rh8)):
        d = code_dist(got, ref)
        # one code wherever the value is clear of the e4m3 subnormal range;
        # near zero the MFMA's group truncation can move a cancelled
        # accumulator by a few subnormal steps
        clear = ref.float().abs() >= 2.0 ** -4
        assert int(d[clear].max()) <= 1 and int(d.max()) <= 8
        assert float((d > 0).float().mean()) < 0.005
        assert O.rel_l2(got.cpu().float(), ref.float()) < 2e-3
    torch.testing.assert_close(amax[1:3].cpu(), torch.stack([ra1, ra2]), rtol=1e-2, atol=0)


@pytest.mark.parametrize("T,D,I", SHAPES)
def test_down_fwd_integer_operands(dev, T, D, I):
    g = torch.Generator().manual_seed(2 + T + D + I)
    h8 = int_fp8((T, I), E4, g)
    wd8 = int_fp8((D, I), E4, g)
    res = torch.randn(T, D, generator=g).to(torch.bfloat16)
    s = torch.tensor([1, 1, 2.0 ** 4, 1, 1])
    ws = torch.tensor([1.0, 2.0 ** 3])
    y = sg.ops.down_fwd(slab(h8, dev), slab(wd8, dev), res.to(dev), s.to(dev), ws.to(dev))
    ry = O.down_fwd(h8, wd8, res, s, ws)
    assert torch.equal(y.cpu(), ry)


# The headline width D = 1024: the persistent dgrad with fewer tiles than CUs
# and with three tiles per work-group (T = 16384); ragged T.
SHAPES_DGRAD_PIPE = [(1000, 1024, 768), (1, 1024, 128), (4099, 1024, 3072), (16384, 1024, 3072)]


@pytest.mark.parametrize("T,D,I", SHAPES + SHAPES_DGRAD_PIPE)
def test_down_dgrad_swiglu_integer_operands(dev, T, D, I):
    g = torch.Generator().manual_seed(3 + T + D + I)
    dy = torch.randint(-8, 9, (T, D), generator=g).float().to(torch.bfloat16)
    wd = torch.randint(-8, 9, (D, I), generator=g).float().to(torch.bfloat16)
    gu8 = O.e4m3(torch.randn(T, 2 * I, generator=g) * 64)
    s = torch.tensor([1, 64.0, 1, 2.0 ** -12, 1])
    amax = torch.zeros(5, device=dev)
    dgu8s, dgu8t = sg.ops.down_dgrad_swiglu(dy.to(dev), slab(wd.t(), dev), slab(gu8, dev), s.to(dev), amax)
    dgu8 = sg.ops.unslab(dgu8s, T)
    assert torch.all(u8(sg.ops.unslab(dgu8s, sg.ops.ldt_of(T)))[T:] == 0)
    rdgu8, ra3, _ = O.down_dgrad_swiglu(dy, wd, gu8, s, I)
    d = code_dist(dgu8, rdgu8)
    assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 0.01
    dt = u8(sg.ops.unslab(dgu8t, 2 * I))
    assert torch.equal(dt[:, :T], u8(dgu8).t())
    assert torch.all(dt[:, T:] == 0)
    torch.testing.assert_close(amax[3].cpu(), ra3, rtol=1e-5, atol=0)
    # without the token-contiguous copy: the same rows and amax
    amax2 = torch.zeros(5, device=dev)
    dgu8b, none = sg.ops.down_dgrad_swiglu(dy.to(dev), slab(wd.t(), dev), slab(gu8, dev), s.to(dev), amax2,
                                           copy=False)
    assert none is None
    assert torch.equal(u8(dgu8b), u8(dgu8s))
    assert torch.equal(amax2, amax)


@pytest.mark.parametrize("T,D,I", [(512, 256, 256), (8192, 1024, 3072)])
def test_down_dgrad_swiglu_every_gate_code(dev, T, D, I):
    """Every e4m3 code as gate and as up value, the two NaN codes included.
    The kernel takes sigmoid(g) and sig*(1 + g*(1 - sig)) from a table over
    the 256 gate codes and multiplies in the reference's order, so only a
    sigmoid that differs from torch's by an ulp can move a byte.  NaN outputs
    must carry a NaN code (the sign of a NaN is not specified)."""
    g = torch.Generator().manual_seed(11)
    dy = torch.randint(-8, 9, (T, D), generator=g).float().to(torch.bfloat16)
    wd = torch.randint(-8, 9, (D, I), generator=g).float().to(torch.bfloat16)
    codes = torch.arange(T * I, dtype=torch.int64)
    gate = (codes % 256).to(torch.uint8).view(T, I)
    up = ((codes * 97 + codes // 256) % 256).to(torch.uint8).view(T, I)
    gu8 = torch.cat([gate, up], dim=1).view(E4)
    s = torch.tensor([1, 64.0, 1, 2.0 ** -6, 1])
    amax = torch.zeros(5, device=dev)
    dgu8s, dgu8t = sg.ops.down_dgrad_swiglu(dy.to(dev), slab(wd.t(), dev), slab(gu8, dev), s.to(dev), amax)
    dgu8 = sg.ops.unslab(dgu8s, T)
    rdgu8, _, _ = O.down_dgrad_swiglu(dy, wd, gu8, s, I)
    nan = torch.isnan(rdgu8.float())
    assert int(nan.sum()) > 0
    got = u8(dgu8)
    assert torch.all((got[nan] & 0x7F) == 0x7F)
    d = code_dist(dgu8, rdgu8)[~nan]
    assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 1e-3
    dt = u8(sg.ops.unslab(dgu8t, 2 * I))
    assert torch.equal(dt[:, :T], got.t())
    # without the token-contiguous copy (at D = 1024 the persistent 256 x 128
    # kernel with the deferred epilogue): the same bytes, NaN codes and
    # exact-path blocks included, and the same amax
    amax2 = torch.zeros(5, device=dev)
    dgu8b, _ = sg.ops.down_dgrad_swiglu(dy.to(dev), slab(wd.t(), dev), slab(gu8, dev), s.to(dev), amax2,
                                        copy=False)
    assert torch.equal(u8(dgu8b), u8(dgu8s))
    assert torch.equal(amax2, amax)


@pytest.mark.parametrize("T,D,I", SHAPES[:3] + SHAPES_DGRAD_PIPE[2:])
def test_down_dgrad_swiglu_random(dev, T, D, I):
    g = torch.Generator().manual_seed(4 + T + D + I)
    dy = (torch.randn(T, D, generator=g) * 1e-3).to(torch.bfloat16)
    wd = (torch.randn(D, I, generator=g) * I ** -0.5).to(torch.bfloat16)
    gu8 = O.e4m3(torch.randn(T, 2 * I, generator=g) * 64)
    s = torch.tensor([1, 64.0, 1, 2.0 ** 18, 1])
    amax = torch.zeros(5, device=dev)
    dgu8s, _ = sg.ops.down_dgrad_swiglu(dy.to(dev), slab(wd.t(), dev), slab(gu8, dev), s.to(dev), amax)
    dgu8 = sg.ops.unslab(dgu8s, T)
    rdgu8, ra3, _ = O.down_dgrad_swiglu(dy, wd, gu8, s, I)
    d = code_dist(dgu8, rdgu8)
    # Where dh = dy @ Wd cancels, the oracle's own fp32 sum can be more than
    # half a bf16 ulp from the exact (fp64) value; its byte there is not
    # pinned (any fp32 order, the kernel's included, may round elsewhere).
    # Such elements must be rare; every other byte is within one code.
    dh32, dh64 = dy.float() @ wd.float(), dy.double() @ wd.double()
    unpinned = (dh32.double() - dh64).abs() > dh64.abs() * 2.0 ** -9
    unpinned = torch.cat([unpinned, unpinned], dim=1)
    assert float(unpinned.float().mean()) < 1e-3
    assert int(d[~unpinned].max()) <= 1 and float((d > 0).float().mean()) < 0.02
    torch.testing.assert_close(amax[3].cpu(), ra3, rtol=1e-2, atol=0)
    amax2 = torch.zeros(5, device=dev)
    dgu8b, _ = sg.ops.down_dgrad_swiglu(dy.to(dev), slab(wd.t(), dev), slab(gu8, dev), s.to(dev), amax2,
                                        copy=False)
    assert torch.equal(u8(dgu8b), u8(dgu8s))
    assert torch.equal(amax2, amax)


@pytest.mark.parametrize("T,D,I", SHAPES)
def test_gateup_dgrad_integer_operands(dev, T, D, I):
    g = torch.Generator().manual_seed(5 + T + D + I)
    dgu8 = int_fp8((T, 2 * I), E5, g)
    w8 = int_fp8((2 * I, D), E4, g)
    s = torch.tensor([1, 1, 1, 2.0 ** 5, 1])
    ws = torch.tensor([2.0 ** 2, 1.0])
    dxn = sg.ops.gateup_dgrad(slab(dgu8, dev), slab(w8.t(), dev), s.to(dev), ws.to(dev), T, D)
    rdxn = O.gateup_dgrad(dgu8, w8, s, ws)
    assert torch.equal(dxn.cpu(), rdxn)


@pytest.mark.parametrize("T,M,N", [(1000, 256, 768), (257, 768, 128), (4099, 1024, 512), (65536, 256, 256)])
def test_wgrad_integer_operands(dev, T, M, N):
    g = torch.Generator().manual_seed(6 + T + M + N)
    ldt = sg.ops.ldt_of(T)
    a = int_fp8((T, M), E5, g, -4, 4)
    b = int_fp8((T, N), E4, g, -4, 4)
    at = torch.zeros(M, ldt, dtype=torch.uint8)
    bt = torch.zeros(N, ldt, dtype=torch.uint8)
    at[:, :T] = u8(a).t()
    bt[:, :T] = u8(b).t()
    sa, sb = torch.tensor([2.0 ** 3]), torch.tensor([0.5])
    at_s = sg.ops.to_slab(at.view(E5)).view(torch.uint8)
    bt_s = sg.ops.to_slab(bt.view(E4)).view(torch.uint8)
    # padding rows (beyond M, N) hold NaN codes: they must not reach the output
    at_s[:, M:] = 0x7F
    bt_s[:, N:] = 0x7F
    out = sg.ops.wgrad(at_s.view(E5).to(dev), bt_s.view(E4).to(dev), M, N, sa.to(dev), sb.to(dev))
    ref = (a.float().t() @ b.float()) / (sa * sb)
    assert torch.equal(out.cpu(), ref)


def test_wgrad_matches_oracle_forms(dev):
    """Both weight gradients of the block through the kernel vs the oracle's
    reference-shaped formulas (down: dy quantized e5m2 in 2 token splits;
    gate/up: d_gu8^T x8)."""
    T, D, I = 1000, 256, 768
    g = torch.Generator().manual_seed(7)
    dy = (torch.randn(T, D, generator=g) * 1e-3).to(torch.bfloat16)
    h8 = O.e4m3(torch.randn(T, I, generator=g) * 30)
    dgu8 = O.e5m2(torch.randn(T, 2 * I, generator=g) * 1000)
    x8 = O.e4m3(torch.randn(T, D, generator=g) * 30)
    s = torch.tensor([16.0, 1, 32.0, 2.0 ** 10, 2.0 ** 15])
    ldt = sg.ops.ldt_of(T)

    def tpad(t8):
        out = torch.zeros(t8.shape[1], ldt, dtype=torch.uint8)
        out[:, :T] = u8(t8).t()
        return sg.ops.to_slab(out.view(t8.dtype)).to(dev)

    dy8 = O.e5m2(dy.float() * s[4])
    sd = s.to(dev)
    dwd = sg.ops.wgrad(tpad(dy8), tpad(h8), D, I, sd[4:5], sd[2:3])
    dwgu = sg.ops.wgrad(tpad(dgu8), tpad(x8), 2 * I, D, sd[3:4], sd[0:1])
    for got, ref in ((dwd, O.down_wgrad(dy, h8, s)), (dwgu, O.gateup_wgrad(dgu8, x8, s))):
        torch.testing.assert_close(got.cpu(), ref, rtol=1e-4, atol=1e-4 * float(ref.abs().max()))
        assert O.rel_l2(got.cpu(), ref) < 1e-4


@pytest.mark.parametrize("M,N", [(256, 100), (300, 36), (64, 4)])
def test_wgrad_ragged_columns_stay_in_bounds(dev, M, N):
    """N % 16 != 0 with one K split (the kernel's own epilogue writes [M, N]):
    every float4 past column N is skipped, so a guard region right after the
    output is untouched and the output equals a float32 matmul."""
    from spark_gpt_amd import _lib

    T = 200
    ldt = sg.ops.ldt_of(T)
    assert _lib.query("sfp8_wgrad_splits", M, N, ldt) == 1
    g = torch.Generator().manual_seed(M + N)
    a = int_fp8((T, M), E5, g, -4, 4)
    b = int_fp8((T, N), E4, g, -4, 4)
    at = torch.zeros(M, ldt, dtype=torch.uint8)
    bt = torch.zeros(N, ldt, dtype=torch.uint8)
    at[:, :T] = u8(a).t()
    bt[:, :T] = u8(b).t()
    at_s = sg.ops.to_slab(at.view(E5)).to(dev)
    bt_s = sg.ops.to_slab(bt.view(E4)).to(dev)
    sa, sb = torch.tensor([1.0], device=dev), torch.tensor([1.0], device=dev)
    guard = 1 << 16
    buf = torch.full((M * N + guard,), 12345.0, device=dev)
    _lib.call("sfp8_gemm_wgrad", at_s.data_ptr(), 1, bt_s.data_ptr(), 0, M, N, ldt, sa.data_ptr(), sb.data_ptr(),
              buf.data_ptr(), None, 0, _lib.stream_of(buf))
    torch.cuda.synchronize()
    ref = a.float().t() @ b.float()
    assert torch.equal(buf[: M * N].view(M, N).cpu(), ref)
    assert bool((buf[M * N:] == 12345.0).all())


@pytest.mark.parametrize("M,N,T,splits", [(6144, 1024, 4096, 2), (1024, 3072, 16384, 5), (1024, 1024, 8192, 4),
                                          (1024, 1024, 16384, 8), (320, 192, 1000, 1), (256, 256, 65536, 32)])
def test_wgrad_rows_equals_token_contiguous(dev, M, N, T, splits):
    """The weight gradient read from the row K-slabs through transposing LDS
    reads gives the bytes of the one read from the token-contiguous copies
    (same values in the same MFMA K positions, same split sums): one split
    and several (2 and 4 splits: each split on 8 / splits XCDs; 5: uneven
    splits, the last shorter, runs of the split-major order crossing split
    boundaries; 8 and 32: whole splits per XCD), ragged tiles, and the same
    operands in both layouts.  The result is also checked against a float64
    matmul of the same operands, which no split mapping shares."""
    from spark_gpt_amd import _lib

    ops = sg.ops
    assert _lib.query("sfp8_wgrad_splits", M, N, ops.ldt_of(T)) == splits
    g = torch.Generator(device=dev).manual_seed(M + N + T)
    a = (torch.randn(T, M, device=dev, generator=g) * 8).to(ops.E5M2)
    b = (torch.randn(T, N, device=dev, generator=g) * 8).to(ops.E4M3)
    ldt = ops.ldt_of(T)
    pad = lambda x: torch.cat([x, torch.zeros(ldt - T, x.shape[1], dtype=x.dtype, device=dev)])
    a_rows, b_rows = ops.to_slab(pad(a)), ops.to_slab(pad(b))      # [M/64, ldt, 64]
    a_t, b_t = ops.to_slab(pad(a).t().contiguous()), ops.to_slab(pad(b).t().contiguous())  # [ldt/64, M, 64]
    sa = torch.tensor([2.0 ** 4], device=dev)
    sb = torch.tensor([2.0 ** -2], device=dev)
    ref = ops.wgrad(a_t, b_t, M, N, sa, sb)
    exact = (a.double().t() @ b.double()) / (sa.double() * sb.double())
    # fp32 accumulation over T products: rel-L2 about 1e-5 at T = 65536
    assert float((ref.double() - exact).norm() / exact.norm()) < 1e-4
    assert torch.equal(ops.wgrad_rows(a_rows, b_rows, M, N, sa, sb), ref)
    assert torch.equal(ops.wgrad_rows(a_rows, b_t, M, N, sa, sb, b_rows=False), ref)
    assert torch.equal(ops.wgrad_rows(a_t, b_rows, M, N, sa, sb, a_rows=False), ref)
