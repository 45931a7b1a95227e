"""CPU tests that pin the oracle (oracle/fp8_mlp.py) before the GPU path is
tested against it.

The reference holds no golden vectors for this path (its only test is a
tolerance test against an fp32 autograd MLP, spark-gpt tests/test_fp8_mlp.py),
so each oracle function is pinned against an independent derivation:

* casts: every bf16 bit pattern x a set of power-of-two scales against the
  closed-form RNE table of oracle/fp8_bits.py, plus OCP known answers;
* scale rules: exact rational floor(log2) with the correctly rounded fp32
  log2 band, invariants, and the two forms of the quotient;
* norm statistics: fp64 closed form and an order-independence property;
* GEMM pieces: fp64 brute force on tiny shapes (exact for fp8 operands);
* the block: the reference's own bound (rel-L2 < 0.12 vs fp32 autograd) at
  the reference's test shape, the amax/scale lifecycle, and planted mistakes
  (a dropped term, a transposed operand, a wrong scale) that must fail it.
"""
import math

import numpy as np
import pytest
import torch

from oracle import fp8_bits, fp8_mlp as O


def all_bf16_finite():
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    return x[torch.isfinite(x)]


# ------------------------------------------------------------------ casts
@pytest.mark.parametrize("log2s", [-20, -9, -1, 0, 3, 9, 20])
def test_e4m3_cast_exhaustive_vs_closed_form(log2s):
    x = all_bf16_finite() * 2.0 ** log2s
    ours = O.e4m3(x).view(torch.uint8).numpy()
    closed = fp8_bits.cast_e4m3(x.clamp(-448, 448).numpy())
    assert np.array_equal(ours, closed)


@pytest.mark.parametrize("log2s", [-30, -12, 0, 5, 14])
def test_e5m2_cast_exhaustive_vs_closed_form(log2s):
    x = all_bf16_finite() * 2.0 ** log2s
    ours = O.e5m2(x).view(torch.uint8).numpy()
    closed = fp8_bits.cast_e5m2(x.clamp(-57344, 57344).numpy())
    assert np.array_equal(ours, closed)


def test_cast_known_answers():
    """OCP FP8 spec values (e4m3fn: bias 7, max 448 = 0x7E, NaN 0x7F, min
    subnormal 2^-9; e5m2: bias 15, max 57344 = 0x7B, min subnormal 2^-16)."""
    kat4 = [(1.0, 0x38), (448.0, 0x7E), (-448.0, 0xFE), (2.0 ** -9, 0x01), (2.0 ** -6, 0x08), (0.0, 0x00),
            (-0.0, 0x80), (1.5 * 2 ** -10, 0x01), (2.0 ** -10, 0x00), (240.0, 0x77), (1.0625, 0x38),
            (1.1875, 0x3A), (1e9, 0x7E), (-1e9, 0xFE)]
    for v, code in kat4:
        assert int(O.e4m3(torch.tensor([v])).view(torch.uint8)) == code, v
    kat5 = [(1.0, 0x3C), (57344.0, 0x7B), (2.0 ** -16, 0x01), (2.0 ** -14, 0x04), (448.0, 0x5F), (1.125, 0x3C),
            (1.375, 0x3E), (1e9, 0x7B), (-0.0, 0x80)]
    for v, code in kat5:
        assert int(O.e5m2(torch.tensor([v])).view(torch.uint8)) == code, v
    for fn in (O.e4m3, O.e5m2):
        b = fn(torch.tensor([float("nan"), -float("nan")])).view(torch.uint8).tolist()
        assert b == [0x7F, 0xFF]


def test_decode_roundtrip():
    for fmt, dt in (("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)):
        codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
        ref = codes.view(dt).float().numpy()
        ours = fp8_bits.decode(codes.numpy(), fmt)
        fin = np.isfinite(ref)
        assert np.array_equal(ours[fin], ref[fin])


# ------------------------------------------------------------------ scale rules
def _exact_floor_log2(r: float) -> int:
    m, e = math.frexp(r)  # r = m * 2^e, 0.5 <= m < 1
    return e - 1


def test_band_table_matches_torch_log2():
    """floor(torch.log2(r)) == the correctly rounded band rule for every r
    within 80 ulps below each power of two, and equals the exact floor
    elsewhere."""
    rs = []
    for K in range(-120, 120):
        b = int(np.float32(2.0 ** K).view(np.uint32))
        rs += [b - n for n in range(0, 80)] + [b + 1, b + 77]
    r = np.array(rs, dtype=np.uint32).view(np.float32)
    ours = fp8_bits.floor_log2_cr(r)
    t = torch.floor(torch.log2(torch.from_numpy(r))).numpy().astype(np.int64)
    assert np.array_equal(ours, t)
    exact = np.array([_exact_floor_log2(float(v)) for v in r])
    diff = ours != exact
    # the band is where the rounded log2 sits on the next integer
    assert diff.any() and np.all(ours[diff] == exact[diff] + 1)


def test_band_table_values():
    t = fp8_bits.band_table()
    # r = 2^K (1 - n 2^-24): rounds to K iff n/(2^24 ln 2) < half-spacing near K
    for K, n in t.items():
        hs = fp8_bits._half_spacing_toward(K)
        assert -math.log2(1 - n * 2.0 ** -24) < float(hs) or n == 0
        assert -math.log2(1 - (n + 1) * 2.0 ** -24) >= float(hs) * (1 - 1e-9)


@pytest.mark.parametrize("fmax,head", [(448.0, 1), (57344.0, 1), (448.0, 0)])
def test_scale_rule_invariants(fmax, head):
    rng = np.random.default_rng(1)
    a = np.exp(rng.uniform(-50, 50, 50000)).astype(np.float32)
    s = fp8_bits.pow2_scale(a, fmax, head)
    m, _ = np.frexp(s)
    assert np.all(m == 0.5)  # powers of two
    prod = a.astype(np.float64) * s
    # (fmax/2^(head+1), fmax/2^head], except in the log2 rounding band
    lo, hi = fmax / 2 ** (head + 1), fmax / 2 ** head
    inside = (prod > lo) & (prod <= hi)
    assert inside.mean() > 0.9999


def test_update_scales_oracle_vs_closed_form():
    rng = np.random.default_rng(2)
    a = np.exp(rng.uniform(-60, 60, 20000)).astype(np.float32)
    a = np.concatenate([a, np.zeros(5, np.float32)])[: (len(a) // 5) * 5]
    amax = torch.from_numpy(a.copy())
    scale = torch.ones_like(amax) * 4.0
    for i in range(0, len(a), 5):
        O.update_scales(scale[i:i + 5], amax[i:i + 5])
    fmax = np.tile(np.array(O.FP8_SITE_MAX, np.float32), len(a) // 5)
    rule = np.where(fmax == 448.0, fp8_bits.pow2_scale(a, 448.0, 1), fp8_bits.pow2_scale(a, 57344.0, 1))
    want = np.where(a > 0, rule, np.float32(4.0))
    assert np.array_equal(scale.numpy(), want.astype(np.float32))
    assert torch.all(amax == 0)


def test_weight_rule_is_reciprocal_then_multiply():
    """`448.0 / tensor` in torch is reciprocal(t) * 448 (two roundings); the
    oracle's weight scale equals the recip-first closed form exactly, and the
    two quotient forms do differ for some amax."""
    rng = np.random.default_rng(3)
    a = np.exp(rng.uniform(-30, 30, 100000)).astype(np.float32)
    extra = []
    for K in range(-20, 20):
        b = int(np.float32(2.0 ** K).view(np.uint32))
        for n in range(0, 48):
            r = np.array([b - n], np.uint32).view(np.float32)[0]
            c = int(np.float32(np.float32(448.0) / r).view(np.uint32))
            extra += [c + d for d in range(-3, 4)]
    a = np.concatenate([a, np.array(extra, np.uint32).view(np.float32)])
    q = np.array([O.quantize_weight(torch.tensor([[v]]))[1].item() for v in a[:3000]] +
                 list(torch.exp2(torch.floor(torch.log2(448.0 / torch.from_numpy(a[3000:]).clamp(min=1e-30))))
                      .numpy()), dtype=np.float32)
    assert np.array_equal(q, fp8_bits.pow2_scale(a, 448.0, 0, recip_first=True))
    assert not np.array_equal(q, fp8_bits.pow2_scale(a, 448.0, 0, recip_first=False))


def test_quantize_weight_bytes():
    g = torch.Generator().manual_seed(4)
    w = torch.randn(96, 64, generator=g) * 0.05
    w8, q = O.quantize_weight(w)
    assert q.item() == fp8_bits.pow2_scale(np.array([w.abs().max().item()], np.float32), 448.0, 0, True)[0]
    assert np.array_equal(w8.view(torch.uint8).numpy(), fp8_bits.cast_e4m3((w * q).clamp(-448, 448).numpy()))
    assert 224 < float(w.abs().max() * q) <= 448


# ------------------------------------------------------------------ norm
def test_norm_stats_closed_form_and_order_independence():
    g = torch.Generator().manual_seed(5)
    h = (torch.randn(64, 512, generator=g) * 3).to(torch.bfloat16)
    r = O.norm_stats(h, 1e-6)
    hd = h.double()
    v = np.float32(np.float32((hd ** 2).sum(1).numpy()) / np.float32(512)) + np.float32(1e-6)
    want = (1.0 / np.sqrt(v.astype(np.float64))).astype(np.float32)
    assert np.array_equal(r.numpy(), want)
    perm = torch.randperm(512, generator=g)
    assert torch.equal(O.norm_stats(h[:, perm], 1e-6), r)
    # close to the plain fp32 formula of the reference
    ref = torch.rsqrt(h.float().pow(2).mean(-1) + 1e-6)
    torch.testing.assert_close(r, ref, rtol=3e-7, atol=0)


def test_norm_quant_matches_fp64():
    g = torch.Generator().manual_seed(6)
    h = torch.randn(33, 256, generator=g).to(torch.bfloat16)
    w = torch.empty(256).uniform_(0.5, 1.5, generator=g)
    x8, x8t, r, a = O.norm_quant(h, w, torch.tensor(32.0), 1e-6)
    n64 = h.double() * r.double()[:, None] * w.double()[None, :]
    assert torch.allclose(O.f(x8), O.e4m3(n64.float() * 32).float())
    assert abs(a.item() - n64.abs().max().item()) < 1e-6 * a.item()
    assert torch.equal(x8t.view(torch.uint8), x8.view(torch.uint8).t())


# ------------------------------------------------------------------ GEMM pieces vs fp64 brute force
def _fp8(shape, dt, g, scale=20.0):
    return (torch.randn(shape, generator=g) * scale).clamp(-400, 400).to(dt)


def test_gemm_pieces_vs_fp64():
    T, D, I = 37, 64, 32
    g = torch.Generator().manual_seed(7)
    s = torch.tensor([4.0, 8.0, 16.0, 2.0 ** 10, 2.0 ** 14])
    ws = torch.tensor([2.0 ** 6, 2.0 ** 7])
    x8 = _fp8((T, D), torch.float8_e4m3fn, g)
    w8 = _fp8((2 * I, D), torch.float8_e4m3fn, g)
    gu8, h8, a1, a2 = O.swiglu_fwd(x8, w8, s, ws, I)
    acc = x8.double() @ w8.double().t() / (4.0 * 2 ** 6)
    gg, uu = O.bf(acc[:, :I].float()), O.bf(acc[:, I:].float())
    assert torch.allclose(O.f(gu8[:, :I]), O.f(O.e4m3(gg * 8.0)))
    hh = gg * torch.sigmoid(gg) * uu
    assert torch.equal(h8.view(torch.uint8), O.e4m3(hh * 16.0).view(torch.uint8))
    assert a1.item() == max(gg.abs().max().item(), uu.abs().max().item())
    # down forward
    wd8 = _fp8((D, I), torch.float8_e4m3fn, g)
    res = torch.randn(T, D, generator=g).to(torch.bfloat16)
    y = O.down_fwd(h8, wd8, res, s, ws)
    want = (res.double() + O.bf((h8.double() @ wd8.double().t() / (16.0 * 2 ** 7)).float()).double())
    torch.testing.assert_close(y.float(), want.float().to(torch.bfloat16).float(), rtol=0, atol=0)
    # gate/up dgrad and weight grads
    dgu8 = _fp8((T, 2 * I), torch.float8_e5m2, g, 1000.0)
    dxn = O.gateup_dgrad(dgu8, w8, s, ws)
    torch.testing.assert_close(dxn.float(), (dgu8.double() @ w8.double() / (2 ** 10 * 2 ** 6)).float()
                               .to(torch.bfloat16).float(), rtol=0, atol=0)
    dwgu = O.gateup_wgrad(dgu8, x8, s)
    ref = dgu8.double().t() @ x8.double() / (2 ** 10 * 4.0)
    torch.testing.assert_close(dwgu.double(), ref, rtol=1e-6, atol=1e-6 * float(ref.abs().max()))
    dy = (torch.randn(T, D, generator=g) * 1e-3).to(torch.bfloat16)
    dwd = O.down_wgrad(dy, h8, s)
    dq = O.e5m2(dy.float() * 2 ** 14).double()
    ref = dq.t() @ h8.double() / (2 ** 14 * 16.0)
    torch.testing.assert_close(dwd.double(), ref, rtol=1e-6, atol=1e-6 * float(ref.abs().max()))


def test_swiglu_backward_is_derivative():
    """The SwiGLU backward formulas of the oracle are the derivative of
    silu(g)*u (autograd in fp64)."""
    g = torch.randn(100, dtype=torch.float64, requires_grad=True)
    u = torch.randn(100, dtype=torch.float64, requires_grad=True)
    dh = torch.randn(100, dtype=torch.float64)
    (torch.nn.functional.silu(g) * u * dh).sum().backward()
    sig = torch.sigmoid(g.detach())
    gd, ud = g.detach(), u.detach()
    torch.testing.assert_close(dh * ud * (sig * (1 + gd * (1 - sig))), g.grad)
    torch.testing.assert_close(dh * gd * sig, u.grad)


def test_down_dgrad_swiglu_is_derivative():
    """O.down_dgrad_swiglu against fp64 autograd of dy @ Wd -> silu(g) * u, with
    g, u the dequantized gu8 it is given: each d_gu code within one e5m2 step
    (the oracle rounds dh to bf16 first), amax slots exact in form."""
    T, D, I = 24, 64, 32
    g = torch.Generator().manual_seed(12)
    s = torch.tensor([1.0, 8.0, 1.0, 2.0 ** 12, 2.0 ** 14])
    gu8 = _fp8((T, 2 * I), torch.float8_e4m3fn, g, 16.0)
    wd = (torch.randn(D, I, generator=g) * 0.2).to(torch.bfloat16)
    dy = (torch.randn(T, D, generator=g) * 1e-2).to(torch.bfloat16)
    dgu8, a3, a4 = O.down_dgrad_swiglu(dy, wd, gu8, s, I)
    gg = (gu8[:, :I].double() / 8.0).requires_grad_(True)
    uu = (gu8[:, I:].double() / 8.0).requires_grad_(True)
    dh = dy.double() @ wd.double()
    dgate, dup = torch.autograd.grad((torch.nn.functional.silu(gg) * uu * dh).sum(), [gg, uu])
    want = torch.cat([dgate, dup], 1)
    got = O.f(dgu8).double() / 2.0 ** 12
    # e5m2 has 2 mantissa bits: one step is 25 % relative; dh's bf16 rounding moves a value < 1 %
    assert torch.all((got - want).abs() <= 0.26 * want.abs() + 2.0 ** -16 / 2.0 ** 12)
    assert abs(a3.item() - want.abs().max().item()) <= 0.01 * want.abs().max().item()
    assert a4.item() == dy.float().abs().max().item()


def test_norm_backward_is_derivative():
    g = torch.Generator().manual_seed(8)
    h = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    w = torch.empty(64).uniform_(0.5, 1.5, generator=g)
    dxn = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    dy = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    rstd = O.norm_stats(h, 1e-6)
    dh, dnw = O.norm_bwd(h, rstd, dxn, dy, w)
    x = h.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    n = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * wd
    gx, gw = torch.autograd.grad((n * dxn.double()).sum() + (x * dy.double()).sum(), [x, wd])
    torch.testing.assert_close(dh.double(), gx.to(torch.bfloat16).double(), rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(dnw.double(), gw, rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------ the block
def _block_inputs(seed=0, T=1000, D=256, I=768, wstd=0.05):
    torch.manual_seed(seed)
    nw = torch.empty(D).uniform_(0.5, 1.5)
    wgu = torch.randn(2 * I, D) * wstd
    wd = torch.randn(D, I) * wstd
    h = torch.randn(T, D).to(torch.bfloat16)
    probe = torch.randn(T, D)
    return h, nw, wgu, wd, probe


def _oracle_step(h, nw, wgu, wd, probe, scale, amax, oracle=O):
    y, saved = oracle.block_forward(h, nw, wgu, wd, scale, amax, 1e-6)
    grads, _ = oracle.block_backward(probe.to(torch.bfloat16), saved, scale, amax)
    return (y,) + grads


def _errors(out, ref, h):
    errs = {}
    for name, a, r in zip(("y", "dh", "dnw", "dwgu", "dwd"), out, ref):
        if name == "y":
            a, r = a.float() - h.float(), r - h.float()
        errs[name] = O.rel_l2(a.float(), r)
    return errs


def test_block_tracks_fp32_reference():
    """spark-gpt tests/test_fp8_mlp.py:10-53 protocol and bound, on the oracle."""
    h, nw, wgu, wd, probe = _block_inputs()
    scale, amax = torch.ones(5), torch.zeros(5)
    _oracle_step(h, nw, wgu, wd, probe, scale, amax)
    assert bool((amax > 0).all())
    O.update_scales(scale, amax)
    assert bool((amax == 0).all())
    out = _oracle_step(h, nw, wgu, wd, probe, scale, amax)
    ref = O.fp32_reference(h, nw, wgu, wd, probe.to(torch.bfloat16).float())
    errs = _errors(out, ref, h)
    assert all(e < 0.12 for e in errs.values()), errs
    # and it is FP8-grade, not exact: 5-8% per element (CHANGES.md:372-373)
    assert all(e > 0.01 for e in errs.values()), errs


def _plant(monkeypatch, kind):
    """Plant one plausible mistake in the oracle."""
    if kind == "swap_gate_up":
        orig = O.swiglu_fwd
        monkeypatch.setattr(O, "swiglu_fwd", lambda x8, w8, s, ws, I: orig(
            x8, torch.cat([w8[I:], w8[:I]]), s, ws, I))
    elif kind == "transposed_down":
        orig = O.down_fwd
        monkeypatch.setattr(O, "down_fwd", lambda h8, wd8, res, s, ws: orig(
            h8, wd8.reshape(wd8.shape[1], wd8.shape[0]).t().contiguous(), res, s, ws))
    elif kind == "drop_residual_grad":
        orig = O.norm_bwd
        monkeypatch.setattr(O, "norm_bwd", lambda h, r, dxn, dy, w: (
            (orig(h, r, dxn, dy, w)[0].float() - dy.float()).to(torch.bfloat16), orig(h, r, dxn, dy, w)[1]))
    elif kind == "wgrad_not_dequantized":
        orig = O.down_wgrad
        monkeypatch.setattr(O, "down_wgrad", lambda dy, h8, s: orig(dy, h8, s) * (s[4] * s[2]))
    elif kind == "sigmoid_of_up":
        orig = O.down_dgrad_swiglu

        def swapped(dy, wd, gu8, s, I):
            return orig(dy, wd, torch.cat([gu8[:, I:], gu8[:, :I]], 1), s, I)
        monkeypatch.setattr(O, "down_dgrad_swiglu", swapped)


@pytest.mark.parametrize("kind", ["swap_gate_up", "transposed_down", "drop_residual_grad",
                                  "wgrad_not_dequantized", "sigmoid_of_up"])
def test_planted_mistakes_fail_the_reference_bound(monkeypatch, kind):
    h, nw, wgu, wd, probe = _block_inputs(seed=1, D=256, I=512)
    _plant(monkeypatch, kind)
    scale, amax = torch.ones(5), torch.zeros(5)
    _oracle_step(h, nw, wgu, wd, probe, scale, amax)
    O.update_scales(scale, amax)
    out = _oracle_step(h, nw, wgu, wd, probe, scale, amax)
    ref = O.fp32_reference(h, nw, wgu, wd, probe.to(torch.bfloat16).float())
    errs = _errors(out, ref, h)
    assert max(errs.values()) > 0.12, errs


def test_transposed_copies_and_saved_state():
    h, nw, wgu, wd, probe = _block_inputs(T=130, D=128, I=256)
    scale, amax = torch.tensor([8.0, 4.0, 4.0, 1024.0, 2.0 ** 14]), torch.zeros(5)
    y, saved = O.block_forward(h, nw, wgu, wd, scale, amax, 1e-6)
    assert torch.equal(saved["x8t"].view(torch.uint8), saved["x8"].view(torch.uint8).t())
    assert saved["gu8"].shape == (130, 512) and saved["h8"].shape == (130, 256)
    assert saved["wd"].dtype == torch.bfloat16
    assert y.dtype == torch.bfloat16
