"""GPU kernels against the committed golden fixtures (tests/golden/): FP8
bytes, scales and amax bit-exact; the block's bf16/fp32 outputs within rel-L2
1e-2 (the MFMA accumulates in a different order than the CPU matmul)."""
import json
import os
import struct

import numpy as np
import pytest
import torch

import spark_gpt_amd as sg

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def hexf(s: str) -> float:
    return struct.unpack(">f", bytes.fromhex(s))[0]


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).cpu().numpy()


def rel_l2(a: torch.Tensor, r: torch.Tensor) -> float:
    a, r = a.detach().double().cpu(), r.detach().double().cpu()
    return float((a - r).norm() / r.norm().clamp(min=1e-300))


def test_quantizer_casts_every_bf16_pattern(dev):
    z = load("cast_bf16_all.npz")
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).reshape(512, 128)
    for i, k in enumerate(z["log2s_e4m3"]):
        scale = torch.tensor([2.0 ** int(k), 1, 1, 1, 1], device=dev)
        x8, x8t = sg.ops.quant_e4m3_rowcol(x.to(dev), scale, torch.zeros(5, device=dev))
        assert np.array_equal(u8(x8).reshape(-1), z["e4m3"][i]), k
        assert np.array_equal(u8(sg.ops.unslab(x8t, 128))[:, :512].T.reshape(-1), z["e4m3"][i]), k


def test_dy_cast_every_bf16_pattern(dev):
    """e5m2 bytes of dy * s4 (the norm backward's transposed copy)."""
    z = load("cast_bf16_all.npz")
    dy = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).reshape(256, 256)
    T, D = dy.shape
    zt = torch.zeros(T, D, dtype=torch.bfloat16, device=dev)
    for i, k in enumerate(z["log2s_e5m2"]):
        scale = torch.tensor([1, 1, 1, 1, 2.0 ** int(k)], device=dev)
        _, _, dy8t = sg.ops.norm_bwd(zt, torch.ones(T, device=dev), zt, dy.to(dev), torch.ones(D, device=dev),
                                     scale, torch.zeros(5, device=dev))
        assert np.array_equal(u8(sg.ops.unslab(dy8t, D))[:, :T].T.reshape(-1), z["e5m2"][i]), k


def test_scale_roll_kat(dev):
    kat = json.load(open(os.path.join(GOLDEN, "scale_kat.json")))
    amax = torch.tensor([hexf(c[0]) for c in kat["cases"]], dtype=torch.float32)
    n = amax.numel()
    scale = torch.full((n * 5,), hexf(kat["old_scale"]), device=dev)
    am = amax[:, None].repeat(1, 5).reshape(-1).contiguous().to(dev)
    sg.ops.update_scales(scale, am)
    s = scale.view(n, 5).cpu()
    want4 = torch.tensor([hexf(c[1]) for c in kat["cases"]])
    want5 = torch.tensor([hexf(c[2]) for c in kat["cases"]])
    for j in range(3):
        assert torch.equal(s[:, j].view(torch.int32), want4.view(torch.int32)), j
    for j in (3, 4):
        assert torch.equal(s[:, j].view(torch.int32), want5.view(torch.int32)), j
    assert torch.all(am.cpu() == 0)


def test_weight_scale_kat(dev):
    """q = 2^floor(log2(448 / amax)) over the band-edge amax values, each as the
    one non-zero element of a 128 x 128 master."""
    kat = json.load(open(os.path.join(GOLDEN, "scale_kat.json")))
    cases = [c for c in kat["cases"] if 0 < hexf(c[0]) < float("inf")]
    q = torch.zeros(1, device=dev)
    w = torch.zeros(128, 128, device=dev)
    got, want = [], []
    for c in cases[::7]:
        w[5, 77] = hexf(c[0])
        sg.ops.weight_quant(w, q)
        got.append(q.clone())
        want.append(hexf(c[3]))
    got = torch.cat(got).cpu()
    assert torch.equal(got.view(torch.int32), torch.tensor(want).view(torch.int32))


def test_quantizer_fixture(dev):
    z = load("quant_64x256.npz")
    scale = torch.tensor([float(z["scale"]), 1, 1, 1, 1], device=dev)
    amax = torch.zeros(5, device=dev)
    x8, x8t = sg.ops.quant_e4m3_rowcol(bf16(z["x"]).to(dev), scale, amax)
    assert np.array_equal(u8(x8), z["x8"])
    xt = u8(sg.ops.unslab(x8t, z["x8t"].shape[0]))
    assert np.array_equal(xt[:, :64], z["x8t"])
    assert np.all(xt[:, 64:] == 0)
    assert np.float32(amax[0].item()) == z["amax"]
    sg.ops.update_scales(scale, amax)
    assert np.float32(scale[0].item()) == z["next_scale"]


def test_norm_quant_fixture(dev):
    z = load("norm_quant_40x128.npz")
    scale = torch.tensor([float(z["s0"]), 1, 1, 1, 1], device=dev)
    amax = torch.zeros(5, device=dev)
    x8, x8t, rstd = sg.ops.norm_quant(bf16(z["h"]).to(dev), torch.from_numpy(z["norm_w"]).to(dev), scale, amax,
                                      float(z["eps"]))
    assert np.array_equal(u8(sg.ops.unslab(x8, z["x8"].shape[0])), z["x8"])
    assert np.array_equal(rstd.cpu().numpy().view(np.uint32), z["rstd"].view(np.uint32))
    assert np.float32(amax[0].item()) == z["amax"]


def test_block_fixture(dev):
    """The whole block at T=80 (ragged), D=128, I=128 with the fixture's rolled
    scales: outputs and grads within rel-L2 1e-2, amax slots 0 and 4 exact,
    the others within 2 %; the norm-quantized activations bit-exact."""
    z = load("block_T80_D128_I128.npz")
    h = bf16(z["h"]).to(dev)
    params = [torch.from_numpy(z[k].copy()).to(dev).requires_grad_(True) for k in ("norm_w", "w_gu", "w_down")]
    scale = torch.from_numpy(z["scale"].copy()).to(dev)
    amax = torch.zeros(5, device=dev)
    x = h.clone().requires_grad_(True)
    y = sg._FP8MLPBlock.apply(x, *params, scale, amax, float(z["eps"]))
    grads = torch.autograd.grad(y, [x] + params, bf16(z["dy"]).to(dev))
    hf = h.float().cpu()
    assert rel_l2(y.float().cpu() - hf, bf16(z["y"]).float() - hf) < 1e-2
    for name, g in zip(("dh", "dnw", "dw_gu", "dw_down"), grads):
        ref = bf16(z[name]).float() if name == "dh" else torch.from_numpy(z[name])
        assert torch.isfinite(g).all(), name
        assert rel_l2(g.float(), ref) < 1e-2, name
    a = amax.cpu().numpy()
    assert a[0] == z["amax"][0] and a[4] == z["amax"][4]
    np.testing.assert_allclose(a, z["amax"], rtol=2e-2)
    x8, _, _ = sg.ops.norm_quant(h, params[0].detach(), scale, torch.zeros(5, device=dev), float(z["eps"]))
    assert np.array_equal(u8(sg.ops.unslab(x8, h.shape[0])), z["x8"])
