"""The oracle against the committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py): bit-exact for every byte, scale and amax; the
oracle's own float outputs to fp32 rounding (torch CPU matmul order)."""
import json
import os
import struct

import numpy as np
import pytest
import torch

from oracle import fp8_bits, fp8_mlp as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def hexf(s: str) -> float:
    return struct.unpack(">f", bytes.fromhex(s))[0]


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).numpy()


def test_cast_fixture_vs_closed_form():
    """torch's library cast (the fixture) and the oracle's closed-form RNE agree
    on every bf16 pattern at every stored scale, NaN and saturation included."""
    z = load("cast_bf16_all.npz")
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float().numpy()
    with np.errstate(over="ignore", invalid="ignore"):
        _check_closed_form(z, x)


def _check_closed_form(z, x):
    for i, k in enumerate(z["log2s_e4m3"]):
        assert np.array_equal(fp8_bits.cast_e4m3(np.clip(x * 2.0 ** int(k), -448, 448)), z["e4m3"][i]), k
    for i, k in enumerate(z["log2s_e5m2"]):
        assert np.array_equal(fp8_bits.cast_e5m2(np.clip(x * 2.0 ** int(k), -57344, 57344)), z["e5m2"][i]), k


def test_cast_fixture_vs_oracle_torch_path():
    z = load("cast_bf16_all.npz")
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    assert np.array_equal(u8(O.e4m3(x * 2.0 ** int(z["log2s_e4m3"][1]))), z["e4m3"][1])
    assert np.array_equal(u8(O.e5m2(x * 2.0 ** int(z["log2s_e5m2"][1]))), z["e5m2"][1])


def test_scale_kat_vs_closed_form():
    """Band-edge amax values: the closed-form pow2 scale (exact exponent plus
    the enumerated log2 band) equals the reference expression's result."""
    kat = json.load(open(os.path.join(GOLDEN, "scale_kat.json")))
    cases = kat["cases"]
    assert len(cases) > 1000
    amax = np.array([hexf(c[0]) for c in cases], np.float32)
    want4 = np.array([hexf(c[1]) for c in cases], np.float32)
    want5 = np.array([hexf(c[2]) for c in cases], np.float32)
    wantq = np.array([hexf(c[3]) for c in cases], np.float32)
    old = np.float32(hexf(kat["old_scale"]))
    pos = amax > 0
    got4 = np.where(pos, fp8_bits.pow2_scale(amax, 448.0, 1), old)
    got5 = np.where(pos, fp8_bits.pow2_scale(amax, 57344.0, 1), old)
    gotq = fp8_bits.pow2_scale(np.maximum(amax, np.float32(1e-30)), 448.0, 0, recip_first=True)
    assert np.array_equal(got4.view(np.uint32), want4.view(np.uint32))
    assert np.array_equal(got5.view(np.uint32), want5.view(np.uint32))
    assert np.array_equal(gotq.view(np.uint32), wantq.view(np.uint32))


def test_scale_kat_vs_oracle_roll():
    kat = json.load(open(os.path.join(GOLDEN, "scale_kat.json")))
    amax = torch.tensor([hexf(c[0]) for c in kat["cases"]], dtype=torch.float32)
    n = amax.numel()
    s = torch.full((n, 5), hexf(kat["old_scale"]))
    am = amax[:, None].repeat(1, 5)
    O.update_scales(s, am)  # one 5-slot set per row
    want4 = torch.tensor([hexf(c[1]) for c in kat["cases"]])
    want5 = torch.tensor([hexf(c[2]) for c in kat["cases"]])
    assert torch.equal(s[:, 0], want4) and torch.equal(s[:, 2], want4)
    assert torch.equal(s[:, 3], want5) and torch.equal(s[:, 4], want5)
    assert torch.all(am == 0)


def test_quant_fixture():
    z = load("quant_64x256.npz")
    x = bf16(z["x"])
    x8, x8t, a = O.quant_rowcol(x, torch.tensor(float(z["scale"])))
    assert np.array_equal(u8(x8), z["x8"]) and np.array_equal(u8(x8t), z["x8t"])
    assert np.float32(a) == z["amax"]
    # the next scale from this amax (one binade of headroom)
    assert fp8_bits.pow2_scale(np.float32(z["amax"]), 448.0, 1) == z["next_scale"]


def test_norm_fixture():
    z = load("norm_quant_40x128.npz")
    x8, _, rstd, a = O.norm_quant(bf16(z["h"]), torch.from_numpy(z["norm_w"]), torch.tensor(float(z["s0"])),
                                  float(z["eps"]))
    assert np.array_equal(u8(x8), z["x8"])
    assert np.array_equal(rstd.numpy().view(np.uint32), z["rstd"].view(np.uint32))
    assert np.float32(a) == z["amax"]
    # the zero row: rstd = 1/sqrt(eps) in the fp64 spec, all-zero bytes
    assert np.all(z["x8"][7] == 0)


def test_block_fixture():
    z = load("block_T80_D128_I128.npz")
    threads = torch.get_num_threads()
    torch.set_num_threads(1)  # the fixture's summation order
    try:
        scale = torch.from_numpy(z["scale"].copy())
        amax = torch.zeros(5)
        params = [torch.from_numpy(z[k].copy()) for k in ("norm_w", "w_gu", "w_down")]
        y, saved = O.block_forward(bf16(z["h"]), *params, scale, amax, float(z["eps"]))
        (dh, dnw, dwgu, dwd), inter = O.block_backward(bf16(z["dy"]), saved, scale, amax)
    finally:
        torch.set_num_threads(threads)
    assert np.array_equal(u8(saved["x8"]), z["x8"])
    assert np.array_equal(saved["wscale"].numpy(), z["wscale"])
    for name, t in (("gu8", saved["gu8"]), ("h8", saved["h8"]), ("dgu8", inter["dgu8"])):
        assert np.array_equal(u8(t), z[name]), name
    for name, t in (("y", y), ("dh", dh)):
        assert np.array_equal(t.view(torch.int16).numpy().view(np.uint16), z[name]), name
    for name, t in (("dnw", dnw), ("dw_gu", dwgu), ("dw_down", dwd), ("amax", amax)):
        np.testing.assert_allclose(t.numpy(), z[name], rtol=1e-6, atol=0, err_msg=name)


@pytest.mark.parametrize("name", ["cast_bf16_all.npz", "quant_64x256.npz", "norm_quant_40x128.npz",
                                  "block_T80_D128_I128.npz"])
def test_fixtures_hold_plain_arrays(name):
    """Fixtures are data only: every member loads without pickle."""
    z = load(name)
    assert all(z[k].dtype != object for k in z.files)
