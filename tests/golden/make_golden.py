"""Writes the golden fixtures of this directory (run from the repository root:
``python tests/golden/make_golden.py``).

The reference holds no golden vectors for the FP8 MLP path (its only test,
spark-gpt tests/test_fp8_mlp.py, is tolerance-based), so the fixtures come from
two sources, named per file:

* library routines -- torch CPU's ``.to(float8_e4m3fn / float8_e5m2)`` cast
  (round-to-nearest-even) and the reference's own torch expressions for the
  scale roll and the weight scale (train.py:942-945, 951), evaluated by torch;
* the oracle (oracle/fp8_mlp.py) for the fused kernels, whose arithmetic no
  library routine covers.  These pin the GPU kernels and any later change of
  the oracle to the values committed here.

Every input is seed-fixed; every array is stored as raw bits (bf16 as uint16,
fp8 as uint8, fp32 as float32) in compressed ``.npz`` files or JSON.
"""
from __future__ import annotations

import json
import os
import struct
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import fp8_mlp as O  # noqa: E402

E4M3_LOG2S = (-9, 0, 7)
E5M2_LOG2S = (-16, 0, 9)


def bits_bf16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def bits_fp8(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).numpy()


def f32_hex(x: float) -> str:
    return struct.pack(">f", x).hex()


def all_bf16() -> torch.Tensor:
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def cast_kat() -> dict:
    """Every bf16 bit pattern times 2^k, clamped to the format maximum and cast
    by torch (train.py:972, 1016, 1094 clamp before the cast)."""
    x = all_bf16().float()
    out = {"log2s_e4m3": np.array(E4M3_LOG2S, np.int32), "log2s_e5m2": np.array(E5M2_LOG2S, np.int32)}
    out["e4m3"] = np.stack([bits_fp8((x * 2.0 ** k).clamp(-448.0, 448.0).to(torch.float8_e4m3fn))
                            for k in E4M3_LOG2S])
    out["e5m2"] = np.stack([bits_fp8((x * 2.0 ** k).clamp(-57344.0, 57344.0).to(torch.float8_e5m2))
                            for k in E5M2_LOG2S])
    return out


def amax_cases() -> list[float]:
    """Amax values around every band edge fmax * 2^-k (a few fp32 ulps either
    side), seed-fixed random values, and the special cases."""
    vals = [0.0, 1e-30, 1e-38, 1e-45, 3.4e38, float("inf")]
    for fmax in (448.0, 57344.0):
        for k in range(-24, 40):
            edge = np.float32(fmax * 2.0 ** -k)
            v = edge
            for _ in range(4):
                v = np.nextafter(v, np.float32(np.inf))
                vals.append(float(v))
            v = edge
            for _ in range(4):
                v = np.nextafter(v, np.float32(0))
                vals.append(float(v))
            vals.append(float(edge))
    g = torch.Generator().manual_seed(11)
    vals += (torch.rand(200, generator=g) * 40 - 20).exp2().tolist()
    return [float(np.float32(v)) for v in vals]


def scale_kat() -> dict:
    """Next scale per amax: the scale roll of train.py:942-945 (five sites, one
    binade of headroom, amax == 0 keeps the old scale) and the weight scale of
    train.py:951 (no headroom), each evaluated with the reference's torch
    expression."""
    amax = torch.tensor(amax_cases(), dtype=torch.float32)
    rows = []
    old = torch.full((5,), 0.25)
    fmax = torch.tensor(O.FP8_SITE_MAX)
    for a in amax:
        am = a.repeat(5)
        new = torch.exp2(torch.floor(torch.log2(fmax / am.clamp(min=1e-30))) - O.FP8_HEADROOM_BINADES)
        roll = torch.where(am > 0, new, old)
        q = torch.exp2(torch.floor(torch.log2(448.0 / a.clamp(min=1e-30))))
        rows.append([f32_hex(float(a)), f32_hex(float(roll[0])), f32_hex(float(roll[3])), f32_hex(float(q))])
    return {"old_scale": f32_hex(0.25), "columns": ["amax", "roll_e4m3", "roll_e5m2", "weight_q"],
            "cases": rows}


def quant_fixture() -> dict:
    """Standalone quantizer: 64 x 256 bf16 ~N(0,1), columns 3 and 200 scaled
    x50; scale from a prewarm roll of the input's own amax."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 256, generator=g)
    x[:, [3, 200]] *= 50
    x = x.to(torch.bfloat16)
    scale = torch.ones(5)
    amax = torch.zeros(5)
    amax[0] = O.amax_of(x)
    O.update_scales(scale, amax)
    x8, x8t, a = O.quant_rowcol(x, scale[0])
    nxt = scale.clone()
    am = torch.zeros(5)
    am[0] = a
    O.update_scales(nxt, am)
    return {"x": bits_bf16(x), "scale": np.float32(scale[0]), "x8": bits_fp8(x8), "x8t": bits_fp8(x8t),
            "amax": np.float32(a), "next_scale": np.float32(nxt[0])}


def norm_fixture() -> dict:
    """Norm-fused quantizer: 40 x 128 bf16 rows (row 7 all zero, row 9 scaled
    x1000), norm weight ~U(0.5, 1.5), s0 = 2^5, eps 1e-6."""
    g = torch.Generator().manual_seed(4)
    h = torch.randn(40, 128, generator=g)
    h[7] = 0
    h[9] *= 1000
    h = h.to(torch.bfloat16)
    nw = torch.rand(128, generator=g) + 0.5
    s0 = torch.tensor(32.0)
    x8, x8t, rstd, a0 = O.norm_quant(h, nw, s0, 1e-6)
    return {"h": bits_bf16(h), "norm_w": nw.numpy(), "s0": np.float32(s0), "eps": np.float32(1e-6),
            "x8": bits_fp8(x8), "rstd": rstd.numpy(), "amax": np.float32(a0)}


def block_fixture() -> dict:
    """Whole block at T=80 (a ragged tail of every 256-row tile), D=128,
    I=128: one prewarm step, the scale roll, then the recorded step."""
    T, D, I = 80, 128, 128
    g = torch.Generator().manual_seed(80)
    h = torch.randn(T, D, generator=g).to(torch.bfloat16)
    nw = torch.rand(D, generator=g) + 0.5
    # bf16-valued fp32 masters (the fixture stores them compactly)
    w_gu = (torch.randn(2 * I, D, generator=g) * D ** -0.5).to(torch.bfloat16).float()
    w_down = (torch.randn(D, I, generator=g) * I ** -0.5).to(torch.bfloat16).float()
    dy = (torch.randn(T, D, generator=g) * 1e-3).to(torch.bfloat16)
    scale, amax = torch.ones(5), torch.zeros(5)
    _, saved = O.block_forward(h, nw, w_gu, w_down, scale, amax, 1e-6)
    O.block_backward(dy, saved, scale, amax)
    O.update_scales(scale, amax)
    s = scale.clone()
    y, saved = O.block_forward(h, nw, w_gu, w_down, scale, amax, 1e-6)
    (dh, dnw, dwgu, dwd), inter = O.block_backward(dy, saved, scale, amax)
    return {"h": bits_bf16(h), "norm_w": nw.numpy(), "w_gu": w_gu.numpy(), "w_down": w_down.numpy(),
            "dy": bits_bf16(dy), "scale": s.numpy(), "eps": np.float32(1e-6),
            "y": bits_bf16(y), "dh": bits_bf16(dh), "dnw": dnw.numpy(), "dw_gu": dwgu.numpy(),
            "dw_down": dwd.numpy(), "amax": amax.numpy(), "wscale": saved["wscale"].numpy(),
            "x8": bits_fp8(saved["x8"]), "gu8": bits_fp8(saved["gu8"]), "h8": bits_fp8(saved["h8"]),
            "dgu8": bits_fp8(inter["dgu8"]), "rstd": saved["rstd"].numpy()}


def main() -> None:
    torch.set_num_threads(1)  # fixed summation order in the oracle's matmuls
    np.savez_compressed(os.path.join(HERE, "cast_bf16_all.npz"), **cast_kat())
    with open(os.path.join(HERE, "scale_kat.json"), "w") as fh:
        json.dump(scale_kat(), fh, separators=(",", ":"))
    np.savez_compressed(os.path.join(HERE, "quant_64x256.npz"), **quant_fixture())
    np.savez_compressed(os.path.join(HERE, "norm_quant_40x128.npz"), **norm_fixture())
    np.savez_compressed(os.path.join(HERE, "block_T80_D128_I128.npz"), **block_fixture())
    for n in sorted(os.listdir(HERE)):
        print(f"{n:32s} {os.path.getsize(os.path.join(HERE, n)):8d} B")


if __name__ == "__main__":
    main()
