"""Benchmark: FP8 SwiGLU MLP block fwd+bwd on one MI355X.

Workload (default): tokens=65536, d_model=1024, ffn=3072 (Qwen3-0.6B width),
bf16 inputs ~N(0,1), weights ~N(0,1/fan_in), upstream grads ~N(0,1e-3),
seed-fixed, after one prewarm step + scale roll.  A step is one forward and
backward of the block (7-argument autograd Function, all kernels on the
current stream).  Value = 18*T*D*I FLOP / step time, in TFLOP/s.

Also reported on the same JSON line:
  roofline      the dominant GEMM kernel, timed alone with HIP events on the
                stream it runs on; algorithmic FLOP per launch / mean duration
                vs the 5.0 PFLOP/s dense FP8 MFMA peak
  quantizer     the standalone quantizer (bf16 65536x4096 with 0.1% x50 outlier
                columns -> e4m3 row-major + transposed + amax): 4 B/element
                algorithmic traffic / mean duration vs 8 TB/s HBM
  kernels       per-kernel mean durations of one step
  cpu_baseline  the same FP8 recipe emulated in torch on the host cores (the
                CPU oracle) on a bounded token sample, in TFLOP/s
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP8_PEAK_TFLOPS = 5033.0   # MI355X dense FP8 MFMA (256 CU x 2.4 GHz x 8192 FLOP/clk)
HBM_PEAK_GBPS = 8000.0     # MI355X HBM3E


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--tokens", type=int, default=65536)
    p.add_argument("--d-model", type=int, default=1024)
    p.add_argument("--ffn", type=int, default=3072)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-tokens", type=int, default=16384)
    p.add_argument("--quant-rows", type=int, default=65536)
    p.add_argument("--quant-cols", type=int, default=4096)
    return p.parse_args()


def timed_launches(fn, reps: int, stream) -> float:
    """Mean ms per call of fn() over reps calls, HIP events on `stream`."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / reps


def cpu_baseline(T: int, D: int, I: int) -> dict:
    """The reference recipe emulated on the host (CPU oracle), T tokens."""
    import torch

    from oracle import fp8_mlp as O

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(2)
    h = torch.randn(T, D, generator=g).to(torch.bfloat16)
    nw = torch.ones(D)
    wgu = torch.randn(2 * I, D, generator=g) * D ** -0.5
    wd = torch.randn(D, I, generator=g) * I ** -0.5
    dy = (torch.randn(T, D, generator=g) * 1e-3).to(torch.bfloat16)
    scale, amax = torch.ones(5), torch.zeros(5)

    def step():
        y, saved = O.block_forward(h, nw, wgu, wd, scale, amax, 1e-6)
        O.block_backward(dy, saved, scale, amax)

    step()
    O.update_scales(scale, amax)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = sorted(times)[1]
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(18.0 * T * D * I / med / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"torch-CPU emulation of the FP8 recipe (oracle), fwd+bwd at tokens={T}, "
                  f"d_model={D}, ffn={I}; median of 3 steps after 1 warm-up; {med:.2f} s/step; "
                  f"cpu={cpu_model}",
    }


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the FP8 MLP path "
              "runs data-parallel with one block per GPU and no collective inside it)", file=sys.stderr)
        sys.exit(2)

    import torch

    import spark_gpt_amd as sg
    from spark_gpt_amd import ops

    dev = torch.device("cuda:0")
    T, D, I = args.tokens, args.d_model, args.ffn
    g = torch.Generator(device=dev).manual_seed(1)
    h = torch.randn(T, D, device=dev, generator=g).to(torch.bfloat16)
    nw = torch.ones(D, device=dev, requires_grad=True)
    wgu = (torch.randn(2 * I, D, device=dev, generator=g) * D ** -0.5).requires_grad_(True)
    wd = (torch.randn(D, I, device=dev, generator=g) * I ** -0.5).requires_grad_(True)
    dy = (torch.randn(T, D, device=dev, generator=g) * 1e-3).to(torch.bfloat16)
    scale = torch.ones(5, device=dev)
    amax = torch.zeros(5, device=dev)
    params = [nw, wgu, wd]

    def step():
        x = h.detach().requires_grad_(True)
        y = sg._FP8MLPBlock.apply(x, *params, scale, amax, 1e-6)
        torch.autograd.backward(y, dy, inputs=[x] + params)
        for p in params:
            p.grad = None

    step()                            # prewarm: records amax under scale 1
    ops.update_scales(scale, amax)    # roll, as the trainer does after the prewarm step
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    flop = 18.0 * T * D * I
    tflops = flop / (ms * 1e-3) / 1e12

    # ---- per-kernel timing (HIP events on the current stream) ----
    stream = torch.cuda.current_stream(dev)
    x8, x8t, rstd = ops.norm_quant(h, nw.detach(), scale, amax, 1e-6)
    wscale = torch.empty(2, device=dev)
    w8, w8t, _ = ops.weight_quant(wgu.detach(), wscale[0:1], w8=True, w8t=True)
    wd8, _, wdt = ops.weight_quant(wd.detach(), wscale[1:2], w8=True, bf16t=True)
    gu8, h8, h8t = ops.gateup_swiglu_fwd(x8, w8, scale, wscale, amax, I)
    dgu8, dgu8t = ops.down_dgrad_swiglu(dy, wdt, gu8, scale, amax)
    dxn = ops.gateup_dgrad(dgu8, w8t, scale, wscale)
    dh, dnw, dy8t = ops.norm_bwd(h, rstd, dxn, dy, nw.detach(), scale, amax)
    reps = 10
    kern = {
        "norm_quant": (lambda: ops.norm_quant(h, nw.detach(), scale, amax, 1e-6), None),
        "weight_quant_gu": (lambda: ops.weight_quant(wgu.detach(), wscale[0:1], w8=True, w8t=True), None),
        "weight_quant_down": (lambda: ops.weight_quant(wd.detach(), wscale[1:2], w8=True, bf16t=True), None),
        "gateup_swiglu_fwd": (lambda: ops.gateup_swiglu_fwd(x8, w8, scale, wscale, amax, I), 4.0 * T * D * I),
        "down_fwd": (lambda: ops.down_fwd(h8, wd8, h, scale, wscale), 2.0 * T * D * I),
        "down_dgrad_swiglu_bf16": (lambda: ops.down_dgrad_swiglu(dy, wdt, gu8, scale, amax), 2.0 * T * D * I),
        "gateup_dgrad": (lambda: ops.gateup_dgrad(dgu8, w8t, scale, wscale), 4.0 * T * D * I),
        "norm_bwd": (lambda: ops.norm_bwd(h, rstd, dxn, dy, nw.detach(), scale, amax), None),
        "wgrad_down": (lambda: ops.wgrad(dy8t, h8t, scale[4:5], scale[2:3]), 2.0 * T * D * I),
        "wgrad_gateup": (lambda: ops.wgrad(dgu8t, x8t, scale[3:4], scale[0:1]), 4.0 * T * D * I),
    }
    kernels = {}
    for name, (fn, fl) in kern.items():
        kms = timed_launches(fn, reps, stream)
        rec = {"ms": round(kms, 4)}
        if fl:
            rec["tflops"] = round(fl / (kms * 1e-3) / 1e12, 1)
        kernels[name] = rec
    # dominant kernel: the GEMM taking the most time
    gemms = {k: v for k, v in kernels.items() if "tflops" in v}
    dom = max(gemms, key=lambda k: gemms[k]["ms"])
    dom_flop = kern[dom][1]
    dom_ms = gemms[dom]["ms"]
    achieved = dom_flop / (dom_ms * 1e-3) / 1e12
    peak = FP8_PEAK_TFLOPS if "bf16" not in dom else FP8_PEAK_TFLOPS / 2
    roofline = {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 1), "peak": peak,
                "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": None,
                "flop_per_launch": dom_flop}

    # ---- standalone quantizer (HBM-bound) ----
    R, C = args.quant_rows, args.quant_cols
    gq = torch.Generator(device=dev).manual_seed(3)
    xq = torch.randn(R, C, device=dev, generator=gq)
    cols = torch.randperm(C, device=dev, generator=gq)[: max(1, C // 1000)]
    xq[:, cols] *= 50.0
    xq = xq.to(torch.bfloat16)
    qs, qa = torch.ones(5, device=dev), torch.zeros(5, device=dev)
    ops.quant_e4m3_rowcol(xq, qs, qa)
    ops.update_scales(qs, qa)
    qms = timed_launches(lambda: ops.quant_e4m3_rowcol(xq, qs, qa), 20, stream)
    qbytes = 4.0 * R * C
    qgbps = qbytes / (qms * 1e-3) / 1e9
    quant = {"rows": R, "cols": C, "ms": round(qms, 4), "GB/s": round(qgbps, 1),
             "frac_hbm": round(qgbps / HBM_PEAK_GBPS, 4), "bytes_per_launch": qbytes}
    del xq

    out = {
        "metric": "FP8 MLP fwd+bwd TFLOP/s (% FP8 MFMA peak); quantize GB/s (% HBM peak)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3/e5m2 (bf16 down dgrad)",
        "data": "synthetic: seed-fixed N(0,1) bf16 activations, N(0,1/fan_in) fp32 weights, N(0,1e-3) bf16 grads",
        "config": {"workload": "fp8_swiglu_mlp_block_fwd_bwd", "tokens": T, "d_model": D, "ffn": I,
                   "flop_per_step": flop, "frac_fp8_peak": round(tflops / FP8_PEAK_TFLOPS, 4)},
        "roofline": roofline,
        "quantizer": quant,
        "kernels": kernels,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_tokens, D, I)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
