"""ctypes binding of ``libsparkfp8.so`` (declared in ``include/sparkfp8.h``).

There is no fallback: if the library is missing, or a tensor is not on a
ROCm device, the call raises.  torch is imported first so the library binds
to the HIP runtime torch already loaded (same soname, one runtime per process).
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsparkfp8.so")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_INT = ctypes.c_int

# name -> (restype, argtypes); must match include/sparkfp8.h
SIGNATURES = {
    "sfp8_quant_e4m3_rowcol": (_INT, [_P, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "sfp8_norm_quant": (_INT, [_P, _P, _I64, _I64, _F32, _P, _P, _P, _P, _I64, _P, _P]),
    "sfp8_weight_quant": (_INT, [_P, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P]),
    "sfp8_update_scales": (_INT, [_P, _P, _I64, _P]),
    "sfp8_block_weight_quant": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P]),
    "sfp8_gemm_gateup_swiglu_fwd": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "sfp8_gemm_down_fwd": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _P]),
    "sfp8_gemm_down_dgrad_swiglu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "sfp8_gemm_gateup_dgrad": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _P]),
    "sfp8_gemm_wgrad": (_INT, [_P, _INT, _P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "sfp8_wgrad_splits": (_I64, [_I64, _I64, _I64]),
    "sfp8_wgrad_workspace_floats": (_I64, [_I64, _I64, _I64]),
    "sfp8_slab_bytes": (_I64, [_I64, _I64]),
    "sfp8_norm_bwd": (_INT, [_P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _I64, _P, _P, _I64, _P]),
    "sfp8_norm_bwd_partials": (_I64, [_I64, _I64]),
    "sfp8_norm_bwd_noalloc": (_INT, [_P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "sfp8_moe_plan_ints": (_I64, [_I64, _I64]),
    "sfp8_moe_padded_rows": (_I64, [_I64, _I64]),
    "sfp8_moe_plan": (_INT, [_P, _I64, _I64, _P, _I64, _P]),
    "sfp8_moe_rows_quant": (_INT, [_P, _I64, _I64, _P, _I64, _P, _I64, _P, _INT, _P, _INT, _INT, _P, _P, _P]),
    "sfp8_weight_quant_experts": (_INT, [_P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P]),
    "sfp8_moe_gemm_gateup_swiglu_fwd": (_INT, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P]),
    "sfp8_moe_gemm_down_fwd": (_INT, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _I64, _P]),
    "sfp8_moe_gemm_down_dgrad_swiglu": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P]),
    "sfp8_moe_gemm_gateup_dgrad": (_INT, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _I64, _P]),
    "sfp8_moe_wgrad_splits": (_I64, [_I64, _I64, _I64]),
    "sfp8_moe_wgrad_workspace_floats": (_I64, [_I64, _I64, _I64]),
    "sfp8_moe_gemm_wgrad": (_INT, [_P, _INT, _P, _INT, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P, _I64, _P]),
    "sfp8_moe_wgrad_rows_workspace_floats": (_I64, [_I64, _I64, _I64]),
    "sfp8_moe_gemm_wgrad_rows": (_INT, [_P, _INT, _INT, _P, _INT, _INT, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P, _I64,
                                        _P]),
    "sfp8_moe_topk_sum": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _P]),
    # bf16 SwiGLU path
    "sfp8_bf16_slab_bytes": (_I64, [_I64, _I64]),
    "sfp8_bf16_weight_slabs": (_INT, [_P, _INT, _P, _I64, _I64, _I64, _P, _P, _P]),
    "sfp8_bf16_rows_prep": (_INT, [_P, _I64, _I64, _P, _I64, _F32, _P, _P, _P, _P]),
    "sfp8_bf16_gemm_swiglu_fwd": (_INT, [_P, _INT, _P, _I64, _I64, _I64, _P, _P, _P, _P]),
    "sfp8_bf16_moe_gemm_swiglu_fwd": (_INT, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P]),
    "sfp8_bf16_swiglu_bwd": (_INT, [_P, _P, _I64, _I64, _P, _P, _I64, _P, _P, _P]),
    "sfp8_bf16_gemm": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "sfp8_bf16_moe_gemm": (_INT, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "sfp8_bf16_norm_dh": (_INT, [_P, _P, _P, _I64, _I64, _P, _P]),
    "sfp8_bf16_wgrad_splits": (_I64, [_I64, _I64, _I64]),
    "sfp8_bf16_wgrad_workspace_floats": (_I64, [_I64, _I64, _I64]),
    "sfp8_bf16_gemm_wgrad": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "sfp8_bf16_moe_wgrad_workspace_floats": (_I64, [_I64, _I64, _I64]),
    "sfp8_bf16_moe_gemm_wgrad": (_INT, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P]),
    "sfp8_bf16_gemm_wgrad_rows": (_INT, [_P, _P, _INT, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "sfp8_bf16_moe_gemm_wgrad_rows": (_INT, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P]),
    "sfp8_bf16_fold_partials": (_I64, [_I64, _I64]),
    "sfp8_bf16_fold_grads": (_INT, [_P, _P, _P, _I64, _I64, _P, _P, _P, _I64, _P]),
    "sfp8_wgrad_rows_workspace_floats": (_I64, [_I64, _I64, _I64]),
    "sfp8_gemm_wgrad_rows": (_INT, [_P, _INT, _INT, _P, _INT, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    # the optimizer's momentum stage, and the weight gradient fused with it
    "sfp8_momentum_stage": (_INT, [_P, _P, _P, _I64, _F32, _F32, _P]),
    "sfp8_wgrad_momentum_workspace_floats": (_I64, [_I64, _I64, _I64]),
    "sfp8_gemm_wgrad_momentum": (_INT, [_P, _INT, _INT, _P, _INT, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _F32, _F32,
                                        _P, _I64, _P]),
}

ERRORS = {
    -1: "null pointer argument",
    -2: "unsupported shape",
    -3: "misaligned pointer (16-byte alignment required)",
    -4: "workspace too small",
    -5: "shape beyond the allocation-free entry point's fixed scratch",
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load the library once (thread-safe); raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                    "(there is no non-HIP fallback)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, name: str) -> None:
    if rc != 0:
        msg = ERRORS.get(rc, f"HIP error {rc}")
        raise RuntimeError(f"{name} failed: {msg}")


def call(name: str, *args) -> None:
    rc = getattr(_lib or load(), name)(*args)
    if rc != 0:
        check(rc, name)


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """Handle of torch's current stream on t's device (the stream every call
    is launched on)."""
    if not t.is_cuda:
        raise RuntimeError("libsparkfp8 kernels need ROCm device tensors")
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
