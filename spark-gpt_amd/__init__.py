"""MI355X-native SwiGLU MLP paths of spark-gpt: the FP8 block and experts, and the
bf16 fused SwiGLU (gfx950 HIP kernels behind a C ABI).

Import as ``spark_gpt_amd`` (the repository-root module of that name loads
this directory as the package).
"""
from .mlp import (FP8_HEADROOM_BINADES, FP8_SITE_MAX, MLP, _FP8MLPBlock, _use_fp8_mlp,
                  fp8_mlp_block, fp8_update_scales, make_fp8_mlp_guard, set_fp8_mlp)
from .moe import _FP8Experts, _use_fp8_moe, make_fp8_moe_guard
from .swiglu import (_FusedSwiGLU, _NormSwiGLU, _use_fused_norm_mlp, _use_fused_swiglu, make_fused_norm_mlp_guard,
                     make_fused_swiglu_guard)
from .muon import _momentum_stage, _momentum_stage_supported
from . import mlp, moe, muon, ops, swiglu, torch_ops

__all__ = [
    "FP8_HEADROOM_BINADES", "FP8_SITE_MAX", "MLP", "_FP8MLPBlock", "_use_fp8_mlp",
    "fp8_mlp_block", "fp8_update_scales", "make_fp8_mlp_guard", "mlp", "ops", "set_fp8_mlp", "torch_ops",
    "_FP8Experts", "_use_fp8_moe", "make_fp8_moe_guard", "moe",
    "_FusedSwiGLU", "_NormSwiGLU", "_use_fused_norm_mlp", "_use_fused_swiglu", "make_fused_norm_mlp_guard",
    "make_fused_swiglu_guard", "swiglu", "_momentum_stage", "_momentum_stage_supported", "muon",
]


def __getattr__(name):
    # FP8_MLP is read from the submodule, where set_fp8_mlp rebinds it
    if name == "FP8_MLP":
        return mlp.FP8_MLP
    raise AttributeError(name)
