"""CPU tests of the host side: the C-ABI library loads and exports exactly the
entry points include/sparkfp8.h declares (no kernel is launched), the device
constant tables match the oracle's derivation, and the Python mirror of the
reference interface (guard, module state, scale roll plumbing) behaves like
spark-gpt train.py:914-946 / 247-262."""
import ctypes
import os
import re

import pytest
import torch
import torch.nn as nn

import spark_gpt_amd as sg
from spark_gpt_amd import _lib, ops
from oracle import fp8_bits

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sparkfp8.h")


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return {n: t for t, n in re.findall(r"^\s*(int|int64_t)\s+(sfp8_\w+)\s*\(", text, flags=re.M)}


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    decl = header_functions()
    assert len(decl) >= 14
    for name in decl:
        assert hasattr(lib, name), name
    # ctypes table covers exactly the declared functions, with matching return types
    assert set(_lib.SIGNATURES) == set(decl)
    for name, ret in decl.items():
        want = ctypes.c_int64 if ret == "int64_t" else ctypes.c_int
        assert _lib.SIGNATURES[name][0] is want, name


def test_header_argument_counts_match_binding():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for m in re.finditer(r"(sfp8_\w+)\s*\(([^)]*)\)\s*;", text):
        name, args = m.group(1), m.group(2)
        n = len([a for a in args.split(",") if a.strip()])
        assert len(_lib.SIGNATURES[name][1]) == n, name


def test_size_queries_need_no_gpu():
    # one partial row per norm work-group (64 tokens each, 65536 / D when
    # fewer), then up to 32 group sums
    assert _lib.query("sfp8_norm_bwd_partials", 1024, 65536) == 65536 // 64 + 32
    assert _lib.query("sfp8_norm_bwd_partials", 2048, 65536) == 65536 // 32 + 32
    assert _lib.query("sfp8_norm_bwd_partials", 4096, 16384) == 16384 // 16 + 32
    assert _lib.query("sfp8_norm_bwd_partials", 128, 256) == 4 + 4  # fewer than 32 rows: one group each
    assert _lib.query("sfp8_norm_bwd_partials", 96, 256) == -1
    # rows of 8192 and more: 64 tokens per work-group
    assert _lib.query("sfp8_norm_bwd_partials", 8192, 65536) == 65536 // 64 + 32
    assert _lib.query("sfp8_norm_bwd_partials", 32768, 256) == 4 + 4
    assert _lib.query("sfp8_norm_bwd_partials", 12288, 256) == 4 + 4  # any multiple of 4096 from 8192
    assert _lib.query("sfp8_norm_bwd_partials", 10240, 256) == -1
    s = _lib.query("sfp8_wgrad_splits", 6144, 1024, 65536)
    # any count, each split a whole number of 128-token stage pairs (the last
    # takes the rest); at the headline shape both gradients take 5
    chunk = -(-(-(-65536 // s)) // 128) * 128
    assert s == 5 and chunk % 128 == 0 and 0 < 65536 - (s - 1) * chunk <= chunk
    assert _lib.query("sfp8_wgrad_splits", 1024, 3072, 65536) == 5
    assert _lib.query("sfp8_wgrad_workspace_floats", 6144, 1024, 65536) == (s * 6144 * 1024 if s > 1 else 0)
    # partials are whole 256 x 256 tiles per split
    s2 = _lib.query("sfp8_wgrad_splits", 384, 128, 65536)
    assert s2 > 1 and _lib.query("sfp8_wgrad_workspace_floats", 384, 128, 65536) == s2 * 2 * 256 * 256
    assert _lib.query("sfp8_wgrad_splits", 256, 256, 256) == 1


def test_invalid_arguments_rejected_before_launch():
    lib = _lib.load()
    # null pointers and bad shapes return negative codes without touching the device
    assert lib.sfp8_update_scales(None, None, 1, None) == -1
    assert lib.sfp8_quant_e4m3_rowcol(None, 4, 100, None, None, None, None, 4, None) == -1
    # x8t is a K-slab over ldt tokens: ldt must be a multiple of 64 and cover the rows
    assert lib.sfp8_quant_e4m3_rowcol(16, 4, 128, 16, 16, 16, 16, 100, None) == -2
    assert lib.sfp8_quant_e4m3_rowcol(16, 100, 128, 16, 16, 16, 16, 64, None) == -2
    assert lib.sfp8_quant_e4m3_rowcol(16, 4, 100, 16, 16, 16, 16, 64, None) == -2
    assert lib.sfp8_gemm_wgrad(16, 0, 16, 0, 256, 256, 256, 16, 16, 16, 16, 0, None) == -2  # A must be e5m2
    # producers of padded K-slabs write every padding token only for ldt = T rounded up to 256
    assert lib.sfp8_gemm_gateup_swiglu_fwd(16, 16, 100, 256, 384, 16, 16, 16, 16, 16, 16, 512, None) == -2
    assert lib.sfp8_gemm_gateup_swiglu_fwd(16, 16, 100, 256, 384, 16, 16, 16, 16, 16, 16, 100, None) == -2
    assert lib.sfp8_gemm_down_dgrad_swiglu(16, 16, 16, 300, 256, 384, 16, 16, 16, 16, 768, None) == -2
    assert lib.sfp8_gemm_wgrad(16, 1, 16, 0, 256, 102, 256, 16, 16, 16, 16, 0, None) == -2  # N % 4
    # the allocation-free norm backward refuses shapes beyond its fixed scratch on the host
    assert lib.sfp8_norm_bwd_noalloc(16, 16, 16, 16, 16, 65536, 4096, 16, 16, 16, 16, 16, None, 65536, None) == -5
    assert lib.sfp8_norm_bwd_noalloc(None, 16, 16, 16, 16, 256, 1024, 16, 16, 16, 16, None, 16, 256, None) == -1
    with pytest.raises(RuntimeError, match="null pointer"):
        _lib.check(-1, "x")
    with pytest.raises(RuntimeError, match="HIP error 1"):
        _lib.check(1, "x")


def test_device_band_table_matches_oracle():
    src = open(os.path.join(ROOT, "spark-gpt_amd", "csrc", "scale.h")).read()
    body = src[src.index("kLog2Band[254] = {") + len("kLog2Band[254] = {"):]
    body = body[: body.index("};")]
    vals = [int(v) for v in body.replace("\n", " ").split(",") if v.strip()]
    want = fp8_bits.band_table(-125, 128)
    assert vals == [want[k] for k in range(-125, 129)]


def test_ops_reject_host_tensors():
    h = torch.zeros(4, 128, dtype=torch.bfloat16)
    with pytest.raises((ValueError, RuntimeError)):
        ops.norm_quant(h, torch.ones(128), torch.ones(5), torch.zeros(5), 1e-6)
    with pytest.raises((ValueError, RuntimeError)):
        ops.quant_e4m3_rowcol(h, torch.ones(5), torch.zeros(5))


def test_slab_layout_roundtrip():
    """K-slab copies: element (r, t) at [t // 64, r, t % 64], rows padded to 256."""
    assert ops.slab_rows(1) == 256 and ops.slab_rows(256) == 256 and ops.slab_rows(768) == 768
    assert ops.slab_rows(384) == 512
    g = torch.Generator().manual_seed(9)
    x = torch.randint(0, 256, (384, 512), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn)
    s = ops.to_slab(x)
    assert s.shape == (8, 512, 64) and s.dtype == x.dtype
    su = s.view(torch.uint8)
    xu = x.view(torch.uint8)
    for r, t in ((0, 0), (383, 511), (17, 64), (200, 300)):
        assert su[t // 64, r, t % 64] == xu[r, t]
    assert torch.all(su[:, 384:] == 0)
    assert torch.equal(ops.unslab(s, 384).view(torch.uint8), xu)
    assert _lib.query("sfp8_slab_bytes", 384, 512) == 512 * 512
    assert _lib.query("sfp8_slab_bytes", 6144, 65536) == 6144 * 65536
    assert _lib.query("sfp8_slab_bytes", 128, 100) == -1


def test_ldt_padding():
    assert ops.ldt_of(0) == 0 and ops.ldt_of(1) == 256 and ops.ldt_of(256) == 256 and ops.ldt_of(1000) == 1024


def test_constants_match_reference_recipe():
    assert sg.FP8_SITE_MAX == (448.0, 448.0, 448.0, 57344.0, 57344.0)
    assert sg.FP8_HEADROOM_BINADES == 1


def test_mlp_module_state_names():
    m = sg.MLP(256, 768)
    assert set(dict(m.named_parameters())) == {"gate_up_proj.weight", "down_proj.weight"}
    assert m.gate_up_proj.weight.shape == (1536, 256) and m.down_proj.weight.shape == (256, 768)
    assert "fp8_scale" not in m.state_dict() and "fp8_amax" not in m.state_dict()
    assert torch.equal(m.fp8_scale, torch.ones(5)) and torch.equal(m.fp8_amax, torch.zeros(5))
    x = torch.randn(3, 256)
    g, u = m.gate_up_proj(x).chunk(2, -1)
    torch.testing.assert_close(m(x), m.down_proj(torch.nn.functional.silu(g) * u))


class _FakeBlock(nn.Module):
    def __init__(self, d, inter, sparse=False):
        super().__init__()
        self.is_sparse = sparse
        if not sparse:
            self.mlp = sg.MLP(d, inter)


class _FakeCudaTensor:
    """Stands in for a device tensor in the guard (it reads only attributes)."""

    def __init__(self, shape, dtype=torch.bfloat16, is_cuda=True):
        self.shape, self.dtype, self.is_cuda = shape, dtype, is_cuda

    def dim(self):
        return len(self.shape)


@pytest.mark.parametrize("d,inter,ok", [(1024, 3072, True), (256, 768, True), (384, 768, False),
                                        (1024, 3000, False), (8192, 1024, True), (16384, 3072, True),
                                        (12288, 3072, False), (128, 128, True), (64, 128, False)])
def test_guard_predicate(monkeypatch, d, inter, ok):
    from spark_gpt_amd import mlp as M

    monkeypatch.setattr(M, "FP8_MLP", True)
    b = _FakeBlock(d, inter).train()
    assert M._use_fp8_mlp(b, _FakeCudaTensor((10, d))) is ok
    b.eval()
    assert M._use_fp8_mlp(b, _FakeCudaTensor((10, d))) is False
    b.train()
    assert M._use_fp8_mlp(b, _FakeCudaTensor((10, d), dtype=torch.float32)) is False
    assert M._use_fp8_mlp(b, _FakeCudaTensor((10, d), is_cuda=False)) is False
    monkeypatch.setattr(M, "FP8_MLP", False)
    assert M._use_fp8_mlp(b, _FakeCudaTensor((10, d))) is False


def test_guard_checks_sparse_first(monkeypatch):
    """Regression of spark-gpt tests/test_fp8_mlp.py:113-140: a sparse block has
    no down_proj and the guard must not touch it."""
    from spark_gpt_amd import mlp as M

    monkeypatch.setattr(M, "FP8_MLP", True)
    b = _FakeBlock(256, 768, sparse=True).train()
    assert M._use_fp8_mlp(b, _FakeCudaTensor((10, 256))) is False


def test_update_scales_walks_every_fp8_module(monkeypatch):
    seen = []
    monkeypatch.setattr(ops, "update_scales", lambda s, a: seen.append((s, a)))
    model = nn.Sequential(sg.MLP(128, 256), nn.Linear(4, 4), nn.Sequential(sg.MLP(128, 256)))
    sg.fp8_update_scales(model)
    assert len(seen) == 2


def test_custom_op_fake_shapes_match_allocations():
    """The fake (shape-only) implementations used under torch.compile return
    the shapes and dtypes the real wrappers allocate (checked with fake CUDA
    tensors: no GPU needed)."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    T, D, I = 300, 256, 384
    with FakeTensorMode():
        dev = "cuda"
        h = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
        nw, wgu, wd = torch.empty(D, device=dev), torch.empty(2 * I, D, device=dev), torch.empty(D, I, device=dev)
        s, a = torch.empty(5, device=dev), torch.empty(5, device=dev)
        out = torch.ops.sparkfp8.block_fwd(h, nw, wgu, wd, s, a, 1e-6)
        grads = torch.ops.sparkfp8.block_bwd(torch.empty(T, D, dtype=torch.bfloat16, device=dev), h, nw, wgu, wd,
                                             *out[1:], s, a)
    meta = "meta"
    want = [torch.empty(T, D, dtype=torch.bfloat16, device=meta),
            ops.kslab_empty(ops.ldt_of(T), D, ops.E4M3, meta),
            torch.empty(T, device=meta),
            ops.kslab_empty(ops.ldt_of(T), 2 * I, ops.E4M3, meta),
            ops.kslab_empty(ops.ldt_of(T), I, ops.E4M3, meta)]
    assert len(out) == len(want)
    for got, w in zip(out, want):
        assert got.shape == w.shape and got.dtype == w.dtype
    assert [tuple(g.shape) for g in grads] == [(T, D), (D,), (2 * I, D), (D, I)]
    assert [g.dtype for g in grads] == [torch.bfloat16] + [torch.float32] * 3


def _integration_snippet():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    tail = text[text.index("<!-- trainer-binding -->"):]
    return tail[tail.index("```python") + len("```python"):tail.index("```", tail.index("```python") + 9)]


# The parts of spark-gpt's train.py this path touches, reduced to what the
# binding needs: the switch (train.py:914), main()'s rebinding of it
# (train.py:3635-3642), Block.forward's dispatch (train.py:2359-2365) and
# Experts.forward's (train.py:2292-2296).
_STUB_TRAINER_HEAD = """
FP8_MLP = False
FUSED_SWIGLU = True
FUSED_NORM_MLP = True
"""
_STUB_TRAINER_TAIL = """
def main(fp8_mlp, fused_norm_mlp=True, fused_swiglu=True):
    global FP8_MLP, FUSED_NORM_MLP, FUSED_SWIGLU
    FP8_MLP = fp8_mlp
    FUSED_NORM_MLP = fused_norm_mlp
    FUSED_SWIGLU = fused_swiglu

class Block:
    def __init__(self, block):
        self.block = block

    def forward(self, h):
        b = self.block
        if _use_fp8_mlp(b, h):
            return _FP8MLPBlock.apply(h, b.norm_w, b.mlp.gate_up_proj.weight, b.mlp.down_proj.weight,
                                      b.mlp.fp8_scale, b.mlp.fp8_amax, 1e-6)
        if _use_fused_norm_mlp(b, h):
            return _NormSwiGLU.apply(h, b.norm_w, b.mlp.gate_up_proj.weight, 1e-6)
        return "bf16"

class Experts:
    def __init__(self, m):
        self.m = m

    def forward(self, x, token_index, inverse_permutation, offsets, top_k):
        m = self.m
        if _use_fp8_moe(m, x):
            return _FP8Experts.apply(x, m.gate_up_proj, m.down_proj, token_index, inverse_permutation, offsets,
                                     top_k, m.fp8_scale, m.fp8_amax)
        return "bf16"
"""


def test_documented_trainer_binding(monkeypatch):
    """INTEGRATION.md's substitution, run in a stub of train.py: after main()
    sets the trainer's own FP8_MLP, a dense training block goes to
    _FP8MLPBlock; before it, and for eval or sparse blocks, it does not."""
    import types

    train = types.ModuleType("train_stub")
    exec(_STUB_TRAINER_HEAD + _integration_snippet() + _STUB_TRAINER_TAIL, train.__dict__)
    assert train._FP8MLPBlock is sg._FP8MLPBlock
    calls = []

    class _Recorder:
        @staticmethod
        def apply(*args):
            calls.append(args)
            return "fp8"

    monkeypatch.setattr(train, "_FP8MLPBlock", _Recorder)
    monkeypatch.setattr(train, "FUSED_NORM_MLP", False)  # the unfused bf16 path, as --no-fused-norm-mlp
    dense = _FakeBlock(1024, 3072).train()
    dense.norm_w = torch.ones(1024)
    blk = train.Block(dense)
    h = _FakeCudaTensor((10, 1024))
    assert blk.forward(h) == "bf16" and not calls  # --fp8-mlp not given
    train.main(True, fused_norm_mlp=False)
    assert sg.mlp.FP8_MLP is False  # the package's own switch is not involved
    assert blk.forward(h) == "fp8" and len(calls) == 1
    assert calls[0][2] is dense.mlp.gate_up_proj.weight
    dense.eval()
    assert blk.forward(h) == "bf16"
    sparse = _FakeBlock(1024, 3072, sparse=True).train()
    assert train._use_fp8_mlp(sparse, h) is False
    train.main(False, fused_norm_mlp=False)
    dense.train()
    assert blk.forward(h) == "bf16"


def test_documented_trainer_binding_bf16(monkeypatch):
    """Without --fp8-mlp the same substitution routes a dense block to
    _NormSwiGLU (the default, train.py:2366-2369); --no-fused-norm-mlp or
    --no-fused-swiglu (main() rebinding the trainer's switches) routes it to
    the unfused path, and a sparse block is never routed (checked first)."""
    import types

    train = types.ModuleType("train_stub")
    exec(_STUB_TRAINER_HEAD + _integration_snippet() + _STUB_TRAINER_TAIL, train.__dict__)
    assert train._NormSwiGLU is sg._NormSwiGLU and train._FusedSwiGLU is sg._FusedSwiGLU
    calls = []

    class _Recorder:
        @staticmethod
        def apply(*args):
            calls.append(args)
            return "bf16-fused"

    monkeypatch.setattr(train, "_NormSwiGLU", _Recorder)
    dense = _FakeBlock(1024, 3072).train()
    dense.norm_w = torch.ones(1024)
    blk = train.Block(dense)
    h = _FakeCudaTensor((10, 1024))
    train.main(False)
    assert blk.forward(h) == "bf16-fused" and len(calls) == 1
    assert calls[0][2] is dense.mlp.gate_up_proj.weight
    dense.eval()
    assert blk.forward(h) == "bf16-fused"  # the fused bf16 path is not training-only
    train.main(False, fused_norm_mlp=False)
    assert blk.forward(h) == "bf16"
    train.main(False, fused_swiglu=False)
    assert blk.forward(h) == "bf16"
    train.main(False)
    assert blk.forward(_FakeCudaTensor((10, 1000))) == "bf16"  # width not a multiple of 64
    sparse = _FakeBlock(1024, 3072, sparse=True)
    assert train._use_fused_norm_mlp(sparse, h) is False
    assert train._use_fused_swiglu(h) is True
    assert train._use_fused_swiglu(_FakeCudaTensor((10, 1024), dtype=torch.float32)) is False


def test_documented_trainer_binding_experts(monkeypatch):
    """The same substitution routes a training Experts module (power-of-two
    hidden size, 128-divisible expert ffn) to _FP8Experts once main() sets
    FP8_MLP, and nothing else."""
    import types

    train = types.ModuleType("train_stub")
    exec(_STUB_TRAINER_HEAD + _integration_snippet() + _STUB_TRAINER_TAIL, train.__dict__)
    assert train._FP8Experts is sg._FP8Experts
    calls = []

    class _Recorder:
        @staticmethod
        def apply(*args):
            calls.append(args)
            return "fp8"

    monkeypatch.setattr(train, "_FP8Experts", _Recorder)
    m = torch.nn.Module()
    m.hidden_dim, m.intermediate_dim = 1024, 768
    m.gate_up_proj = torch.nn.Parameter(torch.zeros(4, 2 * 768, 1024))
    m.down_proj = torch.nn.Parameter(torch.zeros(4, 1024, 768))
    m.fp8_scale, m.fp8_amax = torch.ones(5), torch.zeros(5)
    m.train()
    ex = train.Experts(m)
    x = _FakeCudaTensor((10, 1024))
    args = (None, None, None, 2)
    assert ex.forward(x, *args) == "bf16" and not calls
    train.main(True)
    assert ex.forward(x, *args) == "fp8" and len(calls) == 1
    assert calls[0][1] is m.gate_up_proj and calls[0][6] == 2 and calls[0][8] is m.fp8_amax
    m.eval()
    assert ex.forward(x, *args) == "bf16"
    m.train()
    m.intermediate_dim = 100  # not a multiple of 128
    assert ex.forward(x, *args) == "bf16"
    m.intermediate_dim, m.hidden_dim = 768, 768  # not a power of two
    assert ex.forward(_FakeCudaTensor((10, 768)), *args) == "bf16"
    train.main(False)


def test_set_fp8_mlp_switches_package_guard(monkeypatch):
    from spark_gpt_amd import mlp as M

    monkeypatch.setattr(M, "FP8_MLP", False)
    b = _FakeBlock(256, 768).train()
    h = _FakeCudaTensor((10, 256))
    assert sg._use_fp8_mlp(b, h) is False
    sg.set_fp8_mlp(True)
    assert sg.FP8_MLP is True and sg._use_fp8_mlp(b, h) is True
    sg.set_fp8_mlp(False)
    assert sg._use_fp8_mlp(b, h) is False


def test_weight_cache_keys(monkeypatch):
    """The cache reuses a quantization while the same masters are unchanged,
    re-quantizes when a version counter moves, and fp8_update_scales
    re-quantizes entries whose masters the optimizer may have rewritten
    (quantization replaced by a counter: no GPU)."""
    from spark_gpt_amd import torch_ops as TO

    n = []
    monkeypatch.setattr(TO, "quantize_weights", lambda a, b: n.append(1) or ("q", len(n)))
    TO.clear_weight_cache()
    wgu, wd = torch.zeros(8, 4), torch.zeros(4, 4)
    q1 = TO.cached_weights(wgu, wd)
    assert TO.cached_weights(wgu, wd) is q1 and len(n) == 1
    with torch.no_grad():
        wgu.add_(1)  # in-place update: version counter moves
    q2 = TO.cached_weights(wgu, wd)
    assert q2 is not q1 and len(n) == 2
    other = torch.zeros(4, 4)
    assert TO.cached_weights(wgu, other) is not q2 and len(n) == 3  # another down master
    # a refresh re-quantizes (entries on CPU masters are dropped instead)
    TO.refresh_weight_cache(wgu, other)
    assert TO.cached_weights(wgu, other)[1] == 4
    monkeypatch.setattr(TO, "FP8_WEIGHT_CACHE", False)
    TO.cached_weights(wgu, other)
    TO.cached_weights(wgu, other)
    assert len(n) == 6
    TO.clear_weight_cache()


def test_weight_cache_entry_dies_with_master(monkeypatch):
    import gc

    from spark_gpt_amd import torch_ops as TO

    monkeypatch.setattr(TO, "quantize_weights", lambda a, b: ("q",))
    TO.clear_weight_cache()
    wgu, wd = torch.zeros(8, 4), torch.zeros(4, 4)
    TO.cached_weights(wgu, wd)
    assert len(TO._WCACHE) == 1
    del wgu
    gc.collect()
    assert len(TO._WCACHE) == 0
