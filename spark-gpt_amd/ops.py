"""Torch-facing wrappers of the libsparkfp8 kernels.

Each wrapper validates shapes/dtypes, allocates its outputs with torch's
caching allocator (as the reference allocates with ``torch.empty``), and
launches on torch's current stream.  Nothing here synchronises the device or
reads device values back.
"""
from __future__ import annotations

import torch

from . import _lib

E4M3 = torch.float8_e4m3fn
E5M2 = torch.float8_e5m2
FMT_E4M3 = 0
FMT_E5M2 = 1
TOKEN_ALIGN = 256  # leading dimension of token-contiguous fp8 copies


def ldt_of(T: int) -> int:
    """Tokens covered by the token-contiguous copies (x8t, h8t, d_gu8t, dy8t):
    T rounded up to a multiple of 256, zero past T."""
    return -(-T // TOKEN_ALIGN) * TOKEN_ALIGN


SLAB = 64  # bytes of K per slab row
# bytes per element of the dtypes the K-slabs hold
_ESIZE = {torch.float8_e4m3fn: 1, torch.float8_e5m2: 1, torch.uint8: 1, torch.bfloat16: 2, torch.float16: 2,
          torch.float32: 4}


def _esize(dtype) -> int:
    n = _ESIZE.get(dtype)
    return n if n is not None else torch.empty((), dtype=dtype).element_size()


def slab_rows(R: int) -> int:
    """Rows of a K-slab: R rounded up to the 256-row GEMM tile."""
    return -(-R // 256) * 256


def kslab_empty(R: int, L: int, dtype, device) -> torch.Tensor:
    """A K-slab of a row-major [R, L] matrix (L elements of K per row):
    [L*size/64, slab_rows(R), 64/size] for elements of `size` bytes; element
    (r, l) at [l // n, r, l % n] with n = 64 / size.  Every FP8 GEMM operand
    (and the bf16 W_down^T) uses this layout; one 64-byte K stage of a
    256-row tile is one contiguous 16 KiB block."""
    n = SLAB // _esize(dtype)
    _need(L % n == 0, f"K extent {L} must be a multiple of {n}")
    return torch.empty(L // n, slab_rows(R), n, dtype=dtype, device=device)


def kslab_shape(R: int, L: int, dtype) -> tuple:
    """Shape of kslab_empty(R, L, dtype)."""
    n = SLAB // _esize(dtype)
    _need(L % n == 0, f"K extent {L} must be a multiple of {n}")
    return (L // n, slab_rows(R), n)


def slab_empty(R: int, T: int, dtype, device) -> torch.Tensor:
    """A token-contiguous K-slab copy of R feature rows over ldt_of(T) tokens
    (the weight gradients' operands): [ldt / 64, slab_rows(R), 64]; element
    (r, t) at [t // 64, r, t % 64]."""
    return kslab_empty(R, ldt_of(T), dtype, device)


def unslab(t: torch.Tensor, R: int) -> torch.Tensor:
    """The plain [R, L] matrix of a K-slab tensor (for inspection and tests)."""
    n, rp, _ = t.shape
    return t.view(torch.uint8).permute(1, 0, 2).reshape(rp, n * SLAB)[:R].view(t.dtype)


def to_slab(x: torch.Tensor) -> torch.Tensor:
    """K-slab of a plain [R, L] tensor (64-byte multiple rows); padding rows zero."""
    R, L = x.shape
    nb = L * x.element_size()
    _need(nb % SLAB == 0, "row length must be a multiple of 64 bytes")
    out = torch.zeros(nb // SLAB, slab_rows(R), SLAB, dtype=torch.uint8, device=x.device)
    out[:, :R] = x.contiguous().view(torch.uint8).view(R, nb // SLAB, SLAB).permute(1, 0, 2)
    return out.view(x.dtype)


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _cuda_contig(name: str, t: torch.Tensor, dtype: torch.dtype, ndim: int) -> None:
    _need(t.is_cuda, f"{name} must be a ROCm device tensor")
    _need(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _need(t.dim() == ndim, f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    _need(t.is_contiguous(), f"{name} must be contiguous")


def _state(scale: torch.Tensor, amax: torch.Tensor) -> None:
    for n, t in (("scale", scale), ("amax", amax)):
        _need(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous() and t.numel() >= 5,
              f"{n} must be a contiguous fp32 device tensor of 5 slots")


# ------------------------------------------------------------------ quantizers
def quant_e4m3_rowcol(x: torch.Tensor, scale: torch.Tensor, amax: torch.Tensor):
    """x8 = e4m3(x * scale[0]) row-major [rows, cols]; x8t = the token-contiguous
    K-slab copy of x8^T over ldt_of(rows) tokens ([ldt / 64, slab_rows(cols),
    64], zeros past rows and cols); amax[0] max|x|."""
    _cuda_contig("x", x, torch.bfloat16, 2)
    R, C = x.shape
    _need(C % 128 == 0, "cols must be a multiple of 128")
    ldt = ldt_of(R)
    x8 = torch.empty(R, C, dtype=E4M3, device=x.device)
    x8t = slab_empty(C, R, E4M3, x.device)
    _lib.call("sfp8_quant_e4m3_rowcol", x.data_ptr(), R, C, scale.data_ptr(), amax.data_ptr(),
              x8.data_ptr(), x8t.data_ptr(), ldt, _lib.stream_of(x))
    return x8, x8t


def norm_quant(h: torch.Tensor, norm_w: torch.Tensor, scale: torch.Tensor, amax: torch.Tensor, eps: float, *,
               copy: bool = True):
    """(x8 K-slab of [T, D] ([D/64, ldt, 64]), x8t K-slab of [D, ldt], rstd
    [T]); amax[0] max-accumulated.  copy=False skips the token-contiguous
    x8t (None): the weight gradient then reads x8 itself (wgrad_rows)."""
    _cuda_contig("h", h, torch.bfloat16, 2)
    _cuda_contig("norm_w", norm_w, torch.float32, 1)
    _state(scale, amax)
    T, D = h.shape
    ldt = ldt_of(T)
    x8 = kslab_empty(ldt, D, E4M3, h.device)
    x8t = slab_empty(D, T, E4M3, h.device) if copy else None
    rstd = torch.empty(T, dtype=torch.float32, device=h.device)
    _lib.call("sfp8_norm_quant", h.data_ptr(), norm_w.data_ptr(), T, D, float(eps), scale.data_ptr(),
              amax.data_ptr(), x8.data_ptr(), _lib.ptr(x8t), ldt, rstd.data_ptr(), _lib.stream_of(h))
    return x8, x8t, rstd


def weight_quant(w: torch.Tensor, q_out: torch.Tensor, *, w8: bool = True, w8t: bool = False,
                 bf16t: bool = False):
    """Just-in-time e4m3 copy of an fp32 master [R, C]: returns (w8 K-slab of
    [R, C], w8t K-slab of [C, R], bf16 K-slab of W^T [C, R]), unrequested
    outputs None; the pow2 scale lands in q_out[0] (device)."""
    _cuda_contig("w", w, torch.float32, 2)
    R, C = w.shape
    _need(C % 64 == 0, "weight columns must be a multiple of 64")
    _need(not w8t or R % 64 == 0, "weight rows must be a multiple of 64 for the transposed copy")
    _need(not bf16t or R % 32 == 0, "weight rows must be a multiple of 32 for the bf16 copy")
    dev = w.device
    o8 = kslab_empty(R, C, E4M3, dev) if w8 else None
    o8t = kslab_empty(C, R, E4M3, dev) if w8t else None
    obt = kslab_empty(C, R, torch.bfloat16, dev) if bf16t else None
    parts = torch.empty(512, dtype=torch.float32, device=dev)
    _lib.call("sfp8_weight_quant", w.data_ptr(), R, C, parts.data_ptr(), parts.numel(), q_out.data_ptr(),
              _lib.ptr(o8), _lib.ptr(o8t), _lib.ptr(obt), _lib.stream_of(w))
    return o8, o8t, obt


def block_weight_quant(w_gu: torch.Tensor, w_down: torch.Tensor, scale=None, amax=None):
    """Both weight quantizations of a dense block in two launches:
    (w8, w8t, wd8, wdt, wscale) as weight_quant(w_gu, w8=True, w8t=True) and
    weight_quant(w_down, w8=True, bf16t=True) return them, wscale = [q_gu,
    q_d]; with scale and amax, also the delayed-scale roll of those 5 slots
    (update_scales), in the first launch."""
    _cuda_contig("w_gu", w_gu, torch.float32, 2)
    _cuda_contig("w_down", w_down, torch.float32, 2)
    R0, C0 = w_gu.shape
    R1, C1 = w_down.shape
    _need(R0 % 64 == 0 and C0 % 64 == 0, "gate/up weight rows and columns must be multiples of 64")
    _need(C1 % 64 == 0 and R1 % 32 == 0, "down weight columns must be a multiple of 64, rows of 32")
    _need(w_down.device == w_gu.device, "weights on one device")
    if scale is not None or amax is not None:
        _need(scale is not None and amax is not None, "scale and amax go together")
        _state(scale, amax)
        _need(scale.numel() == 5 and amax.numel() == 5, "one 5-slot set")
        _need(scale.device == w_gu.device and amax.device == w_gu.device, "scale/amax on the weights' device")
    dev = w_gu.device
    w8 = kslab_empty(R0, C0, E4M3, dev)
    w8t = kslab_empty(C0, R0, E4M3, dev)
    wd8 = kslab_empty(R1, C1, E4M3, dev)
    wdt = kslab_empty(C1, R1, torch.bfloat16, dev)
    wscale = torch.empty(2, dtype=torch.float32, device=dev)
    parts = torch.empty(1024, dtype=torch.float32, device=dev)
    _lib.call("sfp8_block_weight_quant", w_gu.data_ptr(), R0, C0, w_down.data_ptr(), R1, C1, parts.data_ptr(),
              parts.numel(), wscale.data_ptr(), w8.data_ptr(), w8t.data_ptr(), wd8.data_ptr(), wdt.data_ptr(),
              _lib.ptr(scale), _lib.ptr(amax), _lib.stream_of(w_gu))
    return w8, w8t, wd8, wdt, wscale


def update_scales(scale: torch.Tensor, amax: torch.Tensor) -> None:
    """In-place delayed-scale roll of one or more contiguous 5-slot sets."""
    _need(scale.is_cuda and amax.is_cuda, "scale/amax must be device tensors")
    _need(scale.dtype == torch.float32 and amax.dtype == torch.float32, "scale/amax must be fp32")
    _need(scale.is_contiguous() and amax.is_contiguous(), "scale/amax must be contiguous")
    _need(scale.numel() == amax.numel() and scale.numel() % 5 == 0, "scale/amax: 5 slots per set")
    _lib.call("sfp8_update_scales", scale.data_ptr(), amax.data_ptr(), scale.numel() // 5,
              _lib.stream_of(scale))


# ------------------------------------------------------------------ GEMMs
def _kslab(name: str, t: torch.Tensor, dtype, R: int, L: int) -> None:
    n = SLAB // _esize(dtype)
    _cuda_contig(name, t, dtype, 3)
    _need(tuple(t.shape) == (L // n, slab_rows(R), n), f"{name} must be a K-slab of [{R}, {L}]")


def gateup_swiglu_fwd(x8, w8, scale, wscale, amax, T: int, I: int, *, copy: bool = True):
    """(gu8 K-slab of [T, 2I], h8 K-slab of [T, I], h8t K-slab of [I, ldt]);
    x8 is the K-slab of [T, D], w8 that of [2I, D]; amax[1], amax[2]
    max-accumulated.  copy=False skips the token-contiguous h8t (None): the
    weight gradient then reads h8 itself (wgrad_rows)."""
    _need(x8.dim() == 3, "x8 must be a K-slab")
    D = x8.shape[0] * SLAB
    ldt = ldt_of(T)
    _kslab("x8", x8, E4M3, ldt, D)
    _kslab("w8", w8, E4M3, 2 * I, D)
    _need(D % 128 == 0 and I % 128 == 0, "D and I must be multiples of 128")
    dev = x8.device
    gu8 = kslab_empty(ldt, 2 * I, E4M3, dev)
    h8 = kslab_empty(ldt, I, E4M3, dev)
    h8t = slab_empty(I, T, E4M3, dev) if copy else None
    _lib.call("sfp8_gemm_gateup_swiglu_fwd", x8.data_ptr(), w8.data_ptr(), T, D, I, scale.data_ptr(),
              wscale.data_ptr(), amax.data_ptr(), gu8.data_ptr(), h8.data_ptr(), h8t.data_ptr() if copy else 0,
              ldt, _lib.stream_of(x8))
    return gu8, h8, h8t


def down_fwd(h8, wd8, res, scale, wscale):
    """y = bf16(res + bf16(h8 @ wd8^T / (s2 * q_d))), [T, D] bf16; h8 is the
    K-slab of [T, I], wd8 that of [D, I]."""
    _cuda_contig("res", res, torch.bfloat16, 2)
    T, D = res.shape
    _need(h8.dim() == 3, "h8 must be a K-slab")
    I = h8.shape[0] * SLAB
    ldt = ldt_of(T)
    _kslab("h8", h8, E4M3, ldt, I)
    _kslab("wd8", wd8, E4M3, D, I)
    _need(I % 128 == 0, "I must be a multiple of 128")
    y = torch.empty(T, D, dtype=torch.bfloat16, device=h8.device)
    _lib.call("sfp8_gemm_down_fwd", h8.data_ptr(), wd8.data_ptr(), res.data_ptr(), T, D, I, scale.data_ptr(),
              wscale.data_ptr(), y.data_ptr(), ldt, _lib.stream_of(h8))
    return y


def down_dgrad_swiglu(dy, wdt, gu8, scale, amax, *, copy: bool = True):
    """(dgu8 K-slab of [T, 2I] e5m2, dgu8t K-slab of [2I, ldt] e5m2); wdt is
    the bf16 K-slab of W_down^T [I, D], gu8 the e4m3 K-slab of [T, 2I] the
    forward wrote; amax[3] max-accumulated.  copy=False skips the
    token-contiguous dgu8t (None): the weight gradient then reads dgu8 itself
    (wgrad_rows)."""
    _cuda_contig("dy", dy, torch.bfloat16, 2)
    T, D = dy.shape
    _need(gu8.dim() == 3, "gu8 must be a K-slab")
    I = gu8.shape[0] * SLAB // 2
    ldt = ldt_of(T)
    _kslab("gu8", gu8, E4M3, ldt, 2 * I)
    _kslab("wdt", wdt, torch.bfloat16, I, D)
    _need(D % 64 == 0 and I % 128 == 0, "D must be a multiple of 64 and I of 128")
    dgu8 = kslab_empty(ldt, 2 * I, E5M2, dy.device)
    dgu8t = slab_empty(2 * I, T, E5M2, dy.device) if copy else None
    _lib.call("sfp8_gemm_down_dgrad_swiglu", dy.data_ptr(), wdt.data_ptr(), gu8.data_ptr(), T, D, I,
              scale.data_ptr(), amax.data_ptr(), dgu8.data_ptr(), dgu8t.data_ptr() if copy else 0, ldt,
              _lib.stream_of(dy))
    return dgu8, dgu8t


def gateup_dgrad(dgu8, w8t, scale, wscale, T: int, D: int):
    """dxn = bf16(dgu8 @ w8 / (s3 * q_gu)), [T, D] bf16; dgu8 is the K-slab
    of [T, 2I], w8t that of W8^T [D, 2I]."""
    _need(dgu8.dim() == 3, "dgu8 must be a K-slab")
    I2 = dgu8.shape[0] * SLAB
    ldt = ldt_of(T)
    _kslab("dgu8", dgu8, E5M2, ldt, I2)
    _kslab("w8t", w8t, E4M3, D, I2)
    _need(I2 % 128 == 0, "2I must be a multiple of 128")
    dxn = torch.empty(T, D, dtype=torch.bfloat16, device=dgu8.device)
    _lib.call("sfp8_gemm_gateup_dgrad", dgu8.data_ptr(), w8t.data_ptr(), T, D, I2 // 2, scale.data_ptr(),
              wscale.data_ptr(), dxn.data_ptr(), ldt, _lib.stream_of(dgu8))
    return dxn


def wgrad(at, bt, M: int, N: int, sa, sb):
    """out[m, n] = sum_t at[m, t] bt[n, t] / (sa * sb), fp32 [M, N]; at e5m2
    and bt e4m3 are K-slab token-contiguous copies of M and N rows (zeros past
    the last token)."""
    _cuda_contig("at", at, E5M2, 3)
    _cuda_contig("bt", bt, E4M3, 3)
    ldt = at.shape[0] * SLAB
    _need(at.shape == (ldt // SLAB, slab_rows(M), SLAB), "at must be a K-slab copy of M rows")
    _need(bt.shape == (ldt // SLAB, slab_rows(N), SLAB), "bt must be a K-slab copy of N rows over the same tokens")
    _need(ldt % TOKEN_ALIGN == 0, "token count must be a multiple of 256")
    out = torch.empty(M, N, dtype=torch.float32, device=at.device)
    nws = _lib.query("sfp8_wgrad_workspace_floats", M, N, ldt)
    ws = torch.empty(max(nws, 1), dtype=torch.float32, device=at.device)
    _lib.call("sfp8_gemm_wgrad", at.data_ptr(), FMT_E5M2, bt.data_ptr(), FMT_E4M3, M, N, ldt, sa.data_ptr(),
              sb.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(at))
    return out


# ------------------------------------------------------------------ norm backward
def wgrad_rows(a8, b8, M: int, N: int, sa, sb, *, a_rows: bool = True, b_rows: bool = True):
    """out [M, N] fp32 = sum over tokens of a8[t, m] b8[t, n] / (sa * sb): a8
    (e5m2) and b8 (e4m3) each either the row K-slab of the token-major
    activation ([rows/64, ldt, 64]: read through transposing LDS reads) or,
    with a_rows / b_rows False, the token-contiguous copy ([ldt/64,
    slab_rows, 64], as for wgrad)."""
    _cuda_contig("a8", a8, E5M2, 3)
    _cuda_contig("b8", b8, E4M3, 3)
    _need(a_rows or b_rows, "at least one row K-slab operand (else use wgrad)")
    ldt = a8.shape[1] if a_rows else a8.shape[0] * SLAB
    _need((b8.shape[1] if b_rows else b8.shape[0] * SLAB) == ldt, "a8, b8 must cover the same tokens")
    _need(not a_rows or a8.shape[0] * SLAB == M, "a8 must be the row K-slab of [ldt, M]")
    _need(not b_rows or b8.shape[0] * SLAB == N, "b8 must be the row K-slab of [ldt, N]")
    out = torch.empty(M, N, dtype=torch.float32, device=a8.device)
    nws = _lib.query("sfp8_wgrad_rows_workspace_floats", M, N, ldt)
    ws = torch.empty(max(nws, 1), dtype=torch.float32, device=a8.device)
    _lib.call("sfp8_gemm_wgrad_rows", a8.data_ptr(), FMT_E5M2, int(a_rows), b8.data_ptr(), FMT_E4M3, int(b_rows), M, N,
              ldt, sa.data_ptr(), sb.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(a8))
    return out


def norm_bwd(h, rstd, dxn, dy, norm_w, scale, amax, *, rows: bool = False):
    """(dh [T, D] bf16, dnw [D] fp32, dy8 e5m2); amax[4] = max|dy|.  dy8 is
    the token-contiguous K-slab copy of D rows ([ldt/64, slab_rows(D), 64]),
    or with rows=True the K-slab of [T, D] ([D/64, ldt, 64], read by
    wgrad_rows)."""
    for n, t in (("h", h), ("dxn", dxn), ("dy", dy)):
        _cuda_contig(n, t, torch.bfloat16, 2)
    _cuda_contig("rstd", rstd, torch.float32, 1)
    _cuda_contig("norm_w", norm_w, torch.float32, 1)
    T, D = h.shape
    ldt = ldt_of(T)
    dev = h.device
    dh = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    dnw = torch.empty(D, dtype=torch.float32, device=dev)
    dy8 = kslab_empty(ldt, D, E5M2, dev) if rows else slab_empty(D, T, E5M2, dev)
    nparts = _lib.query("sfp8_norm_bwd_partials", D, ldt)
    _need(nparts >= 0, f"unsupported hidden size {D}")
    parts = torch.empty(max(nparts * D, 1), dtype=torch.float32, device=dev)
    _lib.call("sfp8_norm_bwd", h.data_ptr(), rstd.data_ptr(), dxn.data_ptr(), dy.data_ptr(), norm_w.data_ptr(),
              T, D, scale.data_ptr(), amax.data_ptr(), dh.data_ptr(), dnw.data_ptr(), parts.data_ptr(),
              parts.numel(), dy8.data_ptr() if rows else 0, 0 if rows else dy8.data_ptr(), ldt, _lib.stream_of(h))
    return dh, dnw, dy8


# ------------------------------------------------------------------ MoE experts (grouped)
def moe_padded_rows(R: int, E: int) -> int:
    """Rows of the padded expert order (every expert's rows from a 256-row
    boundary): the worst case for R rows over E experts."""
    return _lib.query("sfp8_moe_padded_rows", R, E)


def moe_plan(offsets: torch.Tensor, R: int) -> torch.Tensor:
    """The tile table of padded expert order, built on the device from the
    experts' inclusive row-count prefix sums (int32 [E]); no host sync."""
    _need(offsets.is_cuda and offsets.dim() == 1, "offsets must be a 1-D device tensor")
    offsets = offsets.to(torch.int32).contiguous()
    E = offsets.numel()
    n = _lib.query("sfp8_moe_plan_ints", R, E)
    _need(n > 0, f"unsupported expert count {E}")
    plan = torch.empty(n, dtype=torch.int32, device=offsets.device)
    _lib.call("sfp8_moe_plan", offsets.data_ptr(), E, R, plan.data_ptr(), n, _lib.stream_of(offsets))
    return plan


def moe_rows_quant(src: torch.Tensor, index, plan: torch.Tensor, ldp: int, scale, sslot: int, amax, aslot: int,
                   fmt: int, with_rows: bool, with_copy: bool = True):
    """fp8 copies of gathered rows in padded expert order: (xs, xt) = (K-slab of
    [ldp, D] or None, token-contiguous K-slab of [D, ldp] or None); row u of
    the expert order is src[index[u]] (or src[u] without index)."""
    _cuda_contig("src", src, torch.bfloat16, 2)
    n, D = src.shape
    dt = E4M3 if fmt == FMT_E4M3 else E5M2
    _need(with_rows or with_copy, "at least one output layout")
    xs = kslab_empty(ldp, D, E4M3, src.device) if with_rows else None
    xt = kslab_empty(D, ldp, dt, src.device) if with_copy else None
    idx = None
    if index is not None:
        _need(index.is_cuda and index.dtype == torch.int64, "row index must be an int64 device tensor")
        idx = index.contiguous()
    _lib.call("sfp8_moe_rows_quant", src.data_ptr(), n, D, _lib.ptr(idx), 0 if idx is None else idx.numel(),
              plan.data_ptr(), ldp, scale.data_ptr(), sslot, amax.data_ptr(), aslot, fmt, _lib.ptr(xs), _lib.ptr(xt),
              _lib.stream_of(src))
    return xs, xt


def weight_quant_experts(w: torch.Tensor, q_out: torch.Tensor, *, w8: bool = True, w8t: bool = False,
                         bf16t: bool = False):
    """Per-expert e4m3 copies of fp32 masters [E, R, C] (stacked K-slabs, as
    weight_quant per expert); the pow2 scales land in q_out[0:E]."""
    _cuda_contig("w", w, torch.float32, 3)
    E, R, C = w.shape
    _need(q_out.numel() >= E and q_out.is_contiguous(), "q_out must hold E scales")
    dev = w.device
    o8 = torch.empty((E,) + kslab_shape(R, C, E4M3), dtype=E4M3, device=dev) if w8 else None
    o8t = torch.empty((E,) + kslab_shape(C, R, E4M3), dtype=E4M3, device=dev) if w8t else None
    obt = torch.empty((E,) + kslab_shape(C, R, torch.bfloat16), dtype=torch.bfloat16, device=dev) if bf16t else None
    parts = torch.empty(512 * E, dtype=torch.float32, device=dev)
    _lib.call("sfp8_weight_quant_experts", w.data_ptr(), E, R, C, parts.data_ptr(), parts.numel(), q_out.data_ptr(),
              _lib.ptr(o8), _lib.ptr(o8t), _lib.ptr(obt), _lib.stream_of(w))
    return o8, o8t, obt


def moe_gateup_swiglu_fwd(x8, w8, plan, scale, q_gu, amax, I: int, *, copy: bool = True):
    """(gu8, h8, h8t) over padded expert order; x8 the K-slab of [ldp, D], w8
    the stacked per-expert K-slabs of [2I, D].  copy=False skips h8t (None)."""
    D, ldp = x8.shape[0] * SLAB, x8.shape[1]
    E = w8.shape[0]
    dev = x8.device
    gu8 = kslab_empty(ldp, 2 * I, E4M3, dev)
    h8 = kslab_empty(ldp, I, E4M3, dev)
    h8t = kslab_empty(I, ldp, E4M3, dev) if copy else None
    _lib.call("sfp8_moe_gemm_gateup_swiglu_fwd", x8.data_ptr(), w8.data_ptr(), E, D, I, plan.data_ptr(), ldp,
              scale.data_ptr(), q_gu.data_ptr(), amax.data_ptr(), gu8.data_ptr(), h8.data_ptr(), _lib.ptr(h8t),
              _lib.stream_of(x8))
    return gu8, h8, h8t


def moe_down_fwd(h8, wd8, plan, scale, q_d, R: int, D: int):
    """out [R, D] bf16 expert-order rows (no residual)."""
    I, ldp = h8.shape[0] * SLAB, h8.shape[1]
    E = wd8.shape[0]
    out = torch.empty(R, D, dtype=torch.bfloat16, device=h8.device)
    _lib.call("sfp8_moe_gemm_down_fwd", h8.data_ptr(), wd8.data_ptr(), E, D, I, plan.data_ptr(), ldp,
              scale.data_ptr(), q_d.data_ptr(), out.data_ptr(), R, _lib.stream_of(h8))
    return out


def moe_down_dgrad_swiglu(dout, wdt, gu8, plan, scale, amax, *, copy: bool = True):
    """(dgu8, dgu8t) e5m2 over padded expert order; dout [R, D] bf16 expert-order
    rows, wdt the stacked bf16 K-slabs of W_down[e]^T.  copy=False skips dgu8t
    (None)."""
    _cuda_contig("dout", dout, torch.bfloat16, 2)
    R, D = dout.shape
    I2, ldp = gu8.shape[0] * SLAB, gu8.shape[1]
    E = wdt.shape[0]
    dev = dout.device
    dgu8 = kslab_empty(ldp, I2, E5M2, dev)
    dgu8t = kslab_empty(I2, ldp, E5M2, dev) if copy else None
    _lib.call("sfp8_moe_gemm_down_dgrad_swiglu", dout.data_ptr(), wdt.data_ptr(), gu8.data_ptr(), E, D, I2 // 2, R,
              plan.data_ptr(), ldp, scale.data_ptr(), amax.data_ptr(), dgu8.data_ptr(), _lib.ptr(dgu8t),
              _lib.stream_of(dout))
    return dgu8, dgu8t


def moe_gateup_dgrad(dgu8, w8t, plan, scale, q_gu, R: int, D: int):
    """dx [R, D] bf16 expert-order rows."""
    I2, ldp = dgu8.shape[0] * SLAB, dgu8.shape[1]
    E = w8t.shape[0]
    dx = torch.empty(R, D, dtype=torch.bfloat16, device=dgu8.device)
    _lib.call("sfp8_moe_gemm_gateup_dgrad", dgu8.data_ptr(), w8t.data_ptr(), E, D, I2 // 2, plan.data_ptr(), ldp,
              scale.data_ptr(), q_gu.data_ptr(), dx.data_ptr(), R, _lib.stream_of(dgu8))
    return dx


def moe_wgrad(at, bt, M: int, N: int, E: int, plan, sa, sb):
    """out[e] = sum over expert e's rows of at^T bt / (sa * sb), fp32 [E, M, N];
    at (e5m2) and bt (e4m3) token-contiguous K-slab copies over padded expert order."""
    _cuda_contig("at", at, E5M2, 3)
    _cuda_contig("bt", bt, E4M3, 3)
    ldp = at.shape[0] * SLAB
    out = torch.empty(E, M, N, dtype=torch.float32, device=at.device)
    nws = _lib.query("sfp8_moe_wgrad_workspace_floats", M, N, E)
    ws = torch.empty(max(nws, 1), dtype=torch.float32, device=at.device)
    _lib.call("sfp8_moe_gemm_wgrad", at.data_ptr(), FMT_E5M2, bt.data_ptr(), FMT_E4M3, M, N, E, plan.data_ptr(), ldp,
              sa.data_ptr(), sb.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(at))
    return out


def moe_wgrad_rows(a8, b8, M: int, N: int, E: int, plan, sa, sb, *, a_rows: bool = True, b_rows: bool = True):
    """moe_wgrad with a8 (e5m2) and/or b8 (e4m3) the row K-slab of the
    expert-order activation over padded rows ([rows/64, ldp, 64]: read
    through transposing LDS reads) instead of the token-contiguous copy."""
    _cuda_contig("a8", a8, E5M2, 3)
    _cuda_contig("b8", b8, E4M3, 3)
    _need(a_rows or b_rows, "at least one row K-slab operand (else use moe_wgrad)")
    ldp = a8.shape[1] if a_rows else a8.shape[0] * SLAB
    _need((b8.shape[1] if b_rows else b8.shape[0] * SLAB) == ldp, "a8, b8 must cover the same padded rows")
    _need(not a_rows or a8.shape[0] * SLAB == M, "a8 must be the row K-slab of [ldp, M]")
    _need(not b_rows or b8.shape[0] * SLAB == N, "b8 must be the row K-slab of [ldp, N]")
    out = torch.empty(E, M, N, dtype=torch.float32, device=a8.device)
    nws = _lib.query("sfp8_moe_wgrad_rows_workspace_floats", M, N, E)
    ws = torch.empty(max(nws, 1), dtype=torch.float32, device=a8.device)
    _lib.call("sfp8_moe_gemm_wgrad_rows", a8.data_ptr(), FMT_E5M2, int(a_rows), b8.data_ptr(), FMT_E4M3, int(b_rows),
              M, N, E, plan.data_ptr(), ldp, sa.data_ptr(), sb.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
              _lib.stream_of(a8))
    return out


def moe_topk_sum(dx, inverse_permutation, T: int, top_k: int):
    """out[t] = sum of the top_k expert-order rows of token t (bf16 [T, D])."""
    _cuda_contig("dx", dx, torch.bfloat16, 2)
    inv = inverse_permutation.to(torch.int64).contiguous()
    R, D = dx.shape
    out = torch.empty(T, D, dtype=torch.bfloat16, device=dx.device)
    _lib.call("sfp8_moe_topk_sum", dx.data_ptr(), R, D, inv.data_ptr(), T, top_k, out.data_ptr(), _lib.stream_of(dx))
    return out


# ----------------------------------------------------- bf16 SwiGLU path
# The default (non-FP8) MLP path: bf16 K-slabs (32 elements of K per 64-byte
# row), rows dense (no plan) or in padded expert order (a MoE plan).
BF16 = torch.bfloat16


def bf16_weight_slabs(w: torch.Tensor, norm_w=None, *, rows: bool = True, transposed: bool = True):
    """bf16 K-slabs of W [E, R, C] (fp32, times norm_w[c] when given, or bf16):
    (ws: stacked K-slabs of W[e] [R, C] or None, wt: of W[e]^T [C, R] or None)."""
    _need(w.is_cuda and w.dim() == 3 and w.is_contiguous() and w.dtype in (torch.float32, BF16),
          "w must be a contiguous [E, R, C] fp32 or bf16 device tensor")
    E, R, C = w.shape
    _need(R % 64 == 0 and C % 64 == 0, f"weight dims {R} x {C} must be multiples of 64")
    if norm_w is not None:
        _cuda_contig("norm_w", norm_w, torch.float32, 1)
    dev = w.device
    ws = torch.empty((E,) + kslab_shape(R, C, BF16), dtype=BF16, device=dev) if rows else None
    wt = torch.empty((E,) + kslab_shape(C, R, BF16), dtype=BF16, device=dev) if transposed else None
    _lib.call("sfp8_bf16_weight_slabs", w.data_ptr(), int(w.dtype == BF16), _lib.ptr(norm_w), E, R, C, _lib.ptr(ws),
              _lib.ptr(wt), _lib.stream_of(w))
    return ws, wt


def bf16_rows_prep(x: torch.Tensor, plan, ldp: int, eps=None, *, copy: bool = True, rows: bool = False):
    """(rstd [rows] fp32 or None, xt or None, xs or None): xt the
    token-contiguous bf16 K-slab of x^T over ldp padded rows (copy=False
    skips it: bf16_wgrad_rows reads x itself); xs (rows=True) the row K-slab
    of x over the ldp rows, for bf16_swiglu_fwd; rstd = 1/sqrt(mean(x^2) +
    eps) when eps is given (dense rows only)."""
    _cuda_contig("x", x, BF16, 2)
    n, D = x.shape
    _need(copy or rows or eps is not None, "nothing to compute")
    xt = kslab_empty(D, ldp, BF16, x.device) if copy else None
    xs = kslab_empty(ldp, D, BF16, x.device) if rows else None
    rstd = torch.empty(n, dtype=torch.float32, device=x.device) if eps is not None else None
    _lib.call("sfp8_bf16_rows_prep", x.data_ptr(), n, D, _lib.ptr(plan), ldp, float(eps or 0.0), _lib.ptr(rstd),
              _lib.ptr(xt), _lib.ptr(xs), _lib.stream_of(x))
    return rstd, xt, xs


def bf16_swiglu_fwd(x: torch.Tensor, ws: torch.Tensor, I: int, rstd=None, plan=None, ldp: int = 0, xs=None):
    """(gu [rows, 2I], h [rows, I]) bf16: the gate/up GEMM with the SwiGLU
    epilogue, rows scaled by rstd when given (dense) or grouped by a plan.
    Dense: xs, the row K-slab of x from bf16_rows_prep(rows=True), when
    given is read instead of x (the same result, a faster read)."""
    _cuda_contig("x", x, BF16, 2)
    n, D = x.shape
    gu = torch.empty(n, 2 * I, dtype=BF16, device=x.device)
    h = torch.empty(n, I, dtype=BF16, device=x.device)
    if plan is None:
        if xs is not None:
            _kslab("xs", xs, BF16, ldt_of(n), D)
        a = x if xs is None else xs
        _lib.call("sfp8_bf16_gemm_swiglu_fwd", a.data_ptr(), int(xs is not None), ws.data_ptr(), n, D, I,
                  _lib.ptr(rstd), gu.data_ptr(), h.data_ptr(), _lib.stream_of(x))
    else:
        _lib.call("sfp8_bf16_moe_gemm_swiglu_fwd", x.data_ptr(), ws.data_ptr(), ws.shape[0], D, I, plan.data_ptr(),
                  ldp, gu.data_ptr(), h.data_ptr(), _lib.stream_of(x))
    return gu, h


def bf16_swiglu_bwd(gu: torch.Tensor, dout: torch.Tensor, rstd, plan, ldp: int, *, copy: bool = True):
    """(gs, gt): G' = bf16 SwiGLU gradient of the rows (times rstd when given)
    as the K-slab over ldp padded rows and its token-contiguous transpose
    (copy=False skips gt, None: the weight gradient then reads gs itself)."""
    _cuda_contig("gu", gu, BF16, 2)
    _cuda_contig("dout", dout, BF16, 2)
    n, I2 = gu.shape
    _need(dout.shape == (n, I2 // 2), "dout must be [rows, I]")
    gs = kslab_empty(ldp, I2, BF16, gu.device)
    gt = kslab_empty(I2, ldp, BF16, gu.device) if copy else None
    _lib.call("sfp8_bf16_swiglu_bwd", gu.data_ptr(), dout.data_ptr(), n, I2 // 2, _lib.ptr(rstd), _lib.ptr(plan), ldp,
              gs.data_ptr(), _lib.ptr(gt), _lib.stream_of(gu))
    return gs, gt


def bf16_gemm(a: torch.Tensor, b: torch.Tensor, rows: int, N: int, K: int, plan=None):
    """out [rows, N] bf16 = A @ B^T, A a bf16 K-slab over padded rows (dense:
    the first `rows` rows; a plan: the expert-order rows of each tile), B the
    (stacked per expert) bf16 K-slab of [N, K]."""
    lda = a.shape[1]
    out = torch.empty(rows, N, dtype=BF16, device=a.device)
    if plan is None:
        _lib.call("sfp8_bf16_gemm", a.data_ptr(), b.data_ptr(), rows, N, K, lda, out.data_ptr(), _lib.stream_of(a))
    else:
        _lib.call("sfp8_bf16_moe_gemm", a.data_ptr(), b.data_ptr(), b.shape[0], N, K, plan.data_ptr(), lda,
                  out.data_ptr(), _lib.stream_of(a))
    return out


def bf16_norm_dh(p: torch.Tensor, h: torch.Tensor, rstd: torch.Tensor):
    """dh = bf16(p - rstd^2 * sum(h * p) / D * h) per row."""
    _cuda_contig("p", p, BF16, 2)
    _cuda_contig("h", h, BF16, 2)
    T, D = h.shape
    dh = torch.empty_like(h)
    _lib.call("sfp8_bf16_norm_dh", p.data_ptr(), h.data_ptr(), rstd.data_ptr(), T, D, dh.data_ptr(), _lib.stream_of(h))
    return dh


def bf16_wgrad(at: torch.Tensor, bt: torch.Tensor, M: int, N: int, plan=None, E: int = 1):
    """bf16(A^T B) over the padded rows: [M, N] (dense) or [E, M, N] (per
    expert, with a plan); at, bt the token-contiguous bf16 K-slabs of [M, ldp]
    and [N, ldp]."""
    ldp = at.shape[0] * (SLAB // 2)
    dev = at.device
    if plan is None:
        out = torch.empty(M, N, dtype=BF16, device=dev)
        nws = _lib.query("sfp8_bf16_wgrad_workspace_floats", M, N, ldp)
        ws = torch.empty(max(nws, 1), dtype=torch.float32, device=dev)
        _lib.call("sfp8_bf16_gemm_wgrad", at.data_ptr(), bt.data_ptr(), M, N, ldp, out.data_ptr(), ws.data_ptr(),
                  ws.numel(), _lib.stream_of(at))
    else:
        out = torch.empty(E, M, N, dtype=BF16, device=dev)
        nws = _lib.query("sfp8_bf16_moe_wgrad_workspace_floats", M, N, E)
        ws = torch.empty(max(nws, 1), dtype=torch.float32, device=dev)
        _lib.call("sfp8_bf16_moe_gemm_wgrad", at.data_ptr(), bt.data_ptr(), M, N, E, plan.data_ptr(), ldp,
                  out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(at))
    return out


def bf16_wgrad_rows(gs: torch.Tensor, b: torch.Tensor, M: int, N: int, plan=None, E: int = 1, T=None):
    """bf16_wgrad with A read from gs, the bf16 K-slab of G' over the padded
    rows, through transposing LDS reads.  Dense (no plan): b is x itself,
    row-major [T, N] bf16, also transposed on read, or (3-d) the
    token-contiguous K-slab of x^T (bf16_rows_prep; T then gives the tokens);
    with a plan b is the token-contiguous K-slab of x^T over the padded rows."""
    _cuda_contig("gs", gs, BF16, 3)
    ldp = gs.shape[1]
    _need(gs.shape[0] * (SLAB // 2) == M, "gs must be the bf16 K-slab of [ldp, M]")
    dev = gs.device
    if plan is None:
        x_rows = b.dim() == 2
        _cuda_contig("x", b, BF16, 2 if x_rows else 3)
        if x_rows:
            _need(b.shape[1] == N and b.shape[0] <= ldp, "x must be [T, N] with T <= the padded rows")
            T = b.shape[0]
        else:
            _need(b.shape[0] * (SLAB // 2) == ldp and T is not None, "xt must cover the padded rows; give T")
        out = torch.empty(M, N, dtype=BF16, device=dev)
        nws = _lib.query("sfp8_bf16_wgrad_workspace_floats", M, N, ldp)
        ws = torch.empty(max(nws, 1), dtype=torch.float32, device=dev)
        _lib.call("sfp8_bf16_gemm_wgrad_rows", gs.data_ptr(), b.data_ptr(), int(x_rows), M, N, T, ldp, out.data_ptr(),
                  ws.data_ptr(), ws.numel(), _lib.stream_of(gs))
    else:
        _cuda_contig("bt", b, BF16, 3)
        _need(b.shape[0] * (SLAB // 2) == ldp, "bt must cover the same padded rows")
        out = torch.empty(E, M, N, dtype=BF16, device=dev)
        nws = _lib.query("sfp8_bf16_moe_wgrad_workspace_floats", M, N, E)
        ws = torch.empty(max(nws, 1), dtype=torch.float32, device=dev)
        _lib.call("sfp8_bf16_moe_gemm_wgrad_rows", gs.data_ptr(), b.data_ptr(), M, N, E, plan.data_ptr(), ldp,
                  out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(gs))
    return out


def bf16_fold_grads(dwp: torch.Tensor, w: torch.Tensor, norm_w: torch.Tensor):
    """(dw = f32(dwp) * norm_w, dnorm_w = sum over rows of f32(dwp) * w): the
    gradients of the fp32 gate/up master and the norm weight from the bf16
    gradient of the folded weight."""
    M, N = dwp.shape
    dw = torch.empty(M, N, dtype=torch.float32, device=dwp.device)
    dnw = torch.empty(N, dtype=torch.float32, device=dwp.device)
    part = torch.empty(_lib.query("sfp8_bf16_fold_partials", M, N), dtype=torch.float32, device=dwp.device)
    _lib.call("sfp8_bf16_fold_grads", dwp.data_ptr(), w.data_ptr(), norm_w.data_ptr(), M, N, dw.data_ptr(),
              dnw.data_ptr(), part.data_ptr(), part.numel(), _lib.stream_of(dwp))
    return dw, dnw


# ----------------------------------------------------- the optimizer's momentum stage
def _flat_state(name: str, t, dtype: torch.dtype, numel: int, device, align: int) -> None:
    """t is a contiguous `dtype` tensor of `numel` elements on `device` whose
    data pointer is `align`-byte aligned (what the kernels' vector accesses
    need); raises ValueError before anything is launched."""
    _need(isinstance(t, torch.Tensor), f"{name} must be a tensor")
    _need(t.is_cuda and t.device == device, f"{name} must be a ROCm device tensor on {device}")
    _need(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _need(t.is_contiguous(), f"{name} must be contiguous")
    _need(t.numel() == numel, f"{name} must have {numel} elements, got {t.numel()}")
    _need(t.data_ptr() % align == 0, f"{name} must be {align}-byte aligned")


def _momentum_weights(momentum: float) -> None:
    """The kernels take w_v = 1 - momentum and w_u = momentum as fp32 values
    (ctypes rounds them as the reference's launch does) with
    -0.5 < w_v < 0.5 <= w_u."""
    import numpy as np

    w_v, w_u = np.float32(1.0 - momentum), np.float32(momentum)
    _need(bool(-0.5 < w_v < 0.5 <= w_u), f"momentum {momentum} outside the kernel's range (0.5 <= momentum < 1.5)")


def momentum_stage(g: torch.Tensor, v: torch.Tensor, u: torch.Tensor, momentum: float) -> None:
    """v <- lerp(v, g, 1 - momentum) in place; u <- bf16(lerp(g, v, momentum))."""
    _need(isinstance(g, torch.Tensor) and g.is_cuda, "g must be a ROCm device tensor")
    n = g.numel()
    _need(n % 4 == 0, "g, v, u need a multiple of 4 elements")
    _flat_state("g", g, torch.float32, n, g.device, 16)
    _flat_state("v", v, torch.float32, n, g.device, 16)
    _flat_state("u", u, BF16, n, g.device, 8)
    _momentum_weights(momentum)
    _lib.call("sfp8_momentum_stage", g.data_ptr(), v.data_ptr(), u.data_ptr(), n, 1.0 - momentum, momentum,
              _lib.stream_of(g))


def wgrad_momentum(a8, b8, M: int, N: int, sa, sb, v: torch.Tensor, u: torch.Tensor, momentum: float, grad=None, *,
                   a_rows: bool = False, b_rows: bool = False):
    """wgrad (a_rows = b_rows = False) or wgrad_rows of the same operands
    handed straight to the momentum stage: v <- lerp(v, dW, 1 - momentum),
    u <- bf16(lerp(dW, v, momentum)); dW is also written to `grad` when
    given.  v and grad are fp32, u bf16, each [M, N] on the operands' device;
    sa and sb are fp32 scales there."""
    _cuda_contig("a8", a8, E5M2, 3)
    _cuda_contig("b8", b8, E4M3, 3)
    _need(b8.device == a8.device, "a8, b8 must be on the same device")
    _flat_state("v", v, torch.float32, M * N, a8.device, 16)
    _flat_state("u", u, BF16, M * N, a8.device, 8)
    if grad is not None:
        _flat_state("grad", grad, torch.float32, M * N, a8.device, 16)
    for name, t in (("sa", sa), ("sb", sb)):
        _need(isinstance(t, torch.Tensor) and t.is_cuda and t.device == a8.device and t.dtype == torch.float32
              and t.numel() >= 1, f"{name} must be an fp32 scale on {a8.device}")
    _momentum_weights(momentum)
    ldt = a8.shape[1] if a_rows else a8.shape[0] * SLAB
    _need((b8.shape[1] if b_rows else b8.shape[0] * SLAB) == ldt, "a8, b8 must cover the same tokens")
    nws = _lib.query("sfp8_wgrad_momentum_workspace_floats", M, N, ldt)
    ws = torch.empty(max(nws, 1), dtype=torch.float32, device=a8.device)
    _lib.call("sfp8_gemm_wgrad_momentum", a8.data_ptr(), FMT_E5M2, int(a_rows), b8.data_ptr(), FMT_E4M3, int(b_rows),
              M, N, ldt, sa.data_ptr(), sb.data_ptr(), _lib.ptr(grad), v.data_ptr(), u.data_ptr(), 1.0 - momentum,
              momentum, ws.data_ptr(), ws.numel(), _lib.stream_of(a8))
