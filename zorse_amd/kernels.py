"""Tensor-level wrappers of the C ABI.

Each wrapper validates device / dtype / layout in Python (so bad input is a
``ValueError`` before anything is enqueued), allocates outputs and workspaces
with torch's caching allocator, and enqueues the kernel on torch's current
stream.  The C side re-validates and reports through ``zk_last_error``.
Nothing here falls back to another implementation: without the library or a
GPU tensor these functions raise.
"""
from __future__ import annotations

import math

import torch

from . import _abi
from ._abi import check, dtype_code, lib, ptr, stream_handle

_LOWP = (torch.bfloat16, torch.float16)


def _require_gpu(*tensors: torch.Tensor | None) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("zorse_amd kernels need GPU tensors (got a CPU tensor)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev


def _require_contig(name: str, t: torch.Tensor) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# --------------------------------------------------------------- RMSNorm ---

def rmsnorm_fwd(x: torch.Tensor, weight: torch.Tensor, eps: float,
                residual: torch.Tensor | None = None, out=None):
    """y = w * round(h * rsqrt(mean(h^2) + eps)), h = x (+ residual).

    Returns (y, rstd, h); h is x itself when no residual is given.  ``out``
    may supply preallocated (y, rstd) or (y, rstd, h)."""
    dev = _require_gpu(x, weight, residual)
    if x.dtype not in (torch.float32, *_LOWP):
        raise ValueError(f"unsupported activation dtype {x.dtype}")
    hidden = x.shape[-1]
    if weight.shape != (hidden,):
        raise ValueError(f"weight shape {tuple(weight.shape)} != ({hidden},)")
    _require_contig("x", x)
    _require_contig("weight", weight)
    rows = x.numel() // hidden if hidden else 0
    if out is not None:
        y, rstd = out[0], out[1]
        _require_gpu(x, y, rstd)
        if y.shape != x.shape or y.dtype != x.dtype or not y.is_contiguous():
            raise ValueError("out y must match x")
        if rstd.numel() != rows or rstd.dtype != torch.float32 or not rstd.is_contiguous():
            raise ValueError("out rstd must be contiguous fp32 with one value per row")
    else:
        y = torch.empty_like(x)
        rstd = torch.empty(x.shape[:-1], device=dev, dtype=torch.float32)
    h = x
    if residual is not None:
        if residual.shape != x.shape or residual.dtype != x.dtype:
            raise ValueError("residual must match x in shape and dtype")
        _require_contig("residual", residual)
        if out is not None and len(out) > 2:
            h = out[2]
            _require_gpu(h)
            if h.shape != x.shape or h.dtype != x.dtype or not h.is_contiguous() \
                    or h.device != dev:
                raise ValueError("out h must match x (shape, dtype, device, contiguous)")
        else:
            h = torch.empty_like(x)
    check(lib().zk_rmsnorm_fwd(ptr(x), ptr(residual), ptr(h) if residual is not None else None,
                               ptr(weight), ptr(y), ptr(rstd), rows, hidden, float(eps),
                               dtype_code(x.dtype), dtype_code(weight.dtype),
                               stream_handle(dev)), "zk_rmsnorm_fwd")
    return y, rstd, h


def rmsnorm_bwd_workspace_elems(rows: int, hidden: int) -> int:
    """fp32 elements of scratch zk_rmsnorm_bwd needs (the dw partial rows)."""
    return max(int(lib().zk_rmsnorm_bwd_workspace(rows, hidden)), 1)


def rmsnorm_bwd(dy: torch.Tensor, h: torch.Tensor, weight: torch.Tensor,
                rstd: torch.Tensor, dres: torch.Tensor | None = None,
                dw: torch.Tensor | None = None, accumulate: bool = False,
                dw_dtype: torch.dtype | None = None, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None):
    """Returns (dx, dw).  dx includes dres when given; dw is written (or
    accumulated into) ``dw`` if supplied, else a new tensor -- in the weight's
    dtype either way (``dw_dtype``, if given, must be that dtype).  ``out`` /
    ``workspace`` may be preallocated."""
    dev = _require_gpu(dy, h, weight, rstd, dres, dw)
    hidden = h.shape[-1]
    for name, t in (("dy", dy), ("h", h), ("rstd", rstd), ("weight", weight)):
        _require_contig(name, t)
    if dy.shape != h.shape or dy.dtype != h.dtype:
        raise ValueError("dy must match h in shape and dtype")
    rows = h.numel() // hidden if hidden else 0
    if rstd.numel() != rows or rstd.dtype != torch.float32:
        raise ValueError("rstd must be fp32 with one value per row")
    if dres is not None:
        if dres.shape != h.shape or dres.dtype != h.dtype:
            raise ValueError("dres must match h")
        _require_contig("dres", dres)
    if dw_dtype is not None and dw_dtype != weight.dtype:
        raise ValueError(f"dw is written in the weight's dtype {weight.dtype} (got dw_dtype "
                         f"{dw_dtype})")
    if dw is None:
        dw = torch.empty(hidden, device=dev, dtype=weight.dtype)
        accumulate = False
    elif dw.shape != (hidden,) or not dw.is_contiguous() or dw.dtype != weight.dtype:
        raise ValueError(f"dw must be a contiguous [hidden] tensor of the weight's dtype "
                         f"{weight.dtype}")
    if out is not None:
        _require_gpu(h, out)
        if out.shape != h.shape or out.dtype != h.dtype or not out.is_contiguous():
            raise ValueError("out must match h")
        dx = out
    else:
        dx = torch.empty_like(h)
    ws_elems = rmsnorm_bwd_workspace_elems(rows, hidden)
    if workspace is not None:
        _require_gpu(h, workspace)
        if workspace.dtype != torch.float32 or workspace.numel() < ws_elems or \
                not workspace.is_contiguous():
            raise ValueError(f"workspace must be contiguous fp32 with >= {ws_elems} elements")
        ws = workspace
    else:
        ws = torch.empty(ws_elems, device=dev, dtype=torch.float32)
    check(lib().zk_rmsnorm_bwd(ptr(dy), ptr(h), ptr(weight), ptr(rstd), ptr(dres), ptr(dx),
                               ptr(dw), int(accumulate), ptr(ws), ws.numel(), rows, hidden,
                               dtype_code(h.dtype), dtype_code(weight.dtype),
                               stream_handle(dev)), "zk_rmsnorm_bwd")
    return dx, dw


# ----------------------------------------------------------------- SwiGLU --

def _row_view_check(name: str, t: torch.Tensor) -> int:
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D row-major view (unit column stride)")
    return t.stride(0)


def swiglu_fwd(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None):
    """z = round(round(silu(g)) * u) for 2-D views gate/up sharing a row stride."""
    dev = _require_gpu(gate, up, out)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("gate and up must match")
    ld = _row_view_check("gate", gate)
    if _row_view_check("up", up) != ld:
        raise ValueError("gate and up must share a row stride")
    rows, cols = gate.shape
    if out is None:
        out = torch.empty(rows, cols, device=dev, dtype=gate.dtype)
    elif out.shape != (rows, cols) or out.dtype != gate.dtype or out.device != dev:
        raise ValueError("out must be [rows, cols] of gate's dtype on gate's device")
    ldz = _row_view_check("out", out)
    check(lib().zk_swiglu_fwd(ptr(gate), ptr(up), ld, ptr(out), ldz, rows, cols,
                              dtype_code(gate.dtype), stream_handle(dev)), "zk_swiglu_fwd")
    return out


def swiglu_bwd(dz: torch.Tensor, gate: torch.Tensor, up: torch.Tensor,
               dgate: torch.Tensor, dup: torch.Tensor) -> None:
    """Writes dgate / dup (2-D views sharing a row stride)."""
    dev = _require_gpu(dz, gate, up, dgate, dup)
    ld_in = _row_view_check("gate", gate)
    if _row_view_check("up", up) != ld_in:
        raise ValueError("gate and up must share a row stride")
    ld_out = _row_view_check("dgate", dgate)
    if _row_view_check("dup", dup) != ld_out:
        raise ValueError("dgate and dup must share a row stride")
    ld_dz = _row_view_check("dz", dz)
    rows, cols = gate.shape
    for t in (dz, up, dgate, dup):
        if t.shape != (rows, cols) or t.dtype != gate.dtype:
            raise ValueError("swiglu_bwd operands must match gate")
    check(lib().zk_swiglu_bwd(ptr(dz), ld_dz, ptr(gate), ptr(up), ld_in, ptr(dgate),
                              ptr(dup), ld_out, rows, cols, dtype_code(gate.dtype),
                              stream_handle(dev)), "zk_swiglu_bwd")


def gemm_nt_supported(M: int, N: int, K: int) -> bool:
    """Whether an [M, K] x [N, K]^T product is on the MFMA pipeline's grid
    (M, N multiples of 256, K a multiple of 128 and at least 256)."""
    return bool(lib().zk_gemm_nt_supported(M, N, K))


def _gemm_operand(name: str, t: torch.Tensor):
    """(rows, cols, leading dimension) of a 2-D operand with unit column stride
    and non-overlapping rows."""
    if t.dim() != 2:
        raise ValueError(f"gemm: {name} must be 2-D, got shape {tuple(t.shape)}")
    rows, cols = t.shape
    if t.stride(1) != 1 and cols > 1:
        raise ValueError(f"gemm: {name} needs unit column stride")
    ld = t.stride(0) if rows > 1 else max(cols, 1)
    if ld < cols:
        raise ValueError(f"gemm: {name} has overlapping rows (row stride {ld} < {cols})")
    return rows, cols, max(ld, 1)


def gemm(a: torch.Tensor, b: torch.Tensor, *, a_kmajor: bool = False, b_kmajor: bool = False,
         residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """C = op(a) op(b)^T (+ residual) from the hand-written GEMMs (zk_gemm):
    a is [M, K] (``a_kmajor``: [K, M]) and b is [N, K] (``b_kmajor``:
    [K, N]), each with unit column stride -- so x W^T is gemm(x, W), dY W is
    gemm(dY, W, b_kmajor=True) and dY^T X is gemm(dY, X, a_kmajor=True,
    b_kmajor=True), all on the tensors as stored.  bf16 / fp16 (fp32
    accumulation, one rounding) or fp32; every tensor shares the dtype.
    ``out`` / ``residual``: [M, N] with unit column stride."""
    dev = _require_gpu(a, b, residual, out)
    if a.dtype != b.dtype or a.dtype not in (torch.float32, *_LOWP):
        raise ValueError(f"gemm: a and b must share a float dtype, got {a.dtype} and {b.dtype}")
    ra, ca, lda = _gemm_operand("a", a)
    rb, cb, ldb = _gemm_operand("b", b)
    M, K = (ca, ra) if a_kmajor else (ra, ca)
    N, Kb = (cb, rb) if b_kmajor else (rb, cb)
    if Kb != K:
        raise ValueError(f"gemm: reduction sizes differ ({K} and {Kb}) for a {tuple(a.shape)} "
                         f"(k-major {a_kmajor}) and b {tuple(b.shape)} (k-major {b_kmajor})")
    if out is None:
        out = torch.empty(M, N, device=dev, dtype=a.dtype)
    if out.shape != (M, N) or out.dtype != a.dtype:
        raise ValueError(f"gemm: out must be [{M}, {N}] of the operands' dtype")
    _, _, ldc = _gemm_operand("out", out)
    ldr = 0
    if residual is not None:
        if residual.shape != (M, N) or residual.dtype != a.dtype:
            raise ValueError(f"gemm: residual must be [{M}, {N}] of the operands' dtype")
        _, _, ldr = _gemm_operand("residual", residual)
    check(lib().zk_gemm(ptr(a), lda, int(a_kmajor), ptr(b), ldb, int(b_kmajor), ptr(out), ldc,
                        ptr(residual) if residual is not None else None, ldr, M, N, K,
                        dtype_code(a.dtype), stream_handle(dev)), "zk_gemm")
    return out


def gemm_rope(x: torch.Tensor, w: torch.Tensor, *, seq_len: int, rot_cols: int, head_dim: int,
              cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor | None = None,
              interleaved: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """x W^T with the rotary embedding applied to its first ``rot_cols``
    columns (whole heads of ``head_dim``), rows being tokens b * seq_len + s
    (zk_gemm_rope): the q|k|v projection and the RoPE pass in one call, equal
    to gemm(x, w) followed by rope_ on the q and k heads.  cos / sin /
    positions as for rope_."""
    dev = _require_gpu(x, w, cos, sin, positions, out)
    if x.dtype != w.dtype or x.dtype not in (torch.float32, *_LOWP):
        raise ValueError(f"gemm_rope: x and w must share a float dtype, got {x.dtype} and {w.dtype}")
    M, K = x.shape
    N, Kw = w.shape
    if Kw != K:
        raise ValueError(f"gemm_rope: reduction sizes differ ({K} and {Kw})")
    if head_dim <= 0 or head_dim % 2 or rot_cols < 0 or rot_cols % head_dim or rot_cols > N:
        raise ValueError(f"gemm_rope: rot_cols {rot_cols} must be whole heads of {head_dim} within {N}")
    if seq_len <= 0 or M % seq_len:
        raise ValueError(f"gemm_rope: {M} rows are not whole sequences of {seq_len}")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != head_dim // 2 \
                or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 [n_pos, {head_dim // 2}] table")
    if cos.shape != sin.shape:
        raise ValueError("cos and sin tables differ in shape")
    n_pos = cos.shape[0]
    if positions is not None:
        if positions.dtype != torch.int64 or positions.numel() != seq_len \
                or not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int64 [seq_len] tensor")
    elif n_pos < seq_len:
        raise ValueError(f"table holds {n_pos} positions < seq_len={seq_len}")
    _, _, lda = _gemm_operand("x", x)
    _, _, ldb = _gemm_operand("w", w)
    if out is None:
        out = torch.empty(M, N, device=dev, dtype=x.dtype)
    if out.shape != (M, N) or out.dtype != x.dtype:
        raise ValueError(f"gemm_rope: out must be [{M}, {N}] of the operands' dtype")
    _, _, ldc = _gemm_operand("out", out)
    check(lib().zk_gemm_rope(ptr(x), lda, ptr(w), ldb, ptr(out), ldc, M, N, K, seq_len, rot_cols,
                             head_dim, ptr(cos), ptr(sin), n_pos, ptr(positions),
                             _abi.ZK_ROPE_INTERLEAVED if interleaved else _abi.ZK_ROPE_HALF,
                             dtype_code(x.dtype), stream_handle(dev)), "zk_gemm_rope")
    return out


def gemm_path(M: int, N: int, K: int, lda: int, ldb: int, ldc: int, dtype: torch.dtype,
              a_kmajor: bool = False, b_kmajor: bool = False, ldr: int = -1) -> str:
    """Which kernel zk_gemm runs for a launch with 16-byte aligned pointers:
    "tiled" (the 256 x 256 MFMA pipeline) or "general" (host-only query)."""
    code = lib().zk_gemm_path(M, N, K, lda, int(a_kmajor), ldb, int(b_kmajor), ldc, ldr,
                              dtype_code(dtype))
    check(code if code < 0 else 0, "zk_gemm_path")
    return "tiled" if code == 1 else "general"


def gemm_nt(a: torch.Tensor, b: torch.Tensor, residual: torch.Tensor | None = None,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """a @ b.T (+ residual): a [M, K] and b [N, K] with unit column stride
    (contiguous along the reduction); zk_gemm_nt."""
    dev = _require_gpu(a, b, residual, out)
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[1]:
        raise ValueError(f"gemm_nt: a [M, K] and b [N, K] expected, got {tuple(a.shape)} and "
                         f"{tuple(b.shape)}")
    if a.dtype != b.dtype or a.dtype not in (torch.float32, *_LOWP):
        raise ValueError("gemm_nt: a and b must share a float dtype")
    M, K = a.shape
    N = b.shape[0]
    lda = _row_view_check("a", a)
    ldb = _row_view_check("b", b)
    if out is None:
        out = torch.empty(M, N, device=dev, dtype=a.dtype)
    if out.shape != (M, N) or out.dtype != a.dtype:
        raise ValueError("gemm_nt: out must be [M, N] of the operands' dtype")
    ldc = _row_view_check("out", out)
    ldr = 0
    if residual is not None:
        if residual.shape != (M, N) or residual.dtype != a.dtype:
            raise ValueError("gemm_nt: residual must be [M, N] of the operands' dtype")
        ldr = _row_view_check("residual", residual)
    check(lib().zk_gemm_nt(ptr(a), lda, ptr(b), ldb, ptr(out), ldc,
                           ptr(residual) if residual is not None else None, ldr, M, N, K,
                           dtype_code(a.dtype), stream_handle(dev)), "zk_gemm_nt")
    return out


def gemm_swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                gu_out: torch.Tensor | None = None, transposed: bool = False):
    """(gu, z[, z^T]) with gu = [x Wg^T | x Wu^T] ([M, 2F], kept for the
    backward) and z = SwiGLU(g, u), from one hand-written GEMM with the
    activation in its epilogue.  x [M, K], w_gate / w_up [F, K] with unit
    column stride; 2-byte dtypes, K % 64 == 0, M and F multiples of 8."""
    dev = _require_gpu(x, w_gate, w_up, gu_out)
    if x.dim() != 2 or w_gate.dim() != 2 or w_gate.shape != w_up.shape:
        raise ValueError("gemm_swiglu: x [M, K] and two [F, K] weights expected")
    M, K = x.shape
    F = w_gate.shape[0]
    if w_gate.shape[1] != K or x.dtype != w_gate.dtype or w_up.dtype != x.dtype:
        raise ValueError("gemm_swiglu: operands must share K and dtype")
    ld_x = _row_view_check("x", x)
    ld_w = _row_view_check("w_gate", w_gate)
    if _row_view_check("w_up", w_up) != ld_w:
        raise ValueError("w_gate and w_up must share a row stride")
    if gu_out is None:
        gu_out = torch.empty(M, 2 * F, device=dev, dtype=x.dtype)
    if gu_out.shape != (M, 2 * F) or gu_out.dtype != x.dtype or gu_out.stride(1) != 1:
        raise ValueError("gu_out must be [M, 2F] with unit column stride")
    z = torch.empty(M, F, device=dev, dtype=x.dtype)
    zt = torch.empty(F, M, device=dev, dtype=x.dtype) if transposed else None
    check(lib().zk_gemm_swiglu(ptr(x), ld_x, ptr(w_gate), ptr(w_up), ld_w, ptr(gu_out),
                               ptr(gu_out[:, F:]), gu_out.stride(0), ptr(z), F,
                               ptr(zt) if zt is not None else None, M, M, F, K,
                               dtype_code(x.dtype), stream_handle(dev)), "zk_gemm_swiglu")
    return (gu_out, z, zt) if transposed else (gu_out, z)


def swiglu_fwd_t(gate: torch.Tensor, up: torch.Tensor):
    """(z, z^T): the SwiGLU output and its transpose [cols, rows] from one pass
    (2-byte dtypes, rows and cols multiples of 8)."""
    dev = _require_gpu(gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("gate and up must match")
    ld = _row_view_check("gate", gate)
    if _row_view_check("up", up) != ld:
        raise ValueError("gate and up must share a row stride")
    rows, cols = gate.shape
    z = torch.empty(rows, cols, device=dev, dtype=gate.dtype)
    zt = torch.empty(cols, rows, device=dev, dtype=gate.dtype)
    check(lib().zk_swiglu_fwd_t(ptr(gate), ptr(up), ld, ptr(z), cols, ptr(zt), rows, rows, cols,
                                dtype_code(gate.dtype), stream_handle(dev)), "zk_swiglu_fwd_t")
    return z, zt


def swiglu_bwd_t(dz: torch.Tensor, gate: torch.Tensor, up: torch.Tensor,
                 dgate: torch.Tensor, dup: torch.Tensor, dgate_t: torch.Tensor,
                 dup_t: torch.Tensor) -> None:
    """swiglu_bwd that also writes dgate^T / dup^T ([cols, rows] views sharing
    a row stride; 2-byte dtypes, rows and cols multiples of 8)."""
    dev = _require_gpu(dz, gate, up, dgate, dup, dgate_t, dup_t)
    ld_in = _row_view_check("gate", gate)
    if _row_view_check("up", up) != ld_in:
        raise ValueError("gate and up must share a row stride")
    ld_out = _row_view_check("dgate", dgate)
    if _row_view_check("dup", dup) != ld_out:
        raise ValueError("dgate and dup must share a row stride")
    ld_t = _row_view_check("dgate_t", dgate_t)
    if _row_view_check("dup_t", dup_t) != ld_t:
        raise ValueError("dgate_t and dup_t must share a row stride")
    ld_dz = _row_view_check("dz", dz)
    rows, cols = gate.shape
    for t in (dz, up, dgate, dup):
        if t.shape != (rows, cols) or t.dtype != gate.dtype:
            raise ValueError("swiglu_bwd_t operands must match gate")
    for t in (dgate_t, dup_t):
        if t.shape != (cols, rows) or t.dtype != gate.dtype:
            raise ValueError("transposed outputs must be (cols, rows) of gate's dtype")
    check(lib().zk_swiglu_bwd_t(ptr(dz), ld_dz, ptr(gate), ptr(up), ld_in, ptr(dgate), ptr(dup),
                                ld_out, ptr(dgate_t), ptr(dup_t), ld_t, rows, cols,
                                dtype_code(gate.dtype), stream_handle(dev)), "zk_swiglu_bwd_t")


# ------------------------------------------------------------------- RoPE --

def rope_(q: torch.Tensor, k: torch.Tensor | None, cos: torch.Tensor, sin: torch.Tensor,
          positions: torch.Tensor | None = None, interleaved: bool = False,
          inverse: bool = False) -> None:
    """Rotate q [B,S,Hq,d] and k [B,S,Hkv,d] in place (unit stride along d).
    cos / sin: fp32 [n_pos, d/2] tables."""
    dev = _require_gpu(q, k, cos, sin, positions)
    if q.dim() != 4 or q.stride(3) != 1:
        raise ValueError("q must be [B,S,H,d] with unit stride along d")
    B, S, Hq, d = q.shape
    if k is not None:
        if k.dim() != 4 or k.stride(3) != 1 or k.shape[0] != B or k.shape[1] != S \
                or k.shape[3] != d or k.dtype != q.dtype:
            raise ValueError("k must be [B,S,Hkv,d] matching q")
        Hkv = k.shape[2]
        ks = k.stride()
    else:
        Hkv, ks = 0, (0, 0, 0, 1)
    if d % 2:
        raise ValueError("head_dim must be even")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != d // 2 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 [n_pos, {d // 2}] table")
    if cos.shape != sin.shape:
        raise ValueError("cos and sin tables differ in shape")
    n_pos = cos.shape[0]
    if positions is not None:
        if positions.dtype != torch.int64 or positions.numel() != S or not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int64 [S] tensor")
    elif n_pos < S:
        raise ValueError(f"table holds {n_pos} positions < S={S}")
    qs = q.stride()
    check(lib().zk_rope(ptr(q), qs[0], qs[1], qs[2], ptr(k), ks[0], ks[1], ks[2], B, S, Hq,
                        Hkv, d, ptr(cos), ptr(sin), n_pos, ptr(positions),
                        _abi.ZK_ROPE_INTERLEAVED if interleaved else _abi.ZK_ROPE_HALF,
                        int(inverse), dtype_code(q.dtype), stream_handle(dev)), "zk_rope")


# -------------------------------------------------------------- Attention --

def _attn_desc(q, k, v, o, scale, causal, window, dq=None, dk=None, dv=None):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, S, H, d]")
    B, Sq, Hq, d = q.shape
    Bk, Skv, Hkv, dk_ = k.shape
    if Bk != B or dk_ != d or v.shape != k.shape:
        raise ValueError(f"shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if Hq % Hkv:
        raise ValueError(f"Hq={Hq} must be a multiple of Hkv={Hkv}")
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o), ("dq", dq), ("dk", dk), ("dv", dv)):
        if t is not None and t.stride(3) != 1:
            raise ValueError(f"{name} must have unit stride along head_dim")
        if t is not None and t.dtype != q.dtype:
            raise ValueError(f"{name} dtype {t.dtype} != q dtype {q.dtype}")
    if (causal or window) and Sq != Skv:
        raise ValueError("causal / windowed attention needs Sq == Skv")
    desc = _abi.AttnDesc()
    desc.B, desc.Sq, desc.Skv, desc.Hq, desc.Hkv, desc.d = B, Sq, Skv, Hq, Hkv, d
    desc.q_sb, desc.q_ss, desc.q_sh = q.stride(0), q.stride(1), q.stride(2)
    desc.k_sb, desc.k_ss, desc.k_sh = k.stride(0), k.stride(1), k.stride(2)
    desc.v_sb, desc.v_ss, desc.v_sh = v.stride(0), v.stride(1), v.stride(2)
    if o is not None:
        desc.o_sb, desc.o_ss, desc.o_sh = o.stride(0), o.stride(1), o.stride(2)
    for pre, t in (("dq", dq), ("dk", dk), ("dv", dv)):
        if t is not None:
            setattr(desc, pre + "_sb", t.stride(0))
            setattr(desc, pre + "_ss", t.stride(1))
            setattr(desc, pre + "_sh", t.stride(2))
    desc.scale = float(scale)
    desc.causal = int(bool(causal))
    desc.window = int(window or 0)
    desc.dtype = dtype_code(q.dtype)
    return desc


def attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = True,
             window: int = 0, scale: float | None = None, out: torch.Tensor | None = None,
             out_t: torch.Tensor | None = None):
    """Flash attention forward on [B,S,H,d] views.  Returns (o, lse) with o
    [B,Sq,Hq,d] (contiguous unless ``out`` is given) and lse fp32 [B,Hq,Sq].

    ``out_t`` (2-byte types, Sq % 8 == 0): a [Hq d, >= B Sq] buffer with unit
    column stride that also receives O transposed (row head * d + i, column
    batch * Sq + position), from the kernel's epilogue -- the operand of the
    o_proj weight gradient."""
    dev = _require_gpu(q, k, v, out, out_t)
    B, Sq, Hq, d = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty(B, Sq, Hq, d, device=dev, dtype=q.dtype)
    elif out.shape != (B, Sq, Hq, d):
        raise ValueError("out has the wrong shape")
    desc = _attn_desc(q, k, v, out, scale, causal, window)
    lse = torch.empty(B, Hq, Sq, device=dev, dtype=torch.float32)
    if out_t is None:
        check(lib().zk_attn_fwd(desc, ptr(q), ptr(k), ptr(v), ptr(out), ptr(lse),
                                stream_handle(dev)), "zk_attn_fwd")
        return out, lse
    if out_t.dtype != q.dtype or out_t.dim() != 2 or out_t.stride(1) != 1:
        raise ValueError("out_t must be a 2-D q-dtype buffer with unit column stride")
    if out_t.shape[0] != Hq * d or out_t.shape[1] < B * Sq:
        raise ValueError(f"out_t must be [{Hq * d}, >= {B * Sq}], got {tuple(out_t.shape)}")
    check(lib().zk_attn_fwd_t(desc, ptr(q), ptr(k), ptr(v), ptr(out), ptr(lse), ptr(out_t),
                              out_t.stride(0), stream_handle(dev)), "zk_attn_fwd_t")
    return out, lse


def attn_bwd(q, k, v, o, do, lse, *, causal: bool = True, window: int = 0,
             scale: float | None = None, dq=None, dk=None, dv=None, rope=None,
             transposed=None):
    """Flash attention backward.  Returns (dq, dk, dv); outputs may be given
    as (strided) views, e.g. slices of one fused [T, (Hq+2Hkv) d] buffer.

    ``rope`` = (cos, sin, positions, interleaved): q and k were rotated by
    RoPE with these tables (as ``rope_``); dq and dk are then returned
    through the transpose rotation, i.e. with respect to the un-rotated
    q / k -- the inverse rope_ pass fused into the kernels.

    ``transposed`` = (dq_t, dk_t, dv_t): 2-D [H d, B S] buffers (rows
    contiguous, one common row stride, a multiple of 8; 2-byte dtypes, S a
    multiple of 8) that also receive dq / dk / dv transposed -- the operand
    layout of the projections' weight-gradient GEMMs -- from the kernels'
    epilogues."""
    dev = _require_gpu(q, k, v, o, do, lse, dq, dk, dv,
                       *(rope[:3] if rope is not None else ()),
                       *(transposed if transposed is not None else ()))
    d = q.shape[3]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if do.shape != o.shape or do.stride() != o.stride():
        raise ValueError("dO must have the same shape and strides as O")
    if lse.dtype != torch.float32 or lse.shape != (q.shape[0], q.shape[2], q.shape[1]) \
            or not lse.is_contiguous():
        raise ValueError("lse must be contiguous fp32 [B, Hq, Sq]")
    dq = torch.empty_like(q, memory_format=torch.contiguous_format) if dq is None else dq
    dk = torch.empty_like(k, memory_format=torch.contiguous_format) if dk is None else dk
    dv = torch.empty_like(v, memory_format=torch.contiguous_format) if dv is None else dv
    if dq.shape != q.shape or dk.shape != k.shape or dv.shape != v.shape:
        raise ValueError("gradient buffers have the wrong shape")
    desc = _attn_desc(q, k, v, o, scale, causal, window, dq, dk, dv)
    nbytes = lib().zk_attn_bwd_workspace(desc)
    ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    if transposed is not None:
        ld_t = _check_transposed(transposed, q, k)
    if rope is None:
        if transposed is not None:
            dq_t, dk_t, dv_t = transposed
            check(lib().zk_attn_bwd_rope_t(desc, ptr(q), ptr(k), ptr(v), ptr(o), ptr(do),
                                           ptr(lse), ptr(dq), ptr(dk), ptr(dv), ptr(ws), nbytes,
                                           None, None, 0, None, 0, ptr(dq_t), ptr(dk_t),
                                           ptr(dv_t), ld_t, stream_handle(dev)),
                  "zk_attn_bwd_rope_t")
            return dq, dk, dv
        check(lib().zk_attn_bwd(desc, ptr(q), ptr(k), ptr(v), ptr(o), ptr(do), ptr(lse),
                                ptr(dq), ptr(dk), ptr(dv), ptr(ws), nbytes,
                                stream_handle(dev)), "zk_attn_bwd")
        return dq, dk, dv
    cos, sin, positions, interleaved = rope
    d, S = q.shape[3], q.shape[1]
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != d // 2 or \
                not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 [n_pos, {d // 2}] table")
    if cos.shape != sin.shape:
        raise ValueError("cos and sin tables differ in shape")
    if positions is not None:
        if positions.dtype != torch.int64 or positions.numel() != S or \
                not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int64 [S] tensor")
    elif cos.shape[0] < S:
        raise ValueError(f"table holds {cos.shape[0]} positions < S={S}")
    pairing = _abi.ZK_ROPE_INTERLEAVED if interleaved else _abi.ZK_ROPE_HALF
    if transposed is not None:
        dq_t, dk_t, dv_t = transposed
        check(lib().zk_attn_bwd_rope_t(desc, ptr(q), ptr(k), ptr(v), ptr(o), ptr(do), ptr(lse),
                                       ptr(dq), ptr(dk), ptr(dv), ptr(ws), nbytes, ptr(cos),
                                       ptr(sin), cos.shape[0], ptr(positions), pairing,
                                       ptr(dq_t), ptr(dk_t), ptr(dv_t), ld_t,
                                       stream_handle(dev)), "zk_attn_bwd_rope_t")
        return dq, dk, dv
    check(lib().zk_attn_bwd_rope(desc, ptr(q), ptr(k), ptr(v), ptr(o), ptr(do), ptr(lse),
                                 ptr(dq), ptr(dk), ptr(dv), ptr(ws), nbytes, ptr(cos), ptr(sin),
                                 cos.shape[0], ptr(positions), pairing,
                                 stream_handle(dev)), "zk_attn_bwd_rope")
    return dq, dk, dv


def _check_transposed(transposed, q, k):
    """Validates attn_bwd's transposed outputs; returns their row stride."""
    if len(transposed) != 3:
        raise ValueError("transposed must be (dq_t, dk_t, dv_t)")
    B, Sq, Hq, d = q.shape
    Skv, Hkv = k.shape[1], k.shape[2]
    want = ((Hq * d, B * Sq), (Hkv * d, B * Skv), (Hkv * d, B * Skv))
    ld = transposed[0].stride(0) if transposed[0].dim() == 2 else -1
    for name, t, shape in zip(("dq_t", "dk_t", "dv_t"), transposed, want):
        if t.dim() != 2 or tuple(t.shape) != shape:
            raise ValueError(f"{name} must be [{shape[0]}, {shape[1]}]")
        if t.dtype != q.dtype or q.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"{name} must be bf16 / fp16 like q")
        if t.stride(1) != 1 or t.stride(0) != ld or ld % 8 != 0 or t.data_ptr() % 16 != 0:
            raise ValueError("transposed outputs need unit column stride, one common row "
                             "stride that is a multiple of 8, and 16-byte alignment")
    if Sq % 8 != 0 or Skv % 8 != 0:
        raise ValueError("transposed outputs need sequence lengths that are multiples of 8")
    return ld


# ------------------------------------------------------------------ AdamW --

def adamw_step(param: torch.Tensor, grad: torch.Tensor, exp_avg: torch.Tensor,
               exp_avg_sq: torch.Tensor, *, lr: float, beta1: float, beta2: float,
               eps: float, weight_decay: float, step: int,
               lowp_out: torch.Tensor | None = None) -> None:
    """One fused AdamW update of a flat fp32 shard (in place)."""
    dev = _require_gpu(param, grad, exp_avg, exp_avg_sq, lowp_out)
    n = param.numel()
    for name, t in (("param", param), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != n:
            raise ValueError(f"{name} must be contiguous fp32 with {n} elements")
    if grad.numel() != n or not grad.is_contiguous():
        raise ValueError("grad must be contiguous with the same number of elements")
    if lowp_out is not None and (lowp_out.numel() != n or not lowp_out.is_contiguous()):
        raise ValueError("lowp_out must be contiguous with the same number of elements")
    check(lib().zk_adamw_step(ptr(param), ptr(grad), dtype_code(grad.dtype), ptr(exp_avg),
                              ptr(exp_avg_sq), ptr(lowp_out),
                              dtype_code(lowp_out.dtype) if lowp_out is not None else 0,
                              n, float(lr), float(beta1), float(beta2), float(eps),
                              float(weight_decay), int(step), stream_handle(dev)),
          "zk_adamw_step")


def adamw_step_t(param: torch.Tensor, grad: torch.Tensor, exp_avg: torch.Tensor,
                 exp_avg_sq: torch.Tensor, lowp_out: torch.Tensor, regions, *, lr: float,
                 beta1: float, beta2: float, eps: float, weight_decay: float,
                 step: int) -> None:
    """adamw_step over the regions of a flat shard, in one launch.  ``regions``:
    up to 8 ``(offset, rows, cols, lowp_t)`` in increasing offset order -- a
    row-major [rows, cols] matrix at ``offset`` whose rounded update also goes,
    transposed, into ``lowp_t`` ([cols, rows], unit column stride, lowp_out's
    dtype) unless it is None.  Elements outside every region are left alone."""
    import ctypes
    from ._abi import AdamwRegion
    dev = _require_gpu(param, grad, exp_avg, exp_avg_sq, lowp_out)
    n = param.numel()
    for name, t in (("param", param), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != n:
            raise ValueError(f"{name} must be contiguous fp32 with {n} elements")
    for name, t in (("grad", grad), ("lowp_out", lowp_out)):
        if t.numel() != n or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous with {n} elements")
    arr = (AdamwRegion * max(1, len(regions)))()
    for i, (off, rows, cols, lt) in enumerate(regions):
        if off < 0 or off + rows * cols > n:
            raise ValueError("region outside the shard")
        if lt is not None:
            _require_gpu(lt)
            if lt.shape != (cols, rows) or lt.stride(1) != 1 or lt.dtype != lowp_out.dtype:
                raise ValueError("lowp_t must be [cols, rows] with unit column stride")
        arr[i] = AdamwRegion(off, rows, cols, lt.stride(0) if lt is not None else 0,
                             ptr(lt) if lt is not None else None)
    check(lib().zk_adamw_step_t(ptr(param), ptr(grad), dtype_code(grad.dtype), ptr(exp_avg),
                                ptr(exp_avg_sq), ptr(lowp_out), dtype_code(lowp_out.dtype),
                                ctypes.cast(arr, ctypes.c_void_p), len(regions), n, float(lr),
                                float(beta1), float(beta2), float(eps), float(weight_decay),
                                int(step), stream_handle(dev)), "zk_adamw_step_t")


def cast_(src: torch.Tensor, dst: torch.Tensor, accumulate: bool = False) -> torch.Tensor:
    """dst = round(src) (or dst = round(dst + src)); contiguous, same numel."""
    dev = _require_gpu(src, dst)
    if src.numel() != dst.numel() or not src.is_contiguous() or not dst.is_contiguous():
        raise ValueError("cast_ needs contiguous tensors of equal size")
    check(lib().zk_cast(ptr(src), dtype_code(src.dtype), ptr(dst), dtype_code(dst.dtype),
                        src.numel(), int(accumulate), stream_handle(dev)), "zk_cast")
    return dst


def transpose(src: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out = src^T for a 2-D tensor with unit column stride; ``out`` (rows
    with unit stride, shape (cols, rows)) may be supplied."""
    dev = _require_gpu(src, out)
    if src.dim() != 2 or src.stride(1) != 1:
        raise ValueError("transpose needs a 2-D tensor with unit column stride")
    rows, cols = src.shape
    if out is None:
        out = torch.empty(cols, rows, device=dev, dtype=src.dtype)
    if out.shape != (cols, rows) or out.dtype != src.dtype or out.stride(1) != 1:
        raise ValueError("out must be (cols, rows) of the same dtype with unit column stride")
    check(lib().zk_transpose(ptr(src), src.stride(0), ptr(out), out.stride(0), rows, cols,
                             dtype_code(src.dtype), stream_handle(dev)), "zk_transpose")
    return out


def _host_copy_check(name, host, devt):
    if host.device.type != "cpu" or not host.is_pinned():
        raise ValueError(f"{name}: the host tensor must be pinned")
    _require_contig("host tensor", host)
    _require_contig("device tensor", devt)
    nbytes = devt.numel() * devt.element_size()
    if host.numel() * host.element_size() != nbytes:
        raise ValueError(f"{name}: the tensors hold different numbers of bytes")
    return nbytes


def copy_to_host(dst: torch.Tensor, src: torch.Tensor, blocks: int = 16) -> torch.Tensor:
    """dst (pinned host tensor) <- src (device tensor), both contiguous with
    the same number of bytes, on the current stream from at most ``blocks``
    workgroups."""
    dev = _require_gpu(src)
    nbytes = _host_copy_check("copy_to_host", dst, src)
    check(lib().zk_copy_to_host(ptr(dst), ptr(src), nbytes, blocks, stream_handle(dev)),
          "zk_copy_to_host")
    return dst


def copy_from_host(dst: torch.Tensor, src: torch.Tensor, blocks: int = 16) -> torch.Tensor:
    """dst (device tensor) <- src (pinned host tensor), as copy_to_host."""
    dev = _require_gpu(dst)
    nbytes = _host_copy_check("copy_from_host", src, dst)
    check(lib().zk_copy_from_host(ptr(dst), ptr(src), nbytes, blocks, stream_handle(dev)),
          "zk_copy_from_host")
    return dst


def device_info(device: int = 0) -> dict:
    import ctypes
    arch = ctypes.create_string_buffer(64)
    cus, clk, mem = ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
    check(lib().zk_device_info(device, arch, 64, ctypes.byref(cus), ctypes.byref(clk),
                               ctypes.byref(mem)), "zk_device_info")
    return {"arch": arch.value.decode(), "num_cus": cus.value,
            "max_clock_khz": clk.value, "hbm_bytes": mem.value}
