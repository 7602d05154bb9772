"""The allocation-free RMSNorm backward, zk_rmsnorm_bwd_noalloc.

It keeps the dw partial rows in the library's static per-device scratch
array instead of a caller-supplied workspace; its results must be identical
to zk_rmsnorm_bwd's (same kernels, deterministic reduction).  Both entry
points are called through the C ABI directly (ctypes), several times in a
row with shrinking inputs, so a stale partial row from an earlier call would
show.
"""
import ctypes

import pytest
import torch

from zorse_amd import _abi


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def test_noalloc_rejects_sizes_beyond_the_scratch():
    """A shape whose dw partial rows exceed the static array is refused on the
    host with ZK_EWORKSPACE before anything is launched (no GPU needed)."""
    lib = _abi.lib()
    p = ctypes.c_void_p(256)
    # 1024 rows -> 512 partial rows of 16384 floats: 8 Mi floats > 4 Mi
    rc = lib.zk_rmsnorm_bwd_noalloc(p, p, p, p, None, p, p, 0, 1024, 16384, _abi.ZK_BF16,
                                    _abi.ZK_BF16, None)
    assert rc == -5, rc
    assert b"scratch" in lib.zk_last_error()
    # the bad-argument checks come first, as in zk_rmsnorm_bwd
    assert lib.zk_rmsnorm_bwd_noalloc(None, p, p, p, None, p, p, 0, 4, 8, 2, 2, None) == -1
    assert lib.zk_rmsnorm_bwd_noalloc(p, p, p, p, None, p, p, 0, 4, 8, 9, 2, None) == -2


CASES = [
    # rows, hidden, activation dtype, weight dtype, residual gradient, accumulate dw
    (4096, 4096, torch.bfloat16, torch.bfloat16, True, False),   # the 7B layer's shape
    (1000, 2048, torch.float16, torch.float32, False, True),      # smaller, fp32 weight
    (3, 100, torch.bfloat16, torch.bfloat16, True, False),        # scalar kernels
]


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(dev):
    lib = _abi.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    for rows, hidden, adt, wdt, with_res, acc in CASES:
        print(f"rmsnorm_bwd_noalloc rows={rows} hidden={hidden} {adt} w={wdt}", flush=True)
        g = torch.Generator().manual_seed(rows + hidden)
        dy = torch.randn(rows, hidden, generator=g).to(adt).to(dev)
        h = torch.randn(rows, hidden, generator=g).to(adt).to(dev)
        w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(wdt).to(dev)
        rstd = torch.rand(rows, generator=g).add_(0.5).to(dev)
        dres = torch.randn(rows, hidden, generator=g).to(adt).to(dev) if with_res else None
        dw0 = torch.randn(hidden, generator=g).to(wdt).to(dev)
        outs = []
        for noalloc in (False, True):
            dx = torch.full_like(h, float("nan"))
            dw = dw0.clone()
            if noalloc:
                rc = lib.zk_rmsnorm_bwd_noalloc(
                    _ptr(dy), _ptr(h), _ptr(w), _ptr(rstd), _ptr(dres), _ptr(dx), _ptr(dw),
                    int(acc), rows, hidden, _abi.dtype_code(adt), _abi.dtype_code(wdt), stream)
            else:
                n = lib.zk_rmsnorm_bwd_workspace(rows, hidden)
                ws = torch.empty(max(n, 1), device=dev, dtype=torch.float32)
                rc = lib.zk_rmsnorm_bwd(
                    _ptr(dy), _ptr(h), _ptr(w), _ptr(rstd), _ptr(dres), _ptr(dx), _ptr(dw),
                    int(acc), _ptr(ws), ws.numel(), rows, hidden, _abi.dtype_code(adt),
                    _abi.dtype_code(wdt), stream)
            assert rc == 0, lib.zk_last_error()
            torch.cuda.synchronize()
            outs.append((dx, dw))
        (dx_ws, dw_ws), (dx_na, dw_na) = outs
        assert torch.isfinite(dx_na).all()
        assert torch.equal(dx_na, dx_ws), (rows, hidden)
        assert torch.equal(dw_na, dw_ws), (rows, hidden)


@pytest.mark.gpu
def test_noalloc_under_graph_capture(dev):
    """The allocation-free entry point inside a captured HIP graph (what it
    exists for): after one eager call on the device (which resolves the
    scratch address), a call captured with torch.cuda.graph is replayed three
    times, the inputs refilled in place by eager work between replays; every
    replay's dx and dw equal the workspace entry point's eager result on the
    same inputs, bit for bit."""
    lib = _abi.lib()
    rows, hidden, adt = 4096, 4096, torch.bfloat16
    code = _abi.dtype_code(adt)
    dy = torch.empty(rows, hidden, device=dev, dtype=adt)
    h = torch.empty_like(dy)
    dres = torch.empty_like(dy)
    w = torch.empty(hidden, device=dev, dtype=adt)
    rstd = torch.empty(rows, device=dev)
    dx = torch.empty_like(dy)
    dw = torch.empty(hidden, device=dev, dtype=adt)

    def fill(seed):
        g = torch.Generator().manual_seed(seed)
        dy.copy_(torch.randn(rows, hidden, generator=g))
        h.copy_(torch.randn(rows, hidden, generator=g))
        dres.copy_(torch.randn(rows, hidden, generator=g))
        w.copy_(1 + 0.1 * torch.randn(hidden, generator=g))
        rstd.copy_(torch.rand(rows, generator=g) + 0.5)

    def call_noalloc():
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        rc = lib.zk_rmsnorm_bwd_noalloc(_ptr(dy), _ptr(h), _ptr(w), _ptr(rstd), _ptr(dres),
                                        _ptr(dx), _ptr(dw), 0, rows, hidden, code, code, stream)
        assert rc == 0, lib.zk_last_error()

    def reference():
        rdx, rdw = torch.empty_like(dx), torch.empty_like(dw)
        n = lib.zk_rmsnorm_bwd_workspace(rows, hidden)
        ws = torch.empty(n, device=dev, dtype=torch.float32)
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        rc = lib.zk_rmsnorm_bwd(_ptr(dy), _ptr(h), _ptr(w), _ptr(rstd), _ptr(dres), _ptr(rdx),
                                _ptr(rdw), 0, _ptr(ws), n, rows, hidden, code, code, stream)
        assert rc == 0, lib.zk_last_error()
        torch.cuda.synchronize()
        return rdx, rdw

    fill(1)
    call_noalloc()                      # eager: resolves the scratch address
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call_noalloc()
    torch.cuda.synchronize()
    for seed in (2, 3, 4):
        print(f"rmsnorm_bwd_noalloc graph replay, inputs seed {seed}", flush=True)
        fill(seed)
        dx.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got_dx, got_dw = dx.clone(), dw.clone()
        rdx, rdw = reference()
        assert torch.equal(got_dx, rdx), seed
        assert torch.equal(got_dw, rdw), seed
