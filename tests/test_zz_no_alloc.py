"""The allocation-free transposed dequant-GEMM (lrq_dequant_gemm_t_noalloc, include/lrq.h).

It runs the same kernels as lrq_dequant_gemm_t with the library's own device scratch in place
of the caller's workspace, so its results must equal that entry point's bit for bit (same
plan, same summation order).  Two calls in a row, the second with a smaller input, check that
the scratch kept from the first call does not leak into the second.  Called through the C ABI.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib(pkg):
    return pkg._lib


def _with_workspace(L, c, g, n, out_f32):
    t = c.descriptor()
    wsb = L.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(t), n)
    assert wsb >= 0
    ws = torch.empty(((max(wsb, 16) + 15) // 16) * 4, dtype=torch.float32, device=g.device)
    out = torch.empty((c.hidden, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=g.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(g.device).cuda_stream)
    st = L.call_raw("lrq_dequant_gemm_t", ctypes.byref(t), ctypes.c_void_p(g.data_ptr()), n, n,
                    ctypes.c_void_p(out.data_ptr()), n, 1 if out_f32 else 0, ctypes.c_void_p(ws.data_ptr()),
                    ws.numel() * 4, stream)
    assert st == 0, L.status_string(st)
    return out, wsb


def _no_alloc(L, c, g, n, out_f32):
    t = c.descriptor()
    out = torch.full((c.hidden, n), float("nan"), dtype=torch.float32 if out_f32 else torch.bfloat16,
                     device=g.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(g.device).cuda_stream)
    st = L.call_raw("lrq_dequant_gemm_t_noalloc", ctypes.byref(t), ctypes.c_void_p(g.data_ptr()), n, n,
                    ctypes.c_void_p(out.data_ptr()), n, 1 if out_f32 else 0, stream)
    assert st == 0, L.status_string(st)
    return out


def _case(pkg, dev, rows, hidden, rank, bits, group, n, seed):
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=seed).to(dev)
    V = pkg.inputs.basis(hidden, rank, seed=seed).to(dev) if rank else None
    c = pkg.encode(x, V, bits=bits, group_size=group)
    g = pkg.inputs.gradient((rows, n), 0.05, seed=seed).to(dev)
    return c, g


@pytest.mark.parametrize("out_f32", [True, False])
def test_noalloc_matches_workspace_entry_point_twice(pkg, dev, out_f32):
    L = _lib(pkg)
    big = _case(pkg, dev, 16384, 4096, 16, 4, 64, 16, seed=31)   # north-star format, 16 row groups
    small = _case(pkg, dev, 1000, 2048, 16, 4, 64, 32, seed=32)  # smaller input, n = 32
    print(f"[noalloc] out_f32={out_f32} big then small", flush=True)
    ref_big, ws_big = _with_workspace(L, *big, 16, out_f32)
    ref_small, ws_small = _with_workspace(L, *small, 32, out_f32)
    assert 0 < ws_small < ws_big <= L.LRQ_GEMM_T_SCRATCH_BYTES
    got_big = _no_alloc(L, *big, 16, out_f32)
    got_small = _no_alloc(L, *small, 32, out_f32)
    torch.cuda.synchronize()
    assert torch.equal(got_big.view(torch.int16 if not out_f32 else torch.int32),
                       ref_big.view(torch.int16 if not out_f32 else torch.int32))
    assert torch.equal(got_small.view(torch.int16 if not out_f32 else torch.int32),
                       ref_small.view(torch.int16 if not out_f32 else torch.int32))
    # the Python wrapper over the same entry point
    out = torch.empty_like(ref_small)
    pkg.dequant_gemm_t_noalloc(small[0], small[1], out)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_small)


def test_noalloc_rejects_a_workspace_beyond_the_scratch(pkg):
    """Host-side check before any HIP call: a plan whose partials exceed the scratch is refused."""
    L = _lib(pkg)
    t = L.LrqTensors()
    t.rows, t.hidden, t.rank, t.bits, t.group = 16, 262144, 0, 4, 64
    t.codes, t.ld_codes = 0x100000, 262144 // 2
    t.qparams, t.ld_qp = 0x200000, 2 * 262144 // 64
    assert L.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(t), 32) > L.LRQ_GEMM_T_SCRATCH_BYTES
    p = ctypes.c_void_p(0x400000)
    assert L.call_raw("lrq_dequant_gemm_t_noalloc", ctypes.byref(t), p, 32, 32, p, 32, 1, None) == L.LRQ_ERR_WORKSPACE


def test_noalloc_replays_from_a_captured_graph(pkg, dev):
    """The entry point launches kernels only (no allocation, no memset), so a call captured in a
    HIP graph replays correctly: three replays, each after eager calls that reuse the scratch
    with another input and a synchronisation, each bit-identical to the workspace entry point.
    The first call on the device (the scratch address lookup) runs eagerly before the capture."""
    L = _lib(pkg)
    c, g = _case(pkg, dev, 4096, 4096, 16, 4, 64, 16, seed=33)
    other = _case(pkg, dev, 3000, 2048, 16, 4, 64, 32, seed=34)
    ref, _ = _with_workspace(L, c, g, 16, True)
    ref_other, _ = _with_workspace(L, *other, 32, True)
    _no_alloc(L, c, g, 16, True)
    torch.cuda.synchronize()
    out = torch.full((c.hidden, 16), float("nan"), dtype=torch.float32, device=dev)
    t = c.descriptor()
    graph = torch.cuda.CUDAGraph()
    print("[noalloc] capture", flush=True)
    with torch.cuda.graph(graph):
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        st = L.call_raw("lrq_dequant_gemm_t_noalloc", ctypes.byref(t), ctypes.c_void_p(g.data_ptr()), 16, 16,
                        ctypes.c_void_p(out.data_ptr()), 16, 1, stream)
    assert st == 0, L.status_string(st)
    for i in range(3):
        got_other = _no_alloc(L, *other, 32, True)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        print(f"[noalloc] replay {i}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"replay {i}"
        assert torch.equal(got_other.view(torch.int32), ref_other.view(torch.int32))
