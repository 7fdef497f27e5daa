"""bs_compress_noalloc (the compress entry point that allocates nothing: its
scratch is a library-owned device array) against bs_compress / bs_compress_relu
with a caller workspace, called through the C ABI on the same inputs.

Bar: bit-exact (bitmask, prefix, values, cursor outputs, scale, quantized and
relu'd dense copies), on two calls in a row with the second input smaller, so
the state the first call leaves in the shared array cannot leak into the
second."""
import ctypes

import pytest
import torch

from tests.helpers import preact_input

pytestmark = pytest.mark.gpu


def _L():
    from bitsparse_amd import _lib
    return _lib.load()


def _p(t):
    return None if t is None else t.data_ptr()


def _outs(dev, M, N, cap, vdt, quant):
    T = ((M + 63) // 64) * ((N + 63) // 64)
    return dict(bitmask=torch.full((T * 512,), 0xAB, dtype=torch.uint8, device=dev),
                prefix=torch.full((T + 1,), 7, dtype=torch.int32, device=dev),
                vals=torch.zeros(cap, dtype=vdt, device=dev),
                off_out=torch.full((1,), -5, dtype=torch.int64, device=dev),
                start_out=torch.full((1,), -5, dtype=torch.int64, device=dev),
                err=torch.zeros(1, dtype=torch.int32, device=dev),
                scale=torch.zeros((), dtype=torch.float32, device=dev),
                q=torch.zeros((M, N), dtype=torch.uint8, device=dev) if quant else None)


def _run_existing(z, quant, relu, off_in, o, relu_out):
    """bs_compress / bs_compress_relu with a workspace (the existing path)."""
    from bitsparse_amd import _lib
    from bitsparse_amd.src import hip_operators as H
    L = _L()
    M, N = z.shape
    st = torch.cuda.current_stream(z.device).cuda_stream
    ws = _lib.workspace_for(z.device)
    epoch_amax = 0
    if quant:
        epoch_amax = H.amax_into_workspace(z, relu=relu)
    ws.ensure(L.bs_compress_workspace_bytes(M, N))
    epoch = ws.next_epoch()
    args = (z.data_ptr(), 0, M, N, int(quant), ws.amax_slot_ptr() if quant else None, epoch_amax,
            _p(o["scale"]), _p(o["q"]), o["bitmask"].data_ptr(), o["prefix"].data_ptr(), o["vals"].data_ptr(),
            o["vals"].numel(), _p(off_in), 0, o["off_out"].data_ptr(), o["start_out"].data_ptr(), 1,
            o["err"].data_ptr(), ws.buf.data_ptr(), ws.nbytes, epoch)
    if relu:
        rc = L.bs_compress_relu(*args, _p(relu_out), st)
    else:
        rc = L.bs_compress(*args, st)
    assert rc == 0, L.bs_last_error()


def _run_noalloc(z, quant, relu, off_in, o, relu_out):
    L = _L()
    M, N = z.shape
    st = torch.cuda.current_stream(z.device).cuda_stream
    rc = L.bs_compress_noalloc(z.data_ptr(), 0, M, N, int(quant), int(relu), _p(o["scale"]), _p(o["q"]),
                               o["bitmask"].data_ptr(), o["prefix"].data_ptr(), o["vals"].data_ptr(),
                               o["vals"].numel(), _p(off_in), 0, o["off_out"].data_ptr(),
                               o["start_out"].data_ptr(), 1, o["err"].data_ptr(), _p(relu_out), st)
    assert rc == 0, L.bs_last_error()


def _same(a, b, quant):
    keys = ["bitmask", "prefix", "off_out", "start_out", "err"] + (["scale", "q"] if quant else [])
    for k in keys:
        assert torch.equal(a[k], b[k]), k
    n = int(a["prefix"][-1].item())
    base = int(a["start_out"].item())
    va, vb = a["vals"].view(torch.uint8), b["vals"].view(torch.uint8)
    eb = a["vals"].element_size()
    assert torch.equal(va[base * eb:(base + n) * eb], vb[base * eb:(base + n) * eb])


@pytest.mark.parametrize("quant,relu", [(False, False), (False, True), (True, True), (True, False)])
def test_noalloc_matches_workspace_compress_twice(dev, quant, relu):
    vdt = torch.float8_e4m3fn if quant else torch.bfloat16
    for (M, N, seed, off) in ((1024, 1536, 1, 5), (200, 130, 2, 3)):     # second call smaller
        z = preact_input((M, N), seed=seed).to(dev)
        if not relu:
            z = z.relu()
        off_in = torch.full((1,), off, dtype=torch.int64, device=dev)
        cap = M * N + off + 64
        a, b = _outs(dev, M, N, cap, vdt, quant), _outs(dev, M, N, cap, vdt, quant)
        za, zb = z.clone(), z.clone()
        _run_existing(za, quant, relu, off_in, a, za if relu else None)
        _run_noalloc(zb, quant, relu, off_in, b, zb if relu else None)
        torch.cuda.synchronize()
        _same(a, b, quant)
        if relu:
            assert torch.equal(za, zb)                  # relu(z) written in place by both


def test_noalloc_refuses_too_many_tiles(dev):
    L = _L()
    max_tiles = L.bs_compress_noalloc_max_tiles()
    assert max_tiles == 1 << 19
    z = torch.zeros((64, 64), dtype=torch.bfloat16, device=dev)
    pre = torch.full((2,), 9, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    # 1 x 64*(max+1) columns: max + 1 tiles; refused before anything is read or launched
    rc = L.bs_compress_noalloc(z.data_ptr(), 0, 1, 64 * (max_tiles + 1), 0, 0, None, None, None,
                               pre.data_ptr(), None, 0, None, 0, None, None, 0, None, None, st)
    assert rc == 1 and b"tiles" in L.bs_last_error()
    torch.cuda.synchronize()
    assert bool((pre == 9).all())


def test_noalloc_under_graph_capture(dev):
    """Captured once, replayed three times with new input values written
    between replays: every replay matches the workspace path on the current
    input (each call clears its scratch state, so replays do not see the
    previous replay's look-back words)."""
    M, N = 512, 640
    z = preact_input((M, N), seed=4).to(dev).relu()
    off_in = torch.zeros((1,), dtype=torch.int64, device=dev)
    cap = M * N + 64
    o = _outs(dev, M, N, cap, torch.bfloat16, False)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _run_noalloc(z, False, False, off_in, o, None)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        _run_noalloc(z, False, False, off_in, o, None)
    for it in range(3):
        z.copy_(preact_input((M, N), seed=10 + it).to(dev).relu())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = _outs(dev, M, N, cap, torch.bfloat16, False)
        _run_existing(z, False, False, off_in, ref, None)
        torch.cuda.synchronize()
        _same(ref, o, False)
