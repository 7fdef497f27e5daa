"""Workspace growth keeps the amax slot: the first quantize+compress of a
process (small workspace -> grown by the compress) must use the real scale."""
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, %r)
from oracle import oracle as O
from bitsparse_amd.src.functions import quantize_and_compress
from tests.helpers import bits, preact_input
x = preact_input((1024, 2048), seed=5).relu() * 3
q, s, sp = quantize_and_compress(x.cuda(), None)
qo, so = O.to_fp8(bits(x))
assert float(s.item()) == so, (float(s.item()), so)
assert (bits(q) == qo).all()
print("ok")
"""


def test_first_quantize_in_fresh_process(dev):
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", SCRIPT % root], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr[-2000:]


def test_epoch_tagged_entry_points_refuse_graph_capture(dev):
    """bs_compress and bs_amax tag their device state with a per-call epoch;
    a captured graph would replay one epoch and read the previous replay's
    status words / amax as current, so capture is refused with an error
    (nothing is enqueued) and the stream keeps working afterwards."""
    import torch
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src import hip_operators as H
    from bitsparse_amd.src.functions import dense_to_tilesparse
    from tests.helpers import relu_input
    x = relu_input((256, 512), 0.5, seed=90).to(dev)
    buf = TensorBuffer(2 * x.numel(), device=dev)
    ref = dense_to_tilesparse(x, None, buf)            # workspace allocated outside capture
    H.amax_into_workspace(x)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    for fn in (lambda: dense_to_tilesparse(x, None, buf), lambda: H.amax_into_workspace(x)):
        g = torch.cuda.CUDAGraph()
        with pytest.raises(ValueError, match="captured into a HIP graph"):
            with torch.cuda.graph(g, stream=side):
                fn()
    torch.cuda.synchronize()
    buf.reset_buffer()
    again = dense_to_tilesparse(x, None, buf)
    assert torch.equal(again.bitmask, ref.bitmask) and torch.equal(again.prefix, ref.prefix)
    assert torch.equal(again.vals[:x.numel()], ref.vals[:x.numel()])


def test_epoch_wrap_between_amax_and_compress(dev):
    """The workspace epoch wraps (buffer zeroed) only where no amax is
    pending: an amax taken at the last epoch still reaches its compress."""
    import torch
    from bitsparse_amd import _lib
    from bitsparse_amd.fp8 import to_fp8
    from bitsparse_amd.src.functions import dense_to_tilesparse, quantize_and_compress
    from tests.helpers import preact_input
    x = (preact_input((256, 512), seed=7).relu() * 5).to(dev)
    q_ref, s_ref = to_fp8(x)
    sp_ref = dense_to_tilesparse(q_ref, s_ref)
    for start in (_lib._EPOCH_LIMIT - 2, _lib._EPOCH_LIMIT - 1, _lib._EPOCH_LIMIT):
        ws = _lib.workspace_for(x.device)
        ws.epoch = start
        q, s, sp = quantize_and_compress(x, None)
        assert torch.equal(s, s_ref)
        assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8))
        assert torch.equal(sp.bitmask, sp_ref.bitmask) and torch.equal(sp.prefix, sp_ref.prefix)
        assert ws.epoch <= _lib._EPOCH_LIMIT
