"""The launch-timing hook (bs_launch_timing): kernel durations recorded by
the launches themselves, in launch order, without changing any result."""
import pytest
import torch

from tests.helpers import relu_input

pytestmark = pytest.mark.gpu


def test_launch_timer_records_compress_and_decompress(dev):
    from bitsparse_amd import _lib
    from bitsparse_amd.src.functions import dense_to_tilesparse
    from bitsparse_amd.src.hip_operators import unpack_batch_
    x = relu_input((1000, 3000), 0.5, seed=80).to(dev)
    ref = dense_to_tilesparse(x, None)
    out = torch.empty_like(x)
    with _lib.LaunchTimer() as t:
        sp = dense_to_tilesparse(x, None)            # count pass + values pass
        unpack_batch_(sp, out, 0, sp.grid_n, 3000, 1000, sp.grid_m * sp.grid_n)
        sp2 = dense_to_tilesparse(x, None)
    assert [k for k, _ in t.records] == ["compress", "compress", "decompress", "compress", "compress"]
    assert all(0.0 < ms < 1000.0 for _, ms in t.records)
    assert torch.equal(out, x)
    for s in (sp, sp2):
        assert torch.equal(s.bitmask, ref.bitmask) and torch.equal(s.prefix, ref.prefix)
        assert torch.equal(s.vals, ref.vals)
    # off again: nothing recorded
    with _lib.LaunchTimer() as t2:
        pass
    assert t2.records == []
    dense_to_tilesparse(x, None)
    n = __import__("ctypes").c_int(-1)
    assert _lib.load().bs_launch_timing_read(None, None, 0, __import__("ctypes").byref(n)) == 0
    assert n.value == 0
