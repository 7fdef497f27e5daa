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
