"""Guard against a register-allocation hazard in the device code (CPU only:
hipcc cross-compiles gfx950 assembly, nothing runs).

At a join block, where a divergent branch ends, the compiler first restores
the exec mask (``s_or_b64 exec, exec, ...``).  A register spill store placed
in that block ahead of the restore runs with only the branch's lanes on, so a
value that every lane holds is saved for some lanes and reloaded as stale
scratch for the others.  The compress kernel once compiled that way (the
mask byte of one chunk spilled under a branch on the wave index) and
produced a wrong bitmask and value stream for wave 0's tile.  The kernels
now keep wave-uniform conditions in scalar registers; this test checks that
no kernel of the library has a spill store in that position.
"""
import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from bitsparse_amd import build as B

LABEL = re.compile(r"^(\.LBB\S+:|; %bb\.\d+:)")
FUNC = re.compile(r"^(_Z\S+):")
EXEC_RESTORE = re.compile(r"^s_(or|mov)_b64 exec, ")
SPILL = re.compile(r"^(scratch_store|buffer_store)\S*\s.*Spill")


def spills_before_exec_restore(asm: str):
    """(function, line, instruction) of every spill store that sits between
    a block label and that block's exec-mask restore."""
    hits, fn, pending, in_head = [], None, [], False
    for i, line in enumerate(asm.splitlines(), 1):
        m = FUNC.match(line)
        if m:
            fn = m.group(1)
        if LABEL.match(line):
            in_head, pending = True, []
            continue
        t = line.strip()
        if not in_head or not t or t.startswith((";", ".")):
            continue
        if SPILL.match(t):
            pending.append((fn, i, t))
            continue
        if EXEC_RESTORE.match(t):
            hits.extend(pending)
        in_head, pending = False, []
    return hits


def test_scanner_finds_the_pattern():
    asm = "\n".join([
        "_Zkernel:",
        "\ts_and_b64 exec, exec, s[22:23]",
        "\ts_cbranch_execz .LBB9_192",
        "\tglobal_store_byte v[10:11], v18, off offset:256",
        ".LBB9_192:",
        "\tscratch_store_dword off, v19, off       ; 4-byte Folded Spill",
        "\ts_or_b64 exec, exec, s[60:61]",
        "\tscratch_store_dword off, v18, off offset:4 ; 4-byte Folded Spill",
    ])
    hits = spills_before_exec_restore(asm)
    assert [h[1] for h in hits] == [6]


@pytest.mark.skipif(shutil.which(B.hipcc()) is None and not os.path.exists(B.hipcc()), reason="no hipcc")
def test_no_spill_runs_under_a_partial_exec_mask(tmp_path):
    flags = [f for f in B.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]

    def asm_of(src):
        out = tmp_path / (src + ".s")
        cmd = ([B.hipcc()] + flags + ["-S", "--cuda-device-only", "-I", B.INCLUDE, "-I", B.CSRC,
               "-o", str(out), os.path.join(B.CSRC, src)])
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-4000:]
        return src, out.read_text()

    with ThreadPoolExecutor(max_workers=min(len(B.SOURCES), 6)) as ex:
        results = list(ex.map(asm_of, B.SOURCES))
    bad = [(src, *h) for src, asm in results for h in spills_before_exec_restore(asm)]
    assert not bad, "spill stores ahead of an exec restore:\n" + "\n".join(map(str, bad[:20]))
