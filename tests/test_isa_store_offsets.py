"""CPU check of the gfx950 machine code the library is built from: no
12- or 16-byte buffer store may take its offset from an SGPR.

The compiler separates such a store from a later VALU write of its data
registers by wait states only when the store's SGPR offset field holds the
constant 0. With an SGPR there, a data register reused by the very next
instruction was seen to change the stored dword on MI355X (the warp-
specialised GEMM's 16-byte residual stores, about 1 dword in 3.5 million
wrong from one run to the next). The kernels therefore put the whole
offset of a wide buffer store in its VGPR; this test compiles every HIP
source to assembly with the library's own flags and holds them to that.
"""
import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import tempfile

import pytest

from indecis_amd import build as hip_build

WIDE_BUFFER_STORE = re.compile(r"^\s*buffer_store_dwordx[34]\s+(.*)$")


def _device_asm(src, out):
    cmd = [hip_build.HIPCC, *hip_build.FLAGS, *hip_build.EXTRA.get(src, []), "--cuda-device-only", "-S",
           os.path.join(hip_build.CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out


def sgpr_offset_stores(asm_text):
    """(kernel, instruction) of every wide buffer store whose SGPR-offset
    operand (the fourth) is a register rather than a constant."""
    bad, fn = [], None
    for line in asm_text.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            fn = m.group(1)
            continue
        m = WIDE_BUFFER_STORE.match(line.split(";")[0])
        if not m:
            continue
        ops = [t.strip() for t in m.group(1).split(",")]
        if len(ops) >= 4 and re.match(r"^(s\d+|s\[|ttmp|m0)", ops[3].split()[0]):
            bad.append((fn, line.strip()))
    return bad


def test_rule_catches_an_sgpr_offset():
    asm = ("_Zk:\n\tbuffer_store_dwordx4 v[8:11], v140, s[12:15], s45 offen\n"
           "\tbuffer_store_dwordx4 v[0:3], v4, s[4:7], 0 offen\n\tbuffer_store_dword v1, v2, s[4:7], s9 offen\n")
    assert sgpr_offset_stores(asm) == [("_Zk", "buffer_store_dwordx4 v[8:11], v140, s[12:15], s45 offen")]


@pytest.mark.skipif(not shutil.which(hip_build.HIPCC) and not os.path.exists(hip_build.HIPCC),
                    reason="hipcc not available")
def test_no_wide_buffer_store_takes_an_sgpr_offset():
    sources = [s for s in hip_build.SOURCES if s.endswith(".hip")]
    with tempfile.TemporaryDirectory() as d:
        with cf.ThreadPoolExecutor(4) as ex:
            outs = list(ex.map(lambda s: _device_asm(s, os.path.join(d, s + ".s")), sources))
        bad = []
        for src, out in zip(sources, outs):
            bad += [(src, fn, ins) for fn, ins in sgpr_offset_stores(open(out).read())]
    assert not bad, "\n".join(f"{s}: {fn}: {ins}" for s, fn, ins in bad[:20])
