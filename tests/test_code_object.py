"""CPU: a check on the built gfx950 code of libgdn.so.

A buffer store of more than 8 bytes whose scalar offset is a register gets no wait states from the
compiler before the VALU rewrites the store's data registers (the compiler treats that store-data
hazard as absent when the offset is a register). On gfx950, a 16-byte state store of this kind was
followed directly by a VALU write of its data registers. The last lanes of a 16-lane row then
stored the rewritten values: a few rows of one state per run, which varied from run to run. The
kernels avoid the form by keeping the scalar offset of every wide store at the constant 0 (row
steps go into the lane offset). This test disassembles the library's own code objects and fails if
the form comes back.
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

from sorernn_amd import _lib

OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
WIDE_STORE_REG_SOFFSET = re.compile(r"buffer_store_dwordx[34]\s+\S+,\s*\S+,\s*s\[\d+:\d+\],\s*s\d+\b")


def _disassembly() -> str:
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libgdn.so is not built")
    if not os.path.exists(OBJDUMP):
        pytest.skip("llvm-objdump not found")
    out = []
    with tempfile.TemporaryDirectory() as d:
        lib = os.path.join(d, "libgdn.so")
        shutil.copy(_lib.LIB_PATH, lib)
        subprocess.run([OBJDUMP, "--offloading", lib], cwd=d, check=True, capture_output=True)
        objs = sorted(f for f in os.listdir(d) if f.endswith("gfx950"))
        assert objs, "no gfx950 code object in libgdn.so"
        for f in objs:
            res = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", os.path.join(d, f)], check=True,
                                 capture_output=True, text=True)
            out.append(res.stdout)
    return "\n".join(out)


def test_no_wide_buffer_store_with_a_register_scalar_offset():
    asm = _disassembly()
    assert "buffer_store_dwordx4" in asm, "expected the kernels' 16-byte buffer stores in the disassembly"
    bad = [ln.strip() for ln in asm.splitlines() if WIDE_STORE_REG_SOFFSET.search(ln)]
    assert not bad, f"{len(bad)} wide buffer stores with a register scalar offset, e.g. {bad[:3]}"
