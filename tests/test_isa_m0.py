"""The prefill GEMMs write m0 in inline asm right before each direct-to-LDS
load (bq_gemm.hip: dma16).  The compiler treats m0 as reserved and does not
preserve it around asm, so that is only safe while nothing else in those
kernels uses m0.  This checks the built gfx950 code object of bq_gemm.hip:
every instruction that names m0 is an s_mov_b32 into m0 followed (past
s_nop hazard padding) by global_load_lds_dwordx4, and no instruction that
reads m0 implicitly (message sends, relative register indexing, GWS / addtid /
ordered-count LDS ops, other LDS-direct loads) appears.  Runs on the CPU."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OBJ = os.path.join(ROOT, "bruce-engine_amd", "_build", "bq_gemm.o")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"

IMPLICIT_M0 = re.compile(r"\b(s_sendmsg\w*|s_movrel\w*|v_movrel\w*|ds_gws\w*|ds_ordered_count|\w*_addtid\w*|"
                         r"buffer_load_\w+\s.*\blds\b|s_ttracedata)")


def _disasm(tmp_path):
    if not (os.path.exists(OBJ) and os.path.exists(OBJDUMP)):
        pytest.skip("needs the built bq_gemm.o (bruce-engine_amd/build.py) and llvm-objdump")
    obj = tmp_path / "bq_gemm.o"
    shutil.copy(OBJ, obj)
    subprocess.run([OBJDUMP, "--offloading", str(obj)], check=True, capture_output=True, cwd=tmp_path)
    co = [f for f in os.listdir(tmp_path) if f.endswith("gfx950")]
    assert co, "no gfx950 code object in bq_gemm.o"
    r = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", str(tmp_path / co[0])], check=True, capture_output=True,
                       text=True)
    return r.stdout


def test_m0_only_feeds_direct_to_lds_loads(tmp_path):
    text = _disasm(tmp_path)
    kernel, insts = None, []
    for line in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.*)>:$", line)
        if m:
            kernel = m.group(1)
            continue
        ins = line.split("//")[0].strip()
        if ins and kernel:
            insts.append((kernel, ins))
    mmq = [(k, i) for k, i in insts if "k_mmq" in k]
    assert mmq, "no prefill GEMM kernels found"
    writes = 0
    for j, (k, ins) in enumerate(mmq):
        assert not IMPLICIT_M0.search(ins), (k, ins)
        if re.search(r"\bm0\b", ins):
            assert ins.startswith("s_mov_b32 m0,"), (k, ins)
            n = j + 1
            while mmq[n][1].startswith("s_nop"):
                n += 1
            assert mmq[n][1].startswith("global_load_lds_dwordx4"), (k, ins, mmq[n][1])
            writes += 1
        if ins.startswith("global_load_lds"):
            p = j - 1
            while mmq[p][1].startswith("s_nop"):
                p -= 1
            assert mmq[p][1].startswith("s_mov_b32 m0,"), (k, ins, mmq[p][1])
    assert writes > 0
