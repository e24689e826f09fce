"""The decode step's host logic on the CPU: bq_decode.hip built for the host
alone and linked against recorders of every entry point it calls
(tests/host/decode_mock.cpp).  For the two-layer model of the GPU decode tests
(a Q6_K v part in the QKV, norm_before on the first block, norm_after on the
last) and every fold mode and block count, each pointer a call receives must
lie inside a buffer with room for what that call touches, no fused call may
write a row that its workgroups also read, and the 4-block step issues the
expected number of launches: 20 (fold 0; the last block's resid and the
loop-end norm are one launch), 16 (fold 1: the gate norm in O, the silu*mul in
the gate+up epilogue, its norm in down) and 14 (fold 2: also the FFN block's
residual update and the first block's loop-start norm in the QKV GEMV).  The 8-row verify step and
a 40-row prompt chunk (prefill GEMMs with and without the step's xdh and
workspace, the last row's logits) are checked the same way, and a workspace
size without a workspace or rows above BQ_MAX_STEP_ROWS are refused."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _hipcc():
    for p in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if p and os.path.exists(p):
            return p
    return None


def test_decode_call_sequence(tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not found")
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "bruce-engine_amd", "csrc")]
    flags = ["--offload-host-only", "-std=c++17", "-O1"]
    dec, mock, exe = tmp_path / "dec.o", tmp_path / "mock.o", tmp_path / "mock"
    subprocess.run([hipcc, *flags, *inc, "-c", os.path.join(ROOT, "bruce-engine_amd", "csrc", "bq_decode.hip"),
                    "-o", str(dec)], check=True, capture_output=True)
    subprocess.run([hipcc, *flags, *inc, "-c", os.path.join(ROOT, "tests", "host", "decode_mock.cpp"),
                    "-o", str(mock)], check=True, capture_output=True)
    subprocess.run([hipcc, str(dec), str(mock), "-o", str(exe)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60).stdout
    runs = {(int(f), int(b)): (int(c), int(bad), int(sc))
            for f, b, c, bad, sc in re.findall(r"fold (\d) blocks (\d) calls (\d+) bad (\d+) scaled (\d+)", out)}
    assert len(runs) == 12, out
    assert all(r[1] == 0 for r in runs.values()), out
    # fold >= 1: each attention block's QKV launch writes the scaled gate row
    # into ffn_u (blocks 0 and 2), once the step has an FFN block to size ffn_u by
    want = lambda f, nb: 0 if f == 0 or nb == 1 else (nb + 1) // 2
    assert all(runs[(f, nb)][2] == want(f, nb) for f in range(3) for nb in range(1, 5)), runs
    assert runs[(0, 4)][0] == 20 and runs[(1, 4)][0] == 16 and runs[(2, 4)][0] == 14, runs
    # the verify step and a 40-row prompt chunk: the same 20 launches (one
    # prefill GEMM launch per fused GEMV, the last row's logits)
    rows = re.findall(r"rows (\d+) scratch (\d) calls (\d+) bad (\d+)", out)
    assert [(int(r), int(c), int(b)) for r, _, c, b in rows] == [(8, 20, 0), (40, 20, 0), (40, 20, 0)], out
    assert "bad = 0" in out
