"""CPU checks of the C ABI: libbq.so loads, exports every function that
include/bq.h declares, and its host-only entry points match the oracle."""
import ctypes
import os
import re

import numpy as np

from helpers import weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "bq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bq_[a-z0-9_]+)\s*\(", text)))


def test_header_matches_exports():
    import bq
    L = bq.load()
    names = declared_functions()
    assert len(names) >= 18
    for n in names:
        assert hasattr(L, n), n
    assert sorted(names) == sorted(bq.EXPORTS)


def test_library_is_gfx950_hip():
    import bq
    data = open(bq.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    assert bq.load().bq_version().decode().startswith("bq ")


def test_strerror():
    import bq
    assert bq.strerror(0) == "ok"
    assert "unsupported" in bq.strerror(1)


def test_repack_q6k_host_matches_oracle(oracle):
    import bq
    for N, K in [(4, 256), (17, 1024)]:
        raw = weights(77 + N, N, K, "q6k")
        got = bq.repack_q6k_host(raw, K, N)
        assert np.array_equal(got, oracle.repack_q6k_160(raw, K))


def test_repack_sizes():
    import bq
    L = bq.load()
    assert L.bq_repack_q5k_bytes(3072, 9216) == 31850496
    assert L.bq_repack_q5k_min_bytes(3072, 9216) == 1769472
    assert L.bq_repack_q6k_bytes(9216, 3072) == 35389440


def test_host_repack_rejects_bad_shape():
    import bq
    L = bq.load()
    buf = (ctypes.c_uint8 * 1024)()
    assert L.bq_repack_q6k_host(buf, 100, 1, buf) == bq.BQ_EINVAL
    assert L.bq_repack_q6k_host(None, 256, 1, buf) == bq.BQ_EINVAL


def test_quantize_q8s_host_matches_oracle(oracle):
    """bq_quantize_q8s_host (q8k_quant_host, bruce.cu:4843-4867) on the CPU."""
    import bq
    for N, K in [(3, 256), (11, 2560)]:
        w = oracle.f32_to_bf16(oracle.gaussian(500 + N, N * K, 0.0, 0.02).reshape(N, K))
        w[0, :32] = 0
        w[0, 32:64] = oracle.f32_to_bf16(np.full(32, 1e-38, np.float32))   # tiny (denormal half scale)
        w[0, [33, 60]] = 0                                                  # id = inf: zeros stay 0
        w[1, 64:96] = oracle.f32_to_bf16(np.linspace(-3e4, 3e4, 32).astype(np.float32))
        got = bq.quantize_q8s_host(w, K, N)
        assert np.array_equal(got, oracle.quantize_q8s(w))


def test_q8s_sizes_and_rejects():
    import bq
    L = bq.load()
    assert L.bq_q8s_bytes(2560, 131072) == 356515840      # the reference's 356.5 MB logits head
    assert L.bq_q8s_bytes(3072, 131072) == 427819008
    buf = (ctypes.c_uint8 * 1024)()
    assert L.bq_quantize_q8s_host(buf, 100, 1, buf) == bq.BQ_EINVAL
    assert L.bq_quantize_q8s_host(None, 256, 1, buf) == bq.BQ_EINVAL


def _has_gpu():
    import torch
    return torch.cuda.is_available()


def test_workspace_bytes():
    """bq_gemm_workspace_bytes_cus (host arithmetic only): the K-split
    workspace of the prefill GEMMs for a device of `cus` CUs, at most 32 MiB
    for any shape; bq_gemm_workspace_bytes sizes it for the current device,
    and without one (this CPU run) it is 0."""
    import bq
    L = bq.load()
    W = L.bq_gemm_workspace_bytes_cus
    # one token tile of a 9216-row matrix on 256 CUs: 72 tiles -> 7 slices for
    # the 512 slots, evened to 6 over the raw tier's 24 stages (4 each); the
    # 32-token tile (144 tiles, 768 slots) takes 5: the larger is reserved
    assert W(64, 3072, 9216, 256) == 6 * 64 * 9216 * 4
    # 1152 tiles = 4 x 256 + 128 leftover tiles: the W144 tier cuts each
    # leftover tile into 2 K slices of 128 x 128 fp32 partial tiles
    assert W(2048, 3072, 9216, 256) == 128 * 2 * 128 * 128 * 4
    assert W(4096, 3072, 9216, 256) == 0      # 2304 tiles = 9 x 256: no leftover
    assert W(0, 3072, 9216, 256) == 0
    assert W(64, 3072, 9216, 0) == 0
    # the split follows the CU count.  On 304 CUs the 128-token tile's 1152
    # tiles are 3 x 304 + 240 and no leftover split beats 4 rounds by half a
    # tile; the 32-token tile's 4608 are 15 x 304 + 48, whose 48 leftover tiles
    # take 4 K slices of 128 x 32 partials each
    assert W(2048, 3072, 9216, 304) == 48 * 4 * 128 * 32 * 4
    # 80 CUs: 72 tiles fill 160 slots twice over at most -> 2 slices, evened
    # over 24 stages (12 each)
    assert W(64, 3072, 9216, 80) == 2 * 64 * 9216 * 4
    # at most 32 MiB on 256 CUs; in general the uniform split fills the
    # device's slots with 128 x 128 fp32 partial tiles (CUs x 128 KiB) and the
    # leftover split is capped at 32 MiB
    for c in (80, 256, 304):
        worst = max(W(r, 3072, n, c) for r in list(range(1, 600, 7)) + list(range(600, 9000, 97))
                    for n in (128, 1024, 9216, 36864))
        assert worst <= max(32 << 20, c * (128 << 10)), c
        if c == 256:
            assert worst <= 32 << 20
    if not _has_gpu():
        assert L.bq_gemm_workspace_bytes(64, 3072, 9216) == 0


STRUCTS = [("bq_weight", "Weight"), ("bq_gguf_tensor", "GgufTensor"), ("bq_decode_block", "DecodeBlock"),
           ("bq_decode_step", "DecodeStep")]


def header_fields(name):
    """Field names of `typedef struct name { ... } name;` in include/bq.h, in order."""
    text = open(os.path.join(ROOT, "include", "bq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S).group(1)
    out = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        fp = re.search(r"\(\s*\*\s*(\w+)\s*\)", decl)           # function pointer
        if fp:
            out.append(fp.group(1))
            continue
        for part in decl.split(","):
            out.append(re.findall(r"(\w+)\s*(?:\[\s*\d+\s*\])?\s*$", part.strip())[0])
    return out


def test_ctypes_structs_match_header(tmp_path):
    """The ctypes mirrors in bq.py have the header's fields, in order, at the
    offsets a C compiler gives them (a field missing from a mirror makes the
    library read past the caller's struct)."""
    import shutil
    import subprocess
    import bq
    for cname, pyname in STRUCTS:
        assert [f[0] for f in getattr(bq, pyname)._fields_] == header_fields(cname), cname
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        return
    src = ['#include <stddef.h>', '#include <stdio.h>', '#include "bq.h"', 'int main(void) {']
    for cname, _ in STRUCTS:
        src.append('printf("%s size %%zu\\n", sizeof(%s));' % (cname, cname))
        for f in header_fields(cname):
            src.append('printf("%s %s %%zu\\n", offsetof(%s, %s));' % (cname, f, cname, f))
    src.append("return 0; }")
    (tmp_path / "off.c").write_text("\n".join(src))
    exe = tmp_path / "off"
    subprocess.run([cc, "-I", os.path.join(ROOT, "include"), str(tmp_path / "off.c"), "-o", str(exe)], check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                        check=True).stdout.splitlines())
    for cname, pyname in STRUCTS:
        S = getattr(bq, pyname)
        assert int(got[f"{cname} size"]) == ctypes.sizeof(S), cname
        for f, _ in S._fields_:
            assert int(got[f"{cname} {f}"]) == getattr(S, f).offset, (cname, f)
