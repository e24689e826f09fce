"""Committed golden fixtures (tests/golden/golden.npz, written by
tests/golden/make_golden.py from this repository's oracle): the oracle must
still reproduce them bit-exactly (CPU), and the HIP path must match them --
bit-exact for codes, scales, sums and repacked bytes, TOL (1e-4 normwise
relative) for fp32 outputs (GPU)."""
import os

import numpy as np
import pytest

from helpers import dev, host

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
TOL = 1e-4


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def test_oracle_reproduces_golden(oracle, gold):
    g = gold
    xq, xd, xs = oracle.q8_rows(g["q8_x"])
    assert np.array_equal(xq, g["q8_xq"]) and np.array_equal(_bits(xd), _bits(g["q8_xd"]))
    assert np.array_equal(xs, g["q8_xs"])
    assert np.array_equal(oracle.fill_xdh(xd, xs), g["q8_xdh"])
    args5 = (g["gemv_xq"], g["gemv_xd"], g["gemv_xs"])
    assert np.array_equal(_bits(oracle.gemm_q5k(g["gemv_w5"], *args5)), _bits(g["gemv_y5"]))
    assert np.array_equal(_bits(oracle.gemm_q5k_f32(g["gemv_w5"], *args5)), _bits(g["gemv_y5_f32"]))
    assert np.array_equal(_bits(oracle.gemm_q6k(g["gemv_w6"], g["gemv_xq"], g["gemv_xd"])), _bits(g["gemv_y6"]))
    assert np.array_equal(_bits(oracle.gemm_q6k_f32(g["gemv_w6"], g["gemv_xq"], g["gemv_xd"])),
                          _bits(g["gemv_y6_f32"]))
    K = g["gemv_xq"].shape[1]
    w144, dm = oracle.repack_q5k_144(g["gemv_w5"], K)
    assert np.array_equal(w144, g["rep_w144"]) and np.array_equal(dm, g["rep_dm"])
    assert np.array_equal(oracle.repack_q6k_160(g["gemv_w6"], K), g["rep_w160"])
    Kg = g["gemm_xq"].shape[1]
    w144g, dmg = oracle.repack_q5k_144(g["gemm_w5"], Kg)
    xdh = oracle.fill_xdh(g["gemm_xd"], g["gemm_xs"])
    y = oracle.gemm_q5k_144(w144g, dmg, g["gemm_xq"], g["gemm_xd"], xdh, g["gemm_w5"].shape[0])
    assert np.array_equal(_bits(y.astype(np.float32)), _bits(g["gemm_y144"]))
    assert np.array_equal(oracle.quantize_q8s(g["q8s_bf16"]), g["q8s_w"])
    Kh = g["q8s_bf16"].shape[1]
    yh = oracle.gemv_q8s(g["q8s_w"], Kh, g["gemv_xq"][:, :Kh], g["gemv_xd"][:, :Kh // 32], g["q8s_rs"])
    assert np.array_equal(_bits(yh), _bits(g["q8s_y"]))
    for op, args in NORM_ARGS.items():
        got = oracle.norm_rows(op, *[g[k] for k in args])
        assert np.array_equal(_bits(got), _bits(g[f"norm_{op}"])), op


NORM_ARGS = {"norm": ("norm_a",), "add": ("norm_a", "norm_b"), "resid": ("norm_a", "norm_b", "norm_c"),
             "gate": ("norm_a", "norm_b", "norm_c"), "silu": ("norm_b", "norm_a", "norm_c", "norm_d")}


@pytest.mark.gpu
def test_hip_matches_golden(bq, oracle, gold):
    import torch
    g = gold
    gq, gd, gs, gh = bq.quantize_q8(dev(g["q8_x"]), with_xdh=True)
    torch.cuda.synchronize()
    assert np.array_equal(host(gq), g["q8_xq"]) and np.array_equal(_bits(host(gd)), _bits(g["q8_xd"]))
    assert np.array_equal(host(gs), g["q8_xs"]) and np.array_equal(host(gh).view(np.uint16), g["q8_xdh"])
    M, K = g["gemv_xq"].shape
    N = g["gemv_w5"].shape[0]
    xq, xd, xs = dev(g["gemv_xq"]), dev(g["gemv_xd"]), dev(g["gemv_xs"])
    w5, w6 = dev(g["gemv_w5"]), dev(g["gemv_w6"])
    y5 = torch.full((M, N), float("nan"), device="cuda")
    assert bq.verify_fused([y5], [bq.make_weight(w5, bq.TYPE_Q5_K, K, N)], M, xq, xd, xs) == bq.BQ_OK
    y6 = torch.full((M, N), float("nan"), device="cuda")
    bq.gemm_q6k_raw(y6, bq.make_weight(w6, bq.TYPE_Q6_K, K, N), M, xq, xd)
    w144, dm = bq.repack_q5k(w5, K, N)
    w160 = bq.repack_q6k(w6, K, N)
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y5), g["gemv_y5"]) < TOL
    assert oracle.normwise_err(host(y6), g["gemv_y6"]) < TOL
    assert np.array_equal(host(w144).reshape(g["rep_w144"].shape), g["rep_w144"])
    assert np.array_equal(host(dm).view(np.uint16).reshape(g["rep_dm"].shape), g["rep_dm"])
    assert np.array_equal(host(w160).reshape(g["rep_w160"].shape), g["rep_w160"])
    Mg, Kg = g["gemm_xq"].shape
    Ng = g["gemm_w5"].shape[0]
    raw = dev(g["gemm_w5"])
    rw, rdm = bq.repack_q5k(raw, Kg, Ng)
    xdh = torch.empty((Mg, Kg // 32), dtype=torch.float16, device="cuda")
    for w, ref in ((bq.make_weight(raw, bq.TYPE_Q5_K, Kg, Ng, rep=rw, rep_min=rdm), g["gemm_y144"]),
                   (bq.make_weight(raw, bq.TYPE_Q5_K, Kg, Ng), g["gemm_y_exact"])):
        y = torch.full((Mg, Ng), float("nan"), device="cuda")
        assert bq.try_mmq([y], [w], Mg, dev(g["gemm_xq"]), dev(g["gemm_xd"]), dev(g["gemm_xs"]), xdh) == bq.BQ_OK
        torch.cuda.synchronize()
        assert oracle.normwise_err(host(y), ref.astype(np.float64)) < TOL


@pytest.mark.gpu
def test_hip_matches_golden_head_and_producers(bq, oracle, gold):
    import torch
    g = gold
    Nh, Kh = g["q8s_bf16"].shape
    hq = bq.quantize_q8s(dev(g["q8s_bf16"].view(np.int16)), Kh, Nh)
    torch.cuda.synchronize()
    assert np.array_equal(host(hq), g["q8s_w"])
    M = g["gemv_xq"].shape[0]
    y = torch.full((M, Nh), float("nan"), device="cuda")
    xq = dev(np.ascontiguousarray(g["gemv_xq"][:, :Kh]))
    xd = dev(np.ascontiguousarray(g["gemv_xd"][:, :Kh // 32]))
    assert bq.gemv_q8s(y, hq, xq, xd, Kh, Nh, M, dev(g["q8s_rs"])) == bq.BQ_OK
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y), g["q8s_y"]) < TOL
    n = g["norm_a"].shape[1]
    for op, args in NORM_ARGS.items():
        ins = [dev(g[k]) for k in args]
        out = ins[0] if op in ("add", "resid") else torch.empty((2, n), device="cuda")
        kw = dict(out=out, a=ins[0])
        kw.update({k: t for k, t in zip("bcd", ins[1:])})
        r, (q, d_, s_) = bq.norm_q8(op, 2, n, **kw)
        assert r == bq.BQ_OK
        torch.cuda.synchronize()
        o = host(out)
        assert oracle.normwise_err(o, g[f"norm_{op}"]) < 2e-6, op
        rq, rd, rs_ = oracle.q8_rows(o)
        assert np.array_equal(host(q), rq) and np.array_equal(host(s_), rs_), op
