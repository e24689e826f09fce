"""Writes tests/golden/golden.npz: small seeded inputs and the oracle's outputs
for every function of the path (q8 quantizer incl. edge values, Q5_K/Q6_K GEMV
in double and fp32 order, both repacks, the W144 GEMM, the BF16 -> Q8S
conversion and Q8S GEMV of the logits head, and the five q8-producing norms).

These are regression fixtures of this repository's CPU oracle (oracle/), not
vectors produced by the reference: the reference ships none for this path and
its CUDA sources cannot be built here.  test_golden.py checks that the oracle
still reproduces them bit-exactly and that the HIP path matches them, so a
change to either side that alters results is caught without re-deriving them.

    python tests/golden/make_golden.py   # needs oracle/_build (make -C oracle)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402


def main():
    g = {}
    # quantizer: 4 rows x 256 with an all-zero group, a lone tiny value, one
    # huge value, exact ties (v*id = k + 0.5) and negative-only groups
    x = O.gaussian(0xC0DE, 4 * 256, 0.0, 1.0).reshape(4, 256)
    x[0, :32] = 0.0
    x[0, 32:64] = 0.0
    x[0, 40] = 1e-30
    x[1, 64:96] = np.linspace(-127.0, 127.0, 32, dtype=np.float32)   # d = 1: integer grid
    x[1, 96:128] = np.arange(32, dtype=np.float32) - 15.5 + 0.0      # .5 ties once scaled
    x[2, :32] *= 1e6
    x[3, 128:160] = -np.abs(x[3, 128:160])
    g["q8_x"] = x
    g["q8_xq"], g["q8_xd"], g["q8_xs"] = O.q8_rows(x)
    g["q8_xdh"] = O.fill_xdh(g["q8_xd"], g["q8_xs"])
    # GEMV, both formats: N = 48 rows, K = 512, 3 activation rows
    K, N, M = 512, 48, 3
    w5 = O.quantize_q5k(O.gaussian(0xC0DF, N * K, 0.0, 0.02).reshape(N, K))
    w6 = O.quantize_q6k(O.gaussian(0xC0E0, N * K, 0.0, 0.02).reshape(N, K))
    xa = O.gaussian(0xC0E1, M * K, 0.0, 1.0).reshape(M, K)
    xq, xd, xs = O.q8_rows(xa)
    g.update(gemv_w5=w5, gemv_w6=w6, gemv_xq=xq, gemv_xd=xd, gemv_xs=xs)
    g["gemv_y5"] = O.gemm_q5k(w5, xq, xd, xs)
    g["gemv_y5_f32"] = O.gemm_q5k_f32(w5, xq, xd, xs)
    g["gemv_y6"] = O.gemm_q6k(w6, xq, xd)
    g["gemv_y6_f32"] = O.gemm_q6k_f32(w6, xq, xd)
    # repacks
    g["rep_w144"], g["rep_dm"] = O.repack_q5k_144(w5, K)
    g["rep_w160"] = O.repack_q6k_160(w6, K)
    # W144 GEMM: M = 96 tokens (the MMQ minimum), N = 128, K = 512; outputs
    # stored as fp32 (compared with the fp32 tolerance)
    Kg, Ng, Mg = 512, 128, 96
    wg = O.quantize_q5k(O.gaussian(0xC0E2, Ng * Kg, 0.0, 0.02).reshape(Ng, Kg))
    xg = O.gaussian(0xC0E3, Mg * Kg, 0.0, 1.0).reshape(Mg, Kg)
    gq, gd, gs = O.q8_rows(xg)
    w144, dm = O.repack_q5k_144(wg, Kg)
    xdh = O.fill_xdh(gd, gs)
    g.update(gemm_w5=wg, gemm_xq=gq, gemm_xd=gd, gemm_xs=gs)
    g["gemm_y144"] = O.gemm_q5k_144(w144, dm, gq, gd, xdh, Ng).astype(np.float32)
    g["gemm_y_exact"] = O.gemm_q5k(wg, gq, gd, gs).astype(np.float32)
    # Q8_0 logits head: BF16 6 x 512 with a zero group, a denormal-scale group
    # and a +-3e4 group; Q8S GEMV of 3 q8 rows with a per-row scale
    Kh, Nh = 512, 6
    wb = O.f32_to_bf16(O.gaussian(0xC0E4, Nh * Kh, 0.0, 0.02).reshape(Nh, Kh))
    wb[0, :32] = 0
    wb[1, 32:64] = O.f32_to_bf16(np.full(32, 1e-38, np.float32))
    wb[2, 64:96] = O.f32_to_bf16(np.linspace(-3e4, 3e4, 32).astype(np.float32))
    hq = O.quantize_q8s(wb)
    rs = O.gaussian(0xC0E5, Nh, 1.0, 0.2)
    g.update(q8s_bf16=wb, q8s_w=hq, q8s_rs=rs)
    g["q8s_y"] = O.gemv_q8s(hq, Kh, xq[:, :Kh], xd[:, :Kh // 32], rs)
    # q8 producers: 2 rows x 256 per op, fp64 rows of the oracle
    n = 256
    a, b = O.gaussian(0xC0E6, 2 * n).reshape(2, n), O.gaussian(0xC0E7, 2 * n, 0.0, 2.0).reshape(2, n)
    c, d = O.gaussian(0xC0E8, n, 0.5, 0.3), O.gaussian(0xC0E9, n, 1.0, 0.3)
    g.update(norm_a=a, norm_b=b, norm_c=c, norm_d=d)
    for op, args in (("norm", (a,)), ("add", (a, b)), ("resid", (a, b, c)), ("gate", (a, b, c)),
                     ("silu", (b, a, c, d))):
        g[f"norm_{op}"] = O.norm_rows(op, *args)
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **g)
    print("wrote", os.path.join(HERE, "golden.npz"), {k: v.shape for k, v in g.items()})


if __name__ == "__main__":
    main()
