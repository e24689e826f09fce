"""The package's numpy k-quant encoder (used to build benchmark weights) is
byte-identical to the oracle's C encoder on the same float inputs."""
import numpy as np

import synth


def test_q5k_encoder_matches_oracle(oracle):
    w = oracle.gaussian(901, 48 * 1024, 0, 0.02).reshape(48, 1024)
    w[3, :256] = 0.0          # all-zero super-block
    w[4, :32] = 0.5           # constant positive sub-block
    assert np.array_equal(synth.quantize_q5k(w), oracle.quantize_q5k(w))


def test_q6k_encoder_matches_oracle(oracle):
    w = oracle.gaussian(902, 48 * 1024, 0, 0.02).reshape(48, 1024)
    w[3, :256] = 0.0
    w[5, 16:32] = -0.25       # constant negative group
    assert np.array_equal(synth.quantize_q6k(w), oracle.quantize_q6k(w))
