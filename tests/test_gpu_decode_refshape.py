"""The decode step at the reference model's own shapes (engine/src/bruce.cu:43-49:
N_EMBD 2560, N_HEAD 16 x HD 256 = 4096 attention width, N_KV 4 x 256 = 1024
for k and v, N_FF 7168).  These take the run-time-K GEMV instances (the
compile-time ones cover K = 3072 / 4096 / 9216) and the 7168-value fused
down row.  The checks are those of tests/test_gpu_decode.py, run on these
shapes."""
import pytest

import test_gpu_decode as D

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fold", [0, 1, 2])
def test_decode_graph_vs_oracle_reference_shapes(bq, oracle, fold):
    saved = (D.E, D.A, D.FF, D.PARTS)
    D.E, D.A, D.FF = 2560, 4096, 7168
    D.PARTS = [("q", 4096, "q5k"), ("k", 1024, "q5k"), ("gate", 4096, "q5k"), ("v", 1024, "q6k")]
    try:
        D.test_decode_graph_vs_oracle(bq, oracle, fold)
    finally:
        D.E, D.A, D.FF, D.PARTS = saved
