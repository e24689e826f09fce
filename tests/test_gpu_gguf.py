"""GPU checks of the streaming GGUF loader (bq_gguf_load): raw k-quant bytes
land on the device unchanged, the repacks and the BF16 -> Q8S conversion that
follow match the oracle bit for bit, and a GEMV on the loaded weight matches
the oracle.  The BF16 head (82 MB) is larger than one 64 MiB staging slot, so
the double-buffered stream runs over several chunks."""
import numpy as np
import pytest

import gguf_writer as W
from helpers import acts, dev, host

pytestmark = pytest.mark.gpu


def test_gguf_load_and_repack(bq, oracle, tmp_path):
    import torch
    K5, N5 = 4096, 16384
    K6, N6 = 9216, 3072
    KB, NB = 1024, 40000
    q5 = W.random_kquant(11, N5, K5, 176)
    q6 = W.random_kquant(12, N6, K6, 210)
    bf = oracle.f32_to_bf16(oracle.gaussian(13, NB * KB, 0.0, 0.02).reshape(NB, KB))
    path = str(tmp_path / "m.gguf")
    W.write_gguf(path, [("general.alignment", W.T_U32, 256)],
                 [("blk.0.ffn_gate.weight", 13, (K5, N5), q5.tobytes()),
                  ("blk.0.ffn_down.weight", 14, (K6, N6), q6.tobytes()),
                  ("output.weight", 30, (KB, NB), bf.tobytes())], alignment=256)
    print("gguf load: file written", flush=True)
    with bq.Gguf(path) as g:
        # Q5_K + W144 / Dm
        raw5 = torch.empty(q5.size, dtype=torch.uint8, device="cuda")
        w144 = torch.empty(bq.load().bq_repack_q5k_bytes(K5, N5), dtype=torch.uint8, device="cuda")
        dm = torch.empty(N5 * K5 // 32, dtype=torch.int16, device="cuda")
        w5 = g.load(g.find("blk.0.ffn_gate.weight"), raw5, w144, dm)
        # Q6_K + W160
        raw6 = torch.empty(q6.size, dtype=torch.uint8, device="cuda")
        w160 = torch.empty(bq.load().bq_repack_q6k_bytes(K6, N6), dtype=torch.uint8, device="cuda")
        w6 = g.load(g.find("blk.0.ffn_down.weight"), raw6, w160)
        # BF16 -> Q8S head
        stage = torch.empty(bf.size * 2, dtype=torch.uint8, device="cuda")
        q8s = torch.empty(bq.load().bq_q8s_bytes(KB, NB), dtype=torch.uint8, device="cuda")
        wh = g.load(g.find("output.weight"), stage, q8s)
        torch.cuda.synchronize()
    print("gguf load: loaded", flush=True)
    assert (w5.K, w5.N, w5.ggml_type) == (K5, N5, 13) and w5.rep and w5.rep_min
    assert (w6.K, w6.N, w6.ggml_type) == (K6, N6, 14) and w6.rep and not w6.rep_min
    assert (wh.K, wh.N, wh.ggml_type) == (KB, NB, 8) and wh.raw == q8s.data_ptr()
    assert np.array_equal(host(raw5), q5.reshape(-1))
    assert np.array_equal(host(raw6), q6.reshape(-1))
    assert np.array_equal(host(stage).view(np.uint16), bf.reshape(-1))
    r144, rdm = oracle.repack_q5k_144(q5, K5)
    assert np.array_equal(host(w144), r144.reshape(-1))
    assert np.array_equal(host(dm).view(np.uint16), rdm.reshape(-1))
    assert np.array_equal(host(w160), oracle.repack_q6k_160(q6, K6).reshape(-1))
    assert np.array_equal(host(q8s), oracle.quantize_q8s(bf).reshape(-1))
    # a GEMV straight from the loaded descriptor
    _, (xq, xd, xs) = acts(14, 1, K5)
    y = torch.empty(N5, device="cuda")
    bq.gemv(y, w5, dev(xq), dev(xd), dev(xs))
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y)[None], oracle.gemm_q5k(q5, xq, xd, xs)) < 1e-4


def test_gguf_load_rejects(bq, tmp_path):
    import torch
    f32 = np.zeros((4, 256), np.float32)
    q5 = W.random_kquant(15, 2, 256, 176)
    path = str(tmp_path / "r.gguf")
    W.write_gguf(path, [], [("norm", 0, (256, 4), f32.tobytes()), ("w", 13, (256, 2), q5.tobytes()),
                            ("h", 30, (256, 2), np.zeros(512, np.uint16).tobytes())])
    buf = torch.empty(4096, dtype=torch.uint8, device="cuda")
    with bq.Gguf(path) as g:
        with pytest.raises(bq.BqError) as e:
            g.load(0, buf)                               # F32: not a k-quant matrix
        assert e.value.code == bq.BQ_UNSUPPORTED
        with pytest.raises(bq.BqError):
            g.load(1, buf, rep=buf)                      # Q5_K W144 without Dm
        with pytest.raises(bq.BqError):
            g.load(2, buf)                               # BF16 without its Q8S target
        w = g.load(1, buf)                               # raw only
        assert w.rep is None and w.K == 256 and w.N == 2
