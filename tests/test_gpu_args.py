"""Argument checks of the compute entry points that need the device to be
initialised: every kernel reads weights, activations and fp32 rows with
16-byte loads (direct-to-LDS copies included), so a buffer that does not start
16-byte aligned must come back as BQ_EINVAL with nothing enqueued -- the
output stays untouched.  (The reference passes cudaMalloc'd buffers and has no
such check; a misaligned pointer there is undefined.)"""
import pytest

from helpers import acts, dev, weights

pytestmark = pytest.mark.gpu


def _mis(t, elems=1):
    """A view of t starting `elems` elements in (not 16-byte aligned)."""
    return t.view(-1)[elems:]


@pytest.fixture(scope="module")
def setup(bq):
    import torch
    K, N = 256, 128
    raw = dev(weights(901, N, K, "q5k"))
    raw6 = dev(weights(902, N, K, "q6k"))
    rep6 = bq.repack_q6k(raw6, K, N)
    w144, dm = bq.repack_q5k(raw, K, N)
    _, (xq, xd, xs) = acts(903, 96, K)
    x = torch.randn(1, K, device="cuda")
    return dict(K=K, N=N, raw=raw, raw6=raw6, rep6=rep6, w144=w144, dm=dm,
                xq=dev(xq), xd=dev(xd), xs=dev(xs), x=x)


def _expect_einval(bq, fn):
    with pytest.raises(bq.BqError) as e:
        fn()
    assert e.value.code == bq.BQ_EINVAL


def test_gemv_rejects_misaligned(bq, setup):
    import torch
    s = setup
    K, N = s["K"], s["N"]
    w = bq.make_weight(s["raw"], bq.TYPE_Q5_K, K, N)
    y = torch.full((N,), float("nan"), device="cuda")
    print("gemv misaligned xq / xd / xsum / weight", flush=True)
    # a buffer one element in: int8 codes are 1 byte off, xd / xsum 4 bytes off
    _expect_einval(bq, lambda: bq.gemv(y, w, _mis(s["xq"]), s["xd"], s["xs"]))
    _expect_einval(bq, lambda: bq.gemv(y, w, s["xq"], _mis(s["xd"]), s["xs"]))
    _expect_einval(bq, lambda: bq.gemv(y, w, s["xq"], s["xd"], _mis(s["xs"])))
    wm = bq.make_weight(_mis(s["raw"], 8), bq.TYPE_Q5_K, K, N)
    _expect_einval(bq, lambda: bq.gemv(y, wm, s["xq"], s["xd"], s["xs"]))
    w6m = bq.make_weight(_mis(s["raw6"], 2), bq.TYPE_Q6_K, K, N)
    _expect_einval(bq, lambda: bq.gemv(y, w6m, s["xq"], s["xd"], s["xs"]))
    torch.cuda.synchronize()
    assert torch.isnan(y).all()


def test_fused_and_verify_reject_misaligned(bq, setup):
    import torch
    s = setup
    K, N = s["K"], s["N"]
    w = bq.make_weight(s["raw"], bq.TYPE_Q5_K, K, N)
    y = torch.full((N,), float("nan"), device="cuda")
    print("fused / verify / gate_up_silu misaligned inputs", flush=True)
    xbuf = torch.randn(1, K + 4, device="cuda")
    _expect_einval(bq, lambda: bq.gemv_q8_fused([y], [w], _mis(xbuf)))
    _expect_einval(bq, lambda: bq.verify_fused([y], [w], 2, s["xq"], _mis(s["xd"]), s["xs"]))
    h = torch.full((N,), float("nan"), device="cuda")
    sg = torch.ones(N, device="cuda")
    _expect_einval(bq, lambda: bq.gate_up_silu(h, w, w, sg, sg, _mis(s["xq"]), s["xd"], s["xs"]))
    w6 = bq.make_weight(s["raw6"], bq.TYPE_Q6_K, K, N, rep=s["rep6"])
    _expect_einval(bq, lambda: bq.q6_verify_fused([y], [w6], 2, s["xq"], _mis(s["xd"])))
    torch.cuda.synchronize()
    assert torch.isnan(y).all() and torch.isnan(h).all()


def test_gemm_and_quantizer_reject_misaligned(bq, setup):
    import torch
    s = setup
    K, N = s["K"], s["N"]
    rows = 96
    wp = bq.make_weight(s["raw"], bq.TYPE_Q5_K, K, N, rep=s["w144"], rep_min=s["dm"])
    y = torch.full((rows, N), float("nan"), device="cuda")
    xdh = bq.fill_xdh(s["xd"], s["xs"])
    print("try_mmq / gemm_q6k_mma / quantize_q8 misaligned", flush=True)
    _expect_einval(bq, lambda: bq.try_mmq([y], [wp], rows, s["xq"], s["xd"], _mis(s["xs"]), xdh))
    _expect_einval(bq, lambda: bq.try_mmq([y], [wp], rows, s["xq"], s["xd"], s["xs"], _mis(xdh)))
    wpm = bq.make_weight(s["raw"], bq.TYPE_Q5_K, K, N, rep=_mis(s["w144"], 4), rep_min=s["dm"])
    _expect_einval(bq, lambda: bq.try_mmq([y], [wpm], rows, s["xq"], s["xd"], s["xs"], xdh))
    w6 = bq.make_weight(s["raw6"], bq.TYPE_Q6_K, K, N, rep=s["rep6"])
    y6 = torch.full((rows, N), float("nan"), device="cuda")
    _expect_einval(bq, lambda: bq.gemm_q6k_mma(y6, w6, rows, s["xq"], _mis(s["xd"])))
    xb = torch.randn(2, K + 4, device="cuda")
    _expect_einval(bq, lambda: bq.quantize_q8(_mis(xb).view(-1)[: 2 * K].view(2, K)))
    torch.cuda.synchronize()
    assert torch.isnan(y).all() and torch.isnan(y6).all()
