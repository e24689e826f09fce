"""ctypes binding of libbq.so (include/bq.h) over torch device tensors.

torch supplies device memory and the current HIP stream; every computation runs
in libbq's HIP kernels.  There is no fallback: if libbq.so is missing or the
GPU is absent, calls raise.

Host-side mirror of the reference's launchers (engine/src/bruce.cu):
    gemv                  launch_gemv            :5624
    verify_fused          launch_verify_fused    :7141
    q6_verify_fused       launch_q6_verify_fused :7231
    gemm_q6k_dp           launch_gemm_q6k_dp     :7285
    try_mmq               try_launch_mmq         :7366
    gemm_b / gemm_b_fused launch_gemm_b(_fused)  :7421-7568
    repack_q5k            q5k_prepack_launch     :4832
    repack_q6k(_host)     q6k_repack_host        :4783
    quantize_q8           k_q8_quant / k_q8_rows :518, :1081
    quantize_q8s(_host)   k_bf16_to_q8 / q8k_quant_host :5159, :4843
    gemv_q8s              k_gemm_q8_logits       :4409 (launch_logits_b :7570)
    norm_q8 / add_norm_q8 / resid_q8 / gate_norm_q8 / silu_mul_norm_q8
                          k_norm :541, k_add_norm :556, k_resid :571, k_gate_norm :602,
                          k_silu_mul_norm :622 (and their _rows / _vec4 forms)
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbq.so")

BQ_OK, BQ_UNSUPPORTED, BQ_EINVAL, BQ_ETOOBIG = 0, 1, 2, 3
TYPE_Q5_K, TYPE_Q6_K = 13, 14
Q5K_BYTES, Q6K_BYTES = 176, 210
Q8S_BYTES = 272  # Q8_0 logits head: 8 fp16 scales + 256 int8 per (row, 256 values)

EXPORTS = [
    "bq_init", "bq_strerror", "bq_version", "bq_quantize_q8", "bq_fill_xdh", "bq_gemv",
    "bq_verify_fused", "bq_q6_verify_fused", "bq_gemm_q6k_dp", "bq_gemm_q6k_raw", "bq_try_mmq",
    "bq_gemm_q6k_mma", "bq_gemm_b", "bq_gemm_b_fused", "bq_repack_q5k", "bq_repack_q5k_bytes",
    "bq_repack_q5k_min_bytes", "bq_repack_q6k", "bq_repack_q6k_host", "bq_repack_q6k_bytes",
    "bq_time_next_launch", "bq_gemv_q8_fused", "bq_q8s_bytes", "bq_quantize_q8s",
    "bq_quantize_q8s_host", "bq_gemv_q8s", "bq_norm_q8", "bq_add_norm_q8", "bq_resid_q8",
    "bq_gate_norm_q8", "bq_silu_mul_norm_q8", "bq_gguf_open", "bq_gguf_close", "bq_gguf_n_tensors",
    "bq_gguf_find", "bq_gguf_tensor_info", "bq_gguf_kv_num", "bq_gguf_kv_str", "bq_gguf_read", "bq_gguf_load",
    "bq_gemv_norm_fused", "bq_gate_up_silu", "bq_gemm_workspace_bytes", "bq_gemm_workspace_bytes_cus",
    "bq_gemm_b_fused_noalloc",
    "bq_noalloc_scratch_bytes", "bq_decode_enqueue", "bq_decode_graph_create", "bq_decode_graph_launch",
    "bq_decode_graph_destroy",
]


class BqError(RuntimeError):
    def __init__(self, code, what):
        self.code = code
        super().__init__(f"{what}: {strerror(code)} ({code})")


class Weight(ctypes.Structure):
    """bq_weight == the reference's TensorW {d, dp, dm, type, K, N} (bruce.cu:78)."""
    _fields_ = [("raw", ctypes.c_void_p), ("rep", ctypes.c_void_p), ("rep_min", ctypes.c_void_p),
                ("ggml_type", ctypes.c_uint32), ("K", ctypes.c_int32), ("N", ctypes.c_int32)]


class GgufTensor(ctypes.Structure):
    """bq_gguf_tensor (include/bq.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("suffix", ctypes.c_char_p), ("ne", ctypes.c_uint64 * 4),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64), ("ggml_type", ctypes.c_uint32),
                ("ndim", ctypes.c_uint32), ("block", ctypes.c_int32)]


BLOCK_ATTN, BLOCK_FFN = 0, 1
ATTN_HOOK = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p)


class DecodeBlock(ctypes.Structure):
    """bq_decode_block (include/bq.h): one attention or FFN block of the decode step."""
    _fields_ = [("kind", ctypes.c_int), ("norm_before", ctypes.c_int), ("norm_after", ctypes.c_int),
                ("alpha", ctypes.c_void_p),
                ("qkv", ctypes.POINTER(Weight)), ("n_qkv", ctypes.c_int), ("qkv_out", ctypes.POINTER(ctypes.c_void_p)),
                ("attn_out", ctypes.c_void_p), ("attn_gate", ctypes.c_void_p), ("sgate", ctypes.c_void_p),
                ("n_attn", ctypes.c_int), ("o", ctypes.POINTER(Weight)),
                ("gate", ctypes.POINTER(Weight)), ("up", ctypes.POINTER(Weight)),
                ("s_gate", ctypes.c_void_p), ("s_up", ctypes.c_void_p), ("down", ctypes.POINTER(Weight)),
                ("n_ff", ctypes.c_int)]


class DecodeStep(ctypes.Structure):
    """bq_decode_step (include/bq.h): the per-token decode launch sequence."""
    _fields_ = [("n_blocks", ctypes.c_int), ("blocks", ctypes.POINTER(DecodeBlock)), ("n_embd", ctypes.c_int),
                ("fold", ctypes.c_int), ("x", ctypes.c_void_p), ("input_h", ctypes.c_void_p),
                ("xq", ctypes.c_void_p), ("xd", ctypes.c_void_p), ("xsum", ctypes.c_void_p),
                ("proj", ctypes.c_void_p), ("ffn_g", ctypes.c_void_p), ("ffn_u", ctypes.c_void_p),
                ("attention", ATTN_HOOK), ("user", ctypes.c_void_p),
                ("head_q8s", ctypes.c_void_p), ("head_rs", ctypes.c_void_p), ("head", ctypes.POINTER(Weight)),
                ("vocab", ctypes.c_int), ("logits", ctypes.c_void_p), ("rows", ctypes.c_int),
                ("x_alt", ctypes.c_void_p), ("xdh", ctypes.c_void_p), ("work", ctypes.c_void_p),
                ("work_bytes", ctypes.c_size_t)]


_lib = None


def load(path=LIB_PATH):
    """Load libbq.so (raises if it is not built).  Imports torch first so the
    HIP runtime libbq links against is torch's own."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (one HIP runtime per process)
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build()")
    L = ctypes.CDLL(path)
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    WP = ctypes.POINTER(Weight)
    sig = {
        "bq_init": (I, []),
        "bq_strerror": (ctypes.c_char_p, [I]),
        "bq_version": (ctypes.c_char_p, []),
        "bq_quantize_q8": (I, [P, I, I, P, P, P, P, P]),
        "bq_fill_xdh": (I, [P, P, I, P, P]),
        "bq_gemv": (I, [P, WP, P, P, P, P]),
        "bq_verify_fused": (I, [P, P, I, I, P, P, P, I, P]),
        "bq_q6_verify_fused": (I, [P, P, I, I, P, P, I, P]),
        "bq_gemm_q6k_dp": (I, [P, WP, I, P, P, I, P]),
        "bq_gemm_q6k_raw": (I, [P, WP, I, P, P, I, P]),
        "bq_gemm_workspace_bytes": (S, [I, I, I]),
        "bq_gemm_workspace_bytes_cus": (S, [I, I, I, I]),
        "bq_try_mmq": (I, [P, P, I, I, P, P, P, P, P, S, P]),
        "bq_gemm_q6k_mma": (I, [P, WP, I, P, P, P, S, P]),
        "bq_gemm_b": (I, [P, WP, I, P, P, P, P, P, S, P]),
        "bq_gemm_b_fused": (I, [P, P, I, I, P, P, P, P, P, S, P]),
        "bq_gemm_b_fused_noalloc": (I, [P, P, I, I, P, P, P, P]),
        "bq_decode_enqueue": (I, [ctypes.POINTER(DecodeStep), P]),
        "bq_decode_graph_create": (I, [ctypes.POINTER(DecodeStep), P, ctypes.POINTER(P)]),
        "bq_decode_graph_launch": (I, [P, P]),
        "bq_decode_graph_destroy": (None, [P]),
        "bq_noalloc_scratch_bytes": (S, []),
        "bq_repack_q5k": (I, [P, I, I, P, P, P]),
        "bq_repack_q5k_bytes": (S, [I, I]),
        "bq_repack_q5k_min_bytes": (S, [I, I]),
        "bq_repack_q6k": (I, [P, I, I, P, P]),
        "bq_repack_q6k_host": (I, [P, I, I, P]),
        "bq_repack_q6k_bytes": (S, [I, I]),
        "bq_time_next_launch": (I, [P, P]),
        "bq_gemv_q8_fused": (I, [P, P, I, P, P, P, P, P]),
        "bq_gemv_norm_fused": (I, [P, P, I, I, P, P, P, P, P, P, P, P, P]),
        "bq_gate_up_silu": (I, [P, WP, WP, P, P, P, P, P, P]),
        "bq_q8s_bytes": (S, [I, I]),
        "bq_quantize_q8s": (I, [P, I, I, P, P]),
        "bq_quantize_q8s_host": (I, [P, I, I, P]),
        "bq_gemv_q8s": (I, [P, P, P, P, I, I, I, P, P]),
        "bq_norm_q8": (I, [P, P, I, I, P, P, P, P]),
        "bq_add_norm_q8": (I, [P, P, I, I, P, P, P, P]),
        "bq_resid_q8": (I, [P, P, P, I, I, P, P, P, P]),
        "bq_gate_norm_q8": (I, [P, P, P, P, I, I, P, P, P, P]),
        "bq_silu_mul_norm_q8": (I, [P, P, P, P, P, I, I, P, P, P, P]),
        "bq_gguf_open": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "bq_gguf_close": (None, [P]),
        "bq_gguf_n_tensors": (ctypes.c_int64, [P]),
        "bq_gguf_find": (ctypes.c_int64, [P, ctypes.c_char_p]),
        "bq_gguf_tensor_info": (I, [P, ctypes.c_int64, ctypes.POINTER(GgufTensor)]),
        "bq_gguf_kv_num": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
        "bq_gguf_kv_str": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]),
        "bq_gguf_read": (I, [P, ctypes.c_int64, P, S, ctypes.c_uint64]),
        "bq_gguf_load": (I, [P, ctypes.c_int64, P, P, P, WP, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def strerror(code):
    return load().bq_strerror(code).decode()


def _check(code, what):
    if code != BQ_OK:
        raise BqError(code, what)
    return code


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("libbq entry points take device tensors")


def make_weight(raw=None, ggml_type=TYPE_Q5_K, K=0, N=0, rep=None, rep_min=None):
    """Build a bq_weight; the tensors must stay alive while it is used."""
    w = Weight(_ptr(raw).value if raw is not None else None,
               _ptr(rep).value if rep is not None else None,
               _ptr(rep_min).value if rep_min is not None else None, ggml_type, K, N)
    w._keep = (raw, rep, rep_min)
    return w


# ---------------------------------------------------------------- quantizer
def quantize_q8(x, with_xdh=False):
    """x fp32 [rows, K] (device) -> xq int8 [rows,K], xd fp32 [rows,K/32], xsum int32, (xdh)."""
    import torch
    _need_gpu(x)
    x = x.contiguous()
    rows, K = x.shape
    xq = torch.empty((rows, K), dtype=torch.int8, device=x.device)
    xd = torch.empty((rows, K // 32), dtype=torch.float32, device=x.device)
    xs = torch.empty((rows, K // 32), dtype=torch.int32, device=x.device)
    xdh = torch.empty((rows, K // 32), dtype=torch.int16, device=x.device) if with_xdh else None
    _check(load().bq_quantize_q8(_ptr(x), rows, K, _ptr(xq), _ptr(xd), _ptr(xs), _ptr(xdh), _stream()),
           "bq_quantize_q8")
    return (xq, xd, xs, xdh) if with_xdh else (xq, xd, xs)


def fill_xdh(xd, xsum, out=None):
    import torch
    if out is None:
        out = torch.empty(xd.shape, dtype=torch.int16, device=xd.device)
    _check(load().bq_fill_xdh(_ptr(xd), _ptr(xsum), xd.numel(), _ptr(out), _stream()), "bq_fill_xdh")
    return out


# ---------------------------------------------------------------- GEMV / verify
def gemv(y, w, xq, xd, xsum):
    _check(load().bq_gemv(_ptr(y), ctypes.byref(w), _ptr(xq), _ptr(xd), _ptr(xsum), _stream()), "bq_gemv")
    return y


def _arrays(ys, ws):
    n = len(ws)
    yarr = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    warr = (ctypes.POINTER(Weight) * n)(*[ctypes.pointer(w) for w in ws])
    return yarr, warr


def verify_fused(ys, ws, rows, xq, xd, xsum, xoff=0):
    """Returns the raw code (BQ_UNSUPPORTED means nothing ran, as the reference's false)."""
    yarr, warr = _arrays(ys, ws)
    r = load().bq_verify_fused(yarr, warr, len(ws), rows, _ptr(xq), _ptr(xd), _ptr(xsum), xoff, _stream())
    if r not in (BQ_OK, BQ_UNSUPPORTED):
        raise BqError(r, "bq_verify_fused")
    return r


def gemv_q8_fused(ys, ws, x, xq=None, xd=None, xsum=None):
    """Quantize the fp32 row x and run the GEMV over every part in one launch;
    xq/xd/xsum (all or none) receive the q8 row."""
    yarr, warr = _arrays(ys, ws)
    r = load().bq_gemv_q8_fused(yarr, warr, len(ws), _ptr(x), _ptr(xq), _ptr(xd), _ptr(xsum), _stream())
    if r not in (BQ_OK, BQ_UNSUPPORTED):
        raise BqError(r, "bq_gemv_q8_fused")
    return r


OPS = {"norm": 0, "add": 1, "resid": 2, "gate": 3, "silu": 4}


def gemv_norm_fused(ys, ws, op, a, b=None, c=None, d=None, out=None, q8=None):
    """q8 producer (op as norm_q8: norm a; add a+b; resid x=a, upd=b, alpha=c;
    gate aout=a, gate=b, sg=c; silu g=a, u=b, sg=c, su=d) and the GEMV of its
    row over every part, one launch.  out receives the produced fp32 row, q8 =
    (xq, xd, xsum) its q8 row.  Returns the raw code (BQ_UNSUPPORTED: nothing ran)."""
    _need_gpu(a, b, c, d, out)
    yarr, warr = _arrays(ys, ws)
    xq, xd, xs = q8 if q8 is not None else (None, None, None)
    r = load().bq_gemv_norm_fused(yarr, warr, len(ws), OPS[op], _ptr(out), _ptr(a), _ptr(b), _ptr(c), _ptr(d),
                                  _ptr(xq), _ptr(xd), _ptr(xs), _stream())
    if r not in (BQ_OK, BQ_UNSUPPORTED):
        raise BqError(r, "bq_gemv_norm_fused")
    return r


def gate_up_silu(h, wg, wu, sg, su, xq, xd, xsum=None):
    """h = silu(g * sg) * u * su with g = wg x, u = wu x for one q8 row x, one launch."""
    _need_gpu(h, sg, su, xq, xd, xsum)
    _check(load().bq_gate_up_silu(_ptr(h), ctypes.byref(wg), ctypes.byref(wu), _ptr(sg), _ptr(su), _ptr(xq),
                                  _ptr(xd), _ptr(xsum), _stream()), "bq_gate_up_silu")
    return h


def q6_verify_fused(ys, ws, rows, xq, xd, xoff=0):
    yarr, warr = _arrays(ys, ws)
    r = load().bq_q6_verify_fused(yarr, warr, len(ws), rows, _ptr(xq), _ptr(xd), xoff, _stream())
    if r not in (BQ_OK, BQ_UNSUPPORTED):
        raise BqError(r, "bq_q6_verify_fused")
    return r


def gemm_q6k_dp(y, w, rows, xq, xd, xoff=0):
    return _check(load().bq_gemm_q6k_dp(_ptr(y), ctypes.byref(w), rows, _ptr(xq), _ptr(xd), xoff, _stream()),
                  "bq_gemm_q6k_dp")


def gemm_q6k_raw(y, w, rows, xq, xd, xoff=0):
    return _check(load().bq_gemm_q6k_raw(_ptr(y), ctypes.byref(w), rows, _ptr(xq), _ptr(xd), xoff, _stream()),
                  "bq_gemm_q6k_raw")


# ---------------------------------------------------------------- prefill GEMM
def workspace_bytes(rows, K, n_total):
    """bq_gemm_workspace_bytes: K-split workspace that allows the full split."""
    return int(load().bq_gemm_workspace_bytes(rows, K, n_total))


def workspace(rows, K, n_total, device="cuda"):
    """A K-split workspace for GEMMs of rows x (n_total = sum N) x K (None if
    such a launch never splits).  Allocated by torch: libbq itself allocates
    nothing."""
    import torch
    n = workspace_bytes(rows, K, n_total)
    return torch.empty(n // 4, dtype=torch.float32, device=device) if n else None


_ws_cache = {}  # (device, stream) -> the largest workspace handed out there so far


def _work(work, rows, K, n_total):
    """work="auto": a workspace sized for the full split, one per (device,
    stream) reused by every call there (calls on one stream are ordered, so
    they can share it) and grown when a shape needs more; None: no split; a
    tensor: used as given.  Returns (pointer, bytes, tensor kept alive by the
    caller)."""
    if isinstance(work, str):
        assert work == "auto"
        import torch
        n = workspace_bytes(rows, K, n_total)
        if n == 0:
            return None, 0, None
        key = (torch.cuda.current_device(), torch.cuda.current_stream().cuda_stream)
        work = _ws_cache.get(key)
        if work is None or work.numel() * 4 < n:
            work = torch.empty(n // 4, dtype=torch.float32, device="cuda")
            _ws_cache[key] = work
    if work is None:
        return None, 0, None
    return _ptr(work), work.numel() * work.element_size(), work


def try_mmq(ys, ws, rows, xq, xd, xsum, xdh=None, work="auto"):
    wp, wb, keep = _work(work, rows, ws[0].K, sum(w.N for w in ws))
    yarr, warr = _arrays(ys, ws)
    r = load().bq_try_mmq(yarr, warr, len(ws), rows, _ptr(xq), _ptr(xd), _ptr(xsum), _ptr(xdh), wp, wb, _stream())
    if r not in (BQ_OK, BQ_UNSUPPORTED):
        raise BqError(r, "bq_try_mmq")
    return r


def gemm_q6k_mma(y, w, rows, xq, xd, work="auto"):
    wp, wb, keep = _work(work, rows, w.K, w.N)
    return _check(load().bq_gemm_q6k_mma(_ptr(y), ctypes.byref(w), rows, _ptr(xq), _ptr(xd), wp, wb, _stream()),
                  "bq_gemm_q6k_mma")


def gemm_b(y, w, rows, xq, xd, xsum, xdh=None, work="auto"):
    wp, wb, keep = _work(work, rows, w.K, w.N)
    return _check(load().bq_gemm_b(_ptr(y), ctypes.byref(w), rows, _ptr(xq), _ptr(xd), _ptr(xsum),
                                   _ptr(xdh), wp, wb, _stream()), "bq_gemm_b")


def gemm_b_fused(ys, ws, rows, xq, xd, xsum, xdh=None, work="auto"):
    wp, wb, keep = _work(work, rows, ws[0].K, sum(w.N for w in ws))
    yarr, warr = _arrays(ys, ws)
    return _check(load().bq_gemm_b_fused(yarr, warr, len(ws), rows, _ptr(xq), _ptr(xd), _ptr(xsum),
                                         _ptr(xdh), wp, wb, _stream()), "bq_gemm_b_fused")


# ---------------------------------------------------------------- repacks
def repack_q5k(raw, K, N):
    """raw uint8 device [N, K/256*176] -> (W144 uint8 [K/128, N, 144], Dm int16 [N, K/32])."""
    import torch
    w144 = torch.empty((K // 128, N, 144), dtype=torch.uint8, device=raw.device)
    dm = torch.empty((N, K // 32), dtype=torch.int16, device=raw.device)
    _check(load().bq_repack_q5k(_ptr(raw), K, N, _ptr(w144), _ptr(dm), _stream()), "bq_repack_q5k")
    return w144, dm


def repack_q6k(raw, K, N):
    import torch
    out = torch.empty((N, K // 128, 160), dtype=torch.uint8, device=raw.device)
    _check(load().bq_repack_q6k(_ptr(raw), K, N, _ptr(out), _stream()), "bq_repack_q6k")
    return out


def repack_q6k_host(raw_np, K, N):
    """Host twin on numpy arrays (no device)."""
    import numpy as np
    raw_np = np.ascontiguousarray(raw_np, np.uint8)
    out = np.empty((N, K // 128, 160), np.uint8)
    _check(load().bq_repack_q6k_host(raw_np.ctypes.data_as(ctypes.c_void_p), K, N,
                                     out.ctypes.data_as(ctypes.c_void_p)), "bq_repack_q6k_host")
    return out


# ---------------------------------------------------------------- Q8_0 logits head
def quantize_q8s(w_bf16, K, N):
    """bf16 bit patterns (int16/uint16 device tensor [N, K]) -> Q8S uint8 [N, K/256*272]."""
    import torch
    _need_gpu(w_bf16)
    out = torch.empty((N, K // 256 * Q8S_BYTES), dtype=torch.uint8, device=w_bf16.device)
    _check(load().bq_quantize_q8s(_ptr(w_bf16.contiguous()), K, N, _ptr(out), _stream()), "bq_quantize_q8s")
    return out


def quantize_q8s_host(w_bf16_np, K, N):
    """Host twin on a numpy uint16 array (no device)."""
    import numpy as np
    w = np.ascontiguousarray(w_bf16_np, np.uint16)
    out = np.empty((N, K // 256 * Q8S_BYTES), np.uint8)
    _check(load().bq_quantize_q8s_host(w.ctypes.data_as(ctypes.c_void_p), K, N,
                                       out.ctypes.data_as(ctypes.c_void_p)), "bq_quantize_q8s_host")
    return out


def gemv_q8s(y, w, xq, xd, K, N, rows, rs=None):
    """y fp32 [rows, N] = Q8S w [N, K] x q8 rows (xq [rows, K], xd [rows, K/32]), times rs[N]."""
    _need_gpu(y, w, xq, xd, rs)
    r = load().bq_gemv_q8s(_ptr(y), _ptr(w), _ptr(xq), _ptr(xd), K, N, rows, _ptr(rs), _stream())
    if r not in (BQ_OK, BQ_UNSUPPORTED):
        raise BqError(r, "bq_gemv_q8s")
    return r


# ---------------------------------------------------------------- q8 producers
def _q8_out(rows, n, device):
    import torch
    return (torch.empty((rows, n), dtype=torch.int8, device=device),
            torch.empty((rows, n // 32), dtype=torch.float32, device=device),
            torch.empty((rows, n // 32), dtype=torch.int32, device=device))


def norm_q8(op, rows, n, out=None, a=None, b=None, c=None, d=None, q8=None):
    """op in {"norm", "add", "resid", "gate", "silu"}; returns (out, (xq, xd, xsum)).
    norm: out = norm(a); add: a = norm(a + b) in place; resid: a = norm(norm(a) +
    (norm(b) - norm(a))*c) in place; gate: out = norm(a / (1 + exp(-b*c)));
    silu: out = norm(silu(a*c) * b * d)."""
    _need_gpu(out, a, b, c, d)
    if q8 is None:
        q8 = _q8_out(rows, n, a.device)
    xq, xd, xs = q8
    L = load()
    S = _stream()
    if op == "norm":
        r = L.bq_norm_q8(_ptr(out), _ptr(a), rows, n, _ptr(xq), _ptr(xd), _ptr(xs), S)
    elif op == "add":
        r = L.bq_add_norm_q8(_ptr(a), _ptr(b), rows, n, _ptr(xq), _ptr(xd), _ptr(xs), S)
    elif op == "resid":
        r = L.bq_resid_q8(_ptr(a), _ptr(b), _ptr(c), rows, n, _ptr(xq), _ptr(xd), _ptr(xs), S)
    elif op == "gate":
        r = L.bq_gate_norm_q8(_ptr(out), _ptr(a), _ptr(b), _ptr(c), rows, n, _ptr(xq), _ptr(xd), _ptr(xs), S)
    elif op == "silu":
        r = L.bq_silu_mul_norm_q8(_ptr(out), _ptr(a), _ptr(b), _ptr(c), _ptr(d), rows, n, _ptr(xq), _ptr(xd),
                                  _ptr(xs), S)
    else:
        raise ValueError(op)
    if r not in (BQ_OK, BQ_UNSUPPORTED):
        raise BqError(r, f"norm_q8({op})")
    return r, q8


# ---------------------------------------------------------------- GGUF
class Gguf:
    """GGUF v3 file opened by libbq's reader (bq_gguf_*)."""

    def __init__(self, path):
        self._h = ctypes.c_void_p()
        _check(load().bq_gguf_open(os.fsencode(path), ctypes.byref(self._h)), f"bq_gguf_open({path})")

    def close(self):
        if self._h:
            load().bq_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __len__(self):
        return load().bq_gguf_n_tensors(self._h)

    def find(self, name):
        return load().bq_gguf_find(self._h, name.encode())

    def tensor(self, i):
        t = GgufTensor()
        _check(load().bq_gguf_tensor_info(self._h, i, ctypes.byref(t)), "bq_gguf_tensor_info")
        return {"name": t.name.decode(errors="replace"), "suffix": t.suffix.decode(errors="replace"), "ne": list(t.ne)[:t.ndim],
                "offset": t.offset, "nbytes": t.nbytes, "type": t.ggml_type, "ndim": t.ndim, "block": t.block}

    def kv_num(self, key):
        v = ctypes.c_double()
        r = load().bq_gguf_kv_num(self._h, key.encode(), ctypes.byref(v))
        return v.value if r == BQ_OK else None

    def kv_str(self, key):
        v = ctypes.c_char_p()
        r = load().bq_gguf_kv_str(self._h, key.encode(), ctypes.byref(v))
        return v.value.decode(errors="replace") if r == BQ_OK else None

    def read(self, i, n=None, off=0):
        import numpy as np
        nb = self.tensor(i)["nbytes"]
        n = nb - off if n is None else n
        out = np.empty(n, np.uint8)
        _check(load().bq_gguf_read(self._h, i, out.ctypes.data_as(ctypes.c_void_p), n, off), "bq_gguf_read")
        return out

    def load(self, i, raw, rep=None, rep_min=None):
        """Stream tensor i into device tensor `raw` (+ repack into rep / rep_min); returns a Weight."""
        w = Weight()
        r = load().bq_gguf_load(self._h, i, _ptr(raw), _ptr(rep), _ptr(rep_min), ctypes.byref(w), _stream())
        if r != BQ_OK:
            raise BqError(r, "bq_gguf_load")
        w._keep = (raw, rep, rep_min)
        return w


# ---------------------------------------------------------------- decode step
def decode_enqueue(step):
    return _check(load().bq_decode_enqueue(ctypes.byref(step), _stream()), "bq_decode_enqueue")


class DecodeGraph:
    """bq_decode_graph: the captured decode step; launch() replays one token."""

    def __init__(self, step):
        self.step = step   # keeps the ctypes structures alive
        h = ctypes.c_void_p()
        _check(load().bq_decode_graph_create(ctypes.byref(step), _stream(), ctypes.byref(h)),
               "bq_decode_graph_create")
        self.h = h

    def launch(self):
        return _check(load().bq_decode_graph_launch(self.h, _stream()), "bq_decode_graph_launch")

    def close(self):
        if self.h:
            load().bq_decode_graph_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
