"""CPU checks of libbq's GGUF v3 reader (bq_gguf_*; engine/src/gguf.h:146-346)
against files written by tests/gguf_writer.py: metadata of every value type,
the tensor table (types, dims, absolute offsets, byte sizes, blk.N names), the
alignment rule, byte reads, and the malformed files the reader must reject."""
import struct

import numpy as np
import pytest

import gguf_writer as W

KV = [
    ("general.architecture", W.T_STR, "bruce"),
    ("general.alignment", W.T_U32, 64),
    ("u8", W.T_U8, 200), ("i8", W.T_I8, -100), ("u16", W.T_U16, 60000), ("i16", W.T_I16, -30000),
    ("u32", W.T_U32, 4000000000), ("i32", W.T_I32, -2000000000), ("f32", W.T_F32, 1.5),
    ("bool", W.T_BOOL, 1), ("u64", W.T_U64, 2 ** 40), ("i64", W.T_I64, -(2 ** 40)), ("f64", W.T_F64, -2.25),
    ("tokens", W.T_ARR, (W.T_STR, ["a", "bb", ""])),
    ("scores", W.T_ARR, (W.T_F32, [0.5, -1.0])),
    ("ids", W.T_ARR, (W.T_I64, [1, 2, 3])),
]


def make_file(tmp_path, kv=KV):
    q5 = W.random_kquant(1, 16, 512, 176)
    q6 = W.random_kquant(2, 8, 768, 210)
    bf = np.arange(4 * 256, dtype=np.uint16).reshape(4, 256)
    f32 = np.linspace(-1, 1, 100).astype(np.float32)
    tensors = [("blk.0.ffn_gate.weight", 13, (512, 16), q5.tobytes()),
               ("blk.12.ffn_down.weight", 14, (768, 8), q6.tobytes()),
               ("output.weight", 30, (256, 4), bf.tobytes()),
               ("output_norm.weight", 0, (100,), f32.tobytes())]
    path = str(tmp_path / "t.gguf")
    data_off = W.write_gguf(path, kv, tensors, alignment=64)
    return path, data_off, tensors


def test_gguf_metadata_and_table(tmp_path):
    import bq
    path, data_off, tensors = make_file(tmp_path)
    with bq.Gguf(path) as g:
        assert len(g) == 4
        assert g.kv_str("general.architecture") == "bruce"
        expect = {"u8": 200, "i8": -100, "u16": 60000, "i16": -30000, "u32": 4000000000, "i32": -2000000000,
                  "f32": 1.5, "bool": 1, "u64": 2 ** 40, "i64": -(2 ** 40), "f64": -2.25, "general.alignment": 64}
        for k, v in expect.items():
            assert g.kv_num(k) == v, k
        assert g.kv_num("tokens") is None and g.kv_str("u8") is None and g.kv_num("missing") is None
        off = data_off
        for i, (name, gt, ne, payload) in enumerate(tensors):
            t = g.tensor(i)
            assert g.find(name) == i
            assert t["name"] == name and t["type"] == gt and t["ne"] == list(ne) and t["ndim"] == len(ne)
            assert t["nbytes"] == len(payload) and t["offset"] == off and t["offset"] % 64 == 0
            off += (len(payload) + 63) // 64 * 64
            assert g.read(i).tobytes() == payload
            assert g.read(i, 10, 5).tobytes() == payload[5:15]
        assert g.tensor(0)["block"] == 0 and g.tensor(0)["suffix"] == "ffn_gate.weight"
        assert g.tensor(1)["block"] == 12 and g.tensor(1)["suffix"] == "ffn_down.weight"
        assert g.tensor(2)["block"] == -1 and g.tensor(2)["suffix"] == ""
        assert g.find("nope") == -1
        with pytest.raises(bq.BqError):
            g.read(0, 10, len(tensors[0][3]) - 5)          # past the tensor's end


def test_gguf_default_alignment_and_big_header(tmp_path):
    """No general.alignment -> 32; a header larger than the reader's first
    prefix (1 MiB of string array) is still parsed."""
    import bq
    big = [("vocab", W.T_ARR, (W.T_STR, ["tok%06d" % i for i in range(120000)]))]
    q5 = W.random_kquant(3, 4, 256, 176)
    path = str(tmp_path / "b.gguf")
    data_off = W.write_gguf(path, big, [("w", 13, (256, 4), q5.tobytes())])
    assert data_off > (1 << 20) and data_off % 32 == 0
    with bq.Gguf(path) as g:
        t = g.tensor(0)
        assert t["offset"] == data_off and g.read(0).tobytes() == q5.tobytes()


@pytest.mark.parametrize("case", ["magic", "version", "truncated", "kvtype", "ttype", "past_end", "ndim"])
def test_gguf_rejects(tmp_path, case):
    import bq
    q5 = W.random_kquant(4, 2, 256, 176).tobytes()
    kv = [("a", W.T_U32, 1)]
    tensors = [("w", 13, (256, 2), q5)]
    if case == "magic":
        blob, _ = W.gguf_bytes(kv, tensors, magic=0x12345678)
    elif case == "version":
        blob, _ = W.gguf_bytes(kv, tensors, version=2)
    elif case == "truncated":
        blob = W.gguf_bytes(kv, tensors)[0][:30]
    elif case == "kvtype":
        blob, _ = W.gguf_bytes([], tensors)     # n_kv = 0; splice in one pair of value type 99
        blob = blob[:16] + struct.pack("<Q", 1) + W._str("k") + struct.pack("<I", 99) + blob[24:]
    elif case == "ttype":
        blob, _ = W.gguf_bytes(kv, [("w", 77, (256, 2), q5)])
    elif case == "past_end":
        blob = W.gguf_bytes(kv, tensors)[0][:-100]
    else:
        blob, _ = W.gguf_bytes(kv, [("w", 13, (256, 2, 1, 1, 1), q5)])
    path = tmp_path / "bad.gguf"
    path.write_bytes(blob)
    with pytest.raises(bq.BqError):
        bq.Gguf(str(path))
    with pytest.raises(bq.BqError):
        bq.Gguf(str(tmp_path / "missing.gguf"))


def test_gguf_hand_laid_file(tmp_path):
    """A file laid out by hand, field by field from the GGUF v3 layout, not by
    gguf_writer: the tensor table lists A then B, but B's data comes first in
    the data section and A's starts after a 96-byte gap (offsets are free in
    GGUF as long as each is a multiple of general.alignment, here 32).  The
    reader must take every offset from the table, not from the order."""
    import bq
    rng = np.random.default_rng(11)
    a = W.random_kquant(12, 2, 256, 176).tobytes()      # Q5_K 256 x 2: 352 B
    b = rng.integers(0, 256, size=96, dtype=np.uint8).tobytes()   # F16, 48 values
    off_b, off_a = 0, 96 + 96                             # B first, then a gap of 96 B
    hdr = b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", 2) + struct.pack("<Q", 1)
    key = b"general.alignment"
    hdr += struct.pack("<Q", len(key)) + key + struct.pack("<I", 4) + struct.pack("<I", 32)   # u32 KV
    for name, ne, gtype, off in ((b"blk.3.attn_q.weight", (256, 2), 13, off_a), (b"tok", (48,), 1, off_b)):
        hdr += struct.pack("<Q", len(name)) + name + struct.pack("<I", len(ne))
        hdr += b"".join(struct.pack("<Q", n) for n in ne) + struct.pack("<I", gtype) + struct.pack("<Q", off)
    data_start = (len(hdr) + 31) // 32 * 32
    blob = bytearray(hdr + b"\x00" * (data_start - len(hdr)))
    data = bytearray(off_a + len(a))
    data[off_b:off_b + len(b)] = b
    data[off_b + len(b):off_a] = b"\xee" * (off_a - off_b - len(b))   # gap: must never be returned
    data[off_a:off_a + len(a)] = a
    blob += data
    path = tmp_path / "hand.gguf"
    path.write_bytes(bytes(blob))
    with bq.Gguf(str(path)) as g:
        assert len(g) == 2 and g.kv_num("general.alignment") == 32
        ta, tb = g.tensor(0), g.tensor(1)
        assert ta["offset"] == data_start + off_a and tb["offset"] == data_start + off_b
        assert ta["nbytes"] == 352 and tb["nbytes"] == 96
        assert ta["block"] == 3 and ta["suffix"] == "attn_q.weight"
        assert g.read(0).tobytes() == a and g.read(1).tobytes() == b


def test_gguf_mutated_files_never_crash(tmp_path):
    """Seeded mutations of a valid file (byte flips, truncations, huge counts,
    lengths and offsets, unknown type ids in the header): every open either
    parses or raises BqError, and reads stay inside the file.  (An
    AddressSanitizer build of the host code ran 11,000 such files clean.)"""
    import random
    import bq
    kv = [("general.architecture", W.T_STR, "x"), ("general.alignment", W.T_U32, 64),
          ("arr", W.T_ARR, (W.T_STR, ["a", "bb"])), ("f", W.T_ARR, (W.T_F32, [1.0, 2.0]))]
    q5 = W.random_kquant(21, 4, 512, 176)
    tensors = [("blk.0.a", 13, (512, 4), q5.tobytes()), ("b", 0, (10,), np.zeros(10, np.float32).tobytes())]
    base, _ = W.gguf_bytes(kv, tensors, alignment=64)
    rng = random.Random(5)
    path = tmp_path / "m.gguf"
    parsed = 0
    for _ in range(400):
        b = bytearray(base)
        kind = rng.randrange(4)
        if kind == 0:
            for _ in range(rng.randrange(1, 8)):
                b[rng.randrange(400)] = rng.randrange(256)
        elif kind == 1:
            b = b[:rng.randrange(len(b))]
        elif kind == 2:
            pos = rng.randrange(392)
            b[pos:pos + 8] = struct.pack("<Q", rng.choice([0, 1, 2 ** 31, 2 ** 63, 2 ** 64 - 1, rng.randrange(2 ** 64)]))
        else:
            pos = rng.randrange(396)
            b[pos:pos + 4] = struct.pack("<I", rng.choice([0, 4, 9, 12, 13, 99, 2 ** 31, 2 ** 32 - 1]))
        path.write_bytes(bytes(b))
        try:
            with bq.Gguf(str(path)) as g:
                for i in range(len(g)):
                    t = g.tensor(i)
                    assert t["offset"] + t["nbytes"] <= len(b)
                    g.read(i, min(t["nbytes"], 64), 0)
            parsed += 1
        except bq.BqError:
            pass
    assert 0 < parsed < 400
