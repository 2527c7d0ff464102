"""GGUF reader of the library (include/qw6_gguf.h) on files written here.

Three checks pin it:
 - known answers: the writer (qw6_amd.gguf.write_gguf) decides every offset,
   so the parser must report exactly those;
 - qw6's own reader compiled from the reference tree (oracle/_ref): header,
   tensor table, spans, metadata and bind_expert_pack addressing agree on the
   same files, and every corrupt file both reject;
 - the expert-pack rule by its closed form: expert e at
   data_offset + offset + e * rows * row_size.
No device is used: parsing is host code.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

import oracle as O
import qw6_amd as Q
from qw6_amd import gguf as G
from qw6_amd import synth as S

needs_ref = pytest.mark.skipif(O.ref() is None, reason="reference tree not built here")

KV_ALL = [
    ("general.architecture", G.T_STR, "qwen35moe"),
    ("general.name", G.T_STR, "synthetic"),
    ("k.u8", G.T_U8, 200), ("k.i8", G.T_I8, -100), ("k.u16", G.T_U16, 60000),
    ("k.i16", G.T_I16, -30000), ("k.u32", G.T_U32, 4000000000), ("k.i32", G.T_I32, -2000000000),
    ("k.f32", G.T_F32, 1.5e-6), ("k.bool", G.T_BOOL, True), ("k.u64", G.T_U64, 2 ** 63 + 5),
    ("k.i64", G.T_I64, -(2 ** 62)), ("k.f64", G.T_F64, 2.0 ** -30),
    ("k.arr_u32", G.T_ARR, (G.T_U32, list(range(37)))),
    ("k.arr_str", G.T_ARR, (G.T_STR, ["a", "", "tokén", "x" * 300])),
    ("k.arr_f64", G.T_ARR, (G.T_F64, [0.5, -2.0])),
    ("k.empty_arr", G.T_ARR, (G.T_I8, [])),
    ("qwen35moe.expert_count_used", G.T_U32, 8),
    ("k.after_arrays", G.T_I32, 7),
]


_QT = {}


def quant_tensor(q, rows, cols, seed=1, kind=0):
    k = (q, rows, cols, seed, kind)
    if k not in _QT:
        _QT[k] = S.quant_matrix(seed, S.stream_id(0, kind), q, rows, cols)
    return _QT[k]


def mixed_tensors():
    """One tensor of every type the reader sizes, 1-4 dims, odd sizes."""
    rng = np.random.default_rng(3)
    return [
        ("token_embd.weight", G.G_F32, [256, 3], rng.standard_normal(768).astype(np.float32)),
        ("v.f16", G.G_F16, [17], rng.integers(0, 255, 34, dtype=np.uint8)),
        ("v.bf16", G.G_BF16, [5, 3], rng.integers(0, 255, 30, dtype=np.uint8)),
        ("m.q8_0", G.G_Q8_0, [64, 2], rng.integers(0, 255, 136, dtype=np.uint8)),
        ("m.q4k", G.G_Q4_K, [512, 3], quant_tensor(Q.Q_Q4_K_M, 3, 512)),
        ("m.q5k", G.G_Q5_K, [256, 5], quant_tensor(Q.Q_Q5_K, 5, 256)),
        ("m.q6k", G.G_Q6_K, [256, 3, 2], quant_tensor(Q.Q_Q6_K, 6, 256)),
        ("m.iq2xxs", G.G_IQ2_XXS, [256, 1], quant_tensor(Q.Q_IQ2_XXS, 1, 256)),
        ("m.iq2s", G.G_IQ2_S, [256, 2, 1, 2], quant_tensor(Q.Q_IQ2_S, 4, 256)),
        ("m.iq3s", G.G_IQ3_S, [768, 1], quant_tensor(Q.Q_IQ3_S, 1, 768)),
    ]


def pack_tensor(name, q, rows, cols, n=256):
    ex = [quant_tensor(q, rows, cols, seed=5, kind=e % 7) for e in range(n)]
    return (name, G.GGML_OF_QUANT[q], [cols, rows, n], b"".join(e.tobytes() for e in ex))


def check_known_answers(path, kv, tensors, info, alignment):
    with G.GgufFile(path) as f:
        h = f.header()
        assert h["version"] == 3 and h["n_kv"] == len(kv) + (alignment != 32)
        assert h["n_tensors"] == len(tensors) and h["data_offset"] == info["data_offset"]
        assert h["data_offset"] % alignment == 0
        size = h["file_size"]
        for i, ((name, t, dims, data), off) in enumerate(zip(tensors, info["offsets"])):
            d = f.tensor(i)
            assert (d["name"], d["type"], d["dims"], d["offset"]) == (name, t, dims, off)
            nxt = info["offsets"][i + 1] + info["data_offset"] if i + 1 < len(tensors) else size
            assert d["span"] == nxt - (off + info["data_offset"])
            assert f.find(name) == i
        assert f.find("no.such.tensor") == -1
        for key, t, v in kv:
            assert f.kv_type(key) == t
            if t in (G.T_F32, G.T_F64):
                assert f.kv_float(key) == pytest.approx(v, rel=1e-7)
            elif t == G.T_STR:
                assert f.kv_str(key) == v
            elif t != G.T_ARR:
                iv = f.kv_int(key)
                assert iv == (v if t != G.T_U64 else v - 2 ** 64 if v >= 2 ** 63 else v)
        assert f.kv_type("missing.key") == -1 and f.kv_int("missing.key") is None
        assert f.kv_int("general.name") is None and f.kv_str("k.u32") is None


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_parser_known_answers(tmp_path, alignment):
    tensors = mixed_tensors()
    p = tmp_path / "mixed.gguf"
    info = G.write_gguf(p, KV_ALL, tensors, alignment=alignment)
    check_known_answers(p, KV_ALL, tensors, info, alignment)


def test_tensor_data_round_trip(tmp_path):
    """The bytes at data_offset + offset are the tensor's bytes."""
    tensors = mixed_tensors()
    p = tmp_path / "rt.gguf"
    G.write_gguf(p, KV_ALL, tensors)
    raw = p.read_bytes()
    with G.GgufFile(p) as f:
        base = f.header()["data_offset"]
        for i, (_, t, dims, data) in enumerate(tensors):
            d = f.tensor(i)
            n = G.tensor_bytes(t, dims)
            got = np.frombuffer(raw[base + d["offset"]: base + d["offset"] + n], np.uint8)
            assert np.array_equal(got, np.frombuffer(np.ascontiguousarray(data).tobytes(), np.uint8))


@pytest.mark.parametrize("q,rows,cols", [(Q.Q_Q4_K_M, 16, 512), (Q.Q_Q5_K, 8, 256),
                                          (Q.Q_Q6_K, 16, 256), (Q.Q_IQ2_XXS, 8, 512),
                                          (Q.Q_IQ2_S, 4, 256), (Q.Q_IQ3_S, 8, 256)])
def test_expert_pack_closed_form(tmp_path, q, rows, cols):
    tensors = [("blk.0.ffn_gate_inp.weight", G.G_F32, [cols, 256],
                np.zeros(256 * cols, np.float32)), pack_tensor("blk.0.ffn_up_exps.weight", q, rows, cols)]
    p = tmp_path / "pack.gguf"
    info = G.write_gguf(p, KV_ALL, tensors)
    with G.GgufFile(p) as f:
        pk = f.expert_pack(1)
        assert (pk["quant"], pk["rows"], pk["cols"]) == (q, rows, cols)
        assert pk["file_offset"] == info["data_offset"] + info["offsets"][1]
        assert pk["expert_bytes"] == rows * S.row_bytes(q, cols)
        with pytest.raises(Q.Qw6HipError, match=r"is not \[cols, rows, "):
            f.expert_pack(1, n_experts=255)
        with pytest.raises(Q.Qw6HipError, match=r"is not \[cols, rows, "):
            f.expert_pack(0)
    if O.ref() is not None:
        r = O.ref_gguf_pack(p, 1)
        assert r is not None and (r["quant"], r["rows"], r["cols"]) == (q, rows, cols)
        assert r["offsets"] == [pk["file_offset"] + e * pk["expert_bytes"] for e in range(256)]
        assert r["sizes"] == [pk["expert_bytes"]] * 256
        assert O.ref_gguf_pack(p, 0) is None


# ---- qw6's reader on the same files ------------------------------------------------

def assert_same_as_reference(p):
    rh = O.ref_gguf_header(p)
    assert rh is not None
    with G.GgufFile(p) as f:
        assert f.header() == rh
        for i in range(rh["n_tensors"]):
            assert f.tensor(i) == O.ref_gguf_tensor(p, i)
        for key, t, v in KV_ALL + [("general.alignment", G.T_U32, 0)]:
            r = O.ref_gguf_kv(p, key)
            if r is None:
                assert f.kv_type(key) == -1
                continue
            rt, ri, rf, rs = r
            assert f.kv_type(key) == rt
            if rt in (G.T_F32, G.T_F64):
                assert f.kv_float(key) == rf
            elif rt == G.T_STR:
                assert f.kv_str(key) == rs
            elif rt != G.T_ARR:
                assert f.kv_int(key) == ri
    assert O.ref_gguf_valid(p)


@needs_ref
@pytest.mark.parametrize("alignment", [32, 64, 4096])
def test_parser_matches_reference(tmp_path, alignment):
    p = tmp_path / "m.gguf"
    G.write_gguf(p, KV_ALL, mixed_tensors(), alignment=alignment)
    assert_same_as_reference(p)


@needs_ref
def test_alignment_key_forms_match_reference(tmp_path):
    """general.alignment honoured only as UINT32; 0 keeps the default 32 for
    the data offset but is reported as 0; the last of two keys wins."""
    tensors = mixed_tensors()[:2]
    for extra in ([("general.alignment", G.T_U64, 64)], [("general.alignment", G.T_U32, 0)],
                  [("general.alignment", G.T_U32, 128), ("general.alignment", G.T_U32, 16)]):
        p = tmp_path / "al.gguf"
        meta = G.encode_meta(KV_ALL + extra, [(n, d, t, 0 if i == 0 else 3072)
                                              for i, (n, t, d, _) in enumerate(tensors)])
        p.write_bytes(meta + b"\0" * (4096 + 8192))
        assert_same_as_reference(p)


@needs_ref
def test_long_names_and_keys_truncate_like_reference(tmp_path):
    long_key, long_name = "k." + "z" * 200, "blk.0." + "n" * 200
    kv = KV_ALL + [(long_key, G.T_U32, 11)]
    t = [(long_name, G.G_F32, [4], np.ones(4, np.float32))]
    p = tmp_path / "long.gguf"
    G.write_gguf(p, kv, t)
    with G.GgufFile(p) as f:
        d = f.tensor(0)
        assert d == O.ref_gguf_tensor(p, 0) and len(d["name"]) == 127
        assert f.kv_int(long_key[:127]) == 11 == O.ref_gguf_kv(p, long_key[:127])[1]
        assert f.kv_type(long_key) == -1 and O.ref_gguf_kv(p, long_key) is None
        assert f.find(long_name[:127]) == 0


@needs_ref
@pytest.mark.parametrize("q", [Q.Q_Q4_K_M, Q.Q_Q5_K, Q.Q_Q6_K, Q.Q_IQ2_XXS, Q.Q_IQ2_S, Q.Q_IQ3_S])
def test_expert_pack_matches_reference(tmp_path, q):
    """A cfg-shaped layer file (256 experts): every pack's addressing equals
    bind_expert_pack's."""
    router = np.zeros(256 * 512, np.float32)
    packs = [(q, [quant_tensor(q, 256, 512, kind=e % 3) for e in range(256)])] * 2 + \
            [(q, [quant_tensor(q, 512, 256, kind=e % 3) for e in range(256)])]
    p = tmp_path / "layer.gguf"
    G.write_gguf(p, KV_ALL, G.moe_layer_tensors(3, 512, 256, router, packs))
    assert_same_as_reference(p)
    with G.GgufFile(p) as f:
        for nm in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"):
            i = f.find("blk.3.%s.weight" % nm)
            pk, r = f.expert_pack(i), O.ref_gguf_pack(p, i)
            assert (pk["quant"], pk["rows"], pk["cols"]) == (r["quant"], r["rows"], r["cols"])
            assert r["offsets"] == [pk["file_offset"] + e * pk["expert_bytes"] for e in range(256)]


@needs_ref
def test_pack_errors_match_reference(tmp_path):
    """Packs qw6 refuses: 255 experts, a Q8_0 pack (no row size), a span cut
    short by the next tensor's start."""
    good = pack_tensor("blk.0.ffn_gate_exps.weight", Q.Q_Q4_K_M, 2, 256)
    cases = {
        "n255": [("blk.0.ffn_gate_exps.weight", G.G_Q4_K, [256, 2, 255],
                  b"\1" * (144 * 2 * 255))],
        "q8_0": [("blk.0.ffn_gate_exps.weight", G.G_Q8_0, [256, 2, 256],
                  b"\1" * (34 * 8 * 2 * 256))],
    }
    for name, t in cases.items():
        p = tmp_path / (name + ".gguf")
        G.write_gguf(p, KV_ALL, t)
        assert O.ref_gguf_valid(p)
        with G.GgufFile(p) as f:
            with pytest.raises(Q.Qw6HipError):
                f.expert_pack(0)
        assert O.ref_gguf_pack(p, 0) is None
    # a second tensor placed inside the pack's range shortens its span
    p = tmp_path / "short.gguf"
    n = len(good[3])
    meta = G.encode_meta(KV_ALL, [(good[0], good[2], good[1], 0), ("x", [4], G.G_F32, n - 32)])
    data_off = (len(meta) + 31) // 32 * 32
    p.write_bytes(meta + b"\0" * (data_off - len(meta)) + good[3])
    assert O.ref_gguf_valid(p)
    with G.GgufFile(p) as f:
        assert f.tensor(0)["span"] == n - 32 == O.ref_gguf_tensor(p, 0)["span"]
        with pytest.raises(Q.Qw6HipError, match="span"):
            f.expert_pack(0)
    assert O.ref_gguf_pack(p, 0) is None


def corrupt_files():
    """(name, bytes): files qw6's reader rejects at parse or range check."""
    t = [("w", G.G_Q4_K, [256, 2], quant_tensor(Q.Q_Q4_K_M, 2, 256))]
    good = G.encode_meta(KV_ALL, [("w", [256, 2], G.G_Q4_K, 0)])
    data_off = (len(good) + 31) // 32 * 32
    body = good + b"\0" * (data_off - len(good)) + t[0][3].tobytes()
    hdr = struct.calcsize("<IIQQ")
    one_kv = struct.pack("<IIQQ", G.MAGIC, 3, 0, 1)   # no tensors, one pair
    pad = b"\0" * 64
    out = [
        ("magic", b"GGUX" + body[4:]),
        ("version2", body[:4] + struct.pack("<I", 2) + body[8:]),
        ("truncated_meta", body[:len(good) // 2]),
        ("truncated_data", body[:-1]),
        ("header_only", body[:hdr - 3]),
        ("empty", b""),
        ("too_many_tensors", G.encode_meta([], [], n_tensors=4097)),
        ("too_many_kv", G.encode_meta([], [], n_kv=513)),
        ("dims5", G.encode_meta([], [("w", [1, 1, 1, 1, 1], G.G_F32, 0)]) + b"\0" * 64),
        ("kv_type13", one_kv + G._str("k") + struct.pack("<i", 13) + pad),
        ("kv_type_negative", one_kv + G._str("k") + struct.pack("<i", -1) + pad),
        ("array_of_arrays", one_kv + G._str("k") + struct.pack("<iiQ", G.T_ARR, G.T_ARR, 1) + pad),
        ("array_type13", one_kv + G._str("k") + struct.pack("<iiQ", G.T_ARR, 13, 0) + pad),
        ("array_too_long", one_kv + G._str("k") +
         struct.pack("<iiQ", G.T_ARR, G.T_U8, 10 * 2 ** 20 + 1) + pad),
        ("string_too_long", one_kv + G._str("k") + struct.pack("<iQ", G.T_STR, 2 ** 20 + 1) + pad),
        ("key_too_long", struct.pack("<IIQQQ", G.MAGIC, 3, 0, 1, 2 ** 20 + 1) + pad),
    ]
    # tensors qw6 cannot size or place
    bad_t = {
        "type_q4_0": [("w", [256], G.G_Q4_0, 0)],
        "ne0_not_block": [("w", [100, 2], G.G_Q4_K, 0)],
        "negative_dim": [("w", [256, -1], G.G_Q4_K, 0)],
        "zero_dim": [("w", [256, 0], G.G_Q4_K, 0)],
        "no_dims": [("w", [], G.G_F32, 0)],
        "past_end": [("w", [256], G.G_F32, 1 << 20)],
        "offset_overflow": [("w", [256], G.G_F32, 2 ** 64 - 16)],
    }
    for name, infos in bad_t.items():
        m = G.encode_meta(KV_ALL, infos)
        out.append((name, m + b"\0" * (4096 + (32 - len(m) % 32))))
    return out


@pytest.mark.parametrize("name,blob", corrupt_files(), ids=[c[0] for c in corrupt_files()])
def test_corrupt_files_rejected(tmp_path, name, blob):
    p = tmp_path / (name + ".gguf")
    p.write_bytes(blob)
    with pytest.raises(Q.Qw6HipError):
        G.GgufFile(p)
    if O.ref() is not None:
        assert not O.ref_gguf_valid(p), name


def test_missing_file_rejected(tmp_path):
    with pytest.raises(Q.Qw6HipError, match="cannot open"):
        G.GgufFile(tmp_path / "nope.gguf")


def test_zero_tensor_file(tmp_path):
    p = tmp_path / "z.gguf"
    G.write_gguf(p, KV_ALL, [])
    with G.GgufFile(p) as f:
        h = f.header()
        assert h["n_tensors"] == 0 and h["data_offset"] == h["file_size"]
        assert f.find("w") == -1
        with pytest.raises(Q.Qw6HipError, match="out of range"):
            f.tensor(0)
    if O.ref() is not None:
        assert O.ref_gguf_header(p) == h and O.ref_gguf_valid(p)
