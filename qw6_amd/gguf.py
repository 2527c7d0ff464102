"""GGUF v3 files: a writer for synthetic models, and the library's reader.

`GgufFile` wraps include/qw6_gguf.h: parse a file (qw6_gguf_parse,
qw6.c:871-1075, with its range checks, qw6.c:410-457), look up metadata and
tensors, read expert-pack addressing (bind_expert_pack, qw6.c:542-597), and
make tensors or a whole MoE layer resident on a device.

`write_gguf` writes the same format from Python values: the synthetic layers
of qw6_amd.synth as model files, for the loader's tests and for users without
a model file at hand. Tensor data is placed at offsets rounded up to the
file's alignment, as GGUF writers do.
"""
from __future__ import annotations

import ctypes as C
import struct
from pathlib import Path

import numpy as np

from . import Experts, Matrix, MoeLayer, Qw6HipError, _check, lib

# gguf_type_t (qw6.h:328-342)
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
           T_F32: "<f", T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}

# ggml_type_t (qw6.h:345-380), the types qw6 reads
G_F32, G_F16, G_Q4_0, G_Q8_0, G_Q4_K, G_Q5_K, G_Q6_K = 0, 1, 2, 8, 12, 13, 14
G_IQ2_XXS, G_IQ3_S, G_IQ2_S, G_BF16 = 16, 21, 22, 30
# qw6_quant_t -> ggml type of a tensor holding it
GGML_OF_QUANT = {0: G_F32, 4: G_Q4_K, 5: G_Q4_K, 6: G_Q5_K, 7: G_Q6_K, 9: G_IQ3_S,
                 11: G_IQ2_S, 13: G_IQ2_XXS}
MAGIC = 0x46554747


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def encode_value(t: int, v) -> bytes:
    """One metadata value of gguf type t (arrays: v = (elem_type, items))."""
    if t == T_STR:
        return _str(v)
    if t == T_ARR:
        et, items = v
        out = struct.pack("<iQ", et, len(items))
        return out + b"".join(encode_value(et, x) for x in items)
    return struct.pack(_SCALAR[t], v)


def encode_meta(kv, infos, version: int = 3, n_tensors: int | None = None,
                n_kv: int | None = None) -> bytes:
    """Header, key/value pairs and tensor table. kv: (key, type, value);
    infos: (name, dims (ne0 first), ggml type, offset in the data section)."""
    out = [struct.pack("<IIQQ", MAGIC, version, len(infos) if n_tensors is None else n_tensors,
                       len(kv) if n_kv is None else n_kv)]
    for key, t, v in kv:
        out.append(_str(key) + struct.pack("<i", t) + encode_value(t, v))
    for name, dims, t, off in infos:
        out.append(_str(name) + struct.pack("<I", len(dims)) +
                   b"".join(struct.pack("<q", d) for d in dims) + struct.pack("<iQ", t, off))
    return b"".join(out)


def tensor_bytes(ggml_type: int, dims) -> int:
    """Bytes of a tensor (ggml_type_block_elems / _bytes, qw6.c:353-383)."""
    be = {G_Q8_0: 32, G_Q4_K: 256, G_Q5_K: 256, G_Q6_K: 256, G_IQ2_XXS: 256, G_IQ2_S: 256,
          G_IQ3_S: 256}.get(ggml_type, 1)
    bb = {G_F32: 4, G_F16: 2, G_BF16: 2, G_Q8_0: 34, G_Q4_K: 144, G_Q5_K: 176, G_Q6_K: 210,
          G_IQ2_XXS: 66, G_IQ2_S: 82, G_IQ3_S: 110}[ggml_type]
    rows = int(np.prod(dims[1:], dtype=np.int64)) if len(dims) > 1 else 1
    return rows * (dims[0] // be) * bb


def write_gguf(path, kv, tensors, alignment: int = 32) -> dict:
    """Write a GGUF v3 file. tensors: (name, ggml type, dims (ne0 first),
    data as bytes / uint8 array). general.alignment is written when
    alignment != 32. Returns the data offset and each tensor's offset."""
    kv = list(kv)
    if alignment != 32:
        kv.append(("general.alignment", T_U32, alignment))
    offs, pos = [], 0
    for name, t, dims, data in tensors:
        n = data.nbytes if isinstance(data, np.ndarray) else len(data)
        if n != tensor_bytes(t, dims):
            raise ValueError("%s: %d bytes for dims %s type %d" % (name, n, dims, t))
        pos = (pos + alignment - 1) // alignment * alignment
        offs.append(pos)
        pos += n
    meta = encode_meta(kv, [(nm, d, t, o) for (nm, t, d, _), o in zip(tensors, offs)])
    data_off = (len(meta) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(meta)
        f.write(b"\0" * (data_off - len(meta)))
        for (name, t, dims, data), o in zip(tensors, offs):
            here = f.tell() - data_off
            f.write(b"\0" * (o - here))
            f.write(data if isinstance(data, (bytes, bytearray)) else np.ascontiguousarray(data).tobytes())
    return {"data_offset": data_off, "offsets": offs}


def moe_layer_tensors(layer: int, hidden: int, inter: int, router: np.ndarray, packs,
                      shared=None, shared_router: np.ndarray | None = None,
                      norm_w: np.ndarray | None = None):
    """Tensor entries of one MoE block under qw6's names (bind_layer_tensor,
    qw6.c:599-677). packs: (quant, [per-expert bytes]) for gate, up, down --
    one quant per pack, experts concatenated as a GGUF expert pack; shared:
    ((bytes, quant) x 3) or None."""
    n_exp = router.size // hidden
    p = "blk.%d." % layer
    out = [(p + "ffn_gate_inp.weight", G_F32, [hidden, n_exp], router.astype(np.float32).tobytes())]
    shapes = ([hidden, inter], [hidden, inter], [inter, hidden])
    for nm, (q, ex), shp in zip(("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"), packs, shapes):
        out.append((p + nm + ".weight", GGML_OF_QUANT[q], shp + [n_exp],
                    b"".join(np.asarray(e, np.uint8).tobytes() for e in ex)))
    if shared is not None:
        for nm, (b, q), shp in zip(("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp"), shared,
                                   shapes):
            out.append((p + nm + ".weight", GGML_OF_QUANT[q], shp, np.asarray(b, np.uint8).tobytes()))
    if shared_router is not None:
        out.append((p + "ffn_gate_inp_shexp.weight", G_F32, [hidden],
                    shared_router.astype(np.float32).tobytes()))
    if norm_w is not None:
        out.append((p + "post_attention_norm.weight", G_F32, [hidden],
                    norm_w.astype(np.float32).tobytes()))
    return out


_setup = False


def _lib():
    global _setup
    L = lib()
    if not _setup:
        vp, u32p, u64p, i64p = C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(C.c_int64)
        L.qw6_hip_gguf_open.argtypes = [C.c_char_p, C.POINTER(vp)]
        L.qw6_hip_gguf_close.argtypes = [vp]
        L.qw6_hip_gguf_close.restype = None
        L.qw6_hip_gguf_header.argtypes = [vp, u32p, u32p, u32p, u32p, u64p, u64p]
        L.qw6_hip_gguf_tensor.argtypes = [vp, C.c_uint32, C.c_char_p, u32p, i64p,
                                          C.POINTER(C.c_int32), u64p, u64p]
        L.qw6_hip_gguf_find_tensor.argtypes = [vp, C.c_char_p]
        L.qw6_hip_gguf_kv_type.argtypes = [vp, C.c_char_p]
        L.qw6_hip_gguf_kv_type.restype = C.c_int32
        L.qw6_hip_gguf_kv_int.argtypes = [vp, C.c_char_p, i64p]
        L.qw6_hip_gguf_kv_float.argtypes = [vp, C.c_char_p, C.POINTER(C.c_double)]
        L.qw6_hip_gguf_kv_str.argtypes = [vp, C.c_char_p, C.c_char_p, C.c_size_t]
        L.qw6_hip_gguf_expert_pack.argtypes = [vp, C.c_uint32, C.c_uint32, C.POINTER(C.c_int32),
                                               u32p, u32p, u64p, u64p]
        L.qw6_hip_gguf_upload.argtypes = [vp, vp, C.c_uint32, C.POINTER(Matrix)]
        L.qw6_hip_gguf_moe_layer.argtypes = [vp, vp, C.c_uint32, C.POINTER(MoeLayer),
                                             C.POINTER(vp)]
        _setup = True
    return L


class GgufFile:
    """An open GGUF file (qw6_hip_gguf_t)."""

    def __init__(self, path):
        h = C.c_void_p()
        _check(_lib().qw6_hip_gguf_open(str(Path(path)).encode(), C.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            _lib().qw6_hip_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def header(self) -> dict:
        v, nt, nkv, al = (C.c_uint32() for _ in range(4))
        do, fs = C.c_uint64(), C.c_uint64()
        _check(_lib().qw6_hip_gguf_header(self.handle, C.byref(v), C.byref(nt), C.byref(nkv),
                                          C.byref(al), C.byref(do), C.byref(fs)))
        return {"version": v.value, "n_tensors": nt.value, "n_kv": nkv.value,
                "alignment": al.value, "data_offset": do.value, "file_size": fs.value}

    def tensor(self, i: int) -> dict:
        name = C.create_string_buffer(128)
        nd, t = C.c_uint32(), C.c_int32()
        dims = (C.c_int64 * 4)()
        off, span = C.c_uint64(), C.c_uint64()
        _check(_lib().qw6_hip_gguf_tensor(self.handle, i, name, C.byref(nd), dims, C.byref(t),
                                          C.byref(off), C.byref(span)))
        return {"name": name.value.decode(errors="replace"), "dims": list(dims[:nd.value]),
                "type": t.value, "offset": off.value, "span": span.value}

    def tensors(self) -> list:
        return [self.tensor(i) for i in range(self.header()["n_tensors"])]

    def find(self, name: str) -> int:
        return _lib().qw6_hip_gguf_find_tensor(self.handle, name.encode())

    def kv_type(self, key: str) -> int:
        return _lib().qw6_hip_gguf_kv_type(self.handle, key.encode())

    def kv_int(self, key: str):
        v = C.c_int64()
        return v.value if _lib().qw6_hip_gguf_kv_int(self.handle, key.encode(), C.byref(v)) == 0 else None

    def kv_float(self, key: str):
        v = C.c_double()
        return v.value if _lib().qw6_hip_gguf_kv_float(self.handle, key.encode(), C.byref(v)) == 0 else None

    def kv_str(self, key: str, cap: int = 1 << 20):
        b = C.create_string_buffer(cap)
        return b.value.decode(errors="replace") if _lib().qw6_hip_gguf_kv_str(
            self.handle, key.encode(), b, cap) == 0 else None

    def expert_pack(self, i: int, n_experts: int = 0) -> dict:
        q = C.c_int32()
        r, c = C.c_uint32(), C.c_uint32()
        fo, eb = C.c_uint64(), C.c_uint64()
        _check(_lib().qw6_hip_gguf_expert_pack(self.handle, i, n_experts, C.byref(q), C.byref(r),
                                               C.byref(c), C.byref(fo), C.byref(eb)))
        return {"quant": q.value, "rows": r.value, "cols": c.value, "file_offset": fo.value,
                "expert_bytes": eb.value}

    def upload(self, ctx, i: int) -> tuple:
        """Tensor i on ctx's device: (address, quant, rows, cols)."""
        m = Matrix()
        _check(_lib().qw6_hip_gguf_upload(ctx.handle, self.handle, i, C.byref(m)))
        return (m.data, m.quant, m.rows, m.cols)

    def moe_layer(self, ctx, layer: int):
        """(MoeLayer descriptor, Experts) of blk.<layer>, resident on ctx."""
        d = MoeLayer()
        h = C.c_void_p()
        _check(_lib().qw6_hip_gguf_moe_layer(ctx.handle, self.handle, layer, C.byref(d),
                                             C.byref(h)))
        E = Experts.__new__(Experts)
        E.handle, E.n = h, None
        return d, E


__all__ = ["GgufFile", "write_gguf", "encode_meta", "encode_value", "moe_layer_tensors",
           "tensor_bytes", "Qw6HipError"]
