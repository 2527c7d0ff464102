"""ctypes bindings for the oracle (test infrastructure only).

The oracle is the CPU reference the HIP library is compared against: tests,
the smoke check and the CPU-baseline leg of bench.py call it to compute
expected results. The
product never imports this package.

``lib()`` loads the repository's C restatement of qw6's CPU path
(libqw6oracle.so); ``ref()`` loads qw6's own CPU path compiled from the
reference tree (oracle/_ref/libqw6ref.so) when that was built, else None.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "libqw6oracle.so"
REF_SO = HERE / "_ref" / "libqw6ref.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


class OrcMat(C.Structure):
    _fields_ = [("data", C.c_void_p), ("quant", C.c_int32),
                ("rows", C.c_uint32), ("cols", C.c_uint32)]


def build(force: bool = False) -> None:
    if force or not ORACLE_SO.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            build()
        L = C.CDLL(str(ORACLE_SO))
        L.orc_fp16_to_f32.restype = C.c_float
        L.orc_fp16_to_f32.argtypes = [C.c_uint16]
        L.orc_dequant_row.argtypes = [C.c_int, C.c_void_p, C.c_uint32, C.c_uint32, _f32p]
        L.orc_matvec.argtypes = [_f32p, C.POINTER(OrcMat), _f32p, C.c_uint32, C.c_int]
        L.orc_moe_route.argtypes = [_i32p, _f32p, _f32p, C.c_int, C.c_int]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_float]
        L.orc_argmax.restype = C.c_int
        L.orc_argmax.argtypes = [_f32p, C.c_int]
        L.orc_silu.restype = C.c_float
        L.orc_silu.argtypes = [C.c_float]
        L.orc_silu_mul.argtypes = [_f32p, _f32p, _f32p, C.c_uint32]
        L.orc_moe_gather.argtypes = [_f32p, _f32p, C.c_void_p, C.c_float, _f32p,
                                     C.c_uint32, C.c_uint32]
        L.orc_moe_layer.argtypes = [_f32p, _i32p, _f32p, C.c_void_p, C.c_void_p,
                                    C.POINTER(OrcMat), C.c_void_p, C.c_void_p, _f32p,
                                    C.c_uint32, C.c_uint32, C.c_uint32, C.c_int]
        L.orc_iq_tables.argtypes = [C.c_void_p] * 5
        L.orc_scale_min_k4.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
        _lib = L
    return _lib


def ref():
    """qw6's own CPU path (compiled from the reference tree), or None."""
    global _ref
    if _ref is None and REF_SO.exists():
        R = C.CDLL(str(REF_SO))
        R.ref_fp16_to_f32.restype = C.c_float
        R.ref_fp16_to_f32.argtypes = [C.c_uint16]
        R.ref_dequant_row.argtypes = [C.c_int, C.c_void_p, C.c_uint32, C.c_uint32,
                                      C.c_uint32, _f32p]
        R.ref_matvec.argtypes = [_f32p, C.c_int, C.c_void_p, C.c_uint32, C.c_uint32,
                                 _f32p, C.c_uint32]
        R.ref_moe_route.argtypes = [_i32p, _f32p, _f32p, C.c_int, C.c_int]
        R.ref_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int]
        R.ref_moe_layer.argtypes = [_f32p, C.c_void_p, C.c_void_p, _f32p,
                                    C.c_void_p, _i32p, C.c_void_p, _i32p, C.c_void_p, _i32p,
                                    C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                    C.c_void_p, C.c_int, _f32p]
        R.ref_moe_layer_logits.argtypes = R.ref_moe_layer.argtypes
        R.ref_moe_layer_sr.argtypes = R.ref_moe_layer.argtypes + [_f32p]
        R.qw6_cpu_argmax.restype = C.c_int
        R.qw6_cpu_argmax.argtypes = [_f32p, C.c_int]
        u32, u64, i64 = C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(C.c_int64)
        R.ref_gguf_header.argtypes = [C.c_char_p, u32, u32, u32, u32, u64, u64]
        R.ref_gguf_validate.argtypes = [C.c_char_p]
        R.ref_gguf_tensor.argtypes = [C.c_char_p, C.c_uint32, C.c_char_p, u32, i64,
                                      C.POINTER(C.c_int32), u64, u64]
        R.ref_gguf_pack.argtypes = [C.c_char_p, C.c_uint32, C.POINTER(C.c_int32), u32, u32,
                                    u64, u64]
        R.ref_gguf_kv.argtypes = [C.c_char_p, C.c_char_p, C.POINTER(C.c_int32), i64,
                                  C.POINTER(C.c_double), C.c_char_p, C.c_size_t]
        _ref = R
    return _ref


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def _mat(data: np.ndarray, quant: int, rows: int, cols: int) -> OrcMat:
    return OrcMat(data.ctypes.data, quant, rows, cols)


# ---- oracle wrappers --------------------------------------------------------

def fp16_to_f32(h: int) -> float:
    return lib().orc_fp16_to_f32(h)


def dequant_row(quant: int, data: np.ndarray, cols: int, row: int) -> np.ndarray:
    out = np.zeros(cols, np.float32)
    rc = lib().orc_dequant_row(quant, data.ctypes.data, cols, row, out)
    if rc != 0:
        raise ValueError("oracle dequant_row failed (quant %d)" % quant)
    return out


def matvec(quant: int, data: np.ndarray, rows: int, cols: int, x: np.ndarray,
           nthreads: int = 1, max_rows: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(rows, np.float32)
    m = _mat(data, quant, rows, cols)
    if lib().orc_matvec(out, C.byref(m), x, max_rows, nthreads) != 0:
        raise ValueError("oracle matvec failed")
    return out


def moe_route(logits: np.ndarray, top_k: int):
    logits = np.ascontiguousarray(logits, np.float32)
    idx = np.zeros(top_k, np.int32)
    w = np.zeros(top_k, np.float32)
    lib().orc_moe_route(idx, w, logits, logits.size, top_k)
    return idx, w


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    return int(lib().orc_argmax(x, x.size))


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    out = np.zeros_like(x, dtype=np.float32)
    lib().orc_rmsnorm(out, np.ascontiguousarray(x, np.float32),
                      np.ascontiguousarray(w, np.float32), x.size, eps)
    return out


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    out = np.zeros(g.size, np.float32)
    lib().orc_silu_mul(np.ascontiguousarray(g, np.float32),
                       np.ascontiguousarray(u, np.float32), out, g.size)
    return out


def moe_gather(expert_out: np.ndarray, weights: np.ndarray, shared: np.ndarray | None,
               shared_weight: float) -> np.ndarray:
    eo = np.ascontiguousarray(expert_out, np.float32)
    top_k, dim = eo.shape
    out = np.zeros(dim, np.float32)
    sh = None if shared is None else np.ascontiguousarray(shared, np.float32)
    lib().orc_moe_gather(eo.reshape(-1), np.ascontiguousarray(weights, np.float32),
                         _ptr(sh), shared_weight, out, dim, top_k)
    return out


class Layer:
    """Host copy of one MoE layer: per-expert (bytes, quant, rows, cols) for
    gate/up/down (None for experts that are never touched), optional shared
    expert, F32 router or None."""

    def __init__(self, hidden, inter, n_experts, top_k, router, experts, shared,
                 shared_router=None):
        self.hidden, self.inter = hidden, inter
        self.n_experts, self.top_k = n_experts, top_k
        self.router = router
        self.experts = experts          # list of 3-tuples of (arr, quant) or None
        self.shared = shared            # 3-tuple of (arr, quant) or None
        self.shared_router = shared_router

    def mats(self):
        keep = []
        arr = (OrcMat * (3 * self.n_experts))()
        for e in range(self.n_experts):
            ex = self.experts[e]
            shapes = ((self.inter, self.hidden), (self.inter, self.hidden),
                      (self.hidden, self.inter))
            for j in range(3):
                if ex is None:
                    arr[3 * e + j] = OrcMat(None, 0, shapes[j][0], shapes[j][1])
                else:
                    a, q = ex[j]
                    keep.append(a)
                    arr[3 * e + j] = OrcMat(a.ctypes.data, q, shapes[j][0], shapes[j][1])
        sh = None
        if self.shared is not None:
            sh = (OrcMat * 3)()
            shapes = ((self.inter, self.hidden), (self.inter, self.hidden),
                      (self.hidden, self.inter))
            for j in range(3):
                a, q = self.shared[j]
                keep.append(a)
                sh[j] = OrcMat(a.ctypes.data, q, shapes[j][0], shapes[j][1])
        return arr, sh, keep


def moe_layer(layer: Layer, x: np.ndarray, logits: np.ndarray | None = None,
              nthreads: int = 1):
    """(out[hidden], idx[top_k], w[top_k]) of one token through the oracle."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(layer.hidden, np.float32)
    idx = np.zeros(layer.top_k, np.int32)
    w = np.zeros(layer.top_k, np.float32)
    arr, sh, keep = layer.mats()
    lg = None if logits is None else np.ascontiguousarray(logits, np.float32)
    rc = lib().orc_moe_layer(out, idx, w, _ptr(layer.router) if logits is None else None,
                             _ptr(lg), arr, C.cast(sh, C.c_void_p) if sh is not None else None,
                             _ptr(layer.shared_router), x, layer.hidden, layer.n_experts,
                             layer.top_k, nthreads)
    if rc != 0:
        raise ValueError("oracle moe_layer failed")
    return out, idx, w


# ---- reference wrappers ----------------------------------------------------

def ref_matvec(quant, data, rows, cols, x, max_rows=0):
    out = np.zeros(rows, np.float32)
    rc = ref().ref_matvec(out, quant, data.ctypes.data, rows, cols,
                          np.ascontiguousarray(x, np.float32), max_rows)
    if rc != 0:
        raise ValueError("reference matvec failed")
    return out


def ref_dequant_row(quant, data, rows, cols, row):
    out = np.zeros(cols, np.float32)
    if ref().ref_dequant_row(quant, data.ctypes.data, rows, cols, row, out) != 0:
        raise ValueError("reference dequant failed")
    return out


def ref_moe_route(logits, top_k):
    logits = np.ascontiguousarray(logits, np.float32)
    idx = np.zeros(top_k, np.int32)
    w = np.zeros(top_k, np.float32)
    ref().ref_moe_route(idx, w, logits, logits.size, top_k)
    return idx, w


def ref_rmsnorm(x, w):
    out = np.zeros(x.size, np.float32)
    ref().ref_rmsnorm(out, np.ascontiguousarray(x, np.float32),
                      np.ascontiguousarray(w, np.float32), x.size)
    return out


def ref_moe_layer(layer: Layer, x: np.ndarray, logits: np.ndarray | None = None,
                  want_route: bool = True):
    """Reference MoE layer (qw6_apply_layer_moe; with logits given, the same
    composition of reference routines minus the router matvec)."""
    n = layer.n_experts
    ptrs = {k: (C.c_void_p * n)() for k in range(3)}
    qs = {k: np.zeros(n, np.int32) for k in range(3)}
    for e in range(n):
        ex = layer.experts[e]
        for j in range(3):
            if ex is not None:
                ptrs[j][e] = ex[j][0].ctypes.data
                qs[j][e] = ex[j][1]
            else:
                qs[j][e] = 4 if j < 2 else 7
    sh = layer.shared
    sa = [None, 0, None, 0, None, 0] if sh is None else [
        sh[0][0].ctypes.data, sh[0][1], sh[1][0].ctypes.data, sh[1][1],
        sh[2][0].ctypes.data, sh[2][1]]
    out = np.zeros(layer.hidden, np.float32)
    idx = np.zeros(layer.top_k, np.int32)
    w = np.zeros(layer.top_k, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    if logits is None:
        fn, first = ref().ref_moe_layer, layer.router
    else:
        fn, first = ref().ref_moe_layer_logits, np.ascontiguousarray(logits, np.float32)
    route = want_route or logits is not None
    extra = []
    if layer.shared_router is not None:
        if logits is not None:
            raise ValueError("the reference's given-logits composition has no shared gate")
        fn = ref().ref_moe_layer_sr
        extra = [np.ascontiguousarray(layer.shared_router, np.float32)]
    rc = fn(out, idx.ctypes.data if route else None, w.ctypes.data if route else None, first,
            ptrs[0], qs[0], ptrs[1], qs[1], ptrs[2], qs[2], *sa, x, *extra)
    if rc != 0:
        raise ValueError("reference moe layer failed")
    return out, idx, w


# ---- qw6's GGUF reader (reference build) -------------------------------------

def ref_gguf_header(path):
    """qw6_gguf_parse's header facts, or None where it fails."""
    v, nt, nkv, al = (C.c_uint32() for _ in range(4))
    do, fs = C.c_uint64(), C.c_uint64()
    if ref().ref_gguf_header(str(path).encode(), C.byref(v), C.byref(nt), C.byref(nkv),
                             C.byref(al), C.byref(do), C.byref(fs)) != 0:
        return None
    return {"version": v.value, "n_tensors": nt.value, "n_kv": nkv.value,
            "alignment": al.value, "data_offset": do.value, "file_size": fs.value}


def ref_gguf_valid(path) -> bool:
    """qw6_gguf_parse + gguf_validate_tensor_ranges both succeed."""
    return ref().ref_gguf_validate(str(path).encode()) == 0


def ref_gguf_tensor(path, i):
    name = C.create_string_buffer(128)
    nd, t = C.c_uint32(), C.c_int32()
    dims = (C.c_int64 * 4)()
    off, span = C.c_uint64(), C.c_uint64()
    if ref().ref_gguf_tensor(str(path).encode(), i, name, C.byref(nd), dims, C.byref(t),
                             C.byref(off), C.byref(span)) != 0:
        return None
    return {"name": name.value.decode(errors="replace"), "dims": list(dims[:nd.value]),
            "type": t.value, "offset": off.value, "span": span.value}


def ref_gguf_pack(path, i):
    """bind_expert_pack on tensor i: quant, rows, cols, per-expert file
    offsets and sizes (256 experts), or None where it fails."""
    q = C.c_int32()
    r, c = C.c_uint32(), C.c_uint32()
    offs = (C.c_uint64 * 256)()
    sizes = (C.c_uint64 * 256)()
    if ref().ref_gguf_pack(str(path).encode(), i, C.byref(q), C.byref(r), C.byref(c), offs,
                           sizes) != 0:
        return None
    return {"quant": q.value, "rows": r.value, "cols": c.value, "offsets": list(offs),
            "sizes": list(sizes)}


def ref_gguf_kv(path, key):
    """(type, integer value, float value, string) of qw6_gguf_find_kv, or None."""
    t = C.c_int32()
    iv, fv = C.c_int64(), C.c_double()
    sb = C.create_string_buffer(1 << 16)
    if ref().ref_gguf_kv(str(path).encode(), key.encode(), C.byref(t), C.byref(iv), C.byref(fv),
                         sb, 1 << 16) != 0:
        return None
    return t.value, iv.value, fv.value, sb.value.decode(errors="replace")
