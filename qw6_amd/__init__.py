"""qw6_amd: MI355X (gfx950) routed-expert MoE FFN for qw6 models.

Python host layer over the C ABI in include/qw6_hip.h (libqw6_hip.so, built
in-tree by qw6_amd/build.py). Function names and argument meaning follow
qw6's Vulkan host operations (qw6_vk.h:9-56): a failing call raises
Qw6HipError with the library's message where the C function returns -1.

Device memory is owned either by the library context (upload / alloc) or by
the caller (torch tensors on a ROCm device, passed by address).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from . import synth  # noqa: F401

LIB_PATH = Path(__file__).resolve().parent / "libqw6_hip.so"

# qw6_quant_t (qw6.h:76-91)
Q_FP32, Q_Q4_K_M, Q_Q4_K_S, Q_Q5_K, Q_Q6_K = 0, 4, 5, 6, 7
Q_IQ3_S, Q_IQ2_S, Q_IQ2_XXS = 9, 11, 13
QUANT_NAMES = {Q_FP32: "F32", Q_Q4_K_M: "Q4_K", Q_Q4_K_S: "Q4_K", Q_Q5_K: "Q5_K",
               Q_Q6_K: "Q6_K", Q_IQ3_S: "IQ3_S", Q_IQ2_S: "IQ2_S", Q_IQ2_XXS: "IQ2_XXS"}


class Qw6HipError(RuntimeError):
    pass


class Matrix(C.Structure):
    _fields_ = [("data", C.c_void_p), ("quant", C.c_int32),
                ("rows", C.c_uint32), ("cols", C.c_uint32)]


class MoeLayer(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("inter", C.c_uint32), ("top_k", C.c_uint32),
                ("router", C.c_void_p), ("shared_router", C.c_void_p),
                ("experts", C.c_void_p), ("shared_gate", Matrix),
                ("shared_up", Matrix), ("shared_down", Matrix),
                ("norm_w", C.c_void_p), ("norm_eps", C.c_float)]


_lib = None
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


def lib():
    """Load libqw6_hip.so; raises if it was not built (no CPU fallback)."""
    global _lib
    if _lib is None:
        # Load torch's HIP runtime first when torch is present: the library
        # then binds to the same libamdhip64.so.7 instead of a second copy.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not LIB_PATH.exists():
            raise Qw6HipError("%s not built (run python -m qw6_amd.build)" % LIB_PATH)
        L = C.CDLL(str(LIB_PATH))
        L.qw6_hip_last_error.restype = C.c_char_p
        for n in ("q4k", "q5k", "q6k", "iq2xxs", "iq2s", "iq3s"):
            getattr(L, "qw6_hip_matmul_%s_host" % n).argtypes = [
                C.c_void_p, _f32p, _f32p, C.c_uint32, C.c_uint32]
        L.qw6_hip_matvec_f32_host.argtypes = [_f32p, _f32p, _f32p, C.c_uint32, C.c_uint32]
        L.qw6_hip_silu_mul_host.argtypes = [_f32p, _f32p, _f32p, C.c_uint32]
        L.qw6_hip_moe_route_host.argtypes = [_f32p, _u32p, _f32p, C.c_uint32, C.c_uint32]
        L.qw6_hip_moe_gather_host.argtypes = [_f32p, _f32p, C.c_void_p, C.c_float, _f32p,
                                              C.c_uint32, C.c_uint32]
        L.qw6_hip_rmsnorm_host.argtypes = [_f32p, _f32p, _f32p, C.c_uint32, C.c_float]
        L.qw6_hip_ctx_init.argtypes = [C.POINTER(C.c_void_p), C.c_int, C.c_uint32]
        L.qw6_hip_ctx_free.argtypes = [C.c_void_p]
        L.qw6_hip_ctx_free.restype = None
        L.qw6_hip_upload.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]
        L.qw6_hip_alloc.argtypes = [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]
        L.qw6_hip_set_mode.argtypes = [C.c_void_p, C.c_int]
        L.qw6_hip_matvec.argtypes = [C.c_void_p, C.POINTER(Matrix), C.c_void_p, C.c_void_p,
                                     C.c_uint32, C.c_void_p]
        L.qw6_hip_experts_create.argtypes = [C.c_void_p, C.POINTER(Matrix), C.POINTER(Matrix),
                                             C.POINTER(Matrix), C.c_uint32,
                                             C.POINTER(C.c_void_p)]
        L.qw6_hip_experts_free.argtypes = [C.c_void_p]
        L.qw6_hip_experts_free.restype = None
        L.qw6_hip_moe_forward.argtypes = [C.c_void_p, C.POINTER(MoeLayer), C.c_void_p,
                                          C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p,
                                          C.c_void_p, C.c_void_p, C.c_void_p]
        L.qw6_hip_moe_forward_noalloc.argtypes = L.qw6_hip_moe_forward.argtypes
        L.qw6_hip_profile.argtypes = [C.c_void_p, C.c_uint32]
        L.qw6_hip_profile_read.argtypes = [C.c_void_p, C.POINTER(C.c_float),
                                           C.POINTER(C.c_uint32)]
        L.qw6_hip_rmsnorm.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_uint32, C.c_uint32, C.c_float, C.c_void_p]
        L.qw6_hip_argmax.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p]
        L.qw6_hip_argmax_host.argtypes = [_f32p, C.c_uint32, _u32p, C.c_void_p]
        L.qw6_hip_sampling_greedy_host.argtypes = [_f32p, C.c_uint32, _u32p]
        L.qw6_hip_output_greedy.argtypes = [C.c_void_p, C.POINTER(Matrix), C.c_void_p,
                                            C.c_void_p, C.c_float, C.c_void_p, C.c_void_p,
                                            C.c_void_p]
        L.qw6_hip_synth_blocks.argtypes = [C.c_void_p, C.c_int32, C.c_uint64, C.c_uint64,
                                           C.c_uint64, C.c_uint64, C.c_void_p]
        L.qw6_hip_synth_normal.argtypes = [C.c_void_p, C.c_uint64, C.c_float, C.c_float,
                                           C.c_uint64, C.c_uint64, C.c_void_p]
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise Qw6HipError(lib().qw6_hip_last_error().decode(errors="replace"))


# ---- synchronous host operations (qw6_vk.h:9-56) ------------------------------

_HOST_FN = {Q_Q4_K_M: "q4k", Q_Q4_K_S: "q4k", Q_Q5_K: "q5k", Q_Q6_K: "q6k",
            Q_IQ2_XXS: "iq2xxs", Q_IQ2_S: "iq2s", Q_IQ3_S: "iq3s"}


def matmul_host(quant: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """y = deq(W) x (qw6_vk_matmul_<fmt>_host)."""
    y = np.zeros(rows, np.float32)
    if quant == Q_FP32:
        _check(lib().qw6_hip_matvec_f32_host(np.ascontiguousarray(w, np.float32).reshape(-1),
                                             np.ascontiguousarray(x, np.float32), y, rows, cols))
        return y
    w = np.ascontiguousarray(w, np.uint8)
    fn = getattr(lib(), "qw6_hip_matmul_%s_host" % _HOST_FN[quant])
    _check(fn(w.ctypes.data, np.ascontiguousarray(x, np.float32), y, rows, cols))
    return y


def silu_mul_host(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    out = np.zeros(g.size, np.float32)
    _check(lib().qw6_hip_silu_mul_host(np.ascontiguousarray(g, np.float32),
                                       np.ascontiguousarray(u, np.float32), out, g.size))
    return out


def moe_route_host(logits: np.ndarray, top_k: int):
    idx = np.zeros(top_k, np.uint32)
    w = np.zeros(top_k, np.float32)
    logits = np.ascontiguousarray(logits, np.float32)
    _check(lib().qw6_hip_moe_route_host(logits, idx, w, logits.size, top_k))
    return idx, w


def moe_gather_host(expert_out: np.ndarray, weights: np.ndarray, shared: np.ndarray | None,
                    shared_weight: float) -> np.ndarray:
    eo = np.ascontiguousarray(expert_out, np.float32)
    top_k, dim = eo.shape
    out = np.zeros(dim, np.float32)
    sh = None if shared is None else np.ascontiguousarray(shared, np.float32)
    _check(lib().qw6_hip_moe_gather_host(eo.reshape(-1), np.ascontiguousarray(weights, np.float32),
                                         None if sh is None else sh.ctypes.data,
                                         shared_weight, out, dim, top_k))
    return out


def rmsnorm_host(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    y = np.zeros(x.size, np.float32)
    _check(lib().qw6_hip_rmsnorm_host(np.ascontiguousarray(x, np.float32),
                                      np.ascontiguousarray(w, np.float32), y, x.size, eps))
    return y


def argmax_host(x: np.ndarray, with_value: bool = False):
    """First index of the maximum, qw6_cpu_argmax semantics (qw6.c:2858-2863)
    (qw6_vk_argmax_host); with_value: (index, x[index])."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(1, np.uint32)
    val = np.zeros(1, np.float32)
    _check(lib().qw6_hip_argmax_host(x, x.size, out, val.ctypes.data if with_value else None))
    return (int(out[0]), val[0]) if with_value else int(out[0])


def sampling_greedy_host(logits: np.ndarray) -> int:
    """Greedy token of host logits (qw6_vk_sampling_greedy_host)."""
    x = np.ascontiguousarray(logits, np.float32).reshape(-1)
    out = np.zeros(1, np.uint32)
    _check(lib().qw6_hip_sampling_greedy_host(x, x.size, out))
    return int(out[0])


# ---- device-resident API ----------------------------------------------------------

def _addr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream


class Experts:
    """Device expert table of one MoE layer (qw6_hip_experts_create)."""

    def __init__(self, ctx: "Context", gate, up, down):
        n = len(gate)
        arrs = [(Matrix * n)(*[Matrix(*m) for m in mats]) for mats in (gate, up, down)]
        h = C.c_void_p()
        _check(lib().qw6_hip_experts_create(ctx.handle, arrs[0], arrs[1], arrs[2], n,
                                            C.byref(h)))
        self.handle = h
        self.n = n

    def free(self):
        if self.handle:
            lib().qw6_hip_experts_free(self.handle)
            self.handle = None


class Context:
    """qw6_hip_ctx_t: workspace and owned device buffers on one device."""

    def __init__(self, device: int = 0, max_tokens: int = 4):
        h = C.c_void_p()
        _check(lib().qw6_hip_ctx_init(C.byref(h), device, max_tokens))
        self.handle = h
        self.device = device

    def close(self):
        if self.handle:
            lib().qw6_hip_ctx_free(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def upload(self, host: np.ndarray) -> int:
        host = np.ascontiguousarray(host)
        p = C.c_void_p()
        _check(lib().qw6_hip_upload(self.handle, host.ctypes.data, host.nbytes, C.byref(p)))
        return p.value

    def alloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        _check(lib().qw6_hip_alloc(self.handle, nbytes, C.byref(p)))
        return p.value

    def set_mode(self, mode: int):
        _check(lib().qw6_hip_set_mode(self.handle, mode))

    def matvec(self, w: tuple, x, y, n_tok: int = 1, stream=None):
        m = Matrix(*w)
        _check(lib().qw6_hip_matvec(self.handle, C.byref(m), _addr(x), _addr(y), n_tok,
                                    _stream(stream)))

    def experts(self, gate, up, down) -> Experts:
        return Experts(self, gate, up, down)

    def moe_forward(self, layer: MoeLayer, x, out, n_tok: int = 1, logits=None,
                    residual=None, idx=None, w=None, stream=None):
        _check(lib().qw6_hip_moe_forward(self.handle, C.byref(layer), _addr(x), _addr(logits),
                                         _addr(residual), n_tok, _addr(out), _addr(idx),
                                         _addr(w), _stream(stream)))

    def moe_forward_noalloc(self, layer: MoeLayer, x, out, n_tok: int = 1, logits=None,
                            residual=None, idx=None, w=None, stream=None):
        """moe_forward on the library's static per-device workspace: no
        allocation, per-token kernels only (qw6_hip_moe_forward_noalloc)."""
        _check(lib().qw6_hip_moe_forward_noalloc(self.handle, C.byref(layer), _addr(x),
                                                 _addr(logits), _addr(residual), n_tok,
                                                 _addr(out), _addr(idx), _addr(w),
                                                 _stream(stream)))

    def profile(self, max_calls: int):
        _check(lib().qw6_hip_profile(self.handle, max_calls))

    def profile_read(self):
        """Summed ms of [router, gate_up, down] over the recorded calls."""
        ms = (C.c_float * 3)()
        n = C.c_uint32()
        _check(lib().qw6_hip_profile_read(self.handle, ms, C.byref(n)))
        return list(ms), n.value

    def rmsnorm(self, x, w, y, n: int, n_tok: int = 1, eps: float = 1e-6, stream=None):
        _check(lib().qw6_hip_rmsnorm(self.handle, _addr(x), _addr(w), _addr(y), n, n_tok, eps,
                                     _stream(stream)))

    def argmax(self, x, n: int, out, stream=None):
        """out[0] = first index of the maximum of x[:n] (device buffers)."""
        _check(lib().qw6_hip_argmax(self.handle, _addr(x), n, _addr(out), _stream(stream)))

    def output_greedy(self, w: tuple, x, logits, token, norm_w=None, eps: float = 1e-6,
                      stream=None):
        """logits = W rmsnorm(x) * norm_w (no norm without norm_w); token[0] = argmax."""
        m = Matrix(*w)
        _check(lib().qw6_hip_output_greedy(self.handle, C.byref(m), _addr(x), _addr(norm_w), eps,
                                           _addr(logits), _addr(token), _stream(stream)))


def make_layer(hidden: int, inter: int, top_k: int, experts: Experts, router=None,
               shared=None, shared_router=None, norm_w=None, norm_eps: float = 1e-6) -> MoeLayer:
    L = MoeLayer()
    L.hidden, L.inter, L.top_k = hidden, inter, top_k
    L.router = _addr(router)
    L.shared_router = _addr(shared_router)
    L.norm_w = _addr(norm_w)
    L.norm_eps = norm_eps
    L.experts = experts.handle
    if shared is not None:
        L.shared_gate = Matrix(*shared[0])
        L.shared_up = Matrix(*shared[1])
        L.shared_down = Matrix(*shared[2])
    return L


def synth_blocks(dst, quant: int, nblocks: int, seed: int, stream_id: int, first: int = 0,
                 stream=None):
    _check(lib().qw6_hip_synth_blocks(_addr(dst), quant, nblocks, first, seed, stream_id,
                                      _stream(stream)))


def synth_normal(dst, n: int, std: float, seed: int, stream_id: int, mean: float = 0.0,
                 stream=None):
    _check(lib().qw6_hip_synth_normal(_addr(dst), n, mean, std, seed, stream_id,
                                      _stream(stream)))
