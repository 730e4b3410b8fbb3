"""ctypes wrapper around oracle/liboracle.so, the CPU restatement of the
reference's 4-bit MoE path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product (libdismoen_hip.so
and the dismoen package) never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
I64P = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
U8P = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


class OracleError(RuntimeError):
    """Error raised by an oracle function; the message is the reference's."""


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.or_fp16_to_f32.argtypes = [C.c_uint16]
        L.or_fp16_to_f32.restype = C.c_float
        L.or_f32_to_bf16_rne.argtypes = [C.c_float]
        L.or_f32_to_bf16_rne.restype = C.c_uint16
        L.or_expf.argtypes = [C.c_float]
        L.or_expf.restype = C.c_float
        L.or_sigmoid_f32.argtypes = [C.c_float]
        L.or_sigmoid_f32.restype = C.c_float
        L.or_silu_f32.argtypes = [C.c_float]
        L.or_silu_f32.restype = C.c_float
        L.or_pack_4bit_pair.argtypes = [C.c_int, C.c_int, C.POINTER(C.c_uint8)]
        L.or_unpack_4bit_pair.argtypes = [C.c_uint8, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.or_compute_fp16_scale_ceil.argtypes = [C.c_float, C.POINTER(C.c_int)]
        L.or_compute_fp16_scale_ceil.restype = C.c_uint16
        L.or_dequant_q4_bf16.argtypes = [U16P, C.c_int64, U8P, C.c_int64, C.c_int64,
                                         C.c_int, U16P, C.c_char_p, C.c_size_t]
        L.or_dequant_gguf.argtypes = [C.c_int, U8P, C.c_int64, C.c_int64, C.c_int, F32P,
                                      C.c_char_p, C.c_size_t]
        L.or_router_project.argtypes = [F32P, C.c_int64, F32P, C.c_int64, C.c_int, C.c_int,
                                        C.c_int, C.c_int, F32P, C.c_char_p, C.c_size_t]
        L.or_router_softmax.argtypes = [F32P, C.c_int64, C.c_int, C.c_int, C.c_int, F32P,
                                        C.c_char_p, C.c_size_t]
        L.or_select_topk.argtypes = [F32P, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_int,
                                     C.c_int, I32P, F32P, C.c_char_p, C.c_size_t]
        L.or_router_config_validate.argtypes = [C.c_int, C.c_int, C.c_int, C.c_char_p,
                                                C.c_size_t]
        L.or_swiglu_forward.argtypes = [F32P, C.c_int64, F32P, F32P, F32P, C.c_int64,
                                        C.c_int64, C.c_int64, C.c_int, C.c_int, C.c_int,
                                        C.c_int, C.c_int, F32P, C.c_char_p, C.c_size_t]
        L.or_shared_gate_forward.argtypes = [F32P, C.c_int64, F32P, C.c_int64, C.c_int,
                                             C.c_int, C.c_int, C.c_char_p, F32P, C.c_char_p,
                                             C.c_size_t]
        L.or_moe_aggregate.argtypes = [C.c_void_p, F32P, F32P, F32P, F32P, C.c_int, C.c_int,
                                       C.c_int, C.c_int, F32P, C.c_char_p, C.c_size_t]
        L.or_rmsnorm.argtypes = [F32P, C.c_void_p, C.c_int, C.c_float, F32P, C.c_char_p,
                                 C.c_size_t]
        L.or_add_residual.argtypes = [F32P, F32P, C.c_int64, C.c_int, F32P, C.c_char_p,
                                      C.c_size_t]
        L.or_partition_range.argtypes = [C.c_int64, C.c_int64, C.c_int64,
                                         C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
        L.or_pool_create.argtypes = [C.c_int]
        L.or_pool_create.restype = C.c_void_p
        L.or_pool_destroy.argtypes = [C.c_void_p]
        L.or_pool_parallel_moe_experts.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int,
                                                   F32P, F32P, I64P, C.c_void_p, C.c_void_p,
                                                   C.c_void_p]
        L.or_layer_cache_build.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t]
        L.or_layer_cache_build.restype = C.c_void_p
        L.or_layer_cache_build_mt.argtypes = [C.c_void_p, C.c_int, C.c_char_p, C.c_size_t]
        L.or_layer_cache_build_mt.restype = C.c_void_p
        L.or_layer_cache_free.argtypes = [C.c_void_p]
        L.or_moe_layer_q4.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, F32P, C.c_void_p,
                                      C.c_int, C.c_int, F32P, I32P, F32P, F32P, C.c_char_p,
                                      C.c_size_t]
        L.or_rmsnorm_tree256.argtypes = [F32P, C.c_void_p, C.c_int, C.c_float, F32P,
                                         C.c_char_p, C.c_size_t]
        L.or_moe_stack_q4.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                                      F32P, C.c_int, C.c_float, F32P, I32P, F32P, C.c_char_p,
                                      C.c_size_t]
        _lib = L
    return _lib


def _check(st, buf):
    if st:
        raise OracleError(buf.value.decode(errors="replace"))


def _errbuf():
    return C.create_string_buffer(1024)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32).ravel()


# ---- scalar helpers --------------------------------------------------------
def expf(x: float) -> float:
    return lib().or_expf(x)


def sigmoid_f32(z: float) -> float:
    return lib().or_sigmoid_f32(z)


def silu_f32(z: float) -> float:
    return lib().or_silu_f32(z)


def fp16_to_f32(h: int) -> float:
    return lib().or_fp16_to_f32(h)


def f32_to_bf16(f: float) -> int:
    return lib().or_f32_to_bf16_rne(f)


def pack_4bit_pair(w0: int, w1: int) -> int:
    out = C.c_uint8()
    if lib().or_pack_4bit_pair(w0, w1, C.byref(out)):
        raise OracleError("pack_4bit_pair: values must be in [-7, 7] (0x8 reserved)")
    return out.value


def unpack_4bit_pair(b: int):
    a, c = C.c_int(), C.c_int()
    if lib().or_unpack_4bit_pair(b, C.byref(a), C.byref(c)):
        raise OracleError("unpack_4bit_pair: reserved nibble 0x8 (-8)")
    return a.value, c.value


def compute_fp16_scale_ceil(max_abs: float) -> int:
    st = C.c_int()
    v = lib().or_compute_fp16_scale_ceil(max_abs, C.byref(st))
    if st.value:
        raise OracleError("compute_fp16_scale_ceil: NaN/Inf or overflow")
    return v


# ---- dequant ---------------------------------------------------------------
def dequant_q4_bf16(scales_u16, packed_u8, num_elements: int, group_size: int = 128):
    s = np.ascontiguousarray(scales_u16, dtype=np.uint16).ravel()
    p = np.ascontiguousarray(packed_u8, dtype=np.uint8).ravel()
    out = np.zeros(max(int(num_elements), 1), dtype=np.uint16)
    e = _errbuf()
    _check(lib().or_dequant_q4_bf16(s, s.size, p, p.size, num_elements, group_size, out,
                                    e, 1024), e)
    return out[:num_elements]


GGML_F32, GGML_Q8_0, GGML_Q3_K, GGML_Q4_K, GGML_BF16 = 0, 8, 11, 12, 30


def dequant_gguf(ggml_type: int, raw, num_elements: int, q4k_layout: int = 0):
    """GGUF payload -> fp32 (src/format/gguf.mojo:414-626)."""
    r = np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else \
        np.ascontiguousarray(raw, dtype=np.uint8).ravel()
    nbytes = r.size
    if r.size == 0:
        r = np.zeros(1, np.uint8)
    out = np.zeros(max(int(num_elements), 1), dtype=np.float32)
    e = _errbuf()
    _check(lib().or_dequant_gguf(ggml_type, r, nbytes, num_elements, q4k_layout, out, e,
                                 1024), e)
    return out[:num_elements]


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- router ----------------------------------------------------------------
def router_project(x, w, seq_len, hidden, num_experts, layer=0):
    x, w = _f32(x), _f32(w)
    out = np.zeros(max(seq_len * num_experts, 1), np.float32)
    e = _errbuf()
    _check(lib().or_router_project(x, x.size, w, w.size, seq_len, hidden, num_experts, layer,
                                   out, e, 1024), e)
    return out[: seq_len * num_experts]


def router_softmax(z, seq_len, num_experts, layer=0):
    z = _f32(z)
    out = np.zeros(max(z.size, 1), np.float32)
    e = _errbuf()
    _check(lib().or_router_softmax(z, z.size, seq_len, num_experts, layer, out, e, 1024), e)
    return out[: z.size]


def select_topk(probs, seq_len, num_experts, top_k, norm_topk_prob=False, layer=0):
    p = _f32(probs)
    ids = np.zeros(max(seq_len * max(top_k, 1), 1), np.int32)
    vals = np.zeros(max(seq_len * max(top_k, 1), 1), np.float32)
    e = _errbuf()
    _check(lib().or_select_topk(p, p.size, seq_len, num_experts, top_k, int(norm_topk_prob),
                                layer, ids, vals, e, 1024), e)
    n = seq_len * top_k
    return ids[:n].reshape(seq_len, top_k), vals[:n].reshape(seq_len, top_k)


def router_forward(x, w, seq_len, hidden, num_experts, top_k, norm_topk_prob=False, layer=0):
    e = _errbuf()
    _check(lib().or_router_config_validate(num_experts, top_k, int(norm_topk_prob), e, 1024), e)
    z = router_project(x, w, seq_len, hidden, num_experts, layer)
    p = router_softmax(z, seq_len, num_experts, layer)
    return select_topk(p, seq_len, num_experts, top_k, norm_topk_prob, layer)


# ---- experts ---------------------------------------------------------------
def swiglu_forward(x, w_gate, w_up, w_down, seq_len, hidden, inter, layer=0, expert_id=-1):
    x, g, u, d = _f32(x), _f32(w_gate), _f32(w_up), _f32(w_down)
    out = np.zeros(max(seq_len * hidden, 1), np.float32)
    e = _errbuf()
    _check(lib().or_swiglu_forward(x, x.size, g, u, d, g.size, u.size, d.size, seq_len, hidden,
                                   inter, layer, expert_id, out, e, 1024), e)
    return out[: seq_len * hidden]


def shared_gate_forward(x, w, seq_len, hidden, layer=0, gate_mode="sigmoid"):
    x, w = _f32(x), _f32(w)
    out = np.zeros(max(seq_len, 1), np.float32)
    e = _errbuf()
    _check(lib().or_shared_gate_forward(x, x.size, w, w.size, seq_len, hidden, layer,
                                        gate_mode.encode(), out, e, 1024), e)
    return out[:seq_len]


def moe_aggregate(residual, routed, probs, shared_out, gates, seq_len, hidden, top_k, layer=0):
    routed, probs, sh, g = _f32(routed), _f32(probs), _f32(shared_out), _f32(gates)
    res = None if residual is None else _f32(residual)
    out = np.zeros(max(seq_len * hidden, 1), np.float32)
    e = _errbuf()
    rp = None if res is None else res.ctypes.data_as(C.c_void_p)
    _check(lib().or_moe_aggregate(rp, routed, probs, sh, g, seq_len, hidden, top_k, layer, out,
                                  e, 1024), e)
    return out[: seq_len * hidden]


def rmsnorm(x, gamma, eps, tree: bool = False):
    """rmsnorm (src/layers/rmsnorm.mojo:10-48); tree=True: the sum of squares
    in the library's fast-mode order (256 strided partials, halving tree)."""
    x = _f32(x)
    gm = None if gamma is None else _f32(gamma)
    out = np.zeros(max(x.size, 1), np.float32)
    e = _errbuf()
    gp = None if gm is None else gm.ctypes.data_as(C.c_void_p)
    fn = lib().or_rmsnorm_tree256 if tree else lib().or_rmsnorm
    _check(fn(x, gp, x.size, eps, out, e, 1024), e)
    return out[: x.size]


def add_residual(y, x, layer=0):
    y, x = _f32(y), _f32(x)
    out = np.zeros(max(y.size, 1), np.float32)
    e = _errbuf()
    if y.size != x.size:
        raise OracleError('{"error_type":"ATTENTION_ERROR","detail":"residual length mismatch",'
                          '"stage":"residual","layer":%d}' % layer)
    _check(lib().or_add_residual(y, x, y.size, layer, out, e, 1024), e)
    return out[: y.size]


def partition_range(total, tid, n):
    s, e = C.c_int64(), C.c_int64()
    lib().or_partition_range(total, tid, n, C.byref(s), C.byref(e))
    return s.value, e.value


class Pool:
    """The static worker pool (src/core/worker_pool.mojo)."""

    def __init__(self, num_threads: int):
        self.num_threads = num_threads
        self.h = lib().or_pool_create(num_threads)

    def close(self):
        if self.h:
            lib().or_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def parallel_moe_experts(self, top_k, hidden, inter, x_tok, selected, w_gate, w_up, w_down):
        """w_* are lists (by expert id) of fp32 arrays; returns [top_k*hidden]."""
        x = _f32(x_tok)
        out = np.zeros(top_k * hidden, np.float32)
        sel = np.ascontiguousarray(selected, dtype=np.int64)
        keep = [_f32(a) for a in w_gate + w_up + w_down]
        n = len(w_gate)
        tabs = [(C.c_void_p * n)(*[a.ctypes.data for a in keep[i * n:(i + 1) * n]])
                for i in range(3)]
        lib().or_pool_parallel_moe_experts(self.h, top_k, hidden, inter, x, out, sel,
                                           C.cast(tabs[0], C.c_void_p),
                                           C.cast(tabs[1], C.c_void_p),
                                           C.cast(tabs[2], C.c_void_p))
        del keep
        return out


# ---- the 4-bit layer -------------------------------------------------------
class _LayerQ4(C.Structure):
    _fields_ = [("hidden", C.c_int), ("num_experts", C.c_int), ("top_k", C.c_int),
                ("inter", C.c_int), ("inter_sh", C.c_int), ("group_size", C.c_int),
                ("router_bf16", C.c_void_p), ("shgate_bf16", C.c_void_p),
                ("gu_scales", C.c_void_p), ("gu_packed", C.c_void_p),
                ("d_scales", C.c_void_p), ("d_packed", C.c_void_p),
                ("sh_gu_scales", C.c_void_p), ("sh_gu_packed", C.c_void_p),
                ("sh_d_scales", C.c_void_p), ("sh_d_packed", C.c_void_p)]


def _layer_struct(L):
    """L: dismoen.synth.MoELayerQ4 (numpy arrays in the reference layout)."""
    s = _LayerQ4()
    s.hidden, s.num_experts, s.top_k = L.hidden, L.num_experts, L.top_k
    s.inter, s.inter_sh, s.group_size = L.inter, L.inter_sh, L.group_size
    for name in ("router_bf16", "shgate_bf16", "gu_scales", "gu_packed", "d_scales",
                 "d_packed", "sh_gu_scales", "sh_gu_packed", "sh_d_scales", "sh_d_packed"):
        arr = getattr(L, name)
        assert arr.flags["C_CONTIGUOUS"]
        setattr(s, name, arr.ctypes.data)
    return s


class LayerCache:
    """Every expert of a layer dequantized once to fp32 (compute-only bound)."""

    def __init__(self, L, threads: int = 1):
        self._s = _layer_struct(L)
        self._keep = L
        e = _errbuf()
        self.h = lib().or_layer_cache_build_mt(C.byref(self._s), threads, e, 1024)
        if not self.h:
            raise OracleError(e.value.decode())

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_layer_cache_free(self.h)
            self.h = None


def moe_layer_q4(L, x, seq_len, residual=None, pool: Pool | None = None,
                 cache: LayerCache | None = None, layer=0):
    """forward_moe_block over the 4-bit layer; returns (y, ids, probs, shgate)."""
    s = _layer_struct(L)
    x = _f32(x)
    H, K = L.hidden, L.top_k
    y = np.zeros(seq_len * H, np.float32)
    ids = np.zeros(seq_len * K, np.int32)
    probs = np.zeros(seq_len * K, np.float32)
    shg = np.zeros(seq_len, np.float32)
    res = None if residual is None else _f32(residual)
    e = _errbuf()
    _check(lib().or_moe_layer_q4(C.byref(s), cache.h if cache else None,
                                 pool.h if pool else None, x,
                                 None if res is None else res.ctypes.data_as(C.c_void_p),
                                 seq_len, layer, y, ids, probs, shg, e, 1024), e)
    return y.reshape(seq_len, H), ids.reshape(seq_len, K), probs.reshape(seq_len, K), shg


def moe_stack_q4(layers, x, seq_len, eps=1e-6, pool: Pool | None = None, gammas=None,
                 tree: bool = False):
    """The port block's MoE section stacked with identity mixers: per layer
    h <- h + MoE_l(rmsnorm(h, gamma_l, eps)); gammas: per-layer [H] arrays (or
    None entries: gamma = 1); tree=True: the fast-mode norm order."""
    arr = (_LayerQ4 * len(layers))(*[_layer_struct(L) for L in layers])
    x = _f32(x)
    H, K = layers[0].hidden, layers[0].top_k
    out = np.zeros(seq_len * H, np.float32)
    ids = np.zeros(len(layers) * seq_len * K, np.int32)
    probs = np.zeros(len(layers) * seq_len * K, np.float32)
    gkeep = None
    gp = None
    if gammas is not None:
        gkeep = [None if g is None else _f32(g) for g in gammas]
        gp = (C.c_void_p * len(layers))(*[None if g is None else g.ctypes.data for g in gkeep])
    e = _errbuf()
    _check(lib().or_moe_stack_q4(C.cast(arr, C.c_void_p), len(layers),
                                 None if gp is None else C.cast(gp, C.c_void_p), int(tree),
                                 pool.h if pool else None, x, seq_len, eps, out, ids, probs,
                                 e, 1024), e)
    del gkeep
    return (out.reshape(seq_len, H), ids.reshape(len(layers), seq_len, K),
            probs.reshape(len(layers), seq_len, K))
