"""ctypes binding of libdismoen_hip.so (declarations in include/dismoen_hip.h).

The library is the only compute path: when it is missing, importing this
module's `lib()` raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes as C
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# DISMOEN_LIB names another build of the same library (the tracing build of
# phase_trace.py); by default the in-tree libdismoen_hip.so
LIB_PATH = os.environ.get("DISMOEN_LIB") or os.path.join(PKG_ROOT, "libdismoen_hip.so")

DMH_F_DEVICE = 0x1
DMH_F_Q4K_PY_SCALES = 0x10
DMH_F_NORM_TREE = 0x20

ERROR_NAMES = {
    1: "INVALID_ARG", 2: "CONFIG", 3: "HIP", 4: "NO_MEMORY", 5: "DEQUANT", 6: "ACT",
    7: "WEIGHT", 8: "ROUTER", 9: "EXPERT", 10: "SWIGLU", 11: "GATE", 12: "NORM", 13: "FORMAT",
}

# every symbol include/dismoen_hip.h declares
EXPORTS = (
    "dmh_version", "dmh_create", "dmh_destroy", "dmh_set_stream", "dmh_get_stream", "dmh_sync",
    "dmh_upload_moe_layer", "dmh_free_layer", "dmh_layer_bytes", "dmh_moe_forward",
    "dmh_moe_stack_forward", "dmh_router_forward", "dmh_dequant_q4_bf16",
    "dmh_quant_open", "dmh_quant_close", "dmh_quant_num_tensors", "dmh_quant_find",
    "dmh_quant_tensor_info", "dmh_quant_read", "dmh_st_open", "dmh_st_close",
    "dmh_st_num_tensors", "dmh_st_find", "dmh_st_tensor_info", "dmh_st_read",
    "dmh_upload_moe_layer_files", "dmh_experts_forward", "dmh_shared_gate_forward",
    "dmh_moe_aggregate", "dmh_gguf_open", "dmh_gguf_close", "dmh_gguf_get_header",
    "dmh_gguf_num_tensors", "dmh_gguf_find", "dmh_gguf_tensor_info", "dmh_gguf_metadata",
    "dmh_gguf_read", "dmh_dequant_gguf", "dmh_gguf_stream_tensor_f32",
    "dmh_upload_moe_layer_gguf", "dmh_free_layer_gguf", "dmh_moe_forward_gguf",
    "dmh_set_layer_norm", "dmh_port_moe_forward", "dmh_moe_forward_noalloc",
    "dmh_set_spin_limit", "dmh_sync_fallbacks", "dmh_xcd_rotation",
)


class DmhDims(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("num_experts", C.c_int32), ("top_k", C.c_int32),
                ("inter", C.c_int32), ("inter_sh", C.c_int32), ("group_size", C.c_int32),
                ("norm_topk_prob", C.c_int32)]


class DmhWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "router_bf16", "shgate_bf16", "gu_scales", "gu_packed", "d_scales", "d_packed",
        "sh_gu_scales", "sh_gu_packed", "sh_d_scales", "sh_d_packed")]


class DmhTensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_char_p), ("ndim", C.c_int32),
                ("shape", C.c_int64 * 8), ("group_size", C.c_int32), ("num_groups", C.c_int64),
                ("scales_offset", C.c_int64), ("scales_bytes", C.c_int64),
                ("data_offset", C.c_int64), ("data_bytes", C.c_int64)]


class DmhGgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("ndim", C.c_int32), ("dims", C.c_int64 * 8),
                ("ggml_type", C.c_int32), ("offset", C.c_int64), ("file_offset", C.c_int64),
                ("num_elements", C.c_int64), ("raw_bytes", C.c_int64)]


class DmhGgufHeader(C.Structure):
    _fields_ = [("version", C.c_int32), ("tensor_count", C.c_int64),
                ("metadata_kv_count", C.c_int64), ("data_section_offset", C.c_int64),
                ("expected_file_size", C.c_int64), ("alignment", C.c_int64)]


class DismoenError(RuntimeError):
    """A nonzero status from the library; str() is the reference's error text."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code
        self.kind = ERROR_NAMES.get(code, str(code))


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libdismoen_hip.so not built ({LIB_PATH}); run __graft_entry__.build()")
    # One HIP runtime per process.  torch ships its own libamdhip64.so.7; the
    # library binds to whichever copy of that soname is loaded first, and
    # torch does not find a GPU through a runtime of another ROCm release.
    # Loading torch first makes both share torch's.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(LIB_PATH)
    vp, sz, i32, i64, u32 = C.c_void_p, C.c_size_t, C.c_int, C.c_int64, C.c_uint
    L.dmh_version.restype = C.c_char_p
    L.dmh_create.argtypes = [i32, C.POINTER(vp), C.c_char_p, sz]
    L.dmh_destroy.argtypes = [vp]
    L.dmh_set_stream.argtypes = [vp, vp]
    L.dmh_get_stream.argtypes = [vp]
    L.dmh_get_stream.restype = vp
    L.dmh_sync.argtypes = [vp, C.c_char_p, sz]
    L.dmh_set_spin_limit.argtypes = [vp, i64]
    L.dmh_sync_fallbacks.argtypes = [vp, C.POINTER(C.c_int64)]
    L.dmh_xcd_rotation.argtypes = [vp, i32]
    L.dmh_upload_moe_layer.argtypes = [vp, i32, C.POINTER(DmhDims), C.POINTER(DmhWeights), u32,
                                       C.c_char_p, sz]
    L.dmh_free_layer.argtypes = [vp, i32]
    L.dmh_layer_bytes.argtypes = [vp, i32, C.POINTER(C.c_int64)]
    L.dmh_moe_forward.argtypes = [vp, i32, vp, vp, i32, vp, vp, vp, vp, u32, C.c_char_p, sz]
    L.dmh_moe_forward_noalloc.argtypes = [vp, i32, vp, vp, i32, vp, vp, vp, vp, u32, C.c_char_p,
                                          sz]
    L.dmh_moe_stack_forward.argtypes = [vp, i32, i32, C.c_float, vp, i32, vp, vp, vp, u32,
                                        C.c_char_p, sz]
    L.dmh_router_forward.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, vp, u32,
                                     C.c_char_p, sz]
    L.dmh_dequant_q4_bf16.argtypes = [vp, vp, i64, vp, i64, i64, i32, vp, u32, C.c_char_p, sz]
    for pre in ("dmh_quant", "dmh_st"):
        getattr(L, pre + "_open").argtypes = [C.c_char_p, C.POINTER(vp), C.c_char_p, sz]
        getattr(L, pre + "_close").argtypes = [vp]
        getattr(L, pre + "_close").restype = None
        getattr(L, pre + "_num_tensors").argtypes = [vp]
        getattr(L, pre + "_find").argtypes = [vp, C.c_char_p]
        getattr(L, pre + "_tensor_info").argtypes = [vp, i32, C.POINTER(DmhTensorInfo)]
    L.dmh_quant_read.argtypes = [vp, i32, vp, i64, vp, i64, C.c_char_p, sz]
    L.dmh_st_read.argtypes = [vp, i32, vp, i64, C.c_char_p, sz]
    L.dmh_upload_moe_layer_files.argtypes = [vp, i32, C.POINTER(DmhDims), vp, vp, i32, C.c_char_p,
                                             sz]
    L.dmh_experts_forward.argtypes = [vp, i32, vp, i32, vp, i32, vp, vp, u32, C.c_char_p, sz]
    L.dmh_shared_gate_forward.argtypes = [vp, i32, vp, i32, vp, u32, C.c_char_p, sz]
    L.dmh_moe_aggregate.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, u32,
                                    C.c_char_p, sz]
    L.dmh_gguf_open.argtypes = [C.c_char_p, C.POINTER(vp), C.c_char_p, sz]
    L.dmh_gguf_close.argtypes = [vp]
    L.dmh_gguf_close.restype = None
    L.dmh_gguf_get_header.argtypes = [vp, C.POINTER(DmhGgufHeader)]
    L.dmh_gguf_num_tensors.argtypes = [vp]
    L.dmh_gguf_find.argtypes = [vp, C.c_char_p]
    L.dmh_gguf_tensor_info.argtypes = [vp, i32, C.POINTER(DmhGgufTensor)]
    L.dmh_gguf_metadata.argtypes = [vp, C.c_char_p]
    L.dmh_gguf_metadata.restype = C.c_char_p
    L.dmh_gguf_read.argtypes = [vp, i32, vp, i64, C.c_char_p, sz]
    L.dmh_dequant_gguf.argtypes = [vp, i32, vp, i64, i64, vp, u32, C.c_char_p, sz]
    L.dmh_gguf_stream_tensor_f32.argtypes = [vp, vp, C.c_char_p, vp, i64, u32, C.c_char_p, sz]
    L.dmh_upload_moe_layer_gguf.argtypes = [vp, i32, C.POINTER(DmhDims), vp, i32, u32,
                                            C.c_char_p, sz]
    L.dmh_free_layer_gguf.argtypes = [vp, i32]
    L.dmh_moe_forward_gguf.argtypes = [vp, i32, vp, vp, i32, vp, vp, vp, vp, u32, C.c_char_p, sz]
    L.dmh_set_layer_norm.argtypes = [vp, i32, vp, i32, u32, C.c_char_p, sz]
    L.dmh_port_moe_forward.argtypes = [vp, i32, vp, i32, C.c_float, vp, vp, vp, vp, u32,
                                       C.c_char_p, sz]
    _lib = L
    return L


def check(rc: int, buf) -> None:
    if rc:
        raise DismoenError(rc, buf.value.decode(errors="replace"))


def errbuf():
    return C.create_string_buffer(2048)
