"""GGUF files of the reference's Qwen3.6 port decode (src/format/gguf.mojo).

parse_gguf_index reads the container on the host (the C ABI's dmh_gguf_*);
stream_gguf_tensor_f32 and the dequantize_* functions turn a tensor's payload
into fp32 on the GPU (dmh_gguf_stream_tensor_f32, dmh_dequant_gguf).  The
block layouts are the reference's own: Q8_0 34 bytes / 32 weights, Q4_K 144
bytes / 256 weights (scales and mins of sub-blocks 4..7 as gguf.mojo:482-488
unpacks them; py_scales=True selects the packing of the reference's Python
twin, tools/oracle/oracle_port.py:104-110), Q3_K 114 bytes / 256 weights.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import (DMH_F_DEVICE, DMH_F_Q4K_PY_SCALES, DismoenError, DmhGgufHeader,
                   DmhGgufTensor, check, errbuf, lib)

GGML_TYPE_F32, GGML_TYPE_Q8_0, GGML_TYPE_Q3_K, GGML_TYPE_Q4_K, GGML_TYPE_BF16 = 0, 8, 11, 12, 30


class GGUFTensorInfo:
    """GGUFTensorInfo (gguf.mojo:104-114); offset relative to the data section."""

    def __init__(self, t: DmhGgufTensor):
        self.name = t.name.decode("utf-8", "replace")
        self.ndim = int(t.ndim)
        self.dims = [int(t.dims[i]) for i in range(min(self.ndim, 8))]
        self.dtype = int(t.ggml_type)
        self.offset = int(t.offset)
        self.file_offset = int(t.file_offset)
        self.num_elements = int(t.num_elements)
        self.raw_bytes = int(t.raw_bytes)


class GGUFIndex:
    """GGUFIndex (gguf.mojo:117-141), built by parse_gguf_index."""

    def __init__(self, path: str):
        self._lib = lib()
        h = C.c_void_p()
        e = errbuf()
        check(self._lib.dmh_gguf_open(str(path).encode(), C.byref(h), e, len(e)), e)
        self._h = h
        self.file_path = str(path)
        hd = DmhGgufHeader()
        self._lib.dmh_gguf_get_header(h, C.byref(hd))
        self.version = int(hd.version)
        self.tensor_count = int(hd.tensor_count)
        self.metadata_kv_count = int(hd.metadata_kv_count)
        self.data_section_offset = int(hd.data_section_offset)
        self.expected_file_size = int(hd.expected_file_size)
        self.alignment = int(hd.alignment)
        self.tensors = []
        for i in range(self._lib.dmh_gguf_num_tensors(h)):
            t = DmhGgufTensor()
            self._lib.dmh_gguf_tensor_info(h, i, C.byref(t))
            self.tensors.append(GGUFTensorInfo(t))
        self.tensor_map = {}
        for t in self.tensors:
            self.tensor_map[t.name] = self._lib.dmh_gguf_find(h, t.name.encode())

    def metadata(self, key: str):
        v = self._lib.dmh_gguf_metadata(self._h, key.encode())
        return None if v is None else v.decode("utf-8", "replace")

    def read_raw(self, name: str) -> np.ndarray:
        idx = self.tensor_map[name]
        t = self.tensors[idx]
        out = np.empty(max(t.raw_bytes, 1), np.uint8)
        e = errbuf()
        check(self._lib.dmh_gguf_read(self._h, idx, out.ctypes.data, t.raw_bytes, e, len(e)), e)
        return out[:t.raw_bytes]

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            self._lib.dmh_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def parse_gguf_index(file_path: str) -> GGUFIndex:
    return GGUFIndex(file_path)


# ---- writer -----------------------------------------------------------------
def write_gguf(path: str, tensors, metadata=None, alignment: int = 32, version: int = 3) -> None:
    """A GGUF file as parse_gguf_index reads it: tensors is a list of (name,
    dims, ggml_type, raw payload bytes), stored in order at `alignment`-byte
    offsets of the data section; metadata maps keys to str or int (u32)."""
    import struct
    meta = dict(metadata or {})
    if alignment != 32:
        meta["general.alignment"] = alignment

    def gstr(v: str) -> bytes:
        b = v.encode()
        return struct.pack("<Q", len(b)) + b

    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta)))
    for k, v in meta.items():
        out += gstr(k)
        out += struct.pack("<I", 8) + gstr(v) if isinstance(v, str) else struct.pack("<II", 4, v)
    off = 0
    offs = []
    for name, dims, ty, raw in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        out += gstr(name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", int(d)) for d in dims) + struct.pack("<IQ", ty, off)
        off += len(raw)
    out += b"\0" * ((-len(out)) % alignment)
    base = len(out)
    with open(path, "wb") as f:
        f.write(out)
        for (name, dims, ty, raw), o in zip(tensors, offs):
            pos = base + o
            cur = f.tell()
            if pos > cur:
                f.write(b"\0" * (pos - cur))
            f.write(bytes(raw))


def _flags(py_scales: bool) -> int:
    return DMH_F_Q4K_PY_SCALES if py_scales else 0


def stream_gguf_tensor_f32(index: GGUFIndex, tensor_name: str, block,
                           py_scales: bool = False) -> np.ndarray:
    """stream_gguf_tensor_f32 (gguf.mojo:563-626): one tensor, read from the
    file and dequantized on the GPU of `block` (a dismoen.MoEBlock)."""
    idx = index._lib.dmh_gguf_find(index.handle, tensor_name.encode())
    n = index.tensors[idx].num_elements if idx >= 0 else 0
    out = np.empty(max(n, 1), np.float32)
    e = errbuf()
    check(index._lib.dmh_gguf_stream_tensor_f32(block.handle, index.handle, tensor_name.encode(),
                                                out.ctypes.data, n, _flags(py_scales), e, len(e)),
          e)
    return out[:n]


def dequantize(ggml_type: int, raw_bytes, num_elements: int, block,
               py_scales: bool = False) -> np.ndarray:
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw_bytes), np.uint8)
                               if not isinstance(raw_bytes, np.ndarray) else raw_bytes,
                               dtype=np.uint8).ravel()
    out = np.empty(max(int(num_elements), 1), np.float32)
    e = errbuf()
    check(lib().dmh_dequant_gguf(block.handle, ggml_type, raw.ctypes.data if raw.size else None,
                                 raw.size, num_elements, out.ctypes.data, _flags(py_scales), e,
                                 len(e)), e)
    return out[:num_elements]


def dequantize_q8_0(raw_bytes, num_elements: int, block) -> np.ndarray:
    """dequantize_q8_0 (gguf.mojo:414-441)."""
    return dequantize(GGML_TYPE_Q8_0, raw_bytes, num_elements, block)


def dequantize_q4_k(raw_bytes, num_elements: int, block, py_scales: bool = False) -> np.ndarray:
    """dequantize_q4_k (gguf.mojo:444-506)."""
    return dequantize(GGML_TYPE_Q4_K, raw_bytes, num_elements, block, py_scales)


def dequantize_q3_k(raw_bytes, num_elements: int, block) -> np.ndarray:
    """dequantize_q3_k (gguf.mojo:509-560)."""
    return dequantize(GGML_TYPE_Q3_K, raw_bytes, num_elements, block)


def dequantize_device(ggml_type: int, raw_ptr: int, raw_bytes: int, num_elements: int,
                      out_ptr: int, block, py_scales: bool = False) -> None:
    """Device pointers (raw 4-byte, out 16-byte aligned), ordered on the
    block's stream; no synchronisation."""
    e = errbuf()
    check(lib().dmh_dequant_gguf(block.handle, ggml_type, raw_ptr, raw_bytes, num_elements,
                                 out_ptr, DMH_F_DEVICE | _flags(py_scales), e, len(e)), e)


__all__ = ["GGUFIndex", "GGUFTensorInfo", "parse_gguf_index", "stream_gguf_tensor_f32",
           "dequantize", "dequantize_q8_0", "dequantize_q4_k", "dequantize_q3_k",
           "dequantize_device", "DismoenError", "GGML_TYPE_F32", "GGML_TYPE_Q8_0",
           "GGML_TYPE_Q3_K", "GGML_TYPE_Q4_K", "GGML_TYPE_BF16"]
