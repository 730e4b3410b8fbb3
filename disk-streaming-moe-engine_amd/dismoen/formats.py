"""The reference's weight files: readers (over the C ABI) and writers.

Readers mirror src/format/quant_reader.mojo (scan_quant_file,
pread_tensor_quant) and src/format/reader.mojo (read_header); their errors
carry the reference's text.  Writers produce the same layouts:
  quant model   BlockHeader.to_header_bytes + BlockTensorMeta.to_record_bytes
                (quant_reader.mojo:56-94, 228-265): a 256-byte JSON header
                padded with spaces, then per tensor [u32 LE meta length][meta
                JSON][fp16 LE scales][packed codes];
  safetensors   [u64 LE header length][JSON header][payload].
"""
from __future__ import annotations

import ctypes as C
import json
import struct

import numpy as np

from ._lib import DismoenError, DmhTensorInfo, check, errbuf, lib


class FileTensor:
    def __init__(self, info: DmhTensorInfo):
        self.name = info.name.decode("utf-8", "replace")
        self.dtype = info.dtype.decode("utf-8", "replace")
        self.shape = [int(info.shape[i]) for i in range(info.ndim)]
        self.group_size = int(info.group_size)
        self.num_groups = int(info.num_groups)
        self.scales_offset = int(info.scales_offset)
        self.scales_bytes = int(info.scales_bytes)
        self.data_offset = int(info.data_offset)
        self.data_bytes = int(info.data_bytes)

    def num_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


class _Handle:
    _pre = ""

    def __init__(self, path: str):
        self._lib = lib()
        h = C.c_void_p()
        e = errbuf()
        check(getattr(self._lib, self._pre + "_open")(str(path).encode(), C.byref(h), e, len(e)), e)
        self._h = h
        self.path = str(path)
        n = getattr(self._lib, self._pre + "_num_tensors")(h)
        self.tensors = []
        for i in range(n):
            info = DmhTensorInfo()
            getattr(self._lib, self._pre + "_tensor_info")(h, i, C.byref(info))
            self.tensors.append(FileTensor(info))

    def find(self, name: str) -> int:
        return getattr(self._lib, self._pre + "_find")(self._h, name.encode())

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            getattr(self._lib, self._pre + "_close")(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class QuantModelIndex(_Handle):
    """scan_quant_file (src/format/quant_reader.mojo:487-662)."""
    _pre = "dmh_quant"

    def read(self, idx: int):
        """pread_tensor_quant: (fp16 scale bits uint16 [num_groups], packed uint8)."""
        t = self.tensors[idx]
        sc = np.empty(t.num_groups, np.uint16)
        pk = np.empty(t.data_bytes, np.uint8)
        e = errbuf()
        check(self._lib.dmh_quant_read(self._h, idx, sc.ctypes.data, sc.size, pk.ctypes.data,
                                       pk.size, e, len(e)), e)
        return sc, pk


class SafetensorsShard(_Handle):
    """read_header (src/format/reader.mojo:21-297)."""
    _pre = "dmh_st"

    def read(self, idx: int) -> bytes:
        t = self.tensors[idx]
        buf = C.create_string_buffer(max(t.data_bytes, 1))
        e = errbuf()
        check(self._lib.dmh_st_read(self._h, idx, buf, t.data_bytes, e, len(e)), e)
        return buf.raw[:t.data_bytes]


def scan_quant_file(path: str) -> QuantModelIndex:
    return QuantModelIndex(path)


def read_header(path: str) -> SafetensorsShard:
    return SafetensorsShard(path)


# ---- writers ------------------------------------------------------------------
def quant_header_bytes(model: str, num_tensors: int, total_bytes: int, group_size: int,
                       version: int = 1) -> bytes:
    js = json.dumps({"version": version, "model": model,
                     "quantization": {"format": "4-bit per-group", "group_size": group_size,
                                      "scale_dtype": "FP16"},
                     "num_tensors": num_tensors, "total_bytes": total_bytes},
                    separators=(",", ":")).encode()
    if len(js) > 256:
        raise ValueError(f"Header JSON exceeds 256 bytes: {len(js)} > 256")
    return js + b" " * (256 - len(js))


def quant_record_bytes(name: str, shape, scales: np.ndarray, packed: np.ndarray,
                       group_size: int, dtype: str = "BF16") -> bytes:
    n = int(np.prod(shape))
    ng = n // group_size
    js = json.dumps({"name": name, "shape": list(map(int, shape)), "dtype": dtype,
                     "quantized_dtype": "4-bit", "group_size": group_size, "num_groups": ng,
                     "scale_offset": 0, "data_offset": ng * 2},
                    separators=(",", ":")).encode()
    sc = np.ascontiguousarray(scales, dtype="<u2").tobytes()
    pk = np.ascontiguousarray(packed, dtype=np.uint8).tobytes()
    return struct.pack("<I", len(js)) + js + sc + pk


def write_quant_file(path: str, model: str, tensors, group_size: int) -> None:
    """tensors: iterable of (name, shape, fp16 scale bits, packed codes)."""
    recs = [quant_record_bytes(nm, sh, sc, pk, group_size) for nm, sh, sc, pk in tensors]
    total = 256 + sum(len(r) for r in recs)
    with open(path, "wb") as f:
        f.write(quant_header_bytes(model, len(recs), total, group_size))
        for r in recs:
            f.write(r)


def write_safetensors(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """tensors: name -> (dtype, shape, raw bytes), stored in insertion order."""
    hdr, off, blobs = {}, 0, []
    if metadata is not None:
        hdr["__metadata__"] = metadata
    for nm, (dt, shape, raw) in tensors.items():
        hdr[nm] = {"dtype": dt, "shape": list(map(int, shape)),
                   "data_offsets": [off, off + len(raw)]}
        off += len(raw)
        blobs.append(raw)
    js = json.dumps(hdr, separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(js)))
        f.write(js)
        for b in blobs:
            f.write(b)


def write_layer_files(quant_path: str, shard_path: str, L, model_layer: int = 0,
                      model: str = "dismoen-synthetic") -> None:
    """A layer in the reference layout (dismoen.synth.MoELayerQ4 fields) as a
    quant model (per-expert gate/up/down and the shared expert, the tensor
    names of src/layers/quant_loader.mojo:89-136) and a safetensors shard
    holding the bf16 router and shared-expert gate."""
    H, E, I, Ish, G = L.hidden, L.num_experts, L.inter, L.inter_sh, L.group_size
    gus = L.gu_scales.reshape(E, 2, I * H // G)
    gup = L.gu_packed.reshape(E, 2, I * H // 2)
    ds = L.d_scales.reshape(E, H * I // G)
    dp = L.d_packed.reshape(E, H * I // 2)
    sgs = L.sh_gu_scales.reshape(2, Ish * H // G)
    sgp = L.sh_gu_packed.reshape(2, Ish * H // 2)
    pre = f"model.layers.{model_layer}.mlp."
    ts = []
    for e in range(E):
        ts.append((pre + f"experts.{e}.gate_proj.weight", (I, H), gus[e, 0], gup[e, 0]))
        ts.append((pre + f"experts.{e}.up_proj.weight", (I, H), gus[e, 1], gup[e, 1]))
        ts.append((pre + f"experts.{e}.down_proj.weight", (H, I), ds[e], dp[e]))
    ts.append((pre + "shared_expert.gate_proj.weight", (Ish, H), sgs[0], sgp[0]))
    ts.append((pre + "shared_expert.up_proj.weight", (Ish, H), sgs[1], sgp[1]))
    ts.append((pre + "shared_expert.down_proj.weight", (H, Ish), L.sh_d_scales, L.sh_d_packed))
    write_quant_file(quant_path, model, ts, G)
    write_safetensors(shard_path, {
        pre + "gate.weight": ("BF16", (E, H), np.ascontiguousarray(L.router_bf16, "<u2").tobytes()),
        pre + "shared_expert_gate.weight": ("BF16", (1, H),
                                            np.ascontiguousarray(L.shgate_bf16, "<u2").tobytes()),
    })


__all__ = ["QuantModelIndex", "SafetensorsShard", "scan_quant_file", "read_header",
           "write_quant_file", "write_safetensors", "write_layer_files", "quant_header_bytes",
           "quant_record_bytes", "DismoenError"]
