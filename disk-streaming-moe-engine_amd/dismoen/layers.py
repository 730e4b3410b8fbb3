"""Host-side mirror of the reference's MoE layer interface over libdismoen_hip.so.

Names, argument meaning and errors follow the Mojo sources:
  RouterConfig / RoutingInfo      src/layers/router_types.mojo:9-81
  router_forward                  src/layers/router.mojo:188-210
  dequant_kernel_simd             src/quant/dequant_kernel.mojo:22-124
  forward_moe_block               src/layers/moe_block.mojo:20-138
  moe_combine_no_residual         src/layers/forward_layer.mojo:181-247
  forward_port_block MoE section  src/layers/port_scheduler.mojo:381-482
Errors surface as DismoenError whose text is the reference's JSON error.
All compute runs in the HIP library; nothing here computes a result.
"""
from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass, field

import numpy as np

from ._lib import (DMH_F_DEVICE, DMH_F_NORM_TREE, DMH_F_Q4K_PY_SCALES, DismoenError, DmhDims,
                   DmhWeights, check, errbuf, lib)


@dataclass
class RouterConfig:
    """src/layers/router_types.mojo:9-44"""
    num_experts: int
    num_experts_per_tok: int
    norm_topk_prob: bool = False

    def validate(self) -> None:
        def err(kind, detail):
            return DismoenError(2 if kind == "CONFIG_ERROR" else 8, json.dumps(
                {"error_type": kind, "detail": detail, "stage": "router"},
                separators=(",", ":")))
        if self.num_experts <= 0:
            raise err("CONFIG_ERROR", "num_experts must be positive")
        if self.num_experts_per_tok <= 0:
            raise err("CONFIG_ERROR", "num_experts_per_tok must be positive")
        if self.num_experts_per_tok > self.num_experts:
            raise err("CONFIG_ERROR", "num_experts_per_tok cannot exceed num_experts")
        if self.norm_topk_prob:
            raise err("ROUTER_ERROR", "norm_topk_prob=true forbidden; unrenormalized routing"
                      " invariant violated")


@dataclass
class RoutingInfo:
    """src/layers/router_types.mojo:47-81"""
    selected_experts: list = field(default_factory=list)
    router_probs: list = field(default_factory=list)
    num_tokens: int = 0
    top_k: int = 0

    @staticmethod
    def from_arrays(ids: np.ndarray, probs: np.ndarray) -> "RoutingInfo":
        return RoutingInfo([list(map(int, r)) for r in ids],
                           [list(map(float, r)) for r in probs.astype(np.float32)],
                           int(ids.shape[0]), int(ids.shape[1]))

    def to_json(self) -> str:
        sel = ",".join("[" + ",".join(str(e) for e in r) + "]" for r in self.selected_experts)
        pr = ",".join("[" + ",".join(repr(float(np.float32(p))) for p in r) + "]"
                      for r in self.router_probs)
        return '{"selected_experts":[' + sel + '],"router_probs":[' + pr + "]}"


def _ptr(a) -> int:
    return a.ctypes.data if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


_F32, _I32 = np.dtype(np.float32), np.dtype(np.int32)


class MoEBlock:
    """One device context: uploaded layers + the block entry points."""

    def __init__(self, device: int = 0):
        self._lib = lib()
        h = C.c_void_p()
        e = errbuf()
        check(self._lib.dmh_create(device, C.byref(h), e, len(e)), e)
        self._h = h
        self.dims = {}
        self.gguf_dims = {}
        self._ebuf = None  # error buffer reused by forward_into

    # -- lifetime --------------------------------------------------------
    def close(self):
        if getattr(self, "_h", None):
            self._lib.dmh_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def handle(self):
        return self._h

    def set_stream(self, stream_ptr: int | None):
        self._lib.dmh_set_stream(self._h, stream_ptr)

    def stream(self) -> int:
        return self._lib.dmh_get_stream(self._h) or 0

    def sync(self):
        e = errbuf()
        check(self._lib.dmh_sync(self._h, e, len(e)), e)

    def set_spin_limit(self, polls: int | None) -> None:
        """Bound of every wait between the workgroups of the single-token
        kernels (None: the default, 2^20 polls; 0: every wait gives up)."""
        rc = self._lib.dmh_set_spin_limit(self._h, -1 if polls is None else int(polls))
        if rc:
            raise DismoenError(rc, "dmh_set_spin_limit failed")

    def sync_fallbacks(self) -> int:
        """Host-pointer calls rerun on the multi-kernel path after a wait
        of a single-token kernel gave up."""
        n = C.c_int64()
        rc = self._lib.dmh_sync_fallbacks(self._h, C.byref(n))
        if rc:
            raise DismoenError(rc, "dmh_sync_fallbacks failed")
        return int(n.value)

    # -- weights ---------------------------------------------------------
    def upload_layer(self, layer_idx: int, L, norm_topk_prob: bool = False) -> None:
        """Upload a layer given in the reference 4-bit layout (dismoen.synth.MoELayerQ4
        or any object with the same fields)."""
        d = DmhDims(L.hidden, L.num_experts, L.top_k, L.inter, L.inter_sh, L.group_size,
                    int(norm_topk_prob))
        arrs = {}
        w = DmhWeights()
        for name, dt in (("router_bf16", np.uint16), ("shgate_bf16", np.uint16),
                         ("gu_scales", np.uint16), ("gu_packed", np.uint8),
                         ("d_scales", np.uint16), ("d_packed", np.uint8),
                         ("sh_gu_scales", np.uint16), ("sh_gu_packed", np.uint8),
                         ("sh_d_scales", np.uint16), ("sh_d_packed", np.uint8)):
            a = np.ascontiguousarray(getattr(L, name), dtype=dt)
            arrs[name] = a
            setattr(w, name, a.ctypes.data)
        e = errbuf()
        check(self._lib.dmh_upload_moe_layer(self._h, layer_idx, C.byref(d), C.byref(w), 0, e,
                                             len(e)), e)
        self.dims[layer_idx] = (L.hidden, L.num_experts, L.top_k, L.inter, L.inter_sh)

    def upload_layer_device(self, layer_idx: int, dims: tuple, ptrs: dict,
                            group_size: int = 32) -> None:
        """Upload from device buffers (ptrs: field name -> device address)."""
        H, E, K, I, Ish = dims
        d = DmhDims(H, E, K, I, Ish, group_size, 0)
        w = DmhWeights(**ptrs)
        e = errbuf()
        check(self._lib.dmh_upload_moe_layer(self._h, layer_idx, C.byref(d), C.byref(w),
                                             DMH_F_DEVICE, e, len(e)), e)
        self.dims[layer_idx] = dims

    def upload_layer_files(self, layer_idx: int, dims: tuple, quant, shard,
                           model_layer: int = 0, group_size: int = 32) -> None:
        """Upload model layer model_layer from a quant model and a safetensors
        shard (dismoen.formats.QuantModelIndex / SafetensorsShard); group_size is
        the group size of the quant model's expert tensors (32, 64, 128 or 256;
        0: quantization.group_size of the quant model's header)."""
        H, E, K, I, Ish = dims
        d = DmhDims(H, E, K, I, Ish, group_size, 0)
        e = errbuf()
        check(self._lib.dmh_upload_moe_layer_files(self._h, layer_idx, C.byref(d), quant.handle,
                                                   shard.handle, model_layer, e, len(e)), e)
        self.dims[layer_idx] = dims

    # -- GGUF layers (slots of their own) ---------------------------------
    def upload_layer_gguf(self, layer_idx: int, dims: tuple, index, model_layer: int = 0,
                          py_scales: bool = False) -> None:
        """load_port_block_from_gguf's MoE tensors of model layer model_layer
        (src/layers/gguf_port_loader.mojo:207-256) from a dismoen.gguf.GGUFIndex;
        dims = (hidden, num_experts, top_k, inter, inter_sh)."""
        H, E, K, I, Ish = dims
        d = DmhDims(H, E, K, I, Ish, 32, 0)
        e = errbuf()
        check(self._lib.dmh_upload_moe_layer_gguf(self._h, layer_idx, C.byref(d), index.handle,
                                                  model_layer,
                                                  DMH_F_Q4K_PY_SCALES if py_scales else 0, e,
                                                  len(e)), e)
        self.gguf_dims[layer_idx] = dims

    def free_layer_gguf(self, layer_idx: int) -> None:
        self._lib.dmh_free_layer_gguf(self._h, layer_idx)
        self.gguf_dims.pop(layer_idx, None)

    def forward_port_moe_gguf(self, norm_x, x_mid, layer_idx: int, seq_len: int):
        """MoE section of forward_port_block (port_scheduler.mojo:381-482) on a
        GGUF layer: (y [seq_len][H], ids, probs, shared gate) as numpy arrays."""
        H, E, K, I, Ish = self.gguf_dims[layer_idx]
        x = _f32(norm_x).reshape(-1)
        res = None if x_mid is None else _f32(x_mid).reshape(-1)
        y = np.empty(seq_len * H, np.float32)
        ids = np.empty(seq_len * K, np.int32)
        probs = np.empty(seq_len * K, np.float32)
        shg = np.empty(seq_len, np.float32)
        e = errbuf()
        check(self._lib.dmh_moe_forward_gguf(self._h, layer_idx, x.ctypes.data, _ptr(res),
                                             seq_len, y.ctypes.data, ids.ctypes.data,
                                             probs.ctypes.data, shg.ctypes.data, 0, e, len(e)), e)
        return (y.reshape(seq_len, H), ids.reshape(seq_len, K), probs.reshape(seq_len, K), shg)

    def forward_gguf_device(self, layer_idx: int, x_ptr: int, seq_len: int, y_ptr: int,
                            ids_ptr: int | None = None, probs_ptr: int | None = None,
                            residual_ptr: int | None = None) -> None:
        """Stream-ordered call on device buffers; errors are reported by sync()."""
        e = errbuf()
        check(self._lib.dmh_moe_forward_gguf(self._h, layer_idx, x_ptr, residual_ptr, seq_len,
                                             y_ptr, ids_ptr, probs_ptr, None, DMH_F_DEVICE, e,
                                             len(e)), e)

    def free_layer(self, layer_idx: int) -> None:
        self._lib.dmh_free_layer(self._h, layer_idx)
        self.dims.pop(layer_idx, None)

    def layer_bytes(self, layer_idx: int) -> int:
        v = C.c_int64()
        if self._lib.dmh_layer_bytes(self._h, layer_idx, C.byref(v)):
            raise DismoenError(1, f"layer {layer_idx} not uploaded")
        return v.value

    # -- the block -------------------------------------------------------
    def _forward(self, layer_idx, x, residual, seq_len):
        H, E, K, I, Ish = self.dims[layer_idx]
        x = _f32(x).reshape(-1)
        res = None if residual is None else _f32(residual).reshape(-1)
        y = np.empty(seq_len * H, np.float32)
        ids = np.empty(seq_len * K, np.int32)
        probs = np.empty(seq_len * K, np.float32)
        shg = np.empty(seq_len, np.float32)
        e = errbuf()
        check(self._lib.dmh_moe_forward(self._h, layer_idx, x.ctypes.data, _ptr(res), seq_len,
                                        y.ctypes.data, ids.ctypes.data, probs.ctypes.data,
                                        shg.ctypes.data, 0, e, len(e)), e)
        return (y.reshape(seq_len, H), ids.reshape(seq_len, K), probs.reshape(seq_len, K), shg)

    def forward_moe_block(self, x, layer_idx: int, seq_len: int):
        """forward_moe_block: y = sum_k p_k E_k(x) + sigmoid(g_sh) E_sh(x) + x.
        Returns (y [seq_len*H] float32, RoutingInfo)."""
        y, ids, probs, _ = self._forward(layer_idx, x, x, seq_len)
        return y.reshape(-1), RoutingInfo.from_arrays(ids, probs)

    def moe_combine_no_residual(self, x, layer_idx: int, seq_len: int):
        """The same block without the residual (src/layers/forward_layer.mojo:181-247)."""
        y, ids, probs, _ = self._forward(layer_idx, x, None, seq_len)
        return y.reshape(-1), RoutingInfo.from_arrays(ids, probs)

    def forward_port_moe(self, norm_x, x_mid, layer_idx: int, seq_len: int):
        """MoE section of forward_port_block: router/experts on norm_x, residual x_mid."""
        y, ids, probs, _ = self._forward(layer_idx, norm_x, x_mid, seq_len)
        return y.reshape(-1), RoutingInfo.from_arrays(ids, probs)

    def forward_arrays(self, layer_idx: int, x, seq_len: int, residual=None):
        """(y, ids, probs, shared_gate) as numpy arrays."""
        return self._forward(layer_idx, x, residual, seq_len)

    def forward_into(self, layer_idx: int, x, seq_len: int, y, ids=None, probs=None, shg=None,
                     residual=None) -> None:
        """Host-pointer call into caller-owned outputs, as a compiled caller
        makes it: x, residual, y, probs, shg C-contiguous float32, ids int32,
        of the call's sizes (checked here); nothing is allocated per call."""
        H, E, K, I, Ish = self.dims[layer_idx]
        nh, nk = seq_len * H, seq_len * K
        for a, dt, n in ((x, _F32, nh), (y, _F32, nh), (residual, _F32, nh), (ids, _I32, nk),
                         (probs, _F32, nk), (shg, _F32, seq_len)):
            if a is not None and (a.dtype != dt or a.size < n or not a.flags.c_contiguous):
                raise ValueError(f"forward_into: arrays must be C-contiguous {np.dtype(dt)}"
                                 f" with at least {n} elements")
        e = self._ebuf
        if e is None:
            e = self._ebuf = errbuf()
        check(self._lib.dmh_moe_forward(self._h, layer_idx, x.ctypes.data, _ptr(residual), seq_len,
                                        y.ctypes.data, _ptr(ids), _ptr(probs), _ptr(shg), 0, e,
                                        len(e)), e)

    def forward_device(self, layer_idx: int, x_ptr: int, seq_len: int, y_ptr: int,
                       ids_ptr: int | None = None, probs_ptr: int | None = None,
                       shg_ptr: int | None = None, residual_ptr: int | None = None) -> None:
        """Stream-ordered call on device buffers; errors are reported by sync()."""
        e = errbuf()
        check(self._lib.dmh_moe_forward(self._h, layer_idx, x_ptr, residual_ptr, seq_len, y_ptr,
                                        ids_ptr, probs_ptr, shg_ptr, DMH_F_DEVICE, e, len(e)), e)

    # -- the port block's MoE section with its RMSNorm ----------------------
    def set_layer_norm(self, layer_idx: int, gamma) -> None:
        """post_attention_layernorm_gamma of layer layer_idx (None: gamma = 1)."""
        H = self.dims[layer_idx][0]
        g = None if gamma is None else _f32(gamma).reshape(-1)
        e = errbuf()
        check(self._lib.dmh_set_layer_norm(self._h, layer_idx, _ptr(g),
                                           H if g is None else g.size, 0, e, len(e)), e)

    def forward_port_moe_norm(self, x_mid, layer_idx: int, seq_len: int, eps: float = 1e-6,
                              tree: bool = False):
        """MoE section of forward_port_block including its RMSNorm
        (port_scheduler.mojo:381-482): (y = x_mid + MoE(rmsnorm(x_mid)), ids,
        probs, shared gate) as numpy arrays."""
        H, E, K, I, Ish = self.dims[layer_idx]
        x = _f32(x_mid).reshape(-1)
        y = np.empty(seq_len * H, np.float32)
        ids = np.empty(seq_len * K, np.int32)
        probs = np.empty(seq_len * K, np.float32)
        shg = np.empty(seq_len, np.float32)
        e = errbuf()
        check(self._lib.dmh_port_moe_forward(self._h, layer_idx, x.ctypes.data, seq_len, eps,
                                             y.ctypes.data, ids.ctypes.data, probs.ctypes.data,
                                             shg.ctypes.data, DMH_F_NORM_TREE if tree else 0, e,
                                             len(e)), e)
        return (y.reshape(seq_len, H), ids.reshape(seq_len, K), probs.reshape(seq_len, K), shg)

    def forward_port_moe_norm_device(self, layer_idx: int, x_ptr: int, seq_len: int, y_ptr: int,
                                     eps: float = 1e-6, ids_ptr=None, probs_ptr=None,
                                     shg_ptr=None, tree: bool = False) -> None:
        e = errbuf()
        fl = DMH_F_DEVICE | (DMH_F_NORM_TREE if tree else 0)
        check(self._lib.dmh_port_moe_forward(self._h, layer_idx, x_ptr, seq_len, eps, y_ptr,
                                             ids_ptr, probs_ptr, shg_ptr, fl, e, len(e)), e)

    def forward_stack(self, x, first_layer: int, num_layers: int, seq_len: int,
                      eps: float = 1e-6, tree: bool = False):
        """num_layers port MoE sections in sequence (identity mixers); tree=True
        sums the norm's squares in the fast tree order."""
        H, E, K, I, Ish = self.dims[first_layer]
        x = _f32(x).reshape(-1)
        out = np.empty(seq_len * H, np.float32)
        ids = np.empty(num_layers * seq_len * K, np.int32)
        probs = np.empty(num_layers * seq_len * K, np.float32)
        e = errbuf()
        check(self._lib.dmh_moe_stack_forward(self._h, first_layer, num_layers, eps,
                                              x.ctypes.data, seq_len, out.ctypes.data,
                                              ids.ctypes.data, probs.ctypes.data,
                                              DMH_F_NORM_TREE if tree else 0, e, len(e)),
              e)
        return (out.reshape(seq_len, H), ids.reshape(num_layers, seq_len, K),
                probs.reshape(num_layers, seq_len, K))

    def forward_stack_device(self, x_ptr: int, first_layer: int, num_layers: int, seq_len: int,
                             out_ptr: int, eps: float = 1e-6, ids_ptr=None, probs_ptr=None,
                             tree: bool = False):
        e = errbuf()
        fl = DMH_F_DEVICE | (DMH_F_NORM_TREE if tree else 0)
        check(self._lib.dmh_moe_stack_forward(self._h, first_layer, num_layers, eps, x_ptr,
                                              seq_len, out_ptr, ids_ptr, probs_ptr, fl,
                                              e, len(e)), e)

    # -- unit entry points ---------------------------------------------
    def router_forward(self, x, w_router, seq_len: int, hidden_dim: int, cfg: RouterConfig,
                       layer_idx: int = 0) -> RoutingInfo:
        """router_forward with fp32 router weights [E][H]."""
        x = _f32(x).reshape(-1)
        w = _f32(w_router).reshape(-1)
        K, E = cfg.num_experts_per_tok, cfg.num_experts
        n = max(seq_len, 1) * max(K, 1)
        ids = np.zeros(n, np.int32)
        probs = np.zeros(n, np.float32)
        e = errbuf()
        check(self._lib.dmh_router_forward(self._h, x.ctypes.data, w.ctypes.data, seq_len,
                                           hidden_dim, E, K, int(cfg.norm_topk_prob), layer_idx,
                                           ids.ctypes.data, probs.ctypes.data, 0, e, len(e)), e)
        return RoutingInfo.from_arrays(ids.reshape(seq_len, K), probs.reshape(seq_len, K))

    def experts_forward(self, x, ids, layer_idx: int, seq_len: int, with_shared: bool = False):
        """The SwiGLU experts ids [seq_len][k] of an uploaded layer on x, unweighted:
        (out [seq_len][k][H], shared [seq_len][H] or None)."""
        H = self.dims[layer_idx][0]
        x = _f32(x).reshape(-1)
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(seq_len, -1)
        k = ids.shape[1]
        out = np.empty(seq_len * k * H, np.float32)
        sh = np.empty(seq_len * H, np.float32) if with_shared else None
        e = errbuf()
        check(self._lib.dmh_experts_forward(self._h, layer_idx, x.ctypes.data, seq_len,
                                            ids.ctypes.data, k, out.ctypes.data, _ptr(sh), 0, e,
                                            len(e)), e)
        return out.reshape(seq_len, k, H), None if sh is None else sh.reshape(seq_len, H)

    def parallel_moe_experts(self, x_tok, selected_experts, layer_idx: int) -> np.ndarray:
        """WorkerPool.parallel_moe_experts for one token: out_routed [top_k*H]."""
        out, _ = self.experts_forward(x_tok, np.asarray(selected_experts).reshape(1, -1),
                                      layer_idx, 1)
        return out.reshape(-1)

    def swiglu_forward(self, x, seq_len: int, layer_idx: int = 0, expert_id: int = -1):
        """swiglu_forward with an uploaded layer's expert expert_id (-1: the shared
        expert): y [seq_len*H]."""
        if expert_id < 0:
            _, sh = self.experts_forward(x, np.zeros((seq_len, 1), np.int32), layer_idx,
                                         seq_len, with_shared=True)
            return sh.reshape(-1)
        out, _ = self.experts_forward(x, np.full((seq_len, 1), expert_id, np.int32), layer_idx,
                                      seq_len)
        return out.reshape(-1)

    def shared_gate_forward(self, x, seq_len: int, layer_idx: int = 0,
                            gate_mode: str = "sigmoid") -> np.ndarray:
        """shared_gate_forward with the uploaded layer's gate vector: scores [seq_len]."""
        if gate_mode != "sigmoid":
            raise DismoenError(11, '{"error_type":"GATE_ERROR","detail":"shared expert gate must'
                                  ' be sigmoid; non-sigmoid gate forbidden (invariant #2)",'
                                  f'"stage":"shared","layer":{layer_idx}}}')
        x = _f32(x).reshape(-1)
        scores = np.empty(max(seq_len, 1), np.float32)
        e = errbuf()
        check(self._lib.dmh_shared_gate_forward(self._h, layer_idx, x.ctypes.data, seq_len,
                                                scores.ctypes.data, 0, e, len(e)), e)
        return scores[:seq_len]

    def _aggregate(self, x, routed_outputs, router_probs, shared_output, shared_gate_scores,
                   seq_len: int, hidden_dim: int, layer_idx: int):
        def err(detail):
            return DismoenError(9, '{"error_type":"EXPERT_ERROR","detail":"' + detail +
                                '","stage":"aggregation","layer":' + str(layer_idx) + "}")
        if seq_len <= 0 or hidden_dim <= 0:
            raise err("dimensions must be positive")
        sh = _f32(shared_output).reshape(-1)
        if (x is not None and _f32(x).size != seq_len * hidden_dim) or sh.size != seq_len * hidden_dim:
            raise err("length mismatch in aggregation")
        g = _f32(shared_gate_scores).reshape(-1)
        if g.size != seq_len or len(routed_outputs) != seq_len:
            raise err("sequence length mismatch")
        probs = _f32(np.asarray(router_probs, dtype=np.float32).reshape(seq_len, -1))
        k = probs.shape[1]
        routed = _f32(np.asarray(routed_outputs, dtype=np.float32).reshape(seq_len, k * hidden_dim))
        res = None if x is None else _f32(x).reshape(-1)
        y = np.empty(seq_len * hidden_dim, np.float32)
        e = errbuf()
        check(self._lib.dmh_moe_aggregate(self._h, _ptr(res), routed.ctypes.data,
                                          probs.ctypes.data, sh.ctypes.data, g.ctypes.data,
                                          seq_len, hidden_dim, k, layer_idx, y.ctypes.data, 0, e,
                                          len(e)), e)
        return y

    def moe_aggregate_forward(self, x, routed_outputs, router_probs, shared_output,
                              shared_gate_scores, seq_len: int, hidden_dim: int,
                              layer_idx: int = 0) -> np.ndarray:
        """moe_aggregate_forward on given parts: y [seq_len*H]."""
        return self._aggregate(x, routed_outputs, router_probs, shared_output,
                               shared_gate_scores, seq_len, hidden_dim, layer_idx)

    def combine_no_residual(self, routed_outputs, router_probs, shared_output,
                            shared_gate_scores, seq_len: int, hidden_dim: int,
                            layer_idx: int = 0) -> np.ndarray:
        """moe_combine_no_residual (src/layers/forward_layer.mojo:181-247) on given parts."""
        return self._aggregate(None, routed_outputs, router_probs, shared_output,
                               shared_gate_scores, seq_len, hidden_dim, layer_idx)

    def dequant_kernel_simd(self, scales, packed_weights, num_elements: int,
                            group_size: int = 128) -> np.ndarray:
        """Returns bf16 bit patterns (uint16) of bf16(fp32(s_g) * q)."""
        s = np.ascontiguousarray(scales, dtype=np.uint16).reshape(-1)
        p = np.ascontiguousarray(packed_weights, dtype=np.uint8).reshape(-1)
        out = np.empty(max(int(num_elements), 1), np.uint16)
        e = errbuf()
        check(self._lib.dmh_dequant_q4_bf16(self._h, s.ctypes.data, s.size, p.ctypes.data,
                                            p.size, num_elements, group_size, out.ctypes.data, 0,
                                            e, len(e)), e)
        return out[:num_elements]
