"""Seeded synthetic MoE layers in the reference's 4-bit tensor layout.

Layout (src/format/quant_reader.mojo:171-341, docs/format/quant_format.md:117-161):
each 4-bit tensor is fp16 little-endian group scales [N/G] followed by packed
bytes [N/2]; element i sits in byte i//2, low nibble for even i; groups run
over the flattened row-major index, i.e. along the input dimension.  Codes are
signed two's-complement int4 in [-7, 7]; nibble 0x8 is reserved.

Distributions:
  scales   fp16_rne(|N(0, 0.02)| / 7.5), clamped to >= 0x0001 (the smallest
           positive fp16) because the reference rejects non-positive scales
           (src/quant/dequant_kernel.mojo:68-80);
  codes    uniform over the 15 valid values {-7..7} (the "zero point 8" of an
           offset-binary reading: u = q + 8 in [1, 15]);
  router   bf16(N(0, 0.02)) [E, H]; shared-expert gate bf16(N(0, 0.02)) [H];
  x        bf16(N(0, 1)), returned as float32.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# byte value for each of the 225 (q0, q1) pairs: v = (q0 + 7) + 15 * (q1 + 7)
_PAIR_LUT = np.array(
    [((q0 & 0xF) | ((q1 & 0xF) << 4)) for q1 in range(-7, 8) for q0 in range(-7, 8)],
    dtype=np.uint8)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (finite input)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    return (r >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def make_scales(rng: np.random.Generator, n: int) -> np.ndarray:
    s = np.abs(rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)) / np.float32(7.5)
    h = s.astype(np.float16).view(np.uint16).copy()
    h[h == 0] = 1
    return h


def make_codes_packed(rng: np.random.Generator, n: int) -> np.ndarray:
    """n codes (n even) uniform over {-7..7}, packed two per byte."""
    v = rng.integers(0, 225, size=n // 2, dtype=np.uint8)
    return _PAIR_LUT[v]


def make_activations(rng: np.random.Generator, shape) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32)))


@dataclass
class MoELayerQ4:
    hidden: int
    num_experts: int
    top_k: int
    inter: int
    inter_sh: int
    group_size: int
    router_bf16: np.ndarray   # [E*H] uint16
    shgate_bf16: np.ndarray   # [H] uint16
    gu_scales: np.ndarray     # [E*2I*H/G] uint16 (fp16 bits)
    gu_packed: np.ndarray     # [E*2I*H/2] uint8
    d_scales: np.ndarray      # [E*H*I/G]
    d_packed: np.ndarray      # [E*H*I/2]
    sh_gu_scales: np.ndarray  # [2Ish*H/G]
    sh_gu_packed: np.ndarray
    sh_d_scales: np.ndarray   # [H*Ish/G]
    sh_d_packed: np.ndarray


def make_layer(hidden: int, num_experts: int, top_k: int, inter: int, inter_sh: int,
               group_size: int = 32, seed: int = 0) -> MoELayerQ4:
    H, E, I, Ish, G = hidden, num_experts, inter, inter_sh, group_size
    rng = np.random.default_rng(seed)
    router = f32_to_bf16_bits(rng.standard_normal(E * H, dtype=np.float32) * np.float32(0.02))
    shgate = f32_to_bf16_bits(rng.standard_normal(H, dtype=np.float32) * np.float32(0.02))
    gu_s = make_scales(rng, E * 2 * I * H // G)
    gu_p = make_codes_packed(rng, E * 2 * I * H)
    d_s = make_scales(rng, E * H * I // G)
    d_p = make_codes_packed(rng, E * H * I)
    sgu_s = make_scales(rng, 2 * Ish * H // G)
    sgu_p = make_codes_packed(rng, 2 * Ish * H)
    sd_s = make_scales(rng, H * Ish // G)
    sd_p = make_codes_packed(rng, H * Ish)
    return MoELayerQ4(H, E, top_k, I, Ish, G, router, shgate, gu_s, gu_p, d_s, d_p,
                      sgu_s, sgu_p, sd_s, sd_p)


# The five workloads (hidden, experts, top_k, inter, inter_sh).
CONFIG_TOY = dict(hidden=256, num_experts=16, top_k=4, inter=128, inter_sh=128)
CONFIG_QWEN36 = dict(hidden=2048, num_experts=256, top_k=8, inter=512, inter_sh=512)


def zipf_router_bias(num_experts: int, s: float = 1.1, seed: int = 0) -> np.ndarray:
    """log-popularity of Zipf(s) over a seeded permutation of the experts."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(num_experts)
    ranks = np.empty(num_experts, np.float64)
    ranks[perm] = np.arange(1, num_experts + 1)
    return (-s * np.log(ranks)).astype(np.float32)


def with_router_bias(L: MoELayerQ4, bias: np.ndarray) -> MoELayerQ4:
    """A copy of L whose router carries a per-expert logit bias in input
    column 0: W_r[e, 0] = bf16(bias[e]).  With activations whose feature 0 is
    1.0 (bias_feature) the router logit is z_e = bias_e + sum_{h>0} x_h W_r[e, h],
    i.e. a biased router expressed in the reference's unbiased router
    (src/layers/router.mojo:15-106 has no bias term)."""
    import dataclasses
    H, E = L.hidden, L.num_experts
    r = L.router_bf16.reshape(E, H).copy()
    r[:, 0] = f32_to_bf16_bits(np.asarray(bias, np.float32))
    return dataclasses.replace(L, router_bf16=r.reshape(-1))


def bias_feature(x: np.ndarray) -> np.ndarray:
    """Activations with feature 0 set to 1.0, the input of a router bias
    folded in by with_router_bias."""
    x = np.array(x, dtype=np.float32, copy=True)
    x[..., 0] = 1.0
    return x


def expert_bytes(H, I, G=32) -> int:
    """4-bit codes plus fp16 group scales of one expert's gate, up and down."""
    n = 3 * I * H
    return n // 2 + 2 * n // G


def algorithmic_bytes_per_token(H, E, K, I, Ish, G=32, x_bytes=4, y_bytes=4) -> int:
    """Bytes one decode token must move: K routed + 1 shared expert in 4 bits
    with fp16 group scales, the bf16 router and shared gate, x in, y out."""
    return (K * expert_bytes(H, I, G) + expert_bytes(H, Ish, G) + 2 * E * H + 2 * H
            + x_bytes * H + y_bytes * H)


def make_layer_device(hidden: int, num_experts: int, top_k: int, inter: int, inter_sh: int,
                      group_size: int = 32, seed: int = 0, device="cuda") -> dict:
    """The same distributions as make_layer, drawn on the GPU with torch (for
    many-layer workloads whose host generation would take minutes).  Returns
    field name -> contiguous device tensor, for MoEBlock.upload_layer_device."""
    import torch
    H, E, I, Ish, G = hidden, num_experts, inter, inter_sh, group_size
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    lut = torch.from_numpy(_PAIR_LUT).to(device)

    def bf16(n):
        v = torch.randn(n, generator=g, device=device) * 0.02
        return v.to(torch.bfloat16).view(torch.int16)

    def scales(n):
        v = (torch.randn(n, generator=g, device=device).abs() * 0.02 / 7.5).half()
        b = v.view(torch.int16)
        return torch.where(b == 0, torch.ones_like(b), b)

    def codes(n):
        out = torch.empty(n // 2, dtype=torch.uint8, device=device)
        step = 1 << 26
        for o in range(0, n // 2, step):
            m = min(step, n // 2 - o)
            out[o:o + m] = lut[torch.randint(0, 225, (m,), generator=g, device=device)]
        return out

    return {"router_bf16": bf16(E * H), "shgate_bf16": bf16(H),
            "gu_scales": scales(E * 2 * I * H // G), "gu_packed": codes(E * 2 * I * H),
            "d_scales": scales(E * H * I // G), "d_packed": codes(E * H * I),
            "sh_gu_scales": scales(2 * Ish * H // G), "sh_gu_packed": codes(2 * Ish * H),
            "sh_d_scales": scales(H * Ish // G), "sh_d_packed": codes(H * Ish)}


# ---- GGUF layers ------------------------------------------------------------
def gguf_payload(rng, ggml_type: int, n: int, scale: float = 1e-4) -> bytes:
    """Random payload of n weights whose super-scales are fp16 values near
    `scale` (Q8_0: 20 x scale)."""
    import numpy as np
    if ggml_type == 0:
        return (rng.standard_normal(n) * scale * 100).astype("<f4").tobytes()
    bs, bpb, d_off = {8: (32, 34, 0), 12: (256, 144, 0), 11: (256, 114, 112)}[ggml_type]
    nb = -(-n // bs)  # a partial last block is stored whole
    raw = rng.integers(0, 256, size=(nb, bpb), dtype=np.uint8)
    d = (rng.uniform(0.5, 1.5, nb) * scale * (20 if ggml_type == 8 else 1)).astype(np.float16)
    raw[:, d_off:d_off + 2] = d.view(np.uint8).reshape(nb, 2)
    if ggml_type == 12:  # dmin
        raw[:, 2:4] = (rng.uniform(0.5, 1.5, nb) * scale).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return raw.tobytes()


def make_gguf_moe_layer(hidden: int, num_experts: int, inter: int, inter_sh: int, seed: int = 0,
                        expert_type: int = 11, model_layer: int = 0):
    """The MoE tensors of one layer under the names of
    src/layers/gguf_port_loader.mojo:207-256, as (name, dims, type, raw)
    for dismoen.gguf.write_gguf: router Q8_0, experts of expert_type,
    shared-expert gate vector F32."""
    import numpy as np
    rng = np.random.default_rng(seed)
    H, E, I, Ish = hidden, num_experts, inter, inter_sh
    p = f"blk.{model_layer}."
    ts = [(p + "ffn_gate_exps.weight", [H, E], 8, gguf_payload(rng, 8, E * H))]
    for e in range(E):
        ts.append((p + f"ffn_gate.{e}.weight", [H, I], expert_type, gguf_payload(rng, expert_type, I * H)))
        ts.append((p + f"ffn_up.{e}.weight", [H, I], expert_type, gguf_payload(rng, expert_type, I * H)))
        ts.append((p + f"ffn_down.{e}.weight", [I, H], expert_type, gguf_payload(rng, expert_type, I * H)))
    ts.append((p + "ffn_shared_gate.weight", [H, Ish], expert_type, gguf_payload(rng, expert_type, Ish * H)))
    ts.append((p + "ffn_shared_up.weight", [H, Ish], expert_type, gguf_payload(rng, expert_type, Ish * H)))
    ts.append((p + "ffn_shared_down.weight", [Ish, H], expert_type, gguf_payload(rng, expert_type, Ish * H)))
    ts.append((p + "shared_gate.weight", [H], 0, (rng.standard_normal(H) * 0.02).astype("<f4").tobytes()))
    return ts
