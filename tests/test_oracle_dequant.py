"""Pins the oracle's 4-bit dequant and layout helpers.

Reference tests mirrored: tests/unit/test_m6_dequant.mojo:48-157 (225 pairs,
reserved nibble, bad scales), tests/unit/test_m6_quant_format.mojo:139-144
(pack known answers), the G-M6-K seed-42 fixture of
tools/oracle/oracle_dequant.py:93-170 (tests/golden/make_gm6k.py), and
fixtures/m10_quant_mini.bin.  Independent checks: numpy's fp16 widening and
torch's float32 -> bfloat16 cast.
"""
import json
import os
import struct

import numpy as np
import pytest
import torch

from conftest import GOLDEN


def torch_bf16_bits(f32):
    t = torch.from_numpy(np.ascontiguousarray(f32, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def test_fp16_widening_all_patterns(oracle):
    ref = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_f32(i) for i in range(65536)], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ref[finite].view(np.uint32), got[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(np.isinf(ref), np.isinf(got))


def test_bf16_rne_matches_torch(oracle):
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 1e-3,
                        rng.standard_normal(20000).astype(np.float32) * 300,
                        np.array([0.0, -0.0, 1.0, 65504 * 7, 2 ** -24, 3 * 2 ** -24,
                                  1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8], np.float32)])
    # exact ties: bit 15 set, low 15 bits zero
    ties = (rng.integers(0, 2 ** 31, 4000, dtype=np.uint32) & 0x7F7F0000) | 0x8000
    v = np.concatenate([v, ties.view(np.float32)])
    got = np.array([oracle.f32_to_bf16(float(f)) for f in v], dtype=np.uint16)
    assert np.array_equal(got, torch_bf16_bits(v))


def test_pack_known_answers(oracle):
    # tests/unit/test_m6_quant_format.mojo:139-144
    assert oracle.pack_4bit_pair(7, 7) == 0x77
    assert oracle.pack_4bit_pair(-1, -1) == 0xFF
    assert oracle.pack_4bit_pair(-7, -7) == 0x99
    assert oracle.pack_4bit_pair(1, -1) == 0xF1
    with pytest.raises(oracle.OracleError):
        oracle.pack_4bit_pair(-8, 0)
    with pytest.raises(oracle.OracleError):
        oracle.unpack_4bit_pair(0x08)
    with pytest.raises(oracle.OracleError):
        oracle.unpack_4bit_pair(0x80)
    for b in range(256):
        if (b & 0xF) == 8 or (b >> 4) == 8:
            continue
        w0, w1 = oracle.unpack_4bit_pair(b)
        assert oracle.pack_4bit_pair(w0, w1) == b


def all_225_pairs():
    scales = np.array([0.25, 0.5, 1.0, 2.0], np.float16).view(np.uint16)
    packed, w0, w1 = [], [], []
    for v1 in range(-7, 8):
        for v0 in range(-7, 8):
            packed.append(((v1 & 0xF) << 4) | (v0 & 0xF))
            w0.append(v0)
            w1.append(v1)
    while len(packed) < 256:
        packed.append(0); w0.append(0); w1.append(0)
    return scales, np.array(packed, np.uint8), np.array(w0), np.array(w1)


def test_dequant_225_pairs(oracle):
    # tests/unit/test_m6_dequant.mojo:48-86
    scales, packed, w0, w1 = all_225_pairs()
    out = oracle.dequant_q4_bf16(scales, packed, 512, 128)
    s = np.repeat(scales.view(np.float16).astype(np.float32), 64)
    exp0 = torch_bf16_bits(s * w0.astype(np.float32))
    exp1 = torch_bf16_bits(s * w1.astype(np.float32))
    assert np.array_equal(out[0::2], exp0)
    assert np.array_equal(out[1::2], exp1)


def test_dequant_every_scale_every_code(oracle):
    """All 63488 positive finite fp16 scales x all 15 codes vs torch."""
    s_bits = np.array([u for u in range(1, 0x7C00)], np.uint16)
    G = 32
    n_groups = s_bits.size
    codes = np.tile(np.concatenate([np.arange(-7, 8), np.zeros(17, int)]), n_groups)
    lo, hi = codes[0::2], codes[1::2]
    packed = (((hi & 0xF) << 4) | (lo & 0xF)).astype(np.uint8)
    out = oracle.dequant_q4_bf16(s_bits, packed, n_groups * G, G)
    s = np.repeat(s_bits.view(np.float16).astype(np.float32), G)
    assert np.array_equal(out, torch_bf16_bits(s * codes.astype(np.float32)))


def test_dequant_rejections(oracle):
    # tests/unit/test_m6_dequant.mojo:89-157
    one = np.array([0x3C00], np.uint16)
    bad_lo = np.zeros(64, np.uint8); bad_lo[10] = 0x08
    bad_hi = np.zeros(64, np.uint8); bad_hi[10] = 0x80
    for p in (bad_lo, bad_hi):
        with pytest.raises(oracle.OracleError, match="reserved nibble"):
            oracle.dequant_q4_bf16(one, p, 128, 128)
    ok = np.zeros(64, np.uint8)
    for bits, msg in ((0x7E00, "NaN or Inf"), (0x7C00, "NaN or Inf"), (0x0000, "non-positive"),
                      (0x8000, "non-positive"), (0xBC00, "non-positive")):
        with pytest.raises(oracle.OracleError, match=msg):
            oracle.dequant_q4_bf16(np.array([bits], np.uint16), ok, 128, 128)
    with pytest.raises(oracle.OracleError, match="group_size must be in"):
        oracle.dequant_q4_bf16(one, ok, 128, 48)
    with pytest.raises(oracle.OracleError, match="N % G != 0"):
        oracle.dequant_q4_bf16(one, ok, 100, 32)
    with pytest.raises(oracle.OracleError, match="scales length mismatch"):
        oracle.dequant_q4_bf16(np.array([0x3C00, 0x3C00], np.uint16), ok, 128, 128)
    with pytest.raises(oracle.OracleError, match="packed weights length mismatch"):
        oracle.dequant_q4_bf16(one, np.zeros(63, np.uint8), 128, 128)


def load_gm6k():
    sc = np.fromfile(os.path.join(GOLDEN, "fixture_seed42_scales.bin"), np.uint16)
    pk = np.fromfile(os.path.join(GOLDEN, "fixture_seed42_packed.bin"), np.uint8)
    gd = np.fromfile(os.path.join(GOLDEN, "fixture_seed42_golden_bf16.bin"), np.uint16)
    return sc, pk, gd


def test_gm6k_seed42_fixture(oracle):
    sc, pk, gd = load_gm6k()
    assert sc.size == 1024 and pk.size == 65536
    assert list(sc[:5]) == [0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF]
    assert np.array_equal(oracle.dequant_q4_bf16(sc, pk, 131072, 128), gd)
    corrupt = pk.copy()
    corrupt[42] = (corrupt[42] & 0x0F) | 0x80
    with pytest.raises(oracle.OracleError, match="reserved nibble"):
        oracle.dequant_q4_bf16(sc, corrupt, 131072, 128)


def read_m10():
    """quant_model.bin: 256-byte JSON header, then [u32 len][JSON meta][scales][codes]
    (src/format/quant_reader.mojo:520-662)."""
    raw = open(os.path.join(GOLDEN, "m10_quant_mini.bin"), "rb").read()
    hdr = json.loads(raw[:256].split(b"\x00")[0].decode().strip())
    off = 256
    (ml,) = struct.unpack_from("<I", raw, off)
    meta = json.loads(raw[off + 4: off + 4 + ml])
    base = off + 4 + ml
    ng = meta["num_groups"]
    n = int(np.prod(meta["shape"]))
    sc = np.frombuffer(raw, np.uint16, ng, base + meta["scale_offset"])
    pk = np.frombuffer(raw, np.uint8, (n + 1) // 2, base + meta["data_offset"])
    return hdr, meta, sc, pk


def test_m10_quant_mini_fixture(oracle):
    hdr, meta, sc, pk = read_m10()
    assert hdr["quantization"]["group_size"] == 64 and meta["shape"] == [64, 64]
    out = oracle.dequant_q4_bf16(sc, pk, 4096, meta["group_size"])
    s = np.repeat(sc.view(np.float16).astype(np.float32), 64)
    lo = (pk & 0xF).astype(int); hi = (pk >> 4).astype(int)
    q = np.stack([np.where(lo >= 8, lo - 16, lo), np.where(hi >= 8, hi - 16, hi)], 1).ravel()
    assert np.array_equal(out, torch_bf16_bits(s * q.astype(np.float32)))


def test_scale_ceil_rule(oracle):
    # compute_fp16_scale_ceil, src/format/half_float.mojo:77-97
    rng = np.random.default_rng(5)
    for a in np.abs(rng.standard_normal(2000).astype(np.float32)) * 3:
        s = oracle.compute_fp16_scale_ceil(float(a))
        sf = float(np.uint16(s).view(np.float16))
        assert np.float32(sf) * np.float32(7.0) >= a
        if s > 1:
            prev = float(np.uint16(s - 1).view(np.float16))
            assert np.float32(prev) * np.float32(7.0) < a or prev < np.float32(a) / np.float32(7)
    assert oracle.compute_fp16_scale_ceil(0.0) == 0x3C00
