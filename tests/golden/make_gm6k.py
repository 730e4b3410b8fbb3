"""Regenerate the G-M6-K seed-42 dequant conformance fixture.

Restates the generator of the reference's tools/oracle/oracle_dequant.py:93-170
(numpy default_rng(42): five corner fp16 scales then random normal-range
scales; codes drawn from the 15 valid nibbles; 1024 groups x 128) and computes
the golden bf16 output with torch's float32 -> bfloat16 cast of fp32(s) * q,
the single-rounding rule of the reference oracle (oracle_dequant.py:32-90).
Writes fixture_seed42_{scales,packed,golden_bf16}.bin next to this script.
"""
import os
import struct

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def generate(num_groups=1024, group_size=128):
    rng = np.random.default_rng(42)
    scales_u16 = [0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF]
    for _ in range(num_groups - len(scales_u16)):
        exp = rng.integers(1, 31)
        mant = rng.integers(0, 1024)
        scales_u16.append(int((exp << 10) | mant))
    valid = [0, 1, 2, 3, 4, 5, 6, 7, 9, 10, 11, 12, 13, 14, 15]
    total = num_groups * group_size
    packed = bytearray(total // 2)
    for i in range(total // 2):
        n0 = int(rng.choice(valid))
        n1 = int(rng.choice(valid))
        packed[i] = (n1 << 4) | n0
    scales = np.array(scales_u16, dtype=np.uint16)
    return scales, np.frombuffer(bytes(packed), dtype=np.uint8)


def golden(scales, packed, group_size=128):
    s = scales.view(np.float16).astype(np.float32)
    lo = (packed & 0xF).astype(np.int32)
    hi = (packed >> 4).astype(np.int32)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    q = np.stack([lo, hi], axis=1).reshape(-1).astype(np.float32)
    sg = np.repeat(s, group_size)
    y = torch.from_numpy((sg * q).astype(np.float32)).to(torch.bfloat16)
    return y.view(torch.int16).numpy().view(np.uint16)


if __name__ == "__main__":
    sc, pk = generate()
    gd = golden(sc, pk)
    sc.tofile(os.path.join(HERE, "fixture_seed42_scales.bin"))
    pk.tofile(os.path.join(HERE, "fixture_seed42_packed.bin"))
    gd.tofile(os.path.join(HERE, "fixture_seed42_golden_bf16.bin"))
    print(sc.size, pk.size, gd.size, struct.pack("<H", int(gd[0])).hex())
