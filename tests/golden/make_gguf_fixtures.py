"""Writes the GGUF fixtures of the tests from the reference repository.

  m9_port_mini.gguf   copied from fixtures/m9_port_mini.gguf (the reference's
                      synthetic port checkpoint, tools/fixtures/
                      generate_m9_gguf_fixture.py);
  gguf_fuzz.json      every *.gguf case of fixtures/m9-fuzz/manifest.json as
                      an edit of m9_port_mini.gguf (byte patches, a truncated
                      length or appended bytes) with the manifest's expected
                      error, so the 15 MB corpus is not stored;
  gguf_vectors.npz    random Q4_K and Q3_K payloads and their fp32 values as
                      computed by the reference's Python twin of the GGUF
                      dequantizers (tools/oracle/oracle_port.py:86-160), and
                      the twin's values for the Q4_K blocks with scale bytes
                      12..15 replaced by bytes 8..11 (q4k_sub_f32).

Run in a checkout that has the reference at REF (default /root/reference):
    python tests/golden/make_gguf_fixtures.py
"""
import importlib.util
import json
import os
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("REF", "/root/reference")


def fuzz_cases():
    base = open(os.path.join(REF, "fixtures", "m9_port_mini.gguf"), "rb").read()
    man = json.load(open(os.path.join(REF, "fixtures", "m9-fuzz", "manifest.json")))
    out = []
    for c in man["cases"]:
        path = c["args"][1]
        if not path.endswith(".gguf"):
            continue
        d = open(os.path.join(REF, path), "rb").read()
        n = min(len(d), len(base))
        patches = [[i, d[i]] for i in range(n) if d[i] != base[i]]
        out.append({"id": c["id"], "file": os.path.basename(path), "size": len(d),
                    "patches": patches, "append": list(d[len(base):]),
                    "want_exit": c["want_exit"], "want_err": c["want_err"],
                    "description": c["description"]})
    return out


def vectors():
    spec = importlib.util.spec_from_file_location(
        "oracle_port", os.path.join(REF, "tools", "oracle", "oracle_port.py"))
    op = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(op)
    rng = np.random.default_rng(2024)
    res = {}
    for name, bpb, fn in (("q4k", 144, op.dequantize_q4_k), ("q3k", 114, op.dequantize_q3_k)):
        nb = 48
        raw = rng.integers(0, 256, size=(nb, bpb), dtype=np.uint8)
        # finite fp16 super-scales (exponent field < 31) of both signs, some subnormal
        hdr = [0, 2] if name == "q4k" else [112]
        for k, o in enumerate(hdr):
            h = rng.integers(0, 0x7C00, size=nb).astype(np.uint16)
            h[:4] = [0x0001, 0x03FF, 0x3C00, 0x0000]
            h[4:8] ^= 0x8000
            raw[:, o] = h & 0xFF
            raw[:, o + 1] = h >> 8
        res[name + "_raw"] = raw
        res[name + "_f32"] = fn(raw.tobytes(), nb * 256).astype(np.float32)
        if name == "q4k":
            # the same blocks with scale bytes 12..15 replaced by bytes 8..11:
            # where gguf.mojo:482-488 reads them from
            sub = raw.copy()
            sub[:, 12:16] = sub[:, 8:12]
            res["q4k_sub_f32"] = fn(sub.tobytes(), nb * 256).astype(np.float32)
    return res


def main():
    shutil.copyfile(os.path.join(REF, "fixtures", "m9_port_mini.gguf"),
                    os.path.join(HERE, "m9_port_mini.gguf"))
    with open(os.path.join(HERE, "gguf_fuzz.json"), "w") as f:
        json.dump(fuzz_cases(), f, indent=1)
    np.savez_compressed(os.path.join(HERE, "gguf_vectors.npz"), **vectors())
    print("wrote m9_port_mini.gguf, gguf_fuzz.json, gguf_vectors.npz", file=sys.stderr)


if __name__ == "__main__":
    main()
