"""GGUF on the host (no GPU): the container index of src/format/gguf.mojo:
257-411 against the reference's fixture fixtures/m9_port_mini.gguf and its
fuzz corpus fixtures/m9-fuzz (stored as edits of the fixture in
tests/golden/gguf_fuzz.json), and the oracle's dequantizers
(gguf.mojo:414-560) against

  - the closed forms of the synthetic blocks that
    tools/fixtures/generate_m9_gguf_fixture.py:47-91 wrote into the fixture,
  - the reference's Python twin (tools/oracle/oracle_port.py:86-160) on random
    blocks (tests/golden/gguf_vectors.npz, written by make_gguf_fixtures.py),
  - for Q4_K as gguf.mojo unpacks it: the twin on the same blocks with scale
    bytes 12..15 replaced by bytes 8..11, the bytes gguf.mojo:482-488 reads."""
import json
import os

import numpy as np
import pytest

from dismoen import DismoenError, gguf

HERE = os.path.dirname(os.path.abspath(__file__))
MINI = os.path.join(HERE, "golden", "m9_port_mini.gguf")


def _same(a, b):
    """Bit-exact, NaNs compared as NaNs."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and \
        np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


@pytest.fixture(scope="module")
def mini():
    with gguf.parse_gguf_index(MINI) as g:
        yield g


def test_fixture_index(mini):
    """Header and directory of the fixture as its generator wrote them
    (generate_m9_gguf_fixture.py:94-367: version 3, alignment 32, payloads
    packed back to back at 32-byte boundaries)."""
    assert (mini.version, mini.alignment, mini.tensor_count) == (3, 32, 148)
    assert mini.expected_file_size == os.path.getsize(MINI)
    assert mini.data_section_offset % 32 == 0
    t = mini.tensors[mini.tensor_map["token_embd.weight"]]
    # "1024 x 128 = 131072 elems -> 4096 blocks -> 139264 bytes"
    assert (t.dims, t.dtype, t.num_elements, t.raw_bytes, t.offset) == \
        ([128, 1024], 8, 131072, 139264, 0)
    end = 0
    for t in mini.tensors:
        assert t.offset == (end + 31) // 32 * 32
        end = t.offset + t.raw_bytes
    assert mini.data_section_offset + end == os.path.getsize(MINI)
    kinds = {}
    for t in mini.tensors:
        kinds[t.dtype] = kinds.get(t.dtype, 0) + 1
    assert kinds == {8: 6, 0: 16, 12: 14, 11: 112}
    assert mini.metadata("general.architecture") == "qwen3.6"
    assert mini.metadata("no.such.key") is None


def _fuzz_cases():
    return json.load(open(os.path.join(HERE, "golden", "gguf_fuzz.json")))


def _materialise(case, tmp_path):
    base = open(MINI, "rb").read()
    b = bytearray(base[:case["size"]])
    for off, v in case["patches"]:
        b[off] = v
    b += bytes(case["append"])
    assert len(b) == case["size"]
    p = tmp_path / case["file"]
    p.write_bytes(bytes(b))
    return str(p)


# The corpus drives the reference's CLI; cases 01, 02 and 04 are turned away
# by its format detector before parse_gguf_index runs, and the name and dims
# mutations that the index accepts fail later, when the loader looks the
# tensor up or checks its shape.  These are the index's own results.
PARSE_RESULT = {
    "FUZZ_01_CORRUPT_MAGIC": "GGUF_FILE_CORRUPT: invalid magic header (expected 'GGUF')",
    "FUZZ_02_UNSUPPORTED_VERSION": "GGUF_FILE_CORRUPT: unsupported version 99",
    "FUZZ_03_TRUNCATED_HEADER": "GGUF_FILE_CORRUPT: file size 12 too small for header",
    "FUZZ_04_ZERO_BYTE": "GGUF_FILE_CORRUPT: file size 0 too small for header",
    "FUZZ_05_F11B_SIZE_MISMATCH":
        "GGUF_FILE_CORRUPT: actual size 762081 != expected size 762080 (diff: 1 bytes)",
    "FUZZ_06_TRUNCATED_DATA": "GGUF_FILE_CORRUPT: tensor extends beyond file boundary",
    "FUZZ_15_MUTATION_CORRUPT_OFFSET_271": "GGUF_FILE_CORRUPT: tensor ndim invalid: 16447751",
    "FUZZ_18_MUTATION_CORRUPT_OFFSET_322": "GGUF_FILE_CORRUPT: u64 overflow/negative value",
    "FUZZ_21_MUTATION_CORRUPT_OFFSET_373": "GGUF_FILE_CORRUPT: tensor ndim invalid: 0",
    "FUZZ_26_MUTATION_CORRUPT_OFFSET_458": "GGUF_FILE_CORRUPT: tensor ndim invalid: 16711681",
}
BEYOND = ("FUZZ_14", "FUZZ_17", "FUZZ_20", "FUZZ_24", "FUZZ_27")
RENAMED = {"FUZZ_13": "token_embd.weight", "FUZZ_16": "output.weight",
           "FUZZ_19": "output_norm.weight", "FUZZ_22": "blk.0.attn_norm.weight",
           "FUZZ_25": "blk.0.ffn_norm.weight"}


@pytest.mark.parametrize("case", _fuzz_cases(), ids=lambda c: c["id"])
def test_fuzz_corpus(case, tmp_path):
    path = _materialise(case, tmp_path)
    key = case["id"][:7]
    if case["id"] in PARSE_RESULT or key in BEYOND:
        with pytest.raises(DismoenError) as ei:
            gguf.parse_gguf_index(path)
        msg = str(ei.value)
        want = PARSE_RESULT.get(case["id"],
                                 "GGUF_FILE_CORRUPT: tensor extends beyond file boundary")
        assert msg == want
        if case["want_err"].startswith("GGUF"):
            assert case["want_err"] in msg
        return
    with gguf.parse_gguf_index(path) as g:
        if key in RENAMED:
            assert RENAMED[key] not in g.tensor_map  # the loader's lookup fails
        else:  # FUZZ_23: first dim of blk.0.attn_norm.weight 128 -> 127
            assert case["id"] == "FUZZ_23_MUTATION_CORRUPT_OFFSET_407"
            t = g.tensors[g.tensor_map["blk.0.attn_norm.weight"]]
            assert t.dims == [127] and t.raw_bytes == 508


def test_missing_file(tmp_path):
    p = str(tmp_path / "nope.gguf")
    with pytest.raises(DismoenError) as ei:
        gguf.parse_gguf_index(p)
    j = json.loads(str(ei.value))
    assert j["error_type"] == "FILE_NOT_FOUND" and j["shard"] == p


def _gguf(tmp_path, kv=b"", nkv=0, tensors=(), version=3, pad_to=None, payload=b""):
    """A GGUF file: header, nkv metadata bytes kv, tensor directory entries
    (name, dims, type, offset), data section at 32 bytes, payload."""
    import struct
    b = b"GGUF" + struct.pack("<IQQ", version, len(tensors), nkv) + kv
    for name, dims, ty, off in tensors:
        b += struct.pack("<Q", len(name)) + name.encode() + struct.pack("<I", len(dims))
        b += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, off)
    b += b"\0" * ((-len(b)) % (pad_to or 32)) + payload
    p = tmp_path / "t.gguf"
    p.write_bytes(b)
    return str(p)


def _kv(key, vtype, val):
    import struct
    return struct.pack("<Q", len(key)) + key.encode() + struct.pack("<I", vtype) + val


def test_metadata_values_and_alignment(tmp_path):
    import struct
    kv = (_kv("a.u8", 0, b"\xff") + _kv("a.i16", 3, b"\xfe\xff") +
          _kv("a.f32", 6, struct.pack("<f", 1.0)) + _kv("a.str", 8, struct.pack("<Q", 2) + b"hi") +
          _kv("a.arr", 9, struct.pack("<IQ", 9, 2) + struct.pack("<IQ", 0, 1) + b"\x01" +
              struct.pack("<IQ", 8, 1) + struct.pack("<Q", 1) + b"x") +
          _kv("general.alignment", 4, struct.pack("<I", 64)))
    p = _gguf(tmp_path, kv, 6, [("w", [4], 0, 0)], pad_to=64, payload=b"\0" * 16)
    with gguf.parse_gguf_index(p) as g:
        assert g.metadata("a.u8") == "255" and g.metadata("a.i16") == "65534"
        assert g.metadata("a.f32") == str(0x3F800000) and g.metadata("a.str") == "hi"
        assert g.metadata("a.arr") == "[Array of 2 elements]"
        assert g.alignment == 64 and g.data_section_offset % 64 == 0


@pytest.mark.parametrize("case", ["u64_eof", "string_eof", "vtype", "top_bit", "strlen"])
def test_header_errors(tmp_path, case):
    import struct
    kv, pad, msg = {
        "u64_eof": (_kv("k", 10, b"\0\0\0"), 1, "GGUF_FILE_CORRUPT: unexpected EOF reading u64"),
        "string_eof": (struct.pack("<Q", 1000), 1, "GGUF: unexpected EOF reading string"),
        "vtype": (_kv("k", 13, b""), 32, "GGUF: unknown value type 13"),
        "top_bit": (b"\0" * 7 + b"\x80", 32, "GGUF_FILE_CORRUPT: u64 overflow/negative value"),
        "strlen": (struct.pack("<Q", 65537), 32, "GGUF: string length invalid: 65537"),
    }[case]
    p = _gguf(tmp_path, kv, 1, pad_to=pad, payload=b"" if pad == 1 else b"\0" * 64)
    with pytest.raises(DismoenError) as ei:
        gguf.parse_gguf_index(p)
    assert str(ei.value) == msg
    # tensor_count bound, checked before the metadata
    b = bytearray(open(p, "rb").read())
    b[8:16] = struct.pack("<Q", 100001)
    open(p, "wb").write(bytes(b))
    with pytest.raises(DismoenError) as ei:
        gguf.parse_gguf_index(p)
    assert str(ei.value) == "GGUF_FILE_CORRUPT: tensor_count out of bounds: 100001"


def test_offset_overflow_and_duplicates(tmp_path):
    p = _gguf(tmp_path, tensors=[("w", [4], 0, (1 << 63) - 8)])
    with pytest.raises(DismoenError) as ei:
        gguf.parse_gguf_index(p)
    assert str(ei.value) == "GGUF_FILE_CORRUPT: tensor offset integer overflow"
    # a repeated name: the map keeps the last entry (Dict assignment)
    p = _gguf(tmp_path, tensors=[("w", [4], 0, 0), ("w", [8], 0, 32)], payload=b"\0" * 64)
    with gguf.parse_gguf_index(p) as g:
        assert len(g.tensors) == 2 and g.tensor_map["w"] == 1


# ---- oracle dequantizers ------------------------------------------------------
def _payload(g, name):
    return g.read_raw(name), g.tensors[g.tensor_map[name]]


def test_oracle_q8_0_fixture(mini, oracle):
    """token_embd.weight: scale 1.0, codes ((b + j) % 15) - 7."""
    raw, t = _payload(mini, "token_embd.weight")
    y = oracle.dequant_gguf(8, raw, t.num_elements)
    b, j = np.divmod(np.arange(t.num_elements), 32)
    assert _same(y, ((b + j) % 15 - 7).astype(np.float32))


def test_oracle_q4_k_fixture(mini, oracle):
    """d = 0.5, dmin = fp16 0x2E66, every scale byte 10, every code byte 0x23:
    sub-blocks 0-3 have scale 5 and min 10*dmin, 4-7 scale 5 and min 0 (under
    both packings); the low nibble 3 fills the first 16 weights of a
    sub-block, the high nibble 2 the last 16."""
    raw, t = _payload(mini, "blk.0.linear_attn.k.weight")
    dmin = float(np.array([0x2E66], np.uint16).view(np.float16)[0])
    e = np.arange(t.num_elements) % 256
    sub, r = e // 32, e % 32
    m = np.where(sub < 4, np.float32(10 * dmin), np.float32(0))
    want = np.where(r < 16, np.float32(15), np.float32(10)) - m
    for layout in (0, 1):
        assert _same(oracle.dequant_gguf(12, raw, t.num_elements, layout), want.astype(np.float32))


def test_oracle_q3_k_fixture(mini, oracle):
    """hmask 0x55, codes 0xAA, scale bytes 34, d = 0.25: q = 6 at even and 2 at
    odd positions, scale 0.5, so +1, -1, +1, ..."""
    raw, t = _payload(mini, "blk.0.ffn_down_exps.0.weight")
    y = oracle.dequant_gguf(11, raw, t.num_elements)
    want = np.where(np.arange(t.num_elements) % 2 == 0, 1.0, -1.0).astype(np.float32)
    assert _same(y, want)


@pytest.fixture(scope="module")
def vec():
    return np.load(os.path.join(HERE, "golden", "gguf_vectors.npz"))


def test_oracle_vs_python_twin(oracle, vec):
    q4, q3 = vec["q4k_raw"], vec["q3k_raw"]
    assert _same(oracle.dequant_gguf(12, q4.ravel(), q4.shape[0] * 256, 1), vec["q4k_f32"])
    assert _same(oracle.dequant_gguf(11, q3.ravel(), q3.shape[0] * 256), vec["q3k_f32"])


def test_oracle_q4_k_mojo_packing(oracle, vec):
    q4 = vec["q4k_raw"]
    n = q4.shape[0] * 256
    mojo = oracle.dequant_gguf(12, q4.ravel(), n, 0)
    assert _same(mojo, vec["q4k_sub_f32"])
    # the two packings do differ on these blocks, in sub-blocks 4..7 only
    twin = vec["q4k_f32"]
    diff = ~((mojo == twin) | (np.isnan(mojo) & np.isnan(twin)))
    assert diff.any() and not diff.reshape(-1, 8, 32)[:, :4].any()


def test_oracle_tail_and_types(oracle):
    """Elements past the last whole block are 0.0; F32 and BF16 copy."""
    rng = np.random.default_rng(5)
    raw = rng.integers(0, 256, 34 * 2, dtype=np.uint8)
    raw[1] = raw[35] = 0x3C  # finite scales
    y = oracle.dequant_gguf(8, raw, 70)
    assert np.all(y[64:] == 0) and _same(y[:32], oracle.dequant_gguf(8, raw[:34], 32))
    f = rng.standard_normal(9).astype(np.float32)
    assert _same(oracle.dequant_gguf(0, f.view(np.uint8), 9), f)
    bf = rng.integers(0, 65536, 5, dtype=np.uint16)
    assert _same(oracle.dequant_gguf(30, bf.view(np.uint8), 5),
                 (bf.astype(np.uint32) << 16).view(np.float32))
    with pytest.raises(Exception, match="GGUF_UNSUPPORTED_DTYPE: unsupported GGML type 1"):
        oracle.dequant_gguf(1, raw, 32)
