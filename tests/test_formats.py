"""Readers of the reference's weight files through the C ABI (host code, no
GPU): the safetensors header checks against the reference's fuzz fixtures
(fixtures/m0-fuzz with its manifest of expected error types), the quant
model scan against fixtures/m10_quant_mini.bin and the SEC-4 rules of
src/format/quant_reader.mojo:345-433, 487-662, and a written layer read
back byte for byte."""
import json
import os
import struct

import numpy as np
import pytest

from dismoen import DismoenError, formats, synth

HERE = os.path.dirname(os.path.abspath(__file__))
FUZZ = os.path.join(HERE, "golden", "safetensors_fuzz")
M10 = os.path.join(HERE, "golden", "m10_quant_mini.bin")


def _manifest():
    return json.load(open(os.path.join(FUZZ, "manifest.json")))


@pytest.mark.parametrize("case", _manifest(), ids=lambda c: c["file"])
def test_safetensors_fuzz_fixture(case):
    """Every fixture of the reference's fuzz set is accepted or rejected with
    the error type its manifest names."""
    path = os.path.join(FUZZ, case["file"])
    assert os.path.getsize(path) == case["size"]
    if case["want_exit"] == 0:
        with formats.read_header(path) as sh:
            raw = open(path, "rb").read()
            n = struct.unpack("<Q", raw[:8])[0]
            hdr = json.loads(raw[8:8 + n])
            names = [k for k in hdr if k != "__metadata__"]
            assert [t.name for t in sh.tensors] == names
            for t in sh.tensors:
                h = hdr[t.name]
                assert t.dtype == h["dtype"] and t.shape == h["shape"]
                b, e = h["data_offsets"]
                assert (t.data_offset, t.data_bytes) == (8 + n + b, e - b)
                assert sh.read(sh.find(t.name)) == raw[8 + n + b:8 + n + e]
    else:
        with pytest.raises(DismoenError) as ei:
            formats.read_header(path)
        err = json.loads(str(ei.value))
        assert err["error_type"] == case["want_err"], str(ei.value)
        assert err["shard"] == path


def test_safetensors_error_details():
    """The detail texts of src/format/reader.mojo for a few fixtures."""
    def detail(f):
        with pytest.raises(DismoenError) as ei:
            formats.read_header(os.path.join(FUZZ, f))
        return json.loads(str(ei.value))

    assert detail("03_empty_file.st")["detail"] == "file < 8 byte"
    d = detail("16_dup_key.st")
    assert d["detail"].startswith("kunci ganda: ") and d["tensor_name"] == d["detail"][13:]
    assert detail("13_dtype_asing.st")["detail"].startswith("dtype asing: ")
    assert detail("15_layout_mismatch.st")["detail"].startswith("len ")
    assert detail("18_missing_field.st")["detail"] == "field kurang"


def test_quant_fixture_is_padded_so_the_scan_rejects_it():
    """fixtures/m10_quant_mini.bin is zero-padded to 16384 bytes for O_DIRECT
    reads; scan_quant_file requires the records to end at the file end."""
    with pytest.raises(DismoenError) as ei:
        formats.scan_quant_file(M10)
    assert str(ei.value) == ("scan_quant_file: trailing data or size mismatch "
                             "(read 2616 != file_size 16384)")


def test_quant_fixture_trimmed_reads_back(tmp_path):
    raw = open(M10, "rb").read()
    hdr = raw[:256].rstrip(b" ").replace(b'"total_bytes":16384', b'"total_bytes":2616')
    p = tmp_path / "m10_trim.bin"
    p.write_bytes(hdr + b" " * (256 - len(hdr)) + raw[256:2616])
    with formats.scan_quant_file(str(p)) as q:
        assert len(q.tensors) == 1
        t = q.tensors[0]
        assert t.name == "model.layers.0.mlp.experts.0.gate_proj.weight"
        assert t.shape == [64, 64] and t.group_size == 64 and t.num_groups == 64
        assert (t.scales_offset, t.scales_bytes) == (440, 128)
        assert (t.data_offset, t.data_bytes) == (568, 2048)
        sc, pk = q.read(0)
        assert sc.tobytes() == raw[440:568] and pk.tobytes() == raw[568:2616]
        assert q.find(t.name) == 0 and q.find("nope") == -1


def _write(tmp_path, name, header=None, records=None, tail=b""):
    """A quant file from a header dict (fields overriding a valid header) and
    records (meta dict, payload bytes)."""
    records = records if records is not None else [
        ({"name": "w", "shape": [2, 64], "dtype": "BF16", "quantized_dtype": "4-bit",
          "group_size": 64, "num_groups": 2, "scale_offset": 0, "data_offset": 4},
         b"\x00\x3c" * 2 + b"\x11" * 64)]
    body = b""
    for meta, payload in records:
        js = json.dumps(meta, separators=(",", ":")).encode()
        body += struct.pack("<I", len(js)) + js + payload
    body += tail
    h = {"version": 1, "model": "t", "quantization": {"format": "4-bit per-group",
                                                       "group_size": 64, "scale_dtype": "FP16"},
         "num_tensors": len(records), "total_bytes": 256 + len(body)}
    for k, v in (header or {}).items():
        if k in ("format", "group_size", "scale_dtype"):
            h["quantization"][k] = v
        else:
            h[k] = v
    js = json.dumps(h, separators=(",", ":")).encode()
    p = tmp_path / name
    p.write_bytes(js + b" " * (256 - len(js)) + body)
    return str(p)


def _scan_err(path):
    with pytest.raises(DismoenError) as ei:
        formats.scan_quant_file(path)
    return str(ei.value)


def test_quant_scan_accepts_a_valid_file(tmp_path):
    with formats.scan_quant_file(_write(tmp_path, "ok.bin")) as q:
        sc, pk = q.read(0)
        assert sc.tolist() == [0x3C00, 0x3C00] and pk.tolist() == [0x11] * 64


H = "scan_quant_file: header validation failed (SEC-4): "
M = "scan_quant_file: tensor metadata failed SEC-4 validation: "


@pytest.mark.parametrize("hdr,msg", [
    ({"version": 2}, H + "Invalid quant header version: expected 1, got 2"),
    ({"group_size": 48}, H + "Group size must be one of {32, 64, 128, 256}, got 48"),
    ({"group_size": 0}, H + "Group size must be positive, got 0"),
    ({"format": "8-bit"}, H + "Unsupported quantization format: 8-bit"),
    ({"scale_dtype": "BF16"}, H + "Unsupported scale dtype: BF16"),
    ({"num_tensors": 0}, H + "Header num_tensors must be positive, got 0"),
    ({"num_tensors": 100001}, H + "Header num_tensors exceeds configured max: 100001 > 100000"),
    ({"total_bytes": 999}, None),
])
def test_quant_header_checks(tmp_path, hdr, msg):
    p = _write(tmp_path, "h.bin", header=hdr)
    if msg is None:
        msg = H + f"File size mismatch: header total_bytes=999, physical size={os.path.getsize(p)}"
    assert _scan_err(p) == msg


def _meta(**kw):
    m = {"name": "w", "shape": [2, 64], "dtype": "BF16", "quantized_dtype": "4-bit",
         "group_size": 64, "num_groups": 2, "scale_offset": 0, "data_offset": 4}
    m.update(kw)
    return m


@pytest.mark.parametrize("meta,msg", [
    (_meta(name=""), M + "Tensor name cannot be empty"),
    (_meta(name="a" * 513), M + "Tensor name length exceeds configured max: 513 > 512"),
    (_meta(shape=[]), "scan_quant_file: failed parsing tensor metadata JSON at tensor 0: "
                      "BlockTensorMeta: N % G != 0 (tail group not supported)"),
    (_meta(shape=[1] * 7 + [64, 2]), M + "Tensor ndim exceeds configured max: 9 > 8"),
    (_meta(shape=[0, 64]), M + "Dimension must be positive, got 0"),
    (_meta(num_groups=3), M + "num_groups mismatch: meta=3, expected=2"),
    (_meta(group_size=100), "scan_quant_file: failed parsing tensor metadata JSON at tensor 0: "
                            "BlockTensorMeta: group_size not in {32, 64, 128, 256}"),
])
def test_quant_meta_checks(tmp_path, meta, msg):
    p = _write(tmp_path, "m.bin", records=[(meta, b"\x00\x3c" * 2 + b"\x11" * 64)])
    assert _scan_err(p) == msg


def test_quant_framing_checks(tmp_path):
    # payload shorter than the meta promises
    p = _write(tmp_path, "t.bin", records=[(_meta(), b"\x00\x3c" * 2 + b"\x11" * 10)])
    assert _scan_err(p) == ("scan_quant_file: tensor payload truncated: w (offset "
                            f"{os.path.getsize(p) + 54} > {os.path.getsize(p)})")
    # bytes after the last record
    p = _write(tmp_path, "tail.bin", tail=b"\x00" * 7)
    n = os.path.getsize(p)
    assert _scan_err(p) == f"scan_quant_file: trailing data or size mismatch (read {n - 7} != file_size {n})"
    # the header is not JSON
    p = tmp_path / "nj.bin"
    p.write_bytes(b"x" * 300)
    assert _scan_err(str(p)) == (
        'scan_quant_file: failed parsing quant header: {"error_type":"JSON_PARSE_ERROR",'
        '"detail":"expected byte 123 at 0","shard":"quant_header","tensor_name":""}')
    # shorter than the header
    p = tmp_path / "short.bin"
    p.write_bytes(b"{}")
    assert _scan_err(str(p)) == "scan_quant_file: file truncated, size 2 < header size 256"
    # a fraction where the subset allows integers only
    p = _write(tmp_path, "fr.bin", header={"model": "t"})
    raw = open(p, "rb").read().replace(b'"model":"t"', b'"pi":3.1e0')
    open(p, "wb").write(raw)
    assert "pecahan/eksponen di luar subset" in _scan_err(p)


def test_written_layer_reads_back(tmp_path):
    L = synth.make_layer(**synth.CONFIG_TOY, seed=4)
    qp, sp = str(tmp_path / "layer.quant"), str(tmp_path / "layer.safetensors")
    formats.write_layer_files(qp, sp, L, model_layer=3)
    E, I, H, G = L.num_experts, L.inter, L.hidden, L.group_size
    with formats.scan_quant_file(qp) as q, formats.read_header(sp) as s:
        assert len(q.tensors) == 3 * E + 3
        i = q.find(f"model.layers.3.mlp.experts.5.up_proj.weight")
        sc, pk = q.read(i)
        assert np.array_equal(sc, L.gu_scales.reshape(E, 2, -1)[5, 1])
        assert np.array_equal(pk, L.gu_packed.reshape(E, 2, -1)[5, 1])
        r = s.read(s.find("model.layers.3.mlp.gate.weight"))
        assert np.array_equal(np.frombuffer(r, "<u2"), L.router_bf16)


@pytest.mark.parametrize("G", [-1, 48, 512])
def test_file_upload_rejects_group_size_before_reading(tmp_path, G):
    """dmh_upload_moe_layer_files checks the dims (group size in {32, 64,
    128, 256}) before any arithmetic or allocation on them: a negative or
    unsupported group size is a CONFIG_ERROR, not a division by zero, and no
    device is needed to reach the check.  Group size 0 takes the quant
    model's header value instead (below)."""
    import ctypes as C
    from dismoen._lib import DmhDims, lib
    c = synth.CONFIG_TOY
    L = synth.make_layer(**c, seed=70)
    qp, sp = str(tmp_path / "m.quant"), str(tmp_path / "m.safetensors")
    formats.write_layer_files(qp, sp, L, model_layer=0)
    d = DmhDims(c["hidden"], c["num_experts"], c["top_k"], c["inter"], c["inter_sh"], G, 0)
    e = C.create_string_buffer(1024)
    with formats.scan_quant_file(qp) as q, formats.read_header(sp) as s:
        rc = lib().dmh_upload_moe_layer_files(None, 0, C.byref(d), q.handle, s.handle, 0, e,
                                              len(e))
    assert rc == 2, e.value
    assert b'"error_type":"CONFIG_ERROR"' in e.value and b"G=%d" % G in e.value


def test_file_upload_group_size_zero_takes_the_header(tmp_path):
    """Group size 0 in the dims means quantization.group_size of the quant
    model's header (docs/format/quant_format.md:76): the dims check passes
    (the header says 32), and the call goes on to the context check."""
    import ctypes as C
    from dismoen._lib import DmhDims, lib
    c = synth.CONFIG_TOY
    L = synth.make_layer(**c, seed=71)
    qp, sp = str(tmp_path / "m.quant"), str(tmp_path / "m.safetensors")
    formats.write_layer_files(qp, sp, L, model_layer=0)
    d = DmhDims(c["hidden"], c["num_experts"], c["top_k"], c["inter"], c["inter_sh"], 0, 0)
    e = C.create_string_buffer(1024)
    with formats.scan_quant_file(qp) as q, formats.read_header(sp) as s:
        rc = lib().dmh_upload_moe_layer_files(None, 0, C.byref(d), q.handle, s.handle, 0, e,
                                              len(e))
    assert rc == 1 and b"NULL context" in e.value, e.value
