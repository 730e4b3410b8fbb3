"""GPU parity of the GGUF dequantizers (dmh_dequant_gguf,
dmh_gguf_stream_tensor_f32) with the oracle restatement of
src/format/gguf.mojo:414-626, bit-exact (every output is one fp32 product of
exact factors, or for Q4_K one rounded difference), NaNs compared as NaNs:

  - random payloads of every type, both Q4_K packings, non-finite and
    subnormal super-scales, ragged tails (a partial block, n not a multiple
    of 8), host and device pointers, up to 2^24 weights;
  - the reference Python twin's vectors (tests/golden/gguf_vectors.npz);
  - every tensor of the reference's fixture m9_port_mini.gguf streamed from
    the file;
  - the error texts of stream_gguf_tensor_f32."""
import json
import os
import struct

import numpy as np
import pytest

from dismoen import DismoenError, gguf

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
MINI = os.path.join(HERE, "golden", "m9_port_mini.gguf")
SPEC = {0: (1, 4), 30: (1, 2), 8: (32, 34), 12: (256, 144), 11: (256, 114)}


def _same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and \
        np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def _payload(rng, t, n, special=True):
    bs, bpb = SPEC[t]
    nb = -(-n // bs)
    raw = rng.integers(0, 256, size=nb * bpb, dtype=np.uint8)
    if t in (8, 12, 11):
        blk = raw.reshape(nb, bpb)
        offs = {8: [0], 12: [0, 2], 11: [112]}[t]
        for o in offs:
            h = rng.integers(0, 0x7C00, size=nb).astype(np.uint16) | \
                (rng.integers(0, 2, size=nb).astype(np.uint16) << 15)
            if special and nb >= 6:
                h[:6] = [0x7C00, 0xFC00, 0x7E00, 0x0001, 0x8000, 0x03FF]  # inf, -inf, nan, subnormals
            blk[:, o] = h & 0xFF
            blk[:, o + 1] = h >> 8
    return raw


@pytest.mark.parametrize("t,layout", [(8, 0), (12, 0), (12, 1), (11, 0), (0, 0), (30, 0)])
@pytest.mark.parametrize("n", [1, 7, 33, 256, 300, 4096 + 5, 1 << 16])
def test_dequant_host_matches_oracle(block, oracle, t, layout, n):
    rng = np.random.default_rng(n * 31 + t)
    raw = _payload(rng, t, n)
    if t == 0:  # finite floats
        raw = rng.standard_normal(n).astype(np.float32).view(np.uint8)
    y = gguf.dequantize(t, raw, n, block, py_scales=bool(layout))
    assert _same(y, oracle.dequant_gguf(t, raw, n, layout)), (t, layout, n)


def test_twin_vectors(block):
    vec = np.load(os.path.join(HERE, "golden", "gguf_vectors.npz"))
    q4, q3 = vec["q4k_raw"], vec["q3k_raw"]
    n4, n3 = q4.shape[0] * 256, q3.shape[0] * 256
    assert _same(gguf.dequantize_q4_k(q4.ravel(), n4, block, py_scales=True), vec["q4k_f32"])
    assert _same(gguf.dequantize_q4_k(q4.ravel(), n4, block), vec["q4k_sub_f32"])
    assert _same(gguf.dequantize_q3_k(q3.ravel(), n3, block), vec["q3k_f32"])


@pytest.mark.parametrize("t,layout", [(11, 0), (12, 0), (12, 1), (8, 0), (30, 0)])
def test_dequant_device_large(block, oracle, t, layout):
    import torch
    n = (1 << 24) + 256 + 40  # a ragged tail past the last whole block
    rng = np.random.default_rng(77 + t)
    raw = _payload(rng, t, n)
    dev = torch.device("cuda:0")
    draw = torch.from_numpy(raw).to(dev)
    out = torch.full((n,), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    print(f"device dequant type {t} layout {layout} n {n}", flush=True)
    gguf.dequantize_device(t, draw.data_ptr(), raw.size, n, out.data_ptr(), block,
                           py_scales=bool(layout))
    block.sync()
    torch.cuda.synchronize()
    assert _same(out.cpu().numpy(), oracle.dequant_gguf(t, raw, n, layout))


def test_stream_fixture_tensors(block, oracle):
    """Every tensor of fixtures/m9_port_mini.gguf read and dequantized through
    the library equals the oracle on the same bytes."""
    with gguf.parse_gguf_index(MINI) as g:
        for t in g.tensors:
            y = gguf.stream_gguf_tensor_f32(g, t.name, block)
            ref = oracle.dequant_gguf(t.dtype, g.read_raw(t.name), t.num_elements)
            assert _same(y, ref), t.name
            assert np.isfinite(y).all() and y.size == t.num_elements  # test_m9_w3_gguf.mojo


def test_stream_device_out(block, oracle):
    import torch
    with gguf.parse_gguf_index(MINI) as g:
        name = "blk.0.ffn_down_exps.0.weight"
        t = g.tensors[g.tensor_map[name]]
        out = torch.empty(t.num_elements, dtype=torch.float32, device="cuda:0")
        from dismoen._lib import DMH_F_DEVICE, check, errbuf, lib
        e = errbuf()
        check(lib().dmh_gguf_stream_tensor_f32(block.handle, g.handle, name.encode(),
                                               out.data_ptr(), t.num_elements, DMH_F_DEVICE, e,
                                               len(e)), e)
        block.sync()
        assert _same(out.cpu().numpy(), oracle.dequant_gguf(11, g.read_raw(name), t.num_elements))


def _one_tensor_file(path, ty, n, payload):
    name = b"w"
    b = b"GGUF" + struct.pack("<IQQ", 3, 1, 0)
    b += struct.pack("<Q", len(name)) + name + struct.pack("<IQIQ", 1, n, ty, 0)
    b += b"\0" * ((-len(b)) % 32) + payload
    open(path, "wb").write(b)


def test_stream_errors(block, tmp_path):
    with gguf.parse_gguf_index(MINI) as g:
        with pytest.raises(DismoenError) as ei:
            gguf.stream_gguf_tensor_f32(g, "blk.9.missing.weight", block)
        assert json.loads(str(ei.value)) == {"error_type": "WEIGHT_LOAD_FAILED",
                                             "detail": "tensor not found in GGUF index",
                                             "tensor": "blk.9.missing.weight"}
    p = str(tmp_path / "f16.gguf")
    _one_tensor_file(p, 1, 16, b"\0" * 32)  # F16: parsed, not dequantized
    with gguf.parse_gguf_index(p) as g:
        with pytest.raises(DismoenError) as ei:
            gguf.stream_gguf_tensor_f32(g, "w", block)
        assert str(ei.value) == "GGUF_UNSUPPORTED_DTYPE: unsupported GGML type 1 for tensor w"
    p = str(tmp_path / "short.gguf")
    _one_tensor_file(p, 8, 64, b"\0" * 68)
    with gguf.parse_gguf_index(p) as g:
        with open(p, "r+b") as f:  # the file shrinks after the index was built
            f.truncate(os.path.getsize(p) - 10)
        with pytest.raises(DismoenError) as ei:
            gguf.stream_gguf_tensor_f32(g, "w", block)
        assert str(ei.value) == ("GGUF_READ_ERROR: truncated read for tensor w: expected 68 "
                                 "bytes, got 58")


def test_dequant_argument_errors(block):
    with pytest.raises(DismoenError, match="GGUF_UNSUPPORTED_DTYPE: unsupported GGML type 14"):
        gguf.dequantize(14, np.zeros(210, np.uint8), 256, block)
    with pytest.raises(DismoenError, match="payload bytes"):
        gguf.dequantize(11, np.zeros(113, np.uint8), 256, block)
    import torch
    raw = torch.zeros(256, dtype=torch.uint8, device="cuda:0")
    out = torch.zeros(64, dtype=torch.float32, device="cuda:0")
    with pytest.raises(DismoenError, match="aligned"):
        gguf.dequantize_device(8, raw.data_ptr() + 2, 68, 64, out.data_ptr(), block)
    with pytest.raises(DismoenError, match="aligned"):
        gguf.dequantize_device(8, raw.data_ptr(), 68, 60, out.data_ptr() + 4, block)
