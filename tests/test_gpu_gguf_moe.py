"""GPU parity of the MoE section of forward_port_block on GGUF layers
(dmh_upload_moe_layer_gguf, dmh_moe_forward_gguf) against the oracle's
composition of the same reference steps on the dequantized weights
(src/layers/port_scheduler.mojo:381-482: router_forward, swiglu_forward per
selected expert, the shared expert, shared_gate_forward,
moe_aggregate_forward), on the reference's fixtures/m9_port_mini.gguf and
on written GGUF layers of the Qwen3.6 shape (hidden 2048, inter 512, top-8).

Bars: expert ids and probabilities bit-exact; outputs within max-abs-err
<= 1e-3 x RMS of the oracle's no-residual output (the experts accumulate in
another fp32 order); the loader's and the block's error texts."""
import json
import os

import numpy as np
import pytest

from conftest import tol_check
from dismoen import DismoenError, gguf, synth

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
MINI = os.path.join(HERE, "golden", "m9_port_mini.gguf")
MINI_DIMS = (128, 8, 2, 64, 64)  # fixtures/m9_port_config_mini.json


def oracle_port_moe(oracle, g, model_layer, dims, x, residual, layer=0):
    """(y, ids, probs, y_no_residual) of the reference composition."""
    H, E, K, I, Ish = dims
    T = x.shape[0]
    p = f"blk.{model_layer}."

    def deq(name):
        t = g.tensors[g.tensor_map[p + name]]
        return oracle.dequant_gguf(t.dtype, g.read_raw(p + name), t.num_elements)

    ids, probs = oracle.router_forward(x, deq("ffn_gate_exps.weight"), T, H, E, K, layer=layer)
    w = {}
    routed = np.zeros((T, K * H), np.float32)
    for t in range(T):
        for k in range(K):
            e = int(ids[t, k])
            if e not in w:
                w[e] = (deq(f"ffn_gate.{e}.weight"), deq(f"ffn_up.{e}.weight"),
                        deq(f"ffn_down.{e}.weight"))
            routed[t, k * H:(k + 1) * H] = oracle.swiglu_forward(x[t], *w[e], 1, H, I)
    sh = oracle.swiglu_forward(x, deq("ffn_shared_gate.weight"), deq("ffn_shared_up.weight"),
                               deq("ffn_shared_down.weight"), T, H, Ish)
    gates = oracle.shared_gate_forward(x, deq("shared_gate.weight"), T, H, layer=layer)
    y0 = oracle.moe_aggregate(None, routed, probs, sh, gates, T, H, K, layer=layer)
    y = oracle.moe_aggregate(residual, routed, probs, sh, gates, T, H, K, layer=layer)
    return y.reshape(T, H), ids, probs, y0.reshape(T, H)


def _check_layer(block, oracle, g, model_layer, dims, slot, T, seed):
    rng = np.random.default_rng(seed)
    H = dims[0]
    x = synth.make_activations(rng, (T, H))
    res = rng.standard_normal((T, H)).astype(np.float32)
    y, ids, probs, _ = block.forward_port_moe_gguf(x, res, slot, T)
    y0, ids0, probs0, _ = block.forward_port_moe_gguf(x, None, slot, T)
    ref, rid, rp, ref0 = oracle_port_moe(oracle, g, model_layer, dims, x, res, layer=slot)
    assert np.array_equal(ids, rid) and np.array_equal(ids0, rid)
    assert np.array_equal(probs.view(np.uint32), rp.view(np.uint32))
    err, rms, ok = tol_check(y0, ref0)
    assert ok, (err, rms)
    # the residual is added last, in the reference's order
    assert np.array_equal(y.view(np.uint32), (y0 + res).view(np.uint32))
    err, _, _ = tol_check(y, ref)
    assert err <= 1e-3 * rms, err


def test_fixture_layers(block, oracle):
    with gguf.parse_gguf_index(MINI) as g:
        for ml in range(4):
            block.upload_layer_gguf(ml, MINI_DIMS, g, model_layer=ml)
            _check_layer(block, oracle, g, ml, MINI_DIMS, ml, T=3, seed=50 + ml)


@pytest.fixture(scope="module")
def qwen_gguf(tmp_path_factory):
    """A Qwen3.6-shape GGUF layer (hidden 2048, inter 512, shared 512) with 16
    experts of Q3_K, written once."""
    p = str(tmp_path_factory.mktemp("gguf") / "qwen_l3.gguf")
    gguf.write_gguf(p, synth.make_gguf_moe_layer(2048, 16, 512, 512, seed=7, model_layer=3))
    return p


def test_qwen_shape_q3_k(block, oracle, qwen_gguf):
    dims = (2048, 16, 8, 512, 512)
    with gguf.parse_gguf_index(qwen_gguf) as g:
        block.upload_layer_gguf(20, dims, g, model_layer=3)
        print("qwen-shape q3_k layer uploaded", flush=True)
        _check_layer(block, oracle, g, 3, dims, 20, T=1, seed=60)
        _check_layer(block, oracle, g, 3, dims, 20, T=5, seed=61)


def test_many_tokens_grouped_qwen_shape(block, oracle, qwen_gguf):
    """130 tokens on 16 experts: the grouped form's big units (more than 32
    of an expert's tokens, the shared expert's 128 + 2) and small units,
    against the oracle, and rows equal to the same tokens computed alone,
    bit for bit."""
    dims = (2048, 16, 8, 512, 512)
    with gguf.parse_gguf_index(qwen_gguf) as g:
        block.upload_layer_gguf(22, dims, g, model_layer=3)
        print("qwen-shape q3_k layer uploaded (grouped form)", flush=True)
        _check_layer(block, oracle, g, 3, dims, 22, T=130, seed=64)
    x = synth.make_activations(np.random.default_rng(65), (130, 2048))
    y, ids, probs, shg = block.forward_port_moe_gguf(x, None, 22, 130)
    for t in (0, 1, 63, 127, 128, 129):
        y1, i1, p1, s1 = block.forward_port_moe_gguf(x[t:t + 1], None, 22, 1)
        assert np.array_equal(y[t].view(np.uint32), y1[0].view(np.uint32)), t
        assert np.array_equal(ids[t], i1[0]) and np.array_equal(probs[t], p1[0]), t
    # 16 tokens take the lane-chain fp32 router: a non-finite activation is
    # the router stage's error, as in every other form
    xb = x[:16].copy()
    xb[5, 7] = np.nan
    with pytest.raises(DismoenError) as ei:
        block.forward_port_moe_gguf(xb, None, 22, 16)
    assert json.loads(str(ei.value)) == {"error_type": "ACT_LOAD_FAILED",
                                         "detail": "non-finite value in activation",
                                         "stage": "router", "layer": 22}
    y16, i16, p16, _ = block.forward_port_moe_gguf(x[:16], None, 22, 16)
    assert np.array_equal(i16, ids[:16]) and np.array_equal(p16, probs[:16])
    assert np.array_equal(y16.view(np.uint32), y[:16].view(np.uint32))


@pytest.mark.parametrize("ty", [12, 8, 0])
def test_other_expert_types(block, oracle, tmp_path, ty):
    dims = (256, 8, 4, 64, 96)
    p = str(tmp_path / f"t{ty}.gguf")
    gguf.write_gguf(p, synth.make_gguf_moe_layer(256, 8, 64, 96, seed=8 + ty, expert_type=ty))
    with gguf.parse_gguf_index(p) as g:
        block.upload_layer_gguf(21, dims, g)
        _check_layer(block, oracle, g, 0, dims, 21, T=4, seed=70 + ty)


def test_device_pointers_match_host(block, qwen_gguf):
    import torch
    dims = (2048, 16, 8, 512, 512)
    with gguf.parse_gguf_index(qwen_gguf) as g:
        block.upload_layer_gguf(22, dims, g, model_layer=3)
    T, H, K = 3, 2048, 8
    x = synth.make_activations(np.random.default_rng(80), (T, H))
    y_h, ids_h, probs_h, _ = block.forward_port_moe_gguf(x, None, 22, T)
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(x).to(dev)
    yd = torch.empty((T, H), dtype=torch.float32, device=dev)
    idd = torch.empty((T, K), dtype=torch.int32, device=dev)
    pd = torch.empty((T, K), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    block.forward_gguf_device(22, xd.data_ptr(), T, yd.data_ptr(), idd.data_ptr(), pd.data_ptr())
    block.sync()
    assert np.array_equal(yd.cpu().numpy().view(np.uint32), y_h.view(np.uint32))
    assert np.array_equal(idd.cpu().numpy(), ids_h) and np.array_equal(pd.cpu().numpy(), probs_h)


def _layer_file(tmp_path, name, mutate):
    ts = synth.make_gguf_moe_layer(128, 4, 32, 32, seed=9)
    ts = mutate(ts)
    p = str(tmp_path / name)
    gguf.write_gguf(p, ts)
    return gguf.parse_gguf_index(p)


def _upload_err(block, g, dims=(128, 4, 2, 32, 32)):
    with pytest.raises(DismoenError) as ei:
        block.upload_layer_gguf(23, dims, g)
    return str(ei.value)


def test_loader_errors(block, tmp_path):
    g = _layer_file(tmp_path, "miss.gguf", lambda ts: [t for t in ts if t[0] != "blk.0.ffn_up.2.weight"])
    assert json.loads(_upload_err(block, g)) == {
        "error_type": "WEIGHT_LOAD_FAILED", "detail": "tensor not found in GGUF index",
        "tensor": "blk.0.ffn_up.2.weight"}
    # the router of a wrong length fails first, with _expect_len's text
    g = _layer_file(tmp_path, "len.gguf", lambda ts: ts)
    msg = _upload_err(block, g, dims=(128, 5, 2, 32, 32))
    assert msg == ("GGUF_FILE_CORRUPT: dimension mismatch for tensor blk.0.ffn_gate_exps.weight: "
                   "expected 640 elements, got 512")

    def mixed(ts):
        rng = np.random.default_rng(1)
        out = list(ts)
        i = [k for k, t in enumerate(out) if t[0] == "blk.0.ffn_down.1.weight"][0]
        out[i] = (out[i][0], out[i][1], 12, synth.gguf_payload(rng, 12, 32 * 128))
        return out
    g = _layer_file(tmp_path, "mixed.gguf", mixed)
    assert _upload_err(block, g) == ("dmh_upload_moe_layer_gguf: expert tensor "
                                     "blk.0.ffn_down.1.weight has GGML type 12, the others 11")


def test_partial_blocks_rejected(block, oracle, tmp_path):
    # 100 x 36 Q8_0 weights are 112.5 blocks of 32 (F32 experts of that
    # size, blocks of one weight, upload)
    p = str(tmp_path / "f32.gguf")
    gguf.write_gguf(p, synth.make_gguf_moe_layer(100, 2, 36, 36, seed=3, expert_type=0))
    with gguf.parse_gguf_index(p) as g:
        block.upload_layer_gguf(23, (100, 2, 1, 36, 36), g)
        # rows of 100 and 36: the kernels' four-weights-per-lane form
        _check_layer(block, oracle, g, 0, (100, 2, 1, 36, 36), 23, T=3, seed=85)
    rng = np.random.default_rng(4)
    ts = synth.make_gguf_moe_layer(100, 2, 36, 36, seed=4, expert_type=0)
    ts = [(n, d, 8, synth.gguf_payload(rng, 8, -(-(36 * 100) // 32) * 32)) if ty == 0 and
          "shared_gate.weight" != n.split(".", 2)[2] else (n, d, ty, raw) for n, d, ty, raw in ts]
    p = str(tmp_path / "partial.gguf")
    gguf.write_gguf(p, ts)
    with gguf.parse_gguf_index(p) as g:
        assert _upload_err(block, g, dims=(100, 2, 1, 36, 36)) == (
            "dmh_upload_moe_layer_gguf: expert tensor blk.0.ffn_gate.0.weight has 3600 weights, "
            "not whole blocks of 32")


@pytest.mark.parametrize("T", [2, 1])
def test_forward_errors(block, tmp_path, T):
    """Error texts of the block; T = 1 takes the single-launch one-token form
    (k_gguf_one)."""
    dims = (128, 4, 2, 32, 32)
    g = _layer_file(tmp_path, "ok.gguf", lambda ts: ts)
    block.upload_layer_gguf(24, dims, g)
    x = synth.make_activations(np.random.default_rng(90), (T, 128))
    x[T - 1, 3] = np.nan
    with pytest.raises(DismoenError) as ei:
        block.forward_port_moe_gguf(x, None, 24, T)
    assert json.loads(str(ei.value)) == {"error_type": "ACT_LOAD_FAILED",
                                         "detail": "non-finite value in activation",
                                         "stage": "router", "layer": 24}

    # an infinite super-scale in the shared expert's gate: its first row's
    # gate projection is non-finite; the text names hidden and inter_sh the way
    # forward_port_block's swiglu_forward call does
    def bad(ts):
        out = list(ts)
        i = [k for k, t in enumerate(out) if t[0] == "blk.0.ffn_shared_gate.weight"][0]
        raw = bytearray(out[i][3])
        raw[112:114] = b"\x00\x7c"  # fp16 +inf
        out[i] = (out[i][0], out[i][1], out[i][2], bytes(raw))
        return out
    g = _layer_file(tmp_path, "inf.gguf", bad)
    block.upload_layer_gguf(25, dims, g)
    x = synth.make_activations(np.random.default_rng(91), (T, 128))
    with pytest.raises(DismoenError) as ei:
        block.forward_port_moe_gguf(x, None, 25, T)
    j = json.loads(str(ei.value))
    assert j["error_type"] == "EXPERT_ERROR" and j["detail"] == "non-finite in gate projection"
    assert (j["layer"], j["expert_id"]) == (128, 32)
    # the layer recovers: the same layer, finite inputs, other weights fine
    block.upload_layer_gguf(25, dims, _layer_file(tmp_path, "ok2.gguf", lambda ts: ts))
    block.forward_port_moe_gguf(x, None, 25, T)


def _tied_router(ts, E, H):
    """Router rows 2i + 1 copied from rows 2i: every logit appears twice."""
    out = list(ts)
    i = [k for k, t in enumerate(out) if t[0].endswith("ffn_gate_exps.weight")][0]
    raw = bytearray(out[i][3])
    rb = H // 32 * 34  # one Q8_0 row
    for e in range(0, E - 1, 2):
        raw[(e + 1) * rb:(e + 2) * rb] = raw[e * rb:(e + 1) * rb]
    out[i] = (out[i][0], out[i][1], out[i][2], bytes(raw))
    return out


@pytest.mark.parametrize("E,K,ties", [(256, 8, False), (256, 8, True), (256, 7, True),
                                      (300, 8, False), (300, 5, True)])
def test_single_token_routing(block, oracle, tmp_path, E, K, ties):
    """Single-token calls (one k_gguf_one launch) on 256 and 300 experts: the
    top-k on the logits; with duplicated router rows, equal probabilities
    inside the selection (ordered by id) and, for odd K, a tie at the top-k
    boundary (the exact-probability path)."""
    H, I, Ish = 256, 32, 32
    ts = synth.make_gguf_moe_layer(H, E, I, Ish, seed=E + K)
    if ties:
        ts = _tied_router(ts, E, H)
    p = str(tmp_path / "r.gguf")
    gguf.write_gguf(p, ts)
    dims = (H, E, K, I, Ish)
    with gguf.parse_gguf_index(p) as g:
        block.upload_layer_gguf(27, dims, g)
        for t in range(4):
            print(f"E={E} K={K} ties={ties} token {t}", flush=True)
            _check_layer(block, oracle, g, 0, dims, 27, T=1, seed=100 + t)


def test_many_tokens_cross_launch_chunks(block, tmp_path):
    """65537 tokens: the router and down launches split at 65535 tokens, the
    gate/up launch at 65535 / (K + 1); rows on either side of every split
    equal the same tokens computed alone, bit for bit."""
    dims = (128, 4, 2, 32, 32)
    g = _layer_file(tmp_path, "many.gguf", lambda ts: ts)
    block.upload_layer_gguf(26, dims, g)
    T = 65537
    x = synth.make_activations(np.random.default_rng(95), (T, 128))
    y, ids, probs, shg = block.forward_port_moe_gguf(x, None, 26, T)
    for t in (0, 21844, 21845, 43690, 43691, 65534, 65535, 65536):
        y1, i1, p1, s1 = block.forward_port_moe_gguf(x[t:t + 1], None, 26, 1)
        assert np.array_equal(y[t].view(np.uint32), y1[0].view(np.uint32)), t
        assert np.array_equal(ids[t], i1[0]) and np.array_equal(probs[t], p1[0]), t
        assert s1[0] == shg[t], t
