"""GPU parity of the MoE block (dmh_moe_forward / dmh_moe_stack_forward)
against the CPU oracle's restatement of the reference composition.

Bar: selected expert ids and their probabilities bit-exact; the no-residual
output within max-abs-err <= 1e-3 x RMS(oracle output)."""
import numpy as np
import pytest

from conftest import f10, tol_check
from dismoen import DismoenError, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def toy(block):
    L = synth.make_layer(**synth.CONFIG_TOY, seed=0)
    block.upload_layer(0, L)
    return L


@pytest.fixture(scope="module")
def qwen(block):
    L = synth.make_layer(**synth.CONFIG_QWEN36, seed=1)
    block.upload_layer(1, L)
    return L


def check_layer(block, oracle, L, layer, x, residual=None):
    T = x.shape[0]
    y, ids, probs, shg = block.forward_arrays(layer, x, T, residual=residual)
    yo, ido, po, so = oracle.moe_layer_q4(L, x, T, residual=residual)
    assert np.array_equal(ids, ido)
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    assert np.array_equal(shg.view(np.uint32), so.view(np.uint32))
    if residual is None:
        err, rms, ok = tol_check(y, yo)
        assert ok, (err, rms)
    else:
        yn, _, _, _ = block.forward_arrays(layer, x, T)
        err, rms, ok = tol_check(y - residual, yo - residual)
        assert ok, (err, rms)
    return y, yo


def test_toy_layer_single_token(block, oracle, toy):
    x = synth.make_activations(np.random.default_rng(100), (1, 256))
    check_layer(block, oracle, toy, 0, x)


def test_toy_layer_tokens_and_residual(block, oracle, toy):
    x = synth.make_activations(np.random.default_rng(101), (7, 256))
    check_layer(block, oracle, toy, 0, x)
    check_layer(block, oracle, toy, 0, x, residual=x)


def test_toy_reference_api_mirror(block, oracle, toy):
    x = synth.make_activations(np.random.default_rng(102), (3, 256))
    y, info = block.forward_moe_block(x, 0, 3)
    yo, ido, po, _ = oracle.moe_layer_q4(toy, x, 3, residual=x)
    assert info.selected_experts == ido.tolist() and info.num_tokens == 3 and info.top_k == 4
    err, rms, ok = tol_check(y.reshape(3, -1) - x, yo - x)
    assert ok


def test_qwen_layer_decode_tokens(block, oracle, qwen):
    x = synth.make_activations(np.random.default_rng(103), (6, 2048))
    for t in range(6):
        check_layer(block, oracle, qwen, 1, x[t:t + 1])


@pytest.mark.parametrize("T", [1, 8, 32])
def test_qwen_layer_f10_gate(block, oracle, qwen, T):
    """The reference's own MoE-layer comparison gate G-M3-1 (delta_max <= 1e-3,
    epsilon_rel <= 1e-4 over the whole output, compare.rs:1041-1043) on the
    decode kernel (16 single-token calls) and the grouped path (8 and 32
    tokens per call)."""
    x = synth.make_activations(np.random.default_rng(105 + T), (16 if T == 1 else T, 2048))
    if T == 1:
        y = np.concatenate([block.forward_arrays(1, x[t:t + 1], 1)[0] for t in range(16)])
    else:
        y = block.forward_arrays(1, x, T)[0]
    yo = oracle.moe_layer_q4(qwen, x, x.shape[0])[0]
    dmax, eps, ok = f10(yo, y)
    assert ok, (dmax, eps)


def test_deterministic_run_to_run(block, qwen):
    x = synth.make_activations(np.random.default_rng(104), (2, 2048))
    a = block.forward_arrays(1, x, 2)
    b = block.forward_arrays(1, x, 2)
    for u, v in zip(a, b):
        assert np.array_equal(np.asarray(u).view(np.uint8), np.asarray(v).view(np.uint8))


def test_nonfinite_activation_error_matches_oracle(block, oracle, toy):
    x = synth.make_activations(np.random.default_rng(105), (2, 256))
    x[1, 17] = np.nan
    with pytest.raises(oracle.OracleError) as eo:
        oracle.moe_layer_q4(toy, x, 2)
    with pytest.raises(DismoenError) as eg:
        block.forward_arrays(0, x, 2)
    assert str(eg.value) == str(eo.value)
    # the context stays usable after an error
    x[1, 17] = 0.0
    check_layer(block, oracle, toy, 0, x)


def test_single_token_host_pointers_match_device_and_oracle(block, oracle, qwen):
    """The single-token host-pointer call (the kernel reads x and the
    residual from, and writes the outputs into, page-locked host memory, and
    its last workgroup writes the status key there) gives the device-pointer
    call's bits, with and without a residual, and the oracle's routing."""
    import torch
    dev = torch.device("cuda:0")
    H, K = 2048, 8
    x = synth.make_activations(np.random.default_rng(110), (4, H))
    for t in range(4):
        for res in (None, x[t]):
            y = np.empty(H, np.float32)
            ids = np.empty(K, np.int32)
            probs = np.empty(K, np.float32)
            shg = np.empty(1, np.float32)
            block.forward_into(1, x[t], 1, y, ids, probs, shg, residual=res)
            xd = torch.from_numpy(x[t].copy()).to(dev)
            rd = None if res is None else torch.from_numpy(res.copy()).to(dev)
            yd = torch.empty(H, dtype=torch.float32, device=dev)
            idd = torch.empty(K, dtype=torch.int32, device=dev)
            pd = torch.empty(K, dtype=torch.float32, device=dev)
            sd = torch.empty(1, dtype=torch.float32, device=dev)
            torch.cuda.synchronize()  # made on torch's stream, read on the library's
            block.forward_device(1, xd.data_ptr(), 1, yd.data_ptr(), idd.data_ptr(),
                                 pd.data_ptr(), sd.data_ptr(),
                                 None if rd is None else rd.data_ptr())
            block.sync()
            assert np.array_equal(y.view(np.uint32), yd.cpu().numpy().view(np.uint32))
            assert np.array_equal(ids, idd.cpu().numpy())
            assert np.array_equal(probs.view(np.uint32), pd.cpu().numpy().view(np.uint32))
            assert np.array_equal(shg.view(np.uint32), sd.cpu().numpy().view(np.uint32))
            yo, ido, po, so = oracle.moe_layer_q4(qwen, x[t:t + 1], 1,
                                                  residual=None if res is None else res[None])
            assert np.array_equal(ids, ido.reshape(-1))
            assert np.array_equal(probs.view(np.uint32), po.reshape(-1).view(np.uint32))
    with pytest.raises(ValueError):
        block.forward_into(1, x[0].astype(np.float64), 1, np.empty(H, np.float32))


def test_single_token_host_errors_and_recovery(block, oracle, toy):
    """Errors of single-token host-pointer calls (the status key comes back
    from the kernel itself, or from the multi-kernel replay that names the
    failing check) match the oracle's texts, and the call after an error,
    and after a device-pointer call that failed, computes normally."""
    import torch
    x = synth.make_activations(np.random.default_rng(111), (1, 256))
    good = block.forward_arrays(0, x, 1)
    for scale in (1e15, 1e17, 1e19, 1e21, 3e37):
        xs = (x * np.float32(scale)).astype(np.float32)
        msgs = []
        for call in (lambda: block.forward_arrays(0, xs, 1),
                     lambda: oracle.moe_layer_q4(toy, xs, 1)):
            try:
                call()
                msgs.append(None)
            except (DismoenError, oracle.OracleError) as e:
                msgs.append(str(e))
        assert msgs[0] == msgs[1], (scale, msgs)
        again = block.forward_arrays(0, x, 1)
        for u, v in zip(good, again):
            assert np.array_equal(np.asarray(u).view(np.uint8), np.asarray(v).view(np.uint8))
    xn = x.copy()
    xn[0, 3] = np.inf
    with pytest.raises(DismoenError):
        block.forward_arrays(0, xn, 1)
    # a failing device-pointer call leaves a sticky error for sync(); the
    # next host call resets the key first and reports only its own result
    xd = torch.from_numpy(xn).to("cuda:0")
    yd = torch.empty(256, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    block.forward_device(0, xd.data_ptr(), 1, yd.data_ptr())
    again = block.forward_arrays(0, x, 1)
    for u, v in zip(good, again):
        assert np.array_equal(np.asarray(u).view(np.uint8), np.asarray(v).view(np.uint8))
    block.sync()


def test_upload_rejects_reserved_code_and_bad_scale(block):
    L = synth.make_layer(**synth.CONFIG_TOY, seed=7)
    L.d_packed = L.d_packed.copy()
    L.d_packed[1000] = 0x80
    with pytest.raises(DismoenError, match="reserved nibble"):
        block.upload_layer(5, L)
    L = synth.make_layer(**synth.CONFIG_TOY, seed=7)
    L.gu_scales = L.gu_scales.copy()
    L.gu_scales[3] = 0x7E00
    with pytest.raises(DismoenError, match="scale is NaN or Inf at group 3"):
        block.upload_layer(5, L)


def test_stack_of_layers(block, oracle):
    layers = [synth.make_layer(**synth.CONFIG_TOY, seed=20 + l) for l in range(4)]
    for l, L in enumerate(layers):
        block.upload_layer(10 + l, L)
    x = synth.make_activations(np.random.default_rng(106), (3, 256))
    out, ids, probs = block.forward_stack(x, 10, 4, 3, eps=1e-6)
    oo, ido, po = oracle.moe_stack_q4(layers, x, 3, 1e-6)
    assert np.array_equal(ids, ido)
    err, rms, ok = tol_check(out - x, oo - x)
    assert ok, (err, rms)


def test_device_generated_layers_stack_decode(block, oracle):
    """Layers drawn on the GPU and uploaded from device pointers (the path of
    the 40-layer workload), one decode token through two of them."""
    import torch
    cfg = synth.CONFIG_QWEN36
    dims = (cfg["hidden"], cfg["num_experts"], cfg["top_k"], cfg["inter"], cfg["inter_sh"])
    layers = []
    for l in range(2):
        W = synth.make_layer_device(**cfg, seed=500 + l, device="cuda")
        torch.cuda.synchronize()
        block.upload_layer_device(20 + l, dims, {k: v.data_ptr() for k, v in W.items()})
        block.sync()
        host = {k: v.cpu().numpy().view(np.uint16 if v.dtype == torch.int16 else np.uint8)
                for k, v in W.items()}
        layers.append(synth.MoELayerQ4(*dims, 32, **host))
        del W
    x = synth.make_activations(np.random.default_rng(108), (1, 2048))
    out, ids, probs = block.forward_stack(x, 20, 2, 1, eps=1e-6)
    oo, ido, po = oracle.moe_stack_q4(layers, x, 1, 1e-6)
    assert np.array_equal(ids, ido)
    # layer 0 routes the same input bits; deeper layers see the previous
    # layer's output, equal only within the tolerance
    assert np.array_equal(probs[0].view(np.uint32), po[0].view(np.uint32))
    err, rms, ok = tol_check(out - x, oo - x)
    assert ok, (err, rms)
    # the device-pointer form (layer 0 reads x, the last layer writes out) gives
    # the same bits
    xd = torch.from_numpy(x).to("cuda")
    od = torch.empty_like(xd)
    torch.cuda.synchronize()
    block.forward_stack_device(xd.data_ptr(), 20, 2, 1, od.data_ptr(), eps=1e-6)
    block.sync()
    assert np.array_equal(od.cpu().numpy().view(np.uint32), out.view(np.uint32))
    block.free_layer(20)
    block.free_layer(21)


def test_interleaved_layers_of_different_shapes(block, oracle, toy, qwen):
    """Launches of layers with different workgroup counts alternate on one
    context (each layer keeps its own handoff counters)."""
    rng = np.random.default_rng(107)
    for rep in range(3):
        xt = synth.make_activations(rng, (1, 256))
        xq = synth.make_activations(rng, (1, 2048))
        check_layer(block, oracle, toy, 0, xt)
        check_layer(block, oracle, qwen, 1, xq)


@pytest.mark.parametrize("gap_ulp", [0, 1, 2, 3, 4, 8, 64])
def test_routing_near_ties_at_topk_boundary(block, oracle, gap_ulp):
    """Experts 3 and 4 get logits gap_ulp fp32 ulp apart around the 4th place
    (0 = exact tie, lowest id must win); ids and probabilities must equal the
    oracle's bit for bit, including the path that forms the softmax
    normaliser before selecting."""
    L = synth.make_layer(**synth.CONFIG_TOY, seed=30)
    H, E = L.hidden, L.num_experts
    w = np.zeros((E, H), np.float32)
    w[:, 0] = 0.5
    w[0, 0], w[1, 0], w[2, 0] = 1.5, 1.25, 1.125
    w[3, 0], w[4, 0] = 1.0, 1.0
    w[3, 1] = 1.0
    w[4, 1] = 1.0 + gap_ulp * 2.0 ** -7  # z4 - z3 = gap_ulp * 2^-23
    L.router_bf16 = synth.f32_to_bf16_bits(w).reshape(-1)
    assert np.array_equal(synth.bf16_bits_to_f32(L.router_bf16).reshape(E, H)[:, :2], w[:, :2])
    block.upload_layer(40 + gap_ulp % 50, L)
    x = np.zeros((1, H), np.float32)
    x[0, 0], x[0, 1] = 1.0, 2.0 ** -16
    y, ids, probs, shg = block.forward_arrays(40 + gap_ulp % 50, x, 1)
    yo, ido, po, so = oracle.moe_layer_q4(L, x, 1)
    assert np.array_equal(ids, ido), (ids, ido)
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    err, rms, ok = tol_check(y, yo)
    assert ok, (err, rms)


@pytest.mark.parametrize("cfg", ["toy", "qwen"])
def test_upload_from_reference_files(block, tmp_path, cfg):
    """A layer written as the reference's quant model + safetensors shard and
    uploaded from them computes the same bits as the same layer uploaded from
    arrays (single token and a batch)."""
    from dismoen import formats
    c = synth.CONFIG_TOY if cfg == "toy" else synth.CONFIG_QWEN36
    L = synth.make_layer(**c, seed=41)
    qp, sp = str(tmp_path / "m.quant"), str(tmp_path / "m.safetensors")
    formats.write_layer_files(qp, sp, L, model_layer=7)
    dims = (c["hidden"], c["num_experts"], c["top_k"], c["inter"], c["inter_sh"])
    with formats.scan_quant_file(qp) as q, formats.read_header(sp) as s:
        block.upload_layer_files(30, dims, q, s, model_layer=7)
    block.upload_layer(31, L)
    x = synth.make_activations(np.random.default_rng(109), (3, c["hidden"]))
    for T in (1, 3):
        a = block.forward_arrays(30, x[:T], T)
        b = block.forward_arrays(31, x[:T], T)
        for u, v in zip(a, b):
            assert np.array_equal(np.asarray(u).view(np.uint8), np.asarray(v).view(np.uint8))
    block.free_layer(30)
    block.free_layer(31)


def test_upload_from_files_missing_expert(block, tmp_path):
    from dismoen import DismoenError, formats
    c = synth.CONFIG_TOY
    L = synth.make_layer(**c, seed=42)
    qp, sp = str(tmp_path / "m.quant"), str(tmp_path / "m.safetensors")
    formats.write_layer_files(qp, sp, L, model_layer=0)
    dims = (c["hidden"], c["num_experts"], c["top_k"], c["inter"], c["inter_sh"])
    with formats.scan_quant_file(qp) as q, formats.read_header(sp) as s:
        with pytest.raises(DismoenError) as ei:
            block.upload_layer_files(32, dims, q, s, model_layer=1)
    assert str(ei.value) == ('{"error_type":"WEIGHT_LOAD_FAILED","detail":"required router gate'
                             ' tensor not in weight_map: model.layers.1.mlp.gate.weight",'
                             '"shard":"","tensor_name":"model.layers.1.mlp.gate.weight"}')


def test_two_contexts_on_one_device(block, oracle, qwen):
    """With a second live context on the device the single-launch decode
    kernel is launched cooperatively (every workgroup resident); both
    contexts still route and compute as the oracle does."""
    from dismoen import MoEBlock
    x = synth.make_activations(np.random.default_rng(113), (2, 2048))
    with MoEBlock(0) as other:
        other.upload_layer(0, qwen)
        for t in range(2):
            y2, ids2, p2, s2 = other.forward_arrays(0, x[t:t + 1], 1)
            check_layer(block, oracle, qwen, 1, x[t:t + 1])
            yo, ido, po, so = oracle.moe_layer_q4(qwen, x[t:t + 1], 1)
            assert np.array_equal(ids2, ido)
            assert np.array_equal(p2.view(np.uint32), po.view(np.uint32))
            err, rms, ok = tol_check(y2, yo)
            assert ok, (err, rms)
    # back to one context: the plain launch
    check_layer(block, oracle, qwen, 1, x[:1])


def test_two_contexts_from_two_threads_at_once(block, oracle, qwen):
    """Two contexts on one device, each driven by its own host thread at the
    same time (single-token host-pointer calls: cooperative launches of the
    fused decode kernel, which the runtime admits one grid at a time): every
    token of both matches the oracle."""
    import threading

    from dismoen import MoEBlock
    N = 24
    xs = synth.make_activations(np.random.default_rng(114), (2, N, 2048))
    outs = [[None] * N, [None] * N]
    errs = []
    with MoEBlock(0) as other:
        other.upload_layer(1, qwen)
        ctxs = (block, other)

        def run(c):
            try:
                for t in range(N):
                    outs[c][t] = ctxs[c].forward_arrays(1, xs[c, t:t + 1], 1)
            except Exception as e:  # reported below, on the main thread
                errs.append(repr(e))

        th = [threading.Thread(target=run, args=(c,)) for c in range(2)]
        for t in th:
            t.start()
        for t in th:
            t.join()
    assert not errs, errs
    for c in range(2):
        yo, ido, po, so = oracle.moe_layer_q4(qwen, xs[c], N)
        for t in range(N):
            y, ids, probs, shg = outs[c][t]
            assert np.array_equal(ids[0], ido[t]), (c, t)
            assert np.array_equal(probs[0].view(np.uint32), po[t].view(np.uint32)), (c, t)
            err, rms, ok = tol_check(y[0], yo[t])
            assert ok, (c, t, err, rms)
