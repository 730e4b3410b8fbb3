"""GPU parity of the port block's MoE section with its RMSNorm
(dmh_port_moe_forward: xn = rmsnorm(x_mid, gamma, eps), y = x_mid + MoE(xn),
src/layers/port_scheduler.mojo:381-485, src/layers/rmsnorm.mojo:10-48) and of
the stack of such sections (dmh_moe_stack_forward), against the oracle.

Two norm orders: the reference's (squares added in element order,
or_rmsnorm) and the library's fast tree order (DMH_F_NORM_TREE,
or_rmsnorm_tree256).  Given the same input bits the GPU's ids, probabilities
and shared gate equal the oracle's bit for bit in either order; outputs are
within max-abs-err <= 1e-3 x RMS of the no-residual part.  Deeper layers of a
stack are checked on the GPU's own previous output, so each layer is compared
on identical inputs."""
import numpy as np
import pytest

from conftest import tol_check
from dismoen import DismoenError, synth

pytestmark = pytest.mark.gpu


def _gamma(rng, H):
    return (1.0 + 0.25 * rng.standard_normal(H)).astype(np.float32)


def _residual_stream(rng, shape):
    """Activations that are not bf16 values (a residual stream after mixing)."""
    return (rng.standard_normal(shape) * 1.7).astype(np.float32)


def _port_check(block, oracle, L, layer, x, gamma, eps, tree):
    T = x.shape[0]
    y, ids, probs, shg = block.forward_port_moe_norm(x, layer, T, eps=eps, tree=tree)
    xn = np.stack([oracle.rmsnorm(x[t], gamma, eps, tree=tree) for t in range(T)])
    yo, ido, po, so = oracle.moe_layer_q4(L, xn, T, residual=x)
    assert np.array_equal(ids, ido)
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    assert np.array_equal(shg.view(np.uint32), so.view(np.uint32))
    err, rms, ok = tol_check(y - x, yo - x)
    assert ok, (err, rms)
    return y, ids


@pytest.mark.parametrize("tree", [False, True])
@pytest.mark.parametrize("T", [1, 4])
def test_port_moe_with_norm_toy_vs_oracle(block, oracle, tree, T):
    rng = np.random.default_rng(700 + T + 10 * tree)
    L = synth.make_layer(**synth.CONFIG_TOY, seed=70)
    block.upload_layer(70, L)
    g = _gamma(rng, 256)
    block.set_layer_norm(70, g)
    x = _residual_stream(rng, (T, 256))
    _port_check(block, oracle, L, 70, x, g, 1e-6, tree)
    # gamma reset to 1
    block.set_layer_norm(70, None)
    _port_check(block, oracle, L, 70, x, None, 1e-5, tree)
    block.free_layer(70)


@pytest.mark.parametrize("tree", [False, True])
def test_port_moe_with_norm_qwen_vs_oracle(block, oracle, tree):
    rng = np.random.default_rng(710 + tree)
    L = synth.make_layer(**synth.CONFIG_QWEN36, seed=71)
    block.upload_layer(71, L)
    g = _gamma(rng, 2048)
    block.set_layer_norm(71, g)
    x = _residual_stream(rng, (3, 2048))
    for t in range(3):
        _port_check(block, oracle, L, 71, x[t:t + 1], g, 1e-6, tree)
    _port_check(block, oracle, L, 71, x, g, 1e-6, tree)
    block.free_layer(71)


def test_norm_errors_match_reference(block, oracle):
    L = synth.make_layer(**synth.CONFIG_TOY, seed=72)
    block.upload_layer(72, L)
    x = _residual_stream(np.random.default_rng(720), (1, 256))
    for eps in (0.0, -1.0, float("nan"), float("inf")):
        with pytest.raises(DismoenError) as eg:
            block.forward_port_moe_norm(x, 72, 1, eps=eps)
        with pytest.raises(oracle.OracleError) as eo:
            oracle.rmsnorm(x[0], None, eps)
        assert str(eg.value) == str(eo.value)
    with pytest.raises(DismoenError) as eg:
        block.set_layer_norm(72, np.ones(255, np.float32))
    assert str(eg.value) == ('{"error_type":"NORM_ERROR","detail":"length mismatch",'
                             '"stage":"rmsnorm"}')
    block.free_layer(72)


@pytest.mark.parametrize("tree", [False, True])
def test_toy_stack_with_gamma_equals_chain_and_oracle(block, oracle, tree):
    """A stack call equals the chain of port calls bit for bit, and each layer
    of the chain matches the oracle on the chain's own input."""
    rng = np.random.default_rng(730 + tree)
    layers = [synth.make_layer(**synth.CONFIG_TOY, seed=73 + l) for l in range(4)]
    gammas = [_gamma(rng, 256) for _ in layers]
    for l, (L, g) in enumerate(zip(layers, gammas)):
        block.upload_layer(80 + l, L)
        block.set_layer_norm(80 + l, g)
    x = _residual_stream(rng, (3, 256))
    out, ids, probs = block.forward_stack(x, 80, 4, 3, eps=1e-6, tree=tree)
    h = x
    for l, (L, g) in enumerate(zip(layers, gammas)):
        y, lid = _port_check(block, oracle, L, 80 + l, h, g, 1e-6, tree)
        assert np.array_equal(lid, ids[l])
        h = y
    assert np.array_equal(out.view(np.uint32), h.view(np.uint32))
    # and the whole stack against the oracle's own stack (outputs within the bar)
    oo, ido, po = oracle.moe_stack_q4(layers, x, 3, 1e-6, gammas=gammas, tree=tree)
    assert np.array_equal(ido[0], ids[0])
    err, rms, ok = tol_check(out - x, oo - x)
    assert ok, (err, rms)
    for l in range(4):
        block.free_layer(80 + l)


def test_qwen_40_layer_stack_per_layer_vs_oracle(block, oracle):
    """Configuration 2: 40 Qwen3.6-shape layers (drawn on the GPU, uploaded
    from device pointers, each with its own gamma), one decode token through
    all 40 port MoE sections.  Every layer is compared with the oracle on the
    GPU's own input to that layer, in both norm orders: ids and
    probabilities bit-exact, outputs within the bar.  The stack call then
    reproduces the chain of per-layer calls bit for bit."""
    import torch
    cfg = synth.CONFIG_QWEN36
    dims = (cfg["hidden"], cfg["num_experts"], cfg["top_k"], cfg["inter"], cfg["inter_sh"])
    NL, base, eps = 40, 100, 1e-6
    rng = np.random.default_rng(740)
    x = _residual_stream(rng, (1, 2048))
    h_seq, h_tree = x, x
    ids_seq, ids_tree = [], []
    for l in range(NL):
        W = synth.make_layer_device(**cfg, seed=900 + l, device="cuda")
        torch.cuda.synchronize()
        block.upload_layer_device(base + l, dims, {k: v.data_ptr() for k, v in W.items()})
        g = _gamma(rng, 2048)
        block.set_layer_norm(base + l, g)
        block.sync()
        host = {k: v.cpu().numpy().view(np.uint16 if v.dtype == torch.int16 else np.uint8)
                for k, v in W.items()}
        del W
        L = synth.MoELayerQ4(*dims, 32, **host)
        y, ids = _port_check(block, oracle, L, base + l, h_seq, g, eps, tree=False)
        ids_seq.append(ids)
        h_seq = y
        y, ids = _port_check(block, oracle, L, base + l, h_tree, g, eps, tree=True)
        ids_tree.append(ids)
        h_tree = y
        del host, L
        print(f"layer {l} ok", flush=True)
    for tree, h_chain, ids_chain in ((False, h_seq, ids_seq), (True, h_tree, ids_tree)):
        out, ids, probs = block.forward_stack(x, base, NL, 1, eps=eps, tree=tree)
        assert np.array_equal(ids, np.stack(ids_chain))
        assert np.array_equal(out.view(np.uint32), h_chain.view(np.uint32))
    for l in range(NL):
        block.free_layer(base + l)


def test_stream_switch_between_device_calls(block, oracle):
    """dmh_set_stream orders work queued on the old stream before the new
    one: device-pointer calls issued on two streams alternately route as the
    oracle does."""
    import torch
    L = synth.make_layer(**synth.CONFIG_QWEN36, seed=75)
    block.upload_layer(75, L)
    x = synth.make_activations(np.random.default_rng(750), (4, 2048))
    xd = torch.from_numpy(x).to("cuda")
    yd = torch.empty_like(xd)
    idd = torch.empty((4, 8), dtype=torch.int32, device="cuda")
    pd = torch.empty((4, 8), dtype=torch.float32, device="cuda")
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    for t in range(4):
        block.set_stream(side.cuda_stream if t % 2 else None)
        block.forward_device(75, xd[t].data_ptr(), 1, yd[t].data_ptr(), idd[t].data_ptr(),
                             pd[t].data_ptr())
    block.set_stream(None)
    block.sync()
    yo, ido, po, so = oracle.moe_layer_q4(L, x, 4)
    assert np.array_equal(idd.cpu().numpy(), ido)
    assert np.array_equal(pd.cpu().numpy().view(np.uint32), po.view(np.uint32))
    err, rms, ok = tol_check(yd.cpu().numpy(), yo)
    assert ok, (err, rms)
    block.free_layer(75)


@pytest.mark.parametrize("H,cfg", [(256, "toy"), (2048, "qwen")])
def test_norm_order_distinguishing_input(block, oracle, H, cfg):
    """x[0]^2 = 2^24 and every other square 1: added in element order each 1
    is lost, in the tree order they are kept, so the two orders give
    different normalised inputs.  Each GPU mode must match its own oracle
    order bit for bit in the probabilities."""
    c = synth.CONFIG_TOY if cfg == "toy" else synth.CONFIG_QWEN36
    L = synth.make_layer(**c, seed=76)
    block.upload_layer(76, L)
    x = np.ones((1, H), np.float32)
    x[0, 0] = 4096.0
    x[0, 1::2] = -1.0
    assert not np.array_equal(oracle.rmsnorm(x[0], None, 1e-6),
                              oracle.rmsnorm(x[0], None, 1e-6, tree=True))
    for tree in (False, True):
        _port_check(block, oracle, L, 76, x, None, 1e-6, tree)
    block.free_layer(76)
