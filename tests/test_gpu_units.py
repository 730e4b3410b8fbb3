"""GPU parity of the unit entry points of the boundary against the CPU
oracle: dmh_experts_forward (swiglu_forward, WorkerPool.parallel_moe_experts),
dmh_shared_gate_forward (shared_gate_forward) and dmh_moe_aggregate
(moe_aggregate_forward, moe_combine_no_residual).

Bars: expert outputs within max-abs-err <= 1e-3 x RMS of the oracle's fp32
SwiGLU on the same bf16-rounded weights; the shared gate and the aggregation
bit-exact (the same fp32 operations in the reference's order)."""
import json

import numpy as np
import pytest

from conftest import tol_check
from dismoen import DismoenError, synth

pytestmark = pytest.mark.gpu

LAYER_TOY, LAYER_QWEN = 10, 11


@pytest.fixture(scope="module")
def toy(block):
    L = synth.make_layer(**synth.CONFIG_TOY, seed=21)
    block.upload_layer(LAYER_TOY, L)
    return L


@pytest.fixture(scope="module")
def qwen(block):
    L = synth.make_layer(**synth.CONFIG_QWEN36, seed=22)
    block.upload_layer(LAYER_QWEN, L)
    return L


def _deq(oracle, scales, packed, rows, cols, G):
    bits = oracle.dequant_q4_bf16(scales, packed, rows * cols, G)
    return oracle.bf16_bits_to_f32(bits).reshape(rows, cols)


def expert_f32(oracle, L, e):
    """fp32 (bf16-rounded) gate, up, down of routed expert e, or the shared one (e < 0)."""
    H, E, I, Ish, G = L.hidden, L.num_experts, L.inter, L.inter_sh, L.group_size
    if e < 0:
        gs = L.sh_gu_scales.reshape(2, -1)
        gp = L.sh_gu_packed.reshape(2, -1)
        return (_deq(oracle, gs[0], gp[0], Ish, H, G), _deq(oracle, gs[1], gp[1], Ish, H, G),
                _deq(oracle, L.sh_d_scales, L.sh_d_packed, H, Ish, G), Ish)
    gs = L.gu_scales.reshape(E, 2, -1)
    gp = L.gu_packed.reshape(E, 2, -1)
    ds = L.d_scales.reshape(E, -1)
    dp = L.d_packed.reshape(E, -1)
    return (_deq(oracle, gs[e, 0], gp[e, 0], I, H, G), _deq(oracle, gs[e, 1], gp[e, 1], I, H, G),
            _deq(oracle, ds[e], dp[e], H, I, G), I)


def oracle_expert(oracle, L, e, x):
    wg, wu, wd, inter = expert_f32(oracle, L, e)
    T = x.shape[0]
    return oracle.swiglu_forward(x, wg, wu, wd, T, L.hidden, inter, expert_id=e).reshape(T, -1)


@pytest.mark.parametrize("cfg", ["toy", "qwen"])
def test_experts_forward_matches_swiglu(block, oracle, toy, qwen, cfg):
    L, layer = (toy, LAYER_TOY) if cfg == "toy" else (qwen, LAYER_QWEN)
    rng = np.random.default_rng(31)
    T, k = (3, 5) if cfg == "toy" else (2, 8)
    x = synth.make_activations(rng, (T, L.hidden))
    ids = rng.integers(0, L.num_experts, size=(T, k)).astype(np.int32)
    ids[0, 1] = ids[0, 0]  # a repeated expert within a token
    out, sh = block.experts_forward(x, ids, layer, T, with_shared=True)
    assert out.shape == (T, k, L.hidden) and sh.shape == (T, L.hidden)
    cache = {}
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            if e not in cache:
                cache[e] = oracle_expert(oracle, L, e, x)
            err, rms, ok = tol_check(out[t, j], cache[e][t])
            assert ok, (t, j, e, err, rms)
    ref_sh = oracle_expert(oracle, L, -1, x)
    for t in range(T):
        err, rms, ok = tol_check(sh[t], ref_sh[t])
        assert ok, (t, err, rms)


def test_swiglu_forward_mirror(block, oracle, toy):
    x = synth.make_activations(np.random.default_rng(32), (4, toy.hidden))
    for e in (-1, 0, toy.num_experts - 1):
        y = block.swiglu_forward(x, 4, LAYER_TOY, expert_id=e)
        ref = oracle_expert(oracle, toy, e, x).reshape(-1)
        err, rms, ok = tol_check(y, ref)
        assert ok, (e, err, rms)


def test_parallel_moe_experts_mirror(block, oracle, toy):
    """One token, K experts: the layout out_routed[k*H + d] of parallel_moe_experts,
    against the oracle's worker pool on fp32 weight tables."""
    x = synth.make_activations(np.random.default_rng(33), (1, toy.hidden))
    sel = np.array([3, 7, 0, 12], np.int64)
    out = block.parallel_moe_experts(x, sel, LAYER_TOY)
    wg, wu, wd = {}, {}, {}
    for e in range(toy.num_experts):
        wg[e], wu[e], wd[e], _ = expert_f32(oracle, toy, e)
    pool = oracle.Pool(2)
    ref = pool.parallel_moe_experts(len(sel), toy.hidden, toy.inter, x.reshape(-1), sel,
                                    [wg[e] for e in range(toy.num_experts)],
                                    [wu[e] for e in range(toy.num_experts)],
                                    [wd[e] for e in range(toy.num_experts)])
    pool.close()
    for j in range(len(sel)):
        seg = slice(j * toy.hidden, (j + 1) * toy.hidden)
        err, rms, ok = tol_check(out[seg], np.asarray(ref)[seg])
        assert ok, (j, err, rms)


def test_experts_single_token_single_expert_qwen(block, oracle, qwen):
    x = synth.make_activations(np.random.default_rng(34), (1, qwen.hidden))
    out, _ = block.experts_forward(x, np.array([[200]], np.int32), LAYER_QWEN, 1)
    err, rms, ok = tol_check(out.reshape(-1), oracle_expert(oracle, qwen, 200, x).reshape(-1))
    assert ok, (err, rms)


def test_experts_bad_id(block, toy):
    x = synth.make_activations(np.random.default_rng(35), (2, toy.hidden))
    with pytest.raises(DismoenError) as ei:
        block.experts_forward(x, np.array([[1, 2], [3, toy.num_experts]], np.int32), LAYER_TOY, 2)
    j = json.loads(str(ei.value))
    assert j["error_type"] == "EXPERT_ERROR" and j["detail"] == "expert id out of range"
    assert j["expert_id"] == toy.num_experts and j["layer"] == LAYER_TOY


def test_experts_bad_id_device(block, toy):
    """Device pointers: the id is checked on the device, reported by sync()."""
    import torch
    dev = torch.device("cuda:0")
    T, H, k = 2, toy.hidden, 2
    x = torch.from_numpy(synth.make_activations(np.random.default_rng(36), (T, H))).to(dev)
    ids = torch.tensor([[0, 1], [-3, 2]], dtype=torch.int32, device=dev)
    out = torch.empty((T, k, H), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    from dismoen._lib import DMH_F_DEVICE, check, errbuf
    e = errbuf()
    check(block._lib.dmh_experts_forward(block._h, LAYER_TOY, x.data_ptr(), T, ids.data_ptr(),
                                         k, out.data_ptr(), None, DMH_F_DEVICE, e, len(e)), e)
    with pytest.raises(DismoenError) as ei:
        block.sync()
    j = json.loads(str(ei.value))
    assert j["detail"] == "expert id out of range" and j["expert_id"] == -3
    block.sync()  # the error is cleared


def test_experts_nonfinite_activation(block, toy):
    x = synth.make_activations(np.random.default_rng(37), (2, toy.hidden))
    x[1, 5] = np.inf
    with pytest.raises(DismoenError) as ei:
        block.experts_forward(x, np.array([[4], [9]], np.int32), LAYER_TOY, 2)
    j = json.loads(str(ei.value))
    assert j["error_type"] in ("EXPERT_ERROR", "SWIGLU_ERROR") and j["expert_id"] == 9


def test_shared_gate_bit_exact(block, oracle, toy, qwen):
    for L, layer, T in ((toy, LAYER_TOY, 5), (qwen, LAYER_QWEN, 3)):
        x = synth.make_activations(np.random.default_rng(38), (T, L.hidden))
        s = block.shared_gate_forward(x, T, layer)
        w = oracle.bf16_bits_to_f32(L.shgate_bf16)
        ref = oracle.shared_gate_forward(x, w, T, L.hidden, layer=layer)
        assert np.array_equal(np.asarray(s).view(np.uint32),
                              np.asarray(ref, np.float32).view(np.uint32))


def test_shared_gate_errors(block, toy):
    x = synth.make_activations(np.random.default_rng(39), (2, toy.hidden))
    with pytest.raises(DismoenError) as ei:
        block.shared_gate_forward(x, 2, LAYER_TOY, gate_mode="softmax")
    assert json.loads(str(ei.value))["error_type"] == "GATE_ERROR"
    x[0, 3] = np.nan
    with pytest.raises(DismoenError) as ei:
        block.shared_gate_forward(x, 2, LAYER_TOY)
    j = json.loads(str(ei.value))
    assert j == {"error_type": "GATE_ERROR", "detail": "non-finite shared gate logit",
                 "stage": "shared", "layer": LAYER_TOY}


@pytest.mark.parametrize("residual", [True, False])
def test_aggregate_bit_exact(block, oracle, residual):
    rng = np.random.default_rng(40)
    T, H, K = 3, 96, 4
    x = rng.standard_normal((T, H), dtype=np.float32)
    routed = rng.standard_normal((T, K * H), dtype=np.float32)
    probs = rng.random((T, K), dtype=np.float32)
    sh = rng.standard_normal((T, H), dtype=np.float32)
    g = rng.random(T, dtype=np.float32)
    if residual:
        y = block.moe_aggregate_forward(x, routed, probs, sh, g, T, H, layer_idx=2)
    else:
        y = block.combine_no_residual(routed, probs, sh, g, T, H, layer_idx=2)
    ref = oracle.moe_aggregate(x if residual else None, routed, probs, sh, g, T, H, K, layer=2)
    assert np.array_equal(np.asarray(y).view(np.uint32), np.asarray(ref, np.float32).view(np.uint32))


def test_aggregate_errors(block):
    T, H, K = 2, 32, 2
    routed = np.ones((T, K * H), np.float32)
    probs = np.full((T, K), 0.25, np.float32)
    sh = np.ones((T, H), np.float32)
    g = np.full(T, 0.5, np.float32)
    x = np.zeros((T, H), np.float32)
    x[1, 7] = np.inf
    with pytest.raises(DismoenError) as ei:
        block.moe_aggregate_forward(x, routed, probs, sh, g, T, H, layer_idx=4)
    assert json.loads(str(ei.value)) == {"error_type": "EXPERT_ERROR",
                                         "detail": "non-finite value in aggregation",
                                         "stage": "aggregation", "layer": 4}
    with pytest.raises(DismoenError) as ei:
        block.moe_aggregate_forward(np.zeros((T, H + 1), np.float32), routed, probs, sh, g, T, H)
    assert json.loads(str(ei.value))["detail"] == "length mismatch in aggregation"
    with pytest.raises(DismoenError) as ei:
        block.combine_no_residual(routed, probs, sh, g[:1], T, H)
    assert json.loads(str(ei.value))["detail"] == "sequence length mismatch"
