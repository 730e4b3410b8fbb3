"""Routing through the single-token decode kernel at the Qwen3.6 layer shape
(hidden 2048, 256 experts top-8, intermediate 512): the product kernel of
batch-1 decode (dmh_moe_forward with one token, the XCD-sliced fused launch on
MI355X).

Bar: selected expert ids, their probabilities and the shared gate bit-exact
against the oracle (router_project / router_softmax / select_topk,
src/layers/router.mojo:15-210, src/layers/topk.mojo:11-133, and
shared_gate_forward, src/layers/moe.mojo:17-102); outputs within max-abs-err
<= 1e-3 x RMS on a sample.  Covers ten thousand tokens one call each, logits
tied or a few ulp apart at the top-8 boundary (the kernel's exact-probability
fallback), and the order-revealing router rows whose logits the oracle's
closed-form tests pin (tests/test_oracle_router.py)."""
import copy
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import tol_check
from dismoen import RouterConfig, synth
from test_oracle_router import ORDER_H, order_rows

pytestmark = pytest.mark.gpu

SLOT = 70      # the module's Qwen3.6-shape layer
SLOT_MOD = 71  # the same experts under a hand-made router


@pytest.fixture(scope="module")
def qwen(block):
    L = synth.make_layer(**synth.CONFIG_QWEN36, seed=3)
    block.upload_layer(SLOT, L)
    yield L
    block.free_layer(SLOT)


def _router_f32(L):
    return synth.bf16_bits_to_f32(L.router_bf16).reshape(L.num_experts, L.hidden)


def _oracle_route(oracle, x, w, K):
    """oracle.router_forward over token chunks on host threads (the oracle
    releases the GIL), concatenated in token order."""
    T, H = x.shape
    E = w.shape[0]
    n = max(1, min(16, os.cpu_count() or 1, T))
    cuts = np.linspace(0, T, n + 1).astype(int)

    def part(i):
        a, b = int(cuts[i]), int(cuts[i + 1])
        return oracle.router_forward(x[a:b], w, b - a, H, E, K)

    with ThreadPoolExecutor(n) as ex:
        parts = list(ex.map(part, range(n)))
    return np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts])


def _with_router(L, w, shgate=None):
    M = copy.copy(L)
    M.router_bf16 = synth.f32_to_bf16_bits(w).reshape(-1)
    assert np.array_equal(synth.bf16_bits_to_f32(M.router_bf16), w.reshape(-1))
    if shgate is not None:
        M.shgate_bf16 = synth.f32_to_bf16_bits(shgate)
        assert np.array_equal(synth.bf16_bits_to_f32(M.shgate_bf16), shgate)
    return M


def _check_one(block, oracle, L, slot, x):
    y, ids, probs, shg = block.forward_arrays(slot, x, 1)
    yo, ido, po, so = oracle.moe_layer_q4(L, x, 1)
    assert np.array_equal(ids, ido), (ids, ido)
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    assert np.array_equal(shg.view(np.uint32), so.view(np.uint32))
    err, rms, ok = tol_check(y, yo)
    assert ok, (err, rms)
    return ids


def test_single_token_routing_10k_tokens_vs_oracle(block, oracle, qwen):
    """Ten thousand single-token calls (device pointers, one launch per
    token), half with bf16-valued activations (the decode workload's input)
    and half with arbitrary fp32 ones: every token's ids, probabilities and
    shared gate equal the oracle's bit for bit; outputs on a sample."""
    import torch
    T, H, K = 10000, qwen.hidden, qwen.top_k
    rng = np.random.default_rng(12)
    x = synth.make_activations(rng, (T, H))
    x[T // 2:] = rng.standard_normal((T - T // 2, H), dtype=np.float32)
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(x).to(dev)
    yd = torch.empty_like(xd)
    idd = torch.full((T, K), -1, dtype=torch.int32, device=dev)
    pd = torch.empty((T, K), dtype=torch.float32, device=dev)
    sd = torch.empty(T, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()  # written on torch's stream, read on the library's
    xb, yb, ib, pb, sb = (t.data_ptr() for t in (xd, yd, idd, pd, sd))
    for t in range(T):
        block.forward_device(SLOT, xb + 4 * H * t, 1, yb + 4 * H * t, ib + 4 * K * t,
                             pb + 4 * K * t, sb + 4 * t)
    block.sync()
    ids, probs, shg, y = (v.cpu().numpy() for v in (idd, pd, sd, yd))
    ido, po = _oracle_route(oracle, x, _router_f32(qwen), K)
    bad = np.nonzero(~np.all(ids == ido, axis=1))[0]
    assert bad.size == 0, f"{bad.size} tokens route differently, first {bad[:5].tolist()}"
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    so = oracle.shared_gate_forward(x, synth.bf16_bits_to_f32(qwen.shgate_bf16), T, H)
    assert np.array_equal(shg.view(np.uint32), so.view(np.uint32))
    # how close the 8th and 9th probabilities came (the kernel's margin test
    # sends such tokens through its exact-probability selection)
    z = x.astype(np.float64) @ _router_f32(qwen).T.astype(np.float64)
    zs = -np.sort(-z, axis=1)
    close = int(np.sum(zs[:, K - 1] - zs[:, K] < 1e-5 * np.abs(zs[:, K - 1])))
    print(f"tokens whose 8th and 9th logits are within 1e-5 relative: {close}")
    for t in list(range(0, T, 1250)) + [T - 1]:
        yo, _, _, _ = oracle.moe_layer_q4(qwen, x[t:t + 1], 1)
        err, rms, ok = tol_check(y[t], yo[0])
        assert ok, (t, err, rms)


@pytest.mark.parametrize("gap_ulp", [0, 1, 2, 3, 4, 8, 64])
def test_qwen_routing_near_ties_at_top8_boundary(block, oracle, qwen, gap_ulp):
    """Experts 7 and 8 get logits gap_ulp fp32 ulp apart at the 8th place
    (0: an exact tie, the lower id must win; a gap of one ulp can give equal
    probabilities, and then too) above 247 experts tied lower down; ids,
    probabilities and shared gate must equal the oracle's bit for bit,
    through the single-token kernel's margin test and its selection on the
    exact probabilities."""
    H, E = qwen.hidden, qwen.num_experts
    w = np.zeros((E, H), np.float32)
    w[:, 0] = 0.5
    w[:7, 0] = [2.0, 1.875, 1.75, 1.625, 1.5, 1.375, 1.25]
    w[7, 0] = w[8, 0] = 1.0
    w[7, 1] = 1.0
    w[8, 1] = 1.0 + gap_ulp * 2.0 ** -7  # z8 - z7 = gap_ulp * 2^-23 (z ~ 1)
    L = _with_router(qwen, w)
    block.upload_layer(SLOT_MOD, L)
    try:
        x = np.zeros((1, H), np.float32)
        x[0, 0], x[0, 1] = 1.0, 2.0 ** -16
        ids = _check_one(block, oracle, L, SLOT_MOD, x)
        # experts 0-6 and one of the pair (which one the probabilities decide)
        assert sorted(ids[0].tolist())[:7] == list(range(7))
        assert len({7, 8} & set(ids[0].tolist())) == 1
    finally:
        block.free_layer(SLOT_MOD)


def test_order_revealing_router_rows_through_decode_kernel(block, oracle, qwen):
    """Router rows 0-3 carry the patterns whose logits the oracle's
    closed-form tests fix (1 + 2^-23, 1 + 2^-23, 1, 1: lane chains in k
    order, the halving tree, products rounded before their add); the other
    252 logits are 0 and tie at the top-8 boundary; the shared gate row is
    row 1 scaled by -16 (logit -16 - 2^-19).  The single-token kernel must
    give the oracle's bits, and the ids the closed form: 0-3, then the lowest
    ids of the tied zeros."""
    H, E = qwen.hidden, qwen.num_experts
    x1, w4, _ = order_rows(H, tail=False)
    w = np.zeros((E, H), np.float32)
    w[:4] = w4
    L = _with_router(qwen, w, shgate=(-16.0 * w4[1]).astype(np.float32))
    block.upload_layer(SLOT_MOD, L)
    try:
        ids = _check_one(block, oracle, L, SLOT_MOD, x1[None, :])
        assert ids[0].tolist() == list(range(8))
    finally:
        block.free_layer(SLOT_MOD)


@pytest.mark.parametrize("T", [1, 64])
def test_order_revealing_rows_through_router_entry(block, oracle, T):
    """The same rows with the scalar tail (hidden 51: three 16-lane steps and
    three tail elements) through dmh_router_forward: ids and probabilities
    equal the oracle's bits, ids the closed form [0, 1, 2, 3]."""
    x1, w4, _ = order_rows(ORDER_H, tail=True)
    w = np.zeros((8, ORDER_H), np.float32)
    w[:4] = w4
    x = np.tile(x1, (T, 1))
    info = block.router_forward(x, w, T, ORDER_H, RouterConfig(8, 4))
    ido, po = oracle.router_forward(x, w, T, ORDER_H, 8, 4)
    assert np.array_equal(np.array(info.selected_experts), ido)
    assert np.array_equal(np.array(info.router_probs, np.float32).view(np.uint32),
                          po.view(np.uint32))
    assert ido[0].tolist() == [0, 1, 2, 3]
