"""Pins the oracle's expert path: sigmoid/SiLU, swiglu_forward,
shared_gate_forward, the aggregation, the worker-pool partition, and the full
4-bit layer composition.

Reference known answers: tests/unit/test_moe.mojo:23-188 and
tests/unit/test_m11_w1_workerpool.mojo:23-221.  Independent check: a float64
numpy MoE layer over the same dequantised weights.
"""
import math

import numpy as np
import pytest

from dismoen import synth


def test_sigmoid_silu_known_values(oracle):
    assert abs(oracle.sigmoid_f32(0.0) - 0.5) < 1e-6
    assert oracle.sigmoid_f32(-100.0) == 0.0 and oracle.sigmoid_f32(100.0) == 1.0
    for v in (-10.0, -5.0, -1.0, 0.5, 1.0, 5.0, 10.0):
        s = oracle.sigmoid_f32(v)
        assert 0.0 < s < 1.0 and abs(s - 1 / (1 + math.exp(-v))) < 1e-7
    assert oracle.silu_f32(0.0) == 0.0
    assert abs(oracle.silu_f32(2.0) - 1.7615941) < 1e-5
    assert abs(oracle.silu_f32(-2.0) - (-0.23840584)) < 1e-5
    assert math.isnan(oracle.silu_f32(float("nan")))
    assert oracle.silu_f32(float("inf")) == float("inf") and oracle.silu_f32(float("-inf")) == 0.0
    prev = 0.0
    for i in range(-50, 51):
        s = oracle.sigmoid_f32(i * 0.5)
        assert 0.0 <= s <= 1.0 and s >= prev
        prev = s


def test_swiglu_identity_known_values(oracle):
    eye = [1.0, 0.0, 0.0, 1.0]
    out = oracle.swiglu_forward([1.0, 2.0], eye, eye, eye, 1, 2, 2)
    assert abs(out[0] - oracle.silu_f32(1.0)) < 1e-5
    assert abs(out[1] - oracle.silu_f32(2.0) * 2.0) < 1e-5
    with pytest.raises(oracle.OracleError, match="activation length mismatch"):
        oracle.swiglu_forward([1.0], eye, eye, eye, 1, 2, 2)
    with pytest.raises(oracle.OracleError, match="non-finite value in activation"):
        oracle.swiglu_forward([float("nan"), 1.0], eye, eye, eye, 1, 2, 2)


def test_shared_gate_known_values(oracle):
    s = oracle.shared_gate_forward([1.0, 2.0, -1.0, -2.0], [0.5, 0.5], 2, 2)
    assert abs(s[0] - oracle.sigmoid_f32(1.5)) < 1e-5
    assert abs(s[1] - oracle.sigmoid_f32(-1.5)) < 1e-5
    for mode in ("linear", "softmax"):
        with pytest.raises(oracle.OracleError, match="GATE_ERROR"):
            oracle.shared_gate_forward([1.0, 1.0], [0.5, 0.5], 1, 2, gate_mode=mode)


def test_aggregate_known_values(oracle):
    y = oracle.moe_aggregate([1.0, 2.0], [10.0, 20.0, 30.0, 40.0], [0.3, 0.2], [5.0, 6.0],
                             [0.5], 1, 2, 2)
    assert np.allclose(y, [12.5, 19.0], atol=1e-5)
    y0 = oracle.moe_aggregate(None, [10.0, 20.0, 30.0, 40.0], [0.3, 0.2], [5.0, 6.0], [0.5],
                              1, 2, 2)
    assert np.allclose(y0, [11.5, 17.0], atol=1e-5)


def test_partition_range_invariants(oracle):
    for total in range(0, 40):
        for n in range(1, 12):
            parts = [oracle.partition_range(total, t, n) for t in range(n)]
            if n == 1:
                assert parts == [(0, total)]
                continue
            assert parts[0][0] == 0 and parts[-1][1] == total
            for a, b in zip(parts, parts[1:]):
                assert a[1] == b[0]
            sizes = [e - s for s, e in parts]
            assert max(sizes) - min(sizes) <= 1


def test_parallel_experts_bit_exact_vs_serial(oracle):
    rng = np.random.default_rng(7)
    H, I, E, K = 64, 48, 6, 4
    wg = [(rng.standard_normal(I * H) * 0.1).astype(np.float32) for _ in range(E)]
    wu = [(rng.standard_normal(I * H) * 0.1).astype(np.float32) for _ in range(E)]
    wd = [(rng.standard_normal(H * I) * 0.1).astype(np.float32) for _ in range(E)]
    x = rng.standard_normal(H).astype(np.float32)
    sel = [4, 1, 5, 2]
    serial = np.concatenate([oracle.swiglu_forward(x, wg[e], wu[e], wd[e], 1, H, I) for e in sel])
    for nt in (1, 2, 3, 4, 7):
        pool = oracle.Pool(nt)
        for _ in range(3):
            par = pool.parallel_moe_experts(K, H, I, x, sel, wg, wu, wd)
            assert np.array_equal(par.view(np.uint32), serial.view(np.uint32))
        pool.close()


def np_moe(L, x, residual=None):
    """float64 reference of the 4-bit MoE layer over the dequantised weights."""
    from oracle import bf16_bits_to_f32, dequant_q4_bf16
    H, E, K, I, Ish, G = L.hidden, L.num_experts, L.top_k, L.inter, L.inter_sh, L.group_size

    def deq(s, p, n):
        return bf16_bits_to_f32(dequant_q4_bf16(s, p, n, G)).astype(np.float64)

    x64 = x.astype(np.float64)
    wr = synth.bf16_bits_to_f32(L.router_bf16).reshape(E, H).astype(np.float64)
    z = x64 @ wr.T
    pz = np.exp(z - z.max(1, keepdims=True))
    pz /= pz.sum(1, keepdims=True)
    out = np.zeros_like(x64)
    ids = []
    n = I * H
    for t in range(x.shape[0]):
        sel = sorted(range(E), key=lambda e: (-pz[t, e], e))[:K]
        ids.append(sel)
        for e in sel:
            gu = deq(L.gu_scales[e * 2 * n // G:(e + 1) * 2 * n // G],
                     L.gu_packed[e * n:(e + 1) * n], 2 * n).reshape(2 * I, H)
            wd = deq(L.d_scales[e * n // G:(e + 1) * n // G],
                     L.d_packed[e * n // 2:(e + 1) * n // 2], n).reshape(H, I)
            g, u = gu[:I] @ x64[t], gu[I:] @ x64[t]
            out[t] += pz[t, e] * (wd @ (g / (1 + np.exp(-g)) * u))
        ns = Ish * H
        gu = deq(L.sh_gu_scales, L.sh_gu_packed, 2 * ns).reshape(2 * Ish, H)
        wd = deq(L.sh_d_scales, L.sh_d_packed, ns).reshape(H, Ish)
        g, u = gu[:Ish] @ x64[t], gu[Ish:] @ x64[t]
        gs = 1 / (1 + np.exp(-(x64[t] @ synth.bf16_bits_to_f32(L.shgate_bf16).astype(np.float64))))
        out[t] += gs * (wd @ (g / (1 + np.exp(-g)) * u))
    if residual is not None:
        out += residual
    return out, np.array(ids)


def test_layer_composition_vs_float64(oracle):
    L = synth.make_layer(**synth.CONFIG_TOY, seed=0)
    x = synth.make_activations(np.random.default_rng(1), (5, 256))
    y, ids, probs, shg = oracle.moe_layer_q4(L, x, 5)
    ref, rids = np_moe(L, x)
    assert np.array_equal(ids, rids)
    rms = np.sqrt(np.mean(ref ** 2))
    assert np.max(np.abs(y - ref)) <= 1e-5 * rms
    yr, _, _, _ = oracle.moe_layer_q4(L, x, 5, residual=x)
    assert np.max(np.abs(yr - (ref + x))) <= 1e-5 * np.sqrt(np.mean((ref + x) ** 2))
    assert np.all(probs.sum(1) < 1.0)


def test_layer_threads_and_cache_bit_exact(oracle):
    L = synth.make_layer(**synth.CONFIG_TOY, seed=3)
    x = synth.make_activations(np.random.default_rng(2), (3, 256))
    y1, ids1, p1, s1 = oracle.moe_layer_q4(L, x, 3)
    cache = oracle.LayerCache(L)
    pool = oracle.Pool(3)
    y2, ids2, p2, s2 = oracle.moe_layer_q4(L, x, 3, pool=pool, cache=cache)
    pool.close()
    assert np.array_equal(ids1, ids2)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    assert np.array_equal(p1, p2) and np.array_equal(s1, s2)


def test_rmsnorm_and_residual(oracle):
    rng = np.random.default_rng(9)
    x = rng.standard_normal(2048).astype(np.float32)
    a = oracle.rmsnorm(x, None, 1e-6)
    ref = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
    assert np.max(np.abs(a - ref)) < 1e-5
    with pytest.raises(oracle.OracleError, match="rms_norm_eps"):
        oracle.rmsnorm(x, None, 0.0)
    with pytest.raises(oracle.OracleError, match="empty input"):
        oracle.rmsnorm(np.zeros(0, np.float32), None, 1e-6)
    r = oracle.add_residual([1.0, 2.0], [3.0, 4.0])
    assert r.tolist() == [4.0, 6.0]
    with pytest.raises(oracle.OracleError, match="non-finite value in residual"):
        oracle.add_residual([float("inf")], [1.0])


def test_stack_composition(oracle):
    """The oracle's stack is the chain of port MoE sections: per layer
    xn = rmsnorm(h, gamma_l, eps), h <- h + MoE_l(xn), with ids and
    probabilities of every layer and the output equal bit for bit, in both
    norm orders."""
    rng = np.random.default_rng(5)
    layers = [synth.make_layer(**synth.CONFIG_TOY, seed=10 + l) for l in range(3)]
    gammas = [(1.0 + 0.25 * rng.standard_normal(256)).astype(np.float32) for _ in layers]
    gammas[1] = None  # gamma = 1
    x = synth.make_activations(rng, (2, 256))
    outs = {}
    for tree in (False, True):
        out, ids, probs = oracle.moe_stack_q4(layers, x, 2, 1e-6, gammas=gammas, tree=tree)
        h = x.copy()
        for l, L in enumerate(layers):
            xn = np.stack([oracle.rmsnorm(h[t], gammas[l], 1e-6, tree=tree) for t in range(2)])
            y, lid, lp, _ = oracle.moe_layer_q4(L, xn, 2, residual=h)
            assert np.array_equal(lid, ids[l]), (tree, l)
            assert np.array_equal(lp.view(np.uint32), probs[l].view(np.uint32)), (tree, l)
            h = y
        assert np.array_equal(out.view(np.uint32), h.view(np.uint32))
        outs[tree] = out
    # the two norm orders agree within a few ulp, so the stacks within the bar
    rms = np.sqrt(np.mean((outs[False] - x).astype(np.float64) ** 2))
    assert np.max(np.abs(outs[True] - outs[False])) <= 1e-4 * rms


def test_rmsnorm_with_gamma_closed_form(oracle):
    """rmsnorm(x, gamma, eps) against float64 for both orders; and with
    integer x (every partial sum of squares exact in fp32, so both orders give
    the same sum S) bit-exactly against out = (x / denom) * gamma with
    denom = sqrt(S / n + eps), each step one correctly rounded fp32 operation
    (src/layers/rmsnorm.mojo:44-47)."""
    rng = np.random.default_rng(11)
    for n in (256, 2048, 4096):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        g = (1 + 0.5 * rng.standard_normal(n)).astype(np.float32)
        ref = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * g
        for tree in (False, True):
            a = oracle.rmsnorm(x, g, 1e-6, tree=tree)
            assert np.max(np.abs(a - ref)) <= 1e-5 * np.max(np.abs(ref))
        xi = rng.integers(-20, 21, n).astype(np.float32)
        S = np.float32(np.sum(xi.astype(np.int64) ** 2))
        eps = np.float32(1e-5)
        denom = np.sqrt(np.float32(S / np.float32(n)) + eps, dtype=np.float32)
        want = (xi / denom) * g
        for tree in (False, True):
            assert np.array_equal(oracle.rmsnorm(xi, g, float(eps), tree=tree), want)


def test_rmsnorm_order_closed_form(oracle):
    """The two summation orders differ where fp32 rounding tells them apart:
    x[0]^2 = 2^24 and every other square 1.  Added in element order each 1
    is lost (2^24 + 1 rounds to 2^24, ties to even), so the sum stays 2^24
    and denom = sqrt(2^24 / n + eps); the tree adds the ones among
    themselves first and keeps them."""
    for n in (256, 2048):
        x = np.ones(n, np.float32)
        x[0] = 4096.0
        eps = np.float32(1e-6)
        denom = np.sqrt(np.float32(np.float32(2.0 ** 24) / np.float32(n)) + eps, dtype=np.float32)
        seq = oracle.rmsnorm(x, None, float(eps))
        assert np.array_equal(seq, x / denom)
        tree = oracle.rmsnorm(x, None, float(eps), tree=True)
        assert not np.array_equal(tree, seq)
        # the tree keeps the ones: its sum is 2^24 + n - 1 within one ulp (2)
        dt = np.float32(x[1] / tree[1])
        s_tree = (np.float64(dt) ** 2 - 1e-6) * n
        assert abs(s_tree - (2.0 ** 24 + n - 1)) <= 2 * n * 2.0 ** -20 * 2.0 ** 24 / n + 4

def test_layer_cache_threads_and_pool_bit_exact(oracle):
    """The pre-dequantized fp32 cache built by several threads, the pool of
    parallel_moe_experts and dequant-per-use all give the same bits (the CPU
    baseline's four modes compute one result)."""
    L = synth.make_layer(**synth.CONFIG_TOY, seed=12)
    x = synth.make_activations(np.random.default_rng(13), (3, 256))
    ref = oracle.moe_layer_q4(L, x, 3)
    pool = oracle.Pool(4)
    try:
        for cache in (oracle.LayerCache(L, 1), oracle.LayerCache(L, 5)):
            for p in (None, pool):
                got = oracle.moe_layer_q4(L, x, 3, cache=cache, pool=p)
                for u, v in zip(ref, got):
                    assert np.array_equal(np.asarray(u).view(np.uint8), np.asarray(v).view(np.uint8))
    finally:
        pool.close()
