"""GPU parity of the MoE block for several tokens per call (small batches and
prefill: routing, grouping of the tokens by expert, grouped expert GEMMs,
combine) against the CPU oracle.

Bar as for decode: ids and probabilities bit-exact, the no-residual output
within max-abs-err <= 1e-3 x RMS(oracle output).  Every token's output depends
only on its own activation, so at prefill size the oracle is run on a sample
of the batch's tokens and compared with those rows."""
import numpy as np
import pytest

from conftest import tol_check
from dismoen import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qwen(block):
    L = synth.make_layer(**synth.CONFIG_QWEN36, seed=11)
    block.upload_layer(5, L)
    return L


def _check(block, oracle, L, layer, x, residual=None, pool=None):
    T = x.shape[0]
    y, ids, probs, shg = block.forward_arrays(layer, x, T, residual=residual)
    yo, ido, po, so = oracle.moe_layer_q4(L, x, T, residual=residual, pool=pool)
    assert np.array_equal(ids, ido)
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    assert np.array_equal(shg.view(np.uint32), so.view(np.uint32))
    if residual is None:
        err, rms, ok = tol_check(y, yo)
    else:
        err, rms, ok = tol_check(y - residual, yo - residual)
    assert ok, (err, rms)


@pytest.mark.parametrize("cfg", ["toy", "qwen"])
@pytest.mark.parametrize("gap_ulp", [0, 1, 3, 64, 4096])
def test_batch_routing_near_ties_at_topk_boundary(block, oracle, cfg, gap_ulp):
    """The K-th and (K+1)-th experts get logits gap_ulp fp32 ulp apart (0 =
    exact tie, lowest id wins) in every token of a 3-token call: the batch
    front end's top-k has a fast reduction on truncated probability keys and
    must fall back to exact rounds when the truncation could reorder them.
    ids and probabilities bit-exact against the oracle."""
    c = synth.CONFIG_TOY if cfg == "toy" else synth.CONFIG_QWEN36
    L = synth.make_layer(**c, seed=31)
    H, E, K = L.hidden, L.num_experts, L.top_k
    w = np.zeros((E, H), np.float32)
    w[:, 0] = 0.5
    for i in range(K - 1):
        w[i, 0] = 2.0 - i * 0.125
    w[K - 1, 0], w[K, 0] = 1.0, 1.0
    w[K - 1, 1] = 1.0
    w[K, 1] = 1.0 + gap_ulp * 2.0 ** -7  # z_K - z_{K-1} = gap_ulp * 2^-23
    L.router_bf16 = synth.f32_to_bf16_bits(w).reshape(-1)
    assert np.array_equal(synth.bf16_bits_to_f32(L.router_bf16).reshape(E, H)[:, :2], w[:, :2])
    layer = 60 + (gap_ulp % 7) + (10 if cfg == "qwen" else 0)
    block.upload_layer(layer, L)
    x = np.zeros((3, H), np.float32)
    x[:, 0], x[:, 1] = 1.0, 2.0 ** -16
    x[1, 2] = 0.25  # a second row pattern: feature 2 adds nothing (w[:, 2] = 0)
    y, ids, probs, shg = block.forward_arrays(layer, x, 3)
    yo, ido, po, so = oracle.moe_layer_q4(L, x, 3)
    assert np.array_equal(ids, ido), (ids, ido)
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    err, rms, ok = tol_check(y, yo)
    assert ok, (err, rms)
    block.free_layer(layer)


@pytest.mark.parametrize("T", [2, 3, 5, 8, 32])
def test_small_batch_vs_oracle(block, oracle, qwen, T):
    x = synth.make_activations(np.random.default_rng(200 + T), (T, 2048))
    pool = oracle.Pool(8)
    try:
        _check(block, oracle, qwen, 5, x, pool=pool)
        if T == 8:
            _check(block, oracle, qwen, 5, x, residual=x, pool=pool)
    finally:
        pool.close()


@pytest.mark.parametrize("T", [6, 48])
def test_batch_matches_single_token_calls(block, qwen, T):
    """The several-token launch (T = 6) or the grouped path (T = 48) and the
    single-token decode kernel agree token by token: ids and probabilities
    bit for bit, outputs within the bar."""
    x = synth.make_activations(np.random.default_rng(300), (T, 2048))
    y, ids, probs, shg = block.forward_arrays(5, x, T)
    for t in range(0, T, 5 if T > 8 else 1):
        y1, ids1, p1, s1 = block.forward_arrays(5, x[t:t + 1], 1)
        assert np.array_equal(ids[t], ids1[0])
        assert np.array_equal(probs[t].view(np.uint32), p1[0].view(np.uint32))
        err, rms, ok = tol_check(y1[0], y[t])
        assert ok, (t, err, rms)


def test_fp32_activations_need_lo_parts(block, oracle, qwen):
    """Activations that are not bf16 values exercise the bf16 lo pass."""
    rng = np.random.default_rng(301)
    x = rng.standard_normal((12, 2048)).astype(np.float32)
    _check(block, oracle, qwen, 5, x)


def test_prefill_2048_tokens_sampled_vs_oracle(block, oracle, qwen):
    T = 2048
    x = synth.make_activations(np.random.default_rng(302), (T, 2048))
    y, ids, probs, shg = block.forward_arrays(5, x, T)
    sample = np.random.default_rng(303).choice(T, 24, replace=False)
    pool = oracle.Pool(8)
    try:
        yo, ido, po, so = oracle.moe_layer_q4(qwen, x[sample], len(sample), pool=pool)
    finally:
        pool.close()
    assert np.array_equal(ids[sample], ido)
    assert np.array_equal(probs[sample].view(np.uint32), po.view(np.uint32))
    for i, t in enumerate(sample):
        err, rms, ok = tol_check(y[t], yo[i])
        assert ok, (t, err, rms)
    # every token used exactly K distinct experts
    assert all(len(set(r)) == 8 for r in ids.tolist())


def test_batch_deterministic(block, qwen):
    x = synth.make_activations(np.random.default_rng(304), (200, 2048))
    a = block.forward_arrays(5, x, 200)
    b = block.forward_arrays(5, x, 200)
    for u, v in zip(a, b):
        assert np.array_equal(np.asarray(u).view(np.uint8), np.asarray(v).view(np.uint8))


def test_batch_nonfinite_activation_error_matches_oracle(block, oracle, qwen):
    from dismoen import DismoenError
    x = synth.make_activations(np.random.default_rng(305), (5, 2048))
    x[3, 17] = np.nan
    with pytest.raises(DismoenError) as e_gpu:
        block.forward_arrays(5, x, 5)
    with pytest.raises(oracle.OracleError) as e_cpu:
        oracle.moe_layer_q4(qwen, x, 5, layer=5)
    assert str(e_gpu.value) == str(e_cpu.value)


def test_batch_overflow_error_matches_oracle(block, oracle):
    """An overflowing activation in one token of a batch: the first failing
    check (in the reference's order of tokens, phases and rows) gives the same
    error text as the oracle."""
    from dismoen import DismoenError
    L = synth.make_layer(**synth.CONFIG_TOY, seed=7)
    block.upload_layer(6, L)
    x = synth.make_activations(np.random.default_rng(306), (4, 256))
    x[2] *= np.float32(3e37)
    msgs = []
    for call in (lambda: block.forward_arrays(6, x, 4),
                 lambda: oracle.moe_layer_q4(L, x, 4, layer=6)):
        with pytest.raises((DismoenError, oracle.OracleError)) as e:
            call()
        msgs.append(str(e.value))
    assert msgs[0] == msgs[1], msgs


def test_many_tokens_matrix_core_router_vs_oracle(block, oracle, qwen):
    """From 64 tokens on, bf16 activations are routed on the matrix cores
    (one fp32 MFMA step per chain element): every token's ids and
    probabilities bit-exact."""
    T = 96
    x = synth.make_activations(np.random.default_rng(310), (T, 2048))
    pool = oracle.Pool(8)
    try:
        _check(block, oracle, qwen, 5, x, pool=pool)
    finally:
        pool.close()


def test_many_tokens_fp32_activations_vs_oracle(block, oracle, qwen):
    """Activations that are not bf16 values take the lane-chain router."""
    T = 80
    x = np.random.default_rng(311).standard_normal((T, 2048)).astype(np.float32)
    pool = oracle.Pool(8)
    try:
        _check(block, oracle, qwen, 5, x, pool=pool)
    finally:
        pool.close()


def test_fp32_prefill_301_tokens_vs_oracle(block, oracle, qwen):
    """A 301-token chunk of activations that are not bf16 values (the
    lane-chain router, hi and lo passes, the need-lo flag set by thousands of
    waves): sampled tokens and the last five with ids, probabilities and
    shared gates bit-exact."""
    T = 301
    x = np.random.default_rng(312).standard_normal((T, 2048)).astype(np.float32)
    y, ids, probs, shg = block.forward_arrays(5, x, T)
    sample = np.concatenate([np.random.default_rng(313).choice(296, 12, replace=False),
                             np.arange(296, T)])
    pool = oracle.Pool(8)
    try:
        yo, ido, po, so = oracle.moe_layer_q4(qwen, x[sample], len(sample), pool=pool)
    finally:
        pool.close()
    assert np.array_equal(ids[sample], ido)
    assert np.array_equal(probs[sample].view(np.uint32), po.view(np.uint32))
    assert np.array_equal(shg[sample].view(np.uint32), so.view(np.uint32))
    for i, t in enumerate(sample):
        err, rms, ok = tol_check(y[t], yo[i])
        assert ok, (t, err, rms)


@pytest.mark.parametrize("slot,shape", [
    (20, (256, 16, 4, 128, 128)),    # 2 words per chain; one live wave in the last row block
    (21, (512, 40, 4, 128, 128)),    # 4 words; the last block's fourth wave has no rows
    (22, (1024, 64, 6, 256, 256)),   # 8 words
    (23, (384, 24, 4, 128, 128)),    # 3 words: the one-token-at-a-time lane-chain kernel
])
@pytest.mark.parametrize("T", [9, 37])
def test_lane_chain_router_hidden_sizes_vs_oracle(block, oracle, slot, shape, T):
    """Activations that are not bf16 values at several hidden sizes: the
    register-resident lane-chain router (4 tokens a pass, a ragged last
    pass) and its one-token fallback give bit-exact ids, probabilities and
    shared gates."""
    H, E, K, I, Ish = shape
    L = synth.make_layer(H, E, K, I, Ish, seed=slot)
    block.upload_layer(slot, L)
    x = np.random.default_rng(400 + slot + T).standard_normal((T, H)).astype(np.float32)
    _check(block, oracle, L, slot, x)


def test_many_tokens_toy_layer_vs_oracle(block, oracle):
    """Fewer experts than one router workgroup covers (16 < 64), hidden 256."""
    L = synth.make_layer(**synth.CONFIG_TOY, seed=8)
    block.upload_layer(7, L)
    x = synth.make_activations(np.random.default_rng(312), (70, 256))
    _check(block, oracle, L, 7, x)
    _check(block, oracle, L, 7, x, residual=x)


def test_prefill_2048_zipf_skew_vs_oracle(block, oracle):
    """The Zipf(1.1)-skewed 2048-token prefill: a router bias folded into
    router column 0 with activation feature 0 = 1.0 (synth.with_router_bias),
    so hot experts get hundreds of tokens and their full 128-token units run.
    Every token's ids and probabilities are compared with the oracle's
    router_forward (topk.mojo:79-96, lowest id on ties); outputs on a sample
    holding tokens of the hottest expert and of experts with 1-5 tokens."""
    E, H, K, T = 256, 2048, 8, 2048
    L = synth.with_router_bias(synth.make_layer(**synth.CONFIG_QWEN36, seed=13),
                               synth.zipf_router_bias(E, 1.1, seed=7))
    block.upload_layer(8, L)
    x = synth.bias_feature(synth.make_activations(np.random.default_rng(320), (T, H)))
    y, ids, probs, shg = block.forward_arrays(8, x, T)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    hot = int(np.argmax(counts))
    # the routed full-unit path of the grouped kernels (more than one
    # 128-token unit for a routed expert) is exercised
    assert counts[hot] > 128, counts[hot]
    w = synth.bf16_bits_to_f32(L.router_bf16).reshape(E, H)
    ido, po = oracle.router_forward(x, w, T, H, E, K)
    assert np.array_equal(ids, ido)
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    rng = np.random.default_rng(321)
    hot_tokens = np.nonzero((ids == hot).any(axis=1))[0]
    sample = list(rng.choice(hot_tokens, 8, replace=False))
    cold = [e for e in range(E) if 1 <= counts[e] <= 5]
    assert cold, "no expert with 1-5 tokens"
    for e in cold[:16]:
        t = int(np.nonzero((ids == e).any(axis=1))[0][0])
        if t not in sample:
            sample.append(t)
    sample = np.array(sample)
    pool = oracle.Pool(8)
    try:
        yo, ido2, po2, so = oracle.moe_layer_q4(L, x[sample], len(sample), pool=pool)
    finally:
        pool.close()
    assert np.array_equal(ids[sample], ido2)
    assert np.array_equal(shg[sample].view(np.uint32), so.view(np.uint32))
    for i, t in enumerate(sample):
        err, rms, ok = tol_check(y[t], yo[i])
        assert ok, (int(t), err, rms)
    block.free_layer(8)
