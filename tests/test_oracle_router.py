"""Pins the oracle's router: router_project / router_softmax / select_topk /
router_forward (src/layers/router.mojo, topk.mojo, router_types.mojo).

Reference known answers: tests/unit/test_router_ops.mojo:75-183 and
tests/unit/test_router_topk.mojo:26-100.  Independent checks: float64 dot
products and softmax, a brute-force (-p, id) sort, and float64 exp for or_expf.
"""
import json
import math

import numpy as np
import pytest


def test_expf_accuracy_and_monotone(oracle):
    xs = np.concatenate([np.linspace(-103.9, 88.7, 200001, dtype=np.float32),
                         -np.abs(np.random.default_rng(0).standard_normal(50000) * 8)
                         .astype(np.float32)])
    got = np.array([oracle.expf(float(x)) for x in xs], dtype=np.float64)
    ref = np.exp(xs.astype(np.float64))
    normal = ref > 1.2e-38
    ulp = np.spacing(ref[normal].astype(np.float32)).astype(np.float64)
    err_ulp = np.abs(got[normal] - ref[normal]) / ulp
    assert err_ulp.max() <= 2.0, err_ulp.max()
    # consecutive floats just below 0 (the softmax / sigmoid argument range)
    u = np.arange(0x80000000, 0x80000000 + 300000, dtype=np.uint32)
    for start in (np.float32(-0.0), np.float32(-0.69), np.float32(-5.3), np.float32(-20.1)):
        b = np.array([start], np.float32).view(np.uint32)[0]
        seq = (np.arange(300000, dtype=np.uint32) + b).view(np.float32)
        e = np.array([oracle.expf(float(v)) for v in seq[::7]])
        assert np.all(np.diff(e) <= 0)  # x decreasing -> exp non-increasing
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(-200.0) == 0.0
    assert math.isinf(oracle.expf(100.0))
    del u


def test_router_project_known_values(oracle):
    x = [1.0, 2.0, 3.0, 4.0]
    w = [1.0, 0.0, 0.0, 1.0, 1.0, 1.0]
    z = oracle.router_project(x, w, 2, 2, 3)
    assert np.allclose(z, [1, 2, 3, 3, 4, 7], atol=1e-5)


def test_router_project_errors(oracle):
    with pytest.raises(oracle.OracleError, match="activation length mismatch"):
        oracle.router_project([1.0], [1, 2, 3, 4], 1, 2, 2)
    with pytest.raises(oracle.OracleError, match="weight length mismatch"):
        oracle.router_project([1.0, 2.0], [1, 2], 1, 2, 2)
    with pytest.raises(oracle.OracleError, match="dimensions must be"):
        oracle.router_project([1.0, 2.0], [1, 2, 3, 4], 0, 2, 2)
    with pytest.raises(oracle.OracleError, match="non-finite value in activation"):
        oracle.router_project([float("nan"), 1.0], [1, 0, 0, 1], 1, 2, 2)
    with pytest.raises(oracle.OracleError, match="non-finite value in router weight"):
        oracle.router_project([1.0, 2.0], [1, float("nan"), 0, 1], 1, 2, 2)


def test_softmax_shift_invariance_and_sum(oracle):
    p1 = oracle.router_softmax([1.0, 2.0, 5.0, 3.0], 1, 4)
    p2 = oracle.router_softmax([1001.0, 1002.0, 1005.0, 1003.0], 1, 4)
    assert np.allclose(p1, p2, atol=1e-5)
    p = oracle.router_softmax([-2.0, 0.5, 3.0, 1.2, -0.4], 1, 5)
    assert np.all(p > 0) and abs(float(p.sum()) - 1.0) < 1e-5
    with pytest.raises(oracle.OracleError, match="non-finite max logit"):
        oracle.router_softmax([float("inf"), 1.0, 2.0], 1, 3)
    with pytest.raises(oracle.OracleError, match="non-finite exp"):
        oracle.router_softmax([1.0, float("nan"), 2.0], 1, 3)


def test_softmax_matches_float64(oracle):
    rng = np.random.default_rng(1)
    z = rng.standard_normal((50, 256)).astype(np.float32) * 3
    p = oracle.router_softmax(z, 50, 256).reshape(50, 256)
    ref = np.exp(z - z.max(1, keepdims=True))
    ref = ref / ref.sum(1, keepdims=True)
    assert np.max(np.abs(p - ref) / ref) < 3e-6


def test_topk_known_values(oracle):
    ids, vals = oracle.select_topk([0.05, 0.40, 0.10, 0.30, 0.15], 1, 5, 3)
    assert ids.tolist() == [[1, 3, 4]]
    assert np.allclose(vals, [[0.40, 0.30, 0.15]], atol=1e-5)
    ids, vals = oracle.select_topk([1 / 60] * 60, 1, 60, 4)
    assert abs(float(vals.sum()) - 4 / 60) < 1e-5 and ids.tolist() == [[0, 1, 2, 3]]
    with pytest.raises(oracle.OracleError, match="norm_topk_prob=true"):
        oracle.select_topk([0.25, 0.25, 0.25, 0.25, 0.0], 1, 5, 2, norm_topk_prob=True)
    with pytest.raises(oracle.OracleError, match="renormalization leak"):
        oracle.select_topk([0.6, 0.4, 0.05, 0.05], 1, 4, 2)
    with pytest.raises(oracle.OracleError, match="top_k cannot exceed"):
        oracle.select_topk([0.5, 0.5], 1, 2, 3)
    with pytest.raises(oracle.OracleError, match="exceeds 1.0"):
        oracle.select_topk([0.7, 0.7, 0.1], 1, 3, 2)


def test_topk_brute_force_with_ties(oracle):
    rng = np.random.default_rng(2)
    for _ in range(300):
        E = int(rng.integers(2, 40))
        K = int(rng.integers(1, E + 1))
        p = rng.choice(np.array([0.01, 0.02, 0.03, 0.005], np.float32), E)  # many ties
        ids, vals = oracle.select_topk(p, 1, E, K)
        ref = sorted(range(E), key=lambda e: (-float(p[e]), e))[:K]
        assert ids[0].tolist() == ref
        assert np.array_equal(vals[0], p[ref])


def test_router_forward_matches_float64(oracle):
    rng = np.random.default_rng(4)
    T, H, E, K = 64, 2048, 256, 8
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    ids, vals = oracle.router_forward(x, w, T, H, E, K)
    z = oracle.router_project(x, w, T, H, E).reshape(T, E)
    z64 = x.astype(np.float64) @ w.T.astype(np.float64)
    assert np.max(np.abs(z - z64)) < 1e-4
    p64 = np.exp(z64 - z64.max(1, keepdims=True))
    p64 /= p64.sum(1, keepdims=True)
    for t in range(T):
        ref = np.argsort(-p64[t], kind="stable")[:K]
        gap_ok = np.sort(p64[t])[::-1]
        if gap_ok[K - 1] - gap_ok[K] > 1e-6:  # skip near-ties float64 cannot decide
            assert sorted(ids[t].tolist()) == sorted(ref.tolist())
        assert np.allclose(vals[t], p64[t][ids[t]], rtol=2e-5)


def test_router_config_validation(oracle):
    with pytest.raises(oracle.OracleError, match="num_experts must be"):
        oracle.router_forward([1.0], [1.0], 1, 1, 0, 1)
    with pytest.raises(oracle.OracleError, match="cannot exceed num_experts"):
        oracle.router_forward([1.0], [1.0], 1, 1, 1, 2)
    with pytest.raises(oracle.OracleError) as e:
        oracle.router_forward([1.0], [1.0], 1, 1, 1, 1, norm_topk_prob=True)
    assert json.loads(str(e.value))["error_type"] == "ROUTER_ERROR"


# ---- arithmetic order of router_project and router_softmax ------------------
# The reference forms a logit as 16 SIMD lanes, lane l summing the products
# k = l, l+16, ... one after another (router.mojo:84-90), then
# SIMD.reduce_add (:91), then the scalar tail k = 16*floor(H/16) .. H-1
# added to the reduced value in order (:92-96); every product is rounded
# before its add (no contraction).  reduce_add is read as the halving tree
# lane l += lane l+w for w = 8, 4, 2, 1.  router_softmax sums exp(z - max) in
# expert order (:160-170) and multiplies each numerator by 1/S (:180-183).
#
# The patterns below make each step observable in fp32 bits: 1 + 2^-24 is a
# tie that rounds to 1 (even), while 2^-24 + 2^-24 = 2^-23 and 1 + 2^-23 is
# exact, so a logit is 1 + 2^-23 exactly when the two small products meet
# each other before they meet the 1.  Every weight is bf16-representable, so
# the same rows also drive the HIP router.
ORDER_H = 51          # three 16-lane steps and a three-element tail
ORDER_X_FMA = 0x3EFE03FB  # x[19]: x[19] * (1 + 2^-7) = 0.5 + 2^-24 + 0.48 * 2^-24 exactly


def order_rows(H=ORDER_H, tail=True):
    """x [H] and router rows w [4][H]; the logits the reference forms, each
    derived in the comment of its row."""
    t = 2.0 ** -24
    x = np.ones(H, np.float32)
    x[3] = 0.5
    x[19] = np.array([ORDER_X_FMA], np.uint32).view(np.float32)[0]
    w = np.zeros((4, H), np.float32)
    # row 0, one lane's chain in k order: lane 0 adds p0 = 2^-24, p16 = 2^-24,
    # p32 = 1: (2^-24 + 2^-24) + 1 = 1 + 2^-23.  (k order reversed: 1.)
    w[0, 0], w[0, 16], w[0, 32] = t, t, 1.0
    # row 1, the halving tree: lanes 0, 7, 15 hold 1, 2^-24, 2^-24; lane 7
    # meets lane 15 at w = 8 (2^-23), reaches lane 1 at w = 1 and then lane 0:
    # 1 + 2^-23.  (Lanes summed in order, or adjacent pairs: 1.)
    w[1, 0], w[1, 7], w[1, 15] = 1.0, t, t
    # row 2, the tail after the tree: the tree gives 1 (lane 1), then
    # 1 + p48 = 1 + 2^-24 -> 1, + p49 = 0, + p50 -> 1.  (Tail summed first, or
    # folded into lanes 0 and 2 before the tree: 1 + 2^-23.)
    if tail:
        w[2, 1], w[2, 48], w[2, 50] = 1.0, t, t
    else:
        w[2, 1] = 1.0
    # row 3, rounded products: lane 3 adds p3 = 0.5, then p19 whose exact
    # value 0.5 + 1.48 * 2^-24 rounds to 0.5 + 2^-24; 0.5 + (0.5 + 2^-24) =
    # 1 + 2^-24 -> 1.  (A fused multiply-add keeps 1.48 * 2^-24: 1 + 2^-23.)
    w[3, 3], w[3, 19] = 1.0, np.float32(1.0 + 2.0 ** -7)
    z = np.array([1 + 2.0 ** -23, 1 + 2.0 ** -23, 1.0, 1.0], np.float32)
    return x, w, z


def _add(a, b):
    return np.float32(np.float32(a) + np.float32(b))


def _mutant_dot(x, w, chain="strided", tree="halving", tail="after", fma=False):
    """router_project's dot product read in one of the plausible wrong ways."""
    n = len(x)
    m = n // 16 * 16
    if fma:
        def mac(acc, k):  # one rounding of the exact acc + x*w (exact in float64 here)
            return np.float32(float(acc) + float(x[k]) * float(w[k]))
    else:
        def mac(acc, k):
            return _add(acc, np.float32(x[k] * w[k]))
    acc = [np.float32(0)] * 16
    if chain == "strided":
        for k in range(0, m, 16):
            for l in range(16):
                acc[l] = mac(acc[l], k + l)
    elif chain == "reversed":
        for k in range(m - 16, -1, -16):
            for l in range(16):
                acc[l] = mac(acc[l], k + l)
    elif chain == "contiguous":
        c = m // 16
        for l in range(16):
            for i in range(c):
                acc[l] = mac(acc[l], l * c + i)
    if tail == "lanes":
        for k in range(m, n):
            acc[k % 16] = mac(acc[k % 16], k)
    if tree == "halving":
        a = list(acc)
        for wd in (8, 4, 2, 1):
            for l in range(wd):
                a[l] = _add(a[l], a[l + wd])
        s = a[0]
    elif tree == "sequential":
        s = np.float32(0)
        for v in acc:
            s = _add(s, v)
    elif tree == "adjacent":
        a = list(acc)
        while len(a) > 1:
            a = [_add(a[2 * i], a[2 * i + 1]) for i in range(len(a) // 2)]
        s = a[0]
    if tail == "after":
        for k in range(m, n):
            s = mac(s, k)
    elif tail in ("first", "summed"):
        t = np.float32(0)
        for k in range(m, n):
            t = mac(t, k)
        s = _add(t, s) if tail == "first" else _add(s, t)
    return s


MUTANTS = {
    "k order reversed": dict(chain="reversed"),
    "contiguous lane chunks": dict(chain="contiguous"),
    "lanes summed in order": dict(tree="sequential"),
    "adjacent-pair tree": dict(tree="adjacent"),
    "tail folded into lanes": dict(tail="lanes"),
    "tail before the tree": dict(tail="first"),
    "tail summed, then added": dict(tail="summed"),
    "fused multiply-add": dict(fma=True),
}


def test_router_project_order_closed_form(oracle):
    """The oracle's logits equal the closed forms derived above, and every
    plausible misreading of the reference's order gives different bits on at
    least one row."""
    x, w, z = order_rows()
    got = oracle.router_project(x, w.reshape(-1), 1, ORDER_H, 4)
    assert np.array_equal(got.view(np.uint32), z.view(np.uint32)), got
    # the derivations hold for the reading the oracle follows ...
    ref = np.array([_mutant_dot(x, w[e]) for e in range(4)], np.float32)
    assert np.array_equal(ref.view(np.uint32), z.view(np.uint32))
    # ... and each wrong reading fails one of them
    for name, kw in MUTANTS.items():
        mz = np.array([_mutant_dot(x, w[e], **kw) for e in range(4)], np.float32)
        assert not np.array_equal(mz.view(np.uint32), z.view(np.uint32)), name
    # a sequential sum over all of k: rows 0, 2 and 3 agree with it, row 1 does not
    seq = np.float32(0)
    for k in range(ORDER_H):
        seq = _add(seq, np.float32(x[k] * w[1, k]))
    assert seq != z[1]


def test_shared_gate_logit_order_closed_form(oracle):
    """shared_gate_forward reduces its logit in the same order
    (src/layers/moe.mojo:70-84).  Row 1 scaled by -16 gives the logit
    -16 - 2^-19 (the two -2^-20 products meet first); in lane order it would
    be -16, and sigmoid separates the two by about 2^-19 relative."""
    x, w, _ = order_rows()
    g = oracle.shared_gate_forward(x, -16.0 * w[1], 1, ORDER_H)
    want = oracle.sigmoid_f32(float(np.float32(-16.0 - 2.0 ** -19)))
    wrong = oracle.sigmoid_f32(-16.0)
    assert want != wrong
    assert g[0] == np.float32(want)


def test_router_softmax_sequential_sum_closed_form(oracle):
    """S is summed in expert order: with the maximum first and 63 numerators
    e = exp(-18) < 2^-24 each, every add after the first rounds back to 1, so
    S = 1, p_0 = 1 and p_i = e exactly.  A pairwise or reversed sum gives
    S = 1 + 63e ~ 1 + 8 ulp, and p_0 < 1."""
    e = oracle.expf(-18.0)
    assert 0.0 < e < 2.0 ** -24
    z = np.full(64, -18.0, np.float32)
    z[0] = 0.0
    p = oracle.router_softmax(z, 1, 64)
    assert p[0] == 1.0
    assert np.all(p[1:] == np.float32(e))
    # the misreadings
    ev = np.array([1.0] + [e] * 63, np.float32)
    pair = ev.copy()
    while pair.size > 1:
        pair = (pair[0::2] + pair[1::2]).astype(np.float32)
    rev = np.float32(0)
    for v in ev[::-1]:
        rev = _add(rev, v)
    assert pair[0] != 1.0 and rev != 1.0


def test_router_softmax_multiplies_by_reciprocal(oracle):
    """p = e * (1/S), one rounding of the product of two floats, not e / S:
    three maxima and numerators below half an ulp of 3 give S = 3 exactly,
    1/S = fl(1/3) = 0x3EAAAAAB, and every p_i = fl(e_i * 0x3EAAAAAB) (the
    product of two floats is exact in float64, so rounding it once to float32
    is the closed form).  At least one e_i / 3 rounds differently."""
    zs = np.linspace(-18.0, -19.0, 61).astype(np.float32)
    z = np.concatenate([np.zeros(3, np.float32), zs])
    p = oracle.router_softmax(z, 1, z.size)
    inv = np.array([0x3EAAAAAB], np.uint32).view(np.float32)[0]
    assert np.float32(1.0) / np.float32(3.0) == inv
    ev = np.array([oracle.expf(float(v)) for v in zs], np.float32)
    assert np.all(ev < 2.0 ** -23)  # below half an ulp of 3: S stays 3
    want = (ev.astype(np.float64) * np.float64(inv)).astype(np.float32)
    assert np.all(p[:3] == inv)
    assert np.array_equal(p[3:].view(np.uint32), want.view(np.uint32))
    div = (ev / np.float32(3.0)).astype(np.float32)
    assert np.any(div.view(np.uint32) != want.view(np.uint32))
