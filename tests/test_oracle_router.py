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
