"""GPU parity of the unit entry points through the C ABI:
dmh_dequant_q4_bf16 (bit-exact) and dmh_router_forward (ids and probs bit-exact)
against the CPU oracle."""
import json

import numpy as np
import pytest

from dismoen import DismoenError, RouterConfig

pytestmark = pytest.mark.gpu


def test_dequant_225_pairs(block, oracle):
    from test_oracle_dequant import all_225_pairs
    scales, packed, _, _ = all_225_pairs()
    got = block.dequant_kernel_simd(scales, packed, 512, 128)
    assert np.array_equal(got, oracle.dequant_q4_bf16(scales, packed, 512, 128))


def test_dequant_gm6k_fixture(block, oracle):
    from test_oracle_dequant import load_gm6k
    sc, pk, gd = load_gm6k()
    assert np.array_equal(block.dequant_kernel_simd(sc, pk, 131072, 128), gd)
    corrupt = pk.copy()
    corrupt[42] = (corrupt[42] & 0x0F) | 0x80
    with pytest.raises(DismoenError, match="reserved nibble"):
        block.dequant_kernel_simd(sc, corrupt, 131072, 128)


@pytest.mark.parametrize("G", [32, 64, 128, 256])
def test_dequant_random_all_groups(block, oracle, G):
    rng = np.random.default_rng(G)
    n = G * 777
    sc = rng.integers(1, 0x7C00, n // G, dtype=np.uint16)
    v = rng.integers(0, 225, n // 2)
    pk = (((v // 15 - 7) & 0xF) << 4 | ((v % 15 - 7) & 0xF)).astype(np.uint8)
    assert np.array_equal(block.dequant_kernel_simd(sc, pk, n, G),
                          oracle.dequant_q4_bf16(sc, pk, n, G))


def test_dequant_errors_match_oracle(block, oracle):
    pk = np.zeros(64, np.uint8)
    cases = [(np.array([0x7E00], np.uint16), pk, 128, 128),
             (np.array([0x0000], np.uint16), pk, 128, 128),
             (np.array([0x3C00, 0x7C00, 0x8000], np.uint16), np.zeros(48, np.uint8), 96, 32),
             (np.array([0x3C00], np.uint16), np.where(np.arange(64) == 7, 0x80, 0).astype(np.uint8),
              128, 128),
             (np.array([0x3C00], np.uint16), pk, 128, 48),
             (np.array([0x3C00], np.uint16), pk, 100, 32)]
    for sc, p, n, G in cases:
        with pytest.raises(oracle.OracleError) as eo:
            oracle.dequant_q4_bf16(sc, p, n, G)
        with pytest.raises(DismoenError) as eg:
            block.dequant_kernel_simd(sc, p, n, G)
        assert str(eg.value) == str(eo.value)


def test_router_known_values(block):
    info = block.router_forward([1.0, 2.0, 3.0, 4.0], [1.0, 0.0, 0.0, 1.0, 1.0, 1.0], 2, 2,
                                RouterConfig(3, 2))
    assert info.selected_experts == [[2, 1], [2, 1]]
    with pytest.raises(DismoenError) as e:
        block.router_forward([1.0, 2.0], [1.0, 2.0], 1, 2, RouterConfig(1, 1, True))
    assert json.loads(str(e.value))["error_type"] == "ROUTER_ERROR"


@pytest.mark.parametrize("T,H,E,K,scale", [(16, 256, 16, 4, 0.02), (1000, 2048, 256, 8, 0.02),
                                           (64, 100, 60, 4, 0.05), (32, 2048, 256, 8, 0.0),
                                           # rows beyond the LDS form: H > 2048, H % 4 != 0
                                           (8, 4096, 40, 4, 0.02), (8, 2050, 24, 4, 0.02)])
def test_router_bit_exact_vs_oracle(block, oracle, T, H, E, K, scale):
    rng = np.random.default_rng(T + H)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.standard_normal((E, H)) * scale).astype(np.float32)
    if scale == 0.0:  # every logit ties: lowest ids win
        w[:] = 0.0
    info = block.router_forward(x, w, T, H, RouterConfig(E, K))
    ids_o, p_o = oracle.router_forward(x, w, T, H, E, K)
    assert np.array_equal(np.array(info.selected_experts), ids_o)
    assert np.array_equal(np.array(info.router_probs, np.float32).view(np.uint32),
                          p_o.view(np.uint32))


def test_router_bit_exact_bf16_inputs_10k_tokens(block, oracle):
    from dismoen import synth
    rng = np.random.default_rng(11)
    T, H, E, K = 10000, 2048, 256, 8
    x = synth.make_activations(rng, (T, H))
    w = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(
        (rng.standard_normal((E, H)) * 0.02).astype(np.float32)))
    info = block.router_forward(x, w, T, H, RouterConfig(E, K))
    ids_o, p_o = oracle.router_forward(x, w, T, H, E, K)
    assert np.array_equal(np.array(info.selected_experts), ids_o)
    assert np.array_equal(np.array(info.router_probs, np.float32), p_o)


def test_router_errors_match_oracle(block, oracle):
    x = np.ones((2, 32), np.float32)
    w = np.ones((4, 32), np.float32) * 0.1
    xb = x.copy(); xb[1, 3] = np.nan
    wb = w.copy(); wb[2, 5] = np.inf
    for xx, ww in ((xb, w), (x, wb), (xb, wb)):
        with pytest.raises(oracle.OracleError) as eo:
            oracle.router_forward(xx, ww, 2, 32, 4, 2)
        with pytest.raises(DismoenError) as eg:
            block.router_forward(xx, ww, 2, 32, RouterConfig(4, 2))
        assert str(eg.value) == str(eo.value)
