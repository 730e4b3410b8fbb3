"""Host-side logic of the dismoen package (no GPU): RouterConfig validation,
RoutingInfo JSON, and the synthetic generator's invariants."""
import json

import numpy as np
import pytest

from dismoen import DismoenError, RouterConfig, RoutingInfo, synth


def test_router_config_validate_messages():
    RouterConfig(256, 8, False).validate()
    for cfg, kind, detail in ((RouterConfig(0, 1), "CONFIG_ERROR", "num_experts must be positive"),
                              (RouterConfig(4, 0), "CONFIG_ERROR",
                               "num_experts_per_tok must be positive"),
                              (RouterConfig(4, 5), "CONFIG_ERROR",
                               "num_experts_per_tok cannot exceed num_experts"),
                              (RouterConfig(4, 2, True), "ROUTER_ERROR",
                               "norm_topk_prob=true forbidden; unrenormalized routing invariant"
                               " violated")):
        with pytest.raises(DismoenError) as e:
            cfg.validate()
        j = json.loads(str(e.value))
        assert j == {"error_type": kind, "detail": detail, "stage": "router"}


def test_routing_info_json():
    info = RoutingInfo([[5, 12]], [[0.35, 0.25]], 1, 2)
    s = info.to_json()
    assert '"selected_experts":[[5,12]]' in s and '"router_probs":[[' in s
    assert json.loads(s)["selected_experts"] == [[5, 12]]


def test_generator_invariants():
    L = synth.make_layer(**synth.CONFIG_TOY, seed=0)
    for name in ("gu_packed", "d_packed", "sh_gu_packed", "sh_d_packed"):
        p = getattr(L, name)
        assert not np.any((p & 0xF) == 8) and not np.any((p >> 4) == 8)
    for name in ("gu_scales", "d_scales", "sh_gu_scales", "sh_d_scales"):
        s = getattr(L, name)
        assert np.all(s > 0) and np.all(s < 0x7C00)
    codes = np.concatenate([(L.gu_packed & 0xF), (L.gu_packed >> 4)]).astype(int)
    codes = np.where(codes >= 8, codes - 16, codes)
    counts = np.bincount(codes + 7, minlength=15)
    assert counts.min() > 0.9 * counts.mean() and counts.max() < 1.1 * counts.mean()
    assert L.router_bf16.size == 16 * 256 and L.gu_scales.size == 16 * 2 * 128 * 256 // 32
    # deterministic per seed
    L2 = synth.make_layer(**synth.CONFIG_TOY, seed=0)
    assert np.array_equal(L.gu_packed, L2.gu_packed)


def test_algorithmic_bytes():
    # 9 experts x 1 769 472 B + router 1 MiB + shared gate 4 KiB + x, y fp32
    b = synth.algorithmic_bytes_per_token(2048, 256, 8, 512, 512)
    assert b == 9 * 1769472 + 1048576 + 4096 + 8192 + 8192


def test_f10_metrics_known_values():
    """The F10 helper on values whose metrics are known in closed form
    (compare.rs:648-700): ref (3, 4) has norm 5."""
    from conftest import f10
    dmax, eps, ok = f10([3.0, 4.0], [3.0, 4.0 + 2.0 ** -10])
    assert dmax == 2.0 ** -10 and abs(eps - 2.0 ** -10 / 5.0) < 1e-18 and not ok
    dmax, eps, ok = f10([3.0, 4.0], [3.0 + 2.0 ** -20, 4.0])
    assert dmax == 2.0 ** -20 and ok
    assert f10([1.0, -2.0], [1.0, -2.0]) == (0.0, 0.0, True)
