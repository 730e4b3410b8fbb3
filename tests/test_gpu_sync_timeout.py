"""The time-out path of the fused kernels' waits, forced from the host.

The fused kernels (the 4-bit decode kernel, the several-token launch and the
GGUF one-launch kernel) run every workgroup at once and pass data between them
through polled words.  Every such wait is bounded: after the context's bound
of polls it records a sync error and the kernel runs on to its end, so the
grid always drains.  A context whose bound is zero polls
(dmh_set_spin_limit(ctx, 0)) makes every wait give up at once; the kernels
still exit normally (their indices stay in range: selected ids are clamped
to the layer), only their outputs are wrong and flagged.

Checked here, against the oracle (ids and probabilities bit for bit,
outputs within max-abs-err <= 1e-3 x RMS):
- a host-pointer call whose waits gave up is rerun on the multi-kernel path
  (no waits between workgroups) and returns the oracle's result; the context
  counts one fallback (dmh_sync_fallbacks);
- a DMH_F_DEVICE call reports the hand-off error text at dmh_sync;
- with the default bound restored, the next host and device calls run the
  fused kernel again and are correct;
- the several-token launch, the 40-layer stack's host call and the GGUF
  layer's host call fall back the same way."""
import numpy as np
import pytest

from conftest import tol_check
from dismoen import DismoenError, gguf, synth
from test_gpu_gguf_moe import MINI, MINI_DIMS, oracle_port_moe

pytestmark = pytest.mark.gpu

SLOT = 90


def _check(oracle, L, x, y, ids, probs, shg):
    yo, ido, po, so = oracle.moe_layer_q4(L, x, 1)
    assert np.array_equal(ids, ido), (ids, ido)
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    assert np.array_equal(np.asarray(shg, np.float32).view(np.uint32),
                          np.asarray(so, np.float32).view(np.uint32))
    err, rms, ok = tol_check(y, yo)
    assert ok, (err, rms)


@pytest.mark.parametrize("shape", ["toy", "qwen"])
def test_decode_waits_give_up_then_fall_back(block, oracle, shape):
    import torch
    cfg = synth.CONFIG_TOY if shape == "toy" else synth.CONFIG_QWEN36
    L = synth.make_layer(**cfg, seed=91)
    H, K = L.hidden, L.top_k
    rng = np.random.default_rng(92)
    x = synth.make_activations(rng, (4, H))
    block.upload_layer(SLOT, L)
    try:
        print(f"[sync-timeout] {shape}: default bound", flush=True)
        _check(oracle, L, x[0:1], *block.forward_arrays(SLOT, x[0:1], 1))
        n0 = block.sync_fallbacks()
        block.set_spin_limit(0)
        print(f"[sync-timeout] {shape}: zero-poll bound, host call", flush=True)
        _check(oracle, L, x[1:2], *block.forward_arrays(SLOT, x[1:2], 1))
        assert block.sync_fallbacks() == n0 + 1
        print(f"[sync-timeout] {shape}: zero-poll bound, device call", flush=True)
        dev = torch.device("cuda:0")
        dx = torch.from_numpy(x[2:3].copy()).to(dev)
        dy = torch.empty((1, H), dtype=torch.float32, device=dev)
        dids = torch.empty((1, K), dtype=torch.int32, device=dev)
        dpr = torch.empty((1, K), dtype=torch.float32, device=dev)
        dsg = torch.empty((1,), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        block.forward_device(SLOT, dx.data_ptr(), 1, dy.data_ptr(), dids.data_ptr(),
                             dpr.data_ptr(), dsg.data_ptr())
        with pytest.raises(DismoenError) as ei:
            block.sync()
        assert "cross-workgroup handoff timed out" in str(ei.value), str(ei.value)
        block.set_spin_limit(None)
        print(f"[sync-timeout] {shape}: default bound again", flush=True)
        block.forward_device(SLOT, dx.data_ptr(), 1, dy.data_ptr(), dids.data_ptr(),
                             dpr.data_ptr(), dsg.data_ptr())
        block.sync()
        _check(oracle, L, x[2:3], dy.cpu().numpy(), dids.cpu().numpy(), dpr.cpu().numpy(),
               dsg.cpu().numpy())
        _check(oracle, L, x[3:4], *block.forward_arrays(SLOT, x[3:4], 1))
        assert block.sync_fallbacks() == n0 + 1
    finally:
        block.set_spin_limit(None)
        block.free_layer(SLOT)


def test_few_token_waits_give_up_then_fall_back(block, oracle):
    """The several-token launch (each token's block on one XCD) under a
    zero-poll bound: the host call is rerun on the grouped path and matches
    the oracle, a device call reports the hand-off error at dmh_sync, and
    with the default bound restored the launch is correct again."""
    import torch
    L = synth.make_layer(**synth.CONFIG_QWEN36, seed=97)
    H, K, T = L.hidden, L.top_k, 4
    x = synth.make_activations(np.random.default_rng(98), (4 * T, H))

    def check(xs, y, ids, probs, shg):
        yo, ido, po, so = oracle.moe_layer_q4(L, xs, T)
        assert np.array_equal(ids, ido), (ids, ido)
        assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
        assert np.array_equal(np.asarray(shg, np.float32).view(np.uint32),
                              np.asarray(so, np.float32).view(np.uint32))
        err, rms, ok = tol_check(y, yo)
        assert ok, (err, rms)

    block.upload_layer(SLOT, L)
    try:
        print("[sync-timeout] few tokens: default bound", flush=True)
        check(x[:T], *block.forward_arrays(SLOT, x[:T], T))
        n0 = block.sync_fallbacks()
        block.set_spin_limit(0)
        print("[sync-timeout] few tokens: zero-poll bound, host call", flush=True)
        check(x[T:2 * T], *block.forward_arrays(SLOT, x[T:2 * T], T))
        assert block.sync_fallbacks() == n0 + 1
        print("[sync-timeout] few tokens: zero-poll bound, device call", flush=True)
        dev = torch.device("cuda:0")
        dx = torch.from_numpy(x[2 * T:3 * T].copy()).to(dev)
        dy = torch.empty((T, H), dtype=torch.float32, device=dev)
        dids = torch.empty((T, K), dtype=torch.int32, device=dev)
        dpr = torch.empty((T, K), dtype=torch.float32, device=dev)
        dsg = torch.empty((T,), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        block.forward_device(SLOT, dx.data_ptr(), T, dy.data_ptr(), dids.data_ptr(),
                             dpr.data_ptr(), dsg.data_ptr())
        with pytest.raises(DismoenError) as ei:
            block.sync()
        assert "cross-workgroup handoff timed out" in str(ei.value), str(ei.value)
        block.set_spin_limit(None)
        print("[sync-timeout] few tokens: default bound again", flush=True)
        block.forward_device(SLOT, dx.data_ptr(), T, dy.data_ptr(), dids.data_ptr(),
                             dpr.data_ptr(), dsg.data_ptr())
        block.sync()
        check(x[2 * T:3 * T], dy.cpu().numpy(), dids.cpu().numpy(), dpr.cpu().numpy(),
              dsg.cpu().numpy())
        check(x[3 * T:], *block.forward_arrays(SLOT, x[3 * T:], T))
        assert block.sync_fallbacks() == n0 + 1
    finally:
        block.set_spin_limit(None)
        block.free_layer(SLOT)


def test_stack_waits_give_up_then_fall_back(block, oracle):
    nl = 3
    layers = [synth.make_layer(**synth.CONFIG_TOY, seed=93 + i) for i in range(nl)]
    rng = np.random.default_rng(96)
    for i, L in enumerate(layers):
        block.upload_layer(SLOT + i, L)
        block.set_layer_norm(SLOT + i, (1.0 + 0.25 * rng.standard_normal(L.hidden)).astype(np.float32))
    x = (rng.standard_normal((1, 256)) * 1.7).astype(np.float32)
    try:
        out0, ids0, probs0 = block.forward_stack(x, SLOT, nl, 1)
        n0 = block.sync_fallbacks()
        block.set_spin_limit(0)
        print("[sync-timeout] stack: zero-poll bound", flush=True)
        out1, ids1, probs1 = block.forward_stack(x, SLOT, nl, 1)
        assert block.sync_fallbacks() == n0 + 1
        # layer 0 sees the same input bits on both paths; deeper layers see
        # outputs that the multi-kernel path sums in another fp32 order
        assert np.array_equal(ids1, ids0)
        assert np.array_equal(probs1[0].view(np.uint32), probs0[0].view(np.uint32))
        np.testing.assert_allclose(probs1, probs0, rtol=1e-5, atol=0)
        err, rms, ok = tol_check(out1 - x, out0 - x)
        assert ok, (err, rms)
        block.set_spin_limit(None)
        out2, ids2, probs2 = block.forward_stack(x, SLOT, nl, 1)
        assert np.array_equal(ids2, ids0)
        assert np.array_equal(out2.view(np.uint32), out0.view(np.uint32))
        assert block.sync_fallbacks() == n0 + 1
    finally:
        block.set_spin_limit(None)
        for i in range(nl):
            block.free_layer(SLOT + i)


def test_gguf_waits_give_up_then_fall_back(block, oracle):
    rng = np.random.default_rng(97)
    H = MINI_DIMS[0]
    x = synth.make_activations(rng, (2, H))
    with gguf.parse_gguf_index(MINI) as g:
        block.upload_layer_gguf(SLOT, MINI_DIMS, g, model_layer=1)
        try:
            for t, lim in ((0, 0), (1, None)):
                n0 = block.sync_fallbacks()
                block.set_spin_limit(lim)
                print(f"[sync-timeout] gguf: bound {lim}", flush=True)
                y, ids, probs, _ = block.forward_port_moe_gguf(x[t:t + 1], None, SLOT, 1)
                _, rid, rp, ref0 = oracle_port_moe(oracle, g, 1, MINI_DIMS, x[t:t + 1], None,
                                                   layer=SLOT)
                assert np.array_equal(ids, rid)
                assert np.array_equal(probs.view(np.uint32), rp.view(np.uint32))
                err, rms, ok = tol_check(y, ref0)
                assert ok, (err, rms)
                assert block.sync_fallbacks() == n0 + (1 if lim == 0 else 0)
        finally:
            block.set_spin_limit(None)
            block.free_layer_gguf(SLOT)
