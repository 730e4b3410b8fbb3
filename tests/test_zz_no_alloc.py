"""dmh_moe_forward_noalloc: the MoE block with every buffer of the call in the
library's per-device static scratch (no allocation).  Checked through the C
ABI against dmh_moe_forward on the same device buffers, on consecutive calls
whose second input is smaller, single-token and several-token paths, with
and without caller-provided routing outputs."""
import ctypes as C

import numpy as np
import pytest

from conftest import tol_check
from dismoen import synth
from dismoen._lib import DMH_F_DEVICE, errbuf, lib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qwen_na(block):
    L = synth.make_layer(**synth.CONFIG_QWEN36, seed=90)
    block.upload_layer(90, L)
    yield L
    block.free_layer(90)


def _bufs(T, H=2048, K=8):
    import torch
    return {"y": torch.empty((T, H), dtype=torch.float32, device="cuda"),
            "ids": torch.empty((T, K), dtype=torch.int32, device="cuda"),
            "probs": torch.empty((T, K), dtype=torch.float32, device="cuda"),
            "shg": torch.empty((T,), dtype=torch.float32, device="cuda")}


def _call(fn, block, layer, xd, T, b, residual=None, with_routing=True):
    e = errbuf()
    rc = fn(block.handle, layer, xd.data_ptr(), None if residual is None else residual.data_ptr(),
            T, b["y"].data_ptr(), b["ids"].data_ptr() if with_routing else None,
            b["probs"].data_ptr() if with_routing else None,
            b["shg"].data_ptr() if with_routing else None, DMH_F_DEVICE, e, len(e))
    assert rc == 0, e.value
    block.sync()


@pytest.mark.parametrize("sizes", [(32, 8), (5, 1), (1, 1)])
def test_noalloc_matches_moe_forward(block, oracle, qwen_na, sizes):
    import torch
    L = lib()
    rng = np.random.default_rng(900 + sizes[0])
    for T in sizes:
        x = synth.make_activations(rng, (T, 2048))
        xd = torch.from_numpy(x).to("cuda")
        torch.cuda.synchronize()
        a, b = _bufs(T), _bufs(T)
        _call(L.dmh_moe_forward_noalloc, block, 90, xd, T, a)
        _call(L.dmh_moe_forward, block, 90, xd, T, b)
        for k in ("ids", "probs", "shg", "y"):
            assert np.array_equal(a[k].cpu().numpy().view(np.uint8),
                                  b[k].cpu().numpy().view(np.uint8)), (T, k)
        # and the oracle's bar
        yo, ido, po, so = oracle.moe_layer_q4(qwen_na, x, T)
        assert np.array_equal(a["ids"].cpu().numpy(), ido)
        err, rms, ok = tol_check(a["y"].cpu().numpy(), yo)
        assert ok, (T, err, rms)


def test_noalloc_residual_and_scratch_routing_outputs(block, oracle, qwen_na):
    """Routing outputs omitted (they then live in the scratch) and a residual."""
    import torch
    L = lib()
    x = synth.make_activations(np.random.default_rng(910), (12, 2048))
    xd = torch.from_numpy(x).to("cuda")
    torch.cuda.synchronize()
    for T in (12, 3):
        a = _bufs(T)
        _call(L.dmh_moe_forward_noalloc, block, 90, xd[:T], T, a, residual=xd[:T],
              with_routing=False)
        yo, _, _, _ = oracle.moe_layer_q4(qwen_na, x[:T], T, residual=x[:T])
        err, rms, ok = tol_check(a["y"].cpu().numpy() - x[:T], yo - x[:T])
        assert ok, (T, err, rms)


def test_noalloc_rejects_what_it_cannot_do_without_allocating(block, qwen_na):
    import torch
    L = lib()
    e = errbuf()
    x = np.zeros((4, 2048), np.float32)
    y = np.zeros((4, 2048), np.float32)
    rc = L.dmh_moe_forward_noalloc(block.handle, 90, x.ctypes.data, None, 4, y.ctypes.data, None,
                                   None, None, 0, e, len(e))
    assert rc == 1 and b"needs DMH_F_DEVICE" in e.value
    T = 4096
    xd = torch.zeros((T, 2048), dtype=torch.float32, device="cuda")
    yd = torch.empty_like(xd)
    torch.cuda.synchronize()
    rc = L.dmh_moe_forward_noalloc(block.handle, 90, xd.data_ptr(), None, T, yd.data_ptr(), None,
                                   None, None, DMH_F_DEVICE, e, len(e))
    assert rc == 1 and b"bytes of scratch, more than the" in e.value, e.value
