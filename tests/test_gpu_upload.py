"""GPU parity of layers uploaded at every group size the reference's quantizer
allows (src/format/half_float.mojo:9,24-31: {32, 64, 128, 256}, default 128),
from arrays and from the reference's file formats, against the oracle (which
dequantizes each tensor at its own group size, dequant_kernel.mojo:22-124).

Bar: ids, probabilities and shared gate bit-exact; the no-residual output
within max-abs-err <= 1e-3 x RMS(oracle output)."""
import numpy as np
import pytest

from conftest import tol_check
from dismoen import DismoenError, formats, synth

pytestmark = pytest.mark.gpu


def _check(block, oracle, L, layer, x):
    T = x.shape[0]
    y, ids, probs, shg = block.forward_arrays(layer, x, T)
    yo, ido, po, so = oracle.moe_layer_q4(L, x, T)
    assert np.array_equal(ids, ido)
    assert np.array_equal(probs.view(np.uint32), po.view(np.uint32))
    assert np.array_equal(shg.view(np.uint32), so.view(np.uint32))
    err, rms, ok = tol_check(y, yo)
    assert ok, (err, rms)


@pytest.mark.parametrize("G", [64, 128, 256])
def test_toy_layer_group_sizes_vs_oracle(block, oracle, G):
    L = synth.make_layer(**synth.CONFIG_TOY, group_size=G, seed=50 + G)
    block.upload_layer(60, L)
    x = synth.make_activations(np.random.default_rng(600 + G), (5, 256))
    _check(block, oracle, L, 60, x[:1])  # single-launch decode kernel
    _check(block, oracle, L, 60, x)      # grouped path
    block.free_layer(60)


def test_qwen_layer_g128_arrays_and_files_vs_oracle(block, oracle, tmp_path):
    """The reference's default group size at the Qwen3.6 layer shape, uploaded
    from arrays and from a quant model + safetensors shard written in the
    reference's layouts; both compared with the oracle."""
    c = synth.CONFIG_QWEN36
    L = synth.make_layer(**c, group_size=128, seed=61)
    dims = (c["hidden"], c["num_experts"], c["top_k"], c["inter"], c["inter_sh"])
    block.upload_layer(61, L)
    qp, sp = str(tmp_path / "m.quant"), str(tmp_path / "m.safetensors")
    formats.write_layer_files(qp, sp, L, model_layer=3)
    with formats.scan_quant_file(qp) as q, formats.read_header(sp) as s:
        block.upload_layer_files(62, dims, q, s, model_layer=3, group_size=128)
        # group size 0: the quant model's header's quantization.group_size
        block.upload_layer_files(64, dims, q, s, model_layer=3, group_size=0)
    x = synth.make_activations(np.random.default_rng(610), (3, c["hidden"]))
    for layer in (61, 62, 64):
        for t in range(2):
            _check(block, oracle, L, layer, x[t:t + 1])
        _check(block, oracle, L, layer, x)
    for layer in (61, 62, 64):
        block.free_layer(layer)


def test_toy_layer_g32_files_vs_oracle(block, oracle, tmp_path):
    """The file upload at G = 32 against the oracle (not only against the
    array upload)."""
    c = synth.CONFIG_TOY
    L = synth.make_layer(**c, seed=62)
    dims = (c["hidden"], c["num_experts"], c["top_k"], c["inter"], c["inter_sh"])
    qp, sp = str(tmp_path / "m.quant"), str(tmp_path / "m.safetensors")
    formats.write_layer_files(qp, sp, L, model_layer=0)
    with formats.scan_quant_file(qp) as q, formats.read_header(sp) as s:
        block.upload_layer_files(63, dims, q, s, model_layer=0)
    x = synth.make_activations(np.random.default_rng(611), (4, c["hidden"]))
    _check(block, oracle, L, 63, x[:1])
    _check(block, oracle, L, 63, x)
    block.free_layer(63)


@pytest.mark.parametrize("G", [128, 256])
def test_bad_scale_reports_source_group(block, oracle, G):
    """Scale errors name the group in the tensor's own numbering at its own
    group size, as dequant_kernel_simd does (dequant_kernel.mojo:68-80)."""
    L = synth.make_layer(**synth.CONFIG_TOY, group_size=G, seed=63)
    L.gu_scales = L.gu_scales.copy()
    L.gu_scales[5] = 0x7E00
    with pytest.raises(DismoenError, match="scale is NaN or Inf at group 5$"):
        block.upload_layer(64, L)
    L = synth.make_layer(**synth.CONFIG_TOY, group_size=G, seed=63)
    L.d_scales = L.d_scales.copy()
    L.d_scales[3] = 0x8000  # -0.0
    with pytest.raises(DismoenError, match="scale is non-positive at group 3$"):
        block.upload_layer(64, L)
    # the oracle's own dequant of the first tensor raises the same text
    n = L.hidden * L.inter
    with pytest.raises(oracle.OracleError, match="scale is non-positive at group 3$"):
        oracle.dequant_q4_bf16(L.d_scales[: n // G], L.d_packed[: n // 2], n, G)


def test_shared_expert_wider_than_routed_experts(block, oracle):
    """I_sh > E * I: the shared expert's matrices are larger than all routed
    gate/up matrices together (the upload staging is sized for the largest
    tensor group)."""
    L = synth.make_layer(hidden=128, num_experts=2, top_k=1, inter=128, inter_sh=512, seed=64)
    block.upload_layer(65, L)
    x = synth.make_activations(np.random.default_rng(612), (3, 128))
    _check(block, oracle, L, 65, x[:1])
    _check(block, oracle, L, 65, x)
    block.free_layer(65)


@pytest.mark.parametrize("G", [0, -1, 48, 512])
def test_unsupported_group_size_is_config_error(block, G):
    L = synth.make_layer(**synth.CONFIG_TOY, seed=65)
    L.group_size = G
    with pytest.raises(DismoenError, match="CONFIG_ERROR") as ei:
        block.upload_layer(66, L)
    assert ei.value.kind == "CONFIG"
