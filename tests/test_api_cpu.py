"""CPU-side behaviour of the host API: argument checks, loud failure without a GPU path,
config builders.  No kernel runs here."""
import pytest
import torch
from torch import nn

from mindpipe_amd import w4a16 as W4
from mindpipe_amd import smoothquant as SQ


def test_compression_config_matches_reference_schema():
    cfg = W4.build_compression_config(group_size=128, ignored_layers=["lm_head"])
    assert cfg["format"] == "pack-quantized"
    assert cfg["ignore"] == ["lm_head"]
    wq = cfg["config_groups"]["group_0"]["weights"]
    assert wq == {"dynamic": False, "group_size": 128, "num_bits": 4, "observer": "minmax", "observer_kwargs": {},
                  "strategy": "group", "symmetric": True, "type": "int"}
    assert cfg["quant_method"] == "compressed-tensors"


def test_smoothquant_linear_rejects_bad_args():
    with pytest.raises(ValueError):
        SQ.SmoothQuantLinear(8, 8, act_quant="per_tensor")
    with pytest.raises(NotImplementedError):
        SQ.SmoothQuantLinear(8, 8, weight_bits=4)
    with pytest.raises(ValueError):
        SQ.SmoothQuantLinear(8, 8, scale_rule="other")


def test_module_forward_refuses_cpu_tensors():
    mod = SQ.SmoothQuantLinear(16, 8)
    with pytest.raises(RuntimeError, match="GPU"):
        mod(torch.zeros(2, 16, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="GPU"):
        SQ.quantize_activation_per_token_absmax(torch.zeros(2, 16, dtype=torch.float16))
    w4 = W4.W4A16Linear(128, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        w4(torch.zeros(1, 128, dtype=torch.float16))


def test_quantize_model_rejects_unknown_model_type():
    class M(nn.Module):
        config = type("C", (), {"model_type": "gpt2"})()
    with pytest.raises(ValueError, match="Unsupported model type"):
        SQ.quantize_model(M())
    with pytest.raises(ValueError):
        SQ.quantize_model(M(), weight_quant="per_tensor")


def test_w4_module_buffers_and_shapes():
    mod = W4.W4A16Linear(256, 64, group_size=128, zero_point=True)
    assert mod.weight_packed.shape == (64, 32) and mod.weight_packed.dtype == torch.int32
    assert mod.weight_scale.shape == (64, 2) and mod.weight_zero_point.shape == (64, 2)
    assert mod.weight_shape.tolist() == [64, 256]
    with pytest.raises(ValueError):
        W4.W4A16Linear(100, 8, group_size=128)
    with pytest.raises(NotImplementedError):
        W4.pseudo_quantize_tensor(torch.zeros(4, 128, dtype=torch.float16), n_bit=8)


def test_smooth_scales_closed_form_cpu():
    fc = nn.Linear(3, 2, bias=False)
    with torch.no_grad():
        fc.weight.copy_(torch.tensor([[1.0, -0.25, 0.0], [0.5, 0.0625, 0.0]]))
    fc = fc.half()
    s = SQ.compute_smooth_scales(fc, torch.tensor([4.0, 9.0, 0.0]), 0.5)
    assert s.dtype == torch.float16 and s.tolist()[:2] == [2.0, 6.0]
    ln = nn.LayerNorm(3).half()
    SQ.smooth_ln_fcs_llama_like(ln, [fc], torch.tensor([4.0, 9.0, 0.0]), 0.5)
    assert fc.weight[0, 0].item() == 2.0
